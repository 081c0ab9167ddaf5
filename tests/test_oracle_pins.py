"""Pins of the CPU oracle (oracle/w8a8_oracle.c) against what the mathematics fixes, independently of the C code.

Each test is chosen so that a plausible mistake in the restatement (a missing fma contraction, a division instead of
a multiply by the rounded inverse, round-half-away instead of half-even, a transposed operand, a wrong rounding of the
int32 -> float conversion, a missed zero-row rule) fails it:
  * conversions fp16/bf16 <-> fp32: exhaustive (fp16 -> fp32) or large random samples against numpy / torch;
  * silu_h: all 65,536 fp16 and bf16 inputs against exp evaluated with the decimal module at 60 digits and
    correctly rounded to float32, followed by numpy's IEEE float32 add / divide and RN conversion;
  * int32 GEMM: torch._int_mm (oneDNN VNNI) and a float64 matmul, brute force on tiny shapes;
  * epilogues: exact rational arithmetic (fractions.Fraction) with correct rounding at each step the reference
    rounds, plus the float64 closed form of the reference's own test (tests/test_w8a8_mma.py:43-51);
  * per-token quant: hand-computed known answers, invariants, and a case where x / scale differs from x * inverse;
  * int8 LM head (W8A16): the float64 closed form within one 16-bit rounding; gathered rows against the dense result;
  * AR8 group quant: exact scales, ties to even, invariants, and the dequantised rank sum against exact rationals;
  * residual add + RMSNorm + quant: the residual against torch's IEEE float32 add and RN conversion, the normalised
    row against the float64 closed form within one 16-bit ulp, constant and zero rows, the scale bound, invariants.
"""
import decimal
import math
from fractions import Fraction

import numpy as np
import pytest
import torch

import oracle
from oracle import cpu_path

F32 = (24, -126, 127)
F16 = (11, -14, 15)
BF16 = (8, -126, 127)


def rn_bin(x, fmt):
    """Round the rational x to the nearest value of a binary format (p-bit significand, emin, emax); ties to even.
    Returns a Fraction, or +-inf on overflow."""
    p, emin, emax = fmt
    x = Fraction(x)
    if x == 0:
        return Fraction(0)
    s = -1 if x < 0 else 1
    a = abs(x)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, emin)
    ulp = Fraction(2) ** (e - (p - 1))
    n = a / ulp
    fl = n.numerator // n.denominator
    rem = n - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    v = fl * ulp
    if v >= Fraction(2) ** (emax + 1):
        return s * math.inf
    return s * v


def f16_bits(v):
    return int(np.array(float(v), np.float64).astype(np.float16).view(np.uint16)) if math.isfinite(v) else \
        (0x7C00 if v > 0 else 0xFC00)


# ---------------------------------------------------------------------------------------------------------------------
# conversions
# ---------------------------------------------------------------------------------------------------------------------
def test_h2f_exhaustive(oracle_lib):
    L = oracle_lib.lib()
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([L.o_h2f(int(b)) for b in bits], np.float32)
    fin = np.isfinite(ref)
    assert np.array_equal(got[fin].view(np.uint32), ref[fin].view(np.uint32))
    assert np.array_equal(np.isnan(got), np.isnan(ref))


def test_f2h_and_f2bf_random(oracle_lib):
    L = oracle_lib.lib()
    rng = np.random.default_rng(1)
    # random float32 bit patterns around the fp16 / bf16 ranges, plus exact ties and boundaries
    xs = np.concatenate([
        (rng.standard_normal(20000) * 10.0 ** rng.uniform(-9, 5, 20000)).astype(np.float32),
        rng.integers(0, 2 ** 32, 20000, dtype=np.uint64).astype(np.uint32).view(np.float32),
        np.array([65504, 65519.99, 65520, 65536, 2 ** -14, 2 ** -24, 2 ** -25, 3 * 2 ** -26, 1 + 2 ** -11,
                  1 + 3 * 2 ** -11, -0.0, 0.0], np.float32),
    ])
    xs = xs[np.isfinite(xs)]
    with np.errstate(over="ignore"):
        ref_h = xs.astype(np.float16).view(np.uint16)
    got_h = np.array([L.o_f2h(float(x)) for x in xs], np.uint16)
    assert np.array_equal(got_h, ref_h)
    ref_b = torch.from_numpy(xs.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got_b = np.array([L.o_f2bf(float(x)) for x in xs], np.uint16)
    assert np.array_equal(got_b, ref_b)


# ---------------------------------------------------------------------------------------------------------------------
# silu_h: exhaustive against a 60-digit decimal exp
# ---------------------------------------------------------------------------------------------------------------------
def _exp_rn32(x):
    """RN32(exp(x)) for a float x, from a 60-digit decimal exp; exact handling of float64 double rounding."""
    if x > 100.0:
        return np.float32(np.inf)
    if x < -110.0:
        return np.float32(0.0)
    with decimal.localcontext() as ctx:
        ctx.prec = 60
        d = decimal.Decimal(x).exp()
    d64 = float(d)
    with np.errstate(over="ignore"):
        c = np.float32(d64)
    lo = np.nextafter(c, np.float32(0))
    hi = np.nextafter(c, np.float32(np.inf))
    # if d64 sits exactly on a float32 midpoint, the decimal decides; otherwise RN64 then RN32 is correct
    for nb in (lo, hi):
        if np.isfinite(nb) and np.isfinite(c):
            mid = (float(c) + float(nb)) / 2.0
            if d64 == mid:
                return nb if (d > decimal.Decimal(mid)) == (nb > c) else c
    return c


@pytest.mark.parametrize("dtype", [oracle.FP16, oracle.BF16])
def test_silu_exhaustive_vs_decimal(oracle_lib, dtype):
    table = oracle_lib.silu_table(dtype)
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    if dtype == oracle.FP16:
        f = bits.view(np.float16).astype(np.float32)
    else:
        f = (bits.astype(np.uint32) << 16).view(np.float32)
    fin = np.isfinite(f)
    e = np.array([_exp_rn32(-float(v)) if ok else np.float32(0) for v, ok in zip(f, fin)], np.float32)
    with np.errstate(over="ignore", invalid="ignore", divide="ignore"):
        d = np.float32(1.0) + e
        s = f / d
    if dtype == oracle.FP16:
        ref = s.astype(np.float16).view(np.uint16)
    else:
        ref = torch.from_numpy(s.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    # signed zeros: -f / inf is -0 for large negative f; compare bit patterns (finite inputs only)
    assert np.array_equal(table[fin], ref[fin]), np.nonzero(table[fin] != ref[fin])[0][:10]


def test_silu_known_values(oracle_lib):
    # silu(0) = 0, silu(1) = 1 / (1 + e^-1) = 0.731058578..., silu(-1) = -0.268941421...; silu(20) -> 20 in fp16
    h = lambda v: f16_bits(v)
    assert oracle_lib.silu_h(h(0.0)) == 0
    assert oracle_lib.silu_h(h(1.0)) == h(0.7310585786300049)
    assert oracle_lib.silu_h(h(-1.0)) == h(-0.2689414213699951)
    assert oracle_lib.silu_h(h(20.0)) == h(20.0)
    assert oracle_lib.silu_h(h(-30.0)) in (0x8000, h(-30.0 * math.exp(-30.0)))


# ---------------------------------------------------------------------------------------------------------------------
# int32 GEMM
# ---------------------------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("M,N,K", [(1, 1, 16), (3, 5, 32), (16, 64, 5120), (33, 40, 4112)])
def test_gemm_i32_vs_torch_and_f64(oracle_lib, M, N, K):
    g = torch.Generator().manual_seed(M * 1000 + N)
    a = torch.randint(-128, 128, (M, K), dtype=torch.int8, generator=g)
    w = torch.randint(-128, 128, (N, K), dtype=torch.int8, generator=g)
    acc = oracle_lib.gemm_i32(a.numpy(), w.numpy())
    ref64 = a.double() @ w.double().t()
    assert np.array_equal(acc, ref64.numpy().astype(np.int64))
    if M >= 2 or K >= 32:
        # torch._int_mm needs M > 16 on some backends; pad rows to 32
        ap = torch.zeros(max(M, 32), K, dtype=torch.int8)
        ap[:M] = a
        ref = torch._int_mm(ap, w.t().contiguous())[:M]
        assert np.array_equal(acc, ref.numpy())


def test_gemm_i32_extremes(oracle_lib):
    # all -128 x -128 over K = 17408 (the down projection's K): 2.85e8, inside int32
    K = 17408
    a = np.full((1, K), -128, np.int8)
    w = np.full((2, K), -128, np.int8)
    w[1] = 127
    acc = oracle_lib.gemm_i32(a, w)
    assert acc[0, 0] == 128 * 128 * K and acc[0, 1] == -128 * 127 * K


# ---------------------------------------------------------------------------------------------------------------------
# epilogues: exact rational arithmetic with the reference's rounding points
# ---------------------------------------------------------------------------------------------------------------------
def _epi_exact(acc, sa, sw, b, order, fmt):
    fa = rn_bin(Fraction(int(acc)), F32)                       # int32 -> float32 (RN for |acc| > 2^24)
    sa, sw = Fraction(float(sa)), Fraction(float(sw))
    bb = Fraction(float(b)) if b is not None else Fraction(0)
    if order == 0:
        t = rn_bin(fa * sa, F32)
        r = rn_bin(t * sw + bb, F32)                           # fma: one rounding of the exact expression
    else:
        t = rn_bin(fa * sw, F32)
        r = rn_bin(sa * t + bb, F32) if b is not None else rn_bin(sa * t, F32)
    return rn_bin(r, fmt)


@pytest.mark.parametrize("order", [0, 1])
@pytest.mark.parametrize("dtype", [oracle.FP16, oracle.BF16])
@pytest.mark.parametrize("with_bias", [False, True])
def test_epilogue_exact_rational(oracle_lib, order, dtype, with_bias):
    rng = np.random.default_rng(7 + order + 2 * dtype + 4 * with_bias)
    M, N = 6, 97
    acc = rng.integers(-2 ** 28, 2 ** 28, (M, N)).astype(np.int32)
    acc[0, :8] = [0, 1, -1, 2 ** 24 + 1, -(2 ** 24) - 3, 2 ** 27 + 5, 16777217, 33554435]
    sa = rng.uniform(1e-3, 2e-2, M).astype(np.float32)
    sw = rng.uniform(1e-4, 1e-2, N).astype(np.float32)
    tdt = torch.float16 if dtype == oracle.FP16 else torch.bfloat16
    bias_t = torch.from_numpy(rng.standard_normal(N).astype(np.float32) * 4).to(tdt) if with_bias else None
    bias_bits = bias_t.view(torch.int16).numpy().view(np.uint16) if with_bias else None
    out = oracle_lib.epilogue(acc, sa, sw, bias_bits, dtype, order)
    fmt = F16 if dtype == oracle.FP16 else BF16
    outf = out.view(np.float16).astype(np.float64) if dtype == oracle.FP16 else \
        (out.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    for m in range(M):
        for n in range(N):
            b = float(bias_t[n].float()) if with_bias else None
            ref = _epi_exact(acc[m, n], sa[m], sw[n], b, order, fmt)
            assert Fraction(float(outf[m, n])) == ref, (m, n, order)


def test_epilogue_fma_matters(oracle_lib):
    """A case where the contracted small-M expression fma(t, sw, b) and the uncontracted RN(RN(t*sw)+b) differ: the
    oracle must give the contracted one (nvcc's default --fmad=true on csrc/w8a8_gemv.cu:91)."""
    rng = np.random.default_rng(3)
    found = 0
    for _ in range(20000):
        acc = int(rng.integers(-2 ** 20, 2 ** 20))
        sa, sw = np.float32(rng.uniform(1e-3, 1e-2)), np.float32(rng.uniform(1e-3, 1e-2))
        b = np.float32(np.float16(rng.standard_normal()))
        t = np.float32(np.float32(acc) * sa)
        fused = rn_bin(Fraction(float(t)) * Fraction(float(sw)) + Fraction(float(b)), F32)
        unfused = np.float32(np.float32(t * sw) + b)
        if Fraction(float(unfused)) != fused and rn_bin(fused, F16) != rn_bin(Fraction(float(unfused)), F16):
            bias = np.array([np.float16(b).view(np.uint16)], np.uint16)
            out = oracle_lib.epilogue(np.array([[acc]], np.int32), [sa], [sw], bias, oracle.FP16, 0)
            assert Fraction(float(out.view(np.float16)[0, 0])) == rn_bin(fused, F16)
            found += 1
            if found >= 3:
                break
    assert found >= 1


def test_epilogue_vs_reference_closed_form(oracle_lib):
    """The reference's own acceptance check (tests/test_w8a8_mma.py:43-51): float64 closed form, rel err < 4e-3."""
    g = torch.Generator().manual_seed(11)
    M, N, K = 13, 300, 5168
    a = torch.randint(-128, 128, (M, K), dtype=torch.int8, generator=g)
    w = torch.randint(-128, 128, (N, K), dtype=torch.int8, generator=g)
    sa = torch.rand(M, 1, generator=g) * 1e-2
    sb = torch.rand(N, 1, generator=g) * 1e-3
    bias = torch.randn(N, generator=g).half()
    out, _ = oracle_lib.scaled_mm(a.numpy(), w.numpy(), sa.numpy(), sb.numpy(),
                                  bias.view(torch.int16).numpy().view(np.uint16))
    ref = (a.double() @ w.double().t()) * sa.double() * sb.double().view(1, -1) + bias.double()
    o = torch.from_numpy(out.view(np.float16).astype(np.float64))
    err = ((o - ref).abs() / (ref.abs() + 1e-3)).max().item()
    assert err < 4e-3


def test_cpu_path_epilogue_matches_oracle(oracle_lib):
    """oracle/cpu_path.py (the vectorised CPU baseline) gives the same bits as the C oracle."""
    g = torch.Generator().manual_seed(5)
    for M, order, dt in ((4, 0, torch.float16), (40, 1, torch.bfloat16), (8, 0, torch.bfloat16)):
        N, K = 256, 1024
        a = torch.randint(-128, 128, (M, K), dtype=torch.int8, generator=g)
        w = torch.randint(-128, 128, (N, K), dtype=torch.int8, generator=g)
        sa = torch.rand(M, 1, generator=g) * 1e-2
        sw = torch.rand(N, 1, generator=g) * 1e-2
        for bias in (None, torch.randn(N, generator=g).to(dt)):
            out_t, acc_t = cpu_path.scaled_mm(a, w, sa, sw, bias, dt, order)
            code = oracle.FP16 if dt == torch.float16 else oracle.BF16
            bb = None if bias is None else bias.view(torch.int16).numpy().view(np.uint16)
            out_o, acc_o = oracle_lib.scaled_mm(a.numpy(), w.numpy(), sa.numpy(), sw.numpy(), bb, code, order)
            assert np.array_equal(acc_t.numpy(), acc_o)
            assert np.array_equal(out_t.view(torch.int16).numpy().view(np.uint16), out_o)


# ---------------------------------------------------------------------------------------------------------------------
# per-token quant
# ---------------------------------------------------------------------------------------------------------------------
def test_quant_known_answers(oracle_lib):
    # row 0: amax 2 -> inverse 63.5; 1 * 63.5 = 63.5 -> 64 (half to even); -2 -> -127; 0.5 -> 31.75 -> 32
    # row 1: all zero -> q 0, scale 0 (csrc/silu_quant.cu:57-58)
    # row 2: amax 127 -> inverse 1; 2.5 -> 2, 3.5 -> 4, -2.5 -> -2 (ties to even, not away from zero)
    x = np.array([[1.0, -2.0, 0.5, 0.0], [0.0, 0.0, -0.0, 0.0], [2.5, 3.5, -2.5, 127.0]], np.float16)
    q, s = oracle_lib.quant_rows(x)
    assert q.tolist() == [[64, -127, 32, 0], [0, 0, 0, 0], [2, 4, -2, 127]]
    assert s[0] == np.float32(2.0) / np.float32(127.0) and s[1] == 0.0 and s[2] == np.float32(1.0)


def test_quant_multiplies_by_rounded_inverse(oracle_lib):
    """quantfuse.py:23 multiplies by RN32(127 / absmax); dividing by the scale absmax / 127 rounds differently for
    some inputs.  Search a case where the two differ after rounding to int8 and check the oracle takes the product."""
    rng = np.random.default_rng(0)
    for _ in range(200000):
        amax = np.float32(np.float16(rng.uniform(0.5, 60.0)))
        v = np.float32(np.float16(rng.uniform(-1, 1) * float(amax)))
        inv = np.float32(127.0) / amax
        sc = amax / np.float32(127.0)
        by_mul = np.rint(np.float32(v * inv))
        by_div = np.rint(np.float32(v / sc))
        if by_mul != by_div:
            x = np.array([[amax, v]], np.float16)
            q, _ = oracle_lib.quant_rows(x)
            assert q[0, 1] == by_mul
            return
    pytest.fail("no distinguishing case found")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_quant_invariants(oracle_lib, dtype):
    g = torch.Generator().manual_seed(2)
    x = (torch.randn(64, 5120, generator=g) * 3).to(dtype)
    x[3] = 0
    x[5, 17] = 1000
    q, s = oracle_lib.quant_rows(x)
    xf = x.float().numpy()
    assert np.abs(q.astype(np.int32)).max() <= 127
    am = np.abs(xf).argmax(axis=1)
    nz = np.abs(xf).max(axis=1) > 0
    assert np.all(np.abs(q[np.arange(64), am])[nz] == 127)
    assert np.all(q[3] == 0) and s[3] == 0
    # dequantized error is at most half a step (plus float rounding of the scale)
    err = np.abs(q.astype(np.float32) * s[:, None] - xf)
    assert np.all(err <= s[:, None] * 0.5 * (1 + 1e-5) + 1e-30)
    # the torch restatement used as the CPU baseline agrees bit for bit
    qt, st = cpu_path.quant_torch(x)
    assert np.array_equal(qt.numpy(), q) and np.array_equal(st.view(-1).numpy(), s)


def test_silu_mul_quant_composition(oracle_lib):
    g = torch.Generator().manual_seed(4)
    for dt in (torch.float16, torch.bfloat16):
        M, I = 7, 136
        gu = (torch.randn(M, 2 * I, generator=g) * 3).to(dt)
        gu[0, :I] = 0                                     # a zero activation row (tests/test_silu_quant.py:27)
        q, s, act = oracle_lib.silu_mul_quant(gu)
        code = oracle.FP16 if dt == torch.float16 else oracle.BF16
        table = oracle_lib.silu_table(code)
        gb = gu.view(torch.int16).numpy().view(np.uint16)
        sg = torch.from_numpy(table[gb[:, :I]].view(np.int16)).view(dt)
        ref_act = (sg.float() * gu[:, I:].float()).to(dt)          # exact float product, one rounding
        assert np.array_equal(act, ref_act.view(torch.int16).numpy().view(np.uint16))
        q2, s2 = oracle_lib.quant_rows(ref_act)
        assert np.array_equal(q, q2) and np.array_equal(s, s2)
        assert np.all(q[0] == 0) and s[0] == 0


# ---------------------------------------------------------------------------------------------------------------------
# residual add + RMSNorm + per-token quant (vLLM's rms_norm_dynamic_per_token_quant as tailoverlap.py:145 calls it)
# ---------------------------------------------------------------------------------------------------------------------
def _ulp16(v, dt):
    """Spacing of the 16-bit format at |v| (float64 array)."""
    mant, emin = (10, -14) if dt == torch.float16 else (7, -126)
    e = np.floor(np.log2(np.maximum(np.abs(v), 2.0 ** emin)))
    return 2.0 ** (e - mant)


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("with_res", [True, False])
def test_rms_norm_quant_closed_form(oracle_lib, dt, with_res):
    g = torch.Generator().manual_seed(11)
    M, K, eps = 6, 5120, 1e-6
    x = (torch.randn(M, K, generator=g) * 2).to(dt)
    x[1, ::97] *= 40                                       # outlier channels
    r = torch.randn(M, K, generator=g).to(dt) if with_res else None
    w = (torch.rand(K, generator=g) + 0.5).to(dt)
    q, s, rb, y = oracle.rms_norm_quant(x, w, eps, r)
    sf = x.float() + (r.float() if with_res else 0)        # torch IEEE float32 add
    if with_res:
        want = sf.to(dt).view(torch.int16).numpy().view(np.uint16)
        assert np.array_equal(rb, want)
    s64 = sf.double()
    rms64 = 1.0 / torch.sqrt((s64 * s64).mean(dim=1, keepdim=True) + eps)
    t64 = (s64 * rms64).numpy()
    y64 = (s64 * rms64 * w.double()).numpy()
    yv = torch.from_numpy(y.view(np.int16)).view(dt).double().numpy()
    # two 16-bit roundings (of s * rms, then of the product with w): |error| <= ulp(t) w / 2 + ulp(y) / 2
    bound = 0.5 * _ulp16(t64, dt) * w.double().numpy() + 0.5 * _ulp16(y64, dt)
    assert np.all(np.abs(yv - y64) <= bound * (1 + 1e-5))
    # the documented chain with numpy float32 arithmetic and torch's conversions (a second implementation of the
    # contract: a dropped intermediate rounding or a fused product fails here)
    ms = np.float32((sf.double() ** 2).sum(dim=1).numpy() / K)
    rms32 = np.float32(1) / np.sqrt(ms + np.float32(eps))
    t32 = torch.from_numpy(sf.numpy() * rms32[:, None]).to(dt).float()
    y32 = (t32 * w.float()).to(dt)
    assert np.array_equal(y, y32.view(torch.int16).numpy().view(np.uint16))
    # quant: scale = absmax / 127 in float32, q = rint(y * RN32(1 / scale)) saturated, +-127 at the argmax
    absmax = np.abs(yv).max(axis=1).astype(np.float32)
    assert np.array_equal(s, np.maximum(absmax / np.float32(127), np.float32(np.finfo(np.float32).eps)))
    inv = np.float32(1) / s
    ref_q = np.clip(np.rint(yv.astype(np.float32) * inv[:, None]), -128, 127).astype(np.int8)
    assert np.array_equal(q, ref_q)
    assert np.abs(q.astype(int)).max() <= 127
    am = np.abs(yv).argmax(axis=1)
    assert np.all(np.abs(q[np.arange(M), am].astype(int)) == 127)


def test_rms_norm_quant_known_rows(oracle_lib):
    K = 4096
    for dt in (torch.float16, torch.bfloat16):
        x = torch.zeros(3, K, dtype=dt)
        x[0] = 0.75                                        # constant row: y = +1 everywhere -> q = 127, scale 1/127
        x[1] = -3.0                                        # constant negative row, weight 1: q = -127
        w = torch.ones(K, dtype=dt)
        q, s, rb, y = oracle.rms_norm_quant(x, w, 1e-6)
        assert rb is None
        assert np.all(q[0] == 127) and np.all(q[1] == -127)
        assert s[0] == np.float32(1) / np.float32(127) and s[1] == s[0]
        assert np.all(q[2] == 0) and s[2] == np.finfo(np.float32).eps    # zero row: the minimum scale, q = 0
        # residual that cancels the input: s = 0 -> zero output, residual becomes +0 / -0 sums
        r = -x
        q2, s2, rb2, _ = oracle.rms_norm_quant(x, w, 1e-6, r)
        assert np.all(q2 == 0) and np.all(s2 == np.finfo(np.float32).eps)
        assert np.all(torch.from_numpy(rb2.view(np.int16)).view(dt).float().numpy() == 0)


def test_rms_norm_quant_scale_bound(oracle_lib):
    g = torch.Generator().manual_seed(3)
    x = torch.randn(4, 1024, generator=g).half()
    w = torch.ones(1024).half()
    q, s, _, y = oracle.rms_norm_quant(x, w, 1e-5)
    ub = float(s.min()) * 127 / 2                           # below every row's absmax
    q2, s2, _, y2 = oracle.rms_norm_quant(x, w, 1e-5, scale_ub=ub)
    assert np.array_equal(y, y2)
    assert np.all(s2 == np.float32(np.float32(ub) / np.float32(127)))
    # a scale below the row's absmax saturates the largest values at -128 / 127 (vLLM's float_to_int8_rn clamp)
    assert q2.min() >= -128 and q2.max() <= 127
    assert ((q2 == 127) | (q2 == -128)).sum() > ((q == 127) | (q == -128)).sum()
    inv = np.float32(1) / s2
    yv = torch.from_numpy(y2.view(np.int16)).view(torch.float16).float().numpy()
    assert np.array_equal(q2, np.clip(np.rint(yv * inv[:, None]), -128, 127).astype(np.int8))


# ---------------------------------------------------------------------------------------------------------------------
# AR8: int8 + fp16 scale per 128-element group (csrc/host_ar.cu:133-201)
# ---------------------------------------------------------------------------------------------------------------------
def test_ar8_known_group(oracle_lib):
    x = np.zeros(256, np.float16)
    x[0] = 127.0                                           # group 0: absmax 127 -> scale exactly 1, inverse 1
    x[1:9] = [0.5, 1.5, 2.5, -0.5, -1.5, 3.49, -126.5, 63.5]
    p = oracle.ar8_quant(x)
    q = p[:256].view(np.int8)
    sc = p[256:].view(np.float16)
    assert sc[0] == 1.0 and sc[1] == 0.0                   # group 1 is all zero: scale 0 and q = 0
    assert q[:9].tolist() == [127, 0, 2, 2, 0, -2, 3, -126, 64]
    assert np.all(q[128:] == 0)


def test_ar8_invariants(oracle_lib):
    g = torch.Generator().manual_seed(21)
    x = (torch.randn(128 * 64, generator=g) * torch.rand(64, generator=g).repeat_interleave(128) * 30).half()
    x[5 * 128:6 * 128] = 0
    p = oracle.ar8_quant(x)
    n = x.numel()
    q = p[:n].view(np.int8).astype(np.int32).reshape(-1, 128)
    sc = p[n:].view(np.float16).astype(np.float32)
    xf = x.float().numpy().reshape(-1, 128)
    amax = np.abs(xf).max(axis=1)
    assert np.array_equal(sc, (amax / np.float32(127)).astype(np.float16).astype(np.float32))   # RN16(amax / 127)
    assert q.min() >= -127 and q.max() <= 127
    nz = amax > 0
    assert np.all(np.abs(q[nz][np.arange(nz.sum()), np.abs(xf[nz]).argmax(axis=1)]) == 127)
    err = np.abs(xf - q * sc[:, None])
    assert np.all(err <= sc[:, None] / 2 * (1 + 1e-6) + 1e-12)


def test_ar8_dequant_sum_exact(oracle_lib):
    g = torch.Generator().manual_seed(22)
    n = 128 * 6
    xs = [(torch.randn(n, generator=g) * 4).half() for _ in range(3)]
    packed = [oracle.ar8_quant(x) for x in xs]
    for ranks in (1, 2, 3):
        out = oracle.ar8_dequant_sum(np.concatenate(packed[:ranks]), n, ranks)
        for i in list(range(0, n, 37)) + [n - 1]:
            terms = []
            for r in range(ranks):
                q = int(packed[r][i].astype(np.int8))
                s = Fraction(float(packed[r][n:].view(np.float16)[i // 128]))
                terms.append(q * s)
            if ranks <= 2:                                 # one rounding of the exact sum to float32, then to fp16
                acc = rn_bin(sum(terms), F32)
            else:                                          # rank order, each step rounded to float32
                acc = terms[0]
                for t in terms[1:]:
                    acc = rn_bin(acc + t, F32)
            assert int(out[i]) == f16_bits(rn_bin(acc, F16)), (ranks, i)


# ---------------------------------------------------------------------------------------------------------------------
# int8 LM head, W8A16 (csrc/w8a16_gemv.cu)
# ---------------------------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_w8a16_closed_form(oracle_lib, dt):
    g = torch.Generator().manual_seed(31)
    M, N, K = 3, 200, 1024
    x = torch.randn(M, K, generator=g).to(dt)
    w = torch.randint(-127, 128, (N, K), dtype=torch.int8, generator=g)
    s = (torch.rand(N, generator=g) * 1e-3 + 1e-4).float()
    bias = torch.randn(N, generator=g).to(dt)
    out = oracle.w8a16(x, w.numpy(), s.numpy(), bias)
    ref = (x.double() @ w.double().T) * s.double() + bias.double()
    got = torch.from_numpy(out.view(np.int16)).view(dt).double()
    # one rounding to the 16-bit type after the float32 steps (the float64 sum rounded to float32, one fma)
    assert torch.all((got - ref).abs() <= torch.from_numpy(_ulp16(ref.numpy(), dt)) * 0.5001 + ref.abs() * 2 ** -22)
    # without a bias: fma with +0, i.e. the rounded product
    out0 = oracle.w8a16(x, w.numpy(), s.numpy())
    ref0 = ((x.double() @ w.double().T).float() * s).to(dt)
    assert np.array_equal(out0, ref0.view(torch.int16).numpy().view(np.uint16))
    # gathered rows = the same columns of the dense result
    rows = np.array([199, 0, 57, 57, 3], np.int32)
    assert np.array_equal(oracle.w8a16(x, w.numpy(), s.numpy(), bias, rows), out[:, rows])
