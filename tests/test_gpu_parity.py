"""GPU parity of the HIP W8A8 path against the CPU oracle (bit-exact int8 / int32 / scales; fp16 / bf16 outputs
bit-exact where the reference's epilogue is pinned, within the fp64 closed form's tolerance otherwise).

Every kernel is called through the C ABI (directly, or through the package's torch custom ops that wrap it).  The
oracle (oracle/) runs on the CPU on the same seeded inputs; large shapes use the oracle's int32 GEMM restated
through torch._int_mm (pinned equal to it in test_oracle_pins.py).  The benchmark configurations at full size, every
output compared, are in test_gpu_configs.py.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from oracle import cpu_path

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module")
def L(oracle_lib):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from vllm_turing_amd import _lib
    return _lib.lib()


def bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def code(dt):
    return oracle.FP16 if dt == torch.float16 else oracle.BF16


def stream():
    return torch.cuda.current_stream().cuda_stream


def say(msg):
    print(msg, flush=True)


# ---------------------------------------------------------------------------------------------------------------------
# silu: every 16-bit input pattern
# ---------------------------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_silu_device_exhaustive(L, dt):
    say(f"silu_table {dt}")
    out = torch.empty(65536, dtype=torch.int16, device=DEV)
    assert L.silu_table(out.data_ptr(), code(dt), stream()) == 0
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint16)
    ref = oracle.silu_table(code(dt))
    vals = torch.from_numpy(np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.int16)).view(dt).float()
    fin = torch.isfinite(vals).numpy()
    bad = np.nonzero((got != ref) & fin)[0]
    assert bad.size == 0, f"{bad.size} silu mismatches, first {bad[:8]}"


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_silu_table_compiled_in(L, dt):
    """The table the SiLU kernel looks up is compiled into the library (silu_table dtype 2 / 3 copies it out): it equals
    the build's generator bit for bit, and the device's own silu arithmetic wherever that is not NaN (NaN there)."""
    say(f"silu compiled-in table {dt}")
    from vllm_turing_amd import silu_table as gen
    tab = torch.empty(65536, dtype=torch.int16, device=DEV)
    arith = torch.empty(65536, dtype=torch.int16, device=DEV)
    assert L.silu_table(tab.data_ptr(), code(dt) + 2, stream()) == 0
    assert L.silu_table(arith.data_ptr(), code(dt), stream()) == 0
    torch.cuda.synchronize()
    t = tab.cpu().numpy().view(np.uint16)
    a = arith.cpu().numpy().view(np.uint16)
    assert np.array_equal(t, gen.values(code(dt)))
    nan_t = torch.from_numpy(t.view(np.int16)).view(dt).isnan().numpy()
    nan_a = torch.from_numpy(a.view(np.int16)).view(dt).isnan().numpy()
    assert np.array_equal(nan_t, nan_a)
    assert np.array_equal(t[~nan_t], a[~nan_a])


def test_silu_mul_quant_captured_first(L):
    """silu_mul_quant captured in a HIP graph (no set-up call, no host synchronization inside the entry point): every
    replay equals the table kernel's and the direct kernel's eager results bit for bit."""
    say("silu_mul_quant under capture")
    M, I = 64, 17408
    g = torch.Generator().manual_seed(12)
    gu = (torch.randn(M, 2 * I, generator=g) * 3).to(torch.bfloat16).to(DEV)
    q = torch.empty(M, I, dtype=torch.int8, device=DEV)
    s = torch.empty(M, dtype=torch.float32, device=DEV)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        assert L.silu_mul_quant_bf16(gu.data_ptr(), q.data_ptr(), s.data_ptr(), M, I,
                                     torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    refs = []
    for path in (1, 2):
        qr = torch.empty(M, I, dtype=torch.int8, device=DEV)
        sr = torch.empty(M, dtype=torch.float32, device=DEV)
        assert L.silu_mul_quant_path(gu.data_ptr(), qr.data_ptr(), sr.data_ptr(), M, I, 1, path, stream()) == 0
        refs.append((qr, sr))
    for _ in range(3):
        q.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for qr, sr in refs:
            assert torch.equal(q, qr) and torch.equal(s.view(torch.int32), sr.view(torch.int32))


def _rounding_inputs():
    """Every float32 sign / exponent / top-7-mantissa pattern (the bf16 value grid, 65,536 high halves) combined with
    the low halves that decide the rounding: 0, 1, just below / at / above the halfway point, the top, and two random
    ones per high half; the fp16 grid is covered by the same set (its rounding point is bit 12 of the low half)."""
    hi = np.arange(65536, dtype=np.uint32) << 16
    lows = [0x0000, 0x0001, 0x7fff, 0x8000, 0x8001, 0xffff, 0x0fff, 0x1000, 0x1001, 0x2000, 0x3000, 0x5000]
    rng = np.random.default_rng(5)
    cols = [hi | np.uint32(v) for v in lows] + [hi | rng.integers(0, 65536, 65536, dtype=np.uint32) for _ in range(2)]
    # fp16's rounding point sits at bit 12 of the float32 mantissa: the same patterns shifted into place
    cols += [(hi & np.uint32(0xffffe000)) | np.uint32(v) for v in (0x0fff, 0x1000, 0x1001, 0x1fff)]
    u = np.concatenate(cols)
    return u.view(np.float32)


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_device_rounding(L, dt):
    say(f"f32_to_16 {dt}")
    x = _rounding_inputs()
    xd = torch.from_numpy(x).to(DEV)
    out = torch.empty(x.size, dtype=torch.int16, device=DEV)
    assert L.f32_to_16(xd.data_ptr(), out.data_ptr(), x.size, code(dt), stream()) == 0
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint16)
    ref = torch.from_numpy(x).to(dt).view(torch.int16).numpy().view(np.uint16)
    fin = np.isfinite(x)
    bad = np.nonzero((got != ref) & fin)[0]
    assert bad.size == 0, f"{bad.size} rounding mismatches, first inputs {[hex(int(v)) for v in x.view(np.uint32)[bad[:6]]]}"
    nan_in = ~fin & (x != np.inf) & (x != -np.inf)
    g = torch.from_numpy(got[nan_in].view(np.int16)).view(dt).float()
    assert torch.isnan(g).all()


# ---------------------------------------------------------------------------------------------------------------------
# int8 LM head (W8A16): float32 sums in the kernel's own order, so to tolerance against the oracle's float64 sum
# ---------------------------------------------------------------------------------------------------------------------
def _ulp16_t(v, dt):
    mant, emin = (10, -14) if dt == torch.float16 else (7, -126)
    e = torch.floor(torch.log2(torch.clamp(v.abs(), min=2.0 ** emin)))
    return 2.0 ** (e - mant)


# M = 1 (K <= 8192) and M = 2, 3 (K <= 5120) take the VALU kernel, the rest the MFMA kernel
W8A16_CASES = [(1, 17408, 5120), (4, 4096, 5120), (16, 1000, 2048), (5, 333, 4112), (32, 2048, 1024), (17, 64, 16),
               (3, 248320 // 8, 5120), (2, 1000, 2048), (1, 7, 16), (1, 333, 8192), (2, 129, 5120), (1, 100, 8208),
               (2, 31, 5136), (3, 777, 5120), (3, 64, 1024),
               # two (M <= 16) or three (M > 16) 16-row tiles per workgroup, N not a multiple of either
               (8, 31, 5136), (24, 4099, 1040), (12, 48 * 7 + 17, 272)]


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("M,N,K", W8A16_CASES)
def test_w8a16(L, dt, M, N, K):
    say(f"w8a16 M={M} N={N} K={K} {dt}")
    g = torch.Generator().manual_seed(M + N + K)
    x = torch.randn(M, K, generator=g).to(dt)
    w = torch.randint(-128, 128, (N, K), dtype=torch.int8, generator=g)
    s = (torch.rand(N, generator=g) * 2e-3 + 1e-4).float()
    bias = torch.randn(N, generator=g).to(dt) if N % 2 else None
    out = torch.empty(M, N, dtype=dt, device=DEV)
    xd, wd, sd = x.to(DEV), w.to(DEV), s.to(DEV)                  # kept alive until the kernel has run
    bd = bias.to(DEV) if bias is not None else None
    rc = L.w8a16_gemv(xd.data_ptr(), wd.data_ptr(), sd.data_ptr(), bd.data_ptr() if bd is not None else None,
                      out.data_ptr(), M, N, K, code(dt), stream())
    assert rc == 0
    torch.cuda.synchronize()
    ref = torch.from_numpy(oracle.w8a16(x, w.numpy(), s.numpy(), bias).view(np.int16)).view(dt).double()
    got = out.cpu().double()
    # float32 sums in another order than the oracle's (float64, rounded once): at most one 16-bit step apart plus the
    # float32 summation error bound K u sum|w x| s, which dominates where the logit cancels to near zero
    absdot = (x.double().abs() @ w.double().abs().T) * s.double()
    bound = _ulp16_t(ref, dt) * 1.0001 + K * 2.0 ** -24 * absdot
    over = (got - ref).abs() > bound
    assert not over.any(), f"{over.sum().item()} outputs outside the bound"
    assert (got == ref).double().mean() > 0.97
    # and the reference head's own criterion against the float64 closed form (rel <= 1e-3 of the logit scale)
    exact = (x.double() @ w.double().T) * s.double() + (bias.double() if bias is not None else 0)
    assert ((got - exact).abs() / (exact.abs() + 1e-3 * exact.abs().max())).max() < 1e-2 if dt == torch.bfloat16 \
        else ((got - exact).abs() / (exact.abs() + 1e-3 * exact.abs().max())).max() < 2e-3


@pytest.mark.parametrize("M", [1, 2, 3])
def test_w8a16_rows_small_m(L, M):
    """Gathered rows (repeats, the first and last row) on the VALU kernel equal the dense logits' columns."""
    say(f"w8a16 rows M={M}")
    g = torch.Generator().manual_seed(11 + M)
    N, K = 2500, 5120
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(DEV)
    w = torch.randint(-128, 128, (N, K), dtype=torch.int8, generator=g).to(DEV)
    sc = (torch.rand(N, generator=g) * 1e-3 + 1e-4).to(DEV)
    bias = torch.randn(N, generator=g).to(torch.bfloat16).to(DEV)
    rows = torch.tensor([N - 1, 0, 5, 5, 1234, 77], dtype=torch.int32, device=DEV)
    dense = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    sub = torch.empty(M, rows.numel(), dtype=torch.bfloat16, device=DEV)
    assert L.w8a16_gemv(x.data_ptr(), w.data_ptr(), sc.data_ptr(), bias.data_ptr(), dense.data_ptr(), M, N, K, 1,
                        stream()) == 0
    sub_b = torch.empty_like(sub)
    assert L.w8a16_gemv_rows(x.data_ptr(), w.data_ptr(), sc.data_ptr(), bias.data_ptr(), sub.data_ptr(), M,
                             rows.numel(), K, 1, rows.data_ptr(), stream()) == 0
    assert L.w8a16_gemv_rows_bounded(x.data_ptr(), w.data_ptr(), sc.data_ptr(), bias.data_ptr(), sub_b.data_ptr(), M,
                                     rows.numel(), K, 1, rows.data_ptr(), N, stream()) == 0
    torch.cuda.synchronize()
    assert torch.equal(sub.cpu(), dense[:, rows.long()].cpu())
    assert torch.equal(sub_b.cpu(), dense[:, rows.long()].cpu())


def test_w8a16_reference_argtypes(L):
    """The LM-head entry points bound exactly as the reference binds them: w8a16_gemv_rows with
    [c_void_p] * 5 + [c_int] * 4 + [c_void_p, c_void_p] (vllm_turing/draftvocab.py:269, tests/test_dhead.py:83) and
    w8a16_mma with [c_void_p] * 5 + [c_int] * 4 + [c_void_p] (vllm_turing/lmhead.py:36), called as the reference
    calls them (lmhead.py:41-52,77; draftvocab.py:44): outputs equal the package's own head bit for bit, for every cfg,
    and a null rows computes every row."""
    say("w8a16 reference argtypes")
    from vllm_turing_amd import _build, lmhead
    R = ctypes.CDLL(_build.so_path())
    R.w8a16_gemv_rows.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int] * 4 + [ctypes.c_void_p, ctypes.c_void_p]
    R.w8a16_gemv_rows.restype = ctypes.c_int
    R.w8a16_mma.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int] * 4 + [ctypes.c_void_p]
    R.w8a16_mma.restype = ctypes.c_int
    g = torch.Generator().manual_seed(31)
    N, K = 4096, 5120
    w = torch.randint(-127, 128, (N, K), dtype=torch.int8, generator=g).to(DEV)
    sc = (torch.rand(N, generator=g) * 1e-3 + 1e-4).to(DEV)
    bias = torch.randn(N, generator=g).half().to(DEV)
    st = torch.cuda.current_stream().cuda_stream
    for M, cfg in ((5, 2), (16, 2), (30, 2), (33, 1), (64, 1), (20, 0), (64, 0)):
        x = torch.randn(M, K, generator=g).half().to(DEV)
        out = torch.empty(M, N, dtype=torch.float16, device=DEV)
        assert R.w8a16_mma(x.data_ptr(), w.data_ptr(), sc.data_ptr(), bias.data_ptr(), out.data_ptr(), M, N, K, cfg,
                           st) == 0
        ref = lmhead.w8a16_mm(x, w, sc, bias)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), (M, cfg)
    assert R.w8a16_mma(x.data_ptr(), w.data_ptr(), sc.data_ptr(), None, out.data_ptr(), 33, N, K, 2, st) == -2
    for M in (1, 4, 16):
        x = torch.randn(M, K, generator=g).half().to(DEV)
        rows = torch.tensor([N - 1, 0, 9, 9, 2047], dtype=torch.int32, device=DEV)
        sub = torch.empty(M, rows.numel(), dtype=torch.float16, device=DEV)
        full = torch.empty(M, N, dtype=torch.float16, device=DEV)
        assert R.w8a16_gemv_rows(x.data_ptr(), w.data_ptr(), sc.data_ptr(), None, sub.data_ptr(), M, rows.numel(), K,
                                 0, rows.data_ptr(), st) == 0
        assert R.w8a16_gemv_rows(x.data_ptr(), w.data_ptr(), sc.data_ptr(), None, full.data_ptr(), M, N, K, 0, None,
                                 st) == 0
        dense = lmhead.w8a16_mm(x, w, sc)
        torch.cuda.synchronize()
        assert torch.equal(full, dense) and torch.equal(sub, dense[:, rows.long()]), M


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_w8a16_large_m(L, dt):
    """Above 256 rows the head is dequantized in 4096-row chunks and multiplied on the library GEMM, as the reference
    does (vllm_turing/lmhead.py:93-99): out = RN_T(RN_T(x . RN_T(w * s)^T) + bias).  Against the float64 product of x
    and the dequantized rows, within the error of those two roundings plus the float32 summation bound."""
    say(f"w8a16 large M {dt}")
    from vllm_turing_amd import lmhead
    g = torch.Generator().manual_seed(41)
    M, N, K = 300, 4096 + 1000, 2048
    x = torch.randn(M, K, generator=g).to(dt)
    w = torch.randint(-127, 128, (N, K), dtype=torch.int8, generator=g)
    s = (torch.rand(N, generator=g) * 1e-3 + 1e-4).float()
    bias = torch.randn(N, generator=g).to(dt)
    y = lmhead.w8a16_mm(x.to(DEV), w.to(DEV), s.to(DEV), bias.to(DEV))
    torch.cuda.synchronize()
    wd = (w.float() * s[:, None]).to(dt).double()
    exact = x.double() @ wd.T
    want = exact + bias.double()
    u = 2.0 ** -8 if dt == torch.bfloat16 else 2.0 ** -11          # unit roundoff of the 16-bit type
    absdot = x.double().abs() @ wd.abs().T
    bound = 1.01 * u * (exact.abs() + want.abs()) + K * 2.0 ** -24 * absdot + 1e-30
    over = (y.cpu().double() - want).abs() > bound
    assert not over.any(), f"{int(over.sum())} of {over.numel()} logits outside the bound"


def test_w8a16_rows_and_api(L):
    say("w8a16 rows + api")
    from vllm_turing_amd import lmhead
    g = torch.Generator().manual_seed(3)
    N, K = 3000, 5120
    w16 = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    wq, ws = lmhead.quantize_rows(w16.to(DEV))
    # torch divides a GPU tensor by a Python scalar as a multiply by the float32 reciprocal (on CUDA as on ROCm, so the
    # reference's own conversion does the same): scale = amax * RN32(1 / 127), then a true tensor division
    sc = w16.float().abs().amax(1).clamp(min=1e-12) * torch.tensor(1 / 127, dtype=torch.float32)
    assert torch.equal(ws.cpu(), sc)
    wq_ref = torch.round(w16.float() / sc[:, None]).clamp(-128, 127)
    assert torch.equal(wq.cpu(), wq_ref.to(torch.int8))
    x = torch.randn(2, 7, K, generator=g).to(torch.bfloat16)          # 14 rows, leading dims kept
    y = lmhead.w8a16_mm(x.to(DEV), wq, ws)
    rows = torch.tensor([2999, 0, 17, 17, 1234], dtype=torch.int32)
    yr = lmhead.w8a16_mm_rows(x.to(DEV), wq, ws, rows.to(DEV))
    x40 = torch.randn(40, K, generator=g).to(torch.bfloat16)           # two kernel passes (32 + 8 rows)
    y40 = lmhead.w8a16_mm(x40.to(DEV), wq, ws)
    torch.cuda.synchronize()
    assert y.shape == (2, 7, N)
    assert torch.equal(yr.cpu(), y.reshape(14, N)[:, rows.long()].cpu())
    ref40 = torch.from_numpy(oracle.w8a16(x40, wq.cpu().numpy(), ws.cpu().numpy()).view(np.int16)).view(torch.bfloat16)
    assert (y40.cpu() == ref40).double().mean() > 0.97


# ---------------------------------------------------------------------------------------------------------------------
# AR8 group quant / dequantised rank sum
# ---------------------------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("n", [128, 128 * 7, 4096 * 5120, 128 * 1001])
def test_ar8_quant(L, n):
    say(f"ar8_quant n={n}")
    g = torch.Generator().manual_seed(n % 9973)
    x = torch.randn(n, generator=g) * torch.rand(n // 128, generator=g).repeat_interleave(128) * 50
    x = x.half()
    if n >= 128 * 7:
        x[128:256] = 0                                     # a zero group
        x[300] = 65504.0                                   # the largest fp16
        x[600:610] = 1e-6                                  # subnormals
    xd = x.to(DEV)
    packed = torch.empty(n + n // 64, dtype=torch.uint8, device=DEV)
    assert L.ar8_quant(xd.data_ptr(), packed.data_ptr(), n, stream()) == 0
    torch.cuda.synchronize()
    assert np.array_equal(packed.cpu().numpy(), oracle.ar8_quant(x))


@pytest.mark.parametrize("ranks", [1, 2, 3, 8])
def test_ar8_dequant_sum(L, ranks):
    say(f"ar8_dequant_sum ranks={ranks}")
    from vllm_turing_amd import ar8
    n = 128 * 2000
    g = torch.Generator().manual_seed(ranks)
    xs = [(torch.randn(n, generator=g) * 3).half() for _ in range(ranks)]
    gathered = torch.cat([ar8.ar8_quant(x.to(DEV)) for x in xs])
    out = ar8.ar8_dequant_sum(gathered, n, ranks)
    if ranks == 2:                                         # the reference's two-rank entry point
        out2 = torch.empty(n, dtype=torch.float16, device=DEV)
        assert L.ar8_dequant_sum(gathered.data_ptr(), out2.data_ptr(), n, stream()) == 0
        assert torch.equal(out, out2)
    torch.cuda.synchronize()
    ref = oracle.ar8_dequant_sum(np.concatenate([oracle.ar8_quant(x) for x in xs]), n, ranks)
    assert np.array_equal(bits(out), ref)
    # a lossy all-reduce: within half a scale step per rank of the exact sum
    exact = torch.stack([x.float() for x in xs]).sum(0)
    step = sum(x.float().view(-1, 128).abs().amax(1).repeat_interleave(128) / 127 for x in xs)
    assert torch.all((out.cpu().float() - exact).abs() <= step * 0.51 + exact.abs() * 1e-3 + 1e-3)


def test_ar8_all_reduce_composition(L):
    """ar8_all_reduce with the all-gather of two 'ranks' simulated on one GPU: every rank gets the same sum."""
    say("ar8_all_reduce")
    from vllm_turing_amd import ar8
    g = torch.Generator().manual_seed(77)
    a, b = (torch.randn(64, 5120, generator=g).half().to(DEV) for _ in range(2))
    other = ar8.ar8_quant(b)
    r0 = ar8.ar8_all_reduce(a, lambda p: torch.cat([p, other]), 2)
    r1 = ar8.ar8_all_reduce(b, lambda p: torch.cat([ar8.ar8_quant(a), p]), 2)
    torch.cuda.synchronize()
    assert r0.shape == a.shape and torch.equal(r0, r1)


# ---------------------------------------------------------------------------------------------------------------------
# residual add + RMSNorm + per-token quant
# ---------------------------------------------------------------------------------------------------------------------
RNQ_CASES = [(1, 5120), (7, 5120), (300, 5120), (4, 17408), (3, 6144), (2, 136), (5, 8), (3, 5001), (2, 65536),
             (16, 49152)]


@pytest.mark.parametrize("with_res", [True, False])
@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("M,K", RNQ_CASES)
def test_rms_norm_quant(L, dt, M, K, with_res):
    say(f"rms_norm_quant M={M} K={K} {dt} residual={with_res}")
    g = torch.Generator().manual_seed(M * 13 + K)
    x = (torch.randn(M, K, generator=g) * 3).to(dt)
    if K >= 64:
        x[:, ::61] *= 25                                   # outlier channels
    if M > 2:
        x[1] = 0                                           # a zero input row (with a residual: the residual's norm)
    r = torch.randn(M, K, generator=g).to(dt) if with_res else None
    if with_res and M > 2:
        r[1] = 0                                           # zero row: scale FLT_EPSILON, q = 0
    w = (torch.rand(K, generator=g) * 1.5 + 0.25).to(dt)
    xd, wd = x.to(DEV), w.to(DEV)
    rd = r.to(DEV) if with_res else None
    q = torch.empty(M, K, dtype=torch.int8, device=DEV)
    s = torch.empty(M, dtype=torch.float32, device=DEV)
    rc = L.rms_norm_quant(xd.data_ptr(), rd.data_ptr() if with_res else None, wd.data_ptr(), None, 1e-6, q.data_ptr(),
                          s.data_ptr(), M, K, code(dt), stream())
    assert rc == 0
    torch.cuda.synchronize()
    qr, sr, rr, _ = oracle.rms_norm_quant(x, w, 1e-6, r)
    assert np.array_equal(q.cpu().numpy(), qr), f"{int((q.cpu().numpy() != qr).sum())} int8 differ"
    assert np.array_equal(s.cpu().numpy(), sr)
    if with_res:
        assert np.array_equal(bits(rd), rr)


def test_rms_norm_quant_api(L):
    """vLLM's signature: residual updated in place, scale_ub, [rows, 1] scales, leading dims kept."""
    say("rms_norm_dynamic_per_token_quant api")
    from vllm_turing_amd import rms_norm_dynamic_per_token_quant
    g = torch.Generator().manual_seed(5)
    h = torch.randn(2, 3, 5120, generator=g).to(torch.bfloat16)
    res = torch.randn(2, 3, 5120, generator=g).to(torch.bfloat16)
    w = (torch.rand(5120, generator=g) + 0.5).to(torch.bfloat16)
    res_d = res.to(DEV)
    ub = torch.tensor([2.0])
    q, s = rms_norm_dynamic_per_token_quant(h.to(DEV), w.to(DEV), 1e-6, torch.int8, ub.to(DEV), res_d)
    torch.cuda.synchronize()
    assert q.shape == (2, 3, 5120) and s.shape == (6, 1)
    qr, sr, rr, _ = oracle.rms_norm_quant(h.reshape(6, 5120), w, 1e-6, res.reshape(6, 5120), scale_ub=2.0)
    assert np.array_equal(q.reshape(6, 5120).cpu().numpy(), qr)
    assert np.array_equal(s.view(-1).cpu().numpy(), sr)
    assert np.array_equal(bits(res_d).reshape(6, 5120), rr)
    with pytest.raises(NotImplementedError):
        rms_norm_dynamic_per_token_quant(h.to(DEV), w.to(DEV), 1e-6, torch.float8_e4m3fn)


def test_rms_norm_quant_codes(L):
    assert L.rms_norm_quant(None, None, None, None, 1e-6, None, None, 4, 64, 0, None) == -1
    assert L.rms_norm_quant(16, None, 16, None, 1e-6, 16, 16, 4, 64, 2, None) == -1
    assert L.rms_norm_quant(16, None, 16, None, -1.0, 16, 16, 4, 64, 0, None) == -1
    assert L.rms_norm_quant(16, None, 16, None, 1e-6, 16, 16, 0, 64, 0, None) == 0


# ---------------------------------------------------------------------------------------------------------------------
# per-token quant
# ---------------------------------------------------------------------------------------------------------------------
QUANT_CASES = [(1, 5120), (5, 5120), (16, 5120), (300, 5120), (7, 17408), (3, 136), (4, 8), (2, 131072), (9, 5001), (3, 7),
               (64, 4104)]


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("M,K", QUANT_CASES)
def test_per_token_quant(L, dt, M, K):
    say(f"per_token_quant M={M} K={K} {dt}")
    from vllm_turing_amd import per_token_quant
    g = torch.Generator().manual_seed(M * 7 + K)
    x = (torch.randn(M, K, generator=g) * 3).to(dt)
    x[0, :] = 0                                            # zero row
    if M > 2:
        x[2, K // 3] = 900.0                               # outlier
    q, s = per_token_quant(x.to(DEV))
    torch.cuda.synchronize()
    qr, sr = oracle.quant_rows(x)
    assert np.array_equal(q.cpu().numpy(), qr)
    assert np.array_equal(s.cpu().view(-1).numpy(), sr)


def test_per_token_quant_strided_rows(L):
    say("per_token_quant strided")
    from vllm_turing_amd import per_token_quant
    g = torch.Generator().manual_seed(3)
    big = torch.randn(33, 6144, generator=g).half().to(DEV)
    x = big[:, :5120]                                       # row stride 6144
    q, s = per_token_quant(x)
    qr, sr = oracle.quant_rows(x.cpu().contiguous())
    assert np.array_equal(q.cpu().numpy(), qr) and np.array_equal(s.cpu().view(-1).numpy(), sr)


def test_per_token_quant_abi_errors(L):
    assert L.per_token_quant(None, None, None, 4, 16, 16, 0, None) == -1
    assert L.per_token_quant(1, 1, 1, 4, 16, 8, 0, None) == -1     # ldx < K
    assert L.per_token_quant(1, 1, 1, 4, 16, 16, 5, None) == -1    # dtype


# ---------------------------------------------------------------------------------------------------------------------
# SiLU * up + quant
# ---------------------------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
# I <= 40960 takes the table kernel (one persistent block per CU, once the table is built), (520, 65536) and (2, 65536)
# the direct kernel
@pytest.mark.parametrize("M,I", [(1, 8704), (7, 8704), (1680, 8704), (300, 4096), (5, 136), (4, 17408), (2, 65536),
                                 (4096, 17408), (520, 65536), (600, 136), (513, 8),
                                 (520, 40960)])
def test_silu_mul_quant(L, dt, M, I):
    say(f"silu_mul_quant M={M} I={I} {dt}")
    from vllm_turing_amd import silu_mul_quant
    g = torch.Generator().manual_seed(M + I)
    gu = (torch.randn(M, 2 * I, generator=g) * 3).to(dt)   # tests/test_silu_quant.py:26
    gu[0, :I] = 0                                          # a zero activation row (tests/test_silu_quant.py:27)
    q, s = silu_mul_quant(gu.to(DEV))
    torch.cuda.synchronize()
    qr, sr, _ = oracle.silu_mul_quant(gu)
    assert np.array_equal(q.cpu().numpy(), qr), int((q.cpu().numpy() != qr).sum())
    assert np.array_equal(s.cpu().view(-1).numpy(), sr)


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_silu_mul_quant_table_exhaustive(L, dt):
    """Every 16-bit gate pattern (NaN and infinity included) through the table kernel against the direct kernel, at
    512 rows of 128 and at one row of 40960 (the table kernel's longest): bit-identical q and scales; the dispatched
    entry point equals them; rows longer than 40960 are refused by the table path."""
    say(f"silu table kernel exhaustive {dt}")
    g = torch.Generator().manual_seed(5)
    pat = torch.arange(65536, dtype=torch.int32)
    gate = torch.where(pat >= 32768, pat - 65536, pat).to(torch.int16).view(dt)
    for M, I in ((512, 128), (1, 40960)):
        gt = gate[: M * I].view(M, I) if M * I <= 65536 else gate[:I].view(1, I)
        up = (torch.randn(M, I, generator=g) * 2).to(dt)
        gu = torch.cat([gt, up], dim=1).contiguous().to(DEV)
        outs = []
        for path in (1, 2):
            q = torch.empty(M, I, dtype=torch.int8, device=DEV)
            s = torch.empty(M, dtype=torch.float32, device=DEV)
            assert L.silu_mul_quant_path(gu.data_ptr(), q.data_ptr(), s.data_ptr(), M, I, code(dt), path, stream()) == 0
            outs.append((q, s))
        fn = L.silu_mul_quant if dt == torch.float16 else L.silu_mul_quant_bf16
        q0 = torch.empty(M, I, dtype=torch.int8, device=DEV)
        s0 = torch.empty(M, dtype=torch.float32, device=DEV)
        assert fn(gu.data_ptr(), q0.data_ptr(), s0.data_ptr(), M, I, stream()) == 0
        torch.cuda.synchronize()
        (q_d, s_d), (q_t, s_t) = outs
        assert torch.equal(q_t, q_d), int((q_t != q_d).sum())
        assert torch.equal(s_t.view(torch.int32), s_d.view(torch.int32))
        assert torch.equal(q0, q_t) and torch.equal(s0.view(torch.int32), s_t.view(torch.int32))
    g2 = torch.zeros(2, 2 * 65536, dtype=dt, device=DEV)
    qq = torch.empty(2, 65536, dtype=torch.int8, device=DEV)
    ss = torch.empty(2, dtype=torch.float32, device=DEV)
    assert L.silu_mul_quant_path(g2.data_ptr(), qq.data_ptr(), ss.data_ptr(), 2, 65536, code(dt), 2, stream()) == 1


def test_silu_mul_quant_codes(L):
    assert L.silu_mul_quant(None, None, None, 4, 12, None) == 1       # I % 8
    assert L.silu_mul_quant(None, None, None, 0, 16, None) == 0       # M == 0: nothing to do
    assert L.silu_mul_quant_bf16(None, None, None, 4, 65544, None) == 1


# ---------------------------------------------------------------------------------------------------------------------
# int32 accumulators: bit-exact
# ---------------------------------------------------------------------------------------------------------------------
def i32(L, a, w, kernel):
    M, K = a.shape
    N = w.shape[0]
    acc = torch.empty(M, N, dtype=torch.int32, device=DEV)
    rc = L.w8a8_i32(a.data_ptr(), w.data_ptr(), acc.data_ptr(), M, N, K, kernel, stream())
    assert rc == 0, rc
    torch.cuda.synchronize()
    return acc.cpu().numpy()


STREAM_SHAPES = [(1, 64, 128), (1, 17408, 5120), (2, 1000, 5136), (3, 300, 5168), (4, 256, 16), (8, 17408, 5120),
                 (2, 5120, 17408), (3, 17408, 5120), (16, 17408, 5120), (32, 17408, 5120), (20, 5120, 17408),
                 (13, 7168, 5120), (16, 5120, 8704), (17, 40, 4112), (25, 5120, 3072), (32, 300, 5168),
                 (31, 8, 48), (1, 5120, 17408), (4, 5120, 6144), (4, 16384, 5120),
                 # tile counts whose last round of four-wavefront workgroups would be under half full: two-wavefront
                 # workgroups with 3- or 2-step rings, short and ragged K (one wavefront with no K step at K = 16)
                 (12, 13312, 272), (24, 17408, 1040), (9, 13328, 16), (17, 13312, 5136),
                 # 33..64 rows: four 16-row activation tiles per step
                 (33, 1000, 5136), (64, 5120, 2048), (48, 17408, 1040), (40, 12288, 272)]


@pytest.mark.parametrize("M,N,K", STREAM_SHAPES)
def test_i32_stream_kernel(L, M, N, K):
    say(f"i32 stream M={M} N={N} K={K}")
    g = torch.Generator().manual_seed(M * 31 + N + K)
    a = torch.randint(-128, 128, (M, K), dtype=torch.int8, generator=g)
    w = torch.randint(-128, 128, (N, K), dtype=torch.int8, generator=g)
    got = i32(L, a.to(DEV), w.to(DEV), 0)
    ref = oracle.gemm_i32(a.numpy(), w.numpy())
    assert np.array_equal(got, ref), np.argwhere(got != ref)[:5]


DOT4_SHAPES = [(1, 17408, 5120), (2, 17408, 5120), (1, 1000, 5136), (2, 300, 16), (1, 64, 8192), (2, 33, 48),
               (1, 7, 1040), (1, 5120, 17408), (1, 300, 17408), (1, 129, 9232), (1, 64, 12304), (2, 100, 8192),
               (3, 17408, 5120), (3, 129, 8192), (3, 5, 48), (4, 17408, 5120), (5, 300, 5120), (4, 7, 16),
               (5, 1000, 4096)]


@pytest.mark.parametrize("M,N,K", DOT4_SHAPES)
def test_i32_dot4_kernel(L, M, N, K):
    say(f"i32 dot4 M={M} N={N} K={K}")
    g = torch.Generator().manual_seed(M * 13 + N + K)
    a = torch.randint(-128, 128, (M, K), dtype=torch.int8, generator=g)
    w = torch.randint(-128, 128, (N, K), dtype=torch.int8, generator=g)
    got = i32(L, a.to(DEV), w.to(DEV), 2)
    ref = oracle.gemm_i32(a.numpy(), w.numpy())
    assert np.array_equal(got, ref), np.argwhere(got != ref)[:5]


GEMM_SHAPES = [(33, 256, 64), (256, 256, 5120), (300, 1000, 5136), (512, 512, 80), (97, 272, 5120),
               (1024, 768, 1024), (260, 12288, 128), (64, 512, 17408), (513, 256, 5248), (4096, 256, 17408),
               # 33..128 rows: streaming passes (small N), the 4-stage 64 x 128 (N up to 12288) or 64 x 64 tiles
               (100, 12288, 272), (40, 13312, 1040), (128, 9000, 5136), (65, 20480, 144), (50, 17000, 272),
               (128, 34816, 48), (200, 5120, 1040), (256, 8192, 272)]


# prefill kernel as dispatched (1), its small configuration alone (3) and its main configuration alone (4); the
# 320- and 384-super-tile shapes take the split launch (main for the whole rounds over the CUs, small for the rest);
# the 1536- and 1649-super-tile shapes take the long-grid variant of the main configuration (next-stage loads placed
# differently), the second with a small-configuration remainder and a ragged K of three stages
GEMM_SPLIT_SHAPES = [(4096, 5120, 256), (2048, 12288, 128), (4160, 5136, 144), (4096, 24576, 144), (4160, 24592, 272)]


@pytest.mark.parametrize("kernel", [1, 3, 4, 5])
@pytest.mark.parametrize("M,N,K", GEMM_SHAPES + GEMM_SPLIT_SHAPES)
def test_i32_gemm_kernel(L, M, N, K, kernel):
    say(f"i32 gemm kernel {kernel} M={M} N={N} K={K}")
    g = torch.Generator().manual_seed(M * 17 + N + K)
    a = torch.randint(-128, 128, (M, K), dtype=torch.int8, generator=g)
    w = torch.randint(-128, 128, (N, K), dtype=torch.int8, generator=g)
    got = i32(L, a.to(DEV), w.to(DEV), kernel)
    ref = oracle.gemm_i32(a.numpy(), w.numpy()) if M * N * K < 2e9 else \
        cpu_path.scaled_mm(a, w, torch.ones(M, 1), torch.ones(N, 1))[1].numpy()
    assert np.array_equal(got, ref), np.argwhere(got != ref)[:5]


def test_i32_extreme_values(L):
    """All -128 (the largest |product|) at K = 17408: 2.85e8 per output, no overflow or saturation difference."""
    say("i32 extremes")
    K = 17408
    a = torch.full((40, K), -128, dtype=torch.int8)
    w = torch.full((64, K), -128, dtype=torch.int8)
    w[1::2] = 127
    for kernel, aa, ww in ((0, a[:8], w), (0, a[:32], w), (1, a, w), (3, a, w), (2, a[:1], w),
                           (2, a[:2, :8192].contiguous(), w[:, :8192].contiguous())):
        got = i32(L, aa.to(DEV), ww.to(DEV), kernel)
        assert np.array_equal(got, oracle.gemm_i32(aa.numpy(), ww.numpy()))


def test_i32_max_k(L):
    """The largest K the kernels take (131056, K % 16 == 0 and K < 131072): all -128 activations against rows of -128
    and 127 give sums of 2147221504 and -2130446336, within 0.01% of the int32 range, in every matmul kernel that
    takes this K (streaming at M = 8 and 32, prefill as dispatched, quarter-tile and full-tile alone)."""
    say("i32 max K")
    K = 131056
    a = torch.full((40, K), -128, dtype=torch.int8)
    w = torch.full((64, K), -128, dtype=torch.int8)
    w[1::2] = 127
    want = np.where(np.arange(64) % 2 == 0, 131056 * 16384, 131056 * -16256).astype(np.int64)
    assert want.max() < 2 ** 31 and want.min() >= -2 ** 31
    wd = w.to(DEV)
    for kernel, m in ((0, 8), (0, 32), (1, 40), (3, 40), (4, 40)):
        got = i32(L, a[:m].to(DEV), wd, kernel)
        assert np.array_equal(got, np.broadcast_to(want, (m, 64))), (kernel, m)


# ---------------------------------------------------------------------------------------------------------------------
# scaled matmul outputs through the dispatch: bit-exact against the oracle's epilogue for that path
# ---------------------------------------------------------------------------------------------------------------------
def run_scaled_mm(a, w, sa, sw, bias, dt):
    from vllm_turing_amd import cutlass_scaled_mm
    wd = w.to(DEV)
    return cutlass_scaled_mm(a.to(DEV), wd.t(), sa.to(DEV), sw.to(DEV), dt, None if bias is None else bias.to(DEV))


CASES = [
    # M, N, K, dtype, bias, per-tensor sa, expected epilogue order
    (1, 17408, 5120, torch.float16, False, False, 0),      # decode GEMV
    (1, 5120, 17408, torch.bfloat16, True, False, 0),      # VALU kernel at K = 17408
    (3, 5120, 8192, torch.float16, False, True, 0),        # VALU kernel with three rows
    (4, 7168, 5120, torch.bfloat16, True, False, 0),
    (8, 5120, 8704, torch.float16, False, True, 0),
    (12, 1000, 5136, torch.float16, True, False, 0),
    (13, 5120, 8704, torch.float16, False, False, 0),      # mid band
    (31, 8192, 5120, torch.bfloat16, True, False, 0),
    (32, 300, 5168, torch.bfloat16, False, False, 0),
    (33, 5120, 3072, torch.float16, False, False, 1),      # prefill kernel
    (300, 1024, 5120, torch.bfloat16, False, False, 1),
    (512, 12288, 5120, torch.bfloat16, True, False, 1),    # with bias -> general entry, large-M bias chain
    (100, 1000, 5120, torch.float16, False, True, 1),      # per-tensor sa -> general entry
    (4096, 5120, 512, torch.bfloat16, True, False, 1),     # 320 super tiles: main + small launches, bias
    (4160, 5136, 272, torch.float16, False, False, 1),     # ragged edges in both configurations
    (96, 10240, 1040, torch.bfloat16, True, False, 1),     # mid configuration, bias
    (70, 5120, 2064, torch.float16, True, True, 1),        # streaming passes (64 + 6 rows), bias, per-tensor sa
]


@pytest.mark.parametrize("M,N,K,dt,with_bias,per_tensor,order", CASES)
def test_scaled_mm_bits(L, M, N, K, dt, with_bias, per_tensor, order):
    say(f"scaled_mm M={M} N={N} K={K} {dt} bias={with_bias} per_tensor={per_tensor}")
    g = torch.Generator().manual_seed(M + N + K)
    a = torch.randint(-128, 128, (M, K), dtype=torch.int8, generator=g)
    w = torch.randint(-128, 128, (N, K), dtype=torch.int8, generator=g)
    sa = torch.rand(1 if per_tensor else M, 1, generator=g) * 1e-2
    sw = torch.rand(N, 1, generator=g) * 1e-3
    bias = torch.randn(N, generator=g).to(dt) if with_bias else None
    out = run_scaled_mm(a, w, sa, sw, bias, dt)
    torch.cuda.synchronize()
    acc = cpu_path.scaled_mm(a, w, sa, sw)[1] if M * N * K > 2e9 else torch.from_numpy(
        oracle.gemm_i32(a.numpy(), w.numpy()))
    ref = oracle.epilogue(acc.numpy(), sa.numpy(), sw.numpy(), None if bias is None else bits(bias), code(dt), order)
    got = bits(out)
    assert np.array_equal(got, ref), f"{int((got != ref).sum())} of {got.size} differ"
    # and the float64 closed form acc * sa * sw + bias: both chains round to float32 at most three times and then once
    # to the 16-bit type, so every output lies within one 16-bit ulp of the exact value plus 4 float32 roundings of
    # the magnitudes involved (a misplaced or missing rounding step, or a dropped scale, breaks this bound)
    prod = (acc.double() if torch.is_tensor(acc) else torch.from_numpy(acc).double()) * sa.double() * \
        sw.double().view(1, -1)
    b64 = bias.double() if bias is not None else torch.zeros(N, dtype=torch.float64)
    r64 = prod + b64
    bound = _ulp16_t(r64, dt) + 4 * 2.0 ** -24 * (prod.abs() + b64.abs())
    over = (out.cpu().double() - r64).abs() > bound
    assert not over.any(), f"{int(over.sum())} outputs further than one 16-bit ulp from the exact value"


# ---------------------------------------------------------------------------------------------------------------------
# the prefill GEMM's K split (w8a8_scaled_mm_ws): the last partial round of super tiles as K pieces met in a workspace
# ---------------------------------------------------------------------------------------------------------------------
SPLIT_SHAPES = [
    (512, 12288, 5120),     # 96 super tiles x 2 pieces of 20 stages
    (1536, 14336, 17408),   # 256 whole tiles and 80 x 3 pieces in one launch
    (4096, 5120, 17408),    # 256 whole, then 64 x 4 (the MLP down projection)
    (1000, 3000, 17424),    # 48 x 5, ragged M, N and K (K % 128 = 16: the last stage zero-filled)
    (768, 8192, 10240),     # 96 x 2 at 80 stages
    (300, 1000, 17408),     # 8 x 8
    (4096, 9472, 17408),    # 592 tiles: 256 whole in a launch of their own, 256 whole + 80 x 3 in the next
    (64, 16384, 5120),      # 64 x 64 tiles: 256 x 2 pieces
    (37, 13000, 5136),      # 204 x 2, ragged M and N, K % 128 = 16 (41 stages: pieces of 20 and 21)
    (33, 17408, 17408),     # 272 tiles at 136 stages: 240 as halves of 68, 32 as 110 + 26
    (64, 20480, 5120),      # 320 tiles: 192 as halves of 20, 128 as 32 + 8
    (40, 19000, 5136),      # 297 tiles, ragged M and N, 41 stages: 215 as 20 + 21, 82 as 33 + 8
    (64, 12288, 5120),      # 192 64 x 64 tiles x 2 pieces
    (128, 5120, 17408),     # 160 tiles (two tile rows) x 3 pieces
    (100, 1000, 17424),     # 32 tiles x 8 pieces, ragged M, N and K (137 stages)
    (40, 6000, 5136),       # 94 tiles x 2, ragged N and K
    (192, 5120, 17408),     # three tile rows: 240 tiles x 2
    (150, 4000, 17424),     # 189 tiles x 2, ragged M, N and K
]


def split_ws(L, M, N, K):
    need = L.w8a8_scaled_mm_ws_size(M, N, K)
    assert need > 4096, (M, N, K, need)                  # the shape does split
    return torch.zeros(need, dtype=torch.uint8, device=DEV)


def ws_call(L, a, w, sa, sw, bias, out, ws, dcode, sa_rows=1, sw_rows=1):
    M, K = a.shape
    N = w.shape[0]
    ptr = (lambda t: None if t is None else t.data_ptr())
    rc = L.w8a8_scaled_mm_ws(a.data_ptr(), w.data_ptr(), ptr(sa), ptr(sw), ptr(bias), out.data_ptr(), M, N, K,
                             sa_rows, sw_rows, dcode, ws.data_ptr(), ws.numel(), stream())
    assert rc == 0, rc


@pytest.mark.parametrize("M,N,K", SPLIT_SHAPES)
def test_split_i32(L, M, N, K):
    """Raw int32 accumulators of the split path whole against the exact products; the tile counters are back at zero
    and a second call on the same workspace gives the same result."""
    say(f"split i32 M={M} N={N} K={K}")
    g = torch.Generator().manual_seed(M * 3 + N + K)
    a = torch.randint(-128, 128, (M, K), dtype=torch.int8, generator=g)
    w = torch.randint(-128, 128, (N, K), dtype=torch.int8, generator=g)
    ws = split_ws(L, M, N, K)
    ad, wd = a.to(DEV), w.to(DEV)
    acc = torch.empty(M, N, dtype=torch.int32, device=DEV)
    ws_call(L, ad, wd, None, None, None, acc, ws, 2)
    torch.cuda.synchronize()
    ref = torch.from_numpy(oracle.gemm_i32(a.numpy(), w.numpy())) if M * N * K < 2e9 else torch._int_mm(a, w.t())
    got = acc.cpu()
    assert torch.equal(got, ref), f"{int((got != ref).sum())} of {ref.numel()} int32 differ"
    assert int(ws[:4096].count_nonzero()) == 0
    acc.fill_(0)
    ws_call(L, ad, wd, None, None, None, acc, ws, 2)
    torch.cuda.synchronize()
    assert torch.equal(acc.cpu(), ref)


@pytest.mark.parametrize("M,N,K,dt,with_bias", [(512, 12288, 5120, torch.bfloat16, True),
                                                (1000, 3000, 17424, torch.float16, False),
                                                (1536, 14336, 17408, torch.float16, True),
                                                (48, 13312, 5120, torch.bfloat16, True),
                                                (64, 17408, 5120, torch.float16, False),
                                                (40, 19000, 5136, torch.bfloat16, True),
                                                (64, 20480, 5120, torch.float16, True),
                                                (128, 5120, 17408, torch.bfloat16, True),
                                                (72, 8000, 5120, torch.float16, False),
                                                (160, 5120, 17408, torch.bfloat16, True)])
def test_split_bits(L, M, N, K, dt, with_bias):
    """16-bit outputs of the split path bit-identical to w8a8_scaled_mm's (no workspace) and to the oracle's large-M
    epilogue of the exact products."""
    say(f"split bits M={M} N={N} K={K} {dt} bias={with_bias}")
    g = torch.Generator().manual_seed(M + 7 * N + K)
    a = torch.randint(-128, 128, (M, K), dtype=torch.int8, generator=g)
    w = torch.randint(-128, 128, (N, K), dtype=torch.int8, generator=g)
    sa = torch.rand(M, generator=g) * 1e-2
    sw = torch.rand(N, generator=g) * 1e-3
    bias = torch.randn(N, generator=g).to(dt) if with_bias else None
    ad, wd, sad, swd = a.to(DEV), w.to(DEV), sa.to(DEV), sw.to(DEV)
    bd = None if bias is None else bias.to(DEV)
    ws = split_ws(L, M, N, K)
    out = torch.empty(M, N, dtype=dt, device=DEV)
    plain = torch.empty(M, N, dtype=dt, device=DEV)
    ws_call(L, ad, wd, sad, swd, bd, out, ws, code(dt))
    assert L.w8a8_scaled_mm(ad.data_ptr(), wd.data_ptr(), sad.data_ptr(), swd.data_ptr(),
                            None if bd is None else bd.data_ptr(), plain.data_ptr(), M, N, K, 1, 1, code(dt),
                            stream()) == 0
    torch.cuda.synchronize()
    assert np.array_equal(bits(out), bits(plain))
    acc = torch._int_mm(a, w.t())
    ref = oracle.epilogue(acc.numpy(), sa.numpy(), sw.numpy(), None if bias is None else bits(bias), code(dt),
                          oracle.ORDER_LARGE_M)
    got = bits(out)
    assert np.array_equal(got, ref), f"{int((got != ref).sum())} of {got.size} differ"


def test_split_shared_workspace_and_graph(L):
    """One workspace for calls of different shapes in a row, then the split path captured in a HIP graph and replayed
    three times with eager work in between: every result equal to the eager one."""
    say("split shared workspace + graph replay")
    shapes = [(1000, 3000, 17424), (64, 16384, 5120), (300, 1000, 17408), (64, 20480, 5120), (1000, 3000, 17424)]
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    ws = torch.zeros(4096 + cus * 262144, dtype=torch.uint8, device=DEV)
    g = torch.Generator().manual_seed(5)
    ops = []
    for M, N, K in shapes:
        a = torch.randint(-128, 128, (M, K), dtype=torch.int8, generator=g)
        w = torch.randint(-128, 128, (N, K), dtype=torch.int8, generator=g)
        ref = torch._int_mm(a, w.t())
        ops.append((a.to(DEV), w.to(DEV), torch.empty(M, N, dtype=torch.int32, device=DEV), ref))
    for a, w, acc, ref in ops:
        ws_call(L, a, w, None, None, None, acc, ws, 2)
    torch.cuda.synchronize()
    for a, w, acc, ref in ops:
        assert torch.equal(acc.cpu(), ref)
    a, w, acc, ref = ops[0]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        ws_call(L, a, w, None, None, None, acc, ws, 2)
    torch.cuda.synchronize()
    for rep in range(3):
        acc.fill_(-1)
        b2, w2, acc2, ref2 = ops[1]
        ws_call(L, b2, w2, None, None, None, acc2, ws, 2)     # eager use of the same workspace between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(acc.cpu(), ref), rep
        assert torch.equal(acc2.cpu(), ref2), rep
    assert int(ws[:4096].count_nonzero()) == 0


def test_workspace_cache(L):
    """The package's K-split workspaces: one per stream, zeroed, at most WS_STREAMS kept, and the one a captured graph
    uses kept whatever other streams come after."""
    say("workspace cache")
    from vllm_turing_amd import w8a8
    dev = torch.device(DEV, torch.cuda.current_device())
    w8a8._WS.clear()
    w8a8._WS_IN_GRAPHS.clear()
    shape = (512, 12288, 5120)
    graph_stream = torch.cuda.Stream()
    with torch.cuda.stream(graph_stream):
        ws0 = w8a8.workspace(*shape, dev)               # allocated before the capture
    y = torch.zeros(16, device=DEV)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=graph_stream):
        assert w8a8.workspace(*shape, dev) is ws0
        y.add_(1)
    key = (dev.index, graph_stream.cuda_stream)
    assert key in w8a8._WS_IN_GRAPHS
    got, streams = [], [torch.cuda.Stream() for _ in range(w8a8.WS_STREAMS + 3)]   # kept: distinct handles
    for s in streams:
        with torch.cuda.stream(s):
            got.append(w8a8.workspace(*shape, dev))
    assert len(w8a8._WS) == w8a8.WS_STREAMS + 1 and w8a8._WS[key] is ws0
    assert all(int(t[:4096].count_nonzero()) == 0 for t in got)
    assert w8a8.workspace(4096, 12288, 5120, dev) is None   # three whole rounds: no split, no workspace
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(y, torch.ones(16, device=DEV))


GEMV_QUANT_CASES = [
    # M, N, K, dtype, ldx extra, bias, zero row
    (1, 5120, 6144, torch.bfloat16, 0, False, False),     # out_proj / o_proj at M = 1
    (4, 5120, 6144, torch.bfloat16, 0, False, True),      # M = 4 at K = 6144: the fallback (quant kernel + GEMV)
    (2, 5120, 6144, torch.float16, 64, True, True),       # strided rows, bias, a zero row
    (3, 1000, 8192, torch.bfloat16, 8, True, False),
    (1, 5120, 17408, torch.float16, 0, False, False),     # the longest K of the fused kernel at one row
    (5, 333, 5120, torch.float16, 0, True, True),
    (1, 96, 272, torch.bfloat16, 0, False, False),        # K not a multiple of the 1 KB row chunk
    (1, 5120, 17408, torch.bfloat16, 64, True, True),     # the fused kernel: strided row, bias, an all-zero row
    (1, 2000, 16400, torch.float16, 8, True, False),      # the fused kernel: K past every thread's full share
    (8, 4096, 5120, torch.bfloat16, 0, False, True),      # M = 8: fallback
    (12, 2048, 1024, torch.float16, 16, True, False),
]


@pytest.mark.parametrize("M,N,K,dt,extra,with_bias,zero_row", GEMV_QUANT_CASES)
def test_gemv_quant_bits(L, M, N, K, dt, extra, with_bias, zero_row):
    """w8a8_gemv_quant (quantization fused into the GEMV) against per_token_quant + w8a8_gemv and the oracle: the
    int8 rows, scales and outputs bit for bit."""
    say(f"gemv_quant M={M} N={N} K={K} {dt} ldx+{extra} bias={with_bias}")
    from vllm_turing_amd import w8a8
    g = torch.Generator().manual_seed(M * 7 + N + K)
    xf = torch.randn(M, K + extra, generator=g)
    xf[:, torch.randperm(K, generator=g)[:max(1, K // 200)]] *= 20
    if zero_row:
        xf[M // 2] = 0
    xfull = xf.to(dt)
    x = xfull[:, :K]                                              # rows of stride K + extra
    w = torch.randint(-127, 128, (N, K), dtype=torch.int8, generator=g)
    sw = torch.rand(N, 1, generator=g) * 1e-2 + 1e-4
    bias = torch.randn(N, generator=g).to(dt) if with_bias else None
    xd = xfull.to(DEV)[:, :K]
    wd, swd, bd = w.to(DEV), sw.to(DEV), (bias.to(DEV) if bias is not None else None)
    out = torch.empty(M, N, dtype=dt, device=DEV)
    xq = torch.empty(M, K, dtype=torch.int8, device=DEV)
    xs = torch.empty(M, dtype=torch.float32, device=DEV)
    assert L.w8a8_gemv_quant(xd.data_ptr(), xd.stride(0), xq.data_ptr(), xs.data_ptr(), wd.data_ptr(), swd.data_ptr(),
                             bd.data_ptr() if bd is not None else None, out.data_ptr(), M, N, K, 1, code(dt),
                             stream()) == 0
    # the two-launch route
    q2 = torch.empty(M, K, dtype=torch.int8, device=DEV)
    s2 = torch.empty(M, dtype=torch.float32, device=DEV)
    out2 = torch.empty(M, N, dtype=dt, device=DEV)
    assert L.per_token_quant(xd.data_ptr(), q2.data_ptr(), s2.data_ptr(), M, K, xd.stride(0), code(dt), stream()) == 0
    assert L.w8a8_gemv(q2.data_ptr(), wd.data_ptr(), s2.data_ptr(), swd.data_ptr(),
                       bd.data_ptr() if bd is not None else None, out2.data_ptr(), M, N, K, 1, 1, code(dt),
                       stream()) == 0
    y = w8a8.gemv_quant(xd, wd, swd, bd) if w8a8.gemv_quant_ok(xd, wd, swd, bd) else None
    torch.cuda.synchronize()
    assert torch.equal(xq, q2) and torch.equal(xs.view(torch.int32), s2.view(torch.int32))
    assert torch.equal(out, out2)
    qr, sr = oracle.quant_rows(x.contiguous())
    assert np.array_equal(xq.cpu().numpy(), qr) and np.array_equal(xs.cpu().numpy(), sr)
    ref = oracle.epilogue(oracle.gemm_i32(qr, w.numpy()), sr, sw.numpy(), None if bias is None else bits(bias),
                          code(dt), oracle.ORDER_SMALL_M)
    assert np.array_equal(bits(out), ref)
    if y is not None:
        assert torch.equal(y, out)


GEMV_SILU_CASES = [
    # M, I, K, dtype, bias, per-tensor scales
    (1, 17408, 5120, torch.bfloat16, False, False),      # the decode gate_up of the stack at one row
    (1, 2000, 17408, torch.float16, True, False),        # the longest K at one row
    (2, 1000, 8192, torch.float16, False, True),         # per-tensor activation scale
    (3, 333, 5136, torch.bfloat16, True, False),         # K not a multiple of the 1 KB row chunk
    (4, 17408, 5120, torch.float16, False, False),
    (5, 64, 16, torch.bfloat16, True, True),
    (1, 7, 5120, torch.float16, False, False),           # fewer pairs than lanes of one wavefront
]


@pytest.mark.parametrize("M,I,K,dt,with_bias,per_tensor", GEMV_SILU_CASES)
def test_gemv_silu_bits(L, M, I, K, dt, with_bias, per_tensor):
    """w8a8_gemv_silu (SiLU * up in the gate_up GEMV's epilogue) against the oracle: the 16-bit silu(g) * u of the
    oracle's gate_up output bit for bit, and per_token_quant of it equal to the oracle's silu_mul_quant (q and scales),
    i.e. to silu_mul_quant of the GEMV's output; the package's decode MLP equal to its two-GEMM chain."""
    say(f"gemv_silu M={M} I={I} K={K} {dt} bias={with_bias} per_tensor={per_tensor}")
    g = torch.Generator().manual_seed(M * 5 + I + K)
    a = torch.randint(-128, 128, (M, K), dtype=torch.int8, generator=g)
    w = torch.randint(-128, 128, (2 * I, K), dtype=torch.int8, generator=g)
    sa = torch.rand(1 if per_tensor else M, generator=g) * 1e-2 + 1e-4
    sw = torch.rand(1 if per_tensor else 2 * I, generator=g) * 2e-3 + 1e-5
    bias = torch.randn(2 * I, generator=g).to(dt) if with_bias else None
    ad, wd, sad, swd = a.to(DEV), w.to(DEV), sa.to(DEV), sw.to(DEV)
    bd = None if bias is None else bias.to(DEV)
    h = torch.empty(M, I, dtype=dt, device=DEV)
    assert L.w8a8_gemv_silu(ad.data_ptr(), wd.data_ptr(), sad.data_ptr(), swd.data_ptr(),
                            None if bd is None else bd.data_ptr(), h.data_ptr(), M, I, K, int(not per_tensor),
                            int(not per_tensor), code(dt), stream()) == 0
    q = torch.empty(M, I, dtype=torch.int8, device=DEV)
    s = torch.empty(M, dtype=torch.float32, device=DEV)
    assert L.per_token_quant(h.data_ptr(), q.data_ptr(), s.data_ptr(), M, I, I, code(dt), stream()) == 0
    torch.cuda.synchronize()
    gu_bits = oracle.epilogue(oracle.gemm_i32(a.numpy(), w.numpy()), sa.numpy(), sw.numpy(),
                              None if bias is None else bits(bias), code(dt), oracle.ORDER_SMALL_M)
    gu = torch.from_numpy(gu_bits.view(np.int16)).view(dt)
    qr, sr, act = oracle.silu_mul_quant(gu)
    assert np.array_equal(bits(h), act), f"{int((bits(h) != act).sum())} of {act.size} silu * up values differ"
    assert np.array_equal(q.cpu().numpy(), qr) and np.array_equal(s.cpu().numpy(), sr)


@pytest.mark.parametrize("M", [1, 4])
def test_decode_mlp_fused_chain(L, M):
    """mlp_quantized at decode row counts (gemv_silu, then the down GEMV quantizing its own input) against the
    reference's chain through the dispatch (GEMV -> silu_mul_quant -> GEMV): identical outputs."""
    say(f"decode MLP fused chain M={M}")
    from vllm_turing_amd import tailoverlap, w8a8
    H, I = 1024, 2048
    g = torch.Generator().manual_seed(M)
    x_q = torch.randint(-128, 128, (M, H), dtype=torch.int8, generator=g).to(DEV)
    x_s = (torch.rand(M, 1, generator=g) * 1e-2 + 1e-4).to(DEV)
    w_gu = torch.randint(-128, 128, (2 * I, H), dtype=torch.int8, generator=g).to(DEV)
    sw_gu = (torch.rand(2 * I, 1, generator=g) * 2e-3 + 1e-5).to(DEV)
    w_d = torch.randint(-128, 128, (H, I), dtype=torch.int8, generator=g).to(DEV)
    sw_d = (torch.rand(H, 1, generator=g) * 2e-3 + 1e-5).to(DEV)
    assert tailoverlap.gemv_silu_ok(x_q, x_s, w_gu, sw_gu)
    got = tailoverlap.mlp_quantized(x_q, x_s, w_gu, sw_gu, w_d, sw_d, torch.bfloat16)
    gate_up = w8a8.cutlass_scaled_mm(x_q, w_gu.t(), x_s, sw_gu, torch.bfloat16)
    a_q, a_s = tailoverlap.silu_mul_quant(gate_up)
    want = w8a8.cutlass_scaled_mm(a_q, w_d.t(), a_s, sw_d, torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.equal(got, want)


def test_dispatch_paths(L):
    from vllm_turing_amd import w8a8
    K, N = 5120, 1024
    w = torch.zeros(N, K, dtype=torch.int8, device=DEV)
    sb = torch.ones(N, 1, device=DEV)
    for M, want in ((1, "gemv"), (12, "gemv"), (13, "mma"), (32, "mma"), (33, "big")):
        a = torch.zeros(M, K, dtype=torch.int8, device=DEV)
        sa = torch.ones(M, 1, device=DEV)
        o = torch.empty(M, N, dtype=torch.float16, device=DEV)
        got = "gemv" if w8a8.gemv_ok(o, a, w.t(), sa, sb, None) else \
            "mma" if w8a8.mma_ok(o, a, w.t(), sa, sb, None) else \
            "big" if w8a8.big_ok(o, a, w.t(), sa, sb, None) else "general"
        assert got == want, (M, got)


# ---------------------------------------------------------------------------------------------------------------------
# the benchmark configurations at full size
# ---------------------------------------------------------------------------------------------------------------------
def test_cpu_case_end_to_end(L):
    """X fp16 [16, 5120] with 0.5% outlier channels x 20, W int8 [5120, 5120]: quant, GEMV, epilogue all bit-exact."""
    say("cpu case end to end")
    from vllm_turing_amd import workloads, per_token_quant, cutlass_scaled_mm
    c = workloads.cpu_case()
    x_q, x_s = per_token_quant(c["x"].to(DEV))
    out = cutlass_scaled_mm(x_q, c["w"].to(DEV).t(), x_s, c["sw"].to(DEV), torch.float16)
    torch.cuda.synchronize()
    qr, sr = oracle.quant_rows(c["x"])
    assert np.array_equal(x_q.cpu().numpy(), qr) and np.array_equal(x_s.cpu().view(-1).numpy(), sr)
    ref, _ = oracle.scaled_mm(qr, c["w"].numpy(), sr, c["sw"].numpy(), None, oracle.FP16)
    assert np.array_equal(bits(out), ref)


@pytest.mark.parametrize("M", [1, 2, 4, 8])
def test_decode_config_full(L, M):
    say(f"decode config M={M}")
    from vllm_turing_amd import workloads, per_token_quant, cutlass_scaled_mm
    c = workloads.decode(M)
    x_q, x_s = per_token_quant(c["x"].to(DEV))
    out = cutlass_scaled_mm(x_q, c["w"].to(DEV).t(), x_s, c["sw"].to(DEV), torch.float16)
    torch.cuda.synchronize()
    qr, sr = oracle.quant_rows(c["x"])
    ref_out, _ = cpu_path.scaled_mm(torch.from_numpy(qr), c["w"], torch.from_numpy(sr), c["sw"], None, torch.float16, 0)
    assert torch.equal(out.cpu(), ref_out)


def test_mlp_tail_fused(L):
    """tailoverlap.py:145-151's fused tail: residual add + RMSNorm + quant -> gate_up -> SiLU*up+quant -> down, every
    intermediate bit-exact (M = 64, hidden 5120, intermediate 17408, GemmaRMSNorm weight 1 + w)."""
    say("mlp tail fused")
    from vllm_turing_amd import workloads, mlp_tail
    from vllm_turing_amd.normquant import gemma_weight
    c = workloads.mlp(M=64)
    g = torch.Generator().manual_seed(9)
    h = c["x"]
    res = (torch.randn(64, workloads.HIDDEN, generator=g) * 0.5).to(torch.bfloat16)
    w1 = gemma_weight((torch.randn(workloads.HIDDEN, generator=g) * 0.1).to(torch.bfloat16))
    res_d = res.to(DEV)
    wgu, wd = c["w_gate_up"].to(DEV), c["w_down"].to(DEV)
    out = mlp_tail(h.to(DEV), res_d, w1.to(DEV), 1e-6, wgu, c["sw_gate_up"].to(DEV), wd, c["sw_down"].to(DEV))
    torch.cuda.synchronize()
    qr, sr, rr, _ = oracle.rms_norm_quant(h, w1, 1e-6, res)
    assert np.array_equal(bits(res_d), rr)
    gu_ref, _ = cpu_path.scaled_mm(torch.from_numpy(qr), c["w_gate_up"], torch.from_numpy(sr), c["sw_gate_up"], None,
                                   torch.bfloat16, 1)
    aq_r, as_r, _ = oracle.silu_mul_quant(gu_ref)
    o_ref, _ = cpu_path.scaled_mm(torch.from_numpy(aq_r), c["w_down"], torch.from_numpy(as_r), c["sw_down"], None,
                                  torch.bfloat16, 1)
    assert torch.equal(out.cpu(), o_ref)


def test_checkpoint_layers_forward(L, tmp_path):
    """A converted compressed-tensors W8A8 checkpoint loaded onto the GPU: each layer's forward (per-token quant +
    scaled int8 matmul through the dispatch) bit-exact against the oracle, at decode and prefill row counts."""
    say("checkpoint layers forward")
    import sys
    sys.path.insert(0, str(__import__("pathlib").Path(__file__).parent))
    from test_checkpoint import _tiny_model
    from vllm_turing_amd import checkpoint as ck
    src, dst = tmp_path / "src", tmp_path / "dst"
    src.mkdir()
    _tiny_model(str(src))
    ck.convert(str(src), str(dst), "cuda", None, 0.5, log=lambda *a: None)
    layers, _ = ck.load(str(dst), device=DEV)
    g = torch.Generator().manual_seed(8)
    for name in ("model.language_model.layers.0.mlp.down_proj", "model.language_model.layers.0.self_attn.q_proj"):
        layer = layers[name]
        K = layer.weight.shape[1]
        for M in (3, 64):
            x = torch.randn(M, K, generator=g).to(torch.bfloat16)
            out = layer(x.to(DEV))
            torch.cuda.synchronize()
            qr, sr = oracle.quant_rows(x)
            ref, _ = oracle.scaled_mm(qr, layer.weight.cpu().numpy(), sr, layer.weight_scale.cpu().numpy().reshape(-1),
                                      None, oracle.BF16)
            assert np.array_equal(bits(out), ref), (name, M)


def test_mlp_chain_small(L):
    """gate_up GEMM -> silu_mul_quant -> down GEMM, every intermediate bit-exact (M = 64, hidden 5120,
    intermediate 17408)."""
    say("mlp chain")
    from vllm_turing_amd import workloads, per_token_quant, mlp_quantized
    from vllm_turing_amd.tailoverlap import silu_mul_quant
    from vllm_turing_amd import cutlass_scaled_mm
    c = workloads.mlp(M=64)
    x = c["x"]
    x_q, x_s = per_token_quant(x.to(DEV))
    wgu, wd = c["w_gate_up"].to(DEV), c["w_down"].to(DEV)
    gu = cutlass_scaled_mm(x_q, wgu.t(), x_s, c["sw_gate_up"].to(DEV), torch.bfloat16)
    a_q, a_s = silu_mul_quant(gu)
    out = cutlass_scaled_mm(a_q, wd.t(), a_s, c["sw_down"].to(DEV), torch.bfloat16)
    out2 = mlp_quantized(x_q, x_s, wgu, c["sw_gate_up"].to(DEV), wd, c["sw_down"].to(DEV), torch.bfloat16)
    torch.cuda.synchronize()
    qr, sr = oracle.quant_rows(x)
    gu_ref, _ = cpu_path.scaled_mm(torch.from_numpy(qr), c["w_gate_up"], torch.from_numpy(sr), c["sw_gate_up"], None,
                                   torch.bfloat16, 1)
    assert torch.equal(gu.cpu(), gu_ref)
    aq_r, as_r, _ = oracle.silu_mul_quant(gu_ref)
    assert np.array_equal(a_q.cpu().numpy(), aq_r) and np.array_equal(a_s.cpu().view(-1).numpy(), as_r)
    o_ref, _ = cpu_path.scaled_mm(torch.from_numpy(aq_r), c["w_down"], torch.from_numpy(as_r), c["sw_down"], None,
                                  torch.bfloat16, 1)
    assert torch.equal(out.cpu(), o_ref) and torch.equal(out2.cpu(), o_ref)


# ---------------------------------------------------------------------------------------------------------------------
# HIP graph capture: the decode and prefill callers replay captured launches
# ---------------------------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("M", [1, 4, 600])
def test_graph_replay_mlp(L, M):
    """norm + quant -> gate_up -> SiLU*up + quant -> down (bf16) captured in one HIP graph and replayed three rounds
    over three inputs copied in eagerly, with eager work and synchronisations between replays: every replay equals the
    eager run bit for bit (M = 600 takes the SiLU table kernel and the prefill GEMM, M = 1 and 4 the decode kernels)."""
    say(f"graph replay MLP M={M}")
    from vllm_turing_amd import cutlass_scaled_mm, rms_norm_dynamic_per_token_quant, silu_mul_quant
    H, I = 1024, 2048
    g = torch.Generator().manual_seed(M + 77)
    wgu = torch.randint(-127, 128, (2 * I, H), dtype=torch.int8, generator=g).to(DEV)
    sgu = (torch.rand(2 * I, 1, generator=g) * 1e-3 + 1e-4).to(DEV)
    wd = torch.randint(-127, 128, (H, I), dtype=torch.int8, generator=g).to(DEV)
    sd = (torch.rand(H, 1, generator=g) * 1e-3 + 1e-4).to(DEV)
    nw = (1.0 + torch.randn(H, generator=g) * 0.1).to(torch.bfloat16).to(DEV)
    inputs = [torch.randn(M, H, generator=g).to(torch.bfloat16).to(DEV) for _ in range(3)]
    x_in = torch.empty(M, H, dtype=torch.bfloat16, device=DEV)

    def step():
        q, s = rms_norm_dynamic_per_token_quant(x_in, nw, 1e-6)
        gu = cutlass_scaled_mm(q, wgu.t(), s, sgu, torch.bfloat16)
        aq, a_s = silu_mul_quant(gu)
        return cutlass_scaled_mm(aq, wd.t(), a_s, sd, torch.bfloat16)

    refs = []
    for xi in inputs:
        x_in.copy_(xi)
        refs.append(step().clone())
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        x_in.copy_(inputs[0])
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = step()
    torch.cuda.synchronize()
    for rnd in range(3):
        for k, (xi, ref) in enumerate(zip(inputs, refs)):
            x_in.copy_(xi)
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, ref), f"round {rnd} input {k}: {int((out != ref).sum())} outputs differ"
            assert float((x_in.float() * 2).abs().sum()) > 0       # eager work between replays
