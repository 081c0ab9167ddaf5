"""The reference's W8A8 linear restated as a vectorised CPU path: test infrastructure and the CPU baseline leg of
bench.py only.

This is what bench.py times as the CPU baseline (kind "port") and what the tests use to check full-size shapes
cheaply: torch's CPU int8 matmul (torch._int_mm, exact int32 results) plus the same float32 epilogue chains as
w8a8_oracle.c, evaluated with torch CPU tensor arithmetic.
  quant      vllm_turing/quantfuse.py:18-24 with the zero-row rule of csrc/silu_quant.cu:57-58
  int32 mm   csrc/w8a8_gemv.cu:53-81 / csrc/w8a8_big.cu:36-43
  epilogue   order 0: csrc/w8a8_gemv.cu:87-91 (fma of the rounded acc*sa product with sw and the bias)
             order 1: csrc/w8a8_big.cu:26-35 (sa * RN32(acc * sw))
The fma of order 0 is evaluated exactly: the product of two float32 values is exact in float64, and the float64
sum is rounded to odd before the one rounding to float32 (fma32 below).
"""
import torch


def quant_torch(x):
    """Per-row dynamic symmetric int8 quant of x [M, K] (fp16/bf16/fp32) -> (q int8 [M, K], s float32 [M, 1])."""
    xf = x.float()
    amax = xf.abs().amax(dim=-1, keepdim=True)
    # a true float32 division, as the CUDA contract (csrc/silu_quant.cu:57, vLLM's eager op): torch evaluates a
    # python-scalar numerator `127.0 / amax` as reciprocal(amax) * 127, which differs in the last bit for ~25% of rows
    inv = torch.where(amax > 0, torch.full_like(amax, 127.0) / amax, torch.zeros_like(amax))
    q = torch.round(xf * inv).clamp(-128.0, 127.0).to(torch.int8)
    return q, amax / 127.0


def fma32(a, b, c):
    """Correctly rounded float32 fma(a, b, c) on float32 tensors.

    a*b is exact in float64 (48-bit significand product).  The float64 sum p + c can round once; double rounding to
    float32 is avoided by computing the float64 sum with its rounding error (two-sum) and nudging the float64 result
    to the odd neighbour when inexact ("round to odd"), after which one rounding to float32 is correct."""
    p = a.double() * b.double()
    c64 = c.double()
    s = p + c64
    bb = s - p
    err = (p - (s - bb)) + (c64 - bb)                  # exact error of the float64 addition (two-sum)
    bits = s.view(torch.int64)
    inexact = err != 0
    odd = (bits & 1) == 1
    # round to odd: if inexact and the last bit is even, move one ulp toward the exact value
    toward = torch.where(err > 0, torch.ones_like(bits), -torch.ones_like(bits))
    toward = torch.where(s < 0, -toward, toward)
    bits = torch.where(inexact & ~odd, bits + toward, bits)
    return bits.view(torch.float64).float()


def epilogue(acc, sa, sw, bias=None, out_dtype=torch.float16, order=0):
    """acc int32 [M, N]; sa float32 [M, 1] or [1]; sw float32 [N] / [N, 1] / [1]; bias [N] (out_dtype) or None."""
    fa = acc.float()
    sa = sa.reshape(-1, 1).float()
    sw = sw.reshape(1, -1).float()
    b = None if bias is None else bias.float().reshape(1, -1)
    if order == 0:
        t = fa * sa
        r = fma32(t, sw.expand_as(t), (b if b is not None else torch.zeros(1)).expand_as(t))
    else:
        t = fa * sw
        r = fma32(sa.expand_as(t), t, b.expand_as(t)) if b is not None else sa * t
    return r.to(out_dtype)


def scaled_mm(a_q, w_q, sa, sw, bias=None, out_dtype=torch.float16, order=None):
    """int8 a_q [M, K] x int8 w_q [N, K] -> out [M, N] with the reference's epilogue for that M."""
    acc = torch._int_mm(a_q, w_q.t())
    if order is None:
        order = 0 if a_q.shape[0] <= 32 else 1
    return epilogue(acc, sa, sw, bias, out_dtype, order), acc


def linear(x, w_q, sw, bias=None, out_dtype=torch.float16):
    """One W8A8 linear as the reference runs it: per-token quant of x, int8 matmul, scale epilogue."""
    a_q, sa = quant_torch(x)
    out, _ = scaled_mm(a_q, w_q, sa, sw, bias, out_dtype)
    return out
