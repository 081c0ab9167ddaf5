"""CPU oracle of the W8A8 SmoothQuant linear path: TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg import this package, and only as the checker
(or, for the baseline, as the timed CPU restatement).  The product package (vllm_turing_amd) never imports it.

The arithmetic lives in w8a8_oracle.c (plain C, IEEE float32, no contraction), built by oracle/Makefile into
oracle/build/liboracle.so.  This module wraps it with numpy arrays.  Each wrapper names the reference lines it
restates; w8a8_oracle.c states how each function is pinned.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "build", "liboracle.so")
_lib = None

FP16, BF16 = 0, 1
ORDER_SMALL_M, ORDER_LARGE_M = 0, 1


def build():
    """Compile the C restatement (make in oracle/)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_SO):
            raise RuntimeError(f"oracle library missing: {_SO} (run `make -C oracle`)")
        L = ctypes.CDLL(_SO)
        vp, lg, i = ctypes.c_void_p, ctypes.c_long, ctypes.c_int
        L.o_quant_rows.argtypes = [vp, i, lg, lg, lg, vp, vp]
        L.o_gemm_i32.argtypes = [vp, vp, vp, lg, lg, lg]
        L.o_gemm_i32.restype = i
        L.o_epilogue.argtypes = [vp, vp, vp, vp, vp, lg, lg, i, i, i, i]
        L.o_silu_h.argtypes = [ctypes.c_uint16, i]
        L.o_silu_h.restype = ctypes.c_uint16
        L.o_silu_table.argtypes = [i, vp]
        L.o_silu_mul_quant.argtypes = [vp, i, lg, lg, vp, vp, vp]
        L.o_w8a16.argtypes = [vp, vp, vp, vp, vp, vp, lg, lg, lg, i]
        L.o_ar8_quant.argtypes = [vp, lg, vp]
        L.o_ar8_dequant_sum.argtypes = [vp, lg, i, vp]
        L.o_rms_norm_quant.argtypes = [vp, vp, vp, vp, ctypes.c_float, lg, lg, i, vp, vp, vp, vp]
        L.o_h2f.argtypes = [ctypes.c_uint16]
        L.o_h2f.restype = ctypes.c_float
        L.o_f2h.argtypes = [ctypes.c_float]
        L.o_f2h.restype = ctypes.c_uint16
        L.o_bf2f.argtypes = [ctypes.c_uint16]
        L.o_bf2f.restype = ctypes.c_float
        L.o_f2bf.argtypes = [ctypes.c_float]
        L.o_f2bf.restype = ctypes.c_uint16
        _lib = L
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _bits(x):
    """fp16 / bf16 data as uint16 bit patterns (numpy uint16 array) plus its dtype code."""
    if hasattr(x, "dtype") and str(x.dtype) in ("torch.float16", "torch.bfloat16"):
        import torch
        code = FP16 if x.dtype == torch.float16 else BF16
        return np.ascontiguousarray(x.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)), code
    if isinstance(x, np.ndarray) and x.dtype == np.float16:
        return np.ascontiguousarray(x.view(np.uint16)), FP16
    raise TypeError("expected fp16/bf16 torch tensor or fp16 numpy array")


def quant_rows(x):
    """Per-token dynamic int8 quant (quantfuse.py:18-24, zero-row rule silu_quant.cu:57-58).

    x: [M, K] fp16/bf16 (torch or numpy fp16) -> (q int8 [M, K], s float32 [M])."""
    xb, code = _bits(x)
    M, K = xb.shape
    q = np.empty((M, K), np.int8)
    s = np.empty(M, np.float32)
    lib().o_quant_rows(_p(xb), code, M, K, K, _p(q), _p(s))
    return q, s


def gemm_i32(a, w):
    """acc[m, n] = sum_k a[m, k] w[n, k] in exact integer arithmetic (w8a8_gemv.cu:53-81, w8a8_big.cu:36-43)."""
    a = np.ascontiguousarray(a, np.int8)
    w = np.ascontiguousarray(w, np.int8)
    M, K = a.shape
    N = w.shape[0]
    acc = np.empty((M, N), np.int32)
    if lib().o_gemm_i32(_p(a), _p(w), _p(acc), M, N, K) != 0:
        raise ValueError("K too large for exact int32 accumulation")
    return acc


def epilogue(acc, sa, sw, bias=None, dtype=FP16, order=ORDER_SMALL_M):
    """Scale epilogue (order 0: w8a8_gemv.cu:87-91; order 1: w8a8_big.cu:26-35).

    acc int32 [M, N]; sa float32 [M] or [1]; sw float32 [N] or [1]; bias uint16 bits [N] or None.
    Returns uint16 bit patterns [M, N] of fp16 (dtype 0) or bf16 (dtype 1)."""
    acc = np.ascontiguousarray(acc, np.int32)
    sa = np.ascontiguousarray(np.asarray(sa, np.float32).reshape(-1))
    sw = np.ascontiguousarray(np.asarray(sw, np.float32).reshape(-1))
    M, N = acc.shape
    out = np.empty((M, N), np.uint16)
    b = None if bias is None else np.ascontiguousarray(np.asarray(bias, np.uint16).reshape(-1))
    lib().o_epilogue(_p(acc), _p(sa), _p(sw), None if b is None else _p(b), _p(out), M, N,
                     int(sa.size > 1), int(sw.size > 1), dtype, order)
    return out


def silu_h(x_bits, dtype=FP16):
    """silu of one fp16/bf16 bit pattern (silu_quant.cu:11-14) -> bit pattern."""
    return lib().o_silu_h(int(x_bits), dtype)


def silu_table(dtype=FP16):
    """All 65,536 silu_h outputs of one type, indexed by input bit pattern."""
    t = np.empty(65536, np.uint16)
    lib().o_silu_table(dtype, _p(t))
    return t


def silu_mul_quant(gu):
    """SiLU(gate) * up + per-row int8 quant (silu_quant.cu:22-69).

    gu: [M, 2I] fp16/bf16 -> (q int8 [M, I], s float32 [M], act bit patterns uint16 [M, I])."""
    gb, code = _bits(gu)
    M, I2 = gb.shape
    I = I2 // 2
    q = np.empty((M, I), np.int8)
    s = np.empty(M, np.float32)
    act = np.empty((M, I), np.uint16)
    lib().o_silu_mul_quant(_p(gb), code, M, I, _p(q), _p(s), _p(act))
    return q, s, act


def rms_norm_quant(x, weight, eps, residual=None, scale_ub=None):
    """Residual add + RMSNorm + per-token int8 quant (vLLM's rms_norm_dynamic_per_token_quant as the reference calls it,
    vllm_turing/tailoverlap.py:145; the contract of o_rms_norm_quant).

    x, residual: [M, K] fp16/bf16; weight: [K] of the same type; eps: float; scale_ub: float or None.
    Returns (q int8 [M, K], scales float32 [M], new residual bit patterns uint16 [M, K] or None,
    normalised row bit patterns uint16 [M, K])."""
    xb, code = _bits(x)
    wb, wcode = _bits(weight)
    if wcode != code:
        raise TypeError("weight dtype differs from the input's")
    M, K = xb.shape
    rb = None
    if residual is not None:
        rb, rcode = _bits(residual)
        if rcode != code:
            raise TypeError("residual dtype differs from the input's")
        rb = rb.copy()
    q = np.empty((M, K), np.int8)
    s = np.empty(M, np.float32)
    y = np.empty((M, K), np.uint16)
    sbuf = np.empty(K, np.float32)
    ubv = None if scale_ub is None else np.array([scale_ub], np.float32)
    lib().o_rms_norm_quant(_p(xb), None if rb is None else _p(rb), _p(np.ascontiguousarray(wb.reshape(-1))),
                           None if ubv is None else _p(ubv), float(eps), M, K, code, _p(q), _p(s), _p(y), _p(sbuf))
    return q, s, rb, y


def w8a16(x, w, s, bias=None, rows=None):
    """The int8 LM head (csrc/w8a16_gemv.cu:98-117): x fp16/bf16 [M, K], w int8 [w_rows, K], s float32 [w_rows],
    bias [w_rows] of x's dtype or None, rows int32 [N] or None -> out bit patterns uint16 [M, N] (float64 sums rounded
    once to float32, then fma with the scale and bias and one rounding to the 16-bit type)."""
    xb, code = _bits(x)
    M, K = xb.shape
    w = np.ascontiguousarray(np.asarray(w, np.int8))
    s = np.ascontiguousarray(np.asarray(s, np.float32).reshape(-1))
    r = None if rows is None else np.ascontiguousarray(np.asarray(rows, np.int32).reshape(-1))
    N = w.shape[0] if r is None else r.size
    b = None
    if bias is not None:
        b, bcode = _bits(bias)
        b = np.ascontiguousarray(b.reshape(-1))
    out = np.empty((M, N), np.uint16)
    lib().o_w8a16(_p(xb), _p(w), _p(s), None if b is None else _p(b), None if r is None else _p(r), _p(out), M, N, K,
                  code)
    return out


def ar8_quant(x):
    """AR8 group quantization (csrc/host_ar.cu:137-164): fp16 [n] (n % 128 == 0) -> packed uint8 [n + n / 64]
    (n int8 then n / 128 fp16 scales)."""
    xb, code = _bits(x)
    if code != FP16:
        raise TypeError("AR8 takes float16")
    xb = np.ascontiguousarray(xb.reshape(-1))
    n = xb.size
    if n % 128:
        raise ValueError("n % 128 != 0")
    packed = np.empty(n + n // 64, np.uint8)
    lib().o_ar8_quant(_p(xb), n, _p(packed))
    return packed


def ar8_dequant_sum(gathered, n, ranks=2):
    """Sum of the dequantised packed blocks of `ranks` ranks (csrc/host_ar.cu:166-183) -> fp16 bit patterns [n]."""
    g = np.ascontiguousarray(np.asarray(gathered, np.uint8).reshape(-1))
    if g.size != ranks * (n + n // 64):
        raise ValueError("gathered size")
    out = np.empty(n, np.uint16)
    lib().o_ar8_dequant_sum(_p(g), n, ranks, _p(out))
    return out


def scaled_mm(a_q, w_q, sa, sw, bias=None, dtype=FP16, order=None):
    """The whole scaled int8 matmul: acc = a_q . w_q^T, then the epilogue of the reference path that M takes
    (order 0 for M <= 32, the GEMV / MMA kernels; order 1 above, w8a8.py:108-117 dispatch)."""
    acc = gemm_i32(a_q, w_q)
    if order is None:
        order = ORDER_SMALL_M if acc.shape[0] <= 32 else ORDER_LARGE_M
    return epilogue(acc, sa, sw, bias, dtype, order), acc
