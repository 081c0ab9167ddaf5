"""The fused MLP activation of the W8A8 path: SiLU(gate) * up with the down projection's per-token int8 quantization,
and the MLP chain that uses it, on MI355X HIP kernels.

The counterpart of the in-scope part of vllm_turing/tailoverlap.py: silu_mul_quant(gate_up) (:57-66) and the
quantized MLP of _Tail.mlp_partial (:138-157): residual add + RMSNorm + int8 quant -> gate_up W8A8 GEMM -> SiLU * up +
int8 requant -> down W8A8 GEMM.  The token chunking, side streams and all-reduce overlap of that module are multi-GPU
and not part of this path.
"""
import torch

from . import _lib, w8a8
from .normquant import rms_norm_dynamic_per_token_quant
from .quantfuse import per_token_quant
from .w8a8 import cutlass_scaled_mm

_flib = torch.library.Library("vllm_turing_amd", "FRAGMENT")
_flib.define("silu_mul_quant_(Tensor(a!) q, Tensor(b!) scales, Tensor gate_up) -> ()")


def _silu_mul_quant_hip(q, scales, gate_up):
    M, I2 = gate_up.shape
    if M == 0:
        return
    fn = _lib.lib().silu_mul_quant if gate_up.dtype == torch.float16 else _lib.lib().silu_mul_quant_bf16
    rc = fn(gate_up.data_ptr(), q.data_ptr(), scales.data_ptr(), M, I2 // 2, _lib.stream_handle(gate_up.device))
    if rc != 0:
        raise RuntimeError(f"silu_mul_quant failed: {rc}")


torch.library.impl(_flib, "silu_mul_quant_", "CUDA")(_silu_mul_quant_hip)


@torch.library.register_fake("vllm_turing_amd::silu_mul_quant_")
def _silu_mul_quant_fake(q, scales, gate_up):
    return None


def silu_mul_quant(gate_up: torch.Tensor):
    """(M, 2I) fp16 / bf16 -> int8 (M, I) of SiLU(gate) * up and its per-row scales (M, 1) float32
    (vllm_turing/tailoverlap.py:57-66; bf16 is an addition: the reference kernel is fp16 only)."""
    if gate_up.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError(f"silu_mul_quant takes float16 or bfloat16, got {gate_up.dtype}")
    gate_up = gate_up.contiguous()
    M, I2 = gate_up.shape
    q = torch.empty(M, I2 // 2, dtype=torch.int8, device=gate_up.device)
    sc = torch.empty(M, 1, dtype=torch.float32, device=gate_up.device)
    torch.ops.vllm_turing_amd.silu_mul_quant_(q, sc, gate_up)
    return q, sc


_flib.define("gemv_silu_(Tensor(a!) h, Tensor a, Tensor w, Tensor a_scales, Tensor w_scales) -> ()")


def _gemv_silu_hip(h, a, w, a_scales, w_scales):
    M, K = a.shape
    if M == 0:
        return
    rc = _lib.lib().w8a8_gemv_silu(a.data_ptr(), w.data_ptr(), a_scales.data_ptr(), w_scales.data_ptr(), None,
                                   h.data_ptr(), M, w.shape[0] // 2, K, int(a_scales.numel() > 1),
                                   int(w_scales.numel() > 1), _lib.dtype_code(h.dtype), _lib.stream_handle(a.device))
    if rc != 0:
        raise RuntimeError(f"w8a8_gemv_silu failed: {rc}")


torch.library.impl(_flib, "gemv_silu_", "CUDA")(_gemv_silu_hip)


@torch.library.register_fake("vllm_turing_amd::gemv_silu_")
def _gemv_silu_fake(h, a, w, a_scales, w_scales):
    return None


GEMV_SILU_MAX_M = 5


def gemv_silu_ok(x_q, x_s, w_gate_up, sw_gate_up):
    """Whether w8a8_gemv_silu takes the gate_up projection: the reference would run it on w8a8_gemv (M <= the GEMV
    bound), the VALU GEMV takes M and K (M <= 5; K <= 17408 at one row, 8192 at two or three, 5120 above), and the
    layouts are the GEMV's (int8 [M, K] and [2I, K] contiguous, float32 scales of M or 1 and 2I or 1)."""
    M, K = x_q.shape
    kmax = 17408 if M == 1 else 8192 if M <= 3 else 5120
    N2 = w_gate_up.shape[0]
    return (1 <= M <= min(GEMV_SILU_MAX_M, w8a8.MAX_M) and K % 16 == 0 and K <= kmax and N2 % 2 == 0
            and x_q.dtype == torch.int8 and x_q.is_contiguous() and w_gate_up.dtype == torch.int8
            and w_gate_up.is_contiguous() and w_gate_up.shape[1] == K
            and x_q.data_ptr() % 16 == 0 and w_gate_up.data_ptr() % 16 == 0
            and x_s.dtype == torch.float32 and x_s.is_contiguous() and x_s.numel() in (1, M)
            and sw_gate_up.dtype == torch.float32 and sw_gate_up.is_contiguous() and sw_gate_up.numel() in (1, N2))


def gemv_silu(x_q, x_s, w_gate_up, sw_gate_up, out_dtype):
    """The decode MLP's first half in one launch: int8 x_q [M, K] times the gate_up weight [2I, K] with the GEMV's
    small-M epilogue, then SiLU(gate) * up rounded as silu_mul_quant rounds it before quantizing -> [M, I] in
    out_dtype.  per_token_quant of the result equals silu_mul_quant of the GEMV's output bit for bit."""
    h = torch.empty((x_q.shape[0], w_gate_up.shape[0] // 2), dtype=out_dtype, device=x_q.device)
    torch.ops.vllm_turing_amd.gemv_silu_(h, x_q, w_gate_up, x_s, sw_gate_up)
    return h


def mlp_quantized(x_q, x_s, w_gate_up, sw_gate_up, w_down, sw_down, out_dtype):
    """The quantized MLP of vllm_turing/tailoverlap.py:146-151 from an int8 input:
    gate_up = W8A8(x_q, w_gate_up) -> (a_q, a_s) = silu_mul_quant(gate_up) -> W8A8(a_q, w_down).
    w_* are int8 [N, K] row-major weights, sw_* float32 [N, 1] scales.  At decode row counts the same chain runs as
    two launches with the same bits: gemv_silu (SiLU * up in the gate_up GEMV's epilogue), then gemv_quant (the
    down GEMV quantizing its input itself)."""
    if gemv_silu_ok(x_q, x_s, w_gate_up, sw_gate_up):
        h = gemv_silu(x_q, x_s, w_gate_up, sw_gate_up, out_dtype)
        if w8a8.gemv_quant_ok(h, w_down, sw_down, None):
            return w8a8.gemv_quant(h, w_down, sw_down)
        a_q, a_s = per_token_quant(h)
        return cutlass_scaled_mm(a_q, w_down.t(), a_s, sw_down, out_dtype)
    gate_up = cutlass_scaled_mm(x_q, w_gate_up.t(), x_s, sw_gate_up, out_dtype)
    a_q, a_s = silu_mul_quant(gate_up)
    return cutlass_scaled_mm(a_q, w_down.t(), a_s, sw_down, out_dtype)


def mlp(x, w_gate_up, sw_gate_up, w_down, sw_down):
    """The same chain from a floating-point input (per-token quantization of x first)."""
    x_q, x_s = per_token_quant(x)
    return mlp_quantized(x_q, x_s, w_gate_up, sw_gate_up, w_down, sw_down, x.dtype)


def mlp_tail(h, residual, norm_weight, eps, w_gate_up, sw_gate_up, w_down, sw_down):
    """_Tail.mlp_partial's fused path (tailoverlap.py:138-151): residual += h in place, x_q = int8 RMSNorm(residual)
    (norm_weight as the fused op takes it: 1 + w for GemmaRMSNorm), then the quantized MLP; returns the down
    projection in h's dtype."""
    x_q, x_s = rms_norm_dynamic_per_token_quant(h, norm_weight, eps, torch.int8, None, residual)
    return mlp_quantized(x_q, x_s, w_gate_up, sw_gate_up, w_down, sw_down, h.dtype)
