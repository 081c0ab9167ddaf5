"""The fused MLP activation of the W8A8 path: SiLU(gate) * up with the down projection's per-token int8 quantization,
and the MLP chain that uses it, on MI355X HIP kernels.

The counterpart of the in-scope part of vllm_turing/tailoverlap.py: silu_mul_quant(gate_up) (:57-66) and the
quantized MLP of _Tail.mlp_partial (:138-157): residual add + RMSNorm + int8 quant -> gate_up W8A8 GEMM -> SiLU * up +
int8 requant -> down W8A8 GEMM.  The token chunking, side streams and all-reduce overlap of that module are multi-GPU
and not part of this path.
"""
import torch

from . import _lib
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


def mlp_quantized(x_q, x_s, w_gate_up, sw_gate_up, w_down, sw_down, out_dtype):
    """The quantized MLP of vllm_turing/tailoverlap.py:146-151 from an int8 input:
    gate_up = W8A8(x_q, w_gate_up) -> (a_q, a_s) = silu_mul_quant(gate_up) -> W8A8(a_q, w_down).
    w_* are int8 [N, K] row-major weights, sw_* float32 [N, 1] scales."""
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
