"""Residual add + RMSNorm + dynamic per-token int8 quantization in one HIP kernel: the other producer of W8A8 inputs.

The reference's MLP tail normalises the residual stream and quantizes it for the gate_up projection with vLLM's fused
op, ops.rms_norm_dynamic_per_token_quant(h, w1, eps, torch.int8, None, res) (vllm_turing/tailoverlap.py:145), with
w1 = 1 + w precomputed in float32 for GemmaRMSNorm (:123).  This module provides that op with vLLM's signature on the
MI355X kernel rms_norm_quant (csrc/quant.hip), through the opaque custom op vllm_turing_amd::rms_norm_quant_, and
install() routes vLLM's int8 case to it when vLLM is importable.

Arithmetic, per row (x and the residual r of one dtype T, fp16 or bf16):
  s = float(x) + float(r); r <- RN_T(s) in place; rms = 1 / sqrt(RN32(sum(s^2) / K) + eps) (the sum in float64);
  y = RN_T(float(RN_T(s * rms)) * float(w)); scale = max(min(absmax(y), scale_ub) / 127, FLT_EPSILON);
  q = clamp(rint(y * (1 / scale)), -128, 127).
vLLM's kernel sums s^2 in float32 in its block-reduction order and uses rsqrtf; those two CUDA-internal details are
the unpinned residue (they move the last float32 bit of rms, hence a 16-bit y only next to a rounding boundary).
"""
import os

import torch

from . import _lib, hooks

ENABLED = os.environ.get("VLLM_TURING_NORMQUANT", "1") != "0"

_nlib = torch.library.Library("vllm_turing_amd", "FRAGMENT")
_nlib.define("rms_norm_quant_(Tensor(a!) q, Tensor(b!) scales, Tensor x, Tensor weight, float epsilon, "
             "Tensor? scale_ub, Tensor(c!)? residual) -> ()")


def _rms_norm_quant_hip(q, scales, x, weight, epsilon, scale_ub, residual):
    M, K = x.shape
    if M == 0:
        return
    rc = _lib.lib().rms_norm_quant(x.data_ptr(), None if residual is None else residual.data_ptr(), weight.data_ptr(),
                                   None if scale_ub is None else scale_ub.data_ptr(), float(epsilon), q.data_ptr(),
                                   scales.data_ptr(), M, K, _lib.dtype_code(x.dtype), _lib.stream_handle(x.device))
    if rc != 0:
        raise RuntimeError(f"rms_norm_quant failed: {rc}")


torch.library.impl(_nlib, "rms_norm_quant_", "CUDA")(_rms_norm_quant_hip)


@torch.library.register_fake("vllm_turing_amd::rms_norm_quant_")
def _rms_norm_quant_fake(q, scales, x, weight, epsilon, scale_ub, residual):
    return None


def rms_norm_dynamic_per_token_quant(input: torch.Tensor, weight: torch.Tensor, epsilon: float,
                                     quant_dtype: torch.dtype = torch.int8, scale_ub=None, residual=None):
    """vllm._custom_ops.rms_norm_dynamic_per_token_quant's signature -> (q [..., K], scales float32 [rows, 1]).

    input, residual: fp16/bf16 [..., K] (residual updated in place to RN(input + residual)); weight: [K] of the same
    dtype; scale_ub: float32 tensor of one element or None.  Only int8 output is part of the W8A8 path."""
    if quant_dtype != torch.int8:
        raise NotImplementedError("only int8 output is implemented (the W8A8 path)")
    if input.dtype not in (torch.float16, torch.bfloat16) or weight.dtype != input.dtype:
        raise ValueError(f"input and weight must share a float16 / bfloat16 dtype, got {input.dtype}, {weight.dtype}")
    shape = input.shape
    K = shape[-1]
    x2 = input.reshape(-1, K).contiguous()
    w = weight.contiguous()
    if w.numel() != K:
        raise ValueError(f"weight has {w.numel()} elements for rows of {K}")
    r2 = None
    if residual is not None:
        if residual.shape != shape or residual.dtype != input.dtype or not residual.is_contiguous():
            raise ValueError("residual must be a contiguous tensor of the input's shape and dtype")
        r2 = residual.view(-1, K)
    ub = None
    if scale_ub is not None:
        ub = scale_ub.reshape(1).to(device=input.device, dtype=torch.float32)
    q = torch.empty(x2.shape, dtype=torch.int8, device=input.device)
    s = torch.empty((x2.shape[0], 1), dtype=torch.float32, device=input.device)
    torch.ops.vllm_turing_amd.rms_norm_quant_(q, s, x2, w, float(epsilon), ub, r2)
    return q.reshape(shape), s


def gemma_weight(w: torch.Tensor) -> torch.Tensor:
    """The GemmaRMSNorm weight the fused op takes: 1 + w in float32, back to w's dtype (tailoverlap.py:123)."""
    return (1.0 + w.float()).to(w.dtype)


def install():
    """Route vllm._custom_ops.rms_norm_dynamic_per_token_quant's int8 case to the HIP kernel (other output types keep
    vLLM's op) when vLLM is importable on a gfx950 device."""
    if not ENABLED:
        return False
    try:
        from vllm import _custom_ops as ops
    except ImportError:
        return False
    vllm_op = getattr(ops, "rms_norm_dynamic_per_token_quant", None)
    if vllm_op is None or not hooks.on_gfx950():
        return False
    if hooks.ours(vllm_op):
        return True

    def rms_norm_dynamic_per_token_quant_hook(input, weight, epsilon, quant_dtype, scale_ub=None, residual=None):
        if quant_dtype == torch.int8:
            return rms_norm_dynamic_per_token_quant(input, weight, epsilon, quant_dtype, scale_ub, residual)
        return vllm_op(input, weight, epsilon, quant_dtype, scale_ub, residual)

    return hooks.replace(ops, "rms_norm_dynamic_per_token_quant", rms_norm_dynamic_per_token_quant_hook)
