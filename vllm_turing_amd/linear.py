"""A W8A8 linear layer with vLLM's compressed-tensors int8 apply() contract, on the MI355X kernels.

vLLM's W8A8 int8 linear method (third-party, the caller of the reference's hooks; its signature is visible at
vllm_turing/tailoverlap.py:92-95) quantizes the input per token with scaled_int8_quant and multiplies with
cutlass_scaled_mm.  W8A8LinearMethod.apply(layer, x, bias) does the same with this package's kernels, so the hooks are
usable without vLLM.  The layer holds the checkpoint tensors as vLLM presents them (scripts/w8a8_convert.py:165-178):
weight int8 [N, K] (exposed to the matmul as its [K, N] stride-(1, K) view) and weight_scale float32 [N, 1].
"""
import torch

from .quantfuse import scaled_int8_quant
from .w8a8 import cutlass_scaled_mm, gemv_quant, gemv_quant_ok


class W8A8LinearMethod:
    """apply(layer, x, bias): per-token int8 quantization of x, int8 GEMM / GEMV, scale epilogue (+ bias).  At decode
    row counts (the GEMV range) the quantization runs inside the GEMV (one launch, the same bits)."""

    @staticmethod
    def apply(layer, x, bias=None):
        x2 = x.reshape(-1, x.shape[-1])
        if gemv_quant_ok(x2, layer.weight, layer.weight_scale, bias):
            return gemv_quant(x2, layer.weight, layer.weight_scale, bias).view(*x.shape[:-1], layer.weight.shape[0])
        x_q, x_s, _ = scaled_int8_quant(x)
        return cutlass_scaled_mm(x_q, layer.weight.t(), x_s, layer.weight_scale, x.dtype, bias)


class W8A8Linear(torch.nn.Module):
    """int8 weight [N, K] + float32 per-output-channel scale [N, 1] (+ optional bias [N])."""

    def __init__(self, weight: torch.Tensor, weight_scale: torch.Tensor, bias: torch.Tensor = None):
        super().__init__()
        if weight.dtype != torch.int8 or weight.dim() != 2:
            raise ValueError("weight must be int8 [N, K]")
        self.register_buffer("weight", weight.contiguous())
        self.register_buffer("weight_scale", weight_scale.to(torch.float32).reshape(-1, 1).contiguous())
        self.register_buffer("bias", bias)
        self.quant_method = W8A8LinearMethod()

    def forward(self, x):
        return self.quant_method.apply(self, x, self.bias)
