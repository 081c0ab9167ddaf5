"""vllm_turing_amd: the W8A8 SmoothQuant linear path of cookjohn/vllm-turing, rebuilt for AMD Instinct MI355X.

Hand-written gfx950 HIP kernels (per-token int8 quantization, fused SiLU * up + quantization, a weight-streaming
int8 MFMA GEMV for decode and an LDS-tiled int8 MFMA GEMM for prefill, each with the scale epilogue fused) behind a
C ABI (include/w8a8_mi355.h) loaded with ctypes, and Python hooks with the reference plugin's signatures:
  w8a8.cutlass_scaled_mm / torch.ops.vllm_turing_amd.scaled_mm_   (vllm_turing/w8a8.py)
  quantfuse.scaled_int8_quant / quant_torch                         (vllm_turing/quantfuse.py)
  tailoverlap.silu_mul_quant / mlp_tail                             (vllm_turing/tailoverlap.py)
  normquant.rms_norm_dynamic_per_token_quant                        (vLLM's fused op, tailoverlap.py:145)
  lmhead.w8a16_mm / quantize_rows                                   (vllm_turing/lmhead.py, the int8 LM head)
  ar8.ar8_quant / ar8_dequant_sum                                   (vllm_turing/hostar.py, AR8 operand)
register() mirrors the reference plugin entry point (vllm_turing/__init__.py:38-72): with vLLM importable on a gfx950
device it patches vllm._custom_ops; VLLM_TURING_DISABLE=1 turns it off.  Importing the package builds nothing; the
library is built or loaded on first use.
"""
import logging
import os

logger = logging.getLogger("vllm.turing_amd")
_registered = False

from . import ar8, hooks, lmhead, normquant, quantfuse, w8a8  # noqa: E402,F401  (defines the custom ops)
from .linear import W8A8Linear, W8A8LinearMethod  # noqa: E402,F401
from .normquant import rms_norm_dynamic_per_token_quant  # noqa: E402,F401
from .quantfuse import per_token_quant, quant_torch, scaled_int8_quant  # noqa: E402,F401
from .tailoverlap import mlp, mlp_quantized, mlp_tail, silu_mul_quant  # noqa: E402,F401
from .w8a8 import cutlass_scaled_mm  # noqa: E402,F401


def register():
    """The vLLM plugin entry point (vllm_turing/__init__.py:38-72): install the hooks in the reference's order (the
    fused norm + quant producer in tailoverlap's slot, then quantfuse, w8a8, lmhead), once per process; nothing when
    VLLM_TURING_DISABLE=1.  Returns {hook: installed} for this call ({} when disabled or already registered)."""
    global _registered
    if _registered or os.environ.get("VLLM_TURING_DISABLE", "0") == "1":
        return {}
    _registered = True
    done = {}
    for name, mod in (("normquant", normquant), ("quantfuse", quantfuse), ("w8a8", w8a8), ("lmhead", lmhead)):
        done[name] = bool(mod.install())
    logger.info("vllm_turing_amd hooks: %s (GEMV up to M=%d)",
                ", ".join(f"{k} {'on' if v else 'off'}" for k, v in done.items()), w8a8.MAX_M)
    return done
