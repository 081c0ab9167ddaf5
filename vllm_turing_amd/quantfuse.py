"""Dynamic per-token int8 quantization of W8A8 activations, on the MI355X HIP kernel.

The counterpart of vllm_turing/quantfuse.py.  The reference replaces vllm._custom_ops.scaled_int8_quant so that,
while torch.compile traces, the dynamic symmetric case becomes torch ops that inductor fuses into the producer's
Triton kernel; eager calls keep vLLM's CUDA op (quantfuse.py:35-39).  This build has no Triton path: the dynamic
symmetric case always runs the HIP kernel per_token_quant through the opaque custom op
vllm_turing_amd::per_token_quant_ (eager, compiled and graph-captured alike), with the CUDA op's arithmetic:
  scale = absmax / 127, q = clamp(rint(x * (127 / absmax)), -128, 127), and q = 0, scale = 0 for an all-zero row
(float32 absmax of the row; IEEE division).  Fusion into the producers is done by dedicated HIP kernels instead
(silu_mul_quant for the MLP activation).

quant_torch() is the reference's torch formula (quantfuse.py:18-24), kept for API parity.  Note that torch evaluates
its `127.0 / absmax` as reciprocal(absmax) * 127, so it differs from the CUDA op (and from this kernel) in the last
bit of the inverse for some rows: the reference's own test tolerates that (tests/test_quantfuse.py:152).
"""
import os

import torch

from . import _lib, hooks

ENABLED = os.environ.get("VLLM_TURING_QUANTFUSE", "1") != "0"


def quant_torch(x: torch.Tensor):
    """Per-row dynamic symmetric int8 quantization with torch ops: (int8 like x, float32 scales [rows, 1])."""
    shape = x.shape
    xf = x.reshape(-1, shape[-1]).float()
    absmax = xf.abs().amax(dim=-1, keepdim=True)
    q = torch.round(xf * (127.0 / absmax)).clamp(-128.0, 127.0).to(torch.int8)
    return q.reshape(shape), absmax / 127.0


_qlib = torch.library.Library("vllm_turing_amd", "FRAGMENT")
_qlib.define("per_token_quant_(Tensor(a!) q, Tensor(b!) scales, Tensor x) -> ()")


def _per_token_quant_hip(q, scales, x):
    M, K = x.shape
    if M == 0:
        return
    rc = _lib.lib().per_token_quant(x.data_ptr(), q.data_ptr(), scales.data_ptr(), M, K, x.stride(0),
                                    _lib.dtype_code(x.dtype), _lib.stream_handle(x.device))
    if rc != 0:
        raise RuntimeError(f"per_token_quant failed: {rc}")


torch.library.impl(_qlib, "per_token_quant_", "CUDA")(_per_token_quant_hip)


@torch.library.register_fake("vllm_turing_amd::per_token_quant_")
def _per_token_quant_fake(q, scales, x):
    return None


def per_token_quant(x: torch.Tensor):
    """x fp16/bf16 [..., K] -> (q int8 [..., K], scales float32 [rows, 1])."""
    shape = x.shape
    x2 = x.reshape(-1, shape[-1])
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    q = torch.empty(x2.shape, dtype=torch.int8, device=x.device)
    s = torch.empty((x2.shape[0], 1), dtype=torch.float32, device=x.device)
    torch.ops.vllm_turing_amd.per_token_quant_(q, s, x2)
    return q.reshape(shape), s


def scaled_int8_quant(input, scale=None, azp=None, symmetric=True):
    """vllm._custom_ops.scaled_int8_quant's signature -> (q, scale [rows, 1], azp).  The dynamic symmetric case (the
    W8A8 path) runs the HIP kernel; static or asymmetric quantization is not part of this path."""
    if scale is None and azp is None and symmetric:
        q, s = per_token_quant(input)
        return q, s, None
    raise NotImplementedError("only dynamic symmetric per-token quantization is implemented (the W8A8 path)")


def install():
    """Route vllm._custom_ops.scaled_int8_quant's dynamic symmetric case to the HIP kernel (other cases keep vLLM's
    op) when vLLM is importable on a gfx950 device.  The reference takes over that case only while torch.compile
    traces, so that inductor fuses its torch formula into the producer (vllm_turing/quantfuse.py:27-43); without a
    Triton path here, eager and compiled calls alike run the kernel through the opaque op.  As there, the compile cache
    key is extended so a graph traced without the hook is not reused with it (quantfuse.py:45-55)."""
    if not ENABLED:
        return False
    try:
        from vllm import _custom_ops as ops
    except ImportError:
        return False
    if not hooks.on_gfx950():
        return False
    vllm_op = ops.scaled_int8_quant
    if hooks.ours(vllm_op):
        return True

    def scaled_int8_quant_hook(input, scale=None, azp=None, symmetric=True):
        if scale is None and azp is None and symmetric:
            q, s = per_token_quant(input)
            return q, s, None
        return vllm_op(input, scale, azp, symmetric)

    hooks.replace(ops, "scaled_int8_quant", scaled_int8_quant_hook)
    _extend_compile_cache_key()
    return True


def _extend_compile_cache_key():
    try:
        from vllm.compilation import caching
    except ImportError:
        return
    factors = getattr(caching, "aot_compile_hash_factors", None)
    if factors is None or hooks.ours(factors):
        return

    def aot_compile_hash_factors(vllm_config):
        return [*factors(vllm_config), "vllm_turing_amd.per_token_quant"]

    hooks.replace(caching, "aot_compile_hash_factors", aot_compile_hash_factors)
