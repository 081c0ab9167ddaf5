"""The int8 LM head (W8A16): vLLM's unquantized LM head weight replaced after loading by int8 rows with a float32
scale per row (half the memory of fp16), logits from the MI355X kernel w8a16_gemv (csrc/gemm.hip: w8a16_kernel).

The counterpart of vllm_turing/lmhead.py.  The reference routes up to 4 rows to its GEMV, 5..64 to a tensor-core
kernel, 16-row GEMV passes up to 256 rows and chunked dequantisation above (lmhead.py:71-99).  Here the weight-
streaming kernels take up to 32 rows per pass (the VALU kernel at one or two rows, the MFMA kernel above) and every
row count up to GEMV_MAX_M runs in passes of them; above GEMV_MAX_M rows each pass would re-read the whole head, so,
as the reference does, the head is dequantized DEQUANT_ROWS rows at a time ((w * s) rounded to the activation type)
and multiplied with the library GEMM (the matmul is compute-bound there).  VLLM_TURING_LMHEAD=0 disables install().
"""
import os

import torch

from . import _lib, hooks

PASS_ROWS = 32          # rows per kernel launch
GEMV_MAX_M = 256        # above this many rows: chunked dequantization and a library GEMM (lmhead.py:17,93-99)
DEQUANT_ROWS = 4096     # head rows dequantized per chunk (lmhead.py:93)


@torch.no_grad()
def quantize_rows(w: torch.Tensor, chunk: int = 16384):
    """[N, K] float -> int8 [N, K] and float32 per-row scales [N]: symmetric, scale = max(absmax, 1e-12) / 127,
    q = clamp(round_half_even(w / scale), -128, 127) (vllm_turing/lmhead.py:57-67)."""
    q = torch.empty(w.shape, dtype=torch.int8, device=w.device)
    s = torch.empty(w.shape[0], dtype=torch.float32, device=w.device)
    for i in range(0, w.shape[0], chunk):
        wf = w[i:i + chunk].float()
        sc = wf.abs().amax(dim=1).clamp(min=1e-12) / 127.0
        q[i:i + chunk] = torch.round(wf / sc[:, None]).clamp(-128, 127).to(torch.int8)
        s[i:i + chunk] = sc
    return q, s


_hlib = torch.library.Library("vllm_turing_amd", "FRAGMENT")
_hlib.define("w8a16_mm(Tensor x, Tensor w, Tensor s, Tensor? bias) -> Tensor")


def _dequant_mm(x, w, s, bias, out):
    """Rows above GEMV_MAX_M (vllm_turing/lmhead.py:93-99): out[:, chunk] = x @ RN_T(w[chunk] * s[chunk])^T, then
    out += bias, with the chunk's weights dequantized on the device and the product on the library GEMM."""
    N = w.shape[0]
    for j in range(0, N, DEQUANT_ROWS):
        wd = (w[j:j + DEQUANT_ROWS].float() * s[j:j + DEQUANT_ROWS, None]).to(x.dtype)
        out[:, j:j + DEQUANT_ROWS] = torch.mm(x, wd.t().contiguous())
    if bias is not None:
        out += bias
    return out


def _w8a16_mm_hip(x, w, s, bias):
    M, K = x.shape
    N = w.shape[0]
    if x.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError(f"w8a16_mm takes float16 / bfloat16 activations, got {x.dtype}")
    x = x.contiguous()
    out = torch.empty(M, N, dtype=x.dtype, device=x.device)
    if M > GEMV_MAX_M:
        return _dequant_mm(x, w, s, bias, out)
    L = _lib.lib()
    code = _lib.dtype_code(x.dtype)
    st = _lib.stream_handle(x.device)
    for r0 in range(0, M, PASS_ROWS):
        r1 = min(M, r0 + PASS_ROWS)
        rc = L.w8a16_gemv(x[r0:r1].data_ptr(), w.data_ptr(), s.data_ptr(),
                          bias.data_ptr() if bias is not None else None, out[r0:r1].data_ptr(), r1 - r0, N, K, code, st)
        if rc != 0:
            raise RuntimeError(f"w8a16_gemv failed: {rc}")
    return out


torch.library.impl(_hlib, "w8a16_mm", "CUDA")(_w8a16_mm_hip)


@torch.library.register_fake("vllm_turing_amd::w8a16_mm")
def _w8a16_mm_fake(x, w, s, bias):
    return x.new_empty(x.shape[0], w.shape[0])


def w8a16_mm(x: torch.Tensor, w: torch.Tensor, s: torch.Tensor, bias: torch.Tensor = None) -> torch.Tensor:
    """Logits [..., N] of x [..., K] (fp16 / bf16) with the int8 head w [N, K] and scales s [N] (+ bias [N])."""
    shp = x.shape
    y = torch.ops.vllm_turing_amd.w8a16_mm(x.reshape(-1, shp[-1]), w, s, bias)
    return y.view(*shp[:-1], y.shape[-1])


def w8a16_mm_rows(x: torch.Tensor, w: torch.Tensor, s: torch.Tensor, rows: torch.Tensor, bias: torch.Tensor = None):
    """Logits over the gathered head rows rows [N] (int32; e.g. a pruned draft vocabulary) -> [M, N]."""
    x = x.reshape(-1, x.shape[-1]).contiguous()
    M, K = x.shape
    rows = rows.to(torch.int32).contiguous()
    N = rows.numel()
    out = torch.empty(M, N, dtype=x.dtype, device=x.device)
    L = _lib.lib()
    for r0 in range(0, M, PASS_ROWS):
        r1 = min(M, r0 + PASS_ROWS)
        rc = L.w8a16_gemv_rows_bounded(x[r0:r1].data_ptr(), w.data_ptr(), s.data_ptr(),
                                       bias.data_ptr() if bias is not None else None, out[r0:r1].data_ptr(), r1 - r0,
                                       N, K, _lib.dtype_code(x.dtype), rows.data_ptr(), w.shape[0],
                                       _lib.stream_handle(x.device))
        if rc != 0:
            raise RuntimeError(f"w8a16_gemv_rows_bounded failed: {rc}")
    return out


def kernel_takes(n_rows: int, k: int) -> bool:
    """Whether the weight-streaming kernels take an int8 head of n_rows x k (32-bit byte offsets into it)."""
    return k % 16 == 0 and n_rows * k < 2 ** 31


def _to_int8_head(layer):
    """Swap a loaded head's 16-bit weight for int8 rows + float32 scales (layer.turing_w8 / turing_s), freeing it."""
    w16 = layer.weight.data
    layer.turing_w8, layer.turing_s = quantize_rows(w16)
    layer.weight.data = w16.new_empty(0, w16.shape[1])
    del w16
    torch.cuda.empty_cache()


def install():
    """Give vLLM's unquantized LM head an int8 weight after loading and compute its logits with w8a16_mm, when vLLM
    is importable on a gfx950 device (vllm_turing/lmhead.py:104-141 does this on sm75).  Heads the kernels cannot
    address (N * K >= 2^31) keep their 16-bit weight and vLLM's own apply()."""
    if os.environ.get("VLLM_TURING_LMHEAD", "1") == "0":
        return False
    try:
        from vllm.model_executor.layers import vocab_parallel_embedding as vpe
    except ImportError:
        return False
    if not hooks.on_gfx950():
        return False
    method = vpe.UnquantizedEmbeddingMethod
    vllm_load, vllm_apply = method.process_weights_after_loading, method.apply
    if hooks.ours(vllm_load) and hooks.ours(vllm_apply):
        return True

    def process_weights_after_loading(self, layer):
        vllm_load(self, layer)
        w = layer.weight
        if isinstance(layer, vpe.ParallelLMHead) and not hasattr(layer, "turing_w8") and w.dim() == 2 \
                and w.is_cuda and kernel_takes(*w.shape):
            _to_int8_head(layer)

    def apply(self, layer, x, bias=None):
        if not hasattr(layer, "turing_w8"):
            return vllm_apply(self, layer, x, bias)
        return w8a16_mm(x, layer.turing_w8, layer.turing_s, bias)

    hooks.replace(method, "process_weights_after_loading", process_weights_after_loading)
    return hooks.replace(method, "apply", apply)
