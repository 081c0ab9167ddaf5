"""The int8 LM head (W8A16): vLLM's unquantized LM head weight replaced after loading by int8 rows with a float32
scale per row (half the memory of fp16), logits from the MI355X kernel w8a16_gemv (csrc/gemm.hip: w8a16_kernel).

The counterpart of vllm_turing/lmhead.py.  The reference routes up to 4 rows to its GEMV, 5..64 to a tensor-core
kernel, 16-row GEMV passes up to 256 rows and chunked dequantisation above; here one MFMA kernel takes up to 32 rows
per pass and every row count runs in passes of it, so no path leaves the HIP kernel.  VLLM_TURING_LMHEAD=0 disables
install().
"""
import os

import torch

from . import _lib

PASS_ROWS = 32          # rows per kernel launch


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


def _w8a16_mm_hip(x, w, s, bias):
    M, K = x.shape
    N = w.shape[0]
    if x.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError(f"w8a16_mm takes float16 / bfloat16 activations, got {x.dtype}")
    x = x.contiguous()
    out = torch.empty(M, N, dtype=x.dtype, device=x.device)
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
        rc = L.w8a16_gemv_rows(x[r0:r1].data_ptr(), w.data_ptr(), s.data_ptr(),
                               bias.data_ptr() if bias is not None else None, out[r0:r1].data_ptr(), r1 - r0, N, K,
                               _lib.dtype_code(x.dtype), rows.data_ptr(), w.shape[0], _lib.stream_handle(x.device))
        if rc != 0:
            raise RuntimeError(f"w8a16_gemv_rows failed: {rc}")
    return out


def install():
    """After weight loading, replace vLLM's ParallelLMHead weight by int8 rows + scales and compute its logits with
    w8a16_mm (vllm_turing/lmhead.py:104-141), when vLLM is importable on a gfx950 device."""
    if os.environ.get("VLLM_TURING_LMHEAD", "1") == "0":
        return False
    try:
        from vllm.model_executor.layers import vocab_parallel_embedding as vpe
    except ImportError:
        return False
    if not torch.cuda.is_available() or "gfx950" not in torch.cuda.get_device_properties(0).gcnArchName:
        return False
    M = vpe.UnquantizedEmbeddingMethod
    if getattr(M, "_vllm_turing_lmhead", False):
        return True
    orig_pw, orig_apply = M.process_weights_after_loading, M.apply

    def process_weights_after_loading(self, layer):
        orig_pw(self, layer)
        if isinstance(layer, vpe.ParallelLMHead) and not hasattr(layer, "turing_w8") and layer.weight.dim() == 2 \
                and layer.weight.is_cuda and layer.weight.shape[1] % 16 == 0:
            w = layer.weight.data
            layer.turing_w8, layer.turing_s = quantize_rows(w)
            layer.weight.data = torch.empty(0, w.shape[1], dtype=w.dtype, device=w.device)   # free the 16-bit head
            del w
            torch.cuda.empty_cache()

    def apply(self, layer, x, bias=None):
        if hasattr(layer, "turing_w8"):
            return w8a16_mm(x, layer.turing_w8, layer.turing_s, bias)
        return orig_apply(self, layer, x, bias)

    M.process_weights_after_loading = process_weights_after_loading
    M.apply = apply
    M._vllm_turing_lmhead = True
    return True
