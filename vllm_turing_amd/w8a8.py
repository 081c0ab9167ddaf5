"""W8A8 scaled int8 matmul behind vLLM's cutlass_scaled_mm, on MI355X (gfx950) HIP kernels.

The counterpart of vllm_turing/w8a8.py.  vLLM's W8A8 int8 linear layers call
vllm._custom_ops.cutlass_scaled_mm(a, b, scale_a, scale_b, out_dtype, bias); install() replaces that wrapper with one
that runs the custom op vllm_turing_amd::scaled_mm_ (same arguments as vllm_turing::scaled_mm_, w8a8.py:104-122),
which dispatches at run time on the concrete M (also under torch.compile and HIP graph capture, where the batch size
is concrete):
  * M <= VLLM_TURING_GEMV_MAX_M (default 12)           -> w8a8_gemv   (weight-streaming kernels, small-M epilogue:
    v_dot4 VALU kernel at one or two rows, else the LDS-ring int8 MFMA kernel)
  * M <= VLLM_TURING_MMA_MAX_M (default and maximum 32) -> w8a8_mma    (the MFMA kernel, two 16-row activation tiles
    past 16 rows)
  * M > MMA_MAX_M, no bias, per-row / per-column scales -> w8a8_big's prefill MFMA GEMM (large-M epilogue)
  * anything else                                       -> w8a8_scaled_mm (prefill or streaming kernel with the
    large-M epilogue of vLLM's cutlass_scaled_mm, with bias / per-tensor scales; the reference sends these to vLLM's
    CUTLASS op, w8a8.py:117, or to triton_scaled_mm for non-16-multiple shapes, w8a8.py:141-143)
The last two run through w8a8_scaled_mm_ws with a per-device, per-stream workspace (workspace()), so that a last
partial round of 256 x 256 tiles runs split over K; the results are bit-identical to the entries without it.
The predicates gemv_ok / mma_ok / big_ok keep the reference's layout requirements (w8a8.py:38-46,58-66,78-79).
Operands that fail them are made conforming (contiguous copies, zero padding of K to a multiple of 16) for the
general kernel.  Every path runs a HIP kernel; there is no torch fallback.
"""
import collections
import os

import torch

from . import _lib, hooks

MAX_M = int(os.environ.get("VLLM_TURING_GEMV_MAX_M", "12"))
MMA_MAX_M = min(int(os.environ.get("VLLM_TURING_MMA_MAX_M", "32")), 32)
BIG = os.environ.get("VLLM_TURING_BIG", "1") != "0"
GEMV_KERNEL_MAX_M = 16          # what the w8a8_gemv entry point accepts


def lib():
    return _lib.lib()


def gemv_ok(out, a, b, sa, sb, bias, max_m=None):
    """The small-M kernels' layout requirements (vllm_turing/w8a8.py:38-46)."""
    M, K = a.shape
    lim = MAX_M if max_m is None else max_m
    return (1 <= M <= min(lim, GEMV_KERNEL_MAX_M if max_m is None else 32) and K % 16 == 0
            and a.dtype == torch.int8 and a.is_contiguous()
            and b.dtype == torch.int8 and b.stride(0) == 1 and b.stride(1) == K
            and out.is_contiguous() and out.dtype in (torch.float16, torch.bfloat16)
            and sa.dtype == torch.float32 and sb.dtype == torch.float32
            and sa.numel() in (1, M) and sb.numel() in (1, b.shape[1])
            and sa.is_contiguous() and sb.is_contiguous()
            and (bias is None or (bias.dtype == out.dtype and bias.is_contiguous()))
            and a.data_ptr() % 16 == 0 and b.data_ptr() % 16 == 0)


def mma_ok(out, a, b, sa, sb, bias):
    """vllm_turing/w8a8.py:78-79."""
    return a.shape[0] > MAX_M and gemv_ok(out, a, b, sa, sb, bias, MMA_MAX_M)


def big_ok(out, a, b, sa, sb, bias):
    """The prefill kernel's requirements (vllm_turing/w8a8.py:58-66)."""
    M, K = a.shape
    N = b.shape[1]
    return (BIG and M > MMA_MAX_M and bias is None and K % 16 == 0 and N % 16 == 0 and a.dtype == torch.int8
            and a.is_contiguous() and b.dtype == torch.int8 and b.stride(0) == 1 and b.stride(1) == K
            and out.is_contiguous() and out.dtype in (torch.float16, torch.bfloat16)
            and sa.dtype == torch.float32 and sb.dtype == torch.float32 and sa.numel() == M and sb.numel() == N
            and sa.is_contiguous() and sb.is_contiguous() and a.data_ptr() % 16 == 0 and b.data_ptr() % 16 == 0)


def _ptr(t):
    return t.data_ptr() if t is not None else None


def _check(rc, name):
    if rc != 0:
        raise RuntimeError(f"{name} failed: {rc}")


def gemv(out, a, b, sa, sb, bias):
    M, K = a.shape
    N = b.shape[1]
    _check(lib().w8a8_gemv(a.data_ptr(), b.data_ptr(), sa.data_ptr(), sb.data_ptr(), _ptr(bias), out.data_ptr(),
                           M, N, K, int(sa.numel() > 1), int(sb.numel() > 1), _lib.dtype_code(out.dtype),
                           _lib.stream_handle(a.device)), "w8a8_gemv launch")


def mma(out, a, b, sa, sb, bias):
    M, K = a.shape
    N = b.shape[1]
    _check(lib().w8a8_mma(a.data_ptr(), b.data_ptr(), sa.data_ptr(), sb.data_ptr(), _ptr(bias), out.data_ptr(),
                          M, N, K, int(sa.numel() > 1), int(sb.numel() > 1), _lib.dtype_code(out.dtype),
                          _lib.stream_handle(a.device)), "w8a8_mma launch")


_WS = collections.OrderedDict()
_WS_IN_GRAPHS = set()          # workspaces a captured graph uses: kept for the life of the process
WS_STREAMS = 8                 # workspaces kept besides those (the most recently used streams)


def workspace(M, N, K, device):
    """The K-split workspace w8a8_scaled_mm_ws takes for M x N x K on `device`'s current stream (one per device and
    stream, zeroed once, sized for the largest split plan), or None: when the shape does not split, or when the stream
    has none yet and is capturing a graph (a zero fill recorded there would run only at replay).  Besides those a graph
    has captured, at most WS_STREAMS are kept; dropping one is safe, as torch's allocator hands its memory only to
    later allocations on the same stream, which run behind the work already queued there."""
    need = lib().w8a8_scaled_mm_ws_size(M, N, K)
    if need <= 0:
        return None
    stream = torch.cuda.current_stream(device)
    key = (device.index, stream.cuda_stream)
    ws = _WS.get(key)
    capturing = torch.cuda.is_current_stream_capturing()
    if ws is None or ws.numel() < need:
        if capturing:
            return None
        cus = torch.cuda.get_device_properties(device).multi_processor_count
        ws = torch.zeros(max(need, 4096 + cus * 262144), dtype=torch.uint8, device=device)
        _WS[key] = ws
    if capturing:
        _WS_IN_GRAPHS.add(key)
    _WS.move_to_end(key)
    for k in [k for k in _WS if k not in _WS_IN_GRAPHS][:-WS_STREAMS]:
        del _WS[k]
    return ws


def _scaled_mm_ws(a_ptr, w_ptr, sa, sb, bias, out, M, N, K, device, name):
    """The large-M-epilogue entry, with the K-split workspace where the shape has one."""
    ws = workspace(M, N, K, device)
    args = (a_ptr, w_ptr, sa.data_ptr(), sb.data_ptr(), _ptr(bias), out.data_ptr(), M, N, K, int(sa.numel() > 1),
            int(sb.numel() > 1), _lib.dtype_code(out.dtype))
    if ws is None:
        _check(lib().w8a8_scaled_mm(*args, _lib.stream_handle(device)), name)
    else:
        _check(lib().w8a8_scaled_mm_ws(*args, ws.data_ptr(), ws.numel(), _lib.stream_handle(device)), name)


def big(out, a, b, sa, sb):
    """The prefill path of w8a8_big (vllm_turing/w8a8.py:92-101): the same kernels and large-M epilogue, through the
    workspace entry so that a last partial round of tiles runs split over K."""
    M, K = a.shape
    N = b.shape[1]
    _scaled_mm_ws(a.data_ptr(), b.data_ptr(), sa, sb, None, out, M, N, K, a.device, "w8a8_big")


def general(out, a, b, sa, sb, bias):
    """Any layout: conform the operands, then the large-M-epilogue kernel (the CUTLASS-op semantics)."""
    if out.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError(f"cutlass_scaled_mm output must be float16 or bfloat16, got {out.dtype}")
    M, K = a.shape
    N = b.shape[1]
    a = a.to(torch.int8).contiguous()
    w = b.t().to(torch.int8).contiguous()                         # [N, K] row-major
    if K % 16 != 0:                                               # zero columns add nothing to the dot products
        pad = 16 - K % 16
        a = torch.nn.functional.pad(a, (0, pad))
        w = torch.nn.functional.pad(w, (0, pad))
        K += pad
    if a.data_ptr() % 16:
        a = a.clone()
    if w.data_ptr() % 16:
        w = w.clone()
    sa = sa.to(torch.float32).contiguous().reshape(-1)
    sb = sb.to(torch.float32).contiguous().reshape(-1)
    if sa.numel() not in (1, M) or sb.numel() not in (1, N):
        raise ValueError(f"scale shapes {tuple(sa.shape)} / {tuple(sb.shape)} do not match M={M} N={N}")
    if bias is not None:
        bias = bias.to(out.dtype).contiguous().reshape(-1)
    dst = out if out.is_contiguous() else torch.empty((M, N), dtype=out.dtype, device=out.device)
    _scaled_mm_ws(a.data_ptr(), w.data_ptr(), sa, sb, bias, dst, M, N, K, a.device, "w8a8_scaled_mm launch")
    if dst is not out:
        out.copy_(dst)


_lib_def = torch.library.Library("vllm_turing_amd", "DEF")
_lib_def.define("scaled_mm_(Tensor(a!) out, Tensor a, Tensor b, Tensor a_scales, Tensor b_scales, Tensor? bias) -> ()")


def _scaled_mm_hip(out, a, b, a_scales, b_scales, bias):
    """Run-time dispatch of vllm_turing/w8a8.py:108-117 onto the HIP kernels."""
    if a.shape[0] == 0 or b.shape[1] == 0:
        return
    if gemv_ok(out, a, b, a_scales, b_scales, bias):
        gemv(out, a, b, a_scales, b_scales, bias)
    elif mma_ok(out, a, b, a_scales, b_scales, bias):
        mma(out, a, b, a_scales, b_scales, bias)
    elif big_ok(out, a, b, a_scales, b_scales, bias):
        big(out, a, b, a_scales, b_scales)
    else:
        general(out, a, b, a_scales, b_scales, bias)


torch.library.impl(_lib_def, "scaled_mm_", "CUDA")(_scaled_mm_hip)


@torch.library.register_fake("vllm_turing_amd::scaled_mm_")
def _scaled_mm_fake(out, a, b, a_scales, b_scales, bias):
    return None


_lib_def.define("gemv_quant_(Tensor(a!) out, Tensor(b!) xq, Tensor(c!) xs, Tensor x, Tensor w, Tensor w_scale, "
                "Tensor? bias) -> ()")


def _gemv_quant_hip(out, xq, xs, x, w, w_scale, bias):
    M, K = x.shape
    N = w.shape[0]
    if M == 0 or N == 0:
        return
    _check(lib().w8a8_gemv_quant(x.data_ptr(), x.stride(0), xq.data_ptr(), xs.data_ptr(), w.data_ptr(),
                                 w_scale.data_ptr(), _ptr(bias), out.data_ptr(), M, N, K, int(w_scale.numel() > 1),
                                 _lib.dtype_code(x.dtype), _lib.stream_handle(x.device)), "w8a8_gemv_quant")


torch.library.impl(_lib_def, "gemv_quant_", "CUDA")(_gemv_quant_hip)


@torch.library.register_fake("vllm_turing_amd::gemv_quant_")
def _gemv_quant_fake(out, xq, xs, x, w, w_scale, bias):
    return None


def gemv_quant_ok(x, w, w_scale, bias):
    """Whether gemv_quant takes these operands: 1..MAX_M rows of fp16 / bf16 x with unit column stride, int8 w [N, K]
    contiguous, K % 16 == 0, float32 scales of N or 1 elements, bias of x's dtype."""
    if x.dim() != 2 or w.dim() != 2:
        return False
    M, K = x.shape
    return (1 <= M <= min(MAX_M, GEMV_KERNEL_MAX_M) and K % 16 == 0 and x.dtype in (torch.float16, torch.bfloat16)
            and x.stride(1) == 1 and w.dtype == torch.int8 and w.is_contiguous() and w.shape[1] == K
            and w.data_ptr() % 16 == 0 and w_scale.dtype == torch.float32 and w_scale.is_contiguous()
            and w_scale.numel() in (1, w.shape[0])
            and (bias is None or (bias.dtype == x.dtype and bias.is_contiguous() and bias.numel() == w.shape[0])))


def gemv_quant(x, w, w_scale, bias=None):
    """Decode W8A8 linear from 16-bit activations with the quantization fused into the GEMV: x fp16 / bf16 [M, K]
    (M <= 12), w int8 [N, K], w_scale float32 [N, 1] or [1] -> out [M, N] in x's dtype, bit-identical to
    per_token_quant followed by cutlass_scaled_mm (which runs w8a8_gemv at these M)."""
    M, K = x.shape
    out = torch.empty((M, w.shape[0]), dtype=x.dtype, device=x.device)
    xq = torch.empty((M, K), dtype=torch.int8, device=x.device)
    xs = torch.empty((M, 1), dtype=torch.float32, device=x.device)
    torch.ops.vllm_turing_amd.gemv_quant_(out, xq, xs, x, w, w_scale, bias)
    return out


def cutlass_scaled_mm(a, b, scale_a, scale_b, out_dtype, bias=None):
    """vLLM's cutlass_scaled_mm signature (vllm_turing/w8a8.py:136-147): a int8 [..., K], b int8 [K, N] (the stride-
    (1, K) view of the [N, K] weight), scale_a float32 [M, 1] or [1], scale_b float32 [N, 1] or [1] -> out [..., N]."""
    assert out_dtype is torch.bfloat16 or out_dtype is torch.float16
    assert bias is None or bias.numel() == b.shape[1] and bias.dtype == out_dtype
    target_shape = (*a.shape[:-1], b.shape[1])
    a = a.reshape(-1, a.shape[-1])
    out = torch.empty((a.shape[0], b.shape[1]), dtype=out_dtype, device=a.device)
    torch.ops.vllm_turing_amd.scaled_mm_(out, a, b, scale_a, scale_b, bias)
    return out.view(*target_shape)


def install():
    """Route vllm._custom_ops.cutlass_scaled_mm to cutlass_scaled_mm above when vLLM is importable and the device is
    gfx950 (the reference replaces the same function on sm75, vllm_turing/w8a8.py:125-150)."""
    try:
        from vllm import _custom_ops as ops
    except ImportError:
        return False
    if not hooks.on_gfx950():
        return False
    return hooks.replace(ops, "cutlass_scaled_mm", cutlass_scaled_mm)
