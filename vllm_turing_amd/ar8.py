"""AR8: int8 with an fp16 scale per 128 values, the compressed operand of the reference's large (prefill) all-reduce
(vllm_turing/hostar.py:40-98 over csrc/host_ar.cu:133-201), on the MI355X kernels ar8_quant / ar8_dequant_sum.

Each rank quantizes its operand (about half the bytes of fp16), the packed blocks are all-gathered, and every rank
sums the dequantised blocks of all ranks in rank order, so the result is identical on every rank.  The collective
itself is the caller's (RCCL all_gather_into_tensor over xGMI on a multi-GPU node): ar8_all_reduce takes it as a
function.  Lossy by design, as in the reference (VLLM_TURING_AR8 gates it there).
"""
import torch

from . import _lib

GROUP = 128


def ar8_ok(t: torch.Tensor) -> bool:
    """The operands AR8 takes (hostar.py:51-52, without the size threshold): contiguous fp16, numel % 128 == 0."""
    return t.dtype == torch.float16 and t.is_contiguous() and t.numel() % GROUP == 0


def packed_bytes(n: int) -> int:
    return n + n // 64


def ar8_quant(t: torch.Tensor, out: torch.Tensor = None) -> torch.Tensor:
    """fp16 tensor (numel % 128 == 0) -> packed uint8 [n + n / 64]: n int8, then n / 128 fp16 scales."""
    if not ar8_ok(t):
        raise ValueError("AR8 takes a contiguous float16 tensor with numel % 128 == 0")
    n = t.numel()
    packed = out if out is not None else torch.empty(packed_bytes(n), dtype=torch.uint8, device=t.device)
    rc = _lib.lib().ar8_quant(t.data_ptr(), packed.data_ptr(), n, _lib.stream_handle(t.device))
    if rc != 0:
        raise RuntimeError(f"ar8_quant failed: {rc}")
    return packed


def ar8_dequant_sum(gathered: torch.Tensor, n: int, ranks: int = 2) -> torch.Tensor:
    """Rank-order sum of `ranks` packed blocks (ranks x (n + n / 64) bytes) -> fp16 [n]."""
    if gathered.dtype != torch.uint8 or gathered.numel() != ranks * packed_bytes(n) or not gathered.is_contiguous():
        raise ValueError("gathered must be contiguous uint8 of ranks * (n + n / 64) bytes")
    out = torch.empty(n, dtype=torch.float16, device=gathered.device)
    rc = _lib.lib().ar8_dequant_sum_ranks(gathered.data_ptr(), out.data_ptr(), n, ranks,
                                          _lib.stream_handle(gathered.device))
    if rc != 0:
        raise RuntimeError(f"ar8_dequant_sum failed: {rc}")
    return out


def ar8_all_reduce(t: torch.Tensor, all_gather, ranks: int) -> torch.Tensor:
    """The compressed all-reduce of hostar.py:73-98: quantize, all_gather(packed) -> ranks packed blocks in rank order
    (e.g. torch.distributed.all_gather_into_tensor into a [ranks * m] buffer), dequantise and sum."""
    packed = ar8_quant(t)
    gathered = all_gather(packed)
    return ar8_dequant_sum(gathered, t.numel(), ranks).view(t.shape)
