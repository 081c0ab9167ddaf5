"""The allocation-free entry point w8a8_scaled_mm_noalloc (the library's per-GPU scratch in place of a workspace)
against w8a8_scaled_mm_ws with a workspace of its own: the same 16-bit outputs and int32 accumulators bit for bit, on
three calls in a row, each smaller than the one before, and the tile counters of the workspace left at zero by all."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module")
def L():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from vllm_turing_amd import _lib
    return _lib.lib()


def bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def test_noalloc_matches_workspace_entry(L):
    st = torch.cuda.current_stream().cuda_stream
    g = torch.Generator().manual_seed(11)
    # four calls in a row, each with a smaller input; all split over K (M=4096, N=5120, K=17408: 256 whole tiles
    # + 64 x 4 pieces, every slot of the scratch; M=40: 297 64 x 64 tiles x 2 pieces, 82 of them uneven; M=64: 256
    # 64 x 64 tiles x 2 pieces; M=512: 96 x 2 pieces)
    for M, N, K in ((4096, 5120, 17408), (40, 19000, 5136), (64, 16384, 5120), (512, 12288, 5120)):
        print(f"noalloc M={M} N={N} K={K}", flush=True)
        need = L.w8a8_scaled_mm_ws_size(M, N, K)
        assert need > 4096
        a = torch.randint(-128, 128, (M, K), dtype=torch.int8, generator=g).to(DEV)
        w = torch.randint(-128, 128, (N, K), dtype=torch.int8, generator=g).to(DEV)
        sa = (torch.rand(M, generator=g) * 1e-2).to(DEV)
        sw = (torch.rand(N, generator=g) * 1e-3).to(DEV)
        bias = torch.randn(N, generator=g).to(torch.bfloat16).to(DEV)
        ws = torch.zeros(need, dtype=torch.uint8, device=DEV)
        args = (a.data_ptr(), w.data_ptr(), sa.data_ptr(), sw.data_ptr(), bias.data_ptr())
        got = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
        want = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
        assert L.w8a8_scaled_mm_noalloc(*args, got.data_ptr(), M, N, K, 1, 1, 1, st) == 0
        assert L.w8a8_scaled_mm_ws(*args, want.data_ptr(), M, N, K, 1, 1, 1, ws.data_ptr(), need, st) == 0
        acc = torch.empty(M, N, dtype=torch.int32, device=DEV)
        acc_want = torch.empty(M, N, dtype=torch.int32, device=DEV)
        assert L.w8a8_scaled_mm_noalloc(a.data_ptr(), w.data_ptr(), None, None, None, acc.data_ptr(), M, N, K, 0, 0, 2,
                                        st) == 0
        assert L.w8a8_scaled_mm_ws(a.data_ptr(), w.data_ptr(), None, None, None, acc_want.data_ptr(), M, N, K, 0, 0, 2,
                                   ws.data_ptr(), need, st) == 0
        torch.cuda.synchronize()
        assert np.array_equal(bits(got), bits(want)), f"{int((bits(got) != bits(want)).sum())} outputs differ"
        assert torch.equal(acc.cpu(), acc_want.cpu())
        assert torch.equal(acc.cpu(), torch._int_mm(a.cpu(), w.cpu().t()))
        assert int(ws[:4096].count_nonzero()) == 0
