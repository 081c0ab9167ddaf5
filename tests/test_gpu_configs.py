"""The benchmark configurations at full size, every output checked: prefill GEMM at M = 512, 2048, 4096 (K = 5120,
N = 12288, bias, bf16), the MLP chain at M = 4096 (residual add + RMSNorm + quant -> gate_up N = 34816 -> SiLU*up +
quant -> down N = 5120 over K = 17408), every distinct projection shape of the 64-layer stack at M = 1, 4 and 4096, and
one whole 64-layer pass at M = 4.

The GPU runs through the package's custom ops (which call the C ABI); the CPU side is the oracle: exact int32 products
(torch._int_mm, pinned equal to the C oracle's gemm in test_oracle_pins.py) and the C restatements of the epilogue,
the quantizations, RMSNorm and SiLU.  Integer results, scales and every 16-bit output are compared bit for bit.
The int32 accumulators of the prefill kernel are also read raw through the w8a8_i32 test export and compared whole,
as the reference's own test compares its GEMM's outputs whole (tests/test_w8a8_big.py:34-54).
"""
import numpy as np
import pytest
import torch

import oracle
from oracle import cpu_path

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module")
def L(oracle_lib):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from vllm_turing_amd import _lib
    return _lib.lib()


def bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def say(msg):
    print(msg, flush=True)


def ndiff(a, b):
    return int((np.asarray(a) != np.asarray(b)).sum())


@pytest.mark.parametrize("M", [512, 2048, 4096])
def test_prefill_config_full(L, M):
    """Prefill GEMM K = 5120, N = 12288 with bias, bf16 out (the large-M bias chain): the per-token quant, the whole
    int32 result and the whole bf16 output bit-exact."""
    say(f"prefill config M={M} (full output)")
    from vllm_turing_amd import workloads, per_token_quant, cutlass_scaled_mm
    c = workloads.prefill(M)
    x_q, x_s = per_token_quant(c["x"].to(DEV))
    wd = c["w"].to(DEV)
    N, K = wd.shape
    out = cutlass_scaled_mm(x_q, wd.t(), x_s, c["sw"].to(DEV), torch.bfloat16, c["bias"].to(DEV))
    acc = torch.empty(M, N, dtype=torch.int32, device=DEV)
    assert L.w8a8_i32(x_q.data_ptr(), wd.data_ptr(), acc.data_ptr(), M, N, K, 1,
                      torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    qr, sr = oracle.quant_rows(c["x"])
    assert np.array_equal(x_q.cpu().numpy(), qr) and np.array_equal(x_s.cpu().view(-1).numpy(), sr)
    acc_ref = torch._int_mm(torch.from_numpy(qr), c["w"].t())
    got_acc = acc.cpu()
    assert torch.equal(got_acc, acc_ref), f"{int((got_acc != acc_ref).sum())} of {acc_ref.numel()} int32 differ"
    ref = oracle.epilogue(acc_ref.numpy(), sr, c["sw"].numpy(), bits(c["bias"]), oracle.BF16, oracle.ORDER_LARGE_M)
    got = bits(out)
    assert np.array_equal(got, ref), f"{ndiff(got, ref)} of {ref.size} outputs differ"


def test_mlp_chain_config_full(L):
    """The MLP tail at M = 4096 with its real launch plan (256 x 256 tiles over several rounds, quarter tiles for the
    remainder of the down projection, the SiLU table kernel): every intermediate in full, bit-exact."""
    say("mlp chain M=4096 (full output)")
    from vllm_turing_amd import workloads, rms_norm_dynamic_per_token_quant, cutlass_scaled_mm, silu_mul_quant
    from vllm_turing_amd.normquant import gemma_weight
    M, H, I = 4096, workloads.HIDDEN, workloads.INTERMEDIATE
    c = workloads.mlp(M)
    g = torch.Generator().manual_seed(9)
    res = (torch.randn(M, H, generator=g) * 0.5).to(torch.bfloat16)
    w1 = gemma_weight((torch.randn(H, generator=g) * 0.1).to(torch.bfloat16))
    res_d = res.to(DEV)
    wgu, wd = c["w_gate_up"].to(DEV), c["w_down"].to(DEV)
    sgu, sd = c["sw_gate_up"].to(DEV), c["sw_down"].to(DEV)
    x_q, x_s = rms_norm_dynamic_per_token_quant(c["x"].to(DEV), w1.to(DEV), 1e-6, torch.int8, None, res_d)
    gu = cutlass_scaled_mm(x_q, wgu.t(), x_s, sgu, torch.bfloat16)
    a_q, a_s = silu_mul_quant(gu)
    out = cutlass_scaled_mm(a_q, wd.t(), a_s, sd, torch.bfloat16)
    torch.cuda.synchronize()

    qr, sr, rr, _ = oracle.rms_norm_quant(c["x"], w1, 1e-6, res)
    assert np.array_equal(bits(res_d), rr), "residual"
    assert np.array_equal(x_q.cpu().numpy(), qr) and np.array_equal(x_s.cpu().view(-1).numpy(), sr), "norm + quant"
    gu_ref, _ = cpu_path.scaled_mm(torch.from_numpy(qr), c["w_gate_up"], torch.from_numpy(sr), c["sw_gate_up"], None,
                                   torch.bfloat16, oracle.ORDER_LARGE_M)
    gu_c = gu.cpu()
    assert torch.equal(gu_c, gu_ref), f"gate_up: {int((gu_c != gu_ref).sum())} of {gu_ref.numel()} differ"
    del gu_c
    aq_r, as_r, _ = oracle.silu_mul_quant(gu_ref)
    assert np.array_equal(a_q.cpu().numpy(), aq_r) and np.array_equal(a_s.cpu().view(-1).numpy(), as_r), "silu+quant"
    o_ref, _ = cpu_path.scaled_mm(torch.from_numpy(aq_r), c["w_down"], torch.from_numpy(as_r), c["sw_down"], None,
                                  torch.bfloat16, oracle.ORDER_LARGE_M)
    o_c = out.cpu()
    assert torch.equal(o_c, o_ref), f"down: {int((o_c != o_ref).sum())} of {o_ref.numel()} differ"


def _stack_shape_ids():
    from vllm_turing_amd import workloads
    return sorted({(N, K) for (_, _, N, K) in workloads.stack_shapes()})


@pytest.mark.parametrize("M", [1, 4, 4096])
def test_stack_shapes(L, M):
    """Every distinct projection shape of the 64-layer stack (in_proj_qkvz, out_proj / o_proj, qkv, gate_up, down at
    TP1) at M = 1, 4, 4096: per-token quant of bf16 activations and the scaled matmul through the dispatch, whole
    outputs bit-exact (the small-M epilogue at M <= 32, the large-M one above)."""
    from vllm_turing_amd import per_token_quant, cutlass_scaled_mm
    for (N, K) in _stack_shape_ids():
        say(f"stack shape M={M} N={N} K={K}")
        g = torch.Generator().manual_seed(N + K + M)
        x = torch.randn(M, K, generator=g).to(torch.bfloat16)
        w = torch.randint(-127, 128, (N, K), dtype=torch.int8, generator=g)
        sw = torch.rand(N, 1, generator=g) * 9e-3 + 1e-3
        x_q, x_s = per_token_quant(x.to(DEV))
        out = cutlass_scaled_mm(x_q, w.to(DEV).t(), x_s, sw.to(DEV), torch.bfloat16)
        torch.cuda.synchronize()
        qr, sr = oracle.quant_rows(x)
        assert np.array_equal(x_q.cpu().numpy(), qr) and np.array_equal(x_s.cpu().view(-1).numpy(), sr)
        ref, _ = cpu_path.scaled_mm(torch.from_numpy(qr), w, torch.from_numpy(sr), sw, None, torch.bfloat16)
        got = out.cpu()
        assert torch.equal(got, ref), f"N={N} K={K}: {int((got != ref).sum())} of {ref.numel()} differ"


def test_stack_pass_m4(L):
    """One whole pass of the 64-layer stack at M = 4 (24.33 G int8 weights, random per layer), every layer as the
    stack benchmark runs it: residual add + RMSNorm + quant -> mixer in-projection -> out-projection of the mixer
    output with its quantization fused into the GEMV (w8a8_gemv_quant) -> residual add + RMSNorm + quant -> gate_up ->
    SiLU*up + quant -> down.  The mixer core is not on
    the path: its output is stood in for by the first 6144 columns of the in-projection (a strided view, so the
    per-token quant reads rows with a stride), which keeps every layer dependent on the previous one.  The final
    hidden state and residual stream are compared bit for bit with the same pass on the CPU."""
    say("stack pass M=4, 64 layers")
    from vllm_turing_amd import workloads, rms_norm_dynamic_per_token_quant, cutlass_scaled_mm, silu_mul_quant
    from vllm_turing_amd.w8a8 import gemv_quant
    M, H, I = 4, workloads.HIDDEN, workloads.INTERMEDIATE
    shapes = workloads.stack_shapes()
    gdev = torch.Generator(device=DEV).manual_seed(7)
    weights = []
    for (_, _, N, K) in shapes:
        w = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=DEV, generator=gdev)
        sw = (torch.rand(N, 1, device=DEV, generator=gdev) * 9e-3 + 1e-3)
        weights.append((w, sw))
    g = torch.Generator().manual_seed(11)
    h0 = torch.randn(M, H, generator=g).to(torch.bfloat16)
    r0 = torch.randn(M, H, generator=g).to(torch.bfloat16)
    norms = [(1.0 + 0.1 * torch.randn(H, generator=g)).to(torch.bfloat16) for _ in range(2 * 64)]
    core = 6144

    # GPU pass
    h, r = h0.to(DEV), r0.to(DEV)
    norms_d = [w.to(DEV) for w in norms]
    for li in range(64):
        (w_in, s_in), (w_out, s_out), (w_gu, s_gu), (w_dn, s_dn) = weights[4 * li:4 * li + 4]
        q, s = rms_norm_dynamic_per_token_quant(h, norms_d[2 * li], 1e-6, torch.int8, None, r)
        y = cutlass_scaled_mm(q, w_in.t(), s, s_in, torch.bfloat16)
        h = gemv_quant(y[:, :core], w_out, s_out)       # quantization inside the decode GEMV (strided rows)
        q, s = rms_norm_dynamic_per_token_quant(h, norms_d[2 * li + 1], 1e-6, torch.int8, None, r)
        gu = cutlass_scaled_mm(q, w_gu.t(), s, s_gu, torch.bfloat16)
        q, s = silu_mul_quant(gu)
        h = cutlass_scaled_mm(q, w_dn.t(), s, s_dn, torch.bfloat16)
    torch.cuda.synchronize()
    h_gpu, r_gpu = h.cpu(), r.cpu()
    assert torch.isfinite(h_gpu.float()).all() and torch.isfinite(r_gpu.float()).all()

    # CPU pass (the oracle), the same weights copied layer by layer
    def lin(qn, sn, w, sw):
        out, _ = cpu_path.scaled_mm(torch.from_numpy(qn), w.cpu(), torch.from_numpy(sn), sw.cpu(), None,
                                    torch.bfloat16, oracle.ORDER_SMALL_M)
        return out

    hc, rc = h0.clone(), r0.clone()
    for li in range(64):
        (w_in, s_in), (w_out, s_out), (w_gu, s_gu), (w_dn, s_dn) = weights[4 * li:4 * li + 4]
        qn, sn, rb, _ = oracle.rms_norm_quant(hc, norms[2 * li], 1e-6, rc)
        rc = torch.from_numpy(rb.view(np.int16)).view(torch.bfloat16).reshape(M, H)
        y = lin(qn, sn, w_in, s_in)
        qn, sn = oracle.quant_rows(y[:, :core].contiguous())
        hc = lin(qn, sn, w_out, s_out)
        qn, sn, rb, _ = oracle.rms_norm_quant(hc, norms[2 * li + 1], 1e-6, rc)
        rc = torch.from_numpy(rb.view(np.int16)).view(torch.bfloat16).reshape(M, H)
        gu = lin(qn, sn, w_gu, s_gu)
        qn, sn, _ = oracle.silu_mul_quant(gu)
        hc = lin(qn, sn, w_dn, s_dn)
    del weights
    torch.cuda.empty_cache()
    assert torch.equal(r_gpu, rc), f"residual stream: {int((r_gpu != rc).sum())} of {rc.numel()} differ"
    assert torch.equal(h_gpu, hc), f"hidden state: {int((h_gpu != hc).sum())} of {hc.numel()} differ"


# ---------------------------------------------------------------------------------------------------------------------
# the reference's own test grids (tests/test_w8a8.py:11-12,30 and tests/test_w8a8_big.py:14-15,34), every output
# against the oracle instead of vLLM's CUTLASS op
# ---------------------------------------------------------------------------------------------------------------------
def int_mm(a, w):
    """Exact int32 a [M, K] x w [N, K]^T on the CPU (torch._int_mm, rows padded to 32 for its small-M limit)."""
    M = a.shape[0]
    if M >= 32:
        return torch._int_mm(a, w.t().contiguous())
    ap = torch.zeros(32, a.shape[1], dtype=torch.int8)
    ap[:M] = a
    return torch._int_mm(ap, w.t().contiguous())[:M]


SMALL_M_SHAPES = [(8192, 5120), (5120, 3072), (7168, 5120), (17408, 5120), (5120, 8704)]   # TP2 (o_proj = out_proj)


@pytest.mark.parametrize("N,K", SMALL_M_SHAPES)
def test_reference_small_m_grid(L, N, K):
    """tests/test_w8a8.py's grid: M in {1, 3, 4, 5, 6, 8, 10, 14, 16} at the TP2 shapes, a and W uniform in [-128,
    128), sa = rand * 1e-2, sb = rand * 1e-3, fp16 out through the dispatch (the GEMV / MMA small-M chain)."""
    from vllm_turing_amd import cutlass_scaled_mm
    g = torch.Generator().manual_seed(N + K)
    w = torch.randint(-128, 128, (N, K), dtype=torch.int8, generator=g)
    sb = torch.rand(N, 1, generator=g) * 1e-3
    wd, sbd = w.to(DEV), sb.to(DEV)
    for M in (1, 3, 4, 5, 6, 8, 10, 14, 16):
        say(f"reference small-M grid N={N} K={K} M={M}")
        a = torch.randint(-128, 128, (M, K), dtype=torch.int8, generator=g)
        sa = torch.rand(M, 1, generator=g) * 1e-2
        out = cutlass_scaled_mm(a.to(DEV), wd.t(), sa.to(DEV), sbd, torch.float16)
        ref = oracle.epilogue(int_mm(a, w).numpy(), sa.numpy(), sb.numpy(), None, oracle.FP16, oracle.ORDER_SMALL_M)
        assert np.array_equal(bits(out), ref), f"M={M}: {ndiff(bits(out), ref)} of {ref.size} differ"


BIG_SHAPES = [(8704, 5120), (5120, 8704), (8192, 5120), (5120, 3072), (3584, 5120)]   # TP2 (o_proj = out_proj)


@pytest.mark.parametrize("M", [1680, 4096, 6720])
def test_reference_big_grid(L, M):
    """tests/test_w8a8_big.py's grid: M in {1680, 4096, 6720} at its TP2 shapes, fp16 and bf16 out, through the
    dispatch's large-M path (w8a8_big's kernels with the K-split workspace); every output bit for bit."""
    from vllm_turing_amd import cutlass_scaled_mm
    g = torch.Generator().manual_seed(M)
    a = torch.randint(-128, 128, (M, 8704), dtype=torch.int8, generator=g)
    sa = torch.rand(M, 1, generator=g) * 1e-2
    ad, sad = a.to(DEV), sa.to(DEV)
    for i, (N, K) in enumerate(BIG_SHAPES):
        dt = torch.float16 if i % 2 == 0 else torch.bfloat16
        say(f"reference big grid M={M} N={N} K={K} {dt}")
        w = torch.randint(-128, 128, (N, K), dtype=torch.int8, generator=g)
        sb = torch.rand(N, 1, generator=g) * 1e-3
        ak = ad[:, :K].contiguous()
        out = cutlass_scaled_mm(ak, w.to(DEV).t(), sad, sb.to(DEV), dt)
        acc = int_mm(a[:, :K].contiguous(), w)
        ref = oracle.epilogue(acc.numpy(), sa.numpy(), sb.numpy(), None,
                              oracle.FP16 if dt == torch.float16 else oracle.BF16, oracle.ORDER_LARGE_M)
        assert np.array_equal(bits(out), ref), f"N={N} K={K}: {ndiff(bits(out), ref)} of {ref.size} differ"
