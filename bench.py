#!/usr/bin/env python3
"""Benchmark of the W8A8 linear path on one MI355X.

Headline (the `value`): decode GEMV at M=1, K=5120, N=17408 (int8 weights, per-token activation scale, per-channel
weight scale, fp16 out), in GB/s of algorithmic bytes N*K + M*K + 2*M*N + 4*N + 4*M per launch.  One step is one
GEMV launch.  Five weight copies (445 MB) are rotated so the 256 MB Infinity Cache cannot hold them: the weights
stream from HBM.  Launches are captured in a HIP graph of 20 back-to-back launches and replayed, so the timed region
is GPU work only (HIP events on the launch stream, bracketed by synchronizations).

Also reported:
  decode_other_m: the same weights at M = 2, 4, 8, 16, 32, 64 through the entry the reference dispatches at that M
    (GEMV up to 12 rows, the mid-band MMA up to 32, the large-M GEMM above);
  batched_decode_split: M = 64 / 128 rows against N 12288 x K 5120 and N 5120 x K 17408 through the workspace entry
    (64 x 64 tiles split over K), with the same entry's time without a workspace beside it;
  gemm: prefill GEMM at M=4096, K=5120, N=12288 with bias, bf16 out, five weight copies rotated per launch (the
    weights come from HBM), in TOPS of 2*M*N*K ops (MFMA-bound roofline),
    timed after a 2 s untimed run of it that samples the median gfx clock amd-smi reports (sclk_mhz) and settles
    the clock, with the fraction of the peak scaled to that clock (frac_at_sclk; the 5.0 POP/s peak is quoted at
    2400 MHz);
  quant: per-token quant at M=4096, K=5120, SiLU*up+quant at M=4096, I=17408, and the AR8 all-reduce operand
    (quantize; dequantised sum of 2 and 8 ranks) at 4096 x 5120, in GB/s (HBM-bound);
  lm_head_w8a16: the int8 LM head (W8A16) over a 248,320 x 5120 vocabulary at M = 1, 4, 16, GB/s (HBM-bound);
  cpu_baseline: the reference's CPU path restated (oracle/cpu_path.py: torch CPU int8 matmul + dequant), timed on a
    bounded sample on this host's cores;
  mlp_chain: the fused MLP tail at M=4096 as the reference runs it (residual add + RMSNorm + int8 quant -> gate_up
    GEMM N=34816 K=5120 -> SiLU*up+quant I=17408 -> down GEMM N=5120 K=17408, bf16), each kernel's time and roofline
    fraction and the whole chain;
  stack: the 64-layer linear stack of the 27B hybrid model (48 GDN + 16 attention mixers, 64 MLPs, 24.3 G int8
    weights) at M in {1, 4, 4096}: per layer residual add + RMSNorm + quant -> mixer in-projection -> quant -> mixer
    out-projection -> residual add + RMSNorm + quant -> gate_up -> SiLU*up+quant -> down, bf16, one HIP graph per
    pass (the attention / GDN cores between the projections are not part of the path); time per pass and per token.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--sections headline,mlp,stack]
       python bench.py --traffic     (a short fixed launch sequence for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs:
                                      10 GEMVs, 10 fused-quant GEMVs and 10 weight-stream reads over 5 weight copies,
                                      a 256 MB device copy for calibrating the counters, 3 GEMMs, 3 per-token quants,
                                      3 SiLU*up quants; prints nothing else)
"""
import argparse
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "W8A8 GEMM TOPS @M=4096 + GEMV HBM GB/s @M=1 (1×MI355X, % roofline)"
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
INT8_PEAK_TOPS = 5000.0        # MI355X dense int8 MFMA
SCLK_MAX_MHZ = 2400.0          # the gfx clock that peak is quoted at


def traffic_from_profiles(key):
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE, scaled by the copy-kernel
    calibration), as recorded in profiles/*.md lines `traffic[<key>] = <bytes> bytes/launch`."""
    pdir = os.path.join(ROOT, "profiles")
    if not os.path.isdir(pdir):
        return None
    pat = re.compile(r"traffic\[" + re.escape(key) + r"\]\s*=\s*([0-9.eE+]+)\s*bytes/launch")
    for f in sorted(os.listdir(pdir)):
        if f.endswith((".md", ".txt")):
            m = pat.search(open(os.path.join(pdir, f)).read())
            if m:
                return float(m.group(1))
    return None


def graph_time(torch, launch, n_launch_per_graph, steps, warmup, min_warm_s=0.05):
    """Capture n launches in a HIP graph, replay; return ms per launch over `steps` launches (rounded up to whole
    replays) and the number of launches timed.  The untimed warm-up replays are at least `warmup` launches and at
    least `min_warm_s` seconds of GPU work (after an idle gap such as the capture a GEMM's launches were measured
    slowing from 224 to 266 us and settling at 218 us only after ~100 launches, the power management's transient).
    The timed replays are queued right behind the warm-up ones with no host synchronization between them, so the
    timed region starts on a busy GPU instead of paying the restart after an idle gap (a host synchronization there
    added ~1.5 us per launch to a 20-launch timed region of 14.3 us GEMVs)."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(n_launch_per_graph):          # warm up outside capture (loads the code object)
            launch(i)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(n_launch_per_graph):
            launch(i)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    g.replay()                                       # one replay to size the warm-up
    e1.record()
    torch.cuda.synchronize()
    one_s = max(e0.elapsed_time(e1) * 1e-3, 1e-6)
    reps_w = max(1, warmup // n_launch_per_graph, int(min_warm_s / one_s + 0.999))
    reps = max(1, (steps + n_launch_per_graph - 1) // n_launch_per_graph)
    for _ in range(reps_w):
        g.replay()
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1)
    return ms / (reps * n_launch_per_graph), reps * n_launch_per_graph


def sclk_under_load(torch, launch, seconds=2.0):
    """Median gfx clock in MHz (over the XCDs and the samples) that `amd-smi metric -c` reports while `launch` runs
    back to back for about `seconds` (which it does also without amd-smi); None when amd-smi is absent or its output
    does not parse.  The dense int8 MFMA peak (5.0 POP/s) is quoted at the 2400 MHz maximum; under a sustained GEMM
    the clock sits lower."""
    import shutil
    import subprocess
    import threading
    exe = shutil.which("amd-smi")
    clocks, stop = [], threading.Event()

    def poll():
        while not stop.is_set():
            try:
                r = subprocess.run([exe, "metric", "-g", "0", "-c", "--json"], capture_output=True, text=True,
                                   timeout=20)
                d = json.loads(r.stdout)
                d = d["gpu_data"] if isinstance(d, dict) else d
                for key, c in d[0]["clock"].items():
                    if key.startswith("gfx_") and isinstance(c.get("clk"), dict):
                        v = c["clk"].get("value")
                        if isinstance(v, (int, float)) and v > 0:
                            clocks.append(float(v))
            except (OSError, ValueError, KeyError, IndexError, TypeError, subprocess.SubprocessError):
                return

    th = threading.Thread(target=poll, daemon=True) if exe else None
    t_end = time.time() + seconds
    launch()
    torch.cuda.synchronize()
    if th:
        th.start()
    while time.time() < t_end:
        for _ in range(20):
            launch()
        torch.cuda.synchronize()
    stop.set()
    if th:
        th.join(timeout=30)
    if not clocks:
        return None
    clocks.sort()
    return clocks[len(clocks) // 2]


def host_cpu():
    """(os.cpu_count(), the CPU model name lscpu reports or None) of this host."""
    import subprocess
    model = None
    try:
        r = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20)
        for line in r.stdout.splitlines():
            if line.startswith("Model name:"):
                model = line.split(":", 1)[1].strip()
                break
    except (OSError, subprocess.SubprocessError):
        pass
    return os.cpu_count(), model


def cpu_time(fn, budget_s):
    """Median seconds per call of fn over calls fitting in ~budget_s (at least 3, after one warm-up call)."""
    fn()
    ts = []
    t_end = time.time() + budget_s
    while len(ts) < 3 or (time.time() < t_end and len(ts) < 50):
        t = time.time()
        fn()
        ts.append(time.time() - t)
    ts.sort()
    return ts[len(ts) // 2], len(ts)


def traffic_sequence(torch, L, st, dev):
    """Fixed launches for HBM-traffic counters (FETCH_SIZE / WRITE_SIZE per dispatch)."""
    from vllm_turing_amd import workloads
    K, N, M = workloads.HIDDEN, workloads.INTERMEDIATE, 1
    g = torch.Generator(device=dev).manual_seed(1)
    ws = [torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev, generator=g) for _ in range(5)]
    xq = torch.randint(-127, 128, (M, K), dtype=torch.int8, device=dev, generator=g)
    xs = torch.rand(M, device=dev, generator=g) * 1e-2
    sw = torch.rand(N, device=dev, generator=g) * 1e-2
    out = torch.empty(M, N, dtype=torch.float16, device=dev)
    for i in range(10):
        L.w8a8_gemv(xq.data_ptr(), ws[i % 5].data_ptr(), xs.data_ptr(), sw.data_ptr(), None, out.data_ptr(), M, N, K,
                    1, 1, 0, st())
    x16 = (torch.randn(M, K, device=dev, generator=g) * 3).to(torch.float16)
    for i in range(10):
        L.w8a8_gemv_quant(x16.data_ptr(), K, xq.data_ptr(), xs.data_ptr(), ws[i % 5].data_ptr(), sw.data_ptr(), None,
                          out.data_ptr(), M, N, K, 1, 0, st())
    sink = torch.zeros(64, dtype=torch.int32, device=dev)
    for i in range(10):
        L.hbm_read(ws[i % 5].data_ptr(), N, K, sink.data_ptr(), st())
    torch.cuda.synchronize()
    del ws
    src = torch.ones(256 * 1024 * 1024, dtype=torch.uint8, device=dev)   # calibration: 256 MiB read + write
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    Mg, Ng = 4096, 12288
    a = torch.randint(-127, 128, (Mg, K), dtype=torch.int8, device=dev, generator=g)
    w = torch.randint(-127, 128, (Ng, K), dtype=torch.int8, device=dev, generator=g)
    sa = torch.rand(Mg, device=dev, generator=g) * 1e-2
    swg = torch.rand(Ng, device=dev, generator=g) * 1e-2
    bias = torch.randn(Ng, device=dev, generator=g).to(torch.bfloat16)
    og = torch.empty(Mg, Ng, dtype=torch.bfloat16, device=dev)
    for _ in range(3):
        L.w8a8_scaled_mm(a.data_ptr(), w.data_ptr(), sa.data_ptr(), swg.data_ptr(), bias.data_ptr(), og.data_ptr(), Mg,
                         Ng, K, 1, 1, 1, st())
    x = torch.randn(Mg, K, device=dev, generator=g).to(torch.bfloat16)
    q = torch.empty(Mg, K, dtype=torch.int8, device=dev)
    s = torch.empty(Mg, device=dev)
    for _ in range(3):
        L.per_token_quant(x.data_ptr(), q.data_ptr(), s.data_ptr(), Mg, K, K, 1, st())
    I = workloads.INTERMEDIATE
    gu = torch.randn(Mg, 2 * I, device=dev, generator=g).to(torch.bfloat16)
    qs = torch.empty(Mg, I, dtype=torch.int8, device=dev)
    ss = torch.empty(Mg, device=dev)
    for _ in range(3):
        L.silu_mul_quant_bf16(gu.data_ptr(), qs.data_ptr(), ss.data_ptr(), Mg, I, st())
    torch.cuda.synchronize()


_WS = []


def workspace(torch, dev):
    """The prefill GEMM's K-split workspace (zeroed once; every call leaves its counters zero), sized for any shape:
    4 KB of tile counters + 256 KB per CU, as the package's layers hold one per device and stream."""
    if not _WS:
        cus = torch.cuda.get_device_properties(dev).multi_processor_count
        _WS.append(torch.zeros(4096 + cus * 262144, dtype=torch.uint8, device=dev))
    return _WS[0]


def scaled_mm_ws(L, st, a_q, w, a_s, sw, bias, out, M, N, K, dtype_code):
    """The large-M W8A8 GEMM as the package runs it: w8a8_scaled_mm_ws with the workspace (the whole rounds of super
    tiles, then the last partial round split over K; 64-row tiles split over K where they fit two per CU)."""
    ws = _WS[0]
    return L.w8a8_scaled_mm_ws(a_q.data_ptr(), w.data_ptr(), a_s.data_ptr(), sw.data_ptr(),
                               None if bias is None else bias.data_ptr(), out.data_ptr(), M, N, K, 1, 1, dtype_code,
                               ws.data_ptr(), ws.numel(), st())


def linear_launch(L, st, a_q, a_s, w, sw, out, M, N, K, dtype_code):
    """One W8A8 projection through the entry point the reference's dispatch picks for M (no bias): the streaming
    GEMV for M <= 12, the MMA variant for M <= 32, the prefill GEMM above (w8a8_big's kernels, through the workspace
    entry as the package's layers call them)."""
    args = (a_q.data_ptr(), w.data_ptr(), a_s.data_ptr(), sw.data_ptr())
    if M <= 12:
        rc = L.w8a8_gemv(*args, None, out.data_ptr(), M, N, K, 1, 1, dtype_code, st())
    elif M <= 32:
        rc = L.w8a8_mma(*args, None, out.data_ptr(), M, N, K, 1, 1, dtype_code, st())
    else:
        rc = scaled_mm_ws(L, st, a_q, w, a_s, sw, None, out, M, N, K, dtype_code)
    if rc != 0:
        raise RuntimeError(f"W8A8 linear M={M} N={N} K={K}: {rc}")


def bench_mlp(torch, L, st, dev):
    """Fused MLP tail at M=4096, bf16: each kernel timed alone (HIP graph of launches) and the chain as a whole."""
    from vllm_turing_amd import workloads
    M, H, I = 4096, workloads.HIDDEN, workloads.INTERMEDIATE
    c = workloads.mlp(M)
    g = torch.Generator().manual_seed(9)
    x = c["x"].to(dev)
    res = (torch.randn(M, H, generator=g) * 0.5).to(torch.bfloat16).to(dev)
    nw = (1.0 + torch.randn(H, generator=g) * 0.1).to(torch.bfloat16).to(dev)
    # three copies of each weight, rotated per launch (gate_up 3 x 178 MB, down 3 x 89 MB): every launch reads its
    # weights from HBM, as a layer stack does, instead of from the 256 MB MALL
    copies = 3
    gw = torch.Generator(device=dev).manual_seed(31)
    wgus = [c["w_gate_up"].to(dev)] + [torch.randint(-127, 128, (2 * I, H), dtype=torch.int8, device=dev, generator=gw)
                                       for _ in range(copies - 1)]
    wds = [c["w_down"].to(dev)] + [torch.randint(-127, 128, (H, I), dtype=torch.int8, device=dev, generator=gw)
                                   for _ in range(copies - 1)]
    swgu, swd = c["sw_gate_up"].to(dev), c["sw_down"].to(dev)
    x_q = torch.empty(M, H, dtype=torch.int8, device=dev)
    x_s = torch.empty(M, dtype=torch.float32, device=dev)
    gu = torch.empty(M, 2 * I, dtype=torch.bfloat16, device=dev)
    a_q = torch.empty(M, I, dtype=torch.int8, device=dev)
    a_s = torch.empty(M, dtype=torch.float32, device=dev)
    out = torch.empty(M, H, dtype=torch.bfloat16, device=dev)

    def norm_quant(i=0):
        # residual += x in place each call: the values drift, the work per call does not
        if L.rms_norm_quant(x.data_ptr(), res.data_ptr(), nw.data_ptr(), None, 1e-6, x_q.data_ptr(), x_s.data_ptr(),
                            M, H, 1, st()) != 0:
            raise RuntimeError("rms_norm_quant")

    def gate_up(i=0):
        linear_launch(L, st, x_q, x_s, wgus[i % copies], swgu, gu, M, 2 * I, H, 1)

    def silu(i=0):
        if L.silu_mul_quant_bf16(gu.data_ptr(), a_q.data_ptr(), a_s.data_ptr(), M, I, st()) != 0:
            raise RuntimeError("silu_mul_quant_bf16")

    def down(i=0):
        linear_launch(L, st, a_q, a_s, wds[i % copies], swd, out, M, H, I, 1)

    def chain(i=0):
        norm_quant(i); gate_up(i); silu(i); down(i)

    res_d = {"workload": f"MLP tail M={M} as tailoverlap.py:145-151 runs it: residual add + RMSNorm + int8 quant "
                         f"[{M},{H}] -> gate_up N={2 * I} K={H} -> SiLU*up+quant I={I} -> down N={H} K={I}, bf16, "
                         f"SmoothQuant-scaled N(0,1) activations with 0.5% outliers, {copies} weight copies "
                         f"rotated per launch ({copies * 3 * I * H / 1e6:.0f} MB > 256 MB MALL)"}
    # about 1 s of untimed chains first: the clock settles under the GEMMs' load (their first ~20 ms after
    # memory-bound work run ~7% slower)
    t_end = time.time() + 1.0
    while time.time() < t_end:
        chain()
        torch.cuda.synchronize()
    t = {}
    for name, fn, n in (("norm_quant", norm_quant, 10), ("gate_up", gate_up, 3), ("silu_mul_quant", silu, 4),
                        ("down", down, 3), ("chain", chain, 3)):
        ms, _ = graph_time(torch, fn, n, 4 * n, n)
        t[name] = ms
    ops_gu, ops_d = 2.0 * M * 2 * I * H, 2.0 * M * H * I
    b_n, b_s = 7 * M * H + 2 * H + 4 * M, 2 * M * 2 * I + M * I + 4 * M
    res_d["kernels"] = {
        "norm_quant": {"us": round(t["norm_quant"] * 1e3, 2), "gbs": round(b_n / t["norm_quant"] / 1e6, 1),
                       "frac": round(b_n / t["norm_quant"] / 1e6 / HBM_PEAK_GBS, 4)},
        "gate_up": {"us": round(t["gate_up"] * 1e3, 2), "tops": round(ops_gu / t["gate_up"] / 1e9, 1),
                    "frac": round(ops_gu / t["gate_up"] / 1e9 / INT8_PEAK_TOPS, 4)},
        "silu_mul_quant": {"us": round(t["silu_mul_quant"] * 1e3, 2),
                           "gbs": round(b_s / t["silu_mul_quant"] / 1e6, 1),
                           "frac": round(b_s / t["silu_mul_quant"] / 1e6 / HBM_PEAK_GBS, 4)},
        "down": {"us": round(t["down"] * 1e3, 2), "tops": round(ops_d / t["down"] / 1e9, 1),
                 "frac": round(ops_d / t["down"] / 1e9 / INT8_PEAK_TOPS, 4)},
    }
    res_d["chain_us"] = round(t["chain"] * 1e3, 2)
    res_d["chain_tops"] = round((ops_gu + ops_d) / t["chain"] / 1e9, 1)
    k = res_d["kernels"]
    print(f"[bench] MLP tail M={M}: norm+quant {k['norm_quant']['us']} us ({k['norm_quant']['gbs']} GB/s), gate_up "
          f"{k['gate_up']['us']} us ({k['gate_up']['tops']} TOPS), silu_mul_quant {k['silu_mul_quant']['us']} us, "
          f"down {k['down']['us']} us ({k['down']['tops']} TOPS); chain {res_d['chain_us']} us", file=sys.stderr,
          flush=True)
    return res_d


def bench_stack(torch, L, st, dev, ms_list=(1, 4, 4096)):
    """64-layer linear stack (random int8 weights and scales per layer), one HIP graph per pass, bf16."""
    from vllm_turing_amd import workloads
    shapes = workloads.stack_shapes()
    g = torch.Generator(device=dev).manual_seed(7)
    weights = []
    for (_, _, N, K) in shapes:
        w = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev, generator=g)
        sw = torch.rand(N, device=dev, generator=g) * 9e-3 + 1e-3
        weights.append((w, sw))
    n_params = sum(N * K for (_, _, N, K) in shapes)
    H, I = workloads.HIDDEN, workloads.INTERMEDIATE
    res = {"workload": f"64-layer linear stack, {len(shapes)} projections, {n_params / 1e9:.2f} G int8 weights, "
                       f"bf16 activations; per layer residual add + RMSNorm + quant -> mixer in -> quant -> mixer out "
                       f"-> residual add + RMSNorm + quant -> gate_up -> SiLU*up+quant -> down; at M <= 12 the mixer "
                       f"out-projection quantizes its input inside the GEMV (w8a8_gemv_quant); at M <= 5 the MLP runs "
                       f"as the package's decode MLP: SiLU*up in the gate_up GEMV (w8a8_gemv_silu), the down GEMV "
                       f"quantizing its input (w8a8_gemv_quant)", "passes": {}}
    for M in ms_list:
        kmax = max(K for (_, _, _, K) in shapes)
        nmax = max(N for (_, _, N, _) in shapes)
        x = torch.randn(M, H, device=dev, generator=g).to(torch.bfloat16)
        resid = torch.randn(M, H, device=dev, generator=g).to(torch.bfloat16)
        nw = (1.0 + 0.1 * torch.randn(H, device=dev, generator=g)).to(torch.bfloat16)
        y = torch.randn(M, 6144, device=dev, generator=g).to(torch.bfloat16)
        q = torch.empty(M * kmax, dtype=torch.int8, device=dev)
        s = torch.empty(M, dtype=torch.float32, device=dev)
        o = torch.empty(M * nmax, dtype=torch.bfloat16, device=dev)
        d = torch.empty(M, H, dtype=torch.bfloat16, device=dev)

        fused_mlp = M <= 5                                    # the package's decode MLP (tailoverlap.mlp_quantized)

        def one_pass(i=0):
            for li, (_, name, N, K) in enumerate(shapes):
                w, sw = weights[li]
                if name == "gate_up" and fused_mlp:               # SiLU * up in the gate_up GEMV's epilogue
                    if L.rms_norm_quant(x.data_ptr(), resid.data_ptr(), nw.data_ptr(), None, 1e-6, q.data_ptr(),
                                        s.data_ptr(), M, K, 1, st()) != 0:
                        raise RuntimeError("rms_norm_quant")
                    if L.w8a8_gemv_silu(q.data_ptr(), w.data_ptr(), s.data_ptr(), sw.data_ptr(), None, o.data_ptr(),
                                        M, I, K, 1, 1, 1, st()) != 0:
                        raise RuntimeError("w8a8_gemv_silu")
                    continue
                if name == "down" and fused_mlp:                  # the down GEMV quantizes silu(g) * u itself
                    if L.w8a8_gemv_quant(o.data_ptr(), I, q.data_ptr(), s.data_ptr(), w.data_ptr(), sw.data_ptr(),
                                         None, d.data_ptr(), M, N, K, 1, 1, st()) != 0:
                        raise RuntimeError("w8a8_gemv_quant")
                    continue
                if name == "down":
                    src = o[:M * 2 * I].view(M, 2 * I)          # the gate_up output of this layer
                    if L.silu_mul_quant_bf16(src.data_ptr(), q.data_ptr(), s.data_ptr(), M, I, st()) != 0:
                        raise RuntimeError("silu_mul_quant_bf16")
                    dst = d
                elif K == H:                                      # mixer in / gate_up: the normed residual stream
                    if L.rms_norm_quant(x.data_ptr(), resid.data_ptr(), nw.data_ptr(), None, 1e-6, q.data_ptr(),
                                        s.data_ptr(), M, K, 1, st()) != 0:
                        raise RuntimeError("rms_norm_quant")
                    dst = o
                else:                                             # mixer out: the mixer core's output
                    if M <= 12:                                   # quantization fused into the decode GEMV
                        if L.w8a8_gemv_quant(y.data_ptr(), K, q.data_ptr(), s.data_ptr(), w.data_ptr(), sw.data_ptr(),
                                             None, o.data_ptr(), M, N, K, 1, 1, st()) != 0:
                            raise RuntimeError("w8a8_gemv_quant")
                        continue
                    if L.per_token_quant(y.data_ptr(), q.data_ptr(), s.data_ptr(), M, K, K, 1, st()) != 0:
                        raise RuntimeError("per_token_quant")
                    dst = o
                linear_launch(L, st, q, s, w, sw, dst, M, N, K, 1)

        ms, _ = graph_time(torch, one_pass, 1, 3, 1)
        ops = 2.0 * M * n_params
        entry = {"ms_per_pass": round(ms, 3), "us_per_token": round(ms * 1e3 / M, 3)}
        if M <= 32:
            entry["weight_gbs"] = round(n_params / ms / 1e6, 1)
        else:
            entry["tops"] = round(ops / ms / 1e9, 1)
        res["passes"][f"M{M}"] = entry
        print(f"[bench] stack M={M}: {entry}", file=sys.stderr, flush=True)
        del x, resid, nw, y, q, s, o, d
    del weights
    torch.cuda.empty_cache()
    return res


def bench_headline(torch, L, st, dev, args):
    """Decode GEMV (M=1 headline, then M=2/4/8), prefill GEMM at M=4096, the quant kernels, the CPU baseline."""
    from vllm_turing_amd import workloads
    from vllm_turing_amd.quantfuse import per_token_quant

    # ---- decode GEMV, M=1 -----------------------------------------------------------------------------------------
    M, K, N = 1, workloads.HIDDEN, workloads.INTERMEDIATE
    copies = 5
    c = workloads.decode(M)
    x_q, x_s = per_token_quant(c["x"].to(dev))
    gw = torch.Generator(device=dev).manual_seed(1)
    ws = [torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev, generator=gw) for _ in range(copies)]
    sw = c["sw"].to(dev)
    out = torch.empty(M, N, dtype=torch.float16, device=dev)

    def gemv(i):
        rc = L.w8a8_gemv(x_q.data_ptr(), ws[i % copies].data_ptr(), x_s.data_ptr(), sw.data_ptr(), None,
                         out.data_ptr(), M, N, K, 1, 1, 0, st())
        if rc != 0:
            raise RuntimeError(f"w8a8_gemv {rc}")

    print(f"[bench] GEMV M={M} K={K} N={N}, {copies} weight copies", file=sys.stderr, flush=True)
    ms_gemv, n_gemv = graph_time(torch, gemv, 4 * copies, args.steps, args.warmup)
    gemv_bytes = N * K + M * K + 2 * M * N + 4 * N + 4 * M
    gemv_gbs = gemv_bytes / (ms_gemv * 1e-3) / 1e9
    print(f"[bench] GEMV {ms_gemv * 1e3:.2f} us/launch, {gemv_gbs:.0f} GB/s", file=sys.stderr, flush=True)

    # the achievable ceiling: a read-only stream of the same rotated weight copies through the GEMV's load path
    sink = torch.zeros(1, dtype=torch.int32, device=dev)

    def read(i):
        rc = L.hbm_read(ws[i % copies].data_ptr(), N, K, sink.data_ptr(), st())
        if rc != 0:
            raise RuntimeError(f"hbm_read {rc}")

    ms_read, _ = graph_time(torch, read, 4 * copies, args.steps, args.warmup)
    read_gbs = N * K / (ms_read * 1e-3) / 1e9
    read_ceiling = {"workload": f"the M=1 GEMV's weight stream without its math over the same {copies} rotated "
                                f"{N * K / 1e6:.0f} MB weight copies (its grid, 1 KB non-temporal row loads, next row "
                                f"in flight)",
                    "us": round(ms_read * 1e3, 2), "gbs": round(read_gbs, 1),
                    "frac": round(read_gbs / HBM_PEAK_GBS, 4), "gemv_over_read": round(gemv_gbs / read_gbs, 4)}
    print(f"[bench] read ceiling {ms_read * 1e3:.2f} us/launch, {read_gbs:.0f} GB/s", file=sys.stderr, flush=True)

    # the other decode batch sizes of the same projection (M = 2, 4, 8), same weights and method
    decode_m = {}
    workspace(torch, dev)
    for Md in (2, 4, 8, 16, 32, 64):
        cd = workloads.decode(Md)
        xq_d, xs_d = per_token_quant(cd["x"].to(dev))
        out_d = torch.empty(Md, N, dtype=torch.float16, device=dev)

        def gemv_d(i, Md=Md, xq_d=xq_d, xs_d=xs_d, out_d=out_d):
            # the entry the reference's dispatch takes at this M (w8a8.py:108-117): GEMV, mid-band MMA, and above
            # w8a8_big's kernels through the workspace entry, as the package's layers call them
            if Md <= 12:
                rc = L.w8a8_gemv(xq_d.data_ptr(), ws[i % copies].data_ptr(), xs_d.data_ptr(), sw.data_ptr(), None,
                                 out_d.data_ptr(), Md, N, K, 1, 1, 0, st())
            elif Md <= 32:
                rc = L.w8a8_mma(xq_d.data_ptr(), ws[i % copies].data_ptr(), xs_d.data_ptr(), sw.data_ptr(), None,
                                out_d.data_ptr(), Md, N, K, 1, 1, 0, st())
            else:
                rc = scaled_mm_ws(L, st, xq_d, ws[i % copies], xs_d, sw, None, out_d, Md, N, K, 0)
            if rc != 0:
                raise RuntimeError(f"decode M={Md}: {rc}")

        ms_d, _ = graph_time(torch, gemv_d, 4 * copies, 400, 40)
        b_d = N * K + Md * K + 2 * Md * N + 4 * N + 4 * Md
        decode_m[f"M{Md}"] = {"us": round(ms_d * 1e3, 2), "gbs": round(b_d / ms_d / 1e6, 1),
                              "frac": round(b_d / ms_d / 1e6 / HBM_PEAK_GBS, 4)}
    print(f"[bench] GEMV M=2..64: {decode_m}", file=sys.stderr, flush=True)
    del ws

    # batched decode on the other projections (fp16 out, no bias, rotated weights beyond the MALL): the workspace
    # entry, whose 64 x 64 tiles split over K, beside the same entry without a workspace (the streaming passes of at
    # most 64 rows); the two give the same bits (the GPU tests check that)
    mid_split = {}
    gen_m = torch.Generator(device=dev).manual_seed(23)
    for (Mm, Nm, Km) in ((64, 12288, 5120), (64, 5120, 17408), (128, 5120, 17408)):
        mcopies = max(2, int(4.0e8 // (Nm * Km)) + 1)
        wm = [torch.randint(-127, 128, (Nm, Km), dtype=torch.int8, device=dev, generator=gen_m)
              for _ in range(mcopies)]
        am = torch.randint(-127, 128, (Mm, Km), dtype=torch.int8, device=dev, generator=gen_m)
        sam = torch.rand(Mm, device=dev, generator=gen_m) * 1e-2
        swm = torch.rand(Nm, device=dev, generator=gen_m) * 1e-3
        outm = torch.empty(Mm, Nm, dtype=torch.float16, device=dev)

        def split_on(i, Mm=Mm, Nm=Nm, Km=Km, wm=wm, am=am, sam=sam, swm=swm, outm=outm, mcopies=mcopies):
            if scaled_mm_ws(L, st, am, wm[i % mcopies], sam, swm, None, outm, Mm, Nm, Km, 0) != 0:
                raise RuntimeError(f"batched decode M={Mm} N={Nm} K={Km}: workspace entry failed")

        def split_off(i, Mm=Mm, Nm=Nm, Km=Km, wm=wm, am=am, sam=sam, swm=swm, outm=outm, mcopies=mcopies):
            if L.w8a8_scaled_mm(am.data_ptr(), wm[i % mcopies].data_ptr(), sam.data_ptr(), swm.data_ptr(), None,
                                outm.data_ptr(), Mm, Nm, Km, 1, 1, 0, st()) != 0:
                raise RuntimeError(f"batched decode M={Mm} N={Nm} K={Km}: entry failed")

        ms_on, _ = graph_time(torch, split_on, 2 * mcopies, 200, 20)
        ms_off, _ = graph_time(torch, split_off, 2 * mcopies, 200, 20)
        b_m = Nm * Km + Mm * Km + 2 * Mm * Nm + 4 * Nm + 4 * Mm
        mid_split[f"M{Mm}_N{Nm}_K{Km}"] = {"us": round(ms_on * 1e3, 2), "gbs": round(b_m / ms_on / 1e6, 1),
                                           "frac": round(b_m / ms_on / 1e6 / HBM_PEAK_GBS, 4),
                                           "us_without_workspace": round(ms_off * 1e3, 2)}
        del wm
    print(f"[bench] batched decode, K split: {mid_split}", file=sys.stderr, flush=True)

    # ---- prefill GEMM, M=4096, bias, bf16 ---------------------------------------------------------------------------
    Mg, Kg, Ng = 4096, workloads.HIDDEN, 12288
    p = workloads.prefill(Mg)
    a_q, a_s = per_token_quant(p["x"].to(dev))
    # five weight copies (315 MB > the 256 MB MALL), rotated per launch: each launch reads its weights from HBM, as a
    # layer stack does (with one copy the weights stay in the MALL and the GEMM measures ~9% faster)
    gcopies = 5
    gen_w = torch.Generator(device=dev).manual_seed(21)
    wgs = [p["w"].to(dev)] + [torch.randint(-127, 128, (Ng, Kg), dtype=torch.int8, device=dev, generator=gen_w)
                              for _ in range(gcopies - 1)]
    swg = p["sw"].to(dev)
    bias = p["bias"].to(dev)
    outg = torch.empty(Mg, Ng, dtype=torch.bfloat16, device=dev)

    def gemm(i):
        rc = scaled_mm_ws(L, st, a_q, wgs[i % gcopies], a_s, swg, bias, outg, Mg, Ng, Kg, 1)
        if rc != 0:
            raise RuntimeError(f"w8a8_scaled_mm_ws {rc}")

    print(f"[bench] GEMM M={Mg} K={Kg} N={Ng}", file=sys.stderr, flush=True)
    # 2 s of back-to-back GEMMs first, untimed: the clock sample, and the warm-up that lets the clock settle (the
    # first ~100 launches after the memory-bound sections run ~7% slower than the sustained rate)
    rot = iter(range(1 << 30))
    sclk = sclk_under_load(torch, lambda: gemm(next(rot)))   # the same rotation as the timed launches
    print(f"[bench] gfx clock under GEMM load: {sclk} MHz", file=sys.stderr, flush=True)
    gemm_steps = max(20, args.steps // 20)
    ms_gemm, n_gemm = graph_time(torch, gemm, gcopies, gemm_steps, max(4, args.warmup // 20))
    gemm_ops = 2.0 * Mg * Ng * Kg
    gemm_tops = gemm_ops / (ms_gemm * 1e-3) / 1e12
    print(f"[bench] GEMM {ms_gemm * 1e3:.1f} us/launch, {gemm_tops:.0f} TOPS", file=sys.stderr, flush=True)
    # the other prefill chunk sizes of the same projection, same rotated weights: the first Mo rows of the activations
    gemm_other = {}
    for Mo in (512, 2048):
        outo = torch.empty(Mo, Ng, dtype=torch.bfloat16, device=dev)

        def gemm_o(i, Mo=Mo, outo=outo):
            rc = scaled_mm_ws(L, st, a_q, wgs[i % gcopies], a_s, swg, bias, outo, Mo, Ng, Kg, 1)
            if rc != 0:
                raise RuntimeError(f"w8a8_scaled_mm_ws M={Mo}: {rc}")

        ms_o, _ = graph_time(torch, gemm_o, 2 * gcopies, 8 * gcopies, 2 * gcopies)
        tops_o = 2.0 * Mo * Ng * Kg / (ms_o * 1e-3) / 1e12
        gemm_other[f"M{Mo}"] = {"us": round(ms_o * 1e3, 2), "tops": round(tops_o, 1),
                                "frac": round(tops_o / INT8_PEAK_TOPS, 4)}
    print(f"[bench] GEMM M=512 / 2048: {gemm_other}", file=sys.stderr, flush=True)
    del wgs

    # ---- quant kernels ------------------------------------------------------------------------------------------------
    xq_in = torch.randn(Mg, Kg, dtype=torch.bfloat16, device=dev)
    qq = torch.empty(Mg, Kg, dtype=torch.int8, device=dev)
    sq = torch.empty(Mg, dtype=torch.float32, device=dev)

    def quant(i):
        rc = L.per_token_quant(xq_in.data_ptr(), qq.data_ptr(), sq.data_ptr(), Mg, Kg, Kg, 1, st())
        if rc != 0:
            raise RuntimeError(f"per_token_quant {rc}")

    ms_q, _ = graph_time(torch, quant, 10, 200, 20)
    quant_bytes = 3 * Mg * Kg + 4 * Mg
    I = workloads.INTERMEDIATE
    gu = torch.randn(Mg, 2 * I, dtype=torch.bfloat16, device=dev)
    qs = torch.empty(Mg, I, dtype=torch.int8, device=dev)
    ss = torch.empty(Mg, dtype=torch.float32, device=dev)

    def smq(i):
        rc = L.silu_mul_quant_bf16(gu.data_ptr(), qs.data_ptr(), ss.data_ptr(), Mg, I, st())
        if rc != 0:
            raise RuntimeError(f"silu_mul_quant {rc}")

    ms_s, _ = graph_time(torch, smq, 4, 40, 8)
    smq_bytes = 2 * Mg * 2 * I + Mg * I + 4 * Mg
    print(f"[bench] quant {ms_q * 1e3:.1f} us, silu_mul_quant {ms_s * 1e3:.1f} us", file=sys.stderr, flush=True)

    # AR8 operand of a prefill-size all-reduce (4096 x 5120 fp16): quantize, and the dequantised sum of 2 / 8 ranks
    n8 = Mg * Kg
    a8 = torch.randn(n8, device=dev).half()
    p8 = torch.empty(8 * (n8 + n8 // 64), dtype=torch.uint8, device=dev)
    o8 = torch.empty(n8, dtype=torch.float16, device=dev)
    for r in range(8):
        L.ar8_quant(a8.data_ptr(), p8.data_ptr() + r * (n8 + n8 // 64), n8, st())

    def ar8q(i):
        if L.ar8_quant(a8.data_ptr(), p8.data_ptr(), n8, st()) != 0:
            raise RuntimeError("ar8_quant")

    ar8_res = {}
    ms_a, _ = graph_time(torch, ar8q, 10, 200, 20)
    b_a = 2 * n8 + n8 + n8 // 64
    ar8_res["quant_us"], ar8_res["quant_gbs"] = round(ms_a * 1e3, 2), round(b_a / ms_a / 1e6, 1)
    for ranks in (2, 8):
        def ar8s(i, ranks=ranks):
            if L.ar8_dequant_sum_ranks(p8.data_ptr(), o8.data_ptr(), n8, ranks, st()) != 0:
                raise RuntimeError("ar8_dequant_sum")
        ms_d, _ = graph_time(torch, ar8s, 10, 200, 20)
        b_d = ranks * (n8 + n8 // 64) + 2 * n8
        ar8_res[f"dequant_sum_{ranks}ranks_us"] = round(ms_d * 1e3, 2)
        ar8_res[f"dequant_sum_{ranks}ranks_gbs"] = round(b_d / ms_d / 1e6, 1)
    del a8, p8, o8
    print(f"[bench] AR8 n={n8}: {ar8_res}", file=sys.stderr, flush=True)

    # int8 LM head (W8A16) over the 27B model's 248,320-row vocabulary at K = 5120, bf16 logits, M = 1 / 4 / 16
    Nh = 248320
    wh = torch.randint(-127, 128, (Nh, Kg), dtype=torch.int8, device=dev)
    sh = torch.rand(Nh, device=dev) * 1e-3
    head = {}
    for Mh in (1, 4, 16):
        xh = torch.randn(Mh, Kg, device=dev).to(torch.bfloat16)
        oh = torch.empty(Mh, Nh, dtype=torch.bfloat16, device=dev)

        def lmh(i, Mh=Mh, xh=xh, oh=oh):
            if L.w8a16_gemv(xh.data_ptr(), wh.data_ptr(), sh.data_ptr(), None, oh.data_ptr(), Mh, Nh, Kg, 1, st()) != 0:
                raise RuntimeError("w8a16_gemv")
        ms_h, _ = graph_time(torch, lmh, 4, 40, 8)
        b_h = Nh * Kg + 4 * Nh + 2 * Mh * Kg + 2 * Mh * Nh
        head[f"M{Mh}"] = {"us": round(ms_h * 1e3, 2), "gbs": round(b_h / ms_h / 1e6, 1),
                          "frac": round(b_h / ms_h / 1e6 / HBM_PEAK_GBS, 4)}
    del wh, sh
    print(f"[bench] int8 LM head N={Nh} K={Kg}: {head}", file=sys.stderr, flush=True)

    # ---- CPU baseline: the reference's CPU path (torch int8 matmul + dequant), bounded sample ---------------------
    cpu = None
    cpu_gemm = None
    if not args.no_cpu:
        from oracle import cpu_path
        threads = torch.get_num_threads()
        n_cpus, cpu_model = host_cpu()
        xc, wc, swc = c["x"], c["w"], c["sw"]
        t_gemv, n_cpu = cpu_time(lambda: cpu_path.linear(xc, wc, swc, None, torch.float16), 10.0)
        cpu = {"value": round(gemv_bytes / t_gemv / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
               "sample": f"M=1 K={K} N={N} quant+int_mm+dequant, {n_cpu} calls, median",
               "host_cpus": n_cpus, "cpu_model": cpu_model}
        Ms = 256
        xs_ = p["x"][:Ms]
        t_g, n_g = cpu_time(lambda: cpu_path.linear(xs_, p["w"], p["sw"], p["bias"], torch.bfloat16), 10.0)
        cpu_gemm = {"value": round(2.0 * Ms * Ng * Kg / t_g / 1e12, 3), "unit": "TOPS", "cores": threads,
                    "kind": "port", "sample": f"M={Ms} of 4096 rows, K={Kg} N={Ng}, {n_g} calls, median",
                    "host_cpus": n_cpus, "cpu_model": cpu_model}
        print(f"[bench] CPU GEMV {cpu['value']} GB/s, GEMM {cpu_gemm['value']} TOPS on {threads} threads "
              f"(host: {n_cpus} CPUs, {cpu_model})", file=sys.stderr, flush=True)

    result = {
        "metric": METRIC,
        "value": round(gemv_gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": n_gemv,
        "warmup": args.warmup,
        "ms_per_step": round(ms_gemv, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": f"decode W8A8 GEMV M={M} K={K} N={N} (int8 weights, fp16 out), {copies} rotated "
                               f"weight copies ({copies * N * K / 1e6:.0f} MB > 256 MB MALL), HIP-graph replay",
                   "M": M, "K": K, "N": N, "weight_copies": copies},
        "roofline": {"bound": "hbm", "achieved": round(gemv_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gemv_gbs / HBM_PEAK_GBS, 4), "traffic": traffic_from_profiles("gemv_m1")},
        "cpu_baseline": cpu,
        "gemv_read_ceiling": read_ceiling,
        "decode_other_m": {"workload": f"decode W8A8 K={K} N={N}, fp16 out, same rotated weights, the entry the reference "
                                       f"dispatches at each M (w8a8_gemv <= 12, w8a8_mma <= 32, above w8a8_big's "
                                       f"kernels through the workspace entry, split over K where the plan splits)",
                           **decode_m},
        "batched_decode_split": {"workload": "batched decode W8A8 on the other projections, fp16 out, rotated "
                                             "weights: w8a8_scaled_mm_ws (64 x 64 tiles split over K) beside "
                                             "w8a8_scaled_mm without a workspace (streaming passes of <= 64 rows)",
                                 **mid_split},
        "gemm": {"workload": f"prefill W8A8 GEMM M={Mg} K={Kg} N={Ng}, bias, bf16 out, {gcopies} rotated weight copies "
                             f"({gcopies * Ng * Kg / 1e6:.0f} MB > 256 MB MALL)", "ms": round(ms_gemm, 4),
                 "launches": n_gemm, "tops": round(gemm_tops, 1),
                 "roofline": {"bound": "mfma", "achieved": round(gemm_tops, 1), "peak": INT8_PEAK_TOPS,
                              "unit": "TOPS", "frac": round(gemm_tops / INT8_PEAK_TOPS, 4),
                              "traffic": traffic_from_profiles("gemm_m4096")},
                 "other_m": {"workload": f"the same projection (K={Kg}, N={Ng}, bias, bf16, rotated weights) at "
                                         f"the other prefill chunk sizes", **gemm_other},
                 "sclk_mhz": sclk,
                 "frac_at_sclk": (round(gemm_tops / (INT8_PEAK_TOPS * sclk / SCLK_MAX_MHZ), 4) if sclk else None),
                 "cpu_baseline": cpu_gemm},
        "quant": {"per_token_quant_M4096_K5120": {"us": round(ms_q * 1e3, 2),
                                                   "gbs": round(quant_bytes / (ms_q * 1e-3) / 1e9, 1)},
                  "silu_mul_quant_M4096_I17408": {"us": round(ms_s * 1e3, 2),
                                                   "gbs": round(smq_bytes / (ms_s * 1e-3) / 1e9, 1)},
                  "ar8_n20971520": ar8_res},
        "lm_head_w8a16": {"workload": f"int8 LM head N={Nh} K={Kg}, bf16 activations and logits", **head},
    }
    return result


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000, help="timed GEMV launches")
    ap.add_argument("--warmup", type=int, default=200, help="untimed GEMV launches")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--traffic", action="store_true", help="launch sequence for HBM-traffic counter runs")
    ap.add_argument("--sections", default="headline,mlp,stack",
                    help="comma list: headline (GEMV, GEMM, quant kernels, CPU baseline: the contract's JSON fields), "
                         "mlp (MLP chain at M=4096), stack (64-layer sweep); profiling runs select one")
    args = ap.parse_args()
    sections = set(args.sections.split(","))
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this W8A8 path has no multi-GPU mode (asked for --gpus {args.gpus})",
              file=sys.stderr)
        sys.exit(2)

    import torch
    from vllm_turing_amd import _lib

    dev = "cuda:0"
    torch.cuda.set_device(0)
    L = _lib.lib()
    st = lambda: torch.cuda.current_stream().cuda_stream
    workspace(torch, dev)
    if args.traffic:
        traffic_sequence(torch, L, st, dev)
        return

    if "headline" in sections:
        result = bench_headline(torch, L, st, dev, args)
    else:
        result = {"metric": METRIC, "sections": sorted(sections)}
    if "mlp" in sections:
        torch.cuda.empty_cache()
        result["mlp_chain"] = bench_mlp(torch, L, st, dev)
    if "stack" in sections:
        torch.cuda.empty_cache()
        result["stack"] = bench_stack(torch, L, st, dev)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
