"""Seeded synthetic inputs at the shapes and distributions of the W8A8 path's benchmark configurations.

All tensors are generated on the CPU with torch.Generator(seed) (so every machine gets identical bits) and moved to
the device by the caller.  Shapes (N x K is the int8 weight, row-major [N, K]):
  cpu_case:  X fp16 [16, 5120] ~ N(0, 1) with 0.5% outlier channels x 20, W int8 [5120, 5120] uniform in [-127, 127],
             per-output-channel scales ~ U(1e-3, 1e-2), fp16 out.
  decode:    M in {1, 2, 4, 8} activation rows, K = 5120, N = 17408 (the MLP gate/up shard), fp16 out.
  prefill:   M in {512, 2048, 4096}, K = 5120, N = 12288 (fused QKV), bias bf16 ~ N(0, 1), bf16 out.
  mlp:       M = 4096, gate_up N = 2 x 17408 over K = 5120, down N = 5120 over K = 17408, bf16, activations N(0, 1)
             with outlier channels divided by SmoothQuant factors s_j = max|X_j|^0.6 / max|W_j|^0.4
             (alpha 0.6, the fold of scripts/w8a8_convert.py:114 clamped to [1e-2, 1e2]).
  stack:     the 64-layer projection shapes of the 27B hybrid model at TP1 (48 GDN + 16 attention layers, 64 MLPs).
"""
import torch

HIDDEN = 5120
INTERMEDIATE = 17408


def gen(seed):
    return torch.Generator().manual_seed(seed)


def activations(M, K, dtype=torch.float16, outliers=0.005, scale=20.0, seed=0):
    """x ~ N(0, 1) [M, K] with round(outliers * K) channels (chosen by randperm) multiplied by `scale`."""
    g = gen(seed)
    x = torch.randn(M, K, generator=g)
    n_out = int(round(outliers * K))
    if n_out:
        ch = torch.randperm(K, generator=g)[:n_out]
        x[:, ch] *= scale
    return x.to(dtype)


def weight(N, K, seed=1):
    """int8 [N, K] uniform integers in [-127, 127]."""
    return torch.randint(-127, 128, (N, K), dtype=torch.int8, generator=gen(seed))


def weight_scale(N, seed=2, lo=1e-3, hi=1e-2):
    """float32 [N, 1] ~ U(lo, hi)."""
    g = gen(seed)
    return (torch.rand(N, 1, generator=g) * (hi - lo) + lo).to(torch.float32)


def cpu_case(seed=0):
    x = activations(16, HIDDEN, torch.float16, seed=seed)
    return dict(x=x, w=weight(HIDDEN, HIDDEN, seed + 1), sw=weight_scale(HIDDEN, seed + 2), out_dtype=torch.float16)


def decode(M, seed=0, N=INTERMEDIATE, K=HIDDEN):
    x = activations(M, K, torch.float16, outliers=0.0, seed=seed)
    return dict(x=x, w=weight(N, K, seed + 1), sw=weight_scale(N, seed + 2), out_dtype=torch.float16)


def prefill(M, seed=0, N=12288, K=HIDDEN):
    x = activations(M, K, torch.bfloat16, outliers=0.0, seed=seed)
    bias = torch.randn(N, generator=gen(seed + 3)).to(torch.bfloat16)
    return dict(x=x, w=weight(N, K, seed + 1), sw=weight_scale(N, seed + 2), bias=bias, out_dtype=torch.bfloat16)


def smoothquant_activations(M, K, w, alpha=0.6, seed=0):
    """Outlier activations divided by the SmoothQuant factor of each input channel (scripts/w8a8_convert.py:114)."""
    x = activations(M, K, torch.float32, seed=seed)
    xmax = x.abs().amax(dim=0)
    wmax = w.float().abs().amax(dim=0).clamp_min(1e-5)
    s = (xmax.pow(alpha) / wmax.pow(1 - alpha)).clamp(1e-2, 1e2)
    return (x / s).to(torch.bfloat16)


def mlp(M=4096, seed=0):
    w_gu = weight(2 * INTERMEDIATE, HIDDEN, seed + 1)
    w_d = weight(HIDDEN, INTERMEDIATE, seed + 4)
    return dict(x=smoothquant_activations(M, HIDDEN, w_gu, seed=seed), w_gate_up=w_gu,
                sw_gate_up=weight_scale(2 * INTERMEDIATE, seed + 2), w_down=w_d,
                sw_down=weight_scale(HIDDEN, seed + 5), out_dtype=torch.bfloat16)


# per layer type: (name, N, K) of each W8A8 projection at TP1
GDN_LAYER = (("in_proj_qkvz", 16384, HIDDEN), ("out_proj", HIDDEN, 6144))
ATTN_LAYER = (("qkv", 14336, HIDDEN), ("o_proj", HIDDEN, 6144))
MLP_LAYER = (("gate_up", 2 * INTERMEDIATE, HIDDEN), ("down", HIDDEN, INTERMEDIATE))


def stack_shapes(n_layers=64, attn_every=4):
    """(layer, name, N, K) for the 64-layer stack: every attn_every-th layer is attention, the rest GDN."""
    out = []
    for i in range(n_layers):
        mixer = ATTN_LAYER if (i + 1) % attn_every == 0 else GDN_LAYER
        for name, N, K in (*mixer, *MLP_LAYER):
            out.append((i, name, N, K))
    return out
