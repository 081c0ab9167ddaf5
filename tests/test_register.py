"""register() and the install() hooks against stand-in vLLM modules (vLLM itself is not importable here).

The stand-ins carry exactly the attributes the hooks replace: vllm._custom_ops.{cutlass_scaled_mm, scaled_int8_quant,
rms_norm_dynamic_per_token_quant}, vllm.compilation.caching.aot_compile_hash_factors and
vllm.model_executor.layers.vocab_parallel_embedding.{UnquantizedEmbeddingMethod, ParallelLMHead}.  Checked on the CPU
(the device gate forced open where the test says so): the reference's install order (vllm_turing/__init__.py:38-72),
one replacement per attribute however often register() / install() run, VLLM_TURING_DISABLE and the per-hook switches,
no patching off gfx950, and that the cases the hooks do not take reach vLLM's own functions.  On the GPU
(test_registered_ops_give_oracle_bits): the patched vLLM entry points return the oracle's bits.
"""
import sys
import types

import numpy as np
import pytest
import torch

import vllm_turing_amd as pkg
from vllm_turing_amd import hooks, lmhead, quantfuse, normquant

VLLM_OP = "vllm-op"


def _stub_vllm():
    calls = []
    vllm = types.ModuleType("vllm")
    ops = types.ModuleType("vllm._custom_ops")

    def cutlass_scaled_mm(a, b, scale_a, scale_b, out_dtype, bias=None):
        calls.append("cutlass_scaled_mm")
        return VLLM_OP

    def scaled_int8_quant(input, scale=None, azp=None, symmetric=True):
        calls.append("scaled_int8_quant")
        return VLLM_OP

    def rms_norm_dynamic_per_token_quant(input, weight, epsilon, quant_dtype, scale_ub=None, residual=None):
        calls.append("rms_norm_dynamic_per_token_quant")
        return VLLM_OP

    ops.cutlass_scaled_mm = cutlass_scaled_mm
    ops.scaled_int8_quant = scaled_int8_quant
    ops.rms_norm_dynamic_per_token_quant = rms_norm_dynamic_per_token_quant
    vllm._custom_ops = ops

    compilation = types.ModuleType("vllm.compilation")
    caching = types.ModuleType("vllm.compilation.caching")
    caching.aot_compile_hash_factors = lambda cfg: ["upstream"]
    compilation.caching = caching
    vllm.compilation = compilation

    me = types.ModuleType("vllm.model_executor")
    layers = types.ModuleType("vllm.model_executor.layers")
    vpe = types.ModuleType("vllm.model_executor.layers.vocab_parallel_embedding")

    class UnquantizedEmbeddingMethod:
        def process_weights_after_loading(self, layer):
            calls.append("process_weights_after_loading")

        def apply(self, layer, x, bias=None):
            calls.append("apply")
            return VLLM_OP

    class ParallelLMHead(torch.nn.Module):
        def __init__(self, weight):
            super().__init__()
            self.weight = torch.nn.Parameter(weight, requires_grad=False)

    vpe.UnquantizedEmbeddingMethod = UnquantizedEmbeddingMethod
    vpe.ParallelLMHead = ParallelLMHead
    layers.vocab_parallel_embedding = vpe
    me.layers = layers
    vllm.model_executor = me
    mods = {"vllm": vllm, "vllm._custom_ops": ops, "vllm.compilation": compilation,
            "vllm.compilation.caching": caching, "vllm.model_executor": me, "vllm.model_executor.layers": layers,
            "vllm.model_executor.layers.vocab_parallel_embedding": vpe}
    return mods, calls


@pytest.fixture
def stub(monkeypatch):
    mods, calls = _stub_vllm()
    for name, mod in mods.items():
        monkeypatch.setitem(sys.modules, name, mod)
    monkeypatch.setattr(pkg, "_registered", False)
    monkeypatch.setattr(hooks, "INSTALLED", [])
    monkeypatch.delenv("VLLM_TURING_DISABLE", raising=False)
    monkeypatch.delenv("VLLM_TURING_LMHEAD", raising=False)
    return types.SimpleNamespace(ops=mods["vllm._custom_ops"], caching=mods["vllm.compilation.caching"],
                                 vpe=mods["vllm.model_executor.layers.vocab_parallel_embedding"], calls=calls)


@pytest.fixture
def gfx950(monkeypatch):
    monkeypatch.setattr(hooks, "on_gfx950", lambda: True)


def test_register_order_and_targets(stub, gfx950):
    done = pkg.register()
    assert done == {"normquant": True, "quantfuse": True, "w8a8": True, "lmhead": True}
    M = stub.vpe.UnquantizedEmbeddingMethod
    assert [(o, n) for o, n in hooks.INSTALLED] == [
        ("vllm._custom_ops", "rms_norm_dynamic_per_token_quant"),
        ("vllm._custom_ops", "scaled_int8_quant"),
        ("vllm.compilation.caching", "aot_compile_hash_factors"),
        ("vllm._custom_ops", "cutlass_scaled_mm"),
        ("UnquantizedEmbeddingMethod", "process_weights_after_loading"),
        ("UnquantizedEmbeddingMethod", "apply"),
    ]
    assert stub.ops.cutlass_scaled_mm is pkg.w8a8.cutlass_scaled_mm
    for f in (stub.ops.cutlass_scaled_mm, stub.ops.scaled_int8_quant, stub.ops.rms_norm_dynamic_per_token_quant,
              stub.caching.aot_compile_hash_factors, M.process_weights_after_loading, M.apply):
        assert hooks.ours(f)
    assert stub.caching.aot_compile_hash_factors(None) == ["upstream", "vllm_turing_amd.per_token_quant"]


def test_register_once_and_install_idempotent(stub, gfx950):
    pkg.register()
    first = (stub.ops.cutlass_scaled_mm, stub.ops.scaled_int8_quant, stub.ops.rms_norm_dynamic_per_token_quant,
             stub.vpe.UnquantizedEmbeddingMethod.apply, stub.caching.aot_compile_hash_factors)
    n = len(hooks.INSTALLED)
    assert pkg.register() == {}                                       # once per process
    pkg._registered = False
    assert pkg.register() == {"normquant": True, "quantfuse": True, "w8a8": True, "lmhead": True}
    for mod in (quantfuse, normquant, pkg.w8a8, lmhead):
        assert mod.install()
    assert len(hooks.INSTALLED) == n                                  # nothing wrapped twice
    assert (stub.ops.cutlass_scaled_mm, stub.ops.scaled_int8_quant, stub.ops.rms_norm_dynamic_per_token_quant,
            stub.vpe.UnquantizedEmbeddingMethod.apply, stub.caching.aot_compile_hash_factors) == first
    assert stub.caching.aot_compile_hash_factors(None) == ["upstream", "vllm_turing_amd.per_token_quant"]


def test_disable_switch(stub, gfx950, monkeypatch):
    monkeypatch.setenv("VLLM_TURING_DISABLE", "1")
    orig = stub.ops.cutlass_scaled_mm
    assert pkg.register() == {}
    assert stub.ops.cutlass_scaled_mm is orig and not hooks.ours(stub.ops.scaled_int8_quant)
    assert hooks.INSTALLED == []


def test_per_hook_switches(stub, gfx950, monkeypatch):
    monkeypatch.setenv("VLLM_TURING_LMHEAD", "0")
    monkeypatch.setattr(quantfuse, "ENABLED", False)
    monkeypatch.setattr(normquant, "ENABLED", False)
    assert pkg.register() == {"normquant": False, "quantfuse": False, "w8a8": True, "lmhead": False}
    assert not hooks.ours(stub.ops.scaled_int8_quant) and not hooks.ours(stub.ops.rms_norm_dynamic_per_token_quant)
    assert not hooks.ours(stub.vpe.UnquantizedEmbeddingMethod.apply)


def test_no_patching_off_gfx950(stub, monkeypatch):
    monkeypatch.setattr(hooks, "on_gfx950", lambda: False)
    assert pkg.register() == {"normquant": False, "quantfuse": False, "w8a8": False, "lmhead": False}
    assert hooks.INSTALLED == []
    assert not hooks.ours(stub.ops.cutlass_scaled_mm)


def test_untaken_cases_reach_vllm(stub, gfx950):
    pkg.register()
    x = torch.zeros(2, 16, dtype=torch.float16)
    assert stub.ops.scaled_int8_quant(x, scale=torch.ones(1)) == VLLM_OP          # static scale
    assert stub.ops.scaled_int8_quant(x, None, torch.zeros(1), False) == VLLM_OP   # asymmetric
    assert stub.ops.rms_norm_dynamic_per_token_quant(x, x[0], 1e-6, torch.float8_e4m3fn) == VLLM_OP
    assert stub.calls == ["scaled_int8_quant", "scaled_int8_quant", "rms_norm_dynamic_per_token_quant"]
    # the LM head: a head not converted (here on the CPU) keeps vLLM's loading and apply()
    meth = stub.vpe.UnquantizedEmbeddingMethod()
    head = stub.vpe.ParallelLMHead(torch.zeros(64, 32, dtype=torch.bfloat16))
    meth.process_weights_after_loading(head)
    assert not hasattr(head, "turing_w8")
    assert meth.apply(head, torch.zeros(1, 32, dtype=torch.bfloat16)) == VLLM_OP
    assert stub.calls[-2:] == ["process_weights_after_loading", "apply"]


def test_lmhead_skips_heads_the_kernels_cannot_address():
    assert lmhead.kernel_takes(248320, 5120)
    assert not lmhead.kernel_takes(262144, 8192)        # 2^31 bytes
    assert not lmhead.kernel_takes(1000, 5128)          # K % 16


@pytest.mark.gpu
def test_registered_ops_give_oracle_bits(stub, oracle_lib):
    """With the real device gate on an MI355X: the patched vLLM entry points return the oracle's bits (per-token
    quant, fused norm + quant, the scaled matmul at decode and prefill M) and the LM head is converted on loading and
    computed by the int8 kernel."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import oracle
    from oracle import cpu_path
    assert hooks.on_gfx950()
    assert pkg.register() == {"normquant": True, "quantfuse": True, "w8a8": True, "lmhead": True}
    ops, dev = stub.ops, "cuda"
    g = torch.Generator().manual_seed(21)
    K, N = 5120, 1024
    w = torch.randint(-127, 128, (N, K), dtype=torch.int8, generator=g)
    sw = torch.rand(N, 1, generator=g) * 1e-2 + 1e-4
    for M in (4, 300):
        x = torch.randn(M, K, generator=g).to(torch.bfloat16)
        q, s, azp = ops.scaled_int8_quant(x.to(dev))
        out = ops.cutlass_scaled_mm(q, w.to(dev).t(), s, sw.to(dev), torch.bfloat16)
        torch.cuda.synchronize()
        qr, sr = oracle.quant_rows(x)
        assert azp is None and np.array_equal(q.cpu().numpy(), qr) and np.array_equal(s.cpu().view(-1).numpy(), sr)
        ref, _ = cpu_path.scaled_mm(torch.from_numpy(qr), w, torch.from_numpy(sr), sw, None, torch.bfloat16)
        assert torch.equal(out.cpu(), ref), M
    h = torch.randn(8, K, generator=g).to(torch.bfloat16)
    res = torch.randn(8, K, generator=g).to(torch.bfloat16)
    nw = (1.0 + 0.1 * torch.randn(K, generator=g)).to(torch.bfloat16)
    res_d = res.to(dev)
    q, s = ops.rms_norm_dynamic_per_token_quant(h.to(dev), nw.to(dev), 1e-6, torch.int8, None, res_d)
    torch.cuda.synchronize()
    qr, sr, rr, _ = oracle.rms_norm_quant(h, nw, 1e-6, res)
    assert np.array_equal(q.cpu().numpy(), qr) and np.array_equal(s.cpu().view(-1).numpy(), sr)
    assert np.array_equal(res_d.cpu().view(torch.int16).numpy().view(np.uint16), rr)
    assert stub.calls == []                                           # vLLM's own ops never ran
    # the LM head
    meth = stub.vpe.UnquantizedEmbeddingMethod()
    w16 = (torch.randn(3000, K, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    head = stub.vpe.ParallelLMHead(w16.clone())
    meth.process_weights_after_loading(head)
    assert head.weight.numel() == 0 and head.turing_w8.dtype == torch.int8
    wq, ws = lmhead.quantize_rows(w16)
    assert torch.equal(head.turing_w8, wq) and torch.equal(head.turing_s, ws)
    x = torch.randn(3, K, generator=g).to(torch.bfloat16).to(dev)
    y = meth.apply(head, x)
    y_ref = lmhead.w8a16_mm(x, wq, ws)
    torch.cuda.synchronize()
    assert torch.equal(y, y_ref)
    assert stub.calls == ["process_weights_after_loading"]
