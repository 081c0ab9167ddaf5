"""The W8A8 checkpoint format on the input side of the path (vllm_turing_amd/checkpoint.py, following
scripts/w8a8_convert.py): per-channel weight quantization against its closed form, the SmoothQuant fold against the
float64 identity it must preserve (the products of every smoothed group are unchanged before quantization), the
calibration merge rule, and a convert -> load round trip through real safetensors shards."""
import json
import os

import numpy as np
import pytest
import torch

from vllm_turing_amd import checkpoint as ck


def test_quantize_per_channel_closed_form():
    w = torch.tensor([[127.0, 0.5, 1.5, -2.5], [0.0, 0.0, 0.0, 0.0], [-3.0, 1.0, 0.02, 2.9]])
    q, s = ck.quantize_per_channel(w)
    assert q.dtype == torch.int8 and s.shape == (3, 1) and s.dtype == torch.float32
    assert q[0].tolist() == [127, 0, 2, -2]                       # scale 1: round half to even
    assert q[1].tolist() == [0, 0, 0, 0] and s[1, 0] == np.float32(1e-12) / np.float32(127)
    assert q[2, 0] == -127                                          # the row's absmax maps to -127
    g = torch.Generator().manual_seed(0)
    w = torch.randn(64, 300, generator=g) * torch.rand(64, 1, generator=g) * 10
    q, s = ck.quantize_per_channel(w)
    assert torch.all((q.float() * s - w).abs() <= s / 2 * (1 + 1e-6))
    assert torch.all(q.abs().amax(dim=1) == 127)


def _rms_zc(x, w):                                                # zero-centred RMSNorm: x / rms * (1 + w)
    return x / torch.sqrt((x * x).mean(dim=1, keepdim=True) + 1e-6) * (1 + w)


def test_smoothing_preserves_products():
    g = torch.Generator().manual_seed(1)
    T, H, n_q, n_kv, hd, I = 7, 32, 4, 2, 8, 24
    n_vh, vhd = 4, 6
    tc = {"num_attention_heads": n_q, "num_key_value_heads": n_kv, "head_dim": hd,
          "linear_num_value_heads": n_vh, "linear_value_head_dim": vhd}
    d = lambda *s: torch.randn(*s, generator=g, dtype=torch.float64)
    P = "model.language_model.layers.0."
    t = {P + "input_layernorm.weight": d(H) * 0.1, P + "post_attention_layernorm.weight": d(H) * 0.1,
         P + "self_attn.q_proj.weight": d(n_q * hd, H), P + "self_attn.k_proj.weight": d(n_kv * hd, H),
         P + "self_attn.v_proj.weight": d(n_kv * hd, H), P + "self_attn.o_proj.weight": d(H, n_q * hd),
         P + "mlp.gate_proj.weight": d(I, H), P + "mlp.up_proj.weight": d(I, H), P + "mlp.down_proj.weight": d(H, I),
         P + "linear_attn.out_proj.weight": d(H, n_vh * vhd), P + "linear_attn.norm.weight": d(vhd)}
    stats = {P + "self_attn.qkv_proj": d(H).abs() * 5, P + "self_attn.o_proj": d(n_q * hd).abs() * 3,
             P + "mlp.gate_up_proj": d(H).abs() * 7, P + "mlp.down_proj": d(I).abs() * 2,
             P + "linear_attn.out_proj": d(n_vh * vhd).abs() * 4}
    stats = {k: v.float() for k, v in stats.items()}
    wmax = {c: t[c].float().abs().amax(dim=0) for c in ck.Smoothing.consumers(stats) if c in t}
    plan = ck.Smoothing.plan(stats, wmax, tc, 0.5)
    sm = {k: (plan.apply(k, v) if plan.apply(k, v) is not None else v.float()).double() for k, v in t.items()}
    x, z = d(T, H), d(T, n_vh * vhd)
    # qkv after the input norm (v's rows also carry the o_proj group's 1 / s: its outputs are scaled per channel)
    s_o = plan.edits[P + "self_attn.v_proj.weight"].rows.double()
    for proj in ("q_proj", "k_proj", "v_proj"):
        a = _rms_zc(x, t[P + "input_layernorm.weight"]) @ t[P + f"self_attn.{proj}.weight"].T
        b = _rms_zc(x, sm[P + "input_layernorm.weight"]) @ sm[P + f"self_attn.{proj}.weight"].T
        if proj == "v_proj":
            a = a / s_o
        assert torch.allclose(a, b, rtol=1e-5, atol=1e-5)
    # o_proj of the v heads repeated over their q heads (GQA), attention weights of one
    def o_out(nw, v_w, o_w):
        v = _rms_zc(x, nw) @ v_w.T                               # [T, n_kv * hd]
        rep = v.view(T, n_kv, 1, hd).expand(T, n_kv, n_q // n_kv, hd).reshape(T, n_q * hd)
        return rep @ o_w.T
    assert torch.allclose(o_out(t[P + "input_layernorm.weight"], t[P + "self_attn.v_proj.weight"],
                                t[P + "self_attn.o_proj.weight"]),
                          o_out(sm[P + "input_layernorm.weight"], sm[P + "self_attn.v_proj.weight"],
                                sm[P + "self_attn.o_proj.weight"]), rtol=1e-5,
                          atol=1e-5)
    # MLP: gate/up after the post-attention norm, down after silu(gate) * up
    def mlp(tt):
        h = _rms_zc(x, tt[P + "post_attention_layernorm.weight"])
        gte, up = h @ tt[P + "mlp.gate_proj.weight"].T, h @ tt[P + "mlp.up_proj.weight"].T
        return (torch.nn.functional.silu(gte) * up) @ tt[P + "mlp.down_proj.weight"].T
    assert torch.allclose(mlp(t), mlp(sm), rtol=1e-5, atol=1e-5)
    # GDN out_proj after the gated norm (weight per dimension, shared by the value heads)
    def gdn(tt):
        o = x[:, :n_vh * vhd].reshape(T, n_vh, vhd)
        n = o / torch.sqrt((o * o).mean(dim=2, keepdim=True) + 1e-6) * tt[P + "linear_attn.norm.weight"]
        n = n * torch.nn.functional.silu(z.view(T, n_vh, vhd))
        return n.reshape(T, n_vh * vhd) @ tt[P + "linear_attn.out_proj.weight"].T
    assert torch.allclose(gdn(t), gdn(sm), rtol=1e-5, atol=1e-5)
    # the factors themselves: s = x^a / w^(1-a), clamped
    s = plan.edits[P + "mlp.down_proj.weight"].cols
    ref = (stats[P + "mlp.down_proj"].clamp(min=1e-5) ** 0.5 / wmax[P + "mlp.down_proj.weight"].clamp(min=1e-5) ** 0.5)
    assert torch.allclose(s, ref.clamp(1e-2, 1e2))


def test_calibration_merge(tmp_path):
    from safetensors.torch import save_file
    a = {"language_model.model.layers.0.mlp.down_proj": torch.tensor([1.0, 2.0]),
         "language_model.model.layers.0.mlp.gate_up_proj": torch.tensor([1.0, 5.0, 3.0])}
    b = {"language_model.model.layers.0.mlp.down_proj": torch.tensor([3.0, 4.0]),
         "language_model.model.layers.0.mlp.gate_up_proj": torch.tensor([2.0, 1.0, 3.0])}
    save_file(a, str(tmp_path / "rank0.safetensors"))
    save_file(b, str(tmp_path / "rank1.safetensors"))
    st = ck.load_calibration(str(tmp_path))
    assert st["model.language_model.layers.0.mlp.down_proj"].tolist() == [1.0, 2.0, 3.0, 4.0]   # K shards in order
    assert st["model.language_model.layers.0.mlp.gate_up_proj"].tolist() == [2.0, 5.0, 3.0]     # max over ranks
    assert len(st) == 2
    # the MTP draft layers' files (rank<r>_m1, module names model.layers.<i>) merge into mtp.layers.<i>
    m0 = {"model.layers.0.self_attn.o_proj": torch.tensor([7.0]), "model.layers.0.self_attn.qkv_proj": torch.tensor([1.0, 9.0])}
    m1 = {"model.layers.0.self_attn.o_proj": torch.tensor([8.0]), "model.layers.0.self_attn.qkv_proj": torch.tensor([4.0, 2.0])}
    torch.save(m0, str(tmp_path / "rank0_m1.pt"))
    torch.save(m1, str(tmp_path / "rank1_m1.pt"))
    st = ck.load_calibration(str(tmp_path))
    assert st["mtp.layers.0.self_attn.o_proj"].tolist() == [7.0, 8.0]
    assert st["mtp.layers.0.self_attn.qkv_proj"].tolist() == [4.0, 9.0]
    assert st["model.language_model.layers.0.mlp.down_proj"].tolist() == [1.0, 2.0, 3.0, 4.0]
    with pytest.raises(FileNotFoundError):
        ck.load_calibration(str(tmp_path / "missing_dir_is_not_a_file"))


def _tiny_model(d, smooth=False):
    g = torch.Generator().manual_seed(2)
    H, I = 64, 96
    P0, P1 = "model.language_model.layers.0.", "model.language_model.layers.1."
    r = lambda *s: (torch.randn(*s, generator=g) * 0.05).to(torch.bfloat16)
    t = {P0 + "self_attn.q_proj.weight": r(64, H), P0 + "self_attn.k_proj.weight": r(32, H),
         P0 + "self_attn.v_proj.weight": r(32, H), P0 + "self_attn.o_proj.weight": r(H, 64),
         P0 + "input_layernorm.weight": r(H), P0 + "post_attention_layernorm.weight": r(H),
         P0 + "mlp.gate_proj.weight": r(I, H), P0 + "mlp.up_proj.weight": r(I, H), P0 + "mlp.down_proj.weight": r(H, I),
         P1 + "linear_attn.in_proj_qkv.weight": r(96, H), P1 + "linear_attn.in_proj_z.weight": r(32, H),
         P1 + "linear_attn.in_proj_a.weight": r(4, H), P1 + "linear_attn.in_proj_b.weight": r(4, H),
         P1 + "linear_attn.out_proj.weight": r(H, 32), P1 + "linear_attn.norm.weight": r(8),
         P1 + "linear_attn.conv1d.weight": r(96, 1, 4), "lm_head.weight": r(100, H),
         "model.language_model.embed_tokens.weight": r(100, H)}
    names = sorted(t)
    from safetensors.torch import save_file
    sh = {"model-00001-of-00002.safetensors": names[:9], "model-00002-of-00002.safetensors": names[9:]}
    wm = {}
    for f, ns in sh.items():
        save_file({n: t[n] for n in ns}, os.path.join(d, f), metadata={"format": "pt"})
        wm.update({n: f for n in ns})
    json.dump({"metadata": {}, "weight_map": wm}, open(os.path.join(d, "model.safetensors.index.json"), "w"))
    json.dump({"model_type": "tiny", "text_config": {"num_attention_heads": 8, "num_key_value_heads": 4, "head_dim": 8,
                                                     "linear_num_value_heads": 4, "linear_value_head_dim": 8}},
              open(os.path.join(d, "config.json"), "w"))
    open(os.path.join(d, "tokenizer.json"), "w").write("{}")
    return t


@pytest.mark.parametrize("smooth", [False, True])
def test_convert_and_load(tmp_path, smooth):
    src, dst = tmp_path / "src", tmp_path / "dst"
    src.mkdir()
    t = _tiny_model(str(src))
    calib = None
    if smooth:
        from safetensors.torch import save_file
        g = torch.Generator().manual_seed(4)
        st = {"language_model.model.layers.0.self_attn.qkv_proj": torch.rand(64, generator=g) * 8,
              "language_model.model.layers.0.mlp.gate_up_proj": torch.rand(64, generator=g) * 8,
              "language_model.model.layers.0.mlp.down_proj": torch.rand(96, generator=g) * 8,
              "language_model.model.layers.0.self_attn.o_proj": torch.rand(64, generator=g) * 8,
              "language_model.model.layers.1.linear_attn.in_proj_qkvz": torch.rand(64, generator=g) * 8,
              "language_model.model.layers.1.linear_attn.out_proj": torch.rand(32, generator=g) * 8}
        calib = str(tmp_path / "calib.safetensors")
        save_file(st, calib)
    summary = ck.convert(str(src), str(dst), "cpu", calib, 0.5, log=lambda *a: None)
    assert summary["quantized"] == 10                                 # q k v o gate up down in_proj_qkv in_proj_z out_proj
    cfg = json.load(open(dst / "config.json"))
    assert cfg["quantization_config"] == ck.quantization_config() and cfg["model_type"] == "tiny"
    assert (dst / "tokenizer.json").exists()
    idx = json.load(open(dst / "model.safetensors.index.json"))
    from safetensors import safe_open
    got = {}
    for f in set(idx["weight_map"].values()):
        with safe_open(str(dst / f), framework="pt") as h:
            for n in h.keys():
                got[n] = h.get_tensor(n)
    assert set(got) == set(idx["weight_map"])
    for n in t:
        if ck.QUANT_PATTERN.match(n):
            assert got[n].dtype == torch.int8 and got[n + "_scale"].shape == (t[n].shape[0], 1)
            if not smooth:
                q, s = ck.quantize_per_channel(t[n])
                assert torch.equal(got[n], q) and torch.equal(got[n + "_scale"], s)
    for n in ("lm_head.weight", "model.language_model.layers.1.linear_attn.conv1d.weight",
              "model.language_model.embed_tokens.weight"):
        assert torch.equal(got[n], t[n])                              # kept as stored
    if smooth:
        # smoothed producers stored float32; a smoothed and quantized consumer dequantizes close to W * s
        assert got["model.language_model.layers.0.input_layernorm.weight"].dtype == torch.float32
        assert got["model.language_model.layers.1.linear_attn.in_proj_a.weight"].dtype == torch.float32
        assert got["model.language_model.layers.1.linear_attn.norm.weight"].dtype == torch.float32
    else:
        assert got["model.language_model.layers.0.input_layernorm.weight"].dtype == torch.bfloat16
    layers, rest = ck.load(str(dst), device="cpu")
    assert len(layers) == 10 and all(l.weight.dtype == torch.int8 for l in layers.values())
    assert "lm_head.weight" in rest and not any(k.endswith("_scale") for k in rest)
    P = "model.language_model.layers.0.self_attn."
    qkv = ck.fuse([layers[P + "q_proj"], layers[P + "k_proj"], layers[P + "v_proj"]])
    assert qkv.weight.shape == (128, 64) and qkv.weight_scale.shape == (128, 1)
    assert torch.equal(qkv.weight[64:96], layers[P + "k_proj"].weight)


def test_load_rejects_other_formats(tmp_path):
    d = tmp_path / "x"
    d.mkdir()
    _tiny_model(str(d))
    with pytest.raises(ValueError):
        ck.load(str(d), device="cpu")


def test_convert_folds_mtp_layers(tmp_path):
    """Calibration directories carry the MTP draft layers' maxima in rank<r>_m1 files: the fold reaches mtp.layers.*
    (its norm stored float32, its q / k / v quantized from the smoothed weights), exactly as a hand-applied fold."""
    from safetensors.torch import save_file
    src, dst, cal = tmp_path / "src", tmp_path / "dst", tmp_path / "calib"
    src.mkdir()
    cal.mkdir()
    t = _tiny_model(str(src))
    g = torch.Generator().manual_seed(6)
    H = 64
    P = "mtp.layers.0."
    extra = {P + "self_attn.q_proj.weight": (torch.randn(64, H, generator=g) * 0.05).to(torch.bfloat16),
             P + "self_attn.k_proj.weight": (torch.randn(32, H, generator=g) * 0.05).to(torch.bfloat16),
             P + "self_attn.v_proj.weight": (torch.randn(32, H, generator=g) * 0.05).to(torch.bfloat16),
             P + "input_layernorm.weight": (torch.randn(H, generator=g) * 0.05).to(torch.bfloat16)}
    save_file(extra, str(src / "model-mtp.safetensors"), metadata={"format": "pt"})
    idx = json.load(open(src / "model.safetensors.index.json"))
    idx["weight_map"].update({n: "model-mtp.safetensors" for n in extra})
    json.dump(idx, open(src / "model.safetensors.index.json", "w"))
    main = {"language_model.model.layers.0.mlp.down_proj": torch.rand(48, generator=g) * 8}
    save_file(main, str(cal / "rank0.safetensors"))
    save_file({"language_model.model.layers.0.mlp.down_proj": torch.rand(48, generator=g) * 8},
              str(cal / "rank1.safetensors"))
    xm = [torch.rand(H, generator=g) * 8 for _ in range(2)]
    for r in range(2):
        torch.save({"model.layers.0.self_attn.qkv_proj": xm[r]}, str(cal / f"rank{r}_m1.pt"))
    ck.convert(str(src), str(dst), "cpu", str(cal), 0.5, log=lambda *a: None)
    from safetensors import safe_open
    with safe_open(str(dst / "model-mtp.safetensors"), framework="pt") as f:
        got = {n: f.get_tensor(n) for n in f.keys()}
    x = torch.maximum(xm[0], xm[1])
    w = torch.stack([extra[P + f"self_attn.{c}_proj.weight"].float().abs().amax(0) for c in "qkv"]).amax(0)
    s = ck.smoothing_factors(x, w, 0.5)
    assert torch.equal(got[P + "input_layernorm.weight"], (1 + extra[P + "input_layernorm.weight"].float()) / s - 1)
    for c in "qkv":
        q, sc = ck.quantize_per_channel(extra[P + f"self_attn.{c}_proj.weight"].float() * s[None, :])
        assert torch.equal(got[P + f"self_attn.{c}_proj.weight"], q)
        assert torch.equal(got[P + f"self_attn.{c}_proj.weight_scale"], sc)


def test_cli(tmp_path, capsys):
    src, dst = tmp_path / "src", tmp_path / "dst"
    src.mkdir()
    _tiny_model(str(src))
    assert ck.main([str(src), str(dst), "cpu"]) == 0
    out = json.loads(capsys.readouterr().out.strip().splitlines()[-1])
    assert out["quantized"] == 10 and out["max_rel_err"] < 0.02
