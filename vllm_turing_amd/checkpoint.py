"""compressed-tensors int-quantized W8A8 checkpoints: conversion from a bf16 safetensors model and loading into
W8A8Linear layers (the data format on the input side of the W8A8 path).

The format and the conversion arithmetic are the reference converter's (scripts/w8a8_convert.py), which vLLM's
compressed-tensors loader reads:
  * every quantized linear `<name>.weight` becomes int8 [N, K] plus `<name>.weight_scale` float32 [N, 1], symmetric
    per output channel: scale = max(amax(|w_row|), 1e-12) / 127, q = clamp(round_half_even(w / scale), -128, 127)
    (:165-178); activations are quantized per token at run time (config only);
  * config.json gains quantization_config {quant_method compressed-tensors, format int-quantized, config_groups.group_0
    (8-bit symmetric per-channel static weights, 8-bit symmetric per-token dynamic inputs), ignore list} (:209-231);
  * shards keep the source's layout; model.safetensors.index.json is rewritten; other files are copied (:199-206);
  * optional SmoothQuant fold (:60-149): per group of linears sharing one input X, per input channel j,
    s_j = clamp(max|X_j|^a / max|W_j|^(1-a), 1e-2, 1e2); consumers get W[:, j] * s_j; the producer of X absorbs 1 / s_j
    (zero-centred RMSNorm weight (1 + w) / s - 1, plain norm weight w / s, or the rows of the producing linear / s);
    changed unquantized tensors are stored float32.
Which tensors are quantized, which stay as stored, and the calibration-file merge rule are the reference's, kept
alike because they define the checkpoint a vLLM deployment of the reference loads.

Command line: python -m vllm_turing_amd.checkpoint <src dir> <dst dir> [device] [--smooth <calibration file or dir>]
[--alpha a].  Conversion runs with torch on `device` (a GPU by default when one is present, else the CPU).
"""
import json
import os
import re
import shutil
import sys

import torch

from .linear import W8A8Linear

# the linears that become int8 (scripts/w8a8_convert.py:55-57)
QUANT_PATTERN = re.compile(
    r"^(model\.language_model\.layers\.\d+\.(linear_attn\.(in_proj_qkv|in_proj_z|out_proj)"
    r"|self_attn\.(q_proj|k_proj|v_proj|o_proj)|mlp\.(gate_proj|up_proj|down_proj))"
    r"|mtp\.layers\.\d+\.(self_attn\.(q_proj|k_proj|v_proj|o_proj)|mlp\.(gate_proj|up_proj|down_proj)))\.weight$")
# kept as stored (scripts/w8a8_convert.py:224-226)
IGNORE = ["lm_head", "re:.*visual.*", "re:.*conv1d.*", "re:.*mtp\\.fc.*", "re:.*linear_attn\\.in_proj_(a|b)$"]
ROW_PARALLEL = ("o_proj", "down_proj", "out_proj")      # calibration stats of these are K shards in rank order


def quantization_config():
    """The quantization_config block written into config.json (scripts/w8a8_convert.py:209-231)."""
    return {
        "quant_method": "compressed-tensors",
        "format": "int-quantized",
        "quantization_status": "compressed",
        "config_groups": {
            "group_0": {
                "targets": ["Linear"],
                "weights": {"num_bits": 8, "type": "int", "symmetric": True, "strategy": "channel", "dynamic": False,
                            "group_size": None, "observer": "minmax"},
                "input_activations": {"num_bits": 8, "type": "int", "symmetric": True, "strategy": "token",
                                      "dynamic": True, "observer": None},
                "output_activations": None,
                "format": "int-quantized",
            }
        },
        "ignore": list(IGNORE),
        "kv_cache_scheme": None,
        "sparsity_config": {},
        "global_compression_ratio": None,
    }


def quantize_per_channel(w: torch.Tensor):
    """float weight [N, K] -> (int8 [N, K], float32 scale [N, 1]): symmetric per output channel."""
    wf = w.to(torch.float32)
    scale = wf.abs().amax(dim=1, keepdim=True).clamp(min=1e-12) / 127.0
    q = torch.round(wf / scale).clamp(-128, 127).to(torch.int8)
    return q, scale


def smoothing_factors(x_absmax: torch.Tensor, w_absmax: torch.Tensor, alpha: float):
    """s_j = clamp(max|X_j|^alpha / max|W_j|^(1 - alpha), 1e-2, 1e2) (both maxima floored at 1e-5)."""
    return (x_absmax.clamp(min=1e-5) ** alpha / w_absmax.clamp(min=1e-5) ** (1 - alpha)).clamp(1e-2, 1e2)


def _load_stats_file(path):
    if path.endswith(".safetensors"):
        from safetensors.torch import load_file
        return load_file(path)
    return torch.load(path, map_location="cpu", weights_only=True)


def _checkpoint_name(module_name, tag):
    """vLLM module name -> checkpoint tensor prefix (scripts/w8a8_convert.py:76-77): the language model's layers, or
    for a draft-model file (tag "_m1") the MTP layers."""
    if tag:
        return module_name.replace("model.layers.", "mtp.layers.", 1)
    return module_name.replace("language_model.model.layers.", "model.language_model.layers.", 1)


def load_calibration(path, tag=""):
    """Per-input-channel activation maxima {checkpoint module name: float32 [K]}.  `path` is one file ({name:
    tensor}) or a directory of per-rank files rank<r><tag>.pt / .safetensors as the reference's calibration hooks
    write them (vllm_turing/calib.py), merged as its converter does: row-parallel layers' K shards concatenated in rank
    order, the others reduced with max.  Module names are mapped to checkpoint names."""
    if os.path.isfile(path):
        return {_checkpoint_name(k, tag): v.float() for k, v in _load_stats_file(path).items()}
    parts, r = [], 0
    while True:
        f = next((os.path.join(path, f"rank{r}{tag}{ext}") for ext in (".safetensors", ".pt")
                  if os.path.exists(os.path.join(path, f"rank{r}{tag}{ext}"))), None)
        if f is None:
            break
        parts.append(_load_stats_file(f))
        r += 1
    if not parts:
        raise FileNotFoundError(f"no rank<r>{tag} calibration files in {path}")
    out = {}
    for k in parts[0]:
        if k.rsplit(".", 1)[1] in ROW_PARALLEL:
            v = torch.cat([p[k] for p in parts]).float()
        else:
            v = torch.stack([p[k].float() for p in parts]).amax(dim=0)
        out[_checkpoint_name(k, tag)] = v
    return out


def smoothing_groups(stats):
    """(stats key, consumer weight names, producer tensor name, producer kind, reduction) per linear group sharing one
    input (scripts/w8a8_convert.py:85-101): the stats keys are module names …layers.<i>.self_attn.qkv_proj,
    …mlp.gate_up_proj, …mlp.down_proj, …self_attn.o_proj, …linear_attn.in_proj_qkvz, …linear_attn.out_proj."""
    groups = []
    for k in stats:
        p, role = k.rsplit(".", 1)
        blk = p.rsplit(".", 1)[0] + "."
        if role == "qkv_proj":
            groups.append((k, [f"{p}.{c}.weight" for c in ("q_proj", "k_proj", "v_proj")],
                           blk + "input_layernorm.weight", "zc", None))
        elif role == "in_proj_qkvz":
            groups.append((k, [f"{p}.{c}.weight" for c in ("in_proj_qkv", "in_proj_z", "in_proj_a", "in_proj_b")],
                           blk + "input_layernorm.weight", "zc", None))
        elif role == "gate_up_proj":
            groups.append((k, [f"{p}.gate_proj.weight", f"{p}.up_proj.weight"],
                           blk + "post_attention_layernorm.weight", "zc", None))
        elif role == "down_proj":
            groups.append((k, [f"{p}.down_proj.weight"], f"{p}.up_proj.weight", "rows", None))
        elif role == "o_proj":
            groups.append((k, [f"{p}.o_proj.weight"], f"{p}.v_proj.weight", "rows", "gqa"))
        elif role == "out_proj":
            groups.append((k, [f"{p}.out_proj.weight"], f"{p}.norm.weight", "plain", "heads"))
    return groups


def smoothing_plan(stats, weight_absmax, text_config, alpha):
    """(col_scale, row_scale, norm_fix): tensor name -> s for consumer columns (*), producer rows (/), producer norm
    weights ((s, "zc" | "plain")).  weight_absmax maps consumer weight names to their per-input-channel max |W|."""
    n_q, n_kv, hd = (text_config.get(k) for k in ("num_attention_heads", "num_key_value_heads", "head_dim"))
    n_vh, vhd = text_config.get("linear_num_value_heads"), text_config.get("linear_value_head_dim")
    col_scale, row_scale, norm_fix = {}, {}, {}
    for k, cons, prod, kind, red in smoothing_groups(stats):
        cons = [c for c in cons if c in weight_absmax]
        if not cons:
            continue
        w = torch.stack([weight_absmax[c] for c in cons]).amax(dim=0)
        x = stats[k].float()
        if red == "gqa":        # o_proj input channel h * hd + d belongs to v head h // (n_q / n_kv)
            x = x.view(n_kv, n_q // n_kv, hd).amax(dim=1)
            w = w.view(n_kv, n_q // n_kv, hd).amax(dim=1)
        elif red == "heads":    # the gated norm's weight is per dimension, shared by all value heads
            x = x.view(n_vh, vhd).amax(dim=0)
            w = w.view(n_vh, vhd).amax(dim=0)
        s = smoothing_factors(x, w, alpha)
        if red == "gqa":
            s_cols, s_prod = s.repeat_interleave(n_q // n_kv, dim=0).flatten(), s.flatten()
        elif red == "heads":
            s_cols, s_prod = s.repeat(n_vh), s
        else:
            s_cols = s_prod = s
        for c in cons:
            col_scale[c] = s_cols
        if kind == "rows":
            row_scale[prod] = s_prod
        else:
            norm_fix[prod] = (s_prod, kind)
    return col_scale, row_scale, norm_fix


def apply_smoothing(name, t, plan, device="cpu"):
    """The smoothed float32 tensor, or None if the plan leaves `name` untouched."""
    col_scale, row_scale, norm_fix = plan
    if name not in col_scale and name not in row_scale and name not in norm_fix:
        return None
    w = t.to(device, torch.float32)
    if name in col_scale:
        w = w * col_scale[name].to(device)[None, :]
    if name in row_scale:
        w = w / row_scale[name].to(device)[:, None]
    if name in norm_fix:
        s, kind = norm_fix[name]
        s = s.to(device)
        w = (1 + w) / s - 1 if kind == "zc" else w / s
    return w


def convert(src, dst, device=None, calib=None, alpha=0.5, log=print):
    """Convert the bf16 safetensors model in `src` into a W8A8 int-quantized checkpoint in `dst`, one shard at a
    time.  calib: calibration file / directory for the SmoothQuant fold (None: no smoothing).  Returns a summary."""
    from safetensors import safe_open
    from safetensors.torch import save_file

    if device is None:
        device = "cuda" if torch.cuda.is_available() else "cpu"
    os.makedirs(dst, exist_ok=True)
    index = json.load(open(os.path.join(src, "model.safetensors.index.json")))
    shards = sorted(set(index["weight_map"].values()))
    cfg = json.load(open(os.path.join(src, "config.json")))
    plan = ({}, {}, {})
    if calib is not None:
        stats = load_calibration(calib)
        tc = cfg.get("text_config", cfg)
        need = {c for g in smoothing_groups(stats) for c in g[1]}
        wmax = {}
        for shard in shards:
            with safe_open(os.path.join(src, shard), framework="pt") as f:
                for name in f.keys():
                    if name in need:
                        wmax[name] = f.get_tensor(name).to(device, torch.float32).abs().amax(dim=0).cpu()
        plan = smoothing_plan(stats, wmax, tc, alpha)
        log(f"smoothing (alpha {alpha}): {len(plan[0])} consumer weights")
    new_map, total, nq, err_max = {}, 0, 0, 0.0
    for si, shard in enumerate(shards):
        out = {}
        with safe_open(os.path.join(src, shard), framework="pt") as f:
            for name in f.keys():
                t = f.get_tensor(name)
                ts = apply_smoothing(name, t, plan, device)
                if QUANT_PATTERN.match(name):
                    if t.dim() != 2:
                        raise ValueError(f"{name}: a quantized linear must be 2-D, got {tuple(t.shape)}")
                    w = ts if ts is not None else t.to(device, torch.float32)
                    q, scale = quantize_per_channel(w)
                    e = ((q.float() * scale - w).norm() / w.norm().clamp(min=1e-12)).item()
                    err_max, nq = max(err_max, e), nq + 1
                    out[name] = q.cpu()
                    out[name + "_scale"] = scale.cpu()
                elif ts is not None:
                    out[name] = ts.cpu()
                else:
                    out[name] = t
        for name, t in out.items():
            new_map[name] = shard
            total += t.numel() * t.element_size()
        save_file(out, os.path.join(dst, shard), metadata={"format": "pt"})
        log(f"[{si + 1}/{len(shards)}] {shard}: {len(out)} tensors, {nq} quantized so far, max rel err {err_max:.4f}")
    json.dump({"metadata": {"total_size": total}, "weight_map": new_map},
              open(os.path.join(dst, "model.safetensors.index.json"), "w"), indent=2)
    for fn in os.listdir(src):
        if fn.endswith(".safetensors") or fn in ("model.safetensors.index.json", "config.json") or fn.startswith("."):
            continue
        p = os.path.join(src, fn)
        if os.path.isfile(p):
            shutil.copy2(p, os.path.join(dst, fn))
    cfg["quantization_config"] = quantization_config()
    json.dump(cfg, open(os.path.join(dst, "config.json"), "w"), indent=2)
    return {"quantized": nq, "max_rel_err": err_max, "bytes": total}


def _ignored(name, ignore):
    base = name[:-len(".weight")] if name.endswith(".weight") else name
    for pat in ignore:
        if pat.startswith("re:"):
            if re.match(pat[3:], base):
                return True
        elif base == pat or base.endswith("." + pat) or base.startswith(pat + "."):
            return True
    return False


def load(ckpt_dir, device="cuda", names=None):
    """Read a W8A8 int-quantized checkpoint: {linear name: W8A8Linear} for every `<name>.weight` int8 tensor with its
    `<name>.weight_scale`, and {tensor name: tensor} for everything else.  names: optional iterable of tensor names to
    read (default: all).  Raises if config.json is not an int-quantized compressed-tensors W8A8 configuration."""
    from safetensors import safe_open

    cfg = json.load(open(os.path.join(ckpt_dir, "config.json")))
    qc = cfg.get("quantization_config") or {}
    if qc.get("quant_method") != "compressed-tensors" or qc.get("format") != "int-quantized":
        raise ValueError(f"{ckpt_dir}: not an int-quantized compressed-tensors checkpoint")
    g0 = next(iter(qc["config_groups"].values()))
    wq, aq = g0["weights"], g0["input_activations"]
    if not (wq["num_bits"] == 8 and wq["type"] == "int" and wq["symmetric"] and wq["strategy"] == "channel" and aq
            and aq["num_bits"] == 8 and aq["strategy"] == "token" and aq["dynamic"]):
        raise ValueError(f"{ckpt_dir}: config group is not W8A8 per-channel / per-token dynamic")
    index = json.load(open(os.path.join(ckpt_dir, "model.safetensors.index.json")))
    wmap = index["weight_map"]
    want = set(wmap) if names is None else set(names)
    by_shard = {}
    for n in want:
        by_shard.setdefault(wmap[n], []).append(n)
    raw = {}
    for shard, ns in by_shard.items():
        with safe_open(os.path.join(ckpt_dir, shard), framework="pt") as f:
            for n in ns:
                raw[n] = f.get_tensor(n)
    layers, rest = {}, {}
    for n, t in raw.items():
        if n.endswith(".weight") and t.dtype == torch.int8:
            sn = n + "_scale"
            if sn not in raw:
                with safe_open(os.path.join(ckpt_dir, wmap[sn]), framework="pt") as f:
                    raw_scale = f.get_tensor(sn)
            else:
                raw_scale = raw[sn]
            if _ignored(n, qc.get("ignore", [])):
                raise ValueError(f"{n} is int8 but matches the ignore list")
            layers[n[:-len(".weight")]] = W8A8Linear(t.to(device), raw_scale.to(device))
        elif not n.endswith(".weight_scale"):
            rest[n] = t.to(device)
    return layers, rest


def fuse(layers):
    """One W8A8Linear of stacked output channels (vLLM's qkv_proj / gate_up_proj packing): the int8 weights and
    their per-channel scales concatenated along N, in the given order."""
    w = torch.cat([l.weight for l in layers], dim=0)
    s = torch.cat([l.weight_scale for l in layers], dim=0)
    return W8A8Linear(w, s)


def main(argv):
    args = list(argv)
    calib, alpha = None, 0.5
    if "--smooth" in args:
        i = args.index("--smooth")
        calib = args[i + 1]
        del args[i:i + 2]
    if "--alpha" in args:
        i = args.index("--alpha")
        alpha = float(args[i + 1])
        del args[i:i + 2]
    if len(args) < 2:
        print(__doc__)
        return 2
    summary = convert(args[0], args[1], args[2] if len(args) > 2 else None, calib, alpha)
    print(json.dumps(summary))
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
