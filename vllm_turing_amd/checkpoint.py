"""compressed-tensors int-quantized W8A8 checkpoints: conversion from a bf16 safetensors model, and loading into
W8A8Linear layers (the data format on the input side of the W8A8 path).

On-disk format (the one vLLM's compressed-tensors loader reads, as the reference converter writes it:
scripts/w8a8_convert.py:51-53,165-178,209-231):
  * each quantized linear `<name>.weight` is int8 [N, K] with `<name>.weight_scale` float32 [N, 1], symmetric per
    output channel: scale = max(amax |w_row|, 1e-12) / 127, q = clamp(round_half_even(w / scale), -128, 127);
    activations are quantized per token at run time (configuration only);
  * config.json carries quantization_config (compressed-tensors, int-quantized, one config group of 8-bit symmetric
    per-channel static weights and 8-bit symmetric per-token dynamic inputs, and the ignore list);
  * the source's shard layout is kept, the index rewritten, the other files copied.
QUANT_PATTERN, IGNORE and quantization_config() are that format and stay as the reference has them.

Conversion, as this module organises it: a SourceModel reads the source shards one at a time (the model never sits in
memory whole); an optional Smoothing maps tensor names to Edits; convert_tensor turns one source tensor into the
tensors stored for it; write_shard / finish write the output.  The SmoothQuant fold (scripts/w8a8_convert.py:60-149):
for each group of linears sharing one input X (SMOOTH_GROUPS, a table of the model's structure), per input channel j,
  s_j = clamp(max(max|X_j|, 1e-5)^a / max(max|W_j|, 1e-5)^(1-a), 1e-2, 1e2),
the group's weights take W[:, j] * s_j and the producer of X absorbs 1 / s_j: a zero-centred RMSNorm weight becomes
(1 + w) / s - 1, a plain norm weight w / s, a producing linear's output rows W[j, :] / s_j.  Where one factor must
serve several channels (o_proj after GQA v heads; the GDN gated norm shared by the value heads) the maxima are pooled
over those channels first.  Smoothed tensors that stay unquantized are stored float32.  The calibration maxima come
from per-rank files (main model `rank<r>`, MTP draft layers `rank<r>_m1`); row-parallel layers' shards are
concatenated in rank order, the others reduced with max (scripts/w8a8_convert.py:71-82).

Command line: python -m vllm_turing_amd.checkpoint SRC DST [DEVICE] [--smooth CALIB] [--alpha A]
"""
import argparse
import dataclasses
import json
import os
import re
import shutil
import sys

import torch

from .linear import W8A8Linear

# ---- the on-disk format (scripts/w8a8_convert.py:51-53,209-231) -----------------------------------------------------
QUANT_PATTERN = re.compile(
    r"^(model\.language_model\.layers\.\d+\.(linear_attn\.(in_proj_qkv|in_proj_z|out_proj)"
    r"|self_attn\.(q_proj|k_proj|v_proj|o_proj)|mlp\.(gate_proj|up_proj|down_proj))"
    r"|mtp\.layers\.\d+\.(self_attn\.(q_proj|k_proj|v_proj|o_proj)|mlp\.(gate_proj|up_proj|down_proj)))\.weight$")
IGNORE = ["lm_head", "re:.*visual.*", "re:.*conv1d.*", "re:.*mtp\\.fc.*", "re:.*linear_attn\\.in_proj_(a|b)$"]


def quantization_config():
    """The quantization_config block of config.json."""
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
    return torch.round(wf / scale).clamp(-128, 127).to(torch.int8), scale


# ---- calibration maxima ------------------------------------------------------------------------------------------------
# The model's module names in the calibration files, per file tag, and the checkpoint prefix they stand for: the main
# model's decoder layers, and (tag _m1) the MTP draft layers, which the draft model names model.layers.<i>.
CALIB_TAGS = {"": ("language_model.model.layers.", "model.language_model.layers."),
              "_m1": ("model.layers.", "mtp.layers.")}
ROW_PARALLEL = ("o_proj", "down_proj", "out_proj")   # their activation maxima are K shards, one per rank


def _read_stats(path):
    if path.endswith(".safetensors"):
        from safetensors.torch import load_file
        return load_file(path)
    return torch.load(path, map_location="cpu", weights_only=True)


def _rank_files(path, tag):
    files = []
    while True:
        found = [os.path.join(path, f"rank{len(files)}{tag}{ext}") for ext in (".safetensors", ".pt")]
        found = [f for f in found if os.path.exists(f)]
        if not found:
            return files
        files.append(found[0])


def _merge_ranks(parts):
    """{module: maxima} of every rank -> one dict: row-parallel modules concatenated in rank order, others max."""
    merged = {}
    for name in parts[0]:
        vals = [p[name].float() for p in parts]
        merged[name] = torch.cat(vals) if name.rsplit(".", 1)[-1] in ROW_PARALLEL else torch.stack(vals).amax(0)
    return merged


def load_calibration(path):
    """Per-input-channel activation maxima {checkpoint module name: float32 [K]}.

    path: one file of {module name: maxima} (main-model names), or a directory of per-rank files rank<r>.pt /
    rank<r>.safetensors (main model) and rank<r>_m1.* (MTP draft layers), as the calibration hooks write them."""
    if os.path.isfile(path):
        old, new = CALIB_TAGS[""]
        return {k.replace(old, new, 1): v.float() for k, v in _read_stats(path).items()}
    stats = {}
    for tag, (old, new) in CALIB_TAGS.items():
        files = _rank_files(path, tag)
        if not files:
            if tag == "":
                raise FileNotFoundError(f"no rank<r> calibration files in {path}")
            continue
        for k, v in _merge_ranks([_read_stats(f) for f in files]).items():
            stats[k.replace(old, new, 1)] = v
    return stats


# ---- SmoothQuant -------------------------------------------------------------------------------------------------------
@dataclasses.dataclass(frozen=True)
class SmoothGroup:
    """Linears that read one activation, named relative to their decoder layer's prefix.

    module: the calibrated module whose input maxima the group uses; consumers: the weights that read that input;
    producer: the tensor that writes it; fold: how the producer absorbs 1 / s ("zero_centred_norm", "norm", "rows");
    pooling: channels that must share one factor ("none", "kv_head" for o_proj over GQA v heads, "head_dim" for the
    GDN gated norm whose weight is per dimension and shared by the value heads)."""
    module: str
    consumers: tuple
    producer: str
    fold: str
    pooling: str = "none"


SMOOTH_GROUPS = (
    SmoothGroup("self_attn.qkv_proj", ("self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight"),
                "input_layernorm.weight", "zero_centred_norm"),
    SmoothGroup("linear_attn.in_proj_qkvz", ("linear_attn.in_proj_qkv.weight", "linear_attn.in_proj_z.weight",
                                             "linear_attn.in_proj_a.weight", "linear_attn.in_proj_b.weight"),
                "input_layernorm.weight", "zero_centred_norm"),
    SmoothGroup("mlp.gate_up_proj", ("mlp.gate_proj.weight", "mlp.up_proj.weight"), "post_attention_layernorm.weight",
                "zero_centred_norm"),
    SmoothGroup("mlp.down_proj", ("mlp.down_proj.weight",), "mlp.up_proj.weight", "rows"),
    SmoothGroup("self_attn.o_proj", ("self_attn.o_proj.weight",), "self_attn.v_proj.weight", "rows", "kv_head"),
    SmoothGroup("linear_attn.out_proj", ("linear_attn.out_proj.weight",), "linear_attn.norm.weight", "norm",
                "head_dim"),
)
_GROUP_BY_MODULE = {g.module: g for g in SMOOTH_GROUPS}
_LAYER = re.compile(r"^(.*\.layers\.\d+\.)(.+)$")


def smoothing_factors(x_absmax: torch.Tensor, w_absmax: torch.Tensor, alpha: float):
    """s_j = clamp(max(x_j, 1e-5)^alpha / max(w_j, 1e-5)^(1 - alpha), 1e-2, 1e2)."""
    return (x_absmax.clamp(min=1e-5) ** alpha / w_absmax.clamp(min=1e-5) ** (1 - alpha)).clamp(1e-2, 1e2)


def _groups_in(stats):
    """(layer prefix, SmoothGroup) for every calibrated module that heads a group."""
    for key in stats:
        m = _LAYER.match(key)
        if m and m.group(2) in _GROUP_BY_MODULE:
            yield m.group(1), _GROUP_BY_MODULE[m.group(2)]


class _Heads:
    """The head geometry the pooled groups need, from the model's text config."""

    def __init__(self, text_config):
        c = text_config
        self.n_q, self.n_kv, self.hd = c.get("num_attention_heads"), c.get("num_key_value_heads"), c.get("head_dim")
        self.n_vh, self.vhd = c.get("linear_num_value_heads"), c.get("linear_value_head_dim")

    def pool(self, v, pooling):
        """Per-channel maxima -> one value per shared factor (max over the channels that share it)."""
        if pooling == "kv_head":          # o_proj input channel (q head h, d) reads v head h // (n_q / n_kv)
            return v.view(self.n_kv, self.n_q // self.n_kv, self.hd).amax(dim=1)
        if pooling == "head_dim":         # value head h, dimension d share the norm weight of d
            return v.view(self.n_vh, self.vhd).amax(dim=0)
        return v

    def spread(self, s, pooling):
        """Factors per shared slot -> (factor per consumer input column, factor per producer element)."""
        if pooling == "kv_head":
            return s.repeat_interleave(self.n_q // self.n_kv, dim=0).reshape(-1), s.reshape(-1)
        if pooling == "head_dim":
            return s.repeat(self.n_vh), s
        return s, s


@dataclasses.dataclass
class Edit:
    """What the fold does to one tensor: input columns times `cols`, output rows divided by `rows`, and for a norm
    weight division by `norm` (zero_centred: of 1 + w, minus 1 after)."""
    cols: torch.Tensor = None
    rows: torch.Tensor = None
    norm: torch.Tensor = None
    zero_centred: bool = False

    def apply(self, t, device):
        w = t.to(device, torch.float32)
        if self.cols is not None:
            w = w * self.cols.to(device)[None, :]
        if self.rows is not None:
            w = w / self.rows.to(device)[:, None]
        if self.norm is not None:
            s = self.norm.to(device)
            w = (1 + w) / s - 1 if self.zero_centred else w / s
        return w


class Smoothing:
    """The SmoothQuant fold of one model: {tensor name: Edit}."""

    def __init__(self, edits=None):
        self.edits = dict(edits or {})

    @staticmethod
    def consumers(stats):
        """Names of the weights whose per-input-channel maxima the plan needs."""
        return {prefix + c for prefix, g in _groups_in(stats) for c in g.consumers}

    @classmethod
    def plan(cls, stats, weight_colmax, text_config, alpha):
        """stats: {module: input maxima}; weight_colmax: {consumer weight name: max |W| per input channel} (absent
        consumers are skipped); text_config: the model's head geometry."""
        heads = _Heads(text_config)
        edits = {}

        def edit(name):
            return edits.setdefault(name, Edit())

        for prefix, g in _groups_in(stats):
            present = [prefix + c for c in g.consumers if prefix + c in weight_colmax]
            if not present:
                continue
            w = torch.stack([weight_colmax[c] for c in present]).amax(dim=0)
            s = smoothing_factors(heads.pool(stats[prefix + g.module].float(), g.pooling), heads.pool(w, g.pooling),
                                  alpha)
            s_cols, s_prod = heads.spread(s, g.pooling)
            for c in present:
                edit(c).cols = s_cols
            if g.fold == "rows":
                edit(prefix + g.producer).rows = s_prod
            else:
                e = edit(prefix + g.producer)
                e.norm, e.zero_centred = s_prod, g.fold == "zero_centred_norm"
        return cls(edits)

    def apply(self, name, t, device="cpu"):
        """The smoothed float32 tensor, or None when the fold leaves `name` as it is."""
        e = self.edits.get(name)
        return None if e is None else e.apply(t, device)


# ---- conversion --------------------------------------------------------------------------------------------------------
class SourceModel:
    """A safetensors model directory: its index, shards and config, read one shard at a time."""

    def __init__(self, path):
        self.path = path
        self.index = json.load(open(os.path.join(path, "model.safetensors.index.json")))
        self.shards = sorted(set(self.index["weight_map"].values()))
        self.config = json.load(open(os.path.join(path, "config.json")))

    def tensors(self, shard):
        from safetensors import safe_open
        with safe_open(os.path.join(self.path, shard), framework="pt") as f:
            for name in f.keys():
                yield name, f.get_tensor(name)

    def column_maxima(self, names, device):
        """{name: max |W| over the output rows, per input column} for the named 2-D weights present."""
        out = {}
        for shard in self.shards:
            for name, t in self.tensors(shard):
                if name in names:
                    out[name] = t.to(device, torch.float32).abs().amax(dim=0).cpu()
        return out

    def other_files(self):
        skip = {"model.safetensors.index.json", "config.json"}
        for fn in sorted(os.listdir(self.path)):
            p = os.path.join(self.path, fn)
            if os.path.isfile(p) and not fn.startswith(".") and not fn.endswith(".safetensors") and fn not in skip:
                yield fn, p


@dataclasses.dataclass
class Report:
    quantized: int = 0
    max_rel_err: float = 0.0
    sum_rel_err: float = 0.0
    bytes: int = 0

    def note(self, q, scale, w):
        e = ((q.float() * scale - w).norm() / w.norm().clamp(min=1e-12)).item()
        self.quantized += 1
        self.max_rel_err = max(self.max_rel_err, e)
        self.sum_rel_err += e

    def summary(self):
        return {"quantized": self.quantized, "max_rel_err": self.max_rel_err,
                "mean_rel_err": self.sum_rel_err / max(self.quantized, 1), "bytes": self.bytes}


def convert_tensor(name, t, smoothing, device, report):
    """The tensors stored for one source tensor: int8 weight + scale for a quantized linear, the smoothed float32
    tensor for a folded one, else the tensor as stored."""
    folded = smoothing.apply(name, t, device)
    if QUANT_PATTERN.match(name):
        if t.dim() != 2:
            raise ValueError(f"{name}: a quantized linear must be 2-D, got {tuple(t.shape)}")
        w = folded if folded is not None else t.to(device, torch.float32)
        q, scale = quantize_per_channel(w)
        report.note(q, scale, w)
        return {name: q.cpu(), name + "_scale": scale.cpu()}
    return {name: folded.cpu() if folded is not None else t}


def convert(src, dst, device=None, calib=None, alpha=0.5, log=print):
    """Convert the bf16 safetensors model in `src` into a W8A8 int-quantized checkpoint in `dst`, one shard at a
    time; calib: calibration file or directory for the SmoothQuant fold (None: no fold).  Returns a summary dict."""
    from safetensors.torch import save_file

    device = device or ("cuda" if torch.cuda.is_available() else "cpu")
    source = SourceModel(src)
    smoothing = Smoothing()
    if calib is not None:
        stats = load_calibration(calib)
        colmax = source.column_maxima(Smoothing.consumers(stats), device)
        smoothing = Smoothing.plan(stats, colmax, source.config.get("text_config", source.config), alpha)
        log(f"SmoothQuant fold, alpha {alpha}: {len(smoothing.edits)} tensors change")
    os.makedirs(dst, exist_ok=True)
    report, weight_map = Report(), {}
    for i, shard in enumerate(source.shards):
        stored = {}
        for name, t in source.tensors(shard):
            stored.update(convert_tensor(name, t, smoothing, device, report))
        save_file(stored, os.path.join(dst, shard), metadata={"format": "pt"})
        for name, t in stored.items():
            weight_map[name] = shard
            report.bytes += t.numel() * t.element_size()
        log(f"shard {i + 1} of {len(source.shards)} ({shard}) written; {report.quantized} linears quantized, worst "
            f"relative error {report.max_rel_err:.4f}")
    with open(os.path.join(dst, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {"total_size": report.bytes}, "weight_map": weight_map}, f, indent=2)
    for fn, p in source.other_files():
        shutil.copy2(p, os.path.join(dst, fn))
    cfg = dict(source.config, quantization_config=quantization_config())
    with open(os.path.join(dst, "config.json"), "w") as f:
        json.dump(cfg, f, indent=2)
    return report.summary()


# ---- loading -----------------------------------------------------------------------------------------------------------
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
    wmap = json.load(open(os.path.join(ckpt_dir, "model.safetensors.index.json")))["weight_map"]
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
            if sn in raw:
                scale = raw[sn]
            else:
                with safe_open(os.path.join(ckpt_dir, wmap[sn]), framework="pt") as f:
                    scale = f.get_tensor(sn)
            if _ignored(n, qc.get("ignore", [])):
                raise ValueError(f"{n} is int8 but matches the ignore list")
            layers[n[:-len(".weight")]] = W8A8Linear(t.to(device), scale.to(device))
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
    ap = argparse.ArgumentParser(prog="python -m vllm_turing_amd.checkpoint",
                                 description="bf16 safetensors model -> compressed-tensors W8A8 int-quantized checkpoint")
    ap.add_argument("src")
    ap.add_argument("dst")
    ap.add_argument("device", nargs="?", default=None, help="torch device for the conversion (default: a GPU if any)")
    ap.add_argument("--smooth", metavar="CALIB", default=None,
                    help="calibration file or directory of rank<r>[_m1] files: apply the SmoothQuant fold")
    ap.add_argument("--alpha", type=float, default=0.5, help="SmoothQuant migration strength (default 0.5)")
    a = ap.parse_args(argv)
    print(json.dumps(convert(a.src, a.dst, a.device, a.smooth, a.alpha)))
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
