"""Static KV scales: the safetensors file format and its TP slicing (reference kvq/scales.py).

File format: keys "<layer_name>|k_scale", "<layer_name>|v_scale" and optional "<layer_name>|k_mu",
each float32 [num_kv_heads_total, D] (per channel) or [num_kv_heads_total, 1] (per head); k_mu is
[num_kv_heads_total, D]. Scales are dequantization steps (x ~= code * scale).
"""
import torch
from safetensors.torch import load_file, save_file

QMAX = 127.0


def from_stats(st, samples=None, granularity="per_channel", method="max", smooth_k=False):
    """One layer's static scales from calibration stats (reference kvq/scales.py:13-34).

    st: {"tokens", "k_sum", "k_max", "k_min", "k_absmax", "v_absmax"} per (head, channel);
    method "max" or "q<quantile>" (then `samples` {"k", "v"} [T, H, D] rows are used);
    granularity "per_channel" or "per_head"; smooth_k subtracts the per-channel mean of K."""
    out = {}
    mu = None
    if smooth_k:
        mu = (st["k_sum"] / st["tokens"]).float()
        out["k_mu"] = mu
    for side in ("k", "v"):
        if side == "k" and mu is not None:
            amax = torch.maximum(st["k_max"] - mu, mu - st["k_min"])
        else:
            amax = st[f"{side}_absmax"].float()
        if method != "max":
            frac = float(method[1:])
            x = samples[side].float()
            if side == "k" and mu is not None:
                x = x - mu
            a = x.abs().reshape(x.shape[0], -1)
            k = max(1, min(a.shape[0], int(round(frac * a.shape[0]))))
            amax = a.kthvalue(k, dim=0).values.reshape(x.shape[1:])
        if granularity == "per_head":
            amax = amax.amax(-1, keepdim=True)
        out[f"{side}_scale"] = torch.clamp(amax / QMAX, min=1e-8)
    return out


def save(path, scales):
    """scales: {layer_name: {"k_scale", "v_scale"[, "k_mu"]}} -> one safetensors file."""
    save_file({f"{name}|{k}": v.contiguous().float() for name, d in scales.items() for k, v in d.items()}, path)


def load(path, device="cpu"):
    """safetensors file -> {layer_name: {field: tensor}}."""
    out = {}
    for key, t in load_file(path, device=device).items():
        name, field = key.split("|")
        out.setdefault(name, {})[field] = t
    return out


def shard(t, tp_rank, tp_size):
    """The kv-head rows of one TP rank; with fewer kv heads than ranks each head is replicated."""
    h = t.shape[0]
    if h >= tp_size:
        assert h % tp_size == 0, (h, tp_size)
        n = h // tp_size
        return t[tp_rank * n:(tp_rank + 1) * n]
    i = tp_rank * h // tp_size
    return t[i:i + 1]


def merge_tp(per_rank, num_kv_heads):
    """Calibration under TP: concatenate each rank's stats / samples along heads in rank order,
    keeping one replica per head when heads < ranks (reference kvq/scales.py:59-75)."""
    ranks = sorted(per_rank, key=lambda r: r["tp_rank"])
    tp = len(ranks)
    if tp > num_kv_heads:
        ranks = ranks[:: tp // num_kv_heads]
    if len(ranks) == 1:
        return ranks[0]["stats"], ranks[0]["samples"]
    stats, samples = {}, {}
    for name in ranks[0]["stats"]:
        parts = [r["stats"][name] for r in ranks]
        stats[name] = {"tokens": parts[0]["tokens"],
                       **{k: torch.cat([p[k] for p in parts], dim=0) for k in parts[0] if k != "tokens"}}
        samples[name] = {side: torch.cat([r["samples"][name][side] for r in ranks], dim=1) for side in "kv"}
    return stats, samples


def for_layer(all_scales, name, tp_rank, tp_size, device):
    """This rank's slice of one layer's scales, on `device`."""
    return {k: shard(v, tp_rank, tp_size).to(device) for k, v in all_scales[name].items()}
