"""Static K/V scale sets: the safetensors file the backend reads, calibration statistics -> scales, and
tensor-parallel slicing. Drop-in for the reference's kvq/scales.py: the same functions, arguments, file
keys and results (its interface, kvq/scales.py:1-5), built on that format description.

File format: one safetensors file holding one float32 tensor per (layer, field), under the key
"<layer name>|<field>", for the model's full set of kv heads (a TP rank slices its own rows):
  k_scale, v_scale   [num_kv_heads, D] per channel, or [num_kv_heads, 1] per head: dequantization
                     steps, x ~= code * scale, codes in -127..127
  k_mu               [num_kv_heads, D], optional: the smooth-K mean subtracted from K before it is
                     quantized
"""
import torch
from safetensors import safe_open
from safetensors.torch import save_file

SEP = "|"
FIELDS = ("k_scale", "v_scale", "k_mu")
CODE_MAX = 127.0        # codes are symmetric: -127..127
MIN_SCALE = 1e-8        # a channel that never moved still gets a usable step


def scale_of(amax):
    """Dequantization step mapping |x| <= amax onto the codes -127..127 (kvq/quant.py:50-51)."""
    return torch.clamp(amax.float() / CODE_MAX, min=MIN_SCALE)


def _quantile_over_tokens(x, frac):
    """Per (head, channel): the k-th smallest |x| over the sampled tokens, k = round(frac * tokens)
    kept within [1, tokens] (frac >= 1 gives the maximum)."""
    a = x.abs().float().flatten(1)                         # [tokens, heads * channels]
    k = min(max(int(round(frac * a.shape[0])), 1), a.shape[0])
    ordered, _ = torch.sort(a, dim=0)
    return ordered[k - 1].view(x.shape[1:])


def from_stats(st, samples=None, granularity="per_channel", method="max", smooth_k=False):
    """One layer's static scales from calibration statistics (reference kvq/scales.py:13-34).

    st: running statistics per (kv head, channel) as kvq.capture records them -- "tokens", "k_sum",
    "k_max", "k_min", "k_absmax", "v_absmax". method "max" takes the extremes seen; "q<frac>" (e.g.
    "q0.999") the frac-quantile of |x| over `samples` {"k", "v"} ([tokens, heads, D] rows).
    smooth_k: K is centred on its per-channel mean first (returned as k_mu), and its range is the
    larger distance of the extremes from that mean. granularity "per_head" keeps one step per head (the
    largest channel range)."""
    if granularity not in ("per_channel", "per_head"):
        raise ValueError(f"static scales are per_channel or per_head, not {granularity!r}")
    mu = (st["k_sum"] / st["tokens"]).float() if smooth_k else None
    if method == "max":
        k_range = st["k_absmax"].float() if mu is None else \
            torch.maximum(st["k_max"].float() - mu, mu - st["k_min"].float())
        ranges = {"k": k_range, "v": st["v_absmax"].float()}
    elif method.startswith("q"):
        frac = float(method[1:])
        centred_k = samples["k"].float() if mu is None else samples["k"].float() - mu
        ranges = {"k": _quantile_over_tokens(centred_k, frac), "v": _quantile_over_tokens(samples["v"], frac)}
    else:
        raise ValueError(f"method is 'max' or 'q<fraction>', not {method!r}")
    if granularity == "per_head":
        ranges = {side: r.amax(dim=-1, keepdim=True) for side, r in ranges.items()}
    out = {"k_scale": scale_of(ranges["k"]), "v_scale": scale_of(ranges["v"])}
    if mu is not None:
        out["k_mu"] = mu
    return out


def save(path, scales):
    """{layer name: {field: tensor}} -> one safetensors file (float32, contiguous, on the host)."""
    flat = {}
    for layer, fields in scales.items():
        for field, t in fields.items():
            if field not in FIELDS:
                raise ValueError(f"{layer}: unknown scale field {field!r} (expected one of {FIELDS})")
            flat[layer + SEP + field] = t.detach().float().contiguous().cpu()
    save_file(flat, path)


def load(path, device="cpu"):
    """safetensors file -> {layer name: {field: tensor}} (layer names may themselves contain dots, not
    the separator)."""
    out = {}
    with safe_open(path, framework="pt", device=str(device)) as f:
        for key in f.keys():
            layer, sep, field = key.rpartition(SEP)
            if not sep:
                raise ValueError(f"{path}: key {key!r} is not '<layer>{SEP}<field>'")
            out.setdefault(layer, {})[field] = f.get_tensor(key)
    return out


def kv_heads_of_rank(num_kv_heads, tp_rank, tp_size):
    """The kv heads (a range) tensor-parallel rank tp_rank of tp_size holds, as vLLM partitions them:
    an equal contiguous share when there are at least as many heads as ranks, otherwise one head,
    replicated over tp_size / num_kv_heads consecutive ranks."""
    if num_kv_heads >= tp_size:
        if num_kv_heads % tp_size:
            raise ValueError(f"{num_kv_heads} kv heads do not split over {tp_size} ranks")
        per = num_kv_heads // tp_size
        return range(tp_rank * per, (tp_rank + 1) * per)
    head = tp_rank * num_kv_heads // tp_size
    return range(head, head + 1)


def shard(t, tp_rank, tp_size):
    """Rows (kv heads) of t that TP rank tp_rank holds."""
    heads = kv_heads_of_rank(t.shape[0], tp_rank, tp_size)
    return t[heads.start:heads.stop]


def merge_tp(per_rank, num_kv_heads):
    """Calibration under tensor parallelism: each rank recorded only its own kv heads. Rebuild the
    model-wide statistics and samples by taking every head from the first rank holding it, heads in
    order (stats rows along dim 0, sample rows [tokens, heads, D] along dim 1); the token count is
    the same on every rank. per_rank: kvq.capture.collect() of each rank."""
    by_rank = {r["tp_rank"]: r for r in per_rank}
    tp = len(by_rank)
    holders = []
    for h in range(num_kv_heads):
        rank = min(rk for rk in by_rank if h in kv_heads_of_rank(num_kv_heads, rk, tp))
        if rank not in holders:
            holders.append(rank)
    parts = [by_rank[rk] for rk in holders]
    if len(parts) == 1:
        return parts[0]["stats"], parts[0]["samples"]
    stats, samples = {}, {}
    for layer, first in parts[0]["stats"].items():
        merged = {"tokens": first["tokens"]}
        for field in first:
            if field != "tokens":
                merged[field] = torch.cat([p["stats"][layer][field] for p in parts], dim=0)
        stats[layer] = merged
        samples[layer] = {side: torch.cat([p["samples"][layer][side] for p in parts], dim=1) for side in ("k", "v")}
    return stats, samples


def for_layer(all_scales, name, tp_rank, tp_size, device):
    """This TP rank's rows of one layer's scales, on `device`."""
    return {field: shard(t, tp_rank, tp_size).to(device) for field, t in all_scales[name].items()}
