"""KVQ_DEBUG_DUMP: the long-query path's attention call, saved for an offline replay.

The reference saves the metadata of its last FlashAttention call (kvq/cuda_kernels.py:123-127) and
replays it with random tensors of the same shapes (scripts/replay_fa_call.py) -- the tool that located
its mixed-batch memory fault (docs/WALKTHROUGH.md:357-370). Here the long path's consumer is the HIP
prefill kernel, so a dump holds what that call reads: the query start offsets and the device key counts,
the temporary cache's block table and page sources, the work list, and the shapes and strides of q, out
and the temporary cache.

    dump_long_call(path, ...)   called by cuda_kernels.long_attention while KVQ_DEBUG_DUMP=path
    load(path)                  the dump (torch.load with weights_only=True: tensors and plain values)
    check(d)                    host-side bounds report of a dump: the reads the call would make
    replay(d, seed)             the same call on random tensors of the dumped shapes, on the GPU
"""
import torch

FIELDS = ("cu_seqlens_q", "seq_lens", "block_table", "src_req", "src_j", "tile_req", "tile_row")


def dump_long_call(path, q, out, cu_seqlens_q, seq_lens, plan, kt, tile_req, tile_row, max_query_len, rows_per_tile,
                   softmax_scale):
    """Save the prefill call of one long_attention step (synchronises the device: a debugging aid). kt: the
    temporary cache or its shape (with KVQ_PREFILL_DIRECT=1 none is made; the replay runs the two-kernel
    consumer on a temporary cache of that shape)."""
    src_req, src_j, bt = (torch.as_tensor(x) for x in (plan.src_req, plan.src_j, plan.block_table))
    d = {"cu_seqlens_q": cu_seqlens_q.cpu(), "seq_lens": seq_lens.cpu()[:cu_seqlens_q.shape[0] - 1].clone(),
         "block_table": bt.cpu(), "src_req": src_req.cpu(), "src_j": src_j.cpu(), "tile_req": tile_req.cpu(),
         "tile_row": tile_row.cpu(), "max_seqlen_q": int(max_query_len), "max_seqlen_k": int(plan.max_seqlen_k),
         "q_shape": tuple(q.shape), "q_stride": tuple(q.stride()), "out_shape": tuple(out.shape),
         "out_stride": tuple(out.stride()), "kt_shape": tuple(getattr(kt, "shape", kt)), "block_size": int(plan.block_size),
         "rows_per_tile": int(rows_per_tile), "softmax_scale": float(softmax_scale)}
    torch.save(d, path)
    return d


def load(path):
    return torch.load(path, weights_only=True)


def check(d):
    """Every read the prefill call would make, checked on the host: a list of problems (empty if none).
    For each work-list entry (request r, first row r0): its rows lie in r's query rows; r's key count is at
    least its query count; the keys it reads, [0, seq_lens[r]), lie on pages of r's row of the block table,
    and those entries are pages of the temporary cache that were copied from request r, in order."""
    errs = []
    cu, sl, bt = d["cu_seqlens_q"].long(), d["seq_lens"].long(), d["block_table"].long()
    src_req, src_j = d["src_req"].long(), d["src_j"].long()
    T, hq, _ = d["q_shape"]
    P, bs, hkv, _ = d["kt_shape"]
    G = hq // hkv
    n = cu.numel() - 1
    ql = cu[1:] - cu[:-1]
    if int(cu[-1]) > T:
        errs.append(f"cu_seqlens_q[-1] {int(cu[-1])} > {T} query rows")
    if src_req.numel() != P or src_j.numel() != P:
        errs.append(f"{src_req.numel()} page sources for {P} temporary pages")
    for r, r0 in zip(d["tile_req"].long().tolist(), d["tile_row"].long().tolist()):
        if not 0 <= r < n:
            errs.append(f"work entry for request {r} of {n}")
            continue
        if not 0 <= r0 < int(ql[r]) * G:
            errs.append(f"req {r}: work rows from {r0}, request has {int(ql[r]) * G} rows")
        L = int(sl[r])
        if L < int(ql[r]):
            errs.append(f"req {r}: {L} keys < {int(ql[r])} query tokens")
        pages = -(-L // bs)
        if pages > bt.shape[1]:
            errs.append(f"req {r}: {pages} pages > block table width {bt.shape[1]}")
            continue
        ids = bt[r, :pages]
        if pages and (int(ids.min()) < 0 or int(ids.max()) >= P):
            errs.append(f"req {r}: temporary page ids outside [0, {P})")
            continue
        if pages and not (bool((src_req[ids] == r).all()) and torch.equal(src_j[ids], torch.arange(pages))):
            errs.append(f"req {r}: its table row points at pages copied from other requests or out of order")
    return errs


def replay(d, seed=0, device="cuda"):
    """Run the dumped prefill call on random q / temporary K and V of the dumped shapes and strides, on the
    GPU. Returns (q, kt, vt, out): out holds the rows the work list covers, NaN elsewhere."""
    from . import cuda_kernels as ck

    g = torch.Generator(device=device).manual_seed(seed)
    T, hq, D = d["q_shape"]
    qs, os_ = d["q_stride"], d["out_stride"]
    q = torch.randn(T * qs[0], generator=g, device=device).to(torch.bfloat16).as_strided((T, hq, D), qs)
    out = torch.full((T * os_[0],), float("nan"), dtype=torch.bfloat16, device=device).as_strided((T, hq, D), os_)
    kt = torch.randn(d["kt_shape"], generator=g, device=device).to(torch.bfloat16)
    vt = torch.randn(d["kt_shape"], generator=g, device=device).to(torch.bfloat16)
    idx = {k: d[k].to(device=device, dtype=torch.int32) for k in FIELDS}
    ck.ext().paged_prefill_attention(q, kt, vt, out, idx["cu_seqlens_q"], idx["seq_lens"], idx["block_table"],
                                     idx["tile_req"], idx["tile_row"], d["softmax_scale"])
    return q, kt, vt, out
