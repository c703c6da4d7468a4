"""Writes tests/golden/golden.safetensors + golden.json from the REFERENCE's own Python numerics.

Run in the build container only (the reference is not on the GPU box and never leaves it):
    python tests/golden/make_golden.py [/root/reference]
It imports the reference's kvq.quant, kvq.ref_attn and kvq.int8_ref (pure PyTorch, CPU) to produce,
for each case of tests/golden/cases.py:
  <case>|int8_b    (rows of cases.stored_rows) paged_static_attention(Cfg(smooth_k=True, p_tile=32[, per-head]), cache_is_int8=True,
                   short_q=8) output (bf16)  -- kvq/int8_ref.py:162-197, as tests/test_cuda_kernels.py:12-17
  <case>|int8_b_qgroup32  (cases.WITH_QGROUP32) the same with Cfg(..., q_gran="group32")  -- kvq/int8_ref.py:120-129
  <case>|bf16_ref  paged_attention_ref on the original bf16 K/V (bf16)     -- kvq/ref_attn.py:88-90
  codes sha256     of the int8 caches quant.quantize(k - mu, s_k), quant.quantize(v, s_v)  -- kvq/quant.py:50-51
  quant|codes      quant.quantize on the corner-case inputs of cases.quant_special()
These pin the functions no closed form fixes exactly: run_paged's batching and masking, and
implementation B's op order / P tiling / denominator.
"""
import hashlib
import json
import os
import sys

import torch
from safetensors.torch import save_file

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
import cases  # noqa: E402

REF = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
sys.path.insert(0, REF)
from kvq import int8_ref as ref_int8  # noqa: E402  (the reference's modules)
from kvq import quant as ref_quant  # noqa: E402
from kvq import ref_attn as ref_attn  # noqa: E402


def sha(t):
    return hashlib.sha256(t.contiguous().numpy().tobytes()).hexdigest()


def main():
    torch.set_num_threads(min(8, os.cpu_count() or 1))
    tensors, meta = {}, {"reference": "ischencheng/int8-kvcache (kvq/quant.py, kvq/ref_attn.py, kvq/int8_ref.py)",
                         "cases": {}}
    for name in cases.NAMES:
        c = cases.build(name)
        st = c["static"]
        kq = ref_quant.quantize(c["k"].float() - st["k_mu"], st["k_scale"])
        vq = ref_quant.quantize(c["v"], st["v_scale"])
        smooth = bool(st["k_mu"].abs().max() > 0)   # (an INT8 cache already holds k - mu: B does not read it)
        if c["per_channel"]:
            cfg = ref_int8.Cfg(smooth_k=smooth, p_tile=32)
        else:
            cfg = ref_int8.Cfg(smooth_k=smooth, p_tile=32, k_gran="per_head", v_gran="per_head")
        args = (c["cu"], c["seq_lens"], c["block_table"])
        b = ref_int8.paged_static_attention(cfg, st, cache_is_int8=True, short_q=8)(c["q"], kq, vq, *args, c["scale"])
        g = ref_attn.paged_attention_ref(c["q"], c["k"], c["v"], *args, c["scale"]) if name in cases.WITH_BF16_REF else None
        rows = cases.stored_rows(name, c["cu"])
        tensors[f"{name}|int8_b"] = b[rows].contiguous()
        if name in cases.WITH_QGROUP32:
            cfg_g = ref_int8.Cfg(smooth_k=True, p_tile=32, q_gran="group32")
            bg = ref_int8.paged_static_attention(cfg_g, st, cache_is_int8=True, short_q=8)(c["q"], kq, vq, *args,
                                                                                          c["scale"])
            tensors[f"{name}|int8_b_qgroup32"] = bg[rows].contiguous()
        if name in cases.WITH_BF16_REF:
            tensors[f"{name}|bf16_ref"] = g[rows].contiguous()
        meta["cases"][name] = {"k_codes_sha256": sha(kq), "v_codes_sha256": sha(vq),
                               "q_sha256": sha(c["q"].view(torch.int16)), "shape": list(c["q"].shape)}
        print(name, tuple(b.shape), flush=True)
    x, s = cases.quant_special()
    tensors["quant|codes"] = ref_quant.quantize(x, s)
    dq = ref_quant.dequantize(tensors["quant|codes"], s, torch.bfloat16)
    tensors["quant|dequant_bf16"] = dq
    save_file(tensors, os.path.join(HERE, "golden.safetensors"))
    with open(os.path.join(HERE, "golden.json"), "w") as f:
        json.dump(meta, f, indent=1)
    print("wrote", len(tensors), "tensors")


if __name__ == "__main__":
    main()
