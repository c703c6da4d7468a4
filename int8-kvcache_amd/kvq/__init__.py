"""Static INT8 KV cache for vLLM on MI355X (gfx950): drop-in for the reference's `kvq` package.

  kvq.cuda_kernels   operator API (same names as the reference), HIP kernels via a C ABI
  kvq.scales         static-scale safetensors format: load / save / shard / merge_tp / for_layer
  kvq.synth          seeded synthetic workloads of the benchmark configurations
"""
