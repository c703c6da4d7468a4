"""vLLM general-plugin entry point (reference kvq/vllm_plugin.py:9-25).

Install this package where vLLM's workers import from, with an entry point in the
"vllm.general_plugins" group pointing at `kvq.vllm_plugin:register`, e.g. in a pyproject:

    [project.entry-points."vllm.general_plugins"]
    kvq = "kvq.vllm_plugin:register"

vLLM calls register() in every process it starts, before the model is built: it registers the static
INT8 backend as AttentionBackendEnum.CUSTOM (by class path, so the backend module is imported only
when vLLM selects it), warns when the installed vLLM does not know kv_cache_dtype="int8_static" yet
(kvq.vllm_dtype registers it) and, with KVQ_CAPTURE=1, wraps the bf16 attention backend to record the K/V
statistics that calibration turns into static scales (kvq.capture).
"""
import os


def register():
    from vllm.v1.attention.backends.registry import AttentionBackendEnum, register_backend

    register_backend(AttentionBackendEnum.CUSTOM, "kvq.vllm_int8.backend.Int8StaticBackend")
    from kvq import vllm_dtype

    missing = vllm_dtype.missing_tables()
    if missing:  # vLLM would reject kv_cache_dtype="int8_static" before asking any backend
        from vllm.logger import init_logger

        init_logger(__name__).warning(
            "kv_cache_dtype int8_static is not registered in this vLLM (%s); run `python -m kvq.vllm_dtype` once",
            ", ".join(missing))
    if os.environ.get("KVQ_CAPTURE") == "1":
        from kvq import capture

        capture.install()
    for var, what in (("KVQ_ATTN", "the attention-override study backend"), ("KVQ_MLA", "the MLA study path")):
        if os.environ.get(var):
            raise RuntimeError(f"{var} selects {what} of the reference repository, which this package does not "
                               f"provide (it holds the static INT8 KV-cache path only); unset {var}")
