"""Test stand-in for the parts of vLLM 0.32 that the kvq backend, plugin and capture touch (vLLM is not
installed in this image). It models interfaces only: class names, constructor arguments, the metadata
fields the backend reads, and the backend registry. Used by tests/test_vllm_backend.py and
tests/test_gpu_vllm_backend.py, never by the package."""
