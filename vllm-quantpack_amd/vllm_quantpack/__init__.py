"""vllm-quantpack for MI355X: the int4_per_token_head / k8v4_per_token_head KV-cache attention of vllm-quantpack,
re-implemented as hand-written gfx950 HIP kernels behind the plugin's attention-backend API.

Layout:
  attention/  the drop-in Python boundary (int4_kv, int4_prefill, k8v4_kv, rht) over the HIP library
  _hip.py     ctypes binding of libquantpack_hip.so (C ABI: include/quantpack.h)
  tools/      synthetic paged caches for the benchmark and the parity tests

Only the KV-attention part of the reference plugin is here; its EXL3 quantisation, model families and TurboQuant
patches are not.
"""
__version__ = "0.1.0"


def register():
    """vLLM general-plugin entry point: installs the HIP int4 / k8v4 KV attention (reference __init__.py:31-65,
    attention part only)."""
    from vllm.logger import init_logger

    from .attention.int4_kv import patch_int4_kv
    patch_int4_kv(init_logger("vllm.quantpack"))
