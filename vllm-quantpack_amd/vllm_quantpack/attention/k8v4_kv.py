"""k8v4_per_token_head KV cache: int8 keys and int4 values, served by the HIP kernels of this package.

Same format as the reference (k8v4_kv.py:1-24): per (token, KV head) the key is int8 with one fp32 scale and the
value is stored as int4_per_token_head stores it (nibble pairs, fp32 scale with the 4-bit zero point in its low
mantissa bits), both in the randomized-Hadamard domain. Page cell, head size hs:
[K hs int8 | K scale f32 | V hs/2 bytes | V scale f32] = 1.5 hs + 8 bytes (392 at hs 256; int4 264).

The read path is the same split-KV decode / MFMA prefill as the int4 cache with the key half read as int8; the store
is `qp_store` with an int8 key half.
"""
from __future__ import annotations

import dataclasses

import torch

from .. import _hip
from . import rht
from .vllm_hooks import HOOKS, Hook, find

NAME = "k8v4_per_token_head"
SCALE_BYTES = 4


def cell_bytes(head_size: int, head_size_v: int) -> int:
    """Bytes of one (token, KV head) cell: int8 key, packed value, one fp32 scale each (k8v4_kv.py:31-33)."""
    return head_size + head_size_v // 2 + 2 * SCALE_BYTES


def is_k8v4(key_cache: torch.Tensor) -> bool:
    """True for the key view of a k8v4 cache: int8, where int4 cache views are uint8 (k8v4_kv.py:36-38)."""
    return key_cache.dtype == torch.int8


def _scale_view(kv_cache: torch.Tensor, byte_at: int) -> torch.Tensor:
    nblocks, nkv, block_size, _ = kv_cache.shape
    st = kv_cache.stride()
    base = torch.tensor([], dtype=torch.float32, device=kv_cache.device).set_(kv_cache.untyped_storage())
    return torch.as_strided(base, (nblocks, block_size, nkv), (st[0] // 4, st[2] // 4, st[1] // 4),
                            (kv_cache.storage_offset() + byte_at) // 4)


def views(kv_cache: torch.Tensor, head_size: int, head_size_v: int | None = None):
    """(key, value, key scale, value scale) views of the logical (blocks, KV heads, block size, cell) byte cache:
    key (blocks, bs, nkv, hs) int8, value (..., hs_v / 2) uint8, scales (blocks, bs, nkv) fp32 over the same storage.
    Only the cache's strides are used, so a physically NHD cache works too. ValueError for a cell of the wrong size
    or scales that are not 4-byte aligned (k8v4_kv.py:41-65)."""
    head_size_v = head_size if head_size_v is None else head_size_v
    _, _, _, cell = kv_cache.shape
    if kv_cache.element_size() != 1 or cell != cell_bytes(head_size, head_size_v):
        raise ValueError(f"{NAME}: cache cell of {cell} x {kv_cache.element_size()} bytes, expected "
                         f"{cell_bytes(head_size, head_size_v)} for head sizes {head_size} / {head_size_v}")
    st = kv_cache.stride()
    if any(s % 4 for s in st[:3]) or kv_cache.storage_offset() % 4 or head_size % 4 or (head_size_v // 2) % 4:
        raise ValueError(f"{NAME}: fp32 scales are not 4-byte aligned (strides {tuple(st)}, head {head_size})")
    v_at = head_size + SCALE_BYTES
    t = kv_cache.transpose(1, 2)
    key = t[..., :head_size].view(torch.int8)
    value = t[..., v_at:v_at + head_size_v // 2].view(torch.uint8)
    return key, value, _scale_view(kv_cache, head_size), _scale_view(kv_cache, v_at + head_size_v // 2)


def int4_views(kv_cache: torch.Tensor, head_size: int):
    """(key, value, key scale, value scale) views of an int4_per_token_head byte cache (blocks, nkv, bs, hs + 8):
    [K nibbles hs/2 | K word | V nibbles hs/2 | V word] per cell, the views vLLM hands the backend
    (tests/test_int4_kv.py:95-103)."""
    phs = head_size // 2 + SCALE_BYTES
    if kv_cache.element_size() != 1 or kv_cache.shape[3] != 2 * phs:
        raise ValueError(f"int4_per_token_head: cache cell of {kv_cache.shape[3]} bytes, expected {2 * phs}")
    kc, vc = kv_cache.view(torch.uint8).transpose(1, 2).split(phs, dim=-1)
    return kc, vc, _scale_view(kv_cache, head_size // 2), _scale_view(kv_cache, phs + head_size // 2)


def store(stock, key, value, key_cache, value_cache, slot_mapping, *, k_scale_cache, v_scale_cache,
          rotate: bool = True):
    """Rotate (RHT, as the int4 cache), quantise and write key / value into the cache views: int8 keys when
    key_cache is int8 (k8v4), int4 otherwise; values int4. `slot_mapping[i] < 0` skips token i.
    Replaces k8v4_kv.store + _store_k8v4 (k8v4_kv.py:68-86, k8v4_ops.py:11-63). `stock` is accepted for call
    compatibility and not used: the rotation is this package's own (rht.py)."""
    del stock
    num_tokens, nkv, head_size = key.shape
    if value.shape != key.shape:
        raise ValueError(f"{NAME}: key {tuple(key.shape)} and value {tuple(value.shape)} differ")
    if key.dtype != torch.bfloat16 or value.dtype != torch.bfloat16:
        key, value = key.to(torch.bfloat16), value.to(torch.bfloat16)
    if key.stride(-1) != 1:
        key = key.contiguous()
    if value.stride(-1) != 1:
        value = value.contiguous()
    slots = slot_mapping.to(torch.int64) if slot_mapping.dtype != torch.int64 else slot_mapping
    cache = _hip.paged_cache(key_cache, value_cache, k_scale_cache, v_scale_cache, head_size)
    args = _hip.StoreArgs(key.data_ptr(), _hip.I64x2(key.stride(0), key.stride(1)), value.data_ptr(),
                          _hip.I64x2(value.stride(0), value.stride(1)), slots.data_ptr(), num_tokens,
                          rht.signs(head_size, key.device).data_ptr() if rotate else None)
    _hip.check(_hip.lib().qp_store(cache, args, _hip.stream_of(key)), "reshape_and_cache_int4")


def dtype_handler(int4_mode):
    """The dtype registry's entry for k8v4: int8 storage (the int4 cache is uint8, which is how a spec or a cache view
    tells the two formats apart where vLLM passes no dtype string) and the int4 per-token-head quantisation mode, so
    that vLLM's per-token-head code paths (dynamic scales, the Triton backend, the packed dispatch) serve it."""
    return type("K8v4Dtype", (), {"name": NAME, "torch_dtype": lambda self: torch.int8,
                                  "quant_mode": lambda self: int4_mode})


def register_dtype(logger) -> bool:
    """Make `--kv-cache-dtype k8v4_per_token_head` a valid vLLM option through its KV-cache dtype registry
    (k8v4_kv.py:89-110). False on a vLLM without the registry."""
    try:
        _, register, lookup = find("vllm.config.cache", "register_kv_cache_dtype", "get_kv_cache_dtype_handler")
        _, int4_mode = find("vllm.v1.kv_cache_interface", "KVQuantMode.INT4_PER_TOKEN_HEAD")
    except Exception as e:
        logger.debug("vllm-quantpack: no KV-cache dtype registry for %s (%s)", NAME, e)
        return False
    if lookup(NAME) is None:
        register(NAME)(dtype_handler(int4_mode))
    return True


def backend_hooks(triton_attn, int4_mode) -> list:
    """The Triton backend's knowledge of the k8v4 cell: the spec's cell size, and the key / value / scale views the
    attention implementation takes from a layer's byte cache (k8v4_kv.py:113-166). Every other cache dtype is left
    to vLLM's own methods."""
    backend, impl = triton_attn.TritonAttentionBackend, triton_attn.TritonAttentionImpl
    vllm_spec = backend.customize_spec.__func__
    vllm_scales, vllm_views = impl._ensure_scale_caches, impl._pth_key_value_caches

    def k8v4_spec(spec) -> bool:
        return spec.state_content_bytes is None and spec.kv_quant_mode == int4_mode and spec.dtype == torch.int8

    def customize_spec(cls, spec):
        if not k8v4_spec(spec):
            return vllm_spec(cls, spec)
        return dataclasses.replace(spec, state_content_bytes=cell_bytes(spec.head_size, spec.head_size_v))

    def k8v4_views(self, kv_cache):
        """(key, value) views of a k8v4 layer cache; its two scale views go to the layer on first use, every scale
        at 1.0 as vLLM starts per-token-head scales."""
        key, value, k_scales, v_scales = views(kv_cache, self.head_size)
        if self._k_scale_cache is None:
            k_scales.fill_(1.0)
            v_scales.fill_(1.0)
            self._k_scale_cache, self._v_scale_cache = k_scales, v_scales
        return key, value

    def _ensure_scale_caches(self, kv_cache):
        if self.kv_cache_dtype != NAME:
            return vllm_scales(self, kv_cache)
        k8v4_views(self, kv_cache)

    def _pth_key_value_caches(self, kv_cache):
        return k8v4_views(self, kv_cache) if self.kv_cache_dtype == NAME else vllm_views(self, kv_cache)

    dtypes = list(backend.supported_kv_cache_dtypes)
    return [Hook(backend, "customize_spec", classmethod(customize_spec), "k8v4 cell size in the attention spec"),
            Hook(impl, "_ensure_scale_caches", _ensure_scale_caches, "k8v4 scale views"),
            Hook(impl, "_pth_key_value_caches", _pth_key_value_caches, "k8v4 key / value views"),
            Hook(backend, "supported_kv_cache_dtypes", dtypes + [NAME] if NAME not in dtypes else dtypes,
                 "k8v4 among the backend's cache dtypes")]


def patch_backend(stock, logger) -> bool:
    """Install backend_hooks into vLLM's Triton backend. The store and the attention themselves are attached by
    int4_kv.patch_int4_kv (the reference installs its k8v4 store here, k8v4_kv.py:145-166; `stock` is accepted for
    that call signature). False on a vLLM without the backend methods or the int4 quantisation mode."""
    del stock
    try:
        triton_attn, _, _, _ = find("vllm.v1.attention.backends.triton_attn", "TritonAttentionBackend.customize_spec",
                                    "TritonAttentionImpl._ensure_scale_caches",
                                    "TritonAttentionImpl._pth_key_value_caches")
        _, int4_mode = find("vllm.v1.kv_cache_interface", "KVQuantMode.INT4_PER_TOKEN_HEAD")
        hooks = backend_hooks(triton_attn, int4_mode)
    except Exception as e:
        logger.warning("vllm-quantpack: %s not available on this vLLM (%s)", NAME, e)
        return False
    for hook in hooks:
        HOOKS.apply(hook)
    return True
