"""ctypes binding of libquantpack_hip.so (the C ABI declared in include/quantpack.h).

The library is loaded after torch so that its `libamdhip64.so.7` dependency resolves to the HIP runtime torch already
loaded: device pointers and streams are then shared. There is no fallback: if the library is missing, every call
raises.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, Structure, c_char_p, c_float, c_int32, c_int64, c_void_p

import torch  # noqa: F401  (must be loaded first: see module docstring)

LIB_PATH = os.environ.get("QUANTPACK_HIP_LIB") or os.path.join(os.path.dirname(os.path.abspath(__file__)),
                                                                 "libquantpack_hip.so")

QP_OK, QP_ERR_INVALID, QP_ERR_UNSUPPORTED = 0, -1, -2
CODES_INT4, CODES_INT8 = 0, 1
DTYPE_BF16, DTYPE_F32 = 0, 1
DECODE_TILE = 32          # QP_DECODE_TILE: split-KV segments are multiples of this many keys
DECODE_MAX_QUERY = 4      # QP_DECODE_MAX_QUERY

I64x3 = c_int64 * 3
I64x2 = c_int64 * 2


class CacheHalf(Structure):
    _fields_ = [("codes", c_void_p), ("code_stride", I64x3), ("words", c_void_p), ("word_stride", I64x3),
                ("format", c_int32)]


class PagedCache(Structure):
    _fields_ = [("key", CacheHalf), ("value", CacheHalf), ("num_blocks", c_int32), ("block_size", c_int32),
                ("num_kv_heads", c_int32), ("head_size", c_int32)]


class DecodeArgs(Structure):
    _fields_ = [("query", c_void_p), ("query_stride", I64x2), ("cu_seqlens_q", c_void_p), ("seqused_k", c_void_p),
                ("block_table", c_void_p), ("block_table_stride", c_int64), ("num_seqs", c_int32),
                ("num_tokens", c_int32), ("num_q_heads", c_int32), ("max_query_len", c_int32),
                ("num_segments", c_int32), ("softmax_scale", c_float), ("segm_output", c_void_p),
                ("segm_output_stride", I64x3), ("segm_max", c_void_p), ("segm_expsum", c_void_p),
                ("segm_stat_stride", I64x2), ("segm_rows", c_int32), ("query_signs", c_void_p)]


class MergeArgs(Structure):
    _fields_ = [("segm_output", c_void_p), ("segm_output_stride", I64x3), ("segm_max", c_void_p),
                ("segm_expsum", c_void_p), ("segm_stat_stride", I64x2), ("cu_seqlens_q", c_void_p),
                ("seqused_k", c_void_p), ("num_seqs", c_int32), ("num_tokens", c_int32), ("num_q_heads", c_int32),
                ("head_size", c_int32), ("num_segments", c_int32), ("out", c_void_p), ("out_stride", I64x2),
                ("lse", c_void_p), ("lse_stride", I64x2), ("rht_signs", c_void_p), ("rht_out_scale", c_float)]


class PrefillArgs(Structure):
    _fields_ = [("query", c_void_p), ("query_stride", I64x2), ("cu_seqlens_q", c_void_p), ("seqused_k", c_void_p),
                ("block_table", c_void_p), ("block_table_stride", c_int64), ("num_seqs", c_int32),
                ("num_tokens", c_int32), ("num_q_heads", c_int32), ("max_query_len", c_int32),
                ("max_seqlen_k", c_int32), ("num_splits", c_int32), ("softmax_scale", c_float), ("out", c_void_p),
                ("out_stride", I64x2), ("workspace", c_void_p), ("workspace_bytes", c_int64),
                ("rht_signs", c_void_p), ("rht_out_scale", c_float), ("query_signs", c_void_p)]


class AttentionArgs(Structure):
    _fields_ = [("query", c_void_p), ("query_stride", I64x2), ("cu_seqlens_q", c_void_p), ("seqused_k", c_void_p),
                ("block_table", c_void_p), ("block_table_stride", c_int64), ("num_seqs", c_int32),
                ("num_tokens", c_int32), ("num_q_heads", c_int32), ("max_query_len", c_int32),
                ("max_seqlen_k", c_int32), ("softmax_scale", c_float), ("out", c_void_p), ("out_stride", I64x2),
                ("segm_output", c_void_p), ("segm_output_stride", I64x3), ("segm_max", c_void_p),
                ("segm_expsum", c_void_p), ("segm_stat_stride", I64x2), ("segm_rows", c_int32),
                ("num_segments", c_int32), ("max_decode_rows", c_int32), ("rht_signs", c_void_p),
                ("rht_out_scale", c_float),
                ("workspace", c_void_p), ("workspace_bytes", c_int64)]


class StoreArgs(Structure):
    _fields_ = [("key", c_void_p), ("key_stride", I64x2), ("value", c_void_p), ("value_stride", I64x2),
                ("slot_mapping", c_void_p), ("num_tokens", c_int32), ("rht_signs", c_void_p)]


# Every entry point of include/quantpack.h with its ctypes signature.
SIGNATURES = {
    "qp_unpack_segment": (c_int32, [POINTER(CacheHalf), c_int32, c_int32, c_int32, c_void_p, c_int32, c_int32,
                                    c_void_p, POINTER(c_int64), c_void_p]),
    "qp_decode_splitkv": (c_int32, [POINTER(PagedCache), POINTER(DecodeArgs), c_void_p]),
    "qp_merge_segments": (c_int32, [POINTER(MergeArgs), c_void_p]),
    "qp_prefill": (c_int32, [POINTER(PagedCache), POINTER(PrefillArgs), c_void_p]),
    "qp_prefill_workspace_size": (c_int64, [POINTER(PagedCache), POINTER(PrefillArgs)]),
    "qp_attention": (c_int32, [POINTER(PagedCache), POINTER(AttentionArgs), c_void_p]),
    "qp_attention_workspace_size": (c_int64, [POINTER(PagedCache), POINTER(AttentionArgs)]),
    "qp_attention_noalloc": (c_int32, [POINTER(PagedCache), POINTER(AttentionArgs), c_void_p]),
    "qp_store": (c_int32, [POINTER(PagedCache), POINTER(StoreArgs), c_void_p]),
    "qp_rht": (c_int32, [c_void_p, c_int32, c_int64, c_void_p, c_int32, c_int64, c_int64, c_int32, c_void_p,
                         c_int32, c_float, c_void_p]),
    "qp_last_error": (c_char_p, []),
    "qp_version": (c_char_p, []),
}

_lib = None


class HipLibraryMissing(RuntimeError):
    pass


def lib():
    """The loaded library; raises HipLibraryMissing when it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise HipLibraryMissing(f"{LIB_PATH} is missing: build it with `python vllm-quantpack_amd/build.py` "
                                    "(this package has no CPU or Triton fallback)")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def check(status: int, what: str) -> None:
    if status == QP_OK:
        return
    msg = lib().qp_last_error().decode()
    if status == QP_ERR_INVALID:
        raise ValueError(f"{what}: {msg}")
    if status == QP_ERR_UNSUPPORTED:
        raise NotImplementedError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: HIP error {status}: {msg}")


def stream_of(t: torch.Tensor):
    return c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def ptr(t):
    return None if t is None else c_void_p(t.data_ptr())


def cache_half(codes: torch.Tensor, words: torch.Tensor) -> CacheHalf:
    """A (blocks, bs, nkv, bytes) code view (uint8 nibble pairs or int8) and its (blocks, bs, nkv) fp32 word view."""
    if codes.element_size() != 1:
        raise ValueError(f"cache codes must be a byte view, got {codes.dtype}")
    if words.dtype not in (torch.float32, torch.int32, torch.uint32):
        raise ValueError(f"scale words must be 4-byte elements, got {words.dtype}")
    fmt = CODES_INT8 if codes.dtype == torch.int8 else CODES_INT4
    return CacheHalf(codes.data_ptr(), I64x3(*codes.stride()[:3]), words.data_ptr(), I64x3(*words.stride()[:3]),
                     fmt)


def paged_cache(k_cache, v_cache, k_scale_cache, v_scale_cache, head_size: int) -> PagedCache:
    if v_cache.dtype == torch.int8:
        raise ValueError("value codes must be uint8 nibble pairs")
    return PagedCache(cache_half(k_cache, k_scale_cache), cache_half(v_cache, v_scale_cache), k_cache.shape[0],
                      k_cache.shape[1], k_cache.shape[2], head_size)
