"""ctypes binding of libquantpack_hip.so (the C ABI declared in include/quantpack.h).

The library is loaded after torch so that its `libamdhip64.so.7` dependency resolves to the HIP runtime torch already
loaded: device pointers and streams are then shared. There is no fallback: if the library is missing, every call
raises.
"""
from __future__ import annotations

import ctypes
import os
import struct
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


_CODES = {c_void_p: "Q", c_int64: "q", c_int32: "i", c_float: "f"}


def _scalars(struct_type, base=0):
    """(byte offset, struct code) of every scalar of a ctypes Structure, nested structures and arrays flattened, in
    field order."""
    out = []
    for name, t in struct_type._fields_:
        off = base + getattr(struct_type, name).offset
        if issubclass(t, Structure):
            out += _scalars(t, off)
        elif issubclass(t, ctypes.Array):
            out += [(off + i * ctypes.sizeof(t._type_), _CODES[t._type_]) for i in range(t._length_)]
        else:
            out.append((off, _CODES[t]))
    return out


class Packer:
    """Fills every field of a ctypes Structure in one `struct.pack_into` (about 0.1 us, against about 1 us per
    nested structure and field for ctypes' own constructor): values in field order, nested structures and arrays
    flattened, 0 for a null pointer. The format is derived from the Structure's own field offsets, so it has the
    C layout ctypes computed."""

    def __init__(self, struct_type):
        fmt, pos = "<", 0
        for off, code in _scalars(struct_type):
            if off > pos:
                fmt += f"{off - pos}x"
            fmt += code
            pos = off + struct.calcsize(code)
        size = ctypes.sizeof(struct_type)
        if size > pos:
            fmt += f"{size - pos}x"
        self._s = struct.Struct(fmt)
        if self._s.size != size:
            raise AssertionError(f"{struct_type.__name__}: packed size {self._s.size} != {size}")
        self.type = struct_type
        self.fields = len(_scalars(struct_type))

    def pack(self, dst, *values) -> None:
        self._s.pack_into(dst, 0, *values)


# Every entry point of include/quantpack.h with its ctypes signature.
SIGNATURES = {
    "qp_unpack_segment": (c_int32, [POINTER(CacheHalf), c_int32, c_int32, c_int32, c_void_p, c_int32, c_int32,
                                    c_void_p, POINTER(c_int64), c_void_p]),
    "qp_decode_splitkv": (c_int32, [POINTER(PagedCache), POINTER(DecodeArgs), c_void_p]),
    "qp_merge_segments": (c_int32, [POINTER(MergeArgs), c_void_p]),
    "qp_prefill": (c_int32, [POINTER(PagedCache), POINTER(PrefillArgs), c_void_p]),
    "qp_prefill_workspace_size": (c_int64, [POINTER(PagedCache), POINTER(PrefillArgs)]),
    "qp_prefill_i8": (c_int32, [POINTER(PagedCache), POINTER(PrefillArgs), c_void_p]),
    "qp_prefill_i8_workspace_size": (c_int64, [POINTER(PagedCache), POINTER(PrefillArgs)]),
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


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(t: torch.Tensor):
    """The current HIP stream of t's device (torch's raw-stream query when it has one: no Stream object)."""
    if _raw_stream is not None and t.is_cuda:
        return c_void_p(_raw_stream(t.get_device()))
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


_WORD_DTYPES = (torch.float32, torch.int32, torch.uint32)
_PAGED = None


def pack_paged_cache(dst: PagedCache, k_cache, v_cache, k_scale_cache, v_scale_cache, head_size: int) -> PagedCache:
    """Fill dst with the cache views' pointers, strides and sizes (the checks of cache_half / paged_cache)."""
    global _PAGED
    if _PAGED is None:
        _PAGED = Packer(PagedCache)
    if k_cache.element_size() != 1 or v_cache.element_size() != 1:
        raise ValueError(f"cache codes must be a byte view, got {k_cache.dtype} / {v_cache.dtype}")
    if v_cache.dtype == torch.int8:
        raise ValueError("value codes must be uint8 nibble pairs")
    if k_scale_cache.dtype not in _WORD_DTYPES or v_scale_cache.dtype not in _WORD_DTYPES:
        raise ValueError(f"scale words must be 4-byte elements, got {k_scale_cache.dtype} / {v_scale_cache.dtype}")
    ks, kws, vs, vws = k_cache.stride(), k_scale_cache.stride(), v_cache.stride(), v_scale_cache.stride()
    shape = k_cache.shape
    _PAGED.pack(dst, k_cache.data_ptr(), ks[0], ks[1], ks[2], k_scale_cache.data_ptr(), kws[0], kws[1], kws[2],
                CODES_INT8 if k_cache.dtype == torch.int8 else CODES_INT4,
                v_cache.data_ptr(), vs[0], vs[1], vs[2], v_scale_cache.data_ptr(), vws[0], vws[1], vws[2], CODES_INT4,
                shape[0], shape[1], shape[2], head_size)
    return dst


def paged_cache(k_cache, v_cache, k_scale_cache, v_scale_cache, head_size: int) -> PagedCache:
    return pack_paged_cache(PagedCache(), k_cache, v_cache, k_scale_cache, v_scale_cache, head_size)
