"""int4_per_token_head / k8v4_per_token_head KV-cache attention on MI355X, behind vLLM's Triton-backend API.

The reference fixes vLLM's Triton kernel by text edits and routes long prefills to FlashAttention (int4_kv.py:1-29).
This package replaces the whole read path with hand-written gfx950 kernels reached through libquantpack_hip.so:

* one library call per attention layer (`qp_attention`): the randomized Hadamard rotation of the queries happens as
  the kernels load them, a route table written on the device sends each sequence of 1..4 query tokens (decode / MTP
  verify) to the split-KV kernel and every other sequence to the batched MFMA prefill kernel, and the output is
  rotated back inside the merge or the prefill epilogue before its single bf16 store;
* the split-KV kernel holds every query row of a GQA group per workgroup (the cache is read once per step), and a
  log-sum-exp merge finishes it;
* the store (`reshape_and_cache_int4`) rotates, quantises and scatters new tokens, int4 or int8 keys.

The arithmetic is the reference's exact kernel: bf16 query and exact-integer nibble operands, fp32 accumulation, and
the value zero point removed with the same bf16-rounded P * s_v that feeds the PV product (int4_kv.py:80-95).
Nothing here copies to or waits for the host; a batch of short sequences allocates nothing either, so decode steps
can be captured in HIP graphs.
"""
from __future__ import annotations

import contextlib
import os
import threading

import torch

from .. import _hip
from . import int4_prefill, k8v4_kv, rht
from .rht import single_rht  # noqa: F401  (re-exported: the stock module's name)
from .vllm_hooks import HOOKS, Hook, find, module_value

MODULE = "vllm.v1.attention.ops.int4_per_token_head"
PACKED_DTYPES = ("int4_per_token_head", "k8v4_per_token_head")
MAX_Q_SPLIT_KV = _hip.DECODE_MAX_QUERY       # MTP / EAGLE verification with up to 3 draft tokens
# The reference's Triton tile tables (int4_kv.py:42-56), kept with their override formats. The HIP kernels have
# fixed tiles; of the decode setting, the segment count sizes the split-KV buffers and the optional fourth value caps
# the query rows one split-KV workgroup holds (16: one row tile, tokens beyond it read the segment again).
PREFILL_TILES_BY_MAJOR = {8: (64, 64, 8, 2), 12: (64, 64, 8, 2)}
PREFILL_TILES_DEFAULT = (64, 64, 8, 2)
DECODE_TILES_DEFAULT = (64, 4, "auto")
DECODE_MAX_M = 64
MIN_SEGMENTS, MAX_SEGMENTS = 16, 128
MAX_DECODE_ROWS = 32                          # query rows (tokens x GQA heads) one split-KV workgroup holds
RHT_HEAD_SIZES = (64, 128, 256, 512)          # sign vectors made when the package is installed


def prefill_tiles(major):
    """(BLOCK_M, TILE, warps, stages) from VLLM_QUANTPACK_INT4_TILES or the table (int4_kv.py:59-63)."""
    env = os.environ.get("VLLM_QUANTPACK_INT4_TILES")
    if env:
        return tuple(int(x) for x in env.split(","))
    return PREFILL_TILES_BY_MAJOR.get(major, PREFILL_TILES_DEFAULT)


def segments_for(sms):
    """Split-KV segments per sequence for a GPU with `sms` compute units: next power of two of sms / 4, clamped to
    [16, 128] (int4_kv.py:66-69). MI355X (256 CUs): 64, i.e. 4 KV heads x 64 segments = one workgroup per CU."""
    n = 1 << max(0, -(-sms // 4) - 1).bit_length()
    return min(MAX_SEGMENTS, max(MIN_SEGMENTS, n))


def decode_segments(requested, num_seqs, num_kv_heads, sms):
    """Segments per (sequence, KV head) the split-KV decode actually uses: the caller's count (the capacity of its
    segment buffers), lowered for batches so that one launch holds about 8 workgroups per CU. Longer segments stream
    more keys per workgroup: the 32-request ragged k8v4 batch runs 232 us at 16 segments against 331 us at 64, while a
    single sequence keeps all 64 (4 KV heads x 64 = one workgroup per CU). Any count gives the same result up to fp32
    rounding (the merge takes the same count)."""
    want = -(-8 * max(1, sms) // max(1, num_seqs * num_kv_heads))
    return max(1, min(int(requested), want))


def decode_tiles(sms):
    """(tile, warps, segments[, rows]) from VLLM_QUANTPACK_INT4_DECODE="tile,warps,segments|auto[,rows]" or the
    default (int4_kv.py:72-77)."""
    env = os.environ.get("VLLM_QUANTPACK_INT4_DECODE")
    tile, warps, segments, *max_m = env.split(",") if env else DECODE_TILES_DEFAULT
    segments = segments_for(sms) if str(segments).strip() == "auto" else int(segments)
    return (int(tile), int(warps), segments) + tuple(int(m) for m in max_m[:1])


_ROW_CAP: dict = {}


def decode_row_cap(sms) -> int:
    """The query-row cap of VLLM_QUANTPACK_INT4_DECODE's optional fourth value (DECODE_MAX_M by default), as the
    library takes it: 16 keeps one row tile per split-KV workgroup, anything from 32 up allows two. Parsed once per
    value of the variable."""
    key = (os.environ.get("VLLM_QUANTPACK_INT4_DECODE"), sms)
    cap = _ROW_CAP.get(key)
    if cap is None:
        tiles = decode_tiles(sms)
        rows = tiles[3] if len(tiles) > 3 else DECODE_MAX_M
        cap = _ROW_CAP[key] = 16 if rows < 32 else MAX_DECODE_ROWS
    return cap


_CUS: dict = {}


def _device_cus(t: torch.Tensor) -> int:
    """Compute units of the GPU that holds t."""
    idx = t.get_device()
    cus = _CUS.get(idx)
    if cus is None:
        cus = _CUS[idx] = torch.cuda.get_device_properties(idx).multi_processor_count
    return cus


def _plain(q, window_size, softcap, sinks, alibi_slopes, qq_bias, output_scale, mm_prefix_range):
    unsupported = [name for name, bad in (
        ("sliding window", window_size is not None and window_size[0] >= 0),
        ("softcap", bool(softcap)), ("sinks", sinks is not None), ("ALiBi", alibi_slopes is not None),
        ("qq_bias", qq_bias is not None), ("fp8 output_scale", output_scale is not None),
        ("mm_prefix_range", mm_prefix_range is not None)) if bad]
    if unsupported:
        raise NotImplementedError("int4 KV attention (HIP): " + ", ".join(unsupported) + " not supported")


def _check_batch(q, cu_seqlens_q, seqused_k, block_table):
    """The tensors the kernels index: bf16 queries with contiguous channels, int32 index tensors (host-side checks
    only; nothing is copied)."""
    if q.dtype != torch.bfloat16:
        raise NotImplementedError(f"int4 KV attention (HIP): bf16 queries only, got {q.dtype}")
    if q.stride(-1) != 1:
        raise ValueError("int4 KV attention: query channels must be contiguous")
    for name, t in (("cu_seqlens_q", cu_seqlens_q), ("seqused_k", seqused_k), ("block_table", block_table)):
        if t.dtype != torch.int32:
            raise ValueError(f"int4 KV attention: {name} must be int32, got {t.dtype}")


_ATTENTION = _hip.Packer(_hip.AttentionArgs)
_NO_SEGMENTS = (0,) * 10
_TLS = threading.local()


def _pack_attention(dst, q, out, *, cu_seqlens_q, seqused_k, block_table, max_seqlen_q, max_seqlen_k, softmax_scale,
                    num_segments=0, softmax_segm_output=None, softmax_segm_max=None, softmax_segm_expsum=None,
                    rht_signs=None, rht_out_scale=1.0, max_decode_rows=0):
    so, sm, ss = softmax_segm_output, softmax_segm_max, softmax_segm_expsum
    if so is None or sm is None or ss is None:
        segm = _NO_SEGMENTS
    else:
        st = sm.stride()
        if st != ss.stride() or st[2] != 1:
            raise ValueError("segment max / expsum buffers must share strides with contiguous segments")
        sost = so.stride()
        segm = (so.data_ptr(), sost[0], sost[1], sost[2], sm.data_ptr(), ss.data_ptr(), st[0], st[1], so.shape[0],
                int(num_segments))
    qs, ost = q.stride(), out.stride()
    _ATTENTION.pack(dst, q.data_ptr(), qs[0], qs[1], cu_seqlens_q.data_ptr(), seqused_k.data_ptr(),
                    block_table.data_ptr(), block_table.stride(0), seqused_k.shape[0], q.shape[0], q.shape[1],
                    int(max_seqlen_q), int(min(max_seqlen_k, 2**31 - 1)), float(softmax_scale), out.data_ptr(), ost[0],
                    ost[1], *segm, int(max_decode_rows), 0 if rht_signs is None else rht_signs.data_ptr(),
                    float(rht_out_scale), 0, 0)
    return dst


def attention_args(q, out, **kw) -> _hip.AttentionArgs:
    """The qp_attention arguments of one call (no workspace yet). q and out bf16 [T, NQ, hs]; keywords: cu_seqlens_q,
    seqused_k, block_table, max_seqlen_q, max_seqlen_k, softmax_scale, and optionally num_segments with the three
    segment buffers softmax_segm_output / _max / _expsum, rht_signs with rht_out_scale, max_decode_rows."""
    return _pack_attention(_hip.AttentionArgs(), q, out, **kw)


def _scratch():
    """This thread's argument structs for attend (the library reads them during the call only)."""
    s = getattr(_TLS, "structs", None)
    if s is None:
        s = _TLS.structs = (_hip.PagedCache(), _hip.AttentionArgs())
    return s


def attend(q, k_cache, v_cache, k_scale_cache, v_scale_cache, out, **kw) -> None:
    """One qp_attention call (see attention_args for the keywords): the library routes the batch between split-KV
    decode and prefill on the device. A workspace is taken from torch's caching allocator only when the batch has
    sequences of more than 4 query tokens (a batch of short sequences needs none)."""
    cache, args = _scratch()
    _hip.pack_paged_cache(cache, k_cache, v_cache, k_scale_cache, v_scale_cache, q.shape[2])
    _pack_attention(args, q, out, **kw)
    lib = _hip.lib()
    need = lib.qp_attention_workspace_size(cache, args)
    if need > 0:
        ws = torch.empty(need, dtype=torch.uint8, device=q.device)
        args.workspace = ws.data_ptr()
        args.workspace_bytes = need
    _hip.check(lib.qp_attention(cache, args, _hip.stream_of(q)), "int4 KV attention")


def paged_decode(q, k_cache, v_cache, k_scale_cache, v_scale_cache, out, *, cu_seqlens_q, seqused_k, block_table,
                 max_seqlen_q, softmax_scale, num_segments, softmax_segm_output, softmax_segm_max,
                 softmax_segm_expsum, rht_signs=None, rht_out_scale=1.0, lse=None, query_signs=None) -> None:
    """Split-KV decode + merge as two library calls (qp_decode_splitkv, qp_merge_segments), q in the cache's domain
    unless query_signs rotates it on load (bf16 [T, NQ, hs]); out bf16 [T, NQ, hs]. With rht_signs the merge rotates
    the result back (out = (x H D) * rht_out_scale); lse (fp32 [T, NQ]) receives the natural-log LSE of each row.
    The segment buffers are the caller's: output fp32 [rows >= T, NQ, >= num_segments, >= hs], max / expsum fp32
    [rows, NQ, >= num_segments]."""
    hs = q.shape[2]
    cache = _hip.paged_cache(k_cache, v_cache, k_scale_cache, v_scale_cache, hs)
    so, sm, ss = softmax_segm_output, softmax_segm_max, softmax_segm_expsum
    if sm.stride() != ss.stride() or sm.stride(2) != 1:
        raise ValueError("segment max / expsum buffers must share strides with contiguous segments")
    args = _hip.DecodeArgs(q.data_ptr(), _hip.I64x2(q.stride(0), q.stride(1)), cu_seqlens_q.data_ptr(),
                           seqused_k.data_ptr(), block_table.data_ptr(), block_table.stride(0), len(seqused_k),
                           q.shape[0], q.shape[1], int(max_seqlen_q), int(num_segments), float(softmax_scale),
                           so.data_ptr(), _hip.I64x3(*so.stride()[:3]), sm.data_ptr(), ss.data_ptr(),
                           _hip.I64x2(sm.stride(0), sm.stride(1)), so.shape[0], _hip.ptr(query_signs))
    stream = _hip.stream_of(q)
    _hip.check(_hip.lib().qp_decode_splitkv(cache, args, stream), "split-KV decode")
    margs = _hip.MergeArgs(so.data_ptr(), _hip.I64x3(*so.stride()[:3]), sm.data_ptr(), ss.data_ptr(),
                           _hip.I64x2(sm.stride(0), sm.stride(1)), cu_seqlens_q.data_ptr(), seqused_k.data_ptr(),
                           len(seqused_k), q.shape[0], q.shape[1], hs, int(num_segments), out.data_ptr(),
                           _hip.I64x2(out.stride(0), out.stride(1)), _hip.ptr(lse),
                           _hip.I64x2(*(lse.stride() if lse is not None else (0, 0))), _hip.ptr(rht_signs),
                           float(rht_out_scale))
    _hip.check(_hip.lib().qp_merge_segments(margs, stream), "split-KV merge")


def unified_attention_int4(q, k_cache, v_cache, out, *, cu_seqlens_q, max_seqlen_q, seqused_k, max_seqlen_k,
                           softmax_scale, window_size, block_table, softcap, sinks, alibi_slopes, use_alibi_sqrt,
                           qq_bias, output_scale, mm_prefix_range, k_scale_cache, v_scale_cache, seq_threshold_3D=None,
                           num_par_softmax_segments=None, softmax_segm_output=None, softmax_segm_max=None,
                           softmax_segm_expsum=None, **kw):
    """Attention of unrotated bf16 queries q [T, NQ, hs] over an int4 (uint8 key view) or k8v4 (int8 key view) paged
    cache stored in the rotated domain; writes out in place, returns None. Same signature as the stock function and
    the reference's router (int4_kv.py:294-296; full call tests/test_int4_kv.py:150-156).

    One library call: sequences with at most MAX_Q_SPLIT_KV query tokens take the split-KV decode (when the caller
    passes segment buffers; int4_kv.py:101-112 and the sub-batch of :308-323), the others the MFMA prefill kernel,
    both routed on the device. q is rotated as the kernels load it and the output rotated back before its store
    (single_rht framing, :326-329). No host synchronisation; no allocation for a batch of short sequences."""
    del use_alibi_sqrt, seq_threshold_3D, kw
    _plain(q, window_size, softcap, sinks, alibi_slopes, qq_bias, output_scale, mm_prefix_range)
    _check_batch(q, cu_seqlens_q, seqused_k, block_table)
    hs = q.shape[2]
    target = out if (out.dtype == torch.bfloat16 and out.stride(-1) == 1) else torch.empty(
        q.shape, dtype=torch.bfloat16, device=q.device)
    segments = rows = 0
    if softmax_segm_output is not None and num_par_softmax_segments:
        cus = _device_cus(q)
        segments = decode_segments(num_par_softmax_segments, seqused_k.shape[0], k_cache.shape[2], cus)
        rows = decode_row_cap(cus)
    attend(q, k_cache, v_cache, k_scale_cache, v_scale_cache, target, cu_seqlens_q=cu_seqlens_q,
           seqused_k=seqused_k, block_table=block_table, max_seqlen_q=max_seqlen_q, max_seqlen_k=max_seqlen_k,
           softmax_scale=float(softmax_scale) / hs,        # <R q, R k> = hs <q, k>
           num_segments=segments, softmax_segm_output=softmax_segm_output, softmax_segm_max=softmax_segm_max,
           softmax_segm_expsum=softmax_segm_expsum, rht_signs=rht.signs(hs, q.device), rht_out_scale=1.0 / hs,
           max_decode_rows=rows)
    if target is not out:
        out.copy_(target)
    return None


def reshape_and_cache_int4(key, value, key_cache, value_cache, slot_mapping, *, k_scale_cache, v_scale_cache):
    """Store new tokens: rotate, quantise (int8 keys for a k8v4 key view, int4 otherwise; int4 values) and scatter to
    `slot_mapping`; negative slots are skipped. The stock store's and the reference's k8v4 override's signature
    (k8v4_kv.py:152-157)."""
    k8v4_kv.store(None, key, value, key_cache, value_cache, slot_mapping, k_scale_cache=k_scale_cache,
                  v_scale_cache=v_scale_cache)


# ------------------------------------------------------------------------------------------ vLLM integration

def segment_buffer_hook(triton_attn, segments) -> Hook:
    """Let vLLM's Triton metadata builder size the split-KV segment buffers of packed caches for `segments`
    segments. The builder reads the module constant NUM_PAR_SOFTMAX_SEGMENTS while it allocates, so a packed cache's
    builder is constructed with that constant at `segments`; other caches keep vLLM's value."""
    builder = triton_attn.TritonAttentionMetadataBuilder
    stock_init = builder.__init__

    def __init__(self, kv_cache_spec, layer_names, vllm_config, device):
        packed = vllm_config.cache_config.cache_dtype in PACKED_DTYPES
        sized = module_value(triton_attn, "NUM_PAR_SOFTMAX_SEGMENTS", segments) if packed else contextlib.nullcontext()
        with sized:
            stock_init(self, kv_cache_spec, layer_names, vllm_config, device)

    return Hook(builder, "__init__", __init__, f"split-KV buffers of packed caches for {segments} segments")


def _patch_decode_segments(segments, logger):
    """Install segment_buffer_hook (int4_kv.py:229-257): the segment count on success, 0 when `segments` is not a
    power of two (vLLM's split-KV layout) or when this vLLM has no Triton metadata builder to attach to."""
    if segments < 1 or segments & (segments - 1):
        logger.warning("vllm-quantpack: %d split-KV segments is not a power of two; vLLM's count kept", segments)
        return 0
    try:
        triton_attn, _, _ = find("vllm.v1.attention.backends.triton_attn", "TritonAttentionMetadataBuilder",
                                 "NUM_PAR_SOFTMAX_SEGMENTS")
    except Exception as e:
        logger.info("vllm-quantpack: split-KV segment count left to vLLM (%s)", e)
        return 0
    HOOKS.apply(segment_buffer_hook(triton_attn, segments))
    return segments


def patch_int4_kv(logger):
    """Attach the HIP attention and store to vLLM's int4 KV module, size the split-KV buffers for this GPU, register
    the k8v4 dtype and make the rotation's sign vectors (int4_kv.py:190-226). False when switched off
    (VLLM_QUANTPACK_INT4_KV=0), when vLLM has no int4 KV mode, or when the HIP library cannot be loaded: vLLM is then
    left as it was."""
    if os.environ.get("VLLM_QUANTPACK_INT4_KV", "1") == "0":
        return False
    try:
        (stock,) = find(MODULE)
    except Exception as e:
        logger.debug("vllm-quantpack: this vLLM has no int4 KV mode (%s)", e)
        return False
    try:
        _hip.lib()
        cus = torch.cuda.get_device_properties(0).multi_processor_count if torch.cuda.is_available() else 0
        segments = decode_tiles(cus)[2]
        if torch.cuda.is_available():
            for hs in RHT_HEAD_SIZES:       # before any graph capture can ask for them
                rht.signs(hs, torch.device("cuda", torch.cuda.current_device()))
    except Exception as e:
        logger.warning("vllm-quantpack: int4 KV attention left to vLLM (%s)", e)
        return False
    fresh = HOOKS.apply(Hook(stock, "unified_attention_int4", unified_attention_int4, "int4 attention on HIP"))
    HOOKS.apply(Hook(stock, "reshape_and_cache_int4", reshape_and_cache_int4, "int4 / k8v4 store on HIP"))
    if not fresh:
        return True
    segments = _patch_decode_segments(segments, logger)
    k8v4 = k8v4_kv.patch_backend(stock, logger) and k8v4_kv.register_dtype(logger)
    logger.info("vllm-quantpack: int4_per_token_head attention on MI355X HIP kernels (split-KV decode up to %d query "
                "tokens, %s segments; MFMA prefill)", MAX_Q_SPLIT_KV, segments or "vLLM's")
    if k8v4:
        logger.info("vllm-quantpack: KV cache dtype %s available (int8 keys, int4 values)", k8v4_kv.NAME)
    return True


# ------------------------------------------------------------------------------------------- prepared calls

class DecodePlan:
    """A decode step with every C-ABI argument prepared once, for loops that replay the same shapes (benchmarks,
    HIP-graph capture): `run()` is one qp_attention call (the whole layer: rotation, split-KV decode, merge),
    `decode()` / `merge()` the two kernel-level calls of the same step for timing them apart. Tensors are referenced,
    not copied; their contents may change between runs, their storage and strides may not. With rotate_query the
    query is unrotated and rotated on load (the drop-in path); otherwise it is already in the cache's domain."""

    def __init__(self, q, k_cache, v_cache, k_scale_cache, v_scale_cache, out, *, cu_seqlens_q, seqused_k,
                 block_table, max_seqlen_q, softmax_scale, num_segments, softmax_segm_output, softmax_segm_max,
                 softmax_segm_expsum, rht_signs=None, rht_out_scale=1.0, rotate_query=False):
        hs = q.shape[2]
        so, sm, ss = softmax_segm_output, softmax_segm_max, softmax_segm_expsum
        qsigns = rht_signs if rotate_query else None
        self._keep = (q, k_cache, v_cache, k_scale_cache, v_scale_cache, out, cu_seqlens_q, seqused_k, block_table,
                      so, sm, ss, rht_signs)
        self.cache = _hip.paged_cache(k_cache, v_cache, k_scale_cache, v_scale_cache, hs)
        self.args = _hip.DecodeArgs(q.data_ptr(), _hip.I64x2(q.stride(0), q.stride(1)), cu_seqlens_q.data_ptr(),
                                    seqused_k.data_ptr(), block_table.data_ptr(), block_table.stride(0),
                                    len(seqused_k), q.shape[0], q.shape[1], int(max_seqlen_q), int(num_segments),
                                    float(softmax_scale), so.data_ptr(), _hip.I64x3(*so.stride()[:3]), sm.data_ptr(),
                                    ss.data_ptr(), _hip.I64x2(sm.stride(0), sm.stride(1)), so.shape[0],
                                    _hip.ptr(qsigns))
        self.margs = _hip.MergeArgs(so.data_ptr(), _hip.I64x3(*so.stride()[:3]), sm.data_ptr(), ss.data_ptr(),
                                    _hip.I64x2(sm.stride(0), sm.stride(1)), cu_seqlens_q.data_ptr(),
                                    seqused_k.data_ptr(), len(seqused_k), q.shape[0], q.shape[1], hs,
                                    int(num_segments), out.data_ptr(), _hip.I64x2(out.stride(0), out.stride(1)),
                                    None, _hip.I64x2(0, 0), _hip.ptr(rht_signs), float(rht_out_scale))
        self.aargs = attention_args(q, out, cu_seqlens_q=cu_seqlens_q, seqused_k=seqused_k, block_table=block_table,
                                    max_seqlen_q=max_seqlen_q, max_seqlen_k=2**31 - 1, softmax_scale=softmax_scale,
                                    num_segments=num_segments, softmax_segm_output=so, softmax_segm_max=sm,
                                    softmax_segm_expsum=ss, rht_signs=None, rht_out_scale=rht_out_scale)
        self.aargs.rht_signs = _hip.ptr(rht_signs)
        if rht_signs is not None and not rotate_query:
            raise ValueError("DecodePlan: one qp_attention call rotates both ways; pass rotate_query=True with "
                             "rht_signs, or no signs")
        self.stream = _hip.stream_of(q)
        self._lib = _hip.lib()
        if self._lib.qp_attention_workspace_size(self.cache, self.aargs) != 0:
            raise ValueError("DecodePlan: not a batch of short sequences that fit the segment buffers")

    def decode(self):
        _hip.check(self._lib.qp_decode_splitkv(self.cache, self.args, self.stream), "split-KV decode")

    def merge(self):
        _hip.check(self._lib.qp_merge_segments(self.margs, self.stream), "split-KV merge")

    def run(self):
        _hip.check(self._lib.qp_attention(self.cache, self.aargs, self.stream), "int4 KV attention")
