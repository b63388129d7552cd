"""int4_per_token_head / k8v4_per_token_head KV-cache attention on MI355X, behind vLLM's Triton-backend API.

The reference fixes vLLM's Triton kernel by text edits and routes long prefills to FlashAttention (int4_kv.py:1-29).
This package replaces the whole read path with hand-written gfx950 kernels reached through libquantpack_hip.so:

* decode / MTP verify (1..4 query tokens per sequence): split-KV kernel holding every query row of a GQA group per
  workgroup (the cache is read once per step), then a log-sum-exp merge that also rotates the output back;
* everything else (prefill chunks, mixed batches): one batched MFMA prefill kernel over the packed cache;
* the store (`reshape_and_cache_int4`) quantises and scatters new tokens, int4 or int8 keys.

The arithmetic is the reference's exact kernel: bf16 query and exact-integer nibble operands, fp32 accumulation, and
the value zero point removed with the same bf16-rounded P * s_v that feeds the PV product (int4_kv.py:80-95).
Nothing here copies to or waits for the host, so decode steps can be captured in HIP graphs.
"""
from __future__ import annotations

import os

import torch

from .. import _hip
from . import int4_prefill, k8v4_kv
from .rht import single_rht  # noqa: F401  (re-exported: the stock module's name)

MODULE = "vllm.v1.attention.ops.int4_per_token_head"
PACKED_DTYPES = ("int4_per_token_head", "k8v4_per_token_head")
MAX_Q_SPLIT_KV = _hip.DECODE_MAX_QUERY       # MTP / EAGLE verification with up to 3 draft tokens
# The reference's Triton tile tables (int4_kv.py:42-56). The HIP kernels have fixed geometry (4 waves, 32-key chunks
# for decode); only the split-KV segment count and the query-row cap of the decode setting take effect here.
PREFILL_TILES_BY_MAJOR = {8: (64, 64, 8, 2), 12: (64, 64, 8, 2)}
PREFILL_TILES_DEFAULT = (64, 64, 8, 2)
DECODE_TILES_DEFAULT = (64, 4, "auto")
DECODE_MAX_M = 64
MIN_SEGMENTS, MAX_SEGMENTS = 16, 128
MAX_DECODE_ROWS = 32                          # query rows (tokens x GQA heads) one split-KV workgroup holds


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


def _device_cus(device):
    idx = device.index if device.index is not None else torch.cuda.current_device()
    cus = _CUS.get(idx)
    if cus is None:
        cus = _CUS[idx] = torch.cuda.get_device_properties(idx).multi_processor_count
    return cus


_CUS = {}


def decode_tiles(sms):
    """(tile, warps, segments[, rows]) from VLLM_QUANTPACK_INT4_DECODE="tile,warps,segments|auto[,rows]" or the
    default (int4_kv.py:72-77)."""
    env = os.environ.get("VLLM_QUANTPACK_INT4_DECODE")
    tile, warps, segments, *max_m = env.split(",") if env else DECODE_TILES_DEFAULT
    segments = segments_for(sms) if str(segments).strip() == "auto" else int(segments)
    return (int(tile), int(warps), segments) + tuple(int(m) for m in max_m[:1])


def _plain(q, window_size, softcap, sinks, alibi_slopes, qq_bias, output_scale, mm_prefix_range):
    unsupported = [name for name, bad in (
        ("sliding window", window_size is not None and window_size[0] >= 0),
        ("softcap", bool(softcap)), ("sinks", sinks is not None), ("ALiBi", alibi_slopes is not None),
        ("qq_bias", qq_bias is not None), ("fp8 output_scale", output_scale is not None),
        ("mm_prefix_range", mm_prefix_range is not None)) if bad]
    if unsupported:
        raise NotImplementedError("int4 KV attention (HIP): " + ", ".join(unsupported) + " not supported")


def paged_decode(q, k_cache, v_cache, k_scale_cache, v_scale_cache, out, *, cu_seqlens_q, seqused_k, block_table,
                 max_seqlen_q, softmax_scale, num_segments, softmax_segm_output, softmax_segm_max,
                 softmax_segm_expsum, rht_signs=None, rht_out_scale=1.0, lse=None) -> None:
    """Split-KV decode + merge, q in the cache's domain (bf16 [T, NQ, hs]); out bf16 [T, NQ, hs]. With rht_signs the
    merge rotates the result back (out = (x H D) * rht_out_scale). The segment buffers are the caller's:
    output fp32 [rows >= T, NQ, >= num_segments, >= hs], max / expsum fp32 [rows, NQ, >= num_segments]."""
    hs = q.shape[2]
    cache = _hip.paged_cache(k_cache, v_cache, k_scale_cache, v_scale_cache, hs)
    so, sm, ss = softmax_segm_output, softmax_segm_max, softmax_segm_expsum
    if sm.stride() != ss.stride() or sm.stride(2) != 1:
        raise ValueError("segment max / expsum buffers must share strides with contiguous segments")
    args = _hip.DecodeArgs(q.data_ptr(), _hip.I64x2(q.stride(0), q.stride(1)), cu_seqlens_q.data_ptr(),
                           seqused_k.data_ptr(), block_table.data_ptr(), block_table.stride(0), len(seqused_k),
                           q.shape[0], q.shape[1], int(max_seqlen_q), int(num_segments), float(softmax_scale),
                           so.data_ptr(), _hip.I64x3(*so.stride()[:3]), sm.data_ptr(), ss.data_ptr(),
                           _hip.I64x2(sm.stride(0), sm.stride(1)), so.shape[0])
    stream = _hip.stream_of(q)
    _hip.check(_hip.lib().qp_decode_splitkv(cache, args, stream), "split-KV decode")
    margs = _hip.MergeArgs(so.data_ptr(), _hip.I64x3(*so.stride()[:3]), sm.data_ptr(), ss.data_ptr(),
                           _hip.I64x2(sm.stride(0), sm.stride(1)), cu_seqlens_q.data_ptr(), seqused_k.data_ptr(),
                           len(seqused_k), q.shape[0], q.shape[1], hs, int(num_segments), out.data_ptr(),
                           _hip.I64x2(out.stride(0), out.stride(1)), lse.data_ptr() if lse is not None else None,
                           _hip.I64x2(*(lse.stride() if lse is not None else (0, 0))),
                           rht_signs.data_ptr() if rht_signs is not None else None, float(rht_out_scale))
    _hip.check(_hip.lib().qp_merge_segments(margs, stream), "split-KV merge")


def unified_attention_int4(q, k_cache, v_cache, out, *, cu_seqlens_q, max_seqlen_q, seqused_k, max_seqlen_k,
                           softmax_scale, window_size, block_table, softcap, sinks, alibi_slopes, use_alibi_sqrt,
                           qq_bias, output_scale, mm_prefix_range, k_scale_cache, v_scale_cache, seq_threshold_3D=None,
                           num_par_softmax_segments=None, softmax_segm_output=None, softmax_segm_max=None,
                           softmax_segm_expsum=None, **kw):
    """Attention of unrotated bf16 queries q [T, NQ, hs] over an int4 (uint8 key view) or k8v4 (int8 key view) paged
    cache stored in the rotated domain; writes out in place, returns None. Same signature as the stock function and
    the reference's router (int4_kv.py:294-296; full call tests/test_int4_kv.py:150-156).

    Split-KV decode when every sequence has <= MAX_Q_SPLIT_KV query tokens, q fits the segment buffers and the GQA
    group times the tokens fits one workgroup (int4_kv.py:101-112); the batched MFMA prefill kernel otherwise."""
    del use_alibi_sqrt, seq_threshold_3D, kw
    _plain(q, window_size, softcap, sinks, alibi_slopes, qq_bias, output_scale, mm_prefix_range)
    hs = q.shape[2]
    scale = float(softmax_scale) / hs           # <R q, R k> = hs <q, k>
    q_rot = single_rht(q, out_dtype=torch.bfloat16)
    signs = k8v4_kv.rht.signs(hs, q.device)
    nkv = k_cache.shape[2]
    rows = int(max_seqlen_q) * (q.shape[1] // nkv)
    decode = (int(max_seqlen_q) <= MAX_Q_SPLIT_KV and rows <= MAX_DECODE_ROWS and softmax_segm_output is not None
              and q.shape[0] <= softmax_segm_output.shape[0] and num_par_softmax_segments
              and hs in (128, 256, 512))
    if decode:
        target = out if (out.dtype == torch.bfloat16 and out.stride(-1) == 1) else torch.empty_like(q)
        paged_decode(q_rot, k_cache, v_cache, k_scale_cache, v_scale_cache, target, cu_seqlens_q=cu_seqlens_q,
                     seqused_k=seqused_k, block_table=block_table, max_seqlen_q=max_seqlen_q, softmax_scale=scale,
                     num_segments=decode_segments(num_par_softmax_segments, len(seqused_k), nkv,
                                                  _device_cus(q.device)),
                     softmax_segm_output=softmax_segm_output,
                     softmax_segm_max=softmax_segm_max, softmax_segm_expsum=softmax_segm_expsum, rht_signs=signs,
                     rht_out_scale=1.0 / hs)
        if target is not out:
            out.copy_(target)
        return None
    # the prefill kernel (or its split merge) rotates the result back itself
    target = out if (out.dtype == torch.bfloat16 and out.is_contiguous()) else torch.empty_like(q)
    int4_prefill.prefill_attention(q_rot, k_cache, v_cache, k_scale_cache, v_scale_cache, target,
                                   cu_seqlens_q=cu_seqlens_q, seqused_k=seqused_k, block_table=block_table,
                                   max_seqlen_q=max_seqlen_q, softmax_scale=scale, max_seqlen_k=max_seqlen_k,
                                   rht_signs=signs, rht_out_scale=1.0 / hs)
    if target is not out:
        out.copy_(target)
    return None


def reshape_and_cache_int4(key, value, key_cache, value_cache, slot_mapping, *, k_scale_cache, v_scale_cache):
    """Store new tokens: rotate, quantise (int8 keys for a k8v4 key view, int4 otherwise; int4 values) and scatter to
    `slot_mapping`; negative slots are skipped. The stock store's and the reference's k8v4 override's signature
    (k8v4_kv.py:152-157)."""
    k8v4_kv.store(None, key, value, key_cache, value_cache, slot_mapping, k_scale_cache=k_scale_cache,
                  v_scale_cache=v_scale_cache)


def patch_int4_kv(logger):
    """Install the HIP store and attention into vLLM's int4 module, size the split-KV segment buffers for this GPU
    and register the k8v4 dtype (int4_kv.py:190-226). False when disabled (VLLM_QUANTPACK_INT4_KV=0), when vLLM has
    no int4 KV mode, or when the HIP library cannot be loaded; vLLM is then left untouched."""
    if os.environ.get("VLLM_QUANTPACK_INT4_KV", "1") == "0":
        return False
    try:
        import importlib
        stock = importlib.import_module(MODULE)
    except Exception as e:      # vLLM without the int4 KV mode
        logger.debug("vllm-quantpack: int4 KV attention not patched (%s)", e)
        return False
    if getattr(stock.unified_attention_int4, "_quantpack", False):
        return True
    try:
        _hip.lib()
        sms = torch.cuda.get_device_properties(0).multi_processor_count if torch.cuda.is_available() else 0
        decode = decode_tiles(sms)
    except Exception as e:
        logger.warning("vllm-quantpack: int4_per_token_head attention left stock (%s)", e)
        return False

    def attention(*args, **kwargs):
        return unified_attention_int4(*args, **kwargs)

    def store(*args, **kwargs):
        return reshape_and_cache_int4(*args, **kwargs)

    attention._quantpack = store._quantpack = True
    stock.unified_attention_int4 = attention     # looked up in the module globals at call time
    stock.reshape_and_cache_int4 = store
    segments = _patch_decode_segments(decode[2], logger)
    k8v4 = k8v4_kv.patch_backend(stock, logger) and k8v4_kv.register_dtype(logger)
    logger.info("vllm-quantpack: int4_per_token_head KV attention on MI355X HIP kernels (split-KV decode with MTP, "
                "%s segments, MFMA prefill)", segments or "stock")
    if k8v4:
        logger.info("vllm-quantpack: KV cache dtype %s available (int8 keys, int4 values)", k8v4_kv.NAME)
    return True


def _patch_decode_segments(segments, logger):
    """Allocate the split-KV segment buffers of int4 and k8v4 caches for `segments` segments instead of vLLM's 16
    (int4_kv.py:229-257). 0 when vLLM's builder is absent or segments is not a power of two."""
    try:
        from vllm.v1.attention.backends import triton_attn
        builder = triton_attn.TritonAttentionMetadataBuilder
        stock_init = builder.__init__
        triton_attn.NUM_PAR_SOFTMAX_SEGMENTS   # the anchor this relies on
    except Exception as e:
        logger.info("vllm-quantpack: int4 split-KV segments left stock (%s)", e)
        return 0
    if getattr(stock_init, "_quantpack", False):
        return segments
    if segments < 1 or segments & (segments - 1):
        logger.warning("vllm-quantpack: int4 split-KV segments must be a power of two, got %d: left stock", segments)
        return 0

    def __init__(self, kv_cache_spec, layer_names, vllm_config, device):
        if vllm_config.cache_config.cache_dtype not in PACKED_DTYPES:
            return stock_init(self, kv_cache_spec, layer_names, vllm_config, device)
        saved = triton_attn.NUM_PAR_SOFTMAX_SEGMENTS
        triton_attn.NUM_PAR_SOFTMAX_SEGMENTS = segments   # read once, in __init__, to size the buffers
        try:
            stock_init(self, kv_cache_spec, layer_names, vllm_config, device)
        finally:
            triton_attn.NUM_PAR_SOFTMAX_SEGMENTS = saved

    __init__._quantpack = True
    builder.__init__ = __init__
    return segments


class DecodePlan:
    """A split-KV decode + merge with every C-ABI argument prepared once: `run()` is two library calls and nothing
    else, for loops that replay the same shapes (benchmarks, HIP-graph capture). Tensors are referenced, not
    copied; their contents may change between runs, their storage and strides may not."""

    def __init__(self, q, k_cache, v_cache, k_scale_cache, v_scale_cache, out, *, cu_seqlens_q, seqused_k,
                 block_table, max_seqlen_q, softmax_scale, num_segments, softmax_segm_output, softmax_segm_max,
                 softmax_segm_expsum, rht_signs=None, rht_out_scale=1.0):
        hs = q.shape[2]
        so, sm, ss = softmax_segm_output, softmax_segm_max, softmax_segm_expsum
        self._keep = (q, k_cache, v_cache, k_scale_cache, v_scale_cache, out, cu_seqlens_q, seqused_k, block_table,
                      so, sm, ss, rht_signs)
        self.cache = _hip.paged_cache(k_cache, v_cache, k_scale_cache, v_scale_cache, hs)
        self.args = _hip.DecodeArgs(q.data_ptr(), _hip.I64x2(q.stride(0), q.stride(1)), cu_seqlens_q.data_ptr(),
                                    seqused_k.data_ptr(), block_table.data_ptr(), block_table.stride(0),
                                    len(seqused_k), q.shape[0], q.shape[1], int(max_seqlen_q), int(num_segments),
                                    float(softmax_scale), so.data_ptr(), _hip.I64x3(*so.stride()[:3]), sm.data_ptr(),
                                    ss.data_ptr(), _hip.I64x2(sm.stride(0), sm.stride(1)), so.shape[0])
        self.margs = _hip.MergeArgs(so.data_ptr(), _hip.I64x3(*so.stride()[:3]), sm.data_ptr(), ss.data_ptr(),
                                    _hip.I64x2(sm.stride(0), sm.stride(1)), cu_seqlens_q.data_ptr(),
                                    seqused_k.data_ptr(), len(seqused_k), q.shape[0], q.shape[1], hs,
                                    int(num_segments), out.data_ptr(), _hip.I64x2(out.stride(0), out.stride(1)),
                                    None, _hip.I64x2(0, 0),
                                    rht_signs.data_ptr() if rht_signs is not None else None, float(rht_out_scale))
        self.stream = _hip.stream_of(q)
        self._lib = _hip.lib()

    def decode(self):
        _hip.check(self._lib.qp_decode_splitkv(self.cache, self.args, self.stream), "split-KV decode")

    def merge(self):
        _hip.check(self._lib.qp_merge_segments(self.margs, self.stream), "split-KV merge")

    def run(self):
        self.decode()
        self.merge()
