"""Prefill over the int4_per_token_head / k8v4_per_token_head cache, and the bit-exact segment unpack.

The reference walks a long context in 16k-token segments, unpacks each to bf16 scratch with a Triton kernel,
attends with FlashAttention 2 and folds the segments by log-sum-exp (int4_prefill.py:1-14, 203-232). Here one HIP
kernel (`qp_prefill`) reads the packed cache directly: it dequantises K/V tiles to exact bf16 integers in LDS and runs
QK^T and PV on bf16 MFMA with an online softmax, so there is no scratch, no segment loop and no host synchronisation.
`unpack_segment` remains, bit-exact with the reference's `_unpack_segment` / `_unpack_segment_i8`, for callers that
want bf16 K/V. `prefill_sequence_i8` keeps the reference's single-kernel alternative and its arithmetic (an int8
split of the query, integer QK^T on the raw nibbles, fp16 PV: int4_prefill.py:95-200) on its own HIP kernel
(`qp_prefill_i8`).
"""
from __future__ import annotations

import numpy as np
import torch

from .. import _hip

LOG2E = 1.4426950408889634

MAX_HEAD = 512       # largest head size of the MFMA prefill kernels (head 512: the wide kernel with int4 keys)
SEGMENT = 16384      # the reference's unpack segment; kept for callers that size bf16 scratch the same way
MIN_QUERY = 64       # chunks at least this long take the prefill kernel even when they could take split-KV decode
MIN_CONTEXT = 8192   # kept for API compatibility: the HIP prefill has no context threshold


def unpack_segment(cache: torch.Tensor, scales: torch.Tensor, block_row: torch.Tensor, start: int, length: int,
                   out: torch.Tensor) -> None:
    """Unpack cache positions [start, start + length) of one sequence into out[:length] (L, KV heads, head size),
    bf16. An int8 cache view holds one code per channel (k8v4 keys); a uint8 one, two nibbles per byte, low nibble =
    even channel. out = bf16(fp32(code - zp) * scale) or bf16(fp32(int8) * scale), bit-exact with the reference
    (int4_prefill.py:25-84)."""
    if out.dtype != torch.bfloat16:
        raise ValueError(f"unpack_segment: bf16 output, got {out.dtype}")
    if out.stride(-1) != 1:
        raise ValueError("unpack_segment: output channels must be contiguous")
    nkv, head = cache.shape[2], out.shape[2]
    if block_row.dtype != torch.int32:
        block_row = block_row.to(torch.int32)
    half = _hip.cache_half(cache, scales)
    strides = (_hip.c_int64 * 2)(out.stride(0), out.stride(1))
    _hip.check(_hip.lib().qp_unpack_segment(half, cache.shape[1], nkv, head, _hip.ptr(block_row), int(start),
                                            int(length), _hip.ptr(out), strides, _hip.stream_of(out)),
               "unpack_segment")


def _cu_seqlens(length: int, device) -> torch.Tensor:
    """[0, length] as int32 on the device, written by fill kernels rather than copied from the host
    (int4_prefill.py:87-92)."""
    cu = torch.full((2,), length, dtype=torch.int32, device=device)
    cu[0].zero_()
    return cu


def prefill_attention(q, k_cache, v_cache, k_scale_cache, v_scale_cache, out, *, cu_seqlens_q, seqused_k,
                      block_table, max_seqlen_q, softmax_scale, max_seqlen_k=None, num_splits=0, rht_signs=None,
                      rht_out_scale=1.0, query_signs=None) -> None:
    """Batched causal attention of the query tokens of every sequence (the last cu_seqlens_q[i+1] - cu_seqlens_q[i]
    positions of a context of seqused_k[i] tokens) over the paged cache: q and out bf16 [T, NQ, hs] in the cache's
    domain, softmax_scale multiplies q.k in that domain. With rht_signs the result is rotated back,
    out = (o H D) * rht_out_scale; with query_signs q is unrotated and each row is rotated, (q D) H, as it loads.
    When the chunk alone cannot fill the GPU, the keys are split over workgroups
    (num_splits, 0 = automatic) and merged; the fp32 partials go to a workspace from torch's caching allocator.
    max_seqlen_k bounds the automatic split count; without it the block table's capacity stands in (no host sync).
    Rows are (token, query head) pairs, so any GQA width fills the kernels' tiles. Head 128 from 8 query heads per KV
    head, and head 512 with int4 keys, run the library's wide kernel (32x32x16 MFMAs; at head 512 always key-split, so
    it takes a workspace); head 512 with int8
    keys runs the split-KV decode kernel over causal query slices of the chunk and merges (the library picks the
    path)."""
    cache, args = _prefill_args(q, k_cache, v_cache, k_scale_cache, v_scale_cache, out, cu_seqlens_q, seqused_k,
                                block_table, max_seqlen_q, softmax_scale, max_seqlen_k, num_splits)
    args.rht_signs = _hip.ptr(rht_signs)
    args.rht_out_scale = float(rht_out_scale)
    args.query_signs = _hip.ptr(query_signs)
    lib = _hip.lib()
    need = lib.qp_prefill_workspace_size(cache, args)
    ws = torch.empty(need, dtype=torch.uint8, device=q.device) if need > 0 else None
    args.workspace = _hip.ptr(ws)
    args.workspace_bytes = need
    _hip.check(lib.qp_prefill(cache, args, _hip.stream_of(q)), "prefill")


def _prefill_args(q, k_cache, v_cache, k_scale_cache, v_scale_cache, out, cu_seqlens_q, seqused_k, block_table,
                  max_seqlen_q, softmax_scale, max_seqlen_k, num_splits):
    """(qp_paged_cache, qp_prefill_args) of a prefill call, without workspace or rotations."""
    hs = q.shape[2]
    cache = _hip.paged_cache(k_cache, v_cache, k_scale_cache, v_scale_cache, hs)
    if max_seqlen_k is None:
        max_seqlen_k = block_table.shape[1] * k_cache.shape[1]
    args = _hip.PrefillArgs()
    args.query = q.data_ptr()
    args.query_stride = _hip.I64x2(q.stride(0), q.stride(1))
    args.cu_seqlens_q = cu_seqlens_q.data_ptr()
    args.seqused_k = seqused_k.data_ptr()
    args.block_table = block_table.data_ptr()
    args.block_table_stride = block_table.stride(0)
    args.num_seqs = len(seqused_k)
    args.num_tokens = q.shape[0]
    args.num_q_heads = q.shape[1]
    args.max_query_len = int(max_seqlen_q)
    args.max_seqlen_k = int(min(max_seqlen_k, 2**31 - 1))
    args.num_splits = int(num_splits)
    args.softmax_scale = float(softmax_scale)
    args.out = out.data_ptr()
    args.out_stride = _hip.I64x2(out.stride(0), out.stride(1))
    args.rht_out_scale = 1.0
    return cache, args


def prefill_attention_i8(q, k_cache, v_cache, k_scale_cache, v_scale_cache, out, *, cu_seqlens_q, seqused_k,
                         block_table, max_seqlen_q, softmax_scale, max_seqlen_k=None, num_splits=0) -> None:
    """prefill_attention with the arithmetic of the reference's single-kernel alternative (`_attn_i8`,
    int4_prefill.py:95-172), on int4 caches with q and out in the cache's domain: each query row is split into two
    int8 parts in log2 units (q_scale (hi + lo / 254), the split of int4_prefill.py:181-189, done in the kernel), QK^T
    runs on int8 MFMAs over the raw key nibbles and PV on fp16 MFMAs with P16 = fp16(p s_v)."""
    cache, args = _prefill_args(q, k_cache, v_cache, k_scale_cache, v_scale_cache, out, cu_seqlens_q, seqused_k,
                                block_table, max_seqlen_q, softmax_scale, max_seqlen_k, num_splits)
    # the reference multiplies the fp32 query by softmax_scale * LOG2E, which torch rounds to fp32 first
    args.softmax_scale = float(np.float32(softmax_scale * LOG2E))
    lib = _hip.lib()
    need = lib.qp_prefill_i8_workspace_size(cache, args)
    ws = torch.empty(need, dtype=torch.uint8, device=q.device) if need > 0 else None
    args.workspace = _hip.ptr(ws)
    args.workspace_bytes = need
    _hip.check(lib.qp_prefill_i8(cache, args, _hip.stream_of(q)), "prefill (int8 query split)")


def prefill_sequence(q_rot, k_cache, v_cache, k_scales, v_scales, block_row, n, softmax_scale, fa=None):
    """Attention of q_rot (one chunk's queries, already rotated; the last len(q_rot) positions of a context of n
    tokens) over the whole cached context, in one HIP kernel. Returns the output in the rotated domain in q_rot's
    dtype. `fa` (the reference's FlashAttention function, int4_prefill.py:203) is accepted and not used."""
    del fa
    qlen = q_rot.shape[0]
    q = q_rot if q_rot.dtype == torch.bfloat16 else q_rot.to(torch.bfloat16)
    out = torch.empty_like(q)
    dev = q.device
    cu = _cu_seqlens(qlen, dev)
    used = torch.full((1,), int(n), dtype=torch.int32, device=dev)
    table = block_row.reshape(1, -1)
    if table.dtype != torch.int32:
        table = table.to(torch.int32)
    prefill_attention(q, k_cache, v_cache, k_scales, v_scales, out, cu_seqlens_q=cu, seqused_k=used,
                      block_table=table, max_seqlen_q=qlen, softmax_scale=softmax_scale)
    return out if q_rot.dtype == torch.bfloat16 else out.to(q_rot.dtype)


def prefill_sequence_i8(q_rot, k_cache, v_cache, k_scales, v_scales, block_row, n, softmax_scale, block_m=64,
                        block_n=64, num_warps=8, num_stages=2):
    """The reference's single-kernel alternative (int4_prefill.py:176-200) with the same contract as
    prefill_sequence, and its arithmetic (prefill_attention_i8): the int8 query split, int8 QK^T on the raw nibbles,
    fp16 PV. Its Triton tile arguments are accepted and not used (the HIP kernel has its own tiles)."""
    del block_m, block_n, num_warps, num_stages
    qlen = q_rot.shape[0]
    q = q_rot if q_rot.dtype == torch.bfloat16 else q_rot.to(torch.bfloat16)
    out = torch.empty_like(q)
    dev = q.device
    cu = _cu_seqlens(qlen, dev)
    used = torch.full((1,), int(n), dtype=torch.int32, device=dev)
    table = block_row.reshape(1, -1)
    if table.dtype != torch.int32:
        table = table.to(torch.int32)
    prefill_attention_i8(q, k_cache, v_cache, k_scales, v_scales, out, cu_seqlens_q=cu, seqused_k=used,
                         block_table=table, max_seqlen_q=qlen, softmax_scale=softmax_scale)
    return out if q_rot.dtype == torch.bfloat16 else out.to(q_rot.dtype)
