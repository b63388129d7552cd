"""Prefill over the int4_per_token_head / k8v4_per_token_head cache, and the bit-exact segment unpack.

The reference walks a long context in 16k-token segments, unpacks each to bf16 scratch with a Triton kernel,
attends with FlashAttention 2 and folds the segments by log-sum-exp (int4_prefill.py:1-14, 203-232). Here one HIP
kernel (`qp_prefill`) reads the packed cache directly: it dequantises K/V tiles to exact bf16 integers in LDS and runs
QK^T and PV on bf16 MFMA with an online softmax, so there is no scratch, no segment loop and no host synchronisation.
`unpack_segment` remains, bit-exact with the reference's `_unpack_segment` / `_unpack_segment_i8`, for callers that
want bf16 K/V.
"""
from __future__ import annotations

import torch

from .. import _hip

MAX_HEAD = 256       # largest head size of the MFMA prefill kernel
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
                      block_table, max_seqlen_q, softmax_scale) -> None:
    """Batched causal attention of the query tokens of every sequence (the last cu_seqlens_q[i+1] - cu_seqlens_q[i]
    positions of a context of seqused_k[i] tokens) over the paged cache: q and out bf16 [T, NQ, hs] in the cache's
    domain, softmax_scale multiplies q.k in that domain."""
    hs = q.shape[2]
    cache = _hip.paged_cache(k_cache, v_cache, k_scale_cache, v_scale_cache, hs)
    args = _hip.PrefillArgs(q.data_ptr(), _hip.I64x2(q.stride(0), q.stride(1)), cu_seqlens_q.data_ptr(),
                            seqused_k.data_ptr(), block_table.data_ptr(), block_table.stride(0),
                            len(seqused_k), q.shape[0], q.shape[1], int(max_seqlen_q), float(softmax_scale),
                            out.data_ptr(), _hip.I64x2(out.stride(0), out.stride(1)))
    _hip.check(_hip.lib().qp_prefill(cache, args, _hip.stream_of(q)), "prefill")


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


# The reference's single-kernel INT8-QK alternative (int4_prefill.py:176-200) has the same contract; the MFMA kernel
# serves both names.
prefill_sequence_i8 = prefill_sequence
