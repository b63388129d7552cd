"""Numpy restatement of vllm-quantpack's int4_per_token_head / k8v4_per_token_head KV-cache attention arithmetic.

TEST INFRASTRUCTURE: the results the tests compare the HIP kernels with, and the CPU baseline of the benchmark.
Nothing in the product package imports this module.

Every function cites the reference file:line it restates (paths relative to the reference repository root). The
kernels the plugin edits live in vLLM (`vllm.v1.attention.ops.int4_per_token_head`), which the reference does not
vendor; where a detail comes from vLLM and not from the plugin's own text, the docstring says "inferred".

Pinning (the checks that tie each function to something other than its own formula) is done in
tests/test_oracle_pinning.py; the table there names, per function, the known answers, closed forms and planted
mistakes used. Every function below is pinned by at least one of them. Parity unpinned at bit level, and said so in
the docstrings concerned: the fused multiply-add assumed in the int4 store's `v * inv + zp` (`_fma32`), the correctly
rounded fp32 divisions assumed in the store (`k / k_scale`, `(max - min) / 15`, `-min / scale` and `1 / scale`,
k8v4_ops.py:35-36,52-54: the text does not say how the compiled Triton store divides, and an approximate division
would move codes that sit on a rounding boundary), vLLM's own RHT sign vector (`rht_signs`), and the int4 store's key
half (inferred equal to its value half). Those are pinned only to tolerance, through the fp64 closed form (the
divisions also by the known answers on rows whose quotients are exact or far from a boundary).
"""
from __future__ import annotations

import math
from typing import NamedTuple

import numpy as np

LOG2E = 1.4426950408889634

# ---------------------------------------------------------------------------------------------------------- bf16


def f32_to_bf16_bits(x) -> np.ndarray:
    """float32 -> bfloat16 bits, round to nearest even (torch `.to(torch.bfloat16)`, Triton `.to(tl.bfloat16)`:
    the stores of int4_prefill.py:46-47,67-68 round through `out_ptr.dtype.element_ty`). NaN stays a quiet NaN."""
    x = np.array(x, dtype=np.float32, copy=True)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        r = np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)
    return r


def bf16_bits_to_f32(b) -> np.ndarray:
    return (np.array(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(x) -> np.ndarray:
    """float32 values rounded to the nearest bfloat16 (returned as float32)."""
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


# ------------------------------------------------------------------------------------------- cache cells and views

class CacheViews(NamedTuple):
    """Numpy views of one paged cache, indexed (block, slot, kv head[, byte])."""
    key: np.ndarray          # int4: (blocks, bs, nkv, hs/2) uint8 nibble pairs; k8v4: (blocks, bs, nkv, hs) int8
    value: np.ndarray        # (blocks, bs, nkv, hs_v/2) uint8 nibble pairs
    key_word: np.ndarray     # (blocks, bs, nkv) uint32: int4 = fp32 scale bits with zp in the low 4; k8v4 = fp32 scale
    value_word: np.ndarray   # (blocks, bs, nkv) uint32: fp32 scale bits with zp in the low 4
    key_format: str          # "int4" | "int8"


def int4_cell_bytes(head_size: int) -> int:
    """[K nibbles hs/2 | K word 4 | V nibbles hs/2 | V word 4]: tests/test_int4_kv.py:96-102,
    tools/int4_kv_bench.py:24-30 (264 B at head 256)."""
    return head_size + 8


def k8v4_cell_bytes(head_size: int, head_size_v: int | None = None) -> int:
    """[K int8 hs | K scale 4 | V nibbles hs_v/2 | V word 4]: k8v4_kv.py:31-33 (392 B at head 256)."""
    head_size_v = head_size if head_size_v is None else head_size_v
    return head_size + head_size_v // 2 + 8


def new_cache(num_blocks: int, num_kv_heads: int, block_size: int, cell: int, layout: str = "hnd",
              dtype=np.uint8) -> np.ndarray:
    """Zeroed byte cache with logical shape (blocks, kv heads, block size, cell); NHD stores (blocks, bs, heads, cell)
    and returns the transposed view, as tests/test_k8v4_kv.py:29-32 builds it."""
    if layout == "hnd":
        return np.zeros((num_blocks, num_kv_heads, block_size, cell), dtype=dtype)
    if layout == "nhd":
        return np.zeros((num_blocks, block_size, num_kv_heads, cell), dtype=dtype).transpose(0, 2, 1, 3)
    raise ValueError(layout)


def _root(a: np.ndarray) -> np.ndarray:
    while isinstance(a.base, np.ndarray):
        a = a.base
    return a


def _word_view(kv: np.ndarray, byte_at: int) -> np.ndarray:
    """uint32 (blocks, bs, nkv) view of the 4 bytes at `byte_at` of every cell of kv (blocks, nkv, bs, cell)."""
    root = _root(kv)
    off = kv.__array_interface__["data"][0] - root.__array_interface__["data"][0] + byte_at
    s = kv.strides
    return np.ndarray((kv.shape[0], kv.shape[2], kv.shape[1]), dtype="<u4", buffer=root, offset=off,
                      strides=(s[0], s[2], s[1]))


def int4_views(kv: np.ndarray, head_size: int) -> CacheViews:
    """Views of an int4_per_token_head byte cache, as tests/test_int4_kv.py:95-103 builds them with torch: the key
    view is the first hs/2 bytes of each cell, the value view starts at hs/2 + 4, the fp32 words follow each half."""
    half = head_size // 2
    if kv.shape[3] != int4_cell_bytes(head_size):
        raise ValueError(f"int4 cell of {kv.shape[3]} bytes, expected {int4_cell_bytes(head_size)}")
    t = kv.transpose(0, 2, 1, 3)
    return CacheViews(t[..., :half], t[..., half + 4:2 * half + 4], _word_view(kv, half),
                      _word_view(kv, 2 * half + 4), "int4")


def k8v4_views(kv: np.ndarray, head_size: int, head_size_v: int | None = None) -> CacheViews:
    """k8v4_kv.py:41-65: key int8 (blocks, bs, nkv, hs), value uint8 (..., hs_v/2), two fp32 words; ValueError for a
    cell of the wrong size (:48-50) or scales that are not 4-byte aligned (:56-57)."""
    head_size_v = head_size if head_size_v is None else head_size_v
    cell = kv.shape[3]
    if kv.itemsize != 1 or cell != k8v4_cell_bytes(head_size, head_size_v):
        raise ValueError(f"k8v4_per_token_head: cache cell of {cell} x {kv.itemsize} bytes, expected "
                         f"{k8v4_cell_bytes(head_size, head_size_v)} for head sizes {head_size} / {head_size_v}")
    st = kv.strides
    if any(s % 4 for s in st[:3]) or head_size % 4 or (head_size_v // 2) % 4:
        raise ValueError("k8v4_per_token_head: fp32 scales are not 4-byte aligned")
    v_at = head_size + 4
    t = kv.transpose(0, 2, 1, 3)
    return CacheViews(t[..., :head_size].view(np.int8), t[..., v_at:v_at + head_size_v // 2].view(np.uint8),
                      _word_view(kv, head_size), _word_view(kv, v_at + head_size_v // 2), "int8")


def gather(views: CacheViews, block_row: np.ndarray, positions: np.ndarray):
    """Cells of cache positions `positions` of one sequence through its block-table row: (key codes, key words,
    value codes, value words), each [P, nkv, ...]. Block lookup `block_row[pos // bs]`, slot `pos % bs`
    (int4_prefill.py:35-36,61-62)."""
    bs = views.key.shape[1]
    positions = np.asarray(positions, dtype=np.int64)
    blk = np.asarray(block_row, dtype=np.int64)[positions // bs]
    slot = positions % bs
    return (views.key[blk, slot], views.key_word[blk, slot], views.value[blk, slot], views.value_word[blk, slot])


# ------------------------------------------------------------------------------------------------ unpack (a12)

def int4_word_parts(words: np.ndarray):
    """(zero point as float32, scale as float32): `zp = bits & 0xF`, `scale = f32(bits & -16)`
    (int4_prefill.py:40-43)."""
    words = np.asarray(words, dtype=np.uint32)
    zp = (words & np.uint32(0xF)).astype(np.float32)
    scale = (words & np.uint32(0xFFFFFFF0)).view(np.float32)
    return zp, scale


def unpack_int4(codes: np.ndarray, words: np.ndarray) -> np.ndarray:
    """bf16 bits of `bf16(fp32(nibble - zp) * scale)`, low nibble = even channel (int4_prefill.py:44-46):
    an exact fp32 subtraction, one fp32 product rounded to nearest even, one rounding to bf16."""
    zp, scale = int4_word_parts(words)
    lo = ((codes & 0xF).astype(np.float32) - zp[..., None]) * scale[..., None]
    hi = (((codes >> 4) & 0xF).astype(np.float32) - zp[..., None]) * scale[..., None]
    out = np.empty(codes.shape[:-1] + (2 * codes.shape[-1],), np.float32)
    out[..., 0::2] = lo
    out[..., 1::2] = hi
    return f32_to_bf16_bits(out)


def unpack_i8(codes: np.ndarray, words: np.ndarray) -> np.ndarray:
    """bf16 bits of `bf16(fp32(int8) * scale)` for k8v4 keys (int4_prefill.py:63-67)."""
    scale = np.asarray(words, dtype=np.uint32).view(np.float32)
    return f32_to_bf16_bits(codes.astype(np.float32) * scale[..., None])


def unpack_segment(views: CacheViews, block_row, start: int, length: int, which: str = "key") -> np.ndarray:
    """`unpack_segment(cache, scales, block_row, start, length, out)` (int4_prefill.py:71-84): positions
    [start, start + length) to bf16 bits [length, nkv, hs]. `which` picks the key or the value half."""
    kc, kw, vc, vw = gather(views, block_row, np.arange(start, start + length))
    if which == "value":
        return unpack_int4(vc, vw)
    return unpack_i8(kc, kw) if views.key_format == "int8" else unpack_int4(kc, kw)


# ----------------------------------------------------------------------------------------- fp64 closed form

def dequant_f64(views: CacheViews, block_row, n: int):
    """(K, V) in fp64, [n, nkv, hs]: `(u - zp) * scale` (tests/test_int4_kv.py:119-123) or `int8 * scale`
    (tests/test_k8v4_kv.py:116-121), computed without any rounding."""
    kc, kw, vc, vw = gather(views, block_row, np.arange(n))

    def int4(c, w):
        u = np.empty(c.shape[:-1] + (2 * c.shape[-1],), np.float64)
        u[..., 0::2] = c & 0xF
        u[..., 1::2] = (c >> 4) & 0xF
        zp, scale = int4_word_parts(w)
        return (u - zp[..., None].astype(np.float64)) * scale[..., None].astype(np.float64)

    if views.key_format == "int8":
        K = kc.astype(np.float64) * np.asarray(kw, np.uint32).view(np.float32)[..., None].astype(np.float64)
    else:
        K = int4(kc, kw)
    return K, int4(vc, vw)


def attention_f64(q: np.ndarray, K: np.ndarray, V: np.ndarray, n: int, scale: float) -> np.ndarray:
    """Causal attention of q [T, NQ, hs] (the last T positions of a context of n tokens) over K/V [n, nkv, hs] in
    fp64 (tests/test_int4_kv.py:126-133, tools/int4_kv_bench.py:53-59). Query head h reads KV head h // (NQ/nkv)."""
    T, NQ, _ = q.shape
    nkv = K.shape[1]
    g = NQ // nkv
    q = q.astype(np.float64)
    pos = n - T + np.arange(T)
    mask = np.arange(n)[None, :] > pos[:, None]
    out = np.empty(q.shape, np.float64)
    for h in range(NQ):
        s = q[:, h] @ K[:, h // g].T * scale
        s = np.where(mask, -np.inf, s)
        s = s - s.max(axis=1, keepdims=True)
        p = np.exp(s)
        out[:, h] = (p / p.sum(axis=1, keepdims=True)) @ V[:, h // g]
    return out


def relerr(o, ref) -> float:
    """Relative Frobenius error `||o - ref|| / ||ref||` (tests/test_int4_kv.py:160-161)."""
    o = np.asarray(o, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.linalg.norm(o - ref) / np.linalg.norm(ref))


def max_row_relerr(o, ref) -> float:
    """Largest relative error of one output row (the head_size vector of one (token, head)):
    max_r ||o_r - ref_r|| / ||ref_r||. A stricter reading of "max relative error" than the Frobenius figure of the
    reference's own test, which a few bad rows among many cannot hide in."""
    o = np.asarray(o, np.float64)
    ref = np.asarray(ref, np.float64)
    hs = ref.shape[-1]
    num = np.linalg.norm((o - ref).reshape(-1, hs), axis=1)
    den = np.linalg.norm(ref.reshape(-1, hs), axis=1)
    return float((num / np.where(den > 0, den, 1.0)).max())


# ------------------------------------------------------------------------- exact read kernel emulation (a7-a9)

def value_probabilities(P: np.ndarray, s_v: np.ndarray, zp_v: np.ndarray):
    """(P_v16, zero-point sum) of one tile: P_v16 = bf16(P * s_v) is the PV operand, and the zero-point correction
    sum_j fp32(P_v16_j) * zp_v_j is taken on that same rounded P_v16, not on the fp32 P * s_v (int4_kv.py:90-94:
    `P_v16 = P_v.to(...)`, `Pv_zp_sum = tl.sum(P_v16.to(tl.float32) * v_zp[None, :], axis=1)`). P [rows, keys]."""
    P16 = round_bf16(P * s_v[None, :])
    return P16, (P16 * zp_v[None, :]).sum(axis=1, dtype=np.float32)


def segment_length(n: int, num_segments: int, tile: int) -> int:
    """Keys per split-KV segment: `cdiv(n, S * tile) * tile` (the 3D kernel's tiles_per_segment; inferred from
    vLLM's split-KV layout that int4_kv.py:98-122 configures)."""
    return -(-n // (num_segments * tile)) * tile


def decode_partials(q: np.ndarray, views: CacheViews, block_row, n: int, scale: float, num_segments: int,
                    tile: int = 64):
    """One sequence of the generated `_attn_packed_qp` / `_attn_k8v4_qp` split-KV kernel (int4_kv.py:80-95,
    127-142 applied to vLLM's `_attn_packed`), per KV head and segment: returns (acc, m, l) with acc
    [T, NQ, S, hs] fp32 (unnormalised, channel order restored), m and l [T, NQ, S] fp32, m in log2 units.

    Arithmetic per 64-key tile, every query row of a KV head's GQA group at once (int4_kv.py:108-112):
      raw = Q_even . K_lo + Q_odd . K_hi   (bf16 operands: q is bf16, nibbles are exact; fp32 accumulation)
      S   = (raw - Q_sum * zp_k) * s_k * scale * log2(e)            int4 keys (int4_kv.py:82-87)
      S   = raw_int8 * s_k * scale * log2(e)                         k8v4 keys (int4_kv.py:136-141)
      causal mask key j <= n - T + t; online softmax in fp32 with exp2 (exp vs exp2: inferred)
      P_v16 = bf16(P * s_v); acc += P_v16 . V_u - sum(fp32(P_v16) * zp_v)   (int4_kv.py:90-94)
      l from the unrounded P.
    """
    T, NQ, hs = q.shape
    nkv = views.key.shape[2]
    g = NQ // nkv
    qf = round_bf16(np.asarray(q, np.float32))
    seg = segment_length(n, num_segments, tile)
    acc = np.zeros((T, NQ, num_segments, hs), np.float32)
    m_out = np.full((T, NQ, num_segments), -np.inf, np.float32)
    l_out = np.zeros((T, NQ, num_segments), np.float32)
    pos = n - T + np.arange(T)
    c = np.float32(scale * LOG2E)
    for h in range(nkv):
        rows = qf[:, h * g:(h + 1) * g].reshape(T * g, hs)          # row = t * g + j
        row_pos = np.repeat(pos, g)
        q_even, q_odd = rows[:, 0::2], rows[:, 1::2]
        q_sum = q_even.sum(axis=1, dtype=np.float32) + q_odd.sum(axis=1, dtype=np.float32)
        for s in range(num_segments):
            start, end = s * seg, min(n, (s + 1) * seg)
            if start >= end:
                continue
            m = np.full(T * g, -np.inf, np.float32)
            l = np.zeros(T * g, np.float32)
            a_even = np.zeros((T * g, hs // 2), np.float32)
            a_odd = np.zeros((T * g, hs // 2), np.float32)
            for t0 in range(start, end, tile):
                keys = np.arange(t0, min(end, t0 + tile))
                kc, kw, vc, vw = gather(views, block_row, keys)
                kc, kw, vc, vw = kc[:, h], kw[:, h], vc[:, h], vw[:, h]
                if views.key_format == "int8":
                    s_k = np.asarray(kw, np.uint32).view(np.float32)
                    raw = rows @ kc.astype(np.float32).T
                    S = raw * (s_k * c)
                else:
                    zp_k, s_k = int4_word_parts(kw)
                    raw = q_even @ (kc & 0xF).astype(np.float32).T + q_odd @ ((kc >> 4) & 0xF).astype(np.float32).T
                    S = (raw - q_sum[:, None] * zp_k[None, :]) * (s_k * c)[None, :]
                S = np.where(keys[None, :] > row_pos[:, None], np.float32(-np.inf), S).astype(np.float32)
                m_new = np.maximum(m, S.max(axis=1))
                m_safe = np.where(np.isneginf(m_new), np.float32(0), m_new)
                P = np.exp2(S - m_safe[:, None]).astype(np.float32)
                alpha = np.exp2(m - m_safe).astype(np.float32)
                l = l * alpha + P.sum(axis=1, dtype=np.float32)
                m = m_new
                zp_v, s_v = int4_word_parts(vw)
                P16, corr = value_probabilities(P, s_v, zp_v)
                a_even = a_even * alpha[:, None] + (P16 @ (vc & 0xF).astype(np.float32)) - corr[:, None]
                a_odd = a_odd * alpha[:, None] + (P16 @ ((vc >> 4) & 0xF).astype(np.float32)) - corr[:, None]
            out = np.empty((T * g, hs), np.float32)
            out[:, 0::2] = a_even
            out[:, 1::2] = a_odd
            acc[:, h * g:(h + 1) * g, s] = out.reshape(T, g, hs)
            m_out[:, h * g:(h + 1) * g, s] = m.reshape(T, g)
            l_out[:, h * g:(h + 1) * g, s] = l.reshape(T, g)
    return acc, m_out, l_out


def merge_partials(acc: np.ndarray, m: np.ndarray, l: np.ndarray) -> np.ndarray:
    """Split-KV segment reduce (vLLM's reduce kernel, absent; algebra as int4_prefill.py:224-230 merges its
    segments): M = max_s m_s, out = sum_s acc_s 2^(m_s - M) / sum_s l_s 2^(m_s - M), in fp32. Returns fp32."""
    M = m.max(axis=-1)
    M = np.where(np.isneginf(M), np.float32(0), M)
    w = np.exp2(m - M[..., None]).astype(np.float32)
    w = np.where(np.isneginf(m), np.float32(0), w)
    L = (l * w).sum(axis=-1, dtype=np.float32)
    num = (acc * w[..., None]).sum(axis=-2, dtype=np.float32)
    return (num / np.where(L == 0, np.float32(1), L)[..., None]).astype(np.float32)


def segment_lse(m: np.ndarray, l: np.ndarray) -> np.ndarray:
    """Natural-log LSE of a segment from (m in log2 units, l): (m + log2 l) * ln 2; -inf for an empty one
    (m = -inf, l = 0). The per-segment LSE the split-KV path carries, in the natural-log units of the `lse` that
    int4_prefill.py:223-230 folds with `logaddexp`."""
    m = np.asarray(m, np.float64)
    l = np.asarray(l, np.float64)
    with np.errstate(divide="ignore", invalid="ignore"):
        out = (m + np.log2(l)) * math.log(2)
    return np.where((l > 0) & np.isfinite(m), out, -np.inf).astype(np.float32)


def merge_lse(m: np.ndarray, l: np.ndarray) -> np.ndarray:
    """Natural-log LSE of whole rows from their segments' statistics (last axis = segment): ln sum_s l_s 2^(m_s),
    the `logaddexp` fold of int4_prefill.py:223-230 over the segments. -inf when every segment is empty."""
    m = np.asarray(m, np.float64)
    l = np.asarray(l, np.float64)
    M = m.max(axis=-1)
    Ms = np.where(np.isfinite(M), M, 0.0)
    with np.errstate(invalid="ignore"):
        w = np.where(np.isfinite(m), np.exp2(m - Ms[..., None]), 0.0)
    L = (l * w).sum(axis=-1)
    with np.errstate(divide="ignore"):
        out = (Ms + np.log2(L)) * math.log(2)
    return np.where(L > 0, out, -np.inf).astype(np.float32)


def decode_emulated(q, views, block_row, n, scale, num_segments=1, tile=64) -> np.ndarray:
    """Segment partials merged and rounded to bf16 (the output dtype): float32 values of the bf16 result."""
    acc, m, l = decode_partials(q, views, block_row, n, scale, num_segments, tile)
    return round_bf16(merge_partials(acc, m, l))


# ---------------------------------------------------------------------- dequantise-then-attend (a11, CPU path)

def unpack_torch(codes, words, key_format: str = "int4"):
    """`unpack_int4` / `unpack_i8` in torch on the CPU (multi-threaded), returning the bf16 values as fp32:
    codes [..., bytes] uint8 (int8 for keys of a k8v4 cache), words [...] uint32 numpy arrays."""
    import torch
    c = torch.from_numpy(np.ascontiguousarray(codes))
    w = torch.from_numpy(np.ascontiguousarray(words).view(np.int32))
    if key_format == "int8":
        scale = w.view(torch.float32)
        return (c.view(torch.int8).float() * scale[..., None]).to(torch.bfloat16).float()
    zp = (w & 0xF).float()
    scale = (w & -16).view(torch.float32)
    c = c.to(torch.int32)
    lo = ((c & 0xF).float() - zp[..., None]) * scale[..., None]
    hi = ((c >> 4).float() - zp[..., None]) * scale[..., None]
    return torch.stack((lo, hi), dim=-1).flatten(-2).to(torch.bfloat16).float()


def prefill_dequant_attend(q_rot, views: CacheViews, block_row, n: int, scale: float, segment: int = 16384,
                           threads: int | None = None):
    """`prefill_sequence` (int4_prefill.py:203-232) restated in torch on the CPU: newest-first segments of `segment`
    tokens, each K/V segment gathered through the block table and unpacked to bf16 exactly as `unpack_segment`
    (:25-68), attention in fp32 with its log-sum-exp (causal on the newest segment only, :222), segments folded by
    `logaddexp` (:223-230). FlashAttention's own arithmetic is replaced by plain fp32 attention (its internals are not
    in the reference). This is also the benchmark's CPU baseline. q_rot: [T, NQ, hs] array of bf16 values.
    Returns fp32 [T, NQ, hs] (before the final bf16 store)."""
    import torch
    if threads:
        torch.set_num_threads(threads)
    q = torch.from_numpy(round_bf16(np.asarray(q_rot, np.float32)))
    T, NQ, hs = q.shape
    nkv = views.key.shape[2]
    g = NQ // nkv
    qh = q.reshape(T, nkv, g, hs).permute(1, 0, 2, 3).reshape(nkv, T * g, hs)   # [nkv, rows, hs]
    row_pos = torch.arange(n - T, n).repeat_interleave(g)
    acc = acc_lse = None
    end = n
    while end > 0:
        start = max(0, end - segment)
        kc, kw, vc, vw = gather(views, block_row, np.arange(start, end))
        kb = unpack_torch(kc, kw, views.key_format)                                 # [L, nkv, hs]
        vb = unpack_torch(vc, vw)
        s = torch.bmm(qh, kb.permute(1, 2, 0).contiguous()) * scale                 # [nkv, rows, L]
        if end == n:
            keys = torch.arange(start, end)
            s = s.masked_fill(keys[None, None, :] > row_pos[None, :, None], float("-inf"))
        lse = torch.logsumexp(s, dim=-1)                                            # [nkv, rows]
        o = torch.bmm(torch.softmax(s, dim=-1), vb.permute(1, 0, 2).contiguous())   # [nkv, rows, hs]
        if acc is None:
            acc, acc_lse = o, lse
        else:
            new = torch.logaddexp(acc_lse, lse)
            acc = acc * torch.exp(acc_lse - new)[..., None] + o * torch.exp(lse - new)[..., None]
            acc_lse = new
        end = start
    out = acc.reshape(nkv, T, g, hs).permute(1, 0, 2, 3).reshape(T, NQ, hs)
    return out.numpy()


# ------------------------------------------------------------------ single-kernel int8 prefill (a14, _attn_i8)

Q_LO = 254  # weight of the high int8 part of the query (int4_prefill.py:173)


def quantize_query_i8(q_rot_bits, softmax_scale: float):
    """The query split of `prefill_sequence_i8` (int4_prefill.py:181-189), in fp32 as torch runs it:
    q = f32(q_rot) * f32(softmax_scale * LOG2E) (torch rounds the Python scalar to the tensor's fp32 first);
    q_scale = max(max|q| / 127, 1e-20) per (token, head); qn = q / q_scale; hi = round(qn) and
    lo = clamp(round((qn - hi) * 254), -127, 127), rounding half to even (torch.round); q_sum = sum(hi) * 254 + sum(lo)
    (exact: the fp32 sums of these integers stay below 2^24).
    q_rot_bits: bf16 bits [T, NQ, hs]. Returns (hi int8, lo int8, q_scale fp32 [T, NQ], q_sum int64 [T, NQ])."""
    q = bf16_bits_to_f32(q_rot_bits) * np.float32(softmax_scale * LOG2E)
    qs = np.maximum(np.abs(q).max(axis=-1) / np.float32(127.0), np.float32(1e-20)).astype(np.float32)
    qn = (q / qs[..., None]).astype(np.float32)
    hi = np.rint(qn).astype(np.float32)
    lo = np.clip(np.rint((qn - hi) * np.float32(Q_LO)), -127, 127).astype(np.float32)
    q_sum = hi.astype(np.int64).sum(-1) * Q_LO + lo.astype(np.int64).sum(-1)
    return hi.astype(np.int8), lo.astype(np.int8), qs, q_sum


def i8_scores(hi, lo, q_sum, qs, kcodes, kwords) -> np.ndarray:
    """The scores of `_attn_i8` (int4_prefill.py:136-138) of one query head over keys of one KV head, in log2 units:
    S = ((hi . k) * 254 + lo . k - q_sum * zp_k), an exact int32 on the raw nibbles k (low nibble = even channel),
    then fp32, times q_scale / 254 (fp32), times s_k. hi, lo: int8 [T, hs]; q_sum int [T]; qs fp32 [T];
    kcodes uint8 [n, hs/2]; kwords uint32 [n]. Returns fp32 [T, n]."""
    k = np.empty((kcodes.shape[0], 2 * kcodes.shape[1]), np.int64)
    k[:, 0::2] = kcodes & 0xF
    k[:, 1::2] = kcodes >> 4
    zp, ks = int4_word_parts(kwords)
    si = (hi.astype(np.int64) @ k.T) * Q_LO + lo.astype(np.int64) @ k.T - q_sum[:, None] * zp.astype(np.int64)[None, :]
    qs_lo = (qs / np.float32(Q_LO)).astype(np.float32)
    return (si.astype(np.float32) * qs_lo[:, None]).astype(np.float32) * ks[None, :]


def prefill_i8_emulated(q_rot_bits, views: CacheViews, block_row, n: int, softmax_scale: float) -> np.ndarray:
    """`_attn_i8` over one sequence (int4_prefill.py:95-172): the chunk's queries (the last T positions of a context of
    n tokens, causal) against an int4 cache. Scores from i8_scores; softmax in base 2 against the row maximum; the
    value operand nibble - zp (exact) and P16 = fp16(p * s_v) (:161-163); l the sum of the unrounded p; out = acc / l.
    The reference adds each 64-key tile's fp16-accumulated PV into fp32 and rescales by its running maximum; here
    everything after P16 is summed in fp64 against the final maximum (fp16 rounding is relative, so only values in
    fp16's subnormal range depend on which maximum p is taken against). Returns fp64 [T, NQ, hs] (before the bf16
    store)."""
    hi, lo, qs, q_sum = quantize_query_i8(q_rot_bits, softmax_scale)
    T, NQ, hs = hi.shape
    kc, kw, vc, vw = gather(views, block_row, np.arange(n))
    nkv = kc.shape[1]
    g = NQ // nkv
    pos = n - T + np.arange(T)
    mask = np.arange(n)[None, :] > pos[:, None]
    out = np.zeros((T, NQ, hs), np.float64)
    for kvh in range(nkv):
        v = np.empty((n, hs), np.float64)
        v[:, 0::2] = vc[:, kvh] & 0xF
        v[:, 1::2] = vc[:, kvh] >> 4
        zp_v, s_v = int4_word_parts(vw[:, kvh])
        v -= zp_v.astype(np.float64)[:, None]
        for h in range(kvh * g, (kvh + 1) * g):
            s = i8_scores(hi[:, h], lo[:, h], q_sum[:, h], qs[:, h], kc[:, kvh], kw[:, kvh]).astype(np.float64)
            s = np.where(mask, -np.inf, s)
            mx = s.max(axis=1, keepdims=True)
            ok = np.isfinite(mx)
            p = np.where(ok, np.exp2(s - np.where(ok, mx, 0.0)), 0.0)
            p16 = (p.astype(np.float32) * s_v[None, :]).astype(np.float16).astype(np.float64)
            l = p.sum(axis=1, keepdims=True)
            out[:, h] = (p16 @ v) / np.where(l > 0, l, 1.0)
    return out


# ------------------------------------------------------------------------------------------- store (next-1)

def round_half_away(x: np.ndarray) -> np.ndarray:
    """`_round` (k8v4_ops.py:5-8): fp32 `x +/- 0.5`, then truncation toward zero."""
    x = np.asarray(x, np.float32)
    return np.where(x >= 0, np.trunc(x + np.float32(0.5)), np.trunc(x - np.float32(0.5))).astype(np.float32)


def _fma32(a, b, c) -> np.ndarray:
    """fp32 fused multiply-add: the fp64 product of two fp32 values plus a small integer is exact, so one rounding
    to fp32 gives the correctly rounded result. Used for `v * inv_v + v_zp` (k8v4_ops.py:55-56) on the assumption
    that Triton contracts it into one FMA (its `enable_fp_fusion` compile option is on by default). Parity unpinned:
    Triton cannot run here, and the reference holds no stored codes that would show which of the two it does; a
    mul-then-add store differs from this one in the codes of a few channels near a rounding boundary."""
    return (np.asarray(a, np.float64) * np.asarray(b, np.float64) + np.asarray(c, np.float64)).astype(np.float32)


def quantize_int4(v: np.ndarray):
    """Asymmetric int4 per (token, head) as the value half of `_store_k8v4` (k8v4_ops.py:42-63), which states it
    follows vLLM's int4 store (:22; the int4 store itself is in vLLM: its key half is inferred to be the same).
    v: [..., hs] fp32 values. Returns (nibble-pair bytes [..., hs/2] uint8, word [...] uint32). The divisions are taken
    as correctly rounded fp32 (numpy's), an assumption about the compiled store: parity unpinned there."""
    v = np.asarray(v, np.float32)
    vmin = v.min(axis=-1)
    vmax = v.max(axis=-1)
    scale = np.maximum((vmax - vmin) / np.float32(15.0), np.float32(1e-6)).astype(np.float32)
    zp = np.clip(round_half_away(-vmin / scale), 0, 15).astype(np.float32)
    inv = (np.float32(1.0) / scale).astype(np.float32)
    q = np.clip(round_half_away(_fma32(v, inv[..., None], zp[..., None])), 0, 15).astype(np.uint8)
    codes = (q[..., 0::2] & 0xF) | ((q[..., 1::2] & 0xF) << 4)
    word = (scale.view(np.uint32) & np.uint32(0xFFFFFFF0)) | zp.astype(np.uint32)
    return codes.astype(np.uint8), word.astype(np.uint32)


def quantize_int8(k: np.ndarray):
    """Key half of `_store_k8v4` (k8v4_ops.py:30-39): scale = max(absmax / 127, 1e-6), codes =
    clamp(round(k / scale), -127, 127). Returns (int8 codes [..., hs], fp32 scale bits [...] uint32). The divisions
    are taken as correctly rounded fp32 (numpy's), an assumption about the compiled store: parity unpinned there."""
    k = np.asarray(k, np.float32)
    scale = np.maximum(np.abs(k).max(axis=-1) / np.float32(127.0), np.float32(1e-6)).astype(np.float32)
    q = np.clip(round_half_away(k / scale[..., None]), -127, 127).astype(np.int8)
    return q, scale.view(np.uint32)


def store(views: CacheViews, key: np.ndarray, value: np.ndarray, slots: np.ndarray) -> None:
    """`reshape_and_cache_int4` semantics on the oracle's views (k8v4_kv.py:68-86, k8v4_ops.py:11-63): token i goes
    to slot `slots[i]` (block slot // bs, offset slot % bs); negative slots are skipped (:26-27). key/value: fp32
    [N, nkv, hs] already in the cache's (rotated) domain."""
    bs = views.key.shape[1]
    if views.key_format == "int8":
        kc, kw = quantize_int8(key)
    else:
        kc, kw = quantize_int4(key)
    vc, vw = quantize_int4(value)
    for i, slot in enumerate(np.asarray(slots, np.int64)):
        if slot < 0:
            continue
        b, o = slot // bs, slot % bs
        views.key[b, o] = kc[i]
        views.key_word[b, o] = kw[i]
        views.value[b, o] = vc[i]
        views.value_word[b, o] = vw[i]


# ----------------------------------------------------------------------------------------------- RHT (next-2)

def rht_signs(head_size: int, seed: int = 0) -> np.ndarray:
    """The +/-1 diagonal D of the randomized Hadamard rotation R = H D: sign of channel c is bit 0 of the
    `lowbias32` integer hash (C. Wellons) of c + seed * 0x9E3779B9. vLLM's own sign vector is not in the reference
    (`single_rht` lives in vLLM); only its unnormalised orthogonality R R^T = hs I is (tests/test_int4_kv.py:126-133)."""
    x = (np.arange(head_size, dtype=np.uint64) + np.uint64(seed) * np.uint64(0x9E3779B9)) & np.uint64(0xFFFFFFFF)
    x ^= x >> np.uint64(16)
    x = (x * np.uint64(0x7FEB352D)) & np.uint64(0xFFFFFFFF)
    x ^= x >> np.uint64(15)
    x = (x * np.uint64(0x846CA68B)) & np.uint64(0xFFFFFFFF)
    x ^= x >> np.uint64(16)
    return np.where(x & np.uint64(1), -1.0, 1.0)


def sylvester(n: int) -> np.ndarray:
    """Sylvester Hadamard matrix H_n (n a power of two), entries +/-1, H H^T = n I."""
    h = np.ones((1, 1))
    while h.shape[0] < n:
        h = np.block([[h, h], [h, -h]])
    return h


def rht(x: np.ndarray, inverse: bool = False, seed: int = 0) -> np.ndarray:
    """`single_rht(x)` = x R^T (rows rotated by R = H D); `single_rht(x, inverse=True)` = x R (unnormalised: the
    caller divides by hs, int4_kv.py:329). fp64."""
    hs = x.shape[-1]
    H = sylvester(hs)
    D = rht_signs(hs, seed)
    x = np.asarray(x, np.float64)
    if inverse:
        return (x @ H) * D          # D H y: rows y -> y H^T D = y H D (H symmetric)
    return (x * D) @ H.T            # H D x as rows: x D H^T
