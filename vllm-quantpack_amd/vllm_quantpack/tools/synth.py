"""Seeded synthetic paged caches and queries for the benchmark and the parity tests.

Workloads (24 query / 4 KV heads, head 256, block 16 unless stated):
  decode-int4-4k-t1        4096 cached tokens, 1 query token, 256 shuffled blocks
  decode-int4-128k-t2      131072 tokens, 2 query tokens (MTP 1), 8192 shuffled blocks
  decode-int4-256k-t4      262144 tokens, 4 query tokens (MTP 3), 16384 shuffled blocks
  prefill-int4-128k-c1024  131072 cached tokens + a 1024-token chunk whose bf16 K/V are quantised by the store
  decode-k8v4-ragged-b32   32 requests of 1 or 2 query tokens, contexts lognormal(ln 16384, 1) clipped to
                           [2048, 65536], int8 keys, queries rotated into the Hadamard domain
  prefill-k8v4-128k-c1024  the prefill chunk workload over a k8v4 cache (int8 keys stored by the store as well)
  prefill-int4-h512-128k-c1024  the prefill chunk workload at head 512 with 16 query / 2 KV heads (the shape of a
                           Gemma-style global attention layer)
  prefill-int4-g16-32k-c1024  a 1024-token chunk over 32768 cached tokens with 32 query / 2 KV heads (16 query heads
                           per KV head), head 256
  prefill-int4-g8-128k-c1024  the prefill chunk workload with 64 query / 8 KV heads at head 128 (the attention of a
                           Llama-3-70B-class layer on one GPU: 8 query heads per KV head)
  prefill-int4-g4-128k-c1024  the prefill chunk workload with 32 query / 8 KV heads at head 128 (a Llama-3-8B or
                           Mistral-7B-class layer: 4 query heads per KV head)

int4 cells: nibbles uniform 0..15; per (token, KV head) fp32 scale ~ lognormal(-3, 0.5) with its low 4 mantissa bits
replaced by the zero point round(U(6, 9)). k8v4 keys: int8 uniform -127..127, fp32 scale ~ lognormal(-4, 0.5).
Queries bf16 N(0, 1). Block tables are seeded permutations of the physical blocks. Seed = 1000 + workload index.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

NQ, NKV, HS, BS = 24, 4, 256, 16

WORKLOADS = ("decode-int4-4k-t1", "decode-int4-128k-t2", "decode-int4-256k-t4", "prefill-int4-128k-c1024",
             "decode-k8v4-ragged-b32", "prefill-k8v4-128k-c1024", "prefill-int4-h512-128k-c1024",
             "prefill-int4-g16-32k-c1024", "prefill-int4-g8-128k-c1024", "prefill-int4-g4-128k-c1024")


@dataclass
class Workload:
    name: str
    kv: np.ndarray                 # uint8 byte cache (blocks, nkv, bs, cell), HND
    key_format: str                # "int4" | "int8"
    q: np.ndarray                  # uint16 bf16 bits [T, NQ, hs]
    cu_seqlens_q: np.ndarray       # int32 [num_seqs + 1]
    seqused_k: np.ndarray          # int32 [num_seqs]
    block_table: np.ndarray        # int32 [num_seqs, width]
    softmax_scale: float           # multiplies q.k in the cache's domain
    head_size: int = HS
    num_q_heads: int = NQ
    num_kv_heads: int = NKV
    block_size: int = BS
    new_key: np.ndarray | None = None    # uint16 bf16 bits [chunk, nkv, hs]: tokens the store writes first
    new_value: np.ndarray | None = None
    new_slots: np.ndarray | None = None  # int64 [chunk]
    meta: dict = field(default_factory=dict)

    @property
    def num_tokens(self) -> int:
        return int(self.q.shape[0])

    @property
    def max_query_len(self) -> int:
        return int(np.diff(self.cu_seqlens_q).max())


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits, round to nearest even."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def int4_words(rng, shape, mu=-3.0, sigma=0.5, zp_lo=6.0, zp_hi=9.0) -> np.ndarray:
    scale = rng.lognormal(mu, sigma, size=shape).astype(np.float32)
    zp = np.rint(rng.uniform(zp_lo, zp_hi, size=shape)).astype(np.uint32)
    return (scale.view(np.uint32) & np.uint32(0xFFFFFFF0)) | zp


def fill_int4_cache(rng, num_blocks, nkv=NKV, bs=BS, hs=HS) -> np.ndarray:
    half = hs // 2
    kv = np.empty((num_blocks, nkv, bs, hs + 8), np.uint8)
    kv[..., :half] = rng.integers(0, 256, size=(num_blocks, nkv, bs, half), dtype=np.uint8)
    kv[..., half + 4:2 * half + 4] = rng.integers(0, 256, size=(num_blocks, nkv, bs, half), dtype=np.uint8)
    kv[..., half:half + 4] = int4_words(rng, (num_blocks, nkv, bs)).view(np.uint8).reshape(num_blocks, nkv, bs, 4)
    kv[..., 2 * half + 4:] = int4_words(rng, (num_blocks, nkv, bs)).view(np.uint8).reshape(num_blocks, nkv, bs, 4)
    return kv


def fill_k8v4_cache(rng, num_blocks, nkv=NKV, bs=BS, hs=HS) -> np.ndarray:
    half = hs // 2
    cell = hs + half + 8
    kv = np.empty((num_blocks, nkv, bs, cell), np.uint8)
    kv[..., :hs] = rng.integers(-127, 128, size=(num_blocks, nkv, bs, hs), dtype=np.int8).view(np.uint8)
    ks = rng.lognormal(-4.0, 0.5, size=(num_blocks, nkv, bs)).astype(np.float32)
    kv[..., hs:hs + 4] = ks.view(np.uint8).reshape(num_blocks, nkv, bs, 4)
    kv[..., hs + 4:hs + 4 + half] = rng.integers(0, 256, size=(num_blocks, nkv, bs, half), dtype=np.uint8)
    kv[..., hs + 4 + half:] = int4_words(rng, (num_blocks, nkv, bs)).view(np.uint8).reshape(num_blocks, nkv, bs, 4)
    return kv


def _rotate_rows(x: np.ndarray, seed: int = 0) -> np.ndarray:
    """x D H (unnormalised randomized Hadamard rotation of the last axis), the package's single_rht."""
    from ..attention.rht import signs_np
    hs = x.shape[-1]
    y = (x * signs_np(hs, seed)).astype(np.float64)
    h = 1
    while h < hs:      # fast Walsh-Hadamard transform over the last axis
        y = y.reshape(*y.shape[:-1], hs // (2 * h), 2, h)
        a, b = y[..., 0, :], y[..., 1, :]
        y = np.stack((a + b, a - b), axis=-2).reshape(*x.shape[:-1], hs)
        h *= 2
    return y.astype(np.float32)


def _single(name, rng, n, T, nblocks_total=None, scale=1.0 / 16) -> Workload:
    nb = -(-n // BS)
    total = nblocks_total or nb
    kv = fill_int4_cache(rng, total)
    table = rng.permutation(total)[:nb].astype(np.int32)[None, :]
    q = bf16_bits(rng.standard_normal((T, NQ, HS)).astype(np.float32))
    return Workload(name, kv, "int4", q, np.array([0, T], np.int32), np.array([n], np.int32), table, scale)


def make(name: str, *, small: bool = False) -> Workload:
    """The named workload. small=True shrinks context lengths 16x (parity tests) keeping every other property."""
    idx = WORKLOADS.index(name)
    rng = np.random.Generator(np.random.PCG64(1000 + idx))
    div = 16 if small else 1
    if name == "decode-int4-4k-t1":
        return _single(name, rng, 4096 // div, 1)
    if name == "decode-int4-128k-t2":
        return _single(name, rng, 131072 // div, 2)
    if name == "decode-int4-256k-t4":
        return _single(name, rng, 262144 // div, 4)
    if name in ("prefill-int4-128k-c1024", "prefill-k8v4-128k-c1024", "prefill-int4-h512-128k-c1024",
                "prefill-int4-g16-32k-c1024", "prefill-int4-g8-128k-c1024", "prefill-int4-g4-128k-c1024"):
        k8v4 = name.startswith("prefill-k8v4")
        shapes = {"-h512-": (16, 2, 512), "-g16-": (32, 2, HS), "-g8-": (64, 8, 128), "-g4-": (32, 8, 128)}
        nq, nkv, hs = next((v for k, v in shapes.items() if k in name), (NQ, NKV, HS))
        cached, chunk = (32768 if "-32k-" in name else 131072) // div, 1024 // (4 if small else 1)
        n = cached + chunk
        nb = -(-n // BS)
        kv = fill_k8v4_cache(rng, nb, nkv, BS, hs) if k8v4 else fill_int4_cache(rng, nb, nkv, BS, hs)
        table = rng.permutation(nb).astype(np.int32)
        q = bf16_bits(rng.standard_normal((chunk, nq, hs)).astype(np.float32))
        nk = bf16_bits(rng.standard_normal((chunk, nkv, hs)).astype(np.float32))
        nv = bf16_bits(rng.standard_normal((chunk, nkv, hs)).astype(np.float32))
        pos = np.arange(cached, n)
        slots = (table[pos // BS].astype(np.int64) * BS + pos % BS)
        return Workload(name, kv, "int8" if k8v4 else "int4", q, np.array([0, chunk], np.int32),
                        np.array([n], np.int32), table[None, :], hs ** -0.5, head_size=hs, num_q_heads=nq,
                        num_kv_heads=nkv, new_key=nk, new_value=nv, new_slots=slots, meta={"cached": cached})
    if name == "decode-k8v4-ragged-b32":
        seqs = 32
        T = rng.integers(1, 3, size=seqs)
        n = np.clip(rng.lognormal(np.log(16384), 1.0, size=seqs), 2048, 65536).astype(np.int64) // div
        n = np.maximum(n, T)
        nb = -(-n // BS)
        total = int(nb.sum())
        kv = fill_k8v4_cache(rng, total)
        pool = rng.permutation(total).astype(np.int32)
        width = int(nb.max())
        table = np.zeros((seqs, width), np.int32)
        at = 0
        for i in range(seqs):
            table[i, :nb[i]] = pool[at:at + nb[i]]
            at += nb[i]
        q = _rotate_rows(rng.standard_normal((int(T.sum()), NQ, HS)).astype(np.float32))
        cu = np.concatenate(([0], np.cumsum(T))).astype(np.int32)
        return Workload(name, kv, "int8", bf16_bits(q), cu, n.astype(np.int32), table, 1.0 / 16 / HS,
                        meta={"sum_n": int(n.sum()), "sum_T": int(T.sum()), "mu": float(np.log(16384)),
                              "sigma": 1.0})
    raise KeyError(name)


def cache_bytes(w: Workload) -> int:
    """Algorithmic HBM bytes of one decode / prefill call: the KV cells every query reads, the block-table entries,
    q and out (segment partials excluded)."""
    cell = w.kv.shape[3]
    nb = -(-w.seqused_k.astype(np.int64) // w.block_size)
    return int(w.seqused_k.astype(np.int64).sum() * w.num_kv_heads * cell + 4 * nb.sum()
               + 2 * w.q.size * 2)


def to_device(w: Workload, device):
    """Torch tensors of the workload on `device`: dict with the byte cache, its views and the metadata."""
    import torch

    from ..attention import k8v4_kv
    kv = torch.from_numpy(w.kv).to(device)
    if w.key_format == "int8":
        kc, vc, ks, vs = k8v4_kv.views(kv, w.head_size)
    else:
        kc, vc, ks, vs = k8v4_kv.int4_views(kv, w.head_size)
    q = torch.from_numpy(w.q.view(np.int16)).to(device).view(torch.bfloat16)
    d = dict(kv=kv, k_cache=kc, v_cache=vc, k_scale_cache=ks, v_scale_cache=vs, q=q,
             cu_seqlens_q=torch.from_numpy(w.cu_seqlens_q).to(device),
             seqused_k=torch.from_numpy(w.seqused_k).to(device),
             block_table=torch.from_numpy(w.block_table).to(device))
    if w.new_key is not None:
        d["new_key"] = torch.from_numpy(w.new_key.view(np.int16)).to(device).view(torch.bfloat16)
        d["new_value"] = torch.from_numpy(w.new_value.view(np.int16)).to(device).view(torch.bfloat16)
        d["new_slots"] = torch.from_numpy(w.new_slots).to(device)
    return d
