"""Writes tests/golden/int4_small.npz: a small int4_per_token_head case (24 query / 4 KV heads, head 256, block 16,
96 cached tokens over a permuted block table) with its expected results from the oracle.

Contents:
  cache (uint8 blocks x heads x slots x 264), table (int32), n, scale;
  decode: q_decode (bf16 bits, 2 tokens), decode_emu / decode_ref (fp16: the oracle's emulation of the reference
          kernel and the fp64 closed form, rounded to fp16), decode_segments;
  prefill: q_prefill (bf16 bits, the last 4 positions), prefill_emu / prefill_ref (fp16);
  unpack: unpack_start, unpack_key / unpack_value (bf16 bits of positions [start, start + 16));
  store: store_key / store_value (bf16 bits, 4 tokens, some rows all zero or constant), store_slots, store_cells
         (uint8 cells after the store).

The fixture is produced by the oracle only (no reference code runs); tests/test_golden.py checks that the oracle
still reproduces it exactly and that the HIP kernels meet it.

    python tests/golden/make_fixtures.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [REPO, os.path.dirname(HERE)]

from oracle import qp_oracle as O  # noqa: E402
from qp_testlib import random_cache  # noqa: E402

PATH = os.path.join(HERE, "int4_small.npz")
NQ, NKV, HS, BS, N = 24, 4, 256, 16, 96


def build():
    rng = np.random.default_rng(20260)
    nb = N // BS + 1
    kv, v = random_cache(rng, nb, NKV, BS, HS, "int4", "hnd")
    table = rng.permutation(nb).astype(np.int32)[:N // BS]
    scale = HS ** -0.5
    f = {"cache": np.ascontiguousarray(kv), "table": table, "n": np.int32(N), "scale": np.float32(scale)}
    q = O.f32_to_bf16_bits(rng.standard_normal((2, NQ, HS)).astype(np.float32))
    qf = O.bf16_bits_to_f32(q)
    K, V = O.dequant_f64(v, table, N)
    f["q_decode"] = q
    f["decode_segments"] = np.int32(3)
    f["decode_emu"] = O.decode_emulated(qf, v, table, N, scale, num_segments=3, tile=32).astype(np.float16)
    f["decode_ref"] = O.attention_f64(qf, K, V, N, scale).astype(np.float16)
    qp = O.f32_to_bf16_bits(rng.standard_normal((4, NQ, HS)).astype(np.float32))
    qpf = O.bf16_bits_to_f32(qp)
    f["q_prefill"] = qp
    f["prefill_emu"] = O.decode_emulated(qpf, v, table, N, scale, num_segments=1, tile=64).astype(np.float16)
    f["prefill_ref"] = O.attention_f64(qpf, K, V, N, scale).astype(np.float16)
    f["unpack_start"] = np.int32(21)
    f["unpack_key"] = O.unpack_segment(v, table, 21, 16, "key")
    f["unpack_value"] = O.unpack_segment(v, table, 21, 16, "value")
    sk = O.f32_to_bf16_bits(rng.standard_normal((4, NKV, HS)).astype(np.float32))
    sv = O.f32_to_bf16_bits(rng.standard_normal((4, NKV, HS)).astype(np.float32))
    # rows without spread (all zero, constant): the store's 1e-6 scale floors set their words and codes
    for (t, h), c in zip([(0, 1), (2, 2), (3, 3), (2, 0)], [0.0, 0.5, -0.5, 1e-5]):
        sk[t, h] = O.f32_to_bf16_bits(np.full(HS, c, np.float32))
        sv[t, (h + 1) % NKV] = O.f32_to_bf16_bits(np.full(HS, c, np.float32))
    slots = np.array([3, -1, 17, 30], np.int64)          # block 0 slot 3, skipped, block 1 slot 1, block 1 slot 14
    fresh = O.new_cache(2, NKV, BS, O.int4_cell_bytes(HS))
    O.store(O.int4_views(fresh, HS), O.bf16_bits_to_f32(sk), O.bf16_bits_to_f32(sv), slots)
    f["store_key"], f["store_value"], f["store_slots"], f["store_cells"] = sk, sv, slots, fresh
    return f


def main():
    np.savez_compressed(PATH, **build())
    print(PATH, os.path.getsize(PATH), "bytes")


if __name__ == "__main__":
    main()
