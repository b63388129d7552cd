"""Parity of the HIP kernel of the reference's single-kernel alternative prefill (`prefill_sequence_i8` / `_attn_i8`,
int4_prefill.py:95-200: an int8 split of the query, integer QK^T on the raw key nibbles, fp16 PV) with the oracle's
restatement of that arithmetic (`prefill_i8_emulated`), on seeded int4 caches.

Bars: within 1e-2 relative of the emulation (Frobenius and every (token, head) row), as for the other kernels against
the reference's own, and within 0.5 % of the fp64 closed form. The reference accumulates each 64-key tile's PV in fp16
and the kernel in fp32, so the two agree to tolerance, not bit for bit.
"""
import numpy as np
import pytest

from oracle import qp_oracle as O
from qp_testlib import assert_emulation, bf16_tensor, i32, random_cache, to_f32, torch_cache

pytestmark = pytest.mark.gpu


def _case(device, rng, lens, hs=256, nq=24, nkv=4, bs=16, layout="hnd", splits=0, big_keys=()):
    """lens = [(T_i, n_i)]: one batched prefill_attention_i8 call; returns (gpu out, emulation, fp64 reference)."""
    import torch

    from vllm_quantpack.attention import int4_prefill
    nbs = [-(-n // bs) for _, n in lens]
    total = sum(nbs) + 2
    kv, v = random_cache(rng, total, nkv, bs, hs, "int4", layout)
    pool = rng.permutation(total).astype(np.int32)
    table = np.zeros((len(lens), max(nbs)), np.int32)
    at = 0
    for i, nb in enumerate(nbs):
        table[i, :nb] = pool[at:at + nb]
        at += nb
    for pos, sc in big_keys:
        for i in range(len(lens)):
            words = v.key_word[table[i, pos // bs], pos % bs]
            words[:] = (words & np.uint32(0xF)) | (np.float32(sc).view(np.uint32) & np.uint32(0xFFFFFFF0))
    _, (kc, vc, ks, vs) = torch_cache(kv, hs, "int4", device)
    Ts = [t for t, _ in lens]
    q = O.f32_to_bf16_bits(rng.standard_normal((sum(Ts), nq, hs)).astype(np.float32))
    cu = np.concatenate(([0], np.cumsum(Ts))).astype(np.int32)
    scale = hs ** -0.5
    qt = bf16_tensor(q, device)
    out = torch.full_like(qt, float("nan"))
    int4_prefill.prefill_attention_i8(qt, kc, vc, ks, vs, out, cu_seqlens_q=i32(cu, device),
                                      seqused_k=i32([n for _, n in lens], device), block_table=i32(table, device),
                                      max_seqlen_q=max(Ts), softmax_scale=scale, num_splits=splits)
    torch.cuda.synchronize()
    qf = O.bf16_bits_to_f32(q)
    emus, refs = [], []
    for i, (T, n) in enumerate(lens):
        emus.append(O.prefill_i8_emulated(q[cu[i]:cu[i + 1]], v, table[i], n, scale))
        K, V = O.dequant_f64(v, table[i], n)
        refs.append(O.attention_f64(qf[cu[i]:cu[i + 1]], K, V, n, scale))
    return to_f32(out), O.round_bf16(np.concatenate(emus).astype(np.float32)), np.concatenate(refs)


@pytest.mark.parametrize("hs,nq,nkv", [(256, 24, 4), (128, 16, 2), (512, 16, 2)])
def test_prefill_i8_matches_the_emulation(device, hs, nq, nkv):
    rng = np.random.default_rng(700 + hs)
    out, emu, ref = _case(device, rng, [(100, 3000)], hs=hs, nq=nq, nkv=nkv)
    assert np.isfinite(out).all()
    assert_emulation(out, emu, f"head {hs}")
    assert O.relerr(out, ref) < 5e-3, O.relerr(out, ref)


@pytest.mark.parametrize("splits", [1, 3])
@pytest.mark.parametrize("layout,bs", [("hnd", 16), ("nhd", 48)])
def test_prefill_i8_ragged_batch(device, splits, layout, bs):
    """Three sequences of different chunk and context lengths (one whose chunk is its whole context), key splits
    merged by the split-KV merge, span and strided cache layouts."""
    rng = np.random.default_rng(710 + splits)
    out, emu, ref = _case(device, rng, [(48, 2600), (7, 300), (33, 33)], layout=layout, bs=bs, splits=splits)
    assert np.isfinite(out).all()
    assert_emulation(out, emu, (splits, layout, bs))
    assert O.relerr(out, ref) < 5e-3, O.relerr(out, ref)


def test_prefill_i8_scores_far_above_the_first_tile(device):
    """Keys whose scales sit 2^7 to 2^12 above the others raise the rows' running maxima well past the headroom of
    8 log2 units, several times per row: every rescale must keep acc, l and the fp16 probabilities consistent."""
    rng = np.random.default_rng(720)
    big = [(300, 2.0 ** 4), (900, 2.0 ** 6), (1700, 2.0 ** 9)]
    out, emu, ref = _case(device, rng, [(64, 2000)], big_keys=big)
    assert np.isfinite(out).all()
    assert_emulation(out, emu)
    assert O.relerr(out, ref) < 5e-3, O.relerr(out, ref)


def test_prefill_i8_repeats_bit_for_bit(device):
    """Five identical calls (key splits merged) give the same bits: the kernel's work split does not follow timing."""
    import torch

    from vllm_quantpack.attention import int4_prefill
    rng = np.random.default_rng(735)
    hs, nq, nkv, bs, n, T = 256, 24, 4, 16, 3000, 40
    nb = -(-n // bs)
    kv, _ = random_cache(rng, nb, nkv, bs, hs, "int4")
    _, (kc, vc, ks, vs) = torch_cache(kv, hs, "int4", device)
    q = bf16_tensor(O.f32_to_bf16_bits(rng.standard_normal((T, nq, hs)).astype(np.float32)), device)
    kw = dict(cu_seqlens_q=i32([0, T], device), seqused_k=i32([n], device),
              block_table=i32(rng.permutation(nb).astype(np.int32)[None], device), max_seqlen_q=T,
              softmax_scale=hs ** -0.5, num_splits=3)
    outs = []
    for _ in range(5):
        out = torch.full_like(q, float("nan"))
        int4_prefill.prefill_attention_i8(q, kc, vc, ks, vs, out, **kw)
        torch.cuda.synchronize()
        outs.append(to_f32(out))
    assert np.isfinite(outs[0]).all()
    for k in range(1, 5):
        assert np.array_equal(outs[k], outs[0]), (k, int((outs[k] != outs[0]).sum()))


def test_prefill_sequence_i8_contract(device):
    """The reference's call (int4_prefill.py:176): one chunk's rotated queries, the nibble and scale views, a block
    row and n; the output in the queries' dtype, against the emulation."""
    import torch

    from vllm_quantpack.attention import int4_prefill
    rng = np.random.default_rng(730)
    hs, nq, nkv, bs, n, T = 256, 24, 4, 16, 1500, 80
    nb = -(-n // bs) + 1
    kv, v = random_cache(rng, nb, nkv, bs, hs, "int4")
    row = rng.permutation(nb)[: -(-n // bs)].astype(np.int32)
    _, (kc, vc, ks, vs) = torch_cache(kv, hs, "int4", device)
    q = O.f32_to_bf16_bits(rng.standard_normal((T, nq, hs)).astype(np.float32))
    out = int4_prefill.prefill_sequence_i8(bf16_tensor(q, device), kc, vc, ks, vs, i32(row, device), n, hs ** -0.5,
                                           block_m=64, block_n=64, num_warps=8, num_stages=2)
    torch.cuda.synchronize()
    assert out.dtype == torch.bfloat16 and out.shape == (T, nq, hs)
    emu = O.round_bf16(O.prefill_i8_emulated(q, v, row, n, hs ** -0.5).astype(np.float32))
    assert_emulation(to_f32(out), emu)


def test_prefill_i8_rejects_int8_keys(device):
    import torch

    from vllm_quantpack.attention import int4_prefill
    rng = np.random.default_rng(740)
    kv, v = random_cache(rng, 4, 4, 16, 256, "int8")
    _, (kc, vc, ks, vs) = torch_cache(kv, 256, "int8", device)
    q = torch.zeros((8, 24, 256), dtype=torch.bfloat16, device=device)
    with pytest.raises(NotImplementedError, match="int4 caches only"):
        int4_prefill.prefill_attention_i8(q, kc, vc, ks, vs, torch.empty_like(q), cu_seqlens_q=i32([0, 8], device),
                                          seqused_k=i32([40], device), block_table=i32([[0, 1, 2]], device),
                                          max_seqlen_q=8, softmax_scale=0.0625)
