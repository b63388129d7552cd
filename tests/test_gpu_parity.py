"""Parity of the HIP kernels with the CPU oracle, on seeded inputs (runs on the MI355X through the C ABI).

Bars: the unpack and the store are bit-exact; attention is within 1e-2 relative of the oracle's emulation of the
reference's exact kernel, both as the reference's own test metric (Frobenius over the whole output,
tests/test_int4_kv.py:160-161,190) and row by row (the largest error of any (token, head) output vector), and within
0.5 % (Frobenius) of the fp64 closed form.
"""
import numpy as np
import pytest

from oracle import qp_oracle as O
from test_oracle_pinning import degenerate_rows, fma_rows
from qp_testlib import assert_emulation, bf16_tensor, i32, random_cache, run_decode, to_f32, torch_cache

pytestmark = pytest.mark.gpu

NQ, NKV, HS = 24, 4, 256


# ---------------------------------------------------------------------------------------------------- unpack

@pytest.mark.parametrize("fmt,which", [("int4", "key"), ("int4", "value"), ("int8", "key")])
@pytest.mark.parametrize("layout", ["hnd", "nhd"])
@pytest.mark.parametrize("bs", [16, 3072])
def test_unpack_segment_bit_exact(device, fmt, which, layout, bs):
    import torch

    from vllm_quantpack.attention import int4_prefill
    rng = np.random.default_rng(hash((fmt, which, layout, bs)) % 2**32)
    nb = 40 if bs == 16 else 3
    kv, v = random_cache(rng, nb, NKV, bs, HS, fmt, layout)
    _, (kc, vc, ks, vs) = torch_cache(kv, HS, fmt, device)
    row = rng.permutation(nb).astype(np.int32)
    start, length = (37, 500) if bs == 16 else (1000, 4500)
    out = torch.full((length + 3, NKV, HS), float("nan"), dtype=torch.bfloat16, device=device)
    cache, scales = (kc, ks) if which == "key" else (vc, vs)
    int4_prefill.unpack_segment(cache, scales, i32(row, device), start, length, out)
    torch.cuda.synchronize()
    got = out[:length].view(torch.int16).cpu().numpy().view(np.uint16)
    want = O.unpack_segment(v, row, start, length, which)
    assert (got == want).all()
    assert torch.isnan(out[length:].float()).all()        # nothing written past `length`


# ---------------------------------------------------------------------------------------------------- decode

def _decode_case(device, rng, fmt, lens, layout="hnd", bs=16, segments=8, nq=NQ, nkv=NKV, hs=HS, scale=None,
                 big_keys=()):
    """lens = [(T_i, n_i)]: one call over the batch; returns (gpu out, oracle emulation, fp64 refs). big_keys =
    [(first position, count, factor)] multiplies the key scales of those positions of every sequence by factor."""
    nbs = [-(-n // bs) for _, n in lens]
    total = sum(nbs) + 3
    kv, v = random_cache(rng, total, nkv, bs, hs, fmt, layout)
    pool = rng.permutation(total).astype(np.int32)
    width = max(nbs)
    table = np.zeros((len(lens), width), np.int32)
    at = 0
    for i, nb in enumerate(nbs):
        table[i, :nb] = pool[at:at + nb]
        at += nb
    for first, count, factor in big_keys:
        for i in range(len(lens)):
            for pos in range(first, first + count):
                blk, slot = table[i, pos // bs], pos % bs
                words = v.key_word[blk, slot]
                if fmt == "int4":
                    big = (words & np.uint32(0xFFFFFFF0)).view(np.float32) * np.float32(factor)
                    words[:] = (big.view(np.uint32) & np.uint32(0xFFFFFFF0)) | (words & np.uint32(0xF))
                else:
                    words[:] = (words.view(np.float32) * np.float32(factor)).view(np.uint32)
    _, views = torch_cache(kv, hs, fmt, device)
    Ts = [t for t, _ in lens]
    q = O.f32_to_bf16_bits(rng.standard_normal((sum(Ts), nq, hs)).astype(np.float32))
    cu = np.concatenate(([0], np.cumsum(Ts))).astype(np.int32)
    used = np.array([n for _, n in lens], np.int32)
    scale = scale or hs ** -0.5
    out, bufs = run_decode(views, bf16_tensor(q, device), i32(cu, device), i32(used, device), i32(table, device),
                           max(Ts), scale, segments, device)
    qf = O.bf16_bits_to_f32(q)
    emus, refs = [], []
    for i, (T, n) in enumerate(lens):
        qs = qf[cu[i]:cu[i + 1]]
        emus.append(O.decode_emulated(qs, v, table[i], n, scale, num_segments=segments, tile=32))
        K, V = O.dequant_f64(v, table[i], n)
        refs.append(O.attention_f64(qs, K, V, n, scale))
    return out, np.concatenate(emus), np.concatenate(refs), dict(bufs=bufs, views=v, table=table, q=qf)


@pytest.mark.parametrize("fmt", ["int4", "int8"])
@pytest.mark.parametrize("T", [1, 2, 3, 4])
def test_decode_matches_oracle(device, fmt, T):
    rng = np.random.default_rng(100 + T + (10 if fmt == "int8" else 0))
    out, emu, ref, _ = _decode_case(device, rng, fmt, [(T, 5003)], segments=7)
    assert_emulation(out, emu)
    assert O.relerr(out, ref) < 5e-3, O.relerr(out, ref)


@pytest.mark.parametrize("fmt", ["int4", "int8"])
@pytest.mark.parametrize("T", [1, 4])
def test_decode_scores_far_above_the_running_maximum(device, fmt, T):
    """Key blocks with larger key scales. The first two (int4 8x and 20x, int8 2.5x and 5x) give scores 10-60 (log2
    units) above the maximum the waves hold when they reach them: inside the lazy maximum's 64-unit headroom, so they
    accumulate with probabilities up to 2^60 while the keys before them keep a share of the probability mass (median
    1-12 %, up to 38 % and more per row), which a mis-scaled sum or accumulator shows against fp64. A second case adds
    a third block (int4 256x, int8 64x) up to 250-500 units above, in a chunk that some wave claims after others of its
    own (chunk 10 of its segment): the accumulators are rescaled mid-segment (by assembly on AGPR tiles for the two
    row tiles of T = 4: 4 tokens x 6 query heads per KV head)."""
    f1, f2, f3 = (8.0, 20.0, 256.0) if fmt == "int4" else (2.5, 5.0, 64.0)
    for big in ([(1504, 16, f1), (2900, 8, f2)], [(1504, 16, f1), (2900, 8, f2), (3790, 8, f3)]):
        rng = np.random.default_rng(400 + T + (10 if fmt == "int8" else 0))
        out, emu, ref, _ = _decode_case(device, rng, fmt, [(T, 4000)], segments=7, nq=12, nkv=2, big_keys=big)
        assert np.isfinite(out).all()
        assert O.relerr(out, ref) < 5e-3, (len(big), O.relerr(out, ref))
        assert_emulation(out, emu)


@pytest.mark.parametrize("fmt,segments,lens", [("int4", 8, [8192]), ("int4", 5, [8192]), ("int4", 64, [32768]),
                                               ("int8", 16, [8192, 32768])])
def test_decode_counts_every_chunk_once(device, fmt, segments, lens):
    """Exact key coverage of the split-KV decode. Zero queries make the softmax uniform, and the value codes light
    channel c % 256 for the keys of 32-key chunk c (code 1 there, 0 elsewhere; zero point 0, scale 1), so every
    output channel must equal 32 * (chunks on it) / n exactly, launch after launch: a chunk skipped or taken twice
    (by two waves, or by two segments) moves its channel by a quarter or more, below any tolerance-based test's
    reach at these lengths. 5 segments leave a partial last segment; the batch covers two sequences at once."""
    import torch
    hs, nkv, nq, bs = 256, 2, 4, 16
    nbs = [n // bs for n in lens]
    cell = O.int4_cell_bytes(hs) if fmt == "int4" else O.k8v4_cell_bytes(hs)
    kv = O.new_cache(sum(nbs), nkv, bs, cell, "hnd")
    v = O.int4_views(kv, hs) if fmt == "int4" else O.k8v4_views(kv, hs)
    table = np.zeros((len(lens), max(nbs)), np.int32)
    at = 0
    for i, (n, nb) in enumerate(zip(lens, nbs)):
        table[i, :nb] = np.arange(at, at + nb)
        keys = np.arange(n)
        ch = (keys // 32) % hs
        v.value[at + keys // bs, keys % bs, :, ch // 2] = (1 << (4 * (ch % 2))).astype(np.uint8)[:, None]
        at += nb
    v.value_word[...] = np.float32(1.0).view(np.uint32)
    v.key_word[...] = np.float32(1.0).view(np.uint32)
    _, views = torch_cache(kv, hs, fmt, device)
    q = torch.zeros((len(lens), nq, hs), dtype=torch.bfloat16, device=device)
    cu = i32(np.arange(len(lens) + 1), device)
    expect = np.zeros((len(lens), nq, hs), np.float32)
    for i, n in enumerate(lens):
        per = np.bincount((np.arange(n // 32)) % hs, minlength=hs)
        expect[i] = (32.0 * per / n)[None, :]
    for _ in range(3):
        out, _ = run_decode(views, q, cu, i32(lens, device), i32(table, device), 1, hs ** -0.5, segments, device)
        assert np.array_equal(out, expect), np.abs(out - expect).max()


@pytest.mark.parametrize("layout,bs", [("nhd", 16), ("hnd", 32), ("hnd", 3072), ("nhd", 48)])
def test_decode_layouts_and_block_sizes(device, layout, bs):
    rng = np.random.default_rng(7 + bs)
    out, emu, ref, _ = _decode_case(device, rng, "int4", [(2, 4100)], layout=layout, bs=bs, segments=5)
    assert_emulation(out, emu)
    assert O.relerr(out, ref) < 5e-3


@pytest.mark.parametrize("fmt,T", [("int4", 1), ("int4", 2), ("int4", 4), ("int8", 2)])
def test_decode_span_and_row_loaders_agree(device, fmt, T):
    """The HND page-span kernel (HBM -> LDS copies) and the generic strided-row kernel on the same cache contents:
    the same seed fills the same logical cells, stored HND (whole 16-cell page runs, the span kernel) and NHD (slots of
    one head strided by the KV heads, the strided kernel)."""
    a, emu, ref, _ = _decode_case(device, np.random.default_rng(5), fmt, [(T, 3000), (1, 200)], segments=9)
    b, _, _, _ = _decode_case(device, np.random.default_rng(5), fmt, [(T, 3000), (1, 200)], layout="nhd", segments=9)
    assert_emulation(a, emu)
    assert_emulation(b, emu)
    assert O.relerr(a, ref) < 5e-3 and O.relerr(b, ref) < 5e-3
    assert O.relerr(a, b) < 5e-3


def test_decode_ragged_batch(device):
    """Sequences of 4, 3, 1 and 2 query tokens and very different lengths in one call (tests/test_int4_kv.py:230-249
    with k8v4 keys, as the ragged k8v4 workload)."""
    rng = np.random.default_rng(21)
    lens = [(4, 2000), (3, 900), (1, 3333), (2, 64), (1, 1)]
    out, emu, ref, _ = _decode_case(device, rng, "int8", lens, segments=16)
    at = 0
    for T, n in lens:
        sl = slice(at, at + T)
        assert_emulation(out[sl], emu[sl], (T, n))
        assert O.relerr(out[sl], ref[sl]) < 5e-3, (T, n)
        at += T


@pytest.mark.parametrize("fmt", ["int4", "int8"])
def test_decode_short_contexts(device, fmt):
    """Contexts of a few keys: as many keys as query tokens (each token sees only the keys up to itself), one
    partial 32-key chunk, a chunk and one key, with most of the 16 segments of every sequence empty. 6 query heads
    per KV head make 24 query rows (two row tiles) at 4 tokens."""
    rng = np.random.default_rng(71 + (10 if fmt == "int8" else 0))
    lens = [(1, 1), (2, 2), (4, 4), (3, 17), (1, 33), (4, 31), (2, 47)]
    out, emu, ref, _ = _decode_case(device, rng, fmt, lens, nq=12, nkv=2, segments=16)
    assert np.isfinite(out).all()
    at = 0
    for T, n in lens:
        sl = slice(at, at + T)
        assert_emulation(out[sl], emu[sl], (T, n))
        assert O.relerr(out[sl], ref[sl]) < 5e-3, (T, n)
        at += T


def test_decode_segment_count_invariance(device):
    rng = np.random.default_rng(31)
    outs = []
    for S in (1, 4, 64, 200):
        out, _, ref, _ = _decode_case(device, np.random.default_rng(31), "int4", [(2, 6000)], segments=S)
        outs.append(out)
        assert O.relerr(out, ref) < 5e-3, S
    for o in outs[1:]:      # each is ~2e-3 from fp64 (bf16 P_v and output rounding): independent roundings
        assert O.relerr(o, outs[0]) < 5e-3


def test_decode_partials_match_the_emulation(device):
    """Per-segment (acc, m, l) against the emulation run with the kernel's 32-key segmentation."""
    rng = np.random.default_rng(41)
    T, n, S = 2, 3000, 6
    out, emu, ref, ctx = _decode_case(device, rng, "int4", [(T, n)], segments=S)
    so, sm, ss = ctx["bufs"]
    acc, m, l_ = O.decode_partials(ctx["q"], ctx["views"], ctx["table"][0], n, HS ** -0.5, S, tile=32)
    active = -(-n // O.segment_length(n, S, 32))
    gm, gl, go = to_f32(sm)[:, :, :active], to_f32(ss)[:, :, :active], to_f32(so)[:, :, :active]
    assert np.isfinite(gm).all() and np.isfinite(gl).all() and np.isfinite(go).all()
    # the kernel may keep a different (lazily updated) reference maximum: compare rescaled to the oracle's
    f = np.exp2(gm - m[:, :, :active])
    assert np.allclose(gl * f, l_[:, :, :active], rtol=1e-3)
    assert O.relerr(go * f[..., None], acc[:, :, :active]) < 1e-2


@pytest.mark.parametrize("fmt,lens,segments", [("int4", [(2, 4096)], 64), ("int4", [(1, 900)], 8),
                                                ("int8", [(1, 2100), (2, 5000), (1, 3000), (2, 2048)], 16)],
                         ids=["mtp1-4096", "decode-900", "k8v4-ragged"])
def test_merge_lse_matches_the_oracle(device, fmt, lens, segments):
    """The merge's optional lse output (natural log, per token and query head) against the oracle's fold of the
    emulated segment statistics and against the fp64 logsumexp of the scores over the visible keys: the per-row
    log-sum-exp a caller folds with other partial attentions (the `logaddexp` merge of int4_prefill.py:223-230)."""
    import torch
    from scipy.special import logsumexp

    from vllm_quantpack.attention import int4_kv
    rng = np.random.default_rng(sum(t * n for t, n in lens) % 1000)
    _, _, _, ctx = _decode_case(device, rng, fmt, lens, segments=segments)
    so, sm, ss = ctx["bufs"]
    Ts = [t for t, _ in lens]
    cu = np.concatenate(([0], np.cumsum(Ts))).astype(np.int32)
    lse = torch.full((sum(Ts), NQ), float("nan"), dtype=torch.float32, device=device)
    out = torch.empty((sum(Ts), NQ, HS), dtype=torch.bfloat16, device=device)
    cu_t, used_t = i32(cu, device), i32([n for _, n in lens], device)   # held until the merge has run
    margs = int4_kv._hip.MergeArgs(so.data_ptr(), int4_kv._hip.I64x3(*so.stride()[:3]), sm.data_ptr(),
                                   ss.data_ptr(), int4_kv._hip.I64x2(sm.stride(0), sm.stride(1)), cu_t.data_ptr(),
                                   used_t.data_ptr(), len(lens), sum(Ts), NQ, HS, segments, out.data_ptr(),
                                   int4_kv._hip.I64x2(out.stride(0), out.stride(1)), lse.data_ptr(),
                                   int4_kv._hip.I64x2(lse.stride(0), lse.stride(1)), None, 1.0)
    int4_kv._hip.check(int4_kv._hip.lib().qp_merge_segments(margs, int4_kv._hip.stream_of(out)), "merge")
    torch.cuda.synchronize()
    got = to_f32(lse)
    scale = HS ** -0.5
    for i, (T, n) in enumerate(lens):
        qs = ctx["q"][cu[i]:cu[i + 1]]
        _, m, l_ = O.decode_partials(qs, ctx["views"], ctx["table"][i], n, scale, segments, tile=32)
        want = O.merge_lse(m, l_)
        assert np.abs(got[cu[i]:cu[i + 1]] - want).max() < 1e-4, i
        K, _ = O.dequant_f64(ctx["views"], ctx["table"][i], n)
        for t in range(T):
            vis = n - T + t + 1
            for h in range(0, NQ, 5):
                ref = logsumexp(scale * (K[:vis, h // (NQ // NKV)] @ qs[t, h].astype(np.float64)))
                assert abs(got[cu[i] + t, h] - ref) < 1e-4, (i, t, h)


def _dead_value_cache(rng, fmt, n, bs=16, live=2):
    """A cache whose value codes equal their zero points (value 0) on all keys but `live` ones."""
    nb = -(-n // bs)
    kv, v = random_cache(rng, nb, NKV, bs, HS, fmt)
    zp = (v.value_word & np.uint32(0xF)).astype(np.uint8)
    v.value[...] = zp[..., None] | (zp[..., None] << 4)
    for pos in rng.choice(n, live, replace=False):
        v.value[pos // bs, pos % bs] = rng.integers(0, 256, v.value.shape[-1:], dtype=np.uint8)
    return kv, v, np.arange(nb, dtype=np.int32)


@pytest.mark.parametrize("fmt", ["int4", "int8"])
def test_zero_point_sum_uses_the_rounded_probabilities(device, fmt):
    """int4_kv.py:90-94 through both kernels: the zero-point correction sum_j P16_j zp_j must come from the same
    bf16-rounded P16 = bf16(P s_v) that the PV product takes. With values at their zero points on all keys but two,
    the true output is small and a sum on the unrounded P s_v misses fp64 by 3-28 % (the oracle's planted variant);
    both the decode and the prefill kernel stay within the usual bar."""
    import torch

    from vllm_quantpack.attention import int4_prefill
    rng = np.random.default_rng(95 + (1 if fmt == "int8" else 0))
    n = 3000
    kv, v, table = _dead_value_cache(rng, fmt, n)
    _, (kc, vc, ks, vs) = torch_cache(kv, HS, fmt, device)
    for T in (2, 64):
        q = O.f32_to_bf16_bits(rng.standard_normal((T, NQ, HS)).astype(np.float32))
        qf = O.bf16_bits_to_f32(q)
        K, V = O.dequant_f64(v, table, n)
        ref = O.attention_f64(qf, K, V, n, HS ** -0.5)
        if T <= 4:
            out, _ = run_decode((kc, vc, ks, vs), bf16_tensor(q, device), i32([0, T], device), i32([n], device),
                                i32(table[None], device), T, HS ** -0.5, 16, device)
        else:
            o = torch.empty((T, NQ, HS), dtype=torch.bfloat16, device=device)
            int4_prefill.prefill_attention(bf16_tensor(q, device), kc, vc, ks, vs, o,
                                           cu_seqlens_q=i32([0, T], device), seqused_k=i32([n], device),
                                           block_table=i32(table[None], device), max_seqlen_q=T,
                                           softmax_scale=HS ** -0.5)
            torch.cuda.synchronize()
            out = to_f32(o)
        assert O.relerr(out, ref) < 5e-3, (T, O.relerr(out, ref))


def test_decode_plan_graph_replays(device):
    """DecodePlan recorded in a HIP graph: three replays, each after eager work that changes the query, each equal
    to an eager run on the same query and within the fp64 bar."""
    import torch

    from vllm_quantpack.attention import int4_kv
    rng = np.random.default_rng(71)
    T, n, S = 2, 4000, 16
    nb = -(-n // 16)
    kv, v = random_cache(rng, nb + 2, NKV, 16, HS, "int4", "hnd")
    _, (kc, vc, ks, vs) = torch_cache(kv, HS, "int4", device)
    table = rng.permutation(nb + 2).astype(np.int32)[None, :nb]
    cu, used, tab = i32([0, T], device), i32([n], device), i32(table, device)
    q = torch.empty((T, NQ, HS), dtype=torch.bfloat16, device=device)
    so = torch.empty((T, NQ, S, HS), dtype=torch.float32, device=device)
    sm = torch.empty((T, NQ, S), dtype=torch.float32, device=device)
    ss = torch.empty((T, NQ, S), dtype=torch.float32, device=device)
    out = torch.empty((T, NQ, HS), dtype=torch.bfloat16, device=device)
    kw = dict(cu_seqlens_q=cu, seqused_k=used, block_table=tab, max_seqlen_q=T, softmax_scale=HS ** -0.5,
              num_segments=S, softmax_segm_output=so, softmax_segm_max=sm, softmax_segm_expsum=ss)
    eager = int4_kv.DecodePlan(q, kc, vc, ks, vs, out, **kw)
    queries = [O.f32_to_bf16_bits(rng.standard_normal((T, NQ, HS)).astype(np.float32)) for _ in range(4)]
    q.copy_(bf16_tensor(queries[0], device))
    eager.run()                                        # warm up on the capture-free path first
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            captured = int4_kv.DecodePlan(q, kc, vc, ks, vs, out, **kw)   # launches on the capture stream
            captured.run()
    torch.cuda.synchronize()
    for qb in queries[1:]:
        q.copy_(bf16_tensor(qb, device))
        eager.run()
        torch.cuda.synchronize()
        want = to_f32(out).copy()
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = to_f32(out)
        assert np.array_equal(got, want)
        K, V = O.dequant_f64(v, table[0], n)
        assert O.relerr(got, O.attention_f64(O.bf16_bits_to_f32(qb), K, V, n, HS ** -0.5)) < 5e-3


@pytest.mark.parametrize("fmt", ["int4", "int8"])
@pytest.mark.parametrize("T", [1, 2, 3, 4])
def test_decode_head_512(device, fmt, T):
    """Head 512 with 8 query heads per KV head (Gemma 4 global layers: tests/test_int4_kv.py:194-210,
    tests/test_k8v4_kv.py:208-225). 3 and 4 tokens make 24 / 32 query rows: they run as workgroups of two tokens
    (one row tile each), the last group of 3 tokens holding a single token."""
    rng = np.random.default_rng(300 + T + (10 if fmt == "int8" else 0))
    out, emu, ref, _ = _decode_case(device, rng, fmt, [(T, 3000), (1, 900)], nq=16, nkv=2, hs=512, segments=6)
    assert_emulation(out, emu)
    assert O.relerr(out, ref) < 5e-3


@pytest.mark.parametrize("fmt,T,layout", [("int4", 1, "hnd"), ("int4", 2, "nhd"), ("int4", 3, "hnd"),
                                           ("int4", 4, "hnd"), ("int8", 1, "hnd"), ("int8", 4, "nhd")])
def test_decode_head_64(device, fmt, T, layout):
    """Head 64 (Llama 3.2 1B-class models: 8 query heads per KV head): 72-byte int4 and 104-byte k8v4 cells, one
    channel block of PV, two row tiles at 4 tokens; both loaders."""
    rng = np.random.default_rng(320 + T + (10 if fmt == "int8" else 0))
    out, emu, ref, _ = _decode_case(device, rng, fmt, [(T, 3000), (1, 900), (2, 17)], nq=16, nkv=2, hs=64,
                                    segments=6, layout=layout)
    assert_emulation(out, emu)
    assert O.relerr(out, ref) < 5e-3


@pytest.mark.parametrize("T", [1, 2])
def test_decode_head_512_row_loader(device, T):
    """Head 512 int4 cache stored NHD (slots of one head strided by the KV heads): the generic strided-row kernel,
    whose scale words are read through one lane-chosen pointer, against the same cells stored HND."""
    a, emu, ref, _ = _decode_case(device, np.random.default_rng(310 + T), "int4", [(T, 2500), (1, 700)], nq=16, nkv=2,
                                  hs=512, segments=5)
    b, _, _, _ = _decode_case(device, np.random.default_rng(310 + T), "int4", [(T, 2500), (1, 700)], nq=16, nkv=2,
                              hs=512, segments=5, layout="nhd")
    assert_emulation(b, emu)
    assert O.relerr(b, ref) < 5e-3
    assert O.relerr(a, b) < 5e-3


@pytest.mark.parametrize("fmt", ["int4", "int8"])
def test_decode_gqa_8_and_head_128(device, fmt):
    """Head 128, 8 query heads per KV head: 4 tokens are two row tiles (AGPR accumulators), 1 token one row tile
    (8 waves; one stage each with int8 keys)."""
    rng = np.random.default_rng(51 + (10 if fmt == "int8" else 0))
    out, emu, ref, _ = _decode_case(device, rng, fmt, [(4, 2500), (1, 700)], nq=16, nkv=2, hs=128, segments=9)
    assert_emulation(out, emu)
    assert O.relerr(out, ref) < 5e-3


# ------------------------------------------------------------------------------------------------------ store

@pytest.mark.parametrize("fmt", ["int4", "int8"])
@pytest.mark.parametrize("layout", ["hnd", "nhd"])
@pytest.mark.parametrize("hs", [256, 64])
def test_store_bit_exact(device, fmt, layout, hs):
    """Bit-exact stores; head 64 holds one channel per lane, so each int4 byte joins two lanes."""
    import torch

    from vllm_quantpack.attention import k8v4_kv
    HS = hs
    rng = np.random.default_rng(61)
    nb, bs, n = 20, 16, 200
    kv_np = O.new_cache(nb, NKV, bs, O.int4_cell_bytes(HS) if fmt == "int4" else O.k8v4_cell_bytes(HS), layout)
    t, (kc, vc, ks, vs) = torch_cache(kv_np, HS, fmt, device)
    key = O.f32_to_bf16_bits(rng.standard_normal((n, NKV, HS)).astype(np.float32) * 2)
    val = O.f32_to_bf16_bits(rng.standard_normal((n, NKV, HS)).astype(np.float32))
    # rows whose probe channel rounds differently under a fused multiply-add and a mul-then-add (int4 halves)
    rows, _ = fma_rows(HS)
    val[1:1 + len(rows), 0] = O.f32_to_bf16_bits(rows)
    if fmt == "int4":
        key[1:1 + len(rows), 1] = O.f32_to_bf16_bits(rows)
    # all-zero and constant rows, where the scale floors of both halves decide the word and the codes
    flat = degenerate_rows(HS)
    val[10:10 + len(flat), 2] = O.f32_to_bf16_bits(flat)
    key[10:10 + len(flat), 3] = O.f32_to_bf16_bits(flat)
    key[20:20 + len(flat)] = O.f32_to_bf16_bits(flat)[:, None, :]
    slots = rng.permutation(nb * bs)[:n].astype(np.int64)
    slots[::17] = -1
    k8v4_kv.store(None, bf16_tensor(key, device), bf16_tensor(val, device), kc, vc,
                  torch.from_numpy(slots).to(device), k_scale_cache=ks, v_scale_cache=vs, rotate=False)
    torch.cuda.synchronize()
    views = O.int4_views(kv_np, HS) if fmt == "int4" else O.k8v4_views(kv_np, HS)
    O.store(views, O.bf16_bits_to_f32(key), O.bf16_bits_to_f32(val), slots)
    got = t.cpu().numpy().view(np.uint8)            # logical (blocks, heads, slots, cell) order
    assert (got == kv_np).all()


def test_store_with_rotation_equals_rotate_then_store(device):
    import torch

    from vllm_quantpack.attention import k8v4_kv, rht
    rng = np.random.default_rng(62)
    nb, bs, n = 10, 16, 150
    kv_a = O.new_cache(nb, NKV, bs, O.k8v4_cell_bytes(HS))
    kv_b = O.new_cache(nb, NKV, bs, O.k8v4_cell_bytes(HS))
    ta, va = torch_cache(kv_a, HS, "int8", device)
    tb, vb = torch_cache(kv_b, HS, "int8", device)
    key = bf16_tensor(O.f32_to_bf16_bits(rng.standard_normal((n, NKV, HS)).astype(np.float32)), device)
    val = bf16_tensor(O.f32_to_bf16_bits(rng.standard_normal((n, NKV, HS)).astype(np.float32)), device)
    slots = torch.arange(n, device=device)
    k8v4_kv.store(None, key, val, va[0], va[1], slots, k_scale_cache=va[2], v_scale_cache=va[3])
    k8v4_kv.store(None, rht.single_rht(key), rht.single_rht(val), vb[0], vb[1], slots, k_scale_cache=vb[2],
                  v_scale_cache=vb[3], rotate=False)
    torch.cuda.synchronize()
    assert torch.equal(ta, tb)


# -------------------------------------------------------------------------------------------------------- RHT

def test_rht_matches_fp64_and_inverts(device):
    import torch

    from vllm_quantpack.attention import rht
    rng = np.random.default_rng(71)
    x = rng.standard_normal((33, HS)).astype(np.float32)
    xt = torch.from_numpy(x).to(device)
    y = rht.single_rht(xt)
    want = O.rht(x)
    assert np.allclose(to_f32(y), want, rtol=1e-5, atol=1e-4)
    back = rht.single_rht(y, inverse=True, out_scale=1.0 / HS)
    assert np.allclose(to_f32(back), x, atol=1e-5)
    yb = rht.single_rht(xt.to(torch.bfloat16))
    assert (to_f32(yb) == O.round_bf16(O.rht(O.round_bf16(x)).astype(np.float32))).mean() > 0.99


# --------------------------------------------------------------------------------- end-to-end drop-in router

@pytest.mark.parametrize("fmt", ["int4", "int8"])
@pytest.mark.parametrize("qlen", [1, 2, 4])
def test_unified_attention_decode_matches_fp64(device, fmt, qlen):
    """The reference's end-to-end check (tests/test_int4_kv.py:172-191 / tests/test_k8v4_kv.py:159-173): random bf16 K/V
    stored through reshape_and_cache_int4, attention of unrotated queries against fp64, error < 1e-2 (and < 0.5 %)."""
    import torch

    from vllm_quantpack.attention import int4_kv
    rng = np.random.default_rng(81 + qlen)
    n, bs = 6000, 16
    nb = -(-n // bs)
    kv_np = O.new_cache(nb, NKV, bs, O.int4_cell_bytes(HS) if fmt == "int4" else O.k8v4_cell_bytes(HS))
    _, (kc, vc, ks, vs) = torch_cache(kv_np, HS, fmt, device)
    g = torch.Generator(device=device).manual_seed(0)
    k = torch.randn((n, NKV, HS), generator=g, device=device, dtype=torch.bfloat16)
    v = torch.randn((n, NKV, HS), generator=g, device=device, dtype=torch.bfloat16)
    int4_kv.reshape_and_cache_int4(k, v, kc, vc, torch.arange(n, device=device), k_scale_cache=ks,
                                   v_scale_cache=vs)
    q = torch.randn((qlen, NQ, HS), generator=g, device=device, dtype=torch.bfloat16)
    S = 64
    rows = 32
    segm = (torch.empty((rows, NQ, S, HS), dtype=torch.float32, device=device),
            torch.empty((rows, NQ, S), dtype=torch.float32, device=device),
            torch.empty((rows, NQ, S), dtype=torch.float32, device=device))
    out = torch.empty_like(q)
    int4_kv.unified_attention_int4(
        q, kc, vc, out, cu_seqlens_q=i32([0, qlen], device), max_seqlen_q=qlen, seqused_k=i32([n], device),
        max_seqlen_k=n, softmax_scale=HS ** -0.5, window_size=(-1, -1),
        block_table=torch.arange(nb, dtype=torch.int32, device=device)[None], softcap=0.0, sinks=None,
        alibi_slopes=None, use_alibi_sqrt=False, qq_bias=None, output_scale=None, mm_prefix_range=None,
        k_scale_cache=ks, v_scale_cache=vs, seq_threshold_3D=rows, num_par_softmax_segments=S,
        softmax_segm_output=segm[0], softmax_segm_max=segm[1], softmax_segm_expsum=segm[2])
    torch.cuda.synchronize()
    # fp64 reference from the stored bytes (the cache is in the rotated domain)
    views = O.int4_views if fmt == "int4" else O.k8v4_views
    root = _host_cache(kc, vc, ks, vs, fmt)
    K, V = O.dequant_f64(views(root, HS), np.arange(nb), n)
    qr = O.rht(to_f32(q).astype(np.float64))
    ref = O.rht(O.attention_f64(qr, K, V, n, HS ** -0.5 / HS), inverse=True) / HS
    err = O.relerr(to_f32(out), ref)
    assert err < 5e-3, err


@pytest.mark.parametrize("fmt", ["int4", "int8"])
def test_unified_attention_decode_batch_matches_fp64(device, fmt):
    """The router on a ragged batch of 12 sequences (1 or 2 query tokens, 300 to 3000 cached tokens): it lowers the
    caller's 64 segments to 43 for the batch; every sequence within 0.5 % of fp64."""
    import torch

    from vllm_quantpack.attention import int4_kv
    rng = np.random.default_rng(91)
    seqs, bs = 12, 16
    T = rng.integers(1, 3, size=seqs)
    n = rng.integers(300, 3001, size=seqs)
    nb = -(-n // bs)
    total = int(nb.sum())
    kv_np = O.new_cache(total, NKV, bs, O.int4_cell_bytes(HS) if fmt == "int4" else O.k8v4_cell_bytes(HS))
    _, (kc, vc, ks, vs) = torch_cache(kv_np, HS, fmt, device)
    pool = rng.permutation(total).astype(np.int32)
    table = np.zeros((seqs, int(nb.max())), np.int32)
    at = 0
    g = torch.Generator(device=device).manual_seed(1)
    for i in range(seqs):
        table[i, :nb[i]] = pool[at:at + nb[i]]
        at += nb[i]
        slots = torch.as_tensor(table[i, :nb[i]].astype(np.int64), device=device)[:, None] * bs + torch.arange(
            bs, device=device)
        slots = slots.flatten()[:n[i]]
        k = torch.randn((int(n[i]), NKV, HS), generator=g, device=device, dtype=torch.bfloat16)
        v = torch.randn((int(n[i]), NKV, HS), generator=g, device=device, dtype=torch.bfloat16)
        int4_kv.reshape_and_cache_int4(k, v, kc, vc, slots, k_scale_cache=ks, v_scale_cache=vs)
    q = torch.randn((int(T.sum()), NQ, HS), generator=g, device=device, dtype=torch.bfloat16)
    cu = np.concatenate(([0], np.cumsum(T))).astype(np.int32)
    S, rows = 64, int(T.sum())
    segm = (torch.empty((rows, NQ, S, HS), dtype=torch.float32, device=device),
            torch.empty((rows, NQ, S), dtype=torch.float32, device=device),
            torch.empty((rows, NQ, S), dtype=torch.float32, device=device))
    out = torch.empty_like(q)
    assert int4_kv.decode_segments(S, seqs, NKV, torch.cuda.get_device_properties(device).multi_processor_count) < S
    int4_kv.unified_attention_int4(
        q, kc, vc, out, cu_seqlens_q=i32(cu, device), max_seqlen_q=int(T.max()), seqused_k=i32(n, device),
        max_seqlen_k=int(n.max()), softmax_scale=HS ** -0.5, window_size=(-1, -1), block_table=i32(table, device),
        softcap=0.0, sinks=None, alibi_slopes=None, use_alibi_sqrt=False, qq_bias=None, output_scale=None,
        mm_prefix_range=None, k_scale_cache=ks, v_scale_cache=vs, seq_threshold_3D=rows, num_par_softmax_segments=S,
        softmax_segm_output=segm[0], softmax_segm_max=segm[1], softmax_segm_expsum=segm[2])
    torch.cuda.synchronize()
    views = O.int4_views if fmt == "int4" else O.k8v4_views
    root = _host_cache(kc, vc, ks, vs, fmt)
    got = to_f32(out)
    qr = O.rht(to_f32(q).astype(np.float64))
    for i in range(seqs):
        K, V = O.dequant_f64(views(root, HS), table[i], int(n[i]))
        ref = O.rht(O.attention_f64(qr[cu[i]:cu[i + 1]], K, V, int(n[i]), HS ** -0.5 / HS), inverse=True) / HS
        assert O.relerr(got[cu[i]:cu[i + 1]], ref) < 5e-3, i


def _host_cache(kc, vc, ks, vs, fmt, hs=HS):
    """The byte cache behind the views, copied to the host as a numpy (blocks, heads, slots, cell) array."""
    import torch
    st = kc.untyped_storage()
    nbytes = st.nbytes()
    base = torch.empty(nbytes, dtype=torch.uint8, device=kc.device)
    base.set_(st, 0, (nbytes,), (1,))
    arr = base.cpu().numpy()
    nb, bs, nkv = kc.shape[0], kc.shape[1], kc.shape[2]
    cell = O.int4_cell_bytes(hs) if fmt == "int4" else O.k8v4_cell_bytes(hs)
    return arr.reshape(nb, nkv, bs, cell)


# ---------------------------------------------------------------------------------------------------- prefill

def _prefill_case(device, rng, fmt, lens, layout="hnd", bs=16, nq=NQ, nkv=NKV, hs=HS, scale=None, splits=0,
                  big_keys=()):
    """lens = [(T_i, n_i)]: one batched prefill call; returns (gpu out, emulation, fp64 reference). big_keys =
    [(position, scale)] gives those key positions of every sequence a large key scale (scores far above the first
    tile's maximum)."""
    import torch

    from vllm_quantpack.attention import int4_prefill
    nbs = [-(-n // bs) for _, n in lens]
    total = sum(nbs) + 2
    kv, v = random_cache(rng, total, nkv, bs, hs, fmt, layout)
    pool = rng.permutation(total).astype(np.int32)
    table = np.zeros((len(lens), max(nbs)), np.int32)
    at = 0
    for i, nb in enumerate(nbs):
        table[i, :nb] = pool[at:at + nb]
        at += nb
    for pos, sc in big_keys:
        for i in range(len(lens)):
            blk, slot = table[i, pos // bs], pos % bs
            words = v.key_word[blk, slot]
            bits = np.float32(sc).view(np.uint32) & np.uint32(0xFFFFFFF0)
            words[:] = (words & np.uint32(0xF)) | bits if fmt == "int4" else np.float32(sc).view(np.uint32)
    _, (kc, vc, ks, vs) = torch_cache(kv, hs, fmt, device)
    Ts = [t for t, _ in lens]
    q = O.f32_to_bf16_bits(rng.standard_normal((sum(Ts), nq, hs)).astype(np.float32))
    cu = np.concatenate(([0], np.cumsum(Ts))).astype(np.int32)
    scale = scale or hs ** -0.5
    qt = bf16_tensor(q, device)
    out = torch.full_like(qt, float("nan"))
    int4_prefill.prefill_attention(qt, kc, vc, ks, vs, out, cu_seqlens_q=i32(cu, device),
                                   seqused_k=i32([n for _, n in lens], device), block_table=i32(table, device),
                                   max_seqlen_q=max(Ts), softmax_scale=scale, num_splits=splits)
    torch.cuda.synchronize()
    qf = O.bf16_bits_to_f32(q)
    emus, refs = [], []
    for i, (T, n) in enumerate(lens):
        qs = qf[cu[i]:cu[i + 1]]
        emus.append(O.decode_emulated(qs, v, table[i], n, scale, num_segments=1, tile=64))
        K, V = O.dequant_f64(v, table[i], n)
        refs.append(O.attention_f64(qs, K, V, n, scale))
    return to_f32(out), np.concatenate(emus), np.concatenate(refs)


@pytest.mark.parametrize("fmt", ["int4", "int8"])
@pytest.mark.parametrize("layout", ["hnd", "nhd"])
def test_prefill_matches_oracle(device, fmt, layout):
    rng = np.random.default_rng(201)
    out, emu, ref = _prefill_case(device, rng, fmt, [(100, 3000)], layout=layout)
    assert np.isfinite(out).all()
    assert_emulation(out, emu)
    assert O.relerr(out, ref) < 5e-3, O.relerr(out, ref)


@pytest.mark.parametrize("splits", [1, 2, 5])
def test_prefill_key_splits_agree(device, splits):
    """Keys split over 1, 2 or 5 workgroups per query block and merged: the same attention (the split ranges follow
    the split-KV segment rule, so some sequences get empty splits)."""
    rng = np.random.default_rng(210)
    lens = [(48, 2600), (7, 300), (33, 33)]
    out, emu, ref = _prefill_case(device, rng, "int4", lens, splits=splits)
    assert np.isfinite(out).all()
    assert_emulation(out, emu)
    assert O.relerr(out, ref) < 5e-3, O.relerr(out, ref)


@pytest.mark.parametrize("fmt", ["int4", "int8"])
@pytest.mark.parametrize("bs,splits", [(16, 1), (16, 2), (32, 1)])
def test_prefill_loop_boundaries(device, fmt, bs, splits):
    """Contexts whose 32-key tile counts straddle the kernel's loop boundaries: the six-tile unrolled loop (int4 keys)
    and the steady loops run only while at least 12 (7) tiles remain, and a split's last tile may hold 1..31 keys; with
    16-token blocks the run pairs come from a stepping table pointer. 20 query tokens per sequence, so every tile past
    the chunk is unmasked."""
    rng = np.random.default_rng(230 + (1 if fmt == "int8" else 0) + 2 * bs + splits)
    ns = [161, 192, 193, 351, 352, 353, 383, 385, 545, 640, 701]
    out, emu, ref = _prefill_case(device, rng, fmt, [(20, n) for n in ns], bs=bs, splits=splits)
    assert np.isfinite(out).all()
    assert_emulation(out, emu)
    at = 0
    for n in ns:
        sl = slice(at, at + 20)
        assert O.relerr(out[sl], ref[sl]) < 5e-3, n
        at += 20


@pytest.mark.parametrize("splits", [1, 0])
@pytest.mark.parametrize("hs,nq,nkv,fmt", [(256, 24, 4, "int4"), (256, 24, 4, "int8"), (128, 64, 8, "int4"),
                                           (128, 64, 8, "int8"), (512, 16, 2, "int4"), (512, 16, 2, "int8")])
def test_prefill_repeats_bit_for_bit(device, fmt, splits, hs, nq, nkv):
    """The same call five times gives the same bits. Nothing in the kernels depends on timing, so a race between
    waves (a copy landing in a slot that is still read, an LDS buffer rewritten before a barrier) or a work split that
    follows the waves' timing shows up here as differing rows, well inside the accuracy bars the other tests hold.
    40 tokens over 3000 keys: at head 256 (6 query heads per KV head) two row blocks of the tile kernel through its
    unrolled and steady loops; head 128 with 8 per KV head and head 512 on the wide kernel; head 512 with int8 keys as
    query slices on the decode kernel; one split, or the host's choice (split partials merged)."""
    import torch

    from vllm_quantpack.attention import int4_prefill
    rng = np.random.default_rng(260 + splits + (2 if fmt == "int8" else 0) + hs)
    n, T, bs = 3000, 40, 16
    nb = -(-n // bs)
    kv, _ = random_cache(rng, nb, nkv, bs, hs, fmt)
    _, (kc, vc, ks, vs) = torch_cache(kv, hs, fmt, device)
    q = bf16_tensor(O.f32_to_bf16_bits(rng.standard_normal((T, nq, hs)).astype(np.float32)), device)
    kw = dict(cu_seqlens_q=i32([0, T], device), seqused_k=i32([n], device),
              block_table=i32(rng.permutation(nb).astype(np.int32)[None], device), max_seqlen_q=T,
              softmax_scale=hs ** -0.5, num_splits=splits)
    outs = []
    for _ in range(5):
        out = torch.full_like(q, float("nan"))
        int4_prefill.prefill_attention(q, kc, vc, ks, vs, out, **kw)
        torch.cuda.synchronize()
        outs.append(to_f32(out))
    assert np.isfinite(outs[0]).all()
    for k in range(1, 5):
        diff = np.argwhere(outs[k] != outs[0])
        assert not len(diff), (k, len(diff), sorted({(int(t), int(h)) for t, h, _ in diff})[:8])


@pytest.mark.parametrize("fmt,n", [("int4", 330), ("int4", 1009), ("int8", 1000), ("int8", 721)])
def test_prefill_table_row_exactly_as_long_as_the_context(device, fmt, n):
    """One sequence whose block table holds exactly ceil(n / 16) entries and whose last tile has 1..16 keys: the
    kernel's table reads ahead of the copies stay inside the row (the CPU walk in test_prefill_table_walk checks the
    indices; this runs the same shapes)."""
    rng = np.random.default_rng(250 + n)
    out, emu, ref = _prefill_case(device, rng, fmt, [(20, n)])
    assert np.isfinite(out).all()
    assert_emulation(out, emu)
    assert O.relerr(out, ref) < 5e-3, O.relerr(out, ref)


@pytest.mark.parametrize("fmt", ["int4", "int8"])
@pytest.mark.parametrize("bs", [16, 48])
def test_prefill_head_128(device, fmt, bs):
    """Head 128 (GQA 6): 136- and 200-byte cells, so a 16-cell page run is two or three full 64-lane copies plus an
    8-lane tail, and the copy slots mix runs; 16-token blocks take the stepping table pointer, 48-token blocks the
    general run arithmetic."""
    rng = np.random.default_rng(240 + bs + (1 if fmt == "int8" else 0))
    out, emu, ref = _prefill_case(device, rng, fmt, [(70, 1900), (12, 500), (3, 37)], bs=bs, hs=128)
    assert np.isfinite(out).all()
    assert_emulation(out, emu)
    assert O.relerr(out, ref) < 5e-3, O.relerr(out, ref)


@pytest.mark.parametrize("fmt", ["int4", "int8"])
def test_prefill_scores_far_above_the_first_tile(device, fmt):
    """Keys with scales 2^7 .. 2^12 late in the context push scores thousands of log2 units above the first tile's
    maximum: each row raises its maximum where the scores exceed it, scaling its sum and accumulators down in place
    (by assembly on the AGPR tiles), and the result still matches."""
    rng = np.random.default_rng(211)
    big = [(700, 2.0 ** 7), (1300, 2.0 ** 9), (1901, 2.0 ** 12)]
    out, emu, ref = _prefill_case(device, rng, fmt, [(40, 2000), (9, 1400)], splits=1, big_keys=big)
    assert np.isfinite(out).all()
    assert O.relerr(out, ref) < 5e-3, O.relerr(out, ref)


def test_prefill_fused_rotation(device):
    """rht_signs rotates the output back inside the library, with and without key splits."""
    import torch

    from vllm_quantpack.attention import int4_prefill, rht
    rng = np.random.default_rng(212)
    n, qlen, bs = 3000, 64, 16
    nb = -(-n // bs)
    kv, v = random_cache(rng, nb, NKV, bs, HS)
    _, (kc, vc, ks, vs) = torch_cache(kv, HS, "int4", device)
    q = O.f32_to_bf16_bits(rng.standard_normal((qlen, NQ, HS)).astype(np.float32))
    qt = bf16_tensor(q, device)
    table = torch.arange(nb, dtype=torch.int32, device=device)[None]
    signs = rht.signs(HS, device)
    plain = torch.empty_like(qt)
    int4_prefill.prefill_attention(qt, kc, vc, ks, vs, plain, cu_seqlens_q=i32([0, qlen], device),
                                   seqused_k=i32([n], device), block_table=table, max_seqlen_q=qlen,
                                   softmax_scale=0.06, num_splits=1)
    want = O.rht(to_f32(plain).astype(np.float64), inverse=True) / HS
    for splits in (1, 3):
        got = torch.empty_like(qt)
        int4_prefill.prefill_attention(qt, kc, vc, ks, vs, got, cu_seqlens_q=i32([0, qlen], device),
                                       seqused_k=i32([n], device), block_table=table, max_seqlen_q=qlen,
                                       softmax_scale=0.06, num_splits=splits, rht_signs=signs, rht_out_scale=1 / HS)
        torch.cuda.synchronize()
        assert O.relerr(to_f32(got), want) < 1e-2, splits


@pytest.mark.parametrize("fmt", ["int4", "int8"])
def test_prefill_varlen_batch(device, fmt):
    """A batch mixing a long chunk, a first chunk (context == chunk), short chunks and single tokens."""
    rng = np.random.default_rng(202 + (10 if fmt == "int8" else 0))
    lens = [(70, 2500), (5, 900), (1, 1), (33, 33), (16, 4000), (17, 64)]
    out, emu, ref = _prefill_case(device, rng, fmt, lens)
    at = 0
    for T, n in lens:
        sl = slice(at, at + T)
        assert_emulation(out[sl], emu[sl], (T, n))
        assert O.relerr(out[sl], ref[sl]) < 5e-3, (T, n)
        at += T


@pytest.mark.parametrize("bs", [32, 3072])
def test_prefill_block_sizes_and_gqa(device, bs):
    rng = np.random.default_rng(203 + bs)
    out, emu, ref = _prefill_case(device, rng, "int4", [(40, 2000)], bs=bs, nq=16, nkv=2, hs=128)
    assert_emulation(out, emu)
    assert O.relerr(out, ref) < 5e-3


@pytest.mark.parametrize("fmt", ["int4", "int8"])
def test_prefill_head_512(device, fmt):
    """Head 512: int4 keys take the wide kernel (K operands from the packed codes, always key-split), int8 keys the
    split-KV kernel over causal query slices, then the merge (the reference keeps these on its Triton kernel:
    tests/test_int4_kv.py:194-210, tests/test_k8v4_kv.py:208-225). Ragged batch."""
    rng = np.random.default_rng(401 + (1 if fmt == "int8" else 0))
    out, emu, ref = _prefill_case(device, rng, fmt, [(37, 2100), (5, 600), (1, 64)], nq=16, nkv=2, hs=512)
    assert_emulation(out, emu)
    assert O.relerr(out, ref) < 5e-3


@pytest.mark.parametrize("fmt", ["int4", "int8"])
def test_prefill_head_64(device, fmt):
    """Head 64 prefills over causal query slices of the split-KV kernel (the reference's kernels take any head size:
    int4_kv.py:130-131). Ragged batch, with a first chunk (context == chunk)."""
    rng = np.random.default_rng(407 + (1 if fmt == "int8" else 0))
    out, emu, ref = _prefill_case(device, rng, fmt, [(37, 2100), (20, 20), (1, 64)], nq=16, nkv=2, hs=64)
    assert_emulation(out, emu)
    assert O.relerr(out, ref) < 5e-3


@pytest.mark.parametrize("nq,nkv,hs", [(12, 4, 256), (20, 4, 256), (28, 4, 128), (32, 4, 256), (32, 2, 256),
                                       (16, 4, 128)])
def test_prefill_tile_rows_at_any_gqa_width(device, nq, nkv, hs):
    """The tile kernel's 192-row blocks of (token, query head) pairs at GQA 3, 5, 7, 8 and 16 (and 4 at head 128): a
    ragged batch whose blocks straddle tokens and sequences end mid-block, against the emulation and fp64."""
    rng = np.random.default_rng(410 + nq + hs)
    lens = [(70, 2500), (5, 900), (1, 1), (33, 33), (17, 64)]
    out, emu, ref = _prefill_case(device, rng, "int4", lens, nq=nq, nkv=nkv, hs=hs)
    assert np.isfinite(out).all()
    assert_emulation(out, emu)
    assert O.relerr(out, ref) < 5e-3, O.relerr(out, ref)


def test_prefill_wide_gqa(device):
    """16 query heads per KV head is past the 16-row-tile kernel's 12: the wide kernel (32x32x16 MFMAs, rows as
    (token, head) pairs) serves it."""
    rng = np.random.default_rng(405)
    out, emu, ref = _prefill_case(device, rng, "int4", [(20, 1500), (3, 200)], nq=16, nkv=1, hs=128)
    assert_emulation(out, emu)
    assert O.relerr(out, ref) < 5e-3


@pytest.mark.parametrize("fmt", ["int4", "int8"])
@pytest.mark.parametrize("hs,splits", [(256, 1), (256, 3), (128, 1), (128, 2), (512, 1), (512, 3)])
def test_prefill_wide_kernel_batches(device, fmt, hs, splits):
    """16 query heads per KV head on a batch whose row blocks (256 rows at head 128 and 128 at head 512 on the wide
    kernel, 192 at head 256 on the tile kernel) straddle tokens and end mid-block: a long chunk, a first chunk (context
    == chunk), a single token, a 130-token chunk; 32 query heads on 2 KV heads; with key splits, some of them empty
    (head 512 runs at least 2; with int8 keys it takes the query slices)."""
    rng = np.random.default_rng(260 + hs + splits + (1 if fmt == "int8" else 0))
    lens = [(40, 3000), (7, 7), (1, 500), (130, 900)]
    out, emu, ref = _prefill_case(device, rng, fmt, lens, nq=32, nkv=2, hs=hs, splits=splits)
    assert np.isfinite(out).all()
    assert_emulation(out, emu)
    assert O.relerr(out, ref) < 5e-3, O.relerr(out, ref)


@pytest.mark.parametrize("fmt,n,hs", [("int4", 330, 128), ("int8", 1000, 128), ("int4", 1009, 512), ("int4", 353, 512)])
def test_prefill_wide_table_row_exactly_as_long_as_the_context(device, fmt, n, hs):
    """One sequence whose block table holds exactly ceil(n / 16) entries and whose last tile has 1..16 keys, on the
    wide kernel (the CPU walk in test_prefill_table_walk checks its table reads)."""
    rng = np.random.default_rng(270 + n)
    out, emu, ref = _prefill_case(device, rng, fmt, [(20, n)], nq=16, nkv=1, hs=hs)
    assert_emulation(out, emu)
    assert O.relerr(out, ref) < 5e-3, O.relerr(out, ref)


@pytest.mark.parametrize("hs", [128, 256, 512])
def test_prefill_wide_rows_without_keys_are_zero(device, hs):
    """A sequence whose context holds no keys (seqused_k = 0 beside a query chunk; vLLM does not send these) leaves
    the row blocks without a tile (the wide kernel at heads 128 and 512, the tile kernel at 256): its rows come out
    zero, with one split (the epilogue's normalisation of empty accumulators) and with several (every split empty for
    the merge), and the other sequence is unaffected."""
    import torch

    from vllm_quantpack.attention import int4_prefill
    rng = np.random.default_rng(285 + hs)
    bs, nq, nkv, n = 16, 16, 1, 700
    nb = -(-n // bs)
    kv, v = random_cache(rng, nb + 1, nkv, bs, hs)
    _, (kc, vc, ks, vs) = torch_cache(kv, hs, "int4", device)
    table = np.zeros((2, nb), np.int32)
    table[0] = np.arange(nb)
    q = O.f32_to_bf16_bits(rng.standard_normal((13, nq, hs)).astype(np.float32))
    qt = bf16_tensor(q, device)
    scale = hs ** -0.5
    for splits in (1, 3):
        out = torch.full_like(qt, float("nan"))
        int4_prefill.prefill_attention(qt, kc, vc, ks, vs, out, cu_seqlens_q=i32([0, 8, 13], device),
                                       seqused_k=i32([n, 0], device), block_table=i32(table, device), max_seqlen_q=8,
                                       softmax_scale=scale, num_splits=splits)
        torch.cuda.synchronize()
        got = to_f32(out)
        assert np.all(got[8:] == 0), splits
        emu = O.decode_emulated(O.bf16_bits_to_f32(q)[:8], v, table[0], n, scale, num_segments=1, tile=64)
        assert_emulation(got[:8], emu, splits)


@pytest.mark.parametrize("fmt,hs", [("int4", 128), ("int8", 128), ("int4", 512)])
def test_prefill_wide_scores_far_above_the_first_tile(device, fmt, hs):
    """Key scales of 2^7 .. 2^12 late in the context put scores thousands of log2 units above the first tile's
    maximum, past the wide kernel's headroom: the workgroup runs its split again with the raised maxima (once per
    jump), and the result still matches."""
    rng = np.random.default_rng(280 + (1 if fmt == "int8" else 0) + hs)
    big = [(700, 2.0 ** 7), (1300, 2.0 ** 9), (1901, 2.0 ** 12)]
    out, emu, ref = _prefill_case(device, rng, fmt, [(40, 2000), (9, 1400)], nq=16, nkv=1, hs=hs, splits=1,
                                  big_keys=big)
    assert np.isfinite(out).all()
    assert O.relerr(out, ref) < 5e-3, O.relerr(out, ref)


@pytest.mark.parametrize("hs", [128, 512])
def test_prefill_wide_fused_rotations(device, hs):
    """On the wide kernel: the query rotated on load gives the bits of rotating it first, and the output rotated back
    in the epilogue (one split) or by the merge (three; at head 512 the kernel always splits) matches a separate
    inverse rotation."""
    import torch

    from vllm_quantpack.attention import int4_prefill, rht
    rng = np.random.default_rng(290 + hs)
    n, qlen, bs, nq, nkv = 2500, 50, 16, 32, 2
    HS = hs
    nb = -(-n // bs)
    kv, _ = random_cache(rng, nb, nkv, bs, HS)
    _, (kc, vc, ks, vs) = torch_cache(kv, HS, "int4", device)
    q = bf16_tensor(O.f32_to_bf16_bits(rng.standard_normal((qlen, nq, HS)).astype(np.float32)), device)
    table = torch.arange(nb, dtype=torch.int32, device=device)[None]
    signs = rht.signs(HS, device)
    kw = dict(cu_seqlens_q=i32([0, qlen], device), seqused_k=i32([n], device), block_table=table, max_seqlen_q=qlen,
              softmax_scale=0.004)
    a, b = torch.empty_like(q), torch.empty_like(q)
    int4_prefill.prefill_attention(rht.single_rht(q), kc, vc, ks, vs, a, **kw, num_splits=1)
    int4_prefill.prefill_attention(q, kc, vc, ks, vs, b, **kw, num_splits=1, query_signs=signs)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    want = O.rht(to_f32(a).astype(np.float64), inverse=True) / HS
    for splits in (1, 3):
        got = torch.empty_like(q)
        int4_prefill.prefill_attention(q, kc, vc, ks, vs, got, **kw, num_splits=splits, query_signs=signs,
                                       rht_signs=signs, rht_out_scale=1 / HS)
        torch.cuda.synchronize()
        assert O.relerr(to_f32(got), want) < 1e-2, splits


@pytest.mark.parametrize("fmt,hs,nq", [("int8", 256, NQ), ("int4", 512, 16), ("int8", 128, 16)])
def test_prefill_span_and_row_loaders_agree(device, fmt, hs, nq):
    """The page-run copies (HND) and the strided gather (NHD) of the tile kernel (head 256) and the wide one (head 128
    with 8 query heads per KV head, head 512) on the same cache contents."""
    case = dict(hs=hs, nq=nq, nkv=2 if hs in (128, 512) else NKV)
    a, emu, ref = _prefill_case(device, np.random.default_rng(204), fmt, [(64, 1500), (3, 700)], **case)
    b, _, _ = _prefill_case(device, np.random.default_rng(204), fmt, [(64, 1500), (3, 700)], layout="nhd", **case)
    assert_emulation(a, emu)
    assert_emulation(b, emu)
    assert O.relerr(a, b) < 5e-3


@pytest.mark.parametrize("fmt", ["int4", "int8"])
@pytest.mark.parametrize("nq,nkv,hs", [(NQ, NKV, HS), (16, 2, 512)], ids=["head256", "head512"])
def test_unified_attention_prefill_matches_fp64(device, fmt, nq, nkv, hs):
    """tests/test_int4_kv.py:172-191 prefill rows: a 256-token chunk over a 6000-token context through the router;
    head 512 with 16 / 2 heads as tests/test_int4_kv.py:194-210 and tests/test_k8v4_kv.py:208-225."""
    import torch

    from vllm_quantpack.attention import int4_kv
    rng = np.random.default_rng(205)
    n, bs, qlen = 6000, 16, 256
    nb = -(-n // bs)
    kv_np = O.new_cache(nb, nkv, bs, O.int4_cell_bytes(hs) if fmt == "int4" else O.k8v4_cell_bytes(hs))
    _, (kc, vc, ks, vs) = torch_cache(kv_np, hs, fmt, device)
    g = torch.Generator(device=device).manual_seed(1)
    k = torch.randn((n, nkv, hs), generator=g, device=device, dtype=torch.bfloat16)
    v = torch.randn((n, nkv, hs), generator=g, device=device, dtype=torch.bfloat16)
    int4_kv.reshape_and_cache_int4(k, v, kc, vc, torch.arange(n, device=device), k_scale_cache=ks,
                                   v_scale_cache=vs)
    q = torch.randn((qlen, nq, hs), generator=g, device=device, dtype=torch.bfloat16)
    out = torch.empty_like(q)
    segm = (torch.empty((32, nq, 16, hs), dtype=torch.float32, device=device),
            torch.empty((32, nq, 16), dtype=torch.float32, device=device),
            torch.empty((32, nq, 16), dtype=torch.float32, device=device))
    int4_kv.unified_attention_int4(
        q, kc, vc, out, cu_seqlens_q=i32([0, qlen], device), max_seqlen_q=qlen, seqused_k=i32([n], device),
        max_seqlen_k=n, softmax_scale=hs ** -0.5, window_size=(-1, -1),
        block_table=torch.arange(nb, dtype=torch.int32, device=device)[None], softcap=0.0, sinks=None,
        alibi_slopes=None, use_alibi_sqrt=False, qq_bias=None, output_scale=None, mm_prefix_range=None,
        k_scale_cache=ks, v_scale_cache=vs, seq_threshold_3D=32, num_par_softmax_segments=16,
        softmax_segm_output=segm[0], softmax_segm_max=segm[1], softmax_segm_expsum=segm[2])
    torch.cuda.synchronize()
    views = O.int4_views if fmt == "int4" else O.k8v4_views
    K, V = O.dequant_f64(views(_host_cache(kc, vc, ks, vs, fmt, hs), hs), np.arange(nb), n)
    qr = O.rht(to_f32(q).astype(np.float64))
    ref = O.rht(O.attention_f64(qr, K, V, n, hs ** -0.5 / hs), inverse=True) / hs
    err = O.relerr(to_f32(out), ref)
    assert err < 5e-3, err


def test_prefill_sequence_reference_signature(device):
    """int4_prefill.prefill_sequence(q_rot, k_cache, v_cache, k_scales, v_scales, block_row, n, scale, fa) as the
    reference calls it (int4_kv.py:327-328): output in the rotated domain, q_rot's dtype."""
    import torch

    from vllm_quantpack.attention import int4_prefill
    rng = np.random.default_rng(206)
    n, qlen = 2000, 80
    kv, v = random_cache(rng, -(-n // 16), NKV, 16, HS)
    _, (kc, vc, ks, vs) = torch_cache(kv, HS, "int4", device)
    q = O.f32_to_bf16_bits(rng.standard_normal((qlen, NQ, HS)).astype(np.float32))
    o = int4_prefill.prefill_sequence(bf16_tensor(q, device), kc, vc, ks, vs,
                                      torch.arange(-(-n // 16), dtype=torch.int32, device=device), n, 0.05, None)
    assert o.dtype == torch.bfloat16 and tuple(o.shape) == (qlen, NQ, HS)
    K, V = O.dequant_f64(v, np.arange(-(-n // 16)), n)
    ref = O.attention_f64(O.bf16_bits_to_f32(q), K, V, n, 0.05)
    assert O.relerr(to_f32(o), ref) < 5e-3
    # the reference's undispatched single-kernel variant (int4_prefill.py:176-200) has the same contract
    o8 = int4_prefill.prefill_sequence_i8(bf16_tensor(q, device), kc, vc, ks, vs,
                                          torch.arange(-(-n // 16), dtype=torch.int32, device=device), n, 0.05)
    assert o8.dtype == torch.bfloat16 and O.relerr(to_f32(o8), ref) < 5e-3
