"""The drop-in attention (unified_attention_int4 -> qp_attention) on the MI355X: mixed batches routed on the device,
the query rotation fused into the kernels' loads, the decode row cap, no host synchronisation, HIP-graph capture.

References: the mixed prefill + MTP step of tests/test_int4_kv.py:213-227 and tests/test_k8v4_kv.py:176-192, the
batched MTP decodes with capped query rows of tests/test_int4_kv.py:230-249, and the host-sync checks of
tests/test_int4_kv.py:252-315. Every output is checked against the fp64 closed form computed from the stored bytes.
"""
import numpy as np
import pytest

from oracle import qp_oracle as O
from qp_testlib import i32, to_f32, torch_cache

pytestmark = pytest.mark.gpu

NQ, NKV, HS, BS = 24, 4, 256, 16


def _stored_cache(device, fmt, lens, seed, nkv=NKV, hs=HS, spare=3):
    """A paged cache holding random bf16 K/V stored through reshape_and_cache_int4 for sequences of lens[i] tokens
    (shuffled blocks from a shared pool, `spare` blocks never used). Returns (views, table, host views)."""
    import torch

    from vllm_quantpack.attention import int4_kv
    rng = np.random.default_rng(seed)
    nbs = [-(-n // BS) for n in lens]
    total = sum(nbs) + spare
    kv_np = O.new_cache(total, nkv, BS, O.int4_cell_bytes(hs) if fmt == "int4" else O.k8v4_cell_bytes(hs))
    t, (kc, vc, ks, vs) = torch_cache(kv_np, hs, fmt, device)
    pool = rng.permutation(total).astype(np.int32)
    table = np.zeros((len(lens), max(nbs)), np.int32)
    at = 0
    g = torch.Generator(device=device).manual_seed(seed)
    for i, n in enumerate(lens):
        table[i, :nbs[i]] = pool[at:at + nbs[i]]
        at += nbs[i]
        slots = (torch.as_tensor(table[i, :nbs[i]].astype(np.int64), device=device)[:, None] * BS
                 + torch.arange(BS, device=device)).flatten()[:n]
        k = torch.randn((n, nkv, hs), generator=g, device=device, dtype=torch.bfloat16)
        v = torch.randn((n, nkv, hs), generator=g, device=device, dtype=torch.bfloat16)
        int4_kv.reshape_and_cache_int4(k, v, kc, vc, slots, k_scale_cache=ks, v_scale_cache=vs)
    torch.cuda.synchronize()
    host = t.cpu().numpy().view(np.uint8)
    if host.shape != kv_np.shape:
        host = host.transpose(0, 2, 1, 3)
    views = O.int4_views(np.ascontiguousarray(host), hs) if fmt == "int4" else O.k8v4_views(
        np.ascontiguousarray(host), hs)
    return (kc, vc, ks, vs), table, views


def _fp64(q, views, table, lens, qlens, hs=HS):
    """Reference outputs of unrotated queries: rotate, attend in the stored domain (scale hs^-0.5 / hs), rotate back."""
    out = []
    at = 0
    qr = O.rht(q.astype(np.float64))
    for i, (n, T) in enumerate(zip(lens, qlens)):
        K, V = O.dequant_f64(views, table[i], n)
        o = O.attention_f64(qr[at:at + T], K, V, n, hs ** -0.5 / hs)
        out.append(O.rht(o, inverse=True) / hs)
        at += T
    return np.concatenate(out)


def _segm(device, rows, segments, nq=NQ, hs=HS):
    import torch
    return (torch.full((rows, nq, segments, hs), float("nan"), dtype=torch.float32, device=device),
            torch.full((rows, nq, segments), float("nan"), dtype=torch.float32, device=device),
            torch.full((rows, nq, segments), float("nan"), dtype=torch.float32, device=device))


def _call(views, q, out, cu, used, table, max_q, max_k, segm, segments, hs=HS):
    from vllm_quantpack.attention import int4_kv
    kc, vc, ks, vs = views
    int4_kv.unified_attention_int4(
        q, kc, vc, out, cu_seqlens_q=cu, max_seqlen_q=max_q, seqused_k=used, max_seqlen_k=max_k,
        softmax_scale=hs ** -0.5, window_size=(-1, -1), block_table=table, softcap=0.0, sinks=None, alibi_slopes=None,
        use_alibi_sqrt=False, qq_bias=None, output_scale=None, mm_prefix_range=None, k_scale_cache=ks,
        v_scale_cache=vs, seq_threshold_3D=segm[0].shape[0] if segm else None,
        num_par_softmax_segments=segments if segm else None, softmax_segm_output=segm[0] if segm else None,
        softmax_segm_max=segm[1] if segm else None, softmax_segm_expsum=segm[2] if segm else None)


def _batch(device, seqs, fmt, seed, nkv=NKV, hs=HS, nq=NQ):
    import torch
    lens = [n for _, n in seqs]
    qlens = [T for T, _ in seqs]
    views, table, host = _stored_cache(device, fmt, lens, seed, nkv=nkv, hs=hs)
    g = torch.Generator(device=device).manual_seed(seed + 1)
    q = torch.randn((sum(qlens), nq, hs), generator=g, device=device, dtype=torch.bfloat16)
    cu = np.concatenate(([0], np.cumsum(qlens))).astype(np.int32)
    ref = _fp64(to_f32(q), host, table, lens, qlens, hs)
    return views, table, q, cu, lens, qlens, ref


@pytest.mark.parametrize("fmt", ["int4", "int8"])
def test_mixed_batch_long_prefill_and_mtp_decodes(device, fmt):
    """One step with a 256-token chunk over 40000 keys and MTP decodes of 4, 3 and 1 query tokens (the reference's
    mixed steps): the short sequences take the split-KV kernel through the device route table, the chunk the
    prefill kernel, in one call; every sequence within 0.5 % of fp64."""
    import torch
    seqs = [(256, 40000), (4, 20000), (3, 9000), (1, 16384)]
    views, table, q, cu, lens, qlens, ref = _batch(device, seqs, fmt, 500 + (fmt == "int8"))
    out = torch.full_like(q, float("nan"))
    segm = _segm(device, 32, 64)
    _call(views, q, out, i32(cu, device), i32(lens, device), i32(table, device), max(qlens), max(lens), segm, 64)
    torch.cuda.synchronize()
    got = to_f32(out)
    for i in range(len(seqs)):
        sl = slice(cu[i], cu[i + 1])
        assert O.relerr(got[sl], ref[sl]) < 5e-3, (i, O.relerr(got[sl], ref[sl]))
    # the short sequences' partials went to the first segment-buffer rows (4 + 3 + 1 of them), not to token rows
    assert np.isfinite(to_f32(segm[1])[:8, :, 0]).all() and np.isnan(to_f32(segm[1])[8:]).all()


@pytest.mark.parametrize("fmt", ["int4", "int8"])
def test_mixed_batch_head_64(device, fmt):
    """Head 64 through the drop-in: a 40-token chunk (query slices of the split-KV kernel) beside decodes of 4 and 1
    tokens, the rotations fused, 16 query heads on 2 KV heads; within 0.5 % of fp64."""
    import torch
    seqs = [(40, 3000), (4, 2000), (1, 700)]
    views, table, q, cu, lens, qlens, ref = _batch(device, seqs, fmt, 520 + (fmt == "int8"), nkv=2, hs=64, nq=16)
    out = torch.full_like(q, float("nan"))
    segm = _segm(device, 32, 16, nq=16, hs=64)
    _call(views, q, out, i32(cu, device), i32(lens, device), i32(table, device), max(qlens), max(lens), segm, 16,
          hs=64)
    torch.cuda.synchronize()
    got = to_f32(out)
    for i in range(len(seqs)):
        sl = slice(cu[i], cu[i + 1])
        assert O.relerr(got[sl], ref[sl]) < 5e-3, (i, O.relerr(got[sl], ref[sl]))


def test_mixed_batch_short_rows_beyond_the_segment_buffers(device):
    """Segment buffers of 5 rows take the first two short sequences (4 + 1 rows); the next short sequence no longer
    fits and the prefill kernel serves it, as it does the chunk. Ragged lengths, first chunk without cached keys."""
    import torch
    seqs = [(4, 5000), (40, 40), (1, 3000), (2, 7000), (70, 2600), (3, 100)]
    views, table, q, cu, lens, qlens, ref = _batch(device, seqs, "int4", 510)
    out = torch.full_like(q, float("nan"))
    segm = _segm(device, 5, 16)
    _call(views, q, out, i32(cu, device), i32(lens, device), i32(table, device), max(qlens), max(lens), segm, 16)
    torch.cuda.synchronize()
    got = to_f32(out)
    for i in range(len(seqs)):
        sl = slice(cu[i], cu[i + 1])
        assert O.relerr(got[sl], ref[sl]) < 5e-3, i


def test_batch_without_segment_buffers_takes_the_prefill(device):
    """Without segment buffers every sequence, short ones included, goes through the prefill kernel."""
    import torch
    seqs = [(2, 3000), (1, 500), (33, 1200)]
    views, table, q, cu, lens, qlens, ref = _batch(device, seqs, "int8", 520)
    out = torch.empty_like(q)
    _call(views, q, out, i32(cu, device), i32(lens, device), i32(table, device), max(qlens), max(lens), None, 0)
    torch.cuda.synchronize()
    assert O.relerr(to_f32(out), ref) < 5e-3


@pytest.mark.parametrize("max_m", ["64", "32", "16"], ids=["one-program", "capped-32", "stock-rows"])
def test_batched_mtp_decodes_with_capped_query_rows(device, monkeypatch, max_m):
    """tests/test_int4_kv.py:230-249: 4, 3 and 1 query tokens in one step with the decode row cap of
    VLLM_QUANTPACK_INT4_DECODE; at 16 the 4- and 3-token sequences run as token groups of one row tile."""
    import torch

    from vllm_quantpack.attention import int4_kv
    monkeypatch.setenv("VLLM_QUANTPACK_INT4_DECODE", f"64,4,auto,{max_m}")
    assert int4_kv.decode_row_cap(256) == (16 if max_m == "16" else 32)
    seqs = [(4, 20000), (3, 9000), (1, 16384), (4, 3072)]
    views, table, q, cu, lens, qlens, ref = _batch(device, seqs, "int4", 530)
    out = torch.empty_like(q)
    _call(views, q, out, i32(cu, device), i32(lens, device), i32(table, device), 4, max(lens), _segm(device, 16, 64),
          64)
    torch.cuda.synchronize()
    got = to_f32(out)
    for i in range(len(seqs)):
        sl = slice(cu[i], cu[i + 1])
        assert O.relerr(got[sl], ref[sl]) < 5e-3, i


@pytest.mark.parametrize("fmt", ["int4", "int8"])
def test_fused_query_rotation_is_bit_identical(device, fmt):
    """Rotating q inside the kernels' loads gives the same bits as rotating it first (qp_rht) and attending in the
    cache's domain: decode (one and two row tiles) and prefill."""
    import torch

    from qp_testlib import random_cache
    from vllm_quantpack.attention import int4_kv, int4_prefill, rht
    rng = np.random.default_rng(540)
    n = 3000
    nb = -(-n // BS)
    kv, _ = random_cache(rng, nb, NKV, BS, HS, fmt)
    _, views = torch_cache(kv, HS, fmt, device)
    kc, vc, ks, vs = views
    signs = rht.signs(HS, device)
    table = torch.arange(nb, dtype=torch.int32, device=device)[None]
    for T in (1, 4, 40):
        q = torch.randn((T, NQ, HS), device=device, dtype=torch.bfloat16)
        q_rot = rht.single_rht(q)
        cu, used = i32([0, T], device), i32([n], device)
        a, b = torch.empty_like(q), torch.empty_like(q)
        if T <= 4:
            kw = dict(cu_seqlens_q=cu, seqused_k=used, block_table=table, max_seqlen_q=T, softmax_scale=0.004,
                      num_segments=16)
            int4_kv.paged_decode(q_rot, kc, vc, ks, vs, a, **kw, softmax_segm_output=_segm(device, T, 16)[0],
                                 softmax_segm_max=_segm(device, T, 16)[1], softmax_segm_expsum=_segm(device, T, 16)[2])
            s2 = _segm(device, T, 16)
            int4_kv.paged_decode(q, kc, vc, ks, vs, b, **kw, softmax_segm_output=s2[0], softmax_segm_max=s2[1],
                                 softmax_segm_expsum=s2[2], query_signs=signs)
        else:
            kw = dict(cu_seqlens_q=cu, seqused_k=used, block_table=table, max_seqlen_q=T, softmax_scale=0.004)
            int4_prefill.prefill_attention(q_rot, kc, vc, ks, vs, a, **kw)
            int4_prefill.prefill_attention(q, kc, vc, ks, vs, b, **kw, query_signs=signs)
        torch.cuda.synchronize()
        assert torch.equal(a, b), T


@pytest.mark.parametrize("case", ["decode", "mixed", "prefill"])
def test_drop_in_attention_does_not_wait_for_the_gpu(device, case):
    """tests/test_int4_kv.py:252-315: no host synchronisation inside the drop-in call, for a decode step, a mixed
    step and a prefill chunk (the rotation signs exist already, as patch_int4_kv makes them)."""
    import torch

    from vllm_quantpack.attention import rht
    seqs = {"decode": [(2, 6000), (1, 3000)], "mixed": [(256, 9000), (3, 5000)], "prefill": [(300, 8000)]}[case]
    views, table, q, cu, lens, qlens, ref = _batch(device, seqs, "int4", 550)
    rht.signs(HS, device)
    args = (i32(cu, device), i32(lens, device), i32(table, device), max(qlens), max(lens), _segm(device, 32, 64), 64)
    out = torch.empty_like(q)
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        _call(views, q, out, *args)
    finally:
        torch.cuda.set_sync_debug_mode("default")
    torch.cuda.synchronize()
    assert O.relerr(to_f32(out), ref) < 5e-3


def test_prefill_sequence_does_not_wait_for_the_gpu(device):
    """The reference's prefill_sequence(q_rot, ...) call (tests/test_int4_kv.py:252-276) under sync debug mode."""
    import torch

    from qp_testlib import bf16_tensor, random_cache
    from vllm_quantpack.attention import int4_prefill
    rng = np.random.default_rng(560)
    n, qlen = 9000, 256
    nb = -(-n // BS)
    kv, v = random_cache(rng, nb, NKV, BS, HS)
    _, (kc, vc, ks, vs) = torch_cache(kv, HS, "int4", device)
    q = O.f32_to_bf16_bits(rng.standard_normal((qlen, NQ, HS)).astype(np.float32))
    qt = bf16_tensor(q, device)
    table = torch.arange(nb, dtype=torch.int32, device=device)
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        o = int4_prefill.prefill_sequence(qt, kc, vc, ks, vs, table, n, 0.05, None)
    finally:
        torch.cuda.set_sync_debug_mode("default")
    K, V = O.dequant_f64(v, np.arange(nb), n)
    assert O.relerr(to_f32(o), O.attention_f64(O.bf16_bits_to_f32(q), K, V, n, 0.05)) < 5e-3


def test_drop_in_attention_in_a_hip_graph(device):
    """unified_attention_int4 itself recorded in a HIP graph (a decode step of two sequences): three replays, each
    after eager work that changes the queries and the contexts, each equal to an eager call on the same inputs."""
    import torch
    seqs = [(2, 7000), (1, 4000)]
    views, table, q0, cu, lens, qlens, _ = _batch(device, seqs, "int8", 570)
    q = q0.clone()
    used = i32(lens, device)
    segm = _segm(device, 8, 64)
    args = (i32(cu, device), used, i32(table, device), 2, max(lens), segm, 64)
    out = torch.empty_like(q)
    _call(views, q, out, *args)                 # warm-up outside the capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            _call(views, q, out, *args)
    torch.cuda.synchronize()
    gen = torch.Generator(device=device).manual_seed(5)
    for step in range(3):
        q.copy_(torch.randn(q.shape, generator=gen, device=device, dtype=torch.bfloat16))
        used.copy_(i32([lens[0] - 100 * step, lens[1] - 7 * step], device))
        _call(views, q, out, *args)
        torch.cuda.synchronize()
        want = out.clone()
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), step
