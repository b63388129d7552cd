"""qp_attention_noalloc: a decode step whose split-KV partials live in the library's static device buffer, against
qp_attention with the caller's segment buffers (the same kernels and segment count, so the same bits), on two calls in
a row, the second with a smaller batch, and against the fp64 closed form."""
import ctypes

import numpy as np
import pytest

from oracle import qp_oracle as O
from qp_testlib import i32, to_f32, torch_cache

pytestmark = pytest.mark.gpu

NQ, NKV, HS, BS = 24, 4, 256, 16


def _case(device, seed, seqs, fmt):
    import torch

    from vllm_quantpack.attention import int4_kv
    rng = np.random.default_rng(seed)
    lens = [n for _, n in seqs]
    nbs = [-(-n // BS) for n in lens]
    total = sum(nbs) + 2
    kv_np = O.new_cache(total, NKV, BS, O.int4_cell_bytes(HS) if fmt == "int4" else O.k8v4_cell_bytes(HS))
    t, (kc, vc, ks, vs) = torch_cache(kv_np, HS, fmt, device)
    pool = rng.permutation(total).astype(np.int32)
    table = np.zeros((len(seqs), max(nbs)), np.int32)
    at = 0
    g = torch.Generator(device=device).manual_seed(seed)
    for i, n in enumerate(lens):
        table[i, :nbs[i]] = pool[at:at + nbs[i]]
        at += nbs[i]
        slots = (torch.as_tensor(table[i, :nbs[i]].astype(np.int64), device=device)[:, None] * BS
                 + torch.arange(BS, device=device)).flatten()[:n]
        k = torch.randn((n, NKV, HS), generator=g, device=device, dtype=torch.bfloat16)
        v = torch.randn((n, NKV, HS), generator=g, device=device, dtype=torch.bfloat16)
        int4_kv.reshape_and_cache_int4(k, v, kc, vc, slots, k_scale_cache=ks, v_scale_cache=vs)
    qlens = [T for T, _ in seqs]
    q = torch.randn((sum(qlens), NQ, HS), generator=g, device=device, dtype=torch.bfloat16)
    cu = np.concatenate(([0], np.cumsum(qlens))).astype(np.int32)
    torch.cuda.synchronize()
    host = t.cpu().numpy().view(np.uint8)
    views = O.int4_views(host, HS) if fmt == "int4" else O.k8v4_views(host, HS)
    ref = []
    qr = O.rht(to_f32(q).astype(np.float64))
    for i, (T, n) in enumerate(seqs):
        K, V = O.dequant_f64(views, table[i], n)
        o = O.attention_f64(qr[cu[i]:cu[i + 1]], K, V, n, HS ** -0.5 / HS)
        ref.append(O.rht(o, inverse=True) / HS)
    return (kc, vc, ks, vs), q, i32(cu, device), i32(lens, device), i32(table, device), max(qlens), np.concatenate(ref)


def test_noalloc_matches_qp_attention_on_two_calls(device):
    import torch

    from vllm_quantpack import _hip
    from vllm_quantpack.attention import int4_kv, rht
    lib = _hip.lib()
    signs = rht.signs(HS, device)
    for seed, seqs, fmt, S in ((800, [(2, 6000), (1, 3000)], "int4", 64), (801, [(1, 900)], "int8", 16)):
        (kc, vc, ks, vs), q, cu, used, table, max_q, ref = _case(device, seed, seqs, fmt)
        segm = (torch.empty((q.shape[0], NQ, S, HS), dtype=torch.float32, device=device),
                torch.empty((q.shape[0], NQ, S), dtype=torch.float32, device=device),
                torch.empty((q.shape[0], NQ, S), dtype=torch.float32, device=device))
        cache = _hip.paged_cache(kc, vc, ks, vs, HS)
        want = torch.full_like(q, float("nan"))
        args = int4_kv.attention_args(q, want, cu_seqlens_q=cu, seqused_k=used, block_table=table,
                                      max_seqlen_q=max_q, max_seqlen_k=int(used.max()), softmax_scale=HS ** -0.5 / HS,
                                      num_segments=S, softmax_segm_output=segm[0], softmax_segm_max=segm[1],
                                      softmax_segm_expsum=segm[2], rht_signs=signs, rht_out_scale=1.0 / HS)
        assert lib.qp_attention_workspace_size(cache, args) == 0
        _hip.check(lib.qp_attention(cache, args, _hip.stream_of(q)), "qp_attention")
        got = torch.full_like(q, float("nan"))
        args.out = got.data_ptr()
        args.segm_output = args.segm_max = args.segm_expsum = None      # not read by the static-buffer variant
        torch.cuda.synchronize()
        before = torch.cuda.memory_allocated(device)
        _hip.check(lib.qp_attention_noalloc(cache, args, _hip.stream_of(q)), "qp_attention_noalloc")
        torch.cuda.synchronize()
        assert torch.cuda.memory_allocated(device) == before
        assert torch.equal(got, want), seqs
        assert O.relerr(to_f32(got), ref) < 5e-3


def test_noalloc_rejects_a_batch_beyond_its_buffer():
    """Checked on the host before anything runs: partials of 64 tokens x 24 heads x 256 segments x 258 floats do not
    fit the 32 MiB buffer."""
    import torch

    from vllm_quantpack import _hip
    lib = _hip.lib()
    cache = _hip.PagedCache()
    cache.num_kv_heads, cache.head_size, cache.block_size = NKV, HS, BS
    args = _hip.AttentionArgs()
    args.num_seqs, args.num_tokens, args.num_q_heads, args.max_query_len, args.num_segments = 32, 64, NQ, 2, 256
    st = lib.qp_attention_noalloc(ctypes.byref(cache), ctypes.byref(args), None)
    assert st == _hip.QP_ERR_UNSUPPORTED
    assert "static buffer" in lib.qp_last_error().decode()
    args.max_query_len = 8                                  # a prefill chunk is not for this entry point
    assert lib.qp_attention_noalloc(ctypes.byref(cache), ctypes.byref(args), None) == _hip.QP_ERR_UNSUPPORTED
    # head 512 with 24 query heads on one KV head: a decode shape qp_attention sends to its prefill path
    cache.num_kv_heads, cache.head_size = 1, 512
    args.num_seqs, args.num_tokens, args.max_query_len, args.num_segments = 1, 1, 1, 4
    assert lib.qp_attention_noalloc(ctypes.byref(cache), ctypes.byref(args), None) == _hip.QP_ERR_UNSUPPORTED
    assert "head 512" in lib.qp_last_error().decode()
    del torch
