"""Every named workload of the package's synthetic set through the public path.

- The small versions (contexts 16x shorter, same layouts, block tables, formats and scales) against the oracle: the
  fp64 closed form within 0.5 % and the reference kernel's emulation within 1e-2.
- The full sizes (the configurations the benchmark is quoted on) against an fp64 dequantise-then-attend computed on
  the GPU from the same cache bytes; the oracle's numpy path would take minutes there. The dequantisation is the
  closed form (code - zp) * scale of the oracle's `dequant_f64`, restated in torch so that it runs on the device.
"""
import numpy as np
import pytest

from oracle import qp_oracle as O
from qp_testlib import assert_emulation, to_f32

DECODE = ["decode-int4-4k-t1", "decode-int4-128k-t2", "decode-int4-256k-t4", "decode-k8v4-ragged-b32"]
PREFILL = ["prefill-int4-128k-c1024", "prefill-k8v4-128k-c1024", "prefill-int4-h512-128k-c1024",
           "prefill-int4-g16-32k-c1024", "prefill-int4-g8-128k-c1024",
           "prefill-int4-g4-128k-c1024"]
SEGMENTS = 64


def _views(w):
    return O.int4_views(w.kv, w.head_size) if w.key_format == "int4" else O.k8v4_views(w.kv, w.head_size)


def _decode(w, device):
    """Split-KV decode + merge of the workload through int4_kv.paged_decode; out fp32 numpy [T, NQ, HS]."""
    import torch

    from vllm_quantpack.attention import int4_kv
    from vllm_quantpack.tools import synth
    d = synth.to_device(w, device)
    T, nq, hs = w.q.shape
    so = torch.empty((T, nq, SEGMENTS, hs), dtype=torch.float32, device=device)
    sm = torch.empty((T, nq, SEGMENTS), dtype=torch.float32, device=device)
    ss = torch.empty((T, nq, SEGMENTS), dtype=torch.float32, device=device)
    out = torch.empty((T, nq, hs), dtype=torch.bfloat16, device=device)
    int4_kv.paged_decode(d["q"], d["k_cache"], d["v_cache"], d["k_scale_cache"], d["v_scale_cache"], out,
                         cu_seqlens_q=d["cu_seqlens_q"], seqused_k=d["seqused_k"], block_table=d["block_table"],
                         max_seqlen_q=w.max_query_len, softmax_scale=w.softmax_scale, num_segments=SEGMENTS,
                         softmax_segm_output=so, softmax_segm_max=sm, softmax_segm_expsum=ss)
    torch.cuda.synchronize()
    return to_f32(out), d


def _prefill(w, device):
    """The chunk's new keys stored into the cache, then the chunked prefill; out fp32 numpy [T, NQ, HS]."""
    import torch

    from vllm_quantpack.attention import int4_prefill, k8v4_kv
    from vllm_quantpack.tools import synth
    d = synth.to_device(w, device)
    k8v4_kv.store(None, d["new_key"], d["new_value"], d["k_cache"], d["v_cache"], d["new_slots"],
                  k_scale_cache=d["k_scale_cache"], v_scale_cache=d["v_scale_cache"], rotate=False)
    out = torch.empty_like(d["q"])
    int4_prefill.prefill_attention(d["q"], d["k_cache"], d["v_cache"], d["k_scale_cache"], d["v_scale_cache"], out,
                                   cu_seqlens_q=d["cu_seqlens_q"], seqused_k=d["seqused_k"],
                                   block_table=d["block_table"], max_seqlen_q=w.max_query_len,
                                   softmax_scale=w.softmax_scale)
    torch.cuda.synchronize()
    return to_f32(out), d


def _prefill_again(w, d):
    """The chunked prefill once more over the cache _prefill stored into; out fp32 numpy [T, NQ, HS]."""
    import torch

    from vllm_quantpack.attention import int4_prefill
    out = torch.empty_like(d["q"])
    int4_prefill.prefill_attention(d["q"], d["k_cache"], d["v_cache"], d["k_scale_cache"], d["v_scale_cache"], out,
                                   cu_seqlens_q=d["cu_seqlens_q"], seqused_k=d["seqused_k"],
                                   block_table=d["block_table"], max_seqlen_q=w.max_query_len,
                                   softmax_scale=w.softmax_scale)
    torch.cuda.synchronize()
    return to_f32(out)


def _oracle_decode(w):
    """fp64 closed form and the reference kernel's emulation, sequence by sequence."""
    views = _views(w)
    ref, emu = np.zeros(w.q.shape), np.zeros(w.q.shape)
    q = O.bf16_bits_to_f32(w.q)
    for i in range(len(w.seqused_k)):
        a, b = int(w.cu_seqlens_q[i]), int(w.cu_seqlens_q[i + 1])
        n = int(w.seqused_k[i])
        row = w.block_table[i]
        K, V = O.dequant_f64(views, row, n)
        ref[a:b] = O.attention_f64(q[a:b].astype(np.float64), K, V, n, w.softmax_scale)
        emu[a:b] = O.decode_emulated(q[a:b], views, row, n, w.softmax_scale, num_segments=SEGMENTS)
    return ref, emu


@pytest.mark.gpu
@pytest.mark.parametrize("name", DECODE)
def test_small_decode_workloads_match_the_oracle(device, name):
    from vllm_quantpack.tools import synth
    w = synth.make(name, small=True)
    out, _ = _decode(w, device)
    ref, emu = _oracle_decode(w)
    assert np.isfinite(out).all()
    assert O.relerr(out, ref) < 5e-3
    assert_emulation(out, emu)


@pytest.mark.gpu
@pytest.mark.parametrize("name", PREFILL)
def test_small_prefill_workload_matches_the_oracle(device, name):
    from vllm_quantpack.tools import synth
    w = synth.make(name, small=True)
    out, _ = _prefill(w, device)
    # the oracle stores the chunk's keys the same way, then attends in fp64
    views = _views(w)
    O.store(views, O.bf16_bits_to_f32(w.new_key), O.bf16_bits_to_f32(w.new_value), w.new_slots)
    n = int(w.seqused_k[0])
    K, V = O.dequant_f64(views, w.block_table[0], n)
    ref = O.attention_f64(O.bf16_bits_to_f32(w.q).astype(np.float64), K, V, n, w.softmax_scale)
    assert np.isfinite(out).all()
    assert O.relerr(out, ref) < 5e-3


def _dequant_gpu(kv, fmt, hs, blocks, n):
    """(K, V) fp64 [n, NKV, HS] of the first n tokens behind `blocks` (torch int64), from the device byte cache
    [num_blocks, NKV, BS, cell] (HND): (code - zp) * scale for int4 halves, code * scale for int8 keys."""
    import torch
    nkv, bs = kv.shape[1], kv.shape[2]
    cells = kv[blocks].permute(0, 2, 1, 3).reshape(-1, nkv, kv.shape[3])[:n]  # token-major
    kb = hs // 2 if fmt == "int4" else hs

    def word(at):
        return cells[..., at:at + 4].contiguous().view(torch.int32)[..., 0]

    def nibbles(codes, w):
        zp = (w & 0xF).to(torch.float64)
        scale = (w & -16).view(torch.float32).to(torch.float64)
        c = (codes.view(torch.uint8) if codes.dtype == torch.int8 else codes).to(torch.int32)
        x = torch.stack(((c & 0xF), (c >> 4)), dim=-1).flatten(-2).to(torch.float64)
        return (x - zp[..., None]) * scale[..., None]

    if fmt == "int4":
        K = nibbles(cells[..., :kb], word(kb))
    else:
        K = cells[..., :kb].view(torch.int8).to(torch.float64) * word(kb).view(torch.float32).to(torch.float64)[..., None]
    V = nibbles(cells[..., kb + 4:kb + 4 + hs // 2], word(kb + 4 + hs // 2))
    return K, V


def _attention_gpu(q, K, V, n, scale):
    """fp64 causal attention of the T query rows (the last T positions of n) on the device, one KV head at a time:
    q [T, NQ, HS] fp64, K / V [n, NKV, HS] fp64."""
    import torch
    T, nq, hs = q.shape
    nkv = K.shape[1]
    G = nq // nkv
    out = torch.empty_like(q)
    pos = n - T + torch.arange(T, device=q.device)
    keys = torch.arange(n, device=q.device)
    mask = keys[None, :] > pos[:, None]
    for h in range(nkv):
        for j in range(G):
            s = (q[:, h * G + j] @ K[:, h].T) * scale
            s.masked_fill_(mask, float("-inf"))
            p = torch.softmax(s, dim=-1)
            out[:, h * G + j] = p @ V[:, h]
    return out


def _full_reference(w, d):
    import torch
    q = d["q"].to(torch.float64)
    out = torch.empty_like(q)
    for i in range(len(w.seqused_k)):
        a, b = int(w.cu_seqlens_q[i]), int(w.cu_seqlens_q[i + 1])
        n = int(w.seqused_k[i])
        nb = -(-n // w.block_size)
        blocks = d["block_table"][i, :nb].to(torch.int64)
        K, V = _dequant_gpu(d["kv"], w.key_format, w.head_size, blocks, n)
        out[a:b] = _attention_gpu(q[a:b], K, V, n, w.softmax_scale)
        del K, V
    torch.cuda.synchronize()
    return to_f32(out)


@pytest.mark.gpu
@pytest.mark.parametrize("name", DECODE)
def test_full_size_decode_workloads_match_fp64(device, name):
    from vllm_quantpack.tools import synth
    w = synth.make(name)
    out, d = _decode(w, device)
    ref = _full_reference(w, d)
    assert np.isfinite(out).all()
    assert O.relerr(out, ref) < 5e-3
    del d
    # the same step again gives the same bits (each wave sums a fixed set of chunks in a fixed order)
    assert np.array_equal(_decode(w, device)[0], out)


@pytest.mark.gpu
@pytest.mark.parametrize("name", PREFILL)
def test_full_size_prefill_workload_matches_fp64(device, name):
    from vllm_quantpack.tools import synth
    w = synth.make(name)
    out, d = _prefill(w, device)          # the cache on the device now holds the stored chunk
    ref = _full_reference(w, d)
    assert np.isfinite(out).all()
    assert O.relerr(out, ref) < 5e-3
    # the same call again gives the same bits (a copy or barrier race shows up here as a few differing rows)
    assert np.array_equal(_prefill_again(w, d), out)


def test_gpu_dequant_restatement_matches_the_oracle():
    """The torch dequantisation above equals the oracle's fp64 dequantisation on a small cache (CPU)."""
    import torch

    from vllm_quantpack.tools import synth
    for name in ("decode-int4-4k-t1", "decode-k8v4-ragged-b32"):
        w = synth.make(name, small=True)
        views = _views(w)
        kv = torch.from_numpy(w.kv if w.key_format == "int4" else w.kv.view(np.int8))
        for i in range(min(3, len(w.seqused_k))):
            n = int(w.seqused_k[i])
            nb = -(-n // w.block_size)
            blocks = torch.from_numpy(w.block_table[i, :nb].astype(np.int64))
            K, V = _dequant_gpu(kv, w.key_format, w.head_size, blocks, n)
            Kr, Vr = O.dequant_f64(views, w.block_table[i], n)
            assert np.array_equal(K.numpy(), Kr) and np.array_equal(V.numpy(), Vr)
