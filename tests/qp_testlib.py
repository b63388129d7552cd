"""Shared helpers of the parity tests: random caches built on the oracle's numpy views, copied byte for byte to the
GPU, and thin wrappers that run the HIP path through the package's public functions."""
import numpy as np

from oracle import qp_oracle as O


def assert_emulation(out, emu, what=None):
    """The bar against the oracle's emulation of the reference's exact kernel: relative error below 1e-2 as the
    reference's own test measures it (Frobenius over the output, tests/test_int4_kv.py:160-161,190) and for every
    (token, head) output row on its own."""
    fro, row = O.relerr(out, emu), O.max_row_relerr(out, emu)
    assert fro < 1e-2 and row < 1e-2, (what, f"frobenius {fro:.3e}, worst row {row:.3e}")


def word(scale, zp):
    return np.uint32((int(np.float32(scale).view(np.uint32)) & 0xFFFFFFF0) | int(zp))


def random_cache(rng, num_blocks, nkv, bs, hs, fmt="int4", layout="hnd"):
    """(byte cache, oracle views) filled like the synthetic workloads: nibbles U{0..15}, scales lognormal(-3, .5)
    with zero points U{6..9}; int8 keys U{-127..127} with lognormal(-4, .5) scales."""
    cell = O.int4_cell_bytes(hs) if fmt == "int4" else O.k8v4_cell_bytes(hs)
    kv = O.new_cache(num_blocks, nkv, bs, cell, layout)
    v = O.int4_views(kv, hs) if fmt == "int4" else O.k8v4_views(kv, hs)
    shape = v.key_word.shape
    if fmt == "int4":
        v.key[...] = rng.integers(0, 256, v.key.shape, dtype=np.uint8)
        sc = rng.lognormal(-3, 0.5, shape).astype(np.float32)
        v.key_word[...] = (sc.view(np.uint32) & np.uint32(0xFFFFFFF0)) | rng.integers(6, 10, shape).astype(np.uint32)
    else:
        v.key[...] = rng.integers(-127, 128, v.key.shape, dtype=np.int8)
        v.key_word[...] = rng.lognormal(-4, 0.5, shape).astype(np.float32).view(np.uint32)
    v.value[...] = rng.integers(0, 256, v.value.shape, dtype=np.uint8)
    sc = rng.lognormal(-3, 0.5, shape).astype(np.float32)
    v.value_word[...] = (sc.view(np.uint32) & np.uint32(0xFFFFFFF0)) | rng.integers(6, 10, shape).astype(np.uint32)
    return kv, v


def torch_cache(kv, hs, fmt, device):
    """The byte cache on the device with the same physical layout, and the package's views of it."""
    import torch

    from vllm_quantpack.attention import k8v4_kv
    root = O._root(kv)
    if fmt == "int8":
        root = root.view(np.int8)
    t = torch.from_numpy(np.ascontiguousarray(root)).to(device)
    if root.shape != kv.shape:          # NHD storage, logical (blocks, heads, slots, cell)
        t = t.transpose(1, 2)
    if fmt == "int8":
        return t, k8v4_kv.views(t, hs)
    return t, k8v4_kv.int4_views(t, hs)


def bf16_tensor(bits, device):
    import torch
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(device).view(torch.bfloat16)


def to_f32(t):
    import torch
    return t.detach().to(torch.float32).cpu().numpy()


def run_decode(views, q, cu, used, table, max_q, scale, segments, device, rows=None):
    """Split-KV decode + merge through int4_kv.paged_decode. Returns (out fp32 numpy, segment buffers)."""
    import torch

    from vllm_quantpack.attention import int4_kv
    kc, vc, ks, vs = views
    T, nq, hs = q.shape
    rows = rows or T
    so = torch.full((rows, nq, segments, hs), float("nan"), dtype=torch.float32, device=device)
    sm = torch.full((rows, nq, segments), float("nan"), dtype=torch.float32, device=device)
    ss = torch.full((rows, nq, segments), float("nan"), dtype=torch.float32, device=device)
    out = torch.empty((T, nq, hs), dtype=torch.bfloat16, device=device)
    int4_kv.paged_decode(q, kc, vc, ks, vs, out, cu_seqlens_q=cu, seqused_k=used, block_table=table,
                         max_seqlen_q=max_q, softmax_scale=scale, num_segments=segments, softmax_segm_output=so,
                         softmax_segm_max=sm, softmax_segm_expsum=ss)
    torch.cuda.synchronize()
    return to_f32(out), (so, sm, ss)


def i32(x, device):
    import torch
    return torch.as_tensor(np.asarray(x, np.int32), device=device)
