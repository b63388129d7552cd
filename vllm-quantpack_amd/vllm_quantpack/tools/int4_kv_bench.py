"""Time this package's int4 / k8v4 KV-cache attention per layer on this GPU, to pick VLLM_QUANTPACK_INT4_DECODE.

The kernels have fixed tiles, so of a decode config "tile,warps,segments[,rows]" only the segment count (the split-KV
segments per sequence and KV head, which also sizes vLLM's segment buffers) and the optional query-row cap (16: one
row tile per split-KV workgroup, 32 or more: two) change anything; tile and warps are parsed and ignored. Per context
length the tool fills a random cache through the package's own store and times, per attention layer,

  decode   one request with 1 + MTP query tokens through unified_attention_int4, for every decode config;
  prefill  one 1024-query chunk at the end of the context through the same call (the MFMA prefill kernel).

Times are CUDA-event averages over --reps calls queued back to back (the drop-in call as vLLM makes it: routing,
fused rotations, split-KV decode and merge, or prefill). Each line also prints the largest per-row relative error
against an fp64 attention over the dequantised cache, so a config that changes the result shows up. The shape
defaults to 24 query / 4 KV heads at head 256 and block size 3072, as the reference's tool (tools/int4_kv_bench.py).

usage: python -m vllm_quantpack.tools.int4_kv_bench [--contexts 32768,131072,262144] [--decode 64,4,16:64,4,32:...]
           [--q-heads 24] [--kv-heads 4] [--head-size 256] [--block-size 3072] [--mtp 1] [--key-format int4|int8]
           [--reps 20]
"""
import argparse
import contextlib
import os
import sys

DEFAULT_SEGMENTS = (16, 32, 64, 128)
ENV = "VLLM_QUANTPACK_INT4_DECODE"


def parse_configs(text):
    """"tile,warps,segments[,rows]" configs separated by ':' -> tuples, segments an int or 'auto'."""
    out = []
    for c in text.split(":"):
        f = [x.strip() for x in c.split(",")]
        if len(f) not in (3, 4):
            raise ValueError(f"decode config {c!r}: expected tile,warps,segments[,rows]")
        seg = f[2] if f[2] == "auto" else int(f[2])
        out.append((int(f[0]), int(f[1]), seg) + tuple(int(x) for x in f[3:]))
    return out


@contextlib.contextmanager
def _env(name, value):
    old = os.environ.get(name)
    os.environ[name] = value
    try:
        yield
    finally:
        if old is None:
            os.environ.pop(name, None)
        else:
            os.environ[name] = old


def _cache(n, nkv, hs, bs, key_format, device):
    """A random cache of n tokens filled by reshape_and_cache_int4 (rotation + quantisation on the GPU), block table
    0..nb-1: the four views and the block count."""
    import torch

    from ..attention import int4_kv, k8v4_kv
    nb = -(-n // bs)
    cell = k8v4_kv.cell_bytes(hs, hs) if key_format == "int8" else hs + 8
    kv = torch.zeros((nb, nkv, bs, cell), dtype=torch.uint8, device=device)
    views = k8v4_kv.views(kv, hs) if key_format == "int8" else k8v4_kv.int4_views(kv, hs)
    g = torch.Generator(device=device).manual_seed(0)
    for s in range(0, n, 16384):
        t = min(16384, n - s)
        k = torch.randn((t, nkv, hs), generator=g, device=device, dtype=torch.bfloat16)
        v = torch.randn((t, nkv, hs), generator=g, device=device, dtype=torch.bfloat16)
        int4_kv.reshape_and_cache_int4(k, v, views[0], views[1], torch.arange(s, s + t, device=device),
                                       k_scale_cache=views[2], v_scale_cache=views[3])
    return (kv,) + tuple(views), nb


def _dequant(views, n, hs):
    """fp64 K, V [n, nkv, hs] of the first n tokens (block table 0..nb-1) from the cache views."""
    import torch
    kc, vc, ks, vs = views
    nkv = kc.shape[2]

    def words(sc):
        bits = sc.reshape(-1, nkv)[:n].contiguous().view(torch.int32)
        return (bits & 0xF).double()[..., None], (bits & -16).view(torch.float32).double()[..., None]

    def nibbles(c):
        b = c.reshape(-1, nkv, c.shape[-1])[:n, :, :hs // 2].to(torch.int16)
        return torch.stack((b & 0xF, b >> 4), -1).reshape(n, nkv, hs).double()

    zv, sv = words(vs)
    V = (nibbles(vc) - zv) * sv
    if kc.dtype == torch.int8:
        K = kc.reshape(-1, nkv, kc.shape[-1])[:n, :, :hs].double() * \
            ks.reshape(-1, nkv)[:n].double()[..., None]
    else:
        zk, sk = words(ks)
        K = (nibbles(kc) - zk) * sk
    return K, V


def _reference(q, K, V, n, rows, scale):
    """fp64 attention of query rows `rows` of q (the last len(q) positions of an n-token context) in the cache's
    rotated domain, rotated back: (softmax(R q . K * scale / hs) V) R^T / hs."""
    import torch

    from ..attention import rht
    nq, hs = q.shape[1], q.shape[2]
    nkv = K.shape[1]
    qr = rht.single_rht(q[rows].float()).double()
    pos = n - len(q) + torch.tensor(rows, device=q.device)
    masked = torch.arange(n, device=q.device)[None] > pos[:, None]
    out = torch.empty((len(rows), nq, hs), dtype=torch.float64, device=q.device)
    for h in range(nq):
        kv = h // (nq // nkv)
        s = (qr[:, h] @ K[:, kv].T) * (scale / hs)
        out[:, h] = torch.softmax(s.masked_fill(masked, float("-inf")), -1) @ V[:, kv]
    return rht.single_rht(out.float(), inverse=True, out_scale=1.0 / hs).double()


def max_row_relerr(o, ref):
    """max over (token, head) rows of |o - ref| / |ref|."""
    d = (o.double() - ref).flatten(0, -2).norm(dim=-1)
    return float((d / ref.flatten(0, -2).norm(dim=-1)).max())


def _timed(fn, reps):
    import torch
    fn()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        fn()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / reps


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0],
                                 epilog=f"Set the chosen config with {ENV}=tile,warps,segments[,rows] "
                                        "(default 64,4,auto).")
    ap.add_argument("--contexts", default="32768,131072,262144")
    ap.add_argument("--decode", default=None, help="tile,warps,segments[,max query rows] configs separated by ':' "
                    "(default: 64,4 with 16, 32, 64 and 128 segments); segments may be 'auto'")
    ap.add_argument("--prefill-tiles", default=None, help="accepted for the reference's command lines; the MFMA "
                    "prefill kernel's tiles are fixed")
    ap.add_argument("--q-heads", type=int, default=24)
    ap.add_argument("--kv-heads", type=int, default=4)
    ap.add_argument("--head-size", type=int, default=256)
    ap.add_argument("--block-size", type=int, default=3072)
    ap.add_argument("--mtp", type=int, default=1, help="draft tokens: decode steps have 1 + MTP query tokens")
    ap.add_argument("--key-format", choices=("int4", "int8"), default="int4",
                    help="int4 keys (int4_per_token_head) or int8 keys (k8v4_per_token_head)")
    ap.add_argument("--reps", type=int, default=20, help="timed decode calls per config (prefill: a quarter)")
    a = ap.parse_args(argv)
    configs = parse_configs(a.decode) if a.decode else [(64, 4, s) for s in DEFAULT_SEGMENTS]
    contexts = [int(x) for x in a.contexts.split(",")]
    if 1 + a.mtp > 4:
        raise SystemExit("--mtp: at most 3 draft tokens (split-KV decode takes 1 to 4 query tokens)")

    import torch

    from ..attention import int4_kv
    if not torch.cuda.is_available():
        raise SystemExit("int4_kv_bench: no GPU")
    dev = torch.device("cuda", torch.cuda.current_device())
    props = torch.cuda.get_device_properties(dev)
    cus = props.multi_processor_count
    nq, nkv, hs, bs = a.q_heads, a.kv_heads, a.head_size, a.block_size
    print(f"{props.name}, {cus} CUs (auto: {int4_kv.segments_for(cus)} segments) | {nq} q / {nkv} KV heads, head "
          f"{hs}, block {bs}, {a.key_format} keys | times per attention layer", flush=True)
    results = []
    for n in contexts:
        (kv, kc, vc, ks, vs), nb = _cache(n, nkv, hs, bs, a.key_format, dev)
        K, V = _dequant((kc, vc, ks, vs), n, hs)
        table = torch.arange(nb, dtype=torch.int32, device=dev)[None]
        used = torch.tensor([n], dtype=torch.int32, device=dev)

        def attend(q, out, segments):
            segm = (torch.empty((32, nq, segments, hs), dtype=torch.float32, device=dev),
                    torch.empty((32, nq, segments), dtype=torch.float32, device=dev),
                    torch.empty((32, nq, segments), dtype=torch.float32, device=dev))
            cu = torch.tensor([0, len(q)], dtype=torch.int32, device=dev)
            return lambda: int4_kv.unified_attention_int4(
                q, kc, vc, out, cu_seqlens_q=cu, max_seqlen_q=len(q), seqused_k=used, max_seqlen_k=n,
                softmax_scale=hs ** -0.5, window_size=(-1, -1), block_table=table, softcap=0.0, sinks=None,
                alibi_slopes=None, use_alibi_sqrt=False, qq_bias=None, output_scale=None, mm_prefix_range=None,
                k_scale_cache=ks, v_scale_cache=vs, seq_threshold_3D=32, num_par_softmax_segments=segments,
                softmax_segm_output=segm[0], softmax_segm_max=segm[1], softmax_segm_expsum=segm[2])

        q = torch.randn((1 + a.mtp, nq, hs), device=dev, dtype=torch.bfloat16)
        ref = _reference(q, K, V, n, list(range(len(q))), hs ** -0.5)
        out = torch.empty_like(q)
        for c in configs:
            segments = int4_kv.segments_for(cus) if c[2] == "auto" else c[2]
            with _env(ENV, ",".join(str(x) for x in c)):
                ms = _timed(attend(q, out, segments), a.reps)
            err = max_row_relerr(out, ref)
            rows = f" max rows {c[3]:>2}" if len(c) > 3 else ""
            print(f"ctx {n:>7} decode  segments {segments:>3}{rows}  {ms * 1e3:9.1f} us  relerr {err:.1e}",
                  flush=True)
            results.append(dict(context=n, kind="decode", config=c, segments=segments, ms=ms, relerr=err))
        chunk = min(1024, n)
        q = torch.randn((chunk, nq, hs), device=dev, dtype=torch.bfloat16)
        rows = sorted({0, chunk // 2, chunk - 1})
        ref = _reference(q, K, V, n, rows, hs ** -0.5)
        out = torch.empty_like(q)
        ms = _timed(attend(q, out, int4_kv.segments_for(cus)), max(1, a.reps // 4))
        err = max_row_relerr(out[rows], ref)
        print(f"ctx {n:>7} prefill {chunk}-token chunk (MFMA)  {ms:9.3f} ms  relerr {err:.1e}", flush=True)
        results.append(dict(context=n, kind="prefill", chunk=chunk, ms=ms, relerr=err))
        del kv, kc, vc, ks, vs, K, V
        torch.cuda.empty_cache()
    print(f"Set the fastest decode config with {ENV}=tile,warps,segments[,rows] (default 64,4,auto).")
    return results


if __name__ == "__main__":
    main()
    sys.exit(0)
