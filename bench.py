"""Benchmark of the int4 KV-cache attention path on one MI355X.

A step is one split-KV decode + log-sum-exp merge of 2 query tokens (MTP 1) over a 131072-token int4 paged cache,
24 query / 4 KV heads, head 256, block 16, 8192 shuffled blocks (workload decode-int4-128k-t2): one attention layer
of one decode step, launched back to back. Inputs are seeded synthetic data resident in HBM before timing; the steps
cycle through --cache-copies independent copies of the cache (4 x 138 MB by default, more than the 256 MB last-level
cache), so each step reads its cache from HBM rather than from the last-level cache.

Prints one JSON line: decode tok/s (value), HBM GB/s and us per layer, the prefill-chunk workload's tok/s when the
prefill kernel is available, the roofline of the decode kernel (algorithmic bytes / its average duration measured with
events on its stream around a run of launches queued behind a spin, so the events see execution only), the drop-in
path's time per layer (unified_attention_int4 with the query rotation, eager and as a graph replay) and the CPU
baselines (the dequantise-then-attend restatement timed on this host, on the decode step and on the whole prefill
chunk).

    python bench.py [--gpus 1] [--steps 200] [--warmup 20] [--segments N] [--no-cpu] [--no-prefill]
    python bench.py --copy-probe MIB     # only a plain device copy of MIB MiB, 10 times (HBM counter calibration)

roofline.traffic is the decode kernel's HBM bytes per launch as the FETCH_SIZE + WRITE_SIZE counters read it, each
scaled by the ratio of known bytes to counted bytes of the plain copy; the figures come from the committed counter
summary profiles/decode_span_kernel_decode-int4-128k-t2_traffic.txt (null when it is absent).
"""
import argparse
import json
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "vllm-quantpack_amd"))

METRIC = "int4-KV decode tok/s + HBM GB/s at 128k ctx; prefill-chunk tok/s"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
DECODE_KERNEL = "qp::decode_span_kernel<256, 0, 1, 8>"
SPIN_CYCLES = 50_000_000


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def decode_bench(torch, args):
    from vllm_quantpack.attention import int4_kv
    from vllm_quantpack.tools import synth
    dev = torch.device("cuda:0")
    w = synth.make("decode-int4-128k-t2")
    # Independent copies of the layer's cache, used in turn: together they exceed the 256 MB last-level cache, so
    # every step streams its cache from HBM as it does in a model whose other layers run in between.
    copies = [synth.to_device(w, dev) for _ in range(args.cache_copies)]
    S = args.segments or int4_kv.segments_for(torch.cuda.get_device_properties(0).multi_processor_count)
    T, NQ, HS = w.q.shape
    so = torch.empty((T, NQ, S, HS), dtype=torch.float32, device=dev)
    sm = torch.empty((T, NQ, S), dtype=torch.float32, device=dev)
    ss = torch.empty((T, NQ, S), dtype=torch.float32, device=dev)
    out = torch.empty((T, NQ, HS), dtype=torch.bfloat16, device=dev)
    plans = [int4_kv.DecodePlan(d["q"], d["k_cache"], d["v_cache"], d["k_scale_cache"], d["v_scale_cache"], out,
                                cu_seqlens_q=d["cu_seqlens_q"], seqused_k=d["seqused_k"],
                                block_table=d["block_table"], max_seqlen_q=w.max_query_len,
                                softmax_scale=w.softmax_scale, num_segments=S, softmax_segm_output=so,
                                softmax_segm_max=sm, softmax_segm_expsum=ss) for d in copies]
    n = len(plans)
    stream = torch.cuda.current_stream(dev)
    # kernel durations: launches queued behind a spin that holds the stream, bracketed by one pair of events on that
    # stream, so the average is the execution time in a full queue (an event pair around every launch would add its
    # own dispatch overhead, about 3 us, to each): the split-KV decode kernel alone (the roofline's kernel) and the
    # step's two launches (decode + merge). At least 200 launches each, whatever --steps is. They run before the timed
    # steps, which therefore start on a GPU at its working clock, as in a serving loop (on an idle GPU the first
    # timed steps measured about 3 us slower each).
    reps = max(200, args.steps)

    def queued(fn):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(SPIN_CYCLES)
        a.record(stream)
        for i in range(reps):
            fn(plans[i % n])
        b.record(stream)
        torch.cuda.synchronize()
        return a.elapsed_time(b) / reps

    kern_ms = queued(lambda pl: pl.decode())
    pair_ms = queued(lambda pl: (pl.decode(), pl.merge()))
    for i in range(args.warmup):
        plans[i % n].run()
    torch.cuda.synchronize()
    # timed region: exactly `steps` decode steps (split-KV decode + merge), launched back to back
    t0 = time.perf_counter()
    for i in range(args.steps):
        plans[i % n].run()
    torch.cuda.synchronize()
    step_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    nbytes = synth.cache_bytes(w)
    result = dict(tokens_per_step=T, step_ms=step_ms, decode_kernel_us=kern_ms * 1e3, bytes=nbytes, segments=S,
                  pair_us=pair_ms * 1e3, out=out, w=w, copies=copies)
    return result


def dropin_bench(torch, args, r):
    """The drop-in path of one layer: unified_attention_int4 on unrotated queries (the query rotation, split-KV
    decode, merge and inverse rotation in one qp_attention call, plus the Python layer's argument checks and
    ctypes structs), timed eagerly over `steps` calls and as replays of one captured HIP graph of 40 layers (a
    serving engine captures a whole forward pass; one graph per layer would time the graph launch instead)."""
    from vllm_quantpack.attention import int4_kv, rht
    from vllm_quantpack.tools import synth
    dev = torch.device("cuda:0")
    w = r["w"]
    d = r["copies"][0]
    copies = r["copies"]
    T, NQ, HS = w.q.shape
    S = r["segments"]
    segm = (torch.empty((T, NQ, S, HS), dtype=torch.float32, device=dev),
            torch.empty((T, NQ, S), dtype=torch.float32, device=dev),
            torch.empty((T, NQ, S), dtype=torch.float32, device=dev))
    out = torch.empty((T, NQ, HS), dtype=torch.bfloat16, device=dev)
    rht.signs(HS, dev)

    def layer(c):
        int4_kv.unified_attention_int4(
            c["q"], c["k_cache"], c["v_cache"], out, cu_seqlens_q=c["cu_seqlens_q"], max_seqlen_q=w.max_query_len,
            seqused_k=c["seqused_k"], max_seqlen_k=int(w.seqused_k.max()), softmax_scale=w.softmax_scale * HS,
            window_size=(-1, -1), block_table=c["block_table"], softcap=0.0, sinks=None, alibi_slopes=None,
            use_alibi_sqrt=False, qq_bias=None, output_scale=None, mm_prefix_range=None,
            k_scale_cache=c["k_scale_cache"], v_scale_cache=c["v_scale_cache"], seq_threshold_3D=T,
            num_par_softmax_segments=S, softmax_segm_output=segm[0], softmax_segm_max=segm[1],
            softmax_segm_expsum=segm[2])

    n = len(copies)
    for i in range(args.warmup):
        layer(copies[i % n])
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        layer(copies[i % n])
    torch.cuda.synchronize()
    eager_us = (time.perf_counter() - t0) * 1e6 / args.steps
    layers = 40
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=side):
            for i in range(layers):
                layer(copies[i % n])
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    # at least 5 replays of the 40-layer graph (200 layers), more with more steps
    replays = max(5, args.steps // layers)
    t0 = time.perf_counter()
    for _ in range(replays):
        g.replay()
    torch.cuda.synchronize()
    graph_us = (time.perf_counter() - t0) * 1e6 / (replays * layers)
    del synth, d
    return dict(eager_us=eager_us, graph_us=graph_us)


def prefill_bench(torch, args):
    from vllm_quantpack.attention import int4_prefill
    from vllm_quantpack.tools import synth
    dev = torch.device("cuda:0")
    w = synth.make("prefill-int4-128k-c1024")
    d = synth.to_device(w, dev)
    out = torch.empty_like(d["q"])

    def step():
        int4_prefill.prefill_attention(d["q"], d["k_cache"], d["v_cache"], d["k_scale_cache"], d["v_scale_cache"],
                                       out, cu_seqlens_q=d["cu_seqlens_q"], seqused_k=d["seqused_k"],
                                       block_table=d["block_table"], max_seqlen_q=w.max_query_len,
                                       softmax_scale=w.softmax_scale)

    from vllm_quantpack.attention import k8v4_kv
    k8v4_kv.store(None, d["new_key"], d["new_value"], d["k_cache"], d["v_cache"], d["new_slots"],
                  k_scale_cache=d["k_scale_cache"], v_scale_cache=d["v_scale_cache"], rotate=False)
    step()
    torch.cuda.synchronize()
    reps = 5
    stream = torch.cuda.current_stream(dev)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(reps):
        step()
    b.record(stream)
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / reps
    chunk = w.q.shape[0]
    n = int(w.seqused_k[0])
    cached = n - chunk
    flops = 4.0 * w.head_size * w.num_q_heads * (chunk * cached + chunk * (chunk + 1) / 2)
    return dict(ms=ms, tok_s=chunk / (ms * 1e-3), tflops=flops / (ms * 1e-3) / 1e12, flops=flops)


def copy_probe(torch, mib):
    """A plain device-to-device copy of known size, the calibration kernel for the HBM byte counters."""
    n = mib << 20
    src = torch.ones(n, dtype=torch.uint8, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"copied {n} bytes 10 times")


def counted_traffic():
    """HBM bytes per decode launch from the committed counter summary, or None."""
    path = os.path.join(HERE, "profiles", "decode_span_kernel_decode-int4-128k-t2_traffic.txt")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch"):
            return int(line.split("=")[1].split()[0])
    return None


def cpu_prefill_baseline(sample_tokens=None):
    """The same dequantise-then-attend restatement on the prefill chunk workload, one rep: the whole 1024-token chunk
    (each token attending to the 131072 cached keys and the chunk's tokens before it; about 10-15 s on 16 host
    cores), or its first `sample_tokens` query tokens when given, reported as tokens per second."""
    import torch

    from oracle import qp_oracle as O
    from vllm_quantpack.tools import synth
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    w = synth.make("prefill-int4-128k-c1024")
    views = O.int4_views(w.kv, w.head_size)
    # the chunk's own keys: the oracle store writes them as the workload's setup does on the device
    O.store(views, O.bf16_bits_to_f32(w.new_key), O.bf16_bits_to_f32(w.new_value), w.new_slots)
    n = int(w.seqused_k[0])
    chunk = w.q.shape[0]
    tokens = chunk if not sample_tokens else min(sample_tokens, chunk)
    q = O.bf16_bits_to_f32(w.q[:tokens])
    t = time.perf_counter()
    O.prefill_dequant_attend(q, views, w.block_table[0], n - chunk + tokens, w.softmax_scale)
    dt = time.perf_counter() - t
    what = "the whole 1024-token chunk" if tokens == chunk else f"the first {tokens} query tokens"
    return dict(value=round(tokens / dt, 2), unit="tok/s", cores=threads, kind="port",
                sample=f"{what} of prefill-int4-128k-c1024 ({n - chunk} cached keys, causal in the chunk), 1 rep, "
                       f"{dt:.2f} s, torch {torch.__version__} CPU")


def cpu_baseline(w, budget_s=20.0):
    """The oracle's dequantise-then-attend restatement of the reference's path, on this host's cores."""
    import numpy as np
    import torch

    from oracle import qp_oracle as O
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    views = O.int4_views(w.kv, w.head_size)
    q = O.bf16_bits_to_f32(w.q)
    n = int(w.seqused_k[0])
    times = []
    t_start = time.perf_counter()
    while len(times) < 3 and (not times or time.perf_counter() - t_start + times[-1] < budget_s):
        t = time.perf_counter()
        O.prefill_dequant_attend(q, views, w.block_table[0], n, w.softmax_scale)
        times.append(time.perf_counter() - t)
    med = float(np.median(times))
    return dict(value=round(q.shape[0] / med, 3), unit="tok/s", cores=threads, kind="port",
                sample=f"full decode-int4-128k-t2 step ({q.shape[0]} query tokens over {n} keys), median of "
                       f"{len(times)} reps, {med:.2f} s each, torch {torch.__version__} CPU")


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--segments", type=int, default=0, help="split-KV segments (default: sized for the CU count)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-prefill", action="store_true", help="skip the prefill-chunk workload")
    ap.add_argument("--no-dropin", action="store_true", help="skip the unified_attention_int4 (drop-in path) timing")
    ap.add_argument("--cache-copies", type=int, default=4,
                    help="copies of the decode cache used in turn (1: the cache stays in the last-level cache)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB", help="only run a plain copy of MIB MiB")
    args = ap.parse_args(argv)
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one MI355X: the int4 KV attention path runs on one GPU here (across GPUs it would "
              "shard by KV head with no exchange). Run with --gpus 1.", file=sys.stderr)
        return 2
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    if args.copy_probe:
        copy_probe(torch, args.copy_probe)
        return 0
    log(f"device {torch.cuda.get_device_name(0)}, {torch.cuda.get_device_properties(0).multi_processor_count} CUs")
    r = decode_bench(torch, args)
    step_s = r["step_ms"] * 1e-3
    kern_s = r["decode_kernel_us"] * 1e-6
    log(f"decode: {r['step_ms'] * 1e3:.1f} us/step, decode kernel {r['decode_kernel_us']:.1f} us "
        f"({r['bytes'] / kern_s / 1e9:.0f} GB/s), decode + merge queued {r['pair_us']:.1f} us")
    line = {
        "metric": METRIC,
        "value": round(r["tokens_per_step"] / step_s, 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["step_ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "decode-int4-128k-t2", "context": 131072, "query_tokens": 2, "q_heads": 24,
                   "kv_heads": 4, "head_size": 256, "block_size": 16, "kv_format": "int4_per_token_head",
                   "segments": r["segments"], "cache_copies": args.cache_copies, "parallelism": "single-gpu"},
        "us_per_layer": round(r["step_ms"] * 1e3, 2),
        "hbm_gbps_step": round(r["bytes"] / step_s / 1e9, 1),
        "hbm_gbps_decode_kernel": round(r["bytes"] / kern_s / 1e9, 1),
        "roofline": {"bound": "hbm", "achieved": round(r["bytes"] / kern_s / 1e9, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(r["bytes"] / kern_s / 1e9 / HBM_PEAK_GBS, 4),
                     "traffic": counted_traffic(), "traffic_source": "FETCH_SIZE + WRITE_SIZE counters of the "
                     "committed summary profiles/decode_span_kernel_decode-int4-128k-t2_traffic.txt (not this run)",
                     "kernel": DECODE_KERNEL,
                     "bytes_per_launch": r["bytes"], "avg_us": round(r["decode_kernel_us"], 2)},
        "decode_plus_merge_queued_us": round(r["pair_us"], 2),
    }
    if not args.no_prefill:
        try:
            p = prefill_bench(torch, args)
            line["prefill"] = {"workload": "prefill-int4-128k-c1024", "tok_s": round(p["tok_s"], 1),
                               "ms": round(p["ms"], 3), "tflops": round(p["tflops"], 1),
                               "mfma_frac": round(p["tflops"] / BF16_PEAK_TFLOPS, 4)}
        except NotImplementedError as e:
            line["prefill"] = {"workload": "prefill-int4-128k-c1024", "tok_s": None, "note": str(e)}
    if not args.no_dropin:
        dr = dropin_bench(torch, args, r)
        line["dropin"] = {"what": "unified_attention_int4 per layer on unrotated queries (rotation fused)",
                          "eager_us_per_layer": round(dr["eager_us"], 2), "graph_us_per_layer": round(dr["graph_us"], 2)}
        log(f"drop-in layer: {dr['eager_us']:.1f} us eager, {dr['graph_us']:.1f} us graph replay")
    if not args.no_cpu:
        log("CPU baseline ...")
        line["cpu_baseline"] = cpu_baseline(r["w"])
        if not args.no_prefill:
            line["cpu_baseline_prefill"] = cpu_prefill_baseline()
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
