"""Time the chunked-prefill kernel on a named synthetic prefill workload (one MI355X).

    PYTHONPATH=vllm-quantpack_amd python -m vllm_quantpack.tools.time_prefill [--workload prefill-int4-128k-c1024] \
        [--reps 5] [--splits N] [--i8]

--i8 times the reference's single-kernel alternative arithmetic (qp_prefill_i8) instead of the exact one.

The workload's chunk keys are stored into the cache first (as the benchmark does), then `reps` prefill calls run back
to back between one event pair. Prints one JSON line with the average call time, the attention FLOPs of the chunk
(4 x head size x query heads x visible (query, key) pairs) and the fraction of the 2.5 PFLOP/s dense bf16 MFMA peak.
Run it under `rocprofv3 --kernel-trace --stats` or `--pmc ...` for the per-kernel figures.
"""
import argparse
import json
import sys

BF16_PEAK_TFLOPS = 2500.0


def chunk_flops(w) -> float:
    """4 x hs x NQ x visible pairs: every query token of the chunk sees the cached keys and the chunk up to itself."""
    n = int(w.seqused_k[0])
    chunk = w.q.shape[0]
    cached = n - chunk
    return 4.0 * w.head_size * w.num_q_heads * (chunk * cached + chunk * (chunk + 1) / 2)


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--workload", default="prefill-int4-128k-c1024")
    ap.add_argument("--reps", type=int, default=5)
    ap.add_argument("--splits", type=int, default=0, help="key splits per query block (0: the library's choice)")
    ap.add_argument("--i8", action="store_true",
                    help="the reference's single-kernel alternative arithmetic (int8 query split, qp_prefill_i8)")
    args = ap.parse_args(argv)

    import torch

    from vllm_quantpack.attention import int4_prefill, k8v4_kv
    from vllm_quantpack.tools import synth
    if not args.workload.startswith("prefill-"):
        raise SystemExit(f"{args.workload}: not a prefill workload")
    dev = torch.device("cuda:0")
    w = synth.make(args.workload)
    d = synth.to_device(w, dev)
    k8v4_kv.store(None, d["new_key"], d["new_value"], d["k_cache"], d["v_cache"], d["new_slots"],
                  k_scale_cache=d["k_scale_cache"], v_scale_cache=d["v_scale_cache"], rotate=False)
    out = torch.empty_like(d["q"])

    fn = int4_prefill.prefill_attention_i8 if args.i8 else int4_prefill.prefill_attention

    def step():
        fn(d["q"], d["k_cache"], d["v_cache"], d["k_scale_cache"], d["v_scale_cache"], out,
           cu_seqlens_q=d["cu_seqlens_q"], seqused_k=d["seqused_k"], block_table=d["block_table"],
           max_seqlen_q=w.max_query_len, softmax_scale=w.softmax_scale, max_seqlen_k=int(w.seqused_k.max()),
           num_splits=args.splits)

    step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(args.reps):
        step()
    b.record(stream)
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / args.reps
    flops = chunk_flops(w)
    tflops = flops / (ms * 1e-3) / 1e12
    print(json.dumps({"workload": args.workload, "kernel": "qp_prefill_i8" if args.i8 else "qp_prefill",
                      "reps": args.reps, "ms": round(ms, 4), "flops": flops,
                      "tflops": round(tflops, 1), "mfma_frac": round(tflops / BF16_PEAK_TFLOPS, 4),
                      "tok_s": round(w.q.shape[0] / (ms * 1e-3), 1)}), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
