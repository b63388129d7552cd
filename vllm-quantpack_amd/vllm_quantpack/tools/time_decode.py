"""Time the split-KV decode kernel on one of the named synthetic workloads (one MI355X).

    PYTHONPATH=vllm-quantpack_amd python -m vllm_quantpack.tools.time_decode --workload decode-int4-256k-t4 \
        [--segments N] [--launches 200] [--copies 4]

The workload's cache is put in HBM --copies times and the launches cycle through the copies, so a launch streams its
cache from HBM rather than from the last-level cache (use more copies when one copy is small). The launches are queued
behind a spin that holds the stream and bracketed by one event pair, so the average is the kernel's execution time.
Segments default to what unified_attention_int4 picks for the batch (decode_segments). Prints one JSON line with the
average launch time and the algorithmic bytes per launch (synth.cache_bytes) over that time. Run it under
`rocprofv3 --kernel-trace --stats` for the per-kernel breakdown.
"""
import argparse
import json
import os
import sys

SPIN_CYCLES = 50_000_000


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--workload", default="decode-int4-128k-t2")
    ap.add_argument("--segments", type=int, default=0, help="split-KV segments (default: the router's choice)")
    ap.add_argument("--launches", type=int, default=200)
    ap.add_argument("--copies", type=int, default=4)
    args = ap.parse_args(argv)

    import torch

    from vllm_quantpack import _hip
    from vllm_quantpack.attention import int4_kv
    from vllm_quantpack.tools import synth
    if not args.workload.startswith("decode-"):
        raise SystemExit(f"{args.workload}: not a decode workload")
    dev = torch.device("cuda:0")
    w = synth.make(args.workload)
    copies = [synth.to_device(w, dev) for _ in range(args.copies)]
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    S = args.segments or int4_kv.decode_segments(int4_kv.segments_for(cus), len(w.seqused_k), w.num_kv_heads, cus)
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
    for i in range(10):
        plans[i % len(plans)].run()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(SPIN_CYCLES)
    a.record(stream)
    for i in range(args.launches):
        plans[i % len(plans)].decode()
    b.record(stream)
    torch.cuda.synchronize()
    us = a.elapsed_time(b) / args.launches * 1e3
    nbytes = synth.cache_bytes(w)
    gbps = nbytes / us / 1e3
    print(json.dumps({"workload": args.workload, "segments": S, "launches": args.launches,
                      "decode_kernel_us": round(us, 2), "bytes_per_launch": nbytes, "gbps": round(gbps, 1),
                      "hbm_frac": round(gbps / 8000.0, 4), "library": os.path.basename(_hip.LIB_PATH)}), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
