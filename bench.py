#!/usr/bin/env python3
"""RPA benchmark on one MI355X.

Default workload: BASELINE config 2, the Llama-3-8B-shape decode batch
(64 sequences x 1 query token, 32 q / 8 kv heads, head_dim 128, page_size 16,
bf16 KV, kv_lens ~ U[512, 4096], 20k-page shuffled pool).  One "step" is one
full ragged_paged_attention call (cache write + attention) over that batch with
every input already resident in HBM.

Prints one JSON line:
  value      -- query tokens per second of whole calls: K calls back to back,
                timed both as eager launches and as HIP-graph replays of one
                call; the faster is `value` ("timing" names it, both are
                reported)
  roofline   -- the dominant kernel (the decode kernel when the batch has
                decode rows, else the whole attention call): its algorithmic
                HBM bytes per launch divided by its average launch duration
                (HIP events on the launching stream around graph replays of
                that kernel alone), against MI355X's 8 TB/s; `traffic` is the
                measured HBM bytes per launch from the committed rocprofv3
                FETCH_SIZE / WRITE_SIZE profile of this workload, scaled by the
                copy-kernel calibration stored with it (null without one)
  cpu_baseline -- the CPU oracle (faithful restatement of the reference
                ref_ragged_paged_attention) on the host cores, same workload

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 2]
       python bench.py --copy-probe BYTES   (calibration kernel for rocprofv3 --pmc)
"""

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0
BF16_PEAK_TFLOPS = 2500.0

WORKLOAD_TEXT = {
    1: "C1 CPU-reference decode: 4 seqs x 1 token, 8q/2kv, D128, ps16, bf16, kv~U[64,512]",
    2: "C2 Llama-3-8B-shape decode batch: 64 seqs x 1 token, 32q/8kv, D128, ps16, bf16 KV, "
       "kv_lens~U[512,4096], 20k-page pool",
    3: "C3 mixed: 8x512-token prefill chunks (ctx~U[0,4096]) + 120 decodes (kv~U[1024,8192]), "
       "64q/8kv, D128, ps32, bf16",
    4: "C4 long-context fp8: 16 decodes kv~U[16384,32768], 32q/8kv, D128, ps64, fp8-e4m3 KV",
    5: "C5 Gemma-style: 16 decodes + 16x256 chunks, 16q/8kv, D256, ps16, window 4096, cap 50",
}


def _log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_baseline(w, seconds, call_bytes):
    """Time the CPU oracle (faithful mode, a restatement of the reference's
    ref_ragged_paged_attention) on the same workload: whole calls, the median
    of up to 5 within `seconds` (at least one).  Reports query tokens/s and
    the algorithmic GB/s of those calls."""
    import torch

    from oracle import rpa_oracle as O

    # The cores this process may use (the box's share, OMP_NUM_THREADS when
    # set), not the whole machine's count.
    threads = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else 1
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        threads = min(threads, int(os.environ["OMP_NUM_THREADS"]))
    torch.set_num_threads(max(threads, 1))
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    times = []
    t_start = time.perf_counter()
    while len(times) < 5 and (time.perf_counter() - t_start < seconds or len(times) < 1):
        t0 = time.perf_counter()
        O.ref_ragged_paged_attention(*w.args(), mode="faithful", validate=False, **w.kwargs)
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    return {
        "value": w.num_tokens / med,
        "unit": "tokens/s",
        "gbps": round(call_bytes / med / 1e9, 3),
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"full workload ({w.num_seqs} seqs, {w.num_tokens} query tokens) per call; "
                   f"median of {len(times)} calls; {med * 1e3:.1f} ms/call; "
                   f"oracle faithful mode (torch CPU) on {model}"),
    }


def copy_probe(nbytes, reps):
    """A plain device copy of `nbytes` (src -> dst), `reps` times: the
    reference kernel whose FETCH_SIZE / WRITE_SIZE per dispatch calibrates the
    counters (it moves exactly nbytes in and nbytes out)."""
    import torch

    dev = torch.device("cuda:0")
    n = nbytes // 16
    src = torch.ones(n, 4, dtype=torch.int32, device=dev)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    print(json.dumps({"copy_probe_bytes": n * 16, "reps": reps, "ms": round(ms, 5),
                      "gbps_read_plus_write": round(2 * n * 16 / (ms * 1e-3) / 1e9, 1)}),
          flush=True)


def load_traffic(config, kernel):
    """HBM bytes per launch of `kernel` on config `config` from the committed
    counter profile (profiles/pmc_<kernel>_c<config>.json), or None."""
    path = os.path.join(ROOT, "profiles", f"pmc_{kernel}_c{config}.json")
    if not os.path.exists(path):
        return None
    try:
        with open(path) as f:
            d = json.load(f)
        return int(d["traffic_bytes_per_launch"])
    except (OSError, ValueError, KeyError):
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # 500 whole calls (about 66 ms at C2, 0.4 s at C3): the fixed cost of the
    # first launch and of the closing synchronize is spread over the calls a
    # serving loop runs back to back, not charged to 50 of them.
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", type=int, default=2, choices=[1, 2, 3, 4, 5])
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="BYTES")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}, WORLD_SIZE={world}): "
              "RPA shards by KV heads / sequences with no exchange inside attention, so a "
              "single MI355X's throughput is the measured figure; multi-GPU runs are not part "
              "of this build.", file=sys.stderr)
        sys.exit(2)
    if args.copy_probe:
        copy_probe(args.copy_probe, max(args.steps, 1))
        return

    import torch

    import vllm_torchtpu_amd as R
    import vllm_torchtpu_amd.workloads as W
    from vllm_torchtpu_amd import _native as N

    dev = torch.device("cuda:0")
    _log(f"building workload C{args.config}")
    w = W.baseline_config(args.config)
    g = w.to(dev)
    kw = dict(w.kwargs)
    torch.cuda.synchronize()

    def step():
        return R.ragged_paged_attention(*g.args(), **kw)

    def attn_only():
        return R.ragged_paged_attention(*g.args(), skip_kv_update=True, **kw)

    k_out = torch.empty(g.q.shape, dtype=g.q.dtype, device=dev)

    def decode_only():
        return R.rpa._rpa_forward_impl(
            *g.args(), k_out, use_causal_mask=kw.get("use_causal_mask", True),
            skip_kv_update=True, sm_scale=kw["sm_scale"],
            sliding_window=kw.get("sliding_window"), soft_cap=kw.get("soft_cap"),
            q_scale=kw.get("q_scale"), k_scale=kw.get("k_scale"), v_scale=kw.get("v_scale"),
            path=N.RPA_PATH_DECODE_ONLY)

    has_decode = True
    try:
        decode_only()
    except (NotImplementedError, ValueError, RuntimeError) as e:
        _log(f"decode kernel does not apply ({e}); timing the whole attention call")
        has_decode = False

    _log("warm-up")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # Eager: K whole calls back to back.
    _log(f"timing {args.steps} eager steps")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    eager_s = time.perf_counter() - t0

    def replay_ms(graph):
        # HIP events on the current stream, which the replays launch on.
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(args.steps):
            graph.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / args.steps

    graph_s = attn_ms = kern_ms = median_step_ms = None
    if not args.no_graph:
        _log("capturing HIP graphs")
        fns = [step, attn_only] + ([decode_only] if has_decode else [])
        s = torch.cuda.Stream(dev)
        s.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(s):
            for _ in range(2):
                for fn in fns:
                    fn()
        torch.cuda.current_stream(dev).wait_stream(s)
        torch.cuda.synchronize()
        graphs = []
        for fn in fns:
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr):
                fn()
            graphs.append(gr)
        for _ in range(3):
            for gr in graphs:
                gr.replay()
        torch.cuda.synchronize()
        _log(f"timing {args.steps} graph steps")
        t0 = time.perf_counter()
        for _ in range(args.steps):
            graphs[0].replay()
        torch.cuda.synchronize()
        graph_s = time.perf_counter() - t0
        # Per-step times of graph replays (HIP events around each one).
        per = []
        for _ in range(args.steps):
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record()
            graphs[0].replay()
            e1.record()
            per.append((e0, e1))
        torch.cuda.synchronize()
        median_step_ms = statistics.median(a.elapsed_time(b) for a, b in per)
        attn_ms = replay_ms(graphs[1])
        kern_ms = replay_ms(graphs[2]) if has_decode else attn_ms

    # Both timings cover K whole calls back to back with every input resident
    # in HBM; the faster one is the job's throughput (graph replays pay a
    # per-replay launch gap that back-to-back eager calls can hide).
    timed_s, timing = eager_s, "eager"
    if graph_s is not None and graph_s < eager_s:
        timed_s, timing = graph_s, "graph"
    tokens = w.num_tokens
    value = tokens * args.steps / timed_s
    ms_per_step = timed_s / args.steps * 1e3

    kvl = w.kv_lens.tolist()
    cu = w.cu_q_lens.tolist()
    n = w.num_seqs
    hq, hkv, d = w.q.shape[1], w.k.shape[1], w.q.shape[2]
    dp = w.kv_cache.shape[4]
    ps = w.kv_cache.shape[1]
    kvb = w.kv_cache.element_size()
    qb = w.q.element_size()
    win = kw.get("sliding_window")
    call_bytes = W.algorithmic_bytes(kvl, cu, n, hq, hkv, d, dp, ps, qb, kvb, qb,
                                     sliding_window=win)
    attn_bytes = W.algorithmic_bytes(kvl, cu, n, hq, hkv, d, dp, ps, qb, kvb, qb,
                                     sliding_window=win, kv_write=False)
    dec_bytes = W.decode_kernel_bytes(kvl, cu, n, hq, hkv, d, dp, ps, qb, kvb,
                                      sliding_window=win)
    flops = W.prefill_flops(kvl, cu, n, hq, d, sliding_window=win)

    roofline = None
    if kern_ms is not None:
        kernel = "decode_kernel" if has_decode else "attention_call"
        kbytes = dec_bytes if has_decode else attn_bytes
        achieved = kbytes / (kern_ms * 1e-3) / 1e9
        roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                    "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                    "traffic": load_traffic(args.config, kernel), "kernel": kernel,
                    "kernel_ms": round(kern_ms, 5), "bytes_per_launch": kbytes,
                    "attention_call_ms": round(attn_ms, 5),
                    "attention_call_bytes": attn_bytes}

    # MFMA roofline of the prefill rows: the prefill kernel's share of the
    # batch (the sequences with more than one query token) timed alone as
    # graph replays, and its share of the whole attention call (the call
    # minus the decode kernel alone).
    roofline_mfma = None
    if flops > 0 and not args.no_graph:
        pw = W.prefill_part(w)
        pg = pw.to(dev)
        pkw = dict(pw.kwargs)

        def prefill_only():
            return R.ragged_paged_attention(*pg.args(), skip_kv_update=True, **pkw)

        s2 = torch.cuda.Stream(dev)
        s2.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(s2):
            for _ in range(3):
                prefill_only()
        torch.cuda.current_stream(dev).wait_stream(s2)
        torch.cuda.synchronize()
        pgr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(pgr):
            prefill_only()
        for _ in range(3):
            pgr.replay()
        torch.cuda.synchronize()
        alone_ms = replay_ms(pgr)
        in_call_ms = attn_ms - kern_ms if has_decode else attn_ms
        achieved = flops / (alone_ms * 1e-3) / 1e12
        roofline_mfma = {
            "bound": "mfma", "achieved": round(achieved, 1), "peak": BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s", "frac": round(achieved / BF16_PEAK_TFLOPS, 4),
            "traffic": None, "kernel": "prefill_kernel",
            "flops_per_launch": flops, "alone_ms": round(alone_ms, 5),
            "in_call_ms": round(in_call_ms, 5),
            "in_call_frac": round(flops / (in_call_ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
            "note": ("alone: the batch's multi-token sequences by themselves (distribution "
                     "[0, 0, n]); in_call: attention call minus the decode kernel alone"),
        }

    cpu = None
    if not args.no_cpu_baseline:
        _log("timing CPU oracle baseline")
        cpu = cpu_baseline(w, args.cpu_seconds, call_bytes)

    line = {
        "metric": "RPA tokens/s + achieved HBM GB/s (% of 8 TB/s), Llama-3-8B-shape decode batch",
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if kvb == 2 else ("fp8-e4m3 KV / bf16 q" if kvb == 1 else "f32"),
        "data": "synthetic (seeded N(0,1) Q/K/V, shuffled page pool)",
        "config": {"workload": WORKLOAD_TEXT[args.config], "num_seqs": n,
                   "query_tokens": tokens, "kv_tokens": int(sum(kvl[:n])),
                   "parallelism": "single GPU"},
        "call_bytes": call_bytes,
        "call_gbps": round(call_bytes / (ms_per_step * 1e-3) / 1e9, 1),
        "timing": timing,
        "eager_ms_per_step": round(eager_s / args.steps * 1e3, 5),
        "graph_ms_per_step": None if graph_s is None else round(graph_s / args.steps * 1e3, 5),
        "median_graph_step_ms": None if median_step_ms is None else round(median_step_ms, 5),
        "prefill_flops": flops,
        "roofline": roofline,
        "roofline_mfma": roofline_mfma,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
