"""Decode-step benchmark: KV append + GQA decode attention, Qwen3-VL-2B text-decoder shapes, one MI355X.

Default workload (the headline configuration): batch 8, 16 query / 8 kv heads, head_dim 128, bf16,
28 layers, each sequence prefilled with 2048 tokens (N(0,1), K scaled by 0.5), then decode steps that each
run, for every layer, one KV append (1 token per sequence) and one decode attention over the whole cache.
A step is therefore 28 x {append, attend}; --steps K times exactly K steps (K=128 is one full 128-token
generation), after --warmup W untimed steps. Cache lengths are reset to 2048 between warmup and timing.
The default path runs each layer's append + attend as one launch (aicas_decode_attention_append); the
two-launch path (aicas_kv_append, then aicas_decode_attention) is timed beside it and reported.

Each decode step is captured once as a HIP graph (torch.cuda.CUDAGraph) over per-(step, layer) input and
output buffers, as a serving loop replays one graph per generated token; the timed region is K back-to-back
replays bracketed by torch.cuda.synchronize() and HIP events. --mode eager times the same work issued from
Python without graphs (host-bound).

Printed JSON line: value = microseconds per decode step (lower is better), plus tokens/s, algorithmic HBM
bytes per step and GB/s, the decode kernel's roofline (average duration of the decode kernel from HIP events
bracketing each launch on its stream, algorithmic bytes per launch / that duration), and a CPU baseline: the
oracle (torch.cat append + SDPA over repeat_kv, bf16 eager on the host cores) on the first steps of the same
inputs.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0


def parse_args(argv=None):
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=128)
    p.add_argument("--warmup", type=int, default=16)
    p.add_argument("--mode", choices=("graph", "eager"), default="graph")
    p.add_argument("--path", choices=("fused", "separate"), default="fused",
                   help="fused: one launch per layer appends and attends; separate: append kernel + decode kernel")
    p.add_argument("--compare-paths", type=int, default=1, help="also time the other path (reported, not the value)")
    p.add_argument("--tokens-per-split", type=int, default=0, help="0 = the library's plan")
    p.add_argument("--cpu-baseline-seconds", type=float, default=15.0,
                   help="approximate CPU time budget for the oracle baseline (0 disables it)")
    p.add_argument("--kernel-timing-steps", type=int, default=8,
                   help="steps whose decode launches are bracketed by HIP events for the roofline")
    p.add_argument("--copy-calibration-mib", type=int, default=0,
                   help="also run a plain device copy of this many MiB (reference for profiler byte counters)")
    p.add_argument("--check-steps", type=int, default=2,
                   help="steps whose outputs are compared with the CPU oracle after timing")
    return p.parse_args(argv)


def algorithmic_bytes(batch, hq, hkv, d, lens_after, elem=2):
    """Bytes one layer-step must move: K and V read over each sequence's cache (length after the append),
    new K/V rows read and written, q read and the output written."""
    kv_read = sum(2 * L * hkv * d * elem for L in lens_after)
    new_rows = 2 * batch * hkv * d * 2 + 2 * batch * hkv * d * elem
    q_out = 2 * batch * hq * d * 2
    return kv_read + new_rows + q_out


def decode_kernel_bytes(batch, hq, hkv, d, lens_after, elem=2):
    """Bytes of the decode launch alone: K/V over the cache, q in, out out."""
    return sum(2 * L * hkv * d * elem for L in lens_after) + 2 * batch * hq * d * 2


def cpu_info():
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return model


def main(argv=None) -> int:
    args = parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (this path does not shard "
              "across GPUs here; see DESIGN.md for how it would).", file=sys.stderr)
        return 2

    import torch

    from aicas_amd import ops
    from aicas_amd.workloads import HEAD_DIM, HKV, HQ, SM_SCALE, WORKLOADS, generator, normal

    w = WORKLOADS["c2"]
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    B, D, L0, NL = w.batch, HEAD_DIM, w.prefill, w.layers
    K, W = args.steps, args.warmup
    n_graph_steps = max(K, W)
    cap = L0 + n_graph_steps
    cap = (cap + 63) // 64 * 64

    # ---- inputs, resident in HBM before anything is timed
    g = generator(dev, w.seed)
    kbuf, vbuf = [], []
    for _ in range(NL):
        kb = torch.empty((B, HKV, cap, D), dtype=torch.bfloat16, device=dev)
        vb = torch.empty_like(kb)
        kb[:, :, :L0] = normal((B, HKV, L0, D), g, dev, scale=w.k_scale)
        vb[:, :, :L0] = normal((B, HKV, L0, D), g, dev)
        kb[:, :, L0:].zero_()
        vb[:, :, L0:].zero_()
        kbuf.append(kb)
        vbuf.append(vb)
    q_all = normal((n_graph_steps, NL, B, HQ, 1, D), g, dev)
    kn_all = normal((n_graph_steps, NL, B, HKV, 1, D), g, dev, scale=w.k_scale)
    vn_all = normal((n_graph_steps, NL, B, HKV, 1, D), g, dev)
    out_all = torch.zeros((n_graph_steps, NL, B, HQ, 1, D), dtype=torch.bfloat16, device=dev)
    # fused path: one length tensor for the whole step (tokens cached before it), bumped by the last layer's
    # kernel, as a serving loop keeps it; separate path: each layer's append bumps that layer's lengths
    shared_lens = torch.full((B,), L0, dtype=torch.int32, device=dev)
    lens = [torch.full((B,), L0, dtype=torch.int32, device=dev) for _ in range(NL)]
    lens0 = torch.full((B,), L0, dtype=torch.int32, device=dev)
    views = [ops.KVCacheView(kbuf[i], vbuf[i]) for i in range(NL)]
    # one split size for the whole run, planned at the longest step (the plan's workspace covers every step)
    plan = ops.decode_plan(torch.bfloat16, B, HQ, HKV, D, L0 + n_graph_steps, 0, args.tokens_per_split)
    ws = ops.Workspace.reserve(dev, plan.workspace_bytes)

    def step(s, path, kernel_events=None):
        """One decode step: for every layer append this step's K/V row and attend (L0 + s tokens cached)."""
        for i in range(NL):
            if path == "fused":
                if kernel_events is not None:
                    kernel_events[i][0].record()
                ops.decode_attention_append(
                    q_all[s, i], views[i], kn_all[s, i], vn_all[s, i], shared_lens, sm_scale=SM_SCALE,
                    max_seq_len=L0 + s + 1, min_seq_len=L0 + s,
                    seq_lens_out=shared_lens if i == NL - 1 else None, out=out_all[s, i],
                    tokens_per_split=plan.tokens_per_split, workspace=ws,
                )
                if kernel_events is not None:
                    kernel_events[i][1].record()
            else:
                ops.kv_append(views[i], kn_all[s, i], vn_all[s, i], lens[i], lens[i])
                if kernel_events is not None:
                    kernel_events[i][0].record()
                ops.decode_attention(
                    q_all[s, i], views[i], sm_scale=SM_SCALE, seq_lens=lens[i], max_seq_len=L0 + s + 1,
                    min_seq_len=L0 + s + 1, out=out_all[s, i], tokens_per_split=plan.tokens_per_split, workspace=ws,
                )
                if kernel_events is not None:
                    kernel_events[i][1].record()

    def reset_lens():
        shared_lens.copy_(lens0)
        for t in lens:
            t.copy_(lens0)

    stream = torch.cuda.Stream(device=dev)

    def capture(path):
        graphs = []
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            step(0, path)  # first launch of every kernel outside capture
            torch.cuda.synchronize()
            reset_lens()
            torch.cuda.synchronize()
            for s in range(n_graph_steps):
                gr = torch.cuda.CUDAGraph()
                with torch.cuda.graph(gr, stream=stream):
                    step(s, path)
                graphs.append(gr)
            torch.cuda.synchronize()
        return graphs

    def run_steps(path, graphs, first, count):
        if graphs is not None:
            for s in range(first, first + count):
                graphs[s].replay()
        else:
            for s in range(first, first + count):
                step(s, path)

    def timed(path, graphs):
        with torch.cuda.stream(stream):
            reset_lens()
            run_steps(path, graphs, 0, W)
            torch.cuda.synchronize()
            reset_lens()
            torch.cuda.synchronize()
            ev0 = torch.cuda.Event(enable_timing=True)
            ev1 = torch.cuda.Event(enable_timing=True)
            t0 = time.perf_counter()
            ev0.record()
            run_steps(path, graphs, 0, K)
            ev1.record()
            torch.cuda.synchronize()
            t1 = time.perf_counter()
        return ev0.elapsed_time(ev1), (t1 - t0) * 1e3

    path = args.path
    other = "separate" if path == "fused" else "fused"
    graphs = capture(path) if args.mode == "graph" else None
    gpu_ms, wall_ms = timed(path, graphs)
    us_per_step = gpu_ms * 1e3 / K
    other_us = None
    if args.compare_paths:
        graphs_other = capture(other) if args.mode == "graph" else None
        other_us = timed(other, graphs_other)[0] * 1e3 / K
        del graphs_other

    lens_per_step = [[L0 + s + 1] * B for s in range(K)]
    bytes_steps = [NL * algorithmic_bytes(B, HQ, HKV, D, la) for la in lens_per_step]
    bytes_per_step = sum(bytes_steps) / K
    gbps = bytes_per_step / (us_per_step * 1e-6) / 1e9

    # ---- the dominant kernel's average duration. On the fused path every launch of the timed region is that
    # kernel (NL per step, back to back in the replayed graphs), so the HIP-event time of the timed region over
    # the number of launches is its average launch duration (launch gaps included). The separate path's
    # decode launches are bracketed by events instead (queued behind a GPU sleep, so the host is ahead).
    kt_steps = min(args.kernel_timing_steps, K)
    durations = []
    if kt_steps > 0:
        with torch.cuda.stream(stream):
            reset_lens()
            torch.cuda.synchronize()
            evs = [[[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(NL)]
                   for _ in range(kt_steps)]
            torch.cuda._sleep(int(1.0e8))
            for s in range(kt_steps):
                step(s, path, kernel_events=evs[s])
            torch.cuda.synchronize()
            for s in range(kt_steps):
                for i in range(NL):
                    durations.append(evs[s][i][0].elapsed_time(evs[s][i][1]) * 1e3)  # us
    if path == "fused":
        dec_us = us_per_step / NL
        dec_bytes = bytes_per_step / NL  # the fused kernel moves every algorithmic byte of the layer-step
        dec_launches = K * NL
    else:
        dec_us = sum(durations) / len(durations)
        dec_bytes = sum(decode_kernel_bytes(B, HQ, HKV, D, lens_per_step[s]) for s in range(kt_steps)) / kt_steps
        dec_launches = len(durations)
    dec_gbps = dec_bytes / (dec_us * 1e-6) / 1e9

    # ---- a plain device copy of known size, for scaling the FETCH_SIZE / WRITE_SIZE counters of a profile run
    if args.copy_calibration_mib > 0:
        n = args.copy_calibration_mib << 20
        src = torch.empty(n, dtype=torch.uint8, device=dev).random_(0, 255)
        dst = torch.empty_like(src)
        for _ in range(4):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    # ---- parity of the timed run's first steps against the oracle (outputs of the timed replay)
    from oracle import reference_path as ref

    max_err = 0.0
    check_steps = min(args.check_steps, K)
    if check_steps > 0:
        with torch.cuda.stream(stream):
            reset_lens()
            torch.cuda.synchronize()
            run_steps(path, graphs, 0, check_steps)
            torch.cuda.synchronize()
        for i in range(NL):
            kc = kbuf[i][:, :, :L0].cpu()
            vc = vbuf[i][:, :, :L0].cpu()
            for s in range(check_steps):
                kc, vc = ref.dynamic_layer_update(kc, vc, kn_all[s, i].cpu(), vn_all[s, i].cpu())
                expect = ref.sdpa_decode(q_all[s, i].cpu(), kc, vc, SM_SCALE, HQ // HKV).float()
                err = (out_all[s, i].float().cpu() - expect).abs().max().item()
                max_err = max(max_err, err)
            # the appended rows are bit-identical to the torch.cat cache
            assert torch.equal(kbuf[i][:, :, : L0 + check_steps].cpu().view(torch.int16), kc.view(torch.int16))

    # ---- CPU baseline: the oracle (reference PyTorch path) on the host cores, same inputs, first steps
    cpu = None
    if args.cpu_baseline_seconds > 0:
        threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or min(16, os.cpu_count() or 1)
        torch.set_num_threads(threads)
        kc = [kbuf[i][:, :, :L0].cpu() for i in range(NL)]
        vc = [vbuf[i][:, :, :L0].cpu() for i in range(NL)]
        inputs = [(q_all[s].cpu(), kn_all[s].cpu(), vn_all[s].cpu()) for s in range(min(K, 64))]
        step_times = []
        budget_t0 = time.perf_counter()
        for s in range(len(inputs)):
            qs, kns, vns = inputs[s]
            t_s = time.perf_counter()
            for i in range(NL):
                kc[i], vc[i] = ref.dynamic_layer_update(kc[i], vc[i], kns[i], vns[i])
                ref.sdpa_decode(qs[i], kc[i], vc[i], SM_SCALE, HQ // HKV)
            step_times.append(time.perf_counter() - t_s)
            if time.perf_counter() - budget_t0 > args.cpu_baseline_seconds and len(step_times) >= 2:
                break
        cpu_us = sum(step_times[1:]) / max(1, len(step_times) - 1) * 1e6 if len(step_times) > 1 else step_times[0] * 1e6
        cpu = {
            "value": round(cpu_us, 1),
            "unit": "us/step",
            "cores": threads,
            "kind": "port",
            "sample": f"first {len(step_times)} of the {K} decode steps (28 layers each: torch.cat append + "
                      f"SDPA over repeat_kv, bf16, torch {torch.__version__} eager), mean of steps 2..{len(step_times)}",
            "cpu_model": cpu_info(),
            "cpu_capability": torch.backends.cpu.get_cpu_capability(),
            "tokens_per_s": round(B / (cpu_us * 1e-6), 1),
        }

    # HBM traffic per launch of the fused kernel, from the copy-calibrated FETCH_SIZE / WRITE_SIZE profile runs
    traffic = None
    traffic_file = os.path.join(ROOT, "profiles", "decode_append_c2_hbm_traffic.json")
    if path == "fused" and os.path.exists(traffic_file):
        with open(traffic_file) as f:
            traffic = json.load(f)

    result = {
        "metric": "us/decode-step & achieved HBM GB/s (% of 8 TB/s), B=8 L=2048 28 layers",
        "value": round(us_per_step, 2),
        "unit": "us/step",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(us_per_step / 1e3, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1), K x0.5)",
        "config": {
            "workload": "qwen3vl-2b decode: B=8, 16q/8kv heads, head_dim 128, bf16, 28 layers, prefill 2048, "
                        "128 steps of append 1 + attend",
            "batch": B, "layers": NL, "prefill": L0, "q_heads": HQ, "kv_heads": HKV, "head_dim": D,
            "mode": args.mode, "path": path, "tokens_per_split": plan.tokens_per_split,
            "num_splits": plan.num_splits,
        },
        "tokens_per_s": round(B / (us_per_step * 1e-6), 1),
        "hbm_bytes_per_step": int(bytes_per_step),
        "hbm_gbps": round(gbps, 1),
        "hbm_frac": round(gbps / HBM_PEAK_GBPS, 4),
        "wall_ms": round(wall_ms, 3),
        f"{other}_path_us_per_step": None if other_us is None else round(other_us, 2),
        "roofline": {
            "bound": "hbm",
            "kernel": "decode_attn_kernel<bf16,bf16,D=128,G=2,contiguous,"
                      + ("append>" if path == "fused" else "no-append>"),
            "achieved": round(dec_gbps, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(dec_gbps / HBM_PEAK_GBPS, 4),
            "traffic": None if traffic is None else traffic["traffic_bytes_per_launch"],
            "traffic_note": None if traffic is None else (
                f"rocprofv3 FETCH_SIZE x{traffic['fetch_scale']} + WRITE_SIZE x{traffic['write_scale']} "
                f"(scales from a 256 MiB copy), {traffic['profiled_lengths']}; "
                f"{traffic['traffic_over_algorithmic']} of the algorithmic bytes at those lengths "
                "(profiles/decode_append_c2_hbm_traffic.md)"),
            "avg_launch_us": round(dec_us, 3),
            "avg_launch_us_event_bracketed": round(sum(durations) / len(durations), 3) if durations else None,
            "bytes_per_launch": int(dec_bytes),
            "launches_timed": dec_launches,
        },
        "cpu_baseline": cpu,
        "parity_max_abs_err": max_err,
    }
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
