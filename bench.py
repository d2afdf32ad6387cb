"""Decode-step benchmark: KV append + GQA decode attention, Qwen3-VL-2B text-decoder shapes, one MI355X.

Default workload (the headline configuration, --config c2): batch 8, 16 query / 8 kv heads, head_dim 128,
bf16, 28 layers, each sequence prefilled with 2048 tokens (N(0,1), K scaled by 0.5), then decode steps that
each run, for every layer, one KV append (1 token per sequence) and one decode attention over the whole
cache. A step is therefore 28 x {append, attend}; --steps K times exactly K steps (K=128 is one full
128-token generation), after --warmup W untimed steps. Cache lengths are reset between warmup and timing.
The default path runs each layer's append + attend as one launch (aicas_decode_attention_append); the
two-launch path (aicas_kv_append, then aicas_decode_attention) is timed beside it and reported, and so is the
fused launch with the model's q/k preparation inside it (aicas_decode_attention_append_qk: q/k RMSNorm and the
rotary embedding applied to the raw projections, prepared q written out), which does more than the headline
step and is never the value.

The other seeded configurations of aicas_amd.workloads run with --config:
  c1  B=1, 1 layer, 1024 cached, one step (append at 1024, attend over 1025), repeated;
  c3  B=1, 1 layer, 32768 cached, 64 growing steps;
  c4  B=64, 28 layers, ragged lengths ~ U{512..4096}, one step, repeated;
  c5  B=32, 1 layer, ragged lengths ~ U{256..8192}, paged fp8 (16-token pages, permuted block table, 1%
      outliers), one step, repeated.
and, reported separately from the headline, --config model: a whole decode step of a Qwen3-VL-2B-shaped text
decoder (28 layers, hidden 2048, 16/8 heads, head_dim 128, MLP 6144, vocabulary 151936; random bf16 weights)
per generated token at batch 1 after a --prompt-len prefill, three ways: HF eager (DynamicCache + SDPA, the
reference's default decode), eager with every layer's attention as one fused launch (install_fused_decode +
AicasDecodeCache), and the step captured once as a HIP graph and replayed (AicasGraphDecodeRunner).
A one-layer configuration whose cache is smaller than 512 MB keeps several instances of it (>= 4, > 512 MB in
all) and steps through them in turn, so that the 256 MB MALL cannot serve the reads; its step time is the
per-layer time. One-step configurations repeat their step with the positions held, so every repeat appends
at the same position and attends over the same lengths.

The step is captured once as a HIP graph (torch.cuda.CUDAGraph) and replayed for every generated token, as a
serving loop (and AicasGraphDecodeRunner) runs it: its launches are bounded by the cache capacity and by the
prefill length (the lengths only grow from there), read the step-0 input buffers, and bump the lengths on the
device, so each replay appends one more token and attends over one more. --capture per-step instead captures
one graph per step with that step's exact bounds and inputs (timed beside it, never the value). The timed region
is K back-to-back replays bracketed by torch.cuda.synchronize() and HIP events (one event between replays gives
the per-step median and p90). --mode eager times the same work issued from Python without graphs (host-bound).

Printed JSON line: value = microseconds per decode step (lower is better), plus tokens/s, algorithmic HBM
bytes per step and GB/s, the decode kernel's roofline (algorithmic bytes per launch / average launch
duration on its stream), and a CPU baseline: the oracle (torch.cat append + SDPA over repeat_kv, bf16 eager
on the host cores; for the paged fp8 configuration, dequantise + SDPA) on a bounded sample of the same steps.
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
MALL_BYTES = 256 << 20


def parse_args(argv=None):
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--config", choices=("c1", "c2", "c3", "c4", "c5", "model", "microbench", "calib", "gather",
                                        "prefill"),
                   default="c2",
                   help="model: the whole text-decoder step per generated token; microbench: the shape of the "
                        "reference's published decode microbenchmark (both reported separately)")
    p.add_argument("--prompt-len", type=int, default=1024, help="model: cached tokens before the timed steps")
    p.add_argument("--steps", type=int, default=0, help="timed steps (0: the configuration's default)")
    p.add_argument("--warmup", type=int, default=None,
                   help="untimed warmup steps (default 16; 64 for the one-layer configurations, whose steps are "
                        "short: their time settles only after about 50 passes over the cache instances)")
    p.add_argument("--mode", choices=("graph", "eager"), default="graph")
    p.add_argument("--capture", choices=("once", "per-step"), default="once",
                   help="once: one graph per path, captured with the capacity and the prefill length as the "
                        "length bounds and replayed for every step while the lengths grow on the device (what "
                        "a serving loop and AicasGraphDecodeRunner run); per-step: one graph per step with that "
                        "step's exact bounds")
    p.add_argument("--compare-capture", type=int, default=1,
                   help="also time the other capture mode (reported, not the value)")
    p.add_argument("--path", choices=("fused", "separate"), default="fused",
                   help="fused: one launch per layer appends and attends; separate: append kernel + decode kernel")
    p.add_argument("--compare-paths", type=int, default=1, help="also time the other path (reported, not the value)")
    p.add_argument("--compare-pool", type=int, default=1,
                   help="paged configurations: also time the fused path with a device page allocation before "
                        "each launch (aicas_block_alloc; reported, not the value)")
    p.add_argument("--compare-qk", type=int, default=1,
                   help="also time the fused path with the q/k RMSNorm + rotary prologue (reported, not the value)")
    p.add_argument("--tokens-per-split", type=int, default=0, help="0 = the library's plan")
    p.add_argument("--cache-instances", type=int, default=0,
                   help="one-layer configurations: cache instances stepped through (0: enough to exceed twice the "
                        "256 MB memory-side cache, at least 4; 1 lets that cache serve the reads)")
    p.add_argument("--cpu-baseline-seconds", type=float, default=15.0,
                   help="approximate CPU time budget for the oracle baseline (0 disables it)")
    p.add_argument("--kernel-timing-steps", type=int, default=8,
                   help="steps whose launches are bracketed by HIP events (two-launch path roofline)")
    p.add_argument("--copy-calibration-mib", type=int, default=0,
                   help="also run a plain device copy of this many MiB (reference for profiler byte counters)")
    p.add_argument("--check-steps", type=int, default=2,
                   help="steps whose outputs are compared with the CPU oracle after timing")
    return p.parse_args(argv)


def kv_elem_bytes(fp8):
    """Bytes per cached element and per (token, kv head) scale."""
    return (1, 4) if fp8 else (2, 0)


def algorithmic_bytes(batch, hq, hkv, d, lens_after, fp8=False, page=0):
    """Bytes one layer-step must move: K and V read over each sequence's cache (length after the append),
    new K/V rows read (bf16) and written (cache format), q read and the output written, and for paged caches
    the block-table entries and lengths read."""
    e, s = kv_elem_bytes(fp8)
    kv_read = sum(2 * L * hkv * (d * e + s) for L in lens_after)
    new_rows = 2 * batch * hkv * d * 2 + 2 * batch * hkv * (d * e + s)
    q_out = 2 * batch * hq * d * 2
    table = (sum((L + page - 1) // page * 4 for L in lens_after) + batch * 4) if page else 0
    return kv_read + new_rows + q_out + table


def decode_kernel_bytes(batch, hq, hkv, d, lens_after, fp8=False, page=0):
    """Bytes of the decode launch alone (two-launch path): K/V over the cache, q in, out out, table."""
    e, s = kv_elem_bytes(fp8)
    table = (sum((L + page - 1) // page * 4 for L in lens_after) + batch * 4) if page else 0
    return sum(2 * L * hkv * (d * e + s) for L in lens_after) + 2 * batch * hq * d * 2 + table


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


def host_cores():
    """(cores this process may run on, details): the CPU affinity mask, capped by a cgroup CPU quota when one is
    set (a container's share of a larger host); os.cpu_count() is the host's total and is recorded beside it."""
    total = os.cpu_count() or 1
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = total
    quota = None
    for path in ("/sys/fs/cgroup/cpu.max", "/sys/fs/cgroup/cpu/cpu.cfs_quota_us"):
        try:
            with open(path) as f:
                fields = f.read().split()
        except OSError:
            continue
        if path.endswith("cpu.max") and fields and fields[0] != "max":
            quota = int(fields[0]) / int(fields[1])
        elif path.endswith("cfs_quota_us") and fields and int(fields[0]) > 0:
            with open("/sys/fs/cgroup/cpu/cpu.cfs_period_us") as f:
                quota = int(fields[0]) / int(f.read().split()[0])
        break
    usable = affinity if quota is None else max(1, min(affinity, int(quota)))
    return usable, {"host_cpu_count": total, "affinity_cpus": affinity,
                    "cgroup_cpu_quota": None if quota is None else round(quota, 2)}


def percentile(xs, p):
    ys = sorted(xs)
    if not ys:
        return None
    k = (len(ys) - 1) * p
    lo, hi = math.floor(k), math.ceil(k)
    return ys[lo] + (ys[hi] - ys[lo]) * (k - lo)


def model_step(args) -> int:
    """--config model: µs per generated token for the whole text-decoder step (see the module docstring)."""
    import copy

    import torch
    from transformers.cache_utils import DynamicCache
    from transformers.models.qwen3_vl.configuration_qwen3_vl import Qwen3VLTextConfig
    from transformers.models.qwen3_vl.modeling_qwen3_vl import Qwen3VLTextModel

    import aicas_amd.fused_attention as fa
    from aicas_amd.graph_runner import AicasGraphDecodeRunner
    from aicas_amd.kv_cache import AicasDecodeCache

    t_start = time.perf_counter()

    def progress(what):
        print(f"[model +{time.perf_counter() - t_start:.1f}s] {what}", file=sys.stderr, flush=True)

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    K, W, P = args.steps or 64, max(16 if args.warmup is None else args.warmup, 2), args.prompt_len
    cfg = Qwen3VLTextConfig(vocab_size=151936, hidden_size=2048, intermediate_size=6144, num_hidden_layers=28,
                            num_attention_heads=16, num_key_value_heads=8, head_dim=128, rms_norm_eps=1e-6,
                            rope_theta=5e6, max_position_embeddings=P + K + W + 64)
    cfg._attn_implementation = "sdpa"
    torch.manual_seed(0)
    progress("building the model")
    default_dtype = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device(dev):
            model = Qwen3VLTextModel(cfg).eval()
            lm_head = torch.nn.Linear(2048, 151936, bias=False)
    finally:
        torch.set_default_dtype(default_dtype)
    progress("model built")
    gen = torch.Generator(device=dev).manual_seed(1)
    prompt = torch.randint(0, 151936, (1, P), generator=gen, device=dev)
    with torch.no_grad():
        prefix = DynamicCache(config=cfg)
        h = model(input_ids=prompt, past_key_values=prefix, use_cache=True).last_hidden_state
        tok0 = lm_head(h[:, -1:, :]).argmax(-1)
    torch.cuda.synchronize()
    progress(f"prefill of {P} tokens done")
    cap = P + K + W + 8

    def timed(step, n):
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(n):
            step()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / n

    results = {}
    with torch.no_grad():
        # HF eager: DynamicCache (torch.cat per layer and step) + SDPA
        cache = copy.deepcopy(prefix)
        state = {"tok": tok0.clone(), "pos": torch.full((1, 1), P, dtype=torch.long, device=dev)}

        def hf_step():
            hh = model(input_ids=state["tok"], past_key_values=cache, use_cache=True,
                       position_ids=state["pos"]).last_hidden_state
            state["tok"] = lm_head(hh[:, -1:, :]).argmax(-1)
            state["pos"] = state["pos"] + 1

        for _ in range(W):
            hf_step()
        results["hf_eager_us"] = timed(hf_step, K)
        progress(f"HF eager: {results['hf_eager_us']:.1f} us/token")
        del cache
        # eager, attention fused (q/k norm + rotary + append + attend in one launch per layer)
        acache = AicasDecodeCache(num_layers=28, max_cache_len=cap)
        for src, dst in zip(prefix.layers, acache.layers):
            dst.load_prefix(src.keys, src.values)
        fa.install_fused_decode(model)
        state = {"tok": tok0.clone(), "pos": torch.full((1, 1), P, dtype=torch.long, device=dev)}

        def fused_step():
            hh = model(input_ids=state["tok"], past_key_values=acache, use_cache=True,
                       position_ids=state["pos"]).last_hidden_state
            state["tok"] = lm_head(hh[:, -1:, :]).argmax(-1)
            state["pos"] = state["pos"] + 1

        for _ in range(W):
            fused_step()
        results["fused_eager_us"] = timed(fused_step, K)
        progress(f"fused eager: {results['fused_eager_us']:.1f} us/token")
        del acache
        # the step captured once as a HIP graph
        runner = AicasGraphDecodeRunner(model, lm_head, max_cache_len=cap)
        pos = torch.full((1, 1), P, dtype=torch.long, device=dev)
        assert runner.maybe_capture(prefix, P, tok0, pos)
        progress("graph captured")
        state = {"pos": pos}

        def graph_step():
            runner.prepare_step(runner.static_next_token, state["pos"])
            runner.replay()
            state["pos"] = state["pos"] + 1

        for _ in range(W):
            graph_step()
        results["graph_us"] = timed(graph_step, K)
        progress(f"graph: {results['graph_us']:.1f} us/token")
        runner.release()
        fa.uninstall_fused_decode(model)
    out = {
        "metric": "us per generated token, whole Qwen3-VL-2B text-decoder decode step (reported beside the "
                  "headline, not the headline)",
        "value": round(results["graph_us"], 1),
        "unit": "us/token",
        "n_gpus": 1, "steps": K, "warmup": W, "ms_per_step": round(results["graph_us"] / 1e3, 4),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (random bf16 weights and prompt)",
        "config": {"workload": f"qwen3vl-2b text decoder step, B=1, {P} cached tokens, 28 layers, vocab 151936",
                   "batch": 1, "cached_before": P},
        "hf_eager_us_per_token": round(results["hf_eager_us"], 1),
        "fused_eager_us_per_token": round(results["fused_eager_us"], 1),
        "graph_us_per_token": round(results["graph_us"], 1),
        "tokens_per_s_graph": round(1e6 / results["graph_us"], 1),
        "speedup_graph_vs_hf_eager": round(results["hf_eager_us"] / results["graph_us"], 2),
    }
    print(json.dumps(out), flush=True)
    return 0


def microbench(args) -> int:
    """--config microbench: the shape the reference publishes decode numbers for (message/
    run_triton_attention_microbench.py:39-44: B=1, 16 query / 4 kv heads, head_dim 128, 8192 cached tokens;
    0.2299 ms per gqa_decode_attention call in fp16 on an RTX 3070 Laptop, message/triton_attention_microbench.json:13),
    timed the reference's way — host wall time per call of the public gqa_decode_attention, SDPA over repeat_kv
    beside it — and as the kernel alone (one launch per call, captured in a graph). 32 cache instances (537 MB)
    are stepped through in turn so that the 256 MB memory-side cache cannot serve the reads. Context, not a
    headline: reported beside the configuration the metric is quoted on."""
    import torch
    import torch.nn.functional as F

    from aicas_amd import ops
    from aicas_amd.fallback import repeat_kv
    from aicas_amd.gqa_decode_attention import gqa_decode_attention

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    B, HQ, HKV, D, L, NL = 1, 16, 4, 128, 8192, 32
    iters, warm = args.steps or 100, max(16 if args.warmup is None else args.warmup, 20)
    scale = D ** -0.5
    results = {}
    for name, dtype in (("fp16", torch.float16), ("bf16", torch.bfloat16)):
        gen = torch.Generator(device=dev).manual_seed(0)
        qs = [torch.randn((B, HQ, 1, D), generator=gen, device=dev).to(dtype) for _ in range(NL)]
        ks = [torch.randn((B, HKV, L, D), generator=gen, device=dev).to(dtype) for _ in range(NL)]
        vs = [torch.randn((B, HKV, L, D), generator=gen, device=dev).to(dtype) for _ in range(NL)]

        def ours(i):
            return gqa_decode_attention(qs[i], ks[i], vs[i], sm_scale=scale, num_key_value_groups=HQ // HKV)

        def sdpa(i):
            return F.scaled_dot_product_attention(qs[i], repeat_kv(ks[i], HQ // HKV), repeat_kv(vs[i], HQ // HKV),
                                                  scale=scale)

        def wall_ms(fn):
            for j in range(warm):
                fn(j % NL)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for j in range(iters):
                fn(j % NL)
            torch.cuda.synchronize()
            return (time.perf_counter() - t0) * 1e3 / iters

        err = max(float((ours(i).float() - sdpa(i).float()).abs().max()) for i in range(4))
        ours_ms, sdpa_ms = wall_ms(ours), wall_ms(sdpa)
        # the kernel alone: one decode launch per cache instance, captured once, replayed
        outs = [torch.empty_like(q) for q in qs]
        views = [ops.KVCacheView(k, v) for k, v in zip(ks, vs)]
        stream = torch.cuda.Stream(device=dev)
        with torch.cuda.stream(stream):
            for i in range(NL):
                ops.decode_attention(qs[i], views[i], sm_scale=scale, out=outs[i])
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                for i in range(NL):
                    ops.decode_attention(qs[i], views[i], sm_scale=scale, out=outs[i])
            for _ in range(3):
                graph.replay()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            reps = max(1, iters // NL)
            e0.record()
            for _ in range(reps):
                graph.replay()
            e1.record()
            torch.cuda.synchronize()
        kernel_us = e0.elapsed_time(e1) * 1e3 / (reps * NL)
        nbytes = 2 * B * HKV * L * D * 2 + 2 * B * HQ * D * 2
        results[name] = {
            "gqa_decode_attention_wall_ms": round(ours_ms, 4), "sdpa_repeat_kv_wall_ms": round(sdpa_ms, 4),
            "speedup_vs_sdpa": round(sdpa_ms / ours_ms, 3), "kernel_us_per_launch": round(kernel_us, 2),
            "kernel_hbm_gbps": round(nbytes / (kernel_us * 1e-6) / 1e9, 1), "max_abs_err_vs_sdpa": err,
        }
        del qs, ks, vs, views, outs, graph
    out = {
        "metric": "ms per q_len=1 GQA decode call, B=1 16q/4kv head_dim 128, 8192 cached tokens (the reference's "
                  "published microbenchmark shape; reported beside the headline, not the headline)",
        "value": results["fp16"]["gqa_decode_attention_wall_ms"], "unit": "ms/call", "n_gpus": 1, "steps": iters,
        "warmup": warm, "ms_per_step": results["fp16"]["gqa_decode_attention_wall_ms"], "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp16", "data": "synthetic (seeded N(0,1))",
        "config": {"workload": "gqa decode microbenchmark: B=1, 16 q / 4 kv heads, head_dim 128, L=8192, "
                               f"{NL} rotated cache instances", "batch": B, "kv_len": L},
        "reference_published": {"triton_ms": 0.2299, "sdpa_ms": 0.2959, "gpu": "RTX 3070 Laptop, fp16",
                                "source": "message/triton_attention_microbench.json"},
        "results": results,
    }
    print(json.dumps(out), flush=True)
    return 0


def calib(args) -> int:
    """--config calib: the per-launch streaming ceiling the headline launch is measured against, from committed
    code. One layer of the headline workload (B=8, 8 kv heads, head_dim 128, 2112 tokens: the mean length of a
    128-step run, 69.2 MB of K and V) is read by, per launch: the fused append + attend launch itself; a pure
    streaming read with the attention's grid and access pattern (libaicas_calib.so, at the plan's 4 splits per
    (batch, kv head) pair and at 8); a flat read of the same bytes in 4096 workgroups; and an empty launch. 28
    distinct layers (1.9 GB) are launched back to back in a graph, so the 256 MB memory-side cache cannot serve
    the reads; µs per launch = graph time / launches."""
    import ctypes

    import torch

    from aicas_amd import ops
    from aicas_amd.build import CALIB_OUTPUT

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    B, HQ, HKV, D, L, NL = 8, 16, 8, 128, 2112, 28
    reps = args.steps or 20
    lib = ctypes.CDLL(CALIB_OUTPUT, mode=ctypes.RTLD_LOCAL)
    P, I32, I64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
    lib.aicas_calib_stream_read.argtypes = [P, P, I64, I64, I32, I32, I32, I32, P, P]
    lib.aicas_calib_flat_read.argtypes = [P, P, I64, I32, P, P]
    lib.aicas_calib_empty.argtypes = [P]
    gen = torch.Generator(device=dev).manual_seed(2)
    ks = [torch.randn((B, HKV, L + 1, D), generator=gen, device=dev).to(torch.bfloat16) for _ in range(NL)]
    vs = [torch.randn((B, HKV, L + 1, D), generator=gen, device=dev).to(torch.bfloat16) for _ in range(NL)]
    q = torch.randn((NL, B, HQ, 1, D), generator=gen, device=dev).to(torch.bfloat16)
    kn = torch.randn((NL, B, HKV, 1, D), generator=gen, device=dev).to(torch.bfloat16)
    out = torch.empty_like(q)
    pos = torch.full((B,), L - 1, dtype=torch.int32, device=dev)  # attend over L tokens, the last one appended
    plan = ops.decode_plan(torch.bfloat16, B, HQ, HKV, D, L)
    ws = ops.Workspace.reserve(dev, plan.workspace_bytes)
    sink = torch.empty(4096 * 256, dtype=torch.int32, device=dev)
    kv_bytes = 2 * B * HKV * L * D * 2
    stream = torch.cuda.Stream(device=dev)

    def check(rc):
        if rc:
            raise RuntimeError(f"calibration launch failed ({rc})")

    def attention(i):
        ops.decode_attention_append(q[i], ops.KVCacheView(ks[i], vs[i]), kn[i], kn[i], pos, sm_scale=D ** -0.5,
                                    max_seq_len=L, min_seq_len=L - 1, out=out[i], workspace=ws)

    def stream_read(splits):
        return lambda i: check(lib.aicas_calib_stream_read(ks[i].data_ptr(), vs[i].data_ptr(), ks[i].stride(0),
                                                           ks[i].stride(1), B, HKV, L, splits, sink.data_ptr(),
                                                           stream.cuda_stream))

    # the flat read covers each tensor's first B*Hkv*(L+1)*D elements: the L attended tokens plus one row per
    # (batch, kv head) pair, 0.05% more bytes, counted
    flat_bytes = ks[0].numel() * 2

    def flat_read(i):
        check(lib.aicas_calib_flat_read(ks[i].data_ptr(), vs[i].data_ptr(), flat_bytes, 4096, sink.data_ptr(),
                                        stream.cuda_stream))

    def empty(i):
        check(lib.aicas_calib_empty(stream.cuda_stream))

    def per_launch_us(fn):
        with torch.cuda.stream(stream):
            for i in range(NL):
                fn(i)
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                for i in range(NL):
                    fn(i)
            for _ in range(3):
                graph.replay()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                graph.replay()
            e1.record()
            torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / (reps * NL)

    rows = {}
    for name, fn, nbytes in (
        ("fused append + attend launch (the headline kernel)", attention, algorithmic_bytes(B, HQ, HKV, D, [L] * B)),
        (f"streaming read, the attention's grid ({plan.num_splits} splits x 64 pairs)", stream_read(plan.num_splits),
         kv_bytes),
        ("streaming read, the attention's pattern at 8 splits", stream_read(8), kv_bytes),
        ("flat read of the same bytes, 4096 workgroups", flat_read, 2 * flat_bytes),
        ("empty launch", empty, 0),
    ):
        us = per_launch_us(fn)
        rows[name] = {"us_per_launch": round(us, 3), "bytes": nbytes,
                      "gbps": round(nbytes / (us * 1e-6) / 1e9, 1) if nbytes else None,
                      "frac_of_8tbps": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4) if nbytes else None}
        print(f"[calib] {name}: {us:.3f} us per launch", file=sys.stderr, flush=True)
    result = {
        "metric": "us per launch: the headline launch against pure streaming reads of the same bytes and an empty "
                  "launch (calibration, reported beside the headline, not the headline)",
        "value": rows["fused append + attend launch (the headline kernel)"]["us_per_launch"], "unit": "us/launch",
        "n_gpus": 1, "steps": reps, "warmup": 3, "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic (seeded N(0,1))",
        "config": {"workload": f"one layer of the B=8 decode step: 8 kv heads, head_dim 128, {L} tokens, {NL} "
                               "distinct layers per graph", "batch": B, "tokens": L, "splits": plan.num_splits},
        "launches": rows,
    }
    print(json.dumps(result), flush=True)
    return 0


def gather(args) -> int:
    """--config gather: aicas_kv_gather over the C5 cache (B=32, lengths U{256..8192}, 16-token pages over a
    permuted block table, fp8 e4m3 codes + fp32 scales per (token, kv head)) into dense bf16 K and V
    [32, 8, max_len, 128]: what a prefill's attention reads from that cache. Bytes per launch: the cached rows
    read (codes and scales) plus the dense rows written (max_len per sequence, zeros past its length). Two
    distinct caches alternate in the graph, so the 256 MB memory-side cache cannot serve the reads; µs per launch
    = graph time / launches. The CPU baseline is the oracle's gather + dequantisation of the same cache
    (torch on the host cores) over a bounded sample of its sequences."""
    import torch

    from aicas_amd import ops
    from aicas_amd.workloads import HEAD_DIM as D, HKV, PAGE, WORKLOADS, generator, normal, seq_lengths

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    w = WORKLOADS["c5"]
    gen = generator(dev, w.seed)
    lens = seq_lengths(w, gen)
    B, NL, reps = w.batch, 2, args.steps or 20
    max_len = max(lens)
    views = []
    for _ in range(NL):
        per_seq = [(L + PAGE - 1) // PAGE for L in lens]
        nblocks = sum(per_seq)
        perm = torch.randperm(nblocks, generator=gen, device=dev).to(torch.int32)
        bt = torch.full((B, max(per_seq)), -1, dtype=torch.int32, device=dev)
        at = 0
        for b, n in enumerate(per_seq):
            bt[b, :n] = perm[at : at + n]
            at += n
        kp = torch.zeros((nblocks, HKV, PAGE, D), dtype=ops.FP8_DTYPE, device=dev)
        vp = torch.zeros_like(kp)
        ksc = torch.zeros((nblocks, HKV, PAGE), dtype=torch.float32, device=dev)
        vsc = torch.zeros_like(ksc)
        view = ops.KVCacheView(kp, vp, ksc, vsc, bt)
        for b, L in enumerate(lens):
            rows_k = normal((1, HKV, L, D), gen, dev, outlier_frac=w.outlier_frac, outlier_value=w.outlier_value)
            rows_v = normal((1, HKV, L, D), gen, dev, outlier_frac=w.outlier_frac, outlier_value=w.outlier_value)
            ops.kv_append(ops.KVCacheView(kp, vp, ksc, vsc, bt[b : b + 1]), rows_k, rows_v,
                          torch.zeros(1, dtype=torch.int32, device=dev))
        views.append(view)
    seq_lens = torch.tensor(lens, dtype=torch.int32, device=dev)
    k_out = torch.empty((B, HKV, max_len, D), dtype=torch.bfloat16, device=dev)
    v_out = torch.empty_like(k_out)
    read_bytes = 2 * sum(lens) * HKV * (D + 4)
    write_bytes = 2 * B * HKV * max_len * D * 2
    stream = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(stream):
        for v in views:
            ops.kv_gather(v, seq_lens, max_len, out=(k_out, v_out))
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for v in views:
                ops.kv_gather(v, seq_lens, max_len, out=(k_out, v_out))
        for _ in range(3):
            graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            graph.replay()
        e1.record()
        torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / (reps * NL)
    gbps = (read_bytes + write_bytes) / (us * 1e-6) / 1e9

    # parity of the last launch (the second cache) against the oracle, on a few sequences
    from oracle import reference_path as ref

    view = views[-1]
    check = [0, 1, B - 1]
    kc, ks_c, bt_c = view.k.cpu(), view.k_scale.cpu(), view.block_table.cpu()
    max_err = 0
    for b in check:
        codes = ref.paged_gather(kc, bt_c[b : b + 1], [lens[b]])[0]
        scale = ref.paged_gather(ks_c[..., None], bt_c[b : b + 1], [lens[b]])[0][..., 0]
        want = ref.fp8_dequantize_rows(codes, scale).to(torch.bfloat16)
        got = k_out[b, :, : lens[b]].cpu()
        max_err = max(max_err, int((got.view(torch.int16) != want.view(torch.int16)).sum()))

    cpu = None
    if args.cpu_baseline_seconds > 0:
        threads, core_info = host_cores()
        torch.set_num_threads(threads)
        vc, vs_c = view.v.cpu(), view.v_scale.cpu()
        t_s, done, tokens = time.perf_counter(), 0, 0
        for b in range(B):
            for pool, sc in ((kc, ks_c), (vc, vs_c)):
                codes = ref.paged_gather(pool, bt_c[b : b + 1], [lens[b]])[0]
                scale = ref.paged_gather(sc[..., None], bt_c[b : b + 1], [lens[b]])[0][..., 0]
                dense = torch.zeros((HKV, max_len, D), dtype=torch.bfloat16)
                dense[:, : lens[b]] = ref.fp8_dequantize_rows(codes, scale).to(torch.bfloat16)
            done += 1
            tokens += lens[b]
            if time.perf_counter() - t_s > args.cpu_baseline_seconds:
                break
        cpu_s = time.perf_counter() - t_s
        cpu_us = cpu_s / done * B * 1e6
        cpu = {"value": round(cpu_us, 1), "unit": "us/launch", "cores": threads, **core_info, "kind": "port",
               "sample": f"the oracle's paged gather + fp8 dequantisation (torch {torch.__version__}, host) of "
                         f"{done} of the {B} sequences ({tokens} tokens), scaled to all {B}"}
    result = {
        "metric": "us per aicas_kv_gather launch & achieved HBM GB/s (% of 8 TB/s): the C5 paged fp8 cache as "
                  "dense bf16 rows (reported beside the headline, not the headline)",
        "value": round(us, 2), "unit": "us/launch", "n_gpus": 1, "steps": reps, "warmup": 3,
        "ms_per_step": round(us / 1e3, 5), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp8->bf16", "data": "synthetic (seeded N(0,1), 1% outliers +-8)",
        "config": {"workload": f"kv gather: B={B}, 8 kv heads, head_dim 128, lengths U{{256..8192}} (max {max_len}), "
                               "16-token pages, fp8 e4m3 + fp32 scales -> bf16", "batch": B, "max_len": max_len,
                   "cache_instances": NL},
        "roofline": {"bound": "hbm", "kernel": "kv_gather_kernel<fp8,bf16,D=128>", "achieved": round(gbps, 1),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": None,
                     "bytes_per_launch": read_bytes + write_bytes, "read_bytes": read_bytes,
                     "write_bytes": write_bytes, "avg_launch_us": round(us, 3)},
        "cpu_baseline": cpu,
        "parity_mismatched_elements": max_err,
    }
    print(json.dumps(result), flush=True)
    return 0 if max_err == 0 else 1


def prefill_bytes(batch: int, kv_heads: int, n_new: int, head_dim: int, fp8: bool = False, page: int = 0) -> int:
    """Algorithmic bytes of one aicas_kv_append launch writing n_new tokens per sequence from position 0: the
    16-bit source rows read (K and V), the cache rows written (fp8: one code byte per element and a 4-byte scale
    per row; 16-bit: the rows as they are), the block-table entries of the pages written (paged caches) and the
    positions read."""
    rows = 2 * batch * kv_heads * n_new
    src = rows * head_dim * 2
    dst = rows * (head_dim + 4) if fp8 else rows * head_dim * 2
    table = batch * -(-n_new // page) * 4 if page else 0
    return src + dst + table + batch * 4


def prefill(args) -> int:
    """--config prefill: the prefill writer, one aicas_kv_append launch that writes a 2048-token prompt for each
    of 32 sequences (8 kv heads, head_dim 128) into the C5 layout (16-token pages over a permuted block table,
    fp8 e4m3 quantised on write with an fp32 scale per (token, kv head)), and the same into a contiguous bf16
    cache. Bytes per launch: the bf16 rows read plus the cache rows (and scales) written. Two distinct caches
    alternate in the graph; µs per launch = graph time / launches. The CPU baseline is the oracle's quantisation
    and paged scatter of the same rows (torch on the host cores) over a bounded sample of the sequences."""
    import torch

    from aicas_amd import ops
    from aicas_amd.workloads import HEAD_DIM as D, HKV, PAGE, generator, normal

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    B, N, NL, reps = 32, 2048, 2, args.steps or 20
    gen = generator(dev, 6)
    k_src = normal((B, HKV, N, D), gen, dev, outlier_frac=0.01)
    v_src = normal((B, HKV, N, D), gen, dev, outlier_frac=0.01)
    pos = torch.zeros(B, dtype=torch.int32, device=dev)
    per_seq = N // PAGE
    paged, dense = [], []
    for _ in range(NL):
        bt = torch.randperm(B * per_seq, generator=gen, device=dev).to(torch.int32).view(B, per_seq)
        kp = torch.zeros((B * per_seq, HKV, PAGE, D), dtype=ops.FP8_DTYPE, device=dev)
        ks = torch.zeros((B * per_seq, HKV, PAGE), dtype=torch.float32, device=dev)
        paged.append(ops.KVCacheView(kp, torch.zeros_like(kp), ks, torch.zeros_like(ks), bt))
        kd = torch.zeros((B, HKV, N, D), dtype=torch.bfloat16, device=dev)
        dense.append(ops.KVCacheView(kd, torch.zeros_like(kd)))
    stream = torch.cuda.Stream(device=dev)

    def per_launch_us(views):
        with torch.cuda.stream(stream):
            for v in views:
                ops.kv_append(v, k_src, v_src, pos)
            torch.cuda.synchronize()
            if args.mode == "eager":  # every dispatch its own (for counter runs)
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(reps):
                    for v in views:
                        ops.kv_append(v, k_src, v_src, pos)
                e1.record()
                torch.cuda.synchronize()
                return e0.elapsed_time(e1) * 1e3 / (reps * len(views))
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                for v in views:
                    ops.kv_append(v, k_src, v_src, pos)
            for _ in range(3):
                graph.replay()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                graph.replay()
            e1.record()
            torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / (reps * len(views))

    fp8_bytes = prefill_bytes(B, HKV, N, D, fp8=True, page=PAGE)
    bf16_bytes = prefill_bytes(B, HKV, N, D)
    if args.copy_calibration_mib > 0:  # a device copy of known size beside the kernel, for counter runs
        n = args.copy_calibration_mib << 20
        src = torch.empty(n, dtype=torch.uint8, device=dev).random_(0, 255)
        dst = torch.empty_like(src)
        for _ in range(4):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    us_fp8 = per_launch_us(paged)
    us_bf16 = per_launch_us(dense)

    # parity of the paged fp8 cache against the oracle's quantisation, a few sequences
    from oracle import reference_path as ref

    view = paged[-1]
    kc, ksc, btc = view.k.cpu(), view.k_scale.cpu(), view.block_table.cpu()
    mismatched = 0
    for b in (0, B - 1):
        codes, scale = ref.fp8_quantize_rows(k_src[b].cpu().float())
        got = ref.paged_gather(kc, btc[b : b + 1], [N])[0]
        got_s = ref.paged_gather(ksc[..., None], btc[b : b + 1], [N])[0][..., 0]
        mismatched += int((got.view(torch.uint8) != codes.view(torch.uint8)).sum())
        mismatched += int((got_s != scale).sum())

    cpu = None
    if args.cpu_baseline_seconds > 0:
        threads, core_info = host_cores()
        torch.set_num_threads(threads)
        src = (k_src.cpu(), v_src.cpu())
        pool = torch.zeros((per_seq, HKV, PAGE, D), dtype=ops.FP8_DTYPE)
        spool = torch.zeros((per_seq, HKV, PAGE), dtype=torch.float32)
        table = torch.arange(per_seq, dtype=torch.int32)[None]
        t_s, done = time.perf_counter(), 0
        for b in range(B):
            for x in src:
                codes, scale = ref.fp8_quantize_rows(x[b].float())
                for t in range(0, N, PAGE):  # one page of rows at a time into its block
                    blk = int(table[0, t // PAGE])
                    pool[blk] = codes[:, t : t + PAGE]
                    spool[blk] = scale[:, t : t + PAGE]
            done += 1
            if time.perf_counter() - t_s > args.cpu_baseline_seconds:
                break
        cpu_us = (time.perf_counter() - t_s) / done * B * 1e6
        cpu = {"value": round(cpu_us, 1), "unit": "us/launch", "cores": threads, **core_info, "kind": "port",
               "sample": f"the oracle's fp8 quantisation + paged scatter (torch {torch.__version__}, host) of "
                         f"{done} of the {B} sequences, scaled to all {B}"}
    gbps = fp8_bytes / (us_fp8 * 1e-6) / 1e9
    result = {
        "metric": "us per aicas_kv_append prefill launch & achieved HBM GB/s (% of 8 TB/s): a 2048-token prompt "
                  "for 32 sequences into the C5 paged fp8 layout (reported beside the headline, not the headline)",
        "value": round(us_fp8, 2), "unit": "us/launch", "n_gpus": 1, "steps": reps, "warmup": 3,
        "ms_per_step": round(us_fp8 / 1e3, 5), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16->fp8", "data": "synthetic (seeded N(0,1), 1% outliers +-8)",
        "config": {"workload": f"kv append (prefill): B={B}, 8 kv heads, head_dim 128, {N} new tokens per "
                               "sequence, 16-token pages, fp8 e4m3 + fp32 scales", "batch": B, "new_tokens": N,
                   "cache_instances": NL},
        "roofline": {"bound": "hbm", "kernel": "kv_append_kernel<bf16,fp8,D=128>", "achieved": round(gbps, 1),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": None,
                     "bytes_per_launch": fp8_bytes, "avg_launch_us": round(us_fp8, 3)},
        "contiguous_bf16": {"us_per_launch": round(us_bf16, 2), "bytes_per_launch": bf16_bytes,
                            "gbps": round(bf16_bytes / (us_bf16 * 1e-6) / 1e9, 1),
                            "frac_of_8tbps": round(bf16_bytes / (us_bf16 * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4)},
        "cpu_baseline": cpu,
        "parity_mismatched_elements": mismatched,
    }
    print(json.dumps(result), flush=True)
    return 0 if mismatched == 0 else 1


def main(argv=None) -> int:
    args = parse_args(argv)
    if args.config == "model" and args.gpus == 1:
        return model_step(args)
    if args.config == "microbench" and args.gpus == 1:
        return microbench(args)
    if args.config == "calib" and args.gpus == 1:
        return calib(args)
    if args.config == "gather" and args.gpus == 1:
        return gather(args)
    if args.config == "prefill" and args.gpus == 1:
        return prefill(args)
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported: each GPU serves its own "
              "sequences (or kv heads), so the step does not shard across GPUs here.", file=sys.stderr)
        return 2

    import torch

    from aicas_amd import ops
    from aicas_amd.workloads import HEAD_DIM, HKV, HQ, PAGE, SM_SCALE, WORKLOADS, generator, normal, seq_lengths

    w = WORKLOADS[args.config]
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    B, D = w.batch, HEAD_DIM
    G = HQ // HKV
    growing = w.steps > 1  # c2, c3: every step appends a new token; c1, c4, c5: one step, repeated
    K = args.steps or (w.steps if growing else 64)
    # one-layer configurations: a step is one short launch per cache instance; measured on MI355X, B=32 paged fp8
    # takes 70.9 us per step after 16 warmup steps and 69.3 after 64 or 256 (B=8 L=2048, 28 layers: 442.5 after 5,
    # 440.2 after 64)
    W = args.warmup if args.warmup is not None else (16 if w.layers > 1 else 64)
    n_graph_steps = max(K, W) if growing else 1
    gen = generator(dev, w.seed)
    base = [w.prefill] * B if w.len_range is None else seq_lengths(w, gen)  # cached before step 0
    page = PAGE if w.paged else 0
    kv_dtype = ops.FP8_DTYPE if w.fp8 else torch.bfloat16
    # cache instances: the configuration's layers, or for one-layer configurations enough copies to exceed
    # twice the MALL (>= 4), stepped through in turn within each step
    one_layer = algorithmic_bytes(B, HQ, HKV, D, [L + n_graph_steps for L in base], w.fp8, page)
    NL = w.layers if w.layers > 1 else max(4, math.ceil(2 * MALL_BYTES / one_layer))
    if w.layers == 1 and args.cache_instances > 0:
        NL = args.cache_instances
    layer_weight = w.layers / NL  # one-layer configs: a step's time is the per-layer time
    cap_seq = max(base) + n_graph_steps

    # ---- inputs, resident in HBM before anything is timed
    views = []
    if not w.paged:
        cap = (cap_seq + 63) // 64 * 64
        for _ in range(NL):
            kb = torch.zeros((B, HKV, cap, D), dtype=torch.bfloat16, device=dev)
            vb = torch.zeros_like(kb)
            for b, L in enumerate(base):
                kb[b, :, :L] = normal((HKV, L, D), gen, dev, scale=w.k_scale)
                vb[b, :, :L] = normal((HKV, L, D), gen, dev)
            views.append(ops.KVCacheView(kb, vb))
    else:
        per_seq = [(L + n_graph_steps + page - 1) // page for L in base]
        width, nblocks = max(per_seq), sum(per_seq)
        for _ in range(NL):
            perm = torch.randperm(nblocks, generator=gen, device=dev).to(torch.int32)
            bt = torch.full((B, width), -1, dtype=torch.int32, device=dev)
            at = 0
            for b, n in enumerate(per_seq):
                bt[b, :n] = perm[at : at + n]
                at += n
            kp = torch.zeros((nblocks, HKV, page, D), dtype=kv_dtype, device=dev)
            vp = torch.zeros_like(kp)
            ks = torch.zeros((nblocks, HKV, page), dtype=torch.float32, device=dev) if w.fp8 else None
            vs = torch.zeros_like(ks) if w.fp8 else None
            for b, L in enumerate(base):
                src_k = normal((1, HKV, L, D), gen, dev, outlier_frac=w.outlier_frac, outlier_value=w.outlier_value)
                src_v = normal((1, HKV, L, D), gen, dev, outlier_frac=w.outlier_frac, outlier_value=w.outlier_value)
                ops.kv_append(ops.KVCacheView(kp, vp, ks, vs, bt[b : b + 1]), src_k, src_v,
                              torch.zeros(1, dtype=torch.int32, device=dev))
            views.append(ops.KVCacheView(kp, vp, ks, vs, bt))
    q_all = normal((n_graph_steps, NL, B, HQ, 1, D), gen, dev)
    kn_all = normal((n_graph_steps, NL, B, HKV, 1, D), gen, dev, scale=w.k_scale,
                    outlier_frac=w.outlier_frac, outlier_value=w.outlier_value)
    vn_all = normal((n_graph_steps, NL, B, HKV, 1, D), gen, dev,
                    outlier_frac=w.outlier_frac, outlier_value=w.outlier_value)
    out_all = torch.zeros((n_graph_steps, NL, B, HQ, 1, D), dtype=torch.bfloat16, device=dev)
    # q/k preparation inputs for the fused_qk path: per-layer norm weights, per-step rotary rows of the text
    # positions (the default rotary base 5e6 over head_dim), prepared q written per layer
    qk_all = None
    if args.compare_qk:
        qn_w = 1 + 0.1 * normal((NL, D), gen, dev)
        kn_w = 1 + 0.1 * normal((NL, D), gen, dev)
        inv_freq = 1.0 / (5.0e6 ** (torch.arange(0, D, 2, dtype=torch.float32, device=dev) / D))
        pos = torch.tensor(base, dtype=torch.float32, device=dev)[None, :] + torch.arange(
            n_graph_steps, dtype=torch.float32, device=dev)[:, None]
        ang = pos[..., None] * inv_freq
        ang = torch.cat([ang, ang], -1)  # [steps, B, D]
        qk_all = (qn_w, kn_w, ang.cos().to(torch.bfloat16), ang.sin().to(torch.bfloat16),
                  torch.zeros((NL, B, HQ, 1, D), dtype=torch.bfloat16, device=dev))
    # fused path: one length tensor for the whole step (tokens cached before it), bumped by the last layer's
    # kernel when the step grows the cache, as a serving loop keeps it; separate path: each layer's append
    # bumps that layer's lengths (and a one-step configuration restores them inside the step)
    lens0 = torch.tensor(base, dtype=torch.int32, device=dev)
    shared_lens = lens0.clone()
    lens = [lens0.clone() for _ in range(NL)]
    # one split size for the whole run, planned at the longest step (the plan's workspace covers every step)
    plan = ops.decode_plan(kv_dtype, B, HQ, HKV, D, cap_seq, page, args.tokens_per_split)
    ws = ops.Workspace.reserve(dev, plan.workspace_bytes)
    lo, hi = min(base), max(base)

    def step(s, path, kernel_events=None, once=False):
        """One decode step: for every layer append this step's K/V row and attend. once: the launches a serving
        loop captures a single time and replays for every token — bounded by the capacity and by the prefill
        length, inputs from the step-0 buffers — instead of this step's own bounds and inputs."""
        hi_s, lo_s = (cap_seq - 1, lo) if once else (hi + s, lo + s)  # bounds on the lengths before the append
        if once:
            s = 0
        for i in range(NL):
            if path == "fused_pool":
                # the device block pool gives the page the append will write a block (when it has none yet)
                pools[i].alloc(views[i].block_table, shared_lens, 1, page)
            if path in ("fused", "fused_qk", "fused_pool"):
                qk = None
                if path == "fused_qk":
                    qn_w, kn_w, cos_all, sin_all, q_prep = qk_all
                    qk = ops.QKPrologue(q_norm_weight=qn_w[i], k_norm_weight=kn_w[i], eps=1e-6,
                                        cos=cos_all[s], sin=sin_all[s], q_out=q_prep[i])
                if kernel_events is not None:
                    kernel_events[i][0].record()
                ops.decode_attention_append(
                    q_all[s, i], views[i], kn_all[s, i], vn_all[s, i], shared_lens, sm_scale=SM_SCALE,
                    max_seq_len=hi_s + 1, min_seq_len=lo_s,
                    seq_lens_out=shared_lens if (growing and i == NL - 1) else None, out=out_all[s, i],
                    tokens_per_split=args.tokens_per_split, workspace=ws, qk=qk,
                )
                if kernel_events is not None:
                    kernel_events[i][1].record()
            else:
                ops.kv_append(views[i], kn_all[s, i], vn_all[s, i], lens[i], lens[i])
                if kernel_events is not None:
                    kernel_events[i][0].record()
                ops.decode_attention(
                    q_all[s, i], views[i], sm_scale=SM_SCALE, seq_lens=lens[i], max_seq_len=hi_s + 1,
                    min_seq_len=lo_s + 1, out=out_all[s, i], tokens_per_split=args.tokens_per_split, workspace=ws,
                )
                if kernel_events is not None:
                    kernel_events[i][1].record()
                if not growing:
                    lens[i].copy_(lens0)

    def reset_lens():
        shared_lens.copy_(lens0)
        for t in lens:
            t.copy_(lens0)

    stream = torch.cuda.Stream(device=dev)

    def capture(path, once):
        """once: one graph, replayed for every step (the lengths grow on the device); else one graph per step."""
        graphs = []
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            step(0, path, once=once)  # first launch of every kernel outside capture
            torch.cuda.synchronize()
            reset_lens()
            torch.cuda.synchronize()
            for s in range(1 if once else n_graph_steps):
                gr = torch.cuda.CUDAGraph()
                with torch.cuda.graph(gr, stream=stream):
                    step(s, path, once=once)
                graphs.append(gr)
            torch.cuda.synchronize()
        return graphs

    def run_steps(path, graphs, first, count, events=None, once=False):
        for j, s in enumerate(range(first, first + count)):
            idx = s if (growing and not once) else 0
            if graphs is not None:
                graphs[idx].replay()
            else:
                step(idx, path, once=once)
            if events is not None:
                events[j].record()

    def timed(path, graphs, once):
        with torch.cuda.stream(stream):
            reset_lens()
            run_steps(path, graphs, 0, W, once=once)
            torch.cuda.synchronize()
            reset_lens()
            torch.cuda.synchronize()
            ev0 = torch.cuda.Event(enable_timing=True)
            evs = [torch.cuda.Event(enable_timing=True) for _ in range(K)]
            t0 = time.perf_counter()
            ev0.record()
            run_steps(path, graphs, 0, K, evs, once=once)
            torch.cuda.synchronize()
            t1 = time.perf_counter()
        per_step = [ev0.elapsed_time(evs[0]) * 1e3] + [evs[j - 1].elapsed_time(evs[j]) * 1e3 for j in range(1, K)]
        return ev0.elapsed_time(evs[-1]), (t1 - t0) * 1e3, per_step

    path = args.path
    other = "separate" if path == "fused" else "fused"
    once = args.capture == "once"
    graphs = capture(path, once) if args.mode == "graph" else None
    gpu_ms, wall_ms, per_step_us = timed(path, graphs, once)
    us_graph_step = gpu_ms * 1e3 / K  # one replay: NL layer-steps
    us_per_step = us_graph_step * layer_weight
    other_capture_us = None
    if args.compare_capture and args.mode == "graph":
        graphs_c = capture(path, not once)
        other_capture_us = timed(path, graphs_c, not once)[0] * 1e3 / K * layer_weight
        del graphs_c
    other_us = None
    if args.compare_paths:
        graphs_other = capture(other, once) if args.mode == "graph" else None
        other_us = timed(other, graphs_other, once)[0] * 1e3 / K * layer_weight
        del graphs_other
    pool_us = None
    if w.paged and args.compare_pool:
        # one pool per cache instance, every block free; the tables were filled at set-up, so a step's
        # allocation scans its pages and pops nothing (a page is new only every page_size steps)
        pools = [ops.BlockPool(views[i].k.shape[0], dev) for i in range(NL)]
        graphs_pool = capture("fused_pool", once) if args.mode == "graph" else None
        pool_us = timed("fused_pool", graphs_pool, once)[0] * 1e3 / K * layer_weight
        del graphs_pool
    qk_us = None
    if args.compare_qk:
        graphs_qk = capture("fused_qk", once) if args.mode == "graph" else None
        qk_us = timed("fused_qk", graphs_qk, once)[0] * 1e3 / K * layer_weight
        del graphs_qk

    lens_per_step = [[L + (s if growing else 0) + 1 for L in base] for s in range(K)]
    layer_bytes = [algorithmic_bytes(B, HQ, HKV, D, la, w.fp8, page) for la in lens_per_step]
    bytes_per_step = sum(layer_bytes) / K * w.layers
    gbps = bytes_per_step / (us_per_step * 1e-6) / 1e9

    # ---- the dominant kernel's average duration. On the fused path every launch of the timed region is that
    # kernel (NL per step, back to back in the replayed graphs), so the HIP-event time of the timed region over
    # the number of launches is its average launch duration (launch gaps included). The two-launch path's
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
                step(s if growing else 0, path, kernel_events=evs[s], once=once)
            torch.cuda.synchronize()
            for s in range(kt_steps):
                for i in range(NL):
                    durations.append(evs[s][i][0].elapsed_time(evs[s][i][1]) * 1e3)  # us
    if path == "fused":
        dec_us = us_graph_step / NL
        dec_bytes = sum(layer_bytes) / K  # the fused kernel moves every algorithmic byte of the layer-step
        dec_launches = K * NL
    else:
        dec_us = sum(durations) / len(durations)
        dec_bytes = sum(decode_kernel_bytes(B, HQ, HKV, D, lens_per_step[s], w.fp8, page)
                        for s in range(kt_steps)) / kt_steps
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

    # ---- parity of the first steps against the oracle (outputs of a replay of the timed graphs)
    from oracle import reference_path as ref

    table = ref.e4m3_decode_table() if w.fp8 else None

    def cached(i, b, L):
        """Sequence b's first L cached rows of layer instance i on the host, as the attention sees them."""
        v = views[i]
        if not w.paged:
            return v.k[b, :, :L].cpu(), v.v[b, :, :L].cpu()
        bt = v.block_table[b : b + 1].cpu()
        k = ref.paged_gather(v.k.cpu() if not w.fp8 else v.k.cpu().view(torch.uint8), bt, [L])[0]
        vv = ref.paged_gather(v.v.cpu() if not w.fp8 else v.v.cpu().view(torch.uint8), bt, [L])[0]
        if w.fp8:
            ks = ref.paged_gather(v.k_scale.cpu(), bt, [L])[0]
            vs = ref.paged_gather(v.v_scale.cpu(), bt, [L])[0]
            k, vv = table[k.long()] * ks[..., None], table[vv.long()] * vs[..., None]
        return k, vv

    max_err = 0.0
    check_steps = min(args.check_steps, K, n_graph_steps)
    if check_steps > 0:
        with torch.cuda.stream(stream):
            reset_lens()
            torch.cuda.synchronize()
            run_steps(path, graphs, 0, check_steps, once=once)
            torch.cuda.synchronize()
        src = (lambda s_: 0) if once else (lambda s_: s_)  # step -> the input buffers its launches read
        seqs = list(range(B)) if B <= 8 else list(range(0, B, B // 8))[:8]
        for i in sorted({0, NL // 2, NL - 1}):
            for b in seqs:
                s = check_steps - 1
                L = base[b] + s + 1
                k, v = cached(i, b, L)
                expect = ref.decode_fp64(q_all[src(s), i, b : b + 1].cpu(), k[None], v[None], SM_SCALE, G)
                err = (out_all[src(s), i, b : b + 1].double().cpu() - expect).abs().max().item()
                max_err = max(max_err, err)
        if not w.paged:
            # the appended rows are bit-identical to the torch.cat cache
            for i in sorted({0, NL - 1}):
                for s in range(check_steps):
                    for b in seqs:
                        assert torch.equal(views[i].k[b, :, base[b] + s].cpu().view(torch.int16),
                                           kn_all[src(s), i, b, :, 0].cpu().view(torch.int16))

    # ---- CPU baseline: the oracle (reference PyTorch path) on the host cores, same inputs, first steps (a
    # one-step configuration repeats its step from the same cache)
    cpu = None
    if args.cpu_baseline_seconds > 0:
        threads, core_info = host_cores()
        torch.set_num_threads(threads)
        # at most ~4 GB of cache on the host: a configuration with more times a sample of its layers and scales
        # the time to all of them
        layer_cache = sum(2 * L * HKV * D * 2 for L in base)
        layers_cpu = max(1, min(w.layers, NL, (4 << 30) // layer_cache))
        uniform = len(set(base)) == 1
        init = []
        for i in range(layers_cpu):
            rows = [cached(i, b, base[b]) for b in range(B)]
            ks = [r[0].to(torch.bfloat16) for r in rows]
            vs = [r[1].to(torch.bfloat16) for r in rows]
            init.append((torch.stack(ks), torch.stack(vs)) if uniform else (ks, vs))
        state = list(init)

        def cpu_step(s):
            qs, kns, vns = q_all[s].cpu(), kn_all[s].cpu(), vn_all[s].cpu()
            t_s = time.perf_counter()
            for i in range(layers_cpu):
                kc, vc = state[i]
                if uniform:
                    kc, vc = ref.dynamic_layer_update(kc, vc, kns[i], vns[i])
                    ref.sdpa_decode(qs[i], kc, vc, SM_SCALE, G)
                else:
                    kc, vc = list(kc), list(vc)
                    for b in range(B):
                        kb, vb = ref.dynamic_layer_update(kc[b][None], vc[b][None], kns[i, b : b + 1],
                                                          vns[i, b : b + 1])
                        ref.sdpa_decode(qs[i, b : b + 1], kb, vb, SM_SCALE, G)
                        kc[b], vc[b] = kb[0], vb[0]
                state[i] = (kc, vc)
            return time.perf_counter() - t_s

        step_times = []
        budget_t0 = time.perf_counter()
        for r in range(64):
            if not growing:
                state[:] = init
            step_times.append(cpu_step(r if growing else 0))
            if len(step_times) >= 2 and (time.perf_counter() - budget_t0 > args.cpu_baseline_seconds
                                         or (growing and r + 1 >= min(K, n_graph_steps))):
                break
        cpu_us = sum(step_times[1:]) / (len(step_times) - 1) * 1e6 * w.layers / layers_cpu
        cpu = {
            "value": round(cpu_us, 1),
            "unit": "us/step",
            "cores": threads,
            "cores_note": "torch threads = every core this process may run on (affinity mask, capped by the "
                          "cgroup CPU quota); the host's total is host_cpu_count",
            **core_info,
            "omp_num_threads_env": os.environ.get("OMP_NUM_THREADS"),
            "kind": "port",
            "sample": (f"first {len(step_times)} decode steps" if growing else f"{len(step_times)} repeats of the step")
                      + f" of this workload ({w.layers} layer(s) each: torch.cat append + SDPA over repeat_kv"
                      + ("" if uniform else " per sequence") + ", bf16"
                      + (" over the dequantised fp8 cache" if w.fp8 else "")
                      + f", torch {torch.__version__} eager), mean of {'steps' if growing else 'repeats'} "
                      + f"2..{len(step_times)}"
                      + ("" if layers_cpu == w.layers else f"; {layers_cpu} of the {w.layers} layers timed, scaled"),
            "cpu_model": cpu_info(),
            "cpu_capability": torch.backends.cpu.get_cpu_capability(),
            "tokens_per_s": round(B / (cpu_us * 1e-6), 1),
        }

    # HBM traffic per launch of the fused kernel, from the copy-calibrated FETCH_SIZE / WRITE_SIZE profile runs
    traffic = None
    traffic_file = os.path.join(ROOT, "profiles", f"decode_append_{args.config}_hbm_traffic.json")
    if path == "fused" and os.path.exists(traffic_file):
        with open(traffic_file) as f:
            traffic = json.load(f)

    kv_name = "fp8" if w.fp8 else "bf16"
    describe = {
        "c1": "B=1, 1 layer, 1024 cached, append 1 + attend over 1025",
        "c2": "B=8, 28 layers, prefill 2048, 128 steps of append 1 + attend",
        "c3": "B=1, 1 layer, 32768 cached, 64 steps of append 1 + attend",
        "c4": "B=64, 28 layers, ragged lengths U{512..4096}, one step",
        "c5": "B=32, 1 layer, ragged lengths U{256..8192}, paged (16-token pages) fp8 e4m3 + fp32 scales, one step",
    }[args.config]
    metric = ("us/decode-step & achieved HBM GB/s (% of 8 TB/s), B=8 L=2048 28 layers" if args.config == "c2"
              else f"us/decode-step & achieved HBM GB/s (% of 8 TB/s), {args.config}")
    result = {
        "metric": metric,
        "value": round(us_per_step, 2),
        "unit": "us/step",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(us_per_step / 1e3, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": kv_name,
        "data": "synthetic (seeded N(0,1)" + (", K x0.5" if w.k_scale != 1.0 else "")
                + (", 1% outliers +-8" if w.outlier_frac else "") + ")",
        "config": {
            "workload": f"qwen3vl-2b decode: 16q/8kv heads, head_dim 128, {kv_name} KV, {describe}",
            "name": args.config, "batch": B, "layers": w.layers, "cache_instances": NL,
            "cached_before": base[0] if w.len_range is None else [lo, hi],
            "q_heads": HQ, "kv_heads": HKV, "head_dim": D, "paged": w.paged, "page_size": page,
            "mode": args.mode, "capture": args.capture, "path": path,
            "tokens_per_split": plan.tokens_per_split, "num_splits": plan.num_splits,
        },
        "us_per_step_median": round(percentile(per_step_us, 0.5) * layer_weight, 2),
        "us_per_step_p90": round(percentile(per_step_us, 0.9) * layer_weight, 2),
        "tokens_per_s": round(B / (us_per_step * 1e-6), 1),
        "hbm_bytes_per_step": int(bytes_per_step),
        "hbm_gbps": round(gbps, 1),
        "hbm_frac": round(gbps / HBM_PEAK_GBPS, 4),
        "wall_ms": round(wall_ms, 3),
        f"{other}_path_us_per_step": None if other_us is None else round(other_us, 2),
        ("per_step_capture_us_per_step" if once else "single_capture_us_per_step"):
            None if other_capture_us is None else round(other_capture_us, 2),
        "fused_qk_path_us_per_step": None if qk_us is None else round(qk_us, 2),
        "fused_with_block_pool_us_per_step": None if pool_us is None else round(pool_us, 2),
        "roofline": {
            "bound": "hbm",
            "kernel": f"decode_attn_kernel<bf16,{kv_name},D=128,G=2,{'paged' if w.paged else 'contiguous'},"
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
                f"(profiles/decode_append_{args.config}_hbm_traffic.md)"),
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
