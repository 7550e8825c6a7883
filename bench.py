#!/usr/bin/env python3
"""MoE-layer throughput of the gfx950 MXFP4 MoE block on one MI355X.

Default workload: GPT-OSS-20B-shape MoE decode at
batch 64 over all 24 layers' expert weights resident in HBM (~10 GB MXFP4),
32 experts, top-4, router logits injected so expert popularity follows
Zipf(1.1). A step is one pass of the 64-token batch through the 24 MoE layers;
`value` is layer-tokens/s (tokens through one MoE layer per second, the unit of
BASELINE.md's CPU figures). Inputs and weights are resident before timing.

Prints one JSON line. The per-kernel roofline uses the library's hipEvent
profiler on the stream the kernels run on; `cpu_baseline` times the oracle's
faithful Auto lane (x8 AVX2 GEMV for single-row buckets, scalar matmul for
multi-row buckets, one thread, as moe_batch runs it) on layer 0 of the same
batch after checking that the GPU's layer-0 output is bit-identical to it.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "gpt-oss-rs_amd"))

import gossmx as G  # noqa: E402
import synth  # noqa: E402

METRIC = "MoE-layer tokens/s + achieved HBM GB/s (% of peak), 20B shape bs=1/64"
HBM_PEAK_GBPS = 8000.0
GATE_UP_BYTES = 5760 * 90 * 17   # 8,812,800 B per expert
DOWN_BYTES = 2880 * 90 * 17      # 4,406,400 B per expert
SEED = 20251201


def stable_topk_sets(logits: np.ndarray, k: int) -> np.ndarray:
    """Selected experts per row (descending logit, ties to the lower index)."""
    order = np.lexsort((np.arange(logits.shape[1])[None, :].repeat(logits.shape[0], 0), -logits), axis=1)
    return order[:, :k]


def build_workload(ctx, layers: int, experts: int, m: int, zipf_s: float, rng):
    import torch

    dev = torch.device("cuda", 0)
    x = synth.hidden_rows(rng, m)
    x_dev = torch.from_numpy(x.view(np.int16)).to(dev)
    state = []
    for layer in range(layers):
        gu = G.Weights.generate(ctx, SEED, 16 * layer + 4, experts, 5760, 90)
        dn = G.Weights.generate(ctx, SEED, 16 * layer + 5, experts, 2880, 90)
        p = synth.dense_layer_params(np.random.default_rng(SEED + layer), experts)
        moe = G.MoeLayer(ctx, experts, 2880, 2880, 4, p["router_weight"], p["router_bias"], gu, p["gate_up_bias"],
                         dn, p["down_bias"])
        logits = synth.zipf_logits(rng, m, experts, 4, zipf_s)
        state.append({
            "moe": moe, "gu": gu, "dn": dn, "params": p, "logits": logits,
            "logits_dev": torch.from_numpy(logits).to(dev),
            "out_dev": torch.empty((m, 2880), dtype=torch.float32, device=dev),
            "touched": len(np.unique(stable_topk_sets(logits, 4))),
        })
    return x, x_dev, state


def cpu_baseline(x, st0, layer_out_gpu, threads: int):
    """Oracle lanes on layer 0 of the batch; checks GPU bits first."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    p = st0["params"]
    host = O.MoeLayerHost(p["router_weight"], p["router_bias"], O.gen_mxfp4(SEED, 4, 32, 5760, 90),
                          p["gate_up_bias"], O.gen_mxfp4(SEED, 5, 32, 2880, 90), p["down_bias"], 32, 2880, 2880, 4)
    m = x.shape[0]
    t0 = time.perf_counter()
    ref = O.moe_batch(host, x, injected_logits=st0["logits"], auto_lane=True, threads=1)
    t_auto = time.perf_counter() - t0
    assert ref["status"] == O.OK
    same = bool((ref["output"].view(np.uint32) == layer_out_gpu.view(np.uint32)).all())
    t0 = time.perf_counter()
    ref_mt = O.moe_batch(host, x, injected_logits=st0["logits"], auto_lane=True, threads=threads)
    t_all = time.perf_counter() - t0
    same_mt = bool((ref_mt["output"].view(np.uint32) == ref["output"].view(np.uint32)).all())
    return {
        "value": m / t_auto, "unit": "layer-tokens/s", "cores": 1, "kind": "port",
        "sample": f"layer 0 of the batch ({m} tokens, {4 * m} routes), oracle Auto lane (x8 AVX2 GEMV at M=1, "
                  f"scalar matmul for M>1 buckets, cpu_runner.rs:3409-3416), {t_auto:.1f} s",
        "gpu_bits_equal": same,
        "all_cores": {"value": m / t_all, "cores": threads, "seconds": round(t_all, 2), "bits_equal": same_mt},
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--layers", type=int, default=24)
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--zipf", type=float, default=1.1)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-graph", dest="graph", action="store_false",
                    help="time eager launches instead of the captured HIP graph of the step")
    ap.add_argument("--cpu-threads", type=int, default=min(16, os.cpu_count() or 1))
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="only run a device-to-device copy of this many MiB (calibrates HBM byte counters)")
    args = ap.parse_args()
    if args.copy_probe_mib:
        import torch

        src = torch.empty(args.copy_probe_mib << 20, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": args.copy_probe_mib << 20}))
        return 0
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures the single-GPU MoE block only; multi-GPU runs are not part of this build "
              "(expert-parallel sharding is a design note, not an implementation)", file=sys.stderr)
        return 2

    import torch

    torch.cuda.init()
    stream = torch.cuda.Stream()
    rng = np.random.default_rng(SEED)
    ctx = G.Context(0, stream=stream.cuda_stream)
    ctx.selftest()
    x, x_dev, state = build_workload(ctx, args.layers, 32, args.batch, args.zipf, rng)
    torch.cuda.synchronize()

    def step():
        for st in state:
            st["moe"].forward_device(x_dev, args.batch, st["out_dev"], injected_logits=st["logits_dev"])

    def timed(fn) -> float:
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record(stream)
        for _ in range(args.steps):
            fn()
        end.record(stream)
        torch.cuda.synchronize()
        ctx.synchronize()  # raises if a device-side check failed
        return start.elapsed_time(end)

    graph = None
    with torch.cuda.stream(stream):
        for _ in range(args.warmup):
            step()
        ctx.synchronize()
        # Eager pass with the library's hipEvent profiler on the kernels' stream:
        # per-kernel durations for the roofline and the stage breakdown.
        ctx.profile(True)
        ctx.profile_reset()
        ms_eager = timed(step)
        prof = ctx.profile_read()
        ctx.profile(False)
        if args.graph:
            # The same 24-layer step captured once as a HIP graph and replayed:
            # identical kernels and arguments, without per-launch gaps.
            ctx.capture_begin()
            step()
            graph = ctx.capture_end()
            for _ in range(args.warmup):
                graph.launch()
            ctx.synchronize()
            ms_total = timed(graph.launch)
        else:
            ms_total = ms_eager

    ms_step = ms_total / args.steps
    layer_tokens = args.batch * args.layers
    touched = sum(st["touched"] for st in state)
    weight_bytes = touched * (GATE_UP_BYTES + DOWN_BYTES)
    bias_bytes = touched * (5760 + 2880) * 4
    act_bytes = args.layers * args.batch * (2880 * 2 + 32 * 4 + 2880 * 4)
    step_bytes = weight_bytes + bias_bytes + act_bytes
    gbps = step_bytes / (ms_step * 1e-3) / 1e9

    gu = prof["gate_up"]
    gu_avg_ms = gu["total_ms"] / max(gu["launches"], 1)
    gu_bytes_per_launch = touched * GATE_UP_BYTES / args.layers
    gu_gbps = gu_bytes_per_launch / (gu_avg_ms * 1e-3) / 1e9

    out0 = state[0]["out_dev"].cpu().numpy()
    result = {
        "metric": METRIC,
        "value": layer_tokens / (ms_step * 1e-3),
        "unit": "layer-tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "mxfp4xq8->f32",
        "data": "synthetic (seeded; random-init GPT-OSS-20B MoE weights generated on the device)",
        "config": {
            "workload": "configs[1]: GPT-OSS-20B-shape MoE decode, batch 64, all 24 layers resident, "
                        f"Zipf({args.zipf}) injected routing, top-4 of 32 experts",
            "batch": args.batch, "layers": args.layers, "experts": 32, "top_k": 4, "hidden": 2880,
            "intermediate": 2880, "touched_experts": touched,
        },
        "tokens_per_s_through_all_layers": args.batch / (ms_step * 1e-3),
        "hbm_gbps": gbps,
        "hbm_frac": gbps / HBM_PEAK_GBPS,
        "algorithmic_bytes_per_step": step_bytes,
        "roofline": {
            "kernel": "gemm_kernel<kGateUp> (gate_up MXFP4 GEMM + SwiGLU + down-input quantization)",
            "bound": "hbm", "achieved": gu_gbps, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "frac": gu_gbps / HBM_PEAK_GBPS, "traffic": None,
            "avg_launch_ms": gu_avg_ms, "bytes_per_launch": gu_bytes_per_launch,
        },
        "stage_ms_per_step": {k: v["total_ms"] / args.steps for k, v in prof.items() if v["launches"]},
        "launch": "hip-graph" if args.graph else "eager",
        "eager_ms_per_step": ms_eager / args.steps,
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(x, state[0], out0, args.cpu_threads)
    if graph is not None:
        graph.close()
    for st in state:
        st["moe"].close()
        st["gu"].close()
        st["dn"].close()
    ctx.close()
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
