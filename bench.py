#!/usr/bin/env python3
"""MoE-layer throughput of the gfx950 MXFP4 MoE block on one MI355X.

Default workload: GPT-OSS-20B-shape MoE decode at
batch 64 over all 24 layers' expert weights resident in HBM (~10 GB MXFP4),
32 experts, top-4, router logits injected so expert popularity follows
Zipf(1.1). A step is one pass of the batch through every layer; `value` is
layer-tokens/s (tokens through one MoE layer per second, the unit of
BASELINE.md's CPU figures). Inputs and weights are resident before timing.

`--config` selects the other measured workloads of the same metric:
  0  decode of 1 token, router computed, rotating over 12 layer copies
     (5 GB of weights, far beyond the 256 MB Infinity Cache);
  2  prefill of 2048 tokens through one layer, near-uniform top-4
     (MFMA roofline: 407.69 GFLOP per layer);
  4  GPT-OSS-120B shape: 128 experts, all 36 layers resident (61 GB),
     decode batch 256 with Zipf(1.2) routing.

  4 --prefill  the same 120B-shape layers, prefill of 4096 tokens with
     near-uniform routing (MFMA roofline).

With no --config (and no overrides) the line also carries configs[0]'s
figures under "configs0": the same measurement of the 1-token workload
(us_per_layer, value, roofline with its own traffic probe, host-memory rate
and CPU baseline), run after the configs[1] measurement; `value` stays
configs[1]'s.

Prints one JSON line. The per-kernel roofline uses the library's hipEvent
profiler on the stream the kernels run on (the GEMM launches record their own
start and stop events, so the interval is the kernel's execution). For every
workload roofline.traffic (HBM bytes per gate_up launch) is measured in the
same run: two child
processes under rocprofv3 --pmc (FETCH_SIZE, then WRITE_SIZE) run a 1 GiB
device copy, which calibrates each counter, and then the workload, before
this process touches the GPU (--no-traffic skips them). `cpu_baseline` times
the oracle's faithful Auto lane (x8 AVX2 GEMV for single-row buckets, scalar
matmul for multi-row buckets, one thread, as moe_batch runs it) and its
fastest forced panel lane on a bounded sample of layer 0 of the same batch,
after checking that the GPU's rows are bit-identical to it (and the last
layer's rows on the forced lane); the exit status is 1 if any bit differs.
"""
from __future__ import annotations

import argparse
import csv
import gc
import glob
import json
import os
import re
import shutil
import subprocess
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "gpt-oss-rs_amd"))

import gossmx as G  # noqa: E402
import synth  # noqa: E402

METRIC = "MoE-layer tokens/s + achieved HBM GB/s (% of peak), 20B shape bs=1/64"
HBM_PEAK_GBPS = 8000.0
F16_MFMA_PEAK_TFLOPS = 2500.0     # dense f16 MFMA, the instruction the expert GEMM issues
MXFP4_MFMA_PEAK_TFLOPS = 10100.0  # dense MXFP4 MFMA, the peak BASELINE.json's prefill target names
HIDDEN = INTER = 2880
BLOCKS = HIDDEN // 32
GATE_UP_BYTES = 2 * INTER * BLOCKS * 17   # 8,812,800 B per expert
DOWN_BYTES = HIDDEN * BLOCKS * 17         # 4,406,400 B per expert
SEED = 20251201
RMS_EPS = 1e-5  # GPT-OSS rms_norm_eps
COPY_PROBE_BYTES = 1 << 30  # device copy that calibrates the HBM byte counters
GATE_UP_KERNEL = re.compile(r"gemm_kernel<.*>, 1, (true|false)>|gemv_kernel<1, \d+, \d+>|route_gemv_kernel")

CONFIGS = {
    0: {"batch": 1, "layers": 12, "experts": 32, "routing": "router", "zipf": None, "roofline": "hbm",
        "workload": "configs[0]: GPT-OSS-20B-shape MoE decode, 1 token, router computed, rotating over {layers} "
                    "layer copies resident (weights far beyond the 256 MB Infinity Cache), top-4 of 32 experts",
        "sample_rows": 1},
    1: {"batch": 64, "layers": 24, "experts": 32, "routing": "zipf", "zipf": 1.1, "roofline": "hbm",
        "workload": "configs[1]: GPT-OSS-20B-shape MoE decode, batch {batch}, all {layers} layers resident, "
                    "Zipf({zipf}) injected routing, top-4 of 32 experts",
        "sample_rows": 64},
    2: {"batch": 2048, "layers": 1, "experts": 32, "routing": "uniform", "zipf": None, "roofline": "mfma",
        "workload": "configs[2]: GPT-OSS-20B-shape MoE prefill, {batch} tokens, {layers} layer, near-uniform "
                    "injected routing, top-4 of 32 experts",
        "sample_rows": 32},
    4: {"batch": 256, "layers": 36, "experts": 128, "routing": "zipf", "zipf": 1.2, "roofline": "hbm",
        "workload": "configs[4]: GPT-OSS-120B-shape MoE decode, batch {batch}, all {layers} layers resident, "
                    "Zipf({zipf}) injected routing, top-4 of 128 experts",
        "sample_rows": 32},
}
# configs[4]'s second workload (--config 4 --prefill).
PREFILL_4 = {"batch": 4096, "layers": 36, "experts": 128, "routing": "uniform", "zipf": None, "roofline": "mfma",
             "workload": "configs[4]: GPT-OSS-120B-shape MoE prefill, {batch} tokens, all {layers} layers resident, "
                         "near-uniform injected routing, top-4 of 128 experts",
             "sample_rows": 16}


def stable_topk_sets(logits: np.ndarray, k: int) -> np.ndarray:
    """Selected experts per row (descending logit, ties to the lower index)."""
    order = np.lexsort((np.arange(logits.shape[1])[None, :].repeat(logits.shape[0], 0), -logits), axis=1)
    return order[:, :k]


def build_workload(ctx, cfg: dict, rng):
    import torch

    dev = torch.device("cuda", 0)
    m, E = cfg["batch"], cfg["experts"]
    x = synth.hidden_rows(rng, m)
    x_dev = torch.from_numpy(x.view(np.int16)).to(dev)
    state = []
    for layer in range(cfg["layers"]):
        gu = G.Weights.generate(ctx, SEED, 16 * layer + 4, E, 2 * INTER, BLOCKS)
        dn = G.Weights.generate(ctx, SEED, 16 * layer + 5, E, HIDDEN, BLOCKS)
        p = synth.dense_layer_params(np.random.default_rng(SEED + layer), E)
        moe = G.MoeLayer(ctx, E, HIDDEN, INTER, 4, p["router_weight"], p["router_bias"], gu, p["gate_up_bias"],
                         dn, p["down_bias"])
        if cfg["routing"] == "zipf":
            logits = synth.zipf_logits(rng, m, E, 4, cfg["zipf"])
        elif cfg["routing"] == "uniform":
            logits = synth.uniform_logits(rng, m, E)
        else:
            logits = None
        state.append({
            "moe": moe, "gu": gu, "dn": dn, "params": p, "logits": logits,
            "logits_dev": None if logits is None else torch.from_numpy(logits).to(dev),
            "out_dev": torch.empty((m, HIDDEN), dtype=torch.float32, device=dev),
            "sel_dev": torch.empty((m, 4), dtype=torch.int32, device=dev),
            # --residual: the layer's post-attention norm weight and the next residual stream
            "norm_dev": torch.from_numpy((1.0 + 0.25 * rng.standard_normal(HIDDEN)).astype(np.float32)).to(dev),
            "next_dev": torch.empty((m, HIDDEN), dtype=torch.int16, device=dev),
        })
    return x, x_dev, state


def host_layer(O, cfg: dict, st, layer: int):
    p = st["params"]
    E = cfg["experts"]
    return O.MoeLayerHost(p["router_weight"], p["router_bias"], O.gen_mxfp4(SEED, 16 * layer + 4, E, 2 * INTER, BLOCKS),
                          p["gate_up_bias"], O.gen_mxfp4(SEED, 16 * layer + 5, E, HIDDEN, BLOCKS), p["down_bias"], E,
                          HIDDEN, INTER, 4)


def cpu_baseline(cfg: dict, x, state, threads: int):
    """Oracle lanes on a bounded sample of rows: layer 0 on the Auto lane (one
    thread, then all threads) and on the host's fastest forced panel lane, and
    the last layer on the forced lane over all threads; each result is
    checked bit for bit against the GPU's rows first."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    st0 = state[0]
    layer_out_gpu = st0["out_dev"].cpu().numpy()
    host = host_layer(O, cfg, st0, 0)
    n = min(cfg["sample_rows"], x.shape[0])
    rows = np.linspace(0, x.shape[0] - 1, n).astype(np.int64) if n < x.shape[0] else np.arange(n)
    xs = x[rows]
    inj = None if st0["logits"] is None else st0["logits"][rows]
    t0 = time.perf_counter()
    ref = O.moe_batch(host, xs, injected_logits=inj, auto_lane=True, threads=1)
    t_auto = time.perf_counter() - t0
    assert ref["status"] == O.OK
    same = bool((ref["output"].view(np.uint32) == layer_out_gpu[rows].view(np.uint32)).all())
    t0 = time.perf_counter()
    ref_mt = O.moe_batch(host, xs, injected_logits=inj, auto_lane=True, threads=threads)
    t_all = time.perf_counter() - t0
    same_mt = bool((ref_mt["output"].view(np.uint32) == ref["output"].view(np.uint32)).all())
    lane = O.fastest_lane()
    lane_name = {O.LANE_AVX512_8X8: "avx512-vnni 8x8 panel", O.LANE_AVX2_4X8: "avx2 4x8 panel",
                 O.LANE_SCALAR: "scalar"}[lane]
    t0 = time.perf_counter()
    ref_lane = O.moe_batch(host, xs, injected_logits=inj, lane=lane, threads=1)
    t_lane = time.perf_counter() - t0
    same_lane = bool((ref_lane["output"].view(np.uint32) == ref["output"].view(np.uint32)).all())
    last = len(state) - 1
    same_last = None
    if last > 0:
        stl = state[last]
        inj_l = None if stl["logits"] is None else stl["logits"][rows]
        ref_l = O.moe_batch(host_layer(O, cfg, stl, last), xs, injected_logits=inj_l, lane=lane, threads=threads)
        same_last = bool((ref_l["output"].view(np.uint32) ==
                          stl["out_dev"].cpu().numpy()[rows].view(np.uint32)).all())
    whole = "the whole batch" if n == x.shape[0] else f"{n} evenly spaced rows of the {x.shape[0]}-token batch"
    return {
        "value": n / t_auto, "unit": "layer-tokens/s", "cores": 1, "kind": "port",
        "sample": f"layer 0, {whole} ({n} tokens, {4 * n} routes), oracle Auto lane (x8 AVX2 GEMV at M=1, "
                  f"scalar matmul for M>1 buckets, cpu_runner.rs:3409-3416), {t_auto:.1f} s",
        "gpu_bits_equal": same,
        "all_cores": {"value": n / t_all, "cores": threads, "seconds": round(t_all, 2), "bits_equal": same_mt},
        "forced_lane": {"lane": lane_name, "value": n / t_lane, "cores": 1, "seconds": round(t_lane, 2),
                        "bits_equal": same_lane,
                        "source": "x86.rs:449-520 (AVX2 4x8), 660-732 (AVX-512-VNNI 8x8) restated in the oracle"},
        "last_layer_bits_equal": same_last,
    }


def probe_traffic(args, config=None) -> dict:
    """HBM bytes per gate_up launch, measured in this run: two child processes
    under rocprofv3 --pmc (FETCH_SIZE, then WRITE_SIZE: the counters do not
    fit one pass), each running a 1 GiB device copy and then the workload
    (--traffic-probe). Each counter is scaled by copy bytes / what it reads for
    the copy; traffic = FETCH x that + WRITE x that, averaged over the gate_up
    dispatches. Runs before this process touches the GPU."""
    rp = shutil.which("rocprofv3")
    if rp is None:
        return {"traffic": None, "traffic_source": "not measured: rocprofv3 not found"}
    env = dict(os.environ, TMPDIR="/tmp")
    per, codes = {}, {}
    for ctr in ("FETCH_SIZE", "WRITE_SIZE"):
        d = tempfile.mkdtemp(prefix="gossmx_pmc_", dir="/tmp")
        cmd = [rp, "--pmc", ctr, "--output-format", "csv", "-d", d, "-o", "p", "--", sys.executable,
               os.path.abspath(__file__), "--traffic-probe", "--config", str(args.config if config is None else config)]
        if config is None:
            for key in ("layers", "batch", "zipf"):
                if getattr(args, key) is not None:
                    cmd += [f"--{key}", str(getattr(args, key))]
            if args.prefill:
                cmd.append("--prefill")
        try:
            # The child prints "probe done" as its last line; its exit status
            # and that line are recorded in traffic_source.
            proc = subprocess.run(cmd, timeout=240, stdout=subprocess.PIPE, stderr=subprocess.DEVNULL, env=env,
                                  cwd="/tmp", text=True)
        except subprocess.TimeoutExpired:
            return {"traffic": None, "traffic_source": f"not measured: rocprofv3 --pmc {ctr} pass timed out"}
        finished = "probe done" in (proc.stdout or "")
        codes[ctr] = f"exit {proc.returncode}" + ("" if finished else ", the workload did not finish")
        files = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)
        if not files or not finished:
            return {"traffic": None,
                    "traffic_source": f"not measured: rocprofv3 --pmc {ctr} ({codes[ctr]}) wrote no counters"
                    if not files else f"not measured: rocprofv3 --pmc {ctr} ({codes[ctr]})"}
        copy_kib, gate_up = 0.0, []
        with open(files[0]) as f:
            for row in csv.DictReader(f):
                if row.get("Counter_Name") != ctr:
                    continue
                name, val = row.get("Kernel_Name", ""), float(row.get("Counter_Value", "nan"))
                if "copyBuffer" in name:
                    copy_kib = max(copy_kib, val)
                elif GATE_UP_KERNEL.search(name):
                    gate_up.append(val)
        shutil.rmtree(d, ignore_errors=True)
        if copy_kib <= 0 or not gate_up:
            return {"traffic": None, "traffic_source": f"not measured: {ctr} rows for the copy or gate_up missing"}
        per[ctr] = (float(np.mean(gate_up)), copy_kib, len(gate_up))
    (fk, fc, n), (wk, wc, _) = per["FETCH_SIZE"], per["WRITE_SIZE"]
    f_scale, w_scale = COPY_PROBE_BYTES / (fc * 1024), COPY_PROBE_BYTES / (wc * 1024)
    traffic = fk * 1024 * f_scale + wk * 1024 * w_scale
    return {"traffic": traffic,
            "traffic_source": f"rocprofv3 --pmc FETCH_SIZE then WRITE_SIZE in this run, {n} gate_up dispatches: "
                              f"{fk:.0f} KiB x {f_scale:.3f} + {wk:.0f} KiB x {w_scale:.3f} (scales from a 1 GiB "
                              f"device copy: FETCH {fc:.0f} KiB, WRITE {wc:.0f} KiB); profiler children: "
                              f"FETCH {codes['FETCH_SIZE']}, WRITE {codes['WRITE_SIZE']}"}


def run_traffic_probe(args, cfg: dict) -> int:
    """Child of probe_traffic: a 1 GiB device copy, then one untimed pass and
    one step of the workload (two layers at most), eager."""
    import torch

    torch.cuda.init()
    src = torch.empty(COPY_PROBE_BYTES, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    cfg = dict(cfg, layers=min(cfg["layers"], 2))
    ctx = G.Context(0)
    x, x_dev, state = build_workload(ctx, cfg, np.random.default_rng(SEED))
    m = cfg["batch"]
    for _ in range(2):
        for st in state:
            st["moe"].forward_device(x_dev, m, st["out_dev"], injected_logits=st["logits_dev"])
    ctx.synchronize()
    for st in state:
        st["moe"].close()
        st["gu"].close()
        st["dn"].close()
    ctx.close()
    release_torch()
    print("probe done", flush=True)
    return 0


def release_torch():
    """Ends the process's GPU work before the interpreter exits: waits for the
    device and returns torch's cached blocks, so that nothing of this program
    is in flight or cached while the runtime (and a profiler's library, when
    one is loaded) tears down."""
    import torch

    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def run_model(args) -> int:
    """the random-init GPT-OSS-20B forward, a 63-token prefill and 8
    greedy decode steps through gossmx_model_*: norms, RoPE, attention and the
    KV cache on host threads, the Q/K/V/O projections, lm_head and every
    layer's MoE block on the GPU. Times whole generations and splits
    them into dense and MoE wall time; the CPU baseline is the oracle's
    whole-model run (dense path and MoE on the host) on the same weights, whose
    tokens and logits bits must equal the product's."""
    import torch

    torch.cuda.init()
    ctx = G.Context(0)
    ctx.selftest()
    layers = args.layers or 24
    cfg = dict(G.GPT_OSS_20B, layers=layers, context_cap=4096)
    gen = torch.Generator(device="cuda:0")
    gen.manual_seed(SEED)

    def normal(n, std):
        t = torch.randn(n, generator=gen, device="cuda:0", dtype=torch.float32).mul_(std).to(torch.bfloat16)
        return t.view(torch.int16).cpu().numpy().view(np.uint16)

    w = synth.model_weights(cfg, normal)
    rng = np.random.default_rng(SEED)
    keep, dense_layers = [], []
    for i, L in enumerate(w["layers"]):
        gu = G.Weights.generate(ctx, SEED, 16 * i + 4, 32, 2 * INTER, BLOCKS)
        dn = G.Weights.generate(ctx, SEED, 16 * i + 5, 32, HIDDEN, BLOCKS)
        p = synth.dense_layer_params(rng, 32)
        moe = G.MoeLayer(ctx, 32, HIDDEN, INTER, 4, p["router_weight"], p["router_bias"], gu, p["gate_up_bias"], dn,
                         p["down_bias"])
        keep.append((gu, dn, moe, p))
        dense_layers.append(dict(L, moe=moe))
    model = G.Model(ctx, G.model_config(threads=args.cpu_threads, **cfg), w["embedding"], w["final_norm"],
                    w["lm_head"], dense_layers)
    prompt = rng.integers(0, cfg["vocab"], 63).astype(np.uint32)
    decode_steps = 8
    for _ in range(args.warmup):
        model.generate(prompt, decode_steps)
    d0, m0 = model.times()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        tokens, logits = model.generate(prompt, decode_steps)
    wall = (time.perf_counter() - t0) / args.steps
    d1, m1 = model.times()
    dense_s, moe_s = (d1 - d0) / args.steps, (m1 - m0) / args.steps
    forwards = prompt.size + decode_steps
    line = {
        "metric": "configs[3] GPT-OSS-20B forward: token forwards/s (63-token prefill + 8 greedy decodes)",
        "value": forwards / wall, "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": wall * 1e3, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16 projections and lm_head (GPU), bf16 attention (host) + MXFP4 x residual-Q8 MoE (GPU)",
        "data": "synthetic (random-init weights, random prompt)",
        "config": {"workload": f"configs[3]: random-init GPT-OSS-20B, {layers} layers, 63-token prefill + "
                               f"{decode_steps} greedy decode steps, projections on the GPU, attention on {args.cpu_threads} host threads",
                   "layers": layers, "prompt": int(prompt.size), "decode_steps": decode_steps},
        "dense_s": dense_s, "moe_s": moe_s, "moe_share": moe_s / wall, "greedy_tokens": tokens.tolist(),
        "roofline": None, "cpu_baseline": None,
    }
    if not args.no_cpu_baseline:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle as O

        for L, (gu, dn, moe, p) in zip(w["layers"], keep):
            L["moe_host"] = O.MoeLayerHost(p["router_weight"], p["router_bias"], gu.export_canonical(),
                                           p["gate_up_bias"], dn.export_canonical(), p["down_bias"], 32, HIDDEN,
                                           INTER, 4)
        host = O.ModelHost(cfg, w["embedding"], w["final_norm"], w["lm_head"], w["layers"])
        t0 = time.perf_counter()
        st, want_tokens, want_logits = O.model_generate(host, prompt, decode_steps, threads=args.cpu_threads)
        cpu_wall = time.perf_counter() - t0
        line["cpu_baseline"] = {
            "value": forwards / cpu_wall, "unit": "tokens/s", "cores": args.cpu_threads, "kind": "port",
            "sample": f"the whole generation once: oracle dense path and MoE (Auto lane) on the host, "
                      f"{args.cpu_threads} threads for projections and expert matmuls, {cpu_wall:.1f} s",
            "greedy_match": bool(st == 0 and (want_tokens == tokens).all()),
            "logits_bits_equal": bool(st == 0 and (want_logits.view(np.uint32) == logits.view(np.uint32)).all()),
        }
    model.close()
    for gu, dn, moe, _ in keep:
        moe.close()
        gu.close()
        dn.close()
    ctx.close()
    release_torch()
    print(json.dumps(line))
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", type=int, default=None, choices=sorted(CONFIGS) + [3],
                    help="BASELINE.json configs[] index of the workload (default 1; with no --config the line "
                         "also carries configs[0]'s figures under configs0)")
    ap.add_argument("--layers", type=int, default=None, help="override the config's layer count")
    ap.add_argument("--batch", type=int, default=None, help="override the config's batch")
    ap.add_argument("--zipf", type=float, default=None, help="override the config's Zipf exponent")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--host-steps", type=int, default=3,
                    help="steps of the host-memory (PCIe-inclusive) rate reported beside value; 0 skips it")
    ap.add_argument("--residual", action="store_true",
                    help="time gossmx_moe_forward_residual (post-attention RMSNorm + block + residual add) "
                         "instead of the block alone; no CPU baseline")
    ap.add_argument("--no-graph", dest="graph", action="store_false",
                    help="time eager launches instead of the captured HIP graph of the step")
    ap.add_argument("--cpu-threads", type=int, default=min(16, os.cpu_count() or 1))
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="only run a device-to-device copy of this many MiB (calibrates HBM byte counters)")
    ap.add_argument("--prefill", action="store_true",
                    help="with --config 4: the 4096-token prefill workload instead of decode 256")
    ap.add_argument("--no-traffic", action="store_true",
                    help="skip the rocprofv3 --pmc passes that measure roofline.traffic")
    ap.add_argument("--traffic-probe", action="store_true", help=argparse.SUPPRESS)
    args = ap.parse_args()
    # The default line (no --config, no overrides) also times configs[0].
    both = args.config is None and not args.residual and not args.prefill and \
        all(getattr(args, k) is None for k in ("layers", "batch", "zipf"))
    if args.config is None:
        args.config = 1
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
    if args.config == 3:
        return run_model(args)
    if args.prefill and args.config != 4:
        print("--prefill applies to --config 4 only", file=sys.stderr)
        return 2
    cfg = dict(PREFILL_4 if args.prefill else CONFIGS[args.config])
    for key in ("layers", "batch", "zipf"):
        if getattr(args, key) is not None:
            cfg[key] = getattr(args, key)
    m, E, L = cfg["batch"], cfg["experts"], cfg["layers"]
    if args.traffic_probe:
        return run_traffic_probe(args, cfg)
    # The counter passes run in child processes before this one touches the GPU.
    probe = probe0 = None
    if not args.no_traffic and not args.residual:
        probe = probe_traffic(args)
        if both:
            probe0 = probe_traffic(args, config=0)

    import torch

    torch.cuda.init()
    stream = torch.cuda.Stream()
    ctx = G.Context(0, stream=stream.cuda_stream)
    ctx.selftest()

    def measure(cfg: dict, probe, host_steps: int):
        """One workload: build, time (eager with the profiler, then graph
        replay), the host-memory rate; returns the result fields and what
        the CPU baseline and the clean-up need."""
        m, E, L = cfg["batch"], cfg["experts"], cfg["layers"]
        rng = np.random.default_rng(SEED)
        x, x_dev, state = build_workload(ctx, cfg, rng)
        torch.cuda.synchronize()

        def step():
            for st in state:
                if args.residual:
                    st["moe"].forward_residual_device(x_dev, m, st["norm_dev"], RMS_EPS, st["next_dev"],
                                                      injected_logits=st["logits_dev"])
                else:
                    st["moe"].forward_device(x_dev, m, st["out_dev"], injected_logits=st["logits_dev"])

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
            # One untimed pass that also returns the selections (touched experts).
            for st in state:
                if args.residual:
                    st["moe"].forward_residual_device(x_dev, m, st["norm_dev"], RMS_EPS, st["next_dev"],
                                                      injected_logits=st["logits_dev"], selected=st["sel_dev"])
                else:
                    st["moe"].forward_device(x_dev, m, st["out_dev"], injected_logits=st["logits_dev"],
                                             selected=st["sel_dev"])
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
                # The same step captured once as a HIP graph and replayed: identical
                # kernels and arguments, without per-launch gaps.
                ctx.capture_begin()
                step()
                graph = ctx.capture_end()
                for _ in range(args.warmup):
                    graph.launch()
                ctx.synchronize()
                ms_total = timed(graph.launch)
            else:
                ms_total = ms_eager

        # Host-memory mode (GOSSMX_MEM_HOST, the direct drop-in for Rust slices):
        # every layer call copies x and the logits in and the outputs out (one
        # copy each way), then synchronizes. PCIe-inclusive, reported beside value, never as value.
        # Python's cyclic collector is paused for the timed calls: a full
        # collection of the interpreter's objects (torch's included) takes tens of
        # ms and would land inside some call; a native caller has no such pause.
        host_ms = None
        if not args.residual and host_steps > 0:
            for st in state:  # one untimed pass (host staging buffers)
                st["moe"].forward(x, injected_logits=st["logits"])
            gc.collect()
            gc.disable()
            try:
                t0 = time.perf_counter()
                for _ in range(host_steps):
                    for st in state:
                        st["moe"].forward(x, injected_logits=st["logits"])
                host_ms = (time.perf_counter() - t0) * 1e3 / host_steps
            finally:
                gc.enable()

        sel = [st["sel_dev"].cpu().numpy() for st in state]
        if cfg["routing"] != "router":
            assert all((s == stable_topk_sets(st["logits"], 4)).all() for s, st in zip(sel, state))
        touched = sum(len(np.unique(s)) for s in sel)
        routes = m * 4

        ms_step = ms_total / args.steps
        layer_tokens = m * L
        weight_bytes = touched * (GATE_UP_BYTES + DOWN_BYTES)
        bias_bytes = touched * (2 * INTER + HIDDEN) * 4
        router_bytes = L * (E * HIDDEN * 2 + E * 4) if cfg["routing"] == "router" else 0
        act_bytes = L * m * (HIDDEN * 2 + E * 4 + HIDDEN * 4)
        step_bytes = weight_bytes + bias_bytes + router_bytes + act_bytes
        gbps = step_bytes / (ms_step * 1e-3) / 1e9

        gu = prof["gate_up"]
        gu_avg_ms = gu["total_ms"] / max(gu["launches"], 1)
        gu_bytes_per_launch = touched * GATE_UP_BYTES / L
        gu_gbps = gu_bytes_per_launch / (gu_avg_ms * 1e-3) / 1e9
        if m == 1 and cfg["routing"] == "router":
            kernel = ("route_gemv_kernel (top-k selection per work-group + block-packed MXFP4 GEMV, P=8 + SwiGLU + "
                      "down-input quantization)")
        elif m <= 4:
            kernel = (f"gemv_kernel<kGateUp, P={8 // (1 if m == 1 else 2 if m == 2 else 4)}> (block-packed small-batch "
                      "MXFP4 GEMV + SwiGLU + down-input quantization)")
        else:
            kernel = "gemm_kernel<kGateUp> (gate_up MXFP4 GEMM + SwiGLU + down-input quantization)"
        if cfg["roofline"] == "hbm":
            roofline = {"kernel": kernel, "bound": "hbm", "achieved": gu_gbps, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                        "frac": gu_gbps / HBM_PEAK_GBPS, "traffic": None, "avg_launch_ms": gu_avg_ms,
                        "bytes_per_launch": gu_bytes_per_launch}
            roofline.update(probe or {"traffic_source": "not measured (--no-traffic or --residual)"})
        else:
            flops = 2.0 * routes * (2 * INTER) * HIDDEN
            tflops = flops / (gu_avg_ms * 1e-3) / 1e12
            roofline = {"kernel": kernel, "bound": "mfma", "achieved": tflops, "peak": F16_MFMA_PEAK_TFLOPS,
                        "unit": "TFLOP/s", "frac": tflops / F16_MFMA_PEAK_TFLOPS, "traffic": None,
                        "frac_of_mxfp4_peak": tflops / MXFP4_MFMA_PEAK_TFLOPS, "mxfp4_peak": MXFP4_MFMA_PEAK_TFLOPS,
                        "avg_launch_ms": gu_avg_ms, "flops_per_launch": flops, "hbm_gbps": gu_gbps,
                        "weight_bytes_per_launch": gu_bytes_per_launch}
            roofline.update(probe or {"traffic_source": "not measured (--no-traffic or --residual)"})

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
            "dtype": "mxfp4 x residual-q8 (two integer dots per block) -> f32 holding bf16 values",
            "data": f"synthetic (seeded; random-init GPT-OSS-{'120B' if E == 128 else '20B'} MoE weights generated "
                    "on the device)",
            "config": {
                "workload": cfg["workload"].format(**cfg) + (
                    "; MoE half of the decoder layer: post-attention RMSNorm + block + residual add"
                    if args.residual else ""),
                "residual": bool(args.residual),
                "batch": m, "layers": L, "experts": E, "top_k": 4, "hidden": HIDDEN,
                "intermediate": INTER, "touched_experts": touched,
            },
            "tokens_per_s_through_all_layers": m / (ms_step * 1e-3),
            "hbm_gbps": gbps,
            "hbm_frac": gbps / HBM_PEAK_GBPS,
            "algorithmic_bytes_per_step": step_bytes,
            "roofline": roofline,
            "stage_ms_per_step": {k: v["total_ms"] / args.steps for k, v in prof.items() if v["launches"]},
            "launch": "hip-graph" if args.graph else "eager",
            "eager_ms_per_step": ms_eager / args.steps,
        }
        if host_ms is not None:
            result["host_memory"] = {
                "ms_per_step": host_ms, "value": layer_tokens / (host_ms * 1e-3), "unit": "layer-tokens/s",
                "steps": host_steps,
                "note": ("GOSSMX_MEM_HOST calls (eager launches): x and logits in one copy from pinned staging; "
                         "every CpuMoeStep output (router logits, selection, routing weights, route order, output "
                         "rows) and the device error flags written by the kernels into pinned host memory; one "
                         "synchronization per layer"),
            }
        return result, x, state, graph

    def release(state, graph):
        if graph is not None:
            graph.close()
        for st in state:
            st["moe"].close()
            st["gu"].close()
            st["dn"].close()

    result, x, state, graph = measure(cfg, probe, args.host_steps)
    bits_ok = True
    if not args.no_cpu_baseline and not args.residual:
        cb = cpu_baseline(cfg, x, state, args.cpu_threads)
        result["cpu_baseline"] = cb
        bits_ok = cb["gpu_bits_equal"] and cb["all_cores"]["bits_equal"] and cb["forced_lane"]["bits_equal"] and \
            cb["last_layer_bits_equal"] is not False
    release(state, graph)
    if both:
        # The bs=1 half of the metric, timed the same way after
        # the configs[1] line's measurement; reported beside it, not in value.
        r0, x0, state0, graph0 = measure(dict(CONFIGS[0]), probe0, args.host_steps)
        cb0 = None
        if not args.no_cpu_baseline:
            cb0 = cpu_baseline(dict(CONFIGS[0]), x0, state0, args.cpu_threads)
            bits_ok = bits_ok and cb0["gpu_bits_equal"] and cb0["all_cores"]["bits_equal"] and \
                cb0["forced_lane"]["bits_equal"] and cb0["last_layer_bits_equal"] is not False
        release(state0, graph0)
        result["configs0"] = {
            "workload": r0["config"]["workload"],
            "value": r0["value"], "unit": r0["unit"], "ms_per_step": r0["ms_per_step"],
            "us_per_layer": r0["ms_per_step"] * 1e3 / r0["config"]["layers"],
            "touched_experts": r0["config"]["touched_experts"],
            "hbm_gbps": r0["hbm_gbps"], "hbm_frac": r0["hbm_frac"],
            "roofline": r0["roofline"], "stage_ms_per_step": r0["stage_ms_per_step"],
            "host_memory": r0.get("host_memory"), "cpu_baseline": cb0,
        }
    ctx.close()
    release_torch()
    print(json.dumps(result))
    if not bits_ok:
        print("GPU rows differ from the oracle's bits (cpu_baseline)", file=sys.stderr)
        return 1
    return 0


if __name__ == "__main__":
    sys.exit(main())
