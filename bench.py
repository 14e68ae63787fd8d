"""Benchmark of the MI355X FP8 block-scaled linear on Qwen3-4B projection shapes.

Metric: FP8 block GEMM TFLOPS at M=2048 and HBM GB/s at M=8 over the four
merged Qwen3-4B projections (qkv, o_proj, gate_up, down), on one GPU.

* A step is one pass of the block GEMM over the four projections for one batch: the
  prefill step at M=2048 (``value`` = TFLOPS = sum 2MNK / sum GEMM time) and the decode
  step at M=8 (``decode.gbps`` = op-level bytes / GEMM time).  Activations are quantized
  before the timed region (the quantizer is timed separately, ``quant``) and all inputs
  are resident in HBM.
* Weights rotate through enough independent sets (> 512 MB) that no step reads weights
  that are still in the 256 MB MALL from the step before.
* Timing: each projection's launches (one per weight set) are captured in a HIP graph
  and replayed K times between two HIP events recorded on the stream the kernels run on;
  the per-launch time is the elapsed time over K x sets launches, so
  ``roofline.achieved`` is the average per-launch rate of the dominant kernel.
* ``cpu_baseline`` times the C oracle (a CPU restatement of the reference arithmetic) on
  a bounded sample: the same four projections at ``--cpu-rows`` rows.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(ROOT, "mini-inference-engine_amd"), os.path.join(ROOT, "oracle")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

PEAK_FP8_TFLOPS = 5000.0   # MI355X dense OCP-FP8 MFMA
PEAK_HBM_GBPS = 8000.0     # MI355X HBM3E
SEED = 20261008


def parse_args(argv=None):
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--prefill-m", type=int, default=2048)
    p.add_argument("--decode-m", type=int, default=8)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--cpu-rows", type=int, default=1024)
    return p.parse_args(argv)


def main(argv=None) -> int:
    args = parse_args(argv)
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the FP8 linear's sharding is a design note); run with --gpus 1", file=sys.stderr)
        return 2

    import torch

    from minillm_amd import mi355x_fp8 as fp8
    from minillm_amd.validation import (
        QWEN3_4B_PROJECTIONS, gemm_bytes, linear_flops, make_baseline_activations, make_baseline_weights,
        quant_bytes,
    )

    dev = torch.device("cuda:0")
    if not fp8.mi355x_available(dev):
        print("bench.py needs an MI355X (gfx950) GPU", file=sys.stderr)
        return 2
    torch.cuda.set_device(dev)
    projs = QWEN3_4B_PROJECTIONS
    layer_bytes = sum(p.n * p.k for p in projs)
    sets = max(2, -(-512 * 2**20 // layer_bytes) + 1)
    print(f"generating {sets} weight sets of {layer_bytes / 2**20:.1f} MiB", file=sys.stderr, flush=True)
    weights = [[make_baseline_weights(p, SEED + 1000 * s, device="cuda") for p in projs] for s in range(sets)]

    def prepare(m, outliers):
        xs, qs, out = [], [], []
        for p in projs:
            x = make_baseline_activations(m, p.k, SEED, outliers=outliers, device="cuda")
            xs.append(x)
            qs.append(fp8.quantize_mi355x_fp8_activation(x, scale_layout="kgroup"))
            out.append(torch.empty((m, p.n), dtype=torch.bfloat16, device=dev))
        return xs, qs, out

    def run_phase(m, outliers):
        """Per projection: one HIP graph of `sets` back-to-back GEMM launches (one per
        weight set), replayed `steps` times between two HIP events on the launch stream.
        Graph replay removes the host's launch gaps, so the events time the kernels."""

        xs, qs, outs = prepare(m, outliers)
        stream = torch.cuda.Stream()
        per_launch_ms, graphs = [], []
        with torch.cuda.stream(stream):
            for i, p in enumerate(projs):
                for r in range(sets):  # eager warm-up outside capture
                    fp8.launch_block_gemm(qs[i][0], weights[r][i][0], outs[i], qs[i][1], weights[r][i][1])
                stream.synchronize()
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph, stream=stream):
                    for r in range(sets):
                        fp8.launch_block_gemm(qs[i][0], weights[r][i][0], outs[i], qs[i][1], weights[r][i][1])
                graphs.append(graph)
            for i, p in enumerate(projs):
                for _ in range(args.warmup):
                    graphs[i].replay()
                start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                stream.synchronize()
                start.record(stream)
                for _ in range(args.steps):
                    graphs[i].replay()
                end.record(stream)
                end.synchronize()
                per_launch_ms.append(start.elapsed_time(end) / (args.steps * sets))
            # Quantizer timing (separate: not part of the GEMM metric).
            quant_ms = []
            for i, p in enumerate(projs):
                fp8.quantize_mi355x_fp8_activation(xs[i], scale_layout="kgroup")
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph, stream=stream):
                    for _ in range(sets):
                        fp8.quantize_mi355x_fp8_activation(xs[i], scale_layout="kgroup")
                graph.replay()
                start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                stream.synchronize()
                start.record(stream)
                for _ in range(args.steps):
                    graph.replay()
                end.record(stream)
                end.synchronize()
                quant_ms.append(start.elapsed_time(end) / (args.steps * sets))
        torch.cuda.synchronize()
        return per_launch_ms, quant_ms

    results = {}
    for phase, m, outliers in (("prefill", args.prefill_m, True), ("decode", args.decode_m, False)):
        print(f"timing {phase} M={m}", file=sys.stderr, flush=True)
        mean, quant_ms = run_phase(m, outliers)
        flops = [linear_flops(m, p.n, p.k) for p in projs]
        nbytes = [gemm_bytes(m, p.n, p.k) for p in projs]
        results[phase] = {
            "m": m,
            "step_ms": sum(mean),
            "tflops": sum(flops) / (sum(mean) * 1e9),
            "gbps": sum(nbytes) / (sum(mean) * 1e6),
            "per_proj": {p.name: {"mean_us": 1e3 * mean[i],
                                  "tflops": flops[i] / (mean[i] * 1e9), "gbps": nbytes[i] / (mean[i] * 1e6)}
                         for i, p in enumerate(projs)},
            "quant": {p.name: {"us": 1e3 * quant_ms[i], "gbps": quant_bytes(m, p.k) / (quant_ms[i] * 1e6)}
                      for i, p in enumerate(projs)},
        }

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(args.cpu_rows)

    pre, dec = results["prefill"], results["decode"]
    line = {
        "metric": "FP8 block GEMM TFLOPS @M=2048 + HBM GB/s @M=8, Qwen3-4B shapes, 1 GPU",
        "value": round(pre["tflops"], 2),
        "unit": "TFLOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(pre["step_ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8e4m3 (fp32 accumulate, bf16 out)",
        "data": "synthetic: seeded N(0,1) bf16 activations (1% outlier channels x20 at M=2048), "
                "N(0,0.02) weights block-quantized to e4m3 with 128x128 fp32 scales",
        "config": {"workload": "Qwen3-4B merged projections qkv/o_proj/gate_up/down; prefill M=2048 "
                               "(value) and decode M=8 (decode.gbps); GEMM on pre-quantized activations",
                   "prefill_m": pre["m"], "decode_m": dec["m"], "weight_sets": sets},
        "decode": {"gbps": round(dec["gbps"], 1), "ms_per_step": round(dec["step_ms"], 4),
                   "frac_of_hbm": round(dec["gbps"] / PEAK_HBM_GBPS, 4)},
        "roofline": {"bound": "mfma", "kernel": "tile_gemm_kernel (prefill M=2048, 4 projections)",
                     "achieved": round(pre["tflops"], 2), "peak": PEAK_FP8_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(pre["tflops"] / PEAK_FP8_TFLOPS, 4), "traffic": None},
        "roofline_decode": {"bound": "hbm", "kernel": "stream_gemm_kernel (decode M=8, 4 projections)",
                            "achieved": round(dec["gbps"], 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                            "frac": round(dec["gbps"] / PEAK_HBM_GBPS, 4), "traffic": None},
        "detail": results,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


def cpu_baseline(rows: int) -> dict:
    """The C oracle on the host cores: the four projections at ``rows`` rows."""

    import numpy as np
    import torch

    import oracle
    from minillm_amd.validation import QWEN3_4B_PROJECTIONS, make_baseline_activations, make_baseline_weights

    threads = min(os.cpu_count() or 1, 16)
    total_flops, total_s = 0, 0.0
    for p in QWEN3_4B_PROJECTIONS:
        w, ws = make_baseline_weights(p, SEED)
        x = make_baseline_activations(rows, p.k, SEED, outliers=True)
        q, s = oracle.act_quant(x.view(torch.int16).numpy().view(np.uint16))
        wc = w.view(torch.uint8).numpy()
        wsn = ws.numpy()
        t0 = time.perf_counter()
        oracle.block_gemm(q, s, wc, wsn, threads=threads)
        total_s += time.perf_counter() - t0
        total_flops += 2 * rows * p.n * p.k
    return {"value": round(total_flops / total_s / 1e12, 5), "unit": "TFLOPS", "cores": threads,
            "kind": "port",
            "sample": f"C oracle block GEMM (exact fp64 per-group dots, fp32 scaling) over the 4 projections "
                      f"at M={rows}, {total_s:.1f} s"}


if __name__ == "__main__":
    raise SystemExit(main())
