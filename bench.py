"""Benchmark of the MI355X FP8 block-scaled linear on Qwen3-4B projection shapes.

Metric: FP8 block GEMM TFLOPS at M=2048 and HBM GB/s at M=8 over the four
merged Qwen3-4B projections (qkv, o_proj, gate_up, down), on one GPU.

* A step is one pass of the block GEMM over the four projections for one batch: the
  prefill step at M=2048 (``value`` = TFLOPS = sum 2MNK / sum GEMM time) and the decode
  step at M=8 (``decode.gbps`` = op-level bytes / GEMM time).  Activations are quantized
  before the timed region (the quantizer is timed separately, ``quant``) and all inputs are
  resident in HBM.  The GEMM reads K-group-major activation scales, the layout
  ``fp8_linear`` hands it.
* Weights rotate so that no launch reads weights still in the 256 MB MALL: each projection
  is timed over its own ring of weight buffers of more than 600 MiB (the 7 generated sets
  plus copies of them at other addresses; qkv 40 buffers, o_proj 60, gate_up 13, down 26),
  and the decode chain streams 7 whole layers (707 MB) per replay.
* Timing: each projection's launches (one per weight set) are captured in a HIP graph and
  replayed K times between two HIP events recorded on the stream the kernels run on; the
  per-launch time is the elapsed time over K x sets launches, so ``roofline.achieved`` is
  the average per-launch rate of the dominant kernel.
* Also reported: baseline config 4 (the MLP block at M=512: gate_up -> SiLU*up + requant ->
  down, ``extras.mlp``) and config 5 (one continuous-batching step of the 36-layer linear
  stack, 144 full linears with independent weights at M = 512 + 24 = 536, ``extras.stack``).
* ``cpu_baseline`` times the C oracle (a CPU restatement of the reference arithmetic) on a
  bounded sample: the same four projections at ``--cpu-rows`` rows.
* ``roofline.traffic`` / ``roofline_decode.traffic`` are the measured HBM bytes per launch
  from the committed rocprofv3 PMC summary (profiles/hbm_traffic_qwen3.txt), when present.

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
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic_qwen3.txt")


def parse_args(argv=None):
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--prefill-m", type=int, default=2048)
    p.add_argument("--decode-m", type=int, default=8)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--cpu-rows", type=int, default=4096)
    p.add_argument("--no-extras", action="store_true", help="skip the MLP-block and 36-layer-stack configs")
    p.add_argument("--no-sweep", action="store_true", help="skip the M sweep (detail.sweep)")
    p.add_argument("--sweep-ms", default="1,16,64,256,1024,2048,4096,8192,16384",
                   help="row counts of the M sweep (the reference's benchmark range)")
    p.add_argument("--eager", action="store_true",
                   help="launch kernels directly instead of through HIP graphs (for counter collection)")
    p.add_argument("--only", choices=["prefill", "decode"], help="time one phase only")
    p.add_argument("--copy-calibration", type=int, metavar="MIB", default=0,
                   help="only run a device-to-device copy of MIB MiB a few times (PMC calibration) and exit")
    return p.parse_args(argv)


def timed_graph(torch, stream, fn, launches_per_call, steps, warmup, eager):
    """Average ms per launch of ``fn`` (which issues ``launches_per_call`` launches)."""

    with torch.cuda.stream(stream):
        fn()  # warm-up outside capture: sizes workspaces, so the capture allocates nothing new
        stream.synchronize()
        if eager:
            run = fn
        else:
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                fn()
            run = graph.replay
        for _ in range(warmup):
            run()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        stream.synchronize()
        start.record(stream)
        for _ in range(steps):
            run()
        end.record(stream)
        end.synchronize()
    return start.elapsed_time(end) / (steps * launches_per_call)


def read_traffic():
    """Bytes per launch measured by rocprofv3 (FETCH_SIZE + WRITE_SIZE, calibrated), from
    the committed summary: lines ``TRAFFIC <phase> <projection> <bytes>``."""

    out = {}
    if os.path.exists(TRAFFIC_FILE):
        for line in open(TRAFFIC_FILE):
            parts = line.split()
            if len(parts) == 4 and parts[0] == "TRAFFIC":
                out[(parts[1], parts[2])] = float(parts[3])
    return out


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
    stream = torch.cuda.Stream()

    if args.copy_calibration:
        n = args.copy_calibration << 20
        src = torch.ones(n, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": n, "launches": 5}), flush=True)
        return 0

    projs = QWEN3_4B_PROJECTIONS
    layer_bytes = sum(p.n * p.k for p in projs)
    sets = max(2, -(-512 * 2**20 // layer_bytes) + 1)
    print(f"generating {sets} weight sets of {layer_bytes / 2**20:.1f} MiB", file=sys.stderr, flush=True)
    weights = [[make_baseline_weights(p, SEED + 1000 * s, device="cuda") for p in projs] for s in range(sets)]
    # Per projection, a ring of weight buffers larger than the MALL: the generated sets, then
    # copies of them (the same bytes at other addresses miss the caches just the same).
    ring_bytes = 600 * 2**20
    rings = []
    for i, p in enumerate(projs):
        ring = [weights[r][i] for r in range(sets)]
        while len(ring) * p.n * p.k < ring_bytes:
            w, ws = weights[len(ring) % sets][i]
            ring.append((w.clone(), ws.clone()))
        rings.append(ring)

    lib = fp8._lib.load()
    sink = torch.empty(8 * 1024, dtype=torch.int32, device=dev)

    def run_phase(m, outliers, full_linear, probe=False):
        per_launch, quant, linear, probes = [], [], [], []
        for i, p in enumerate(projs):
            x = make_baseline_activations(m, p.k, SEED, outliers=outliers, device="cuda")
            q, s = fp8.quantize_mi355x_fp8_activation(x, scale_layout="kgroup")
            out = torch.empty((m, p.n), dtype=torch.bfloat16, device=dev)

            ring = rings[i]

            def gemms(ring=ring, q=q, s=s, out=out):
                for w, ws in ring:
                    fp8.launch_block_gemm(q, w, out, s, ws)

            def quants(x=x):
                for _ in range(sets):
                    fp8.quantize_mi355x_fp8_activation(x, scale_layout="kgroup")

            def linears(ring=ring, x=x):
                for w, ws in ring:
                    fp8.mi355x_fp8_linear(x, w, ws, [128, 128])

            def reads(ring=ring):
                for w8, _ in ring:
                    fp8._lib.check(lib.mi355x_fp8_read_probe(w8.data_ptr(), w8.numel(), sink.data_ptr(), sink.numel(),
                                                             torch.cuda.current_stream().cuda_stream))

            per_launch.append(timed_graph(torch, stream, gemms, len(ring), args.steps, args.warmup, args.eager))
            if probe:
                probes.append(timed_graph(torch, stream, reads, len(ring), args.steps, args.warmup, args.eager))
            quant.append(timed_graph(torch, stream, quants, sets, args.steps, args.warmup, args.eager))
            if full_linear:
                linear.append(timed_graph(torch, stream, linears, len(ring), args.steps, args.warmup, args.eager))
        return per_launch, quant, linear, probes

    results = {}
    for phase, m, outliers in (("prefill", args.prefill_m, True), ("decode", args.decode_m, False)):
        if args.only and phase != args.only:
            continue
        print(f"timing {phase} M={m}", file=sys.stderr, flush=True)
        mean, quant_ms, linear_ms, probe_ms = run_phase(m, outliers, full_linear=True, probe=phase == "decode")
        flops = [linear_flops(m, p.n, p.k) for p in projs]
        nbytes = [gemm_bytes(m, p.n, p.k) for p in projs]
        results[phase] = {
            "m": m,
            "step_ms": sum(mean),
            "tflops": sum(flops) / (sum(mean) * 1e9),
            "gbps": sum(nbytes) / (sum(mean) * 1e6),
            "per_proj": {p.name: {"mean_us": 1e3 * mean[i], "tflops": flops[i] / (mean[i] * 1e9),
                                  "gbps": nbytes[i] / (mean[i] * 1e6), "algorithmic_bytes": nbytes[i],
                                  "flops": flops[i]}
                         for i, p in enumerate(projs)},
            "quant": {p.name: {"us": 1e3 * quant_ms[i], "gbps": quant_bytes(m, p.k) / (quant_ms[i] * 1e6)}
                      for i, p in enumerate(projs)},
        }
        if probe_ms:
            # The same launches, each a plain streaming read of its weight bytes: what one launch
            # over these bytes reaches (launch, ramp-up and drain included).
            results[phase]["read_ceiling"] = {
                "step_ms": sum(probe_ms), "gbps": sum(nbytes) / (sum(probe_ms) * 1e6),
                "per_proj_us": {p.name: 1e3 * probe_ms[i] for i, p in enumerate(projs)}}
        if linear_ms:
            # The whole linear from bf16 activations (quantization included), as a model calls
            # it; same algorithmic bytes (gemm_bytes counts the activations as bf16).
            lbytes = nbytes
            results[phase]["linear"] = {
                "step_ms": sum(linear_ms), "gbps": sum(lbytes) / (sum(linear_ms) * 1e6),
                "tflops": sum(flops) / (sum(linear_ms) * 1e9),
                "per_proj": {p.name: {"us": 1e3 * linear_ms[i], "gbps": lbytes[i] / (linear_ms[i] * 1e6)}
                             for i, p in enumerate(projs)}}
    if args.only:
        print(json.dumps({"phase": args.only, "detail": results}), flush=True)
        return 0
    if "decode" in results:
        print("timing the decode layer chain", file=sys.stderr, flush=True)
        results["decode"]["layer_chain"] = bench_decode_layers(torch, fp8, stream, args, weights, projs)
    if not args.no_sweep:
        print("timing the M sweep", file=sys.stderr, flush=True)
        results["sweep"] = bench_sweep(torch, fp8, stream, args, rings, projs)
    ring_sizes = {p.name: len(r) for p, r in zip(projs, rings)}
    del weights, rings
    torch.cuda.empty_cache()

    extras = {}
    if not args.no_extras:
        print("timing MLP block and 36-layer stack", file=sys.stderr, flush=True)
        extras["mlp"] = bench_mlp(torch, fp8, stream, args, make_baseline_weights, make_baseline_activations)
        extras["rmsnorm_quant"] = bench_rmsnorm_quant(torch, fp8, stream, args)
        extras["stack"] = bench_stack(torch, fp8, stream, args, make_baseline_weights, make_baseline_activations,
                                      projs)

    cpu = None if args.no_cpu else cpu_baseline(args.cpu_rows)
    traffic = read_traffic()

    def traffic_per_launch(phase):
        vals = [traffic.get((phase, p.name)) for p in projs]
        return None if any(v is None for v in vals) else round(sum(vals) / len(vals))

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
                   "prefill_m": pre["m"], "decode_m": dec["m"], "weight_sets": sets,
                   "weight_ring_buffers": ring_sizes},
        "decode": {"gbps": round(dec["gbps"], 1), "ms_per_step": round(dec["step_ms"], 4),
                   "frac_of_hbm": round(dec["gbps"] / PEAK_HBM_GBPS, 4),
                   "linear_gbps": round(dec["linear"]["gbps"], 1),
                   "linear_ms_per_step": round(dec["linear"]["step_ms"], 4),
                   "layer_chain_gbps": dec["layer_chain"]["weight_gbps"],
                   "layer_chain_us_per_layer": dec["layer_chain"]["us_per_layer"]},
        "prefill_linear": {"tflops": round(pre["linear"]["tflops"], 1), "ms_per_step": round(pre["linear"]["step_ms"], 4),
                           "frac": round(pre["linear"]["tflops"] / PEAK_FP8_TFLOPS, 4)},
        "roofline": {"bound": "mfma", "kernel": "prefill block GEMM (M=2048, mean over the 4 projections)",
                     "achieved": round(pre["tflops"], 2), "peak": PEAK_FP8_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(pre["tflops"] / PEAK_FP8_TFLOPS, 4), "traffic": traffic_per_launch("prefill")},
        "roofline_decode": {"bound": "hbm", "kernel": "stream_gemm_kernel (decode M=8, mean over the 4 projections)",
                            "achieved": round(dec["gbps"], 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                            "frac": round(dec["gbps"] / PEAK_HBM_GBPS, 4), "traffic": traffic_per_launch("decode"),
                            "ceiling": round(dec["read_ceiling"]["gbps"], 1),
                            "frac_of_ceiling": round(dec["gbps"] / dec["read_ceiling"]["gbps"], 4)},
        "extras": extras,
        "detail": results,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


def bench_sweep(torch, fp8, stream, args, rings, projs):
    """GEMM-only and whole-linear (quantizer included) rate of each projection over the
    reference's benchmark row counts (BENCH_MS, engine/kernels/sm89_fp8_validation.py:33),
    so the dispatch crossovers show: per M, per projection, µs, TFLOPS and GB/s (op-level
    bytes), and the kernel the dispatch picked.  Weights rotate through the same rings as the
    headline phases; steps shrink with M so the sweep stays within a minute."""

    from minillm_amd.validation import gemm_bytes, linear_flops, make_baseline_activations

    lib = fp8._lib.load()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    out = {}
    for m in (int(v) for v in args.sweep_ms.split(",") if v):
        steps = max(2, min(args.steps, (args.steps * 256) // max(m, 256)))
        row = {}
        tot = {"gemm_us": 0.0, "linear_us": 0.0, "flops": 0, "bytes": 0}
        for i, p in enumerate(projs):
            x = make_baseline_activations(m, p.k, SEED + 17, outliers=m > 64, device="cuda")
            q, s = fp8.quantize_mi355x_fp8_activation(x, scale_layout="kgroup")
            o = torch.empty((m, p.n), dtype=torch.bfloat16, device="cuda")

            ring = rings[i]

            def gemms(ring=ring, q=q, s=s, o=o):
                for w, ws in ring:
                    fp8.launch_block_gemm(q, w, o, s, ws)

            def linears(ring=ring, x=x):
                for w, ws in ring:
                    fp8.mi355x_fp8_linear(x, w, ws, [128, 128])

            g_ms = timed_graph(torch, stream, gemms, len(ring), steps, 1, args.eager)
            l_ms = timed_graph(torch, stream, linears, len(ring), steps, 1, args.eager)
            flops, nbytes = linear_flops(m, p.n, p.k), gemm_bytes(m, p.n, p.k)
            kernel = fp8.dispatch_name(m, p.n, p.k, cus)
            row[p.name] = {"kernel": kernel, "gemm_us": round(g_ms * 1e3, 2), "linear_us": round(l_ms * 1e3, 2),
                           "gemm_tflops": round(flops / (g_ms * 1e9), 1),
                           "linear_tflops": round(flops / (l_ms * 1e9), 1),
                           "gemm_gbps": round(nbytes / (g_ms * 1e6), 1),
                           "linear_gbps": round(nbytes / (l_ms * 1e6), 1)}
            tot["gemm_us"] += g_ms * 1e3
            tot["linear_us"] += l_ms * 1e3
            tot["flops"] += flops
            tot["bytes"] += nbytes
            del x, q, s, o
        row["all"] = {"gemm_us": round(tot["gemm_us"], 2), "linear_us": round(tot["linear_us"], 2),
                      "gemm_tflops": round(tot["flops"] / (tot["gemm_us"] * 1e6), 1),
                      "linear_tflops": round(tot["flops"] / (tot["linear_us"] * 1e6), 1),
                      "gemm_gbps": round(tot["bytes"] / (tot["gemm_us"] * 1e3), 1),
                      "linear_gbps": round(tot["bytes"] / (tot["linear_us"] * 1e3), 1)}
        out[str(m)] = row
        print(f"  sweep M={m}: GEMM {row['all']['gemm_tflops']} TFLOPS, linear {row['all']['linear_tflops']} TFLOPS",
              file=sys.stderr, flush=True)
        torch.cuda.empty_cache()
    return out


def bench_decode_layers(torch, fp8, stream, args, weights, projs):
    """The decode linears as a model runs them, chained over the rotating weight sets (one
    set per layer): residual add + RMSNorm + quantizer -> qkv GEMM; the q columns (the
    attention stand-in) -> quantizer + o_proj GEMM; residual add + RMSNorm + quantizer ->
    gate_up GEMM -> SiLU*up; quantizer -> down GEMM.  Four launches per layer up to 8 rows
    (the two norms, every quantizer and the SiLU*up run inside the GEMM launches), eight
    above.  Reported: time per layer and the layer's weight bytes per second, and the same
    chain with SiLU*up + quantizer as a launch of its own."""

    m, hidden, eps = args.decode_m, 2560, 1e-6
    gen = torch.Generator().manual_seed(SEED + 3)
    h0 = torch.randn(m, hidden, generator=gen).to(torch.bfloat16).cuda()
    r0 = torch.randn(m, hidden, generator=gen).to(torch.bfloat16).cuda()
    norms = [((torch.rand(hidden, generator=gen) + 0.5).to(torch.bfloat16).cuda(),
              (torch.rand(hidden, generator=gen) + 0.5).to(torch.bfloat16).cuda()) for _ in weights]
    inter = projs[3].k
    out = torch.empty((m, hidden), dtype=torch.bfloat16, device="cuda")

    def chain():
        h, res = h0, r0
        for (qkv_w, o_w, gu_w, d_w), (n1, n2) in zip(weights, norms):
            qkv, summed = fp8.rmsnorm_linear_mi355x_fp8(h, n1, eps, qkv_w[0], qkv_w[1], residual=res)
            o = fp8.mi355x_fp8_linear(qkv[:, :projs[1].k], o_w[0], o_w[1], [128, 128])
            act, res = fp8.rmsnorm_gate_up_silu_mi355x_fp8(o, n2, eps, gu_w[0], gu_w[1], residual=summed)
            h = fp8.mi355x_fp8_linear(act, d_w[0], d_w[1], [128, 128])

    def chain_separate():
        # The same layer with the SiLU*up + quantizer as its own launch after the gate_up
        # norm-linear, the down GEMM on its codes (the form before the gate_up/SiLU fusion).
        h, res = h0, r0
        for (qkv_w, o_w, gu_w, d_w), (n1, n2) in zip(weights, norms):
            qkv, summed = fp8.rmsnorm_linear_mi355x_fp8(h, n1, eps, qkv_w[0], qkv_w[1], residual=res)
            o = fp8.mi355x_fp8_linear(qkv[:, :projs[1].k], o_w[0], o_w[1], [128, 128])
            gu, res = fp8.rmsnorm_linear_mi355x_fp8(o, n2, eps, gu_w[0], gu_w[1], residual=summed)
            q3, s3 = fp8.silu_mul_quant_mi355x_fp8(gu[:, :inter], gu[:, inter:])
            fp8.launch_block_gemm(q3, d_w[0], out, s3, d_w[1])
            h = out

    ms = timed_graph(torch, stream, chain, len(weights), args.steps, args.warmup, args.eager)
    ms_sep = timed_graph(torch, stream, chain_separate, len(weights), args.steps, args.warmup, args.eager)
    nbytes = sum(p.n * p.k + 4 * ((p.n + 127) // 128) * ((p.k + 127) // 128) for p in projs)
    return {"us_per_layer": round(ms * 1e3, 2), "weight_gbps": round(nbytes / (ms * 1e6), 1),
            "launches_per_layer": 4 if m <= 8 else 8,
            "separate_silu_us_per_layer": round(ms_sep * 1e3, 2)}


def bench_rmsnorm_quant(torch, fp8, stream, args):
    """The fused residual add + RMSNorm + 1x128 quantizer in front of qkv / gate_up (hidden
    2560), at the prefill and decode row counts; bytes = 2K x + 2K residual + 2K residual
    sum + K codes + 4 K/128 scales per row."""

    out = {}
    gen = torch.Generator().manual_seed(SEED)
    for m in (args.prefill_m, args.decode_m):
        k = 2560
        x = torch.randn(m, k, generator=gen).to(torch.bfloat16).cuda()
        r = torch.randn(m, k, generator=gen).to(torch.bfloat16).cuda()
        w = (torch.rand(k, generator=gen) + 0.5).to(torch.bfloat16).cuda()
        calls = 16  # per graph replay, so the replay's own launch cost is spread out

        def run():
            for _ in range(calls):
                fp8.rmsnorm_quant_mi355x_fp8(x, w, 1e-6, r)

        ms = timed_graph(torch, stream, run, calls, args.steps, args.warmup, args.eager)
        nbytes = m * (6 * k + k + 4 * (k // 128))
        out[f"m{m}"] = {"us": round(ms * 1e3, 2), "gbps": round(nbytes / (ms * 1e6), 1)}
    return out


def bench_mlp(torch, fp8, stream, args, make_w, make_x):
    """Baseline config 4: x[512, 2560] -> gate_up -> SiLU(gate)*up + requant -> down."""

    from minillm_amd.validation import QWEN3_4B_PROJECTIONS

    gu, down = QWEN3_4B_PROJECTIONS[2], QWEN3_4B_PROJECTIONS[3]
    m = 512
    wgu, sgu = make_w(gu, SEED, device="cuda")
    wd, sd = make_w(down, SEED + 1, device="cuda")
    x = make_x(m, gu.k, SEED, outliers=True, device="cuda")
    # Copies of the block's 75 MB of weights at other addresses, more than 600 MiB in all, so
    # that no call finds its weights in the MALL.
    copies = [(wgu, sgu, wd, sd)]
    while len(copies) * (gu.n * gu.k + down.n * down.k) < 600 * 2**20:
        copies.append((wgu.clone(), sgu.clone(), wd.clone(), sd.clone()))

    def blocks():
        for a, b, c, d in copies:
            fp8.mlp_forward_mi355x_fp8(x, a, b, c, d)

    ms = timed_graph(torch, stream, blocks, len(copies), args.steps, args.warmup, args.eager)
    flops = 2 * m * (gu.n * gu.k + down.n * down.k)
    del copies
    return {"config": "MLP block M=512 (gate_up, fused SiLU*up + requant, down; incl. the input quantizer; "
                      "weights rotated over > 600 MiB of copies)",
            "us": round(ms * 1e3, 2), "tflops": round(flops / (ms * 1e9), 1)}


def bench_stack(torch, fp8, stream, args, make_w, make_x, projs):
    """Baseline config 5: 36 layers x 4 full linears (quantizer + GEMM), independent weights,
    M = 512-token prefill chunk + 24 decode tokens = 536."""

    m, layers = 536, 36
    weights = [[make_w(p, SEED + 7919 * layer + i, device="cuda") for i, p in enumerate(projs)]
               for layer in range(layers)]
    xs = [make_x(m, p.k, SEED + i, outliers=True, device="cuda") for i, p in enumerate(projs)]

    def step():
        for layer in range(layers):
            for i in range(len(projs)):
                w, s = weights[layer][i]
                fp8.mi355x_fp8_linear(xs[i], w, s, [128, 128])

    ms = timed_graph(torch, stream, step, 1, max(2, args.steps // 4), 2, args.eager)
    flops = layers * sum(2 * m * p.n * p.k for p in projs)
    nbytes = layers * sum(p.n * p.k for p in projs)

    # Per projection, over the same 36 independent weight sets: the GEMM on pre-quantized
    # activations, the quantizer alone, and the whole linear (what the stack runs).
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    per_proj = {}
    for i, p in enumerate(projs):
        q, s = fp8.quantize_mi355x_fp8_activation(xs[i], scale_layout="kgroup")
        o = torch.empty((m, p.n), dtype=torch.bfloat16, device="cuda")

        def gemms(i=i, q=q, s=s, o=o):
            for layer in range(layers):
                fp8.launch_block_gemm(q, weights[layer][i][0], o, s, weights[layer][i][1])

        def quants(i=i):
            for _ in range(layers):
                fp8.quantize_mi355x_fp8_activation(xs[i], scale_layout="kgroup")

        def linears(i=i):
            for layer in range(layers):
                fp8.mi355x_fp8_linear(xs[i], weights[layer][i][0], weights[layer][i][1], [128, 128])

        steps = max(2, args.steps // 4)
        g = timed_graph(torch, stream, gemms, layers, steps, 1, args.eager)
        qt = timed_graph(torch, stream, quants, layers, steps, 1, args.eager)
        ln = timed_graph(torch, stream, linears, layers, steps, 1, args.eager)
        f = 2 * m * p.n * p.k
        per_proj[p.name] = {"kernel": fp8.dispatch_name(m, p.n, p.k, cus), "gemm_us": round(g * 1e3, 2),
                            "quant_us": round(qt * 1e3, 2), "linear_us": round(ln * 1e3, 2),
                            "gemm_tflops": round(f / (g * 1e9), 1),
                            "gemm_frac_of_fp8_peak": round(f / (g * 1e9) / PEAK_FP8_TFLOPS, 4)}
    del weights
    torch.cuda.empty_cache()
    return {"config": "36-layer linear stack, 144 linears (quantizer + GEMM), M=536, independent weights",
            "ms": round(ms, 3), "tflops": round(flops / (ms * 1e9), 1),
            "weight_gbps": round(nbytes / (ms * 1e6), 1),
            "frac_of_fp8_peak": round(flops / (ms * 1e9) / PEAK_FP8_TFLOPS, 4),
            "per_proj": per_proj}


def cpu_baseline(rows: int) -> dict:
    """The C oracle on the host cores: the four projections at ``rows`` rows."""

    import numpy as np
    import torch

    import oracle
    from minillm_amd.validation import QWEN3_4B_PROJECTIONS, make_baseline_activations, make_baseline_weights

    host_cpus = os.cpu_count() or 1
    # The GPU box's CPU share is 16 cores per GPU (the pool's rule), whatever the host shows.
    threads = min(host_cpus, 16)
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
    # Config 1 of the baseline as the reference's CPU path runs it: the merged qkv linear
    # (quantizer + GEMM) on 16 tokens, single-threaded and with the same thread count.
    qkv = QWEN3_4B_PROJECTIONS[0]
    w, ws = make_baseline_weights(qkv, SEED)
    x16 = make_baseline_activations(16, qkv.k, SEED).view(torch.int16).numpy().view(np.uint16)
    wc, wsn = w.view(torch.uint8).numpy(), ws.numpy()
    config1 = {}
    for label, th in (("1_thread", 1), (f"{threads}_threads", threads)):
        t0 = time.perf_counter()
        reps = 3
        for _ in range(reps):
            oracle.linear(x16, wc, wsn, threads=th)
        config1[label + "_ms"] = round((time.perf_counter() - t0) / reps * 1e3, 2)
    return {"value": round(total_flops / total_s / 1e12, 5), "unit": "TFLOPS", "cores": threads,
            "host_cpus": host_cpus, "config1_qkv_m16": config1,
            "kind": "port",
            "sample": f"C oracle block GEMM (exact fp64 per-group dots, fp32 scaling) over the 4 projections "
                      f"at M={rows}, {total_s:.1f} s"}


if __name__ == "__main__":
    raise SystemExit(main())
