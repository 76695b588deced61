"""Benchmark of the W8A8 quantized Linear path on one MI355X.

Default workload: the FP8 (OCP E4M3) W8A8 state-pass GEMMs at M = 4096 tokens,
hidden K = 4096: fused QKV (N = 6144), o_proj (N = 4096), fused gate_up
(N = 2 x 12288) and down (K = 12288, N = 4096). One step = one pass of the hot
path over each shape: per-token activation quantization of the resident bf16
input, then the GEMM with its dequant epilogue to bf16 (QuantLinear.forward's
work, called through the C ABI wrappers).

Prints one JSON line: whole-path TOPS, the dominant kernel's roofline (timed
live with HIP events on the launch stream), per-shape figures, and the CPU
oracle's throughput on a bounded sample of the same workload.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "d3-turbo-trt_amd"))
sys.path.insert(0, ROOT)

METRIC = "W8A8 GEMM TOPS & % MI355X MFMA peak; state4096+16Q linear-stack ms"
PEAK_TOPS = {"fp8": 5000.0, "int8": 5000.0}  # MI355X dense MFMA, TFLOP/s (TOPS for int8)
PEAK_HBM_GBS = 8000.0

STATE_SHAPES = [  # (name, M, N, K)
    ("qkv", 4096, 6144, 4096),
    ("o_proj", 4096, 4096, 4096),
    ("gate_up", 4096, 24576, 4096),
    ("down", 4096, 4096, 12288),
]


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def build_state_pass(mode: str, dev):
    import torch

    from d3trt_amd import QuantLinear
    from oracle import quant_ref as R  # input generators only (seeded draws)

    g = torch.Generator().manual_seed(0)
    layers = []
    for name, M, N, K in STATE_SHAPES:
        x = R.outlier_activations(g, M, K).to(dev)
        w = R.gaussian_weight(g, N, K).to(dev)
        lin = QuantLinear(K, N, mode=mode, dtype=torch.bfloat16, device=dev)
        lin.load_full(w)
        del w
        layers.append((name, M, N, K, x, lin))
    torch.cuda.synchronize()
    return layers


def run_state_pass(args, mode: str):
    import torch

    from d3trt_amd import _lib
    from d3trt_amd import kernels as KK

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    layers = build_state_pass(mode, dev)
    n = len(layers)

    def step(events=None):
        for i, (_, M, N, K, x, lin) in enumerate(layers):
            if events is not None:
                events[i][0].record()
            q, s = KK.quantize_rows(x, mode)
            if events is not None:
                events[i][1].record()
            KK.gemm(mode, q, s.view(-1), lin.weight, lin.weight_scale, epilogue=_lib.EPI_DEQUANT,
                    out_dtype=torch.bfloat16)
            if events is not None:
                events[i][2].record()

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    ev = [[[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(n)] for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for k in range(args.steps):
        step(ev[k])
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_per_step = (t1 - t0) * 1000.0 / args.steps

    total_ops = sum(2.0 * M * N * K for _, M, N, K, _, _ in layers)
    shapes = {}
    for i, (name, M, N, K, _, _) in enumerate(layers):
        q_ms = sum(ev[k][i][0].elapsed_time(ev[k][i][1]) for k in range(args.steps)) / args.steps
        g_ms = sum(ev[k][i][1].elapsed_time(ev[k][i][2]) for k in range(args.steps)) / args.steps
        ops = 2.0 * M * N * K
        gemm_bytes = M * K + N * K + 2 * M * N + 4 * (M + N)
        quant_bytes = 2 * M * K + M * K + 4 * M
        shapes[name] = {
            "M": M, "N": N, "K": K,
            "gemm_ms": round(g_ms, 5),
            "gemm_tops": round(ops / (g_ms * 1e-3) / 1e12, 1),
            "gemm_frac_peak": round(ops / (g_ms * 1e-3) / 1e12 / PEAK_TOPS[mode], 4),
            "gemm_algo_bytes": gemm_bytes,
            "quant_ms": round(q_ms, 5),
            "quant_gbs": round(quant_bytes / (q_ms * 1e-3) / 1e9, 1),
            "quant_frac_hbm": round(quant_bytes / (q_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
        }
    dom = max(shapes, key=lambda s: shapes[s]["gemm_ms"])
    d = shapes[dom]
    achieved = d["gemm_tops"]
    roofline = {
        "bound": "mfma",
        "kernel": f"gemm_w8a8 {mode} {dom} {d['M']}x{d['N']}x{d['K']}",
        "achieved": achieved,
        "peak": PEAK_TOPS[mode],
        "unit": "TFLOP/s" if mode == "fp8" else "TOPS",
        "frac": round(achieved / PEAK_TOPS[mode], 4),
        "traffic": None,
        "algo_ops_per_launch": 2.0 * d["M"] * d["N"] * d["K"],
        "avg_launch_ms": d["gemm_ms"],
    }
    value = total_ops / (ms_per_step * 1e-3) / 1e12
    result = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8" if mode == "fp8" else "int8",
        "data": "synthetic (seeded N(0,1) bf16 activations with 1% x20 outlier channels; N(0,0.02) weights)",
        "config": {
            "workload": f"state_pass_{mode}_m4096: quantize_rows + W8A8 GEMM + dequant for "
                        "qkv 4096x6144x4096, o_proj 4096x4096x4096, gate_up 4096x24576x4096, "
                        "down 4096x4096x12288",
            "frac_of_mfma_peak": round(value / PEAK_TOPS[mode], 4),
        },
        "roofline": roofline,
        "shapes": shapes,
    }
    return result, layers


def cpu_baseline_state_pass(layers, mode: str, rows: int):
    """The oracle's restatement of the reference CPU path (quant.py:158-162) on `rows` rows per shape."""
    import torch

    from oracle import quant_ref as R

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    work = []
    for _, M, N, K, x, lin in layers:
        work.append((x[:rows].cpu(), lin.weight.cpu(), lin.weight_scale.cpu(), N, K))
    ops = sum(2.0 * rows * N * K for _, _, _, N, K in work)
    reps = 0
    t0 = time.perf_counter()
    while True:
        for xs, wq, ws, _, _ in work:
            R.emulated_linear(xs, wq, ws, mode, torch.bfloat16)
        reps += 1
        if time.perf_counter() - t0 > 10.0 or reps >= 5:
            break
    dt = (time.perf_counter() - t0) / reps
    return {
        "value": round(ops / dt / 1e12, 4),
        "unit": "TOPS",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"{rows} of 4096 rows of each of the 4 state-pass shapes, {reps} reps; oracle emulated_linear "
                  f"(torch CPU: quantize_rows, fp32 matmul, dequant); host {_cpu_model()}",
    }


def single_pass(mode: str) -> int:
    """One plain copy of known size (64 MiB read + 64 MiB written, the counter calibration) and
    then one step of the workload, for hardware-counter runs that count per dispatch."""
    import torch

    from d3trt_amd import _lib
    from d3trt_amd import kernels as KK

    dev = torch.device("cuda:0")
    src = torch.ones(64 << 20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    layers = build_state_pass(mode, dev)
    torch.cuda.synchronize()
    dst.copy_(src)
    for _, M, N, K, x, lin in layers:
        q, s = KK.quantize_rows(x, mode)
        KK.gemm(mode, q, s.view(-1), lin.weight, lin.weight_scale, epilogue=_lib.EPI_DEQUANT,
                out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    print(json.dumps({"single_pass": mode, "copy_bytes": src.numel()}))
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--mode", choices=["fp8", "int8"], default="fp8")
    ap.add_argument("--cpu-rows", type=int, default=128)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--single", action="store_true",
                    help="run one untimed step after a 64 MiB copy (for rocprofv3 --pmc passes)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this benchmark runs on exactly one GPU; multi-GPU sharding of the W8A8 "
                                   "path is a design note only (rows or output channels split with no "
                                   "communication)", "n_gpus": args.gpus}))
        return 2
    import torch

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU available"}))
        return 2
    if args.single:
        return single_pass(args.mode)
    result, layers = run_state_pass(args, args.mode)
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline_state_pass(layers, args.mode, args.cpu_rows)
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
