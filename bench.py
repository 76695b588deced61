"""Benchmark of the W8A8 quantized Linear path on one MI355X.

Headline workload (the JSON line's ``value``): the FP8 (OCP E4M3) W8A8
state-pass GEMMs at M = 4096 tokens, hidden K = 4096 -- fused QKV
(N = 6144), o_proj (N = 4096), fused gate_up (N = 2 x 12288) and down
(K = 12288, N = 4096). One step = one pass over the four shapes: per-token
quantization of the resident bf16 activations, then the GEMM with its dequant
epilogue to bf16 (QuantLinear.forward's work). ``value`` is the step's
algorithmic ops (2 M N K summed over the shapes) per second of the step.

The same line carries, under ``configs``, the other synthetic workloads of
the path, each timed on the GPU with HIP events on the launch stream:
  single_int8_linear   128 x 1024 x 1024 INT8 linear (quant + GEMM)
  ragged_int8          16 question blocks, lengths in [32, 128], packed into one
                       launch per projection (K = 4096; N = 6144, 4096, 24576)
  mlp_block_int8       norm + quant -> gate_up + SwiGLU -> requant -> down + residual,
                       M = 4096, hidden 4096, intermediate 12288
  gated_o_proj_quant_fp8  quantize_rows(out * sigmoid(gate)) fused, 4096 x 4096, the gate read in
                       place from the q_proj output
  gdn_norm_quant_fp8   gated RMSNorm over 32 heads of 128 + quantize fused, 4096 x 4096
  question_gemms_fp8_m128  the four projections at M = 128 (a batch of 8 question blocks),
                       weights streamed from HBM (pool > Infinity Cache): HBM GB/s
  linear_stack_fp8     48 layers of QKV / o_proj / MLP block, identity mixer: one
                       8192-token state pass, then 255 question blocks of 16 tokens
                       (ragged batches of 8 blocks, and of all 255)
plus ``roofline`` for the dominant kernel and ``cpu_baseline``: the oracle's
restatement of the reference CPU path timed on this host on a bounded sample.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "d3-turbo-trt_amd"))
sys.path.insert(0, ROOT)

METRIC = "W8A8 GEMM TOPS & % MI355X MFMA peak; state4096+16Q linear-stack ms"
PEAK_TOPS = {"fp8": 5000.0, "int8": 5000.0}  # MI355X dense MFMA: FP8 TFLOP/s, INT8 TOPS
PEAK_HBM_GBS = 8000.0
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gemm_w8a8_fp8_state_pass_hbm_traffic.txt")

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


def gemm_bytes(M, N, K, residual=False):
    """Algorithmic HBM bytes of one W8A8 GEMM: 8-bit operands, bf16 output, fp32 scales."""
    return M * K + N * K + 2 * M * N + 4 * (M + N) + (2 * M * N if residual else 0)


def quant_bytes(M, K):
    """bf16 row in, 8-bit row out, one fp32 scale per row."""
    return 2 * M * K + M * K + 4 * M


class Timer:
    """Per-label HIP-event timing of launches on the current stream."""

    def __init__(self):
        import torch

        self.torch = torch
        self.marks = {}

    def run(self, label, fn):
        ev0 = self.torch.cuda.Event(enable_timing=True)
        ev1 = self.torch.cuda.Event(enable_timing=True)
        ev0.record()
        out = fn()
        ev1.record()
        self.marks.setdefault(label, []).append((ev0, ev1))
        return out

    def ms(self, label):
        pairs = self.marks[label]
        return sum(a.elapsed_time(b) for a, b in pairs) / len(pairs)

    def reset(self):
        self.marks = {}


def timed_steps(step, steps, warmup):
    """Warm up, then time exactly ``steps`` calls bracketed by device syncs."""
    import torch

    for _ in range(warmup):
        step(None)
    torch.cuda.synchronize()
    timer = Timer()
    t0 = time.perf_counter()
    for _ in range(steps):
        step(timer)
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1000.0 / steps, timer


SETTLE_MS = 150.0


def settle_clock(step, min_ms: float = SETTLE_MS) -> int:
    """Run ``step`` untimed, in batches of 10, until ``min_ms`` of wall time have passed; return the
    number of steps run. Under sustained load the GPU's clock ramps up over the first ~15 ms after a
    lighter phase (measured on the FP8 state pass: 0.74 ms per step timed after 5 warmup steps, 0.66 ms
    after 60 or 200), so steps timed after this run at the clock a serving loop holds."""
    import torch

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    n = 0
    while True:
        for _ in range(10):
            step(None)
        n += 10
        torch.cuda.synchronize()
        if (time.perf_counter() - t0) * 1000.0 >= min_ms:
            return n


def timed_settled(step, steps, warmup):
    """(ms per step timed from where the GPU stands, ms per step after settle_clock, settle steps):
    both timings are `warmup` untimed steps, then exactly `steps` timed ones."""
    ms_idle, _ = timed_steps(step, steps, warmup)
    n = settle_clock(step)
    ms, _ = timed_steps(step, steps, warmup)
    return ms_idle, ms, n


def _call(timer, label, fn):
    return fn() if timer is None else timer.run(label, fn)


# ---------------------------------------------------------------------------------------------
# headline: FP8 state-pass GEMMs at M = 4096
# ---------------------------------------------------------------------------------------------
def build_state_pass(mode: str, dev):
    import torch

    from d3trt_amd import QuantLinear
    from oracle import quant_ref as R  # seeded input generators only

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


def read_traffic():
    """HBM bytes per launch of each state-pass GEMM, from the committed rocprofv3 PMC summary."""
    out = {}
    try:
        for line in open(TRAFFIC_FILE):
            m = re.match(r"\s*traffic_bytes_per_launch\s+(\w+)\s+(\d+)", line)
            if m:
                out[m.group(1)] = int(m.group(2))
    except OSError:
        pass
    return out


def launch_us(fn_of, n_launches: int, rounds: int = 21) -> float:
    """Duration (us) per launch of back-to-back launches fn_of(0), ..., fn_of(n_launches - 1): the launches
    are captured once in a HIP graph, whose replay is timed between two HIP events on the current stream
    (the stream the kernels run on), so host latency never leaves the GPU waiting. The median over
    `rounds` replays (at least 20)."""
    import torch

    cur = torch.cuda.current_stream()
    side = torch.cuda.Stream()
    side.wait_stream(cur)
    with torch.cuda.stream(side):
        fn_of(0)  # warm-up: allocations and the stream's split-K workspace stay outside the capture
    cur.wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        for i in range(n_launches):
            fn_of(i)
    graph.replay()
    torch.cuda.synchronize()
    times = []
    for _ in range(max(rounds, 20)):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        graph.replay()
        e1.record()
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1) * 1e3 / n_launches)
    del graph
    times.sort()
    return times[len(times) // 2]


ROTATE_BYTES = 320 << 20  # > the 256 MB Infinity Cache: rotated operands come from HBM


def run_state_pass(args, mode: str):
    import torch

    from d3trt_amd import _lib
    from d3trt_amd import kernels as KK

    dev = torch.device("cuda:0")
    layers = build_state_pass(mode, dev)

    def step(_timer=None):
        outs = []
        for name, M, N, K, x, lin in layers:
            q, s = KK.quantize_rows(x, mode, kblock=lin.kblock)
            outs.append(KK.gemm(mode, q, s.view(-1), lin.weight, lin.weight_scale,
                                epilogue=_lib.EPI_DEQUANT, out_dtype=torch.bfloat16))
        return outs

    eager_outs = step()
    # the same launches captured once in a HIP graph and replayed: the step as a serving loop runs it
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):  # the stream warmed up above (its split-K workspace exists)
        graph_outs = step()
    graph.replay()
    torch.cuda.synchronize()
    for e, g in zip(eager_outs, graph_outs):
        if not torch.equal(e, g):
            raise RuntimeError("graph replay differs from the eager state pass")
    ms_idle, ms_per_step, n_settle = timed_settled(lambda _t: graph.replay(), args.steps, args.warmup)
    # eager: the module-path calls one by one (host launch latency included), at the settled clock
    ms_eager, _ = timed_steps(step, args.steps, args.warmup)

    # per-kernel durations: back-to-back launches; quantize inputs and GEMM weights rotate over copies
    # larger than the Infinity Cache (every layer of a stack brings its own weights from HBM), the GEMM
    # reads the quantized activations the step's quantize just wrote
    shapes = {}
    for name, M, N, K, x, lin in layers:
        n_x = max(2, -(-ROTATE_BYTES // x.numel() // x.element_size()))
        xs = [x.clone() for _ in range(n_x)]
        q, s = KK.quantize_rows(x, mode, kblock=lin.kblock)
        qb = torch.empty_like(q)
        sb = torch.empty(M, dtype=torch.float32, device=dev)
        mc, ldq = (KK.mode_code(mode) | _lib.KBLOCK, M) if lin.kblock else (KK.mode_code(mode), K)
        q_us = launch_us(lambda i: _lib.check(_lib.load().d3w8a8_quantize_rows(
            mc, KK.dtype_code(x.dtype), xs[i % n_x].data_ptr(), K, M, K, qb.data_ptr(), ldq,
            sb.data_ptr(), torch.cuda.current_stream().cuda_stream), "quantize_rows"), 4 * n_x)
        del xs
        n_w = max(2, -(-ROTATE_BYTES // lin.weight.numel()))
        ws = [lin.weight.clone() for _ in range(n_w)]
        out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
        g_us = launch_us(lambda i: KK.gemm(mode, q, s.view(-1), ws[i % n_w], lin.weight_scale, out=out,
                                           epilogue=_lib.EPI_DEQUANT, out_dtype=torch.bfloat16), 4 * n_w)
        del ws
        g_ms, q_ms = g_us * 1e-3, q_us * 1e-3
        ops = 2.0 * M * N * K
        shapes[name] = {
            "M": M, "N": N, "K": K,
            "gemm_ms": round(g_ms, 5),
            "gemm_tops": round(ops / (g_ms * 1e-3) / 1e12, 1),
            "gemm_frac_peak": round(ops / (g_ms * 1e-3) / 1e12 / PEAK_TOPS[mode], 4),
            "gemm_algo_bytes": gemm_bytes(M, N, K),
            "gemm_launches_timed": 4 * n_w,
            "quant_ms": round(q_ms, 5),
            "quant_gbs": round(quant_bytes(M, K) / (q_ms * 1e-3) / 1e9, 1),
            "quant_frac_hbm": round(quant_bytes(M, K) / (q_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
        }
    total_ops = sum(2.0 * M * N * K for _, M, N, K, _, _ in layers)
    dom = max(shapes, key=lambda s: shapes[s]["gemm_ms"])
    d = shapes[dom]
    traffic = read_traffic().get(dom)
    roofline = {
        "bound": "mfma",
        "achieved": d["gemm_tops"],
        "peak": PEAK_TOPS[mode],
        "unit": "TFLOP/s" if mode == "fp8" else "TOPS",
        "frac": round(d["gemm_tops"] / PEAK_TOPS[mode], 4),
        "traffic": traffic,
        "kernel": f"gemm_w8a8_dma {mode} {dom} {d['M']}x{d['N']}x{d['K']}",
        "timing": "HIP events around a graph replay of back-to-back launches on the launch stream, weights "
                  "rotated over > 256 MB of copies (streamed from HBM), quantized activations as the step "
                  "leaves them",
        "algo_ops_per_launch": 2.0 * d["M"] * d["N"] * d["K"],
        "algo_bytes_per_launch": d["gemm_algo_bytes"],
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
        "dtype": mode,
        "data": "synthetic: seeded N(0,1) bf16 activations with 1% of channels x20, N(0,0.02) weights",
        "config": {
            "workload": f"state_pass_{mode}_m4096: per-token quantize + W8A8 GEMM + dequant to bf16 for "
                        "qkv 4096x6144x4096, o_proj 4096x4096x4096, gate_up 4096x24576x4096, "
                        "down 4096x4096x12288",
            "frac_of_mfma_peak": round(value / PEAK_TOPS[mode], 4),
            "step": "one HIP graph replay of the 8 launches (graph output checked equal to the eager pass)",
            "clock": f"the timed steps follow {n_settle} untimed replays ({SETTLE_MS:.0f} ms): the clock a "
                     "sustained run holds; ms_per_step_from_idle times the same warmup + steps before them",
            "ms_per_step_from_idle": round(ms_idle, 4),
            "tops_from_idle": round(total_ops / (ms_idle * 1e-3) / 1e12, 1),
            "ms_per_step_eager": round(ms_eager, 4),
            "tops_eager": round(total_ops / (ms_eager * 1e-3) / 1e12, 1),
            "shapes": shapes,
        },
        "roofline": roofline,
    }
    return result, layers


# ---------------------------------------------------------------------------------------------
# the other workloads of the path
# ---------------------------------------------------------------------------------------------
def run_single_linear(args):
    """128 x 1024 x 1024 INT8 linear (quantize_rows + GEMM + dequant), seed 0."""
    import torch

    from d3trt_amd import QuantLinear
    from oracle import quant_ref as R

    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(0)
    M, K, N = 128, 1024, 1024
    x = R.outlier_activations(g, M, K).to(dev)
    lin = QuantLinear(K, N, mode="int8", dtype=torch.bfloat16, device=dev)
    lin.load_full(R.gaussian_weight(g, N, K).to(dev))
    ms, timer = timed_steps(lambda t: _call(t, "fwd", lambda: lin(x)), max(args.steps, 50), args.warmup)
    fwd_ms = timer.ms("fwd")
    # device time: the forward's two launches, back to back in a graph (host latency excluded)
    dev_us = launch_us(lambda i: lin(x), 50)
    byts = quant_bytes(M, K) + gemm_bytes(M, N, K)
    cpu = None
    if not args.no_cpu:
        xc, wq, ws = x.cpu(), lin.weight_rows().cpu(), lin.weight_scale.cpu()
        cpu = cpu_rate(lambda: R.emulated_linear(xc, wq, ws, "int8", torch.bfloat16), 2.0 * M * N * K, 2.0,
                       "the whole workload: oracle emulated_linear (quant.py:158-162), 128 x 1024 x 1024")
    return {
        "cpu_baseline": cpu,
        "shape": f"{M}x{N}x{K}", "mode": "int8", "forward_us": round(fwd_ms * 1e3, 2),
        "forward_note": "eager module call timed by an event pair: host latency included",
        "device_us": round(dev_us, 2),
        "tops": round(2.0 * M * N * K / (dev_us * 1e-6) / 1e12, 2),
        "hbm_gbs": round(byts / (dev_us * 1e-6) / 1e9, 1),
        "bound": "hbm (arithmetic intensity 186 ops/B); launch-latency bound at this size",
    }


def run_ragged(args):
    """16 question blocks, lengths uniform in [32, 128] (seed 0), packed into one launch per projection."""
    import torch

    from d3trt_amd import QuantLinear
    from oracle import quant_ref as R

    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(0)
    lengths = torch.randint(32, 129, (16,), generator=g).tolist()
    W, K = max(lengths), 4096
    x = torch.zeros(16, W, K, dtype=torch.bfloat16)
    for b, n in enumerate(lengths):
        x[b, :n] = R.outlier_activations(g, n, K)
    x = x.to(dev)
    T = sum(lengths)
    out = {"lengths": lengths, "rows": T, "shapes": {},
           "timing": "graph replay of back-to-back forward_ragged calls (ragged quantize + one GEMM each), "
                     "median of >= 20 replays"}
    cpu_work = []
    for N in (6144, 4096, 24576):
        lin = QuantLinear(K, N, mode="int8", dtype=torch.bfloat16, device=dev)
        lin.load_full(R.gaussian_weight(g, N, K).to(dev))
        us = launch_us(lambda i: lin.forward_ragged(x, lengths), 8)
        ops = 2.0 * T * N * K
        out["shapes"][f"N{N}"] = {"us": round(us, 2), "tops": round(ops / (us * 1e-6) / 1e12, 1),
                                  "frac_peak": round(ops / (us * 1e-6) / 1e12 / PEAK_TOPS["int8"], 4)}
        if not args.no_cpu:
            cpu_work.append((lin.weight_rows().cpu(), lin.weight_scale.cpu()))
        del lin
    if cpu_work:
        xb = [x[b, :n].cpu() for b, n in enumerate(lengths[:2])]  # the first two blocks of the batch
        rows = sum(t.shape[0] for t in xb)
        ops = sum(2.0 * rows * wq.shape[0] * K for wq, _ in cpu_work)
        full = sum(2.0 * T * wq.shape[0] * K for wq, _ in cpu_work)
        out["cpu_baseline"] = cpu_rate(
            lambda: [R.emulated_linear(xi, wq, ws, "int8", torch.bfloat16) for wq, ws in cpu_work for xi in xb],
            ops, 3.0, f"the first 2 of the 16 blocks ({rows} rows) through the three projections, block by "
                      "block (the reference runs them right-padded, backends/trtllm.py:149-179)", full)
    return out


def run_mlp_block(args):
    """INT8 MLP block at M = 4096, hidden 4096, intermediate 12288 (norm weight N(1, 0.1), eps 1e-6)."""
    import torch

    from d3trt_amd import QuantMLP
    from d3trt_amd import _lib
    from d3trt_amd import kernels as KK
    from oracle import quant_ref as R

    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(0)
    M, H, I = 4096, 4096, 12288
    x = R.outlier_activations(g, M, H).to(dev)
    mlp = QuantMLP(H, I, mode="int8", dtype=torch.bfloat16, device=dev)
    gate_up = torch.cat([R.gaussian_weight(g, I, H), R.gaussian_weight(g, I, H)]).to(dev)
    mlp.load_full(gate_up, R.gaussian_weight(g, H, I).to(dev))
    del gate_up
    # N(1, 0.1) gain stored as the zero-centred weight w = gain - 1, so the applied gain is N(1, 0.1)
    nw = (0.1 * torch.randn(H, generator=g)).to(torch.bfloat16).to(dev)
    amax = torch.empty(M, dtype=torch.float32, device=dev)
    h = torch.empty(M, I, dtype=torch.bfloat16, device=dev)
    gu, dn = mlp.gate_up_proj, mlp.down_proj

    def step(_t=None):
        q1, s1, _ = KK.rmsnorm_quantize(x, nw, 1e-6, "int8", clear_amax=amax, kblock=True)
        KK.gemm("int8", q1, s1.view(-1), gu.weight, gu.weight_scale, epilogue=_lib.EPI_SWIGLU, out=h, row_amax=amax)
        q2, s2 = KK.quantize_rows_amax(h, amax, "int8", kblock=True)
        return KK.gemm("int8", q2, s2.view(-1), dn.weight, dn.weight_scale, epilogue=_lib.EPI_RESIDUAL,
                       residual=x)

    eager_out = step().clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):  # the stream warmed up above (its split-K workspace exists)
        graph_out = step()
    graph.replay()
    torch.cuda.synchronize()
    if not torch.equal(eager_out, graph_out):
        raise RuntimeError("graph replay differs from the eager MLP block")
    ms_idle, ms, n_settle = timed_settled(lambda _t: graph.replay(), args.steps, args.warmup)
    ms_eager, _ = timed_steps(step, args.steps, args.warmup)

    # per-kernel: back-to-back launches; norm inputs, h and the weights rotate over > 256 MB of copies
    st = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731
    lib = _lib.load()
    k = {}
    q1, s1, _ = KK.rmsnorm_quantize(x, nw, 1e-6, "int8", clear_amax=amax, kblock=True)
    i8k = KK.mode_code("int8") | _lib.KBLOCK  # K-blocked q, as the block runs it
    for rows in (M, 2 * M):
        xr = x if rows == M else torch.cat([x, x])
        n_x = max(2, -(-ROTATE_BYTES // (rows * H * 2)))
        xs = [xr.clone() for _ in range(n_x)]
        qb = torch.empty(rows, H, dtype=torch.int8, device=dev)
        sb = torch.empty(rows, dtype=torch.float32, device=dev)
        us = launch_us(lambda i: _lib.check(lib.d3w8a8_rmsnorm_quantize(
            i8k, KK.dtype_code(x.dtype), xs[i % n_x].data_ptr(), H, KK.dtype_code(nw.dtype),
            nw.data_ptr(), rows, H, 1e-6, 1, qb.data_ptr(), rows, sb.data_ptr(), None, 0, None, st()),
            "rmsnorm_quantize"), 4 * n_x)
        nq = quant_bytes(rows, H) + 2 * H
        key = "norm_quant" if rows == M else f"norm_quant_m{rows}"
        k[key] = {"us": round(us, 2), "gbs": round(nq / (us * 1e-6) / 1e9, 1),
                  "frac_hbm": round(nq / (us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4)}
        del xs
    n_w = max(2, -(-ROTATE_BYTES // gu.weight.numel()))
    wgs = [gu.weight.clone() for _ in range(n_w)]
    us = launch_us(lambda i: KK.gemm("int8", q1, s1.view(-1), wgs[i % n_w], gu.weight_scale,
                                     epilogue=_lib.EPI_SWIGLU, out=h, row_amax=amax), 4 * n_w)
    del wgs
    ops = 2.0 * M * (2 * I) * H
    k["gate_up_swiglu"] = {"us": round(us, 2), "tops": round(ops / (us * 1e-6) / 1e12, 1),
                           "frac_peak": round(ops / (us * 1e-6) / 1e12 / PEAK_TOPS["int8"], 4)}
    n_h = max(2, -(-ROTATE_BYTES // (h.numel() * 2)))
    hs = [h.clone() for _ in range(n_h)]
    q2, s2 = KK.quantize_rows_amax(h, amax, "int8", kblock=True)
    us = launch_us(lambda i: _lib.check(lib.d3w8a8_quantize_rows_amax(
        i8k, KK.dtype_code(h.dtype), hs[i % n_h].data_ptr(), I, amax.data_ptr(), M, I,
        q2.data_ptr(), M, s2.data_ptr(), st()), "quantize_rows_amax"), 4 * n_h)
    del hs
    rq = 2 * M * I + M * I + 4 * M
    k["requant"] = {"us": round(us, 2), "gbs": round(rq / (us * 1e-6) / 1e9, 1),
                    "frac_hbm": round(rq / (us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4)}
    # reference for the HBM-bound kernels: torch's bf16 -> e4m3 cast of the same shapes moves the same
    # bytes (2 read + 1 written per element) with no row reduction, inputs rotated over > 256 MB
    for name, cols in (("reference_cast_4096x4096", H), ("reference_cast_4096x12288", I)):
        n_c = max(2, -(-ROTATE_BYTES // (M * cols * 2)))
        srcs = [torch.randn(M, cols, device=dev).to(torch.bfloat16) for _ in range(n_c)]
        dst = torch.empty(M, cols, dtype=torch.float8_e4m3fn, device=dev)
        us = launch_us(lambda i: dst.copy_(srcs[i % n_c]), 4 * n_c)
        byts = 3 * M * cols
        k[name] = {"us": round(us, 2), "gbs": round(byts / (us * 1e-6) / 1e9, 1),
                   "frac_hbm": round(byts / (us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4),
                   "what": "torch bf16->float8_e4m3fn copy_, same bytes as a quantize, no row reduction"}
        del srcs
    n_w = max(2, -(-ROTATE_BYTES // dn.weight.numel()))
    wds = [dn.weight.clone() for _ in range(n_w)]
    out = torch.empty(M, H, dtype=torch.bfloat16, device=dev)
    us = launch_us(lambda i: KK.gemm("int8", q2, s2.view(-1), wds[i % n_w], dn.weight_scale,
                                     epilogue=_lib.EPI_RESIDUAL, residual=x, out=out), 4 * n_w)
    del wds
    ops = 2.0 * M * H * I
    k["down_residual"] = {"us": round(us, 2), "tops": round(ops / (us * 1e-6) / 1e12, 1),
                          "frac_peak": round(ops / (us * 1e-6) / 1e12 / PEAK_TOPS["int8"], 4)}
    total_ops = 2.0 * M * (2 * I) * H + 2.0 * M * H * I
    cpu = None
    if not args.no_cpu:
        rows = 32
        xs, nwc = x[:rows].cpu(), nw.cpu()
        wgu_q = KK.deinterleave_gate_up(gu.weight_rows().view(torch.uint8)).view(gu.weight.dtype).cpu()
        wgu_s = KK.deinterleave_gate_up(gu.weight_scale).cpu()
        wd_q, wd_s = dn.weight_rows().cpu(), dn.weight_scale.cpu()
        cpu = cpu_rate(lambda: R.mlp_block(xs, nwc, 1e-6, wgu_q, wgu_s, wd_q, wd_s, "int8"),
                       total_ops * rows / M, 4.0, f"{rows} of the 4096 rows through the oracle's block "
                       "(norm, quantize, gate_up, SwiGLU, requantize, down, residual)", total_ops)
    return {"cpu_baseline": cpu, "ms": round(ms, 4), "tops": round(total_ops / (ms * 1e-3) / 1e12, 1),
            "step": "one HIP graph replay (checked equal to the eager block)",
            "clock": f"timed after {n_settle} untimed replays ({SETTLE_MS:.0f} ms)",
            "ms_from_idle": round(ms_idle, 4), "ms_eager": round(ms_eager, 4), "kernels": k,
            "kernel_timing": "graph replay of back-to-back launches between HIP events; inputs / weights rotated "
                             "over > 256 MB",
            "norm_gain": "N(1, 0.1) applied as (1 + w), w ~ N(0, 0.1)"}


def run_gated_quant(args):
    """The gated attention output projection's input, quantize_rows(out * sigmoid(gate)) fused
    (core.py:297), at 4096 tokens x 4096: the gate read in place from the q_proj output [4096, 8192]
    (head_dim 256), inputs rotated over > 256 MB (cold). HBM bytes: out and gate in, codes and scales out."""
    import torch

    from d3trt_amd import _lib
    from d3trt_amd import kernels as KK

    dev = torch.device("cuda:0")
    M, K, hd = 4096, 4096, 256
    g = torch.Generator(device=dev).manual_seed(0)
    per = M * K * 2 * 3  # out + the q_proj output (query and gate halves)
    n = max(2, -(-ROTATE_BYTES // per))
    outs = [torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16) for _ in range(n)]
    qps = [torch.randn(M, 2 * K, generator=g, device=dev).to(torch.bfloat16) for _ in range(n)]
    q = torch.empty(M, K, dtype=torch.float8_e4m3fn, device=dev)
    s = torch.empty(M, dtype=torch.float32, device=dev)
    lib = _lib.load()
    us = launch_us(lambda i: _lib.check(lib.d3w8a8_gate_quantize(
        KK.mode_code("fp8") | _lib.KBLOCK, KK.dtype_code(torch.bfloat16), outs[i % n].data_ptr(), K,
        qps[i % n].data_ptr(), 2 * K, hd, M, K, q.data_ptr(), M, s.data_ptr(), None, 0,
        torch.cuda.current_stream().cuda_stream), "gate_quantize"), 4 * n)
    byts = M * K * 2 + M * K * 2 + M * K + 4 * M
    return {"shape": f"{M}x{K}", "head_dim": hd, "us": round(us, 2), "gbs": round(byts / (us * 1e-6) / 1e9, 1),
            "frac_hbm": round(byts / (us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4),
            "algo_bytes": byts, "note": "out and gate (in place in the q_proj output) in, e4m3 codes + scales out"}


def run_gdn_norm_quant(args):
    """The GDN output projection's input: Qwen3_5RMSNormGated over 32 heads of 128 fused with the per-token
    quantize (core.py:390-391), 4096 tokens x 4096, inputs rotated over > 256 MB (cold). HBM bytes: the
    core output and z in, codes and scales out."""
    import torch

    from d3trt_amd import _lib
    from d3trt_amd import kernels as KK

    dev = torch.device("cuda:0")
    M, K, hd = 4096, 4096, 128
    g = torch.Generator(device=dev).manual_seed(0)
    n = max(2, -(-ROTATE_BYTES // (M * K * 2 * 2)))
    xs = [torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16) for _ in range(n)]
    zs = [torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16) for _ in range(n)]
    w = (1 + 0.1 * torch.randn(hd, generator=g, device=dev)).to(torch.bfloat16)
    q = torch.empty(M, K, dtype=torch.float8_e4m3fn, device=dev)
    s = torch.empty(M, dtype=torch.float32, device=dev)
    lib = _lib.load()
    us = launch_us(lambda i: _lib.check(lib.d3w8a8_gdn_norm_quantize(
        KK.mode_code("fp8") | _lib.KBLOCK, KK.dtype_code(torch.bfloat16), xs[i % n].data_ptr(), K,
        zs[i % n].data_ptr(), K, KK.dtype_code(w.dtype), w.data_ptr(), hd, 1e-6, M, K, q.data_ptr(), M,
        s.data_ptr(), None, 0,
        torch.cuda.current_stream().cuda_stream), "gdn_norm_quantize"), 4 * n)
    byts = 2 * M * K * 2 + M * K + 4 * M + 2 * hd
    return {"shape": f"{M}x{K}", "heads": K // hd, "head_dim": hd, "us": round(us, 2),
            "gbs": round(byts / (us * 1e-6) / 1e9, 1), "frac_hbm": round(byts / (us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4),
            "algo_bytes": byts}


def run_reference_scaled_mm(args):
    """The reference's own FP8 GEMM call on this GPU, rowwise torch._scaled_mm(q, w.t(), scale_a [M, 1],
    scale_b [1, N], out_dtype=bf16) (d3trt/model/quant.py:171-177; hipBLASLt serves it on ROCm), at the
    four state-pass shapes: weights rotated over > 256 MB (from HBM), back-to-back launches replayed from a
    HIP graph, median of >= 20 replays. The library GEMM the W8A8 kernels replace, timed like them (its
    quantize and padding excluded), with the tensorwise form (one scalar scale each) beside it."""
    import torch

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(0)
    out = {}
    for name, M, N, Kd in (("qkv", 4096, 6144, 4096), ("o_proj", 4096, 4096, 4096), ("gate_up", 4096, 24576, 4096),
                           ("down", 4096, 4096, 12288)):
        a = (torch.randn(M, Kd, generator=gen, device=dev) * 8).to(torch.float8_e4m3fn)
        n = max(2, -(-ROTATE_BYTES // (N * Kd)))
        ws = [(torch.randn(N, Kd, generator=gen, device=dev) * 8).to(torch.float8_e4m3fn) for _ in range(n)]
        sa = torch.rand(M, 1, generator=gen, device=dev) * 1e-3
        sb = torch.rand(1, N, generator=gen, device=dev) * 1e-3
        one = torch.ones((), device=dev)
        ops = 2.0 * M * N * Kd
        e = {"M": M, "N": N, "K": Kd}
        for label, (s_a, s_b) in (("rowwise", (sa, sb)), ("tensorwise", (one, one))):
            try:
                us = launch_us(lambda i: torch._scaled_mm(a, ws[i % n].t(), scale_a=s_a, scale_b=s_b,
                                                          out_dtype=torch.bfloat16), 4 * n)
                e[f"{label}_us"] = round(us, 2)
                e[f"{label}_frac_peak"] = round(ops / (us * 1e-6) / 1e12 / PEAK_TOPS["fp8"], 4)
            except (RuntimeError, NotImplementedError) as ex:
                e[f"{label}_error"] = str(ex)[:200]
        out[name] = e
        del ws
        torch.cuda.empty_cache()
    out["note"] = ("rowwise = the reference's call (per-token and per-channel scales, bf16 out); tensorwise = "
                   "one scale per operand, which the reference falls back to where rowwise is missing")
    return out


def run_linear_stack(args):
    """48-layer FP8 projection stack (identity mixer): state pass of 8192 tokens, then 255 question
    blocks of 16 tokens in ragged batches of 8 blocks and of all 255 blocks."""
    import torch

    from d3trt_amd import LinearStack

    dev = torch.device("cuda:0")
    layers = args.stack_layers
    stack = LinearStack(layers, 4096, 6144, 12288, mode="fp8", device=dev)
    gen = torch.Generator(device=dev).manual_seed(0)
    stack.init_random(gen)
    state = torch.randn(8192, 4096, generator=gen, device=dev, dtype=torch.float32).to(torch.bfloat16)
    nq, qlen = 255, 16
    questions = torch.randn(nq, qlen, 4096, generator=gen, device=dev, dtype=torch.float32).to(torch.bfloat16)
    lengths = [qlen] * nq

    def state_pass():
        return stack(state)

    def question_pass(batch):
        # each ragged batch replays the stack as one HIP graph per packed row count
        for b0 in range(0, nq, batch):
            stack.forward_ragged(questions[b0:b0 + batch], lengths[b0:b0 + batch], graph=True)

    res = {"layers": layers, "hidden": 4096, "qkv_out": 6144, "intermediate": 12288, "mode": "fp8",
           "question_pass": "packed rows, one HIP graph replay of the 48 layers per batch"}
    steps = max(1, min(args.steps, 3))
    for label, fn in (("state_ms", state_pass), ("questions_b8_ms", lambda: question_pass(8)),
                      ("questions_b255_ms", lambda: question_pass(nq))):
        ms, _ = timed_steps(lambda t: fn(), steps, 1)
        res[label] = round(ms, 3)
    state_ops = 2.0 * 8192 * 4096 * (6144 + 4096 + 24576 + 4096 * 3) * layers
    q_ops = 2.0 * nq * qlen * 4096 * (6144 + 4096 + 24576 + 4096 * 3) * layers
    res["state_tops"] = round(state_ops / (res["state_ms"] * 1e-3) / 1e12, 1)
    res["questions_b255_tops"] = round(q_ops / (res["questions_b255_ms"] * 1e-3) / 1e12, 1)
    res["total_ms_b8"] = round(res["state_ms"] + res["questions_b8_ms"], 3)
    res["total_ms_b255"] = round(res["state_ms"] + res["questions_b255_ms"], 3)
    weight_bytes = layers * ((6144 + 4096 + 24576) * 4096 + 4096 * 12288)  # 8-bit weights of one sweep
    res["weight_bytes_per_sweep"] = weight_bytes
    res["questions_b8_weight_gbs"] = round(weight_bytes * -(-nq // 8) / (res["questions_b8_ms"] * 1e-3) / 1e9, 1)
    res["per_shape"] = stack_per_shape(stack, gen)
    if not args.no_cpu:
        from d3trt_amd import kernels as KK
        from oracle import quant_ref as R

        lay = stack.layers[0]
        gu = lay.mlp.gate_up_proj
        w = dict(w_in=lay.input_layernorm.cpu(), w_post=lay.post_attention_layernorm.cpu(),
                 wqkv_q=lay.qkv_proj.weight_rows().cpu(), wqkv_s=lay.qkv_proj.weight_scale.cpu(),
                 wo_q=lay.o_proj.weight_rows().cpu(), wo_s=lay.o_proj.weight_scale.cpu(),
                 wgu_q=KK.deinterleave_gate_up(gu.weight_rows().view(torch.uint8)).view(gu.weight.dtype).cpu(),
                 wgu_s=KK.deinterleave_gate_up(gu.weight_scale).cpu(),
                 wd_q=lay.mlp.down_proj.weight_rows().cpu(), wd_s=lay.mlp.down_proj.weight_scale.cpu())
        rows = 8
        xs = state[:rows].cpu()
        per_token_layer = 2.0 * 4096 * (6144 + 4096 + 24576) + 2.0 * 12288 * 4096
        full = per_token_layer * layers * (8192 + nq * qlen)
        res["cpu_baseline"] = cpu_rate(lambda: R.stack_layer(xs, mode="fp8", **w), per_token_layer * rows, 4.0,
                                       f"{rows} tokens through one layer of the oracle's FP8 stack (float64 "
                                       f"products); the projection covers {layers} layers x (8192 state + "
                                       f"{nq * qlen} question tokens)", full)
    del stack
    torch.cuda.empty_cache()
    return res


def stack_per_shape(stack, gen) -> dict:
    """Each launch of a stack layer alone, at the state pass's M = 8192 and a question batch's M = 128:
    back-to-back launches over the stack's own layers (each launch brings its layer's weights from HBM),
    replayed from a HIP graph, median of >= 20 replays. GEMMs against the FP8 MFMA peak at M = 8192 and
    against HBM at M = 128; the quantize kernels against HBM."""
    import torch

    from d3trt_amd import _lib
    from d3trt_amd import kernels as KK

    dev = next(stack.buffers()).device
    L = stack.layers
    n = len(L)
    H, Q, I = 4096, 6144, 12288
    lib = _lib.load()
    st = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731
    out = {}
    for M in (8192, 128):
        x = torch.randn(M, H, generator=gen, device=dev).to(torch.bfloat16)
        # K-blocked [K / 64, M, 64], as the stack's quantize kernels write them
        q_in = (torch.randn(I // 64, M, 64, generator=gen, device=dev) * 8).to(torch.float8_e4m3fn)
        s_in = torch.rand(M, generator=gen, device=dev) * 1e-3
        qkv = torch.empty(M, Q, dtype=torch.bfloat16, device=dev)
        hbuf = torch.empty(M, I, dtype=torch.bfloat16, device=dev)
        amax = torch.zeros(M, dtype=torch.float32, device=dev)
        o = torch.empty(M, H, dtype=torch.bfloat16, device=dev)
        qb = torch.empty(M, I, dtype=torch.float8_e4m3fn, device=dev)
        sb = torch.empty(M, dtype=torch.float32, device=dev)
        a4 = q_in[: H // 64]
        gemms = {
            "qkv": (lambda i: KK.gemm("fp8", a4, s_in, L[i % n].qkv_proj.weight, L[i % n].qkv_proj.weight_scale,
                                      out=qkv), Q, H, 0),
            "o_proj+residual": (lambda i: KK.gemm("fp8", a4, s_in, L[i % n].o_proj.weight,
                                                  L[i % n].o_proj.weight_scale, out=o, residual=x,
                                                  epilogue=_lib.EPI_RESIDUAL), H, H, 1),
            "gate_up+swiglu": (lambda i: KK.gemm("fp8", a4, s_in, L[i % n].mlp.gate_up_proj.weight,
                                                 L[i % n].mlp.gate_up_proj.weight_scale, out=hbuf, row_amax=amax,
                                                 epilogue=_lib.EPI_SWIGLU), 2 * I, H, 0),
            "down+residual": (lambda i: KK.gemm("fp8", q_in, s_in, L[i % n].mlp.down_proj.weight,
                                                L[i % n].mlp.down_proj.weight_scale, out=o, residual=x,
                                                epilogue=_lib.EPI_RESIDUAL), H, I, 1),
        }
        shapes = {}
        for name, (fn, N, Kd, res_) in gemms.items():
            us = launch_us(fn, n)
            ops = 2.0 * M * N * Kd
            n_out = N // 2 if "swiglu" in name else N  # SwiGLU stores half the columns
            byts = M * Kd + N * Kd + 2 * M * n_out + 4 * (M + N) + (2 * M * N if res_ else 0)
            e = {"us": round(us, 2), "tops": round(ops / (us * 1e-6) / 1e12, 1),
                 "frac_mfma": round(ops / (us * 1e-6) / 1e12 / PEAK_TOPS["fp8"], 4),
                 "gbs": round(byts / (us * 1e-6) / 1e9, 1),
                 "frac_hbm": round(byts / (us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4)}
            e["bound"] = "mfma" if ops / byts > PEAK_TOPS["fp8"] * 1e12 / (PEAK_HBM_GBS * 1e9) else "hbm"
            shapes[name] = e
        xs = [torch.randn(M, H, generator=gen, device=dev).to(torch.bfloat16) for _ in range(4)]
        hs = [torch.randn(M, I, generator=gen, device=dev).to(torch.bfloat16) for _ in range(2)]
        amax_h = torch.full((M,), 4.0, device=dev)
        f8k = KK.mode_code("fp8") | _lib.KBLOCK  # K-blocked q, as the stack writes it
        quant = {
            "norm+quantize": (lambda i: _lib.check(lib.d3w8a8_rmsnorm_quantize(
                f8k, 0, xs[i % 4].data_ptr(), H, 0, L[i % n].input_layernorm.data_ptr(), M, H, 1e-6, 1,
                qb.data_ptr(), M, sb.data_ptr(), None, 0, None, st()), "norm"), quant_bytes(M, H) + 2 * H),
            "quantize(q block)": (lambda i: _lib.check(lib.d3w8a8_quantize_rows(
                f8k, 0, xs[i % 4].data_ptr(), H, M, H, qb.data_ptr(), M, sb.data_ptr(), st()), "quant"),
                quant_bytes(M, H)),
            "requantize(h)": (lambda i: _lib.check(lib.d3w8a8_quantize_rows_amax(
                f8k, 0, hs[i % 2].data_ptr(), I, amax_h.data_ptr(), M, I, qb.data_ptr(), M, sb.data_ptr(), st()),
                "requant"), quant_bytes(M, I)),
        }
        for name, (fn, byts) in quant.items():
            us = launch_us(fn, 16)
            shapes[name] = {"us": round(us, 2), "gbs": round(byts / (us * 1e-6) / 1e9, 1),
                            "frac_hbm": round(byts / (us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4), "bound": "hbm"}
        out[f"M{M}"] = shapes
        del x, q_in, qkv, hbuf, o, qb, xs, hs
        torch.cuda.empty_cache()
    out["note"] = ("M8192: the state pass's launches, GEMMs against the 5.0 PF FP8 peak; M128: a question batch "
                   "of 8 x 16 tokens, GEMMs against 8 TB/s (weights streamed); back-to-back over the stack's "
                   "layers (weights from HBM), median of >= 20 graph replays")
    return out


def run_question_gemms(args):
    """The four projections at question-batch M = 128 (8 blocks x 16 tokens), FP8: HBM-bound weight
    streams. Back-to-back launches replayed from a HIP graph, each reading a different weight copy from a
    pool of > 600 MB, so no launch finds its weights in the 256 MB Infinity Cache; median of >= 20
    replays. Weight GB/s and algorithmic GB/s against 8 TB/s, for the automatic tile and, for
    comparison, the weight-streaming tile chosen explicitly."""
    import torch

    from d3trt_amd import _lib
    from d3trt_amd import kernels as K

    dev = torch.device("cuda:0")
    M, out = 128, {}
    gen = torch.Generator(device=dev).manual_seed(0)
    for name, (N, Kd) in (("qkv", (6144, 4096)), ("o_proj", (4096, 4096)), ("gate_up", (24576, 4096)),
                          ("down", (4096, 12288))):
        copies = max(2, -(-(600 << 20) // (N * Kd)))
        ws = [(torch.randn(N, Kd, generator=gen, device=dev) * 8).to(torch.float8_e4m3fn) for _ in range(copies)]
        w_s = torch.rand(N, generator=gen, device=dev) * 1e-3
        # K-blocked activations [K / 64, M, 64], as the module's quantize kernels hand them to the GEMM
        a = (torch.randn(Kd // 64, M, 64, generator=gen, device=dev) * 8).to(torch.float8_e4m3fn)
        a_s = torch.rand(M, generator=gen, device=dev) * 1e-3
        y = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
        res = {"M": M, "N": N, "K": Kd}
        for label, tile in (("", _lib.TILE_AUTO), ("ws_tile_", _lib.TILE_WS)):
            us = launch_us(lambda i: K.gemm("fp8", a, a_s, ws[i % copies], w_s, out=y, tile=tile), 2 * copies)
            res[label + "us"] = round(us, 2)
            res[label + "frac_hbm"] = round(gemm_bytes(M, N, Kd) / (us * 1e-6) / 1e9 / PEAK_HBM_GBS, 3)
            if not label:
                res["weight_gbs"] = round(N * Kd / (us * 1e-6) / 1e9, 1)
                res["algo_gbs"] = round(gemm_bytes(M, N, Kd) / (us * 1e-6) / 1e9, 1)
        if name == "gate_up":  # as the layer runs it: SwiGLU epilogue, half-width output, row amax
            h = torch.empty(M, N // 2, dtype=torch.bfloat16, device=dev)
            amax = torch.zeros(M, device=dev)
            us = launch_us(lambda i: K.gemm("fp8", a, a_s, ws[i % copies], w_s, epilogue=_lib.EPI_SWIGLU, out=h,
                                             row_amax=amax), 2 * copies)
            sw_bytes = M * Kd + N * Kd + M * N + 4 * (2 * M + N)
            res["swiglu_us"] = round(us, 2)
            res["swiglu_frac_hbm"] = round(sw_bytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBS, 3)
        out[name] = res
        del ws
        torch.cuda.empty_cache()
    out["note"] = ("graph replay of back-to-back launches (median of >= 20), weights rotated over > 600 MB; "
                   "automatic tile = the planner's choice at M <= 128: the weight-streaming tile where K <= 4096 "
                   "and its slabs fit one round of CUs (qkv, o_proj, gate_up with SwiGLU), else 128x128 with "
                   "128-byte K steps and split-K (down; gate_up with a plain dequant epilogue); ws_tile_* = the "
                   "weight-streaming tile chosen explicitly; gate_up swiglu_* = the layer's own gate_up launch "
                   "(SwiGLU epilogue, half-width output, row amax)")
    return out


# ---------------------------------------------------------------------------------------------
# CPU baseline: the oracle's restatement of the reference CPU path
# ---------------------------------------------------------------------------------------------
def cpu_rate(fn, ops: float, seconds: float, sample: str, full_ops: float | None = None) -> dict:
    """Time fn() (the oracle on the host cores) for about `seconds`; report its TOPS on `ops` per call and,
    given the full workload's ops, the projected time of the whole configuration."""
    import torch

    torch.set_num_threads(os.cpu_count() or 1)
    reps = 0
    t0 = time.perf_counter()
    while True:
        fn()
        reps += 1
        if time.perf_counter() - t0 > seconds:
            break
    dt = (time.perf_counter() - t0) / reps
    out = {"value": round(ops / dt / 1e12, 4), "unit": "TOPS", "cores": torch.get_num_threads(), "kind": "port",
           "sample": f"{sample}; {reps} reps ({time.perf_counter() - t0:.1f} s); host {_cpu_model()}"}
    if full_ops is not None:
        out["projected_full_ms"] = round(full_ops / (ops / dt) * 1e3, 1)
    return out


def cpu_baseline_state_pass(layers, mode: str, rows: int, seconds: float):
    """QuantLinear._emulated (quant.py:158-162, restated by the oracle) on `rows` rows of each
    state-pass shape, repeated for about `seconds` of wall time on every host core."""
    import torch

    from oracle import quant_ref as R

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    work = [(x[:rows].cpu(), lin.weight_rows().cpu(), lin.weight_scale.cpu(), N, K) for _, M, N, K, x, lin in layers]
    ops = sum(2.0 * rows * N * K for _, _, _, N, K in work)
    reps = 0
    t0 = time.perf_counter()
    while True:
        for xs, wq, ws, _, _ in work:
            R.emulated_linear(xs, wq, ws, mode, torch.bfloat16)
        reps += 1
        if time.perf_counter() - t0 > seconds:
            break
    dt = (time.perf_counter() - t0) / reps
    return {
        "value": round(ops / dt / 1e12, 4),
        "unit": "TOPS",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"{rows} of the 4096 rows of each of the 4 state-pass shapes, {reps} reps "
                  f"({time.perf_counter() - t0:.1f} s); oracle emulated_linear (torch CPU: quantize_rows, "
                  f"fp32 matmul, dequant); host {_cpu_model()}",
    }


def single_pass(mode: str) -> int:
    """Counter calibration, then one step of the headline workload, for hardware-counter runs that count
    per dispatch: a 1 GiB device copy whose source has been pushed out of L2 and the 256 MB Infinity
    Cache by a 1 GiB write (so the copy reads 1 GiB from HBM and writes 1 GiB), then the step."""
    import torch

    from d3trt_amd import _lib
    from d3trt_amd import kernels as KK

    dev = torch.device("cuda:0")
    layers = build_state_pass(mode, dev)
    src = torch.ones(1 << 30, dtype=torch.uint8, device=dev)
    flush = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    flush.fill_(7)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, flush, dst
    for _, M, N, K, x, lin in layers:
        q, s = KK.quantize_rows(x, mode, kblock=lin.kblock)
        KK.gemm(mode, q, s.view(-1), lin.weight, lin.weight_scale, epilogue=_lib.EPI_DEQUANT,
                out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    print(json.dumps({"single_pass": mode, "copy_bytes": 1 << 30}))
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--mode", choices=["fp8", "int8"], default="fp8")
    ap.add_argument("--cpu-rows", type=int, default=128)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--headline-only", action="store_true", help="skip the other workloads")
    ap.add_argument("--stack-layers", type=int, default=48)
    ap.add_argument("--single", action="store_true",
                    help="run a 1 GiB calibration copy, then one untimed step (for rocprofv3 --pmc passes)")
    ap.add_argument("--config", default=None,
                    help="run only this entry of `configs` (no headline step) and print it: for profiling one "
                         "workload, e.g. question_gemms_fp8_m128")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this benchmark runs on exactly one GPU: the W8A8 path shards by token "
                                   "rows or output channels with no communication, and multi-GPU runs are "
                                   "not part of this build", "n_gpus": args.gpus}))
        return 2
    import torch

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU available"}))
        return 2
    torch.cuda.set_device(0)
    if args.single:
        return single_pass(args.mode)
    workloads = (("single_int8_linear", run_single_linear), ("ragged_int8", run_ragged),
                 ("mlp_block_int8", run_mlp_block), ("gated_o_proj_quant_fp8", run_gated_quant),
                 ("gdn_norm_quant_fp8", run_gdn_norm_quant),
                 ("question_gemms_fp8_m128", run_question_gemms),
                 ("reference_scaled_mm_fp8", run_reference_scaled_mm),
                 ("linear_stack_fp8", run_linear_stack))
    if args.config:
        fns = dict(workloads)
        if args.config not in fns:
            print(json.dumps({"error": f"unknown config {args.config!r}", "configs": list(fns)}))
            return 2
        print(json.dumps({"config": args.config, "result": fns[args.config](args)}))
        return 0
    result, layers = run_state_pass(args, args.mode)
    if not args.headline_only:
        configs = {}
        for name, fn in workloads:
            configs[name] = fn(args)
            print(json.dumps({"progress": name, "done": True}), file=sys.stderr, flush=True)
        result["configs"] = configs
    result["cpu_baseline"] = None if args.no_cpu else cpu_baseline_state_pass(layers, args.mode, args.cpu_rows,
                                                                               args.cpu_seconds)
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
