#!/usr/bin/env python
"""Benchmark of the MI355X ratchet-linear hot path (one GPU).

Workload (value): one int8 ratchet linear training step at M=16384 tokens
(batch 32 x seq 512), K=512, N=2048, quinary codes, fp32 row scales U[0.02, 0.1],
BF16 activations N(0,1) quantized per token, BF16 upstream gradient N(0, 1e-2):
per-token quant -> W8A8 forward GEMM (packed codes) -> SR gradient quant ->
int8 grad_input GEMM -> BF16 grad_weight GEMM -> fused normalize+update. It runs
through the drop-in DiscreteRatchetLinear autograd path. ``value`` is the step's
operations per second over its three GEMMs (3 x 2*M*N*K: two int8 GEMMs and one bf16
GEMM), inputs resident in HBM. ``split`` reports the two kinds against their own peaks:
int8 TOPS of the forward and grad_input GEMMs against the int8 MFMA peak, bf16 TFLOP/s of
grad_weight against the bf16 MFMA peak, each over the step time and over the kernels' own
launch times.

Also reported on the same line:
  kernels        per-kernel average launch time (HIP events on the launch stream) and
                 achieved TOPS / GB/s against the MI355X peaks
  roofline       the dominant hand-written kernel against its roofline
  train_tokens_per_s  the 25M ratchet transformer (8 layers, d 512, 8 heads, FFN 2048,
                 vocab 8192, seq 512, batch 32, int8 + int8_backward) full training step
  update_1b      the fused update of every layer of the 1B model (973 M weights) from its
                 grad_weight split partials: HBM GB/s against 8 TB/s
  train_1b       the 1B septenary ratchet transformer (24 layers, d 2048, 16 heads, FFN
                 5632, vocab 8192, seq 1024, batch 8) training step, tokens/s
  decode         KV-cached int8 decode of the 1B model at batch 1 and 16, tokens/s
  cpu_baseline   the reference's fp32 eager CPU path for the same op on a bounded
                 token sample, timed on this host's cores
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
for _p in (str(REPO), str(REPO / "local-ai-training_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "ratchet-linear TOPS (% int8 MFMA peak) + train tokens/s, 25M model, 1 GPU"
PEAK_INT8_OPS = 5.0e15
PEAK_BF16_FLOPS = 2.5e15
PEAK_HBM_BPS = 8.0e12

M_TOK, K_IN, N_OUT, MAX_CODE = 16384, 512, 2048, 2


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def parse_args() -> argparse.Namespace:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    # sustained training throughput: 8 warmup steps, then 30 timed steps with a sync only at
    # both ends (the reference's scripts/int8_training_throughput.py:89-102 method)
    ap.add_argument("--model-steps", type=int, default=30)
    ap.add_argument("--model-warmup", type=int, default=8)
    ap.add_argument("--no-model", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-update-1b", action="store_true")
    ap.add_argument("--no-train-1b", action="store_true")
    ap.add_argument("--train-1b-steps", type=int, default=30)
    ap.add_argument("--train-1b-warmup", type=int, default=8)
    ap.add_argument("--update-1b-only", action="store_true",
                    help="run only the 1B fused-update sweep (for profiling)")
    ap.add_argument("--hbm-probe", action="store_true",
                    help="run only the HBM streaming probe (practical read / copy bandwidth)")
    ap.add_argument("--gemm-sweep", action="store_true",
                    help="run only the forward GEMM on packed codes at large-K shapes")
    ap.add_argument("--immediate-updates", action="store_true",
                    help="--train-only: update each ratchet layer inside backward instead of "
                         "batching the updates after it (A/B runs)")
    ap.add_argument("--decode-only", action="store_true",
                    help="run only the decode bench and print its JSON (for profiling)")
    ap.add_argument("--decode-steps", type=int, default=64)
    ap.add_argument("--decode-batches", type=int, nargs="+", default=[1, 16])
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--kernel-iters", type=int, default=20)
    ap.add_argument("--no-graph", action="store_true",
                    help="time the eager autograd step instead of its HIP-graph replay")
    ap.add_argument("--pmc-probe", action="store_true",
                    help="run each op-step stage and a calibration copy (for rocprofv3 --pmc)")
    ap.add_argument("--traffic-summary", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="write the HBM traffic summary from two rocprofv3 counter CSVs")
    ap.add_argument("--counter-summary", nargs="+", metavar="CSV",
                    help="per-stage SQ/GRBM counter averages of --pmc-probe runs (rocprofv3 "
                         "counter_collection CSVs), with MFMA and VALU busy fractions")
    ap.add_argument("--train-only", choices=["25m", "1b"],
                    help="run only the graph-replayed training step of one model, --steps "
                         "timed steps after --warmup (for kernel traces)")
    ap.add_argument("--step-summary", nargs=2, metavar=("KERNEL_TRACE_CSV", "STEPS"),
                    help="bucket a rocprofv3 kernel trace of --train-only into kernel classes "
                         "per training step")
    return ap.parse_args()


def synthetic_layer(device):
    import torch

    from local_ai_training.ratchet import DiscreteRatchetLinear, pack_code_pressure

    gen = torch.Generator().manual_seed(1337)
    layer = DiscreteRatchetLinear(K_IN, N_OUT, max_code=MAX_CODE, matmul_mode="int8",
                                  int8_backward=True, fuse_backward_update=True)
    code = torch.randint(-MAX_CODE, MAX_CODE + 1, (N_OUT, K_IN), generator=gen,
                         dtype=torch.int8)
    layer.packed.copy_(pack_code_pressure(code, torch.zeros_like(code), MAX_CODE))
    layer._scale.copy_(torch.rand(N_OUT, generator=gen) * 0.08 + 0.02)
    x = torch.randn(M_TOK, K_IN, generator=gen).to(torch.bfloat16)
    g = (torch.randn(M_TOK, N_OUT, generator=gen) * 1e-2).to(torch.bfloat16)
    return layer.to(device).train(), x.to(device), g.to(device)


def op_bench(args, device):
    import torch

    from local_ai_training.int8_matmul import CapturedSeeds, quantize_rows

    layer, x, g = synthetic_layer(device)
    x.requires_grad_(True)

    def step():
        q, s = quantize_rows(x.detach())
        out = layer(x, inputs_int8=q, inputs_scale=s)
        out.backward(g)
        x.grad = None
        layer.ratchet_update(validate=False)

    def timed(fn, steps):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / steps

    for _ in range(args.warmup):
        step()
    eager_s = timed(step, args.steps)
    if args.no_graph:
        return eager_s, eager_s, layer, x.detach(), g
    # The whole step (quant, forward, backward, fused update) captured once into a HIP
    # graph and replayed: every replay launches the same kernels on the same buffers, so
    # the host-side autograd and launch overhead of the eager step disappears. The SR seed
    # is read from a device slot that the host fills before each replay with a fresh draw
    # from the CPU generator (the eager step's draw), inside the timed step.
    seeds = CapturedSeeds(device)
    side = torch.cuda.Stream(device=device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream(device).wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with seeds.recording(), torch.cuda.graph(graph):
        step()

    def replay():
        seeds.refill()
        graph.replay()

    for _ in range(args.warmup):
        replay()
    graph_s = timed(replay, args.steps)
    return graph_s, eager_s, layer, x.detach(), g


def stage_work(m: int, n: int, k: int, g_elem: int, nsplit: int) -> dict:
    """Algorithmic work per launch of each op-step stage: name -> (kind, amount[, bytes]);
    kind "bytes", "ops" (int8 MFMA) or "flops" (bf16 MFMA). Bytes count each operand
    read once and each result written once. grad_weight's result is its float32 split
    partials (nsplit per weight), which the update then reads."""
    mnk2 = 2.0 * m * n * k
    return {
        "quant_rows": ("bytes", m * k * 2 + m * k + m * 4),
        "fwd_gemm_packed": ("ops", mnk2, m * k + n * k + m * n * 2 + m * 4 + n * 4),
        "sr_quant_rows": ("bytes", m * n * 2 + m * n + m * 4 + n * 4),
        "grad_input_gemm": ("ops", mnk2, m * n + n * k + m * k * 2 + m * 4),
        "grad_weight_partials": ("flops", mnk2, m * n * g_elem + m * k + m * 4 + n * k * 4 * nsplit),
        "ratchet_update_partials": ("bytes", n * k * (1 + 4 * nsplit + 1) + n * 4),
    }


def op_stages(layer, x, g):
    """The launches of one op step as separately callable stages (same shapes, buffers and
    kernels as the autograd step), with each stage's algorithmic work (stage_work)."""
    import torch

    from local_ai_training import _native as nat
    from local_ai_training.int8_matmul import grad_weight_splits
    from local_ai_training.ops import ratchet

    ops = ratchet()
    dev = x.device
    m, k = x.shape
    n = layer.out_features
    packed, scale = layer.packed, layer.scale.float().contiguous()
    q, s = ops.quantize_rows(x)
    gq, gs = ops.quantize_rows(g, scale, True, 12345)
    splits = grad_weight_splits(m, n, k)
    gw_work = torch.empty(splits, n, k, dtype=torch.float32, device=dev)
    counts = torch.zeros(4, dtype=torch.int64, device=dev)
    row_rms = torch.empty(n, dtype=torch.float32, device=dev)
    flag = torch.zeros(1, dtype=torch.int32, device=dev)

    def update():
        # the update kernel alone (the step's separate one-block mean of row_rms is not part
        # of this stage), through the C ABI with its fixed buffers
        nat.call("rk_ratchet_update_partials", packed.data_ptr(), k, gw_work.data_ptr(), splits,
                 n, k, MAX_CODE, 8, 0.5, 1.5, 1e-8, None, 0.0, 1.0, counts.data_ptr(),
                 row_rms.data_ptr(), None, flag.data_ptr(), None, None, k,
                 nat.stream_handle(dev))

    # each stage is the operator the autograd step calls, with the step's arguments
    stages = [
        ("quant_rows", lambda: ops.quantize_rows(x)),
        ("fwd_gemm_packed", lambda: ops.packed_mm(q, packed, MAX_CODE, s, scale,
                                                  torch.bfloat16)),
        ("sr_quant_rows", lambda: ops.quantize_rows(g, scale, True, 12345)),
        ("grad_input_gemm", lambda: ops.packed_mm_t(gq, packed, MAX_CODE, gs, None,
                                                    torch.bfloat16)),
        ("grad_weight_partials", lambda: ops.grad_weight_partials(g, q, s, gw_work)),
        ("ratchet_update_partials", update),
    ]
    work = stage_work(m, n, k, g.element_size(), splits)
    return stages, work


def kernel_breakdown(layer, x, g, iters: int):
    """Average device time of each launch of one op step: `iters` back-to-back launches of
    the stage captured in a HIP graph and replayed between HIP events on the replay stream
    (no host launch time inside the interval; consecutive graph kernels start back to
    back, as the kernel trace shows)."""
    import torch

    stages, work = op_stages(layer, x, g)
    dev = x.device
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        for _, fn in stages:  # warm, outside the capture
            fn()
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize()
    avg_ms = {}
    for name, fn in stages:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(iters):
                fn()
        graph.replay()
        torch.cuda.synchronize()
        best = None
        for _ in range(3):  # the fastest of three replays (graph launch hiccups excluded)
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record()
            graph.replay()
            e1.record()
            torch.cuda.synchronize()
            ms = e0.elapsed_time(e1) / iters
            best = ms if best is None else min(best, ms)
        avg_ms[name] = best

    report = {}
    for name, ms in avg_ms.items():
        sec = ms * 1e-3
        w = work[name]
        entry = {"avg_us": round(ms * 1e3, 2)}
        if w[0] == "bytes":
            entry["alg_bytes"] = w[1]
            entry["GBps"] = round(w[1] / sec / 1e9, 1)
            entry["hbm_frac"] = round(w[1] / sec / PEAK_HBM_BPS, 4)
        else:
            peak = PEAK_INT8_OPS if w[0] == "ops" else PEAK_BF16_FLOPS
            entry["kind"] = "int8" if w[0] == "ops" else "bf16"
            entry["alg_ops"] = w[1]
            entry["alg_bytes"] = w[2]
            entry["TOPS"] = round(w[1] / sec / 1e12, 1)
            entry["mfma_frac"] = round(w[1] / sec / peak, 4)
            ai = w[1] / w[2]
            cap = min(peak, ai * PEAK_HBM_BPS)
            entry["roofline_cap_frac"] = round(cap / peak, 4)
            entry["roofline_frac"] = round(w[1] / sec / cap, 4)
        report[name] = entry
    return report


# ---------------------------------------------------------------------------
# HBM traffic per launch from rocprofv3 counters. `--pmc-probe` runs each op-step stage
# and a plain 256 MiB device copy a few times; run it once under
# `rocprofv3 --pmc FETCH_SIZE` and once under `--pmc WRITE_SIZE`, then
# `--traffic-summary FETCH_CSV WRITE_CSV` scales each stage's per-dispatch KiB by what the
# same counter reads for the copy (bytes known) and writes the summary that the default
# run reads for roofline.traffic.
# ---------------------------------------------------------------------------
TRAFFIC_FILE = REPO / "profiles" / f"op_step_M{M_TOK}_K{K_IN}_N{N_OUT}_hbm_traffic.md"
COPY_BYTES = 256 << 20
# rocprofv3 kernel-name fragments of each stage's launches (summed per launch)
STAGE_KERNELS = {
    "quant_rows": ["quant_rows_kernel<1, 0, false"],
    "fwd_gemm_packed": ["int8_gemm_m32_kernel<1,"],
    "sr_quant_rows": ["quant_rows_kernel<1, 0, true"],
    "grad_input_gemm": ["int8_gemm_m32_kernel<2,"],
    "grad_weight_partials": ["grad_weight_partial_kernel"],
    "ratchet_update_partials": ["ratchet_update_grad_kernel<2,"],
}
PROBE_REPEATS = 5


def pmc_probe(device) -> None:
    import torch

    layer, x, g = synthetic_layer(device)
    stages, _ = op_stages(layer, x, g)
    for _, fn in stages:
        fn()
    src = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device=device)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(PROBE_REPEATS):
        for _, fn in stages:
            fn()
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"pmc probe: {PROBE_REPEATS} x {len(stages)} stages + {COPY_BYTES} B copy")


def _per_dispatch_kib(csv_path: str, counter: str) -> list[tuple[str, float]]:
    import csv

    rows = []
    with open(csv_path, newline="") as f:
        for r in csv.DictReader(f):
            if r["Counter_Name"] == counter:
                rows.append((int(r["Dispatch_Id"]), r["Kernel_Name"], float(r["Counter_Value"])))
    rows.sort()
    return [(name, kib) for _, name, kib in rows]


def _stage_means(rows: list[tuple[str, float]]) -> tuple[dict, float]:
    """Mean KiB per launch of each stage (its kernels summed), and of the copy."""
    sums = {name: 0.0 for name in STAGE_KERNELS}
    counts = {name: 0 for name in STAGE_KERNELS}
    copies = [kib for name, kib in rows if "copy" in name.lower() and "rk::" not in name]
    # the calibration copies (setup copies of small tensors excluded)
    copy = [kib for kib in copies if kib >= 0.25 * max(copies, default=0.0)]
    for name, kib in rows:
        for stage, frags in STAGE_KERNELS.items():
            if any(f in name for f in frags):
                sums[stage] += kib
                counts[stage] += 1
    # every launch of a stage does the same work (the warm-up and the setup launches that
    # produce later stages' inputs included): the mean over all of them
    return ({k: v / max(counts[k], 1) for k, v in sums.items()},
            sum(copy) / max(len(copy), 1))


def traffic_summary(fetch_csv: str, write_csv: str) -> dict:
    fetch, fcopy = _stage_means(_per_dispatch_kib(fetch_csv, "FETCH_SIZE"))
    write, wcopy = _stage_means(_per_dispatch_kib(write_csv, "WRITE_SIZE"))
    f_scale = fcopy * 1024 / COPY_BYTES
    w_scale = wcopy * 1024 / COPY_BYTES
    from local_ai_training.int8_matmul import grad_weight_splits

    # the op step's gradient is bfloat16; the split count is the library's (host-side)
    work = stage_work(M_TOK, N_OUT, K_IN, 2, grad_weight_splits(M_TOK, N_OUT, K_IN))
    alg = {name: w[2] if len(w) > 2 else w[1] for name, w in work.items()}
    kernels = {}
    for stage in STAGE_KERNELS:
        fb = fetch[stage] * 1024 / f_scale
        wb = write[stage] * 1024 / w_scale
        kernels[stage] = {"fetch_bytes": round(fb), "write_bytes": round(wb),
                          "traffic_bytes": round(fb + wb), "alg_bytes": alg[stage],
                          "traffic_over_alg": round((fb + wb) / alg[stage], 3)}
    return {"copy_bytes": COPY_BYTES, "fetch_scale": round(f_scale, 4),
            "write_scale": round(w_scale, 4), "kernels": kernels}


def write_traffic_file(summary: dict, fetch_csv: str, write_csv: str) -> None:
    lines = [
        f"# HBM traffic per launch: int8 ratchet linear op step (M={M_TOK}, K={K_IN}, "
        f"N={N_OUT})",
        "",
        "Commands (repository root R on the MI355X box; the second runs the same probe with "
        "WRITE_SIZE):",
        "",
        "```",
        "cd /tmp && export TMPDIR=/tmp && rocprofv3 --pmc FETCH_SIZE -d $R/gpurun_out/pmc_fetch "
        "-o p --output-format csv -- python3 $R/bench.py --pmc-probe",
        "cd /tmp && export TMPDIR=/tmp && rocprofv3 --pmc WRITE_SIZE -d $R/gpurun_out/pmc_write "
        "-o p --output-format csv -- python3 $R/bench.py --pmc-probe",
        f"python3 $R/bench.py --traffic-summary {fetch_csv} {write_csv}",
        "```",
        "",
        f"Counters are KiB per dispatch. Calibration: a {COPY_BYTES >> 20} MiB device copy "
        f"reads FETCH_SIZE x {summary['fetch_scale']} and WRITE_SIZE x "
        f"{summary['write_scale']} of its true bytes; every figure below is divided by "
        "that factor.",
        "",
        "| stage | HBM read B | HBM write B | traffic B | algorithmic B | traffic / alg |",
        "|---|---:|---:|---:|---:|---:|",
    ]
    for stage, e in summary["kernels"].items():
        lines.append(f"| {stage} | {e['fetch_bytes']} | {e['write_bytes']} | "
                     f"{e['traffic_bytes']} | {e['alg_bytes']} | {e['traffic_over_alg']} |")
    lines += ["", "```json", json.dumps(summary), "```", ""]
    TRAFFIC_FILE.write_text("\n".join(lines))


# VALU issue peak: every SIMD issues one wave64 VALU instruction per 4 cycles (16 lanes per
# cycle; packed float32 doubles the lanes of its own instructions only).
PEAK_VALU_WAVE_INSTS = 1024 * 2.4e9 / 4
COUNTERS_FILE = REPO / "profiles" / f"op_step_M{M_TOK}_K{K_IN}_N{N_OUT}_counters.md"


def measured_valu_insts(kernel: str):
    """VALU wave instructions per launch of `kernel` from the committed counter summary."""
    if not COUNTERS_FILE.is_file():
        return None
    text = COUNTERS_FILE.read_text()
    start = text.find("```json")
    if start < 0:
        return None
    body = text[start + 7:text.find("```", start + 7)]
    try:
        return json.loads(body)[kernel]["VALU_insts"]
    except (ValueError, KeyError):
        return None


def measured_traffic(kernel: str):
    """HBM bytes per launch of `kernel` from the committed counter summary, or None."""
    if not TRAFFIC_FILE.is_file():
        return None
    text = TRAFFIC_FILE.read_text()
    start = text.find("```json")
    if start < 0:
        return None
    body = text[start + 7:text.find("```", start + 7)]
    try:
        return json.loads(body)["kernels"][kernel]["traffic_bytes"]
    except (ValueError, KeyError):
        return None


def headline_split(step_s: float, kernels: dict) -> dict:
    """The step's GEMM work by arithmetic: int8 (forward + grad_input, 2 x 2MNK ops) against
    the int8 MFMA peak and bf16 (grad_weight, 2MNK FLOPs) against the bf16 MFMA peak, per
    step time and per the kernels' own average launch times."""
    mnk2 = 2.0 * M_TOK * N_OUT * K_IN
    int8_us = kernels["fwd_gemm_packed"]["avg_us"] + kernels["grad_input_gemm"]["avg_us"]
    bf16_us = kernels["grad_weight_partials"]["avg_us"]
    int8_ops, bf16_flops = 2 * mnk2, mnk2
    return {
        "int8": {"ops_per_step": int8_ops, "kernels": ["fwd_gemm_packed", "grad_input_gemm"],
                 "TOPS_over_step": round(int8_ops / step_s / 1e12, 1),
                 "frac_int8_peak_over_step": round(int8_ops / step_s / PEAK_INT8_OPS, 4),
                 "kernel_us": round(int8_us, 2),
                 "TOPS_over_kernels": round(int8_ops / (int8_us * 1e-6) / 1e12, 1),
                 "frac_int8_peak_over_kernels": round(int8_ops / (int8_us * 1e-6) / PEAK_INT8_OPS,
                                                      4)},
        "bf16": {"flops_per_step": bf16_flops, "kernels": ["grad_weight_partials"],
                 "TFLOPs_over_step": round(bf16_flops / step_s / 1e12, 1),
                 "frac_bf16_peak_over_step": round(bf16_flops / step_s / PEAK_BF16_FLOPS, 4),
                 "kernel_us": round(bf16_us, 2),
                 "TFLOPs_over_kernels": round(bf16_flops / (bf16_us * 1e-6) / 1e12, 1),
                 "frac_bf16_peak_over_kernels": round(
                     bf16_flops / (bf16_us * 1e-6) / PEAK_BF16_FLOPS, 4)},
    }


def roofline_entry(kernels: dict) -> dict:
    """The dominant hand-written kernel (largest average time) against its roofline: MFMA
    kernels against their MFMA peak (int8 or bf16) unless their algorithmic bytes bound
    them first, elementwise kernels against HBM bandwidth. `traffic` is the measured HBM
    bytes per launch (counter summary), null if not measured."""
    name = max(kernels, key=lambda k: kernels[k]["avg_us"])
    e = kernels[name]
    sec = e["avg_us"] * 1e-6
    traffic = measured_traffic(name)
    if "alg_ops" in e:
        peak = PEAK_INT8_OPS if e.get("kind") == "int8" else PEAK_BF16_FLOPS
        ai = e["alg_ops"] / e["alg_bytes"]
        if ai * PEAK_HBM_BPS >= peak:
            achieved = e["alg_ops"] / sec / 1e12
            return {"kernel": name, "bound": "mfma", "achieved": round(achieved, 1),
                    "peak": peak / 1e12, "unit": "TFLOP/s",
                    "frac": round(achieved * 1e12 / peak, 4), "traffic": traffic,
                    "alg_ops_per_launch": e["alg_ops"], "alg_bytes_per_launch": e["alg_bytes"],
                    "avg_us": e["avg_us"]}
    achieved = e["alg_bytes"] / sec / 1e9
    entry = {"kernel": name, "bound": "hbm", "achieved": round(achieved, 1),
             "peak": PEAK_HBM_BPS / 1e9, "unit": "GB/s",
             "frac": round(achieved * 1e9 / PEAK_HBM_BPS, 4), "traffic": traffic,
             "alg_bytes_per_launch": e["alg_bytes"], "avg_us": e["avg_us"]}
    insts = measured_valu_insts(name)
    if insts:
        # the stochastic-rounding quant issues ~50 VALU instructions per element (Philox):
        # its binding roofline is VALU issue, reported beside the HBM one
        rate = insts / sec
        entry["valu"] = {"insts_per_launch": insts, "achieved": round(rate / 1e9, 1),
                         "peak": PEAK_VALU_WAVE_INSTS / 1e9, "unit": "G wave-instr/s",
                         "frac": round(rate / PEAK_VALU_WAVE_INSTS, 4)}
    return entry


# ---------------------------------------------------------------------------
# Per-stage SQ/GRBM counters of the op step (`--pmc-probe` under rocprofv3 --pmc, one run
# per counter group), averaged per launch. Derived figures use AMD's own definitions of
# the derived metrics rocprofv3 lists for gfx950:
#   MfmaUtil        = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE * SIMDs)
#   VALUBusy        = SQ_ACTIVE_INST_VALU / (CUs * GRBM_GUI_ACTIVE)
#   LDSBankConflict = SQ_LDS_BANK_CONFLICT / (CUs * GRBM_GUI_ACTIVE)
#   wait fraction   = SQ_WAIT_INST_ANY / SQ_WAVE_CYCLES (both in wave quad-cycles)
# GRBM_GUI_ACTIVE is taken per XCD (the CSV sums its 8 XCD instances; the metric takes the
# maximum, which for one kernel on the whole chip is the sum / 8).
# ---------------------------------------------------------------------------
MI355X_CUS, MI355X_SIMDS, MI355X_XCDS = 256, 1024, 8


def _counter_rows(csv_paths: list[str]) -> dict:
    """{dispatch id: {"name": kernel, counter: value, ...}} over every CSV."""
    import csv

    out: dict = {}
    for i, path in enumerate(csv_paths):
        with open(path, newline="") as f:
            for r in csv.DictReader(f):
                key = (i, int(r["Dispatch_Id"]))
                d = out.setdefault(key, {"name": r["Kernel_Name"]})
                d[r["Counter_Name"]] = d.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
    return out


def counter_summary(csv_paths: list[str]) -> str:
    rows = _counter_rows(csv_paths)
    per_stage: dict = {s: {} for s in STAGE_KERNELS}
    for d in rows.values():
        for stage, frags in STAGE_KERNELS.items():
            if any(f in d["name"] for f in frags):
                for c, v in d.items():
                    if c != "name":
                        per_stage[stage].setdefault(c, []).append(v)
    lines = ["| stage | counter | mean per launch | launches |", "|---|---|---:|---:|"]
    derived = {}
    for stage, cs in per_stage.items():
        mean = {c: sum(v) / len(v) for c, v in cs.items()}
        for c in sorted(mean):
            lines.append(f"| {stage} | {c} | {mean[c]:.4g} | {len(cs[c])} |")
        grbm = mean.get("GRBM_GUI_ACTIVE")
        d = {}
        if grbm:
            cyc = grbm / MI355X_XCDS
            d["gpu_cycles"] = round(cyc)
            d["us_at_2.4GHz"] = round(cyc / 2.4e3, 2)
            if "SQ_VALU_MFMA_BUSY_CYCLES" in mean:
                d["MfmaUtil"] = round(mean["SQ_VALU_MFMA_BUSY_CYCLES"] / (cyc * MI355X_SIMDS), 4)
            if "SQ_ACTIVE_INST_VALU" in mean:
                d["VALUBusy"] = round(mean["SQ_ACTIVE_INST_VALU"] / (cyc * MI355X_CUS), 4)
            if "SQ_LDS_BANK_CONFLICT" in mean:
                d["LDSBankConflict"] = round(mean["SQ_LDS_BANK_CONFLICT"] / (cyc * MI355X_CUS), 4)
        if mean.get("SQ_WAVE_CYCLES"):
            if "SQ_WAIT_INST_ANY" in mean:
                d["wait_inst_frac"] = round(mean["SQ_WAIT_INST_ANY"] / mean["SQ_WAVE_CYCLES"], 4)
            if "SQ_WAIT_ANY" in mean:
                d["wait_any_frac"] = round(mean["SQ_WAIT_ANY"] / mean["SQ_WAVE_CYCLES"], 4)
        if mean.get("SQ_INSTS_VALU_MFMA_MOPS_I8"):
            d["mfma_i8_ops"] = mean["SQ_INSTS_VALU_MFMA_MOPS_I8"] * 512
        if mean.get("SQ_INSTS_VALU_MFMA_MOPS_BF16"):
            d["mfma_bf16_flops"] = mean["SQ_INSTS_VALU_MFMA_MOPS_BF16"] * 512
        if "SQ_INSTS_VALU" in mean:
            d["VALU_insts"] = round(mean["SQ_INSTS_VALU"])  # wave instructions per launch
        if mean.get("SQ_WAVES"):
            for c in ("SQ_INSTS_VALU", "SQ_INSTS_MFMA", "SQ_INSTS_LDS", "SQ_INSTS_SALU",
                      "SQ_INSTS_VMEM_RD", "SQ_INSTS_VMEM_WR"):
                if c in mean:
                    d[c.replace("SQ_INSTS_", "") + "_per_wave"] = round(mean[c] / mean["SQ_WAVES"], 1)
        derived[stage] = d
    lines += ["", "Derived (per launch):", "", "```json", json.dumps(derived, indent=1), "```"]
    return "\n".join(lines)


# ---------------------------------------------------------------------------
# Per-step kernel classes of a training step (the reference buckets its step the same way
# in scripts/int8_step_profile.py:26-38), from a rocprofv3 --kernel-trace CSV of
# `--train-only`: the timed steps are the last STEPS repeats of the replayed kernel
# sequence.
# ---------------------------------------------------------------------------
STEP_CLASSES = [
    ("int8 GEMM forward (W8A8, packed codes)", r"int8_gemm_(m32|nt|pipe)_kernel<[01],|int8_gemv"),
    ("int8 GEMM grad_input (packed codes, in place)", r"int8_gemm_(m32|pipe)_kernel<2,"),
    ("SR gradient quant (Philox)", r"quant_rows_kernel<\d+, \d+, true"),
    ("activation quant prologues (RMSNorm/GELU/transpose)", r"quant_rows_kernel<\d+, \d+, false"),
    ("bf16 grad_weight (MFMA)", r"grad_weight_(partial|reduce)_kernel"),
    ("fused ratchet update", r"ratchet_update|row_rms_(segment_)?mean"),
    ("prologue backward (RMSNorm/GELU)", r"rmsnorm_bwd|rmsnorm_gw_reduce|gelu_bwd"),
    ("attention (HIP forward, torch memory-efficient backward)", r"attn|fmha|flash|bwd_preprocess|bwd_postprocess"),
    ("bf16 grad_input (lm_head, MFMA on packed codes)", r"grad_input_bf16_kernel|effective_fragments"),
    ("bf16 GEMM (hipBLASLt)", r"Cijk_|gemm"),
    ("effective bf16 weights", r"effective_bf16"),
    ("optimizer (AdamW)", r"multi_tensor|adam"),
    ("loss (cross-entropy) / reductions", r"xent|reduce|softmax|nll|cross_entropy"),
    ("elementwise / cast / copy", r"elementwise|copy|cast|fill|vectorized|index|embedding"),
]


def step_summary(trace_csv: str, steps: int) -> str:
    import csv
    import re

    recs = []
    with open(trace_csv, newline="") as f:
        for r in csv.DictReader(f):
            recs.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"]))
    recs.sort()
    names = [n for _, _, n in recs]
    # the replayed step's kernels: the shortest period p whose last `steps` windows launch
    # the same kernels (as multisets: kernels of two streams may start in either order)
    from collections import Counter

    period = None
    for p in range(1, len(names) // steps + 1):
        tail = names[len(names) - p * steps:]
        first = Counter(tail[:p])
        if all(Counter(tail[i * p:(i + 1) * p]) == first for i in range(1, steps)):
            period = p
            break
    if period is None:
        raise SystemExit("no repeated step sequence in the trace")
    timed = recs[len(recs) - period * steps:]
    wall_ns = timed[-1][1] - timed[0][0]
    classes: dict = {}
    for s, e, n in timed:
        label = next((lab for lab, pat in STEP_CLASSES if re.search(pat, n, re.I)),
                     "other: " + n[:60])
        c = classes.setdefault(label, [0.0, 0])
        c[0] += (e - s) / 1e3
        c[1] += 1
    busy = sum(v[0] for v in classes.values())
    lines = [f"kernels per step: {period}; wall per step (first start to last end over "
             f"{steps} steps): {wall_ns / 1e3 / steps:.1f} us; kernel time per step: "
             f"{busy / steps:.1f} us ({busy * 1e3 / wall_ns * 100:.1f}% of wall)", "",
             "| kernel class | us / step | % of kernel time | launches / step |",
             "|---|---:|---:|---:|"]
    for label, (us, cnt) in sorted(classes.items(), key=lambda kv: -kv[1][0]):
        lines.append(f"| {label} | {us / steps:.1f} | {us / busy * 100:.1f} | "
                     f"{cnt // steps} |")
    return "\n".join(lines)


TRAIN_25M = dict(model="ratchet-gpt-25M", vocab=8192, block=512, batch=32, n_layer=8, n_head=8,
                 n_embd=512, ffn=2048, max_code=MAX_CODE, codes="quinary")
TRAIN_1B = dict(model="ratchet-gpt-1B", vocab=8192, block=1024, batch=8, n_layer=24, n_head=16,
                n_embd=2048, ffn=5632, max_code=3, codes="septenary")


def train_bench(shape: dict, steps: int, warmup: int, device, graph: bool,
                defer_updates: bool = True):
    """Training tokens/s of a ratchet transformer (int8 + int8_backward, fused update every
    step, AdamW on the float parameters, Zipf(1.1) token ids), sustained: syncs only at both
    ends of the timed steps. ``graph``: the step is captured once as a HIP graph and
    replayed (training.CapturedTrainingStep: SR seeds drawn on the host per replay, in the
    eager order; capturable AdamW); otherwise the eager step (training.training_step)."""
    import numpy as np
    import torch

    from local_ai_training.model import ModelConfig, build_seeded_model
    from local_ai_training.training import CapturedTrainingStep, training_step

    vocab, block, batch = shape["vocab"], shape["block"], shape["batch"]
    config = ModelConfig(vocab_size=vocab, block_size=block, n_layer=shape["n_layer"],
                         n_head=shape["n_head"], n_embd=shape["n_embd"],
                         ffn_hidden=shape["ffn"], matmul_mode="int8", int8_backward=True)
    model = build_seeded_model(config, max_code=shape["max_code"], seed=1337).to(device).train()
    # the layers' fused updates batched after backward (a few launches for the whole model);
    # defer_updates=False keeps one update launch per layer inside backward (A/B runs)
    model.defer_ratchet_updates(defer_updates)
    # capturable (device-side step count) in both modes: the same AdamW arithmetic, so the
    # eager and graph runs of the same steps end at the same loss; torch's fused AdamW (one
    # kernel for every parameter; the same update as the reference's foreach AdamW up to
    # float rounding)
    optimizer = torch.optim.AdamW(model.parameters(), lr=3e-4, weight_decay=0.0,
                                  capturable=True, fused=True)
    rng = np.random.default_rng(1337)
    ids = (rng.zipf(1.1, size=batch * (block + 1)) - 1) % vocab  # Zipf(s=1.1) token ids
    tokens = torch.from_numpy(ids.astype(np.uint16).astype(np.int64)).view(batch, block + 1)
    tokens = tokens.to(device)
    inputs, targets = tokens[:, :block], tokens[:, 1:]
    # the SR seeds come from the CPU generator (one draw per int8-backward layer and step):
    # seed it, so the run (and its loss) does not depend on what ran before
    torch.manual_seed(1337)
    if graph:
        # the capture's own warm-up steps count toward `warmup`
        step = CapturedTrainingStep(model, optimizer, inputs, targets, warmup_steps=2)
        warmup = max(warmup - 2, 0)
    else:
        def step():
            return training_step(model, optimizer, inputs, targets, check_finite=False,
                                 autocast_cache=False)[0]
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        loss = step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    final_loss = float(loss.detach())
    del model, optimizer, step
    torch.cuda.empty_cache()
    return batch * block * steps / elapsed, elapsed / steps, final_loss


def model_bench(args, device, graph: bool):
    """25M ratchet transformer training tokens/s."""
    return train_bench(TRAIN_25M, args.model_steps, args.model_warmup, device, graph)


def hbm_probe(device, gib: float = 1.0) -> dict:
    """Practical HBM bandwidth of a plain streaming kernel (rk_hbm_stream): read-only and
    copy over `gib` GiB, swept over loads in flight per thread and grid size; the best of
    each and the full sweep. Copy counts read + write bytes."""
    import torch

    from local_ai_training import _native as nat

    nbytes = int(gib * (1 << 30))
    src = torch.empty(nbytes // 4, dtype=torch.int32, device=device).random_()
    dst = torch.empty(nbytes // 4, dtype=torch.int32, device=device)
    stream = nat.stream_handle(device)
    sweep = []
    for copy in (0, 1):
        for unroll in (2, 4, 8):
            for blocks in (1024, 2048, 4096, 8192):
                def run():
                    nat.call("rk_hbm_stream", src.data_ptr(), dst.data_ptr(), nbytes, copy,
                             unroll, blocks, stream)
                run()
                torch.cuda.synchronize()
                best = None
                for _ in range(3):
                    e0 = torch.cuda.Event(enable_timing=True)
                    e1 = torch.cuda.Event(enable_timing=True)
                    e0.record()
                    for _ in range(5):
                        run()
                    e1.record()
                    torch.cuda.synchronize()
                    ms = e0.elapsed_time(e1) / 5
                    best = ms if best is None else min(best, ms)
                moved = nbytes * (2 if copy else 1)
                sweep.append({"mode": "copy" if copy else "read", "unroll": unroll,
                              "blocks": blocks, "us": round(best * 1e3, 1),
                              "TB_s": round(moved / (best * 1e-3) / 1e12, 3)})
    del src, dst
    torch.cuda.empty_cache()
    out = {"bytes": nbytes, "sweep": sweep}
    for mode in ("read", "copy"):
        top = max((e for e in sweep if e["mode"] == mode), key=lambda e: e["TB_s"])
        out[mode] = {"TB_s": top["TB_s"], "frac_hbm": round(top["TB_s"] * 1e12 / PEAK_HBM_BPS, 4),
                     "unroll": top["unroll"], "blocks": top["blocks"]}
    return out


def update_1b_bench(device, iters: int) -> dict:
    """The fused update of one 1B training step at full scale: every ratchet layer of the 1B
    septenary model (24 x qkv 6144x2048, proj 2048x2048, expand 5632x2048, contract
    2048x5632, then lm_head 8192x2048; 973 M weights), in model order, from what the
    training step hands it: the bf16 gradient grad_weight writes itself where it takes one
    split of 8192 tokens (2 B per weight), its float32 split partials elsewhere (4 B per
    weight and split). Packed states are 1 B read + 1 B written per weight. Beside it, the
    same sweep with every layer fed float32 partials (the earlier path). The data exceed the
    last-level cache, so every sweep streams them from HBM."""
    import torch

    from local_ai_training import _native as nat
    from local_ai_training.int8_matmul import grad_weight_splits

    tokens, mc = 8192, 3
    shapes = [(6144, 2048), (2048, 2048), (5632, 2048), (2048, 5632)] * 24 + [(8192, 2048)]
    gen = torch.Generator().manual_seed(11)
    counts = torch.zeros(4, dtype=torch.int64, device=device)
    flag = torch.zeros(1, dtype=torch.int32, device=device)
    stream = nat.stream_handle(device)

    def run(all_partials: bool) -> dict:
        layers = []
        for n, k in shapes:
            nsplit = grad_weight_splits(tokens, n, k)
            code = torch.randint(-mc, mc + 1, (n, k), generator=gen, dtype=torch.int8)
            packed = (((code + mc) & 0x0F) | (7 << 4)).to(torch.uint8).to(device)
            if nsplit == 1 and not all_partials:
                grad = torch.empty(n, k, device=device).normal_(0.0, 1e-3).to(torch.bfloat16)
            else:
                grad = torch.empty(nsplit, n, k, device=device).normal_(0.0, 1e-3)
            layers.append((packed, grad, nsplit, n, k, torch.empty(n, device=device)))

        def sweep():
            for packed, grad, nsplit, n, k, row_rms in layers:
                if grad.dtype == torch.bfloat16:
                    nat.call("rk_ratchet_update_grad", packed.data_ptr(), k, grad.data_ptr(),
                             nat.RK_BF16, k, n, k, mc, 8, 0.5, 1.5, 1e-8, None, 0.0, 1.0,
                             counts.data_ptr(), row_rms.data_ptr(), None, flag.data_ptr(),
                             None, stream)
                else:
                    nat.call("rk_ratchet_update_partials", packed.data_ptr(), k,
                             grad.data_ptr(), nsplit, n, k, mc, 8, 0.5, 1.5, 1e-8, None, 0.0,
                             1.0, counts.data_ptr(), row_rms.data_ptr(), None, flag.data_ptr(),
                             None, None, k, stream)

        # the batched form the training step takes (RatchetGPT.defer_ratchet_updates): one
        # rk_ratchet_update_multi launch per gradient source and row-length class
        groups: dict = {}
        for packed, grad, nsplit, n, k, row_rms in layers:
            src = nat.RK_BF16 if grad.dtype == torch.bfloat16 else nat.RK_UPDATE_SRC_SPLITS
            chunks = (k + 511) // 512
            groups.setdefault((src, 4 if chunks <= 4 else 12, nsplit == 1), []).append(
                (packed, grad, nsplit, n, k, row_rms))
        tables = []
        for (src, _, _), group in groups.items():
            entries = (nat.UpdateLayer * len(group))()
            row = 0
            for d, (packed, grad, nsplit, n, k, row_rms) in zip(entries, group):
                d.packed, d.g = packed.data_ptr(), grad.data_ptr()
                d.counts, d.row_rms, d.nonfinite = (counts.data_ptr(), row_rms.data_ptr(),
                                                    flag.data_ptr())
                d.ldp, d.ldg, d.rows, d.K, d.row_begin = k, k, n, k, row
                d.max_code, d.threshold, d.nsplit = mc, 8, nsplit
                d.low, d.high, d.eps, d.beta1, d.beta2 = 0.5, 1.5, 1e-8, 0.0, 1.0
                row += n
            host = torch.frombuffer(bytearray(ctypes.string_at(ctypes.addressof(entries),
                                                               ctypes.sizeof(entries))),
                                    dtype=torch.uint8)
            tables.append((src, len(group), host, host.to(device)))

        def batched():
            for src, count, host, dev in tables:
                nat.call("rk_ratchet_update_multi", host.data_ptr(), dev.data_ptr(), count, src,
                         stream)

        def timed(fn) -> float:
            fn()
            torch.cuda.synchronize()
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(iters):
                fn()
            e1.record()
            torch.cuda.synchronize()
            return e0.elapsed_time(e1) * 1e-3 / iters

        sweep_s = timed(sweep)
        batched_s = timed(batched)
        alg = sum(n * k * (2 + (2 if g.dtype == torch.bfloat16 else 4 * nsp)) + 4 * n
                  for _, g, nsp, n, k, _ in layers)
        del layers, tables
        torch.cuda.empty_cache()

        def rate(sec: float) -> dict:
            return {"ms": round(sec * 1e3, 3), "GB_s": round(alg / sec / 1e9, 1),
                    "frac_hbm": round(alg / sec / PEAK_HBM_BPS, 4)}

        return {"alg_bytes": alg, "launches": len(groups), **rate(batched_s),
                "per_layer": {"launches": len(shapes), **rate(sweep_s)}}

    step = run(False)
    partials = run(True)
    return {"workload": "fused update of every 1B ratchet layer from what its backward hands "
                        "it (bf16 gradient at one split, float32 split partials otherwise), "
                        "batched per gradient source and row length (rk_ratchet_update_multi); "
                        "per_layer: one launch per layer",
            "weights": sum(n * k for n, k in shapes), **step,
            "all_partials": {"workload": "every layer from float32 split partials", **partials}}


DECODE_LAYERS = dict(vocab=8192, block=1024, n_layer=24, n_head=16, n_embd=2048, ffn=5632)
DECODE_MAX_CODE = 3


def decode_model(device):
    """The 1B septenary ratchet transformer (24 layers, d 2048, 16 heads, FFN 5632, vocab
    8192, block 1024) in int8 inference mode."""
    from local_ai_training.model import ModelConfig, build_seeded_model

    d = DECODE_LAYERS
    config = ModelConfig(vocab_size=d["vocab"], block_size=d["block"], n_layer=d["n_layer"],
                         n_head=d["n_head"], n_embd=d["n_embd"], ffn_hidden=d["ffn"],
                         matmul_mode="int8")
    return build_seeded_model(config, max_code=DECODE_MAX_CODE, seed=1337).to(device).eval()


def decode_weight_bytes(model) -> int:
    """Bytes every decode step must stream: packed codes + fp32 row scales of every ratchet
    layer (the GEMVs read each weight once per step)."""
    from local_ai_training.ratchet import DiscreteRatchetLinear

    return sum(m.packed.numel() + 4 * m.packed.shape[0] for m in model.modules()
               if isinstance(m, DiscreteRatchetLinear))


def gemv_chain(model, batch: int, device, iters: int) -> dict:
    """Every ratchet GEMV of one decode step as the fused decode path runs it (qkv and
    expand: RMSNorm+quant prologue; proj and contract: per-token quant prologue with the
    residual add; lm_head: RMSNorm prologue), in model order over all 24 layers (0.97 GB
    of packed codes, more than the last-level cache), on seeded float32 activations. HIP
    events on the launch stream around each launch give the per-kind averages."""
    import torch

    from local_ai_training import decode as dec

    gen = torch.Generator().manual_seed(3)
    c, f = model.config.n_embd, model.config.hidden_size

    def rows(width):
        return (torch.randn(batch, width, generator=gen) * 2.0).to(device)

    hidden, att, ffn_in = rows(c), rows(c), rows(f)
    qkv = torch.empty(batch, 3 * c, dtype=torch.bfloat16, device=device)
    ffn = torch.empty(batch, f, dtype=torch.float32, device=device)
    logits = torch.empty(batch, model.config.vocab_size, dtype=torch.float32, device=device)
    residual = rows(c)
    calls = []
    for block in model.blocks:
        calls += [
            ("qkv", block.attention.qkv, qkv, dict(prologue=dec.PRO_RMSNORM,
             epilogue=dec.EPI_STORE, x=hidden, norm_weight=block.attention_norm.weight,
             eps=dec.BLOCK_NORM_EPS)),
            ("projection", block.attention.projection, residual,
             dict(prologue=dec.PRO_PLAIN, epilogue=dec.EPI_ADD, x=att)),
            ("expand", block.feed_forward.expand, ffn, dict(prologue=dec.PRO_RMSNORM,
             epilogue=dec.EPI_GELU, x=hidden, norm_weight=block.feed_forward_norm.weight,
             eps=dec.BLOCK_NORM_EPS)),
            ("contract", block.feed_forward.contract, residual,
             dict(prologue=dec.PRO_PLAIN, epilogue=dec.EPI_ADD, x=ffn_in)),
        ]
    calls.append(("lm_head", model.lm_head, logits, dict(prologue=dec.PRO_RMSNORM,
                  epilogue=dec.EPI_STORE, x=hidden, norm_weight=model.final_norm.weight,
                  eps=float(torch.finfo(torch.float32).eps))))

    def run(events=None):
        for i, (_, layer, out, kw) in enumerate(calls):
            if events is not None:
                events[i][0].record()
            dec.decode_gemv(layer, out, **kw)
            if events is not None:
                events[i][1].record()

    run()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(iters):
        run()
    torch.cuda.synchronize()
    chain_s = (time.perf_counter() - t0) / iters
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in calls]
    per_kind: dict = {}
    for _ in range(iters):
        run(events)
        torch.cuda.synchronize()
        for (kind, layer, _, _), (e0, e1) in zip(calls, events):
            n, k = layer.packed.shape
            e = per_kind.setdefault(kind, {"N": n, "K": k, "count": 0, "us": 0.0})
            e["count"] += 1
            e["us"] += e0.elapsed_time(e1) * 1e3

    def alg_bytes(n, k):
        # packed codes + row scales, activation rows (f32) in, outputs (bf16 / f32) out
        return n * k + 4 * n + 4 * batch * k + 4 * batch * n

    kinds = {}
    for kind, e in per_kind.items():
        n, k = e["N"], e["K"]
        us = e["us"] / e["count"]
        alg = alg_bytes(n, k)
        kinds[kind] = {"N": n, "K": k, "avg_us": round(us, 2), "alg_bytes": alg,
                       "GB_s": round(alg / us / 1e3, 1),
                       "frac": round(alg / us * 1e6 / PEAK_HBM_BPS, 4)}
    total = sum(alg_bytes(*layer.packed.shape) for _, layer, _, _ in calls)
    return {"launches": len(calls), "chain_us": round(chain_s * 1e6, 1),
            "chain_GB_s": round(total / chain_s / 1e9, 1),
            "chain_frac": round(total / chain_s / PEAK_HBM_BPS, 4), "kinds": kinds}


def decode_bench(args, device) -> dict:
    """KV-cached int8 decode of the 1B model at a 1024-token window: batch 1 and 16, a
    prompt of 1024 - steps tokens prefilled, then `steps` greedy decode steps replayed as
    one HIP graph each (argmax feeds the next token on the device, no host sync)."""
    import numpy as np
    import torch

    from local_ai_training.decode import fused_decode_supported
    from local_ai_training.generate import DecodeGraph

    d = DECODE_LAYERS
    model = decode_model(device)
    weight_bytes = decode_weight_bytes(model)
    steps = min(args.decode_steps, d["block"] - 1)
    prompt_len = d["block"] - steps
    head = d["n_embd"] // d["n_head"]
    out = {"config": {"workload": "KV-cached int8 decode, 1B septenary ratchet transformer",
                      "n_layer": d["n_layer"], "n_embd": d["n_embd"], "n_head": d["n_head"],
                      "ffn": d["ffn"], "vocab": d["vocab"], "window": d["block"],
                      "prompt": prompt_len, "steps": steps, "kv_dtype": "bf16",
                      "codes": "septenary"},
           "weight_bytes_per_step": weight_bytes}
    rng = np.random.default_rng(1337)
    for batch in args.decode_batches:
        ids = (rng.zipf(1.1, size=(batch, prompt_len)) - 1) % d["vocab"]
        tokens = torch.from_numpy(ids.astype(np.int64)).to(device)
        cache = model.new_cache(batch, dtype=torch.bfloat16)
        logits = model.prefill(tokens, cache)
        # the greedy graph picks each step's argmax into its token buffer and advances the
        # position itself
        graph = DecodeGraph(model, cache, greedy=True)
        first = logits.argmax(-1, keepdim=True)

        def run(count):
            for _ in range(count):
                graph.next_greedy()

        graph.tokens.copy_(first)
        run(min(args.warmup, steps))
        cache.length = prompt_len  # rewind: the timed steps rewrite the same positions
        cache.pos.fill_(prompt_len)
        graph.tokens.copy_(first)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        run(steps)
        torch.cuda.synchronize()
        step_s = (time.perf_counter() - t0) / steps
        # keys+values the attention reads per step (positions 0..p, bf16; p averaged over
        # the timed steps)
        mean_len = prompt_len + (steps + 1) / 2
        kv_bytes = int(d["n_layer"] * 2 * batch * d["n_head"] * mean_len * head * 2)
        chain = gemv_chain(model, batch, device, args.kernel_iters)
        entry = {"tokens_per_s": round(batch / step_s, 1), "ms_per_step": round(step_s * 1e3, 4),
                 "path": "fused" if fused_decode_supported(model, cache) else "modules",
                 "launches_per_step": 6 * d["n_layer"] + 3,  # + embed, lm_head, greedy pick
                 "weight_GB_s": round(weight_bytes / step_s / 1e9, 1),
                 "step_bytes": weight_bytes + kv_bytes,
                 "step_frac_hbm": round((weight_bytes + kv_bytes) / step_s / PEAK_HBM_BPS, 4),
                 "gemv": chain}
        out[f"batch_{batch}"] = entry
        log(f"decode B={batch}: {step_s * 1e3:.3f} ms/step -> {batch / step_s:.0f} tok/s; "
            f"GEMV chain {chain['chain_us']} us ({chain['chain_GB_s']} GB/s)")
        del graph, cache
        torch.cuda.empty_cache()
    return out


GEMM_SWEEP_SHAPES = [(16384, 512, 2048), (16384, 2048, 2048), (16384, 512, 8192),
                     (4096, 4096, 4096), (8192, 8192, 8192)]


def gemm_sweep(device, iters: int) -> list:
    """Forward GEMM on packed quinary codes (bf16 out, row and column scales) at the op
    shape and at larger K, where the 256 x 256 block tiles take over (K >= 1024): device
    time per launch from HIP events on the launch stream, TOPS and % of the int8 peak."""
    import torch

    from local_ai_training.int8_matmul import packed_int8_mm

    out_rows = []
    gen = torch.Generator().manual_seed(5)
    for m, k, n in GEMM_SWEEP_SHAPES:
        q = torch.randint(-127, 128, (m, k), generator=gen, dtype=torch.int8).to(device)
        ls = (torch.rand(m, generator=gen) + 0.5).to(device)
        code = torch.randint(-MAX_CODE, MAX_CODE + 1, (n, k), generator=gen)
        packed = (((code + MAX_CODE) & 0x0F) | (7 << 4)).to(torch.uint8).to(device)
        rs = (torch.rand(n, generator=gen) * 0.08 + 0.02).to(device)

        def run():
            packed_int8_mm(q, packed, MAX_CODE, ls, rs)

        for _ in range(3):
            run()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(iters):
            run()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) / iters * 1e3
        tops = 2.0 * m * n * k / us / 1e6
        out_rows.append({"M": m, "K": k, "N": n, "avg_us": round(us, 2), "TOPS": round(tops, 1),
                         "mfma_frac": round(tops * 1e12 / PEAK_INT8_OPS, 4),
                         "tiles": "256x256" if k >= 1024 else "128x128"})
        log(f"  gemm {m}x{k}x{n}: {us:.1f} us {tops:.0f} TOPS")
    return out_rows


def host_info() -> dict:
    """The host CPU's model string (first "model name" of /proc/cpuinfo) and the torch
    version the CPU baseline ran on."""
    import platform

    import torch

    model = platform.processor() or "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "torch": torch.__version__}


def cpu_baseline(seconds: float) -> dict:
    import torch

    from oracle.cpu_reference import fp32_ratchet_linear_step

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    m_sample = M_TOK
    gen = torch.Generator().manual_seed(7)
    code = torch.randint(-MAX_CODE, MAX_CODE + 1, (N_OUT, K_IN), generator=gen)
    packed = (((code + MAX_CODE) & 0x0F) | (7 << 4)).to(torch.uint8)
    scale = torch.rand(N_OUT, generator=gen) * 0.08 + 0.02
    x = torch.randn(m_sample, K_IN, generator=gen)
    g = torch.randn(m_sample, N_OUT, generator=gen) * 1e-2
    fp32_ratchet_linear_step(x, packed, scale, g, MAX_CODE)  # warm
    iters, t0 = 0, time.perf_counter()
    while True:
        fp32_ratchet_linear_step(x, packed, scale, g, MAX_CODE)
        iters += 1
        if time.perf_counter() - t0 >= seconds and iters >= 2:
            break
    per_step = (time.perf_counter() - t0) / iters
    ops = 3 * 2.0 * m_sample * N_OUT * K_IN
    return {"value": round(ops / per_step / 1e12, 4), "unit": "TOPS", "cores": threads,
            "kind": "port", **host_info(),
            "sample": f"fp32 eager torch ratchet linear fwd+bwd+tiled update, M={m_sample} of "
                      f"{M_TOK} tokens, K={K_IN}, N={N_OUT}, {iters} steps, "
                      f"{per_step * 1e3:.1f} ms/step"}


def cpu_baseline_model() -> dict:
    """The reference's CPU training path at its tiny CPU config (2 layers, d 128, 4 heads,
    FFN 512, byte vocab 256, seq 64, batch 8, quinary codes; fp32 ratchet linears with the
    update fused into backward, bf16 autocast, AdamW): 20 steps, tokens/s over steps 3-20,
    on the host's cores."""
    import torch

    from oracle.cpu_reference import tiny_training_tokens_per_s

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    r = tiny_training_tokens_per_s()
    return {"value": round(r["tokens_per_s"], 1), "unit": "tokens/s", "cores": threads,
            "kind": "port", **host_info(),
            "sample": f"tiny ratchet transformer (2L, d128, 4h, FFN 512, vocab 256, seq 64, "
                      f"batch 8) fp32 eager + bf16 autocast training, {r['timed_steps']} of "
                      f"{r['steps']} steps timed, {r['ms_per_step']:.1f} ms/step, loss "
                      f"{r['first_loss']:.3f} -> {r['last_loss']:.3f}"}


def main() -> int:
    args = parse_args()
    if args.traffic_summary:
        summary = traffic_summary(*args.traffic_summary)
        write_traffic_file(summary, *args.traffic_summary)
        print(json.dumps(summary), flush=True)
        return 0
    if args.counter_summary:
        print(counter_summary(args.counter_summary), flush=True)
        return 0
    if args.step_summary:
        print(step_summary(args.step_summary[0], int(args.step_summary[1])), flush=True)
        return 0
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported by this "
              "build (single-GPU ratchet-linear path)", file=sys.stderr)
        return 2
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 1
    device = torch.device("cuda:0")
    if args.pmc_probe:
        pmc_probe(device)
        return 0
    if args.decode_only:
        print(json.dumps({"decode": decode_bench(args, device)}), flush=True)
        return 0
    if args.hbm_probe:
        print(json.dumps({"hbm_probe": hbm_probe(device)}), flush=True)
        return 0
    if args.update_1b_only:
        print(json.dumps({"update_1b": update_1b_bench(device, 5)}), flush=True)
        return 0
    if args.gemm_sweep:
        print(json.dumps({"gemm_sweep": gemm_sweep(device, args.kernel_iters)}), flush=True)
        return 0
    if args.train_only:
        shape = TRAIN_25M if args.train_only == "25m" else TRAIN_1B
        log(f"training only: {shape['model']}, warmup={args.warmup} steps={args.steps}")
        tok_s, step_s, loss = train_bench(shape, args.steps, args.warmup, device,
                                          graph=not args.no_graph,
                                          defer_updates=not args.immediate_updates)
        print(json.dumps({"model": shape["model"], "tokens_per_s": round(tok_s, 1),
                          "ms_per_step": round(step_s * 1e3, 3), "loss": round(loss, 5),
                          "steps": args.steps, "graph": not args.no_graph,
                          "deferred_updates": not args.immediate_updates}), flush=True)
        return 0
    log(f"op bench: M={M_TOK} K={K_IN} N={N_OUT} warmup={args.warmup} steps={args.steps}")
    step_s, eager_s, layer, x, g = op_bench(args, device)
    ops = 3 * 2.0 * M_TOK * N_OUT * K_IN
    tops = ops / step_s / 1e12
    log(f"op step {step_s * 1e3:.3f} ms -> {tops:.1f} TOPS (eager autograd step "
        f"{eager_s * 1e3:.3f} ms)")
    kernels = kernel_breakdown(layer, x, g, args.kernel_iters)
    for name, e in kernels.items():
        log(f"  {name}: {e}")
    result = {
        "metric": METRIC,
        "value": round(tops, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_s * 1e3, 4),
        "eager_ms_per_step": round(eager_s * 1e3, 4),
        "step_mode": "eager" if args.no_graph else "hip_graph",
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "int8 ratchet linear fwd+bwd+fused update (int8_backward)",
                   "M": M_TOK, "K": K_IN, "N": N_OUT, "codes": "quinary",
                   "batch": 32, "seq_len": 512, "parallelism": "none"},
        "split": headline_split(step_s, kernels),
        "kernels": kernels,
        "roofline": roofline_entry(kernels),
    }
    if not args.no_model:
        log(f"model bench: 25M int8, warmup={args.model_warmup} steps={args.model_steps}")
        tok_s, step_m, loss = model_bench(args, device, graph=True)
        log(f"model (HIP graph) {step_m * 1e3:.2f} ms/step -> {tok_s:.0f} tok/s "
            f"(loss {loss:.4f})")
        tok_e, step_e, loss_e = model_bench(args, device, graph=False)
        log(f"model (eager) {step_e * 1e3:.2f} ms/step -> {tok_e:.0f} tok/s (loss {loss_e:.4f})")
        result["train_tokens_per_s"] = round(tok_s, 1)
        result["train_ms_per_step"] = round(step_m * 1e3, 3)
        result["train_step_mode"] = "hip_graph"
        result["train_eager"] = {"tokens_per_s": round(tok_e, 1),
                                 "ms_per_step": round(step_e * 1e3, 3)}
        result["train_loss"] = {"hip_graph": round(loss, 5), "eager": round(loss_e, 5)}
        result["train_config"] = {"model": "ratchet-gpt-25M", "n_layer": 8, "n_embd": 512,
                                  "n_head": 8, "ffn": 2048, "vocab": 8192, "seq_len": 512,
                                  "batch": 32, "matmul_mode": "int8", "int8_backward": True,
                                  "steps": args.model_steps, "warmup": args.model_warmup}
    if not args.no_update_1b:
        log("update bench: the fused update of every 1B layer from split partials")
        result["update_1b"] = update_1b_bench(device, 5)
        log(f"  {result['update_1b']}")
    if not args.no_train_1b:
        log(f"1B training bench: warmup={args.train_1b_warmup} steps={args.train_1b_steps}")
        tok_s, step_1b, loss_1b = train_bench(TRAIN_1B, args.train_1b_steps,
                                              args.train_1b_warmup, device, graph=True)
        log(f"1B model (HIP graph) {step_1b * 1e3:.1f} ms/step -> {tok_s:.0f} tok/s "
            f"(loss {loss_1b:.3f})")
        tok_e, step_e, loss_e = train_bench(TRAIN_1B, args.train_1b_steps,
                                            args.train_1b_warmup, device, graph=False)
        log(f"1B model (eager) {step_e * 1e3:.1f} ms/step -> {tok_e:.0f} tok/s")
        result["train_1b"] = {"tokens_per_s": round(tok_s, 1),
                              "ms_per_step": round(step_1b * 1e3, 2), "step_mode": "hip_graph",
                              "eager": {"tokens_per_s": round(tok_e, 1),
                                        "ms_per_step": round(step_e * 1e3, 2)},
                              "loss": {"hip_graph": round(loss_1b, 4), "eager": round(loss_e, 4)},
                              "loss_note": "runs differ: torch's memory-efficient attention "
                                           "backward at head size 128 sums dq in a varying "
                                           "order (deterministic mode uses the flash kernel "
                                           "and repeats)",
                              "config": {k: TRAIN_1B[k] for k in TRAIN_1B},
                              "matmul_mode": "int8", "int8_backward": True}
    if not args.no_decode:
        log(f"decode bench: 1B int8, batches {args.decode_batches}, {args.decode_steps} steps")
        result["decode"] = decode_bench(args, device)
    if not args.no_cpu:
        log(f"cpu baseline: ~{args.cpu_seconds:.0f} s of fp32 eager CPU work")
        result["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
        result["cpu_baseline_model"] = cpu_baseline_model()
        log(f"  {result['cpu_baseline_model']}")
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
