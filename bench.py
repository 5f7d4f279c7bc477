#!/usr/bin/env python
"""Benchmark of the MI355X ratchet-linear hot path (one GPU).

Workload (value): one int8 ratchet linear training step at M=16384 tokens
(batch 32 x seq 512), K=512, N=2048, quinary codes, fp32 row scales U[0.02, 0.1],
BF16 activations N(0,1) quantized per token, BF16 upstream gradient N(0, 1e-2):
per-token quant -> W8A8 forward GEMM (packed codes) -> SR gradient quant ->
int8 grad_input GEMM -> BF16 grad_weight GEMM -> fused normalize+update. It runs
through the drop-in DiscreteRatchetLinear autograd path. ``value`` is the step's
TOPS over its three GEMMs (3 x 2*M*N*K ops; the int8 and bf16 halves are also
reported separately), inputs resident in HBM.

Also reported on the same line:
  kernels        per-kernel average launch time (HIP events on the launch stream) and
                 achieved TOPS / GB/s against the MI355X peaks
  roofline       the dominant hand-written kernel against its roofline
  train_tokens_per_s  the 25M ratchet transformer (8 layers, d 512, 8 heads, FFN 2048,
                 vocab 8192, seq 512, batch 32, int8 + int8_backward) full training step
  cpu_baseline   the reference's fp32 eager CPU path for the same op on a bounded
                 token sample, timed on this host's cores
"""

from __future__ import annotations

import argparse
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
    ap.add_argument("--model-steps", type=int, default=10)
    ap.add_argument("--model-warmup", type=int, default=3)
    ap.add_argument("--no-model", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--kernel-iters", type=int, default=20)
    ap.add_argument("--no-graph", action="store_true",
                    help="time the eager autograd step instead of its HIP-graph replay")
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

    from local_ai_training.int8_matmul import quantize_rows_into

    layer, x, g = synthetic_layer(device)
    x.requires_grad_(True)
    q = torch.empty(M_TOK, K_IN, dtype=torch.int8, device=device)
    s = torch.empty(M_TOK, dtype=torch.float32, device=device)

    def step():
        quantize_rows_into(x.detach(), q, s)
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
    # the host-side autograd and launch overhead of the eager step disappears. The SR
    # seed drawn on the host at capture time is part of the graph (same work per step).
    side = torch.cuda.Stream(device=device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream(device).wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for _ in range(args.warmup):
        graph.replay()
    graph_s = timed(graph.replay, args.steps)
    return graph_s, eager_s, layer, x.detach(), g


def kernel_breakdown(layer, x, g, iters: int):
    """Average device time of each launch of one op step, HIP events on the launch stream."""
    import torch

    from local_ai_training import _native as nat
    from local_ai_training.int8_matmul import (
        grad_weight_bf16,
        grad_weight_splits,
        int8_mm_nt,
        packed_int8_mm,
        quantize_rows_into,
        unpack_transpose,
    )

    dev = x.device
    m, k = x.shape
    n = layer.out_features
    packed, scale = layer.packed, layer.scale.float().contiguous()
    q = torch.empty(m, k, dtype=torch.int8, device=dev)
    s = torch.empty(m, dtype=torch.float32, device=dev)
    out = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
    gq = torch.empty(m, n, dtype=torch.int8, device=dev)
    gs = torch.empty(m, dtype=torch.float32, device=dev)
    gin = torch.empty(m, k, dtype=torch.bfloat16, device=dev)
    gw = torch.empty(n, k, dtype=torch.bfloat16, device=dev)
    splits = grad_weight_splits(m, n, k)
    gw_work = torch.empty(splits, n, k, dtype=torch.float32, device=dev)
    counts = torch.zeros(4, dtype=torch.int64, device=dev)
    row_rms = torch.empty(n, dtype=torch.float32, device=dev)
    flag = torch.zeros(1, dtype=torch.int32, device=dev)
    holder = {}

    def update():
        nat.call("rk_ratchet_update_grad", packed.data_ptr(), k, gw.data_ptr(), nat.RK_BF16, k,
                 n, k, MAX_CODE, 8, 0.5, 1.5, 1e-8, None, 0.0, 1.0, counts.data_ptr(),
                 row_rms.data_ptr(), None, flag.data_ptr(), nat.stream_handle(dev))

    stages = [
        ("quant_rows", lambda: quantize_rows_into(x, q, s)),
        ("fwd_gemm_packed", lambda: packed_int8_mm(q, packed, MAX_CODE, s, scale, out=out)),
        ("sr_quant_rows", lambda: quantize_rows_into(g, gq, gs, col_scale=scale,
                                                     stochastic=True, seed=12345)),
        ("unpack_transpose", lambda: holder.__setitem__("ct", unpack_transpose(packed,
                                                                               MAX_CODE))),
        ("grad_input_gemm", lambda: int8_mm_nt(gq, holder["ct"], gs, None, out=gin)),
        ("grad_weight_bf16", lambda: grad_weight_bf16(g, q, s, splits, out=gw, work=gw_work)),
        ("ratchet_update_grad", update),
    ]
    for _, fn in stages:  # warm
        fn()
    torch.cuda.synchronize()
    events = {name: [] for name, _ in stages}
    for _ in range(iters):
        for name, fn in stages:
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record()
            fn()
            e1.record()
            events[name].append((e0, e1))
    torch.cuda.synchronize()
    avg_ms = {name: sum(a.elapsed_time(b) for a, b in ev) / len(ev) for name, ev in events.items()}

    mnk2 = 2.0 * m * n * k
    work = {  # name: (kind, algorithmic amount per launch)
        "quant_rows": ("bytes", m * k * 2 + m * k + m * 4),
        "fwd_gemm_packed": ("ops", mnk2, m * k + n * k + m * n * 2 + m * 4 + n * 4),
        "sr_quant_rows": ("bytes", m * n * 2 + m * n + m * 4 + n * 4),
        "unpack_transpose": ("bytes", 2 * n * k),
        "grad_input_gemm": ("ops", mnk2, m * n + n * k + m * k * 2 + m * 4),
        "grad_weight_bf16": ("flops", mnk2, m * n * g.element_size() + m * k + m * 4
                             + n * k * 2),
        "ratchet_update_grad": ("bytes", n * k * (1 + 2 + 1) + n * 4),
    }
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


def roofline_entry(kernels: dict) -> dict:
    """The dominant hand-written kernel (largest average time, BLAS excluded)."""
    own = {k: v for k, v in kernels.items() if not k.endswith("_blas")}
    name = max(own, key=lambda k: own[k]["avg_us"])
    e = own[name]
    sec = e["avg_us"] * 1e-6
    if "alg_ops" in e:
        ai = e["alg_ops"] / e["alg_bytes"]
        if ai * PEAK_HBM_BPS < PEAK_INT8_OPS:
            achieved = e["alg_bytes"] / sec / 1e9
            return {"kernel": name, "bound": "hbm", "achieved": round(achieved, 1),
                    "peak": PEAK_HBM_BPS / 1e9, "unit": "GB/s",
                    "frac": round(achieved * 1e9 / PEAK_HBM_BPS, 4), "traffic": None,
                    "alg_bytes_per_launch": e["alg_bytes"], "avg_us": e["avg_us"]}
        achieved = e["alg_ops"] / sec / 1e12
        return {"kernel": name, "bound": "mfma", "achieved": round(achieved, 1),
                "peak": PEAK_INT8_OPS / 1e12, "unit": "TFLOP/s",
                "frac": round(achieved * 1e12 / PEAK_INT8_OPS, 4), "traffic": None,
                "alg_ops_per_launch": e["alg_ops"], "avg_us": e["avg_us"]}
    achieved = e["alg_bytes"] / sec / 1e9
    return {"kernel": name, "bound": "hbm", "achieved": round(achieved, 1),
            "peak": PEAK_HBM_BPS / 1e9, "unit": "GB/s",
            "frac": round(achieved * 1e9 / PEAK_HBM_BPS, 4), "traffic": None,
            "alg_bytes_per_launch": e["alg_bytes"], "avg_us": e["avg_us"]}


def model_bench(args, device):
    """25M ratchet transformer training steps/s (sustained, syncs only at both ends)."""
    import numpy as np
    import torch

    from local_ai_training.model import ModelConfig, build_seeded_model

    vocab, block, batch = 8192, 512, 32
    config = ModelConfig(vocab_size=vocab, block_size=block, n_layer=8, n_head=8, n_embd=512,
                         matmul_mode="int8", int8_backward=True)
    model = build_seeded_model(config, max_code=MAX_CODE, seed=1337).to(device).train()
    optimizer = torch.optim.AdamW(model.parameters(), lr=3e-4, weight_decay=0.0)
    rng = np.random.default_rng(1337)
    ids = (rng.zipf(1.1, size=batch * (block + 1)) - 1) % vocab  # Zipf(s=1.1) token ids
    tokens = torch.from_numpy(ids.astype(np.uint16).astype(np.int64)).view(batch, block + 1)
    tokens = tokens.to(device)
    inputs, targets = tokens[:, :block], tokens[:, 1:]

    def step():
        optimizer.zero_grad(set_to_none=True)
        with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
            _, loss = model(inputs, targets)
        loss.backward()
        model.ratchet_update(validate=False)
        optimizer.step()
        return loss

    for _ in range(args.model_warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.model_steps):
        loss = step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    return batch * block * args.model_steps / elapsed, elapsed / args.model_steps, float(loss)


def cpu_baseline(seconds: float) -> dict:
    import torch

    from oracle.cpu_reference import fp32_ratchet_linear_step

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    m_sample = 2048
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
            "kind": "port",
            "sample": f"fp32 eager torch ratchet linear fwd+bwd+tiled update, M={m_sample} of "
                      f"{M_TOK} tokens, K={K_IN}, N={N_OUT}, {iters} steps, "
                      f"{per_step * 1e3:.1f} ms/step"}


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported by this "
              "build (single-GPU ratchet-linear path)", file=sys.stderr)
        return 2
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 1
    device = torch.device("cuda:0")
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
        "pct_int8_mfma_peak": round(tops * 1e12 / PEAK_INT8_OPS * 100, 2),
        "kernels": kernels,
        "roofline": roofline_entry(kernels),
    }
    if not args.no_model:
        log(f"model bench: 25M int8, warmup={args.model_warmup} steps={args.model_steps}")
        tok_s, step_m, loss = model_bench(args, device)
        log(f"model {step_m * 1e3:.2f} ms/step -> {tok_s:.0f} tok/s (loss {loss:.3f})")
        result["train_tokens_per_s"] = round(tok_s, 1)
        result["train_ms_per_step"] = round(step_m * 1e3, 3)
        result["train_config"] = {"model": "ratchet-gpt-25M", "n_layer": 8, "n_embd": 512,
                                  "n_head": 8, "ffn": 2048, "vocab": 8192, "seq_len": 512,
                                  "batch": 32, "matmul_mode": "int8", "int8_backward": True}
    if not args.no_cpu:
        log(f"cpu baseline: ~{args.cpu_seconds:.0f} s of fp32 eager CPU work")
        result["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
