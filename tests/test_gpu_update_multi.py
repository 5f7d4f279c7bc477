"""The multi-layer fused update (rk_ratchet_update_multi, torch.ops.ratchet.update_multi) and the
model's deferred updates built on it.

* Several layers in one launch equal each layer's own update launch bit for bit: packed state,
  move counts, row rms, rms EMA and the non-finite flag, for bf16 / float32 gradients and
  float32 split partials, ragged and unaligned rows, an empty layer and a non-finite row.
* The operator refuses a table whose rows do not follow each other and a table that writes
  outside the tensors it lists.
* A model with deferred updates trains exactly like one that updates inside backward
  (losses, states, move counts, rms means, parameters), eagerly and in a captured graph.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from helpers import synthetic_state
from local_ai_training import _native, ops
from local_ai_training.model import ModelConfig, build_seeded_model
from local_ai_training.ratchet import DiscreteRatchetLinear
from local_ai_training.training import CapturedTrainingStep, training_step

pytestmark = pytest.mark.gpu

RULE = dict(max_code=3, threshold=8, low=0.5, high=1.5, eps=1e-8)


def make_layer(rows, k, cuda, seed, src, nsplit=1, ema=False, bad_row=None):
    packed, _ = synthetic_state(rows, k, RULE["max_code"], seed=seed)
    g = torch.Generator().manual_seed(seed + 1)
    if src == _native.RK_UPDATE_SRC_SPLITS:
        grad = (torch.randn(nsplit, rows, k, generator=g) * 1e-3).to(cuda)
    else:
        dtype = torch.bfloat16 if src == _native.RK_BF16 else torch.float32
        grad = (torch.randn(rows, k, generator=g) * 1e-3).to(dtype).to(cuda)
    if bad_row is not None and rows > bad_row:
        if grad.dim() == 3:
            grad[0, bad_row, 1] = float("nan")
        else:
            grad[bad_row, 1] = float("inf")
    return dict(
        packed=torch.from_numpy(packed).to(cuda), grad=grad, nsplit=nsplit, rows=rows, k=k,
        counts=torch.zeros(4, dtype=torch.int64, device=cuda),
        row_rms=torch.zeros(rows, device=cuda),
        ema=(torch.rand(rows, generator=g) * 1e-6).to(cuda) if ema else None,
        nonfinite=torch.zeros(1, dtype=torch.int32, device=cuda))


def clone_layer(layer):
    return {k: (v.clone() if isinstance(v, torch.Tensor) else v) for k, v in layer.items()}


def table_of(layers, src, beta=0.9):
    entries = (_native.UpdateLayer * len(layers))()
    row = 0
    for d, ly in zip(entries, layers):
        g = ly["grad"]
        d.packed, d.g = ly["packed"].data_ptr(), g.data_ptr()
        d.counts, d.row_rms = ly["counts"].data_ptr(), ly["row_rms"].data_ptr()
        d.rms_ema = ly["ema"].data_ptr() if ly["ema"] is not None else 0
        d.nonfinite = ly["nonfinite"].data_ptr()
        # (an empty tensor's row stride says nothing: a row of K elements then)
        d.ldp = ly["packed"].stride(0) if ly["rows"] else ly["k"]
        d.ldg = g.stride(-2) if ly["rows"] else ly["k"]
        d.rows, d.K, d.row_begin = ly["rows"], ly["k"], row
        d.max_code, d.threshold, d.nsplit = RULE["max_code"], RULE["threshold"], ly["nsplit"]
        d.low, d.high, d.eps = RULE["low"], RULE["high"], RULE["eps"]
        d.beta1 = beta
        d.beta2 = float(np.float32(1.0) - np.float32(beta))
        row += ly["rows"]
    host = torch.frombuffer(bytearray(ctypes.string_at(ctypes.addressof(entries),
                                                       ctypes.sizeof(entries))), dtype=torch.uint8)
    return host


def written_of(layers):
    out = []
    for ly in layers:
        out += [ly["packed"], ly["counts"], ly["row_rms"], ly["nonfinite"]]
        if ly["ema"] is not None:
            out.append(ly["ema"])
    return out


def per_layer(layers, src, beta=0.9):
    R = ops.ratchet()
    rule = (RULE["max_code"], RULE["threshold"], RULE["low"], RULE["high"], RULE["eps"])
    for ly in layers:
        if ly["rows"] == 0:
            continue  # nothing to update (the per-layer operators check an empty state's strides)
        b = beta if ly["ema"] is not None else 0.0
        if src == _native.RK_UPDATE_SRC_SPLITS:
            R.update_from_partials(ly["packed"], ly["grad"], *rule, ly["ema"], b, ly["counts"],
                                   ly["row_rms"], None, ly["nonfinite"], None, None)
        else:
            R.update_from_grad(ly["packed"], ly["grad"], *rule, ly["ema"], b, ly["counts"],
                               ly["row_rms"], None, ly["nonfinite"], None)


SHAPES = [  # (rows, K, nsplit, ema, bad_row)
    (100, 512, 3, False, None),
    (0, 256, 2, False, None),
    (37, 2048, 1, True, None),
    (513, 1000, 4, False, 7),
    (8, 64, 2, True, None),
    (300, 1536, 11, False, None),
]


@pytest.mark.parametrize("src", [_native.RK_BF16, _native.RK_F32, _native.RK_UPDATE_SRC_SPLITS])
def test_multi_layer_update_equals_per_layer_updates(cuda, src):
    print(f"update_multi src={src}", flush=True)
    shapes = [s for s in SHAPES if src != _native.RK_UPDATE_SRC_SPLITS or s[1] % 8 == 0]
    layers = [make_layer(r, k, cuda, 10 + i, src, ns, ema, bad)
              for i, (r, k, ns, ema, bad) in enumerate(shapes)]
    ref = [clone_layer(ly) for ly in layers]
    per_layer(ref, src)
    host = table_of(layers, src)
    ops.ratchet().update_multi(host, host.to(cuda), src, written_of(layers))
    torch.cuda.synchronize()
    moved = 0
    for a, b in zip(layers, ref):
        for key in ("packed", "counts", "row_rms", "nonfinite", "ema"):
            if a[key] is None:
                continue
            assert torch.equal(a[key].view(torch.uint8) if a[key].dtype != torch.uint8 else a[key],
                               b[key].view(torch.uint8) if b[key].dtype != torch.uint8 else b[key]), key
        moved += int(a["counts"][:2].sum())
    assert moved > 0
    assert any(int(a["nonfinite"]) for a in layers) == any(s[4] is not None for s in shapes)


def test_multi_layer_update_rejects_bad_tables(cuda):
    src = _native.RK_BF16
    layers = [make_layer(64, 256, cuda, 1, src), make_layer(32, 512, cuda, 2, src)]
    host = table_of(layers, src)
    R = ops.ratchet()
    bad = host.clone()
    # the second layer's row_begin (offset 96 of entry 1) no longer follows the first layer
    bad[160 + 96] = 1
    with pytest.raises(RuntimeError, match="row_begin"):
        R.update_multi(bad, bad.to(cuda), src, written_of(layers))
    with pytest.raises(RuntimeError, match="packed state is not among the written"):
        R.update_multi(host, host.to(cuda), src, written_of(layers)[1:])


def tiny_config():
    return ModelConfig(vocab_size=256, block_size=64, n_layer=2, n_head=4, n_embd=128,
                       matmul_mode="int8", int8_backward=True)


def batches(cuda, n=6):
    gen = torch.Generator().manual_seed(4)
    return [torch.randint(0, 256, (8, 65), generator=gen).to(cuda) for _ in range(n)]


def ratchet_layers(model):
    return [m for m in model.modules() if isinstance(m, DiscreteRatchetLinear)]


@pytest.mark.parametrize("captured", [False, True])
def test_deferred_updates_train_like_updates_in_backward(cuda, captured):
    # the same seeded model and batches, updating inside backward or deferring to one
    # batched launch per group: identical losses, statistics, states and parameters
    print(f"deferred updates, captured={captured}", flush=True)
    data = batches(cuda)
    runs = []
    for deferred in (False, True):
        model = build_seeded_model(tiny_config(), max_code=2, seed=21).to(cuda).train()
        if deferred:
            model.defer_ratchet_updates(True)
        optimizer = torch.optim.AdamW(model.parameters(), lr=3e-3, weight_decay=0.0,
                                      capturable=True, fused=True)
        torch.manual_seed(8)
        losses, stats = [], []
        if captured:
            step = CapturedTrainingStep(model, optimizer, data[0][:, :-1], data[0][:, 1:],
                                        warmup_steps=2)
            for b in data[2:]:
                losses.append(float(step(b[:, :-1], b[:, 1:])))
                stats.append(step.stats.materialize())
        else:
            for b in data:
                loss, st = training_step(model, optimizer, b[:, :-1], b[:, 1:], validate=True,
                                         autocast_cache=False)
                losses.append(float(loss))
                stats.append(st)
        torch.cuda.synchronize()
        runs.append((losses, stats, [m.packed.clone() for m in ratchet_layers(model)],
                     [p.detach().clone() for p in model.parameters()]))
    (l0, s0, k0, p0), (l1, s1, k1, p1) = runs
    assert l0 == l1
    assert s0 == s1
    assert sum(s.code_moves for s in s1) > 0
    assert all(torch.equal(a, b) for a, b in zip(k0, k1))
    assert all(torch.equal(a, b) for a, b in zip(p0, p1))


def test_deferred_update_is_applied_before_the_layer_runs_again(cuda):
    model = build_seeded_model(tiny_config(), max_code=2, seed=21).to(cuda).train()
    model.defer_ratchet_updates(True)
    b = batches(cuda, 1)[0]
    x, y = b[:, :-1], b[:, 1:]
    layers = ratchet_layers(model)
    before = [m.packed.clone() for m in layers]
    with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        _, loss = model(x, y)
    loss.backward()
    assert all(m._queued for m in layers)  # backward queued the updates
    assert all(torch.equal(m.packed, p) for m, p in zip(layers, before))  # not yet applied
    with torch.no_grad(), torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        model(x, y)  # the next forward applies them first
    assert not any(m._queued for m in layers)
    assert sum(not torch.equal(m.packed, p) for m, p in zip(layers, before)) > 0
    model.ratchet_update(validate=True)


def test_reading_the_state_applies_a_queued_update(cuda):
    # state_dict() and the code / pressure views flush the queue: after backward they show
    # the updated state, as with updates inside backward
    data = batches(cuda, 1)[0]
    x, y = data[:, :-1], data[:, 1:]
    states = []
    for deferred in (False, True):
        model = build_seeded_model(tiny_config(), max_code=2, seed=21).to(cuda).train()
        model.defer_ratchet_updates(deferred)
        torch.manual_seed(8)
        with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
            _, loss = model(x, y)
        loss.backward()
        layers = ratchet_layers(model)
        if deferred:
            assert all(m._queued for m in layers)
            codes = layers[0].code  # flushes the whole queue
            assert not any(m._queued for m in layers)
            assert torch.equal(codes, states[0][1])
        sd = {k: v.clone() for k, v in model.state_dict().items() if k.endswith("packed")}
        states.append((sd, layers[0].code.clone()))
        model.ratchet_update(validate=True)
    assert states[0][0].keys() == states[1][0].keys()
    assert all(torch.equal(states[0][0][k], states[1][0][k]) for k in states[0][0])
