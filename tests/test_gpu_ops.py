"""torch.library.opcheck over every torch.ops.ratchet operator on the GPU.

opcheck runs each operator for real and checks: that it mutates exactly the arguments its
schema declares (test_schema), that its fake kernel reproduces the real results' metadata
(test_faketensor), that it traces and runs through AOT dispatch with dynamic shapes, where
mutating operators are functionalized (test_aot_dispatch_dynamic), and its autograd
registration. Values are checked against the oracle elsewhere; here the operators'
torch integration is.
"""

from __future__ import annotations

import pytest
import torch

from helpers import synthetic_state
from local_ai_training import ops

pytestmark = pytest.mark.gpu

M, K, N, MC = 96, 128, 256, 2


def gen(seed):
    return torch.Generator().manual_seed(seed)


@pytest.fixture(scope="module")
def t(cuda):
    g = gen(1)
    packed, scale = synthetic_state(N, K, MC, seed=3)
    packed_kn, _ = synthetic_state(K, N, MC, seed=4)
    x = torch.randn(M, K, generator=g)
    return dict(
        x=x.to(cuda), xb=x.to(torch.bfloat16).to(cuda),
        q=torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8).to(cuda),
        s=(torch.rand(M, generator=g) * 0.05 + 1e-3).to(cuda),
        gq=torch.randint(-127, 128, (M, N), generator=g, dtype=torch.int8).to(cuda),
        b=torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8).to(cuda),
        packed=torch.from_numpy(packed).to(cuda), packed_kn=torch.from_numpy(packed_kn).to(cuda),
        scale=torch.from_numpy(scale).to(cuda),
        g=(torch.randn(M, N, generator=g) * 1e-2).to(torch.bfloat16).to(cuda),
        gf=(torch.randn(M, N, generator=g) * 1e-2).to(cuda),
        res=torch.randn(M, N, generator=g).to(cuda),
        gw=torch.randn(N, K, generator=g).to(cuda),
        att=torch.randn(2, 4, 48, 32, generator=g).to(torch.bfloat16).to(cuda),
    )


def cases(t, cuda):
    R = ops.ratchet()
    counts = lambda: torch.zeros(4, dtype=torch.int64, device=cuda)  # noqa: E731
    rows = lambda: torch.zeros(N, device=cuda)  # noqa: E731
    flag = lambda: torch.zeros(1, dtype=torch.int32, device=cuda)  # noqa: E731
    nsplit = R.grad_weight_splits(M, N, K)
    work = lambda: torch.zeros(nsplit, N, K, device=cuda)  # noqa: E731
    partials = torch.randn(nsplit, N, K, generator=gen(9)).mul_(1e-3).to(cuda)
    seed = torch.tensor([1234], dtype=torch.int64, device=cuda)
    rule = (MC, 8, 0.5, 1.5, 1e-8)
    whole = (torch.randn(M, 3 * N, generator=gen(11)) * 1e-2).to(torch.bfloat16).to(cuda)
    tgt = torch.randint(0, K, (M,), generator=gen(12)).to(cuda)
    tgt_ignored = torch.where(torch.arange(M, device=cuda) % 7 == 0, -1, tgt)
    att_qkv = tuple(torch.randn(2, 2, 48, 64, generator=gen(13 + i)).to(torch.bfloat16).to(cuda)
                    for i in range(3))
    xent_b = R.cross_entropy_forward(t["xb"], tgt)
    xent_f = R.cross_entropy_forward(t["x"], tgt_ignored, -1)
    parts = list(whole.chunk(3, dim=-1))
    work3 = torch.zeros(R.grad_weight_splits(M, 3 * N, K), 3 * N, K, device=cuda)
    return [
        (R.quantize_rows, (t["x"],), {}),
        (R.quantize_rows, (t["gf"], t["scale"], True, 77), {"x_bf16": torch.empty_like(t["g"])}),
        (R.quantize_rows, (t["g"], t["scale"], True, 0, seed), {}),
        (R.int8_mm_nt, (t["q"], t["b"], t["s"], t["scale"], torch.bfloat16), {}),
        (R.packed_mm, (t["q"], t["packed"], MC, t["s"], t["scale"], torch.float32), {}),
        (R.packed_mm_residual, (t["q"], t["packed"], MC, t["s"], t["scale"], t["res"]), {}),
        (R.packed_mm_accumulate, (t["q"], t["packed"], MC, t["s"], t["scale"],
                                  t["res"].clone()), {}),
        (R.packed_mm_t, (t["gq"], t["packed"], MC, t["s"], None, torch.bfloat16), {}),
        (R.unpack_transpose, (t["packed"], MC), {}),
        (R.unpack, (t["packed"], MC), {}),
        (R.effective_bf16, (t["packed"], MC, t["scale"]), {}),
        (R.grad_input_bf16, (t["g"], t["packed"], MC, t["scale"], torch.float32), {}),
        (R.dequant_bf16, (t["q"], t["s"]), {}),
        (R.transpose_bf16, (t["x"],), {}),
        (R.dequant_transpose_bf16, (t["q"], t["s"]), {}),
        (R.grad_weight, (t["g"], t["q"], t["s"]), {}),
        (R.grad_weight_x, (t["gf"], t["xb"]), {}),
        (R.grad_weight_partials, (t["g"], t["q"], t["s"], work()), {}),
        (R.grad_weight_partials_x, (t["g"], t["x"], work()), {}),
        (R.update_from_z, (t["packed"].clone(), t["gw"], MC, 8, 0.5, 1.5, counts()), {}),
        (R.update_from_grad, (t["packed"].clone(), t["gw"], *rule, None, 0.0, counts(), rows(),
                              rows(), flag(), torch.zeros((), device=cuda)), {}),
        (R.update_from_grad, (t["packed"].clone(), t["gw"], *rule, rows().fill_(1.0), 0.9,
                              counts(), None, None, None, None), {}),
        (R.update_from_partials, (t["packed"].clone(), partials, *rule, None, 0.0, counts(),
                                  rows(), rows(), flag(), torch.zeros((), device=cuda),
                                  torch.empty(N, K, dtype=torch.bfloat16, device=cuda)), {}),
        (R.normalize_rows, (t["gw"], 1e-8, None, 0.0), {}),
        (R.normalize_rows, (t["gw"], 1e-8, rows().fill_(1.0), 0.5), {}),
        (R.pressure_leak, (t["packed"].clone(), MC), {}),
        (R.validate_state, (t["packed"], MC, t["scale"]), {}),
        (R.rmsnorm_quantize, (t["x"], torch.ones(K, device=cuda), 1e-5), {}),
        (R.gelu_quantize, (t["xb"],), {}),
        (R.transpose_quantize, (t["att"],), {}),
        (R.rmsnorm_backward, (t["xb"], t["xb"], torch.ones(K, device=cuda), 1e-5), {}),
        (R.rmsnorm_backward, (t["xb"], t["x"], torch.ones(K, device=cuda), 1e-5, t["x"] * 0.5),
         {}),
        (R.gelu_backward, (t["x"], t["x"]), {}),
        (R.embedding_backward, (t["x"], torch.randint(0, 40, (M,), generator=gen(5)).to(cuda),
                                40), {}),
        (R.quantize_rows_parts, (parts, t["scale"].repeat(3), True, 5), {}),
        (R.quantize_rows_parts, ([p.contiguous() for p in parts[:2]],), {}),
        (R.grad_weight_partials_parts, (parts, t["q"], t["s"], work3), {}),
        (R.grad_weight_partials_parts, (parts, t["xb"], None, work3.clone()), {}),
        (R.row_rms_means, (t["x"][0].abs().contiguous(),
                           torch.tensor([0, 5, 100, K], dtype=torch.int64, device=cuda)), {}),
        (R.attention_forward, (*att_qkv, 0.125), {}),
        (R.cross_entropy_forward, (t["xb"], tgt), {}),
        (R.cross_entropy_forward, (t["x"], tgt_ignored, -1), {}),
        (R.cross_entropy_backward, (torch.ones((), device=cuda), t["xb"], tgt, *xent_b[1:]), {}),
        (R.cross_entropy_backward, (torch.full((), 0.5, device=cuda), t["x"], tgt_ignored,
                                    *xent_f[1:], -1), {}),
    ]


N_CASES = 44


def test_every_operator_has_an_opcheck_case(t, cuda):
    covered = {case[0]._qualified_op_name.split("::")[1] for case in cases(t, cuda)}
    # update_multi writes through the device addresses of its layer table, so opcheck's
    # copies of the written tensors cannot stand in for the originals (the operator refuses
    # them); its values, writes and refusals are tested in test_gpu_update_multi.py
    assert covered == set(ops.OPERATORS) - {"grad_weight_splits", "update_multi"}
    assert len(cases(t, cuda)) == N_CASES


@pytest.mark.parametrize("index", range(N_CASES))
def test_opcheck(t, cuda, index):
    op, args, kwargs, *utils = cases(t, cuda)[index]
    print(f"opcheck {op._qualified_op_name} case {index}", flush=True)
    if utils:
        torch.library.opcheck(op, args, kwargs, test_utils=utils[0])
    else:
        torch.library.opcheck(op, args, kwargs)
    torch.cuda.synchronize()
