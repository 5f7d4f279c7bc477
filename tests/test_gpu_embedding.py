"""The token-embedding weight gradient on the GPU (rk_embedding_backward through
torch.ops.ratchet.embedding_backward and the C ABI) against the oracle's fixed-order sum,
bit for bit: the 25M and 1B training shapes with Zipf-distributed ids, ragged and one-id
cases, bf16 gradients, int32 ids, an empty batch; replays of a captured graph against the
eager result; argument errors; and the model's lookup against torch's own backward."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from local_ai_training import _native as nat
from local_ai_training.ops import ratchet
from oracle.embedding import embedding_backward

pytestmark = pytest.mark.gpu


def zipf_ids(t: int, v: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return np.minimum(rng.zipf(1.1, t) - 1, v - 1).astype(np.int64)


CASES = [
    # (T, V, D, grad dtype, ids dtype, id pattern)
    (16384, 8192, 512, torch.float32, torch.int64, "zipf"),     # 25M training step
    (8192, 8192, 2048, torch.float32, torch.int64, "zipf"),     # 1B training step
    (1000, 300, 132, torch.bfloat16, torch.int64, "uniform"),   # ragged chunk and columns
    (4096, 16, 64, torch.float32, torch.int32, "one"),          # one id everywhere
    (777, 5000, 4096, torch.bfloat16, torch.int32, "uniform"),  # widest rows, sparse hits
    (64, 1, 4, torch.float32, torch.int64, "one"),
]


@pytest.mark.parametrize("t,v,d,gdt,idt,pattern", CASES)
def test_embedding_backward_matches_oracle_bit_exact(cuda, t, v, d, gdt, idt, pattern):
    print(f"embedding backward T={t} V={v} D={d} {gdt} {idt} {pattern}", flush=True)
    rng = np.random.default_rng(t + v + d)
    if pattern == "zipf":
        ids = zipf_ids(t, v, seed=t)
    elif pattern == "one":
        ids = np.full(t, v // 2, dtype=np.int64)
    else:
        ids = rng.integers(0, v, t)
    g = torch.from_numpy(rng.standard_normal((t, d)).astype(np.float32) * 1e-3).to(gdt)
    want = embedding_backward(g.float().numpy(), ids, v)
    got = ratchet().embedding_backward(g.to(cuda), torch.from_numpy(ids).to(idt).to(cuda), v)
    assert got.dtype == torch.float32 and got.shape == (v, d)
    assert np.array_equal(got.cpu().numpy().view(np.int32), want.view(np.int32))


def test_embedding_backward_3d_gradient_and_empty_batch(cuda):
    g = torch.randn(4, 96, 64) * 1e-2
    ids = torch.randint(0, 37, (4, 96))
    got = ratchet().embedding_backward(g.to(cuda), ids.to(cuda), 37).cpu().numpy()
    assert np.array_equal(got, embedding_backward(g.numpy(), ids.numpy(), 37))
    empty = ratchet().embedding_backward(torch.empty(0, 8, device=cuda),
                                         torch.empty(0, dtype=torch.int64, device=cuda), 5)
    assert empty.shape == (5, 8) and not empty.any()


def test_embedding_backward_through_the_c_abi_with_ids_outside_the_table(cuda):
    t, v, d = 300, 40, 16
    g = torch.randn(t, d, device=cuda)
    ids = torch.randint(-3, v + 3, (t,), device=cuda)
    out = torch.full((v, d), float("nan"), device=cuda)
    nbytes = int(nat.load_library().rk_embedding_backward_workspace(t, v, d))
    work = torch.empty(nbytes, dtype=torch.uint8, device=cuda)
    nat.call("rk_embedding_backward", g.data_ptr(), nat.RK_F32, d, ids.data_ptr(), 1, t, v, d,
             out.data_ptr(), d, work.data_ptr(), nbytes, nat.stream_handle(cuda))
    torch.cuda.synchronize()
    want = embedding_backward(g.cpu().numpy(), ids.cpu().numpy(), v)
    assert np.array_equal(out.cpu().numpy(), want)


def test_embedding_backward_rejects_bad_arguments(cuda):
    g = torch.randn(8, 6, device=cuda)
    ids = torch.zeros(8, dtype=torch.int64, device=cuda)
    with pytest.raises(RuntimeError, match="multiple of 4"):
        ratchet().embedding_backward(g, ids, 4)
    with pytest.raises(RuntimeError, match="at most 4096"):
        ratchet().embedding_backward(torch.randn(2, 4100, device=cuda), ids[:2], 4)
    with pytest.raises(RuntimeError, match="rows for"):
        ratchet().embedding_backward(torch.randn(7, 8, device=cuda), ids, 4)
    work = torch.empty(16, dtype=torch.uint8, device=cuda)
    out = torch.empty(4, 8, device=cuda)
    with pytest.raises(nat.NativeError, match="workspace"):
        nat.call("rk_embedding_backward", g.data_ptr(), nat.RK_F32, 8, ids.data_ptr(), 1, 8, 4,
                 8, out.data_ptr(), 8, work.data_ptr(), 16, nat.stream_handle(cuda))


def test_embedding_backward_replays_of_a_captured_graph_match_eager(cuda):
    t, v, d = 4096, 1000, 256
    g = torch.randn(t, d, device=cuda) * 1e-2
    ids = torch.from_numpy(zipf_ids(t, v, seed=3)).to(cuda)
    R = ratchet()
    R.embedding_backward(g, ids, v)  # warm (allocator, library load)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = R.embedding_backward(g, ids, v)
    for replay in range(4):
        g.copy_(torch.randn(t, d, device=cuda) * 1e-2)
        ids.copy_(torch.from_numpy(zipf_ids(t, v, seed=10 + replay)).to(cuda))
        want = R.embedding_backward(g, ids, v)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int32), want.view(torch.int32)), replay


def test_model_token_lookup_gradient_close_to_torch_backward(cuda):
    from local_ai_training.model import ModelConfig, RatchetGPT, build_seeded_model

    config = ModelConfig(vocab_size=300, block_size=128, n_layer=1, n_head=2, n_embd=64,
                         matmul_mode="int8", int8_backward=True)
    tokens = torch.from_numpy(zipf_ids(32 * 128, 300, seed=5).reshape(32, 128)).to(cuda)
    grads = []
    for hip in (True, False):
        RatchetGPT.hip_embedding_backward = hip
        torch.manual_seed(0)  # the SR seeds of the int8 backward come from the CPU generator
        try:
            model = build_seeded_model(config, max_code=2, seed=11).to(cuda)
            with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
                _, loss = model(tokens[:, :-1], tokens[:, 1:])
            loss.backward()
            model.discard_pending_gradients()
            grads.append(model.token_embedding.weight.grad.clone())
        finally:
            RatchetGPT.hip_embedding_backward = True
    torch.testing.assert_close(grads[0], grads[1], rtol=1e-5, atol=1e-8)
