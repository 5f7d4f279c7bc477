"""The reference's CPU path for one ratchet linear, restated in eager torch (CPU baseline).

Test / baseline infrastructure only. The reference's int8 path is GPU-only
(``int8_matmul.py:257-258``); its CPU path is ``matmul_mode="fp32"`` with the update
fused into backward over 256-row tiles. One step here is that path:

* forward  ``out = x @ (code * scale)^T``                      (ratchet.py:57-59)
* backward ``grad_input = g @ (code * scale)``                 (ratchet.py:120-124)
* per 256-row tile: ``G_w = g[:, tile]^T @ x``,
  ``z = G_w / (sqrt(mean G_w^2) + eps)``, integer update      (ratchet.py:150-169,
  539-556, 265-301)

It is timed on the host cores as the ``cpu_baseline`` of bench.py, in the same unit
(TOPS over the three GEMMs' 2*M*N*K each) as the GPU path.
"""

from __future__ import annotations

import torch


def _update_core(packed, z, max_code, threshold, low, high):
    mag = z.abs()
    inc = -torch.sign(z).to(torch.int16) * ((mag >= high).to(torch.int16)
                                            + (mag >= low).to(torch.int16))
    v = packed.to(torch.int16)
    code = (v & 0x0F) - max_code
    p = (v >> 4) - 7 + inc
    pr = p >= threshold
    nr = p <= -threshold
    pm = pr & (code < max_code)
    nm = nr & (code > -max_code)
    code = code + pm.to(torch.int16) - nm.to(torch.int16)
    p = (p - pr.to(torch.int16) * threshold + nr.to(torch.int16) * threshold).clamp(-128, 127)
    new = ((code + max_code) & 0x0F) | (((p + 7) & 0x0F) << 4)
    return new.to(torch.uint8), pm.sum() + nm.sum()


def fp32_ratchet_linear_step(x: torch.Tensor, packed: torch.Tensor, scale: torch.Tensor,
                             grad_out: torch.Tensor, max_code: int, threshold: int = 8,
                             low: float = 0.5, high: float = 1.5, eps: float = 1e-8,
                             tile_size: int = 256):
    """One fp32 forward + backward + fused update; mutates ``packed``. Returns
    (output, grad_input, code_moves)."""
    code = ((packed.to(torch.int16) & 0x0F) - max_code).to(torch.float32)
    effective = code * scale[:, None]
    out = x @ effective.t()
    grad_input = grad_out @ effective
    moves = torch.zeros((), dtype=torch.int64)
    grad_t = grad_out.t()
    for t0 in range(0, packed.shape[0], tile_size):
        t1 = min(t0 + tile_size, packed.shape[0])
        gw = grad_t[t0:t1] @ x
        rms = gw.square().mean(dim=1, keepdim=True).sqrt()
        z = gw / (rms + eps)
        new, m = _update_core(packed[t0:t1], z, max_code, threshold, low, high)
        packed[t0:t1] = new
        moves += m
    return out, grad_input, moves


# ---------------------------------------------------------------------------
# The reference's CPU training step for a whole model (the C1 tiny config), restated in
# eager torch: train.py:248-277 (zero_grad, bf16 autocast forward, backward with the
# ratchet update fused into each linear's backward, AdamW on the float parameters), the
# decoder of model.py (sinusoidal positions, pre-RMSNorm blocks, causal attention, GELU
# feed-forward, ratchet linears in fp32 mode) and ratchet.py's fp32 _RatchetMatmul.
# ---------------------------------------------------------------------------


class _RatchetLinearFn(torch.autograd.Function):
    """fp32-mode ratchet linear: out = x @ (code * scale)^T; the backward returns
    grad_input and updates the packed state over 256-row tiles (ratchet.py:57-59,
    120-124, 150-169)."""

    @staticmethod
    def forward(ctx, x, packed, scale, max_code):
        code = ((packed.to(torch.int16) & 0x0F) - max_code).to(torch.float32)
        weight = code * scale[:, None]
        ctx.save_for_backward(x, weight)
        ctx.packed, ctx.max_code = packed, max_code
        return x @ weight.t().to(x.dtype)

    @staticmethod
    def backward(ctx, grad_out):
        x, weight = ctx.saved_tensors
        grad_input = grad_out @ weight.to(grad_out.dtype)
        g = grad_out.reshape(-1, grad_out.shape[-1]).float().t()
        xf = x.reshape(-1, x.shape[-1]).float()
        packed = ctx.packed
        for t0 in range(0, packed.shape[0], 256):
            t1 = min(t0 + 256, packed.shape[0])
            gw = g[t0:t1] @ xf
            rms = gw.square().mean(dim=1, keepdim=True).sqrt()
            new, _ = _update_core(packed[t0:t1], gw / (rms + 1e-8), ctx.max_code, 8, 0.5, 1.5)
            packed[t0:t1] = new
        return grad_input, None, None, None


class _RatchetLinear(torch.nn.Module):
    def __init__(self, n_in: int, n_out: int, max_code: int, gen: torch.Generator):
        super().__init__()
        code = torch.randint(-max_code, max_code + 1, (n_out, n_in), generator=gen)
        self.register_buffer("packed", (((code + max_code) & 0x0F) | (7 << 4)).to(torch.uint8))
        self.register_buffer("scale", torch.rand(n_out, generator=gen) * 0.08 + 0.02)
        self.max_code = max_code

    def forward(self, x):
        return _RatchetLinearFn.apply(x, self.packed, self.scale, self.max_code)


class TinyRatchetGPT(torch.nn.Module):
    """Decoder-only ratchet transformer in the reference's fp32 mode."""

    def __init__(self, vocab: int, n_embd: int, n_head: int, n_layer: int, ffn: int,
                 block: int, max_code: int, seed: int):
        super().__init__()
        gen = torch.Generator().manual_seed(seed)
        nn = torch.nn
        self.n_head = n_head
        self.embed = nn.Embedding(vocab, n_embd)
        pos = torch.arange(block, dtype=torch.float32)[:, None]
        freq = torch.exp(torch.arange(0, n_embd, 2, dtype=torch.float32)
                         * (-torch.log(torch.tensor(10000.0)) / n_embd))
        pe = torch.zeros(block, n_embd)
        pe[:, 0::2] = torch.sin(pos * freq)
        pe[:, 1::2] = torch.cos(pos * freq)
        self.register_buffer("pe", pe)
        self.blocks = nn.ModuleList()
        for _ in range(n_layer):
            self.blocks.append(nn.ModuleDict({
                "n1": nn.RMSNorm(n_embd), "qkv": _RatchetLinear(n_embd, 3 * n_embd, max_code, gen),
                "proj": _RatchetLinear(n_embd, n_embd, max_code, gen), "n2": nn.RMSNorm(n_embd),
                "expand": _RatchetLinear(n_embd, ffn, max_code, gen),
                "contract": _RatchetLinear(ffn, n_embd, max_code, gen)}))
        self.norm = nn.RMSNorm(n_embd)
        self.head = _RatchetLinear(n_embd, vocab, max_code, gen)

    def forward(self, tokens, targets):
        b, s = tokens.shape
        x = self.embed(tokens) + self.pe[:s]
        for blk in self.blocks:
            q, k, v = blk["qkv"](blk["n1"](x)).chunk(3, dim=-1)
            heads = lambda t: t.view(b, s, self.n_head, -1).transpose(1, 2)
            att = torch.nn.functional.scaled_dot_product_attention(
                heads(q), heads(k), heads(v), is_causal=True)
            x = x + blk["proj"](att.transpose(1, 2).reshape(b, s, -1))
            x = x + blk["contract"](torch.nn.functional.gelu(blk["expand"](blk["n2"](x))))
        logits = self.head(self.norm(x))
        return torch.nn.functional.cross_entropy(logits.flatten(0, 1).float(), targets.flatten())


def tiny_training_tokens_per_s(steps: int = 20, timed_from: int = 3, seed: int = 1337) -> dict:
    """The C1 config (2 layers, d 128, 4 heads, FFN 512, byte vocab 256, seq 64, batch 8,
    quinary codes): `steps` training steps, tokens/s over steps timed_from..steps."""
    import time

    vocab, block, batch = 256, 64, 8
    model = TinyRatchetGPT(vocab, 128, 4, 2, 512, block, 2, seed)
    opt = torch.optim.AdamW([p for p in model.parameters() if p.requires_grad], lr=3e-4)
    gen = torch.Generator().manual_seed(seed + 1)
    t0 = None
    losses = []
    for step in range(1, steps + 1):
        if step == timed_from:
            t0 = time.perf_counter()
        data = torch.randint(0, vocab, (batch, block + 1), generator=gen)
        opt.zero_grad(set_to_none=True)
        with torch.autocast(device_type="cpu", dtype=torch.bfloat16):
            loss = model(data[:, :-1], data[:, 1:])
        loss.backward()
        opt.step()
        losses.append(float(loss.detach()))
    dt = time.perf_counter() - t0
    timed = steps - timed_from + 1
    return {"tokens_per_s": batch * block * timed / dt, "ms_per_step": dt / timed * 1e3,
            "steps": steps, "timed_steps": timed, "first_loss": losses[0], "last_loss": losses[-1]}
