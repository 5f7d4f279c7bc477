"""One KV-cached decode step of the ratchet transformer on the fused HIP decode kernels.

The reference produces every generated token by running the whole window through the
model (``generate.py:183-201``). The cached step computes the last position only, and
for up to 16 sequences it does so in 6 launches per layer (``rk_decode_*`` in
include/ratchet_hip.h):

    qkv       = GEMV(RMSNorm-quant(hidden))                 bf16 (exact: the GEMM rounds
                                                             its output to bf16)
    att       = attention(qkv, cache, pos)                   float32; appends k, v at pos
                                                             (two launches)
    hidden   += GEMV(quant(att))                             residual add in the epilogue
    ffn       = GELU(GEMV(RMSNorm-quant(hidden)))           float32
    hidden   += GEMV(quant(ffn))

then ``logits = GEMV(RMSNorm-quant(hidden))`` through ``lm_head``. The quantized rows
equal what the training kernels compute for the same float rows (``rk_rmsnorm_quantize``,
``rk_quantize_rows``, ``rk_gelu_quantize``), and each GEMV's int32 sums and bf16 outputs
equal ``rk_int8_gemm_packed``'s; the attention runs in float32 with its positions split
across workgroups, so its result differs from the window forward's attention only by
float summation order. Every kernel reads the position from ``cache.pos`` on the device,
so the step can be captured once as a HIP graph and replayed.
"""

from __future__ import annotations

import math

import torch
from torch import Tensor, nn

from . import _native as nat
from .ratchet import DiscreteRatchetLinear

PRO_INT8, PRO_PLAIN, PRO_RMSNORM = 0, 1, 2
EPI_STORE, EPI_GELU, EPI_ADD = 0, 1, 2
MAX_ROWS = 16
MAX_K = 6144
BLOCK_NORM_EPS = 1e-5  # FusedRMSNormQuantizeFn's eps (int8_fused.py:14-39)


def decode_gemv(layer: DiscreteRatchetLinear, out: Tensor, *, prologue: int, epilogue: int,
                x: Tensor | None = None, xq: Tensor | None = None, xs: Tensor | None = None,
                norm_weight: Tensor | None = None, eps: float = 0.0) -> Tensor:
    """out = epilogue(GEMV(prologue(rows))) with `layer`'s packed codes and row scales."""
    packed = layer.packed
    n, k = packed.shape
    m = out.shape[0]
    scale = layer.scale.detach()
    if scale.dtype != torch.float32 or not scale.is_contiguous():
        scale = scale.float().contiguous()
    nat.call(
        "rk_decode_gemv", nat.ptr(x), x.stride(0) if x is not None else 0, nat.ptr(xq),
        xq.stride(0) if xq is not None else 0, nat.ptr(xs), prologue, nat.ptr(norm_weight),
        float(eps), packed.data_ptr(), packed.stride(0), layer.max_code, scale.data_ptr(),
        out.data_ptr(), nat.dtype_code(out.dtype), out.stride(0), epilogue, m, n, k,
        nat.stream_handle(out.device),
    )
    return out


def decode_attention(qkv: Tensor, keys: Tensor, values: Tensor, pos: Tensor, n_head: int,
                     work: Tensor, out: Tensor) -> Tensor:
    """Append this step's k, v at `pos`; out [B, H*D] float32 = the attention rows."""
    batch, _, max_len, head = keys.shape
    nat.call(
        "rk_decode_attention", qkv.data_ptr(), nat.dtype_code(qkv.dtype), qkv.stride(0),
        keys.data_ptr(), values.data_ptr(), nat.dtype_code(keys.dtype), keys.stride(0),
        keys.stride(1), keys.stride(2), pos.data_ptr(), batch, n_head, head, max_len,
        1.0 / math.sqrt(head), work.data_ptr(), work.numel(), out.data_ptr(), out.stride(0),
        nat.stream_handle(qkv.device),
    )
    return out


def decode_greedy(logits: Tensor, tokens: Tensor, pos: Tensor | None = None) -> Tensor:
    """tokens[b, 0] = argmax of logits row b (torch.argmax's pick: the first largest value,
    NaN above every number), then ``pos += 1`` when `pos` is given: the greedy choice of
    ``generate.py:188-189`` and the window's growth by that token (``generate.py:200``) in
    one launch (``rk_decode_greedy``). `logits` float32 with unit column stride, `tokens`
    int64 [B, 1]."""
    if logits.dtype != torch.float32 or logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("decode_greedy expects float32 logits [B, V] with unit column stride")
    if tokens.dtype != torch.long or tokens.shape[0] != logits.shape[0]:
        raise ValueError("decode_greedy expects int64 tokens with one row per logits row")
    if pos is not None and (pos.dtype != torch.long or pos.numel() != 1):
        raise ValueError("decode_greedy expects a one-element int64 position")
    nat.call("rk_decode_greedy", logits.data_ptr(), logits.stride(0), logits.shape[0],
             logits.shape[1], tokens.data_ptr(), tokens.stride(0), nat.ptr(pos),
             nat.stream_handle(logits.device))
    return tokens


def attention_workspace_floats(batch: int, n_head: int, head: int, max_len: int) -> int:
    splits = int(nat.load_library().rk_decode_attention_splits(batch, n_head, max_len))
    return batch * n_head * splits * (head + 4)


def _ratchet_layers(model) -> list:
    layers = [model.lm_head]
    for block in model.blocks:
        layers += [block.attention.qkv, block.attention.projection, block.feed_forward.expand,
                   block.feed_forward.contract]
    return layers


def fused_decode_supported(model, cache) -> bool:
    """True when the fused kernels cover this model and cache: a ROCm device, at most 16
    sequences, int8 ratchet layers with N % 16 == 0, K % 64 == 0, K <= 6144, head size
    64/128/256, a plain float32 token embedding, eval mode."""
    config = model.config
    if cache.device.type != "cuda" or cache.batch > MAX_ROWS or model.training:
        return False
    if not isinstance(model.token_embedding, nn.Embedding):
        return False
    if model.token_embedding.weight.dtype != torch.float32:
        return False
    head = config.n_embd // config.n_head
    if head not in (64, 128, 256):
        return False
    for layer in _ratchet_layers(model):
        if not isinstance(layer, DiscreteRatchetLinear) or layer.matmul_mode != "int8":
            return False
        n, k = layer.packed.shape
        if n % 16 or k % 64 or k > MAX_K or not layer.packed.is_cuda:
            return False
    return True


def _step_buffers(model, cache) -> dict[str, Tensor]:
    bufs = cache.step_buffers
    if not bufs:
        config, batch, device = model.config, cache.batch, cache.device
        c, head = config.n_embd, config.n_embd // config.n_head
        f32 = dict(dtype=torch.float32, device=device)
        bufs.update(
            tokens=torch.zeros(batch, dtype=torch.long, device=device),
            hidden=torch.empty(batch, c, **f32),
            qkv=torch.empty(batch, 3 * c, dtype=torch.bfloat16, device=device),
            attn=torch.empty(batch, c, **f32),
            ffn=torch.empty(batch, config.hidden_size, **f32),
            logits=torch.empty(batch, config.vocab_size, **f32),
            work=torch.empty(attention_workspace_floats(batch, config.n_head, head,
                                                        cache.max_len), **f32),
        )
    return bufs


@torch.no_grad()
def fused_decode_logits(model, tokens: Tensor, cache) -> Tensor:
    """Logits [B, vocab] (float32 holding bf16 values, as the int8 lm_head writes them) of
    `tokens` [B, 1] at position ``cache.pos``; appends every layer's key/value there. The
    cache is not advanced. The returned buffer is overwritten by the next step."""
    config = model.config
    batch = cache.batch
    if tokens.shape != (batch, 1):
        raise ValueError(f"decode step expects tokens of shape ({batch}, 1)")
    bufs = _step_buffers(model, cache)
    ids = tokens
    if tokens.dtype != torch.long or not tokens.is_contiguous() or not tokens.is_cuda:
        ids = bufs["tokens"]
        ids.copy_(tokens.reshape(batch))
    hidden, qkv, ffn = bufs["hidden"], bufs["qkv"], bufs["ffn"]
    stream = nat.stream_handle(hidden.device)
    table = model.token_embedding.weight
    positions = model.position_encoding
    nat.call("rk_decode_embed", ids.data_ptr(), batch, table.data_ptr(), table.shape[0],
             config.n_embd, positions.data_ptr(), positions.shape[0], cache.pos.data_ptr(),
             hidden.data_ptr(), hidden.stride(0), stream)
    for index, block in enumerate(model.blocks):
        attention, feed_forward = block.attention, block.feed_forward
        decode_gemv(attention.qkv, qkv, prologue=PRO_RMSNORM, epilogue=EPI_STORE, x=hidden,
                    norm_weight=block.attention_norm.weight, eps=BLOCK_NORM_EPS)
        keys, values = cache.buffers(index, qkv)
        att = decode_attention(qkv, keys, values, cache.pos, config.n_head, bufs["work"],
                               bufs["attn"])
        decode_gemv(attention.projection, hidden, prologue=PRO_PLAIN, epilogue=EPI_ADD, x=att)
        decode_gemv(feed_forward.expand, ffn, prologue=PRO_RMSNORM, epilogue=EPI_GELU,
                    x=hidden, norm_weight=block.feed_forward_norm.weight, eps=BLOCK_NORM_EPS)
        decode_gemv(feed_forward.contract, hidden, prologue=PRO_PLAIN, epilogue=EPI_ADD, x=ffn)
    final_eps = model.final_norm.eps
    if final_eps is None:  # nn.RMSNorm's default: the float32 machine epsilon
        final_eps = torch.finfo(torch.float32).eps
    return decode_gemv(model.lm_head, bufs["logits"], prologue=PRO_RMSNORM, epilogue=EPI_STORE,
                       x=hidden, norm_weight=model.final_norm.weight, eps=final_eps)
