"""Decoder-only ratchet GPT (drop-in for ``model.py``), the host caller of the int8 path.

Same architecture and switches as the reference (``model.py:23-285``): sinusoidal
positions, RMSNorm, causal SDPA, tanh-GELU FFN in int8 mode (erf-GELU otherwise),
untied ratchet ``lm_head``, every dense matrix a ``DiscreteRatchetLinear`` with the
update fused into backward. In ``matmul_mode="int8"`` the RMSNorm / GELU / head-merge
prologues quantize on the GPU and hand int8 rows straight to the ratchet GEMMs.

Additions: ``ffn_hidden`` (default ``4 * n_embd``, the reference's hard-coded width,
``model.py:137``) so 1B-class shapes with FFN 5632 can be built.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Literal

import torch
from torch import Tensor, nn
from torch.nn import functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel

from .attention import CausalAttentionFn, attention_supported
from .cross_entropy import cross_entropy
from .int8_fused import (
    FusedGELUQuantizeFn,
    FusedRMSNormQuantizeFn,
    FusedRMSNormQuantizeResidualFn,
    FusedTransposeQuantizeFn,
)
from .ratchet import DiscreteRatchetLinear, RatchetEmbedding, RatchetUpdateStats, UpdateQueue


@dataclass(frozen=True)
class ModelConfig:
    vocab_size: int
    block_size: int = 128
    n_layer: int = 2
    n_head: int = 4
    n_embd: int = 128
    dropout: float = 0.0
    pressure_threshold: int = 8
    bucket_low: float = 0.5
    bucket_high: float = 1.5
    trainable_scale: bool = False
    rms_ema_beta: float = 0.0
    pressure_leak_period: int = 0
    compile_update: bool = False
    gradient_checkpointing: bool = False
    matmul_mode: Literal["fp32", "bf16", "int8"] = "fp32"
    int8_backward: bool = False
    qat: bool = False
    ratchet_embedding: bool = False
    ffn_hidden: int | None = None

    def __post_init__(self) -> None:
        if min(self.vocab_size, self.block_size, self.n_layer, self.n_head, self.n_embd) <= 0:
            raise ValueError("model dimensions must be positive")
        if self.n_embd % self.n_head != 0:
            raise ValueError("n_embd must be divisible by n_head")
        if not 0 <= self.dropout < 1:
            raise ValueError("dropout must be in [0, 1)")
        if self.matmul_mode not in {"fp32", "bf16", "int8"}:
            raise ValueError("matmul_mode must be fp32, bf16, or int8")
        if self.ffn_hidden is not None and self.ffn_hidden <= 0:
            raise ValueError("ffn_hidden must be positive")
        if self.qat:
            raise ValueError("the QAT control arm is not part of the ratchet-linear build")

    @property
    def hidden_size(self) -> int:
        return self.ffn_hidden if self.ffn_hidden is not None else 4 * self.n_embd


def _sinusoidal_positions(block_size: int, n_embd: int) -> Tensor:
    positions = torch.arange(block_size, dtype=torch.float32)[:, None]
    even = torch.arange(0, n_embd, 2, dtype=torch.float32)
    frequencies = torch.exp(-math.log(10_000.0) * even / n_embd)
    encoding = torch.zeros(block_size, n_embd, dtype=torch.float32)
    encoding[:, 0::2] = torch.sin(positions * frequencies)
    if n_embd > 1:
        encoding[:, 1::2] = torch.cos(positions * frequencies[: encoding[:, 1::2].shape[1]])
    return encoding


def _linear(config: ModelConfig, in_features: int, out_features: int, max_code: int | None):
    if max_code is None:
        return nn.Linear(in_features, out_features, bias=False)
    return DiscreteRatchetLinear(
        in_features, out_features, max_code=max_code,
        pressure_threshold=config.pressure_threshold, bucket_low=config.bucket_low,
        bucket_high=config.bucket_high, trainable_scale=config.trainable_scale,
        rms_ema_beta=config.rms_ema_beta, pressure_leak_period=config.pressure_leak_period,
        compile_update=config.compile_update, matmul_mode=config.matmul_mode,
        fuse_backward_update=True, int8_backward=config.int8_backward,
    )


def _is_int8(layer: nn.Module) -> bool:
    return getattr(layer, "matmul_mode", "fp32") == "int8"


class KVCache:
    """Per-layer keys/values [B, H, max_len, D] for incremental decoding, plus the number of
    filled positions. ``pos`` is that number as a device tensor, so a decode step (which
    reads the position and the mask from it) has fixed shapes and can be replayed as a HIP
    graph; ``length`` is the host copy."""

    def __init__(self, n_layer: int, batch: int, n_head: int, head_size: int, max_len: int,
                 device: torch.device, dtype: torch.dtype | None = None) -> None:
        self.n_layer, self.batch, self.n_head = n_layer, batch, n_head
        self.head_size, self.max_len, self.device = head_size, max_len, device
        self.dtype = dtype
        self.keys: list[Tensor | None] = [None] * n_layer
        self.values: list[Tensor | None] = [None] * n_layer
        self.length = 0
        self.pos = torch.zeros(1, dtype=torch.long, device=device)
        self._arange = torch.arange(max_len, device=device)
        self._mask: Tensor | None = None
        self.step_buffers: dict[str, Tensor] = {}  # fixed-shape work buffers of a step

    def buffers(self, layer: int, like: Tensor) -> tuple[Tensor, Tensor]:
        """The layer's key/value buffers, allocated on first use in the cache dtype
        (``like``'s when none was given) and kept from then on (later steps convert to
        their dtype, so keys written by a prefill are never dropped)."""
        if self.keys[layer] is None:
            dtype = self.dtype or like.dtype
            shape = (self.batch, self.n_head, self.max_len, self.head_size)
            self.keys[layer] = torch.zeros(shape, dtype=dtype, device=self.device)
            self.values[layer] = torch.zeros(shape, dtype=dtype, device=self.device)
        return self.keys[layer], self.values[layer]

    def decode_mask(self, dtype: torch.dtype) -> Tensor:
        """Additive mask [1, 1, 1, max_len] for a one-token step at position ``pos``:
        0 for keys 0..pos, -inf after (computed on the device from ``pos``). Built once per
        step (``begin_step``) and shared by the layers."""
        if self._mask is None or self._mask.dtype != dtype:
            valid = self._arange <= self.pos
            zero = torch.zeros((), dtype=dtype, device=self.device)
            ninf = torch.full((), float("-inf"), dtype=dtype, device=self.device)
            self._mask = torch.where(valid, zero, ninf).view(1, 1, 1, self.max_len)
        return self._mask

    def begin_step(self) -> None:
        self._mask = None

    def advance(self, steps: int) -> None:
        self.length += steps
        self.pos.add_(steps)


# causal training attention: the HIP forward (rk_attention_forward) where it applies, with
# torch's memory-efficient backward (False: torch's forward too)
hip_attention_forward = True
_FAST_ATTENTION = [SDPBackend.EFFICIENT_ATTENTION, SDPBackend.FLASH_ATTENTION]
_DETERMINISTIC_ATTENTION = [SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]


def _attend(q: Tensor, k: Tensor, v: Tensor, **kwargs) -> Tensor:
    """scaled_dot_product_attention; 16-bit GPU inputs go to the fused kernels only (the
    math fallback runs 16-bit batched products on transposed views, avoided here). The
    memory-efficient kernel comes first: on MI355X its causal forward + backward takes
    260 us against the flash kernel's 348 us at B 32, H 8, S 512, D 64, and 550 against
    885 us at B 8, H 16, S 1024, D 128, with the same forward output. Its backward at head
    size 128 accumulates dq in an order that varies from run to run (measured: dk, dv and
    the output repeat bit for bit, dq does not; the flash kernel repeats at both shapes), so
    under torch.use_deterministic_algorithms(True) the flash kernel comes first."""
    if q.is_cuda and q.dtype in (torch.bfloat16, torch.float16):
        deterministic = torch.are_deterministic_algorithms_enabled()
        if (hip_attention_forward and not deterministic and kwargs.get("is_causal")
                and not kwargs.get("dropout_p") and kwargs.keys() <= {"is_causal", "dropout_p"}
                and attention_supported(q, k, v)):
            # the HIP forward with torch's memory-efficient backward (attention.py)
            return CausalAttentionFn.apply(q, k, v)
        order = _DETERMINISTIC_ATTENTION if deterministic else _FAST_ATTENTION
        with sdpa_kernel(order, set_priority=True):
            return F.scaled_dot_product_attention(q, k, v, **kwargs)
    return F.scaled_dot_product_attention(q, k, v, **kwargs)


class _TokenLookup(torch.autograd.Function):
    """``embedding(tokens, weight)`` whose weight gradient comes from the HIP kernels
    (``rk_embedding_backward``): a fixed-order float32 sum per vocabulary row, made of plain
    kernel launches. torch's own backward sorts the ids on the device and clears the sort's
    state with a memset, which a captured training step would record as a memset node."""

    @staticmethod
    def forward(ctx, tokens: Tensor, weight: Tensor) -> Tensor:
        ctx.save_for_backward(tokens)
        ctx.num_weights = weight.shape[0]
        ctx.weight_dtype = weight.dtype
        return F.embedding(tokens, weight)

    @staticmethod
    def backward(ctx, grad_output: Tensor):
        (tokens,) = ctx.saved_tensors
        from .ops import ratchet as _ops

        grad = _ops().embedding_backward(grad_output, tokens, ctx.num_weights)
        return None, grad.to(ctx.weight_dtype)


def _hip_lookup_config_ok(embedding: nn.Module) -> bool:
    """Whether the HIP embedding-gradient kernels take this embedding (devices aside): a
    plain nn.Embedding in float32 or bf16 without padding_idx, max_norm, sparse gradients or
    scale_grad_by_freq, rows of a multiple of 4 and at most 4096 columns."""
    if type(embedding) is not nn.Embedding:
        return False
    w = embedding.weight
    return (w.dtype in (torch.float32, torch.bfloat16)
            and embedding.padding_idx is None and embedding.max_norm is None
            and not embedding.sparse and not embedding.scale_grad_by_freq
            and w.shape[1] % 4 == 0 and w.shape[1] <= 4096 and w.shape[0] < 2**31 - 1)


def _hip_lookup_supported(embedding: nn.Module, tokens: Tensor) -> bool:
    return (embedding.weight.is_cuda and tokens.is_cuda
            and _hip_lookup_config_ok(embedding))


def _autocast_bf16(t: Tensor) -> torch.dtype | None:
    """torch.bfloat16 when `t`'s device runs under bf16 autocast, else None."""
    dev = t.device.type
    if torch.is_autocast_enabled(dev) and torch.get_autocast_dtype(dev) == torch.bfloat16:
        return torch.bfloat16
    return None


class CausalSelfAttention(nn.Module):
    # int8 qkv: the layer returns q, k, v as chunks whose gradients it reads in place
    split_qkv_grad: bool = True

    def __init__(self, config: ModelConfig, *, max_code: int | None) -> None:
        super().__init__()
        self.qkv = _linear(config, config.n_embd, 3 * config.n_embd, max_code)
        self.projection = _linear(config, config.n_embd, config.n_embd, max_code)
        self.n_head = config.n_head
        self.head_size = config.n_embd // config.n_head
        self.dropout = config.dropout

    def forward(self, inputs: Tensor, *, inputs_int8: Tensor | None = None,
                inputs_scale: Tensor | None = None, cache: KVCache | None = None,
                layer: int = 0, decode: bool = False,
                residual: Tensor | None = None) -> Tensor:
        """``residual``: return residual + attention output (int8 projection: added in the
        GEMM epilogue)."""
        batch_size, sequence_length, channels = inputs.shape
        if inputs_int8 is not None:
            # Under bf16 autocast the attention casts q, k, v to bf16 (and their gradients
            # back): take the GEMM's bf16 result directly instead (the same values; no cast
            # kernels). The layer returns the three chunks itself, so their gradients reach
            # its backward separately and are read there in place (no concatenation).
            kw = {"split": 3} if self.split_qkv_grad else {}
            qkv = self.qkv(inputs, inputs_int8=inputs_int8, inputs_scale=inputs_scale,
                           out_dtype=_autocast_bf16(inputs), **kw)
        else:
            qkv = self.qkv(inputs)
        query, key, value = qkv if isinstance(qkv, tuple) else qkv.chunk(3, dim=-1)

        def heads(t: Tensor) -> Tensor:
            return t.view(batch_size, sequence_length, self.n_head, self.head_size).transpose(1, 2)

        q, k, v = heads(query), heads(key), heads(value)
        dropout_p = self.dropout if self.training else 0.0
        if cache is not None:
            attended = self._cached_attention(q, k, v, cache, layer, decode)
        else:
            attended = _attend(q, k, v, dropout_p=dropout_p, is_causal=True)
        if _is_int8(self.projection):
            attn_int8, attn_scale, dummy = FusedTransposeQuantizeFn.apply(attended)
            return self.projection(dummy, inputs_int8=attn_int8, inputs_scale=attn_scale,
                                   residual=residual)
        joined = attended.transpose(1, 2).contiguous().view(batch_size, sequence_length, channels)
        out = self.projection(joined)
        return out if residual is None else residual + out

    def _cached_attention(self, q: Tensor, k: Tensor, v: Tensor, cache: KVCache, layer: int,
                          decode: bool) -> Tensor:
        """Attention of the new positions against the cache, after appending their keys and
        values. ``decode``: one token at the device-side position ``cache.pos``, attending
        over the whole buffer under a mask (fixed shapes); otherwise a prompt of S tokens
        written at the host-side ``cache.length`` (causal among themselves)."""
        keys, values = cache.buffers(layer, k)
        out_dtype = q.dtype
        if keys.dtype != q.dtype:
            q, k, v = q.to(keys.dtype), k.to(keys.dtype), v.to(keys.dtype)
        if decode:
            keys.index_copy_(2, cache.pos, k)
            values.index_copy_(2, cache.pos, v)
            out = _attend(q, keys, values, attn_mask=cache.decode_mask(q.dtype))
            return out.to(out_dtype)
        start, length = cache.length, q.shape[2]
        end = start + length
        if end > cache.max_len:
            raise ValueError("KV cache is full")
        keys[:, :, start:end] = k
        values[:, :, start:end] = v
        if start == 0:
            return _attend(q, k, v, is_causal=True).to(out_dtype)
        mask = torch.ones(length, end, dtype=torch.bool, device=q.device).tril(diagonal=start)
        out = _attend(q, keys[:, :, :end], values[:, :, :end], attn_mask=mask)
        return out.to(out_dtype)


class FeedForward(nn.Module):
    # Under bf16 autocast an int8 expansion hands its bf16 GEMM result to the GELU prologue
    # (the float32 result is that value widened): the expansion's output, the contraction's
    # grad_input, the GELU backward and the expansion's gradient then move 2-byte values.
    # The contraction keeps the input's dtype for its own output and gradient, as with a
    # float32 expansion.
    bf16_expand: bool = True

    def __init__(self, config: ModelConfig, *, max_code: int | None) -> None:
        super().__init__()
        hidden = config.hidden_size
        self.expand = _linear(config, config.n_embd, hidden, max_code)
        self.contract = _linear(config, hidden, config.n_embd, max_code)
        self.dropout = config.dropout

    def forward(self, inputs: Tensor, *, inputs_int8: Tensor | None = None,
                inputs_scale: Tensor | None = None,
                residual: Tensor | None = None) -> Tensor:
        """``residual``: return residual + feed-forward output (int8 contraction without
        active dropout: added in the GEMM epilogue)."""
        int8_contract = _is_int8(self.contract)
        bf16_out = _autocast_bf16(inputs) if int8_contract and self.bf16_expand else None
        kw = {"out_dtype": bf16_out} if bf16_out is not None else {}
        if inputs_int8 is not None:
            expanded = self.expand(inputs, inputs_int8=inputs_int8, inputs_scale=inputs_scale,
                                   **kw)
        else:
            expanded = self.expand(inputs, **kw)
        no_dropout = self.dropout == 0.0 or not self.training
        if int8_contract:
            gelu_int8, gelu_scale, dummy = FusedGELUQuantizeFn.apply(expanded)
            kw = {"out_dtype": inputs.dtype} if expanded.dtype != inputs.dtype else {}
            if no_dropout:
                return self.contract(dummy, inputs_int8=gelu_int8, inputs_scale=gelu_scale,
                                     residual=residual, **kw)
            contracted = self.contract(dummy, inputs_int8=gelu_int8, inputs_scale=gelu_scale,
                                       **kw)
        else:
            contracted = self.contract(F.gelu(expanded))
        out = F.dropout(contracted, p=self.dropout, training=self.training)
        return out if residual is None else residual + out


class TransformerBlock(nn.Module):
    # int8 blocks hand the residual stream to the attention projection and the feed-forward
    # contraction, whose GEMMs add it in their epilogue (the same float32 add)
    fuse_residual: bool = True
    # with fuse_residual: the block input's two gradients are added in the RMSNorm backward
    # kernel's store instead of by autograd (the same float32 add)
    fuse_residual_grad: bool = True

    def __init__(self, config: ModelConfig, *, max_code: int | None) -> None:
        super().__init__()
        self.attention_norm = nn.RMSNorm(config.n_embd)
        self.attention = CausalSelfAttention(config, max_code=max_code)
        self.feed_forward_norm = nn.RMSNorm(config.n_embd)
        self.feed_forward = FeedForward(config, max_code=max_code)

    def forward(self, inputs: Tensor, *, cache: KVCache | None = None, layer: int = 0,
                decode: bool = False) -> Tensor:
        kv = dict(cache=cache, layer=layer, decode=decode) if cache is not None else {}
        fuse_grad = self.fuse_residual and self.fuse_residual_grad
        if _is_int8(self.attention.qkv):
            if fuse_grad:
                # the block input's two gradients (normalized path, residual stream) meet
                # in the RMSNorm backward's store instead of a separate add
                q, s, dummy, res = FusedRMSNormQuantizeResidualFn.apply(
                    inputs, self.attention_norm.weight, 1e-5)
                inputs = self.attention(dummy, inputs_int8=q, inputs_scale=s, residual=res,
                                        **kv)
            else:
                q, s, dummy = FusedRMSNormQuantizeFn.apply(inputs, self.attention_norm.weight,
                                                           1e-5)
                if self.fuse_residual:
                    inputs = self.attention(dummy, inputs_int8=q, inputs_scale=s,
                                            residual=inputs, **kv)
                else:
                    inputs = inputs + self.attention(dummy, inputs_int8=q, inputs_scale=s,
                                                     **kv)
        else:
            inputs = inputs + self.attention(self.attention_norm(inputs), **kv)
        if _is_int8(self.feed_forward.expand):
            if fuse_grad:
                q, s, dummy, res = FusedRMSNormQuantizeResidualFn.apply(
                    inputs, self.feed_forward_norm.weight, 1e-5)
                inputs = self.feed_forward(dummy, inputs_int8=q, inputs_scale=s, residual=res)
            else:
                q, s, dummy = FusedRMSNormQuantizeFn.apply(inputs, self.feed_forward_norm.weight,
                                                           1e-5)
                if self.fuse_residual:
                    inputs = self.feed_forward(dummy, inputs_int8=q, inputs_scale=s,
                                               residual=inputs)
                else:
                    inputs = inputs + self.feed_forward(dummy, inputs_int8=q, inputs_scale=s)
        else:
            inputs = inputs + self.feed_forward(self.feed_forward_norm(inputs))
        return inputs


def _total(values):
    """Sum of per-layer statistics: device scalars are stacked and summed in one
    reduction (not one addition kernel per layer); host numbers are added as numbers."""
    values = list(values)
    tensors = [v.reshape(()) for v in values if isinstance(v, Tensor)]
    host = sum(v for v in values if not isinstance(v, Tensor))
    if not tensors:
        return host
    total = torch.stack(tensors).sum()
    return total + host if host else total


class RatchetGPT(nn.Module):
    # decode steps use the fused HIP decode kernels where supported (False: the module
    # forwards, e.g. to compare the two)
    fused_decode: bool = True
    # the token embedding's weight gradient from the HIP kernels (False: torch's backward)
    hip_embedding_backward: bool = True
    # the layers' move counts in one model-level buffer, summed and cleared once per step
    shared_move_counts: bool = True
    # the training loss from the HIP cross-entropy kernels (False: F.cross_entropy); with an
    # int8 lm_head the logits of a forward with targets are then bfloat16 (the same values)
    fused_cross_entropy: bool = True

    def __init__(self, config: ModelConfig, *, max_code: int | None) -> None:
        super().__init__()
        self.config = config
        self.max_code = max_code
        if max_code is not None and config.ratchet_embedding:
            self.token_embedding = RatchetEmbedding(
                config.vocab_size, config.n_embd, max_code=max_code,
                pressure_threshold=config.pressure_threshold, bucket_low=config.bucket_low,
                bucket_high=config.bucket_high, trainable_scale=config.trainable_scale,
                compile_update=config.compile_update, rms_ema_beta=config.rms_ema_beta,
                pressure_leak_period=config.pressure_leak_period,
            )
        else:
            self.token_embedding = nn.Embedding(config.vocab_size, config.n_embd)
        self.register_buffer(
            "position_encoding", _sinusoidal_positions(config.block_size, config.n_embd)
        )
        self.blocks = nn.ModuleList(
            TransformerBlock(config, max_code=max_code) for _ in range(config.n_layer)
        )
        self.final_norm = nn.RMSNorm(config.n_embd)
        self.lm_head = _linear(config, config.n_embd, config.vocab_size, max_code)

    def embedding_backward_is_sort_based(self) -> bool:
        """Whether a training step takes the token embedding's weight gradient from torch's
        sort-based embedding backward (``embedding_dense_backward``) instead of the HIP
        kernels: a ratchet embedding (its effective weight goes through F.embedding), the
        HIP path switched off, or an embedding those kernels do not take (padding_idx,
        max_norm, sparse or scale_grad_by_freq, width not a multiple of 4 or above 4096).
        Under graph capture that backward records a memset node that clears its sort's
        state, which is not safe on replays."""
        emb = self.token_embedding
        if type(emb) is not nn.Embedding:
            return True
        if not emb.weight.requires_grad:
            return False
        return not (self.hip_embedding_backward and _hip_lookup_config_ok(emb))

    def forward(self, tokens: Tensor, targets: Tensor | None = None
                ) -> tuple[Tensor, Tensor | None]:
        if tokens.ndim != 2:
            raise ValueError("tokens must have shape (batch, sequence)")
        sequence_length = tokens.shape[1]
        if sequence_length > self.config.block_size:
            raise ValueError("token sequence exceeds configured block_size")
        if self.training and torch.is_grad_enabled() and self.shared_move_counts:
            self._attach_count_slots()
        if self.hip_embedding_backward and _hip_lookup_supported(self.token_embedding, tokens):
            looked_up = _TokenLookup.apply(tokens, self.token_embedding.weight)
        else:
            looked_up = self.token_embedding(tokens)
        hidden = looked_up + self.position_encoding[:sequence_length]
        for block in self.blocks:
            if self.config.gradient_checkpointing and self.training:
                from torch.utils.checkpoint import checkpoint

                hidden = checkpoint(block, hidden, use_reentrant=False)
            else:
                hidden = block(hidden)
        if targets is not None and targets.shape != tokens.shape:
            raise ValueError("targets must have the same shape as tokens")
        fused_loss = (targets is not None and self.fused_cross_entropy and hidden.is_cuda
                      and targets.dtype == torch.int64)
        if fused_loss and _is_int8(self.lm_head):
            # the int8 lm_head's float32 output is its bf16 result widened: the loss reads
            # the bf16 logits (the same values) and hands their gradient back as bf16
            logits = self.lm_head(self.final_norm(hidden), out_dtype=torch.bfloat16)
        else:
            logits = self.lm_head(self.final_norm(hidden))
        loss = None
        if fused_loss:
            loss = cross_entropy(logits.flatten(0, 1), targets.flatten())
        elif targets is not None:
            loss = F.cross_entropy(logits.flatten(0, 1), targets.flatten())
        return logits, loss

    # -- incremental decoding ---------------------------------------------------
    def new_cache(self, batch: int, max_len: int | None = None,
                  dtype: torch.dtype | None = None) -> KVCache:
        """An empty KV cache for `batch` sequences of up to `max_len` (<= block_size) tokens.
        `dtype` (e.g. bfloat16) stores keys/values and runs the cached attention in that
        type; by default they keep the activations' dtype."""
        max_len = max_len or self.config.block_size
        if max_len > self.config.block_size:
            raise ValueError("a cache cannot outgrow block_size (positions are absolute)")
        device = self.position_encoding.device
        return KVCache(self.config.n_layer, batch, self.config.n_head,
                       self.config.n_embd // self.config.n_head, max_len, device, dtype)

    @torch.no_grad()
    def prefill(self, tokens: Tensor, cache: KVCache) -> Tensor:
        """Run `tokens` [B, S] at positions cache.length .. +S, append their keys/values, and
        return the logits of the last position [B, vocab]."""
        start, length = cache.length, tokens.shape[1]
        hidden = self.token_embedding(tokens) + self.position_encoding[start:start + length]
        for index, block in enumerate(self.blocks):
            hidden = block(hidden, cache=cache, layer=index)
        cache.advance(length)
        return self.lm_head(self.final_norm(hidden[:, -1:]))[:, 0]

    @torch.no_grad()
    def decode_step(self, tokens: Tensor, cache: KVCache) -> Tensor:
        """One token per sequence (`tokens` [B, 1]) at the device-side position cache.pos;
        returns its logits [B, vocab] and advances the cache. Shapes do not depend on the
        position, so the step can be captured once and replayed (the caller then advances
        the cache itself)."""
        logits = self.decode_logits(tokens, cache).clone()
        cache.advance(1)
        return logits

    def decode_logits(self, tokens: Tensor, cache: KVCache) -> Tensor:
        """decode_step without advancing the cache (the capturable part). On a ROCm GPU
        with int8 ratchet layers of supported shapes the step runs on the fused decode
        kernels (``decode.fused_decode_logits``; its result buffer is reused by the next
        step); otherwise through the module forwards."""
        from .decode import fused_decode_logits, fused_decode_supported

        if self.fused_decode and fused_decode_supported(self, cache):
            return fused_decode_logits(self, tokens, cache)
        cache.begin_step()
        hidden = self.token_embedding(tokens) + self.position_encoding.index_select(
            0, cache.pos).view(1, 1, -1)
        for index, block in enumerate(self.blocks):
            hidden = block(hidden, cache=cache, layer=index, decode=True)
        return self.lm_head(self.final_norm(hidden))[:, 0]

    def _attach_count_slots(self) -> None:
        """One int64 [layers, 4] move-count buffer for every ratchet layer of the model (each
        layer's update adds into its row): summed and cleared once per step by
        ``ratchet_update`` instead of one zero-filled tensor per layer and step."""
        layers = [m for m in self.modules() if isinstance(m, DiscreteRatchetLinear)]
        if not layers:
            return
        device = layers[0].packed.device
        buf = getattr(self, "_count_slots", None)
        if (buf is not None and buf.device == device and buf.shape[0] == len(layers)
                and all(m._counts_slot is not None for m in layers)):
            return
        buf = torch.zeros(len(layers), 4, dtype=torch.int64, device=device)
        for i, m in enumerate(layers):
            m._counts_slot = buf[i]
            m._slot_dirty = False
        self._count_slots = buf
        # the layers' row rms in one buffer too, segment s = layer s: one launch takes every
        # layer's mean row rms for the step's statistics
        sizes = [m.out_features for m in layers]
        bounds = [0]
        for n in sizes:
            bounds.append(bounds[-1] + n)
        rms = torch.zeros(bounds[-1], dtype=torch.float32, device=device)
        self._rms_slots = rms
        self._rms_offsets = torch.tensor(bounds, dtype=torch.int64, device=device)
        for i, m in enumerate(layers):
            m._rms_slot = rms[bounds[i]:bounds[i + 1]]
            m._rms_slot_bounds = torch.tensor([0, sizes[i]], dtype=torch.int64, device=device)

    def defer_ratchet_updates(self, enabled: bool = True) -> None:
        """Batch the ratchet layers' fused updates: backward queues each layer's update
        instead of launching it, and the next ``ratchet_update()`` (or
        ``flush_ratchet_updates()``, ``discard_pending_gradients()``, or a queued layer's
        next forward) runs them together, a few launches for the whole model. States, move
        counts, row rms and EMA after ``ratchet_update()`` are bit-identical to the
        per-layer updates; between backward and that call the layers hold their pre-update
        states. Layers that need a trainable-scale gradient from backward, or keep their
        weight gradient, still update inside backward."""
        queue = UpdateQueue() if enabled else None
        old = getattr(self, "_update_queue", None)
        if old is not None:
            old.flush()
        for m in self.modules():
            if isinstance(m, DiscreteRatchetLinear):
                m._update_queue = queue
        self._update_queue = queue

    def flush_ratchet_updates(self) -> None:
        """Run the updates backward queued (``defer_ratchet_updates``), if any."""
        queue = getattr(self, "_update_queue", None)
        if queue is not None:
            queue.flush()

    def ratchet_update(self, *, validate: bool = True) -> RatchetUpdateStats:
        self.flush_ratchet_updates()
        layers = [m for m in self.modules() if isinstance(m, DiscreteRatchetLinear)]
        buf = getattr(self, "_count_slots", None)
        shared = (buf is not None and buf.shape[0] == len(layers)
                  and all(m._counts_slot is not None and m._counts_slot.data_ptr()
                          == buf[i].data_ptr() for i, m in enumerate(layers)))
        if shared:
            # slots whose counts a layer-level ratchet_update already reported
            for i, m in enumerate(layers):
                if m._slot_dirty:
                    buf[i].zero_()
                    m._slot_dirty = False
        # every layer's first launch of the step left its row rms in the shared buffer: one
        # launch for all their means (each equal to the per-layer launch's)
        rms = getattr(self, "_rms_slots", None)
        slot_means = None
        if (rms is not None and rms.shape[0] == sum(m.out_features for m in layers)
                and all(m._rms_slot is not None and len(m._pending_rms_means) == 1
                        and m._pending_rms_means[0] is None for m in layers)):
            from .ops import ratchet as _ratchet_ops

            slot_means = _ratchet_ops().row_rms_means(rms, self._rms_offsets)
            for i, m in enumerate(layers):
                m._rms_slot_mean = slot_means[i]
        if shared:
            # one copy of every layer's slot for their stats to own (one launch, where a
            # clone per layer was one small copy each)
            snapshot = buf.clone()
            for i, m in enumerate(layers):
                m._counts_snapshot = snapshot[i]
        try:
            updates = [m.ratchet_update(validate=validate) for m in layers]
        finally:
            for m in layers:
                m._counts_snapshot = None
        if shared:
            # the layers' counts live in one buffer: one reduction for the four totals,
            # then the buffer is cleared for the next step
            totals = snapshot.sum(dim=0)
            moves = (totals[0], totals[1], totals[2], totals[3])
            buf.zero_()
            for m in layers:
                m._slot_dirty = False
        else:
            moves = (_total(u.positive_moves for u in updates),
                     _total(u.negative_moves for u in updates),
                     _total(u.blocked_positive_moves for u in updates),
                     _total(u.blocked_negative_moves for u in updates))
        aggregated = RatchetUpdateStats(
            total_weights=sum(u.total_weights for u in updates),
            positive_moves=moves[0],
            negative_moves=moves[1],
            blocked_positive_moves=moves[2],
            blocked_negative_moves=moves[3],
            # unvalidated, the layers' means are views of one vector: its sum is the sum of
            # their stack (validated, they are host floats, added as floats)
            gradient_rms_mean=(slot_means.sum() / len(updates)
                               if slot_means is not None and not validate
                               else _total(u.gradient_rms_mean for u in updates) / len(updates)
                               if updates else 0.0),
        )
        return aggregated.materialize() if validate else aggregated

    def discard_pending_gradients(self) -> None:
        self.flush_ratchet_updates()
        for module in self.modules():
            if isinstance(module, DiscreteRatchetLinear):
                module.discard_pending_gradient()


def build_seeded_model(config: ModelConfig, *, max_code: int | None, seed: int) -> RatchetGPT:
    """Build matched arms without changing the caller's global CPU RNG state."""
    with torch.random.fork_rng(devices=[]):
        torch.manual_seed(seed)
        return RatchetGPT(config, max_code=max_code)
