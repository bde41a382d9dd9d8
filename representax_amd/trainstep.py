"""INT4-LoRA encoder train step: the harness around the quantized linear path.

A BERT-base-shaped encoder whose every Q/K/V/O/FFN projection is a
``QuantizedLoRALinear`` (the fused INT4-LoRA HIP kernels), trained with the
in-batch multiple-negatives ranking (MNR) loss and AdamW on the fp32 LoRA
masters only. It restates the reference's model and step:

* embeddings (word + position + token type, LayerNorm) and post-LN layers
  with a GELU MLP: src/representax/models/bert/model.py:74-330;
* mean pooling over the attention mask and L2 normalisation:
  src/representax/models/bert/model.py:566-574,
  src/representax/models/components.py:238-270;
* LayerNorm with float32 statistics: src/representax/models/components.py:110-132;
* MNR loss (cosine logits times ``scale``, logsumexp over the in-batch
  documents, forward direction): src/representax/tasks/retrieval/mnr.py:48-158;
* adapters on every layer projection with only ``lora_a``/``lora_b``
  trainable: src/representax/models/adapters.py:201-267.

bf16 compute with fp32 masters follows the ``bfloat16_mixed`` policy
(src/representax/precision.py:19-124). Dropout is off (probability 0, as in
the reference's benchmark configuration). Attention runs as explicit batched
products with contiguous right-hand operands in float32, and through torch's
fused flash / memory-efficient kernels in bf16.

The step follows src/representax/train/step.py:346-393: per-layer activation
rematerialization ("full" by default, config.py:483-490, applied per layer
as in components.py:28-43), the global gradient norm in float32, clipping to
``max_grad_norm`` (1.0 by default, step.py:123) and a step that leaves
parameters and optimizer state unchanged when the loss, the gradients or
their norm are not finite (``optax.tree.where(finite, proposed, state)``).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch.utils.checkpoint import checkpoint

from . import ops
from .adapters import apply_quantized_lora, lora_parameters
from .components import Linear
from .config import PrecisionConfig
from .mlp import gelu_mlp, shared_input_projections, swiglu_mlp
from .precision import (active_compute_views, active_policy, compute_views, precision_context,
                        resolve_precision_policy)


@dataclass(frozen=True)
class BertConfig:
    """Shape of the encoder (BERT-base defaults)."""

    vocab_size: int = 30522
    hidden_size: int = 768
    num_hidden_layers: int = 12
    num_attention_heads: int = 12
    intermediate_size: int = 3072
    max_position_embeddings: int = 512
    type_vocab_size: int = 2
    norm_epsilon: float = 1e-12
    initializer_range: float = 0.02
    pad_token_id: int = 0

    @property
    def head_dimension(self) -> int:
        return self.hidden_size // self.num_attention_heads

    def step_flops(self, batch: int, sequence: int, *, remat: bool = False) -> float:
        """Matrix FLOPs of one train step over ``batch`` sequences (linears,
        attention products; forward, optional recompute, backward)."""

        h, f, s = self.hidden_size, self.intermediate_size, sequence
        tokens = batch * sequence
        linear = 2.0 * tokens * (4 * h * h + 2 * h * f)
        attention = 4.0 * batch * s * s * h
        forward = self.num_hidden_layers * (linear + attention)
        # backward: dX through every linear and both attention products twice
        backward = self.num_hidden_layers * (linear + 2 * attention)
        return forward * (2 if remat else 1) + backward


class LayerNorm(torch.nn.Module):
    """Last-axis LayerNorm with float32 statistics, output in the input dtype."""

    def __init__(self, size: int, eps: float, device=None) -> None:
        super().__init__()
        self.weight = torch.nn.Parameter(torch.ones(size, device=device))
        self.bias = torch.nn.Parameter(torch.zeros(size, device=device))
        self.eps = eps

    def forward(self, value: torch.Tensor) -> torch.Tensor:
        # torch's reduced-precision layer_norm keeps float32 statistics and
        # rounds the normalized, affine-transformed value once
        return F.layer_norm(value, value.shape[-1:], self.weight.to(value.dtype),
                            self.bias.to(value.dtype), self.eps)


REMAT_POLICIES = ("none", "full")


def run_layer(layer: torch.nn.Module, remat: str, *args):
    """One layer, rematerialized in the backward pass under ``"full"`` (the
    reference's nothing-saveable checkpoint around each layer): only the
    layer's inputs are kept, and its forward, INT4 + LoRA kernels included,
    runs again before its backward."""

    if remat == "full" and torch.is_grad_enabled():
        # the recompute runs inside backward(), outside the caller's precision
        # context: it re-enters the policy (and compute views) the forward
        # saw, as jax.checkpoint replays the function traced under them
        policy = active_policy()
        views = active_compute_views()

        def layer_under_policy(*inputs):
            if policy is None:
                return layer(*inputs)
            with precision_context(policy), compute_views(views):
                return layer(*inputs)

        return checkpoint(layer_under_policy, *args, use_reentrant=False,
                          preserve_rng_state=False)
    if remat not in REMAT_POLICIES:
        raise ValueError("rematerialization must be 'none' or 'full'")
    return layer(*args)


class _Attention(torch.autograd.Function):
    """softmax(Q K^T * scale + bias) V over ``[B, H, S, D]`` with every
    batched product taking a contiguous right operand."""

    @staticmethod
    def forward(ctx, q, k, v, bias, scale):
        q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
        s = torch.matmul(q, k.transpose(-1, -2).contiguous()).float() * scale
        if bias is not None:
            s = s + bias
        p = torch.softmax(s, dim=-1).to(q.dtype)
        ctx.save_for_backward(q, k, v, p)
        ctx.scale = scale
        return torch.matmul(p, v)

    @staticmethod
    def backward(ctx, do):
        q, k, v, p = ctx.saved_tensors
        do = do.contiguous()
        dv = torch.matmul(p.transpose(-1, -2).contiguous(), do)
        dp = torch.matmul(do, v.transpose(-1, -2).contiguous()).float()
        pf = p.float()
        ds = (pf * (dp - (dp * pf).sum(-1, keepdim=True)) * ctx.scale).to(q.dtype)
        dq = torch.matmul(ds, k)
        dk = torch.matmul(ds.transpose(-1, -2).contiguous(), q)
        return dq, dk, dv, None, None


def attention(q, k, v, bias, scale):
    """``[B, H, S, D]`` attention. bf16/fp16 inputs use torch's fused flash
    or memory-efficient kernels only (never the unfused math fallback);
    float32 inputs use the explicit products above."""

    if q.dtype in (torch.bfloat16, torch.float16):
        from torch.nn.attention import SDPBackend, sdpa_kernel

        backends = [SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]
        if bias is not None:
            backends = [SDPBackend.EFFICIENT_ATTENTION]
        with sdpa_kernel(backends):
            return F.scaled_dot_product_attention(
                q, k, v, attn_mask=None if bias is None else bias.to(q.dtype), scale=scale)
    return _Attention.apply(q, k, v, bias, scale)


class BertSelfAttention(torch.nn.Module):
    def __init__(self, config: BertConfig, key: int, device=None) -> None:
        super().__init__()
        arg = dict(scale=config.initializer_range, bias=True, device=device)
        h = config.hidden_size
        self.query = Linear.init(h, h, key=key + 0, **arg)
        self.key = Linear.init(h, h, key=key + 1, **arg)
        self.value = Linear.init(h, h, key=key + 2, **arg)
        self.output = Linear.init(h, h, key=key + 3, **arg)
        self.heads = config.num_attention_heads
        self.head_dim = config.head_dimension

    def forward(self, hidden: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
        b, s, h = hidden.shape

        q, k, v = (t.reshape(b, s, self.heads, self.head_dim).transpose(1, 2)
                   for t in shared_input_projections(hidden, (self.query, self.key, self.value)))
        out = attention(q, k, v, bias, 1.0 / math.sqrt(self.head_dim))
        return self.output(out.transpose(1, 2).reshape(b, s, h))


class BertMLP(torch.nn.Module):
    def __init__(self, config: BertConfig, key: int, device=None) -> None:
        super().__init__()
        arg = dict(scale=config.initializer_range, bias=True, device=device)
        self.input = Linear.init(config.hidden_size, config.intermediate_size, key=key, **arg)
        self.output = Linear.init(config.intermediate_size, config.hidden_size, key=key + 1, **arg)

    def forward(self, hidden: torch.Tensor) -> torch.Tensor:
        # output(gelu(input(hidden))), fused when both are INT4 + LoRA
        return gelu_mlp(hidden, self.input, self.output)


class BertLayer(torch.nn.Module):
    def __init__(self, config: BertConfig, key: int, device=None) -> None:
        super().__init__()
        self.attention = BertSelfAttention(config, key, device)
        self.attention_norm = LayerNorm(config.hidden_size, config.norm_epsilon, device)
        self.mlp = BertMLP(config, key + 4, device)
        self.output_norm = LayerNorm(config.hidden_size, config.norm_epsilon, device)

    def forward(self, hidden: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
        hidden = self.attention_norm(hidden + self.attention(hidden, bias))
        return self.output_norm(hidden + self.mlp(hidden))


class BertEncoder(torch.nn.Module):
    """Embeddings, post-LN layers, masked mean pooling, L2 normalisation."""

    def __init__(self, config: BertConfig, seed: int = 0, device=None) -> None:
        super().__init__()
        self.config = config
        g = torch.Generator().manual_seed(seed)

        def table(rows):
            t = config.initializer_range * torch.randn(rows, config.hidden_size, generator=g)
            return torch.nn.Parameter(t.to(device))

        self.word = table(config.vocab_size)
        with torch.no_grad():
            self.word[config.pad_token_id].zero_()
        self.position = table(config.max_position_embeddings)
        self.token_type = table(config.type_vocab_size)
        self.embedding_norm = LayerNorm(config.hidden_size, config.norm_epsilon, device)
        self.layers = torch.nn.ModuleList(
            BertLayer(config, seed * 1000 + 10 * (i + 1), device)
            for i in range(config.num_hidden_layers))
        self.remat = "none"

    def hidden_states(self, input_ids: torch.Tensor, attention_mask: torch.Tensor | None = None,
                      compute_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
        """``attention_mask`` None means every position is a real token."""

        s = input_ids.shape[1]
        hidden = (self.word[input_ids] + self.position[:s][None]
                  + self.token_type[torch.zeros_like(input_ids)])
        hidden = self.embedding_norm(hidden).to(compute_dtype)
        bias = None
        if attention_mask is not None:
            bias = torch.zeros(attention_mask.shape, dtype=torch.float32, device=hidden.device)
            bias = bias.masked_fill(~attention_mask.bool(), float("-inf"))[:, None, None, :]
        for layer in self.layers:
            hidden = run_layer(layer, self.remat, hidden, bias)
        return hidden

    def encode(self, input_ids: torch.Tensor, attention_mask: torch.Tensor | None = None,
               compute_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
        hidden = self.hidden_states(input_ids, attention_mask, compute_dtype).float()
        if attention_mask is None:
            pooled = hidden.mean(1)
        else:
            mask = attention_mask.to(hidden.dtype)[..., None]
            pooled = (hidden * mask).sum(1) / mask.sum(1).clamp_min(1.0)
        return pooled / pooled.norm(dim=-1, keepdim=True).clamp_min(1e-12)


def mnr_loss(queries: torch.Tensor, documents: torch.Tensor, scale: float = 20.0) -> torch.Tensor:
    """Mean over queries of ``logsumexp_j(scale cos(q, d_j)) - scale cos(q, d_q)``
    with each query's own document as its positive
    (src/representax/tasks/retrieval/mnr.py:48-52,132-158,338-341): the
    fused HIP loss, f32 casts and normalisation included."""

    return ops.mnr_loss(queries, documents, scale)


LAYER_LINEARS = r"\.layers\[\d+\]\.(attention\.(query|key|value|output)|mlp\.(input|output|gate|up|down))$"


def build_int4lora_encoder(config: BertConfig, *, rank: int = 16, alpha: float = 32.0,
                           group_size: int | None = 64, seed: int = 0,
                           device: torch.device | str = "cuda") -> BertEncoder:
    """Random-init encoder with every layer projection packed INT4 plus a
    rank-``rank`` adapter; every other parameter is frozen."""

    model = BertEncoder(config, seed=seed, device=device)
    model = apply_quantized_lora(model, rank=rank, alpha=alpha, key=seed,
                                 target_pattern=LAYER_LINEARS, group_size=group_size,
                                 inplace=True)
    trainable = {id(p) for p in lora_parameters(model)}
    for p in model.parameters():
        p.requires_grad_(id(p) in trainable)
    return model


# ---------------------------------------------------------------------------
# Qwen3-VL-shaped text tower (src/representax/models/qwen3_vl/text.py:23-359,
# model.py:212-223): pre-norm causal GQA / SwiGLU decoder layers with per-head
# query/key RMSNorm and rotary positions, final RMSNorm, last-token pooling.
# For text-only inputs the three MRoPE position streams are equal, so the
# interleaved rotary embedding is the ordinary one (text.py:30-61).
# ---------------------------------------------------------------------------
@dataclass(frozen=True)
class Qwen3TextConfig:
    """Shape of the text tower (Qwen3-VL-2B defaults)."""

    vocab_size: int = 151936
    hidden_size: int = 2048
    num_hidden_layers: int = 28
    num_attention_heads: int = 16
    num_key_value_heads: int = 8
    head_dimension: int = 128
    intermediate_size: int = 6144
    rope_theta: float = 5_000_000.0
    norm_epsilon: float = 1e-6
    initializer_range: float = 0.02

    def step_flops(self, batch: int, sequence: int, *, remat: bool = False) -> float:
        h, f, d = self.hidden_size, self.intermediate_size, self.head_dimension
        q = self.num_attention_heads * d
        kv = self.num_key_value_heads * d
        tokens = batch * sequence
        linear = 2.0 * tokens * (h * q + 2 * h * kv + q * h + 3 * h * f)
        # causal attention: half of the score and value products
        attention = 2.0 * batch * sequence * sequence * q
        forward = self.num_hidden_layers * (linear + attention)
        backward = self.num_hidden_layers * (linear + 2 * attention)
        return forward * (2 if remat else 1) + backward


class RMSNorm(torch.nn.Module):
    """Last-axis RMS normalisation with float32 statistics
    (src/representax/models/components.py:134-150)."""

    def __init__(self, size: int, eps: float, device=None) -> None:
        super().__init__()
        self.weight = torch.nn.Parameter(torch.ones(size, device=device))
        self.eps = eps

    def forward(self, value: torch.Tensor) -> torch.Tensor:
        v = value.float()
        v = v * torch.rsqrt(v.square().mean(-1, keepdim=True) + self.eps)
        return (v * self.weight.float()).to(value.dtype)


def _rotate_half(value: torch.Tensor) -> torch.Tensor:
    first, second = value.chunk(2, dim=-1)
    return torch.cat((-second, first), dim=-1)


class Qwen3Attention(torch.nn.Module):
    def __init__(self, config: Qwen3TextConfig, key: int, device=None) -> None:
        super().__init__()
        arg = dict(scale=config.initializer_range, bias=False, device=device)
        h, d = config.hidden_size, config.head_dimension
        self.heads, self.kv_heads, self.head_dim = (config.num_attention_heads,
                                                    config.num_key_value_heads, d)
        self.query = Linear.init(h, self.heads * d, key=key + 0, **arg)
        self.key = Linear.init(h, self.kv_heads * d, key=key + 1, **arg)
        self.value = Linear.init(h, self.kv_heads * d, key=key + 2, **arg)
        self.output = Linear.init(self.heads * d, h, key=key + 3, **arg)
        self.query_norm = RMSNorm(d, config.norm_epsilon, device)
        self.key_norm = RMSNorm(d, config.norm_epsilon, device)

    def forward(self, hidden, cos, sin):
        b, s, _ = hidden.shape
        q, k, v = shared_input_projections(hidden, (self.query, self.key, self.value))
        q = self.query_norm(q.reshape(b, s, self.heads, self.head_dim))
        k = self.key_norm(k.reshape(b, s, self.kv_heads, self.head_dim))
        v = v.reshape(b, s, self.kv_heads, self.head_dim)
        cos, sin = cos[:, :, None], sin[:, :, None]
        q = (q.float() * cos + _rotate_half(q.float()) * sin).to(hidden.dtype)
        k = (k.float() * cos + _rotate_half(k.float()) * sin).to(hidden.dtype)
        rep = self.heads // self.kv_heads
        q, k, v = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
        if rep > 1:
            k = k.repeat_interleave(rep, dim=1)
            v = v.repeat_interleave(rep, dim=1)
        out = causal_attention(q, k, v, 1.0 / math.sqrt(self.head_dim))
        return self.output(out.transpose(1, 2).reshape(b, s, self.heads * self.head_dim))


def causal_attention(q, k, v, scale):
    """Causal ``[B, H, S, D]`` attention; bf16 through torch's fused kernels,
    float32 through explicit products with a -inf upper triangle."""

    if q.dtype in (torch.bfloat16, torch.float16):
        from torch.nn.attention import SDPBackend, sdpa_kernel

        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            return F.scaled_dot_product_attention(q, k, v, is_causal=True, scale=scale)
    s = q.shape[-2]
    bias = torch.full((s, s), float("-inf"), device=q.device).triu(1)
    return _Attention.apply(q, k, v, bias, scale)


class Qwen3MLP(torch.nn.Module):
    def __init__(self, config: Qwen3TextConfig, key: int, device=None) -> None:
        super().__init__()
        arg = dict(scale=config.initializer_range, bias=False, device=device)
        h, f = config.hidden_size, config.intermediate_size
        self.gate = Linear.init(h, f, key=key, **arg)
        self.up = Linear.init(h, f, key=key + 1, **arg)
        self.down = Linear.init(f, h, key=key + 2, **arg)

    def forward(self, hidden):
        # down(silu(gate(hidden)) * up(hidden)), fused when all are INT4 + LoRA
        return swiglu_mlp(hidden, self.gate, self.up, self.down)


class Qwen3Layer(torch.nn.Module):
    def __init__(self, config: Qwen3TextConfig, key: int, device=None) -> None:
        super().__init__()
        self.input_norm = RMSNorm(config.hidden_size, config.norm_epsilon, device)
        self.attention = Qwen3Attention(config, key, device)
        self.post_attention_norm = RMSNorm(config.hidden_size, config.norm_epsilon, device)
        self.mlp = Qwen3MLP(config, key + 4, device)

    def forward(self, hidden, cos, sin):
        hidden = hidden + self.attention(self.input_norm(hidden), cos, sin)
        return hidden + self.mlp(self.post_attention_norm(hidden))


class Qwen3TextEncoder(torch.nn.Module):
    """Token embedding, decoder layers, final norm, last-token pooling and L2
    normalisation (every sequence is full length)."""

    def __init__(self, config: Qwen3TextConfig, seed: int = 0, device=None) -> None:
        super().__init__()
        self.config = config
        g = torch.Generator().manual_seed(seed)
        table = config.initializer_range * torch.randn(config.vocab_size, config.hidden_size,
                                                       generator=g)
        self.embedding = torch.nn.Parameter(table.to(device))
        self.layers = torch.nn.ModuleList(
            Qwen3Layer(config, seed * 1000 + 10 * (i + 1), device)
            for i in range(config.num_hidden_layers))
        self.remat = "none"
        self.final_norm = RMSNorm(config.hidden_size, config.norm_epsilon, device)
        inv = 1.0 / (config.rope_theta ** (torch.arange(0, config.head_dimension, 2,
                                                        dtype=torch.float32)
                                           / config.head_dimension))
        self.register_buffer("inverse_frequency", inv.to(device), persistent=False)

    def rotary(self, sequence: int):
        pos = torch.arange(sequence, device=self.inverse_frequency.device, dtype=torch.float32)
        freq = pos[:, None] * self.inverse_frequency[None]
        emb = torch.cat((freq, freq), dim=-1)
        return emb.cos()[None], emb.sin()[None]

    def encode(self, input_ids: torch.Tensor, attention_mask=None,
               compute_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
        del attention_mask  # full-length sequences: the last token is position S - 1
        hidden = self.embedding[input_ids].to(compute_dtype)
        cos, sin = self.rotary(input_ids.shape[1])
        for layer in self.layers:
            hidden = run_layer(layer, self.remat, hidden, cos, sin)
        pooled = self.final_norm(hidden)[:, -1].float()
        return pooled / pooled.norm(dim=-1, keepdim=True).clamp_min(1e-12)


def build_int4lora_qwen3(config: Qwen3TextConfig, *, rank: int = 32, alpha: float = 64.0,
                         group_size: int | None = 64, seed: int = 0,
                         device: torch.device | str = "cuda") -> Qwen3TextEncoder:
    """Random-init text tower with all seven projections of every layer packed
    INT4 plus a rank-``rank`` adapter; every other parameter is frozen."""

    model = Qwen3TextEncoder(config, seed=seed, device=device)
    model = apply_quantized_lora(model, rank=rank, alpha=alpha, key=seed,
                                 target_pattern=LAYER_LINEARS, group_size=group_size,
                                 inplace=True)
    trainable = {id(p) for p in lora_parameters(model)}
    for p in model.parameters():
        p.requires_grad_(id(p) in trainable)
    return model


class MNRTrainStep:
    """One AdamW step of the MNR loss on (query, document) token batches.

    The step restates src/representax/train/step.py:346-393 for the LoRA
    masters: gradients of the loss (with ``remat`` applied per layer), their
    float32 global norm, clipping by ``min(1, max_grad_norm / (norm + 1e-6))``
    (none when ``max_grad_norm`` is None), an AdamW update, and the whole
    update discarded (parameters and optimizer state restored) unless the
    loss, the gradient norm and hence every gradient are finite.

    The masters live in one flat float32 buffer (the modules' parameters are
    views of it, and so are their gradients), so the norm, the clip, AdamW
    and the finite guard are a handful of kernels per step. Their bf16
    compute views (``compute_parameter``) are slices of one bf16 buffer
    converted from the masters once per step, each a leaf whose gradient is
    left to autograd (no preset ``.grad``, so each view takes its gradient
    tensor as returned, with no accumulate kernel) and then gathered into the
    masters' float32 gradient by one concatenation (the transpose of the
    cast): two kernels per step instead of a cast per parameter use and an
    add per gradient.
    ``capture()`` records forward, backward and the update into one HIP graph
    over static input buffers; ``__call__`` replays it (or runs eagerly
    before capture).
    """

    def __init__(self, model: torch.nn.Module, *, batch: int, sequence: int, lr: float = 1e-4,
                 scale: float = 20.0, seed: int = 6, remat: str = "full",
                 max_grad_norm: float | None = 1.0) -> None:
        if remat not in REMAT_POLICIES:
            raise ValueError("rematerialization must be 'none' or 'full'")
        if max_grad_norm is not None and max_grad_norm <= 0:
            raise ValueError("max_grad_norm must be positive or None")
        self.model = model
        model.remat = remat
        self.remat = remat
        self.max_grad_norm = max_grad_norm
        self.policy = resolve_precision_policy(PrecisionConfig.bfloat16_mixed())
        device = next(model.parameters()).device
        self.params = lora_parameters(model)
        # flat storage: every master (and its gradient) is a view of one buffer
        sizes = [p.numel() for p in self.params]
        self.flat = torch.nn.Parameter(torch.cat([p.detach().reshape(-1) for p in self.params]))
        self.flat.grad = torch.zeros_like(self.flat)
        self.flat_c = torch.zeros(self.flat.numel(), dtype=torch.bfloat16, device=device)
        self.views: dict[int, torch.Tensor] = {}
        self.view_list: list[torch.Tensor] = []
        offset = 0
        for p, n in zip(self.params, sizes):
            p.data = self.flat.data[offset:offset + n].view_as(p)
            p.grad = self.flat.grad[offset:offset + n].view_as(p)
            view = self.flat_c[offset:offset + n].view_as(p).detach().requires_grad_(True)
            self.views[id(p)] = view
            self.view_list.append(view)
            offset += n
        self.optimizer = torch.optim.AdamW([self.flat], lr=lr, weight_decay=0.01,
                                           capturable=True, foreach=False)
        # the state AdamW would create on its first step, made up front so
        # that every step can snapshot it
        self.optimizer.state[self.flat] = {
            "step": torch.zeros((), dtype=torch.float32, device=device),
            "exp_avg": torch.zeros_like(self.flat, memory_format=torch.preserve_format),
            "exp_avg_sq": torch.zeros_like(self.flat, memory_format=torch.preserve_format),
        }
        g = torch.Generator(device="cpu").manual_seed(seed)
        vocab = model.config.vocab_size
        self.query_ids = torch.randint(0, vocab, (batch, sequence), generator=g).to(device)
        self.document_ids = torch.randint(0, vocab, (batch, sequence), generator=g).to(device)
        self.scale = scale
        self.loss = torch.zeros((), dtype=torch.float32, device=device)
        self.grad_norm = torch.zeros((), dtype=torch.float32, device=device)
        self.finite = torch.ones((), dtype=torch.bool, device=device)
        self._backup = None
        self.graph = None

    def _state_tensors(self) -> list[torch.Tensor]:
        st = self.optimizer.state[self.flat]
        return [self.flat.data, st["exp_avg"], st["exp_avg_sq"], st["step"]]

    def _step(self) -> None:
        for view in self.view_list:
            view.grad = None
        with torch.no_grad():
            self.flat_c.copy_(self.flat)
        with precision_context(self.policy), compute_views(self.views):
            ids = torch.cat([self.query_ids, self.document_ids], 0)
            emb = self.model.encode(ids)
            b = self.query_ids.shape[0]
            loss = mnr_loss(emb[:b], emb[b:], self.scale)
        loss.backward()
        grad = self.flat.grad
        # bf16 view gradients -> the masters' float32 gradient, one kernel (a
        # view that took no part in the loss has gradient zero)
        torch.cat([(v.grad if v.grad is not None else torch.zeros_like(v)).reshape(-1)
                   for v in self.view_list], out=grad)
        norm = torch.linalg.vector_norm(grad, dtype=torch.float32)
        finite = torch.isfinite(loss.detach()) & torch.isfinite(norm)
        if self.max_grad_norm is not None:
            coef = torch.clamp(self.max_grad_norm / (norm + 1e-6), max=1.0)
            grad.mul_(coef)
        state = self._state_tensors()
        if self._backup is None:
            self._backup = [t.clone() for t in state]
        else:
            for dst, src in zip(self._backup, state):
                dst.copy_(src)
        self.optimizer.step()
        for t, old in zip(state, self._backup):
            t.copy_(torch.where(finite, t, old))
        self.loss.copy_(loss.detach())
        self.grad_norm.copy_(norm)
        self.finite.copy_(finite)

    def capture(self, warmup: int = 2) -> None:
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(warmup):
                self._step()
        torch.cuda.current_stream().wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self._step()

    def __call__(self) -> torch.Tensor:
        if self.graph is None:
            self._step()
        else:
            self.graph.replay()
        return self.loss


__all__ = [
    "BertConfig",
    "BertEncoder",
    "Qwen3TextConfig",
    "Qwen3TextEncoder",
    "build_int4lora_qwen3",
    "causal_attention",
    "LAYER_LINEARS",
    "MNRTrainStep",
    "REMAT_POLICIES",
    "attention",
    "build_int4lora_encoder",
    "mnr_loss",
    "run_layer",
]
