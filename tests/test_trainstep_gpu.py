"""The INT4-LoRA encoder train step on the GPU: only the LoRA masters move,
and the bf16 fused path agrees with a float32 torch restatement of the same
model (tests/models/test_adapters.py:97-153 for the training invariants)."""

from __future__ import annotations

import math

import pytest
import torch

from representax_amd import QuantizedLoRALinear, lora_parameters
from representax_amd.trainstep import (BertConfig, MNRTrainStep, Qwen3TextConfig,
                                       build_int4lora_encoder, build_int4lora_qwen3, mnr_loss)

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TINY = BertConfig(vocab_size=512, hidden_size=128, num_hidden_layers=2, num_attention_heads=4,
                  intermediate_size=256, max_position_embeddings=64)


def _frozen_state(model):
    state = {n: t.detach().clone() for n, t in model.named_buffers() if t is not None}
    state.update({n: p.detach().clone() for n, p in model.named_parameters() if not p.requires_grad})
    return state


def test_train_step_moves_only_lora_masters():
    model = build_int4lora_encoder(TINY, rank=4, alpha=8.0, group_size=64, seed=3, device=DEV)
    frozen = _frozen_state(model)
    lora = {id(p) for p in lora_parameters(model)}
    assert len(lora) == 2 * 6 * TINY.num_hidden_layers
    assert all(p.requires_grad == (id(p) in lora) for p in model.parameters())
    before = [p.detach().clone() for p in lora_parameters(model)]
    step = MNRTrainStep(model, batch=8, sequence=32, lr=1e-2)
    losses = [float(step()) for _ in range(3)]
    torch.cuda.synchronize()
    assert all(math.isfinite(v) for v in losses)
    after = lora_parameters(model)
    assert all(not torch.equal(b, a.detach()) for b, a in zip(before, after))
    for name, value in _frozen_state(model).items():
        assert torch.equal(value, frozen[name]), name
    # optimizer state exists only for the adapter masters: one flat buffer
    # whose views are exactly the LoRA parameters
    assert list(step.optimizer.state) == [step.flat]
    assert step.flat.numel() == sum(p.numel() for p in after)
    def inside(t, buf):
        return buf.data_ptr() <= t.data_ptr() < buf.data_ptr() + buf.numel() * 4

    assert all(inside(p, step.flat) and inside(p.grad, step.flat.grad) for p in after)
    assert all(p.dtype == torch.float32 for p in after)


def test_graph_replay_matches_eager_steps():
    # capture() runs two eager warm-up steps, then each replay is one step
    def run(capture):
        model = build_int4lora_encoder(TINY, rank=4, alpha=8.0, group_size=None, seed=5,
                                       device=DEV)
        step = MNRTrainStep(model, batch=8, sequence=32, lr=1e-2)
        if capture:
            step.capture(warmup=2)
            out = [float(step()) for _ in range(3)]
        else:
            out = [float(step()) for _ in range(5)][2:]
        torch.cuda.synchronize()
        return out, [p.detach().clone() for p in lora_parameters(model)]

    eager_losses, eager_params = run(False)
    graph_losses, graph_params = run(True)
    assert graph_losses == eager_losses
    assert all(torch.equal(a, b) for a, b in zip(eager_params, graph_params))


def _fp32_adapter_forward(self, value):
    """float32 restatement of the adapter: x W_b^T + (x A^T) B^T * alpha/r + b."""

    w = self.base_weight().float()
    x = value.float()
    y = x @ w.t() + (x @ self.lora_a.t()) @ self.lora_b.t() * (self.alpha / self.rank)
    if self.bias_bits is not None:
        y = y + self.bias_bits.view(torch.bfloat16).float()
    return y


def test_bf16_step_matches_float32_restatement(monkeypatch):
    model = build_int4lora_encoder(TINY, rank=8, alpha=16.0, group_size=64, seed=7, device=DEV)
    g = torch.Generator(device="cpu").manual_seed(11)
    with torch.no_grad():
        for mod in model.modules():
            if isinstance(mod, QuantizedLoRALinear):
                mod.lora_b.copy_(0.05 * torch.randn(mod.lora_b.shape, generator=g))
    ids = torch.randint(0, TINY.vocab_size, (16, 32), generator=g).to(DEV)
    params = lora_parameters(model)

    step = MNRTrainStep(model, batch=8, sequence=32)
    with torch.no_grad():
        step.query_ids.copy_(ids[:8])
        step.document_ids.copy_(ids[8:])
    with torch.autograd.set_grad_enabled(True):
        from representax_amd.precision import precision_context

        with precision_context(step.policy):
            emb = model.encode(ids)
            loss = mnr_loss(emb[:8], emb[8:])
        grads = torch.autograd.grad(loss, params)

    monkeypatch.setattr(QuantizedLoRALinear, "forward", _fp32_adapter_forward)
    emb32 = model.encode(ids, compute_dtype=torch.float32)
    loss32 = mnr_loss(emb32[:8], emb32[8:])
    grads32 = torch.autograd.grad(loss32, params)
    torch.cuda.synchronize()

    assert abs(float(loss.detach()) - float(loss32.detach())) < 2e-2 * max(1.0, abs(float(loss32.detach())))
    num = sum(float((a.float() - b).square().sum()) for a, b in zip(grads, grads32))
    den = sum(float(b.square().sum()) for b in grads32)
    # bf16 activations through two layers versus float32 throughout
    assert math.sqrt(num / den) < 5e-2


QWEN_TINY = Qwen3TextConfig(vocab_size=640, hidden_size=256, num_hidden_layers=2,
                            num_attention_heads=4, num_key_value_heads=2, head_dimension=64,
                            intermediate_size=512)


def test_qwen3_tower_step_moves_only_lora_masters():
    model = build_int4lora_qwen3(QWEN_TINY, rank=8, alpha=16.0, group_size=64, seed=2, device=DEV)
    frozen = _frozen_state(model)
    lora = lora_parameters(model)
    assert len(lora) == 2 * 7 * QWEN_TINY.num_hidden_layers
    before = [p.detach().clone() for p in lora]
    step = MNRTrainStep(model, batch=4, sequence=64, lr=1e-2)
    losses = [float(step()) for _ in range(3)]
    torch.cuda.synchronize()
    assert all(math.isfinite(v) for v in losses)
    assert all(not torch.equal(b, a.detach()) for b, a in zip(before, lora))
    for name, value in _frozen_state(model).items():
        assert torch.equal(value, frozen[name]), name


def test_qwen3_bf16_forward_backward_matches_float32(monkeypatch):
    model = build_int4lora_qwen3(QWEN_TINY, rank=8, alpha=16.0, group_size=64, seed=4, device=DEV)
    g = torch.Generator(device="cpu").manual_seed(12)
    with torch.no_grad():
        for mod in model.modules():
            if isinstance(mod, QuantizedLoRALinear):
                mod.lora_b.copy_(0.05 * torch.randn(mod.lora_b.shape, generator=g))
    ids = torch.randint(0, QWEN_TINY.vocab_size, (8, 64), generator=g).to(DEV)
    params = lora_parameters(model)
    from representax_amd.config import PrecisionConfig
    from representax_amd.precision import precision_context, resolve_precision_policy

    with precision_context(resolve_precision_policy(PrecisionConfig.bfloat16_mixed())):
        emb = model.encode(ids)
        loss = mnr_loss(emb[:4], emb[4:])
    grads = torch.autograd.grad(loss, params)
    monkeypatch.setattr(QuantizedLoRALinear, "forward", _fp32_adapter_forward)
    emb32 = model.encode(ids, compute_dtype=torch.float32)
    loss32 = mnr_loss(emb32[:4], emb32[4:])
    grads32 = torch.autograd.grad(loss32, params)
    torch.cuda.synchronize()
    assert abs(float(loss.detach()) - float(loss32.detach())) < 2e-2 * max(1.0, abs(float(loss32.detach())))
    num = sum(float((a.float() - b).square().sum()) for a, b in zip(grads, grads32))
    den = sum(float(b.square().sum()) for b in grads32)
    assert math.sqrt(num / den) < 5e-2


@pytest.mark.parametrize("which", ["bert", "qwen3"])
def test_rematerialized_layers_give_identical_gradients(which):
    """Per-layer rematerialization (the reference's default, full) re-runs
    each layer's forward, INT4 + LoRA kernels included, before its
    backward: loss and every LoRA gradient equal the saved-activation run
    bit for bit."""

    from representax_amd.precision import precision_context, resolve_precision_policy
    from representax_amd.config import PrecisionConfig

    if which == "bert":
        model = build_int4lora_encoder(TINY, rank=8, alpha=16.0, group_size=64, seed=9, device=DEV)
        shape = (8, 32)
    else:
        model = build_int4lora_qwen3(QWEN_TINY, rank=8, alpha=16.0, group_size=64, seed=9,
                                     device=DEV)
        shape = (8, 64)
    g = torch.Generator(device="cpu").manual_seed(21)
    with torch.no_grad():
        for mod in model.modules():
            if isinstance(mod, QuantizedLoRALinear):
                mod.lora_b.copy_(0.05 * torch.randn(mod.lora_b.shape, generator=g))
    ids = torch.randint(0, model.config.vocab_size, shape, generator=g).to(DEV)
    params = lora_parameters(model)
    policy = resolve_precision_policy(PrecisionConfig.bfloat16_mixed())
    out = {}
    for remat in ("none", "full"):
        model.remat = remat
        with precision_context(policy):
            emb = model.encode(ids)
            loss = mnr_loss(emb[:4], emb[4:])
        out[remat] = (loss.detach(), torch.autograd.grad(loss, params))
    torch.cuda.synchronize()
    assert torch.equal(out["none"][0], out["full"][0])
    assert all(torch.equal(a, b) for a, b in zip(out["none"][1], out["full"][1]))


def test_step_clips_the_global_gradient_norm():
    """The gradients the update sees are scaled by min(1, max / (norm + 1e-6))
    with norm the float32 global norm of the unclipped gradients."""

    model = build_int4lora_encoder(TINY, rank=4, alpha=8.0, group_size=64, seed=13, device=DEV)
    with torch.no_grad():
        for mod in model.modules():
            if isinstance(mod, QuantizedLoRALinear):
                mod.lora_b.normal_(0.0, 0.5)
    step = MNRTrainStep(model, batch=8, sequence=32, max_grad_norm=1e-3)
    step()
    torch.cuda.synchronize()
    norm = float(step.grad_norm)
    clipped = float(torch.linalg.vector_norm(step.flat.grad))
    assert norm > 1e-3 and bool(step.finite)
    assert abs(clipped - 1e-3 * norm / (norm + 1e-6)) < 1e-6 * norm
    free = MNRTrainStep(build_int4lora_encoder(TINY, rank=4, alpha=8.0, group_size=64, seed=13,
                                               device=DEV), batch=8, sequence=32,
                        max_grad_norm=None)
    free()
    torch.cuda.synchronize()
    assert abs(float(torch.linalg.vector_norm(free.flat.grad)) - float(free.grad_norm)) < 1e-6


@pytest.mark.parametrize("captured", [False, True])
def test_non_finite_step_leaves_state_unchanged(captured):
    """A step whose loss is not finite (an inf planted in a frozen embedding
    row the batch uses) changes no parameter and no optimizer state, as the
    reference's optax.tree.where(finite, proposed, state) does; the next
    finite step updates as usual."""

    model = build_int4lora_encoder(TINY, rank=4, alpha=8.0, group_size=64, seed=17, device=DEV)
    step = MNRTrainStep(model, batch=4, sequence=16, lr=1e-2)
    if captured:
        step.capture(warmup=1)
    else:
        step()
    torch.cuda.synchronize()
    token = int(step.query_ids[0, 0])
    saved_row = model.word[token].detach().clone()
    before = [t.clone() for t in step._state_tensors()]
    with torch.no_grad():
        model.word[token] = float("inf")
    step()
    torch.cuda.synchronize()
    assert not bool(step.finite) and not math.isfinite(float(step.loss))
    for a, b in zip(before, step._state_tensors()):
        assert torch.equal(a, b)
    with torch.no_grad():
        model.word[token] = saved_row
    step()
    torch.cuda.synchronize()
    assert bool(step.finite)
    assert not torch.equal(before[0], step._state_tensors()[0])
    assert float(step._state_tensors()[3]) == float(before[3]) + 1
