"""Module-level behaviour on the GPU, mirroring the reference's adapter and
precision tests (tests/models/test_adapters.py, tests/train/test_precision.py)."""

from __future__ import annotations

import io

import numpy as np
import pytest
import torch

import representax_amd as rx
from oracle import lora as olora
from tests.helpers import BF16_REL_TOL, from_dev, rel_l2

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


class _AdapterEncoder(torch.nn.Module):
    """8 -> 6 projection with bias (tests/models/test_adapters.py:28-57)."""

    def __init__(self, key):
        super().__init__()
        self.projection = rx.Linear.init(8, 6, key=key, scale=8 ** -0.5, bias=True, device=DEV)
        with torch.no_grad():
            self.projection.bias.copy_(torch.linspace(-0.5, 0.5, 6))

    def forward(self, x):
        return self.projection(x)


def _adapter(model):
    return rx.apply_quantized_lora(model, rank=2, alpha=4.0, key=2)


def test_packs_base_and_zero_initializes_adapter_output():
    original = _AdapterEncoder(key=1)
    adapted = _adapter(original)
    proj = adapted.projection
    assert isinstance(proj, rx.QuantizedLoRALinear)
    assert proj.packed_weight.dtype == torch.uint8 and proj.packed_weight.numel() == 6 * 4
    assert proj.scale_bits.dtype == torch.uint16
    assert torch.count_nonzero(proj.lora_b) == 0
    values = torch.randn(4, 8, generator=torch.Generator().manual_seed(3)).to(DEV)
    merged = rx.merge_quantized_lora(adapted)
    assert isinstance(merged.projection, rx.Linear)
    torch.testing.assert_close(adapted(values), merged(values), rtol=2e-3, atol=2e-3)
    # the original model is untouched (functional update)
    assert isinstance(original.projection, rx.Linear)


def test_merged_export_matches_oracle_with_nonzero_adapter():
    adapted = _adapter(_AdapterEncoder(key=4))
    with torch.no_grad():
        adapted.projection.lora_b.normal_(0, 0.2)
    p = adapted.projection
    want = olora.merged_weight(p.packed_weight.cpu().numpy(),
                               p.scale_bits.view(torch.int16).cpu().numpy().view(np.uint16),
                               p.lora_a.detach().cpu().numpy(), p.lora_b.detach().cpu().numpy(),
                               alpha=4.0, rank=2, input_size=8)
    np.testing.assert_allclose(p.merged_weight().cpu().numpy(), want, rtol=1e-6, atol=1e-7)


def _cosine_loss(model, left, right, labels):
    a = model(left)
    b = model(right)
    cos = torch.nn.functional.cosine_similarity(a.float(), b.float(), dim=-1)
    return ((cos - labels) ** 2).mean()


def test_adapter_step_changes_only_lora_parameters():
    """One AdamW step: frozen leaves bit-identical, lora_b moves, finite
    (tests/models/test_adapters.py:120-153)."""

    model = _adapter(_AdapterEncoder(key=5))
    opt = torch.optim.AdamW(rx.lora_parameters(model), lr=1e-2, weight_decay=0.0)
    frozen_before = {n: b.clone() for n, b in model.named_buffers()}
    lora_b_before = model.projection.lora_b.detach().clone()
    values = torch.randn(4, 8, generator=torch.Generator().manual_seed(6)).to(DEV)
    right = values.clone()
    right[:, 0] += 0.1
    labels = torch.tensor([0.7, 0.8, 0.9, 0.6], device=DEV)
    bf = rx.resolve_precision_policy(rx.PrecisionConfig.bfloat16_mixed())
    with rx.precision_context(bf):
        loss = _cosine_loss(model, values, right, labels)
    loss.backward()
    opt.step()
    for n, b in model.named_buffers():
        assert torch.equal(b, frozen_before[n]), n
    assert not torch.equal(model.projection.lora_b.detach(), lora_b_before)
    assert torch.isfinite(loss)
    assert all(p.dtype == torch.float32 for p in model.parameters())


def test_adapter_state_round_trips_exactly():
    model = _adapter(_AdapterEncoder(key=7))
    template = _adapter(_AdapterEncoder(key=8))
    buf = io.BytesIO()
    torch.save(model.state_dict(), buf)
    buf.seek(0)
    template.load_state_dict(torch.load(buf, weights_only=True))
    for (n1, t1), (n2, t2) in zip(model.state_dict().items(), template.state_dict().items()):
        assert n1 == n2 and torch.equal(t1, t2)


def test_bf16_module_gradients_match_oracle():
    """QuantizedLoRALinear under the bf16 policy: autograd through the fused
    kernels gives the oracle's x / lora_a / lora_b gradients."""

    g = np.random.Generator(np.random.PCG64(12))
    lin = rx.Linear.init(256, 192, key=1, scale=0.02, bias=True, device=DEV)
    layer = rx.QuantizedLoRALinear.from_linear(lin, rank=16, alpha=32.0, key=3)
    with torch.no_grad():
        layer.lora_b.normal_(0, 0.02)
    x = torch.from_numpy(g.standard_normal((128, 256)).astype(np.float32)).to(DEV)
    x = x.to(torch.bfloat16).requires_grad_(True)
    gy = torch.from_numpy(g.standard_normal((128, 192)).astype(np.float32)).to(DEV)
    gy = gy.to(torch.bfloat16)
    bf = rx.resolve_precision_policy(rx.PrecisionConfig.bfloat16_mixed())
    with rx.precision_context(bf):
        y = layer(x)
    y.backward(gy)
    packed = layer.packed_weight.cpu().numpy()
    scales = layer.scale_bits.view(torch.int16).cpu().numpy().view(np.uint16)
    bias = layer.bias_bits.view(torch.int16).cpu().numpy().view(np.uint16)
    xa = from_dev(x.detach())
    a = layer.lora_a.detach().cpu().numpy()
    b = layer.lora_b.detach().cpu().numpy()
    y_o, h_o = olora.lora_forward(xa, packed, scales, a, b, alpha=32.0, rank=16, bias_bits=bias)
    dx_o, da_o, db_o = olora.lora_backward(from_dev(gy), xa, packed, scales, a, b, h_o,
                                           alpha=32.0, rank=16)
    assert rel_l2(from_dev(y.detach()), y_o) < BF16_REL_TOL
    assert rel_l2(from_dev(x.grad), dx_o) < BF16_REL_TOL
    assert rel_l2(layer.lora_a.grad.cpu().numpy(), da_o) < BF16_REL_TOL
    assert rel_l2(layer.lora_b.grad.cpu().numpy(), db_o) < BF16_REL_TOL
    assert layer.lora_a.grad.dtype == torch.float32


@pytest.mark.parametrize("m", [1, 4, 128])
def test_bf16_module_inference_equals_training_forward(m):
    """Without autograd the module calls the fused forward directly and keeps
    h in the call's scratch; its output is bitwise the output of the
    autograd path (small M runs the skinny kernels, M = 128 the GEMM)."""

    g = np.random.Generator(np.random.PCG64(13 + m))
    lin = rx.Linear.init(2048, 1024, key=4, scale=0.02, bias=True, device=DEV)
    layer = rx.QuantizedLoRALinear.from_linear(lin, rank=32, alpha=64.0, key=5, group_size=64)
    with torch.no_grad():
        layer.lora_b.normal_(0, 0.05)
    x = torch.from_numpy(g.standard_normal((m, 2048)).astype(np.float32)).to(DEV).to(torch.bfloat16)
    bf = rx.resolve_precision_policy(rx.PrecisionConfig.bfloat16_mixed())
    with rx.precision_context(bf):
        y_train = layer(x.clone().requires_grad_(True))
        with torch.no_grad():
            y_infer = layer(x)
    torch.cuda.synchronize()
    assert y_train.grad_fn is not None and y_infer.grad_fn is None
    assert torch.equal(y_train.detach(), y_infer)


def test_float8_step_keeps_master_state_finite_and_fp32():
    """tests/train/test_precision.py:214-228 on a small dense model."""

    torch.manual_seed(9)
    model = torch.nn.Sequential(rx.Linear.init(64, 64, key=1, scale=0.1, device=DEV),
                                rx.Linear.init(64, 32, key=2, scale=0.1, bias=True, device=DEV))
    opt = torch.optim.AdamW(model.parameters(), lr=1e-3, weight_decay=1e-2)
    policy = rx.resolve_precision_policy(rx.PrecisionConfig.float8_mixed())
    x = torch.randn(32, 64, device=DEV)
    with rx.precision_context(policy):
        y = model(x)
    loss = (y.float() ** 2).mean()
    loss.backward()
    opt.step()
    assert torch.isfinite(loss)
    assert all(p.dtype == torch.float32 and torch.isfinite(p).all() for p in model.parameters())
    assert all(torch.isfinite(s).all() for st in opt.state.values() for s in st.values()
               if isinstance(s, torch.Tensor))


def test_stacked_adapter_layers():
    """Stacked [L, N, K] weights pack per layer and run one layer at a time."""

    lin = rx.Linear(torch.randn(3, 96, 64, device=DEV) * 0.05)
    stacked = rx.QuantizedLoRALinear.from_linear(lin, rank=4, alpha=8.0, key=1)
    assert stacked.packed_weight.shape == (3, 96, 32) and stacked.lora_a.shape == (3, 4, 64)
    x = torch.randn(16, 64, device=DEV)
    for i in range(3):
        single = rx.QuantizedLoRALinear.from_linear(rx.Linear(lin.weight[i].detach().clone()),
                                                    rank=4, alpha=8.0, key=1)
        assert torch.equal(stacked[i].packed_weight, single.packed_weight)
        assert torch.equal(stacked[i].scale_bits, single.scale_bits)
        with torch.no_grad():
            single.lora_a.copy_(stacked.lora_a[i])
        torch.testing.assert_close(stacked[i](x), single(x))
    assert stacked.merged_weight().shape == (3, 96, 64)
