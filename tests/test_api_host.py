"""Host logic of the reference-API mirror (CPU only, nothing launched)."""

from __future__ import annotations

import pydantic
import pytest
import torch

import representax_amd as rx
from representax_amd.adapters import _path_name


class _Block(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.query = rx.Linear.init(8, 8, key=1, scale=0.1)
        self.value = rx.Linear.init(8, 8, key=2, scale=0.1)
        self.norm = torch.nn.LayerNorm(8)


class _Model(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.layers = torch.nn.ModuleList([_Block(), _Block()])
        self.head = rx.Linear.init(8, 6, key=3, scale=0.1, bias=True)


def test_path_names_follow_keystr_style():
    assert _path_name("layers.0.query") == ".layers[0].query"
    assert _path_name("head") == ".head"


def test_target_pattern_selects_linear_leaves():
    model = _Model()
    assert rx.matched_linear_paths(model) == [
        "layers.0.query", "layers.0.value", "layers.1.query", "layers.1.value", "head"]
    assert rx.matched_linear_paths(model, r"layers\[1\]\.query") == ["layers.1.query"]
    assert rx.matched_linear_paths(model, r"head$") == ["head"]


def test_apply_rejects_bad_arguments_before_packing():
    model = _Model()
    with pytest.raises(ValueError, match="matched no native Linear"):
        rx.apply_quantized_lora(model, rank=2, alpha=4.0, key=0, target_pattern="nothing")
    with pytest.raises(ValueError, match="rank"):
        rx.apply_quantized_lora(model, rank=0, alpha=4.0, key=0)
    with pytest.raises(ValueError, match="alpha"):
        rx.apply_quantized_lora(model, rank=2, alpha=0.0, key=0)


def _adapter_on_cpu():
    return rx.QuantizedLoRALinear(
        packed_weight=torch.zeros((6, 4), dtype=torch.uint8),
        scale_bits=torch.full((6,), 0x3F80, dtype=torch.uint16),
        bias_bits=torch.zeros(6, dtype=torch.uint16),
        lora_a=torch.zeros((2, 8)), lora_b=torch.zeros((6, 2)),
        input_size=8, output_size=6, rank=2, alpha=4.0)


def test_lora_filter_selects_exactly_the_adapter_arrays():
    """Same selection as tests/models/test_adapters.py:97-117."""

    model = torch.nn.Module()
    model.projection = _adapter_on_cpu()
    model.other = torch.nn.Linear(3, 3)
    chosen = rx.lora_parameter_filter(model)
    assert chosen == {"projection.lora_a": True, "projection.lora_b": True,
                      "other.weight": False, "other.bias": False}
    assert {tuple(p.shape) for p in rx.lora_parameters(model)} == {(2, 8), (6, 2)}
    # frozen integer leaves are buffers, never parameters
    names = {n for n, _ in model.named_buffers()}
    assert {"projection.packed_weight", "projection.scale_bits", "projection.bias_bits"} <= names


def test_forward_on_cpu_fails_loudly():
    with pytest.raises(RuntimeError, match="ROCm"):
        _adapter_on_cpu()(torch.zeros((3, 8)))


def test_quantized_config_validation():
    cfg = rx.QuantizedLoRAConfig(rank=8, alpha=16.0, target_pattern=r"layers.*(attention|mlp)")
    assert cfg.bits == 4 and cfg.group_size is None
    for bad in (dict(rank=0, alpha=1.0), dict(rank=2, alpha=0.0), dict(rank=2, alpha=1.0, bits=8),
                dict(rank=2, alpha=1.0, target_pattern="("), dict(rank=2, alpha=1.0, target_pattern="")):
        with pytest.raises(pydantic.ValidationError):
            rx.QuantizedLoRAConfig(**bad)
    assert rx.QuantizedLoRAConfig.model_validate(cfg.model_dump()) == cfg


def test_precision_config_and_policy():
    cfg = rx.PrecisionConfig.float8_mixed()
    assert (cfg.compute_dtype, cfg.activation_dtype, cfg.resolved_matrix_dtype) == (
        "bfloat16", "bfloat16", "float8_e4m3fn")
    policy = rx.resolve_precision_policy(cfg)
    assert policy.matrix_dtype == torch.float8_e4m3fn
    assert policy.compute_dtype == torch.bfloat16 and policy.parameter_dtype == torch.float32
    bf = rx.resolve_precision_policy(rx.PrecisionConfig.bfloat16_mixed())
    assert bf.matrix_dtype == torch.bfloat16
    with pytest.raises(pydantic.ValidationError):
        rx.PrecisionConfig(compute_dtype="float16")


def test_precision_context_nests_and_restores():
    from representax_amd.precision import active_policy

    bf = rx.resolve_precision_policy(rx.PrecisionConfig.bfloat16_mixed())
    assert active_policy() is None
    with rx.precision_context(bf):
        assert active_policy() is bf
        assert rx.compute_parameter(torch.zeros(2)).dtype == torch.bfloat16
        assert rx.activation_inputs({"x": torch.zeros(2), "ids": torch.zeros(2, dtype=torch.int64)})[
            "ids"].dtype == torch.int64
        with rx.precision_context(rx.FP32_POLICY):
            assert active_policy() is rx.FP32_POLICY
        assert active_policy() is bf
    assert active_policy() is None


def test_linear_matmul_without_fp8_policy_is_a_plain_product():
    a = torch.randn(3, 4, 5)
    b = torch.randn(5, 2)
    torch.testing.assert_close(rx.linear_matmul(a, b), a @ b)
    bf = rx.resolve_precision_policy(rx.PrecisionConfig.bfloat16_mixed())
    with rx.precision_context(bf):
        torch.testing.assert_close(rx.linear_matmul(a, b), a @ b)


def test_fp8_policy_on_cpu_fails_loudly():
    policy = rx.resolve_precision_policy(rx.PrecisionConfig.float8_mixed())
    with rx.precision_context(policy):
        with pytest.raises(RuntimeError, match="ROCm"):
            rx.linear_matmul(torch.randn(4, 8, dtype=torch.bfloat16),
                             torch.randn(8, 2, dtype=torch.bfloat16))


def test_fp8_linear_matmul_rejects_empty_operands():
    """The reference's per-tensor amax is a max-reduction with no identity
    (precision.py:133-135): an empty operand raises, under dynamic and
    delayed scaling alike, before anything touches a device."""

    from representax_amd import DelayedScaling

    st = DelayedScaling(3, device="cpu")
    owner = rx.Linear(torch.zeros(4, 8))
    dynamic = rx.resolve_precision_policy(rx.PrecisionConfig.float8_mixed())
    delayed = rx.resolve_precision_policy(
        rx.PrecisionConfig.float8_mixed(fp8_scaling="delayed"), fp8_state=st)
    cases = [((0, 8), (8, 4)), ((3, 0), (0, 4)), ((3, 8), (8, 0)), ((0, 0), (0, 0))]
    for policy, kw in ((dynamic, {}), (delayed, {"fp8_owner": owner})):
        with rx.precision_context(policy):
            for ls, rs in cases:
                left = torch.zeros(ls, dtype=torch.bfloat16)
                right = torch.zeros(rs, dtype=torch.bfloat16)
                with pytest.raises(ValueError, match="empty operand"):
                    rx.linear_matmul(left, right, **kw)


def test_delayed_slots_follow_module_copies():
    """model_for_compute deep-copies the model every step: the copies keep
    their original's slots (a state sized by for_model lasts any number of
    steps), other modules and other states get their own."""

    import copy

    from representax_amd import DelayedScaling, Linear
    from representax_amd.precision import LINEAR_FORMATS

    model = torch.nn.Sequential(Linear(torch.zeros(4, 8)), Linear(torch.zeros(8, 4)))
    st = DelayedScaling.for_model(model, device="cpu")
    first = [st.slots_for(m, LINEAR_FORMATS) for m in model]
    assert first == [(0, 1, 2), (3, 4, 5)]
    policy = rx.resolve_precision_policy(rx.PrecisionConfig.bfloat16_mixed())
    for _ in range(3):
        view = rx.model_for_compute(model, policy)
        assert [st.slots_for(m, LINEAR_FORMATS) for m in view] == first
    other = DelayedScaling(3, device="cpu")
    assert other.slots_for(model[1], LINEAR_FORMATS) == (0, 1, 2)
    assert st.slots_for(model[1], LINEAR_FORMATS) == (3, 4, 5)
    with pytest.raises(ValueError, match="slots"):
        st.slots_for(Linear(torch.zeros(2, 2)), LINEAR_FORMATS)
    assert copy.deepcopy(model[0])._fp8_delayed_slots == model[0]._fp8_delayed_slots


def test_delayed_scaling_state_and_policy_on_cpu():
    """Slot bookkeeping of the delayed-scale state and the policy's checks
    (the buffers are plain tensors; no kernel runs here)."""

    import torch

    from representax_amd import DelayedScaling, Linear, PrecisionConfig
    from representax_amd.precision import LINEAR_FORMATS, resolve_precision_policy

    st = DelayedScaling(6, history_len=3, device="cpu")
    assert st.scales.tolist() == [1.0] * 6 and st.amax_history.shape == (3, 6)
    a = st.slots_for("layer0", LINEAR_FORMATS)
    b = st.slots_for("layer1", LINEAR_FORMATS)
    assert a == (0, 1, 2) and b == (3, 4, 5) and st.slots_for("layer0", LINEAR_FORMATS) == a
    assert st.fmax.tolist() == [448.0, 448.0, 57344.0] * 2
    with pytest.raises(ValueError, match="slots"):
        st.allocate(("e4m3fn",))
    with pytest.raises(ValueError):
        DelayedScaling(0, device="cpu")
    model = torch.nn.Sequential(Linear(torch.zeros(4, 8)), Linear(torch.zeros(8, 4)))
    assert DelayedScaling.for_model(model, device="cpu").n_slots == 6
    cfg = PrecisionConfig.float8_mixed(fp8_scaling="delayed", amax_history_len=8)
    assert cfg.fp8_scaling == "delayed" and cfg.amax_history_len == 8
    with pytest.raises(ValueError, match="DelayedScaling"):
        resolve_precision_policy(cfg)
    assert resolve_precision_policy(cfg, fp8_state=st).fp8_state is st
    # the dynamic (reference) policy ignores a state
    assert resolve_precision_policy(PrecisionConfig.float8_mixed(), fp8_state=st).fp8_state is None


def test_train_step_rejects_unknown_policies():
    from representax_amd.trainstep import MNRTrainStep, run_layer

    with pytest.raises(ValueError, match="rematerialization"):
        MNRTrainStep(torch.nn.Linear(2, 2), batch=1, sequence=1, remat="selective")
    with pytest.raises(ValueError, match="max_grad_norm"):
        MNRTrainStep(torch.nn.Linear(2, 2), batch=1, sequence=1, max_grad_norm=0.0)
    with torch.no_grad():
        with pytest.raises(ValueError, match="rematerialization"):
            run_layer(torch.nn.Identity(), "sometimes", torch.zeros(1))


def _lora_operands(m=4, k=64, n=32, r=4, group=None):
    packed = torch.zeros((n, (k + 1) // 2), dtype=torch.uint8)
    groups = 1 if group is None else k // group
    scales = torch.zeros((n, groups), dtype=torch.uint16)
    x = torch.zeros((m, k), dtype=torch.bfloat16)
    a = torch.zeros((r, k), dtype=torch.bfloat16)
    b = torch.zeros((n, r), dtype=torch.bfloat16)
    return x, packed, scales, a, b


@pytest.mark.parametrize("case", ["packed_width", "packed_dtype", "scales", "lora_a", "lora_b",
                                  "bias", "x_dim"])
def test_int4lora_forward_rejects_mismatched_extents(case):
    """The C ABI takes pointers and sizes only, so the wrappers check that every
    operand holds what the kernels will read; a mismatch is a ValueError raised
    before any device work (here on CPU tensors, before the device check)."""

    from representax_amd import ops

    x, packed, scales, a, b = _lora_operands(group=16)
    bias = None
    if case == "packed_width":
        packed = torch.zeros((32, 31), dtype=torch.uint8)
    elif case == "packed_dtype":
        packed = packed.to(torch.int16)
    elif case == "scales":
        scales = torch.zeros((32, 1), dtype=torch.uint16)  # group 16 needs 4 per row
    elif case == "lora_a":
        a = torch.zeros((4, 63), dtype=torch.bfloat16)
    elif case == "lora_b":
        b = torch.zeros((32, 5), dtype=torch.bfloat16)
    elif case == "bias":
        bias = torch.zeros(31, dtype=torch.uint16)
    elif case == "x_dim":
        x = x.reshape(1, 4, 64)
    with pytest.raises(ValueError):
        ops.int4lora_forward(x, packed, scales, a, b, scaling=2.0, group_size=16, bias_bits=bias)


def test_int4lora_backward_rejects_mismatched_gradients():
    from representax_amd import ops

    x, packed, scales, a, b = _lora_operands()
    h = torch.zeros((4, 4), dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        ops.int4lora_backward(torch.zeros((4, 31), dtype=torch.bfloat16), x, packed, scales, a, b,
                              h, scaling=2.0)
    with pytest.raises(ValueError):
        ops.int4lora_backward(torch.zeros((4, 32), dtype=torch.bfloat16), x, packed, scales, a, b,
                              torch.zeros((4, 3), dtype=torch.bfloat16), scaling=2.0)
    with pytest.raises(ValueError):
        ops.int4lora_backward_act(torch.zeros((4, 32), dtype=torch.bfloat16), x, packed, scales, a,
                                  b, h, activation="gelu", z=torch.zeros((4, 32)), scaling=2.0)


def test_int4lora_matching_extents_reach_the_device_check():
    """With every extent right, a CPU tensor is refused by the device check
    (no CPU fallback)."""

    from representax_amd import ops

    x, packed, scales, a, b = _lora_operands(group=16)
    with pytest.raises(RuntimeError, match="ROCm"):
        ops.int4lora_forward(x, packed, scales, a, b, scaling=2.0, group_size=16)


def test_fp8_backward_rejects_mismatched_extents():
    from representax_amd import ops

    left = torch.zeros((8, 16), dtype=torch.bfloat16)
    right = torch.zeros((16, 4), dtype=torch.bfloat16)
    scales = torch.ones(2)
    with pytest.raises(ValueError):
        ops.fp8_linear_backward(left, right, torch.zeros((8, 5), dtype=torch.bfloat16), scales)
    codes = (torch.zeros((16, 8), dtype=torch.uint8), torch.zeros((16, 4), dtype=torch.uint8))
    with pytest.raises(ValueError):
        ops.fp8_linear_backward_codes(codes, scales, torch.zeros((8, 4), dtype=torch.bfloat16),
                                      k=15, dtype=torch.bfloat16, right_transposed=False)
    with pytest.raises(ValueError):
        ops.fp8_linear_backward_codes(codes, scales, torch.zeros((9, 4), dtype=torch.bfloat16),
                                      k=16, dtype=torch.bfloat16, right_transposed=False)
