"""Several INT4 + LoRA projections of one input in one call
(rpx_int4lora_forward_multi) against the oracle and against one call per
projection (GPU): the fused small-M form for the q / k / v and gate / up
shapes of the Qwen3-2B tower, the sequential form at larger M and for
mixed ranks, graph replay, and the inference path of
``mlp.shared_input_projections``."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import int4 as oint4
from oracle import lora as olora
from oracle.codecs import f32_to_bf16_bits
from representax_amd import mlp, ops
from tests.helpers import assert_bf16_close, bf16_values, from_dev, rng, to_dev, to_dev_bf16

pytestmark = pytest.mark.gpu


def _proj(g, n, k, r, group, bias):
    w = (g.standard_normal((n, k)) * 0.02).astype(np.float32)
    packed, scales = oint4.pack_int4(w, group)
    a = (g.standard_normal((r, k)) * 0.05).astype(np.float32)
    b = (g.standard_normal((n, r)) * 0.5).astype(np.float32)
    bias_bits = f32_to_bf16_bits((g.standard_normal(n) * 0.5).astype(np.float32)) if bias else None
    host = dict(packed=packed, scales=scales, a=a, b=b, bias=bias_bits, alpha=2.0 * r, r=r, group=group)
    dev = (to_dev(packed), to_dev(scales.view(np.int16)).view(torch.uint16), to_dev_bf16(a),
           to_dev_bf16(b), 2.0, group,
           None if bias_bits is None else to_dev(bias_bits.view(np.int16)).view(torch.uint16))
    return host, dev


SHAPES = [
    pytest.param(2048, [(2048, 32), (1024, 32), (1024, 32)], id="qwen3-qkv"),
    pytest.param(2048, [(6144, 32), (6144, 32)], id="qwen3-gate-up"),
    pytest.param(768, [(768, 16), (768, 16), (768, 16)], id="bert-qkv"),
    pytest.param(512, [(384, 32), (256, 16)], id="mixed-ranks"),
]


@pytest.mark.parametrize("m", [1, 4, 16, 300])
@pytest.mark.parametrize("k,outs", SHAPES)
def test_multi_matches_oracle_and_single_calls(m, k, outs):
    g = rng(600 + m + k + len(outs))
    projs = [_proj(g, n, k, r, 64, bias=(i % 2 == 0)) for i, (n, r) in enumerate(outs)]
    x = bf16_values(g.standard_normal((m, k)))
    xd = to_dev_bf16(x)
    got = ops.int4lora_forward_multi(xd, [d for _, d in projs])
    single = [ops.int4lora_forward(xd, d[0], d[1], d[2], d[3], scaling=d[4], group_size=d[5],
                                   bias_bits=d[6]) for _, d in projs]
    torch.cuda.synchronize()
    for (host, _), (y, h), (ys, hs) in zip(projs, got, single):
        y_o, h_o = olora.lora_forward(x, host["packed"], host["scales"], host["a"], host["b"],
                                      alpha=host["alpha"], rank=host["r"], bias_bits=host["bias"],
                                      group_size=host["group"])
        assert_bf16_close(from_dev(y), y_o, what="y")
        assert_bf16_close(from_dev(h), h_o, what="h")
        if m > 4 or len({r for _, r in outs}) > 1:
            # the sequential form is one call per projection: the same bits
            assert torch.equal(y, ys) and torch.equal(h, hs)


def test_multi_replays_in_a_graph():
    g = rng(650)
    projs = [_proj(g, n, 2048, 32, 64, bias=True) for n in (2048, 1024, 1024)]
    xd = to_dev_bf16(bf16_values(g.standard_normal((1, 2048))))
    eager = ops.int4lora_forward_multi(xd, [d for _, d in projs])
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        ops.int4lora_forward_multi(xd, [d for _, d in projs])
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = ops.int4lora_forward_multi(xd, [d for _, d in projs])
    for _ in range(3):
        for y, h in outs:
            y.zero_()
            h.zero_()
        ops.int4lora_forward_multi(xd, [d for _, d in projs])  # eager work between the replays
        graph.replay()
        torch.cuda.synchronize()
        for (y, h), (ye, he) in zip(outs, eager):
            assert torch.equal(y, ye) and torch.equal(h, he)


def test_multi_one_launch_replays_follow_new_inputs():
    """The one-launch shared-input form replayed in a graph with new x each
    time: every replay's h equals the two-launch form's on the same x, bit
    for bit, and y matches the oracle, so no replay takes partials that its
    previous replay left in the slot."""

    g = rng(660)
    projs = [_proj(g, n, 2048, 32, 64, bias=False) for n in (6144, 6144)]
    xd = to_dev_bf16(bf16_values(g.standard_normal((1, 2048))))
    with ops.tuning(skinny2_one=1):
        ops.int4lora_forward_multi(xd, [d for _, d in projs])
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            ops.int4lora_forward_multi(xd, [d for _, d in projs])
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            outs = ops.int4lora_forward_multi(xd, [d for _, d in projs])
    for i in range(4):
        x = bf16_values(rng(670 + i).standard_normal((1, 2048)))
        xd.copy_(to_dev_bf16(x))
        graph.replay()
        torch.cuda.synchronize()
        with ops.tuning(skinny2_one=0):
            two = ops.int4lora_forward_multi(xd, [d for _, d in projs])
        torch.cuda.synchronize()
        for (host, _), (y, h), (_, h2) in zip(projs, outs, two):
            assert torch.equal(h.view(torch.uint16), h2.view(torch.uint16)), i
            y_o, _ = olora.lora_forward(x, host["packed"], host["scales"], host["a"], host["b"],
                                        alpha=host["alpha"], rank=host["r"], group_size=host["group"])
            assert_bf16_close(from_dev(y), y_o, what="y")
    assert ops.check_device_errors() == 0


def test_shared_input_projections_inference_path():
    from representax_amd import apply_quantized_lora, precision_context
    from representax_amd.config import PrecisionConfig
    from representax_amd.precision import resolve_precision_policy

    from representax_amd import Linear

    arg = dict(scale=0.02, bias=True, device="cuda")
    layers = torch.nn.ModuleDict({
        "query": Linear.init(2048, 2048, key=1, **arg),
        "key": Linear.init(2048, 1024, key=2, **arg),
        "value": Linear.init(2048, 1024, key=3, **arg),
    })
    with torch.no_grad():
        for layer in layers.values():
            layer.bias.normal_(0.0, 0.5)
    model = apply_quantized_lora(layers, rank=32, alpha=64.0, key=0, target_pattern=r".*",
                                 group_size=64)
    with torch.no_grad():
        for layer in model.values():
            layer.lora_b.normal_(0.0, 0.05)
    policy = resolve_precision_policy(PrecisionConfig.bfloat16_mixed())
    x = torch.randn(1, 3, 2048, device="cuda", dtype=torch.bfloat16)
    with precision_context(policy), torch.no_grad():
        fused = mlp.shared_input_projections(x, (model["query"], model["key"], model["value"]))
        separate = [model[name](x) for name in ("query", "key", "value")]
    torch.cuda.synchronize()
    for a, b in zip(fused, separate):
        assert a.shape == b.shape and a.dtype == b.dtype
        assert_bf16_close(from_dev(a), from_dev(b), what="shared-input inference")


@pytest.mark.parametrize("m", [1, 4, 300])
def test_fast_binding_equals_ctypes_binding(m, monkeypatch):
    """The CPython fast-call binding and the ctypes binding reach the same
    entry points: single and multi-projection forwards give identical bits
    either way."""

    from representax_amd import _native as nat

    assert nat.fast() is not None
    g = rng(700 + m)
    k = 2048
    projs = [_proj(g, n, k, 32, 64, bias=(i == 0)) for i, n in enumerate((2048, 1024, 1024))]
    xd = to_dev_bf16(bf16_values(g.standard_normal((m, k))))
    d = projs[0][1]
    y_f, h_f = ops.int4lora_forward(xd, d[0], d[1], d[2], d[3], scaling=d[4], group_size=d[5],
                                    bias_bits=d[6])
    multi_f = ops.int4lora_forward_multi(xd, [p for _, p in projs])
    monkeypatch.setattr(nat, "fast", lambda: None)
    y_c, h_c = ops.int4lora_forward(xd, d[0], d[1], d[2], d[3], scaling=d[4], group_size=d[5],
                                    bias_bits=d[6])
    multi_c = ops.int4lora_forward_multi(xd, [p for _, p in projs])
    torch.cuda.synchronize()
    assert torch.equal(y_f, y_c) and torch.equal(h_f, h_c)
    for (a, b), (c, e) in zip(multi_f, multi_c):
        assert torch.equal(a, c) and torch.equal(b, e)


@pytest.mark.parametrize("fast", [True, False], ids=["fast-binding", "ctypes"])
@pytest.mark.parametrize("m", [1, 4, 64, 300])
def test_forward_without_h_gives_the_same_outputs(m, fast, monkeypatch):
    """need_h=False (inference) keeps h in the call's scratch: y is bitwise
    the y of the call that returns h, for the single and the multi-projection
    forwards on either binding. The outputs of one multi call (one
    allocation at M <= 64) are dense, 16-byte aligned and disjoint."""

    from representax_amd import _native as nat

    if not fast:
        monkeypatch.setattr(nat, "fast", lambda: None)
    g = rng(800 + m)
    k = 2048
    projs = [_proj(g, n, k, 32, 64, bias=(i == 0)) for i, n in enumerate((2048, 1024, 1024))]
    xd = to_dev_bf16(bf16_values(g.standard_normal((m, k))))
    d = projs[0][1]
    y_h, h = ops.int4lora_forward(xd, d[0], d[1], d[2], d[3], scaling=d[4], group_size=d[5],
                                  bias_bits=d[6])
    y_n, no_h = ops.int4lora_forward(xd, d[0], d[1], d[2], d[3], scaling=d[4], group_size=d[5],
                                     bias_bits=d[6], need_h=False)
    multi_h = ops.int4lora_forward_multi(xd, [p for _, p in projs])
    multi_n = ops.int4lora_forward_multi(xd, [p for _, p in projs], need_h=False)
    torch.cuda.synchronize()
    assert no_h is None and h is not None
    assert torch.equal(y_h, y_n)
    for (ya, ha), (yb, hb) in zip(multi_h, multi_n):
        assert hb is None and torch.equal(ya, yb)
    for outs in (multi_h, multi_n):
        spans = []
        for pair in outs:
            for t in pair:
                if t is None:
                    continue
                assert t.is_contiguous() and t.data_ptr() % 16 == 0
                spans.append((t.data_ptr(), t.data_ptr() + t.numel() * t.element_size()))
        spans.sort()
        assert all(end <= start for (_, end), (start, _) in zip(spans, spans[1:]))


@pytest.mark.parametrize("m", [1, 4, 300])
def test_operands_in_other_forms_give_the_same_bits(m):
    """Operands the kernels cannot take as they are (float32 adapters holding
    bf16 values, scale bits typed bf16, bias bits typed int16, a strided or misaligned x)
    go through the general path, which converts them: the same bits as the
    call whose operands are already in the kernels' form."""

    g = rng(900 + m)
    k = 2048
    projs = [_proj(g, n, k, 32, 64, bias=(i == 0)) for i, n in enumerate((2048, 1024, 1024))]
    x = bf16_values(g.standard_normal((m, k)))
    xd = to_dev_bf16(x)
    wide = torch.zeros((m, k + 64), dtype=torch.bfloat16, device="cuda")
    wide[:, 1:1 + k] = xd
    x_strided = wide[:, 1:1 + k]  # strided for M > 1, 2 bytes off alignment at M = 1
    assert not x_strided.is_contiguous() or x_strided.data_ptr() % 16


    def other(d):
        return (d[0], d[1].view(torch.bfloat16), d[2].float(), d[3].float(), d[4], d[5],
                None if d[6] is None else d[6].view(torch.int16))

    for need_h in (True, False):
        d = projs[0][1]
        y_r, h_r = ops.int4lora_forward(xd, d[0], d[1], d[2], d[3], scaling=d[4], group_size=d[5],
                                        bias_bits=d[6], need_h=need_h)
        o = other(d)
        y_o, h_o = ops.int4lora_forward(x_strided, o[0], o[1], o[2], o[3], scaling=o[4],
                                        group_size=o[5], bias_bits=o[6], need_h=need_h)
        multi_r = ops.int4lora_forward_multi(xd, [p for _, p in projs], need_h=need_h)
        multi_o = ops.int4lora_forward_multi(x_strided, [other(p) for _, p in projs],
                                             need_h=need_h)
        torch.cuda.synchronize()
        assert torch.equal(y_r, y_o)
        assert (h_r is None) == (not need_h) and (h_o is None) == (not need_h)
        if need_h:
            assert torch.equal(h_r, h_o)
        for (ya, ha), (yb, hb) in zip(multi_r, multi_o):
            assert torch.equal(ya, yb)
            if need_h:
                assert torch.equal(ha, hb)


@pytest.mark.parametrize("m", [2000, 16384, 32768])
@pytest.mark.parametrize("k,outs", [(768, [(768, 16), (768, 16), (768, 16)]),
                                    (2048, [(6144, 32), (6144, 32)]),
                                    (1024, [(512, 48), (256, 16)]),
                                    (2048, [(2048, 32), (1024, 32), (1024, 32)]),
                                    (512, [(256, 32), (256, 32), (128, 48), (128, 16)]),
                                    (256, [(64, 16)] * 8),
                                    (256, [(64, 16)] * 9)],
                         ids=["bert-qkv", "qwen3-gate-up", "ranks-48-16", "qwen3-qkv",
                              "eight-blocks", "eight-projections", "nine-projections"])
def test_shared_down_projection_equals_single_calls(m, k, outs):
    """Above the small-M sizes the projections' h come from one launch over x
    (row groups of 16, 32 and 64 rows at these M); y and h must equal one
    call per projection bit for bit."""

    g = rng(900 + m + k)
    projs = [_proj(g, n, k, r, 64, bias=(i == 0))[1] for i, (n, r) in enumerate(outs)]
    xd = to_dev_bf16(bf16_values(g.standard_normal((m, k))))
    got = ops.int4lora_forward_multi(xd, projs)
    single = [ops.int4lora_forward(xd, d[0], d[1], d[2], d[3], scaling=d[4], group_size=d[5],
                                   bias_bits=d[6]) for d in projs]
    torch.cuda.synchronize()
    for (y, h), (ys, hs) in zip(got, single):
        assert torch.equal(h, hs)
        assert torch.equal(y, ys)
