"""HIP-graph capture of the hot path: every replay must equal the eager result."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from representax_amd import ops
from tests.helpers import bf16_values, rng, to_dev, to_dev_bf16

pytestmark = pytest.mark.gpu


def _capture(fn):
    fn()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = fn()
    torch.cuda.synchronize()
    return graph, outs


def _check_replays(fn, eager_outs, replays=4):
    graph, outs = _capture(fn)
    for i in range(replays):
        for o in outs:
            o.fill_(float("nan")) if o.is_floating_point() else o.zero_()
        # unrelated eager work between replays
        junk = torch.randn(1024, 1024, device="cuda") @ torch.randn(1024, 1024, device="cuda")
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs, eager_outs):
            assert torch.equal(o, e), f"replay {i} differs from eager"
        del junk


def test_fp8_linear_graph_replays_match_eager():
    g = rng(31)
    x = to_dev_bf16(g.standard_normal((1024, 768)))
    w = to_dev_bf16(g.standard_normal((3072, 768)) * 0.02)
    gy = to_dev_bf16(g.standard_normal((1024, 3072)))

    def fn():
        y, s, codes = ops.fp8_linear_forward(x, w.t(), save_codes=True)
        dl, dr = ops.fp8_linear_backward_codes(codes, s, gy, k=768, dtype=torch.bfloat16,
                                               right_transposed=True)
        return [y, s, dl, dr]

    eager = [t.clone() for t in fn()]
    torch.cuda.synchronize()
    _check_replays(fn, eager)


@pytest.mark.parametrize("group", [None, 64])
def test_int4lora_graph_replays_match_eager(group):
    g = rng(32)
    m, k, n, r = 512, 768, 3072, 16
    x = to_dev_bf16(g.standard_normal((m, k)))
    w = to_dev((g.standard_normal((n, k)) * 0.02).astype(np.float32))
    packed, scales = ops.int4_pack(w, group)
    a = to_dev_bf16(g.standard_normal((r, k)) * 0.02)
    b = to_dev_bf16(g.standard_normal((n, r)) * 0.02)
    gy = to_dev_bf16(bf16_values(g.standard_normal((m, n))))

    def fn():
        y, h = ops.int4lora_forward(x, packed, scales, a, b, scaling=2.0, group_size=group)
        dx, da, db = ops.int4lora_backward(gy, x, packed, scales, a, b, h, scaling=2.0,
                                           group_size=group)
        return [y, h, dx, da, db]

    eager = [t.clone() for t in fn()]
    torch.cuda.synchronize()
    _check_replays(fn, eager)
