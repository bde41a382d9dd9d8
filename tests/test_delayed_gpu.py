"""Delayed-scale fp8 (an extension: the reference's roadmap item,
todo.org:1149-1154): saturating cast with amax record, the one-launch scale
update, and the delayed linear against the dynamic one (GPU)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import fp8 as ofp8
from oracle.codecs import E4M3FN, E5M2
from representax_amd import DelayedScaling, Linear, PrecisionConfig, ops
from representax_amd.precision import precision_context, resolve_precision_policy
from tests.helpers import DEVICE, bf16_values, from_dev, rng, to_dev, to_dev_bf16

pytestmark = pytest.mark.gpu


def _outliers(g, shape, special=True):
    x = g.standard_normal(shape).astype(np.float32)
    x = np.where(g.random(shape) < 1e-2, x * 50.0, x).astype(np.float32)
    if special:
        flat = x.reshape(-1)
        flat[3], flat[7], flat[11] = np.inf, -np.inf, 1e30
    return x


def _hist_f32(state):
    return state.amax_history.cpu().numpy().view(np.float32)


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("shape", [(256, 384), (100, 72), (33, 50)])
@pytest.mark.parametrize("fmt", [E4M3FN, E5M2])
def test_cast_delayed_bit_exact_and_records_amax(fmt, shape, dtype):
    """Tile path (256 x 384), ragged tiles (100 x 72) and the generic path
    (50 columns): saturating codes in both layouts and the recorded amax."""

    g = rng(21)
    x = _outliers(g, shape)
    xv = bf16_values(x) if dtype == "bf16" else x
    xd = to_dev_bf16(x) if dtype == "bf16" else to_dev(x)
    st = DelayedScaling(2, 4, device=DEVICE)
    own = float(ofp8.scale_from_amax(np.float32(50.0), fmt))
    for scale in (1.0, 0.05, 1e-3, own, 3.0e-39):
        st.scales[1] = scale
        out, out_t = ops.fp8_cast_delayed(xd, st, 1, fmt, rowmajor=True, transposed=True)
        torch.cuda.synchronize()
        want = ofp8.cast_saturating(xv, np.float32(scale), fmt)
        assert np.array_equal(out.cpu().numpy(), want), (scale, "row-major")
        assert np.array_equal(out_t.cpu().numpy(), want.T), (scale, "transposed")
    st.update()
    hist = st.amax_history.cpu().numpy()
    assert hist[0, 1] == np.float32(np.inf).view(np.uint32)  # max|x| is the inf entry
    assert hist[0, 0] == 0 and not hist[1:].any()
    assert not st.amax_pending.cpu().numpy().any()  # the update clears the pending maxima
    # a transposed view casts as its buffer, outputs exchanged
    st2 = DelayedScaling(1, 2, device=DEVICE)
    st2.scales[0] = 0.25
    o2, o2t = ops.fp8_cast_delayed(xd.t(), st2, 0, fmt, rowmajor=True, transposed=True)
    want2 = ofp8.cast_saturating(xv.T, np.float32(0.25), fmt)
    assert np.array_equal(o2.cpu().numpy(), want2) and np.array_equal(o2t.cpu().numpy(), want2.T)


def test_recorded_amax_is_the_max_over_casts_and_nan_wins():
    g = rng(22)
    st = DelayedScaling(1, 2, device=DEVICE)
    a = bf16_values(g.standard_normal((128, 128)).astype(np.float32))
    b = bf16_values(g.standard_normal((128, 128)).astype(np.float32) * 3.0)
    for t in (a, b):
        ops.fp8_cast_delayed(to_dev_bf16(t), st, 0)
    st.update()
    torch.cuda.synchronize()
    assert _hist_f32(st)[0, 0] == np.float32(max(np.abs(a).max(), np.abs(b).max()))
    c = b.copy()
    c[5, 5] = np.nan
    ops.fp8_cast_delayed(to_dev_bf16(c), st, 0)
    st.update()
    torch.cuda.synchronize()
    assert st.amax_history.cpu().numpy()[1, 0] > 0x7F800000
    assert np.isnan(st.scales.cpu().numpy()[0])


def test_pair_cast_equals_two_single_casts():
    g = rng(26)
    x = bf16_values(_outliers(g, (192, 256), special=False))
    w = bf16_values(g.standard_normal((384, 256)).astype(np.float32) * 0.02)
    st = DelayedScaling(2, 2, device=DEVICE)
    st.scales[0], st.scales[1] = 0.02, 1e-4
    (a, at), (b, bt) = ops.fp8_cast_delayed2(to_dev_bf16(x), 0, to_dev_bf16(w).t(), 1, st,
                                             rowmajor=True, transposed=True)
    torch.cuda.synchronize()
    wa = ofp8.cast_saturating(x, np.float32(0.02), E4M3FN)
    wb = ofp8.cast_saturating(w.T, np.float32(1e-4), E4M3FN)
    assert np.array_equal(a.cpu().numpy(), wa) and np.array_equal(at.cpu().numpy(), wa.T)
    assert np.array_equal(b.cpu().numpy(), wb) and np.array_equal(bt.cpu().numpy(), wb.T)
    st.update()
    assert np.array_equal(_hist_f32(st)[0], np.array([ofp8.amax(x), ofp8.amax(w)], np.float32))


def test_scale_update_matches_oracle_and_rolls_the_cursor():
    hist = np.array([[0.0, 3.0, 0.0, 448.0],
                     [0.0, 5.0, np.nan, 1.0],
                     [0.0, 1.0, 2.0, 0.0]], np.float32)
    fmts = [E4M3FN, E4M3FN, E5M2, E4M3FN]
    st = DelayedScaling(4, 3, device=DEVICE)
    st.allocate(tuple(fmts))
    old = np.array([0.5, 0.25, 0.125, 2.0], np.float32)
    st.scales.copy_(torch.from_numpy(old))
    st.amax_history.copy_(torch.from_numpy(hist.view(np.uint32).copy()))
    st.cursor.fill_(2)
    # nothing pending: the update writes a zero row 2 and recomputes from the rest
    st.update()
    torch.cuda.synchronize()
    hz = hist.copy()
    hz[2] = 0.0
    want = ofp8.delayed_update(hz, old, fmts)
    got = st.scales.cpu().numpy()
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(got[~np.isnan(want)], want[~np.isnan(want)])
    assert int(st.cursor.item()) == 0
    h2 = st.amax_history.cpu().numpy()
    assert not h2[2].any() and np.array_equal(h2[:2], hist[:2].view(np.uint32))
    # a recorded cast lands in the cursor row at the next update
    x = np.full((8, 16), 3.5, np.float32)
    ops.fp8_cast_delayed(to_dev_bf16(x), st, 1)
    st.update()
    assert int(st.cursor.item()) == 1
    assert _hist_f32(st)[0, 1] == np.float32(3.5)


def _linear_case(seed, m=256, k=384, n=512):
    g = rng(seed)
    x = bf16_values(_outliers(g, (m, k), special=False))
    w = bf16_values(g.standard_normal((n, k)).astype(np.float32) * 0.02)
    gy = bf16_values(g.standard_normal((m, n)).astype(np.float32))
    return x, w, gy


def _run(fn, x, w, gy):
    xd = to_dev_bf16(x).requires_grad_(True)
    wd = to_dev_bf16(w).requires_grad_(True)
    out = fn(xd, wd.t())
    out.backward(to_dev_bf16(gy))
    torch.cuda.synchronize()
    return out.detach(), xd.grad, wd.grad


def test_delayed_linear_equals_dynamic_under_the_tensors_own_scales():
    """With each slot holding the scale the reference computes from that very
    tensor, no quotient saturates and the delayed linear is the dynamic one,
    bit for bit (output, input and weight gradients)."""

    x, w, gy = _linear_case(23)
    dyn = _run(lambda a, b: ops.Fp8LinearFn.apply(a, b, torch.bfloat16), x, w, gy)
    st = DelayedScaling(3, 2, device=DEVICE)
    slots = st.allocate(("e4m3fn", "e4m3fn", "e5m2"))
    st.scales[0] = float(ofp8.scale_from_amax(ofp8.amax(x), E4M3FN))
    st.scales[1] = float(ofp8.scale_from_amax(ofp8.amax(w), E4M3FN))
    st.scales[2] = float(ofp8.scale_from_amax(ofp8.amax(gy), E5M2))
    dly = _run(lambda a, b: ops.Fp8DelayedLinearFn.apply(a, b, torch.bfloat16, st, slots), x, w, gy)
    for name, a, b in zip(("y", "dx", "dW"), dyn, dly):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), name
    st.update()
    rec = _hist_f32(st)[0]
    assert rec[0] == ofp8.amax(x) and rec[1] == ofp8.amax(w) and rec[2] == ofp8.amax(gy)


def test_linear_module_under_the_delayed_policy():
    """Linear under float8_mixed(fp8_scaling='delayed'): the first step runs
    with unit scales, update() sets each slot's scale from the recorded amax,
    and the next step on the same data equals the dynamic path bit for bit."""

    x, w, gy = _linear_case(24, m=128, k=256, n=192)
    lin = Linear(torch.from_numpy(w.astype(np.float32)).to(DEVICE))
    st = DelayedScaling.for_model(lin, history_len=4, device=DEVICE)
    cfg = PrecisionConfig.float8_mixed(fp8_scaling="delayed", amax_history_len=4)
    with pytest.raises(ValueError):
        resolve_precision_policy(cfg)
    policy = resolve_precision_policy(cfg, fp8_state=st)
    xd = to_dev_bf16(x)

    def step():
        lin.zero_grad()
        xin = xd.clone().requires_grad_(True)
        with precision_context(policy):
            y = lin(xin)
        y.backward(to_dev_bf16(gy))
        torch.cuda.synchronize()
        return y.detach(), xin.grad, lin.weight.grad.clone()

    first = step()
    assert all(torch.isfinite(t.float()).all() for t in first)
    st.update()
    torch.cuda.synchronize()
    s = st.scales.cpu().numpy()
    assert s[0] == ofp8.scale_from_amax(ofp8.amax(x), E4M3FN)
    assert s[1] == ofp8.scale_from_amax(ofp8.amax(w), E4M3FN)
    assert int(st.cursor.item()) == 1
    second = step()
    dyn_policy = resolve_precision_policy(PrecisionConfig.float8_mixed())
    lin.zero_grad()
    xin = xd.clone().requires_grad_(True)
    with precision_context(dyn_policy):
        y = lin(xin)
    y.backward(to_dev_bf16(gy))
    torch.cuda.synchronize()
    assert torch.equal(second[0].view(torch.int16), y.detach().view(torch.int16))
    assert torch.equal(second[1].view(torch.int16), xin.grad.view(torch.int16))
    assert torch.equal(second[2], lin.weight.grad)


def test_graph_replays_advance_the_device_cursor():
    """A captured cast + update: each replay records into the current row and
    moves the cursor; every replay's codes equal the eager codes."""

    g = rng(25)
    x = bf16_values(g.standard_normal((256, 256)).astype(np.float32))
    xd = to_dev_bf16(x)
    st = DelayedScaling(1, 3, device=DEVICE)
    st.scales[0] = 0.01
    eager, _ = ops.fp8_cast_delayed(xd, st, 0)
    st.amax_pending.zero_()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph):
            out, _ = ops.fp8_cast_delayed(xd, st, 0)
            ops.fp8_scale_update(st)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    st.amax_pending.zero_()
    st.amax_history.zero_()
    st.cursor.zero_()
    st.scales.fill_(0.01)
    torch.cuda.synchronize()
    want_scale = ofp8.scale_from_amax(ofp8.amax(x), E4M3FN)
    for i in range(4):
        graph.replay()
        torch.cuda.synchronize()
        if i == 0:
            assert torch.equal(out, eager)
        assert int(st.cursor.item()) == (i + 1) % 3
        assert st.scales.cpu().numpy()[0] == want_scale
        _ = (xd.float() * 2).sum().item()  # eager work between replays
