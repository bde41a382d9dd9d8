"""The INT4 + LoRA forward that allocates nothing (rpx_int4lora_forward_static)
against the workspace entry point it mirrors, through the C ABI (GPU)."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from oracle import int4 as oint4
from oracle.codecs import f32_to_bf16_bits
from representax_amd import _native as nat
from representax_amd import ops
from tests.helpers import bf16_values, rng, to_dev, to_dev_bf16

pytestmark = pytest.mark.gpu

STATIC_BYTES = 16 << 20  # RPX_STATIC_SCRATCH_BYTES


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _linear(n, k, r, group, seed):
    g = rng(seed)
    w = (g.standard_normal((n, k)) * 0.02).astype(np.float32)
    packed, scales = oint4.pack_int4(w, group)
    a = to_dev_bf16((g.standard_normal((r, k)) * 0.05).astype(np.float32))
    b = to_dev_bf16((g.standard_normal((n, r)) * 1.0).astype(np.float32))
    bias = to_dev(f32_to_bf16_bits((g.standard_normal(n) * 0.5).astype(np.float32))
                  .view(np.int16)).view(torch.uint16)
    return dict(packed=to_dev(packed), scales=to_dev(scales.view(np.int16)).view(torch.uint16),
                a=a, b=b, bias=bias, group=group, r=r)


def _static_forward(lin, x):
    m, k = x.shape
    n = lin["packed"].shape[0]
    y = torch.empty((m, n), dtype=torch.bfloat16, device=x.device)
    h = torch.empty((m, lin["r"]), dtype=torch.bfloat16, device=x.device)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    nat.call("rpx_int4lora_forward_static", _p(x), nat.DTYPE_BF16, m, k, _p(lin["packed"]),
             _p(lin["scales"]), n, ops.group_arg(lin["group"], k), _p(lin["bias"]), _p(lin["a"]),
             _p(lin["b"]), lin["r"], 2.0, _p(y), _p(h), stream)
    return y, h


# (m_first, m_second, k, n, r, group): the one-launch skinny kernels (M <= 64,
# and M <= 4 at K >= 4096), the two-launch skinny kernels (M <= 4) and the
# MFMA path; the second call of each pair is smaller
CASES = [(64, 16, 2048, 6144, 32, 64), (4, 1, 6144, 2048, 32, 64), (3, 2, 2048, 2048, 32, 64),
         (512, 300, 768, 3072, 16, None)]


@pytest.mark.parametrize("m1,m2,k,n,r,group", CASES)
def test_static_forward_equals_workspace_forward(m1, m2, k, n, r, group):
    lin = _linear(n, k, r, group, seed=k + n + m1)
    for m in (m1, m2):
        x = to_dev_bf16(bf16_values(rng(m + 3).standard_normal((m, k))))
        ys, hs = _static_forward(lin, x)
        yw, hw = ops.int4lora_forward(x, lin["packed"], lin["scales"], lin["a"], lin["b"],
                                      scaling=2.0, group_size=group, bias_bits=lin["bias"])
        torch.cuda.synchronize()
        assert torch.equal(ys, yw) and torch.equal(hs, hw), m


def test_static_forward_rejects_calls_beyond_its_scratch():
    """A shape whose scratch exceeds the static buffer (the generic path of
    a K that is not a multiple of 64) is refused before any launch."""

    m, k, n, r = 2048, 1000, 1024, 8
    need = nat.query("rpx_int4lora_forward_workspace", m, n, k, 0, r, nat.DTYPE_BF16)
    assert need > STATIC_BYTES
    lin = _linear(n, k, r, None, seed=5)
    x = torch.zeros((m, k), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError, match="static buffer"):
        _static_forward(lin, x)
