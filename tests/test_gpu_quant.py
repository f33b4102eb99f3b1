"""The two quantizers on the GPU, bit-exact against the oracle: per-channel weights (load time)
and per-token activations (W8A8 first stage)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import to_bf16_tensor
from oracle import numerics as ora

pytestmark = pytest.mark.gpu


def _quant_weight(pkg, dev, w: np.ndarray):
    q, s = pkg.ops.quantize_weight_per_channel(torch.from_numpy(w).to(dev))
    torch.cuda.synchronize()
    return q.cpu().numpy(), s.cpu().numpy()


@pytest.mark.parametrize("n,k", [(1, 16), (7, 48), (33, 1040), (256, 4096), (4096, 14336)])
def test_weight_quant_bit_exact(pkg, dev, n, k):
    _, w = ora.seeded_inputs(n * 31 + k, 1, n, k)
    q, s = _quant_weight(pkg, dev, w)
    q_ref, s_ref = ora.quantize_weight_per_channel(w)
    np.testing.assert_array_equal(s, s_ref)
    np.testing.assert_array_equal(q, q_ref)


def test_weight_quant_llama_gate_up_full_size(pkg, dev):
    """The largest config-1 weight, (N, K) = (28672, 4096), quantized on the GPU."""
    _, w = ora.seeded_inputs(1002, 1, 28672, 4096)
    q, s = _quant_weight(pkg, dev, w)
    q_ref, s_ref = ora.quantize_weight_per_channel(w)
    np.testing.assert_array_equal(s, s_ref)
    np.testing.assert_array_equal(q, q_ref)


def test_weight_quant_edge_rows(pkg, dev):
    """All-zero row (s = 1, q = 0), exact ties (RNE), a single non-zero, huge and tiny rows."""
    k = 32
    w = np.zeros((6, k), np.float32)
    w[1, :5] = [127.0, 63.5, -1.0, 0.5, 2.5]
    w[2, :4] = [254.0, -3.0, 5.0, 1.0]
    w[3, 9] = -1e-3
    w[4] = np.linspace(-3e38, 3e38, k, dtype=np.float32)
    w[5] = np.linspace(-1e-30, 1e-30, k, dtype=np.float32)
    q, s = _quant_weight(pkg, dev, w)
    q_ref, s_ref = ora.quantize_weight_per_channel(w)
    np.testing.assert_array_equal(s, s_ref)
    np.testing.assert_array_equal(q, q_ref)
    assert s[0] == 1.0 and not q[0].any()
    np.testing.assert_array_equal(q[1, :5], [127, 64, -1, 0, 2])


def test_weight_quant_strided_source(pkg, dev):
    """A weight view with row stride > K (ldw) reads only its own columns."""
    _, w = ora.seeded_inputs(77, 1, 40, 96)
    wide = np.full((40, 128), 1e9, np.float32)
    wide[:, :96] = w
    wt = torch.from_numpy(wide).to(dev)[:, :96]
    lib = pkg.library()
    q = torch.empty((40, 96), dtype=torch.int8, device=dev)
    s = torch.empty((40,), dtype=torch.float32, device=dev)
    st = lib.lse_quantize_weight_per_channel(
        wt.data_ptr(), 128, q.data_ptr(), s.data_ptr(), 40, 96, torch.cuda.current_stream().cuda_stream
    )
    assert st == 0
    torch.cuda.synchronize()
    q_ref, s_ref = ora.quantize_weight_per_channel(w)
    np.testing.assert_array_equal(q.cpu().numpy(), q_ref)
    np.testing.assert_array_equal(s.cpu().numpy(), s_ref)


def _quant_act(pkg, dev, x_bits):
    xq, sx = pkg.ops.quantize_act_per_token(to_bf16_tensor(x_bits, dev))
    torch.cuda.synchronize()
    return xq.cpu().numpy(), sx.cpu().numpy()


@pytest.mark.parametrize("m,k", [(1, 16), (3, 48), (32, 4096), (512, 14336), (4096, 4096),
                                 (7, 3072), (5, 6144), (3, 8192), (2, 8208)])
def test_act_quant_bit_exact_with_outliers(pkg, dev, m, k):
    """Config-3 activations: N(0,1) bf16 with round(0.001 K) columns scaled x20."""
    x_bits, _ = ora.seeded_inputs(3000 + m + k, m, 1, k, outliers=True)
    xq, sx = _quant_act(pkg, dev, x_bits)
    xq_ref, sx_ref = ora.quantize_act_per_token(x_bits)
    np.testing.assert_array_equal(sx, sx_ref)
    np.testing.assert_array_equal(xq, xq_ref)


def test_act_quant_zero_row_and_strided_rows(pkg, dev):
    x_bits, _ = ora.seeded_inputs(41, 5, 1, 64)
    x_bits[2] = 0
    wide = np.zeros((5, 80), np.uint16)
    wide[:, :64] = x_bits
    xt = to_bf16_tensor(wide, dev)[:, :64]
    xq, sx = pkg.ops.quantize_act_per_token(xt)
    torch.cuda.synchronize()
    xq_ref, sx_ref = ora.quantize_act_per_token(x_bits)
    np.testing.assert_array_equal(sx.cpu().numpy(), sx_ref)
    np.testing.assert_array_equal(xq.cpu().numpy(), xq_ref)
    assert sx_ref[2] == 1.0
