"""The committed fixtures (tests/golden/, written by make_golden.py from the CPU oracle) replayed
through the HIP path: weight quantizer, W8A16 in both kernel families, per-token activation
quantizer, W8A8 accumulators and epilogue (two-step and one-launch), on the small ragged case
with its all-zero weight row, exact-tie row and zero activation row; and config 0's weights,
whose digests are committed.

W8A16 outputs are held to the W8A16 rule against the stored fp64 golden (max-abs <= 1e-2
max|golden|, rel <= 1e-2 where |golden| > 1e-3 max|golden|); everything else bit for bit.
"""

from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from helpers import bf16_bits, to_bf16_tensor
from oracle import numerics as ora

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
DECODE, PREFILL = 1, 2


@pytest.fixture(scope="module")
def case():
    with np.load(GOLDEN / "small_cases.npz") as f:
        return {k: f[k] for k in f.files}


def test_weight_quantizer_reproduces_the_fixture(pkg, dev, case):
    q, s = pkg.ops.quantize_weight_per_channel(torch.from_numpy(case["w"]).to(dev))
    np.testing.assert_array_equal(q.cpu().numpy(), case["q"])
    np.testing.assert_array_equal(s.cpu().numpy(), case["s"])
    assert case["s"][3] == 1.0 and not case["q"][3].any(), "zero row: s = 1, q = 0"


@pytest.mark.parametrize("algo,reps", [(DECODE, 1), (DECODE, 12), (PREFILL, 1), (PREFILL, 13)])
def test_w8a16_matches_the_fixture(pkg, dev, case, algo, reps):
    """The 5 fixture tokens once (M = 5) and repeated (M = 60 in the decode kernel, M = 65 in
    the tiled kernel): each row within the W8A16 rule of its stored golden."""
    x = to_bf16_tensor(np.tile(case["x"], (reps, 1)), dev)
    qp = pkg.ops.pack_weight(torch.from_numpy(case["q"]).to(dev))
    y = pkg.ops.w8a16_linear(x, qp, torch.from_numpy(case["s"]).to(dev), algo=algo)
    y_bits = bf16_bits(y)
    for r in range(reps):
        ok, msg = ora.within_tolerance(y_bits[5 * r:5 * r + 5], case["y_w8a16"])
        assert ok, f"rows {5 * r}..: {msg}"
    assert np.all(ora.bf16_bits_to_f32(y_bits[:, 3]) == 0.0), "the all-zero weight row gives 0"


@pytest.mark.parametrize("reps", [1, 13])
def test_w8a8_matches_the_fixture(pkg, dev, case, reps):
    xo = np.tile(case["xo"], (reps, 1))
    xq, sx = pkg.ops.quantize_act_per_token(to_bf16_tensor(xo, dev))
    np.testing.assert_array_equal(xq.cpu().numpy(), np.tile(case["xq"], (reps, 1)))
    np.testing.assert_array_equal(sx.cpu().numpy(), np.tile(case["sx"], reps))
    assert case["sx"][2] == 1.0, "zero activation row: sx = 1"
    qp = pkg.ops.pack_weight(torch.from_numpy(case["q"]).to(dev))
    st = torch.from_numpy(case["s"]).to(dev)
    y, acc = pkg.ops.w8a8_gemm(xq, sx, qp, st, want_acc=True)
    np.testing.assert_array_equal(acc.cpu().numpy(), np.tile(case["acc"], (reps, 1)))
    np.testing.assert_array_equal(bf16_bits(y), np.tile(case["y_w8a8"], (reps, 1)))


def test_w8a8_one_launch_matches_the_fixture(pkg, dev, case):
    """The decode kernel that quantizes x while staging it (lse_w8a8_linear), from bf16."""
    qp = pkg.ops.pack_weight(torch.from_numpy(case["q"]).to(dev))
    y, acc = pkg.ops.w8a8_linear(to_bf16_tensor(case["xo"], dev), qp,
                                 torch.from_numpy(case["s"]).to(dev), want_acc=True,
                                 one_launch=True)
    np.testing.assert_array_equal(acc.cpu().numpy(), case["acc"])
    np.testing.assert_array_equal(bf16_bits(y), case["y_w8a8"])


def test_config0_weights_match_the_committed_digests(pkg, dev):
    """Config 0's seeded weight quantized on the GPU hashes to the committed SHA-256 digests."""
    digests = json.loads((GOLDEN / "config0_digests.json").read_text())
    x_bits, w = ora.seeded_inputs(0, 1, 2048, 2048)
    q, s = pkg.ops.quantize_weight_per_channel(torch.from_numpy(w).to(dev))
    sha = lambda a: hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()  # noqa: E731
    assert sha(x_bits) == digests["x_bits"]
    assert sha(q.cpu().numpy()) == digests["q"]
    assert sha(s.cpu().numpy()) == digests["s"]
