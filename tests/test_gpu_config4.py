"""Config 4 at full size on the GPU: a random-init Llama-3-8B-architecture model (32 layers, hidden
4096, intermediate 14336, 32 q / 8 kv heads of 128, vocab 128256, lm_head kept bf16), 64 sequences
prefilled to 1024 tokens, then one decode step through the runner that follows the reference's
fused decoder path (`decoder_hidden`, src/llm_serving_engine/model/model_runner.py:213-224;
`_step_core`, decode_graph.py:125-140) with the int8 projections swapped in.

Parity is checked layer by layer: every projection of every layer (fused qkv, o_proj, fused
gate_up with its SiLU-mul, down_proj) against the golden of the very input the kernel saw in the
step, so an error in one layer cannot hide in the drift that 32 layers accumulate.
  * W8A16 ("int8"): the W8A16 rule against the fp64 golden (max-abs <= 1e-2 max|golden|, rel <=
    1e-2 where |golden| > 1e-3 max|golden|); gate_up against fp64 silu(g) * u.
  * W8A8: the oracle's per-token quantization of the input, exact integer sums (fp64 GEMM on the
    GPU: integer sums below 2^53), then the epilogue bit for bit; gate_up within 1 bf16 ulp of the
    fp64 silu(g) * u of the exact fp32 g, u.
Whole-step agreement (logits against the eager torch restatement of the same modules, greedy
tokens) is reported and loosely bounded: after 32 layers fp32 summation order moves logits.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import bf16_bits
from oracle import numerics as ora

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(600)]

LAYERS, BATCH, CONTEXT = 32, 64, 1024


@pytest.fixture(scope="module")
def runner(pkg, dev):
    from llm_serving_engine_amd.decode_step import DecodeRunner, random_llama

    print(f"config 4: building {LAYERS} layers, prefilling {BATCH} x {CONTEXT}", flush=True)
    model = random_llama(LAYERS, seed=4000, device=dev)
    r = DecodeRunner(model, BATCH, CONTEXT + 1)
    gen = torch.Generator().manual_seed(4001)
    prompt = torch.randint(0, model.config.vocab_size, (BATCH, CONTEXT), generator=gen).to(dev)
    r.prefill(prompt)
    r.next_token = torch.randint(0, model.config.vocab_size, (BATCH,), generator=gen).to(dev)
    torch.cuda.synchronize()
    yield r
    r.int8 = None
    del r, model
    torch.cuda.empty_cache()


def _traced_step(runner, mode):
    runner.quantize(mode)
    runner.use("int8")
    runner.trace = []
    logits = runner.step(runner.next_token, CONTEXT).float()
    trace, runner.trace = runner.trace, None
    runner.use("int8-torch")
    restated = runner.step(runner.next_token, CONTEXT).float()
    runner.use("int8")
    assert len(trace) == 4 * LAYERS, f"{len(trace)} projections traced"
    return trace, logits, restated


def _exact_acc(xq: np.ndarray, q: torch.Tensor) -> np.ndarray:
    xd = torch.from_numpy(xq).to(q.device).double()
    return (xd @ q.double().t()).round().to(torch.int32).cpu().numpy()


def test_w8a16_every_layer_within_tolerance(runner):
    trace, logits, restated = _traced_step(runner, "int8")
    worst = 0.0
    for i, name, x, y in trace:
        mod = runner.int8[i][name]
        q, s = mod.unpacked_qweight().double(), mod.scales.double()
        xd = x.reshape(-1, x.shape[-1]).double()
        if name == "gate_up":
            inter = mod.intermediate_size
            g = ((xd @ q[:inter].t()) * s[:inter]).cpu().numpy()
            u = ((xd @ q[inter:].t()) * s[inter:]).cpu().numpy()
            golden = ora.silu64(g) * u
        else:
            golden = ((xd @ q.t()) * s).cpu().numpy()
        ok, msg = ora.within_tolerance(bf16_bits(y.reshape(golden.shape)), golden)
        assert ok, f"layer {i} {name}: {msg}"
        err = np.abs(ora.bf16_bits_to_f32(bf16_bits(y.reshape(golden.shape))) - golden).max()
        worst = max(worst, float(err / np.abs(golden).max()))
    rel = float((logits - restated).norm() / restated.norm())
    match = float((logits.argmax(-1) == restated.argmax(-1)).float().mean())
    print(f"W8A16 config 4: worst layer max-abs / max|golden| {worst:.2e}; logits vs restatement "
          f"{rel:.4f}; greedy match {match:.3f}")
    assert rel < 0.05 and match >= 0.75


def test_w8a8_every_layer_bit_exact(runner):
    trace, logits, restated = _traced_step(runner, "w8a8")
    for i, name, x, y in trace:
        mod = runner.int8[i][name]
        q, s = mod.unpacked_qweight(), mod.scales.cpu().numpy()
        x_bits = bf16_bits(x.reshape(-1, x.shape[-1]))
        xq, sx = ora.quantize_act_per_token(x_bits)
        acc = _exact_acc(xq, q)
        y_bits = bf16_bits(y.reshape(acc.shape[0], -1))
        if name == "gate_up":
            ulps = ora.bf16_ulps_apart(y_bits, ora.w8a8_glu_golden(acc, sx, s))
            assert ulps.max() <= 1.0, f"layer {i} gate_up: {ulps.max():.2f} ulps"
        else:
            np.testing.assert_array_equal(y_bits, ora.w8a8_epilogue(acc, sx, s),
                                          err_msg=f"layer {i} {name}")
    # Every layer above is bit-exact on its own input; across 32 layers the torch restatement's
    # SiLU (libm exp against the kernel's hardware exp) moves some bf16 roundings of h by an ulp,
    # and each layer's per-token requantization turns such a flip into a whole quantization step,
    # so the whole-step logits drift more than in W8A16 (8 % measured on MI355X).
    rel = float((logits - restated).norm() / restated.norm())
    match = float((logits.argmax(-1) == restated.argmax(-1)).float().mean())
    print(f"W8A8 config 4: logits vs restatement {rel:.4f}; greedy match {match:.3f}")
    assert rel < 0.2 and match >= 0.75
