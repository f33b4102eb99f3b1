"""Config 4 at small scale on the GPU: the decode-step runner (the reference's fused decoder path
with the int8 linears swapped in) against the same runner on the reference's bf16 linears."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def runner(pkg, dev):
    from llm_serving_engine_amd.decode_step import DecodeRunner, random_llama

    model = random_llama(2, seed=11, device=dev)
    r = DecodeRunner(model, batch=16, capacity=40)
    gen = torch.Generator().manual_seed(12)
    r.prefill(torch.randint(0, model.config.vocab_size, (16, 32), generator=gen).to(dev), chunk=4)
    return r


def test_int8_step_tracks_the_bf16_reference(runner, dev):
    gen = torch.Generator().manual_seed(13)
    vocab = runner.model.config.vocab_size
    tok = torch.randint(0, vocab, (16,), generator=gen).to(dev)
    runner.use("bf16")
    ref, inputs = [], []
    for t in range(3):
        inputs.append(tok)
        logits = runner.step(tok, 32 + t).float()
        ref.append(logits)
        tok = logits.argmax(-1)
    runner.quantize("int8")
    runner.use("int8")
    matches = 0
    for t in range(3):
        logits = runner.step(inputs[t], 32 + t).float()
        rel = (logits - ref[t]).norm() / ref[t].norm()
        assert rel < 0.05, f"step {t}: logits differ by {rel:.3f} (relative norm)"
        matches += int((logits.argmax(-1) == ref[t].argmax(-1)).sum())
    assert matches >= 0.9 * 48, f"greedy match {matches}/48"


def test_int8_kernels_match_the_torch_restatement(runner, dev):
    """The same quantized weights through the HIP kernels and through an eager fp32 torch
    restatement: logits agree to bf16 rounding and fp32 order, and so do the greedy tokens."""
    if runner.int8 is None:
        runner.quantize("int8")
    gen = torch.Generator().manual_seed(14)
    tok = torch.randint(0, runner.model.config.vocab_size, (16,), generator=gen).to(dev)
    runner.use("int8-torch")
    ref = runner.step(tok, 35).float()
    runner.use("int8")
    got = runner.step(tok, 35).float()
    rel = (got - ref).norm() / ref.norm()
    assert rel < 1e-2, f"relative logit difference {rel:.4f}"
    assert int((got.argmax(-1) == ref.argmax(-1)).sum()) >= 15


def test_int8_linear_stack_replays_from_a_graph(runner, dev):
    """All projections of one step captured into one graph: every replay equals eager."""
    if runner.int8 is None:
        runner.quantize("int8")
    runner.use("int8")
    calls = runner.linear_calls(16)
    eager = [mod(x) for mod, x in calls]
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = [mod(x) for mod, x in calls]
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        for a, b in zip(eager, outs):
            assert torch.equal(a, b)


def test_paged_attention_matches_the_torch_attention(runner, dev):
    """One int8 decode step through the HIP paged attention (shuffled 16-slot blocks) and through
    the fp32 torch attention over the contiguous cache: logits agree to the bf16 rounding of the
    probabilities, and so do the greedy tokens."""
    if runner.int8 is None:
        runner.quantize("int8")
    runner.use("int8")
    if runner.k_pool is None:
        runner.enable_paged()
    gen = torch.Generator().manual_seed(15)
    tok = torch.randint(0, runner.model.config.vocab_size, (16,), generator=gen).to(dev)
    runner.use_attention("torch")
    ref = runner.step(tok, 36).float()
    runner.use_attention("paged")
    got = runner.step(tok, 36).float()
    runner.use_attention("torch")
    rel = (got - ref).norm() / ref.norm()
    assert rel < 1e-2, f"relative logit difference {rel:.4f}"
    assert int((got.argmax(-1) == ref.argmax(-1)).sum()) >= 15


def test_whole_step_replays_from_a_graph(runner, dev):
    """The reference's graphed-decode invariant (tests/test_decode_graph.py:53-59: graphed ==
    eager) on the swapped path: one whole decode step (embedding to logits) with the int8 linears
    and the HIP paged attention, captured into a graph, equals the eager step bitwise on every
    replay, with eager steps in between. Each step writes the same K/V values at the same
    position, so every run sees the same state."""
    if runner.int8 is None:
        runner.quantize("int8")
    runner.use("int8")
    if runner.k_pool is None:
        runner.enable_paged()
    runner.use_attention("paged")
    gen = torch.Generator().manual_seed(16)
    tok = torch.randint(0, runner.model.config.vocab_size, (16,), generator=gen).to(dev)
    pos = 37
    eager = runner.step(tok, pos).clone()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        runner.step(tok, pos)
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = runner.step(tok, pos)
    try:
        for i in range(3):
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager), f"replay {i}"
            again = runner.step(tok, pos)
            torch.cuda.synchronize()
            assert torch.equal(again, eager), f"eager after replay {i}"
    finally:
        runner.use_attention("torch")
