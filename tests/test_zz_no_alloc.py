"""lse_w8a16_gemm_noalloc, the W8A16 entry point that allocates nothing (its split-K partial sums
live in the library's static per-device scratch), against lse_w8a16_gemm with a caller workspace,
through the C ABI: bit-identical outputs on consecutive calls, the second one smaller, so what
the first call left in the scratch must not leak into the second."""

from __future__ import annotations

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

MODE_W8A16 = 0


def _weights(pkg, dev, n, k, seed):
    gen = torch.Generator().manual_seed(seed)
    w = (torch.randn(n, k, generator=gen) * 0.02).to(dev)
    q, s = pkg.ops.quantize_weight_per_channel(w)
    return pkg.ops.pack_weight(q), s


def _with_workspace(lib, x, qp, s, m, n, k, stream):
    y = torch.full((m, n), -3.0, dtype=torch.bfloat16, device=x.device)
    nbytes = lib.lse_workspace_bytes(MODE_W8A16, m, n, k)
    ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=x.device)
    st = lib.lse_w8a16_gemm(x.data_ptr(), k, qp.data_ptr(), s.data_ptr(), y.data_ptr(), n,
                            m, n, k, ws.data_ptr(), nbytes, stream)
    assert st == 0, lib.lse_status_string(st)
    return y, nbytes


def _no_alloc(lib, x, qp, s, m, n, k, stream):
    y = torch.full((m, n), -5.0, dtype=torch.bfloat16, device=x.device)
    st = lib.lse_w8a16_gemm_noalloc(x.data_ptr(), k, qp.data_ptr(), s.data_ptr(), y.data_ptr(),
                                    n, m, n, k, stream)
    assert st == 0, lib.lse_status_string(st)
    return y


@pytest.mark.parametrize("k,n,ms", [
    (14336, 4096, (64, 24)),   # down_proj: the split-K decode route, 8 MiB then 3 MiB of partials
    (4096, 6144, (64, 1)),     # fused qkv: no workspace
    (1024, 272, (300, 40)),    # prefill tile, then a ragged decode shape
    (14336, 4096, (200, 70)),  # down_proj on the split tiled route, 25 MiB then 8.75 MiB
])
def test_matches_the_workspace_entry_point(pkg, dev, k, n, ms):
    lib = pkg.library()
    stream = torch.cuda.current_stream().cuda_stream
    qp, s = _weights(pkg, dev, n, k, 90 + k + n)
    gen = torch.Generator().manual_seed(91 + k)
    for m in ms:  # two calls in a row, the second smaller
        x = torch.randn(m, k, generator=gen).to(torch.bfloat16).to(dev)
        ref, nbytes = _with_workspace(lib, x, qp, s, m, n, k, stream)
        got = _no_alloc(lib, x, qp, s, m, n, k, stream)
        torch.cuda.synchronize()
        assert nbytes <= lib.lse_query(5)
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), f"M={m} K={k} N={n}"


def test_ops_wrapper_allocates_nothing(pkg, dev):
    """Through ops.w8a16_linear_noalloc into a preallocated output: the caching allocator's
    counters do not move."""
    k, n = 14336, 4096
    qp, s = _weights(pkg, dev, n, k, 95)
    x = torch.randn(48, k).to(torch.bfloat16).to(dev)
    out = torch.empty(48, n, dtype=torch.bfloat16, device=dev)
    ref = pkg.ops.w8a16_linear(x, qp, s)
    torch.cuda.synchronize()
    before = torch.cuda.memory_stats(dev)["allocation.all.allocated"]
    pkg.ops.w8a16_linear_noalloc(x, qp, s, out)
    torch.cuda.synchronize()
    assert torch.cuda.memory_stats(dev)["allocation.all.allocated"] == before
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))


def test_every_llama_decode_shape_fits_the_scratch(pkg):
    """Every Llama-3-8B projection at 1..256 tokens (decode and the split tiled route)."""
    lib = pkg.library()
    cap = lib.lse_query(5)
    assert cap == 32 << 20
    for k, n in [(4096, 6144), (4096, 4096), (4096, 1024), (4096, 28672), (14336, 4096)]:
        for m in range(1, 257):
            assert lib.lse_workspace_bytes(MODE_W8A16, m, n, k) <= cap, (m, k, n)


def test_rejections_before_any_launch(pkg):
    lib = pkg.library()
    assert lib.lse_w8a16_gemm_noalloc(None, 16, None, None, None, 16, -1, 16, 16, None) == -2
    assert lib.lse_w8a16_gemm_noalloc(None, 16, None, None, None, 16, 1, 16, 17, None) != 0


def test_captured_split_k_calls_replay_bit_identically(pkg, dev):
    """A caller under graph capture: one M = 0 call looks the scratch address up first, then
    down_proj at 24 tokens (split-K decode route) and at 200 (split tiled route) are captured
    into one graph through the no-alloc entry point and replayed several times, with eager work
    between the replays; every replay equals lse_w8a16_gemm with a caller workspace."""
    lib = pkg.library()
    k, n = 14336, 4096
    qp, s = _weights(pkg, dev, n, k, 97)
    gen = torch.Generator().manual_seed(98)
    xs = {m: torch.randn(m, k, generator=gen).to(torch.bfloat16).to(dev) for m in (24, 200)}
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        assert lib.lse_w8a16_gemm_noalloc(None, k, None, None, None, n, 0, n, k,
                                          side.cuda_stream) == 0
        outs = {m: torch.empty(m, n, dtype=torch.bfloat16, device=dev) for m in xs}
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        cap = torch.cuda.current_stream().cuda_stream
        for m, x in xs.items():
            st = lib.lse_w8a16_gemm_noalloc(x.data_ptr(), k, qp.data_ptr(), s.data_ptr(),
                                            outs[m].data_ptr(), n, m, n, k, cap)
            assert st == 0, lib.lse_status_string(st)
    stream = torch.cuda.current_stream().cuda_stream
    for rep in range(3):
        for m in xs:
            xs[m].copy_(torch.randn(m, k, generator=gen).to(torch.bfloat16))
        graph.replay()
        torch.cuda.synchronize()
        for m, x in xs.items():
            ref, _ = _with_workspace(lib, x, qp, s, m, n, k, stream)
            torch.cuda.synchronize()
            assert torch.equal(outs[m].view(torch.int16), ref.view(torch.int16)), (rep, m)
