"""Paged attention on the GPU (the reference's `paged_attention_forward`,
src/llm_serving_engine/kernels/flash_attention.py:287-332) against the fp64 oracle on seeded
inputs, through the C ABI.

Tolerance (`oracle.numerics.attention_within_tolerance`): |o - golden| <= 2^-8 (max|V| + |golden|)
elementwise. The kernel, like the reference, rounds each probability to bf16 before the product
with V (at most 2^-9 max|V|, the output being a convex combination of V rows) and rounds the
output to bf16 (2^-9 |golden|).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import bf16_bits, to_bf16_tensor
from oracle import numerics as ora

pytestmark = pytest.mark.gpu


def _case(seed, entries, h=32, h_kv=8, block_size=16, spare_blocks=3, d=128, max_q_len=None):
    """entries: (q_len, query_offset, context_len) each. Physical blocks shuffled over one pool,
    with `spare_blocks` that no entry owns."""
    rng = np.random.default_rng(seed)
    q_len = np.array([e[0] for e in entries], np.int32)
    qo = np.array([e[1] for e in entries], np.int32)
    ctx = np.array([e[2] for e in entries], np.int32)
    q_start = np.concatenate([[0], np.cumsum(q_len)[:-1]]).astype(np.int32)
    nblk = [max(1, -(-int(c) // block_size)) for c in ctx]
    perm = rng.permutation(sum(nblk) + spare_blocks)
    table = np.zeros((len(entries), max(nblk)), np.int32)
    at = 0
    for e, n in enumerate(nblk):
        table[e, :n] = perm[at:at + n]
        at += n
    tokens = int(q_len.sum())
    q = ora.f32_to_bf16_bits(rng.standard_normal((h, tokens, d), dtype=np.float32))
    shape = (len(perm), block_size, h_kv, d)
    kp = ora.f32_to_bf16_bits(rng.standard_normal(shape, dtype=np.float32))
    vp = ora.f32_to_bf16_bits(rng.standard_normal(shape, dtype=np.float32))
    return dict(q=q, kp=kp, vp=vp, table=table, ctx=ctx, qo=qo, qs=q_start, ql=q_len,
                bs=block_size, max_q_len=max_q_len or int(q_len.max()))


def _run(pkg, dev, c, kp=None, vp=None):
    i32 = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.int32)).to(dev)  # noqa: E731
    o = pkg.ops.paged_attention_forward(
        to_bf16_tensor(c["q"], dev), to_bf16_tensor(c["kp"] if kp is None else kp, dev),
        to_bf16_tensor(c["vp"] if vp is None else vp, dev), i32(c["table"]), i32(c["ctx"]),
        i32(c["qo"]), i32(c["qs"]), i32(c["ql"]), c["bs"], c["max_q_len"])
    torch.cuda.synchronize()
    return bf16_bits(o)


def _check(pkg, dev, c, what=""):
    o = _run(pkg, dev, c)
    golden, covered = ora.paged_attention_golden(c["q"], c["kp"], c["vp"], c["table"], c["ctx"],
                                                 c["qo"], c["qs"], c["ql"], c["bs"])
    vmax = float(np.abs(ora.bf16_bits_to_f32(c["vp"])).max())
    ok, msg = ora.attention_within_tolerance(o, golden, vmax, covered)
    assert ok, f"{what}: {msg}"
    return o


def test_decode_batch(pkg, dev):
    """Decode rows (q_len 1) over contexts from 1 to 1030 tokens, Llama-3-8B heads (32 q, 8 kv)."""
    ctxs = [1, 2, 17, 100, 333, 1024, 1030]
    _check(pkg, dev, _case(1, [(1, c - 1, c) for c in ctxs]), "decode")


def test_mixed_prefill_chunks_and_decode(pkg, dev):
    """A fresh prefill, chunked-prefill continuations (query_offset > 0) and decode rows in one
    launch, with a block size that is not a power of two."""
    entries = [(50, 0, 50), (33, 64, 97), (1, 200, 201), (7, 5, 12), (1, 0, 1), (129, 3, 132)]
    _check(pkg, dev, _case(2, entries, block_size=7), "mixed")


@pytest.mark.parametrize("h,h_kv", [(8, 8), (16, 8), (32, 4), (32, 2), (24, 8), (40, 8), (96, 8)])
def test_head_groupings(pkg, dev, h, h_kv):
    """MHA (1 query head per K/V head) up to 16 query heads per K/V head, including groups that
    do not divide the 16-row tile: 24 over 8 (the reference's default model,
    unsloth/Llama-3.2-3B-Instruct, config.py:29), 5 and 12 per K/V head."""
    entries = [(5, 10, 15), (1, 40, 41), (20, 0, 20), (7, 600, 607)]
    _check(pkg, dev, _case(3 + h_kv + h, entries, h=h, h_kv=h_kv), f"H={h} H_KV={h_kv}")


@pytest.mark.parametrize("ctx", [300, 4096, 9000])
def test_long_contexts_split_into_chunks(pkg, dev, ctx):
    """Few (entry, head) items over contexts longer than one 1024-key chunk take the split path:
    one workgroup per chunk, folded by a second pass. Deterministic: two calls agree bitwise."""
    c = _case(10 + ctx, [(1, ctx - 1, ctx), (3, ctx - 3, ctx)], block_size=32)
    nbytes = pkg.library().lse_paged_attention_workspace_bytes(
        2, 32, 8, 128, c["max_q_len"], c["table"].shape[1], c["bs"])
    assert (nbytes > 0) == (ctx > 1024), "the split path serves contexts of two chunks or more"
    first = _check(pkg, dev, c, f"ctx={ctx}")
    np.testing.assert_array_equal(_run(pkg, dev, c), first)


def _widened(c, bucket, pool_wide=True, scratch_fill=True):
    """The reference's graphed-decode call shape for case c (decode_graph.py:87-212): `bucket`
    entries whose rows past the real ones are padding (q_len 0, context 0, table on a scratch
    block), and a block table as wide as the whole pool (`_alloc`, num_blocks = the scratch id)."""
    e = len(c["ql"])
    nblocks = c["kp"].shape[0]
    width = nblocks if pool_wide else c["table"].shape[1]
    table = np.full((bucket, width), nblocks - 1 if scratch_fill else 0, np.int32)
    table[:e, :c["table"].shape[1]] = c["table"]
    pad = lambda a: np.concatenate([a, np.zeros(bucket - e, np.int32)])  # noqa: E731
    w = dict(c)
    w.update(table=table, ctx=pad(c["ctx"]), qo=pad(c["qo"]), ql=pad(c["ql"]),
             qs=np.concatenate([c["qs"], np.full(bucket - e, int(c["ql"].sum()), np.int32)]))
    return w


def test_rows_do_not_depend_on_batch_or_table_width(pkg, dev):
    """The reference's Triton kernel never splits a row over keys (grid (cdiv(max_q_len, BLOCK_M),
    entries * H), kernels/flash_attention.py:311), so a row's result does not depend on the rest of
    the call: its graphed decode (a bucket of entries padded with q_len = 0 rows, a table as wide
    as the pool, decode_graph.py:97,149) and its eager path (the batch's own entries and table
    width, model_runner.py:268-280) give the same tokens (tests/test_decode_graph.py:53-59). The
    HIP kernel keeps that bitwise: five decode rows over 1 to 2100 keys run as the eager call (40
    items: one workgroup per 1024-key chunk, folded by the second pass), as a 64-entry graph bucket
    over a pool-wide table (512 items: chunks folded inside one workgroup), with a larger
    max_q_len, and reordered inside another batch."""
    ctxs = [2100, 1, 513, 300, 1030]
    c = _case(60, [(1, n - 1, n) for n in ctxs], spare_blocks=40)
    base = _check(pkg, dev, c, "eager shape")
    lib = pkg.library()
    assert lib.lse_paged_attention_workspace_bytes(5, 32, 8, 128, 1, c["table"].shape[1], 16) > 0
    g = _widened(c, 64)
    assert lib.lse_paged_attention_workspace_bytes(64, 32, 8, 128, 1, g["table"].shape[1], 16) == 0
    o = _run(pkg, dev, g)
    np.testing.assert_array_equal(o[:, :len(ctxs)], base, err_msg="graph bucket, pool-wide table")
    g8 = dict(g, max_q_len=8)
    np.testing.assert_array_equal(_run(pkg, dev, g8)[:, :len(ctxs)], base, err_msg="max_q_len 8")
    w = _widened(c, 9, pool_wide=True, scratch_fill=False)
    np.testing.assert_array_equal(_run(pkg, dev, w)[:, :len(ctxs)], base, err_msg="bucket 9")
    # The same rows reversed, after a prefill chunk of another entry, in one call.
    order = list(reversed(range(len(ctxs))))
    other_blocks = list(range(c["kp"].shape[0] - 40, c["kp"].shape[0] - 38))
    table = np.zeros((len(ctxs) + 1, c["table"].shape[1]), np.int32)
    table[0, :2] = other_blocks
    for i, src in enumerate(order):
        table[i + 1] = c["table"][src]
    mixed = dict(c, table=table,
                 ctx=np.array([20] + [c["ctx"][s] for s in order], np.int32),
                 qo=np.array([0] + [c["qo"][s] for s in order], np.int32),
                 ql=np.array([20] + [1] * len(ctxs), np.int32),
                 qs=np.array([0] + list(range(20, 20 + len(ctxs))), np.int32), max_q_len=20)
    q = np.zeros((c["q"].shape[0], 20 + len(ctxs), 128), np.uint16)
    q[:, :20] = c["q"][:, :1]
    for i, src in enumerate(order):
        q[:, 20 + i] = c["q"][:, src]
    mixed["q"] = q
    om = _check(pkg, dev, mixed, "mixed batch")
    for i, src in enumerate(order):
        np.testing.assert_array_equal(om[:, 20 + i], base[:, src], err_msg=f"mixed row {src}")


def test_contexts_beyond_the_split_limit(pkg, dev):
    """A table spanning more than 64 chunks (65536 keys) runs every item in one workgroup; the
    rows still equal the split launch of a narrower table bitwise."""
    c = _case(70, [(1, 2999, 3000), (2, 998, 1000)], block_size=16)
    base = _run(pkg, dev, c)
    wide = dict(c)
    width = 4200  # 67200 keys: 66 chunks, no split
    lib = pkg.library()
    assert lib.lse_paged_attention_workspace_bytes(2, 32, 8, 128, 2, width, 16) == 0
    assert lib.lse_paged_attention_workspace_bytes(2, 32, 8, 128, 2, c["table"].shape[1], 16) > 0
    table = np.zeros((2, width), np.int32)
    table[:, :c["table"].shape[1]] = c["table"]
    wide["table"] = table
    np.testing.assert_array_equal(_run(pkg, dev, wide), base)


def test_graph_bucket_larger_than_the_max_q_len(pkg, dev):
    """max_q_len above every q_len (a graphed decode's bucket) changes nothing."""
    c = _case(20, [(1, 9, 10), (1, 99, 100)])
    base = _run(pkg, dev, c)
    c["max_q_len"] = 8
    np.testing.assert_array_equal(_run(pkg, dev, c), base)


def test_entries_never_see_other_blocks(pkg, dev):
    """Blocks no entry owns, and slots past each entry's context, hold NaN: outputs are finite and
    unchanged (the reference's isolation test, tests/test_fused_forward.py:185)."""
    c = _case(30, [(3, 20, 23), (1, 12, 13), (9, 0, 9)], block_size=8, spare_blocks=4)
    base = _check(pkg, dev, c, "clean")
    kp, vp = c["kp"].copy(), c["vp"].copy()
    nan = np.uint16(0x7FC0)
    owned = set()
    for e, ctx in enumerate(c["ctx"]):
        for n in range(ctx):
            owned.add((int(c["table"][e][n // c["bs"]]), n % c["bs"]))
    for b in range(kp.shape[0]):
        for w in range(kp.shape[1]):
            if (b, w) not in owned:
                kp[b, w] = nan
                vp[b, w] = nan
    np.testing.assert_array_equal(_run(pkg, dev, c, kp, vp), base)


def test_replays_from_a_graph(pkg, dev):
    c = _case(40, [(1, 63, 64), (4, 60, 64), (1, 500, 501)])
    i32 = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.int32)).to(dev)  # noqa: E731
    args = [to_bf16_tensor(c["q"], dev), to_bf16_tensor(c["kp"], dev), to_bf16_tensor(c["vp"], dev),
            i32(c["table"]), i32(c["ctx"]), i32(c["qo"]), i32(c["qs"]), i32(c["ql"])]
    fn = lambda: pkg.ops.paged_attention_forward(*args, c["bs"], c["max_q_len"])  # noqa: E731
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    for i in range(3):
        args[0].copy_(torch.randn_like(args[0], dtype=torch.float32).to(torch.bfloat16))
        g.replay()
        torch.cuda.synchronize()
        eager = fn()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"


def test_rejections(pkg, dev):
    c = _case(50, [(1, 3, 4)])
    i32 = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.int32)).to(dev)  # noqa: E731
    q = to_bf16_tensor(c["q"], dev)
    kp, vp = to_bf16_tensor(c["kp"], dev), to_bf16_tensor(c["vp"], dev)
    idx = [i32(c[k]) for k in ("table", "ctx", "qo", "qs", "ql")]
    with pytest.raises(RuntimeError, match="bf16"):
        pkg.ops.paged_attention_forward(q.float(), kp, vp, *idx, c["bs"], 1)
    with pytest.raises(RuntimeError, match="int32"):
        pkg.ops.paged_attention_forward(q, kp, vp, idx[0].long(), *idx[1:], c["bs"], 1)
    with pytest.raises(RuntimeError, match="unsupported attention shape"):
        pkg.ops.paged_attention_forward(q[:, :, :64].contiguous(), kp[..., :64].contiguous(),
                                        vp[..., :64].contiguous(), *idx, c["bs"], 1)
