"""Pins the CPU oracle (oracle/numerics.py) before anything is checked against it.

The reference holds no golden vectors or known-answer tests for this path (its int8 switch
raises NotImplementedError, src/llm_serving_engine/model/model_runner.py:45-46, pinned by
tests/test_model_runner.py:120-122), so each oracle function is pinned here by something that
does not restate it:
* hand-worked known answers (exact scales 1 and 2, ties that separate round-half-even from
  round-half-away);
* exact rational arithmetic (fractions.Fraction) with an explicit IEEE round-to-nearest-even,
  standing in for fp32 division and multiplication;
* independent library routines: torch's bf16 cast, torch._int_mm, aten._weight_int8pack_mm;
* brute force over tiny shapes, and planted mistakes that the acceptance rule must reject.
"""

from __future__ import annotations

import json
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import numerics as ora

GOLDEN = Path(__file__).resolve().parent / "golden"


def round_to_precision(v: Fraction, p: int) -> Fraction:
    """v rounded to p significant bits, ties to even (normal range only)."""
    if v == 0:
        return Fraction(0)
    sign = -1 if v < 0 else 1
    a = abs(v)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    ulp = Fraction(2) ** (e - (p - 1))
    t = a / ulp
    n = t.numerator // t.denominator
    r = t - n
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return sign * n * ulp


def fl32(v: Fraction) -> Fraction:
    return round_to_precision(v, 24)


def rne_int(v: Fraction) -> int:
    n = v.numerator // v.denominator
    r = v - n
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return n


# ---- bf16 rounding -------------------------------------------------------------------------


def test_bf16_rounding_matches_torch_cast():
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(1e3),
        np.array([0.0, -0.0, 1.0, np.inf, -np.inf, 3.3895314e38, 1e-40, -1e-45], np.float32),
        # exact ties: low 16 bits 0x8000 with even and odd kept parts
        np.array([0x3F808000, 0x3F818000, 0xBF808000, 0x7F7F8000], np.uint32).view(np.float32),
    ])
    ours = ora.f32_to_bf16_bits(vals)
    theirs = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(ours, theirs)
    assert np.isnan(ora.bf16_bits_to_f32(ora.f32_to_bf16_bits(np.array([np.nan], np.float32))))[0]


def test_bf16_roundtrip_is_exact():
    bits = np.arange(0, 65536, dtype=np.uint32).astype(np.uint16)
    finite = np.isfinite(ora.bf16_bits_to_f32(bits))
    np.testing.assert_array_equal(ora.f32_to_bf16_bits(ora.bf16_bits_to_f32(bits))[finite], bits[finite])


# ---- weight quantizer ----------------------------------------------------------------------


def test_weight_quant_known_answers():
    w = np.zeros((4, 5), np.float32)
    w[0] = [127.0, 63.5, -1.0, 0.5, 2.5]  # amax 127 → s = 1 exactly; ties go to even
    w[1] = [254.0, -3.0, 5.0, 1.0, -254.0]  # s = 2 exactly; -1.5 → -2, 2.5 → 2, 0.5 → 0
    w[3] = [0.0, 0.0, 0.0, 0.0, -0.25]  # s = fl32(0.25/127)
    q, s = ora.quantize_weight_per_channel(w)
    assert s[0] == 1.0 and s[1] == 2.0 and s[2] == 1.0
    np.testing.assert_array_equal(q[0], [127, 64, -1, 0, 2])
    np.testing.assert_array_equal(q[1], [127, -2, 2, 0, -127])
    np.testing.assert_array_equal(q[2], 0)  # all-zero row: s = 1, q = 0
    np.testing.assert_array_equal(q[3], [0, 0, 0, 0, -127])
    assert Fraction(float(s[3])) == fl32(Fraction(1, 4) / 127)


def test_weight_quant_matches_exact_rational_ieee():
    """s = fl32(amax/127) and q = rne(fl32(w/s)) computed with exact rationals."""
    _, w = ora.seeded_inputs(123, 1, 6, 40)
    q, s = ora.quantize_weight_per_channel(w)
    for n in range(w.shape[0]):
        amax = max(abs(Fraction(float(v))) for v in w[n])
        s_exact = fl32(amax / 127)
        assert Fraction(float(s[n])) == s_exact
        for k in range(w.shape[1]):
            t = fl32(Fraction(float(w[n, k])) / s_exact)
            assert q[n, k] == max(-127, min(127, rne_int(t))), (n, k)


def test_weight_quant_invariants_at_scale():
    _, w = ora.seeded_inputs(7, 1, 512, 4096)
    q, s = ora.quantize_weight_per_channel(w)
    assert q.dtype == np.int8 and s.dtype == np.float32 and q.shape == w.shape
    assert np.abs(q.astype(np.int32)).max() <= 127
    np.testing.assert_array_equal(np.abs(q.astype(np.int32)).max(axis=1), 127)
    # |q s - W| <= s/2, plus the fp32 rounding of W/s (half an ulp of |W/s| <= 127 is 2^-18 in
    # units of s) and of s itself (2^-24 relative, times |q| <= 127): 2^-16 covers both.
    err = np.abs(q.astype(np.float64) * s[:, None] - w.astype(np.float64))
    assert np.all(err <= s[:, None].astype(np.float64) * (0.5 + 2.0**-16))


# ---- activation quantizer ------------------------------------------------------------------


def test_act_quant_known_answers_and_outliers():
    x = np.zeros((3, 4), np.float32)
    x[0] = [1.0, -0.5, 0.25, 0.0]  # amax 1: s = fl32(1/127)
    x[2] = [-2.0, 2.0, 127.0, -127.0]  # amax 127: s = 1, exact
    xq, sx = ora.quantize_act_per_token(ora.f32_to_bf16_bits(x))
    assert Fraction(float(sx[0])) == fl32(Fraction(1, 127))
    for k, v in enumerate(x[0]):
        assert xq[0, k] == rne_int(fl32(Fraction(float(v)) / Fraction(float(sx[0]))))
    np.testing.assert_array_equal(xq[0], [127, -64, 32, 0])
    assert sx[1] == 1.0 and not xq[1].any()
    np.testing.assert_array_equal(xq[2], [-2, 2, 127, -127])
    x_bits, _ = ora.seeded_inputs(3, 8, 1, 4096, outliers=True)
    xf = ora.bf16_bits_to_f32(x_bits)
    big = np.abs(xf).max(axis=0) > 8.0
    assert 1 <= big.sum() <= 4  # round(0.001 * 4096) = 4 outlier columns, x20


def test_outlier_columns_count():
    for k, expected in ((2048, 2), (4096, 4), (14336, 14)):
        x_plain, _ = ora.seeded_inputs(5, 64, 1, k)
        x_out, _ = ora.seeded_inputs(5, 64, 1, k, outliers=True)
        changed = np.any(x_plain != x_out, axis=0)
        assert changed.sum() == expected


# ---- W8A16 golden --------------------------------------------------------------------------


def test_w8a16_golden_brute_force_rational():
    x_bits, w = ora.seeded_inputs(11, 3, 5, 32)
    q, s = ora.quantize_weight_per_channel(w)
    g = ora.w8a16_golden(x_bits, q, s)
    xf = ora.bf16_bits_to_f32(x_bits)
    for m in range(3):
        for n in range(5):
            exact = Fraction(float(s[n])) * sum(
                Fraction(float(xf[m, k])) * int(q[n, k]) for k in range(32)
            )
            assert abs(Fraction(float(g[m, n])) - exact) <= abs(exact) * Fraction(1, 2**50)


def test_w8a16_golden_unit_vector():
    _, w = ora.seeded_inputs(12, 1, 8, 64)
    q, s = ora.quantize_weight_per_channel(w)
    x = np.zeros((1, 64), np.float32)
    x[0, 9] = 1.0
    g = ora.w8a16_golden(ora.f32_to_bf16_bits(x), q, s)
    np.testing.assert_array_equal(g[0], q[:, 9].astype(np.float64) * s.astype(np.float64))


def test_w8a16_golden_agrees_with_torch_dequantized_linear():
    """torch's own fp64 F.linear on the dequantized weight (q·s applied before the sum, the
    other association) agrees to fp64 rounding. aten._weight_int8pack_mm would be the closer
    library routine, but this image's CPU build of it segfaults on some inputs."""
    x_bits, w = ora.seeded_inputs(13, 4, 96, 512)
    q, s = ora.quantize_weight_per_channel(w)
    x = torch.from_numpy(x_bits.view(np.int16)).view(torch.bfloat16).double()
    w_deq = torch.from_numpy(q).double() * torch.from_numpy(s).double()[:, None]
    y = torch.nn.functional.linear(x, w_deq).numpy()
    g = ora.w8a16_golden(x_bits, q, s)
    np.testing.assert_allclose(g, y, rtol=1e-12, atol=1e-12 * np.abs(g).max())


def test_tolerance_rule_rejects_planted_mistakes():
    """Plausible kernel bugs, planted in the oracle's output on the CPU, all fail the rule."""
    x_bits, w = ora.seeded_inputs(14, 8, 64, 1024)
    q, s = ora.quantize_weight_per_channel(w)
    g = ora.w8a16_golden(x_bits, q, s)
    good = ora.f64_to_bf16_bits(g)
    assert ora.within_tolerance(good, g)[0]
    dropped = ora.f64_to_bf16_bits(ora.w8a16_golden(x_bits[:, :-16], q[:, :-16], s))  # lost K tail
    wrong_scale = ora.f64_to_bf16_bits(g / s[None, :] * s[::-1][None, :])  # scale of another row
    transposed_tile = good.copy()
    transposed_tile[:4, :4] = good[:4, :4].T
    sign = good ^ np.uint16(0x8000)
    for bad in (dropped, wrong_scale, transposed_tile, sign):
        assert not ora.within_tolerance(bad, g)[0]


# ---- W8A8 ----------------------------------------------------------------------------------


def test_w8a8_accumulate_matches_int_mm_and_loops():
    rng = np.random.default_rng(15)
    xq = rng.integers(-127, 128, (33, 128)).astype(np.int8)
    q = rng.integers(-127, 128, (40, 128)).astype(np.int8)
    acc = ora.w8a8_accumulate(xq, q)
    ref = torch._int_mm(torch.from_numpy(xq), torch.from_numpy(q).t().contiguous()).numpy()
    np.testing.assert_array_equal(acc, ref)
    for m, n in ((0, 0), (5, 7), (32, 39)):
        assert acc[m, n] == sum(int(xq[m, k]) * int(q[n, k]) for k in range(128))


def test_w8a8_accumulate_extremes_and_overflow_guard():
    k = 14336
    a = np.full((1, k), 127, np.int8)
    b = np.full((2, k), -127, np.int8)
    assert ora.w8a8_accumulate(a, b)[0, 0] == -127 * 127 * k
    with pytest.raises(OverflowError):
        big = 133_200
        ora.w8a8_accumulate(np.full((1, big), 127, np.int8), np.full((1, big), 127, np.int8))


def test_w8a8_epilogue_order_is_pinned():
    """y = bf16(fl32(fl32(acc * sx) * s)); checked with exact rationals on values where the two
    association orders round differently."""
    rng = np.random.default_rng(16)
    acc = rng.integers(-2**24, 2**24, (6, 7)).astype(np.int32)
    sx = (rng.random(6).astype(np.float32) * np.float32(0.03)).astype(np.float32)
    s = (rng.random(7).astype(np.float32) * np.float32(0.002)).astype(np.float32)
    y = ora.w8a8_epilogue(acc, sx, s)
    differs = 0
    for m in range(6):
        for n in range(7):
            a = Fraction(int(acc[m, n]))
            left = fl32(fl32(a * Fraction(float(sx[m]))) * Fraction(float(s[n])))
            right = fl32(a * fl32(Fraction(float(sx[m])) * Fraction(float(s[n]))))
            expect = round_to_precision(left, 8)
            assert Fraction(float(ora.bf16_bits_to_f32(y[m:m + 1, n])[0])) == expect
            differs += left != right
    assert differs > 0  # the pinned order is observable on these inputs


# ---- committed fixtures --------------------------------------------------------------------


def test_oracle_reproduces_committed_fixtures():
    """tests/golden/*.npz were written by tests/golden/make_golden.py from this oracle; a change
    to the oracle's numerics shows up here."""
    with np.load(GOLDEN / "small_cases.npz") as f:
        q, s = ora.quantize_weight_per_channel(f["w"])
        np.testing.assert_array_equal(q, f["q"])
        np.testing.assert_array_equal(s, f["s"])
        np.testing.assert_array_equal(ora.w8a16_golden(f["x"], q, s), f["y_w8a16"])
        xq, sx = ora.quantize_act_per_token(f["xo"])
        np.testing.assert_array_equal(xq, f["xq"])
        np.testing.assert_array_equal(sx, f["sx"])
        acc = ora.w8a8_accumulate(xq, q)
        np.testing.assert_array_equal(acc, f["acc"])
        np.testing.assert_array_equal(ora.w8a8_epilogue(acc, sx, s), f["y_w8a8"])


def test_config0_digests():
    import hashlib

    digests = json.loads((GOLDEN / "config0_digests.json").read_text())
    x_bits, w = ora.seeded_inputs(0, 1, 2048, 2048)
    q, s = ora.quantize_weight_per_channel(w)
    y = ora.f64_to_bf16_bits(ora.w8a16_golden(x_bits, q, s))
    got = {
        name: hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()
        for name, a in (("x_bits", x_bits), ("q", q), ("s", s), ("y_bits", y))
    }
    assert got == digests


# ---- packed weight layout ------------------------------------------------------------------


def test_pack_weight_matches_the_layout_definition_by_brute_force():
    """Every byte of every tile, walked with explicit loops from the layout's definition,
    including the zero padding past N and K (N=37, K=80: three row tiles, two K steps)."""
    rng = np.random.default_rng(17)
    q = rng.integers(-127, 128, (37, 80)).astype(np.int8)
    qp = ora.pack_weight(q)
    assert qp.shape == (3, 2, 1024) and qp.dtype == np.int8
    for rb in range(3):
        for j in range(2):
            for lane in range(64):
                for i in range(16):
                    row, col = 16 * rb + lane % 16, 64 * j + 16 * (lane // 16) + i
                    expect = q[row, col] if row < 37 and col < 80 else 0
                    assert qp[rb, j, 16 * lane + i] == expect, (rb, j, lane, i)


def test_pack_weight_feeds_the_tile_walk_that_the_kernels_do():
    """A dot product computed the way the kernels consume tiles (lane l of tile (rb, j) holds 16
    K-consecutive weights of row l % 16 starting at 64 j + 16 (l // 16)) reproduces x·qᵀ
    exactly; a transposed or shifted layout would not."""
    rng = np.random.default_rng(18)
    n, k = 48, 192
    q = rng.integers(-127, 128, (n, k)).astype(np.int8)
    x = rng.integers(-5, 6, (3, k)).astype(np.int64)
    qp = ora.pack_weight(q)
    y = np.zeros((3, n), np.int64)
    for rb in range(qp.shape[0]):
        for j in range(qp.shape[1]):
            tile = qp[rb, j].reshape(64, 16).astype(np.int64)
            for lane in range(64):
                row = 16 * rb + lane % 16
                k0 = 64 * j + 16 * (lane // 16)
                y[:, row] += x[:, k0:k0 + 16] @ tile[lane]
    np.testing.assert_array_equal(y, x @ q.astype(np.int64).T)


# ---- fused gate/up -------------------------------------------------------------------------


def test_silu64_matches_torch_silu_and_the_llama_act_fn():
    """silu64 against torch.nn.functional.silu and transformers' SiLUActivation (the act_fn
    LlamaMLP applies, modeling_llama.py:172,175), in fp64, including both tails."""
    from transformers.activations import ACT2FN

    v = np.concatenate([np.linspace(-60, 60, 4001), [-1000.0, -88.7, 0.0, 1e-30, 88.7, 1000.0]])
    ours = ora.silu64(v)
    t = torch.from_numpy(v)
    np.testing.assert_allclose(ours, torch.nn.functional.silu(t).numpy(), rtol=1e-14, atol=1e-300)
    np.testing.assert_allclose(ours, ACT2FN["silu"](t).numpy(), rtol=1e-14, atol=1e-300)
    # closed forms: silu(0) = 0, silu(v) - silu(-v) = v
    assert ours[np.argmax(v == 0.0)] == 0.0
    np.testing.assert_allclose(ora.silu64(v) - ora.silu64(-v), v, rtol=1e-12, atol=1e-12)


def test_glu_golden_is_llama_mlp_in_fp64():
    """With K = I and down_proj set to the identity, transformers' own LlamaMLP in fp64 over the
    dequantized weights computes exactly act_fn(gate(x)) * up(x), the golden's definition."""
    from transformers import LlamaConfig
    from transformers.models.llama.modeling_llama import LlamaMLP

    k = i = 64
    x_bits, w = ora.seeded_inputs(21, 5, 2 * i, k)
    q, s = ora.quantize_weight_per_channel(w)
    mlp = LlamaMLP(LlamaConfig(hidden_size=k, intermediate_size=i, hidden_act="silu")).double()
    deq = torch.from_numpy(q.astype(np.float64) * s.astype(np.float64)[:, None])
    with torch.no_grad():
        mlp.gate_proj.weight.copy_(deq[:i])
        mlp.up_proj.weight.copy_(deq[i:])
        mlp.down_proj.weight.copy_(torch.eye(i, dtype=torch.float64))
        ref = mlp(torch.from_numpy(ora.bf16_bits_to_f32(x_bits).astype(np.float64))).numpy()
    np.testing.assert_allclose(ora.w8a16_glu_golden(x_bits, q, s), ref, rtol=1e-12, atol=1e-14)


def test_pack_glu_matches_the_layout_definition_by_brute_force():
    """Byte 16 l + b of tile (rb, j) is row (rb & 1) I + 16 (rb >> 1) + l % 16 of the stacked
    weight at column 64 j + 16 (l // 16) + b, zero past I or K; ragged I and K."""
    rng = np.random.default_rng(9)
    i, k = 20, 80
    q = rng.integers(-127, 128, (2 * i, k)).astype(np.int8)
    qp = ora.pack_glu(q)
    assert qp.shape == (4, 2, 1024)
    for rb in range(4):
        for j in range(2):
            for lane in range(64):
                for b in range(16):
                    r = 16 * (rb >> 1) + lane % 16
                    c = 64 * j + 16 * (lane // 16) + b
                    want = q[(rb & 1) * i + r, c] if r < i and c < k else 0
                    assert qp[rb, j, 16 * lane + b] == want, (rb, j, lane, b)


def test_w8a8_glu_operands_are_the_pinned_epilogue_before_rounding():
    """g and u rounded to bf16 are exactly the W8A8 epilogue of each half."""
    x_bits, w = ora.seeded_inputs(4, 7, 2 * 48, 256, outliers=True)
    q, s = ora.quantize_weight_per_channel(w)
    xq, sx = ora.quantize_act_per_token(x_bits)
    acc = ora.w8a8_accumulate(xq, q)
    g, u = ora.w8a8_glu_operands(acc, sx, s)
    np.testing.assert_array_equal(ora.f32_to_bf16_bits(g), ora.w8a8_epilogue(acc[:, :48], sx, s[:48]))
    np.testing.assert_array_equal(ora.f32_to_bf16_bits(u), ora.w8a8_epilogue(acc[:, 48:], sx, s[48:]))
    np.testing.assert_allclose(ora.w8a8_glu_golden(acc, sx, s),
                               g / (1 + np.exp(-g.astype(np.float64))) * u, rtol=1e-15)


def test_bf16_ulps_apart_known_answers():
    ys = ora.f32_to_bf16_bits(np.array([1.0, 1.0078125, 3.0, -0.5, 0.0], np.float32))
    gold = np.array([1.0, 1.0, 3.03125, -0.5, 0.0])
    np.testing.assert_allclose(ora.bf16_ulps_apart(ys, gold), [0.0, 1.0, 2.0, 0.0, 0.0])


# ---- paged attention -----------------------------------------------------------------------


def _paged_case(seed, h=8, h_kv=2, d=16, block_size=5, entries=((9, 0, 9), (1, 12, 13), (4, 3, 7))):
    """(q_len, query_offset, context_len) per entry; shuffled physical blocks, one pool."""
    rng = np.random.default_rng(seed)
    q_len = np.array([e[0] for e in entries], np.int32)
    qo = np.array([e[1] for e in entries], np.int32)
    ctx = np.array([e[2] for e in entries], np.int32)
    q_start = np.concatenate([[0], np.cumsum(q_len)[:-1]]).astype(np.int32)
    nblk = [-(-c // block_size) for c in ctx]
    perm = rng.permutation(sum(nblk) + 3)
    table = np.zeros((len(entries), max(nblk)), np.int32)
    at = 0
    for e, n in enumerate(nblk):
        table[e, :n] = perm[at:at + n]
        at += n
    blocks = len(perm)
    tokens = int(q_len.sum())
    q = ora.f32_to_bf16_bits(rng.standard_normal((h, tokens, d), dtype=np.float32))
    kp = ora.f32_to_bf16_bits(rng.standard_normal((blocks, block_size, h_kv, d), dtype=np.float32))
    vp = ora.f32_to_bf16_bits(rng.standard_normal((blocks, block_size, h_kv, d), dtype=np.float32))
    return q, kp, vp, table, ctx, qo, q_start, q_len, block_size


def test_paged_attention_golden_matches_torch_sdpa():
    """Against torch's scaled_dot_product_attention in fp64 on each entry's gathered K/V with an
    explicit causal-offset mask (an independent implementation of the same attention)."""
    q, kp, vp, table, ctx, qo, qs, ql, bs = _paged_case(1)
    out, covered = ora.paged_attention_golden(q, kp, vp, table, ctx, qo, qs, ql, bs)
    assert covered.all()
    qf = torch.from_numpy(ora.bf16_bits_to_f32(q).astype(np.float64))
    kf = torch.from_numpy(ora.bf16_bits_to_f32(kp).astype(np.float64))
    vf = torch.from_numpy(ora.bf16_bits_to_f32(vp).astype(np.float64))
    g = qf.shape[0] // kf.shape[2]
    for e in range(len(ql)):
        pos = torch.arange(int(ctx[e]))
        blk = torch.from_numpy(table[e].astype(np.int64))[pos // bs]
        k = kf[blk, pos % bs].permute(1, 0, 2).repeat_interleave(g, dim=0)  # (H, ctx, D)
        v = vf[blk, pos % bs].permute(1, 0, 2).repeat_interleave(g, dim=0)
        rows = torch.arange(int(ql[e]))
        mask = pos[None, :] <= (int(qo[e]) + rows)[:, None]
        ref = torch.nn.functional.scaled_dot_product_attention(
            qf[:, qs[e]:qs[e] + ql[e]], k, v, attn_mask=mask)
        np.testing.assert_allclose(out[:, qs[e]:qs[e] + ql[e]], ref.numpy(), rtol=1e-10, atol=1e-12)


def test_paged_attention_golden_brute_force_and_closed_forms():
    """Python loops over one tiny entry; a single visible key returns its V row exactly; equal
    scores average the visible V rows."""
    import math

    q, kp, vp, table, ctx, qo, qs, ql, bs = _paged_case(2, h=2, h_kv=1, d=4, block_size=3,
                                                         entries=((2, 2, 4),))
    out, _ = ora.paged_attention_golden(q, kp, vp, table, ctx, qo, qs, ql, bs)
    qf, kf, vf = (ora.bf16_bits_to_f32(a).astype(np.float64) for a in (q, kp, vp))
    for h in range(2):
        for m in range(2):
            n_vis = qo[0] + m + 1
            keys = [(table[0][n // bs], n % bs) for n in range(n_vis)]
            s = [sum(qf[h, m, i] * kf[b, w, 0, i] for i in range(4)) / 2.0 for b, w in keys]
            mx = max(s)
            p = [math.exp(x - mx) for x in s]
            o = [sum(p[j] * vf[b, w, 0, i] for j, (b, w) in enumerate(keys)) / sum(p) for i in range(4)]
            np.testing.assert_allclose(out[h, m], o, rtol=1e-12)
    # first query of a fresh prefill sees only position 0: o = v_0
    q, kp, vp, table, ctx, qo, qs, ql, bs = _paged_case(3, entries=((3, 0, 3),))
    out, _ = ora.paged_attention_golden(q, kp, vp, table, ctx, qo, qs, ql, bs)
    v0 = ora.bf16_bits_to_f32(vp).astype(np.float64)[table[0][0], 0]
    for h in range(out.shape[0]):
        np.testing.assert_array_equal(out[h, 0], v0[h // 4])
    # zero queries: uniform weights over the visible keys
    q0 = np.zeros_like(q)
    out, _ = ora.paged_attention_golden(q0, kp, vp, table, ctx, qo, qs, ql, bs)
    vf = ora.bf16_bits_to_f32(vp).astype(np.float64)
    mean2 = (vf[table[0][0], 0] + vf[table[0][0], 1]) / 2
    np.testing.assert_allclose(out[0, 1], mean2[0], rtol=1e-12)


def test_attention_tolerance_rejects_planted_mistakes():
    """A dropped key, a block read from outside the entry's table and a missing scale all exceed
    the bound; the golden itself rounded to bf16 passes. (Permuting an entry's own blocks would
    not: a row that sees all of them is invariant to their order.)"""
    q, kp, vp, table, ctx, qo, qs, ql, bs = _paged_case(4, d=32, entries=((6, 20, 26), (1, 40, 41)))
    golden, cov = ora.paged_attention_golden(q, kp, vp, table, ctx, qo, qs, ql, bs)
    vmax = float(np.abs(ora.bf16_bits_to_f32(vp)).max())
    ok, msg = ora.attention_within_tolerance(ora.f64_to_bf16_bits(golden), golden, vmax, cov)
    assert ok, msg
    short = ctx.copy()
    short[0] -= 1  # drops the last key of entry 0's last row
    bad, _ = ora.paged_attention_golden(q, kp, vp, table, short, qo, qs, ql, bs)
    bad[:, :5] = golden[:, :5]
    assert not ora.attention_within_tolerance(ora.f64_to_bf16_bits(bad), golden, vmax, cov)[0]
    foreign = table.copy()
    spare = sorted(set(range(kp.shape[0])) - set(table[table >= 0].ravel().tolist()))
    foreign[1, 0] = spare[0]  # a block no entry owns
    bad, _ = ora.paged_attention_golden(q, kp, vp, foreign, ctx, qo, qs, ql, bs)
    assert not ora.attention_within_tolerance(ora.f64_to_bf16_bits(bad), golden, vmax, cov)[0]
    bad, _ = ora.paged_attention_golden(q, kp, vp, table, ctx, qo, qs, ql, bs, scale=1.0)
    assert not ora.attention_within_tolerance(ora.f64_to_bf16_bits(bad), golden, vmax, cov)[0]


# ---- RMSNorm ---------------------------------------------------------------------------------


def test_rmsnorm_matches_llama_rmsnorm():
    """Against transformers' LlamaRMSNorm itself on bf16 rows (CPU): equal bits except where the
    two fp32 variance sums put x * r on opposite sides of a bf16 rounding boundary; that 1-ulp
    difference of the inner rounding, carried through the product with the weight and its own
    rounding, moves the output by at most 2 ulps, and rarely."""
    from transformers.models.llama.modeling_llama import LlamaRMSNorm

    rng = np.random.default_rng(11)
    m, k = 64, 4096
    x = rng.standard_normal((m, k), dtype=np.float32) * np.float32(3.0)
    x[3] = 0.0  # an all-zero row: r = 1/sqrt(eps), h = 0
    x_bits = ora.f32_to_bf16_bits(x)
    w_bits = ora.f32_to_bf16_bits(1.0 + 0.1 * rng.standard_normal(k, dtype=np.float32))
    norm = LlamaRMSNorm(k, eps=1e-5).to(torch.bfloat16)
    with torch.no_grad():
        norm.weight.copy_(torch.from_numpy(w_bits.view(np.int16)).view(torch.bfloat16))
        ref = norm(torch.from_numpy(x_bits.view(np.int16)).view(torch.bfloat16))
    ref_bits = ref.view(torch.int16).numpy().view(np.uint16)
    ours = ora.rmsnorm_bf16(x_bits, w_bits, 1e-5)
    diff = ora.bf16_ulps_apart(ours, ora.bf16_bits_to_f32(ref_bits).astype(np.float64))
    assert diff.max() <= 2.0 and np.mean(diff > 0) < 1e-3, (diff.max(), np.mean(diff > 0))
    assert np.all(ours[3] == 0)
    # eps placement: rows of one repeated value v give h = w * v / sqrt(v^2 + eps)
    v = np.full((1, k), 0.001, np.float32)
    h = ora.bf16_bits_to_f32(ora.rmsnorm_bf16(ora.f32_to_bf16_bits(v), ora.f32_to_bf16_bits(
        np.ones(k, np.float32)), 1e-5))
    vb = float(ora.bf16_bits_to_f32(ora.f32_to_bf16_bits(v))[0, 0])
    np.testing.assert_allclose(h[0, 0], vb / np.sqrt(vb * vb + 1e-5), rtol=2 ** -7)


def test_pack_bf16_weight_matches_the_layout_definition():
    """Brute force over the definition (ragged N and K), and a tile walk: the lo/hi operand pairs
    of every step, contracted with the matching activation slices, give x · wᵀ."""
    rng = np.random.default_rng(12)
    n, k = 20, 80
    w = ora.f32_to_bf16_bits(rng.standard_normal((n, k), dtype=np.float32))
    p = ora.pack_bf16_weight(w)
    assert p.shape == (2, 2, 2, 64, 8)
    for rb in range(2):
        for j in range(2):
            for h in range(2):
                for lane in range(64):
                    for i in range(8):
                        r, c = 16 * rb + lane % 16, 64 * j + 16 * (lane // 16) + 8 * h + i
                        want = w[r, c] if r < n and c < k else 0
                        assert p[rb, j, h, lane, i] == want
    x = ora.f32_to_bf16_bits(rng.standard_normal((3, k), dtype=np.float32))
    xf = np.zeros((3, 128))
    xf[:, :k] = ora.bf16_bits_to_f32(x)
    pf = ora.bf16_bits_to_f32(p)
    y = np.zeros((3, 32))
    for rb in range(2):
        for j in range(2):
            for lane in range(64):
                r, g = lane % 16, lane // 16
                for h in range(2):
                    cols = 64 * j + 16 * g + 8 * h + np.arange(8)
                    y[:, 16 * rb + r] += xf[:, cols] @ pf[rb, j, h, lane].astype(np.float64)
    np.testing.assert_allclose(y[:, :n], ora.bf16_linear_golden(x, w), rtol=1e-12, atol=1e-12)


def test_cpu_baselines_run_on_tiny_layers():
    """bench.py's CPU legs (bf16 F.linear, and torch's int8 kernels beside it) time every case
    and report bytes per second in the int8 layer's algorithmic bytes."""
    from oracle.cpu_baseline import time_bf16_linear_sweep, time_int8_restatements

    shapes, ms = [(64, 32), (128, 48)], [1, 3]
    bf16 = time_bf16_linear_sweep(shapes, ms, budget_s=2.0)
    assert len(bf16["cases"]) == 4 and bf16["gbps"] > 0
    assert bf16["bytes"] == sum(k * n + 4 * n + 2 * m * k + 2 * m * n for k, n in shapes for m in ms)
    r = time_int8_restatements(shapes, ms, budget_s=2.0)
    assert r["threads"] >= 1
    for name in ("w8a16_weight_int8pack_mm", "w8a8_int_mm"):
        assert r[name]["gbps"] > 0 and r[name]["seconds"] > 0
