"""CPU oracle for the int8 quantized Linear forward. TEST INFRASTRUCTURE ONLY.

Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may import
this module, and then only as the checker. No product path routes through it. The product
path runs hand-written HIP kernels and fails when their library is missing.

The reference engine declares the path but does not implement it:
`ModelConfig.quantize` (src/llm_serving_engine/config.py:32) selects "int8", and
`ModelRunner.__init__` raises `NotImplementedError("int8 weight-only quantization")`
(src/llm_serving_engine/model/model_runner.py:45-46). Only the layer being replaced carries
arithmetic: `nn.Linear.forward` → `F.linear(x, W)` with bias=False for every Llama projection
(torch/nn/modules/linear.py:130-134; transformers modeling_llama.py:163-175,230-241). The
numerics below restate the quantized version of that layer as the benchmark configurations
define it:

* per-output-channel weights: s[n] = max_k |W[n,k]| / 127, q = clamp(rne(W / s), -127, 127);
* W8A16: y[m,n] = bf16(s[n] * sum_k x[m,k] * q[n,k]), fp32 accumulation;
* W8A8: sx[m] = max_k |x[m,k]| / 127, xq = clamp(rne(x / sx), -127, 127),
  acc = sum_k xq * q exactly in int32, y = bf16((fp32(acc) * sx[m]) * s[n]);
* fused gate/up (the MLP's `act_fn(gate_proj(x)) * up_proj(x)`, transformers
  modeling_llama.py:175, act_fn = SiLU): h = silu(g) * u with g, u the two projections above,
  silu(v) = v * sigmoid(v) (torch.nn.functional.silu, which transformers' SiLUActivation calls).

All-zero rows are not defined by the specification; this oracle fixes s = 1, q = 0.

Every function is pinned by a check that does not retype it (hand-worked known answers,
closed forms, brute force over exact rationals, torch's independent RNE cast and integer
matmul); those checks live in tests/test_oracle.py.

Dtypes on this boundary: bf16 tensors are carried as their uint16 bit patterns, so numpy
(which has no bfloat16) round-trips them exactly.
"""

from __future__ import annotations

import numpy as np

QMAX = 127


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    """bf16 bit patterns (uint16) → float32. Exact: bf16 is the top half of an fp32."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 → bf16 bit patterns, round-to-nearest-even on the dropped 16 bits.

    NaN inputs stay NaN (quiet bit forced); infinities and overflow to infinity behave as the
    IEEE rounding of the top half does.
    """
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    rounded = ((u + 0x7FFF + lsb) >> 16).astype(np.uint16)
    nan = np.isnan(np.asarray(x, dtype=np.float32))
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), rounded)


def f64_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float64 → bf16 via float32. Double rounding f64→f32→bf16 can differ from a direct
    f64→bf16 rounding by one bf16 ulp; callers compare such values with a tolerance."""
    return f32_to_bf16_bits(np.asarray(x, dtype=np.float64).astype(np.float32))


def quantize_weight_per_channel(w: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """W (N,K) float32 → q (N,K) int8, s (N,) float32.

    s[n] = fl32(amax_n / 127) with IEEE division; q = clamp(rne(fl32(W / s)), -127, 127).
    An all-zero row gets s = 1, q = 0.
    """
    w = np.asarray(w, dtype=np.float32)
    amax = np.max(np.abs(w), axis=1) if w.shape[1] else np.zeros(w.shape[0], np.float32)
    s = np.where(amax > 0, amax / np.float32(QMAX), np.float32(1.0)).astype(np.float32)
    q = np.clip(np.rint(w / s[:, None]), -QMAX, QMAX).astype(np.int8)
    return q, s


def pack_weight(q: np.ndarray) -> np.ndarray:
    """Row-major (N, K) int8 → the kernels' packed tile layout, (ceil(N/16), ceil(K/64), 1024).

    Tile (rb, j) byte 16*l + i holds q[16*rb + l % 16, 64*j + 16*(l // 16) + i], zero past N and
    K. This is a storage permutation, not arithmetic; the layout is this build's own (the
    reference stores row-major `nn.Linear.weight`, torch/nn/modules/linear.py:53).
    """
    q = np.asarray(q, dtype=np.int8)
    n, k = q.shape
    nrb, steps = -(-n // 16), -(-k // 64)
    padded = np.zeros((nrb * 16, steps * 64), np.int8)
    padded[:n, :k] = q
    # [rb][row r][step j][group g][byte i] -> [rb][j][g][r][i]
    t = padded.reshape(nrb, 16, steps, 4, 16).transpose(0, 2, 3, 1, 4)
    return np.ascontiguousarray(t).reshape(nrb, steps, 1024)


def quantize_act_per_token(x_bits: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """x (M,K) bf16 bits → xq (M,K) int8, sx (M,) float32, the same rule as the weights but per
    row of activations: sx[m] = fl32(max_k |x[m,k]| / 127), xq = clamp(rne(fl32(x / sx))).
    An all-zero row gets sx = 1, xq = 0."""
    return quantize_weight_per_channel(bf16_bits_to_f32(x_bits))


def w8a16_golden(x_bits: np.ndarray, q: np.ndarray, s: np.ndarray) -> np.ndarray:
    """fp64 golden of y = s[n] * sum_k x[m,k] q[n,k] (M,N). Every product x*q is exact in fp64
    (8-bit by 8-bit significands) and the fp64 sum's error is far below bf16 resolution."""
    x = bf16_bits_to_f32(x_bits).astype(np.float64)
    return (x @ np.asarray(q, dtype=np.float64).T) * np.asarray(s, dtype=np.float64)[None, :]


def w8a8_accumulate(xq: np.ndarray, q: np.ndarray) -> np.ndarray:
    """Exact int32 accumulators acc[m,n] = sum_k xq[m,k] q[n,k].

    |acc| <= 127 * 127 * K, which stays below 2^31 for K < 133,144, so int64 arithmetic
    followed by the int32 cast is exact for every shape the path accepts.
    """
    acc = np.asarray(xq, dtype=np.int64) @ np.asarray(q, dtype=np.int64).T
    if acc.size and np.max(np.abs(acc)) >= 2**31:
        raise OverflowError("int32 accumulator overflow")
    return acc.astype(np.int32)


def w8a8_epilogue(acc: np.ndarray, sx: np.ndarray, s: np.ndarray) -> np.ndarray:
    """y = bf16_rne((fp32(acc) * sx[m]) * s[n]), two fp32 roundings in this order."""
    a = np.asarray(acc, dtype=np.int32).astype(np.float32)
    y = (a * np.asarray(sx, np.float32)[:, None]) * np.asarray(s, np.float32)[None, :]
    return f32_to_bf16_bits(y.astype(np.float32))


def within_tolerance(y_bits: np.ndarray, golden: np.ndarray, rel: float = 1e-2) -> tuple[bool, str]:
    """The W8A16 acceptance rule: max-abs error <= rel * max|golden|, and elementwise relative
    error <= rel wherever |golden| > 1e-3 * max|golden|."""
    y = bf16_bits_to_f32(y_bits).astype(np.float64)
    g = np.asarray(golden, np.float64)
    if g.size == 0:
        return True, "empty"
    if not np.all(np.isfinite(y)):
        return False, "non-finite output"
    gmax = float(np.max(np.abs(g)))
    err = np.abs(y - g)
    max_abs = float(np.max(err))
    big = np.abs(g) > 1e-3 * gmax
    max_rel = float(np.max(err[big] / np.abs(g[big]))) if np.any(big) else 0.0
    ok = max_abs <= rel * max(gmax, 1e-30) and max_rel <= rel
    return ok, f"max_abs={max_abs:.3e} (gmax={gmax:.3e}) max_rel={max_rel:.3e}"


def seeded_inputs(
    seed: int, m: int, n: int, k: int, outliers: bool = False
) -> tuple[np.ndarray, np.ndarray]:
    """x (M,K) bf16 bits ~ N(0,1) and W (N,K) float32 ~ N(0, 0.02) from one seeded generator.
    With `outliers`, round(0.001*K) activation columns chosen by seeded permutation are
    multiplied by 20 in fp32 before the bf16 rounding."""
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    x = rng.standard_normal((m, k), dtype=np.float32)
    if outliers:
        cols = rng.permutation(k)[: int(round(0.001 * k))]
        x[:, cols] *= np.float32(20.0)
    return f32_to_bf16_bits(x), w


# ---- fused gate/up (LlamaMLP's SiLU-mul) ---------------------------------------------------


def pack_glu(q: np.ndarray) -> np.ndarray:
    """Stacked row-major (2I, K) int8 [gate; up] → the gate/up packed layout,
    (2 ceil(I/16), ceil(K/64), 1024): row tile 2t is pack_weight(gate)'s tile t, row tile 2t+1
    pack_weight(up)'s tile t (zero past I). A storage permutation of this build's own."""
    q = np.asarray(q, dtype=np.int8)
    i = q.shape[0] // 2
    gate, up = pack_weight(q[:i]), pack_weight(q[i:])
    out = np.empty((2 * gate.shape[0],) + gate.shape[1:], np.int8)
    out[0::2], out[1::2] = gate, up
    return out


def silu64(v: np.ndarray) -> np.ndarray:
    """v * sigmoid(v) in fp64, written as v / (1 + e^-v) (e^-v overflowing to inf gives -0 for
    very negative v, the limit)."""
    v = np.asarray(v, np.float64)
    with np.errstate(over="ignore"):
        return v / (1.0 + np.exp(-v))


def w8a16_glu_golden(x_bits: np.ndarray, q: np.ndarray, s: np.ndarray) -> np.ndarray:
    """fp64 golden of h = silu(g) * u (M, I) for the stacked (2I, K) weight q and (2I,) scales s:
    g = w8a16_golden over the gate half, u over the up half."""
    i = np.asarray(q).shape[0] // 2
    g = w8a16_golden(x_bits, q[:i], s[:i])
    u = w8a16_golden(x_bits, q[i:], s[i:])
    return silu64(g) * u


def w8a8_glu_operands(acc: np.ndarray, sx: np.ndarray, s: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """The fp32 gate and up values of the W8A8 gate/up epilogue from the exact int32 sums of the
    stacked weight (M, 2I): (fp32(acc) * sx[m]) * s[n], two fp32 roundings, split in halves."""
    a = np.asarray(acc, dtype=np.int32).astype(np.float32)
    v = (a * np.asarray(sx, np.float32)[:, None]) * np.asarray(s, np.float32)[None, :]
    i = v.shape[1] // 2
    return v[:, :i].astype(np.float32), v[:, i:].astype(np.float32)


def w8a8_glu_golden(acc: np.ndarray, sx: np.ndarray, s: np.ndarray) -> np.ndarray:
    """fp64 h = silu(g) * u from the exact fp32 g, u of `w8a8_glu_operands`; the kernel's
    result is this value rounded once to bf16, up to the fp32 error of its SiLU."""
    g, u = w8a8_glu_operands(acc, sx, s)
    return silu64(g) * u.astype(np.float64)


def bf16_ulps_apart(y_bits: np.ndarray, golden: np.ndarray) -> np.ndarray:
    """|y - golden| in units of the bf16 spacing at golden (2^(e-7) for |golden| in [2^e,
    2^(e+1)); the smallest normal spacing below that)."""
    y = bf16_bits_to_f32(y_bits).astype(np.float64)
    g = np.asarray(golden, np.float64)
    _, e = np.frexp(np.maximum(np.abs(g), np.finfo(np.float32).tiny))
    return np.abs(y - g) / np.ldexp(1.0, e - 8)


# ---- paged attention (the reference's paged_attention_forward) ------------------------------


def paged_attention_golden(
    q_bits: np.ndarray, k_pool_bits: np.ndarray, v_pool_bits: np.ndarray,
    block_table: np.ndarray, context_len: np.ndarray, query_offset: np.ndarray,
    q_start: np.ndarray, q_len: np.ndarray, block_size: int, scale: float | None = None,
) -> tuple[np.ndarray, np.ndarray]:
    """fp64 golden of paged attention (src/llm_serving_engine/kernels/flash_attention.py:201-284):
    q (H, T, D) bf16 bits, pools (blocks, block_size, H_KV, D) bf16 bits. Entry e's query row m
    (q row q_start[e] + m, cache position query_offset[e] + m) of head h attends to positions
    n < context_len[e], n <= query_offset[e] + m, held at pool block block_table[e][n //
    block_size], slot n % block_size, K/V head h // (H // H_KV); softmax of scale * q.k (scale
    1/sqrt(D) by default) times V. Returns (o (H, T, D) fp64, covered (T,) bool): rows no entry
    covers stay zero and are flagged False."""
    q = bf16_bits_to_f32(q_bits).astype(np.float64)
    kp = bf16_bits_to_f32(k_pool_bits).astype(np.float64)
    vp = bf16_bits_to_f32(v_pool_bits).astype(np.float64)
    h_all, t_all, d = q.shape
    g = h_all // kp.shape[2]
    scale = 1.0 / np.sqrt(d) if scale is None else scale
    out = np.zeros_like(q)
    covered = np.zeros(t_all, bool)
    for e in range(len(q_len)):
        ctx, qo, qs, ql = int(context_len[e]), int(query_offset[e]), int(q_start[e]), int(q_len[e])
        if ql == 0:
            continue
        pos = np.arange(ctx)
        blocks = np.asarray(block_table[e])[pos // block_size]
        k = kp[blocks, pos % block_size]  # (ctx, H_KV, D)
        v = vp[blocks, pos % block_size]
        rows = np.arange(ql)
        allowed = pos[None, :] <= (qo + rows)[:, None]  # (ql, ctx)
        covered[qs:qs + ql] = True
        for h in range(h_all):
            s = scale * (q[h, qs:qs + ql] @ k[:, h // g].T)
            s = np.where(allowed, s, -np.inf)
            mx = np.max(s, axis=1, keepdims=True)
            mx = np.where(np.isfinite(mx), mx, 0.0)
            p = np.exp(s - mx)
            den = p.sum(axis=1, keepdims=True)
            out[h, qs:qs + ql] = np.where(den > 0, (p @ v[:, h // g]) / np.where(den > 0, den, 1),
                                          0.0)
    return out, covered


def attention_within_tolerance(o_bits: np.ndarray, golden: np.ndarray, v_absmax: float,
                               covered: np.ndarray | None = None) -> tuple[bool, str]:
    """The paged-attention acceptance rule: |o - golden| <= 2^-8 (max|V| + |golden|) elementwise.
    Rounding each probability to bf16 before the product with V moves the output by at most
    2^-9 max|V| (it is a convex combination of V rows), and the bf16 output by 2^-9 |golden|:
    the bound leaves a factor of two."""
    o = bf16_bits_to_f32(o_bits).astype(np.float64)
    g = np.asarray(golden, np.float64)
    if covered is not None:
        o, g = o[:, covered], g[:, covered]
    if g.size == 0:
        return True, "empty"
    if not np.all(np.isfinite(o)):
        return False, "non-finite output"
    err = np.abs(o - g)
    bound = 2.0 ** -8 * (v_absmax + np.abs(g))
    worst = float(np.max(err / bound))
    return worst <= 1.0, f"max err {float(err.max()):.3e}, worst err/bound {worst:.3f}"


# ---- RMSNorm fused with per-token quantization ----------------------------------------------


def rmsnorm_bf16(x_bits: np.ndarray, w_bits: np.ndarray, eps: float) -> np.ndarray:
    """LlamaRMSNorm's roundings (transformers modeling_llama.py:62-67) on bf16 rows (M, K):
    var = fl32(mean x^2) (the mean in fp64, rounded once), r = fl32(1 / fl32(sqrt(var + eps))),
    h = bf16(w * bf16(fl32(x * r))). Returns h as bf16 bits. Implementations that sum the
    squares in another fp32 order can differ in the last bf16 place where x * r lies at a
    rounding boundary."""
    x = bf16_bits_to_f32(x_bits)
    var = np.mean(x.astype(np.float64) ** 2, axis=1).astype(np.float32)
    r = (np.float32(1.0) / np.sqrt((var + np.float32(eps)).astype(np.float32))).astype(np.float32)
    h = bf16_bits_to_f32(f32_to_bf16_bits((x * r[:, None]).astype(np.float32)))
    w = bf16_bits_to_f32(np.asarray(w_bits, np.uint16))
    return f32_to_bf16_bits((w[None, :] * h).astype(np.float32))


# ---- bf16 decode GEMM (the lm_head kept in bf16) -------------------------------------------


def pack_bf16_weight(w_bits: np.ndarray) -> np.ndarray:
    """Row-major (N, K) bf16 bits → the bf16 tile layout, (ceil(N/16), ceil(K/64), 2, 64, 8)
    uint16: step (rb, j) half h, lane l, element i = w[16 rb + l % 16][64 j + 16 (l // 16) +
    8 h + i], zero past N and K. A storage permutation of this build's own."""
    w = np.asarray(w_bits, np.uint16)
    n, k = w.shape
    nrb, steps = -(-n // 16), -(-k // 64)
    padded = np.zeros((nrb * 16, steps * 64), np.uint16)
    padded[:n, :k] = w
    # [rb][row r][step j][group g][half h][i] -> [rb][j][h][g][r][i]
    t = padded.reshape(nrb, 16, steps, 4, 2, 8).transpose(0, 2, 4, 3, 1, 5)
    return np.ascontiguousarray(t).reshape(nrb, steps, 2, 64, 8)


def bf16_linear_golden(x_bits: np.ndarray, w_bits: np.ndarray) -> np.ndarray:
    """fp64 x · wᵀ of bf16 operands (every product exact in fp64)."""
    return bf16_bits_to_f32(x_bits).astype(np.float64) @ bf16_bits_to_f32(w_bits).astype(np.float64).T
