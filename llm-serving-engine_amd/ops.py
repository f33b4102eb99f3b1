"""Tensor-level ops over the C ABI. Each validates dtypes, devices and layouts in Python,
allocates its outputs with `torch.empty` (so CUDA-graph memory pools own them), and enqueues
the HIP kernel on the current stream without synchronising, which keeps every op capturable
into a graph.

Weights are held in the packed tile layout the kernels stream (`pack_weight`): a (N, K) int8
matrix becomes a (ceil(N/16), ceil(K/64), 1024) int8 tensor whose 1 KB tiles are 16 rows x 64
K-bytes each, in matrix-core operand order. The MLP's gate and up weights share one tensor in the
gate/up layout (`pack_glu`): row tile 2t holds gate rows 16t..16t+15, row tile 2t+1 the same up
rows, so one kernel computes both and applies SiLU-mul before anything leaves registers.
"""

from __future__ import annotations

import torch

from . import _lib

__all__ = [
    "bf16_decode_linear",
    "pack_bf16_weight",
    "packed_bf16_shape",
    "unpack_bf16_weight",
    "paged_attention_forward",
    "pack_glu",
    "pack_weight",
    "packed_glu_shape",
    "packed_shape",
    "quantize_act_per_token",
    "quantize_weight_per_channel",
    "rmsnorm_quantize",
    "unpack_glu",
    "unpack_weight",
    "w8a8_gemm",
    "w8a8_glu",
    "w8a8_glu_quantized",
    "w8a8_linear",
    "w8a16_glu",
    "w8a16_linear",
    "w8a16_linear_noalloc",
    "workspace",
]


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _on_gpu(*tensors: torch.Tensor) -> torch.device:
    dev = tensors[0].device
    _require(dev.type == "cuda", f"int8 kernels need a CUDA (HIP) device, got {dev}")
    for t in tensors[1:]:
        _require(t.device == dev, f"tensors on different devices: {dev} and {t.device}")
    return dev


def _rows(x: torch.Tensor, k: int) -> torch.Tensor:
    """(..., K) → a 2-D (rows, K) view whose last dim is contiguous."""
    _require(x.shape[-1] == k, f"expected last dim {k}, got {tuple(x.shape)}")
    x2 = x.reshape(-1, k)
    strided_rows = x2.shape[0] > 1 and (x2.stride(0) < k or x2.stride(0) % 8)
    if x2.stride(-1) != 1 or strided_rows or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    return x2


# ---- packed weights --------------------------------------------------------------------------


def packed_shape(n: int, k: int) -> tuple[int, int, int]:
    return ((n + 15) // 16, (k + 63) // 64, 1024)


def pack_weight(q: torch.Tensor) -> torch.Tensor:
    """Row-major (N, K) int8 → packed (ceil(N/16), ceil(K/64), 1024) int8, on the GPU."""
    _require(q.dim() == 2 and q.dtype == torch.int8, "q must be a 2-D int8 tensor")
    dev = _on_gpu(q)
    n, k = q.shape
    q = q.contiguous()
    qp = torch.empty(packed_shape(n, k), dtype=torch.int8, device=dev)
    _lib.check(_lib.library().lse_pack_weight(q.data_ptr(), n, k, qp.data_ptr(), _stream(dev)),
               "lse_pack_weight")
    return qp


def unpack_weight(qp: torch.Tensor, n: int, k: int) -> torch.Tensor:
    """Inverse of `pack_weight` (a pure permutation, done with torch views): (N, K) int8."""
    rb, steps, _ = qp.shape
    t = qp.reshape(rb, steps, 4, 16, 16)  # [rb][step][g = lane // 16][row = lane % 16][16 bytes]
    t = t.permute(0, 3, 1, 2, 4).reshape(rb * 16, steps * 64)
    return t[:n, :k].contiguous()


def packed_glu_shape(i: int, k: int) -> tuple[int, int, int]:
    return (2 * ((i + 15) // 16), (k + 63) // 64, 1024)


def pack_glu(q: torch.Tensor) -> torch.Tensor:
    """Stacked row-major (2I, K) int8 [gate; up] → the gate/up layout, (2 ceil(I/16), ceil(K/64),
    1024) int8, on the GPU."""
    _require(q.dim() == 2 and q.dtype == torch.int8 and q.shape[0] % 2 == 0,
             "q must be a 2-D int8 tensor of 2I stacked gate and up rows")
    dev = _on_gpu(q)
    i, k = q.shape[0] // 2, q.shape[1]
    q = q.contiguous()
    qp = torch.empty(packed_glu_shape(i, k), dtype=torch.int8, device=dev)
    _lib.check(_lib.library().lse_pack_glu(q.data_ptr(), i, k, qp.data_ptr(), _stream(dev)),
               "lse_pack_glu")
    return qp


def unpack_glu(qp: torch.Tensor, i: int, k: int) -> torch.Tensor:
    """Inverse of `pack_glu`: the stacked (2I, K) int8 [gate; up]."""
    rows = unpack_weight(qp, qp.shape[0] * 16, k)  # packed rows, tile pairs (gate, up)
    pairs = rows.reshape(-1, 2, 16, k)
    gate = pairs[:, 0].reshape(-1, k)[:i]
    up = pairs[:, 1].reshape(-1, k)[:i]
    return torch.cat([gate, up]).contiguous()


def workspace(mode: int, m: int, n: int, k: int, dev: torch.device) -> torch.Tensor | None:
    """The workspace one GEMM call needs (deep decode shapes and 65..256 tokens over a narrow
    weight add partial sums of K ranges in a second pass), or None. Allocated with torch.empty,
    so graph-pool owned under capture; the caller keeps it alive until the call is enqueued."""
    nbytes = _lib.library().lse_workspace_bytes(mode, m, n, k)
    _require(nbytes >= 0, f"lse_workspace_bytes rejected (M, N, K) = ({m}, {n}, {k})")
    return torch.empty(nbytes, dtype=torch.uint8, device=dev) if nbytes else None


def _ws_args(ws: torch.Tensor | None) -> tuple[int | None, int]:
    return (ws.data_ptr(), ws.numel()) if ws is not None else (None, 0)


def _check_packed(qp: torch.Tensor, n: int, k: int, glu: bool = False) -> None:
    _require(qp.dtype == torch.int8 and qp.is_contiguous(), "packed weight must be contiguous int8")
    want = packed_glu_shape(n, k) if glu else packed_shape(n, k)
    what = "(I, K)" if glu else "(N, K)"
    _require(tuple(qp.shape) == want,
             f"packed weight has shape {tuple(qp.shape)}, {what} = ({n}, {k}) needs {want}")


def _glu_scales(scales: torch.Tensor) -> int:
    _require(scales.dtype == torch.float32 and scales.dim() == 1 and scales.shape[0] % 2 == 0,
             "gate/up scales must be fp32 (2I,) [gate; up]")
    return scales.shape[0] // 2


# ---- ops -------------------------------------------------------------------------------------


def quantize_weight_per_channel(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """W (N, K) → (q (N, K) int8 row-major, s (N,) fp32), s = amax/127 per row, q = clamp(rne(W/s)).

    Runs on the GPU at load time. W is read as fp32 (bf16/fp16 weights widen exactly).
    """
    _require(w.dim() == 2, f"weight must be 2-D, got {tuple(w.shape)}")
    dev = _on_gpu(w)
    n, k = w.shape
    w32 = w.to(torch.float32).contiguous()
    q = torch.empty((n, k), dtype=torch.int8, device=dev)
    s = torch.empty((n,), dtype=torch.float32, device=dev)
    lib = _lib.library()
    _lib.check(
        lib.lse_quantize_weight_per_channel(
            w32.data_ptr(), k, q.data_ptr(), s.data_ptr(), n, k, _stream(dev)
        ),
        "lse_quantize_weight_per_channel",
    )
    return q, s


def w8a16_linear(
    x: torch.Tensor,
    qp: torch.Tensor,
    scales: torch.Tensor,
    algo: int = _lib.ALGO_AUTO,
) -> torch.Tensor:
    """y = bf16(s[n] * sum_k x[..., k] q[n, k]) for x (..., K) bf16 → y (..., N) bf16, with the
    weight q given packed (`pack_weight`)."""
    dev = _on_gpu(x, qp, scales)
    _require(x.dtype == torch.bfloat16, f"W8A16 expects bf16 activations, got {x.dtype}")
    _require(scales.dtype == torch.float32 and scales.dim() == 1, "scales must be fp32 (N,)")
    n, k = scales.shape[0], x.shape[-1]
    _check_packed(qp, n, k)
    x2 = _rows(x, k)
    m = x2.shape[0]
    y = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
    ldx = x2.stride(0) if m > 1 else k
    ws = workspace(_lib.MODE_W8A16, m, n, k, dev)
    _lib.check(
        _lib.library().lse_w8a16_gemm_algo(
            x2.data_ptr(), ldx, qp.data_ptr(), scales.data_ptr(), y.data_ptr(), n,
            m, n, k, algo, *_ws_args(ws), _stream(dev),
        ),
        "lse_w8a16_gemm",
    )
    return y.view(*x.shape[:-1], n)


def w8a16_linear_noalloc(x: torch.Tensor, qp: torch.Tensor, scales: torch.Tensor,
                         out: torch.Tensor) -> torch.Tensor:
    """`w8a16_linear` into a caller-given `out` (M, N) bf16 through `lse_w8a16_gemm_noalloc`:
    nothing is allocated (the decode kernel's split-K partial sums live in the library's static
    per-device scratch). x must already be (M, K) with a contiguous last dim."""
    dev = _on_gpu(x, qp, scales, out)
    _require(x.dtype == torch.bfloat16 and out.dtype == torch.bfloat16, "bf16 x and out expected")
    _require(scales.dtype == torch.float32 and scales.dim() == 1, "scales must be fp32 (N,)")
    _require(x.dim() == 2 and x.stride(-1) == 1, "x must be (M, K) with a contiguous last dim")
    n, (m, k) = scales.shape[0], x.shape
    _check_packed(qp, n, k)
    _require(out.dim() == 2 and tuple(out.shape) == (m, n) and out.stride(-1) == 1,
             f"out must be ({m}, {n}) with a contiguous last dim")
    _lib.check(
        _lib.library().lse_w8a16_gemm_noalloc(
            x.data_ptr(), x.stride(0) if m > 1 else k, qp.data_ptr(), scales.data_ptr(),
            out.data_ptr(), out.stride(0) if m > 1 else n, m, n, k, _stream(dev)),
        "lse_w8a16_gemm_noalloc",
    )
    return out


def quantize_act_per_token(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """x (..., K) bf16 → (xq (rows, K) int8, sx (rows,) fp32), per-row symmetric int8."""
    dev = _on_gpu(x)
    _require(x.dtype == torch.bfloat16, f"W8A8 expects bf16 activations, got {x.dtype}")
    k = x.shape[-1]
    x2 = _rows(x, k)
    m = x2.shape[0]
    xq = torch.empty((m, k), dtype=torch.int8, device=dev)
    sx = torch.empty((m,), dtype=torch.float32, device=dev)
    ldx = x2.stride(0) if m > 1 else k
    _lib.check(
        _lib.library().lse_quantize_act_per_token(
            x2.data_ptr(), ldx, xq.data_ptr(), sx.data_ptr(), m, k, _stream(dev)
        ),
        "lse_quantize_act_per_token",
    )
    return xq, sx


def w8a8_gemm(
    xq: torch.Tensor,
    sx: torch.Tensor,
    qp: torch.Tensor,
    scales: torch.Tensor,
    want_acc: bool = False,
    want_y: bool = True,
) -> tuple[torch.Tensor | None, torch.Tensor | None]:
    """(y (M, N) bf16 or None, acc (M, N) int32 or None) from quantized operands; the weight q
    is given packed."""
    dev = _on_gpu(xq, sx, qp, scales)
    _require(scales.dtype == torch.float32 and scales.dim() == 1, "scales must be fp32 (N,)")
    n = scales.shape[0]
    _require(xq.dim() == 2, "xq must be (M, K) int8")
    m, k = xq.shape
    _require(xq.dtype == torch.int8 and xq.is_contiguous(), "xq must be (M, K) int8")
    _require(sx.dtype == torch.float32 and sx.shape == (m,), "sx must be fp32 (M,)")
    _check_packed(qp, n, k)
    y = torch.empty((m, n), dtype=torch.bfloat16, device=dev) if want_y else None
    acc = torch.empty((m, n), dtype=torch.int32, device=dev) if want_acc else None
    ws = workspace(_lib.MODE_W8A8, m, n, k, dev)
    _lib.check(
        _lib.library().lse_w8a8_gemm(
            xq.data_ptr(), sx.data_ptr(), qp.data_ptr(), scales.data_ptr(),
            y.data_ptr() if y is not None else None, n,
            acc.data_ptr() if acc is not None else None, m, n, k, *_ws_args(ws), _stream(dev),
        ),
        "lse_w8a8_gemm",
    )
    return y, acc


# Elements of x (M * K) up to which w8a8_linear takes the one-launch kernel.
ONE_LAUNCH_W8A8_MAX_ELEMS = 14336


def w8a8_linear(x: torch.Tensor, qp: torch.Tensor, scales: torch.Tensor,
                want_acc: bool = False, one_launch: bool | None = None):
    """Dynamic per-token W8A8: quantize x per row, int8 GEMM with exact int32 accumulation,
    y = bf16((acc * sx[m]) * s[n]). x (..., K) bf16 → y (..., N) bf16 (with want_acc, also the
    (M, N) int32 accumulators). Up to ONE_LAUNCH_W8A8_MAX_ELEMS elements of x (1 to 3 rows of
    4096, 1 row of 14336) run as one kernel that quantizes while it stages x (`lse_w8a8_linear`);
    more quantize first, then run the GEMM. Both give the same bits. The one-launch kernel
    quantizes all of x in every workgroup, so its cost grows with M * K: measured on MI355X over
    the Llama-3-8B shapes it is 3-16 % faster up to 14336 elements, and 6 % slower at 2 x 14336
    (down_proj) and up to 6 % at 4 x 4096. `one_launch` True takes the one-launch kernel wherever
    it runs (`lse_w8a8_linear_supported`), False never."""
    n, k = scales.shape[0], x.shape[-1]
    lib = _lib.library()
    m = x.numel() // k if k else 0
    if one_launch is None:
        one_launch = m * k <= ONE_LAUNCH_W8A8_MAX_ELEMS
    if m and one_launch and lib.lse_w8a8_linear_supported(m, k):
        dev = _on_gpu(x, qp, scales)
        _require(x.dtype == torch.bfloat16, f"W8A8 expects bf16 activations, got {x.dtype}")
        _require(scales.dtype == torch.float32 and scales.dim() == 1, "scales must be fp32 (N,)")
        _check_packed(qp, n, k)
        x2 = _rows(x, k)
        y = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
        acc = torch.empty((m, n), dtype=torch.int32, device=dev) if want_acc else None
        ldx = x2.stride(0) if m > 1 else k
        _lib.check(
            lib.lse_w8a8_linear(
                x2.data_ptr(), ldx, qp.data_ptr(), scales.data_ptr(), y.data_ptr(), n,
                acc.data_ptr() if acc is not None else None, m, n, k, _stream(dev),
            ),
            "lse_w8a8_linear",
        )
    else:
        xq, sx = quantize_act_per_token(x)
        y, acc = w8a8_gemm(xq, sx, qp, scales, want_acc=want_acc)
    y = y.view(*x.shape[:-1], n)
    return (y, acc) if want_acc else y


def w8a16_glu(
    x: torch.Tensor,
    qp: torch.Tensor,
    scales: torch.Tensor,
    algo: int = _lib.ALGO_AUTO,
) -> torch.Tensor:
    """h = bf16(silu(g) * u) for x (..., K) bf16 → h (..., I) bf16, where g and u are the fp32
    W8A16 products of x with the gate and up weights (`pack_glu` layout, scales (2I,) [gate;
    up]); one kernel, one rounding."""
    dev = _on_gpu(x, qp, scales)
    _require(x.dtype == torch.bfloat16, f"W8A16 expects bf16 activations, got {x.dtype}")
    i, k = _glu_scales(scales), x.shape[-1]
    _check_packed(qp, i, k, glu=True)
    x2 = _rows(x, k)
    m = x2.shape[0]
    h = torch.empty((m, i), dtype=torch.bfloat16, device=dev)
    ldx = x2.stride(0) if m > 1 else k
    _lib.check(
        _lib.library().lse_w8a16_glu(
            x2.data_ptr(), ldx, qp.data_ptr(), scales.data_ptr(), h.data_ptr(), i, m, i, k, algo,
            _stream(dev),
        ),
        "lse_w8a16_glu",
    )
    return h.view(*x.shape[:-1], i)


def w8a8_glu(x: torch.Tensor, qp: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """Dynamic per-token W8A8 form of `w8a16_glu`: x quantized per row, exact int32 sums,
    g = (acc_g * sx) * s_g, u likewise, h = bf16(silu(g) * u). x (..., K) → h (..., I)."""
    xq, sx = quantize_act_per_token(x)
    h = w8a8_glu_quantized(xq, sx, qp, scales)
    return h.view(*x.shape[:-1], h.shape[-1])


def w8a8_glu_quantized(xq: torch.Tensor, sx: torch.Tensor, qp: torch.Tensor,
                       scales: torch.Tensor) -> torch.Tensor:
    """`w8a8_glu` from already quantized rows: xq (M, K) int8, sx (M,) fp32 → h (M, I) bf16."""
    dev = _on_gpu(xq, sx, qp, scales)
    i = _glu_scales(scales)
    _require(xq.dim() == 2 and xq.dtype == torch.int8 and xq.is_contiguous(),
             "xq must be contiguous (M, K) int8")
    m, k = xq.shape
    _require(sx.dtype == torch.float32 and sx.shape == (m,), "sx must be fp32 (M,)")
    _check_packed(qp, i, k, glu=True)
    h = torch.empty((m, i), dtype=torch.bfloat16, device=dev)
    _lib.check(
        _lib.library().lse_w8a8_glu(
            xq.data_ptr(), sx.data_ptr(), qp.data_ptr(), scales.data_ptr(), h.data_ptr(), i, m, i,
            k, _stream(dev),
        ),
        "lse_w8a8_glu",
    )
    return h


def paged_attention_forward(
    q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
    block_table: torch.Tensor, context_len: torch.Tensor, query_offset: torch.Tensor,
    q_start: torch.Tensor, q_len: torch.Tensor, block_size: int, max_q_len: int,
) -> torch.Tensor:
    """One launch for a whole batch plan's attention at one layer against a shared paged K/V
    pool, with the reference's signature and meaning (`paged_attention_forward`,
    src/llm_serving_engine/kernels/flash_attention.py:287-332).

    q: (H, total_tokens, D) bf16. k_pool/v_pool: (num_blocks, block_size, H_KV, D) bf16, already
    holding this call's tokens. block_table (entries, max_blocks), context_len, query_offset,
    q_start, q_len (entries,): int32 on the device. max_q_len >= every q_len. Returns o like q.
    Softmax scale 1/sqrt(D). D = 128 and 1 <= H / H_KV <= 16 (24 query heads over 8 K/V
    heads included)."""
    dev = _on_gpu(q, k_pool, v_pool, block_table, context_len, query_offset, q_start, q_len)
    _require(q.dim() == 3 and k_pool.dim() == 4 and v_pool.shape == k_pool.shape,
             "q must be (H, T, D), k_pool/v_pool (num_blocks, block_size, H_KV, D)")
    _require(q.dtype == k_pool.dtype == v_pool.dtype == torch.bfloat16,
             f"paged attention runs on bf16 q/k/v, got {q.dtype}, {k_pool.dtype}, {v_pool.dtype}")
    for name, t in (("block_table", block_table), ("context_len", context_len),
                    ("query_offset", query_offset), ("q_start", q_start), ("q_len", q_len)):
        _require(t.dtype == torch.int32, f"{name} must be int32, got {t.dtype}")
    _require(block_table.dim() == 2 and block_table.stride(1) == 1, "block_table must be (E, B) "
             "with unit column stride")
    entries = block_table.shape[0]
    for name, t in (("context_len", context_len), ("query_offset", query_offset),
                    ("q_start", q_start), ("q_len", q_len)):
        _require(t.dim() == 1 and t.shape[0] == entries and t.stride(0) == 1,
                 f"{name} must be a contiguous ({entries},) tensor")
    h, _tokens, d = q.shape
    _, bs, h_kv, dk = k_pool.shape
    _require(dk == d and bs == block_size, "pool shape does not match q / block_size")
    _require(q.stride(2) == 1 and k_pool.stride(3) == 1 and v_pool.stride() == k_pool.stride(),
             "head dim must be contiguous and k_pool/v_pool must share strides")
    o = torch.empty_like(q)
    lib = _lib.library()
    nbytes = lib.lse_paged_attention_workspace_bytes(entries, h, h_kv, d, max_q_len,
                                                     block_table.shape[1], block_size)
    _require(nbytes >= 0, f"unsupported attention shape: H={h} H_KV={h_kv} D={d}")
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev) if nbytes else None
    _lib.check(
        lib.lse_paged_attention(
            q.data_ptr(), q.stride(0), q.stride(1), k_pool.data_ptr(), v_pool.data_ptr(),
            k_pool.stride(0), k_pool.stride(1), k_pool.stride(2), block_table.data_ptr(),
            block_table.stride(0), context_len.data_ptr(), query_offset.data_ptr(),
            q_start.data_ptr(), q_len.data_ptr(), o.data_ptr(), o.stride(0), o.stride(1),
            entries, h, h_kv, d, block_size, block_table.shape[1], max_q_len, 1.0 / d ** 0.5,
            *_ws_args(ws), _stream(dev),
        ),
        "lse_paged_attention",
    )
    return o


def rmsnorm_quantize(
    x: torch.Tensor, weight: torch.Tensor, eps: float, want_normed: bool = False,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor | None]:
    """LlamaRMSNorm (transformers modeling_llama.py:62-67) and per-token int8 quantization of its
    bf16 output in one kernel: x (..., K) bf16, weight (K,) bf16 → (xq (rows, K) int8, sx (rows,)
    fp32, normed (rows, K) bf16 or None)."""
    dev = _on_gpu(x, weight)
    _require(x.dtype == torch.bfloat16 and weight.dtype == torch.bfloat16,
             f"RMSNorm-quantize takes bf16 x and weight, got {x.dtype}, {weight.dtype}")
    k = x.shape[-1]
    _require(weight.shape == (k,), f"weight must be ({k},), got {tuple(weight.shape)}")
    x2 = _rows(x, k)
    m = x2.shape[0]
    w = weight.contiguous()
    xq = torch.empty((m, k), dtype=torch.int8, device=dev)
    sx = torch.empty((m,), dtype=torch.float32, device=dev)
    normed = torch.empty((m, k), dtype=torch.bfloat16, device=dev) if want_normed else None
    _lib.check(
        _lib.library().lse_rmsnorm_quantize(
            x2.data_ptr(), x2.stride(0) if m > 1 else k, w.data_ptr(), float(eps),
            xq.data_ptr(), sx.data_ptr(), normed.data_ptr() if normed is not None else None, m,
            k, _stream(dev),
        ),
        "lse_rmsnorm_quantize",
    )
    return xq, sx, normed


def packed_bf16_shape(n: int, k: int) -> tuple[int, int, int]:
    return ((n + 15) // 16, (k + 63) // 64, 1024)


def pack_bf16_weight(w: torch.Tensor) -> torch.Tensor:
    """Row-major (N, K) bf16 → the bf16 tile layout, a (ceil(N/16), ceil(K/64), 1024) bf16
    tensor (2 KB per 16-row x 64-K step: the lo and hi MFMA operands), on the GPU."""
    _require(w.dim() == 2 and w.dtype == torch.bfloat16, "w must be a 2-D bf16 tensor")
    dev = _on_gpu(w)
    n, k = w.shape
    w2 = w if w.stride(1) == 1 and w.stride(0) % 8 == 0 and w.data_ptr() % 16 == 0 else w.contiguous()
    wp = torch.empty(packed_bf16_shape(n, k), dtype=torch.bfloat16, device=dev)
    _lib.check(_lib.library().lse_pack_bf16_weight(w2.data_ptr(), w2.stride(0), n, k,
                                                    wp.data_ptr(), _stream(dev)),
               "lse_pack_bf16_weight")
    return wp


def unpack_bf16_weight(wp: torch.Tensor, n: int, k: int) -> torch.Tensor:
    """Inverse of `pack_bf16_weight` (a pure permutation, done with torch views): (N, K) bf16."""
    rb, steps, _ = wp.shape
    t = wp.reshape(rb, steps, 2, 4, 16, 8)  # [rb][step][half][g = lane // 16][row][8 elements]
    t = t.permute(0, 4, 1, 3, 2, 5).reshape(rb * 16, steps * 64)
    return t[:n, :k].contiguous()


def bf16_decode_linear(x: torch.Tensor, wp: torch.Tensor, n: int) -> torch.Tensor:
    """y = bf16(x · wᵀ) for x (..., K) bf16, w given packed (`pack_bf16_weight`) → y (..., N)
    bf16; fp32 accumulation. Built for decode batches (the decode kernel up to 16 rows, bf16
    tiles of the tiled kernel above), correct for any number of rows."""
    dev = _on_gpu(x, wp)
    _require(x.dtype == torch.bfloat16, f"expects bf16 activations, got {x.dtype}")
    k = x.shape[-1]
    _require(wp.dtype == torch.bfloat16 and tuple(wp.shape) == packed_bf16_shape(n, k),
             f"packed weight has shape {tuple(wp.shape)}, (N, K) = ({n}, {k}) needs "
             f"{packed_bf16_shape(n, k)}")
    x2 = _rows(x, k)
    m = x2.shape[0]
    y = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
    _lib.check(
        _lib.library().lse_bf16_decode_gemm(x2.data_ptr(), x2.stride(0) if m > 1 else k,
                                            wp.data_ptr(), y.data_ptr(), n, m, n, k,
                                            _stream(dev)),
        "lse_bf16_decode_gemm",
    )
    return y.view(*x.shape[:-1], n)
