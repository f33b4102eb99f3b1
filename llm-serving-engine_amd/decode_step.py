"""Config 4: the decode-step linear stack of a Llama-3-8B-architecture model, through a runner
that follows the reference's fused decoder path.

The reference's eager path flattens a batch plan into one (1, total_tokens) row of tokens and
runs `decoder_hidden` (src/llm_serving_engine/model/model_runner.py:213-224): embedding, rotary
embedding, then per layer `hidden += attend(input_layernorm(hidden))` and
`hidden += mlp(post_attention_layernorm(hidden))`, then the final norm; `emit_owed`
(model_runner.py:290-308) applies the bf16 lm_head to each sequence's last row and greedy
sampling takes the argmax (sampling.py:34-36). Its attention projects q/k/v with three
`nn.Linear` calls and rotates q and k (`_project_qkv`, model_runner.py:310-326), attends, then
applies o_proj (`attention_output`, model_runner.py:365-369).

`DecodeRunner` runs exactly that sequence over HF Llama modules, with two linear back ends:
  * "bf16": the reference's own `nn.Linear` modules (q, k, v, o, gate, up, down: seven GEMMs a
    layer on the vendor BLAS);
  * "int8" / "w8a8": `Int8Linear` on the fused (4096, 6144) QKV shape the kernels are tuned for
    (split after the GEMM), o_proj and down_proj, and `Int8GateUp` for gate/up: one (4096, 28672)
    weight stream whose epilogue applies the MLP's SiLU-mul, so the (M, 28672) projection never
    leaves the kernel. Per-channel quantization of a row-stacked weight equals quantizing each
    part;
  * "int8-torch": the same quantized weights, applied by an eager torch restatement of each
    module's own arithmetic instead of the HIP kernels (`restate`: W8A16 s·Σ x·q in fp32, W8A8
    per-token quantization, exact integer sums and (acc·sx)·s; gate/up as fp32 g and u with
    silu(g)·u rounded once, as the fused kernel rounds it); it isolates the kernels from the
    quantization itself. Test and measurement use only.
With `trace` set to a list, every int8 projection of a step appends (layer, name, input,
output), so each layer's kernels can be checked on the very input they saw (errors do not
compound over layers).
lm_head stays bf16 in every back end: the vendor BLAS's `nn.Linear` on "bf16" and "int8-torch",
`PackedBf16Linear` (the same bf16 weight in the packed tile layout, `quantize_model_`'s default)
on "int8", in either quantization mode. Attention has two implementations: "torch", fp32 over a
contiguous per-layer KV cache (the reference's `contiguous_attention` path,
model_runner.py:400-418), the same arithmetic for both linear back ends so only the linears
differ; and "paged", the HIP paged attention (`ops.paged_attention_forward`, the reference's
`attend_paged`, model_runner.py:357-363) over a per-layer pool of 16-slot blocks handed to the
sequences in shuffled order, kept in step with the contiguous cache once `enable_paged()` has
allocated it.
"""

from __future__ import annotations

import math

import torch
from torch import nn

from . import ops
from .int8_linear import Int8GateUp, Int8Linear, PackedBf16Linear

LLAMA3_8B = dict(
    hidden_size=4096,
    intermediate_size=14336,
    num_attention_heads=32,
    num_key_value_heads=8,
    head_dim=128,
    vocab_size=128256,
    rope_theta=500000.0,
    rms_norm_eps=1e-5,
    max_position_embeddings=8192,
    initializer_range=0.02,
)


def random_llama(num_layers: int, seed: int, device: torch.device, **overrides) -> nn.Module:
    """A random-init Llama-3-8B-architecture `LlamaForCausalLM` in bf16 on `device` (weights
    ~ N(0, 0.02), the architecture's own initializer_range; there is no checkpoint offline)."""
    from transformers import LlamaConfig, LlamaForCausalLM

    cfg = LlamaConfig(**{**LLAMA3_8B, **overrides, "num_hidden_layers": num_layers})
    torch.manual_seed(seed)
    with torch.device(device):
        model = LlamaForCausalLM._from_config(cfg, dtype=torch.bfloat16)
    model.eval()
    return model


class DecodeRunner:
    """Decode steps of `batch` sequences, one token each, over a contiguous KV cache of
    `capacity` positions per sequence."""

    def __init__(self, model: nn.Module, batch: int, capacity: int) -> None:
        self.model = model
        cfg = model.config
        self.layers = list(model.model.layers)
        self.batch = batch
        self.capacity = capacity
        self.n_heads = cfg.num_attention_heads
        self.n_kv = cfg.num_key_value_heads
        self.head_dim = getattr(cfg, "head_dim", None) or cfg.hidden_size // self.n_heads
        dev = next(model.parameters()).device
        shape = (batch, self.n_kv, capacity, self.head_dim)
        self.k_cache = [torch.zeros(shape, dtype=torch.bfloat16, device=dev) for _ in self.layers]
        self.v_cache = [torch.zeros(shape, dtype=torch.bfloat16, device=dev) for _ in self.layers]
        self.int8: list[dict[str, Int8Linear]] | None = None
        self.head: PackedBf16Linear | None = None
        self.trace: list | None = None
        self.backend = "bf16"
        self.attention = "torch"
        self.k_pool: list[torch.Tensor] | None = None
        self.v_pool: list[torch.Tensor] | None = None

    def enable_paged(self, block_size: int = 16, seed: int = 0) -> None:
        """Allocates a paged K/V pool per layer (the reference's allocate_kv_pool,
        model_runner.py:107-116: (num_blocks + 1, block_size, H_KV, D), the last block a
        scratch row) with each sequence's blocks drawn in shuffled order, and copies in what the
        contiguous cache holds. Call before prefill, or after: both caches then stay in step."""
        dev = self.k_cache[0].device
        per_seq = -(-self.capacity // block_size)
        num_blocks = self.batch * per_seq
        g = torch.Generator().manual_seed(seed)
        perm = torch.randperm(num_blocks, generator=g)
        self.block_size = block_size
        self.tables = perm.reshape(self.batch, per_seq).to(torch.int32).to(dev)
        shape = (num_blocks + 1, block_size, self.n_kv, self.head_dim)
        self.k_pool = [torch.zeros(shape, dtype=torch.bfloat16, device=dev) for _ in self.layers]
        self.v_pool = [torch.zeros(shape, dtype=torch.bfloat16, device=dev) for _ in self.layers]
        for i in range(len(self.layers)):
            self._write_pool(i, self.k_cache[i], self.v_cache[i], 0, self.capacity, slice(None))

    def use_attention(self, kind: str) -> None:
        if kind not in ("torch", "paged"):
            raise ValueError(f"unknown attention {kind!r}")
        if kind == "paged" and self.k_pool is None:
            raise RuntimeError("enable_paged() first")
        self.attention = kind

    def _write_pool(self, i: int, k: torch.Tensor, v: torch.Tensor, start: int, end: int,
                    rows) -> None:
        """k, v (nseq, H_KV, end - start, D) of sequences `rows` at positions [start, end)."""
        pos = torch.arange(start, end, device=k.device)
        blocks = self.tables[rows][:, pos // self.block_size].long()  # (nseq, ntok)
        within = (pos % self.block_size).expand_as(blocks)
        self.k_pool[i][blocks, within] = k.transpose(1, 2)
        self.v_pool[i][blocks, within] = v.transpose(1, 2)

    def _attend_paged(self, i: int, q: torch.Tensor, start: int, end: int, nseq: int,
                      ntok: int) -> torch.Tensor:
        """q (nseq, H, ntok, D) -> (1, nseq * ntok, H * D) through one paged attention launch."""
        dev = q.device
        qh = q.permute(1, 0, 2, 3).reshape(self.n_heads, nseq * ntok, self.head_dim).contiguous()
        table = self.tables[self._rows].contiguous()
        full = lambda v: torch.full((nseq,), v, dtype=torch.int32, device=dev)  # noqa: E731
        q_start = torch.arange(0, nseq * ntok, ntok, dtype=torch.int32, device=dev)
        o = ops.paged_attention_forward(qh, self.k_pool[i], self.v_pool[i], table, full(end),
                                        full(start), q_start, full(ntok), self.block_size, ntok)
        return o.permute(1, 0, 2).reshape(1, nseq * ntok, self.n_heads * self.head_dim)

    # ---- linear back ends ---------------------------------------------------------------------

    @torch.no_grad()
    def quantize(self, mode: str = "int8") -> None:
        """Builds the int8 projections from the bf16 weights (kept, for the bf16 back end)."""
        self.int8 = []
        for layer in self.layers:
            attn, mlp = layer.self_attn, layer.mlp
            qkv = torch.cat([attn.q_proj.weight, attn.k_proj.weight, attn.v_proj.weight])
            self.int8.append({
                "qkv": _int8(qkv, mode),
                "o": _int8(attn.o_proj.weight, mode),
                "gate_up": Int8GateUp.from_linears(mlp.gate_proj, mlp.up_proj, mode),
                "down": _int8(mlp.down_proj.weight, mode),
            })
            del qkv
        head = self.model.lm_head
        self.head = head if isinstance(head, PackedBf16Linear) else PackedBf16Linear.from_linear(head)
        torch.cuda.empty_cache()

    def use(self, backend: str) -> None:
        if backend not in ("bf16", "int8", "int8-torch"):
            raise ValueError(f"unknown back end {backend!r}")
        if backend != "bf16" and self.int8 is None:
            raise RuntimeError("quantize() first")
        self.backend = backend

    def _lin(self, i: int, name: str, x: torch.Tensor) -> torch.Tensor:
        mod = self.int8[i][name]
        if self.backend != "int8":
            return restate(mod, x)
        y = mod(x)
        if self.trace is not None:
            self.trace.append((i, name, x, y))
        return y

    def _qkv(self, i: int, normed: torch.Tensor):
        if self.backend == "bf16":
            attn = self.layers[i].self_attn
            return attn.q_proj(normed), attn.k_proj(normed), attn.v_proj(normed)
        qkv = self._lin(i, "qkv", normed)
        nq, nkv = self.n_heads * self.head_dim, self.n_kv * self.head_dim
        return qkv[..., :nq], qkv[..., nq:nq + nkv], qkv[..., nq + nkv:]

    def _o(self, i: int, x: torch.Tensor) -> torch.Tensor:
        if self.backend == "bf16":
            return self.layers[i].self_attn.o_proj(x)
        return self._lin(i, "o", x)

    def _mlp(self, i: int, x: torch.Tensor) -> torch.Tensor:
        mlp = self.layers[i].mlp
        if self.backend == "bf16":
            return mlp(x)
        return self._lin(i, "down", self._lin(i, "gate_up", x))

    # ---- the step -----------------------------------------------------------------------------

    def _attend(self, i: int, normed: torch.Tensor, rope, start: int, nseq: int,
                ntok: int) -> torch.Tensor:
        """normed (1, nseq*ntok, hidden), sequences contiguous, every sequence at positions
        [start, start + ntok). Writes K/V there and attends causally over [0, end). The
        positions come in as a host int, so a step captures into a graph."""
        from transformers.models.llama.modeling_llama import apply_rotary_pos_emb

        q, k, v = self._qkv(i, normed)
        q = q.reshape(nseq, ntok, self.n_heads, self.head_dim).transpose(1, 2)
        k = k.reshape(nseq, ntok, self.n_kv, self.head_dim).transpose(1, 2)
        v = v.reshape(nseq, ntok, self.n_kv, self.head_dim).transpose(1, 2)
        cos, sin = rope
        q, k = apply_rotary_pos_emb(q, k, cos, sin)
        end = start + ntok
        self.k_cache[i][self._rows, :, start:end] = k
        self.v_cache[i][self._rows, :, start:end] = v
        if self.k_pool is not None:
            self._write_pool(i, k, v, start, end, self._rows)
        if self.attention == "paged":
            return self._o(i, self._attend_paged(i, q, start, end, nseq, ntok))
        keys = self.k_cache[i][self._rows, :, :end].float()
        vals = self.v_cache[i][self._rows, :, :end].float()
        rep = self.n_heads // self.n_kv
        keys = keys.repeat_interleave(rep, dim=1)
        vals = vals.repeat_interleave(rep, dim=1)
        scores = torch.matmul(q.float(), keys.transpose(-1, -2).contiguous())
        scores = scores / math.sqrt(self.head_dim)
        qpos = torch.arange(start, end, device=scores.device)[:, None]
        kpos = torch.arange(end, device=scores.device)[None, :]
        scores = scores.masked_fill(kpos > qpos, float("-inf"))
        out = torch.matmul(torch.softmax(scores, dim=-1), vals)
        out = out.to(torch.bfloat16).transpose(1, 2).reshape(1, nseq * ntok, -1)
        return self._o(i, out)

    @torch.no_grad()
    def forward(self, tokens: torch.Tensor, start: int, rows: slice | None = None) -> torch.Tensor:
        """tokens (nseq, ntok) of sequences `rows` (default: all) at positions [start,
        start + ntok) -> final-norm hidden of every token, (1, nseq*ntok, hidden)."""
        self._rows = rows if rows is not None else slice(None)
        nseq, ntok = tokens.shape
        model = self.model.model
        ids = tokens.reshape(1, nseq * ntok)
        pos = torch.arange(start, start + ntok, device=tokens.device).repeat(nseq, 1)
        hidden = model.embed_tokens(ids)
        cos, sin = model.rotary_emb(hidden, pos.reshape(1, -1))
        rope = (cos.reshape(nseq, ntok, -1), sin.reshape(nseq, ntok, -1))
        for i, layer in enumerate(self.layers):
            hidden = hidden + self._attend(i, layer.input_layernorm(hidden), rope, start, nseq,
                                           ntok)
            hidden = hidden + self._mlp(i, layer.post_attention_layernorm(hidden))
        return model.norm(hidden)

    @torch.no_grad()
    def prefill(self, tokens: torch.Tensor, chunk: int = 8) -> None:
        """Fills positions [0, tokens.shape[1]) of every sequence's cache, `chunk` sequences at a
        time."""
        for s in range(0, tokens.shape[0], chunk):
            self.forward(tokens[s:s + chunk], 0, slice(s, s + chunk))

    @torch.no_grad()
    def step(self, tokens: torch.Tensor, position: int) -> torch.Tensor:
        """One decode step: tokens (batch,) at `position` -> bf16 logits (batch, vocab) from the
        bf16 lm_head (the reference's emit_owed)."""
        hidden = self.forward(tokens[:, None], position)
        return self.lm_head()(hidden[0])

    def lm_head(self) -> nn.Module:
        """The back end's lm_head: the packed bf16 one on "int8", the model's own otherwise."""
        return self.head if self.backend == "int8" and self.head is not None else self.model.lm_head

    # ---- linear-only timing -------------------------------------------------------------------

    def linear_calls(self, m: int) -> list:
        """(module, input) for every projection of one decode step at M = m, with inputs of the
        right shapes (the values do not change the time of a weight stream), and the MLP's
        SiLU-mul between gate/up and down: a call of its own on the bf16 back end, inside the
        fused gate/up kernel on the int8 one."""
        dev = next(self.model.parameters()).device
        g = torch.Generator(device="cpu").manual_seed(7)
        hid = self.model.config.hidden_size
        inter = self.model.config.intermediate_size
        x_h = torch.randn(m, hid, generator=g).to(torch.bfloat16).to(dev)
        x_i = torch.randn(m, inter, generator=g).to(torch.bfloat16).to(dev)
        x_gu = torch.randn(m, 2 * inter, generator=g).to(torch.bfloat16).to(dev)
        calls = []
        for i, layer in enumerate(self.layers):
            if self.backend == "bf16":
                a, p = layer.self_attn, layer.mlp
                calls += [(a.q_proj, x_h), (a.k_proj, x_h), (a.v_proj, x_h), (a.o_proj, x_h),
                          (p.gate_proj, x_h), (p.up_proj, x_h), (SiluMul(p.act_fn), x_gu),
                          (p.down_proj, x_i)]
            else:
                d = self.int8[i]
                calls += [(d["qkv"], x_h), (d["o"], x_h), (d["gate_up"], x_h), (d["down"], x_i)]
        return calls

    def linear_bytes(self, m: int) -> int:
        """Algorithmic bytes of the step's projections (weights, scales, activations in and
        out), excluding lm_head."""
        total = 0
        for mod, x in self.linear_calls(m):
            k = x.shape[-1]
            if isinstance(mod, Int8GateUp):  # both weights in, the SiLU-mul product out
                n = 2 * mod.intermediate_size
                total += k * n + 4 * n + 2 * m * k + 2 * m * (n // 2)
            elif isinstance(mod, SiluMul):  # (M, 2I) in, (M, I) out
                total += 2 * m * k + m * k
            elif isinstance(mod, Int8Linear):
                n = mod.out_features
                total += k * n + 4 * n + 2 * m * k + 2 * m * n
            else:
                n = mod.out_features
                total += 2 * k * n + 2 * m * k + 2 * m * n
        return total


class SiluMul(nn.Module):
    """`act_fn(gate) * up` of LlamaMLP.forward (modeling_llama.py:175) on a stacked (..., 2I)
    [gate | up] input, as a separate call (the bf16 back end's activation between gate/up and
    down)."""

    def __init__(self, act_fn: nn.Module) -> None:
        super().__init__()
        self.act_fn = act_fn

    def forward(self, gu: torch.Tensor) -> torch.Tensor:
        i = gu.shape[-1] // 2
        return self.act_fn(gu[..., :i]) * gu[..., i:]


def _restate_f32(mode: str, x: torch.Tensor, q: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    """fp32 values an int8 projection rounds to bf16, restated in torch: W8A16 s[n]·Σ x·q (fp32
    products and sums); W8A8 sx = amax/127 per token, xq = clamp(rne(x/sx)), acc = Σ xq·q exact
    (an fp64 GEMM: integer sums below 2^53), then (acc·sx)·s."""
    xf = x.float()
    if mode == "int8":
        return (xf @ q.float().t()) * s
    amax = xf.abs().amax(-1, keepdim=True)
    sx = torch.where(amax > 0, amax / 127.0, torch.ones_like(amax))
    xq = torch.clamp(torch.round(xf / sx), -127, 127)
    acc = (xq.double() @ q.double().t()).float()
    return (acc * sx) * s


def restate(mod: nn.Module, x: torch.Tensor) -> torch.Tensor:
    """The eager torch restatement of an `Int8Linear` or `Int8GateUp` call on bf16 x (test and
    measurement only): the module's mode and rounding points, without the HIP kernels. Gate/up:
    h = bf16(silu(g)·u) from fp32 g and u, one rounding as in the fused kernel."""
    q, s = mod.unpacked_qweight(), mod.scales
    if isinstance(mod, Int8GateUp):
        gu = _restate_f32(mod.mode, x, q, s)
        inter = mod.intermediate_size
        return (torch.nn.functional.silu(gu[..., :inter]) * gu[..., inter:]).to(torch.bfloat16)
    return _restate_f32(mod.mode, x, q, s).to(torch.bfloat16)


def _int8(weight: torch.Tensor, mode: str) -> Int8Linear:
    lin = nn.Linear(weight.shape[1], weight.shape[0], bias=False, device=weight.device,
                    dtype=weight.dtype)
    lin.weight.data = weight
    return Int8Linear.from_linear(lin, mode)
