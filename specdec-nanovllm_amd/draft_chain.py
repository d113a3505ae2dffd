"""C5 workload: the draft model's k-step decode chain on this library's kernels.

A random-init Qwen3-0.6B-shaped decoder stack (28 layers, hidden 1024, 16 q /
8 kv heads of 128, intermediate 3072, vocab 151936, RMSNorm eps 1e-6, per-head
q/k RMSNorm, rotate-half RoPE with theta 1e6 — nanovllm/models/qwen3.py:14-216,
layers/layernorm.py, layers/rotary_embedding.py). Every linear (qkv, o, gate_up,
down and lm_head) is W8A16 per-channel int8, quantized once at construction
with ``layers.quant.quantize_weight``; the KV cache is bf16, paged in 256-token
blocks. Its ``ctx_len``-token context per sequence is prefilled from uniform
random token ids (``context="prefill"``): the same decoder stack runs over the
ids at positions 0 .. ctx_len-1 (the linears on the dequantized weights in
bf16, attention on this library's varlen causal prefill kernel) and its k / v
rows are written to the pages; ``context="randn"`` fills the pages with N(0,1)
values instead.

One draft step is the reference's batched single-token forward
(nanovllm/spec_decode/draft_proposer.py:493-510, :527-550): per sequence the
position is ``ctx_len + s``, the slot ``bt[pos // 256] * 256 + pos % 256`` and
the key count ``pos + 1``; the layers call ``store_kvcache``, paged decode
attention and the W8A16 linears of this library, and the next token is the
argmax of the logits (the greedy draft). The hot-path ops run on the gfx950
kernels. The neighbours of the path — RMSNorm (+ residual add), q/k norm +
RoPE and SiLU*mul — are plain eager torch (no torch.compile) with
``fused=False`` (the greedy argmax is this library's sampler in both forms:
torch's argmax over a 151936-wide row clears its reduction semaphores with a
memset, which a captured graph does not replay reliably), or this library's
fused neighbour kernels with ``fused=True``:
add + RMSNorm inside the projection that consumes it (qkv, gate_up, lm_head;
up to 16 rows at hidden 1024, two launches beyond), q/k norm + RoPE + store_kvcache in one
launch on the qkv output (the attention reads q through strides), SiLU*mul in
the gate_up projection's epilogue (one or two rows; the SiLU launch beyond),
the sampler's argmax; the embedding lookup stays a torch index.

``chain()`` runs ``k`` steps back to back, each feeding its tokens to the next,
on static buffers, so the whole chain can be captured in one HIP graph.
"""
from __future__ import annotations

import math

import torch

from . import ops
from .layers.quant import quantize_weight

QWEN3_06B = dict(layers=28, hidden=1024, heads=16, kv_heads=8, head_dim=128, inter=3072,
                 vocab=151936, theta=1e6, eps=1e-6)


class DraftChain:
    """Static-buffer k-step greedy draft decode for ``batch`` sequences."""

    def __init__(self, batch: int, *, ctx_len: int = 2048, k: int = 6, layers: int = 28,
                 hidden: int = 1024, heads: int = 16, kv_heads: int = 8, head_dim: int = 128,
                 inter: int = 3072, vocab: int = 151936, theta: float = 1e6, eps: float = 1e-6,
                 block_size: int = 256, seed: int = 0, device="cuda",
                 dtype: torch.dtype = torch.bfloat16, fused: bool = False,
                 context: str = "prefill"):
        self.B, self.ctx_len, self.k = batch, ctx_len, k
        self.fused = fused
        self.L, self.H, self.Hq, self.Hkv, self.D = layers, hidden, heads, kv_heads, head_dim
        self.I, self.V, self.eps, self.bs = inter, vocab, eps, block_size
        self.dev, self.dtype = torch.device(device), dtype
        self.scale = head_dim ** -0.5
        g = torch.Generator(device=self.dev)
        g.manual_seed(seed)

        def randn(*shape, std=0.02):
            return (torch.randn(shape, generator=g, device=self.dev) * std).to(dtype)

        def qlinear(n_out, n_in):
            q, s = quantize_weight(randn(n_out, n_in))
            return q, s

        self.embed = randn(vocab, hidden)
        self.layers = []
        qkv_out = (heads + 2 * kv_heads) * head_dim
        for _ in range(layers):
            self.layers.append(dict(
                in_norm=1.0 + randn(hidden, std=0.1), post_norm=1.0 + randn(hidden, std=0.1),
                q_norm=1.0 + randn(head_dim, std=0.1), k_norm=1.0 + randn(head_dim, std=0.1),
                qkv=qlinear(qkv_out, hidden), o=qlinear(hidden, heads * head_dim),
                gate_up=qlinear(2 * inter, hidden), down=qlinear(hidden, inter)))
        self.final_norm = 1.0 + randn(hidden, std=0.1)
        self.lm_head = qlinear(vocab, hidden)

        # RoPE cos/sin for the positions the chain touches (rotate-half layout)
        inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32,
                                                 device=self.dev) / head_dim))
        pos = torch.arange(ctx_len + k + 1, dtype=torch.float32, device=self.dev)
        freqs = pos[:, None] * inv_freq[None, :]
        self.cos, self.sin = freqs.cos(), freqs.sin()
        self.cos_sin = torch.cat((self.cos, self.sin), dim=-1).contiguous()  # [cos | sin]

        # paged KV cache: (2, layers, blocks, bs, Hkv, D), a synthetic prefilled
        # context of ctx_len rows per sequence; pages are a seeded shuffle
        self.pages_per_seq = math.ceil((ctx_len + k) / block_size)
        nblk = batch * self.pages_per_seq
        if context == "randn":
            self.kv = torch.randn((2, layers, nblk, block_size, kv_heads, head_dim),
                                  generator=g, device=self.dev).to(dtype)
        elif context == "prefill":
            self.kv = torch.zeros((2, layers, nblk, block_size, kv_heads, head_dim),
                                  device=self.dev, dtype=dtype)
        else:
            raise ValueError(f"unknown context: {context}")
        cg = torch.Generator().manual_seed(seed + 1)
        perm = torch.randperm(nblk, generator=cg).to(torch.int32)
        self.block_table = perm.view(batch, self.pages_per_seq).to(self.dev)
        if context == "prefill":
            ids = torch.randint(0, vocab, (batch, ctx_len), generator=cg).to(self.dev)
            self._prefill(ids)

        # per-step static metadata: positions, slots, key counts
        bt = perm.view(batch, self.pages_per_seq)
        p = torch.arange(k, dtype=torch.int64)[:, None] + ctx_len  # (k, 1)
        pos_k = p.expand(k, batch)
        blk = bt.gather(1, (pos_k // block_size).T.contiguous()).T  # (k, B)
        # row-contiguous (k, B): each step's row is handed to the kernels as is
        self.positions = pos_k.contiguous().to(self.dev)
        self.slots = (blk.to(torch.int64) * block_size + pos_k % block_size).to(torch.int32) \
            .contiguous().to(self.dev)
        self.ctx = (pos_k + 1).to(torch.int32).contiguous().to(self.dev)

        # static token buffers: tokens[0] = the last context token, tokens[s+1] = step s output
        self.tokens = torch.randint(0, vocab, (k + 1, batch), generator=cg).to(self.dev)
        # residual stream of the fused step: the norm fused into a projection
        # writes x + residual to the buffer the current residual is not in
        self._res = torch.empty((2, batch, hidden), device=self.dev, dtype=dtype)

    # -------------------------------------------------------------------- context
    @torch.no_grad()
    def _prefill(self, ids: torch.Tensor) -> None:
        """Prefill of the context: the decoder stack over ``ids`` (batch,
        ctx_len) at positions 0 .. ctx_len-1, its k / v rows written to the
        pages of every layer. Setup, not the measured path: the linears use the
        dequantized weights in bf16 (torch), attention the varlen causal prefill
        kernel on contiguous rows, one layer at a time."""
        B, C, Hq, Hkv, D = self.B, self.ctx_len, self.Hq, self.Hkv, self.D
        if C == 0:
            return
        from .layers.quant import dequantize_weight

        def lin(x, qw):
            return x @ dequantize_weight(*qw).to(self.dtype).T.contiguous()

        pos = torch.arange(C, device=self.dev).repeat(B)
        cos, sin = self.cos[pos], self.sin[pos]
        cu = torch.arange(0, (B + 1) * C, C, dtype=torch.int32, device=self.dev)
        bt = self.block_table.long()
        p = torch.arange(C, device=self.dev)
        slots = (bt[:, p // self.bs] * self.bs + p % self.bs).reshape(-1)  # (B*C,)
        h = self.embed[ids.reshape(-1)]
        residual = None
        for li, lw in enumerate(self.layers):
            if residual is None:
                residual = h
                x = self._rms(h, lw["in_norm"])
            else:
                x, residual = self._add_rms(h, residual, lw["in_norm"])
            q, kk, v = lin(x, lw["qkv"]).split([Hq * D, Hkv * D, Hkv * D], dim=-1)
            q = self._rope(self._rms(q.reshape(-1, Hq, D), lw["q_norm"]), cos, sin)
            kk = self._rope(self._rms(kk.reshape(-1, Hkv, D), lw["k_norm"]), cos, sin)
            v = v.reshape(-1, Hkv, D).contiguous()
            self.kv[0, li].view(-1, Hkv, D)[slots] = kk
            self.kv[1, li].view(-1, Hkv, D)[slots] = v
            o = ops.prefill_attention(q.contiguous(), kk.contiguous(), v, cu, cu, C, self.scale)
            h = lin(o.reshape(-1, Hq * D), lw["o"])
            x, residual = self._add_rms(h, residual, lw["post_norm"])
            gate, up = lin(x, lw["gate_up"]).chunk(2, dim=-1)
            h = lin(torch.nn.functional.silu(gate) * up, lw["down"])
            del q, kk, v, o, x, gate, up

    # ------------------------------------------------------------------ neighbours
    def _rms(self, x, w):
        xf = x.float()
        xf = xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + self.eps)
        return xf.to(x.dtype) * w

    def _add_rms(self, x, residual, w):
        xf = x.float() + residual.float()
        residual = xf.to(x.dtype)
        xf = xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + self.eps)
        return xf.to(x.dtype) * w, residual

    def _rope(self, x, cos, sin):
        x1, x2 = x.float().chunk(2, dim=-1)
        c, s = cos[:, None, :], sin[:, None, :]
        return torch.cat((x1 * c - x2 * s, x2 * c + x1 * s), dim=-1).to(x.dtype)

    # ----------------------------------------------------------------------- step
    def step(self, s: int) -> torch.Tensor:
        """Draft step s: reads tokens[s], writes tokens[s + 1], returns the logits."""
        if self.fused:
            return self._step_fused(s)
        B, Hq, Hkv, D = self.B, self.Hq, self.Hkv, self.D
        pos = self.positions[s]
        cos, sin = self.cos[pos], self.sin[pos]
        slots, ctx = self.slots[s], self.ctx[s]
        h = self.embed[self.tokens[s]]
        residual = None
        for li, lw in enumerate(self.layers):
            if residual is None:
                residual = h
                x = self._rms(h, lw["in_norm"])
            else:
                x, residual = self._add_rms(h, residual, lw["in_norm"])
            qkv = ops.w8a16_linear(x, *lw["qkv"])
            q, kk, v = qkv.split([Hq * D, Hkv * D, Hkv * D], dim=-1)
            q = self._rms(q.reshape(B, Hq, D), lw["q_norm"])
            kk = self._rms(kk.reshape(B, Hkv, D), lw["k_norm"])
            q, kk = self._rope(q, cos, sin), self._rope(kk, cos, sin)
            v = v.reshape(B, Hkv, D)
            kc, vc = self.kv[0, li], self.kv[1, li]
            o = ops.paged_attention(q, kc, vc, self.block_table, self.scale, context_lens=ctx,
                                    key=kk, value=v, slot_mapping=slots)  # store fused
            h = ops.w8a16_linear(o.reshape(B, Hq * D), *lw["o"])
            x, residual = self._add_rms(h, residual, lw["post_norm"])
            gu = ops.w8a16_linear(x, *lw["gate_up"])
            gate, up = gu.chunk(2, dim=-1)
            h = ops.w8a16_linear(torch.nn.functional.silu(gate) * up, *lw["down"])
        x, _ = self._add_rms(h, residual, self.final_norm)
        logits = ops.w8a16_linear(x, *self.lm_head)
        # the greedy argmax on this library's sampler (first index among ties,
        # as torch.argmax): torch's argmax over a vocabulary-wide row is a
        # multi-block reduction whose semaphores are cleared by a memset, and a
        # captured memset node is not reliable on graph replay here
        ops.sample(logits, out=self.tokens[s + 1])
        return logits

    def _step_fused(self, s: int) -> torch.Tensor:
        B, Hq, Hkv, D, eps = self.B, self.Hq, self.Hkv, self.D, self.eps
        pos, slots, ctx = self.positions[s], self.slots[s], self.ctx[s]
        h = self.embed[self.tokens[s]]
        residual, ping = None, 0
        for li, lw in enumerate(self.layers):
            # add + RMSNorm folded into the projection that consumes it
            if residual is None:
                residual = h
                qkv = ops.w8a16_rmsnorm_linear(h, lw["in_norm"], eps, *lw["qkv"])
            else:
                ro, ping = self._res[ping], ping ^ 1
                qkv = ops.w8a16_rmsnorm_linear(h, lw["in_norm"], eps, *lw["qkv"],
                                               residual=residual, residual_out=ro)
                residual = ro
            q = qkv[:, :Hq * D].view(B, Hq, D)
            kk = qkv[:, Hq * D:(Hq + Hkv) * D].view(B, Hkv, D)
            v = qkv[:, (Hq + Hkv) * D:].view(B, Hkv, D)
            # q/k-norm + RoPE + store_kvcache in one launch, then plain paged attention
            ops.qk_norm_rope(q, kk, pos, self.cos_sin, lw["q_norm"], lw["k_norm"], eps, v=v,
                             k_cache=self.kv[0, li], v_cache=self.kv[1, li], slot_mapping=slots)
            o = ops.paged_attention(q, self.kv[0, li], self.kv[1, li], self.block_table,
                                    self.scale, context_lens=ctx)
            h = ops.w8a16_linear(o.reshape(B, Hq * D), *lw["o"])
            ro, ping = self._res[ping], ping ^ 1
            # add + RMSNorm, gate_up and SiLU*mul in one launch (paired gate / up
            # rows) at one or two rows, then the plain down projection
            act = ops.w8a16_gate_up_silu(h, *lw["gate_up"], lw["post_norm"], eps,
                                         residual=residual, residual_out=ro)
            residual = ro
            h = ops.w8a16_linear(act, *lw["down"])
        logits = ops.w8a16_rmsnorm_linear(h, self.final_norm, eps, *self.lm_head,
                                          residual=residual)
        ops.sample(logits, out=self.tokens[s + 1])
        return logits

    def chain(self) -> None:
        for s in range(self.k):
            self.step(s)

    # ------------------------------------------- isolated parts (time shares)
    def attention_chain(self) -> None:
        """Only the attention part of every layer of every step (store_kvcache
        fused with paged attention), on static q / k / v of the step's shape."""
        if not hasattr(self, "_qkv_static"):
            g = torch.Generator(device=self.dev)
            g.manual_seed(7)
            self._qkv_static = (
                torch.randn((self.B, self.Hq, self.D), generator=g, device=self.dev).to(self.dtype),
                torch.randn((self.B, self.Hkv, self.D), generator=g, device=self.dev).to(self.dtype),
                torch.randn((self.B, self.Hkv, self.D), generator=g, device=self.dev).to(self.dtype))
        q, kk, v = self._qkv_static
        for s in range(self.k):
            for li in range(self.L):
                kc, vc = self.kv[0, li], self.kv[1, li]
                ops.paged_attention(q, kc, vc, self.block_table, self.scale,
                                    context_lens=self.ctx[s], key=kk, value=v,
                                    slot_mapping=self.slots[s])

    def gemv_chain(self) -> None:
        """Only the W8A16 linears of every step (4 per layer + lm_head), on static
        activations of the step's shape."""
        if not hasattr(self, "_act_static"):
            g = torch.Generator(device=self.dev)
            g.manual_seed(8)
            self._act_static = (
                torch.randn((self.B, self.H), generator=g, device=self.dev).to(self.dtype),
                torch.randn((self.B, self.Hq * self.D), generator=g, device=self.dev).to(self.dtype),
                torch.randn((self.B, self.I), generator=g, device=self.dev).to(self.dtype))
        xh, xo, xi = self._act_static
        for _ in range(self.k):
            for lw in self.layers:
                ops.w8a16_linear(xh, *lw["qkv"])
                ops.w8a16_linear(xo, *lw["o"])
                ops.w8a16_linear(xh, *lw["gate_up"])
                ops.w8a16_linear(xi, *lw["down"])
            ops.w8a16_linear(xh, *self.lm_head)

    # ----------------------------------------------------------------- accounting
    def step_bytes(self) -> int:
        """Algorithmic HBM bytes of one draft step: every int8 weight and scale
        once, the visible K/V rows of every layer, the embedding rows read."""
        w = 0
        for lw in self.layers:
            for name in ("qkv", "o", "gate_up", "down"):
                q, sc = lw[name]
                w += q.numel() + sc.numel() * sc.element_size()
        q, sc = self.lm_head
        w += q.numel() + sc.numel() * sc.element_size()
        kv = self.L * self.B * (self.ctx_len + 1) * self.Hkv * self.D * 2 * 2
        return w + kv + self.B * self.H * 2
