"""E2B-shaped decode step on the C ABI (host side of the hot path).

`Decoder` owns seeded synthetic weights (generated on the device), the f16 KV
caches and the work buffers of a Gemma-4-E2B-shaped decoder, and enqueues one
decode step in either of two forms:

* ``step_reference`` issues the per-key kernels in the order of the
  reference's encodeTransformerPass (src/engine.ts:1539-1625) and
  sampleNextTokenSubmit (src/engine.ts:1686-1717): rmsNorm, matmulQuant q/k/v,
  v_norm, fusedPerHeadNormRope q/k, kvCacheStore, attnScore, softmax,
  attnOutput, matmulQuant o, fusedNormAdd, rmsNorm, matmulQuant gate/up,
  geluMul, matmulQuant down, fusedNormAdd; then final rmsNorm, LM head,
  softcap, argmax. PLE stages and the embedding lookup are not part of the
  hot path and are not issued.
* ``step_fused`` computes the same step with the fused kernels (norm in the
  matvec prologue, gate/up with the GELU product epilogue, split-K
  flash-decode) and reads the position from device memory, so the whole step
  can be captured once in a HIP graph and replayed token after token.

Shapes follow the layer the benchmark is quoted on: hidden 1536, 8 query heads
and 1 KV head of dim 256, FFN 6144 (Q4_K q/k/v/o/gate/up, Q6_K down), tied
Q6_K LM head [262144 x 1536], softcap 30; layers {4,9,...,34} attend globally
(theta 1e6, proportional RoPE table), the rest use a 512-token window
(theta 1e4) (src/config/gemma4-e2b.ts:16-63).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np

from .device import Buffer, Context, splitmix64

Q4K_BYTES = 144
Q6K_BYTES = 210


@dataclass
class E2BShape:
    hidden: int = 1536
    n_q_heads: int = 8
    n_kv_heads: int = 1
    head_dim: int = 256
    ffn: int = 6144
    vocab: int = 262144
    n_layers: int = 35
    eps: float = 1e-6
    window: int = 512
    theta_local: float = 1e4
    theta_global: float = 1e6
    softcap: float = 30.0
    global_layers: tuple = (4, 9, 14, 19, 24, 29, 34)

    @property
    def q_dim(self) -> int:
        return self.n_q_heads * self.head_dim

    @property
    def kv_dim(self) -> int:
        return self.n_kv_heads * self.head_dim

    def is_global(self, il: int) -> bool:
        return il in self.global_layers

    def layer_weight_bytes(self) -> int:
        H, Q, KV, I = self.hidden, self.q_dim, self.kv_dim, self.ffn
        q4 = (Q * H + 2 * KV * H + H * Q + 2 * I * H) // 256 * Q4K_BYTES
        q6 = (H * I) // 256 * Q6K_BYTES
        return q4 + q6

    def lm_head_bytes(self) -> int:
        return self.vocab * self.hidden // 256 * Q6K_BYTES


@dataclass
class LayerWeights:
    wq: Buffer
    wk: Buffer
    wv: Buffer
    wo: Buffer
    wgate: Buffer
    wup: Buffer
    wdown: Buffer
    attn_norm: Buffer
    post_attn_norm: Buffer
    pre_ffn_norm: Buffer
    post_ffn_norm: Buffer
    q_norm: Buffer
    k_norm: Buffer
    k_cache: Buffer
    v_cache: Buffer


class Decoder:
    def __init__(self, ctx: Context, shape: Optional[E2BShape] = None, max_seq: int = 4096, seed: int = 0,
                 n_layers: Optional[int] = None, lm_head: bool = True):
        self.ctx = ctx
        self.s = shape or E2BShape()
        if n_layers is not None:
            self.s.n_layers = n_layers
        self.max_seq = max_seq
        self.seed = seed
        s = self.s
        self._tid = 0
        self.layers: List[LayerWeights] = []
        for il in range(s.n_layers):
            self.layers.append(LayerWeights(
                wq=self._q4k(s.q_dim, s.hidden), wk=self._q4k(s.kv_dim, s.hidden), wv=self._q4k(s.kv_dim, s.hidden),
                wo=self._q4k(s.hidden, s.q_dim), wgate=self._q4k(s.ffn, s.hidden), wup=self._q4k(s.ffn, s.hidden),
                wdown=self._q6k(s.hidden, s.ffn),
                attn_norm=self._f16(s.hidden), post_attn_norm=self._f16(s.hidden), pre_ffn_norm=self._f16(s.hidden),
                post_ffn_norm=self._f16(s.hidden), q_norm=self._f16(s.head_dim), k_norm=self._f16(s.head_dim),
                k_cache=ctx.zeros(max_seq * s.kv_dim, np.uint16), v_cache=ctx.zeros(max_seq * s.kv_dim, np.uint16)))
        self.final_norm = self._f16(s.hidden)
        self.lm_head = self._q6k(s.vocab, s.hidden) if lm_head else None
        # proportional RoPE divisor table: 1.0 on the first quarter of the pairs,
        # 1e30 (+Inf in f16) after (src/engine.ts:522-537)
        half = s.head_dim // 2
        table = np.where(np.arange(half) < half // 4, 1.0, 1e30).astype(np.float16)
        self.rope_freqs = ctx.from_numpy(table.view(np.uint16))
        f32 = np.float32
        self.hidden = ctx.empty(s.hidden, f32)
        self.hidden2 = ctx.empty(s.hidden, f32)
        self.normed = ctx.empty(s.hidden, f32)
        self.q = ctx.empty(s.q_dim, f32)
        self.k = ctx.empty(s.kv_dim, f32)
        self.v = ctx.empty(s.kv_dim, f32)
        self.attn = ctx.empty(s.q_dim, f32)
        self.o = ctx.empty(s.hidden, f32)
        self.gate = ctx.empty(s.ffn, f32)
        self.up = ctx.empty(s.ffn, f32)
        self.act = ctx.empty(s.ffn, f32)
        self.down = ctx.empty(s.hidden, f32)
        self.logits = ctx.empty(s.vocab, f32)
        self.scores = ctx.empty(s.n_q_heads * max_seq, f32)
        self.token = ctx.zeros(1, np.uint32)
        self.topk = ctx.empty(512, f32)
        self.pos = ctx.zeros(1, np.uint32)
        self.attn_params = []
        for il in range(s.n_layers):
            glob = s.is_global(il)
            self.attn_params.append(ctx.attn_fused_params(
                s.n_q_heads, s.n_kv_heads, s.head_dim, max_seq, 0 if glob else s.window, s.eps,
                s.theta_global if glob else s.theta_local, int(glob)))
        ws = max(max(ctx.attn_workspace_bytes(s.n_q_heads, s.n_kv_heads, s.head_dim, max_seq, w)
                     for w in (0, s.window)),
                 max(ctx.attn_fused_workspace_bytes(p) for p in self.attn_params))
        # split-K partials + arrival counters; zeroed once, the kernels keep the counters zeroed
        self.attn_ws = ctx.zeros(ws, np.uint8)
        ctx.fill_normal_f32(self.hidden, s.hidden, self._seed(), 0.0, 1.0)
        ctx.sync()

    # ---- synthetic weights -------------------------------------------------
    def _seed(self) -> int:
        self._tid += 1
        return splitmix64(self.seed, self._tid)

    def _q4k(self, M: int, N: int) -> Buffer:
        nb = M * N // 256
        b = self.ctx.alloc(nb * Q4K_BYTES)
        self.ctx.fill_q4k(b, nb, self._seed())
        return b

    def _q6k(self, M: int, N: int) -> Buffer:
        nb = M * N // 256
        b = self.ctx.alloc(nb * Q6K_BYTES)
        self.ctx.fill_q6k(b, nb, self._seed())
        return b

    def _f16(self, n: int) -> Buffer:
        b = self.ctx.empty(n, np.uint16)
        self.ctx.fill_normal_f16(b, n, self._seed(), 1.0, 0.1)
        return b

    def fill_kv(self, length: int, seed: int = 1) -> None:
        """Synthetic cached K/V ~ N(0,1) for positions [0, length)."""
        n = length * self.s.kv_dim
        for il, L in enumerate(self.layers):
            self.ctx.fill_normal_f16(L.k_cache, n, splitmix64(seed, 2 * il), 0.0, 1.0)
            self.ctx.fill_normal_f16(L.v_cache, n, splitmix64(seed, 2 * il + 1), 0.0, 1.0)

    def set_position(self, pos: int) -> None:
        self.pos.upload(np.array([pos], np.uint32))

    # ---- the reference's per-key sequence ----------------------------------
    def step_reference(self, position: int, sample: str = "argmax") -> None:
        c, s = self.ctx, self.s
        seq_len = position + 1
        for il, L in enumerate(self.layers):
            glob = s.is_global(il)
            theta = s.theta_global if glob else s.theta_local
            window = 0 if glob else s.window
            c.rmsNorm(self.hidden, L.attn_norm, self.normed, s.hidden, s.eps)
            c.matmulQuant(self.normed, L.wq, self.q, s.q_dim, s.hidden)
            c.matmulQuant(self.normed, L.wk, self.k, s.kv_dim, s.hidden)
            c.matmulQuant(self.normed, L.wv, self.v, s.kv_dim, s.hidden)
            c.perHeadRmsNormNoWeight(self.v, s.n_kv_heads, s.head_dim, s.eps)
            c.fusedPerHeadNormRope(self.q, L.q_norm, s.n_q_heads, s.head_dim, s.eps, position, theta, int(glob),
                                   self.rope_freqs)
            c.fusedPerHeadNormRope(self.k, L.k_norm, s.n_kv_heads, s.head_dim, s.eps, position, theta, int(glob),
                                   self.rope_freqs)
            c.kvCacheStore(self.k, self.v, L.k_cache, L.v_cache, s.n_kv_heads, s.head_dim, position, self.max_seq)
            c.attnScore(self.q, L.k_cache, self.scores, s.n_q_heads, s.n_kv_heads, s.head_dim, seq_len, 1.0, window)
            c.softmax(self.scores, s.n_q_heads, seq_len)
            c.attnOutput(self.scores, L.v_cache, self.attn, s.n_q_heads, s.n_kv_heads, s.head_dim, seq_len)
            c.matmulQuant(self.attn, L.wo, self.o, s.hidden, s.q_dim)
            c.fusedNormAdd(self.o, L.post_attn_norm, self.hidden, self.hidden2, s.hidden, s.eps)
            c.rmsNorm(self.hidden2, L.pre_ffn_norm, self.normed, s.hidden, s.eps)
            c.matmulQuantMR4(self.normed, L.wgate, self.gate, s.ffn, s.hidden)
            c.matmulQuantMR4(self.normed, L.wup, self.up, s.ffn, s.hidden)
            c.geluMul(self.gate, self.up, self.act, s.ffn)
            c.matmulQuant(self.act, L.wdown, self.down, s.hidden, s.ffn, "q6k")
            c.fusedNormAdd(self.down, L.post_ffn_norm, self.hidden2, self.hidden, s.hidden, s.eps)
        self._head(sample)

    def _head(self, sample: str) -> None:
        c, s = self.ctx, self.s
        if self.lm_head is None:
            return
        c.rmsNorm(self.hidden, self.final_norm, self.normed, s.hidden, s.eps)
        c.matmulQuant(self.normed, self.lm_head, self.logits, s.vocab, s.hidden, "q6k")
        c.logitSoftcap(self.logits, s.vocab, s.softcap)
        if sample == "argmax":
            c.argmax(self.logits, self.token, s.vocab)
        else:
            c.topk256(self.logits, self.topk, s.vocab)

    # ---- the fused MI355X step ----------------------------------------------
    def step_fused(self, sample: str = "argmax", advance: bool = True) -> None:
        """One token at position *pos (device), then pos += 1 on the device.

        Five launches per layer:
          1. [post-FFN norm-add of the previous layer ->] attn rmsNorm -> q/k/v matvecs
          2. q/k norm + RoPE, v_norm, KV row store, split-K attention (+ merge)
          3. o matvec
          4. post-attn norm-add -> pre-FFN rmsNorm -> gate/up matvecs -> GELU product
          5. down matvec (Q6_K)
        then the last post-FFN norm-add + final rmsNorm + LM head + softcap in
        one launch, and the argmax.
        """
        c, s = self.ctx, self.s
        for il, L in enumerate(self.layers):
            outs = [self.q, self.k, self.v]
            ws = [L.wq, L.wk, L.wv]
            rows = [s.q_dim, s.kv_dim, s.kv_dim]
            if il == 0:
                c.normAddMatmulSegments("q4k", self.hidden, L.attn_norm, None, None, None, ws, outs, rows,
                                        s.hidden, s.eps)
            else:
                prev = self.layers[il - 1]
                c.normAddMatmulSegments("q4k", self.down, prev.post_ffn_norm, self.hidden2, L.attn_norm,
                                        self.hidden, ws, outs, rows, s.hidden, s.eps)
            c.attnDecodeFused(self.q, self.k, self.v, L.q_norm, L.k_norm, self.rope_freqs, L.k_cache, L.v_cache,
                              self.attn, self.attn_params[il], self.attn_ws, self.pos)
            c.matmulQuant(self.attn, L.wo, self.o, s.hidden, s.q_dim)
            c.normAddGateUpGelu_q4k(self.o, L.post_attn_norm, self.hidden, L.pre_ffn_norm, L.wgate, L.wup,
                                    self.hidden2, self.act, s.ffn, s.hidden, s.eps)
            c.matmulQuant(self.act, L.wdown, self.down, s.hidden, s.ffn, "q6k")
        last = self.layers[-1]
        if self.lm_head is not None:
            c.normAddMatmulSegments("q6k", self.down, last.post_ffn_norm, self.hidden2, self.final_norm,
                                    self.hidden, [self.lm_head], [self.logits], [s.vocab], s.hidden, s.eps,
                                    softcap=s.softcap)
            if sample == "argmax":
                c.argmax(self.logits, self.token, s.vocab)
            else:
                c.topk256(self.logits, self.topk, s.vocab)
        else:
            c.fusedNormAdd(self.down, last.post_ffn_norm, self.hidden2, self.hidden, s.hidden, s.eps)
        if advance:
            c.advancePosition(self.pos, 1)

    def capture_fused(self, sample: str = "argmax"):
        self.ctx.graph_begin()
        try:
            self.step_fused(sample)
        finally:
            g = self.ctx.graph_end()
        return g

    def launches_per_step_fused(self) -> int:
        """Kernel launches of step_fused: 5 per layer (plus the attention merge
        kernel when the split count is too large to merge in-kernel), the head
        (1), argmax (2) and the position advance (1)."""
        return 5 * self.s.n_layers + (3 if self.lm_head is not None else 1) + 1
