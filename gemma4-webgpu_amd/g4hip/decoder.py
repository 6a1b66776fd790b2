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

``BatchDecoder`` runs the same layers for many sequences at once (ragged
continuous-batching decode): every matmul takes all sequences' activation
vectors through the matrix-core kernel (each weight tile read once per
step), and attention reads each sequence's K/V from a paged f16 pool
through a per-sequence page table.

Two layer layouts (src/config/gemma4-e2b.ts:16-63):

* the default ``E2BShape()`` repeats the layer the benchmark is quoted on:
  hidden 1536, 8 query heads and 1 KV head of dim 256, FFN 6144 (Q4_K
  q/k/v/o/gate/up, Q6_K down), tied Q6_K LM head [262144 x 1536], softcap 30;
  layers {4,9,...,34} attend globally (theta 1e6, proportional RoPE table),
  the rest use a 512-token window (theta 1e4);
* ``E2BShape.real()`` is Gemma-4-E2B's own layout on top of that: global
  layers have head dim 512 (of whose 256 RoPE pairs the table rotates the
  first 64), layers 15..34 have FFN 12288 and compute no K/V of their own:
  each reads the cache of the last of layers 0..14 of its attention kind
  (13 local, 14 global) (src/config/gemma4-e2b.ts:151-180,
  src/engine.ts:1149-1152 and 1541-1583).

With ``embed=True`` a step starts from the embedding row of the token the
previous step sampled (src/engine.ts:1505-1514 and 1720-1725: the argmax
result is copied into the embedding lookup's token): the device-side token
feeds the next step without a host round trip.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np

from ._lib import O_SHARES
from .device import Buffer, Context, splitmix64

Q4K_BYTES = 144
Q6K_BYTES = 210
BLOCK_BYTES = {"q4k": Q4K_BYTES, "q6k": Q6K_BYTES}
# the layer matrices and their default formats (Q4_K, the down projection Q6_K)
MATRICES = ("wq", "wk", "wv", "wo", "wgate", "wup", "wdown")
DEFAULT_TYPES = {"wq": "q4k", "wk": "q4k", "wv": "q4k", "wo": "q4k", "wgate": "q4k", "wup": "q4k", "wdown": "q6k"}


@dataclass
class E2BShape:
    hidden: int = 1536
    n_q_heads: int = 8
    n_kv_heads: int = 1
    head_dim: int = 256          # local layers (and global ones when head_dim_global is 0)
    ffn: int = 6144              # layers below n_unshared (all layers when ffn_shared is 0)
    vocab: int = 262144
    n_layers: int = 35
    eps: float = 1e-6
    window: int = 512
    theta_local: float = 1e4
    theta_global: float = 1e6
    softcap: float = 30.0
    global_layers: tuple = (4, 9, 14, 19, 24, 29, 34)
    head_dim_global: int = 0     # head dim of the global layers (0: head_dim)
    ffn_shared: int = 0          # FFN width of layers >= n_unshared (0: ffn)
    n_unshared: int = 0          # layers >= n_unshared read a producer's KV cache (0: every layer owns its cache)
    ple_dim: int = 0             # per-layer embedding width (0: no per-layer embeddings)

    @classmethod
    def real(cls, **kw) -> "E2BShape":
        """Gemma-4-E2B's layer layout (src/config/gemma4-e2b.ts:16-63)."""
        return cls(**{"head_dim_global": 512, "ffn_shared": 12288, "n_unshared": 15, "ple_dim": 256, **kw})

    @property
    def q_dim(self) -> int:
        """The widest layer's q width (buffer sizing)."""
        return self.n_q_heads * self.max_head_dim

    @property
    def kv_dim(self) -> int:
        return self.n_kv_heads * self.max_head_dim

    @property
    def max_head_dim(self) -> int:
        return max(self.head_dim, self.head_dim_global)

    @property
    def max_ffn(self) -> int:
        return max(self.ffn, self.ffn_shared)

    def is_global(self, il: int) -> bool:
        return il in self.global_layers

    def hd(self, il: int) -> int:
        """getHeadDim (src/types.ts:79-81)."""
        return self.head_dim_global if self.is_global(il) and self.head_dim_global else self.head_dim

    def q_dim_of(self, il: int) -> int:
        return self.n_q_heads * self.hd(il)

    def kv_dim_of(self, il: int) -> int:
        return self.n_kv_heads * self.hd(il)

    def ffn_of(self, il: int) -> int:
        """getIntermediateSize (src/types.ts:84-86)."""
        return self.ffn_shared if self.ffn_shared and self.n_unshared and il >= self.n_unshared else self.ffn

    def producer(self, il: int) -> int:
        """The layer whose KV cache layer `il` reads: itself below n_unshared,
        else the last unshared layer of its attention kind
        (computeKvProducerMap, src/config/gemma4-e2b.ts:159-180)."""
        if not self.n_unshared or il < self.n_unshared:
            return il
        same = [j for j in range(min(self.n_unshared, self.n_layers)) if self.is_global(j) == self.is_global(il)]
        if not same:
            raise ValueError(f"layer {il}: no unshared layer of its attention kind")
        return same[-1]

    def is_producer(self, il: int) -> bool:
        return self.producer(il) == il

    def layer_weight_bytes(self, il: int = 0) -> int:
        H, Q, KV, I = self.hidden, self.q_dim_of(il), self.kv_dim_of(il), self.ffn_of(il)
        kv = 2 * KV * H if self.is_producer(il) else 0
        q4 = (Q * H + kv + H * Q + 2 * I * H) // 256 * Q4K_BYTES
        q6 = (H * I) // 256 * Q6K_BYTES
        return q4 + q6

    def weight_bytes(self) -> int:
        """Bytes of every layer's matrices (the LM head apart)."""
        return sum(self.layer_weight_bytes(il) for il in range(self.n_layers))

    def lm_head_bytes(self) -> int:
        return self.vocab * self.hidden // 256 * Q6K_BYTES

    def ple_bytes(self) -> int:
        """Per-layer-embedding bytes one token reads: per_layer_model_proj
        (f16), its table row (Q5_K), every layer's inp_gate and proj (f16)."""
        if not self.ple_dim:
            return 0
        L, D, H = self.n_layers, self.ple_dim, self.hidden
        return L * D * H * 2 + L * 176 + L * 2 * D * H * 2


@dataclass
class LayerWeights:
    wq: Buffer
    wk: Optional[Buffer]   # None in a layer that reads a producer's cache
    wv: Optional[Buffer]
    wo: Buffer
    wgate: Buffer
    wup: Buffer
    wdown: Buffer
    attn_norm: Buffer
    post_attn_norm: Buffer
    pre_ffn_norm: Buffer
    post_ffn_norm: Buffer
    q_norm: Buffer
    k_norm: Optional[Buffer]
    k_cache: Buffer        # the producer's cache in a layer that reads one
    v_cache: Buffer
    qt: dict = field(default_factory=lambda: dict(DEFAULT_TYPES))  # matrix -> "q4k" / "q6k"
    # per-layer embedding stage (src/engine.ts:1608-1616): inp_gate [D x H],
    # proj [H x D], post_norm [H] (f16) and layer_output_scale (f16 [1])
    ple_gate: Optional[Buffer] = None
    ple_proj: Optional[Buffer] = None
    ple_post_norm: Optional[Buffer] = None
    ple_scale: Optional[Buffer] = None


def q4km_types(s: "E2BShape"):
    """A per-matrix format mix of the kind a Q4_K_M file holds: Q4_K
    everywhere except the v projection and the down projection of the first
    and last eighth of their layers and every third layer between, which are
    Q6_K (the k-quant recipe's "more bits" layers)."""
    prod = [il for il in range(s.n_layers) if s.is_producer(il)]

    def more_bits(i: int, n: int) -> bool:
        return i < n // 8 or i >= 7 * n // 8 or (i - n // 8) % 3 == 2

    def qt(il: int, name: str) -> str:
        if name == "wv" and il in prod and more_bits(prod.index(il), len(prod)):
            return "q6k"
        if name == "wdown" and more_bits(il, s.n_layers):
            return "q6k"
        return "q4k"
    return qt


def qkv_groups(L: "LayerWeights", outs, rows):
    """The q/k/v matrices of a layer grouped by format, in order: [(type,
    weights, outputs, rows)] (one launch per group)."""
    names = ("wq", "wk", "wv")[:len(outs)]
    groups = {}
    for nm, o, r in zip(names, outs, rows):
        groups.setdefault(L.qt[nm], ([], [], []))
        g = groups[L.qt[nm]]
        g[0].append(getattr(L, nm))
        g[1].append(o)
        g[2].append(r)
    return [(t, *g) for t, g in groups.items()]


class _SyntheticModel:
    """The model's weights on the device: seeded synthetic E2B-shaped weights
    generated there, or a GGUF file's tensors (`gguf`). Each producer layer's
    k_cache / v_cache is whatever `kv(il)` returns (dense caches or paged
    pools); a layer that reads a producer's cache holds that producer's
    buffers and has no k/v projections or k_norm. `wtypes(il, name)` picks
    each synthetic matrix's format ("q4k" / "q6k"; default Q4_K with a Q6_K
    down projection); a file's matrices keep the file's formats."""

    def _build_weights(self, ctx: Context, shape: Optional[E2BShape], n_layers: Optional[int], seed: int,
                       lm_head: bool, kv, embed: bool = False, wtypes=None, gguf=None) -> None:
        self.ctx = ctx
        self.s = shape or E2BShape()
        if n_layers is not None:
            self.s.n_layers = n_layers
        self.seed = seed
        s = self.s
        self._tid = 0
        self.layers: List[LayerWeights] = []
        for il in range(s.n_layers):
            prod = s.is_producer(il)
            if prod:
                kc, vc = kv(il)
            else:
                src = self.layers[s.producer(il)]
                kc, vc = src.k_cache, src.v_cache
            w = self._file_layer(gguf, il) if gguf is not None else self._synthetic_layer(il, wtypes)
            self.layers.append(LayerWeights(k_cache=kc, v_cache=vc, **w))
        if gguf is not None:
            self._file_globals(gguf, lm_head, embed)
            return
        self.final_norm = self._f16(s.hidden)
        self.lm_type = "q6k"
        self.lm_head = self._q6k(s.vocab, s.hidden) if lm_head else None
        self._synthetic_ple_globals()
        # the f16 token embedding table [vocab x hidden] (shaders/embedding_lookup.wgsl)
        self.embedding = None
        if embed:
            self.embedding = ctx.empty(s.vocab * s.hidden, np.uint16)
            ctx.fill_normal_f16(self.embedding, s.vocab * s.hidden, self._seed(), 0.0, 0.03)
        # proportional RoPE divisor table over the global layers' pairs: 1.0 on
        # the first quarter, 1e30 (+Inf in f16) after (src/engine.ts:522-537)
        half = s.hd(s.global_layers[0]) // 2 if s.global_layers else s.head_dim // 2
        table = np.where(np.arange(half) < half // 4, 1.0, np.inf).astype(np.float16)
        self.rope_freqs = ctx.from_numpy(table.view(np.uint16))

    def _synthetic_layer(self, il: int, wtypes) -> dict:
        s = self.s
        Q, KV, I, hd = s.q_dim_of(il), s.kv_dim_of(il), s.ffn_of(il), s.hd(il)
        prod = s.is_producer(il)
        qt = {nm: (wtypes(il, nm) if wtypes else DEFAULT_TYPES[nm]) for nm in MATRICES}
        mk = lambda nm, M, N: {"q4k": self._q4k, "q6k": self._q6k, "f16": self._f16w}[qt[nm]](M, N)  # noqa: E731
        return dict(
            wq=mk("wq", Q, s.hidden), wk=mk("wk", KV, s.hidden) if prod else None,
            wv=mk("wv", KV, s.hidden) if prod else None,
            wo=mk("wo", s.hidden, Q), wgate=mk("wgate", I, s.hidden), wup=mk("wup", I, s.hidden),
            wdown=mk("wdown", s.hidden, I),
            attn_norm=self._f16(s.hidden), post_attn_norm=self._f16(s.hidden), pre_ffn_norm=self._f16(s.hidden),
            post_ffn_norm=self._f16(s.hidden), q_norm=self._f16(hd), k_norm=self._f16(hd) if prod else None, qt=qt,
            **self._synthetic_ple_layer())

    def _synthetic_ple_layer(self) -> dict:
        s = self.s
        if not s.ple_dim:
            return {}
        D, H = s.ple_dim, s.hidden
        return dict(ple_gate=self._f16(D * H, 0.0, 0.03), ple_proj=self._f16(H * D, 0.0, 0.03),
                    ple_post_norm=self._f16(H), ple_scale=self._f16(2, 0.8, 0.1))

    def _synthetic_ple_globals(self) -> None:
        """per_layer_model_proj [L*D x H], per_layer_proj_norm [D] (f16) and
        the Q5_K per_layer_token_embd table [vocab x L blocks]."""
        s, ctx = self.s, self.ctx
        self.ple_model_proj = self.ple_proj_norm = self.ple_table = None
        if not s.ple_dim:
            return
        if s.ple_dim != 256:
            raise ValueError("per-layer embeddings need ple_dim 256 (one Q5_K block per layer)")
        L, D, H = s.n_layers, s.ple_dim, s.hidden
        self.ple_model_proj = self._f16(L * D * H, 0.0, 0.03)
        self.ple_proj_norm = self._f16(D)
        self.ple_table = ctx.alloc(s.vocab * L * 176)
        ctx.fill_q5k(self.ple_table, s.vocab * L, self._seed())

    # ---- weights from a GGUF file ---------------------------------------------
    # tensor names of a layer (src/engine.ts:59-70; blk.{i}.{name}.weight)
    _FILE_MATRICES = {"wq": "attn_q", "wk": "attn_k", "wv": "attn_v", "wo": "attn_output", "wgate": "ffn_gate",
                      "wup": "ffn_up", "wdown": "ffn_down"}
    _FILE_NORMS = {"attn_norm": "attn_norm", "post_attn_norm": "post_attention_norm", "pre_ffn_norm": "ffn_norm",
                   "post_ffn_norm": "post_ffw_norm", "q_norm": "attn_q_norm", "k_norm": "attn_k_norm"}

    def _file_matrix(self, g, name: str, M: int, N: int):
        from .gguf import MATVEC_TYPES, TYPE_NAMES
        t = g.tensor(name)
        if t.dims != (N, M):
            raise ValueError(f"{name}: dims {t.dims}, the layout needs ({N}, {M})")
        qt = MATVEC_TYPES.get(t.type)
        if qt is not None:
            return g.upload(self.ctx, name), qt
        # other formats become the reference's own f16 rows (tensorToF16,
        # src/engine.ts:570-579) and run through the f16 matvec
        if t.type in (0, 1, 30):
            return g.upload_f16(self.ctx, name), "f16"
        if t.type in (8, 13):
            raw = g.upload(self.ctx, name)
            out = self.ctx.empty(M * N, np.uint16)
            nblk = M * N // (32 if t.type == 8 else 256)
            self.ctx.dequantF16("q8_0" if t.type == 8 else "q5k", raw, nblk, out)
            self.ctx.sync()
            raw.free()
            return out, "f16"
        raise ValueError(f"{name}: {TYPE_NAMES.get(t.type, t.type)} matrices are not supported")

    def _file_vector(self, g, name: str, n: int):
        t = g.tensor(name)
        if t.n_elements != n:
            raise ValueError(f"{name}: {t.n_elements} elements, the layout needs {n}")
        return g.upload_f16(self.ctx, name)

    def _file_layer(self, g, il: int) -> dict:
        s = self.s
        Q, KV, I, hd = s.q_dim_of(il), s.kv_dim_of(il), s.ffn_of(il), s.hd(il)
        prod = s.is_producer(il)
        shapes = {"wq": (Q, s.hidden), "wk": (KV, s.hidden), "wv": (KV, s.hidden), "wo": (s.hidden, Q),
                  "wgate": (I, s.hidden), "wup": (I, s.hidden), "wdown": (s.hidden, I)}
        w, qt = {}, {}
        for nm in MATRICES:
            if nm in ("wk", "wv") and not prod:
                w[nm], qt[nm] = None, DEFAULT_TYPES[nm]
                continue
            w[nm], qt[nm] = self._file_matrix(g, f"blk.{il}.{self._FILE_MATRICES[nm]}.weight", *shapes[nm])
        for nm, fn in self._FILE_NORMS.items():
            if nm == "k_norm" and not prod:
                w[nm] = None
                continue
            w[nm] = self._file_vector(g, f"blk.{il}.{fn}.weight", hd if nm in ("q_norm", "k_norm") else s.hidden)
        w["qt"] = qt
        if s.ple_dim:  # src/engine.ts:63-69 (inp_gate, proj, post_norm, layer_output_scale)
            D, H = s.ple_dim, s.hidden
            w["ple_gate"] = self._file_f16_matrix(g, f"blk.{il}.inp_gate.weight", D, H)
            w["ple_proj"] = self._file_f16_matrix(g, f"blk.{il}.proj.weight", H, D)
            w["ple_post_norm"] = self._file_vector(g, f"blk.{il}.post_norm.weight", H)
            w["ple_scale"] = self._file_vector(g, f"blk.{il}.layer_output_scale.weight", 1)
        return w

    def _file_f16_matrix(self, g, name: str, M: int, N: int):
        t = g.tensor(name)
        if t.dims != (N, M):
            raise ValueError(f"{name}: dims {t.dims}, the layout needs ({N}, {M})")
        return g.upload_f16(self.ctx, name)

    def _file_globals(self, g, lm_head: bool, embed: bool) -> None:
        s, ctx = self.s, self.ctx
        self.final_norm = self._file_vector(g, "output_norm.weight", s.hidden)
        self.lm_head, self.lm_type, self.embedding = None, "q6k", None
        if lm_head or embed:
            name = "output.weight" if lm_head and "output.weight" in g else "token_embd.weight"
            head, self.lm_type = self._file_matrix(g, name, s.vocab, s.hidden)
            if lm_head:
                self.lm_head = head
            if embed:
                # the tied table: the lookup reads f16 rows (src/engine.ts:599-600)
                te, et = (head, self.lm_type) if name == "token_embd.weight" else \
                    self._file_matrix(g, "token_embd.weight", s.vocab, s.hidden)
                if et == "f16":  # already the f16 rows
                    self.embedding = te
                else:
                    self.embedding = ctx.empty(s.vocab * s.hidden, np.uint16)
                    ctx.dequantF16(et, te, s.vocab * s.hidden // 256, self.embedding)
                    if not lm_head or te is not head:
                        ctx.sync()
                        te.free()
        half = s.hd(s.global_layers[0]) // 2 if s.global_layers else s.head_dim // 2
        self.rope_freqs = self._file_vector(g, "rope_freqs.weight", half)
        self.ple_model_proj = self.ple_proj_norm = self.ple_table = None
        if s.ple_dim:  # src/engine.ts:71-77, 599-625, 626-700
            L, D = s.n_layers, s.ple_dim
            if D != 256:
                raise ValueError("per-layer embeddings need per_layer_input_dim 256")
            self.ple_model_proj = self._file_f16_matrix(g, "per_layer_model_proj.weight", L * D, s.hidden)
            self.ple_proj_norm = self._file_vector(g, "per_layer_proj_norm.weight", D)
            t = g.tensor("per_layer_token_embd.weight")
            if t.type != 13 or t.dims != (L * D, s.vocab):
                raise ValueError(f"per_layer_token_embd.weight: {t.type_name} {t.dims}, the layout needs Q5_K "
                                 f"({L * D}, {s.vocab})")
            self.ple_table = g.upload(ctx, "per_layer_token_embd.weight")

    # ---- synthetic weights -------------------------------------------------
    def _seed(self) -> int:
        self._tid += 1
        return splitmix64(self.seed, self._tid)

    def _q4k(self, M: int, N: int) -> Buffer:
        nb = M * N // 256
        b = self.ctx.alloc(nb * Q4K_BYTES)
        self.ctx.fill_q4k(b, nb, self._seed())
        return b

    def _f16w(self, M: int, N: int) -> Buffer:
        """f16 rows ~ N(0, 0.03) (a matrix the file stores in a format the
        matvecs do not read as blocks)."""
        return self._f16(M * N, 0.0, 0.03)

    def _q6k(self, M: int, N: int) -> Buffer:
        nb = M * N // 256
        b = self.ctx.alloc(nb * Q6K_BYTES)
        self.ctx.fill_q6k(b, nb, self._seed())
        return b

    def _rope_tables(self, rows: int) -> dict:
        """RoPE (cos, sin) of positions [0, rows), one table per layer kind: {is_global: table}."""
        s, out = self.s, {}
        self.rope_rows = rows
        for glob in (False, True):
            hd = (s.head_dim_global or s.head_dim) if glob else s.head_dim
            t = self.ctx.empty(rows * hd, np.float32)
            self.ctx.ropeTable(s.theta_global if glob else s.theta_local, int(glob), self.rope_freqs, hd, rows, t)
            out[glob] = t
        return out

    def _f16(self, n: int, mean: float = 1.0, std: float = 0.1) -> Buffer:
        b = self.ctx.empty(n, np.uint16)
        self.ctx.fill_normal_f16(b, n, self._seed(), mean, std)
        return b


class Decoder(_SyntheticModel):
    def __init__(self, ctx: Context, shape: Optional[E2BShape] = None, max_seq: int = 4096, seed: int = 0,
                 n_layers: Optional[int] = None, lm_head: bool = True, embed: bool = False, wtypes=None,
                 gguf=None):
        self.max_seq = max_seq
        self.fuse_qkv = True  # step_fused: q/k/v and the attention in one launch where the shape allows
        # step_fused: where q/k/v take that launch, its chunk merge moves into
        # the o projection (by groups of heads) and the gate/up prologue adds
        # the shares. Off by default: measured in one process on one device,
        # the step takes 1057 us against 1040 with the in-launch merge (the
        # shares the gate/up launch reads ahead of its weights, and the
        # heads launch, cost more than the merge they remove)
        self.heads_o = False
        self._build_weights(ctx, shape, n_layers, seed, lm_head,
                            lambda il: (ctx.zeros(max_seq * self.s.kv_dim_of(il), np.uint16),
                                        ctx.zeros(max_seq * self.s.kv_dim_of(il), np.uint16)), embed=embed,
                            wtypes=wtypes, gguf=gguf)
        s = self.s
        f32 = np.float32
        Q, I = s.q_dim, s.max_ffn
        self.hidden = ctx.empty(s.hidden, f32)
        self.hidden2 = ctx.empty(s.hidden, f32)
        self.normed = ctx.empty(s.hidden, f32)
        self.q = ctx.empty(Q, f32)
        self.k = ctx.empty(s.kv_dim, f32)
        self.v = ctx.empty(s.kv_dim, f32)
        self.attn = ctx.empty(Q, f32)
        self.o = ctx.empty(s.hidden, f32)
        # the o projection's shares by groups of heads (O_SHARES of them; room for one per head)
        self.o_parts = ctx.empty(max(O_SHARES, s.n_q_heads) * s.hidden, f32)
        self.gate = ctx.empty(I, f32)
        self.up = ctx.empty(I, f32)
        self.act = ctx.empty(I, f32)
        self.act_digits = ctx.empty(ctx.digits_bytes(I), np.uint8)  # `act` as the down launch reads it
        self.down = ctx.empty(s.hidden, f32)
        self.logits = ctx.empty(s.vocab, f32)
        self.scores = ctx.empty(s.n_q_heads * max_seq, f32)
        self.token = ctx.zeros(1, np.uint32)
        self.topk = ctx.empty(512, f32)
        self.pos = ctx.zeros(1, np.uint32)
        if s.ple_dim:
            LD = s.n_layers * s.ple_dim
            self.ple_projected = ctx.empty(LD, f32)   # per_layer_model_proj . embedding
            self.ple_inputs = ctx.empty(LD, f32)      # stage 1 output, every layer's slice
            self.ple_gate_out = ctx.empty(s.ple_dim, f32)
            self.ple_gated = ctx.empty(s.ple_dim, f32)
            self.ple_out = ctx.empty(s.hidden, f32)   # proj . gated
            self.ple_normed = ctx.empty(s.hidden, f32)
            self.hidden3 = ctx.empty(s.hidden, f32)   # the post-FFN residual the PLE tail adds to
        self.attn_params = []
        for il in range(s.n_layers):
            glob = s.is_global(il)
            self.attn_params.append(ctx.attn_fused_params(
                s.n_q_heads, s.n_kv_heads, s.hd(il), max_seq, 0 if glob else s.window, s.eps,
                s.theta_global if glob else s.theta_local, int(glob)))
        ws = max(max(ctx.attn_workspace_bytes(s.n_q_heads, s.n_kv_heads, s.hd(il), max_seq, w)
                     for il in range(s.n_layers) for w in (0, s.window)),
                 max(ctx.attn_fused_workspace_bytes(p) for p in self.attn_params))
        # split-K partials + arrival counters; zeroed once, the kernels keep the counters zeroed
        self.attn_ws = ctx.zeros(ws, np.uint8)
        # weights of the gate/up and down launches that follow each attention
        # launch, read into the L2 caches by that launch (the o projection's
        # 1.8 MB arrive in time on their own: measured no faster from L2)
        self.rope_cs = self._rope_tables(max_seq)
        self.warm = [([ctx.matmulWarmRegion("q4k", s.ffn_of(il), s.hidden, L.wgate),
                       ctx.matmulWarmRegion("q4k", s.ffn_of(il), s.hidden, L.wup)] if self._ffn_fused(L) else []) +
                     ([ctx.matmulWarmRegion(L.qt["wdown"], s.hidden, s.ffn_of(il), L.wdown)]
                      if L.qt["wdown"] != "f16" else [])
                     for il, L in enumerate(self.layers)]
        ctx.fill_normal_f32(self.hidden, s.hidden, self._seed(), 0.0, 1.0)
        ctx.sync()

    def fill_kv(self, length: int, seed: int = 1) -> None:
        """Synthetic cached K/V ~ N(0,1) for positions [0, length) of every
        cache (the producer layers')."""
        for il, L in enumerate(self.layers):
            if not self.s.is_producer(il):
                continue
            n = length * self.s.kv_dim_of(il)
            self.ctx.fill_normal_f16(L.k_cache, n, splitmix64(seed, 2 * il), 0.0, 1.0)
            self.ctx.fill_normal_f16(L.v_cache, n, splitmix64(seed, 2 * il + 1), 0.0, 1.0)

    def set_position(self, pos: int) -> None:
        self.pos.upload(np.array([pos], np.uint32))

    def set_token(self, token: int) -> None:
        self.token.upload(np.array([token], np.uint32))

    # ---- the reference's per-key sequence ----------------------------------
    def _ple_stage1(self) -> None:
        """PLE stage 1 (src/engine.ts:1516-1535) from the step's input vector
        and the device-side token."""
        c, s = self.ctx, self.s
        L, D = s.n_layers, s.ple_dim
        c.matmulF16(self.hidden, self.ple_model_proj, self.ple_projected, L * D, s.hidden)
        c.pleStage1Fuse(self.ple_projected, self.ple_proj_norm, self.ple_table, s.vocab, self.ple_inputs, L, D,
                        s.eps, tokens_dev=self.token)

    def step_reference(self, position: int, sample: str = "argmax") -> None:
        c, s = self.ctx, self.s
        seq_len = position + 1
        if self.embedding is not None:
            c.embeddingLookup(self.embedding, s.vocab, self.hidden, s.hidden, token_dev=self.token)
        if s.ple_dim:
            self._ple_stage1()
        for il, L in enumerate(self.layers):
            glob = s.is_global(il)
            theta = s.theta_global if glob else s.theta_local
            window = 0 if glob else s.window
            hd, Q, KV, I = s.hd(il), s.q_dim_of(il), s.kv_dim_of(il), s.ffn_of(il)
            prod = s.is_producer(il)
            c.rmsNorm(self.hidden, L.attn_norm, self.normed, s.hidden, s.eps)
            c.matmulQuant(self.normed, L.wq, self.q, Q, s.hidden, L.qt["wq"])
            if prod:
                c.matmulQuant(self.normed, L.wk, self.k, KV, s.hidden, L.qt["wk"])
                c.matmulQuant(self.normed, L.wv, self.v, KV, s.hidden, L.qt["wv"])
                c.perHeadRmsNormNoWeight(self.v, s.n_kv_heads, hd, s.eps)
            c.fusedPerHeadNormRope(self.q, L.q_norm, s.n_q_heads, hd, s.eps, position, theta, int(glob),
                                   self.rope_freqs)
            if prod:
                c.fusedPerHeadNormRope(self.k, L.k_norm, s.n_kv_heads, hd, s.eps, position, theta, int(glob),
                                       self.rope_freqs)
                c.kvCacheStore(self.k, self.v, L.k_cache, L.v_cache, s.n_kv_heads, hd, position, self.max_seq)
            c.attnScore(self.q, L.k_cache, self.scores, s.n_q_heads, s.n_kv_heads, hd, seq_len, 1.0, window)
            c.softmax(self.scores, s.n_q_heads, seq_len)
            c.attnOutput(self.scores, L.v_cache, self.attn, s.n_q_heads, s.n_kv_heads, hd, seq_len)
            c.matmulQuant(self.attn, L.wo, self.o, s.hidden, Q, L.qt["wo"])
            c.fusedNormAdd(self.o, L.post_attn_norm, self.hidden, self.hidden2, s.hidden, s.eps)
            c.rmsNorm(self.hidden2, L.pre_ffn_norm, self.normed, s.hidden, s.eps)
            for w, y, nm in ((L.wgate, self.gate, "wgate"), (L.wup, self.up, "wup")):
                if L.qt[nm] == "q4k":
                    c.matmulQuantMR4(self.normed, w, y, I, s.hidden)
                else:
                    c.matmulQuant(self.normed, w, y, I, s.hidden, L.qt[nm])
            c.geluMul(self.gate, self.up, self.act, I)
            c.matmulQuant(self.act, L.wdown, self.down, s.hidden, I, L.qt["wdown"])
            c.fusedNormAdd(self.down, L.post_ffn_norm, self.hidden2, self.hidden, s.hidden, s.eps)
            if s.ple_dim:  # PLE stage 2 (src/engine.ts:1608-1616)
                D = s.ple_dim
                c.matmulF16(self.hidden, L.ple_gate, self.ple_gate_out, D, s.hidden)
                c.pleGeluMul(self.ple_gate_out, self.ple_inputs, self.ple_gated, il * D, D)
                c.matmulF16(self.ple_gated, L.ple_proj, self.ple_out, s.hidden, D)
                c.rmsNorm(self.ple_out, L.ple_post_norm, self.ple_normed, s.hidden, s.eps)
                c.pleSkipScaleAdd(self.hidden, self.ple_normed, L.ple_scale, s.hidden)
        self._head(sample)

    def _head(self, sample: str) -> None:
        c, s = self.ctx, self.s
        if self.lm_head is None:
            return
        c.rmsNorm(self.hidden, self.final_norm, self.normed, s.hidden, s.eps)
        c.matmulQuant(self.normed, self.lm_head, self.logits, s.vocab, s.hidden, self.lm_type)
        c.logitSoftcap(self.logits, s.vocab, s.softcap)
        if sample == "argmax":
            c.argmax(self.logits, self.token, s.vocab)
        else:
            c.topk256(self.logits, self.topk, s.vocab)

    # ---- the fused MI355X step ----------------------------------------------
    def _layer_input(self, il: int):
        """The prologue that forms layer il's normalised input: (x, w1,
        residual, scale, w2). Layer 0 normalises the step's input; later
        layers add the previous layer's post-FFN output (or, with per-layer
        embeddings, its PLE tail) to the residual stream first."""
        L = self.layers[il]
        if il == 0:
            return self.hidden, L.attn_norm, None, None, None
        prev = self.layers[il - 1]
        if self.s.ple_dim:  # (h + norm(proj out)) * layer_output_scale
            return self.ple_out, prev.ple_post_norm, self.hidden3, prev.ple_scale, L.attn_norm
        return self.down, prev.post_ffn_norm, self.hidden2, None, L.attn_norm

    def _mv(self, qt: str, x, w, y, M: int, N: int) -> None:
        if qt == "f16":
            self.ctx.matmulF16(x, w, y, M, N)
        else:
            self.ctx.matmulQuant(x, w, y, M, N, qt)

    def _qkv_fused(self, groups) -> bool:
        """q/k/v through qkvAttnDecodeFusedWarm: every one of them Q4_K (one
        group), unless `fuse_qkv` is off."""
        return self.fuse_qkv and len(groups) == 1 and groups[0][0] == "q4k"

    @staticmethod
    def _ffn_fused(L) -> bool:
        """gate/up in one launch (Q4_K pair; the digit hand-off when down is Q6_K)."""
        return L.qt["wgate"] == "q4k" and L.qt["wup"] == "q4k"

    def _heads_path(self, il: int, groups) -> bool:
        """Layer il runs q/k/v + attention without the merge, the per-head
        merge + o projection, and the gate/up over the head shares: its q/k/v
        take the one launch (own K/V, Q4_K, hidden 1536, one KV head of 256,
        window <= 1024), its o is Q4_K over 8 heads and its gate/up is one
        Q4_K launch."""
        s, L = self.s, self.layers[il]
        return (self.heads_o and s.is_producer(il) and self._qkv_fused(groups) and L.qt["wo"] == "q4k"
                and self._ffn_fused(L) and s.n_q_heads == 8
                and self.ctx.qkv_attn_single_launch(self.attn_params[il], s.hidden, 3))

    def step_fused(self, sample: str = "argmax", advance: bool = True, warm: bool = True) -> None:
        """One token at position *pos (device), then pos += 1 on the device.

        Five launches per layer:
          1. [post-FFN norm-add of the previous layer ->] attn rmsNorm -> q/k/v matvecs
          2. q/k norm + RoPE (cos/sin from the per-theta table), v_norm, KV row
             store, split-K attention (+ merge)
          3. o matvec
          4. post-attn norm-add -> pre-FFN rmsNorm -> gate/up matvecs -> GELU product
             (also written as the digit block the down launch reads)
          5. down matvec (Q6_K) over those digits
        Where the shape allows (_heads_path), four: 1 and 2 in one launch
        whose attention workgroups store their chunk partials and end; the
        per-head chunk merge with the o projection by head (8 shares of o);
        4 with the shares added in head order; 5.
        then the last post-FFN norm-add + final rmsNorm + LM head + softcap in
        one launch; its workgroups also leave their argmax candidates (argmax
        sampling), which a one-workgroup launch reduces to the token and the
        position advance, or their per-residue top-k candidates (top-k
        sampling), which a second launch reduces to the 256 pairs. With `warm`, each attention launch also
        reads the gate/up and down weights of its layer into the L2 caches
        (on the CUs the attention leaves idle).
        A layer that reads a producer's cache projects q only, and its
        attention launch forms and stores no K/V row. With the embedding
        table, an embedding lookup of the device-side token (the previous
        step's sample) starts the step.

        Matrices held as f16 rows (a file's Q5_K, Q8_0, F16, BF16 or F32
        matrices) take the f16 matvec: their group's norm is formed by a
        launch of its own, and an f16 gate or up makes the FFN unfused
        (norm launch, two matvecs, GELU product); an f16 LM head is followed
        by the softcap and the argmax / top-k launches.
        """
        c, s = self.ctx, self.s
        H = s.hidden
        if self.embedding is not None:
            c.embeddingLookup(self.embedding, s.vocab, self.hidden, H, token_dev=self.token)
        if s.ple_dim:
            self._ple_stage1()
        for il, L in enumerate(self.layers):
            Q, KV, I = s.q_dim_of(il), s.kv_dim_of(il), s.ffn_of(il)
            prod = s.is_producer(il)
            outs, rows = ([self.q, self.k, self.v], [Q, KV, KV]) if prod else ([self.q], [Q])
            x, w1, res, scale, w2 = self._layer_input(il)
            groups = qkv_groups(L, outs, rows)
            warm_il = self.warm[il] if warm else []
            if self._heads_path(il, groups):
                # q/k/v + attention (chunk partials), per-head merge + o, gate/up over the shares, down
                c.qkvAttnDecodePartials(x, w1, res, scale, w2, None if il == 0 else self.hidden, groups[0][1], outs,
                                        H, s.eps, L.q_norm, L.k_norm, self.rope_freqs, L.k_cache, L.v_cache,
                                        self.attn_params[il], self.attn_ws, self.pos, warm_il,
                                        self.rope_cs[s.is_global(il)], self.rope_rows)
                c.attnHeadsMatmul_q4k(self.attn_ws, self.attn_params[il], self.pos, L.wo, self.o_parts, H)
                c.normAddPartsGateUpGeluDigits_q4k(self.o_parts, L.post_attn_norm, self.hidden, L.pre_ffn_norm,
                                                   L.wgate, L.wup, self.hidden2, self.act, self.act_digits, I, H,
                                                   s.eps)
                if L.qt["wdown"] == "q6k":
                    c.matmulQuantDigits_q6k(self.act_digits, L.wdown, self.down, H, I)
                else:
                    self._mv(L.qt["wdown"], self.act, L.wdown, self.down, H, I)
                if s.ple_dim:
                    self._ple_tail(il, L)
                continue
            if self._qkv_fused(groups):  # q/k/v and the attention block: one launch where the shape allows
                c.qkvAttnDecodeFusedWarm(x, w1, res, scale, w2, None if il == 0 else self.hidden, groups[0][1], outs,
                                         H, s.eps, L.q_norm, L.k_norm, self.rope_freqs, L.k_cache, L.v_cache,
                                         self.attn, self.attn_params[il], self.attn_ws, self.pos, warm_il,
                                         self.rope_cs[s.is_global(il)], self.rope_rows)
            else:
                # one launch per weight format among q/k/v; a later launch
                # recomputes the norm from the same inputs and writes no h_out
                for gi, (qt, ws, go, gr) in enumerate(groups):
                    h_out = None if gi or il == 0 else self.hidden
                    if qt == "f16":
                        c.batchPrepScale(x, 1, w1, res, scale, w2, h_out, self.normed, H, 1, s.eps)
                        for w, y, r in zip(ws, go, gr):
                            c.matmulF16(self.normed, w, y, r, H)
                    else:
                        c.normAddScaleMatmulSegments(qt, x, w1, res, scale, w2, h_out, ws, go, gr, H, s.eps)
                c.attnDecodeFusedWarm(self.q, self.k if prod else None, self.v if prod else None, L.q_norm,
                                      L.k_norm, self.rope_freqs, L.k_cache, L.v_cache, self.attn,
                                      self.attn_params[il], self.attn_ws, self.pos, warm_il,
                                      self.rope_cs[s.is_global(il)], self.rope_rows)
            self._mv(L.qt["wo"], self.attn, L.wo, self.o, H, Q)
            if self._ffn_fused(L):
                c.normAddGateUpGeluDigits_q4k(self.o, L.post_attn_norm, self.hidden, L.pre_ffn_norm, L.wgate, L.wup,
                                              self.hidden2, self.act, self.act_digits, I, H, s.eps)
            else:
                c.batchPrepScale(self.o, 1, L.post_attn_norm, self.hidden, None, L.pre_ffn_norm, self.hidden2,
                                 self.normed, H, 1, s.eps)
                self._mv(L.qt["wgate"], self.normed, L.wgate, self.gate, I, H)
                self._mv(L.qt["wup"], self.normed, L.wup, self.up, I, H)
                c.geluMul(self.gate, self.up, self.act, I)
            if L.qt["wdown"] == "q6k" and self._ffn_fused(L):
                c.matmulQuantDigits_q6k(self.act_digits, L.wdown, self.down, H, I)
            else:
                self._mv(L.qt["wdown"], self.act, L.wdown, self.down, H, I)
            if s.ple_dim:
                self._ple_tail(il, L)
        last = self.layers[-1]
        if s.ple_dim:
            # the last PLE tail on its own (one vector), then the head normalises it
            c.batchPrepScale(self.ple_out, 1, last.ple_post_norm, self.hidden3, last.ple_scale, None, self.hidden,
                             self.normed, H, 1, s.eps)
            x, w1, res, w2, h_out = self.hidden, self.final_norm, None, None, None
        else:
            x, w1, res, w2, h_out = self.down, last.post_ffn_norm, self.hidden2, self.final_norm, self.hidden
        if self.lm_head is None:
            if not s.ple_dim:
                c.fusedNormAdd(self.down, last.post_ffn_norm, self.hidden2, self.hidden, H, s.eps)
        elif self.lm_type == "f16":
            c.batchPrepScale(x, 1, w1, res, None, w2, h_out, self.normed, H, 1, s.eps)
            c.matmulF16(self.normed, self.lm_head, self.logits, s.vocab, H)
            c.logitSoftcap(self.logits, s.vocab, s.softcap)
            if sample == "argmax":
                if advance:
                    c.argmaxAdvance(self.logits, self.token, s.vocab, 1, self.pos, 1)
                    return
                c.argmax(self.logits, self.token, s.vocab)
            else:
                c.topk256(self.logits, self.topk, s.vocab)
        elif sample == "argmax":
            c.normAddMatmulArgmax(self.lm_type, x, w1, res, w2, h_out, self.lm_head, self.logits, s.vocab, H,
                                  self.token, s.eps, softcap=s.softcap, positions=self.pos if advance else None,
                                  delta=1)
            return
        else:
            c.normAddMatmulTopk(self.lm_type, x, w1, res, w2, h_out, self.lm_head, self.logits, s.vocab, H,
                                self.topk, s.eps, softcap=s.softcap)
        if advance:
            c.advancePosition(self.pos, 1)

    def _ple_tail(self, il: int, L) -> None:
        """Post-FFN norm-add -> inp_gate -> gelu * ple_inputs, then proj (the
        layer's per-layer-embedding tail, src/engine.ts:1608-1616)."""
        c, s = self.ctx, self.s
        D = s.ple_dim
        c.pleGate(self.down, L.post_ffn_norm, self.hidden2, self.hidden3, L.ple_gate, self.ple_inputs, 0, il * D,
                  self.ple_gated, D, s.hidden, s.eps)
        c.matmulF16(self.ple_gated, L.ple_proj, self.ple_out, s.hidden, D)

    def capture_fused(self, sample: str = "argmax", warm: bool = True):
        self.ctx.graph_begin()
        try:
            self.step_fused(sample, warm=warm)
        finally:
            g = self.ctx.graph_end()
        return g

    def launches_per_step_fused(self) -> int:
        """Kernel launches of step_fused with argmax sampling: 5 per layer (4
        where the q/k/v matvec and the attention share one launch; 6 where
        the attention takes a launch and a merge: a window longer than 1024
        positions), the head with its argmax
        candidates (1) and their reduction, which also advances the position
        (1), and the embedding lookup when there is a table; with per-layer
        embeddings 2 before the layers, 2 per layer and the last tail; more
        where a layer's matrices mix formats or are f16 rows."""
        s, n = self.s, 2 + (self.embedding is not None)
        if s.ple_dim:  # stage 1 (2), two per layer, the last tail (1)
            n += 3 + 2 * s.n_layers
        if self.lm_head is not None and self.lm_type == "f16":  # norm, matvec, softcap, two argmax stages
            n += 3
        for il, L in enumerate(self.layers):
            groups = qkv_groups(L, [0, 0, 0][:3 if s.is_producer(il) else 1], [0, 0, 0])
            if self._qkv_fused(groups) and self.ctx.qkv_attn_single_launch(self.attn_params[il], s.hidden,
                                                                          3 if s.is_producer(il) else 1):
                n += 4  # q/k/v with the attention block, o, gate/up, down
            else:
                n += 4 + (not self.ctx.attn_fused_single_launch(self.attn_params[il]))
                for qt, ws, _, _ in groups:
                    n += 1 + (len(ws) if qt == "f16" else 0)
            if not self._ffn_fused(L):
                n += 3  # norm, second matvec, GELU product
        return n


class BatchDecoder(_SyntheticModel):
    """Ragged multi-sequence decode: `num_seqs` sequences with their own cached
    lengths share one set of weights and, per layer, one paged f16 K/V pool.

    Pages are handed out on the host when the decoder is built: sequence i
    owns ceil((context_lens[i] + reserve) / page_size) pages, taken from a
    shuffled free list so that a sequence's pages are scattered over the
    pool, as they are after a serving loop has run a while. `seq_lens` holds
    every sequence's length on the device; a step appends one token to each
    sequence (seq_lens += 1) and may be captured once and replayed while the
    reserve lasts.

    The split-K matmuls leave their chunks' partial sums in per-purpose
    buffers; the next launch adds them in chunk order (the per-vector norm
    prologue, or the attention prologue), so no launch waits on another's
    workgroups and the step is deterministic.
    """

    def __init__(self, ctx: Context, context_lens, shape: Optional[E2BShape] = None, page_size: int = 16,
                 reserve: int = 64, seed: int = 0, n_layers: Optional[int] = None, lm_head: bool = True,
                 page_seed: int = 7, shared_pages: bool = False, embed: bool = False, wtypes=None, gguf=None):
        """shared_pages: every row reads and appends through one page list
        (the rows are tokens of one sequence: batched prefill). embed: an f16
        token table; each step starts from the embedding of every row's
        token in `tokens` (the previous step's sample, or the prompt)."""
        lens = np.asarray(context_lens, dtype=np.int64)
        if lens.ndim != 1 or lens.size == 0 or lens.size > 64 or np.any(lens < 0):
            raise ValueError("context_lens: 1..64 non-negative lengths")
        s0 = shape or E2BShape()
        self.B = int(lens.size)
        self.page_size = page_size
        self.shared_pages = shared_pages
        self.max_seq = int(lens.max()) + reserve
        self.max_pages = -(-self.max_seq // page_size)
        per_seq = [self.max_pages] if shared_pages else [-(-(int(L) + reserve) // page_size) for L in lens]
        self.num_pages = int(sum(per_seq))
        order = np.random.default_rng(page_seed).permutation(self.num_pages).astype(np.int32)
        table = np.full((self.B, self.max_pages), -1, np.int32)
        if shared_pages:
            table[:, :] = order[None, :self.max_pages]
        else:
            at = 0
            for i, n in enumerate(per_seq):
                table[i, :n] = order[at:at + n]
                at += n
        self.page_table_host = table
        self.lens_host = lens.astype(np.uint32)
        rows = self.num_pages * page_size
        self._build_weights(ctx, shape, n_layers, seed, lm_head,
                            lambda il: (ctx.zeros(rows * self.s.kv_dim_of(il), np.uint16),
                                        ctx.zeros(rows * self.s.kv_dim_of(il), np.uint16)), embed=embed,
                            wtypes=wtypes, gguf=gguf)
        s, B, f32 = self.s, self.B, np.float32
        self.page_table = ctx.from_numpy(table)
        self.seq_lens = ctx.from_numpy(self.lens_host)
        self.hidden = ctx.empty(B * s.hidden, f32)
        self.hidden2 = ctx.empty(B * s.hidden, f32)
        self.xn = ctx.empty(B * s.hidden, f32)        # normalised input of the next matmul
        self.xops = ctx.empty(ctx.batch_operand_bytes(s.hidden, B), np.uint8)  # its operand blocks
        self.ks_h = s.hidden // 256                    # most K chunks of a matmul over the hidden width
        self.ks_q = s.q_dim // 256                     # (over the widest layer's q / FFN width)
        self.ks_f = s.max_ffn // 256
        self.q_parts = ctx.empty(self.ks_h * B * s.q_dim, f32)
        self.k_parts = ctx.empty(self.ks_h * B * s.kv_dim, f32)
        self.v_parts = ctx.empty(self.ks_h * B * s.kv_dim, f32)
        self.q = ctx.empty(B * s.q_dim, f32)           # q after q_norm + RoPE
        self.attn = ctx.empty(B * s.q_dim, f32)
        # the attention output also as the o projection's operand blocks
        # (written by the attention's merge when a head is whole super-blocks)
        self.aops = ctx.empty(ctx.batch_operand_bytes(s.q_dim, B), np.uint8) if s.head_dim % 256 == 0 else None
        self.o_parts = ctx.empty(self.ks_q * B * s.hidden, f32)
        self.act = ctx.empty(B * s.max_ffn, f32)
        self.down_parts = ctx.empty(self.ks_f * B * s.hidden, f32)
        # the FFN product handed to the down projection as sub-block-scaled
        # operand blocks (a Q4_K gate/up pair over a Q6_K down)
        self.dops = (ctx.empty(ctx.batch_sub_operand_bytes(s.max_ffn, B), np.uint8)
                     if any(self._ffn_handoff(il) for il in range(s.n_layers)) else None)
        if any(not (L.qt["wgate"] == "q4k" and L.qt["wup"] == "q4k") for L in self.layers):
            self.gate_b = ctx.empty(B * s.max_ffn, f32)  # gate and up of a layer that does not pair them
            self.up_b = ctx.empty(B * s.max_ffn, f32)
        self.logits = ctx.empty(B * s.vocab, f32) if lm_head else None
        self.tokens = ctx.zeros(B, np.uint32)
        self.topk = ctx.empty(B * 512, f32)
        if s.ple_dim:
            LD = s.n_layers * s.ple_dim
            self.ple_projected = ctx.empty(B * LD, f32)
            self.ple_inputs = ctx.empty(B * LD, f32)
            self.ple_gated = ctx.empty(B * s.ple_dim, f32)
            self.ple_out = ctx.empty(B * s.hidden, f32)
            self.hidden3 = ctx.empty(B * s.hidden, f32)
        self.pro_params, self.attn_params = [], []
        for il in range(s.n_layers):
            glob = s.is_global(il)
            window = 0 if glob else s.window
            self.pro_params.append(ctx.paged_fused_params(
                B, s.n_q_heads, s.n_kv_heads, s.hd(il), page_size, self.max_pages, self.max_seq, self.num_pages,
                window, s.eps, s.theta_global if glob else s.theta_local, int(glob)))
            self.attn_params.append(ctx.paged_params(
                B, s.n_q_heads, s.n_kv_heads, s.hd(il), page_size, self.max_pages, self.max_seq, self.num_pages,
                1.0, window))
        # the attention block of each layer in one launch (g4_pagedAttnBlock),
        # except where the rows share pages (prefill), whose prologue must
        # append every row before the attention reads any
        # (its own workspace: its arrival counters stay zero between calls)
        self.block_attn = not shared_pages
        self.attn_ws = ctx.zeros(max(ctx.paged_workspace_bytes(p) for p in self.attn_params), np.uint8)
        self.block_ws = ctx.zeros(max(ctx.paged_block_workspace_bytes(p, self.ks_h) for p in self.pro_params),
                                  np.uint8)
        self.rope_cs = self._rope_tables(self.max_seq)
        ctx.fill_normal_f32(self.hidden, B * s.hidden, self._seed(), 0.0, 1.0)
        ctx.sync()

    def fill_kv(self, seed: int = 1) -> None:
        """Synthetic cached K/V ~ N(0,1) over every page of every pool (the producer layers')."""
        for il, L in enumerate(self.layers):
            if not self.s.is_producer(il):
                continue
            n = self.num_pages * self.page_size * self.s.kv_dim_of(il)
            self.ctx.fill_normal_f16(L.k_cache, n, splitmix64(seed, 2 * il), 0.0, 1.0)
            self.ctx.fill_normal_f16(L.v_cache, n, splitmix64(seed, 2 * il + 1), 0.0, 1.0)

    def set_lengths(self, lens) -> None:
        lens = np.asarray(lens, dtype=np.uint32)
        if lens.shape != (self.B,) or int(lens.max()) >= self.max_seq:
            raise ValueError("set_lengths: one length per sequence, below the reserved capacity")
        self.lens_host = lens
        self.seq_lens.upload(lens)

    def pool_row(self, seq: int, pos: int) -> int:
        """Pool row of sequence `seq`'s logical position `pos`."""
        return int(self.page_table_host[seq, pos // self.page_size]) * self.page_size + pos % self.page_size

    def kv_bytes_per_step(self) -> int:
        """K/V bytes one step reads: every sequence's window in every layer
        (lengths after the step's append)."""
        s, total = self.s, 0
        for il in range(s.n_layers):
            for L in self.lens_host:
                n = int(L) + 1
                if not s.is_global(il):
                    n = min(n, s.window)
                total += n * 2 * s.kv_dim_of(il) * 2
        return total

    def step(self, sample: str = "argmax", probe=None, head: bool = True) -> None:
        """One token for every sequence. Per layer:
          1. [sum of the previous down chunks -> post-FFN norm-add ->] attn rmsNorm
          2. q/k/v projections (split-K partial sums)
          3. attention prologue: q/k norm + RoPE, v_norm, K/V append into the pages
          4. paged split-K attention (+ merge, which also writes the o
             projection's operand blocks)
          5. o projection (partial sums)
          6. post-attn norm-add -> pre-FFN rmsNorm
          7. gate/up -> GELU product
          8. down projection (Q6_K, partial sums)
        then the last norm-add + final rmsNorm, the LM head + softcap, and the
        per-sequence argmax (or top-k 256).

        probe (tests): called as probe(stage, il, chunks) once the stage's
        launches are enqueued, so that a test can read the stage's buffers:
        "prep" (layer il's normalised input `xn` and residual `hidden`; il =
        n_layers for the final norm), "attn" (roped `q`, the appended K/V
        rows, `attn`), "ffn_in" (`hidden2` and `xn` after the post-attention
        norm-add), "ffn" (the down projection's `chunks` partial sums in
        `down_parts`), "head" (`logits`). Not for captured steps.

        head=False stops after the layers (no final norm, LM head or sample):
        a prefill chunk whose logits nobody reads (the reference's prefill
        forwards run no LM head either, src/engine.ts:1896-1900)."""
        c, s, B = self.ctx, self.s, self.B
        H = s.hidden
        if self.embedding is not None:
            c.embeddingLookupBatch(self.embedding, s.vocab, self.hidden, H, self.tokens, B)
        if s.ple_dim:  # PLE stage 1 for every row (src/engine.ts:1516-1535)
            LD = s.n_layers * s.ple_dim
            c.matmulF16(self.hidden, self.ple_model_proj, self.ple_projected, LD, H, B)
            c.pleStage1Fuse(self.ple_projected, self.ple_proj_norm, self.ple_table, s.vocab, self.ple_inputs,
                            s.n_layers, s.ple_dim, s.eps, tokens_dev=self.tokens, count=B)
        c.advanceSeqLens(self.seq_lens, B, 1)
        nd = 0
        for il, L in enumerate(self.layers):
            Q, KV, I = s.q_dim_of(il), s.kv_dim_of(il), s.ffn_of(il)
            prod = s.is_producer(il)
            if il == 0:
                c.batchPrep(self.hidden, 1, L.attn_norm, None, None, None, self.xn, H, B, s.eps, ops=self.xops)
            elif s.ple_dim:  # the previous layer's PLE tail: (h + norm(proj out)) * scale
                prev = self.layers[il - 1]
                c.batchPrepScale(self.ple_out, 1, prev.ple_post_norm, self.hidden3, prev.ple_scale, L.attn_norm,
                                 self.hidden, self.xn, H, B, s.eps, ops=self.xops)
            else:
                prev = self.layers[il - 1]
                c.batchPrep(self.down_parts, nd, prev.post_ffn_norm, self.hidden2, L.attn_norm, self.hidden,
                            self.xn, H, B, s.eps, ops=self.xops)
            if probe:
                probe("prep", il, 0)
            # a layer reading a producer's pool projects q only and appends no row
            outs = [self.q_parts, self.k_parts, self.v_parts] if prod else [self.q_parts]
            groups = qkv_groups(L, outs, [Q, KV, KV] if prod else [Q])
            # f16 rows write whole sums (one chunk), so the block formats then split K once too
            nq = 1 if any(g[0] == "f16" for g in groups) else 0
            for qt, ws, go, gr in groups:
                if qt == "f16":
                    for w, y, r in zip(ws, go, gr):
                        c.matmulF16(self.xn, w, y, r, H, B)
                    continue
                # a later format's launch takes the first one's K split (the
                # prologue adds one chunk count): its fewer rows never pick fewer
                k = c.matmulSegmentsBatchPartial(qt, self.xn, ws, go, gr, H, B, nq or self.ks_h, ops=self.xops)
                if nq and k != nq:
                    raise RuntimeError(f"layer {il}: q/k/v launches split K {nq} and {k} ways")
                nq = k
            ops = self.aops if s.hd(il) % 256 == 0 else None
            if self.block_attn:  # prologue and attention in one launch where the window allows
                c.pagedAttnBlock(self.q_parts, self.k_parts if prod else None, self.v_parts if prod else None, nq,
                                 L.q_norm, L.k_norm, self.rope_freqs, self.q, L.k_cache, L.v_cache, self.page_table,
                                 self.seq_lens, self.attn, self.pro_params[il], self.block_ws, ops=ops,
                                 rope_cs=self.rope_cs[s.is_global(il)], rope_rows=self.rope_rows)
            else:
                c.pagedAttnPrologue(self.q_parts, self.k_parts if prod else None, self.v_parts if prod else None, nq,
                                    L.q_norm, L.k_norm, self.rope_freqs, self.q, L.k_cache if prod else None,
                                    L.v_cache if prod else None, self.page_table, self.seq_lens, self.pro_params[il],
                                    self.rope_cs[s.is_global(il)], self.rope_rows)
                c.pagedAttnDecode(self.q, L.k_cache, L.v_cache, self.page_table, self.seq_lens, self.attn,
                                  self.attn_params[il], self.attn_ws, ops=ops)
            if probe:
                probe("attn", il, 0)
            no = self._mm_batch(L.qt["wo"], self.attn, L.wo, self.o_parts, H, Q, self.ks_q, ops)
            c.batchPrep(self.o_parts, no, L.post_attn_norm, self.hidden, L.pre_ffn_norm, self.hidden2, self.xn, H, B,
                        s.eps, ops=self.xops)
            if probe:
                probe("ffn_in", il, 0)
            if self._ffn_handoff(il):
                # the product goes to the down projection as operand blocks only;
                # K in chunks of 3 super-blocks (one workgroup per CU)
                c.gateUpGeluBatchOps(self.xn, self.xops, L.wgate, L.wup, None, self.dops, I, H, B)
                nd = c.matmulSubBatchPartial(self.dops, L.wdown, self.down_parts, H, I, B, I // 768)
            else:
                if L.qt["wgate"] == "q4k" and L.qt["wup"] == "q4k":
                    c.gateUpGeluBatch(self.xn, L.wgate, L.wup, self.act, I, H, B, ops=self.xops)
                else:  # gate and up apart (whole sums), then the GELU product
                    self._mm_batch(L.qt["wgate"], self.xn, L.wgate, self.gate_b, I, H, 1, self.xops)
                    self._mm_batch(L.qt["wup"], self.xn, L.wup, self.up_b, I, H, 1, self.xops)
                    c.geluMul(self.gate_b, self.up_b, self.act, B * I)
                nd = self._mm_batch(L.qt["wdown"], self.act, L.wdown, self.down_parts, H, I, self.ks_f, None)
            if probe:
                probe("ffn", il, nd)
            if s.ple_dim:
                # post-FFN norm-add (h, no second norm) -> inp_gate -> gelu * ple_inputs -> proj
                D = s.ple_dim
                c.batchPrepScale(self.down_parts, nd, L.post_ffn_norm, self.hidden2, None, None, None, self.hidden3,
                                 H, B, s.eps)
                c.pleGate(self.hidden3, None, None, None, L.ple_gate, self.ple_inputs, s.n_layers * D, il * D,
                          self.ple_gated, D, H, s.eps, batch=B)
                c.matmulF16(self.ple_gated, L.ple_proj, self.ple_out, H, D, B)
        if not head:
            self.lens_host = self.lens_host + 1
            return
        last = self.layers[-1]
        if s.ple_dim:
            c.batchPrepScale(self.ple_out, 1, last.ple_post_norm, self.hidden3, last.ple_scale, self.final_norm,
                             self.hidden, self.xn, H, B, s.eps, ops=self.xops)
        else:
            c.batchPrep(self.down_parts, nd, last.post_ffn_norm, self.hidden2, self.final_norm, self.hidden, self.xn,
                        H, B, s.eps, ops=self.xops)
        if probe:
            probe("prep", s.n_layers, 0)
        if self.lm_head is not None:
            if self.lm_type == "f16":
                c.matmulF16(self.xn, self.lm_head, self.logits, s.vocab, H, B)
                c.logitSoftcap(self.logits, B * s.vocab, s.softcap)
            else:
                c.matmulSegmentsBatchPartial(self.lm_type, self.xn, [self.lm_head], [self.logits], [s.vocab], H, B,
                                             1, ops=self.xops, softcap=s.softcap)
            if sample == "argmax":
                c.argmaxBatch(self.logits, self.tokens, s.vocab, B)
            else:
                c.topk256Batch(self.logits, self.topk, s.vocab, B)
            if probe:
                probe("head", s.n_layers, 0)
        self.lens_host = self.lens_host + 1

    def _ffn_handoff(self, il: int) -> bool:
        """Layer il's gate/up launch hands its product to the down projection
        as sub-block-scaled operand blocks: a Q4_K gate/up pair, a Q6_K down,
        FFN width 6144 or 12288."""
        L = self.layers[il]
        return (L.qt["wgate"] == "q4k" and L.qt["wup"] == "q4k" and L.qt["wdown"] == "q6k"
                and self.s.ffn_of(il) in (6144, 12288))

    def _mm_batch(self, qt: str, x, w, y, M: int, N: int, max_ksplit: int, ops) -> int:
        """y = W . x for the B rows: f16 rows through the f16 matvec (one
        chunk), block formats split-K into at most max_ksplit chunks. Returns
        the chunk count."""
        if qt == "f16":
            self.ctx.matmulF16(x, w, y, M, N, self.B)
            return 1
        return self.ctx.matmulSegmentsBatchPartial(qt, x, [w], [y], [M], N, self.B, max_ksplit, ops=ops)

    def prefill(self, tokens, start: int = 0, sample: str = "argmax", probe=None) -> int:
        """Batched prefill of one sequence (a shared_pages decoder with an
        embedding table): the prompt's tokens at positions start, start + 1,
        ... go through the layers B at a time, each chunk one step of the
        ragged path in which row r embeds its token, appends its K/V row at
        its own position and attends to the positions up to it (the
        prologue launch appends every row of the chunk before the attention
        launch reads them, so the chunk is causal). The reference runs one
        full forward per prompt token instead (src/engine.ts:1923-1938) and
        samples from the last one (src/engine.ts:2014-2017); as there, only
        the last chunk runs the LM head. A short last
        chunk repeats its last token and position in the spare rows
        (identical rows, identical writes). Returns the row of the final
        chunk that holds the prompt's last token: its logits and `tokens`
        entry are the first sample. probe (tests): passed to every chunk's
        step."""
        if not self.shared_pages or self.embedding is None:
            raise ValueError("prefill needs a shared_pages decoder with an embedding table")
        toks = np.asarray(tokens, np.uint32)
        T, B = int(toks.size), self.B
        if T == 0 or start + T > self.max_seq - 1:
            raise ValueError(f"prefill: {T} tokens from {start} do not fit {self.max_seq} positions")
        nch = -(-T // B)
        n = T - (nch - 1) * B
        pad = nch * B - T
        # every chunk's tokens and lengths (before the step appends each row)
        # uploaded once; the chunks then run back to back on the stream
        ctok = np.concatenate([toks, np.repeat(toks[-1], pad)]).astype(np.uint32)
        cpos = np.concatenate([start + np.arange(T), np.repeat(start + T - 1, pad)]).astype(np.uint32)
        dtok, dpos = self.ctx.from_numpy(ctok), self.ctx.from_numpy(cpos)
        for k in range(nch):
            self.ctx.copy(self.tokens, dtok.offset(4 * B * k), 4 * B)
            self.ctx.copy(self.seq_lens, dpos.offset(4 * B * k), 4 * B)
            self.lens_host = cpos[B * k:B * (k + 1)].copy()
            self.step(sample, probe=probe, head=k == nch - 1)
        self.ctx.sync()
        dtok.free()
        dpos.free()
        return n - 1

    def capture(self, sample: str = "argmax"):
        """The step as a HIP graph; each replay appends one token per sequence."""
        lens = self.lens_host.copy()
        self.ctx.graph_begin()
        try:
            self.step(sample)
        finally:
            g = self.ctx.graph_end()
        self.lens_host = lens  # capture enqueues nothing
        return g


def open_gguf(path_or_file, max_context_length: Optional[int] = None, n_layers: Optional[int] = None):
    """(GGUFFile, configFromGGUF result, decoder layout) of a Gemma 4 GGUF;
    the layout's vocabulary is the token table's row count."""
    from .gguf import GGUFFile, config_from_gguf, shape_from_config
    g = path_or_file if isinstance(path_or_file, GGUFFile) else GGUFFile(str(path_or_file))
    cfg = config_from_gguf(g, max_context_length)
    emb = g.find("token_embd.weight")
    shape = shape_from_config(cfg, vocab=emb.dims[1] if emb is not None and len(emb.dims) == 2 else None)
    # per-layer embeddings when the file carries their table (Gemma 4 E2B does)
    shape.ple_dim = cfg["per_layer_input_dim"] if "per_layer_token_embd.weight" in g else 0
    if n_layers is not None:
        shape.n_layers = n_layers
    return g, cfg, shape


def decoder_from_gguf(ctx: Context, path_or_file, max_seq: Optional[int] = None, batch=None, **kw):
    """A Decoder (batch None) or BatchDecoder (batch = the context lengths)
    holding a GGUF file's weights: the layer matrices as the file's Q4_K /
    Q6_K blocks, norms and the RoPE table as f16, the tied token table as
    the LM head's blocks and (embed=True, the default) the lookup's f16
    rows. max_seq defaults to the file's context length capped at 2048 (as
    configFromGGUF)."""
    g, cfg, shape = open_gguf(path_or_file, max_seq, kw.pop("n_layers", None))
    kw.setdefault("embed", True)
    if batch is None:
        return Decoder(ctx, shape, max_seq=max_seq or cfg["context_length"], gguf=g, **kw)
    return BatchDecoder(ctx, batch, shape, gguf=g, **kw)
