"""Oracle composition of one E2B-shaped decode step for one sequence (the
order of src/engine.ts:1539-1625 and the head of src/engine.ts:1686-1717),
over weights downloaded once from a decoder's device buffers."""
import numpy as np

import oracle as O
from g4hip.decoder import DEFAULT_TYPES


def gelu_mul_f32(gate, up):
    """shaders/gelu_mul.wgsl:10-16 evaluated in f32 operations in the shader's
    order (tanh correctly rounded to f32): another faithful evaluation of the
    reference, used to measure how sensitive a step is to the last bits of
    the GELU (the oracle's gelu_mul forms the tanh argument in f64)."""
    x = np.asarray(gate, np.float32)
    f = np.float32
    t = np.clip(f(0.7978845608028654) * x * (f(1.0) + f(0.044715) * x * x), f(-15.0), f(15.0))
    th = np.tanh(t.astype(np.float64)).astype(np.float32)
    return (f(0.5) * x * (f(1.0) + th) * np.asarray(up, np.float32)).astype(np.float32)


def f16_toward_zero(x):
    """f32 -> f16 bits rounded toward zero: one f16 ulp from round-to-nearest
    wherever that rounded away from zero."""
    x = np.asarray(x, np.float32)
    with np.errstate(over="ignore"):
        h = x.astype(np.float16)
    bits = h.view(np.uint16).copy()
    away = np.abs(h.astype(np.float32)) > np.abs(x)
    bits[away] -= 1
    return bits


class HostModel:
    """A decoder's weights on the host. Layers that read a producer's cache
    (no k/v projections) index the producer's entry of the cache lists the
    step is given (src/engine.ts:1149-1152)."""

    def __init__(self, dec):
        self.s = s = dec.s
        u8, u16 = np.uint8, np.uint16
        self.table = dec.rope_freqs.download(u16)
        self.layers = []
        for L in dec.layers:
            self.layers.append({k: getattr(L, k).download(u8 if k.startswith("w") else u16)
                                for k in ("wq", "wk", "wv", "wo", "wgate", "wup", "wdown", "attn_norm",
                                          "post_attn_norm", "pre_ffn_norm", "post_ffn_norm", "q_norm", "k_norm",
                                          "ple_gate", "ple_proj", "ple_post_norm", "ple_scale")
                                if getattr(L, k, None) is not None})
        # per-layer embeddings: the projection and its norm on the host, the
        # Q5_K table's rows fetched per token
        self.ple = None
        if s.ple_dim:
            self.ple = dict(model_proj=dec.ple_model_proj.download(u16), proj_norm=dec.ple_proj_norm.download(u16),
                            table=dec.ple_table)
        self.qt = [dict(getattr(L, "qt", DEFAULT_TYPES)) for L in dec.layers]  # each matrix's format
        for W, qt in zip(self.layers, self.qt):  # f16 rows as f16 bits
            for k, t in qt.items():
                if t == "f16" and k in W:
                    W[k] = W[k].view(np.uint16)
        self.final_norm = dec.final_norm.download(u16)
        self.lm_type = getattr(dec, "lm_type", "q6k")
        self.lm_head = dec.lm_head.download(u8) if dec.lm_head is not None else None
        if self.lm_head is not None and self.lm_type == "f16":
            self.lm_head = self.lm_head.view(np.uint16)
        self.embedding = getattr(dec, "embedding", None)  # device table: rows are fetched on demand

    def embed(self, token: int):
        """shaders/embedding_lookup.wgsl for one token (the oracle's embedding_lookup on its row)."""
        H = self.s.hidden
        row = self.embedding.download(np.uint16, H, offset=int(token) * H * 2)
        return O.embedding_lookup(row.view(np.float16), H, 0)

    def ple_inputs(self, x0, token: int):
        """PLE stage 1 (src/engine.ts:1516-1535) for the step's input vector:
        per_layer_model_proj . x0, then shaders/ple_stage1_fuse.wgsl per layer
        over the token's table row, dequantized (src/gguf.ts:218-257) and
        rounded to f16 as the reference uploads it."""
        s = self.s
        L, D = s.n_layers, s.ple_dim
        blocks = self.ple["table"].download(np.uint8, L * 176, offset=int(token) * L * 176)
        row = O.dequant_q5k(blocks).astype(np.float16).view(np.uint16)
        return O.ple_project(x0, self.ple["model_proj"], self.ple["proj_norm"], row, L, D, s.eps)

    def step(self, hidden, kcs, vcs, pos, gelu=O.gelu_mul, row_toward_zero=False, token=0, rows=None):
        """Decode position `pos`: kcs/vcs are this sequence's dense f16 caches
        (one per layer, >= pos + 1 rows; a consumer layer's entry is not
        used), updated in place. Returns the new hidden state and the
        softcapped logits (None without an LM head). `row_toward_zero`
        stores the new K/V rows rounded toward zero instead of to nearest (a
        one-ulp change of the f16 cache, to measure how much the step depends
        on the cache's resolution). `token` picks the per-layer-embedding
        table row. `rows`, a dict, receives each producer layer's new K and V
        rows in f32, before the cache's f16 rounding."""
        s, x = self.s, hidden.copy()
        pin = self.ple_inputs(x, token) if self.ple is not None else None
        for il, W in enumerate(self.layers):
            glob = s.is_global(il)
            theta = s.theta_global if glob else s.theta_local
            window = 0 if glob else s.window
            hd, Q, KV, I = s.hd(il), s.q_dim_of(il), s.kv_dim_of(il), s.ffn_of(il)
            src = s.producer(il)
            qt = self.qt[il]
            n = O.rms_norm(x, W["attn_norm"], s.eps)
            q = O.matmul(n, W["wq"], Q, s.hidden, qt["wq"])
            q = O.fused_per_head_norm_rope(q, W["q_norm"], s.n_q_heads, hd, s.eps, pos, theta, int(glob), self.table)
            if src == il:
                k = O.matmul(n, W["wk"], KV, s.hidden, qt["wk"])
                v = O.matmul(n, W["wv"], KV, s.hidden, qt["wv"])
                v = O.per_head_rms_norm_no_weight(v, s.n_kv_heads, hd, s.eps)
                k = O.fused_per_head_norm_rope(k, W["k_norm"], s.n_kv_heads, hd, s.eps, pos, theta, int(glob),
                                               self.table)
                O.kv_cache_store_f16(k, v, kcs[il], vcs[il], s.n_kv_heads, hd, pos)
                if rows is not None:
                    rows[il] = (np.asarray(k, np.float32).copy(), np.asarray(v, np.float32).copy())
                if row_toward_zero:
                    row = slice(pos * KV, (pos + 1) * KV)
                    kcs[il][row] = f16_toward_zero(k)
                    vcs[il][row] = f16_toward_zero(v)
            a = O.attention(q, kcs[src], vcs[src], s.n_q_heads, s.n_kv_heads, hd, pos + 1, 1.0, window)
            o = O.matmul(a, W["wo"], s.hidden, Q, qt["wo"])
            h = O.fused_norm_add(o, W["post_attn_norm"], x, s.eps)
            n2 = O.rms_norm(h, W["pre_ffn_norm"], s.eps)
            g = O.matmul(n2, W["wgate"], I, s.hidden, qt["wgate"])
            u = O.matmul(n2, W["wup"], I, s.hidden, qt["wup"])
            dn = O.matmul(gelu(g, u), W["wdown"], s.hidden, I, qt["wdown"])
            x = O.fused_norm_add(dn, W["post_ffn_norm"], h, s.eps)
            if pin is not None:  # PLE stage 2 (src/engine.ts:1608-1616)
                D = s.ple_dim
                x = O.ple_layer_tail(x, W["ple_gate"], W["ple_proj"], W["ple_post_norm"], W["ple_scale"][0],
                                     pin[il * D:(il + 1) * D], s.eps)
        if self.lm_head is None:
            return x, None
        n = O.rms_norm(x, self.final_norm, s.eps)
        return x, O.logit_softcap(O.matmul(n, self.lm_head, s.vocab, s.hidden, self.lm_type), s.softcap)
