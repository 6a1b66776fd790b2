"""Oracle composition of one E2B-shaped decode step for one sequence (the
order of src/engine.ts:1539-1625 and the head of src/engine.ts:1686-1717),
over weights downloaded once from a decoder's device buffers."""
import numpy as np

import oracle as O


class HostModel:
    def __init__(self, dec):
        self.s = s = dec.s
        u8, u16 = np.uint8, np.uint16
        self.table = dec.rope_freqs.download(u16)
        self.layers = []
        for L in dec.layers:
            self.layers.append({k: getattr(L, k).download(u8 if k.startswith("w") else u16)
                                for k in ("wq", "wk", "wv", "wo", "wgate", "wup", "wdown", "attn_norm",
                                          "post_attn_norm", "pre_ffn_norm", "post_ffn_norm", "q_norm", "k_norm")})
        self.final_norm = dec.final_norm.download(u16)
        self.lm_head = dec.lm_head.download(u8) if dec.lm_head is not None else None

    def step(self, hidden, kcs, vcs, pos):
        """Decode position `pos`: kcs/vcs are this sequence's dense f16 caches
        (one per layer, >= pos + 1 rows), updated in place. Returns the new
        hidden state and the softcapped logits (None without an LM head)."""
        s, x = self.s, hidden.copy()
        for il, W in enumerate(self.layers):
            glob = s.is_global(il)
            theta = s.theta_global if glob else s.theta_local
            window = 0 if glob else s.window
            n = O.rms_norm(x, W["attn_norm"], s.eps)
            q = O.matmul(n, W["wq"], s.q_dim, s.hidden, "q4k")
            k = O.matmul(n, W["wk"], s.kv_dim, s.hidden, "q4k")
            v = O.matmul(n, W["wv"], s.kv_dim, s.hidden, "q4k")
            v = O.per_head_rms_norm_no_weight(v, s.n_kv_heads, s.head_dim, s.eps)
            q = O.fused_per_head_norm_rope(q, W["q_norm"], s.n_q_heads, s.head_dim, s.eps, pos, theta, int(glob),
                                           self.table)
            k = O.fused_per_head_norm_rope(k, W["k_norm"], s.n_kv_heads, s.head_dim, s.eps, pos, theta, int(glob),
                                           self.table)
            O.kv_cache_store_f16(k, v, kcs[il], vcs[il], s.n_kv_heads, s.head_dim, pos)
            a = O.attention(q, kcs[il], vcs[il], s.n_q_heads, s.n_kv_heads, s.head_dim, pos + 1, 1.0, window)
            o = O.matmul(a, W["wo"], s.hidden, s.q_dim, "q4k")
            h = O.fused_norm_add(o, W["post_attn_norm"], x, s.eps)
            n2 = O.rms_norm(h, W["pre_ffn_norm"], s.eps)
            g = O.matmul(n2, W["wgate"], s.ffn, s.hidden, "q4k")
            u = O.matmul(n2, W["wup"], s.ffn, s.hidden, "q4k")
            dn = O.matmul(O.gelu_mul(g, u), W["wdown"], s.hidden, s.ffn, "q6k")
            x = O.fused_norm_add(dn, W["post_ffn_norm"], h, s.eps)
        if self.lm_head is None:
            return x, None
        n = O.rms_norm(x, self.final_norm, s.eps)
        return x, O.logit_softcap(O.matmul(n, self.lm_head, s.vocab, s.hidden, "q6k"), s.softcap)
