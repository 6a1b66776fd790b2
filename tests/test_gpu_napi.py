"""The Node host path on the GPU: HipBackend (gemma4-webgpu_amd/node/
hip_backend.js) dispatching the reference's per-key pass order through the
N-API addon, on a four-layer model with Gemma-4-E2B's layer kinds (layer 0
local and 1 global own their caches; 2 local reads 0's, 3 global reads 1's;
head dims 256 / 512, FFN 6144 / 12288) and a 4096-token vocabulary.

The model is written here from the oracle's seeded generators; the Node
program (tests/node/napi_forward.js) uploads it and runs three greedy
forwards: token and position as arguments, then the sampled token read on
the device, then that with the position read on the device from a captured
graph. Each forward's hidden state and logits are checked against the
oracle's step at rel-L2 1e-3 / cosine 0.9999, and its token is the argmax
of its logits (bit-exact)."""
import json
import os
import shutil
import subprocess
import tempfile
from types import SimpleNamespace

import numpy as np
import pytest

import oracle as O
from decode_oracle import HostModel
from g4hip.decoder import E2BShape
from gpu_util import assert_close

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
POS = 600
MAX_SEQ = 1024
TOKEN = 1234


class _Host:
    """A host array with the device Buffer's download interface."""

    def __init__(self, a):
        self.a = np.ascontiguousarray(a)

    def download(self, dtype, count=None, offset=0):
        v = self.a.view(np.uint8)[offset:].view(dtype)
        return (v if count is None else v[:count]).copy()


def _model(shape):
    """Seeded weights in the decoder's tensor order; returns the files the
    Node program reads and a HostModel over the same arrays."""
    s, seed, files = shape, [100], {}

    def nxt():
        seed[0] += 1
        return seed[0]

    def q4(M, N):
        return O.gen_q4k(nxt(), M * N // 256)

    def q6(M, N):
        return O.gen_q6k(nxt(), M * N // 256)

    def f16(n, mean=1.0, std=0.1):
        return O.gen_normal_f16(nxt(), n, mean, std)

    layers = []
    for il in range(s.n_layers):
        hd, Q, KV, I, H = s.hd(il), s.q_dim_of(il), s.kv_dim_of(il), s.ffn_of(il), s.hidden
        prod = s.is_producer(il)
        t = {"attn_norm": f16(H), "attn_q": q4(Q, H), "attn_k": q4(KV, H) if prod else None,
             "attn_v": q4(KV, H) if prod else None, "attn_q_norm": f16(hd), "attn_k_norm": f16(hd) if prod else None,
             "attn_output": q4(H, Q), "post_attention_norm": f16(H), "ffn_norm": f16(H), "ffn_gate": q4(I, H),
             "ffn_up": q4(I, H), "ffn_down": q6(H, I), "post_ffw_norm": f16(H)}
        for k, v in t.items():
            if v is not None:
                files[f"L{il}.{k}"] = v
        layers.append(SimpleNamespace(
            wq=_Host(t["attn_q"]), wk=_Host(t["attn_k"]) if prod else None, wv=_Host(t["attn_v"]) if prod else None,
            wo=_Host(t["attn_output"]), wgate=_Host(t["ffn_gate"]), wup=_Host(t["ffn_up"]),
            wdown=_Host(t["ffn_down"]), attn_norm=_Host(t["attn_norm"]),
            post_attn_norm=_Host(t["post_attention_norm"]), pre_ffn_norm=_Host(t["ffn_norm"]),
            post_ffn_norm=_Host(t["post_ffw_norm"]), q_norm=_Host(t["attn_q_norm"]),
            k_norm=_Host(t["attn_k_norm"]) if prod else None))
    final_norm = f16(s.hidden)
    lm_head = q6(s.vocab, s.hidden)
    emb = O.gen_normal_f16(nxt(), s.vocab * s.hidden, 0.0, 0.03)
    half = s.head_dim_global // 2
    table = np.where(np.arange(half) < half // 4, 1.0, np.inf).astype(np.float16).view(np.uint16)
    files.update({"finalNorm": final_norm, "lmHead": lm_head, "tokenEmbed": emb, "rope_freqs": table})
    kcs, vcs = [], []
    for il in range(s.n_layers):
        n = MAX_SEQ * s.kv_dim_of(il)
        k, v = np.zeros(n, np.uint16), np.zeros(n, np.uint16)
        if s.is_producer(il):
            k[:POS * s.kv_dim_of(il)] = O.gen_normal_f16(nxt(), POS * s.kv_dim_of(il), 0.0, 1.0)
            v[:POS * s.kv_dim_of(il)] = O.gen_normal_f16(nxt(), POS * s.kv_dim_of(il), 0.0, 1.0)
            files[f"kv{il}.k"], files[f"kv{il}.v"] = k, v
        kcs.append(k.copy())
        vcs.append(v.copy())
    dec = SimpleNamespace(s=s, rope_freqs=_Host(table), layers=layers, final_norm=_Host(final_norm),
                          lm_head=_Host(lm_head), embedding=_Host(emb))
    return files, HostModel(dec), kcs, vcs


@pytest.mark.skipif(shutil.which("node") is None, reason="no node binary")
def test_node_backend_forwards_vs_oracle():
    addon = os.path.join(ROOT, "gemma4-webgpu_amd", "node", "g4hip.node")
    assert os.path.exists(addon), "g4hip.node is not built"
    shape = E2BShape.real(n_layers=4, n_unshared=2, global_layers=(1, 3), vocab=4096)
    files, hm, kcs, vcs = _model(shape)
    cfg = {"overrides": {"num_layers": 4, "num_unshared_layers": 2, "global_layers": [1, 3], "vocab_size": 4096},
           "maxSeqLen": MAX_SEQ, "position": POS, "token": TOKEN}
    with tempfile.TemporaryDirectory() as d:
        for name, arr in files.items():
            np.ascontiguousarray(arr).tofile(os.path.join(d, name + ".bin"))
        with open(os.path.join(d, "config.json"), "w") as f:
            json.dump(cfg, f)
        print("[napi] running the Node forwards", flush=True)
        r = subprocess.run(["node", os.path.join(ROOT, "tests", "node", "napi_forward.js"), d], capture_output=True,
                           text=True, timeout=240)
        print(r.stdout, r.stderr, flush=True)
        assert r.returncode == 0, r.stderr
        out = np.fromfile(os.path.join(d, "out.bin"), np.uint8)
    H, V = shape.hidden, shape.vocab
    per = 4 * H + 4 * V + 4
    assert out.size == 3 * per
    tok = TOKEN
    for i in range(3):
        blk = out[i * per:(i + 1) * per]
        hidden = blk[:4 * H].view(np.float32)
        logits = blk[4 * H:4 * H + 4 * V].view(np.float32)
        got_tok = int(blk[4 * H + 4 * V:].view(np.uint32)[0])
        x_ref, lg_ref = hm.step(hm.embed(tok), kcs, vcs, POS + i)
        print(f"[napi] forward {i + 1}: token in {tok}, hidden rel-L2 {O.rel_l2(hidden, x_ref):.2e}, "
              f"logits rel-L2 {O.rel_l2(logits, lg_ref):.2e}, sampled {got_tok}", flush=True)
        assert_close(hidden, x_ref, what=f"hidden forward {i + 1}")
        assert_close(logits, lg_ref, what=f"logits forward {i + 1}")
        assert got_tok == O.argmax(logits)
        assert lg_ref[got_tok] >= lg_ref.max() - 1e-3 * np.abs(lg_ref).max()
        tok = got_tok
