"""The Node host path on the GPU: HipBackend (gemma4-webgpu_amd/node/
hip_backend.js) dispatching the reference's per-key pass order through the
N-API addon, on a four-layer model with Gemma-4-E2B's layer kinds (layer 0
local and 1 global own their caches; 2 local reads 0's, 3 global reads 1's;
head dims 256 / 512, FFN 6144 / 12288, per-layer embeddings) and a
4096-token vocabulary, its matrices in a Q4_K_M-style mix of Q4_K and Q6_K.

The model is written here from the oracle's seeded generators; the Node
program (tests/node/napi_forward.js) uploads it and runs three greedy
forwards: token and position as arguments, then the sampled token read on
the device, then that with the position read on the device from a captured
graph. Each forward's hidden state and logits are checked against the
oracle's step at rel-L2 1e-3 / cosine 0.9999, and its token is the argmax
of its logits (bit-exact). The same three steps run again through the fused
MI355X step (HipBackend.encodeFusedStep / captureFusedStep)."""
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
from g4hip.decoder import DEFAULT_TYPES, E2BShape, q4km_types
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

    fmt_of = q4km_types(s)
    names = dict(wq="attn_q", wk="attn_k", wv="attn_v", wo="attn_output", wgate="ffn_gate", wup="ffn_up",
                 wdown="ffn_down")
    layers, formats = [], []
    D = s.ple_dim
    for il in range(s.n_layers):
        hd, Q, KV, I, H = s.hd(il), s.q_dim_of(il), s.kv_dim_of(il), s.ffn_of(il), s.hidden
        prod = s.is_producer(il)
        qt = {nm: fmt_of(il, nm) for nm in names}

        def mat(nm, M, N):
            return q4(M, N) if qt[nm] == "q4k" else q6(M, N)

        t = {"attn_norm": f16(H), "attn_q": mat("wq", Q, H), "attn_k": mat("wk", KV, H) if prod else None,
             "attn_v": mat("wv", KV, H) if prod else None, "attn_q_norm": f16(hd),
             "attn_k_norm": f16(hd) if prod else None, "attn_output": mat("wo", H, Q), "post_attention_norm": f16(H),
             "ffn_norm": f16(H), "ffn_gate": mat("wgate", I, H), "ffn_up": mat("wup", I, H),
             "ffn_down": mat("wdown", H, I), "post_ffw_norm": f16(H)}
        if D:
            t.update({"inp_gate": f16(D * H, 0.0, 0.03), "proj": f16(H * D, 0.0, 0.03), "post_norm": f16(H),
                      "layer_output_scale": f16(2, 0.8, 0.1)})
        for k, v in t.items():
            if v is not None:
                files[f"L{il}.{k}"] = v
        formats.append({names[nm]: f for nm, f in qt.items() if f != DEFAULT_TYPES[nm]})
        ple = {}
        if D:
            ple = dict(ple_gate=_Host(t["inp_gate"]), ple_proj=_Host(t["proj"]), ple_post_norm=_Host(t["post_norm"]),
                       ple_scale=_Host(t["layer_output_scale"]))
        layers.append(SimpleNamespace(qt=qt, **ple,
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
    ple_globals = {}
    if D:
        pmp, ppn = f16(s.n_layers * D * s.hidden, 0.0, 0.03), f16(D)
        rng = np.random.default_rng(nxt())
        tbl = rng.integers(0, 256, (s.vocab * s.n_layers, 176), dtype=np.uint8)
        n = tbl.shape[0]
        tbl[:, 0:2] = np.abs(rng.standard_normal(n) * 2e-3).astype(np.float16).view(np.uint8).reshape(n, 2)
        tbl[:, 2:4] = np.abs(rng.standard_normal(n) * 1e-3).astype(np.float16).view(np.uint8).reshape(n, 2)
        tbl = tbl.reshape(-1)
        files.update({"perLayerModelProj": pmp, "perLayerProjNorm": ppn, "perLayerTable": tbl})
        ple_globals = dict(ple_model_proj=_Host(pmp), ple_proj_norm=_Host(ppn), ple_table=_Host(tbl))
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
                          lm_head=_Host(lm_head), embedding=_Host(emb), **ple_globals)
    return files, formats, HostModel(dec), kcs, vcs


@pytest.mark.skipif(shutil.which("node") is None, reason="no node binary")
@pytest.mark.parametrize("fused", [False, True], ids=["key_by_key", "fused_step"])
def test_node_backend_forwards_vs_oracle(fused):
    addon = os.path.join(ROOT, "gemma4-webgpu_amd", "node", "g4hip.node")
    assert os.path.exists(addon), "g4hip.node is not built"
    shape = E2BShape.real(n_layers=4, n_unshared=2, global_layers=(1, 3), vocab=4096)
    files, formats, hm, kcs, vcs = _model(shape)
    assert any(formats), "the model mixes block formats"
    cfg = {"overrides": {"num_layers": 4, "num_unshared_layers": 2, "global_layers": [1, 3], "vocab_size": 4096},
           "maxSeqLen": MAX_SEQ, "position": POS, "token": TOKEN, "formats": formats, "fused": fused}
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
        x_ref, lg_ref = hm.step(hm.embed(tok), kcs, vcs, POS + i, token=tok)
        print(f"[napi] forward {i + 1}: token in {tok}, hidden rel-L2 {O.rel_l2(hidden, x_ref):.2e}, "
              f"logits rel-L2 {O.rel_l2(logits, lg_ref):.2e}, sampled {got_tok}", flush=True)
        assert_close(hidden, x_ref, what=f"hidden forward {i + 1}")
        assert_close(logits, lg_ref, what=f"logits forward {i + 1}")
        assert got_tok == O.argmax(logits)
        assert lg_ref[got_tok] >= lg_ref.max() - 1e-3 * np.abs(lg_ref).max()
        tok = got_tok


@pytest.mark.skipif(shutil.which("node") is None, reason="no node binary")
def test_node_backend_pipelined_generate_vs_oracle():
    """HipBackend.generate on the GPU: the reference's depth-2 loop
    (src/engine.ts:2041-2124: step N + 1 submitted before step N's token is
    read back, asynchronously) gives the same tokens as the depth-1 loop, and
    each token is a maximum of the oracle's logits for the step that the
    previous token starts (within the logits' tolerance)."""
    N = 6
    shape = E2BShape.real(n_layers=4, n_unshared=2, global_layers=(1, 3), vocab=4096)
    files, formats, hm, kcs, vcs = _model(shape)
    cfg = {"overrides": {"num_layers": 4, "num_unshared_layers": 2, "global_layers": [1, 3], "vocab_size": 4096},
           "maxSeqLen": MAX_SEQ, "position": POS, "token": TOKEN, "formats": formats, "generate": N}
    with tempfile.TemporaryDirectory() as d:
        for name, arr in files.items():
            np.ascontiguousarray(arr).tofile(os.path.join(d, name + ".bin"))
        with open(os.path.join(d, "config.json"), "w") as f:
            json.dump(cfg, f)
        print("[napi] running the Node generate loop", flush=True)
        r = subprocess.run(["node", os.path.join(ROOT, "tests", "node", "napi_forward.js"), d], capture_output=True,
                           text=True, timeout=240)
        print(r.stdout, r.stderr, flush=True)
        assert r.returncode == 0, r.stderr
        toks = np.fromfile(os.path.join(d, "out.bin"), np.uint32)
    assert toks.size == 2 * N
    assert np.array_equal(toks[:N], toks[N:]), "depth 2 and depth 1 differ"
    tok = TOKEN
    for i in range(N):
        _, lg = hm.step(hm.embed(tok), kcs, vcs, POS + i, token=tok)
        got = int(toks[i])
        print(f"[napi] generate step {i}: in {tok}, out {got}, oracle argmax {O.argmax(lg)}", flush=True)
        assert lg[got] >= lg.max() - 1e-3 * np.abs(lg).max(), i
        tok = got


def _run_node(cfg, files):
    with tempfile.TemporaryDirectory() as d:
        for name, arr in files.items():
            np.ascontiguousarray(arr).tofile(os.path.join(d, name + ".bin"))
        with open(os.path.join(d, "config.json"), "w") as f:
            json.dump(cfg, f)
        r = subprocess.run(["node", os.path.join(ROOT, "tests", "node", "napi_forward.js"), d], capture_output=True,
                           text=True, timeout=240)
        print(r.stdout, r.stderr, flush=True)
        assert r.returncode == 0, r.stderr
        return np.fromfile(os.path.join(d, "out.bin"), np.uint8)


@pytest.mark.skipif(shutil.which("node") is None, reason="no node binary")
@pytest.mark.parametrize("rows,T", [(8, 20), (64, 70)])
def test_node_backend_batched_prefill_vs_oracle(rows, T):
    """HipBackend.prefill on the GPU: the prompt through the batched step,
    `rows` tokens per chunk (the last one short), over the backend's own
    caches (an identity page table), against the reference's prefill of one
    forward per token (src/engine.ts:1923-1938; here the oracle's steps
    from position 600, past the 512 window). Every K/V row the prompt
    appended (f16) is checked against the oracle's f32 row of its position,
    the sample is a maximum of the oracle's logits for the last token, and
    the fused step that follows (from the sample, at position 600 + T, over
    the prefilled caches) matches the oracle's step."""
    shape = E2BShape.real(n_layers=4, n_unshared=2, global_layers=(1, 3), vocab=4096)
    files, formats, hm, kcs, vcs = _model(shape)
    toks = np.random.default_rng(T).integers(0, shape.vocab, T).astype(np.uint32)
    cfg = {"overrides": {"num_layers": 4, "num_unshared_layers": 2, "global_layers": [1, 3], "vocab_size": 4096},
           "maxSeqLen": MAX_SEQ, "position": POS, "token": 0, "formats": formats, "prefill": toks.tolist(),
           "rows": rows}
    print(f"[napi] prefill of {T} tokens in chunks of {rows}", flush=True)
    out = _run_node(cfg, files)
    first = int(out[:4].view(np.uint32)[0])
    at = 4
    got_rows = {}
    for il in range(shape.n_layers):
        if not shape.is_producer(il):
            continue
        n = 2 * shape.kv_dim_of(il) * T
        got_rows[il] = [out[at + j * n:at + (j + 1) * n].view(np.float16).astype(np.float32).reshape(T, -1)
                        for j in range(2)]
        at += 2 * n
    H, V = shape.hidden, shape.vocab
    hidden = out[at:at + 4 * H].view(np.float32)
    logits = out[at + 4 * H:at + 4 * H + 4 * V].view(np.float32)
    step_tok = int(out[at + 4 * H + 4 * V:].view(np.uint32)[0])
    lg = None
    for t in range(T):
        want = {}
        _, lg = hm.step(hm.embed(int(toks[t])), kcs, vcs, POS + t, token=int(toks[t]), rows=want)
        for il, (k, v) in got_rows.items():
            assert_close(k[t], want[il][0], what=f"k row {POS + t} layer {il}")
            assert_close(v[t], want[il][1], what=f"v row {POS + t} layer {il}")
    print(f"[napi] prefill sample {first}, oracle argmax {O.argmax(lg)}", flush=True)
    assert lg[first] >= lg.max() - 1e-3 * np.abs(lg).max()
    x_ref, lg_ref = hm.step(hm.embed(first), kcs, vcs, POS + T, token=first)
    print(f"[napi] step after prefill: hidden rel-L2 {O.rel_l2(hidden, x_ref):.2e}, logits rel-L2 "
          f"{O.rel_l2(logits, lg_ref):.2e}", flush=True)
    assert_close(hidden, x_ref, what="hidden of the step after prefill")
    assert_close(logits, lg_ref, what="logits of the step after prefill")
    assert step_tok == O.argmax(logits)
