"""GPU side of the GGUF loader: tensors uploaded from a file and a decoder
built from one.

* g4_gguf_upload: every tensor type's bytes arrive unchanged;
  g4_gguf_upload_f16: F32 / BF16 / F16 tensors equal numpy's IEEE
  round-to-nearest-even f16 conversion bit for bit, over every exponent,
  ties, subnormals, overflow, infinities and NaN;
* g4_dequantF16: Q4_K and Q6_K blocks to f16 equal the oracle's f32 dequant
  (bit-exact with src/gguf.ts:168-210 / :323-368) rounded by numpy;
* a Gemma-4-E2B-layout file (four layers, layer kinds as the real model:
  a global head-dim-512 layer, FFN 12288 and shared caches past the
  unshared layers) with mixed formats as a Q4_K_M file holds them (a Q6_K
  v projection beside Q4_K q/k, Q4_K and Q6_K down projections), written
  by the test-side writer: the decoder built from it holds the file's
  bytes, and its fused step (embedding of the sampled token, captured and
  replayed) and ragged step match the oracle composition over the same
  weights at rel-L2 1e-3 / cosine 0.9999, the sampled tokens bit-exact on
  the device's logits."""
import json
import os
import shutil
import subprocess
import tempfile

import numpy as np
import pytest

import oracle as O
from decode_oracle import HostModel
from g4hip.decoder import E2BShape, decoder_from_gguf, q4km_types
from g4hip.gguf import GGUFFile
from gguf_writer import BOOL, F32, GGUFWriter, I32, STR, U32
from gpu_util import assert_close
from test_gpu_batch_step import _step_vs_oracle

pytestmark = pytest.mark.gpu

T_F32, T_F16, T_Q4_K, T_Q5_K, T_Q6_K, T_BF16, T_Q8_0 = 0, 1, 12, 13, 14, 30, 8


def _f32_sweep() -> np.ndarray:
    """f32 bit patterns over every exponent: each exponent's extreme and
    middle mantissas, the f16 rounding ties and their neighbours, plus
    random patterns, zeros, infinities and NaNs."""
    e = np.arange(256, dtype=np.uint32) << 23
    m = np.array([0, 1, 0xfff, 0x1000, 0x1001, 0x2000, 0x3000, 0x400000, 0x7fe000, 0x7ff000, 0x7fffff],
                 np.uint32)
    grid = (e[:, None] | m[None, :]).ravel()
    rnd = np.random.default_rng(3).integers(0, 2**32, 1 << 16, dtype=np.uint64).astype(np.uint32)
    # around the f16 subnormal and overflow edges
    edges = np.concatenate([np.arange(0x33000000 - 64, 0x33000000 + 64), np.arange(0x387fe000, 0x38802000, 16),
                            np.arange(0x477fe000, 0x47800100, 16)]).astype(np.uint32)
    b = np.concatenate([grid, grid | 0x80000000, rnd, edges, [0x7fc00000, 0xffc00001]]).astype(np.uint32)
    return b.view(np.float32)


def _np_f16_bits(x32: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore", invalid="ignore"):
        h = x32.astype(np.float16).view(np.uint16).copy()
    nan = np.isnan(x32)
    h[nan] = (h[nan] & 0x8000) | 0x7e00  # canonical quiet NaN (payloads are not compared)
    return h


def _nan_canon(h: np.ndarray) -> np.ndarray:
    h = h.copy()
    nan = ((h & 0x7c00) == 0x7c00) & ((h & 0x3ff) != 0)
    h[nan] = (h[nan] & 0x8000) | 0x7e00
    return h


def test_upload_bytes_and_f16(ctx, tmp_path):
    rng = np.random.default_rng(9)
    x = _f32_sweep()
    n = x.size
    bf = (rng.integers(0, 2**16, 4096, dtype=np.uint32)).astype(np.uint16)
    f16 = rng.integers(0, 2**16, 2048, dtype=np.uint32).astype(np.uint16)
    q = {T_Q4_K: O.gen_q4k(4, 40), T_Q6_K: O.gen_q6k(5, 40), T_Q5_K: rng.integers(0, 256, 176 * 8, dtype=np.uint8),
         T_Q8_0: rng.integers(0, 256, 34 * 16, dtype=np.uint8)}
    w = GGUFWriter()
    w.tensor("x32", (n,), T_F32, x).tensor("bf", (bf.size,), T_BF16, bf).tensor("h", (f16.size,), T_F16, f16)
    for t, blob in q.items():
        w.tensor(f"q{t}", (blob.size // {T_Q4_K: 144, T_Q6_K: 210, T_Q5_K: 176, T_Q8_0: 34}[t] *
                            (256 if t != T_Q8_0 else 32),), t, blob)
    g = GGUFFile(w.write(str(tmp_path / "u.gguf")))
    print(f"[gguf upload] {n} f32 patterns, {len(g.tensors)} tensors", flush=True)
    for t in g.tensors:
        got = g.upload(ctx, t.name).download(np.uint8, t.nbytes)
        assert np.array_equal(got, g.data(t.name)), t.name
    got = g.upload_f16(ctx, "x32").download(np.uint16, n)
    assert np.array_equal(_nan_canon(got), _np_f16_bits(x))
    got = g.upload_f16(ctx, "bf").download(np.uint16, bf.size)
    want = _np_f16_bits((bf.astype(np.uint32) << 16).view(np.float32))
    assert np.array_equal(_nan_canon(got), want)
    assert np.array_equal(g.upload_f16(ctx, "h").download(np.uint16, f16.size), f16)
    with pytest.raises(Exception):
        g.upload_f16(ctx, f"q{T_Q4_K}")
    small = ctx.alloc(16)
    with pytest.raises(Exception):
        g.upload(ctx, "x32", dst=small)


@pytest.mark.parametrize("wtype", ["q4k", "q6k"])
def test_dequant_f16(ctx, wtype):
    nb = 3000
    blocks = O.gen_q4k(11, nb) if wtype == "q4k" else O.gen_q6k(12, nb)
    ref = (O.dequant_q4k if wtype == "q4k" else O.dequant_q6k)(blocks)
    out = ctx.empty(nb * 256, np.uint16)
    ctx.dequantF16(wtype, ctx.from_numpy(blocks), nb, out)
    got = out.download(np.uint16)
    assert np.array_equal(_nan_canon(got), _np_f16_bits(ref))


# ---- a small Gemma-4-E2B-layout model in a file --------------------------------

N_LAYERS, N_UNSHARED, GLOBALS, VOCAB = 4, 2, (1, 3), 4096


def _q5k_blocks(seed: int, n: int) -> np.ndarray:
    """Q5_K blocks: f16 d ~ |N(0, 2e-3)|, dmin ~ |N(0, 1e-3)|, the other bytes uniform."""
    rng = np.random.default_rng(seed)
    b = rng.integers(0, 256, (n, 176), dtype=np.uint8)
    b[:, 0:2] = np.abs(rng.standard_normal(n) * 2e-3).astype(np.float16).view(np.uint8).reshape(n, 2)
    b[:, 2:4] = np.abs(rng.standard_normal(n) * 1e-3).astype(np.float16).view(np.uint8).reshape(n, 2)
    return b.reshape(-1)


def _shape() -> E2BShape:
    return E2BShape.real(n_layers=N_LAYERS, n_unshared=N_UNSHARED, global_layers=GLOBALS, vocab=VOCAB)


def _model_file(path: str) -> str:
    s = _shape()
    qt = q4km_types(s)
    w = GGUFWriter()
    w.kv("general.architecture", STR, "gemma4")
    w.kv("gemma4.embedding_length", U32, s.hidden).kv("gemma4.block_count", U32, N_LAYERS)
    w.kv("gemma4.attention.head_count", U32, 8).kv("gemma4.attention.head_count_kv", U32, 1)
    w.kv("gemma4.context_length", U32, 131072)
    w.array("gemma4.feed_forward_length", I32, [s.ffn_of(i) for i in range(N_LAYERS)])
    w.kv("gemma4.attention.key_length", U32, 512).kv("gemma4.attention.key_length_swa", U32, 256)
    w.kv("gemma4.rope.freq_base", F32, 1e6).kv("gemma4.rope.freq_base_swa", F32, 1e4)
    w.kv("gemma4.attention.sliding_window", U32, 512)
    w.array("gemma4.attention.sliding_window_pattern", BOOL, [i not in GLOBALS for i in range(N_LAYERS)])
    w.kv("gemma4.final_logit_softcapping", F32, 30.0)
    w.kv("gemma4.attention.shared_kv_layers", U32, N_LAYERS - N_UNSHARED)
    seed = [100]

    def mat(name, M, N, t):
        seed[0] += 1
        if t == "q4k":
            w.tensor(name, (N, M), T_Q4_K, O.gen_q4k(seed[0], M * N // 256))
        else:
            w.tensor(name, (N, M), T_Q6_K, O.gen_q6k(seed[0], M * N // 256))

    def vec(name, n, mean=1.0, std=0.1):
        seed[0] += 1
        w.tensor(name, (n,), T_F32, O.gen_normal_f32(seed[0], n, mean, std))

    def f32mat(name, M, N):
        seed[0] += 1
        w.tensor(name, (N, M), T_F32, O.gen_normal_f32(seed[0], M * N, 0.0, 0.03))

    for il in range(N_LAYERS):
        H, Q, KV, I, hd = s.hidden, s.q_dim_of(il), s.kv_dim_of(il), s.ffn_of(il), s.hd(il)
        p = f"blk.{il}."
        vec(p + "attn_norm.weight", H)
        mat(p + "attn_q.weight", Q, H, qt(il, "wq"))
        if s.is_producer(il):
            mat(p + "attn_k.weight", KV, H, qt(il, "wk"))
            mat(p + "attn_v.weight", KV, H, qt(il, "wv"))
            vec(p + "attn_k_norm.weight", hd)
        vec(p + "attn_q_norm.weight", hd)
        mat(p + "attn_output.weight", H, Q, qt(il, "wo"))
        vec(p + "post_attention_norm.weight", H)
        vec(p + "ffn_norm.weight", H)
        mat(p + "ffn_gate.weight", I, H, "q4k")
        mat(p + "ffn_up.weight", I, H, "q4k")
        mat(p + "ffn_down.weight", H, I, qt(il, "wdown"))
        vec(p + "post_ffw_norm.weight", H)
    vec("output_norm.weight", s.hidden)
    # per-layer embeddings as the real file holds them: a BF16 projection,
    # an F32 norm, the Q5_K table and F32 per-layer matrices
    L, D = N_LAYERS, s.ple_dim
    seed[0] += 1
    pm = (O.gen_normal_f32(seed[0], L * D * s.hidden, 0.0, 0.03).view(np.uint32) >> 16).astype(np.uint16)
    w.tensor("per_layer_model_proj.weight", (s.hidden, L * D), T_BF16, pm)
    vec("per_layer_proj_norm.weight", D)
    seed[0] += 1
    w.tensor("per_layer_token_embd.weight", (L * D, VOCAB), T_Q5_K, _q5k_blocks(seed[0], VOCAB * L))
    for il in range(N_LAYERS):
        f32mat(f"blk.{il}.inp_gate.weight", D, s.hidden)
        f32mat(f"blk.{il}.proj.weight", s.hidden, D)
        vec(f"blk.{il}.post_norm.weight", s.hidden)
        vec(f"blk.{il}.layer_output_scale.weight", 1, 0.8, 0.1)
    # the tied table (the LM head's blocks, the lookup's f16 rows)
    seed[0] += 1
    te = O.gen_q6k(seed[0], VOCAB * s.hidden // 256)
    w.tensor("token_embd.weight", (s.hidden, VOCAB), T_Q6_K, te)
    w.tensor("rope_freqs.weight", (256,), T_F32, np.where(np.arange(256) < 64, 1.0, 1e30).astype(np.float32))
    return w.write(path)


@pytest.fixture(scope="module")
def model_path(tmp_path_factory):
    return _model_file(str(tmp_path_factory.mktemp("gguf") / "e2b4.gguf"))


def test_decoder_holds_the_file(ctx, model_path):
    g = GGUFFile(model_path)
    d = decoder_from_gguf(ctx, g, max_seq=1024)
    s = d.s
    assert (s.n_layers, s.vocab, s.n_unshared, s.global_layers, s.head_dim_global, s.ffn_shared) == \
        (N_LAYERS, VOCAB, N_UNSHARED, GLOBALS, 512, 12288)
    names = dict(wq="attn_q", wk="attn_k", wv="attn_v", wo="attn_output", wgate="ffn_gate", wup="ffn_up",
                 wdown="ffn_down")
    formats = set()
    for il, L in enumerate(d.layers):
        for nm, fn in names.items():
            b = getattr(L, nm)
            if b is None:
                assert not s.is_producer(il) and nm in ("wk", "wv")
                continue
            t = g.tensor(f"blk.{il}.{fn}.weight")
            assert np.array_equal(b.download(np.uint8, t.nbytes), g.data(t.name)), t.name
            assert L.qt[nm] == {T_Q4_K: "q4k", T_Q6_K: "q6k"}[t.type]
            formats.add((nm, L.qt[nm]))
        want = g.data(f"blk.{il}.attn_norm.weight").view(np.float32).astype(np.float16).view(np.uint16)
        assert np.array_equal(L.attn_norm.download(np.uint16), want)
    assert {("wv", "q6k"), ("wv", "q4k"), ("wdown", "q4k"), ("wdown", "q6k")} <= formats
    te = g.data("token_embd.weight")
    assert np.array_equal(d.lm_head.download(np.uint8, te.size), te)
    emb = d.embedding.download(np.uint16)
    assert np.array_equal(_nan_canon(emb), _np_f16_bits(O.dequant_q6k(te)))
    rf = d.rope_freqs.download(np.uint16).view(np.float16)
    assert np.all(rf[:64] == 1.0) and np.all(np.isinf(rf[64:]))
    # per-layer embeddings: BF16 / F32 tensors as f16, the Q5_K table as is
    assert s.ple_dim == 256
    pm = g.data("per_layer_model_proj.weight").view(np.uint16)
    want = _np_f16_bits((pm.astype(np.uint32) << 16).view(np.float32))
    assert np.array_equal(_nan_canon(d.ple_model_proj.download(np.uint16)), want)
    assert np.array_equal(d.ple_table.download(np.uint8), g.data("per_layer_token_embd.weight"))
    for il, L in enumerate(d.layers):
        for nm, fn in (("ple_gate", "inp_gate"), ("ple_proj", "proj"), ("ple_post_norm", "post_norm")):
            want = g.data(f"blk.{il}.{fn}.weight").view(np.float32).astype(np.float16).view(np.uint16)
            assert np.array_equal(getattr(L, nm).download(np.uint16), want), (il, nm)
        sc = g.data(f"blk.{il}.layer_output_scale.weight").view(np.float32).astype(np.float16).view(np.uint16)
        assert L.ple_scale.download(np.uint16)[0] == sc[0]
    del d


def test_file_model_fused_step_with_token_feedback(ctx, model_path):
    POS = 600
    d = decoder_from_gguf(ctx, model_path, max_seq=1024)
    d.fill_kv(POS, seed=24)
    T0 = 1234
    d.set_token(T0)
    d.set_position(POS)
    ctx.sync()
    hm = HostModel(d)
    kcs = [L.k_cache.download(np.uint16) for L in d.layers]
    vcs = [L.v_cache.download(np.uint16) for L in d.layers]
    # 5 per layer, + a merge launch on the two head-dim-512 layers, + the
    # second q/k/v launch of layer 1 (Q6_K v), + embedding, head, argmax,
    # + per-layer embeddings: stage 1 (2), 2 per layer, the last tail (1)
    assert d.layers[1].qt["wv"] == "q6k" and d.layers[1].qt["wq"] == "q4k"
    assert d.launches_per_step_fused() == 5 * N_LAYERS + 2 + 1 + 3 + 3 + 2 * N_LAYERS
    g = d.capture_fused()
    try:
        tok = T0
        for i in range(2):
            ctx.graph_launch(g)
            ctx.sync()
            x_ref, lg_ref = hm.step(hm.embed(tok), kcs, vcs, POS + i, token=tok)
            lg = d.logits.download(np.float32)
            print(f"[gguf model] replay {i}: token {tok}, hidden rel-L2 "
                  f"{O.rel_l2(d.hidden.download(np.float32), x_ref):.2e}, logits {O.rel_l2(lg, lg_ref):.2e}",
                  flush=True)
            assert_close(d.hidden.download(np.float32), x_ref, what=f"hidden replay {i}")
            assert_close(lg, lg_ref, what=f"logits replay {i}")
            new = int(d.token.download(np.uint32)[0])
            assert new == O.argmax(lg)
            assert lg_ref[new] >= lg_ref.max() - 1e-3 * np.abs(lg_ref).max()
            tok = new
    finally:
        ctx.graph_destroy(g)
    del d


def test_file_model_reference_order_step(ctx, model_path):
    POS = 300
    d = decoder_from_gguf(ctx, model_path, max_seq=1024, embed=False)
    d.fill_kv(POS, seed=25)
    ctx.sync()
    hm = HostModel(d)
    x0 = d.hidden.download(np.float32)
    kcs = [L.k_cache.download(np.uint16) for L in d.layers]
    vcs = [L.v_cache.download(np.uint16) for L in d.layers]
    x_ref, lg_ref = hm.step(x0, kcs, vcs, POS)
    d.step_reference(POS)
    ctx.sync()
    assert_close(d.hidden.download(np.float32), x_ref, what="per-key hidden")
    assert_close(d.logits.download(np.float32), lg_ref, what="per-key logits")
    del d


def test_file_model_ragged_step(ctx, model_path):
    LENS = [5, 700, 130]
    d = decoder_from_gguf(ctx, model_path, batch=LENS, embed=False, reserve=8, seed=3)
    d.fill_kv(seed=27)
    ctx.sync()
    print(f"[gguf model] ragged step B={d.B}", flush=True)
    _step_vs_oracle(ctx, d, LENS)
    del d


@pytest.mark.skipif(shutil.which("node") is None, reason="no node binary")
def test_node_backend_from_gguf(ctx, model_path):
    """HipBackend.fromGGUF (the N-API addon's reader and uploads, the Node
    backend's configFromGGUF) on the same file: three greedy forwards from
    position 0 with zero caches against the oracle over the Python
    decoder's copy of the file's weights."""
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    d = decoder_from_gguf(ctx, model_path, max_seq=1024)
    ctx.sync()
    hm = HostModel(d)
    s = d.s
    kcs = [np.zeros(1024 * s.kv_dim_of(il), np.uint16) for il in range(s.n_layers)]
    vcs = [np.zeros(1024 * s.kv_dim_of(il), np.uint16) for il in range(s.n_layers)]
    del d
    with tempfile.TemporaryDirectory() as td:
        with open(os.path.join(td, "config.json"), "w") as f:
            json.dump({"gguf": model_path, "maxSeqLen": 1024, "position": 0, "token": 1234}, f)
        print("[gguf node] running the Node forwards", flush=True)
        r = subprocess.run(["node", os.path.join(root, "tests", "node", "napi_forward.js"), td], capture_output=True,
                           text=True, timeout=240)
        print(r.stdout, r.stderr, flush=True)
        assert r.returncode == 0, r.stderr
        out = np.fromfile(os.path.join(td, "out.bin"), np.uint8)
    H, V = s.hidden, s.vocab
    per = 4 * H + 4 * V + 4
    assert out.size == 3 * per
    tok = 1234
    for i in range(3):
        blk = out[i * per:(i + 1) * per]
        hidden = blk[:4 * H].view(np.float32)
        logits = blk[4 * H:4 * H + 4 * V].view(np.float32)
        got = int(blk[4 * H + 4 * V:].view(np.uint32)[0])
        x_ref, lg_ref = hm.step(hm.embed(tok), kcs, vcs, i, token=tok)
        print(f"[gguf node] forward {i + 1}: token {tok}, hidden rel-L2 {O.rel_l2(hidden, x_ref):.2e}", flush=True)
        assert_close(hidden, x_ref, what=f"hidden forward {i + 1}")
        assert_close(logits, lg_ref, what=f"logits forward {i + 1}")
        assert got == O.argmax(logits)
        tok = got
