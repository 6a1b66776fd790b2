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
from g4hip.decoder import E2BShape, decoder_from_gguf, q4km_types, qkv_groups
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


def _report_mismatch(got: np.ndarray, want: np.ndarray, raw: np.ndarray, block_bytes: int, per_block: int,
                     what: str) -> None:
    bad = np.flatnonzero(_nan_canon(got) != _nan_canon(want))
    if bad.size:
        print(f"[{what}] {bad.size} of {got.size} values differ", flush=True)
        for i in bad[:8]:
            b = int(i) // per_block
            print(f"  value {i} (block {b}): got {got[i]:#06x} want {want[i]:#06x}, block head "
                  f"{raw[b * block_bytes:b * block_bytes + 4].tolist()}", flush=True)
    assert bad.size == 0, what


@pytest.mark.parametrize("wtype", ["q4k", "q6k", "q8_0"])
def test_dequant_f16(ctx, wtype):
    nb = 3000
    if wtype == "q8_0":
        blocks = _q8_0_blocks(13, nb * 8)
        # d over the f16 range (subnormal, largest, negative, zero) and q = -128
        blocks.reshape(-1, 34)[:8, 0:2] = np.array([0x0001, 0x03ff, 0x0400, 0x7bff, 0x0000, 0x8400, 0xbc00, 0x1234],
                                                   np.uint16).view(np.uint8).reshape(8, 2)
        blocks.reshape(-1, 34)[:8, 2] = 0x80
        ref = O.dequant_q8_0(blocks)
        n = nb * 8
    else:
        blocks = O.gen_q4k(11, nb) if wtype == "q4k" else O.gen_q6k(12, nb)
        ref = (O.dequant_q4k if wtype == "q4k" else O.dequant_q6k)(blocks)
        n = nb
    out = ctx.empty(nb * 256, np.uint16)
    ctx.dequantF16(wtype, ctx.from_numpy(blocks), n, out)
    got = out.download(np.uint16)
    with np.errstate(over="ignore", invalid="ignore"):
        want = ref.astype(np.float16).view(np.uint16)
    _report_mismatch(got, want, blocks, 34 if wtype == "q8_0" else (144 if wtype == "q4k" else 210),
                     32 if wtype == "q8_0" else 256, f"dequant {wtype}")


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


def _q5k_matrix_blocks(seed: int, n: int) -> np.ndarray:
    """Q5_K blocks of a zero-mean matrix: d ~ |N(0, 5e-4)| and dmin = 15.5 d,
    the mean of d*sc*q over q, so that the sub-block offsets cancel on
    average (a biased matrix would make the test model ill-conditioned:
    its products would hinge on sums of the activations)."""
    b = _q5k_blocks(seed, n).reshape(n, 176)
    rng = np.random.default_rng(seed + 1)
    d = np.abs(rng.standard_normal(n) * 5e-4).astype(np.float16)
    b[:, 0:2] = d.view(np.uint8).reshape(n, 2)
    b[:, 2:4] = (d.astype(np.float32) * 15.5).astype(np.float16).view(np.uint8).reshape(n, 2)
    return b.reshape(-1)


def _q8_0_blocks(seed: int, n: int) -> np.ndarray:
    """Q8_0 blocks: f16 d ~ |N(0, 1e-3)|, 32 uniform int8."""
    rng = np.random.default_rng(seed)
    b = rng.integers(0, 256, (n, 34), dtype=np.uint8)
    b[:, 0:2] = np.abs(rng.standard_normal(n) * 1e-3).astype(np.float16).view(np.uint8).reshape(n, 2)
    return b.reshape(-1)


def _q4k_zero_mean(blocks: np.ndarray) -> np.ndarray:
    """Q4_K blocks with dmin = 7.5 d (the mean of d*sc*q over q): the
    sub-block offsets cancel on average, as in a trained matrix."""
    b = blocks.reshape(-1, 144).copy()
    d = b[:, 0:2].copy().view(np.float16).reshape(-1)
    b[:, 2:4] = (d.astype(np.float32) * 7.5).astype(np.float16).view(np.uint8).reshape(-1, 2)
    return b.reshape(-1)


def _matrix_bytes(t: int, seed: int, M: int, N: int, zero_mean: bool = False) -> np.ndarray:
    """An M x N matrix of GGUF type t from the seeded generators."""
    if t == T_Q4_K:
        b = O.gen_q4k(seed, M * N // 256)
        return _q4k_zero_mean(b) if zero_mean else b
    if t == T_Q6_K:
        return O.gen_q6k(seed, M * N // 256)
    if t == T_Q5_K:
        return _q5k_matrix_blocks(seed, M * N // 256)
    if t == T_Q8_0:
        return _q8_0_blocks(seed, M * N // 32)
    f = O.gen_normal_f32(seed, M * N, 0.0, 0.03)
    if t == T_F32:
        return f
    if t == T_F16:
        return f.astype(np.float16)
    return (f.view(np.uint32) >> 16).astype(np.uint16)  # BF16


def _model_file(path: str, fmt=None, head_type: int = T_Q6_K, q_norm: float = 1.0, zero_mean: bool = False) -> str:
    """fmt(il, name) -> GGUF type of each layer matrix (default: the
    Q4_K_M-style mix with Q4_K gate/up); q_norm is the mean of the q-norm
    weights (the attention scores scale with it); zero_mean makes the Q4_K
    matrices zero-mean."""
    s = _shape()
    if fmt is None:
        qt = q4km_types(s)
        fmt = lambda il, nm: {"q4k": T_Q4_K, "q6k": T_Q6_K}[qt(il, nm) if nm not in ("wgate", "wup") else "q4k"]  # noqa
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
        w.tensor(name, (N, M), t, _matrix_bytes(t, seed[0], M, N, zero_mean))

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
        mat(p + "attn_q.weight", Q, H, fmt(il, "wq"))
        if s.is_producer(il):
            mat(p + "attn_k.weight", KV, H, fmt(il, "wk"))
            mat(p + "attn_v.weight", KV, H, fmt(il, "wv"))
            vec(p + "attn_k_norm.weight", hd)
        vec(p + "attn_q_norm.weight", hd, q_norm, 0.1 * q_norm)
        mat(p + "attn_output.weight", H, Q, fmt(il, "wo"))
        vec(p + "post_attention_norm.weight", H)
        vec(p + "ffn_norm.weight", H)
        mat(p + "ffn_gate.weight", I, H, fmt(il, "wgate"))
        mat(p + "ffn_up.weight", I, H, fmt(il, "wup"))
        mat(p + "ffn_down.weight", H, I, fmt(il, "wdown"))
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
    w.tensor("token_embd.weight", (s.hidden, VOCAB), head_type, _matrix_bytes(head_type, seed[0], VOCAB, s.hidden))
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
    # 5 per layer (the head-dim-512 layers' attention merges in its launch),
    # + the second q/k/v launch of layer 1 (Q6_K v), + embedding, head, argmax,
    # + per-layer embeddings: stage 1 (2), 2 per layer, the last tail (1),
    # - one on each layer whose Q4_K q/k/v share the attention's launch
    # (layer 0, the head-dim-256 producer with Q4_K q/k/v)
    assert d.layers[1].qt["wv"] == "q6k" and d.layers[1].qt["wq"] == "q4k"
    shared = [il for il in range(N_LAYERS)
              if d._qkv_fused(qkv_groups(d.layers[il], [0, 0, 0], [0, 0, 0]))
              and ctx.qkv_attn_single_launch(d.attn_params[il], d.s.hidden, 3 if d.s.is_producer(il) else 1)]
    assert shared == [0]
    assert d.launches_per_step_fused() == 5 * N_LAYERS + 1 + 3 + 3 + 2 * N_LAYERS - len(shared)
    g = d.capture_fused()
    assert ctx.graph_kernel_nodes(g) == d.launches_per_step_fused()
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


def _node_from_gguf(ctx, model_path, fused=False):
    """HipBackend.fromGGUF (the N-API addon's reader and uploads, the Node
    backend's configFromGGUF) on a file: three greedy forwards from
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
            json.dump({"gguf": model_path, "maxSeqLen": 1024, "position": 0, "token": 1234, "fused": fused}, f)
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


@pytest.mark.skipif(shutil.which("node") is None, reason="no node binary")
@pytest.mark.parametrize("fused", [False, True], ids=["key_by_key", "fused_step"])
def test_node_backend_from_gguf(ctx, model_path, fused):
    _node_from_gguf(ctx, model_path, fused)


# A file whose matrices are in every format the reference loads: the layers
# mix Q8_0, Q5_K, F16, BF16 and F32 matrices with Q4_K / Q6_K ones (a Q5_K
# gate makes layer 1's FFN unfused; layer 2's gate and up are both F16), and
# the tied table is Q8_0. The formats the matvecs do not read as blocks are
# held as the reference's f16 rows (tensorToF16, src/engine.ts:570-579).
# Its embedding rows are small next to the layers' outputs, so the residual
# stream does not hide the layers' errors. To keep the model well
# conditioned, the q-norm weights (mean 0.25) hold the attention scores at a
# standard deviation of about 4 over the N(0, 1) caches (with mean 1, about
# 16: a softmax whose near-ties amplify any rounding), and the Q4_K and Q5_K
# matrices are zero-mean (a common offset on every row makes the products
# hinge on sums of the activations).
_FORMATS = {
    0: {"wq": T_Q8_0, "wk": T_Q5_K, "wv": T_F16, "wo": T_BF16, "wgate": T_Q4_K, "wup": T_Q4_K, "wdown": T_Q8_0},
    1: {"wq": T_Q4_K, "wk": T_Q4_K, "wv": T_Q6_K, "wo": T_F32, "wgate": T_Q5_K, "wup": T_Q4_K, "wdown": T_Q6_K},
    2: {"wq": T_F16, "wo": T_Q4_K, "wgate": T_F16, "wup": T_F16, "wdown": T_Q4_K},
}


@pytest.fixture(scope="module")
def formats_path(tmp_path_factory):
    fmt = lambda il, nm: _FORMATS.get(il, {}).get(nm, T_Q6_K if nm == "wdown" else T_Q4_K)  # noqa: E731
    return _model_file(str(tmp_path_factory.mktemp("gguf") / "formats.gguf"), fmt, head_type=T_Q8_0, q_norm=0.25,
                       zero_mean=True)


def test_every_format_as_f16_rows(ctx, formats_path):
    g = GGUFFile(formats_path)
    d = decoder_from_gguf(ctx, g, max_seq=1024)
    names = dict(wq="attn_q", wk="attn_k", wv="attn_v", wo="attn_output", wgate="ffn_gate", wup="ffn_up",
                 wdown="ffn_down")
    for il, L in enumerate(d.layers):
        for nm, fn in names.items():
            b = getattr(L, nm)
            if b is None:
                continue
            t = g.tensor(f"blk.{il}.{fn}.weight")
            if t.type in (T_Q4_K, T_Q6_K):
                assert L.qt[nm] == {T_Q4_K: "q4k", T_Q6_K: "q6k"}[t.type]
                assert np.array_equal(b.download(np.uint8, t.nbytes), g.data(t.name))
            else:
                assert L.qt[nm] == "f16", (il, nm)
                got = b.download(np.uint16, t.n_elements)
                bb, per = {T_Q8_0: (34, 32), T_Q5_K: (176, 256)}.get(t.type, (2, 1))
                _report_mismatch(got, O.dequant_f16_rows(g.data(t.name), t.type), g.data(t.name), bb, per,
                                 f"layer {il} {nm} {t.type_name}")
    te = g.tensor("token_embd.weight")
    assert d.lm_type == "f16" and d.embedding is d.lm_head
    assert np.array_equal(d.lm_head.download(np.uint16), O.dequant_f16_rows(g.data(te.name), te.type))
    del d


def test_every_format_fused_step(ctx, formats_path):
    POS = 600
    d = decoder_from_gguf(ctx, formats_path, max_seq=1024)
    d.fill_kv(POS, seed=34)
    d.set_token(77)
    d.set_position(POS)
    ctx.sync()
    hm = HostModel(d)
    kcs = [L.k_cache.download(np.uint16) for L in d.layers]
    vcs = [L.v_cache.download(np.uint16) for L in d.layers]
    # embedding, head (norm, matvec, softcap, two argmax stages); PLE 3 + 2 per layer;
    # layer 0: one f16 q/k/v group (norm + 3 matvecs), attention, o, fused FFN (2);
    # layer 1: a Q4_K (q, k) and a Q6_K (v) launch, attention (head dim 512, its
    # merge in the launch), o, unfused FFN (norm, gate, up, GELU product, down);
    # layer 2: f16 q (norm + matvec), attention, o, unfused FFN; layer 3: q,
    # attention (head dim 512), o, fused FFN
    assert d.launches_per_step_fused() == 1 + 5 + (3 + 2 * N_LAYERS) + 8 + 9 + 9 + 5
    g = d.capture_fused()
    assert ctx.graph_kernel_nodes(g) == d.launches_per_step_fused()
    try:
        tok = 77
        for i in range(2):
            ctx.graph_launch(g)
            ctx.sync()
            x_ref, lg_ref = hm.step(hm.embed(tok), kcs, vcs, POS + i, token=tok)
            lg = d.logits.download(np.float32)
            print(f"[gguf formats] replay {i}: hidden rel-L2 {O.rel_l2(d.hidden.download(np.float32), x_ref):.2e}",
                  flush=True)
            assert_close(d.hidden.download(np.float32), x_ref, what=f"hidden replay {i}")
            assert_close(lg, lg_ref, what=f"logits replay {i}")
            new = int(d.token.download(np.uint32)[0])
            assert new == O.argmax(lg)
            tok = new
        assert int(d.pos.download(np.uint32)[0]) == POS + 2
    finally:
        ctx.graph_destroy(g)
    # the reference-order step on the same weights
    d.set_token(5)
    d.set_position(POS)
    x0 = d.hidden.download(np.float32)
    d.fill_kv(POS, seed=34)
    ctx.sync()
    kcs = [L.k_cache.download(np.uint16) for L in d.layers]
    vcs = [L.v_cache.download(np.uint16) for L in d.layers]
    d.step_reference(POS)
    ctx.sync()
    x_ref, lg_ref = hm.step(hm.embed(5), kcs, vcs, POS, token=5)
    assert_close(d.hidden.download(np.float32), x_ref, what="per-key hidden")
    assert_close(d.logits.download(np.float32), lg_ref, what="per-key logits")
    del d


def test_every_format_ragged_step(ctx, formats_path):
    LENS = [9, 650, 200]
    d = decoder_from_gguf(ctx, formats_path, batch=LENS, embed=False, reserve=8, seed=3)
    d.fill_kv(seed=35)
    ctx.sync()
    _step_vs_oracle(ctx, d, LENS)
    del d


@pytest.mark.skipif(shutil.which("node") is None, reason="no node binary")
@pytest.mark.parametrize("fused", [False, True], ids=["key_by_key", "fused_step"])
def test_every_format_node_backend(ctx, formats_path, fused):
    _node_from_gguf(ctx, formats_path, fused)
