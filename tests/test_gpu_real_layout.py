"""GPU parity of Gemma-4-E2B's own layer layout (src/config/gemma4-e2b.ts:16-63,
src/engine.ts:1149-1152 and 1539-1625): head dim 512 on the global layers,
FFN 12288 and no K/V of their own on the layers past the unshared ones, which
attend over the cache of the last unshared layer of their attention kind.

A six-layer model keeps every case and the oracle quick: layers 0 (local),
1 (global) and 2 (local) own their caches; 3 and 5 (local) read layer 2's,
4 (global) reads layer 1's.

* the shared-cache forms of the fused attention (the one-launch matrix-core
  plan at head dims 256 and 512) and of the paged prologue equal the unfused
  path on the same inputs and leave the caches untouched;
* the per-key sequence and the fused step against the oracle's step, the
  fused step's K/V rows only in the producers' caches;
* the step that starts from the embedding row of the device-side token the
  previous step sampled, replayed from a HIP graph, against the oracle
  composition of the two steps;
* the ragged multi-sequence step against the oracle per sequence.
"""
import numpy as np
import pytest

import oracle as O
from decode_oracle import HostModel
from g4hip.decoder import BatchDecoder, Decoder, E2BShape
from gpu_util import assert_close, bits_equal
from test_gpu_batch_step import _step_vs_oracle

pytestmark = pytest.mark.gpu

MAX_SEQ = 1024
POS = 600  # past the 512 window


def small_real(**kw):
    return E2BShape.real(n_layers=6, n_unshared=3, global_layers=(1, 4), vocab=16384, **kw)


@pytest.fixture(scope="module")
def rdec(ctx):
    d = Decoder(ctx, small_real(), max_seq=MAX_SEQ, seed=21)
    d.fill_kv(POS, seed=22)
    ctx.sync()
    return d


def _snapshot(d):
    return (d.hidden.download(np.float32), [L.k_cache.download(np.uint16) for L in d.layers],
            [L.v_cache.download(np.uint16) for L in d.layers], d.token.download(np.uint32))


def _restore(d, snap):
    """hidden state, caches and the device token (the per-layer-embedding row
    a step reads; the previous step's sample overwrote it)."""
    d.hidden.upload(snap[0])
    for L, k, v in zip(d.layers, snap[1], snap[2]):
        L.k_cache.upload(k)
        L.v_cache.upload(v)
    d.token.upload(snap[3])


@pytest.mark.parametrize("layer", [2, 1])  # head dim 256, 512
def test_fused_attention_over_a_producer_cache(ctx, rdec, layer):
    """k_raw = v_raw = k_norm_w = NULL: q_norm + RoPE and attention over the
    cache as it is, equal to fusedPerHeadNormRope + attnDecode over it
    (1e-5: the fused form rounds q to hi + lo f16 parts); nothing stored."""
    d, s = rdec, rdec.s
    L = d.layers[layer]
    hd, glob = s.hd(layer), s.is_global(layer)
    theta = s.theta_global if glob else s.theta_local
    window = 0 if glob else s.window
    q0 = O.gen_normal_f32(31 + layer, s.n_q_heads * hd)
    kc0, vc0 = L.k_cache.download(np.uint16), L.v_cache.download(np.uint16)
    for pos in (0, 17, POS - 1):
        d.q.upload(q0)
        d.set_position(pos)
        print(f"[shared attn] layer {layer} hd {hd} pos {pos}", flush=True)
        ctx.attnDecodeFused(d.q, None, None, L.q_norm, None, d.rope_freqs, L.k_cache, L.v_cache, d.attn,
                            d.attn_params[layer], d.attn_ws, d.pos)
        ctx.sync()
        got = d.attn.download(np.float32, s.n_q_heads * hd)
        d.q.upload(q0)
        ctx.fusedPerHeadNormRope(d.q, L.q_norm, s.n_q_heads, hd, s.eps, pos, theta, int(glob), d.rope_freqs)
        ctx.attnDecode(d.q, L.k_cache, L.v_cache, d.attn, s.n_q_heads, s.n_kv_heads, hd, pos + 1,
                       1.0, window)
        ctx.sync()
        want = d.attn.download(np.float32, s.n_q_heads * hd)
        assert_close(got, want, rel=1e-5, what=f"shared-cache attention layer {layer} pos {pos}")
        qn = d.q.download(np.float32, s.n_q_heads * hd)
        ref = O.attention(qn, kc0, vc0, s.n_q_heads, s.n_kv_heads, hd, pos + 1, 1.0, window)
        assert_close(got, ref, what=f"shared-cache attention vs oracle layer {layer} pos {pos}")
        assert np.array_equal(L.k_cache.download(np.uint16), kc0)
        assert np.array_equal(L.v_cache.download(np.uint16), vc0)


def test_real_layout_step_vs_oracle(ctx, rdec):
    d, s = rdec, rdec.s
    snap = _snapshot(d)
    kcs, vcs = [k.copy() for k in snap[1]], [v.copy() for v in snap[2]]
    x_ref, logits_ref = HostModel(d).step(snap[0], kcs, vcs, POS)

    d.step_reference(POS)
    ctx.sync()
    print(f"[real layout] per-key hidden rel-L2 {O.rel_l2(d.hidden.download(np.float32), x_ref):.2e}", flush=True)
    assert_close(d.hidden.download(np.float32), x_ref, what="per-key hidden")
    assert_close(d.logits.download(np.float32), logits_ref, what="per-key logits")

    _restore(d, snap)
    d.set_position(POS)
    d.step_fused()
    ctx.sync()
    print(f"[real layout] fused hidden rel-L2 {O.rel_l2(d.hidden.download(np.float32), x_ref):.2e}", flush=True)
    assert_close(d.hidden.download(np.float32), x_ref, what="fused hidden")
    lg = d.logits.download(np.float32)
    assert_close(lg, logits_ref, what="fused logits")
    assert int(d.token.download(np.uint32)[0]) == O.argmax(lg)
    # the producers' caches took the oracle's rows at POS and changed nowhere else
    for il in range(s.n_layers):
        if not s.is_producer(il):
            continue
        kv = s.kv_dim_of(il)
        row = slice(POS * kv, (POS + 1) * kv)
        for nm, got, want, before in (("k", d.layers[il].k_cache.download(np.uint16), kcs[il], snap[1][il]),
                                      ("v", d.layers[il].v_cache.download(np.uint16), vcs[il], snap[2][il])):
            assert_close(got[row].view(np.float16).astype(np.float32),
                         want[row].view(np.float16).astype(np.float32), what=f"{nm} row layer {il}")
            other = np.ones(got.size, bool)
            other[row] = False
            assert np.array_equal(got[other], before[other]), (nm, il)
    _restore(d, snap)


def test_embedding_token_feedback_graph(ctx):
    """Two replays of the captured step with the embedding table: the first
    starts from token T0's row, the second from the row of the token the
    first sampled on the device."""
    d = Decoder(ctx, small_real(), max_seq=MAX_SEQ, seed=23, embed=True)
    d.fill_kv(POS, seed=24)
    s = d.s
    T0 = 4242
    d.set_token(T0)
    d.set_position(POS)
    ctx.sync()
    hm = HostModel(d)
    kcs = [L.k_cache.download(np.uint16) for L in d.layers]
    vcs = [L.v_cache.download(np.uint16) for L in d.layers]
    g = d.capture_fused()
    assert ctx.graph_kernel_nodes(g) == d.launches_per_step_fused()
    try:
        x_prev = None
        tok = T0
        for i in range(2):
            ctx.graph_launch(g)
            ctx.sync()
            x_ref, lg_ref = hm.step(hm.embed(tok), kcs, vcs, POS + i, token=tok)
            lg = d.logits.download(np.float32)
            print(f"[embed feedback] replay {i}: token in {tok}, hidden rel-L2 "
                  f"{O.rel_l2(d.hidden.download(np.float32), x_ref):.2e}", flush=True)
            assert_close(d.hidden.download(np.float32), x_ref, what=f"hidden replay {i}")
            assert_close(lg, lg_ref, what=f"logits replay {i}")
            new = int(d.token.download(np.uint32)[0])
            assert new == O.argmax(lg)  # bit-exact on the device's logits
            # on the oracle's logits the sampled token is a maximum up to the logits' tolerance
            assert lg_ref[new] >= lg_ref.max() - 1e-3 * np.abs(lg_ref).max()
            if x_prev is not None:
                assert not np.array_equal(x_prev, d.hidden.download(np.float32))
            x_prev = d.hidden.download(np.float32)
            tok = new
        assert int(d.pos.download(np.uint32)[0]) == POS + 2
    finally:
        ctx.graph_destroy(g)
    del d


def test_paged_prologue_q_only(ctx):
    """g4_pagedAttnPrologue without k/v parts: q_out as the full prologue
    writes it, pools untouched."""
    lens = [0, 17, 513]
    d = BatchDecoder(ctx, lens, small_real(), seed=25, reserve=4)
    d.fill_kv(seed=26)
    s, B = d.s, d.B
    il = 1  # global, head dim 512
    Q, KV = s.q_dim_of(il), s.kv_dim_of(il)
    L = d.layers[il]
    qp = O.gen_normal_f32(41, 2 * B * Q)
    kp = O.gen_normal_f32(42, 2 * B * KV)
    vp = O.gen_normal_f32(43, 2 * B * KV)
    d.q_parts.upload(qp)
    d.k_parts.upload(kp)
    d.v_parts.upload(vp)
    d.seq_lens.upload(np.asarray(lens, np.uint32) + 1)
    k0, v0 = L.k_cache.download(np.uint16), L.v_cache.download(np.uint16)
    ctx.pagedAttnPrologue(d.q_parts, None, None, 2, L.q_norm, None, d.rope_freqs, d.q, None, None, d.page_table,
                          d.seq_lens, d.pro_params[il], d.rope_cs[True], d.rope_rows)
    ctx.sync()
    q_only = d.q.download(np.float32, B * Q)
    assert np.array_equal(L.k_cache.download(np.uint16), k0)
    assert np.array_equal(L.v_cache.download(np.uint16), v0)
    ctx.pagedAttnPrologue(d.q_parts, d.k_parts, d.v_parts, 2, L.q_norm, L.k_norm, d.rope_freqs, d.q, L.k_cache,
                          L.v_cache, d.page_table, d.seq_lens, d.pro_params[il], d.rope_cs[True], d.rope_rows)
    ctx.sync()
    assert bits_equal(q_only, d.q.download(np.float32, B * Q))
    assert not np.array_equal(L.k_cache.download(np.uint16), k0)
    del d


def test_real_layout_batch_step_vs_oracle(ctx):
    lens = [0, 1, 17, 300, 513, 700]
    d = BatchDecoder(ctx, lens, small_real(), seed=27, reserve=4)
    d.fill_kv(seed=28)
    ctx.sync()
    print(f"[real layout batch] B={d.B}", flush=True)
    _step_vs_oracle(ctx, d, lens)
    del d
