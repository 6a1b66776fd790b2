"""GPU parity of the ragged multi-sequence decode step.

* The paged attention block on identical inputs: per sequence within rel-L2
  1e-5 of the single-sequence fused kernel over a dense copy of its pages (the
  two merge chunks and sum squares in different orders), within rel-L2 1e-3
  of the oracle, K/V rows appended only where the table says.
* The whole step: every sequence against the oracle's single-sequence step on
  its own dense caches, at rel-L2 1e-3 / cosine 0.9999 (or, for the rare
  sequence whose step is that sensitive to one f16 ulp of its newest K/V
  row, the oracle's own movement under such a change): the 18 edge lengths
  above, and the ragged serving shape of 32 sequences with lengths drawn from
  U(128, 8192), once with the benchmark's weight generator and once with
  real-model-like weights (zero-mean Q4_K, Q6_K scales over the whole int8
  range, which the matrix-core weight operand rounds once above 2048).
  With the benchmark's generator the Q4_K weights have a mean near +0.35, so
  for sequences whose normalised FFN input sums negative every GELU input is
  far below -5.5 and f32 tanh saturates: the product is exactly 0 (as in the
  reference's f32 shader and the oracle, which carries tanh as an f32 value),
  and the post-FFN RMSNorm then sees an all-zero vector.
* HIP-graph replays equal eager steps bit for bit."""
import numpy as np
import pytest

import oracle as O
import synth
from decode_oracle import HostModel, gelu_mul_f32
from g4hip.decoder import BatchDecoder, E2BShape
from gpu_util import assert_close, bits_equal

pytestmark = pytest.mark.gpu

# lengths cover: the first token, page edges (15/16/17), the window edge
# (511/512/513) and beyond it, and a long global context
LENS = [0, 1, 15, 16, 17, 31, 300, 511, 512, 513, 530, 700, 1000, 5, 64, 100, 255, 256]


@pytest.fixture(scope="module")
def bdec(ctx):
    # layer 0 local (window 512), layer 1 global; a smaller vocabulary keeps the oracle quick
    shape = E2BShape(n_layers=2, global_layers=(1,), vocab=16384)
    d = BatchDecoder(ctx, LENS, shape, seed=11, reserve=8)
    d.fill_kv(seed=12)
    ctx.sync()
    return d


def _pools(d):
    return [(L.k_cache.download(np.uint16), L.v_cache.download(np.uint16)) for L in d.layers]


def _restore(d, hidden, pools, lens):
    d.hidden.upload(hidden)
    for L, (k, v) in zip(d.layers, pools):
        L.k_cache.upload(k)
        L.v_cache.upload(v)
    d.set_lengths(lens)


def _dense(d, pool, seq, n, kv=None):
    """Sequence `seq`'s first n rows gathered from a pool of rows of kv
    values (default: the uniform layer's), as a dense cache with one spare
    row."""
    kv = kv or d.s.kv_dim
    P = pool.reshape(-1, kv)
    out = np.zeros((n + 1, kv), np.uint16)
    for t in range(n):
        out[t] = P[d.pool_row(seq, t)]
    return out.reshape(-1)


STEP_REL = 1e-3
# A sequence whose oracle step itself moves by more than STEP_REL when its
# newest f16 K/V row is rounded toward zero instead of to nearest (one ulp of
# the cache; a k that differs in its last f32 bits flips such ulps) is held
# to that movement; likewise, times GELU_MARGIN, for the GELU's all-f32 form.
GELU_MARGIN = 4.0


def test_paged_attention_block_matches_dense_and_oracle(ctx, bdec):
    d, s, B = bdec, bdec.s, bdec.B
    kv, table = s.kv_dim, d.rope_freqs.download(np.uint16)
    rng = np.random.default_rng(21)
    Q = rng.normal(0, 2, (B, s.q_dim)).astype(np.float32)
    K = rng.normal(0, 2, (B, kv)).astype(np.float32)
    V = rng.normal(0, 2, (B, kv)).astype(np.float32)
    dq, dk, dv = ctx.from_numpy(Q), ctx.from_numpy(K), ctx.from_numpy(V)
    for il, L in enumerate(d.layers):
        glob = s.is_global(il)
        theta = s.theta_global if glob else s.theta_local
        window = 0 if glob else s.window
        k0 = L.k_cache.download(np.uint16)
        v0 = L.v_cache.download(np.uint16)
        d.set_lengths(np.array(LENS, np.uint32) + 1)  # the step's advance already applied
        ctx.pagedAttnDecodeFused(dq, dk, dv, L.q_norm, L.k_norm, d.rope_freqs, L.k_cache, L.v_cache,
                                 d.page_table, d.seq_lens, d.attn, d.pro_params[il], d.attn_ws)
        A = d.attn.download(np.float32).reshape(B, -1)
        k1 = L.k_cache.download(np.uint16).reshape(-1, kv)
        v1 = L.v_cache.download(np.uint16).reshape(-1, kv)
        qn, kn = L.q_norm.download(np.uint16), L.k_norm.download(np.uint16)
        for b, pos in enumerate(LENS):
            # dense copy of the sequence's pages, then the single-sequence kernel
            kc, vc = _dense(d, k0, b, pos), _dense(d, v0, b, pos)
            kdev, vdev = ctx.from_numpy(kc), ctx.from_numpy(vc)
            ap = ctx.attn_fused_params(s.n_q_heads, s.n_kv_heads, s.head_dim, pos + 1, window, s.eps, theta,
                                       int(glob))
            ws = ctx.zeros(ctx.attn_fused_workspace_bytes(ap), np.uint8)
            out = ctx.empty(s.q_dim, np.float32)
            ctx.attnDecodeFused(ctx.from_numpy(Q[b]), ctx.from_numpy(K[b]), ctx.from_numpy(V[b]), L.q_norm,
                                L.k_norm, d.rope_freqs, kdev, vdev, out, ap, ws,
                                ctx.from_numpy(np.array([pos], np.uint32)))
            # the single-sequence kernel merges its chunks in another order and
            # sums the norms' squares in another order: f32 rounding apart
            assert_close(A[b], out.download(np.float32), rel=1e-5, cos=0.9999999, what=f"dense {il} {b}")
            r = d.pool_row(b, pos)
            kd = kdev.download(np.uint16).reshape(-1, kv)
            vd = vdev.download(np.uint16).reshape(-1, kv)
            for got, want in ((k1[r], kd[pos]), (v1[r], vd[pos])):
                assert np.max(np.abs(got.astype(np.int32) - want.astype(np.int32))) <= 1, (il, b)
            # the oracle on the same inputs
            q = O.fused_per_head_norm_rope(Q[b], qn, s.n_q_heads, s.head_dim, s.eps, pos, theta, int(glob), table)
            k = O.fused_per_head_norm_rope(K[b], kn, s.n_kv_heads, s.head_dim, s.eps, pos, theta, int(glob), table)
            v = O.per_head_rms_norm_no_weight(V[b], s.n_kv_heads, s.head_dim, s.eps)
            O.kv_cache_store_f16(k, v, kc, vc, s.n_kv_heads, s.head_dim, pos)
            a = O.attention(q, kc, vc, s.n_q_heads, s.n_kv_heads, s.head_dim, pos + 1, 1.0, window)
            assert_close(A[b], a, what=f"layer {il} seq {b} len {pos}")
            for got, want in ((k1[r], kc.reshape(-1, kv)[pos]), (v1[r], vc.reshape(-1, kv)[pos])):
                g16, w16 = got.view(np.float16).astype(np.float32), want.view(np.float16).astype(np.float32)
                assert np.all(np.abs(g16 - w16) <= 2.0 ** -10 * np.maximum(np.abs(w16), 2.0 ** -14)), (il, b)
        written = {d.pool_row(b, pos) for b, pos in enumerate(LENS)}
        for before, after in ((k0, k1), (v0, v1)):
            diff = np.nonzero(np.any(before.reshape(-1, kv) != after, axis=1))[0]
            assert set(diff.tolist()) <= written
        L.k_cache.upload(k0)
        L.v_cache.upload(v0)
    d.set_lengths(np.array(LENS, np.uint32))


def test_prologue_then_paged_decode_matches_fused_and_oracle(ctx, bdec):
    """The step's attention path (prologue over split-K partial sums, then the
    paged decode) against the one-launch fused block and the oracle."""
    d, s, B = bdec, bdec.s, bdec.B
    kv, table = s.kv_dim, d.rope_freqs.download(np.uint16)
    rng = np.random.default_rng(31)
    Q = rng.normal(0, 2, (B, s.q_dim)).astype(np.float32)
    K = rng.normal(0, 2, (B, kv)).astype(np.float32)
    V = rng.normal(0, 2, (B, kv)).astype(np.float32)
    # two chunks whose in-order sum is exactly Q (K, V)
    parts = [ctx.from_numpy(np.concatenate([0.5 * A, 0.5 * A])) for A in (Q, K, V)]
    dq, dk, dv = ctx.from_numpy(Q), ctx.from_numpy(K), ctx.from_numpy(V)
    for il, L in enumerate(d.layers):
        glob = s.is_global(il)
        theta = s.theta_global if glob else s.theta_local
        window = 0 if glob else s.window
        k0, v0 = L.k_cache.download(np.uint16), L.v_cache.download(np.uint16)
        d.set_lengths(np.array(LENS, np.uint32) + 1)
        ctx.pagedAttnDecodeFused(dq, dk, dv, L.q_norm, L.k_norm, d.rope_freqs, L.k_cache, L.v_cache, d.page_table,
                                 d.seq_lens, d.attn, d.pro_params[il], d.attn_ws)
        A_fused = d.attn.download(np.float32).reshape(B, -1)
        kf, vf = L.k_cache.download(np.uint16).reshape(-1, kv), L.v_cache.download(np.uint16).reshape(-1, kv)
        L.k_cache.upload(k0)
        L.v_cache.upload(v0)
        ctx.pagedAttnPrologue(parts[0], parts[1], parts[2], 2, L.q_norm, L.k_norm, d.rope_freqs, d.q, L.k_cache,
                              L.v_cache, d.page_table, d.seq_lens, d.pro_params[il])
        ctx.pagedAttnDecode(d.q, L.k_cache, L.v_cache, d.page_table, d.seq_lens, d.attn, d.attn_params[il],
                            d.attn_ws)
        A = d.attn.download(np.float32).reshape(B, -1)
        QR = d.q.download(np.float32).reshape(B, -1)
        kp, vp = L.k_cache.download(np.uint16).reshape(-1, kv), L.v_cache.download(np.uint16).reshape(-1, kv)
        qn, kn = L.q_norm.download(np.uint16), L.k_norm.download(np.uint16)
        for b, pos in enumerate(LENS):
            q = O.fused_per_head_norm_rope(Q[b], qn, s.n_q_heads, s.head_dim, s.eps, pos, theta, int(glob), table)
            assert_close(QR[b], q, rel=1e-5, cos=0.9999999, what=f"roped q layer {il} seq {b}")
            r = d.pool_row(b, pos)
            for got, want in ((kp[r], kf[r]), (vp[r], vf[r])):  # the fused block's f16 rows, to 1 ulp
                g16, w16 = got.view(np.float16).astype(np.float32), want.view(np.float16).astype(np.float32)
                assert np.all(np.abs(g16 - w16) <= 2.0 ** -10 * np.maximum(np.abs(w16), 2.0 ** -14)), (il, b)
            kc, vc = _dense(d, k0, b, pos), _dense(d, v0, b, pos)
            kc.reshape(-1, kv)[pos] = kp[r]
            vc.reshape(-1, kv)[pos] = vp[r]
            a = O.attention(q, kc, vc, s.n_q_heads, s.n_kv_heads, s.head_dim, pos + 1, 1.0, window)
            assert_close(A[b], a, what=f"attention layer {il} seq {b} len {pos}")
            assert_close(A[b], A_fused[b], what=f"vs fused layer {il} seq {b}")
        L.k_cache.upload(k0)
        L.v_cache.upload(v0)
    d.set_lengths(np.array(LENS, np.uint32))


def test_batch_step_matches_oracle_per_sequence(ctx, bdec):
    _step_vs_oracle(ctx, bdec, LENS)


@pytest.mark.parametrize("weights", ["benchmark", "realistic"])
def test_batch_step_serving_shape(ctx, weights):
    """32 sequences, lengths ~ U(128, 8192) (seeded), a local and a global
    layer, 16384-token vocabulary."""
    lens = np.random.default_rng(2024).integers(128, 8193, 32)
    shape = E2BShape(n_layers=2, global_layers=(1,), vocab=16384)
    d = BatchDecoder(ctx, lens, shape, seed=17, reserve=4)
    if weights == "realistic":
        synth.make_realistic(d)
    d.fill_kv(seed=18)
    ctx.sync()
    print(f"[batch step] B=32 {weights}: mean length {lens.mean():.0f}, {d.num_pages} pages", flush=True)
    _step_vs_oracle(ctx, d, [int(x) for x in lens])
    del d


def _step_vs_oracle(ctx, d, LENS):
    s, B = d.s, d.B
    hm = HostModel(d)
    hidden0 = d.hidden.download(np.float32).reshape(B, s.hidden)
    tokens0 = d.tokens.download(np.uint32)  # (the per-layer-embedding rows)
    pools0 = _pools(d)
    lens0 = d.lens_host.copy()

    d.step()
    ctx.sync()
    assert np.array_equal(d.seq_lens.download(np.uint32), lens0 + 1)
    H = d.hidden.download(np.float32).reshape(B, s.hidden)
    LG = d.logits.download(np.float32).reshape(B, s.vocab)
    TOK = d.tokens.download(np.uint32)
    pools1 = _pools(d)
    kvs = [s.kv_dim_of(il) for il in range(s.n_layers)]
    refs, tol = [], []
    for b, L in enumerate(LENS):
        # (a layer reading a producer's pool has that pool here; the oracle reads the producer's entry)
        kcs = [_dense(d, k, b, L, kvs[il]) for il, (k, _) in enumerate(pools0)]
        vcs = [_dense(d, v, b, L, kvs[il]) for il, (_, v) in enumerate(pools0)]
        x, logits = hm.step(hidden0[b], kcs, vcs, L, token=int(tokens0[b]))
        refs.append((x, logits, kcs, vcs))
        # the step's own dependence on the f16 cache's resolution: the oracle
        # against itself with its new K/V rows one ulp off (rounded toward
        # zero), and on the last bits of the GELU (the shader's all-f32 form)
        kz = [_dense(d, k, b, L, kvs[il]) for il, (k, _) in enumerate(pools0)]
        vz = [_dense(d, v, b, L, kvs[il]) for il, (_, v) in enumerate(pools0)]
        xz, lgz = hm.step(hidden0[b], kz, vz, L, row_toward_zero=True, token=int(tokens0[b]))
        x32, lg32 = hm.step(hidden0[b], [k.copy() for k in kcs], [v.copy() for v in vcs], L, gelu=gelu_mul_f32,
                            token=int(tokens0[b]))
        tol.append(max(STEP_REL, O.rel_l2(xz, x), O.rel_l2(lgz, logits),
                       GELU_MARGIN * O.rel_l2(x32, x), GELU_MARGIN * O.rel_l2(lg32, logits)))
    rh = [O.rel_l2(H[b], r[0]) for b, r in enumerate(refs)]
    rl = [O.rel_l2(LG[b], r[1]) for b, r in enumerate(refs)]
    print(f"[batch step] B={B}: max rel-L2 hidden {max(rh):.2e} logits {max(rl):.2e}, "
          f"median hidden {np.median(rh):.2e}; sequences whose own sensitivity sets the bound "
          f"(seq, len, bound, error): "
          f"{[(b, LENS[b], round(t, 5), round(rh[b], 5)) for b, t in enumerate(tol) if t > STEP_REL]}", flush=True)
    for b, L in enumerate(LENS):
        x, logits, kcs, vcs = refs[b]
        assert_close(H[b], x, rel=tol[b], what=f"hidden seq {b} len {L}")
        assert_close(LG[b], logits, rel=tol[b], what=f"logits seq {b} len {L}")
        assert TOK[b] == O.argmax(LG[b]), b
        r = d.pool_row(b, L)
        for il in range(s.n_layers):
            if not s.is_producer(il):
                continue
            for got, ref, nm in ((pools1[il][0], kcs[il], "k"), (pools1[il][1], vcs[il], "v")):
                row = got.reshape(-1, kvs[il])[r].view(np.float16).astype(np.float32)
                want = ref.reshape(-1, kvs[il])[L].view(np.float16).astype(np.float32)
                # layer 0's rows depend on the input only; later rows on the layers before
                assert_close(row, want, rel=STEP_REL if il == 0 else tol[b], what=f"{nm} row seq {b} layer {il}")
    # nothing but the appended rows changed in the pools
    written = sorted(d.pool_row(b, L) for b, L in enumerate(LENS))
    for il in range(s.n_layers):
        for before, after in ((pools0[il][0], pools1[il][0]), (pools0[il][1], pools1[il][1])):
            diff = np.nonzero(np.any(before.reshape(-1, kvs[il]) != after.reshape(-1, kvs[il]), axis=1))[0]
            assert set(diff.tolist()) <= set(written)
    _restore(d, hidden0.reshape(-1), pools0, lens0)


def test_batch_graph_replay_matches_eager(ctx, bdec):
    d, B = bdec, bdec.B
    hidden0 = d.hidden.download(np.float32)
    pools0 = _pools(d)
    lens0 = d.lens_host.copy()
    eager = []
    for _ in range(3):
        d.step()
        ctx.sync()
        eager.append((d.hidden.download(np.float32), d.logits.download(np.float32), d.tokens.download(np.uint32)))
    _restore(d, hidden0, pools0, lens0)
    g = d.capture()
    try:
        for i in range(3):
            ctx.graph_launch(g)
            ctx.sync()
            _ = d.seq_lens.download(np.uint32)  # eager work between replays
            assert bits_equal(d.hidden.download(np.float32), eager[i][0]), i
            assert bits_equal(d.logits.download(np.float32), eager[i][1]), i
            assert np.array_equal(d.tokens.download(np.uint32), eager[i][2]), i
        assert np.array_equal(d.seq_lens.download(np.uint32), lens0 + 3)
    finally:
        ctx.graph_destroy(g)
        _restore(d, hidden0, pools0, lens0)


def test_paged_fused_rejects_bad_shapes(ctx, bdec):
    d = bdec
    p = d.pro_params[0]
    bad = ctx.paged_fused_params(d.B, 8, 1, 256, 16, 2, 64, d.num_pages, 0, 1e-6, 1e4, 0)
    with pytest.raises(Exception, match="exceeds the page table"):
        ctx.pagedAttnDecodeFused(d.q, d.q, d.q, d.layers[0].q_norm, d.layers[0].k_norm, None, d.layers[0].k_cache,
                                 d.layers[0].v_cache, d.page_table, d.seq_lens, d.attn, bad, d.attn_ws)
    small = ctx.zeros(16, np.uint8)
    with pytest.raises(Exception, match="workspace"):
        ctx.pagedAttnDecodeFused(d.q, d.q, d.q, d.layers[0].q_norm, d.layers[0].k_norm, None, d.layers[0].k_cache,
                                 d.layers[0].v_cache, d.page_table, d.seq_lens, d.attn, p, small)


def test_attention_writes_o_projection_operands(ctx, bdec):
    """The paged attention's merge also writes its output as the o
    projection's matrix-core operand blocks: the f16 hi/lo planes and the
    scales equal what the prep kernel builds from the same f32 output, the
    sub-block sums agree to f32 rounding, and the o projection from them
    matches the one that converts the f32 activations itself."""
    d, s, B = bdec, bdec.s, bdec.B
    L = d.layers[1]
    d.set_lengths(np.array(LENS, np.uint32) + 1)
    ctx.pagedAttnDecode(d.q, L.k_cache, L.v_cache, d.page_table, d.seq_lens, d.attn, d.attn_params[1], d.attn_ws,
                        ops=d.aops)
    got_ops = d.aops.download(np.uint8)
    ref_ops = ctx.zeros(d.aops.nbytes, np.uint8)
    ctx.batchPrep(d.attn, 1, None, None, None, None, ctx.empty(B * s.q_dim, np.float32), s.q_dim, B, s.eps,
                  ops=ref_ops)
    want = ref_ops.download(np.uint8)
    ntv = 2 if B > 16 else 1
    blk = ntv * (8 * 2 * 1024 + 1024 + 64)
    main, sums = ntv * 8 * 2 * 1024, ntv * 1024
    g3, w3 = got_ops.reshape(-1, blk), want.reshape(-1, blk)
    assert g3.shape[0] == s.q_dim // 256
    live = np.zeros((ntv * 16,), bool)
    live[:B] = True
    # main planes: [t][s][h][lane] 16 B, lane = c + 16 q (vector 16 t + c)
    gm = g3[:, :main].reshape(-1, ntv, 8, 2, 4, 16, 16)
    wm = w3[:, :main].reshape(-1, ntv, 8, 2, 4, 16, 16)
    lv = live.reshape(ntv, 16)
    for t in range(ntv):
        assert np.array_equal(gm[:, t][:, :, :, :, lv[t]], wm[:, t][:, :, :, :, lv[t]]), t
    gs = g3[:, main + sums:].reshape(-1, ntv, 16, 4).view(np.float32)
    ws_ = w3[:, main + sums:].reshape(-1, ntv, 16, 4).view(np.float32)
    assert np.array_equal(gs[:, :, :, 0][:, lv], ws_[:, :, :, 0][:, lv])
    # sums: [t][lane] 16 B, lane = c + 16 (s >> 1), 4 halves (3 parts + 0) per sub-block s
    gsum = g3[:, main:main + sums].reshape(-1, ntv, 4, 16, 16).view(np.float16).reshape(-1, ntv, 4, 16, 2, 4)
    wsum = w3[:, main:main + sums].reshape(-1, ntv, 4, 16, 16).view(np.float16).reshape(-1, ntv, 4, 16, 2, 4)
    gsum = gsum.astype(np.float64).sum(-1)
    wsum = wsum.astype(np.float64).sum(-1)
    for t in range(ntv):
        g_, w_ = gsum[:, t][:, :, lv[t]], wsum[:, t][:, :, lv[t]]
        assert np.allclose(g_, w_, rtol=1e-6, atol=1e-6 * np.abs(w_).max()), t
    a = ctx.empty(d.ks_q * B * s.hidden, np.float32)
    b = ctx.empty(d.ks_q * B * s.hidden, np.float32)
    na = ctx.matmulSegmentsBatchPartial("q4k", d.attn, [L.wo], [a], [s.hidden], s.q_dim, B, d.ks_q, ops=d.aops)
    nb = ctx.matmulSegmentsBatchPartial("q4k", d.attn, [L.wo], [b], [s.hidden], s.q_dim, B, d.ks_q)
    A = a.download(np.float32)[:na * B * s.hidden].reshape(na, B, -1).sum(0)
    Bm = b.download(np.float32)[:nb * B * s.hidden].reshape(nb, B, -1).sum(0)
    wo = L.wo.download(np.uint8)
    X = d.attn.download(np.float32).reshape(B, -1)
    for v in range(B):
        assert_close(A[v], Bm[v], rel=1e-6, cos=0.99999999, what=f"o with operand blocks, seq {v}")
        assert_close(A[v], O.matmul(X[v], wo, s.hidden, s.q_dim, "q4k"), what=f"o vs oracle, seq {v}")
    d.set_lengths(np.array(LENS, np.uint32))
