"""GPU parity: norms, per-head norm + RoPE, GELU, softcap, KV store (f16 bits
exact), argmax / topk256 (indices bit-exact on identical logits)."""
import numpy as np
import pytest

import oracle as O
from gpu_util import assert_close, bits_equal
from test_oracle import _rule_argmax

pytestmark = pytest.mark.gpu


def test_rms_norm_and_fused_norm_add(ctx):
    for n in (1536, 2048, 100):
        x = O.gen_normal_f32(n, n, 0.5, 4.0)
        w = O.gen_normal_f16(n + 1, n, 1.0, 0.1)
        r = O.gen_normal_f32(n + 2, n)
        dx, dw, dr = ctx.from_numpy(x), ctx.from_numpy(w), ctx.from_numpy(r)
        out = ctx.empty(n, np.float32)
        ctx.rmsNorm(dx, dw, out, n, 1e-6)
        assert_close(out.download(np.float32), O.rms_norm(x, w, 1e-6), rel=1e-6, cos=0.99999999)
        ctx.fusedNormAdd(dx, dw, dr, out, n, 1e-6)
        assert_close(out.download(np.float32), O.fused_norm_add(x, w, r, 1e-6), rel=1e-6, cos=0.99999999)


def test_v_norm(ctx):
    for nh, hd in [(1, 256), (1, 512), (4, 256)]:
        x = O.gen_normal_f32(hd, nh * hd, 0.0, 67.0)
        d = ctx.from_numpy(x)
        ctx.perHeadRmsNormNoWeight(d, nh, hd, 1e-6)
        assert_close(d.download(np.float32), O.per_head_rms_norm_no_weight(x, nh, hd, 1e-6), rel=1e-6,
                     cos=0.99999999)


ROPE_CASES = [
    # (heads, head_dim, position, theta, apply_divisor): local layers (theta 1e4,
    # no divisor), global layers (theta 1e6, proportional table), long positions
    (8, 256, 0, 1e4, 0),
    (8, 256, 14, 1e4, 0),
    (1, 256, 511, 1e4, 0),
    (8, 512, 4095, 1e6, 1),
    (1, 512, 32767, 1e6, 1),
    (8, 256, 32767, 1e6, 0),
]


@pytest.mark.parametrize("nh,hd,pos,theta,div", ROPE_CASES)
def test_fused_per_head_norm_rope(ctx, nh, hd, pos, theta, div):
    x = O.gen_normal_f32(pos + hd, nh * hd, 0.0, 2.0)
    w = O.gen_normal_f16(pos + 1, hd, 1.0, 0.1)
    # real E2B table: 1.0 for the first quarter of the pairs, 1e30 (-> +Inf in f16) after
    table = np.where(np.arange(hd // 2) < hd // 8, 1.0, np.inf).astype(np.float16).view(np.uint16)
    ref = O.fused_per_head_norm_rope(x, w, nh, hd, 1e-6, pos, theta, div, table)
    d = ctx.from_numpy(x)
    ctx.fusedPerHeadNormRope(d, ctx.from_numpy(w), nh, hd, 1e-6, pos, theta, div, ctx.from_numpy(table))
    got = d.download(np.float32)
    assert_close(got, ref, rel=2e-6, cos=0.9999999, what=f"rope pos={pos}")
    # device-position variant
    d2 = ctx.from_numpy(x)
    pdev = ctx.from_numpy(np.array([pos], np.uint32))
    ctx.fusedPerHeadNormRope(d2, ctx.from_numpy(w), nh, hd, 1e-6, 0, theta, div, ctx.from_numpy(table),
                             position_dev=pdev)
    assert bits_equal(d2.download(np.float32), got)


def test_gelu_mul_and_softcap(ctx):
    n = 6144
    g = O.gen_normal_f32(1, n, 0.0, 3.0)
    u = O.gen_normal_f32(2, n)
    out = ctx.empty(n, np.float32)
    ctx.geluMul(ctx.from_numpy(g), ctx.from_numpy(u), out, n)
    assert_close(out.download(np.float32), O.gelu_mul(g, u), rel=1e-6, cos=0.99999999)
    x = np.concatenate([O.gen_normal_f32(3, 262144 - 8, 0.0, 20.0),
                        np.array([0, 450, 451, -1e6, 1e6, 30, -30, 1e-3], np.float32)])
    d = ctx.from_numpy(x)
    ctx.logitSoftcap(d, x.size, 30.0)
    y = d.download(np.float32)
    assert_close(y, O.logit_softcap(x, 30.0), rel=1e-6, cos=0.99999999)
    assert np.max(np.abs(y)) <= 30.0


def test_kv_cache_store_f16_bits(ctx):
    nkh, hd, max_seq = 1, 256, 64
    kc = ctx.zeros(max_seq * hd, np.uint16)
    vc = ctx.zeros(max_seq * hd, np.uint16)
    hk = np.zeros(max_seq * hd, np.uint16)
    hv = np.zeros(max_seq * hd, np.uint16)
    for pos in (0, 5, 63):
        k = O.gen_normal_f32(pos, hd, 0.0, 2.0)
        v = O.gen_normal_f32(pos + 100, hd, 0.0, 1e-5)    # f16 subnormal range
        k[:4] = [65504, 65520, -1e9, 6e-8]
        ctx.kvCacheStore(ctx.from_numpy(k), ctx.from_numpy(v), kc, vc, nkh, hd, pos, max_seq)
        O.kv_cache_store_f16(k, v, hk, hv, nkh, hd, pos)
    assert np.array_equal(kc.download(np.uint16), hk)
    assert np.array_equal(vc.download(np.uint16), hv)
    # device-position variant writes the same row
    kc2 = ctx.zeros(max_seq * hd, np.uint16)
    vc2 = ctx.zeros(max_seq * hd, np.uint16)
    k = O.gen_normal_f32(9, hd)
    pdev = ctx.from_numpy(np.array([17], np.uint32))
    ctx.kvCacheStore(ctx.from_numpy(k), ctx.from_numpy(k), kc2, vc2, nkh, hd, 0, max_seq, position_dev=pdev)
    row = kc2.download(np.uint16).reshape(max_seq, hd)
    assert np.array_equal(row[17], np.array([O.f32_to_f16_rne(float(a)) for a in k], np.uint16))
    assert not row[np.arange(max_seq) != 17].any()


def _argmax_topk(ctx, x):
    d = ctx.from_numpy(x)
    r = ctx.zeros(1, np.uint32)
    ctx.argmax(d, r, x.size)
    t = ctx.empty(512, np.float32)
    ctx.topk256(d, t, x.size)
    return int(r.download(np.uint32)[0]), t.download(np.float32)


def test_argmax_topk_fixture_logits(ctx):
    import os
    from conftest import GOLDEN

    lg = np.load(os.path.join(GOLDEN, "ref_fixtures.npz"), allow_pickle=False)["logits_pos14"]
    a, t = _argmax_topk(ctx, lg)
    assert a == O.argmax(lg) == 236777
    assert bits_equal(t, O.topk256(lg))


def test_argmax_topk_ties_and_specials(ctx):
    rng = np.random.default_rng(5)
    for trial in range(40):
        n = int(rng.choice([1, 255, 256, 257, 1000, 4096, 262144]))
        x = rng.integers(-3, 4, n).astype(np.float32)
        if trial % 5 == 0:
            x[rng.integers(0, n, 7)] = np.nan
        if trial % 7 == 0:
            x[:] = -np.inf
        if trial % 11 == 0:
            x[:] = np.float32(-1e30)
            x[rng.integers(0, n)] = np.float32(-1e29)
        if trial % 3 == 0:
            x[rng.integers(0, n, 3)] = -0.0
        a, t = _argmax_topk(ctx, x)
        assert a == O.argmax(x) == _rule_argmax(x), trial
        assert bits_equal(t, O.topk256(x)), trial


@pytest.mark.parametrize("size,batch", [(262144, 8), (262144, 32), (1000, 5), (257, 64)])
def test_argmax_topk_batch_rows(ctx, size, batch):
    """Sampling over many rows: each row's result equals the one-row rule."""
    rng = np.random.default_rng(size + batch)
    X = rng.integers(-3, 4, (batch, size)).astype(np.float32)
    X[1::3, rng.integers(0, size, 5)] = np.nan
    X[2] = -np.inf
    d = ctx.from_numpy(X)
    r = ctx.zeros(batch, np.uint32)
    t = ctx.empty(batch * 512, np.float32)
    ctx.argmaxBatch(d, r, size, batch)
    ctx.topk256Batch(d, t, size, batch)
    R = r.download(np.uint32)
    T = t.download(np.float32).reshape(batch, 512)
    for b in range(batch):
        assert R[b] == O.argmax(X[b]), b
        assert bits_equal(T[b], O.topk256(X[b])), b


@pytest.mark.parametrize("size,batch", [(262144, 1), (1000, 7), (4097, 32)])
def test_argmax_advance(ctx, size, batch):
    """Each row's argmax (the one-row rule, ties included) and
    positions[r] += delta, over three calls in a row."""
    rng = np.random.default_rng(size * 3 + batch)
    pos0 = rng.integers(0, 1000, batch).astype(np.uint32)
    p = ctx.from_numpy(pos0)
    r = ctx.zeros(batch, np.uint32)
    for call in range(3):
        X = rng.integers(-3, 4, (batch, size)).astype(np.float32)
        X[::2, rng.integers(0, size, 3)] = np.nan
        ctx.argmaxAdvance(ctx.from_numpy(X), r, size, batch, p, 2)
        R = r.download(np.uint32)
        for b in range(batch):
            assert R[b] == O.argmax(X[b]), (call, b)
        assert np.array_equal(p.download(np.uint32), pos0 + 2 * (call + 1)), call


def test_embedding_lookup(ctx):
    """shaders/embedding_lookup.wgsl: E2B's H = 1536 (vector path), an odd H
    (scalar path), host and device token ids, and an out-of-range device token."""
    rng = np.random.default_rng(11)
    for H, rows in ((1536, 97), (250, 13)):
        table = (rng.standard_normal((rows, H)) * 0.05).astype(np.float16)
        d_tab = ctx.from_numpy(table.view(np.uint16))
        out = ctx.empty(H, np.float32)
        for tok in (0, rows // 2, rows - 1):
            ctx.embeddingLookup(d_tab, rows, out, H, tok)
            assert bits_equal(out.download(np.float32), O.embedding_lookup(table, H, tok))
            tdev = ctx.from_numpy(np.array([tok], np.uint32))
            ctx.embeddingLookup(d_tab, rows, out, H, 0, token_dev=tdev)
            assert bits_equal(out.download(np.float32), O.embedding_lookup(table, H, tok))
        tdev = ctx.from_numpy(np.array([rows], np.uint32))
        ctx.embeddingLookup(d_tab, rows, out, H, 0, token_dev=tdev)
        assert not out.download(np.float32).any()
        with pytest.raises(Exception):
            ctx.embeddingLookup(d_tab, rows, out, H, rows)


@pytest.mark.parametrize("policy", [0, 1, 2])
def test_stream_read_probe_reads_every_word_once(ctx, policy):
    """The streaming probe's workgroups together read every 16-byte chunk
    once: the xor of their words is the xor of the buffer's words."""
    rng = np.random.default_rng(policy)
    words = rng.integers(0, 2 ** 32, 1 << 20, dtype=np.uint64).astype(np.uint32)
    for nbytes, nwgs in ((words.nbytes, 300), (words.nbytes - 16 * 77, 1), (4096 + 16 * 3, 1000)):
        buf = ctx.from_numpy(words)
        sink = ctx.zeros(nwgs, np.uint32)
        ctx.streamRead(buf, nbytes, policy, nwgs, sink)
        got = np.bitwise_xor.reduce(sink.download(np.uint32))
        assert got == np.bitwise_xor.reduce(words[:nbytes // 4]), (nbytes, nwgs)
