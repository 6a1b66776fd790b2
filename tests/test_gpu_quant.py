"""GPU parity: Q4_K/Q6_K unpack (bit-exact), quantized matvec (rel-L2 <= 1e-3,
cos >= 0.9999 against the f64 oracle), the fused norm/GELU matvecs, and the
device-side synthetic generators (bit-exact against the oracle's)."""
import struct

import numpy as np
import pytest

import oracle as O
from gpu_util import assert_close, bits_equal
from test_oracle import q4k_edge_blocks

pytestmark = pytest.mark.gpu


def test_dequant_q4k_bit_exact(ctx):
    rng = np.random.default_rng(0)
    b = q4k_edge_blocks(rng, 3000)
    n = b.size // 144
    db = ctx.from_numpy(b)
    out = ctx.empty(n * 256, np.float32)
    ctx.dequant_q4k(db, n, out)
    assert bits_equal(out.download(np.float32), O.dequant_q4k(b))


def test_dequant_q6k_bit_exact(ctx):
    b = O.gen_q6k(3, 3001).reshape(3001, 210).copy()
    b[::7, 208:210] = np.frombuffer(struct.pack("<H", 0x0001), np.uint8)
    b[1::7, 208:210] = np.frombuffer(struct.pack("<H", 0xbc00), np.uint8)
    b[2::7, 208:210] = np.frombuffer(struct.pack("<H", 0x7bff), np.uint8)
    b = b.reshape(-1)
    db = ctx.from_numpy(b)
    out = ctx.empty(3001 * 256, np.float32)
    ctx.dequant_q6k(db, 3001, out)
    assert bits_equal(out.download(np.float32), O.dequant_q6k(b))


def _f16_ulps(a, b):
    return np.abs(a.astype(np.int32) - b.astype(np.int32))


def test_generators_match_oracle(ctx):
    """Integer fields (scales, quants) are bit-exact; the f16 super-scales come
    from f64 Box-Muller (log, cos), whose last bit may differ between the
    device math library and the host libm, so they may differ by one f16 ulp
    in rare blocks."""
    n4, n6, nf = 5000, 3001, 100001
    b4 = ctx.alloc(n4 * 144)
    ctx.fill_q4k(b4, n4, 42)
    got, ref = b4.download(np.uint8).reshape(n4, 144), O.gen_q4k(42, n4).reshape(n4, 144)
    assert np.array_equal(got[:, 4:], ref[:, 4:])
    dd = _f16_ulps(got[:, :4].copy().view(np.uint16), ref[:, :4].copy().view(np.uint16))
    print(f"q4k d/dmin differing: {np.count_nonzero(dd)} of {2 * n4}", flush=True)
    assert dd.max() <= 1 and np.count_nonzero(dd) <= 0.001 * 2 * n4
    b6 = ctx.alloc(n6 * 210)
    ctx.fill_q6k(b6, n6, 43)
    got, ref = b6.download(np.uint8).reshape(n6, 210), O.gen_q6k(43, n6).reshape(n6, 210)
    assert np.array_equal(got[:, :208], ref[:, :208])
    dd = _f16_ulps(got[:, 208:].copy().view(np.uint16), ref[:, 208:].copy().view(np.uint16))
    print(f"q6k d differing: {np.count_nonzero(dd)} of {n6}", flush=True)
    assert dd.max() <= 1 and np.count_nonzero(dd) <= 0.001 * n6
    x = ctx.empty(nf, np.float32)
    ctx.fill_normal_f32(x, nf, 44, 0.0, 1.0)
    got = x.download(np.float32)
    ref = O.gen_normal_f32(44, nf, 0.0, 1.0)
    # Box-Muller runs in f64 on both sides; a last-bit difference of the
    # device's log/cos could flip one f32 rounding, so allow one ulp
    assert np.max(np.abs(got.view(np.int32) - ref.view(np.int32))) <= 1
    h = ctx.empty(nf, np.uint16)
    ctx.fill_normal_f16(h, nf, 45, 1.0, 0.1)
    d = np.abs(h.download(np.uint16).astype(np.int32) - O.gen_normal_f16(45, nf, 1.0, 0.1).astype(np.int32))
    assert d.max() <= 1


MATVEC_CASES = [
    # (wtype, M, N): config-0 GEMV, E2B q/k/v/o/gate/up (Q4_K), down (Q6_K, I=6144 and
    # 12288), global-layer shapes (HD=512), a ragged M and a shape on the generic path
    ("q4k", 6144, 1536),
    ("q4k", 2048, 1536),
    ("q4k", 256, 1536),
    ("q4k", 1536, 2048),
    ("q4k", 4096, 1536),
    ("q4k", 1536, 4096),
    ("q4k", 100, 1536),
    ("q4k", 33, 2560),
    ("q6k", 1536, 6144),
    ("q6k", 1536, 12288),
    ("q6k", 8192, 1536),
    ("q6k", 77, 1536),
    ("q6k", 40, 2560),
    # past two workgroups per CU of tiles: one workgroup per CU walks its
    # tiles through the LDS ring (5 buffers for Q4_K, 3 for Q6_K), with a
    # last partial tile
    ("q4k", 65536, 1536),
    ("q6k", 65536, 1536),
    ("q4k", 65531, 2048),
]


@pytest.mark.parametrize("wtype,M,N", MATVEC_CASES)
def test_matmul_quant(ctx, wtype, M, N):
    bpb = 144 if wtype == "q4k" else 210
    nb = M * N // 256
    W = O.gen_q4k(M * 7 + N, nb) if wtype == "q4k" else O.gen_q6k(M * 7 + N, nb)
    x = O.gen_normal_f32(N, N)
    ref = O.matmul(x, W, M, N, wtype)
    dW, dx = ctx.from_numpy(W), ctx.from_numpy(x)
    dy = ctx.empty(M, np.float32)
    ctx.matmulQuant(dx, dW, dy, M, N, wtype)
    assert_close(dy.download(np.float32), ref, what=f"{wtype} {M}x{N}")
    if wtype == "q4k":
        dy2 = ctx.empty(M, np.float32)
        ctx.matmulQuantMR4(dx, dW, dy2, M, N)
        assert bits_equal(dy2.download(np.float32), dy.download(np.float32))
    assert nb * bpb == W.size


def test_matmul_quant_special_inputs(ctx):
    M, N = 512, 1536
    W = O.gen_q4k(1, M * N // 256)
    dW = ctx.from_numpy(W)
    dy = ctx.empty(M, np.float32)
    # x = 0 gives exactly 0
    ctx.matmulQuant(ctx.zeros(N, np.float32), dW, dy, M, N)
    assert np.all(dy.download(np.float32) == 0)
    # widely ranged x (sub-block scales differ by 1e6)
    x = O.gen_normal_f32(2, N) * np.repeat(10.0 ** np.arange(-3, 3), 256).astype(np.float32)
    ctx.matmulQuant(ctx.from_numpy(x), dW, dy, M, N)
    assert_close(dy.download(np.float32), O.matmul(x, W, M, N, "q4k"), what="ranged x")


def test_matmul_f16_reference_format(ctx):
    M, N = 1000, 1536
    W = O.gen_normal_f16(5, M * N, 0.0, 0.02)
    x = O.gen_normal_f32(6, N)
    dy = ctx.empty(M, np.float32)
    ctx.matmulQuant(ctx.from_numpy(x), ctx.from_numpy(W), dy, M, N, "f16")
    assert_close(dy.download(np.float32), O.matmul(x, W, M, N, "f16"), rel=1e-5, cos=0.9999999)


@pytest.mark.parametrize("wtype,M,N,batch", [("q4k", 2048, 1536, 3), ("q4k", 6144, 1536, 8),
                                             ("q6k", 4096, 1536, 8), ("q6k", 1536, 6144, 5),
                                             ("q4k", 1536, 2048, 16)])
def test_matmul_quant_batched(ctx, wtype, M, N, batch):
    nb = M * N // 256
    W = O.gen_q4k(9, nb) if wtype == "q4k" else O.gen_q6k(9, nb)
    X = O.gen_normal_f32(10, batch * N).reshape(batch, N)
    dY = ctx.empty(batch * M, np.float32)
    ctx.matmulQuantBatch(ctx.from_numpy(X), ctx.from_numpy(W), dY, M, N, batch, wtype)
    Y = dY.download(np.float32).reshape(batch, M)
    for b in range(batch):
        assert_close(Y[b], O.matmul(X[b], W, M, N, wtype), what=f"vector {b}")


def test_rms_norm_matmul(ctx):
    M, N = 2560, 1536
    W = O.gen_q4k(20, M * N // 256)
    x = O.gen_normal_f32(21, N, 0.0, 3.0)
    w = O.gen_normal_f16(22, N, 1.0, 0.1)
    ref = O.matmul(O.rms_norm(x, w, 1e-6), W, M, N, "q4k")
    dy = ctx.empty(M, np.float32)
    ctx.rmsNormMatmul_q4k(ctx.from_numpy(x), ctx.from_numpy(w), ctx.from_numpy(W), dy, M, N, 1e-6)
    assert_close(dy.download(np.float32), ref, what="rmsNorm->matmulQuant")


@pytest.mark.parametrize("I,N", [(6144, 1536), (512, 2048)])
def test_norm_add_gate_up_gelu(ctx, I, N):
    Wg = O.gen_q4k(30, I * N // 256)
    Wu = O.gen_q4k(31, I * N // 256)
    o = O.gen_normal_f32(32, N, 0.0, 2.0)
    res = O.gen_normal_f32(33, N)
    w_post = O.gen_normal_f16(34, N, 1.0, 0.1)
    w_pre = O.gen_normal_f16(35, N, 1.0, 0.1)
    h = O.fused_norm_add(o, w_post, res, 1e-6)
    x = O.rms_norm(h, w_pre, 1e-6)
    ref = O.gelu_mul(O.matmul(x, Wg, I, N, "q4k"), O.matmul(x, Wu, I, N, "q4k"))
    dh = ctx.empty(N, np.float32)
    dout = ctx.empty(I, np.float32)
    ctx.normAddGateUpGelu_q4k(ctx.from_numpy(o), ctx.from_numpy(w_post), ctx.from_numpy(res),
                              ctx.from_numpy(w_pre), ctx.from_numpy(Wg), ctx.from_numpy(Wu), dh, dout, I, N, 1e-6)
    assert_close(dh.download(np.float32), h, rel=1e-6, cos=0.99999999, what="h")
    assert_close(dout.download(np.float32), ref, what="gelu(gate)*up")


def test_lm_head_q6k_full_size(ctx):
    """The tied LM head at its real shape: [262144 x 1536] Q6_K (330 MB)."""
    M, N = 262144, 1536
    W = ctx.alloc(M * N // 256 * 210)
    ctx.fill_q6k(W, M * N // 256, 7)
    x = O.gen_normal_f32(8, N)
    dy = ctx.empty(M, np.float32)
    ctx.matmulQuant(ctx.from_numpy(x), W, dy, M, N, "q6k")
    y = dy.download(np.float32)
    # check a strided subset of rows against the oracle (the full oracle takes ~1 s)
    rows = np.arange(0, M, 97)
    Wh = W.download(np.uint8).reshape(M, -1)[rows]
    assert_close(y[rows], O.matmul(x, Wh.reshape(-1), rows.size, N, "q6k"), what="LM head rows")


@pytest.mark.parametrize("mode", ["norm", "normadd"])
def test_norm_add_matmul_segments_qkv(ctx, mode):
    """q/k/v projections in one launch, with the RMSNorm (and, between layers,
    the post-FFN residual add) in the prologue."""
    N = 1536
    segs = [(2048, 40), (256, 41), (256, 42)]
    Ws = [O.gen_q4k(s, M * N // 256) for M, s in segs]
    x = O.gen_normal_f32(43, N, 0.0, 2.0)
    res = O.gen_normal_f32(44, N)
    w1 = O.gen_normal_f16(45, N, 1.0, 0.1)
    w2 = O.gen_normal_f16(46, N, 1.0, 0.1)
    if mode == "norm":
        xn = O.rms_norm(x, w1, 1e-6)
    else:
        h = O.fused_norm_add(x, w1, res, 1e-6)
        xn = O.rms_norm(h, w2, 1e-6)
    outs = [ctx.empty(M, np.float32) for M, _ in segs]
    dh = ctx.empty(N, np.float32)
    ctx.normAddMatmulSegments("q4k", ctx.from_numpy(x), ctx.from_numpy(w1),
                              ctx.from_numpy(res) if mode == "normadd" else None,
                              ctx.from_numpy(w2) if mode == "normadd" else None,
                              dh if mode == "normadd" else None,
                              [ctx.from_numpy(W) for W in Ws], outs, [M for M, _ in segs], N)
    for (M, _), W, o in zip(segs, Ws, outs):
        assert_close(o.download(np.float32), O.matmul(xn, W, M, N, "q4k"), what=f"{mode} M={M}")
    if mode == "normadd":
        assert_close(dh.download(np.float32), h, rel=1e-6, cos=0.99999999, what="h_out")


def test_norm_add_matmul_q6k_softcap(ctx):
    """post-FFN add + final norm + tied Q6_K LM head + softcap in one launch."""
    M, N = 20000, 1536
    W = O.gen_q6k(50, M * N // 256)
    x = O.gen_normal_f32(51, N, 0.0, 2.0)
    res = O.gen_normal_f32(52, N, 0.0, 5.0)
    w1 = O.gen_normal_f16(53, N, 1.0, 0.1)
    w2 = O.gen_normal_f16(54, N, 1.0, 0.1)
    h = O.fused_norm_add(x, w1, res, 1e-6)
    # scale the final-norm weight 20x so that logits reach the softcap's knee
    w2s = (w2.view(np.float16).astype(np.float32) * 20).astype(np.float16).view(np.uint16)
    ref = O.logit_softcap(O.matmul(O.rms_norm(h, w2s, 1e-6), W, M, N, "q6k"), 30.0)
    y = ctx.empty(M, np.float32)
    dh = ctx.empty(N, np.float32)
    ctx.normAddMatmulSegments("q6k", ctx.from_numpy(x), ctx.from_numpy(w1), ctx.from_numpy(res),
                              ctx.from_numpy(w2s), dh, [ctx.from_numpy(W)], [y], [M], N, 1e-6, softcap=30.0)
    got = y.download(np.float32)
    assert np.max(np.abs(got)) <= 30.0 and np.max(np.abs(ref)) > 20.0
    assert_close(got, ref, what="lm head + softcap")


@pytest.mark.parametrize("M,scale,specials", [(20000, 20.0, False), (3000, 20.0, False), (20000, 2000.0, False),
                                              (3000, 2000.0, True), (262144, 20.0, False)])
def test_norm_add_matmul_argmax(ctx, M, scale, specials):
    """LM head + softcap with the argmax taken from the matvec's own per-workgroup
    candidates: the logits are those of normAddMatmulSegments bit for bit, and the
    index is the reference rule's argmax of them (ties and NaN included). A
    2000x final-norm weight drives many logits to exactly 30.0 (tanh saturates),
    so the residue tie order decides; NaN block scales make NaN rows, kept as
    NaN logits by running that case without the softcap (whose clamp maps NaN
    to -cap)."""
    N = 1536
    W = O.gen_q6k(60, M * N // 256).reshape(M, -1).copy()
    if specials:
        W[5::97, 208:210] = np.frombuffer(struct.pack("<H", 0x7e00), np.uint8)  # d = NaN
    W = W.reshape(-1)
    x = O.gen_normal_f32(61, N, 0.0, 2.0)
    res = O.gen_normal_f32(62, N, 0.0, 5.0)
    w1 = O.gen_normal_f16(63, N, 1.0, 0.1)
    w2 = O.gen_normal_f16(64, N, 1.0, 0.1)
    w2s = (w2.view(np.float16).astype(np.float32) * scale).astype(np.float16).view(np.uint16)
    cap = 0.0 if specials else 30.0
    dx, dw1, dres, dw2, dW = (ctx.from_numpy(a) for a in (x, w1, res, w2s, W))
    y_ref = ctx.empty(M, np.float32)
    ctx.normAddMatmulSegments("q6k", dx, dw1, dres, dw2, None, [dW], [y_ref], [M], N, 1e-6, softcap=cap)
    want = y_ref.download(np.float32)
    y = ctx.empty(M, np.float32)
    dh = ctx.empty(N, np.float32)
    r = ctx.zeros(1, np.uint32)
    pos0 = np.array([77], np.uint32)
    p = ctx.from_numpy(pos0)
    for call in range(2):
        ctx.normAddMatmulArgmax("q6k", dx, dw1, dres, dw2, dh, dW, y, M, N, r, 1e-6, softcap=cap,
                                positions=p, delta=3)
        got = y.download(np.float32)
        assert bits_equal(got, want), call
        idx = int(r.download(np.uint32)[0])
        assert idx == O.argmax(got), (call, idx, O.argmax(got))
        assert p.download(np.uint32)[0] == 77 + 3 * (call + 1)
    if scale > 100 and not specials:
        assert np.count_nonzero(got == np.float32(30.0)) > 8
    if specials:
        assert np.isnan(got).any()
    assert_close(dh.download(np.float32), O.fused_norm_add(x, w1, res, 1e-6), rel=1e-6, cos=0.99999999,
                 what="h_out")
    # no positions: the index only
    r2 = ctx.zeros(1, np.uint32)
    ctx.normAddMatmulArgmax("q6k", dx, dw1, dres, dw2, None, dW, y, M, N, r2, 1e-6, softcap=cap)
    assert int(r2.download(np.uint32)[0]) == idx
    assert p.download(np.uint32)[0] == 77 + 6


@pytest.mark.parametrize("M,scale,specials", [(20000, 20.0, False), (3000, 20.0, False), (20000, 2000.0, False),
                                              (3000, 2000.0, True), (262144, 20.0, False), (262144, 2000.0, False),
                                              (300, 20.0, False)])
def test_norm_add_matmul_topk(ctx, M, scale, specials):
    """LM head + softcap with the top-k256 pairs taken from the matvec's own
    per-workgroup residue-class candidates (src/engine.ts:1735-1740,
    shaders/topk256.wgsl): the logits are those of normAddMatmulSegments bit
    for bit and the 512 words equal the reference scan of them bit for bit,
    with saturated ties (2000x final-norm weight), NaN rows (no softcap),
    fewer rows than classes, and the full 262144-row head (workgroups walking
    512 rows each). Twice in a row: every call restarts its class tables."""
    N = 1536
    W = O.gen_q6k(70, M * N // 256).reshape(M, -1).copy()
    if specials:
        W[5::97, 208:210] = np.frombuffer(struct.pack("<H", 0x7e00), np.uint8)  # d = NaN
    W = W.reshape(-1)
    x = O.gen_normal_f32(71, N, 0.0, 2.0)
    res = O.gen_normal_f32(72, N, 0.0, 5.0)
    w1 = O.gen_normal_f16(73, N, 1.0, 0.1)
    w2 = O.gen_normal_f16(74, N, 1.0, 0.1)
    w2s = (w2.view(np.float16).astype(np.float32) * scale).astype(np.float16).view(np.uint16)
    cap = 0.0 if specials else 30.0
    dx, dw1, dres, dw2, dW = (ctx.from_numpy(a) for a in (x, w1, res, w2s, W))
    y_ref = ctx.empty(M, np.float32)
    ctx.normAddMatmulSegments("q6k", dx, dw1, dres, dw2, None, [dW], [y_ref], [M], N, 1e-6, softcap=cap)
    want = y_ref.download(np.float32)
    y = ctx.empty(M, np.float32)
    dh = ctx.empty(N, np.float32)
    t = ctx.zeros(512, np.float32)
    for call in range(2):
        ctx.normAddMatmulTopk("q6k", dx, dw1, dres, dw2, dh, dW, y, M, N, t, 1e-6, softcap=cap)
        got = y.download(np.float32)
        assert bits_equal(got, want), call
        assert bits_equal(t.download(np.float32), O.topk256(got)), call
    if scale > 100 and not specials:
        assert np.count_nonzero(got == np.float32(30.0)) > 8
    if specials:
        assert np.isnan(got).any()
    # the standalone two-stage top-k over the written logits agrees
    t2 = ctx.zeros(512, np.float32)
    ctx.topk256(y, t2, M)
    assert bits_equal(t2.download(np.float32), t.download(np.float32))


def _check_digit_block(blk, x):
    """The digit block a gate/up launch writes for its outputs x: per 8
    elements, x ~ s * (256 hi + lo) to within one digit step (the scale is
    max|x| / 32512 over the 8), |256 hi + lo| <= 32512, and the offsets are
    32 x the digit sums."""
    K = x.size
    hi = blk[:K].view(np.int8).astype(np.int64)
    lo = blk[K:2 * K].view(np.int8).astype(np.int64)
    s = blk[2 * K:2 * K + 4 * (K // 8)].view(np.float32)
    c = blk[2 * K + 4 * (K // 8):2 * K + 12 * (K // 8)].view(np.int32).reshape(-1, 2)
    g = x.reshape(-1, 8).astype(np.float64)
    am = np.abs(g).max(axis=1)
    assert np.allclose(s, am / 32512.0, rtol=1e-6, atol=0)
    q = (256 * hi + lo).reshape(-1, 8)
    assert np.abs(q).max() <= 32512
    rec = s.astype(np.float64)[:, None] * q
    assert np.all(np.abs(rec - g) <= 1.0001 * s.astype(np.float64)[:, None])
    assert np.array_equal(c[:, 0], 32 * hi.reshape(-1, 8).sum(axis=1))
    assert np.array_equal(c[:, 1], 32 * lo.reshape(-1, 8).sum(axis=1))


@pytest.mark.parametrize("I", [6144, 12288])
def test_gate_up_digits_then_down(ctx, I):
    """The FFN with the GELU product handed to the down projection as digits:
    the f32 product equals normAddGateUpGelu_q4k's bit for bit, the digit
    block restates it (per-8 scales, digit sums), and the down matvec over
    the digits matches the oracle's down projection of the f32 product."""
    N = 1536
    Wg = O.gen_q4k(40, I * N // 256)
    Wu = O.gen_q4k(41, I * N // 256)
    Wd = O.gen_q6k(42, N * I // 256)
    o = O.gen_normal_f32(43, N, 0.0, 2.0)
    res = O.gen_normal_f32(44, N)
    w_post = O.gen_normal_f16(45, N, 1.0, 0.1)
    w_pre = O.gen_normal_f16(46, N, 1.0, 0.1)
    args = [ctx.from_numpy(a) for a in (o, w_post, res, w_pre, Wg, Wu)]
    ref_out = ctx.empty(I, np.float32)
    ctx.normAddGateUpGelu_q4k(*args, ctx.empty(N, np.float32), ref_out, I, N, 1e-6)
    out = ctx.empty(I, np.float32)
    dig = ctx.zeros(ctx.digits_bytes(I), np.uint8)
    dW = ctx.from_numpy(Wd)
    y = ctx.empty(N, np.float32)
    for rep in range(2):
        ctx.normAddGateUpGeluDigits_q4k(*args, ctx.empty(N, np.float32), out, dig, I, N, 1e-6)
        x = out.download(np.float32)
        assert bits_equal(x, ref_out.download(np.float32))
        _check_digit_block(dig.download(np.uint8), x)
        ctx.matmulQuantDigits_q6k(dig, dW, y, N, I)
        assert_close(y.download(np.float32), O.matmul(x, Wd, N, I, "q6k"), what=f"down over digits I={I}")


NON_FINITE = [float("nan"), float("inf"), float("-inf")]


def _non_finite_like_reference(got, ref, what):
    """A non-finite input reaches every row, as in the reference's f32
    matvec (shaders/matmul_quant.wgsl:38-47): NaN where the reference has
    NaN, and NaN or the reference's signed infinity where it has one (the
    input's 32-element sub-block carries it as a NaN scale, so an infinity
    arrives as NaN; the norm that reads the result would turn it into NaN in
    the reference as well)."""
    assert not np.any(np.isfinite(ref)), f"{what}: the oracle has finite rows"
    assert not np.any(np.isfinite(got)), f"{what}: {np.count_nonzero(np.isfinite(got))} finite rows"
    assert np.all(np.isnan(got[np.isnan(ref)])), what
    inf = np.isinf(got)
    assert np.array_equal(got[inf], ref[inf]), what


@pytest.mark.parametrize("wtype,M,N", [("q4k", 6144, 1536), ("q4k", 1536, 2048), ("q6k", 1536, 6144),
                                       ("q6k", 8192, 1536)])
@pytest.mark.parametrize("special", NON_FINITE)
def test_matmul_quant_non_finite_input(ctx, wtype, M, N, special):
    """The one-vector launches with a NaN / +Inf / -Inf activation element,
    then a finite vector through the same buffers (nothing non-finite stays
    behind)."""
    nb = M * N // 256
    W = O.gen_q4k(M + N + 5, nb) if wtype == "q4k" else O.gen_q6k(M + N + 5, nb)
    x = O.gen_normal_f32(N + 1, N)
    xb = x.copy()
    xb[N // 3 + 5] = special
    with np.errstate(invalid="ignore", over="ignore"):
        ref = O.matmul(xb, W, M, N, wtype)
    dW, dy = ctx.from_numpy(W), ctx.empty(M, np.float32)
    dx = ctx.from_numpy(xb)
    ctx.matmulQuant(dx, dW, dy, M, N, wtype)
    _non_finite_like_reference(dy.download(np.float32), ref, f"{wtype} {M}x{N} x={special}")
    dx.upload(x)
    ctx.matmulQuant(dx, dW, dy, M, N, wtype)
    assert_close(dy.download(np.float32), O.matmul(x, W, M, N, wtype), what=f"{wtype} {M}x{N} after {special}")


@pytest.mark.parametrize("special", NON_FINITE)
def test_norm_prologue_and_digit_hand_off_non_finite(ctx, special):
    """The rmsNorm-prologue matvec and the FFN whose GELU product reaches the
    Q6_K down launch as digits: one non-finite element of the input makes
    every output row NaN, as the reference's rms_norm (mean of squares
    non-finite) does before its matvec."""
    N, M, I = 1536, 2048, 6144
    W = O.gen_q4k(50, M * N // 256)
    nw = O.gen_normal_f16(51, N, 1.0, 0.1)
    x = O.gen_normal_f32(52, N, 0.0, 2.0)
    x[700] = special
    with np.errstate(invalid="ignore", over="ignore"):
        ref = O.matmul(O.rms_norm(x, nw, 1e-6), W, M, N, "q4k")
    y = ctx.empty(M, np.float32)
    ctx.rmsNormMatmul_q4k(ctx.from_numpy(x), ctx.from_numpy(nw), ctx.from_numpy(W), y, M, N, 1e-6)
    got = y.download(np.float32)
    assert np.all(np.isnan(got)) and np.all(np.isnan(ref)), special
    Wg, Wu, Wd = O.gen_q4k(53, I * N // 256), O.gen_q4k(54, I * N // 256), O.gen_q6k(55, N * I // 256)
    res = O.gen_normal_f32(56, N)
    w_post, w_pre = O.gen_normal_f16(57, N, 1.0, 0.1), O.gen_normal_f16(58, N, 1.0, 0.1)
    args = [ctx.from_numpy(a) for a in (x, w_post, res, w_pre, Wg, Wu)]
    act = ctx.empty(I, np.float32)
    dig = ctx.zeros(ctx.digits_bytes(I), np.uint8)
    ctx.normAddGateUpGeluDigits_q4k(*args, ctx.empty(N, np.float32), act, dig, I, N, 1e-6)
    down = ctx.empty(N, np.float32)
    ctx.matmulQuantDigits_q6k(dig, ctx.from_numpy(Wd), down, N, I)
    assert np.all(np.isnan(act.download(np.float32))), special
    assert np.all(np.isnan(down.download(np.float32))), special


def test_digit_entries_reject_bad_shapes(ctx):
    """Shapes the digit hand-off does not cover fail with an error, not a launch."""
    N, I = 2048, 6144
    z = ctx.zeros(I * 8, np.float32)
    dig = ctx.zeros(ctx.digits_bytes(I), np.uint8)
    with pytest.raises(RuntimeError):  # hidden width 2048: 32 lanes reduce a row, no 8-row groups in a wave
        ctx.normAddGateUpGeluDigits_q4k(z, z, z, z, z, z, None, z, dig, I, N, 1e-6)
    with pytest.raises(RuntimeError):  # FFN width not covered
        ctx.matmulQuantDigits_q6k(dig, z, z, 1536, 4096)
    with pytest.raises(RuntimeError):
        ctx.digits_bytes(100)
