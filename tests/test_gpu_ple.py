"""GPU parity of the per-layer-embedding (PLE) kernels against the oracle
(shaders/ple_stage1_fuse.wgsl, ple_gelu_mul.wgsl, ple_skip_scale_add.wgsl,
matmul_quant.wgsl over f16 weights; src/engine.ts:1516-1535, 1608-1616).

* Q5_K blocks to f16: bit-exact with the oracle's dequant (src/gguf.ts:218-257)
  rounded by numpy;
* stage 1 over every layer of several rows (device tokens, a token past the
  table), pleGeluMul and pleSkipScaleAdd at rel-L2 1e-6 (f32 arithmetic in
  another order);
* the f16 matvec over 1..13 vectors, every row length it takes (256 to
  12288) and row counts that do not fill a workgroup, the gate with and without its norm-add prologue, the scaled
  norm-add prologue of the quantized matvec and of the batch prologue, at
  rel-L2 1e-3 / cosine 0.9999 (the matvec's tolerance).
"""
import numpy as np
import pytest

import oracle as O
from gpu_util import assert_close

pytestmark = pytest.mark.gpu


def _q5k_blocks(seed: int, n: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    b = rng.integers(0, 256, (n, 176), dtype=np.uint8)
    b[:, 0:2] = np.abs(rng.standard_normal(n) * 2e-3).astype(np.float16).view(np.uint8).reshape(n, 2)
    b[:, 2:4] = np.abs(rng.standard_normal(n) * 1e-3).astype(np.float16).view(np.uint8).reshape(n, 2)
    return b.reshape(-1)


def _f16(x) -> np.ndarray:
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def test_q5k_to_f16_bit_exact(ctx):
    host = _q5k_blocks(1, 500)
    # d / dmin over the whole f16 range, subnormals, zero and a negative d
    host.reshape(-1, 176)[:8, 0:2] = np.array([0x0001, 0x03ff, 0x0400, 0x7bff, 0x0000, 0x8400, 0x3c00, 0x1234],
                                              np.uint16).view(np.uint8).reshape(8, 2)
    dev = ctx.alloc(400 * 176)
    ctx.fill_q5k(dev, 400, 99)
    for name, blocks in (("host", host), ("generated", dev.download(np.uint8))):
        n = blocks.size // 176
        out = ctx.empty(n * 256, np.uint16)
        ctx.dequantF16("q5k", ctx.from_numpy(blocks), n, out)
        with np.errstate(over="ignore", invalid="ignore"):
            want = O.dequant_q5k(blocks).astype(np.float16).view(np.uint16)
        got = out.download(np.uint16)
        assert np.array_equal(got, want), name


@pytest.mark.parametrize("count", [1, 3])
def test_stage1(ctx, count):
    L, D, V = 5, 256, 300
    rng = np.random.default_rng(2 + count)
    table = _q5k_blocks(3, V * L)
    proj = rng.standard_normal(count * L * D).astype(np.float32) * 2
    w = _f16(rng.standard_normal(D) * 0.1 + 1)
    toks = np.array([7, 299, 1000][:count], np.uint32)  # the last one past the table
    out = ctx.empty(count * L * D, np.float32)
    dt = ctx.from_numpy(table)
    if count == 1:
        ctx.pleStage1Fuse(ctx.from_numpy(proj), ctx.from_numpy(w), dt, V, out, L, D, 1e-6, token=int(toks[0]))
    else:
        ctx.pleStage1Fuse(ctx.from_numpy(proj), ctx.from_numpy(w), dt, V, out, L, D, 1e-6,
                          tokens_dev=ctx.from_numpy(toks), count=count)
    got = out.download(np.float32).reshape(count, L * D)
    for b, t in enumerate(toks):
        if t < V:
            row = O.dequant_q5k(table[int(t) * L * 176:(int(t) + 1) * L * 176]).astype(np.float16).view(np.uint16)
        else:
            row = np.zeros(L * D, np.uint16)
        want = O.ple_stage1(proj[b * L * D:(b + 1) * L * D], w, row, L, D, 1e-6)
        print(f"[ple stage1] row {b} token {t}: rel-L2 {O.rel_l2(got[b], want):.2e}", flush=True)
        assert_close(got[b], want, rel=1e-6, cos=0.999999, what=f"stage 1 row {b}")


def test_gelu_mul_and_skip_scale_add(ctx):
    rng = np.random.default_rng(4)
    gate = rng.standard_normal(256).astype(np.float32) * 3
    ple = rng.standard_normal(4 * 256).astype(np.float32)
    out = ctx.empty(256, np.float32)
    ctx.pleGeluMul(ctx.from_numpy(gate), ctx.from_numpy(ple), out, 512, 256)
    assert_close(out.download(np.float32), O.ple_gelu_mul(gate, ple, 512), rel=1e-6, cos=0.999999, what="gelu mul")
    h = rng.standard_normal(1536).astype(np.float32)
    n = rng.standard_normal(1536).astype(np.float32)
    sc = _f16([0.8125, 0])
    dh = ctx.from_numpy(h)
    ctx.pleSkipScaleAdd(dh, ctx.from_numpy(n), ctx.from_numpy(sc), 1536)
    # (the shader rounds the sum, then the product; the oracle rounds once)
    assert_close(dh.download(np.float32), O.ple_skip_scale_add(h, n, int(sc[0])), rel=1e-6, cos=0.999999,
                 what="skip scale add")


@pytest.mark.parametrize("M,N", [(256, 1536), (1536, 256), (1001, 1536), (77, 2048), (4480, 1536), (1536, 4096),
                                 (333, 6144), (1536, 12288)])
@pytest.mark.parametrize("batch", [1, 3, 8, 13])
def test_matmul_f16(ctx, M, N, batch):
    rng = np.random.default_rng(M + N + batch)
    W = _f16(rng.standard_normal(M * N) * 0.05)
    x = rng.standard_normal(batch * N).astype(np.float32)
    y = ctx.empty(batch * M, np.float32)
    ctx.matmulF16(ctx.from_numpy(x), ctx.from_numpy(W), y, M, N, batch)
    got = y.download(np.float32).reshape(batch, M)
    for b in range(batch):
        assert_close(got[b], O.matmul(x[b * N:(b + 1) * N], W, M, N, "f16"), what=f"f16 matvec {M}x{N} vec {b}")


@pytest.mark.parametrize("batch", [1, 5])
def test_ple_gate(ctx, batch):
    D, H, L = 256, 1536, 4
    rng = np.random.default_rng(10 + batch)
    Wg = _f16(rng.standard_normal(D * H) * 0.03)
    ple = rng.standard_normal(batch * L * D).astype(np.float32)
    out = ctx.empty(batch * D, np.float32)
    il = 2
    if batch == 1:  # the post-FFN norm-add prologue
        down = rng.standard_normal(H).astype(np.float32) * 4
        res = rng.standard_normal(H).astype(np.float32)
        w1 = _f16(rng.standard_normal(H) * 0.1 + 1)
        h_out = ctx.empty(H, np.float32)
        ctx.pleGate(ctx.from_numpy(down), ctx.from_numpy(w1), ctx.from_numpy(res), h_out, ctx.from_numpy(Wg),
                    ctx.from_numpy(ple), 0, il * D, out, D, H, 1e-6)
        h = O.fused_norm_add(down, w1, res, 1e-6)
        assert_close(h_out.download(np.float32), h, rel=1e-6, cos=0.999999, what="gate prologue h")
        xs = [h]
    else:
        x = rng.standard_normal(batch * H).astype(np.float32)
        ctx.pleGate(ctx.from_numpy(x), None, None, None, ctx.from_numpy(Wg), ctx.from_numpy(ple), L * D, il * D,
                    out, D, H, 1e-6, batch=batch)
        xs = [x[b * H:(b + 1) * H] for b in range(batch)]
    got = out.download(np.float32).reshape(batch, D)
    for b, xv in enumerate(xs):
        want = O.ple_gelu_mul(O.matmul(xv, Wg, D, H, "f16"), ple[b * L * D:(b + 1) * L * D], il * D)
        assert_close(got[b], want, what=f"gate row {b}")


@pytest.mark.parametrize("wtype", ["q4k", "q6k"])
def test_scaled_norm_add_segments(ctx, wtype):
    H, M = 1536, 512
    rng = np.random.default_rng(20)
    x = rng.standard_normal(H).astype(np.float32) * 3
    res = rng.standard_normal(H).astype(np.float32)
    w1 = _f16(rng.standard_normal(H) * 0.1 + 1)
    w2 = _f16(rng.standard_normal(H) * 0.1 + 1)
    sc = _f16([0.6875, 0])
    W = (O.gen_q4k if wtype == "q4k" else O.gen_q6k)(21, M * H // 256)
    y = ctx.empty(M, np.float32)
    h_out = ctx.empty(H, np.float32)
    ctx.normAddScaleMatmulSegments(wtype, ctx.from_numpy(x), ctx.from_numpy(w1), ctx.from_numpy(res),
                                   ctx.from_numpy(sc), ctx.from_numpy(w2), h_out, [ctx.from_numpy(W)], [y], [M], H)
    h = O.ple_skip_scale_add(res, O.rms_norm(x, w1, 1e-6), int(sc[0]))
    assert_close(h_out.download(np.float32), h, rel=1e-6, cos=0.999999, what="scaled h")
    assert_close(y.download(np.float32), O.matmul(O.rms_norm(h, w2, 1e-6), W, M, H, wtype), what="scaled matvec")


@pytest.mark.parametrize("second_norm", [True, False])
def test_batch_prep_scale(ctx, second_norm):
    H, B, P = 1536, 6, 3
    rng = np.random.default_rng(30)
    parts = rng.standard_normal(P * B * H).astype(np.float32)
    res = rng.standard_normal(B * H).astype(np.float32)
    w1 = _f16(rng.standard_normal(H) * 0.1 + 1)
    w2 = _f16(rng.standard_normal(H) * 0.1 + 1)
    sc = _f16([1.25, 0])
    out = ctx.empty(B * H, np.float32)
    h_out = ctx.empty(B * H, np.float32)
    ctx.batchPrepScale(ctx.from_numpy(parts), P, ctx.from_numpy(w1), ctx.from_numpy(res), ctx.from_numpy(sc),
                       ctx.from_numpy(w2) if second_norm else None, h_out, out, H, B, 1e-6)
    got, gh = out.download(np.float32).reshape(B, H), h_out.download(np.float32).reshape(B, H)
    xs = parts.reshape(P, B, H).astype(np.float64).sum(0).astype(np.float32)
    for b in range(B):
        h = O.ple_skip_scale_add(res[b * H:(b + 1) * H], O.rms_norm(xs[b], w1, 1e-6), int(sc[0]))
        assert_close(gh[b], h, rel=1e-6, cos=0.999999, what=f"h row {b}")
        want = O.rms_norm(h, w2, 1e-6) if second_norm else h
        assert_close(got[b], want, rel=1e-6, cos=0.999999, what=f"out row {b}")
