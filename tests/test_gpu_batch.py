"""GPU parity of the matrix-core matmul over many activation vectors (ragged
multi-sequence decode): every vector of the batch against the f64 oracle's
matvec (rel-L2 <= 1e-3, cos >= 0.9999), with the norm prologues, several
matrices per launch and the softcap epilogue."""
import numpy as np
import pytest

import oracle as O
import synth
from gpu_util import assert_close

pytestmark = pytest.mark.gpu


def _weights(wtype, seed, M, N):
    nb = M * N // 256
    if wtype == "q6k_wide":
        return synth.q6k_wide(seed, nb)
    if wtype == "q4k_centered":
        return synth.q4k_centered(seed, nb)
    return O.gen_q4k(seed, nb) if wtype == "q4k" else O.gen_q6k(seed, nb)


@pytest.mark.parametrize("gen,M,N,batch", [
    ("q4k", 2048, 1536, 32),   # E2B q projection at B=32
    ("q4k", 1536, 2048, 16),   # o projection
    ("q4k", 6144, 1536, 64),   # gate/up at B=64
    ("q4k", 100, 1536, 17),    # ragged rows and batch
    ("q6k", 1536, 6144, 32),   # down projection
    ("q6k", 1000, 1536, 33),   # LM-head-like K, ragged
    ("q6k", 777, 12288, 16),   # wide FFN down, rows not a multiple of 16
    # real GGUF scales span the int8 range: |sc * (q - 32)| up to 4096, where
    # the f16 weight operand rounds once (2^-12 relative at most)
    ("q6k_wide", 1536, 6144, 32),
    ("q6k_wide", 1000, 1536, 33),
    ("q6k_wide", 1536, 6144, 64),
    ("q4k_centered", 2048, 1536, 32),
])
def test_batched_matmul_matches_oracle(ctx, gen, M, N, batch):
    wtype = gen[:3]
    W = _weights(gen, 60, M, N)
    X = O.gen_normal_f32(61, batch * N, 0.0, 1.5).reshape(batch, N)
    X[batch // 2] *= 40.0  # one vector with a very different scale
    dY = ctx.empty(batch * M, np.float32)
    ctx.matmulQuantBatch(ctx.from_numpy(X), ctx.from_numpy(W), dY, M, N, batch, wtype)
    Y = dY.download(np.float32).reshape(batch, M)
    for b in range(batch):
        assert_close(Y[b], O.matmul(X[b], W, M, N, wtype), what=f"{wtype} {M}x{N} vector {b}")


@pytest.mark.parametrize("mode", ["plain", "norm", "normadd"])
def test_batched_segments_with_prologues(ctx, mode):
    """q/k/v of 32 sequences in one launch, with the per-sequence RMSNorm (or
    residual add + RMSNorm) prologue."""
    N, B = 1536, 32
    segs = [(2048, 70), (256, 71), (256, 72)]
    Ws = [O.gen_q4k(s, M * N // 256) for M, s in segs]
    X = O.gen_normal_f32(73, B * N, 0.0, 2.0).reshape(B, N)
    R = O.gen_normal_f32(74, B * N).reshape(B, N)
    w1 = O.gen_normal_f16(75, N, 1.0, 0.1)
    w2 = O.gen_normal_f16(76, N, 1.0, 0.1)
    outs = [ctx.empty(B * M, np.float32) for M, _ in segs]
    dh = ctx.empty(B * N, np.float32)
    ctx.normAddMatmulSegmentsBatch(
        "q4k", ctx.from_numpy(X), ctx.from_numpy(w1) if mode != "plain" else None,
        ctx.from_numpy(R) if mode == "normadd" else None, ctx.from_numpy(w2) if mode == "normadd" else None,
        dh if mode == "normadd" else None, [ctx.from_numpy(W) for W in Ws], outs, [M for M, _ in segs], N, B)
    H = dh.download(np.float32).reshape(B, N)
    for b in range(B):
        if mode == "plain":
            xn = X[b]
        elif mode == "norm":
            xn = O.rms_norm(X[b], w1, 1e-6)
        else:
            h = O.fused_norm_add(X[b], w1, R[b], 1e-6)
            assert_close(H[b], h, rel=1e-6, cos=0.99999999, what=f"h_out {b}")
            xn = O.rms_norm(h, w2, 1e-6)
        for (M, _), W, o in zip(segs, Ws, outs):
            got = o.download(np.float32).reshape(B, M)[b]
            assert_close(got, O.matmul(xn, W, M, N, "q4k"), what=f"{mode} seq {b} M={M}")


def test_batched_lm_head_softcap(ctx):
    """Final norm-add + tied Q6_K LM head + softcap for 16 sequences."""
    M, N, B = 8192, 1536, 16
    W = O.gen_q6k(80, M * N // 256)
    X = O.gen_normal_f32(81, B * N, 0.0, 2.0).reshape(B, N)
    R = O.gen_normal_f32(82, B * N, 0.0, 5.0).reshape(B, N)
    w1 = O.gen_normal_f16(83, N, 1.0, 0.1)
    w2 = (O.gen_normal_f16(84, N, 1.0, 0.1).view(np.float16).astype(np.float32) * 20).astype(np.float16)
    w2 = w2.view(np.uint16)
    dY = ctx.empty(B * M, np.float32)
    ctx.normAddMatmulSegmentsBatch("q6k", ctx.from_numpy(X), ctx.from_numpy(w1), ctx.from_numpy(R),
                                   ctx.from_numpy(w2), None, [ctx.from_numpy(W)], [dY], [M], N, B, softcap=30.0)
    Y = dY.download(np.float32).reshape(B, M)
    assert np.max(np.abs(Y)) <= 30.0
    for b in range(B):
        h = O.fused_norm_add(X[b], w1, R[b], 1e-6)
        ref = O.logit_softcap(O.matmul(O.rms_norm(h, w2, 1e-6), W, M, N, "q6k"), 30.0)
        assert_close(Y[b], ref, what=f"lm head seq {b}")


def test_batched_matmul_rejects_bad_shapes(ctx):
    W = O.gen_q4k(90, 64 * 1536 // 256)
    X = O.gen_normal_f32(91, 65 * 1536)
    dY = ctx.empty(65 * 64, np.float32)
    with pytest.raises(Exception, match="batch 65"):
        ctx.normAddMatmulSegmentsBatch("q4k", ctx.from_numpy(X), None, None, None, None, [ctx.from_numpy(W)],
                                       [dY], [64], 1536, 65)


@pytest.mark.parametrize("B", [5, 32, 64])
def test_batched_gate_up_gelu(ctx, B):
    """Post-attention norm-add + pre-FFN norm + gate/up + GELU product for B
    sequences in one launch."""
    M, N = 6144, 1536
    Wg = O.gen_q4k(100, M * N // 256)
    Wu = O.gen_q4k(101, M * N // 256)
    X = O.gen_normal_f32(102, B * N, 0.0, 2.0).reshape(B, N)
    R = O.gen_normal_f32(103, B * N).reshape(B, N)
    w1 = O.gen_normal_f16(104, N, 1.0, 0.1)
    w2 = O.gen_normal_f16(105, N, 1.0, 0.1)
    dh = ctx.empty(B * N, np.float32)
    dA = ctx.empty(B * M, np.float32)
    ctx.normAddGateUpGeluBatch(ctx.from_numpy(X), ctx.from_numpy(w1), ctx.from_numpy(R), ctx.from_numpy(w2),
                               ctx.from_numpy(Wg), ctx.from_numpy(Wu), dh, dA, M, N, B)
    H = dh.download(np.float32).reshape(B, N)
    A = dA.download(np.float32).reshape(B, M)
    for b in range(B):
        h = O.fused_norm_add(X[b], w1, R[b], 1e-6)
        assert_close(H[b], h, rel=1e-6, cos=0.99999999, what=f"h_out {b}")
        xn = O.rms_norm(h, w2, 1e-6)
        ref = O.gelu_mul(O.matmul(xn, Wg, M, N, "q4k"), O.matmul(xn, Wu, M, N, "q4k"))
        assert_close(A[b], ref, what=f"gelu(gate)*up seq {b}")


def _decode_sub_operands(raw: np.ndarray, M: int, B: int) -> np.ndarray:
    """Values [16 * ntv][M] of sub-block-scaled operand blocks: per super-block
    and 16-vector tile, f16 hi / lo at [sub-block][hi|lo][8-group][vector][8]
    (16384 B per tile), then the f32 2^-e at [tile][sub-block][vector]."""
    ntv = (16 if B <= 16 else 32 if B <= 32 else 64) // 16
    main_t, nsb = 16384, M // 256
    blk = raw.reshape(nsb, ntv * (main_t + 512))
    hl = blk[:, :ntv * main_t].copy().view(np.float16).reshape(nsb, ntv, 8, 2, 4, 16, 8).astype(np.float64)
    fs = blk[:, ntv * main_t:].copy().view(np.float32).reshape(nsb, ntv, 8, 16).astype(np.float64)
    val = (hl[:, :, :, 0] + hl[:, :, :, 1]) * fs[:, :, :, None, :, None]  # (kb, t, s, qq, c, e)
    return val.transpose(1, 4, 0, 2, 3, 5).reshape(16 * ntv, M)


@pytest.mark.parametrize("B,M", [(5, 6144), (32, 6144), (64, 6144), (16, 12288)])
def test_ffn_handoff_operands(ctx, B, M):
    """The gate/up launch's product as sub-block-scaled operand blocks: the
    f32 product equals the plain launch's, the blocks hold it to 2^-19 of the
    largest |value| of each 32-value sub-block (f16 hi + lo), padded vectors
    are zero, and the Q6_K down projection over them (split K, int8 scales
    over their whole range) matches the oracle's matvec of the product."""
    N = 1536
    Wg = O.gen_q4k(110, M * N // 256)
    Wu = O.gen_q4k(111, M * N // 256)
    Wd = synth.q6k_wide(112, N * M // 256)
    X = O.gen_normal_f32(113, B * N, 0.0, 2.0).reshape(B, N)
    X[B // 2] *= 30.0
    w1 = O.gen_normal_f16(114, N, 1.0, 0.1)
    xn = ctx.empty(B * N, np.float32)
    xops = ctx.empty(ctx.batch_operand_bytes(N, B), np.uint8)
    ctx.batchPrep(ctx.from_numpy(X), 1, ctx.from_numpy(w1), None, None, None, xn, N, B, ops=xops)
    dWg, dWu, dWd = ctx.from_numpy(Wg), ctx.from_numpy(Wu), ctx.from_numpy(Wd)
    a_ref = ctx.empty(B * M, np.float32)
    ctx.gateUpGeluBatch(xn, dWg, dWu, a_ref, M, N, B, ops=xops)
    a2 = ctx.empty(B * M, np.float32)
    dops = ctx.empty(ctx.batch_sub_operand_bytes(M, B), np.uint8)
    ctx.gateUpGeluBatchOps(xn, xops, dWg, dWu, a2, dops, M, N, B)
    A = a_ref.download(np.float32).reshape(B, M)
    assert np.array_equal(a2.download(np.float32).reshape(B, M), A)
    dec = _decode_sub_operands(dops.download(np.uint8), M, B)
    assert np.all(dec[B:] == 0)
    sub_max = np.abs(A.astype(np.float64)).reshape(B, M // 32, 32).max(axis=2, keepdims=True)
    err = np.abs(dec[:B] - A).reshape(B, M // 32, 32)
    assert np.all(err <= sub_max * 2.0 ** -19), float((err / np.maximum(sub_max, 1e-30)).max())
    ks_max = M // 768
    parts = ctx.empty(ks_max * B * N, np.float32)
    ks = ctx.matmulSubBatchPartial(dops, dWd, parts, N, M, B, ks_max)
    assert 1 <= ks <= ks_max and (M // 256) % ks == 0
    P = parts.download(np.float32)[:ks * B * N].reshape(ks, B, N)
    Y = P[0].copy()
    for k in range(1, ks):
        Y += P[k]
    for b in range(B):
        assert_close(Y[b], O.matmul(A[b], Wd, N, M, "q6k"), what=f"down over the hand-off, vector {b}")


@pytest.mark.parametrize("B", [3, 32])
def test_batch_prep_adds_partials_then_norms(ctx, B):
    """fusedNormAdd -> rmsNorm over x given as 3 chunks added in order."""
    N = 1536
    X = O.gen_normal_f32(110, 3 * B * N, 0.0, 1.0).reshape(3, B, N)
    R = O.gen_normal_f32(111, B * N).reshape(B, N)
    w1 = O.gen_normal_f16(112, N, 1.0, 0.1)
    w2 = O.gen_normal_f16(113, N, 1.0, 0.1)
    dh, dout = ctx.empty(B * N, np.float32), ctx.empty(B * N, np.float32)
    ctx.batchPrep(ctx.from_numpy(X), 3, ctx.from_numpy(w1), ctx.from_numpy(R), ctx.from_numpy(w2), dh, dout, N, B)
    # the same with operand blocks, then a matmul that takes them: equal to the one that rebuilds them
    dops = ctx.empty(ctx.batch_operand_bytes(N, B), np.uint8)
    ctx.batchPrep(ctx.from_numpy(X), 3, ctx.from_numpy(w1), ctx.from_numpy(R), ctx.from_numpy(w2), None, dout, N, B,
                  ops=dops)
    Wm = O.gen_q4k(114, 512 * N // 256)
    y1, y2 = ctx.empty(B * 512, np.float32), ctx.empty(B * 512, np.float32)
    ctx.matmulSegmentsBatchPartial("q4k", dout, [ctx.from_numpy(Wm)], [y1], [512], N, B, 1)
    ctx.matmulSegmentsBatchPartial("q4k", dout, [ctx.from_numpy(Wm)], [y2], [512], N, B, 1, ops=dops)
    assert_close(y2.download(np.float32), y1.download(np.float32), rel=1e-6, cos=0.99999999, what="ops vs rebuilt")
    H, Y = dh.download(np.float32).reshape(B, N), dout.download(np.float32).reshape(B, N)
    S = (X[0] + X[1]) + X[2]  # f32, chunk order
    for b in range(B):
        h = O.fused_norm_add(S[b], w1, R[b], 1e-6)
        assert_close(H[b], h, rel=1e-6, cos=0.99999999, what=f"h {b}")
        assert_close(Y[b], O.rms_norm(h, w2, 1e-6), rel=1e-6, cos=0.99999999, what=f"x' {b}")
    ctx.batchPrep(ctx.from_numpy(X), 1, ctx.from_numpy(w1), None, None, None, dout, N, B)
    Y = dout.download(np.float32).reshape(B, N)
    for b in range(B):
        assert_close(Y[b], O.rms_norm(X[0][b], w1, 1e-6), rel=1e-6, cos=0.99999999, what=f"norm {b}")


@pytest.mark.parametrize("wtype,segs,N,B,max_ks", [
    ("q4k", (2048, 256, 256), 1536, 32, 6),   # q/k/v
    ("q4k", (1536,), 2048, 17, 8),            # o
    ("q6k", (1536,), 6144, 32, 24),           # down
    ("q6k", (1536,), 6144, 64, 1),            # no split allowed
])
def test_matmul_partials_add_up(ctx, wtype, segs, N, B, max_ks):
    Ws = [_weights(wtype, 120 + i, M, N) for i, M in enumerate(segs)]
    X = O.gen_normal_f32(125, B * N, 0.0, 1.5).reshape(B, N)
    outs = [ctx.empty(max_ks * B * M, np.float32) for M in segs]
    ks = ctx.matmulSegmentsBatchPartial(wtype, ctx.from_numpy(X), [ctx.from_numpy(W) for W in Ws], outs,
                                        list(segs), N, B, max_ks)
    assert 1 <= ks <= max_ks and (N // 256) % ks == 0
    for M, W, o in zip(segs, Ws, outs):
        P = o.download(np.float32)[:ks * B * M].reshape(ks, B, M)
        Y = P[0].copy()
        for c in range(1, ks):
            Y += P[c]
        for b in range(B):
            assert_close(Y[b], O.matmul(X[b], W, M, N, wtype), what=f"{wtype} M={M} vector {b} ({ks} chunks)")
