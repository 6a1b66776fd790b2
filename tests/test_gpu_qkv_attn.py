"""g4_qkvAttnDecodeFusedWarm: the q/k/v matvecs (src/engine.ts:1550-1555,
over the attention rmsNorm of the residual stream) and the attention block
(src/engine.ts:1556-1584) in one launch. Its results are those of the two
calls it replaces (normAddScaleMatmulSegments, then attnDecodeFusedWarm),
bit for bit: the attention output, q/k/v, the new residual and the caches.
Both calls are pinned against the oracle by their own tests.

Cases: a producer layer with the norm-add prologue, layer 0's plain rmsNorm,
a layer reading its producer's cache (q only: two launches), windows merged
in the launch (one launch) and a global window past 1024 positions (two
launches), each
called three times on one workspace (the flags the launch sets must be clear
again for the next call), and with a per-layer output scale.
"""
import numpy as np
import pytest

from gpu_util import bits_equal

pytestmark = pytest.mark.gpu

H, HD, NQH = 1536, 256, 8


def _setup(ctx, seed, pos, window, cap):
    rng = np.random.default_rng(seed)
    f16 = lambda a: np.asarray(a, np.float32).astype(np.float16).view(np.uint16)  # noqa: E731
    host = {
        "x": rng.standard_normal(H).astype(np.float32) * 2,
        "res": rng.standard_normal(H).astype(np.float32),
        "w1": f16(rng.standard_normal(H) * 0.1 + 1),
        "w2": f16(rng.standard_normal(H) * 0.1 + 1),
        "qn": f16(rng.standard_normal(HD) * 0.1 + 1),
        "kn": f16(rng.standard_normal(HD) * 0.1 + 1),
        "k": f16(rng.standard_normal(cap * HD)),
        "v": f16(rng.standard_normal(cap * HD)),
        "scale": f16([0.75, 0]),
    }
    dev = {n: ctx.from_numpy(a) for n, a in host.items() if n not in ("k", "v")}
    W = []
    for i, M in enumerate((NQH * HD, HD, HD)):
        nb = M * H // 256
        w = ctx.alloc(nb * 144)
        ctx.fill_q4k(w, nb, seed * 10 + i)
        W.append(w)
    theta, div = (1e6, 1) if window == 0 else (1e4, 0)
    table = ctx.from_numpy(np.where(np.arange(HD // 2) < HD // 8, 1.0, np.inf).astype(np.float16).view(np.uint16))
    rope = ctx.empty(cap * HD, np.float32)
    ctx.ropeTable(theta, div, table, HD, cap, rope)
    p = ctx.attn_fused_params(NQH, 1, HD, cap, window, 1e-6, theta, div)
    regions = []
    for M, N in ((6144, 1536), (1536, 6144)):
        nb = M * N // 256
        w = ctx.alloc(nb * 144)
        ctx.fill_q4k(w, nb, M)
        regions.append(ctx.matmulWarmRegion("q4k", M, N, w))
        W.append(w)
    return host, dev, W, table, rope, p, regions


@pytest.mark.parametrize("pos,window,cap,form", [
    (700, 512, 1024, "norm_add"),
    (700, 512, 1024, "first"),
    (700, 512, 1024, "consumer"),
    (700, 512, 1024, "scaled"),
    (600, 0, 1024, "norm_add"),
    (5, 0, 1024, "norm_add"),
    (3000, 0, 4096, "norm_add"),
])
def test_qkv_attn_matches_two_calls(ctx, pos, window, cap, form):
    host, dev, W, table, rope, p, regions = _setup(ctx, pos + cap + len(form), pos, window, cap)
    nseg = 1 if form == "consumer" else 3
    res = None if form == "first" else dev["res"]
    w2 = None if form == "first" else dev["w2"]
    scale = dev["scale"] if form == "scaled" else None
    kn = None if form == "consumer" else dev["kn"]
    one = ctx.qkv_attn_single_launch(p, H, nseg)
    print(f"[qkv+attn] pos={pos} window={window} cap={cap} {form}: one launch {one}", flush=True)
    assert one == (cap <= 1024 and nseg == 3)
    results = []
    ws_two = ctx.zeros(ctx.attn_fused_workspace_bytes(p), np.uint8)
    ws_one = ctx.zeros(ctx.attn_fused_workspace_bytes(p), np.uint8)
    for fused in (False, True, True, True):
        ws = ws_one if fused else ws_two
        dk, dv = ctx.from_numpy(host["k"]), ctx.from_numpy(host["v"])
        q, k, v = (ctx.empty(n, np.float32) for n in (NQH * HD, HD, HD))
        outs = [q, k, v][:nseg]
        h_out = None if form == "first" else ctx.empty(H, np.float32)
        out = ctx.empty(NQH * HD, np.float32)
        pdev = ctx.from_numpy(np.array([pos], np.uint32))
        if fused:
            ctx.qkvAttnDecodeFusedWarm(dev["x"], dev["w1"], res, scale, w2, h_out, W[:nseg], outs, H, 1e-6,
                                       dev["qn"], kn, table, dk, dv, out, p, ws, pdev, regions, rope, cap)
        else:
            ctx.normAddScaleMatmulSegments("q4k", dev["x"], dev["w1"], res, scale, w2, h_out, W[:nseg], outs,
                                           [NQH * HD, HD, HD][:nseg], H, 1e-6)
            ctx.attnDecodeFusedWarm(q, k if nseg == 3 else None, v if nseg == 3 else None, dev["qn"], kn, table,
                                    dk, dv, out, p, ws, pdev, regions, rope, cap)
        got = [out.download(np.float32), dk.download(np.uint16), dv.download(np.uint16)]
        got += [t.download(np.float32) for t in outs]
        if h_out is not None:
            got.append(h_out.download(np.float32))
        results.append(got)
    assert np.all(np.isfinite(results[0][0]))
    for r in results[1:]:
        assert len(r) == len(results[0])
        for i, (a, b) in enumerate(zip(results[0], r)):
            assert bits_equal(a, b), f"output {i} differs"
    for w in W:
        w.free()


def test_qkv_attn_flags_clear_across_layers(ctx):
    """Two layers of different windows alternate on one workspace (as the
    decode step's layers do), each call checked against the two-call result."""
    cap = 1024
    A = _setup(ctx, 7, 700, 512, cap)
    B = _setup(ctx, 8, 700, 0, cap)
    ws = ctx.zeros(max(ctx.attn_fused_workspace_bytes(A[5]), ctx.attn_fused_workspace_bytes(B[5])), np.uint8)
    ws2 = ctx.zeros(ws.nbytes, np.uint8)
    for rnd in range(3):
        for host, dev, W, table, rope, p, regions in (A, B):
            got = []
            for fused, w in ((False, ws2), (True, ws)):
                dk, dv = ctx.from_numpy(host["k"]), ctx.from_numpy(host["v"])
                q, k, v = (ctx.empty(n, np.float32) for n in (NQH * HD, HD, HD))
                h_out, out = ctx.empty(H, np.float32), ctx.empty(NQH * HD, np.float32)
                pdev = ctx.from_numpy(np.array([700 + rnd], np.uint32))
                if fused:
                    ctx.qkvAttnDecodeFusedWarm(dev["x"], dev["w1"], dev["res"], None, dev["w2"], h_out, W[:3],
                                               [q, k, v], H, 1e-6, dev["qn"], dev["kn"], table, dk, dv, out, p, w,
                                               pdev, regions, rope, cap)
                else:
                    ctx.normAddScaleMatmulSegments("q4k", dev["x"], dev["w1"], dev["res"], None, dev["w2"], h_out,
                                                   W[:3], [q, k, v], [NQH * HD, HD, HD], H, 1e-6)
                    ctx.attnDecodeFusedWarm(q, k, v, dev["qn"], dev["kn"], table, dk, dv, out, p, w, pdev,
                                            regions, rope, cap)
                got.append([out.download(np.float32), dk.download(np.uint16), q.download(np.float32)])
            for a, b in zip(*got):
                assert bits_equal(a, b), f"round {rnd} window {p.sliding_window}"
    for S in (A, B):
        for w in S[2]:
            w.free()
