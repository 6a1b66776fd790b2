"""GPU parity: decode attention over an f16 KV cache — the per-key trio and
the split-K flash-decode (dense, device-position and paged/ragged forms)
against the f64 oracle (rel-L2 <= 1e-3, cos >= 0.9999)."""
import numpy as np
import pytest

import oracle as O
from gpu_util import assert_close, bits_equal

pytestmark = pytest.mark.gpu


def kv(seed, L, nkh, hd):
    k = O.gen_normal_f16(seed, L * nkh * hd)
    v = O.gen_normal_f16(seed + 1, L * nkh * hd)
    return k, v


def unit_q(seed, nqh, hd):
    # q after q_norm (unit RMS, weights ~ N(1, 0.1))
    q = O.gen_normal_f32(seed, nqh * hd)
    w = O.gen_normal_f16(seed + 2, hd, 1.0, 0.1)
    no = np.ones(hd // 2, np.float16).view(np.uint16)
    return O.fused_per_head_norm_rope(q, w, nqh, hd, 1e-6, 0, 1e4, 0, no)


@pytest.mark.parametrize("L,window", [(1, 0), (7, 0), (33, 512), (600, 512), (600, 0)])
def test_trio(ctx, L, window):
    nqh, nkh, hd = 8, 1, 256
    k, v = kv(L, L, nkh, hd)
    q = unit_q(L + 3, nqh, hd)
    dq, dk, dv = ctx.from_numpy(q), ctx.from_numpy(k), ctx.from_numpy(v)
    sc = ctx.empty(nqh * L, np.float32)
    ctx.attnScore(dq, dk, sc, nqh, nkh, hd, L, 1.0, window)
    s_ref = O.attn_score(q, k, nqh, nkh, hd, L, 1.0, window)
    s = sc.download(np.float32)
    masked = s_ref == np.float32(-1e30)
    assert np.array_equal(s == np.float32(-1e30), masked)
    assert_close(s[~masked], s_ref[~masked], rel=1e-6, cos=0.99999999, what="scores")
    ctx.softmax(sc, nqh, L)
    out = ctx.empty(nqh * hd, np.float32)
    ctx.attnOutput(sc, dv, out, nqh, nkh, hd, L)
    assert_close(out.download(np.float32), O.attention(q, k, v, nqh, nkh, hd, L, 1.0, window), what="trio")


def test_trio_dev_graph_replay(ctx):
    """The trio with seq_len read from the device (src/engine.ts:1496-1504
    patches it per forward): one captured graph replayed at positions 40, 41,
    42 (a device-side position advance ends each replay) gives the oracle's
    attention at every length, with the scores rows at stride seq_len, and
    memset / upload / download / stream sync are refused inside the capture."""
    nqh, nkh, hd, max_len, window = 8, 1, 256, 64, 32
    k, v = kv(91, max_len, nkh, hd)
    q = unit_q(93, nqh, hd)
    dq, dk, dv = ctx.from_numpy(q), ctx.from_numpy(k), ctx.from_numpy(v)
    sc = ctx.zeros(nqh * max_len, np.float32)
    out = ctx.empty(nqh * hd, np.float32)
    pos = ctx.from_numpy(np.array([40], np.uint32))
    ctx.graph_begin()
    try:
        ctx.attnScore(dq, dk, sc, nqh, nkh, hd, max_len, 1.0, window, position_dev=pos)
        ctx.softmax(sc, nqh, max_len, position_dev=pos)
        ctx.attnOutput(sc, dv, out, nqh, nkh, hd, max_len, position_dev=pos)
        ctx.advancePosition(pos, 1)
        for bad in (lambda: sc.zero(), lambda: pos.upload(np.array([1], np.uint32)),
                    lambda: pos.download(np.uint32), lambda: ctx.sync()):
            with pytest.raises(Exception, match="while a graph is being captured"):
                bad()
    finally:
        g = ctx.graph_end()
    try:
        for p in (40, 41, 42):
            ctx.graph_launch(g)
            ctx.sync()
            L = p + 1
            got = out.download(np.float32)
            assert_close(got, O.attention(q, k, v, nqh, nkh, hd, L, 1.0, window), what=f"dev trio L={L}")
            probs = sc.download(np.float32)[:nqh * L].reshape(nqh, L)
            assert np.allclose(probs.sum(axis=1), 1.0, rtol=1e-5)
            assert np.all(probs[:, :L - window] == 0)          # masked rows: exp(-1e30 - max) = 0
        assert int(pos.download(np.uint32)[0]) == 43
    finally:
        ctx.graph_destroy(g)
    # a device position past the maximum is clamped to it
    pos.upload(np.array([1000], np.uint32))
    ctx.attnScore(dq, dk, sc, nqh, nkh, hd, max_len, 1.0, window, position_dev=pos)
    ctx.softmax(sc, nqh, max_len, position_dev=pos)
    ctx.attnOutput(sc, dv, out, nqh, nkh, hd, max_len, position_dev=pos)
    assert_close(out.download(np.float32), O.attention(q, k, v, nqh, nkh, hd, max_len, 1.0, window), what="clamped")


DECODE_CASES = [
    # (L, window, head_dim): short, E2B local (W=512), the config-3 contexts
    (1, 0, 256), (7, 0, 256), (64, 0, 256), (65, 0, 256), (600, 512, 256), (600, 0, 256),
    (512, 0, 256), (4096, 0, 256), (4096, 512, 256), (32768, 0, 256), (5000, 0, 512), (777, 0, 128),
]


@pytest.mark.parametrize("L,window,hd", DECODE_CASES)
def test_attn_decode(ctx, L, window, hd):
    nqh, nkh = 8, 1
    k, v = kv(L * 3 + hd, L, nkh, hd)
    q = unit_q(L + 5, nqh, hd)
    ref = O.attention(q, k, v, nqh, nkh, hd, L, 1.0, window)
    out = ctx.empty(nqh * hd, np.float32)
    ws = ctx.zeros(ctx.attn_workspace_bytes(nqh, nkh, hd, L, window), np.uint8)
    dk, dv = ctx.from_numpy(k), ctx.from_numpy(v)
    ctx.attnDecode(ctx.from_numpy(q), dk, dv, out, nqh, nkh, hd, L, 1.0, window, workspace=ws)
    assert_close(out.download(np.float32), ref, what=f"L={L} W={window}")


def test_attn_decode_gqa_groups(ctx):
    for nqh, nkh in [(8, 2), (4, 4), (8, 8)]:
        hd, L = 256, 300
        k, v = kv(nqh * 10 + nkh, L, nkh, hd)
        q = O.gen_normal_f32(nqh, nqh * hd)
        out = ctx.empty(nqh * hd, np.float32)
        ctx.attnDecode(ctx.from_numpy(q), ctx.from_numpy(k), ctx.from_numpy(v), out, nqh, nkh, hd, L)
        assert_close(out.download(np.float32), O.attention(q, k, v, nqh, nkh, hd, L), what=f"{nqh}/{nkh}")


def test_attn_decode_dev_position(ctx):
    """Capacity-sized plan, live length read on the device (graph replay form)."""
    nqh, nkh, hd, cap = 8, 1, 256, 8192
    k, v = kv(99, cap, nkh, hd)
    q = unit_q(98, nqh, hd)
    dk, dv, dq = ctx.from_numpy(k), ctx.from_numpy(v), ctx.from_numpy(q)
    ws = ctx.zeros(ctx.attn_workspace_bytes(nqh, nkh, hd, cap, 0), np.uint8)
    out = ctx.empty(nqh * hd, np.float32)
    for pos in (0, 100, 4095, cap - 1):
        pdev = ctx.from_numpy(np.array([pos], np.uint32))
        ctx.attnDecode(dq, dk, dv, out, nqh, nkh, hd, cap, 1.0, 0, workspace=ws, position_dev=pdev)
        assert_close(out.download(np.float32), O.attention(q, k, v, nqh, nkh, hd, pos + 1), what=f"pos={pos}")


@pytest.mark.parametrize("B,window", [(4, 0), (32, 0), (32, 512), (64, 0), (64, 512)])
def test_paged_ragged(ctx, B, window):
    nqh, nkh, hd, P = 8, 1, 256, 16
    rng = np.random.default_rng(B + window)
    lens = rng.integers(128, 8193, B).astype(np.uint32) if B > 4 else np.array([1, 16, 17, 1000], np.uint32)
    max_len = int(lens.max())
    max_pages = (max_len + P - 1) // P
    total_pages = int(sum((int(L) + P - 1) // P for L in lens)) + 7
    perm = rng.permutation(total_pages).astype(np.int32)
    table = np.zeros((B, max_pages), np.int32)
    k_pool = O.gen_normal_f16(1, total_pages * P * hd).reshape(-1, hd)
    v_pool = O.gen_normal_f16(2, total_pages * P * hd).reshape(-1, hd)
    c = 0
    for s in range(B):
        n = (int(lens[s]) + P - 1) // P
        table[s, :n] = perm[c:c + n]
        c += n
    q = O.gen_normal_f32(3, B * nqh * hd).reshape(B, nqh * hd)
    p = ctx.paged_params(B, nqh, nkh, hd, P, max_pages, max_len, total_pages, 1.0, window)
    ws = ctx.zeros(ctx.paged_workspace_bytes(p), np.uint8)
    out = ctx.empty(B * nqh * hd, np.float32)
    ctx.pagedAttnDecode(ctx.from_numpy(q), ctx.from_numpy(k_pool), ctx.from_numpy(v_pool), ctx.from_numpy(table),
                        ctx.from_numpy(lens), out, p, ws)
    got = out.download(np.float32).reshape(B, -1)
    for s in range(B):
        ref = O.attention_paged(q[s], k_pool.reshape(-1), v_pool.reshape(-1), table[s], P, nqh, nkh, hd,
                                int(lens[s]), 1.0, window)
        assert_close(got[s], ref, what=f"seq {s} len {lens[s]}")


def test_paged_kv_store(ctx):
    nkh, hd, P, B = 1, 256, 16, 3
    lens = np.array([1, 17, 32], np.uint32)
    table = np.array([[2, 0], [5, 1], [3, 4]], np.int32)
    kp = ctx.zeros(6 * P * hd, np.uint16)
    vp = ctx.zeros(6 * P * hd, np.uint16)
    k = O.gen_normal_f32(1, B * hd)
    v = O.gen_normal_f32(2, B * hd)
    p = ctx.paged_params(B, 8, nkh, hd, P, 2, 32, 6)
    ctx.pagedKvStore(ctx.from_numpy(k), ctx.from_numpy(v), kp, vp, ctx.from_numpy(table), ctx.from_numpy(lens), p)
    K = kp.download(np.uint16).reshape(-1, hd)
    V = vp.download(np.uint16).reshape(-1, hd)
    for s in range(B):
        pos = int(lens[s]) - 1
        row = table[s, pos // P] * P + pos % P
        assert np.array_equal(K[row], k.reshape(B, hd)[s].astype(np.float16).view(np.uint16))
        assert np.array_equal(V[row], v.reshape(B, hd)[s].astype(np.float16).view(np.uint16))
    assert np.count_nonzero(K.any(axis=1)) == B


FUSED_CASES = [
    # (position, window, head_dim, theta, apply_divisor): local layer (W=512,
    # theta 1e4), global layer (proportional table), short and long positions
    (0, 512, 256, 1e4, 0),
    (14, 512, 256, 1e4, 0),
    (700, 512, 256, 1e4, 0),
    (700, 0, 256, 1e6, 1),
    (3000, 0, 256, 1e6, 1),
    (900, 0, 512, 1e6, 1),
    # head dim 512 (Gemma-4-E2B's global layers): steps of 32 positions, two
    # per chunk; the first position, step and chunk edges, the benchmark's
    # context, a window, the merge launch past 16 chunks
    (0, 0, 512, 1e6, 1),
    (31, 0, 512, 1e6, 1),
    (32, 0, 512, 1e6, 1),
    (64, 0, 512, 1e6, 1),
    (512, 0, 512, 1e6, 1),
    (700, 512, 512, 1e4, 0),
    (1100, 0, 512, 1e6, 1),
    # long contexts: chunk partials merged in groups, then the groups
    (20000, 0, 256, 1e6, 1),
    (32767, 0, 256, 1e6, 1),
    (32767, 512, 256, 1e4, 0),
    (32767, 0, 512, 1e6, 1),
]


def _fused_inputs(pos, window, hd, theta, div):
    nqh, nkh = 8, 1
    cap = 4096 if pos < 4096 else 32768
    k, v = kv(pos + 11, cap, nkh, hd)
    qr = O.gen_normal_f32(pos + 1, nqh * hd, 0.0, 3.0)
    kr = O.gen_normal_f32(pos + 2, nkh * hd, 0.0, 3.0)
    vr = O.gen_normal_f32(pos + 3, nkh * hd, 0.0, 60.0)
    qw = O.gen_normal_f16(pos + 4, hd, 1.0, 0.1)
    kw = O.gen_normal_f16(pos + 5, hd, 1.0, 0.1)
    table = np.where(np.arange(hd // 2) < hd // 8, 1.0, np.inf).astype(np.float16).view(np.uint16)
    # oracle: the reference's per-key order (src/engine.ts:1562-1584)
    vq = O.per_head_rms_norm_no_weight(vr, nkh, hd, 1e-6)
    q = O.fused_per_head_norm_rope(qr, qw, nqh, hd, 1e-6, pos, theta, div, table)
    kk = O.fused_per_head_norm_rope(kr, kw, nkh, hd, 1e-6, pos, theta, div, table)
    k_ref, v_ref = k.copy(), v.copy()
    O.kv_cache_store_f16(kk, vq, k_ref, v_ref, nkh, hd, pos)
    ref = O.attention(q, k_ref, v_ref, nqh, nkh, hd, pos + 1, 1.0, window)
    return dict(nqh=nqh, nkh=nkh, cap=cap, k=k, v=v, qr=qr, kr=kr, vr=vr, qw=qw, kw=kw, table=table,
                k_ref=k_ref, v_ref=v_ref, ref=ref)


@pytest.mark.parametrize("pos,window,hd,theta,div", FUSED_CASES)
def test_attn_decode_fused(ctx, pos, window, hd, theta, div):
    """norm + RoPE on q/k, v_norm, KV store and attention in one launch equals
    the reference's per-key sequence restated by the oracle."""
    c = _fused_inputs(pos, window, hd, theta, div)
    nqh, nkh, cap = c["nqh"], c["nkh"], c["cap"]
    p = ctx.attn_fused_params(nqh, nkh, hd, cap, window, 1e-6, theta, div)
    ws = ctx.zeros(ctx.attn_fused_workspace_bytes(p), np.uint8)
    dk, dv = ctx.from_numpy(c["k"]), ctx.from_numpy(c["v"])
    out = ctx.empty(nqh * hd, np.float32)
    dq = ctx.from_numpy(c["qr"])
    pdev = ctx.from_numpy(np.array([pos], np.uint32))
    for rep in range(2):  # the arrival counters must be left zeroed for the next call
        ctx.attnDecodeFused(dq, ctx.from_numpy(c["kr"]), ctx.from_numpy(c["vr"]), ctx.from_numpy(c["qw"]),
                            ctx.from_numpy(c["kw"]), ctx.from_numpy(c["table"]), dk, dv, out, p, ws, pdev)
        assert_close(out.download(np.float32), c["ref"], what=f"fused pos={pos} rep={rep}")
    # the stored row: within an f16 rounding of the oracle's (the norm's f32
    # rounding differs from the oracle's f64 one); no other row touched
    k, v, k_ref, v_ref = c["k"], c["v"], c["k_ref"], c["v_ref"]
    kc, vc = dk.download(np.uint16).reshape(cap, hd), dv.download(np.uint16).reshape(cap, hd)
    assert np.max(np.abs(vc[pos].astype(np.int32) - v_ref.reshape(cap, hd)[pos].astype(np.int32))) <= 1
    assert np.max(np.abs(kc[pos].view(np.float16).astype(np.float32) -
                         k_ref.reshape(cap, hd)[pos].view(np.float16).astype(np.float32))) <= 2e-3
    other = np.arange(cap) != pos
    assert np.array_equal(kc[other], k.reshape(cap, hd)[other])
    assert np.array_equal(vc[other], v.reshape(cap, hd)[other])
    assert np.array_equal(c["qr"], dq.download(np.float32))   # q_raw is not modified


def test_attn_decode_fused_shared_workspace(ctx):
    """Layers of different windows, lengths and head sizes (the one-launch
    form and the two-launch form) share one workspace, as a decode step's
    layers do, over two rounds."""
    cases = [(700, 0, 256, 1e6, 1), (900, 0, 512, 1e6, 1), (3000, 512, 256, 1e4, 0), (3000, 0, 256, 1e6, 1),
             (20, 512, 256, 1e4, 0)]
    prepared = []
    need = 0
    for pos, window, hd, theta, div in cases:
        c = _fused_inputs(pos, window, hd, theta, div)
        p = ctx.attn_fused_params(c["nqh"], c["nkh"], hd, c["cap"], window, 1e-6, theta, div)
        need = max(need, ctx.attn_fused_workspace_bytes(p))
        dev = {n: ctx.from_numpy(c[n]) for n in ("qr", "kr", "vr", "qw", "kw", "table")}
        prepared.append((pos, hd, c, p, dev))
    ws = ctx.zeros(need, np.uint8)
    for rnd in range(2):
        for pos, hd, c, p, dev in prepared:
            dk, dv = ctx.from_numpy(c["k"]), ctx.from_numpy(c["v"])
            out = ctx.empty(c["nqh"] * hd, np.float32)
            ctx.attnDecodeFused(dev["qr"], dev["kr"], dev["vr"], dev["qw"], dev["kw"], dev["table"], dk, dv, out, p,
                                ws, ctx.from_numpy(np.array([pos], np.uint32)))
            assert_close(out.download(np.float32), c["ref"], what=f"shared ws round {rnd} pos={pos} hd={hd}")


@pytest.mark.parametrize("pos,window,hd", [(700, 512, 256), (3000, 0, 256), (20, 512, 256), (900, 0, 512)])
def test_attn_decode_fused_warm_matches(ctx, pos, window, hd):
    """The launch that also reads the following matvecs' weights into the L2
    caches and takes the RoPE cos/sin from a precomputed table computes
    exactly what the plain one does (output and caches bit for bit); the warm
    regions describe the matvec launches' own tiling, with sizes that are
    not multiples of a tile (a partial last tile reads past no matrix end)."""
    theta, div = (1e6 if window == 0 else 1e4), int(window == 0)
    c = _fused_inputs(pos, window, hd, theta, div)
    p = ctx.attn_fused_params(c["nqh"], c["nkh"], hd, c["cap"], window, 1e-6, theta, div)
    ws = ctx.zeros(ctx.attn_fused_workspace_bytes(p), np.uint8)
    dev = {n: ctx.from_numpy(c[n]) for n in ("qr", "kr", "vr", "qw", "kw", "table")}
    shapes = [("q4k", 1536, 2048), ("q4k", 6144, 1536), ("q4k", 1000, 1536), ("q6k", 1537, 6144)]
    mats, regions = [], []
    for wt, M, N in shapes:
        nb = M * N // 256
        w = ctx.alloc(nb * (144 if wt == "q4k" else 210))
        (ctx.fill_q4k if wt == "q4k" else ctx.fill_q6k)(w, nb, M + N)
        r = ctx.matmulWarmRegion(wt, M, N, w)
        assert r.total_bytes == nb * (144 if wt == "q4k" else 210)
        assert r.nwgs >= 1 and r.wg_bytes * r.nwgs >= r.total_bytes
        assert r.wg_bytes * (r.nwgs - 1) < r.total_bytes  # every workgroup has rows
        mats.append(w)
        regions.append(r)
    rope = ctx.empty(c["cap"] * hd, np.float32)
    ctx.ropeTable(theta, div, dev["table"], hd, c["cap"], rope)
    outs = []
    for warm in (False, True, True):
        dk, dv = ctx.from_numpy(c["k"]), ctx.from_numpy(c["v"])
        out = ctx.empty(c["nqh"] * hd, np.float32)
        args = (dev["qr"], dev["kr"], dev["vr"], dev["qw"], dev["kw"], dev["table"], dk, dv, out, p, ws,
                ctx.from_numpy(np.array([pos], np.uint32)))
        if warm:  # L2 warming and the RoPE table
            ctx.attnDecodeFusedWarm(*args, regions, rope, c["cap"])
        else:
            ctx.attnDecodeFused(*args)
        outs.append((out.download(np.float32), dk.download(np.uint16), dv.download(np.uint16)))
    for o in outs[1:]:
        for a, b in zip(outs[0], o):
            assert bits_equal(a, b)
    assert_close(outs[0][0], c["ref"], what=f"warm pos={pos}")
    with pytest.raises(RuntimeError):  # a table shorter than the cache
        ctx.attnDecodeFusedWarm(*args, regions, rope, c["cap"] - 1)
    for w in mats:
        w.free()


@pytest.mark.parametrize("theta,div,hd", [(1e4, 0, 256), (1e6, 1, 256), (1e6, 1, 512)])
def test_rope_table(ctx, theta, div, hd):
    """ropeTable: cos/sin of t * freq_i with freq_i the f32 of 1/theta^(2i/hd)
    (divided by the f16 divisor), the angle an f32 product
    (shaders/fused_per_head_norm_rope.wgsl:50-55), against f64 cos/sin of the
    same f32 angle; positions up to 32767 (large angles)."""
    rows = 32768
    half = hd // 2
    table = np.where(np.arange(half) < hd // 8, 1.0, np.inf).astype(np.float16)
    out = ctx.empty(rows * hd, np.float32)
    ctx.ropeTable(theta, div, ctx.from_numpy(table.view(np.uint16)), hd, rows, out)
    got = out.download(np.float32).reshape(rows, half, 2)
    i = np.arange(half)
    f = (1.0 / np.power(np.float64(theta), 2.0 * i / hd)).astype(np.float32)
    if div:
        f = (f / table.astype(np.float32)).astype(np.float32)
    t = np.arange(rows, dtype=np.float32)[:, None]
    ang = (t * f[None, :]).astype(np.float32).astype(np.float64)
    assert np.max(np.abs(got[..., 0] - np.cos(ang))) < 1e-6
    assert np.max(np.abs(got[..., 1] - np.sin(ang))) < 1e-6
