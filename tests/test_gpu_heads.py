"""The attention merge moved into the o projection, by head.

g4_qkvAttnDecodePartials runs the q/k/v matvec and the attention block in
one launch whose attention workgroups end after storing their chunk partials;
g4_attnHeadsMatmul_q4k merges each head's chunks and multiplies the heads of
each group with their input columns of W_o (out[g] = sum over the group's
heads h of W_o[:, 256h:256h+256] . o_h); and
g4_normAddPartsGateUpGeluDigits_q4k adds the O_SHARES shares in order before
the post-attention norm-add (src/engine.ts:1550-1602 is the sequence these
three launches compute).

Checked against the oracle at rel-L2 1e-3 / cosine 0.9999: every share
against the oracle's matvec of its heads' attention output, and their sum
against the oracle's o projection; q/k/v and the stored K/V rows equal
the one-launch form with the merge (g4_qkvAttnDecodeFusedWarm) bit for bit;
the gate/up over the shares equals the gate/up over their in-order f32 sum
bit for bit. Repeated calls on one workspace (the heads launch clears the
staged q/k/v for the next one), the benchmark's global and local windows,
and an expired hand-off (NaN shares, G4_ERR_STALLED).
"""
import numpy as np
import pytest

import g4hip
import oracle as O
from g4hip._lib import O_SHARES, G4Error
from gpu_util import assert_close, bits_equal
from test_gpu_qkv_attn import H, HD, NQH, _setup

pytestmark = pytest.mark.gpu


def _wo(ctx, seed):
    W = O.gen_q4k(seed, H * NQH * HD // 256)
    return W, ctx.from_numpy(W)


HPS = NQH // O_SHARES  # heads per share


def _group_blocks(W, g):
    """Super-blocks HPS g .. HPS g + HPS - 1 of every row of W_o [H][8 * 256]
    (Q4_K): the columns of the heads of share g."""
    return np.ascontiguousarray(W.reshape(H, NQH, 144)[:, HPS * g:HPS * (g + 1), :]).reshape(-1)


def _run(ctx, S, ws, dwo, pos, cap, partials):
    host, dev, W, table, rope, p, regions = S
    dk, dv = ctx.from_numpy(host["k"]), ctx.from_numpy(host["v"])
    q, k, v = (ctx.empty(n, np.float32) for n in (NQH * HD, HD, HD))
    h_out = ctx.empty(H, np.float32)
    pdev = ctx.from_numpy(np.array([pos], np.uint32))
    if partials:
        parts = ctx.empty(O_SHARES * H, np.float32)
        ctx.qkvAttnDecodePartials(dev["x"], dev["w1"], dev["res"], None, dev["w2"], h_out, W[:3], [q, k, v], H, 1e-6,
                                  dev["qn"], dev["kn"], table, dk, dv, p, ws, pdev, regions, rope, cap)
        ctx.attnHeadsMatmul_q4k(ws, p, pdev, dwo, parts, H)
        return {"parts": parts.download(np.float32).reshape(O_SHARES, H), "k": dk.download(np.uint16),
                "v": dv.download(np.uint16), "q": q.download(np.float32), "h": h_out.download(np.float32)}
    out = ctx.empty(NQH * HD, np.float32)
    ctx.qkvAttnDecodeFusedWarm(dev["x"], dev["w1"], dev["res"], None, dev["w2"], h_out, W[:3], [q, k, v], H, 1e-6,
                               dev["qn"], dev["kn"], table, dk, dv, out, p, ws, pdev, regions, rope, cap)
    return {"attn": out.download(np.float32), "k": dk.download(np.uint16), "v": dv.download(np.uint16),
            "q": q.download(np.float32), "h": h_out.download(np.float32)}


@pytest.mark.parametrize("pos,window,cap", [(700, 512, 1024), (600, 0, 1024), (5, 0, 1024), (1023, 512, 1024),
                                            (40, 512, 1024)])
def test_heads_match_oracle_and_merged_form(ctx, pos, window, cap):
    S = _setup(ctx, 90 + pos + window, pos, window, cap)
    p = S[5]
    assert ctx.qkv_attn_single_launch(p, H, 3)
    W, dwo = _wo(ctx, 77 + pos)
    ws_m = ctx.zeros(ctx.attn_fused_workspace_bytes(p), np.uint8)
    ws_p = ctx.zeros(ctx.attn_fused_workspace_bytes(p), np.uint8)
    merged = _run(ctx, S, ws_m, dwo, pos, cap, False)
    attn = merged["attn"].reshape(NQH, HD)
    for rep in range(3):  # one workspace: the heads launch clears what the next partials launch polls
        got = _run(ctx, S, ws_p, dwo, pos, cap, True)
        for key in ("q", "k", "v", "h"):
            assert bits_equal(got[key], merged[key]), (rep, key)
        for g in range(O_SHARES):
            assert_close(got["parts"][g], O.matmul(attn[HPS * g:HPS * (g + 1)].reshape(-1), _group_blocks(W, g), H,
                                                   HPS * HD, "q4k"), what=f"share {g}, pos {pos} window {window}")
        total = got["parts"].astype(np.float32)
        acc = total[0].copy()
        for g in range(1, O_SHARES):
            acc = (acc + total[g]).astype(np.float32)
        assert_close(acc, O.matmul(merged["attn"], W, H, NQH * HD, "q4k"), what=f"o, pos {pos} window {window}")
    for w in S[2]:
        w.free()


def test_gate_up_over_shares_equals_over_their_sum(ctx):
    I = 6144
    parts = O.gen_normal_f32(61, O_SHARES * H, 0.0, 0.3).reshape(O_SHARES, H)
    acc = parts[0].copy()
    for g in range(1, O_SHARES):
        acc = (acc + parts[g]).astype(np.float32)
    res = O.gen_normal_f32(62, H)
    w_post, w_pre = O.gen_normal_f16(63, H, 1.0, 0.1), O.gen_normal_f16(64, H, 1.0, 0.1)
    Wg, Wu = O.gen_q4k(65, I * H // 256), O.gen_q4k(66, I * H // 256)
    d = {n: ctx.from_numpy(a) for n, a in (("res", res), ("wpost", w_post), ("wpre", w_pre), ("wg", Wg), ("wu", Wu))}
    outs = []
    for form in ("shares", "sum"):
        h_out, out = ctx.empty(H, np.float32), ctx.empty(I, np.float32)
        dig = ctx.zeros(ctx.digits_bytes(I), np.uint8)
        if form == "shares":
            ctx.normAddPartsGateUpGeluDigits_q4k(ctx.from_numpy(parts), d["wpost"], d["res"], d["wpre"], d["wg"],
                                                 d["wu"], h_out, out, dig, I, H, 1e-6)
        else:
            ctx.normAddGateUpGeluDigits_q4k(ctx.from_numpy(acc), d["wpost"], d["res"], d["wpre"], d["wg"], d["wu"],
                                            h_out, out, dig, I, H, 1e-6)
        outs.append([h_out.download(np.float32), out.download(np.float32), dig.download(np.uint8)])
    for a, b in zip(*outs):
        assert bits_equal(a, b)
    # and the oracle's FFN input on the summed o
    h = O.fused_norm_add(acc, w_post, res, 1e-6)
    assert_close(outs[0][0], h, what="h over the shares")


def test_heads_after_expired_hand_off_are_nan():
    """An expired hand-off in the partials launch: the heads launch that
    follows writes NaN shares and the synchronisation reports the stall. A
    2 GiB fill ahead of both launches keeps the stream busy while the host
    enqueues them (so neither entry sees the stall before it is enqueued)."""
    ctx = g4hip.Context(0)
    try:
        pos, window, cap = 700, 512, 1024
        S = _setup(ctx, 31, pos, window, cap)
        host, dev, W, table, rope, p, regions = S
        _, dwo = _wo(ctx, 32)
        ws = ctx.zeros(ctx.attn_fused_workspace_bytes(p), np.uint8)
        parts = ctx.empty(O_SHARES * H, np.float32)
        pdev = ctx.from_numpy(np.array([pos], np.uint32))
        qkv = [ctx.empty(NQH * HD, np.float32), ctx.empty(HD, np.float32), ctx.empty(HD, np.float32)]
        dk, dv = ctx.from_numpy(host["k"]), ctx.from_numpy(host["v"])
        busy = ctx.empty(1 << 29, np.float32)
        ctx.sync()
        ctx.test_stage_wait(64, True)
        ctx.fill_normal_f32(busy, 1 << 29, 5, 0.0, 1.0)
        ctx.qkvAttnDecodePartials(dev["x"], dev["w1"], dev["res"], None, dev["w2"], None, W[:3], qkv, H, 1e-6,
                                  dev["qn"], dev["kn"], table, dk, dv, p, ws, pdev, regions, rope, cap)
        ctx.attnHeadsMatmul_q4k(ws, p, pdev, dwo, parts, H)
        with pytest.raises(G4Error) as e:
            ctx.sync()
        assert e.value.code == -7
        ctx.clear_stall()
        ctx.test_stage_wait(0, False)
        got = parts.download(np.float32)
        assert np.all(np.isnan(got)), f"{np.count_nonzero(~np.isnan(got))} shares are not NaN"
        busy.free()
        for w in S[2]:
            w.free()
    finally:
        ctx.clear_stall()
        ctx.close()


def test_partials_entry_rejects_shapes_without_the_one_launch(ctx):
    pos, window, cap = 3000, 0, 4096  # a global window past 1024 positions
    S = _setup(ctx, 41, pos, window, cap)
    host, dev, W, table, rope, p, regions = S
    ws = ctx.zeros(ctx.attn_fused_workspace_bytes(p), np.uint8)
    q, k, v = (ctx.empty(n, np.float32) for n in (NQH * HD, HD, HD))
    pdev = ctx.from_numpy(np.array([pos], np.uint32))
    with pytest.raises(G4Error, match="one q/k/v"):
        ctx.qkvAttnDecodePartials(dev["x"], dev["w1"], dev["res"], None, dev["w2"], None, W[:3], [q, k, v], H, 1e-6,
                                  dev["qn"], dev["kn"], table, ctx.from_numpy(host["k"]), ctx.from_numpy(host["v"]),
                                  p, ws, pdev, regions, rope, cap)
    _, dwo = _wo(ctx, 42)
    with pytest.raises(G4Error, match="long attention form"):
        ctx.attnHeadsMatmul_q4k(ws, p, pdev, dwo, ctx.empty(O_SHARES * H, np.float32), H)
    for w in S[2]:
        w.free()
