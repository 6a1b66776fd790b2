"""The bounded q/k/v hand-off of g4_qkvAttnDecodeFusedWarm fails loudly.

The one q/k/v + attention launch has its attention workgroups poll for the
q/k/v values its matvec workgroups stage (src/engine.ts:1547-1584 is the
dependency it fuses). The poll is bounded so that every workgroup ends; when
it expires the launch must not pass for a good one: its attention output and
the K/V row it stores are NaN, and the context reports G4_ERR_STALLED at the
synchronisation that follows and at every later call until g4_clear_stall.

The expiry is forced from the host (g4_test_stage_wait: a 64-poll limit and
no matvec workgroups, so nothing is ever staged): every kernel still ends
normally. Each test runs on a context of its own so that the sticky status
cannot reach other tests.
"""
import ctypes

import numpy as np
import pytest

import g4hip
from g4hip._lib import G4Error, lib
from gpu_util import bits_equal
from test_gpu_qkv_attn import H, HD, NQH, _setup

pytestmark = pytest.mark.gpu

STALLED = -7
POS, WINDOW, CAP = 700, 512, 1024


def _prepare(ctx, host, dev, W, table, rope, p, regions, ws):
    """Buffers of one call (uploaded now), and the launch, which enqueues only."""
    dk, dv = ctx.from_numpy(host["k"]), ctx.from_numpy(host["v"])
    q, k, v = (ctx.empty(n, np.float32) for n in (NQH * HD, HD, HD))
    h_out, out = ctx.empty(H, np.float32), ctx.empty(NQH * HD, np.float32)
    pdev = ctx.from_numpy(np.array([POS], np.uint32))

    def launch():
        ctx.qkvAttnDecodeFusedWarm(dev["x"], dev["w1"], dev["res"], None, dev["w2"], h_out, W[:3], [q, k, v], H,
                                   1e-6, dev["qn"], dev["kn"], table, dk, dv, out, p, ws, pdev, regions, rope, CAP)
    return launch, out, dk, dv


def _call(ctx, *S):
    launch, out, dk, dv = _prepare(ctx, *S)
    launch()
    return out, dk, dv


def _expect_stalled(fn):
    with pytest.raises(G4Error) as e:
        fn()
    assert e.value.code == STALLED, str(e.value)
    assert "bounded wait" in str(e.value)


@pytest.fixture()
def own_ctx():
    c = g4hip.Context(0)
    yield c
    c.clear_stall()
    c.close()


def test_expired_hand_off_is_reported_and_poisons(own_ctx):
    ctx = own_ctx
    S = _setup(ctx, 11, POS, WINDOW, CAP)
    host, dev, W, table, rope, p, regions = S
    assert ctx.qkv_attn_single_launch(p, H, 3)
    ws = ctx.zeros(ctx.attn_fused_workspace_bytes(p), np.uint8)
    out, dk, dv = _call(ctx, *S, ws)
    good = [out.download(np.float32), dk.download(np.uint16), dv.download(np.uint16)]
    assert np.all(np.isfinite(good[0]))

    ctx.test_stage_wait(64, True)
    print("[stall] forced expiry: 64 polls, no matvec workgroups", flush=True)
    out2, dk2, dv2 = _call(ctx, *S, ws)
    _expect_stalled(ctx.sync)
    # sticky: a later call and a download report it too
    _expect_stalled(lambda: ctx.test_stage_wait(0, False))
    _expect_stalled(lambda: out2.download(np.float32))
    ctx.clear_stall()
    ctx.test_stage_wait(0, False)
    got = out2.download(np.float32)
    assert np.all(np.isnan(got)), f"{np.count_nonzero(~np.isnan(got))} outputs are not NaN"
    row = slice(POS * HD, (POS + 1) * HD)
    for cache in (dk2, dv2):
        c = cache.download(np.uint16).view(np.float16)
        assert np.all(np.isnan(c[row])), "the stored K/V row is not NaN"
        assert np.array_equal(np.delete(c.view(np.uint16), np.arange(row.start, row.stop)),
                              np.delete(host["k" if cache is dk2 else "v"], np.arange(row.start, row.stop)))

    # after the acknowledgement and a zeroed workspace, the launch is good again
    ws.zero()
    out3, dk3, dv3 = _call(ctx, *S, ws)
    again = [out3.download(np.float32), dk3.download(np.uint16), dv3.download(np.uint16)]
    for a, b in zip(good, again):
        assert bits_equal(a, b)
    for w in W:
        w.free()


def test_expired_hand_off_is_reported_by_events(own_ctx):
    """An event recorded behind the stalled launch reports the stall once it
    completes (g4_event_wait, g4_event_query). A 2 GiB fill ahead of the
    launch keeps the stream busy well past the host's record call, so the
    record itself precedes the stall."""
    ctx = own_ctx
    S = _setup(ctx, 12, POS, WINDOW, CAP)
    ws = ctx.zeros(ctx.attn_fused_workspace_bytes(S[5]), np.uint8)
    busy = ctx.empty(1 << 29, np.float32)
    launch, out, _, _ = _prepare(ctx, *S, ws)
    ctx.sync()
    ctx.test_stage_wait(64, True)
    ctx.fill_normal_f32(busy, 1 << 29, 3, 0.0, 1.0)
    launch()
    ev = ctypes.c_void_p()
    rc = lib().g4_event_record(ctx.h, ctypes.byref(ev))
    if rc == 0:
        assert lib().g4_event_wait(ev) == STALLED
        assert lib().g4_event_query(ev) == STALLED
        ctx.destroy_event(ev)
    else:  # the stream drained before the record: the record reports it
        assert rc == STALLED
    print(f"[stall] reported by {'g4_event_wait' if rc == 0 else 'g4_event_record'}", flush=True)
    ctx.clear_stall()
    assert np.all(np.isnan(out.download(np.float32)))
    ctx.test_stage_wait(0, False)
    ctx.sync()
    busy.free()
    for w in S[2]:
        w.free()


def test_spin_limit_alone_keeps_results(own_ctx):
    """A lowered poll limit with the matvec present: the hand-off completes
    well within 4096 polls, and the results are the normal launch's."""
    ctx = own_ctx
    S = _setup(ctx, 13, POS, WINDOW, CAP)
    ws = ctx.zeros(ctx.attn_fused_workspace_bytes(S[5]), np.uint8)
    out, dk, _ = _call(ctx, *S, ws)
    ref = [out.download(np.float32), dk.download(np.uint16)]
    ctx.test_stage_wait(4096, False)
    out2, dk2, _ = _call(ctx, *S, ws)
    ctx.sync()
    ctx.test_stage_wait(0, False)
    assert bits_equal(ref[0], out2.download(np.float32))
    assert bits_equal(ref[1], dk2.download(np.uint16))
    for w in S[2]:
        w.free()
