"""The allocation-free decode attention entry point (g4_attnDecode_noalloc)
against the workspace entry point it varies (g4_attnDecode): same kernels,
so the outputs are bit-identical, and both within rel-L2 1e-3 of the f64
oracle. Two calls in a row, the second with a smaller input, share the
static partials array; a shape whose partials exceed it is refused."""
import numpy as np
import pytest

import oracle as O
from g4hip import G4Error
from gpu_util import assert_close, bits_equal

pytestmark = pytest.mark.gpu


def _case(ctx, L, window, hd, seed):
    nqh, nkh = 8, 1
    k = O.gen_normal_f16(seed, L * nkh * hd)
    v = O.gen_normal_f16(seed + 1, L * nkh * hd)
    q = O.fused_per_head_norm_rope(O.gen_normal_f32(seed + 2, nqh * hd), O.gen_normal_f16(seed + 3, hd, 1.0, 0.1),
                                   nqh, hd, 1e-6, 0, 1e4, 0, np.ones(hd // 2, np.float16).view(np.uint16))
    dq, dk, dv = ctx.from_numpy(q), ctx.from_numpy(k), ctx.from_numpy(v)
    ws = ctx.zeros(ctx.attn_workspace_bytes(nqh, nkh, hd, L, window), np.uint8)
    ref = ctx.empty(nqh * hd, np.float32)
    ctx.attnDecode(dq, dk, dv, ref, nqh, nkh, hd, L, 1.0, window, workspace=ws)
    out = ctx.empty(nqh * hd, np.float32)
    print(f"[noalloc] L={L} window={window} hd={hd}", flush=True)
    ctx.attnDecodeNoAlloc(dq, dk, dv, out, nqh, nkh, hd, L, 1.0, window)
    got, want = out.download(np.float32), ref.download(np.float32)
    assert bits_equal(got, want), (L, window, hd)
    assert_close(got, O.attention(q, k, v, nqh, nkh, hd, L, 1.0, window), what=f"noalloc L={L}")
    return got


def test_noalloc_matches_workspace_entry(ctx):
    a = _case(ctx, 32768, 0, 512, 501)     # the largest E2B global shape (8.4 MB of partials)
    b = _case(ctx, 600, 512, 256, 601)     # then a smaller one over the same array
    assert a.shape == (8 * 512,) and b.shape == (8 * 256,)
    c = _case(ctx, 4096, 0, 256, 701)
    assert np.all(np.isfinite(c))


def test_noalloc_refuses_oversized_partials(ctx):
    nqh, hd = 8, 512
    buf = ctx.zeros(4096, np.uint8)
    with pytest.raises(G4Error, match="static scratch"):
        ctx.attnDecodeNoAlloc(buf, buf, buf, buf, nqh, 1, hd, 65536, 1.0, 0)
