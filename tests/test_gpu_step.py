"""GPU parity of a whole decode step (E2B-shaped layers + tied Q6_K LM head):
the oracle composition, the per-key kernel sequence (the reference's
encodeTransformerPass order), the fused step and its HIP-graph replays."""
import numpy as np
import pytest

import oracle as O
from decode_oracle import HostModel
from g4hip.decoder import Decoder, E2BShape, qkv_groups
from gpu_util import assert_close, bits_equal

pytestmark = pytest.mark.gpu

N_LAYERS = 2
MAX_SEQ = 1024
POS = 600  # > window so the local layer masks


@pytest.fixture(scope="module")
def dec(ctx):
    # layer 0 local (window 512), layer 1 global
    shape = E2BShape(n_layers=N_LAYERS, global_layers=(1,))
    d = Decoder(ctx, shape, max_seq=MAX_SEQ, seed=3)
    d.fill_kv(POS, seed=4)
    ctx.sync()
    return d


def host(buf, dtype):
    return buf.download(dtype)


def oracle_step(d: Decoder, hidden, kcs, vcs, pos):
    return HostModel(d).step(hidden, kcs, vcs, pos)


def snapshot(d):
    return (host(d.hidden, np.float32), [host(L.k_cache, np.uint16) for L in d.layers],
            [host(L.v_cache, np.uint16) for L in d.layers])


def restore(d, snap):
    d.hidden.upload(snap[0])
    for L, k, v in zip(d.layers, snap[1], snap[2]):
        L.k_cache.upload(k)
        L.v_cache.upload(v)


def check_token(d, logits_gpu, what):
    tok = int(host(d.token, np.uint32)[0])
    assert tok == O.argmax(logits_gpu), what   # indices bit-exact on identical logits


def test_step_reference_and_fused_vs_oracle(ctx, dec):
    snap = snapshot(dec)
    kcs, vcs = [k.copy() for k in snap[1]], [v.copy() for v in snap[2]]
    x_ref, logits_ref = oracle_step(dec, snap[0], kcs, vcs, POS)   # stores the oracle's rows at POS
    kv = dec.s.kv_dim
    row = slice(POS * kv, (POS + 1) * kv)

    dec.step_reference(POS)
    ctx.sync()
    print(f"[step] per-key: hidden rel-L2 {O.rel_l2(host(dec.hidden, np.float32), x_ref):.2e}", flush=True)
    assert_close(host(dec.hidden, np.float32), x_ref, what="per-key hidden")
    lg = host(dec.logits, np.float32)
    assert_close(lg, logits_ref, what="per-key logits")
    check_token(dec, lg, "per-key token")
    perkey_rows = [(host(L.k_cache, np.uint16)[row], host(L.v_cache, np.uint16)[row]) for L in dec.layers]

    restore(dec, snap)
    dec.set_position(POS)
    dec.step_fused()
    ctx.sync()
    assert int(host(dec.pos, np.uint32)[0]) == POS + 1
    print(f"[step] fused: hidden rel-L2 {O.rel_l2(host(dec.hidden, np.float32), x_ref):.2e}", flush=True)
    assert_close(host(dec.hidden, np.float32), x_ref, what="fused hidden")
    lg = host(dec.logits, np.float32)
    assert_close(lg, logits_ref, what="fused logits")
    check_token(dec, lg, "fused token")
    # the K/V rows written at POS: the fused path's f16 rows within one f16
    # ulp of the per-key path's (the two round f32 values that differ in
    # their last bits), both within the tolerance of the oracle's rows, and
    # nothing else of the caches changed
    for il, L in enumerate(dec.layers):
        kall, vall = host(L.k_cache, np.uint16), host(L.v_cache, np.uint16)
        for nm, fused, perkey, ref, before in (("k", kall, perkey_rows[il][0], kcs[il], snap[1][il]),
                                               ("v", vall, perkey_rows[il][1], vcs[il], snap[2][il])):
            f16 = fused[row].view(np.float16).astype(np.float32)
            p16 = perkey.view(np.float16).astype(np.float32)
            assert np.all(np.abs(f16 - p16) <= 2.0 ** -10 * np.maximum(np.abs(p16), 2.0 ** -14)), (nm, il)
            want = ref[row].view(np.float16).astype(np.float32)
            assert_close(f16, want, what=f"fused {nm} row layer {il}")
            assert_close(p16, want, what=f"per-key {nm} row layer {il}")
            assert not np.array_equal(fused[row], before[row])
            other = np.ones(fused.size, bool)
            other[row] = False
            assert np.array_equal(fused[other], before[other])
    restore(dec, snap)


def test_graph_replay_matches_eager(ctx, dec):
    snap = snapshot(dec)
    eager = []
    dec.set_position(POS)
    for _ in range(3):
        dec.step_fused()
        ctx.sync()
        eager.append((host(dec.hidden, np.float32), host(dec.logits, np.float32), int(host(dec.token, np.uint32)[0])))
    restore(dec, snap)
    dec.set_position(POS)
    g = dec.capture_fused()
    assert ctx.graph_kernel_nodes(g) == dec.launches_per_step_fused()
    try:
        for i in range(3):
            ctx.graph_launch(g)
            ctx.sync()
            # eager work between replays, as a host program would do
            _ = host(dec.pos, np.uint32)
            assert bits_equal(host(dec.hidden, np.float32), eager[i][0]), i
            assert bits_equal(host(dec.logits, np.float32), eager[i][1]), i
            assert int(host(dec.token, np.uint32)[0]) == eager[i][2]
        assert int(host(dec.pos, np.uint32)[0]) == POS + 3
    finally:
        ctx.graph_destroy(g)
        restore(dec, snap)


# Layer format mixes of the fused step (wtypes(il, name)): Q4_K q/k/v in one
# launch with the attention block over an FFN that is not one gate/up launch
# (an f16 gate; a Q6_K up), and q/k/v split over two formats.
MIXES = {
    "qkv_one_launch_f16_gate": lambda il, nm: "f16" if nm == "wgate" else ("q6k" if nm == "wdown" else "q4k"),
    "qkv_one_launch_q6k_up": lambda il, nm: "q6k" if nm in ("wup", "wdown") else "q4k",
    "q6k_v": lambda il, nm: "q6k" if nm in ("wv", "wdown") else "q4k",
}


@pytest.mark.parametrize("mix", sorted(MIXES))
def test_fused_step_layer_mixes(ctx, mix):
    """The fused step of each mix against the oracle (hidden, logits, token),
    and the kernel launches of its captured graph against
    launches_per_step_fused."""
    shape = E2BShape(n_layers=N_LAYERS, global_layers=(1,), vocab=16384)
    d = Decoder(ctx, shape, max_seq=MAX_SEQ, seed=5, wtypes=MIXES[mix])
    d.fill_kv(POS, seed=6)
    ctx.sync()
    # layer 0 (local, its own K/V) takes the one q/k/v + attention launch unless v is Q6_K
    one = (d._qkv_fused(qkv_groups(d.layers[0], [0, 0, 0], [0, 0, 0]))
           and ctx.qkv_attn_single_launch(d.attn_params[0], shape.hidden, 3))
    assert one == (mix != "q6k_v"), mix
    snap = snapshot(d)
    kcs, vcs = [k.copy() for k in snap[1]], [v.copy() for v in snap[2]]
    x_ref, logits_ref = oracle_step(d, snap[0], kcs, vcs, POS)
    d.set_position(POS)
    d.step_fused()
    ctx.sync()
    print(f"[step mix] {mix}: hidden rel-L2 {O.rel_l2(host(d.hidden, np.float32), x_ref):.2e}", flush=True)
    assert_close(host(d.hidden, np.float32), x_ref, what=f"{mix} hidden")
    lg = host(d.logits, np.float32)
    assert_close(lg, logits_ref, what=f"{mix} logits")
    check_token(d, lg, f"{mix} token")
    restore(d, snap)
    d.set_position(POS)
    g = d.capture_fused()
    try:
        assert ctx.graph_kernel_nodes(g) == d.launches_per_step_fused(), mix
        ctx.graph_launch(g)
        ctx.sync()
        assert_close(host(d.hidden, np.float32), x_ref, what=f"{mix} hidden (graph)")
    finally:
        ctx.graph_destroy(g)
    del d
