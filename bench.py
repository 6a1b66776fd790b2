#!/usr/bin/env python3
"""Benchmark of the gemma4 decode hot path on one MI355X.

Workload (one "step" = one decoded token at batch 1): 35 Gemma-4-E2B-shaped
decoder layers (hidden 1536; Q4_K q 2048x1536, k/v 256x1536, o 1536x2048,
gate/up 6144x1536; Q6_K down 1536x6144; 8 query / 1 KV head of dim 256;
layers 4,9,...,34 global, the rest with a 512-token window), then the tied
Q6_K LM head [262144 x 1536], softcap 30 and argmax. Weights are seeded
synthetic data generated on the device; the KV cache is pre-filled with
N(0,1) f16 rows up to the start position. The fused step is captured once as
a HIP graph and replayed; each replay advances the device-side position.

The ragged multi-sequence step (B sequences with context lengths ~ U(128,
8192) in a paged f16 pool of 16-token pages, every projection on the
matrix-core kernel) is timed the same way at B = 32 and swept over B = 1, 8
and 64; those figures go in `batch_decode` (aggregate tokens/s).

Prints one JSON line. `value` is decoded tokens/s; `roofline` describes the
kernel with the largest share of a step, timed with HIP events on the
library's stream; `cpu_baseline` times the CPU oracle on a bounded sample.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "gemma4-webgpu_amd"))

import numpy as np  # noqa: E402

import g4hip  # noqa: E402
from g4hip.decoder import BatchDecoder, Decoder, E2BShape  # noqa: E402

METRIC = "Q4_K GEMV GB/s (% of 8 TB/s peak); E2B decode tok/s at B=1 and B=32"
HBM_PEAK_GBPS = 8000.0
START_POS = 512


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def time_launches(ctx, fn, iters):
    """Average ms per call of fn() (enqueue-only work) over `iters` calls."""
    fn()
    ctx.sync()
    a = ctx.record()
    for i in range(iters):
        fn(i)
    b = ctx.record()
    ms = ctx.elapsed_ms(a, b)
    ctx.destroy_event(a)
    ctx.destroy_event(b)
    return ms / iters


def kernel_census(ctx, dec: Decoder, reps: int):
    """Average duration of each kernel of the fused step. Each kind is
    captured as a graph of its launches over all 35 layers (so weights rotate
    through HBM as in a real step, and no host launch overhead is timed),
    replayed `reps` times between HIP events on the library's stream.
    Algorithmic bytes: weights + activations read/written by one launch.

    The step's four launches per layer:
    - `qkv_attn`: the q/k/v matvec with its norm prologue and the attention
      block (RoPE cos/sin from the per-theta table, the new K/V row stored,
      the chunks merged in the launch), with the step's L2 warming (its
      reads are the next launches' weights, charged to those launches);
    - `o_matvec`;
    - `gateup_gelu`: post-attention norm-add, pre-FFN norm, gate/up, GELU
      product and its digit block;
    - `down_matvec_q6k` over those digits.
    The kinds of the per-head o split (Decoder.heads_o) are timed as well:
    `qkv_attn_partials` (the same launch without its merge; it leaves the
    staged q/k/v for `attn_heads` to clear, so it is timed in a graph of
    pairs, less the `attn_heads` graph's time), `attn_heads` (per-head
    merge + o by groups of heads) and `gateup_gelu_shares`. Kinds the step
    does not issue, and those of the two-launch form the step takes for
    other shapes (`qkv_normadd_matvec`, `attn_fused`), have per_step 0. The
    matvecs run with cold weights."""
    s, c = dec.s, ctx
    dec.set_position(START_POS)
    Ls = dec.layers
    nl = len(Ls)
    H, Q, KV, I, V = s.hidden, s.q_dim, s.kv_dim, s.ffn, s.vocab
    q4 = lambda M, N: M * N // 256 * 144  # noqa: E731
    q6 = lambda M, N: M * N // 256 * 210  # noqa: E731
    n_glob = sum(1 for il in range(nl) if s.is_global(il))
    L_loc, L_glob = min(START_POS + 1, s.window), START_POS + 1
    kv_avg = ((nl - n_glob) * L_loc + n_glob * L_glob) * KV * 2 * 2 // nl  # f16 K + V rows read
    ch_avg = ((nl - n_glob) * -(-L_loc // 64) + n_glob * -(-L_glob // 64)) / nl  # live 64-position chunks
    parts = int(ch_avg * s.n_q_heads * (s.head_dim + 2) * 4)  # chunk partials (m, l, o) written / read
    dig = ctx.digits_bytes(I)  # the GELU product as the down launch's digit block
    shares = g4hip.O_SHARES * H * 4

    qkv_bytes = q4(Q + 2 * KV, H) + 5 * H * 4 + (Q + 2 * KV) * 4
    qkv_args = lambda il, L: (  # noqa: E731
        dec.down, L.post_ffn_norm, dec.hidden2, None, L.attn_norm, dec.hidden, [L.wq, L.wk, L.wv],
        [dec.q, dec.k, dec.v], H, s.eps, L.q_norm, L.k_norm, dec.rope_freqs, L.k_cache, L.v_cache)
    rope = lambda il: (dec.rope_cs[s.is_global(il)], dec.rope_rows)  # noqa: E731
    heads = lambda il, L: c.attnHeadsMatmul_q4k(dec.attn_ws, dec.attn_params[il], dec.pos, L.wo, dec.o_parts, H)  # noqa

    def pair(il, L):
        c.qkvAttnDecodePartials(*qkv_args(il, L), dec.attn_params[il], dec.attn_ws, dec.pos, dec.warm[il], *rope(il))
        heads(il, L)

    hs = nl if dec.heads_o else 0  # launches per step of the per-head o split's kinds
    ms = nl - hs                     # of the in-launch merge's
    kinds = {
        # name: (per-layer body, launches per body, launches per step of this kind, algorithmic bytes per launch)
        "qkv_attn": (
            lambda il, L: c.qkvAttnDecodeFusedWarm(*qkv_args(il, L), dec.attn, dec.attn_params[il], dec.attn_ws,
                                                   dec.pos, dec.warm[il], *rope(il)),
            1, ms, qkv_bytes + kv_avg + 2 * KV * 2 + Q * 4),
        "o_matvec": (
            lambda il, L: c.matmulQuant(dec.attn, L.wo, dec.o, H, Q),
            1, ms, q4(H, Q) + Q * 4 + H * 4),
        "gateup_gelu": (
            lambda il, L: c.normAddGateUpGeluDigits_q4k(dec.o, L.post_attn_norm, dec.hidden, L.pre_ffn_norm,
                                                        L.wgate, L.wup, dec.hidden2, dec.act, dec.act_digits, I, H,
                                                        s.eps),
            1, ms, 2 * q4(I, H) + 4 * H * 4 + I * 4 + dig),
        "down_matvec_q6k": (
            lambda il, L: c.matmulQuantDigits_q6k(dec.act_digits, L.wdown, dec.down, H, I),
            1, nl, q6(H, I) + dig + H * 4),
        "qkv_attn_partials+attn_heads": (pair, 2, 0, 0),
        "attn_heads": (heads, 1, hs, parts + q4(H, Q) + shares),
        "gateup_gelu_shares": (
            lambda il, L: c.normAddPartsGateUpGeluDigits_q4k(dec.o_parts, L.post_attn_norm, dec.hidden,
                                                             L.pre_ffn_norm, L.wgate, L.wup, dec.hidden2, dec.act,
                                                             dec.act_digits, I, H, s.eps),
            1, hs, 2 * q4(I, H) + 3 * H * 4 + shares + I * 4 + dig),
        "qkv_normadd_matvec": (
            lambda il, L: c.normAddMatmulSegments(
                "q4k", dec.down, L.post_ffn_norm, dec.hidden2, L.attn_norm, dec.hidden, [L.wq, L.wk, L.wv],
                [dec.q, dec.k, dec.v], [Q, KV, KV], H, s.eps),
            1, 0, qkv_bytes),
        "attn_fused": (
            lambda il, L: c.attnDecodeFusedWarm(dec.q, dec.k, dec.v, L.q_norm, L.k_norm, dec.rope_freqs, L.k_cache,
                                                L.v_cache, dec.attn, dec.attn_params[il], dec.attn_ws, dec.pos, [],
                                                *rope(il)),
            1, 0, kv_avg + (Q + 2 * KV) * 4 + 2 * KV * 2 + Q * 4),
    }
    out = {}
    for name, (body, per_body, per_step, nbytes) in kinds.items():
        ctx.graph_begin()
        try:
            for il, L in enumerate(Ls):
                body(il, L)
        finally:
            g = ctx.graph_end()
        us = time_launches(ctx, lambda _i=0: ctx.graph_launch(g), reps) * 1e3 / nl
        ctx.graph_destroy(g)
        out[name] = {"us": us, "per_step": per_step, "bytes": nbytes,
                     "gbps": nbytes / (us * 1e-6) / 1e9 if nbytes else None}
    # the partials launch: its pairs' time less the heads launch's
    us = out["qkv_attn_partials+attn_heads"]["us"] - out["attn_heads"]["us"]
    nbytes = qkv_bytes + kv_avg + 2 * KV * 2 + parts
    out["qkv_attn_partials"] = {"us": us, "per_step": hs, "bytes": nbytes, "gbps": nbytes / (us * 1e-6) / 1e9,
                                "timed_as": "qkv_attn_partials+attn_heads less attn_heads"}
    # LM head with the final norm-add, softcap and the argmax candidates,
    # then their reduction, as the step runs them (330 MB: larger than the
    # 256 MB last-level cache, so no rotation is needed)
    last = Ls[-1]
    ctx.graph_begin()
    try:
        c.normAddMatmulArgmax("q6k", dec.down, last.post_ffn_norm, dec.hidden2, dec.final_norm, dec.hidden,
                              dec.lm_head, dec.logits, V, H, dec.token, s.eps, softcap=s.softcap)
    finally:
        g = ctx.graph_end()
    us = time_launches(ctx, lambda _i=0: ctx.graph_launch(g), max(5, reps)) * 1e3
    ctx.graph_destroy(g)
    nbytes = s.lm_head_bytes() + 5 * H * 4 + V * 4
    out["lm_head_q6k_softcap_argmax"] = {"us": us, "per_step": 1, "launches": 2, "bytes": nbytes,
                                         "gbps": nbytes / (us * 1e-6) / 1e9}
    return out


def measured_traffic(kind):
    """HBM bytes per launch of a census kind, from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary (scaled by the copy calibration), or None
    when that summary does not cover the kind."""
    path = os.path.join(ROOT, "profiles", "decode_b1_e2b_hbm_traffic.json")
    try:
        with open(path) as f:
            entry = json.load(f)["entries"].get(kind)
    except (OSError, ValueError, KeyError):
        return None
    return None if entry is None else (entry["bytes_per_launch"], entry.get("warming_bytes", 0))


def gemv_cfg0(ctx, copies=101, rounds=5):
    """Config-0 GEMV: W [6144 x 1536] Q4_K, x f32[1536], y f32[6144]; weights
    rotated over `copies` buffers (> 2x the 256 MB last-level cache)."""
    M, N = 6144, 1536
    nb = M * N // 256
    wb = nb * 144
    W = ctx.alloc(wb * copies)
    ctx.fill_q4k(W, nb * copies, 12345)
    x = ctx.empty(N, np.float32)
    ctx.fill_normal_f32(x, N, 1, 0.0, 1.0)
    y = ctx.empty(M, np.float32)
    ptrs = [W.ptr + i * wb for i in range(copies)]

    def one(i=0):
        ctx.matmulQuant(x, ptrs[i % copies], y, M, N, "q4k")
    ms = time_launches(ctx, one, copies * rounds)
    alg = wb + N * 4 + M * 4
    W.free()
    return {"shape": [M, N], "us": ms * 1e3, "bytes": alg, "gbps": alg / (ms * 1e-3) / 1e9,
            "frac": alg / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, "copies": copies}


def gemv_q4k_amortised(ctx, M=262144, N=1536, copies=2, rounds=10):
    """The config-0 kernel family at a size that amortises the launch: the
    one-vector Q4_K matvec (mv_kernel, 12-wave workgroups walking tiles
    through the LDS ring, one workgroup per CU) over W [M x N], 226 MB per
    copy, rotated over `copies` (> the 256 MB last-level cache)."""
    nb = M * N // 256
    wb = nb * 144
    W = ctx.alloc(wb * copies)
    ctx.fill_q4k(W, nb * copies, 4321)
    x = ctx.empty(N, np.float32)
    ctx.fill_normal_f32(x, N, 2, 0.0, 1.0)
    y = ctx.empty(M, np.float32)
    ptrs = [W.ptr + i * wb for i in range(copies)]

    def one(i=0):
        ctx.matmulQuant(x, ptrs[i % copies], y, M, N, "q4k")
    ms = time_launches(ctx, one, copies * rounds)
    alg = wb + N * 4 + M * 4
    W.free()
    # the pure-streaming rate of the same bytes (the probe read of the same
    # rotation), so that the matvec's rate reads against what a launch of
    # this size can stream at all
    fl = stream_floor(ctx, nbytes=wb, copies=copies, rounds=rounds, wg_list=(1024, 2048, 4096))
    return {"shape": [M, N], "us": ms * 1e3, "bytes": alg, "gbps": alg / (ms * 1e-3) / 1e9,
            "frac": alg / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, "copies": copies,
            "stream_floor": {k: fl[k] for k in ("launches", "best_us", "best_gbps", "best_frac")}}


def stream_floor(ctx, nbytes=5339136, copies=101, rounds=5, wg_list=(256, 648, 1024, 2048)):
    """The pure-streaming floor of one launch that reads `nbytes` (config 0's
    5.34 MB by default) from HBM: g4_streamRead over `copies` rotated buffers
    (> 2x the 256 MB last-level cache), timed like the config-0 GEMV."""
    nb = (nbytes + 255) // 256 * 256
    buf = ctx.alloc(nb * copies)  # contents are irrelevant to a read-only stream
    sink = ctx.empty(65535, np.uint32)
    ptrs = [buf.ptr + i * nb for i in range(copies)]
    out = {}
    for pol, name in ((1, "nontemporal"), (0, "plain")):
        for nw in wg_list:
            def one(i=0, pol=pol, nw=nw):
                ctx.streamRead(ptrs[i % copies], nb, pol, nw, sink)
            ms = time_launches(ctx, one, copies * rounds)
            out[f"{name}_wg{nw}"] = {"us": round(ms * 1e3, 3), "gbps": round(nb / (ms * 1e-3) / 1e9, 1)}
    buf.free()
    best = min(out.values(), key=lambda v: v["us"])
    return {"bytes": nb, "copies": copies, "launches": out, "best_us": best["us"], "best_gbps": best["gbps"],
            "best_frac": round(best["gbps"] / HBM_PEAK_GBPS, 4)}


def calibration_reads(ctx, nbytes=256 << 20):
    """One 256 MiB read per cache policy (the streaming probe), for the HBM
    byte counters' calibration under the profiler."""
    buf = ctx.zeros(nbytes, np.uint8)
    sink = ctx.empty(4096, np.uint32)
    for pol in (0, 1, 2):
        ctx.streamRead(buf, nbytes, pol, 4096, sink)
    ctx.sync()
    buf.free()
    return {"bytes": nbytes, "policies": ["plain", "nontemporal", "device_scope"], "workgroups": 4096}


def graph_us(ctx, body, reps):
    """Average us of one replay of a graph holding body()'s launches."""
    ctx.graph_begin()
    try:
        body()
    finally:
        g = ctx.graph_end()
    ms = time_launches(ctx, lambda _i=0: ctx.graph_launch(g), reps)
    ctx.graph_destroy(g)
    return ms * 1e3


def attention_cfg3(ctx, reps=3):
    """Decode attention: 8 query heads, 1 KV head, head_dim 256 (and the
    fused block at head_dim 512, `hd512_*`), f16 K/V ~
    N(0,1), one sequence, contexts 512 / 4096 / 32768, globally (no window)
    and with the 512-position window; `us` is attention alone (normed q in),
    `fused_block_us` the whole block (q/k norm + RoPE, v_norm, KV store,
    attention) in its one launch. Every launch of a replay reads a different
    window of a 302 MB K/V region (more than the 256 MB last-level cache).
    Algorithmic bytes: L_eff * 1024 (f16 K and V rows) + q + output."""
    nqh, nkh, hd, P = 8, 1, 256, 288 * 1024
    k = ctx.empty(P * hd, np.uint16)
    v = ctx.empty(P * hd, np.uint16)
    ctx.fill_normal_f16(k, P * hd, 31, 0.0, 1.0)
    ctx.fill_normal_f16(v, P * hd, 32, 0.0, 1.0)
    q = ctx.empty(nqh * hd, np.float32)
    ctx.fill_normal_f32(q, nqh * hd, 33, 0.0, 1.0)
    out = ctx.empty(nqh * hd, np.float32)
    # the whole block: raw q/k/v, norm weights ~ N(1, 0.1), proportional RoPE table
    k_raw = ctx.empty(nkh * hd, np.float32)
    v_raw = ctx.empty(nkh * hd, np.float32)
    ctx.fill_normal_f32(k_raw, nkh * hd, 34, 0.0, 1.0)
    ctx.fill_normal_f32(v_raw, nkh * hd, 35, 0.0, 1.0)
    q_w = ctx.empty(hd, np.uint16)
    k_w = ctx.empty(hd, np.uint16)
    ctx.fill_normal_f16(q_w, hd, 36, 1.0, 0.1)
    ctx.fill_normal_f16(k_w, hd, 37, 1.0, 0.1)
    table = ctx.from_numpy(np.where(np.arange(hd // 2) < hd // 8, 1.0, np.inf).astype(np.float16).view(np.uint16))
    res = {}
    for L in (512, 4096, 32768):
        for window in (0, 512):
            if window and L <= window:
                continue
            ws = ctx.zeros(ctx.attn_workspace_bytes(nqh, nkh, hd, L, window), np.uint8)
            n_rot = P // L

            def body():
                for r in range(n_rot):
                    off = r * L * hd * 2
                    ctx.attnDecode(q, k.offset(off), v.offset(off), out, nqh, nkh, hd, L, 1.0, window, workspace=ws)
            us = graph_us(ctx, body, reps) / n_rot
            # fused block: q_norm + RoPE, k_norm + RoPE, v_norm, KV store at
            # position L - 1, attention (theta 1e6 global, 1e4 local)
            glob = window == 0
            fp = ctx.attn_fused_params(nqh, nkh, hd, L, window, 1e-6, 1e6 if glob else 1e4, int(glob))
            fws = ctx.zeros(ctx.attn_fused_workspace_bytes(fp), np.uint8)
            pdev = ctx.from_numpy(np.array([L - 1], np.uint32))

            def fused():
                for r in range(n_rot):
                    off = r * L * hd * 2
                    ctx.attnDecodeFused(q, k_raw, v_raw, q_w, k_w, table, k.offset(off), v.offset(off), out, fp, fws,
                                        pdev)
            us_f = graph_us(ctx, fused, reps) / n_rot
            l_eff = min(L, window) if window else L
            nbytes = l_eff * 1024 + 2 * nqh * hd * 4
            res[f"ctx{L}_{'window512' if window else 'global'}"] = {
                "us": round(us, 2), "bytes": nbytes, "gbps": round(nbytes / (us * 1e-6) / 1e9, 1),
                "frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4),
                "fused_block_us": round(us_f, 2), "fused_block_gbps": round(nbytes / (us_f * 1e-6) / 1e9, 1)}
            fws.free()
            ws.free()
    for b in (k, v, k_raw, v_raw, q_w, k_w, table):
        b.free()
    # the fused block at head dim 512 (Gemma-4-E2B's global layers: no
    # window, theta 1e6 with the divisor table), K/V rotated over 604 MB
    hd = 512
    k = ctx.empty(P * hd, np.uint16)
    v = ctx.empty(P * hd, np.uint16)
    ctx.fill_normal_f16(k, P * hd, 41, 0.0, 1.0)
    ctx.fill_normal_f16(v, P * hd, 42, 0.0, 1.0)
    q = ctx.empty(nqh * hd, np.float32)
    ctx.fill_normal_f32(q, nqh * hd, 43, 0.0, 1.0)
    out = ctx.empty(nqh * hd, np.float32)
    k_raw = ctx.empty(hd, np.float32)
    v_raw = ctx.empty(hd, np.float32)
    ctx.fill_normal_f32(k_raw, hd, 44, 0.0, 1.0)
    ctx.fill_normal_f32(v_raw, hd, 45, 0.0, 1.0)
    q_w = ctx.empty(hd, np.uint16)
    k_w = ctx.empty(hd, np.uint16)
    ctx.fill_normal_f16(q_w, hd, 46, 1.0, 0.1)
    ctx.fill_normal_f16(k_w, hd, 47, 1.0, 0.1)
    table = ctx.from_numpy(np.where(np.arange(hd // 2) < hd // 8, 1.0, np.inf).astype(np.float16).view(np.uint16))
    for L in (513, 4096):
        fp = ctx.attn_fused_params(nqh, nkh, hd, L, 0, 1e-6, 1e6, 1)
        fws = ctx.zeros(ctx.attn_fused_workspace_bytes(fp), np.uint8)
        pdev = ctx.from_numpy(np.array([L - 1], np.uint32))
        n_rot = P // L

        def fused512():
            for r in range(n_rot):
                off = r * L * hd * 2
                ctx.attnDecodeFused(q, k_raw, v_raw, q_w, k_w, table, k.offset(off), v.offset(off), out, fp, fws,
                                    pdev)
        us_f = graph_us(ctx, fused512, reps) / n_rot
        nbytes = L * 2048 + 2 * nqh * hd * 4
        res[f"hd512_ctx{L}_global"] = {"fused_block_us": round(us_f, 2), "bytes": nbytes,
                                       "fused_block_gbps": round(nbytes / (us_f * 1e-6) / 1e9, 1)}
        fws.free()
    for b in (k, v, q, out, k_raw, v_raw, q_w, k_w, table):
        b.free()
    return res


def lm_head_sampling(ctx, reps=10):
    """Tied Q6_K LM head [262144 x 1536] + softcap 30 + argmax and top-k 256,
    at M = 1 and M = 8 hidden vectors ~ N(0,1) (the 330 MB matrix exceeds the
    last-level cache, so replays stream it from HBM)."""
    V, H = 262144, 1536
    nb = V * H // 256
    W = ctx.alloc(nb * 210)
    ctx.fill_q6k(W, nb, 41)
    res = {}
    for M in (1, 8):
        x = ctx.empty(M * H, np.float32)
        ctx.fill_normal_f32(x, M * H, 42, 0.0, 1.0)
        lg = ctx.empty(M * V, np.float32)
        tok = ctx.empty(M, np.uint32)
        tk = ctx.empty(M * 512, np.float32)

        def head():
            if M == 1:
                ctx.matmulQuant(x, W, lg, V, H, "q6k")
                ctx.logitSoftcap(lg, V, 30.0)
            else:
                ctx.normAddMatmulSegmentsBatch("q6k", x, None, None, None, None, [W], [lg], [V], H, M,
                                               softcap=30.0)
        us_head = graph_us(ctx, head, reps)
        us_arg = graph_us(ctx, lambda: ctx.argmaxBatch(lg, tok, V, M), reps)
        us_topk = graph_us(ctx, lambda: ctx.topk256Batch(lg, tk, V, M), reps)
        nbytes = nb * 210 + M * H * 4 + M * V * 4
        res[f"M={M}"] = {"head_softcap_us": round(us_head, 2), "argmax_us": round(us_arg, 2),
                         "topk256_us": round(us_topk, 2), "head_bytes": nbytes,
                         "head_gbps": round(nbytes / (us_head * 1e-6) / 1e9, 1)}
        if M == 1:
            # the whole sampling step as the decode step runs it: final norm + LM
            # head + softcap with the argmax / top-k candidates as the matvec's
            # epilogue, then their reduction (two launches each)
            w = ctx.empty(H, np.uint16)
            ctx.fill_normal_f16(w, H, 43, 1.0, 0.1)
            res["M=1"]["fused_argmax_us"] = round(graph_us(
                ctx, lambda: ctx.normAddMatmulArgmax("q6k", x, w, None, None, None, W, lg, V, H, tok,
                                                     softcap=30.0), reps), 2)
            res["M=1"]["fused_topk256_us"] = round(graph_us(
                ctx, lambda: ctx.normAddMatmulTopk("q6k", x, w, None, None, None, W, lg, V, H, tk,
                                                   softcap=30.0), reps), 2)
            w.free()
    W.free()
    return res


def batch_census(ctx, bd, reps=10):
    """Average us per launch kind of the ragged step, each kind captured over
    all 35 layers (weights rotate through HBM as in the step). Algorithmic
    bytes per launch: the weights once, the activations read (f32 or their
    operand blocks) and the outputs written; the attention kinds read every
    sequence's K/V window of one layer."""
    c, s, B = ctx, bd.s, bd.B
    H, Q, KV, I = s.hidden, s.q_dim, s.kv_dim, s.ffn
    Ls = bd.layers
    q4 = lambda M, N: M * N // 256 * 144  # noqa: E731
    q6 = lambda M, N: M * N // 256 * 210  # noqa: E731
    n_glob = sum(1 for il in range(s.n_layers) if s.is_global(il))
    kv_glob = sum(int(L) + 1 for L in bd.lens_host) * KV * 4
    kv_loc = sum(min(int(L) + 1, s.window) for L in bd.lens_host) * KV * 4
    act = lambda N: ctx.batch_operand_bytes(N, B)  # noqa: E731
    sub = lambda K: ctx.batch_sub_operand_bytes(K, B)  # noqa: E731
    # the gate/up launch hands its product to the down projection as
    # sub-block-scaled operand blocks (every layer of this shape)
    handoff = bd.dops is not None
    ks_down = (I // 768) if handoff else bd.ks_f
    nbytes = {
        "qkv": q4(Q + 2 * KV, H) + act(H) + bd.ks_h * B * (Q + 2 * KV) * 4,
        "attn_global": kv_glob + B * Q * 4 * 2,
        # (the one-launch block also reads the q/k/v partials and writes the K/V row)
        "attn_window512": kv_loc + B * Q * 4 * 2 + (bd.ks_h * B * (Q + 2 * KV) * 4 + B * KV * 4
                                                    if bd.block_attn else 0),
        "o": q4(H, Q) + act(Q) + bd.ks_q * B * H * 4,
        "gate_up_gelu": 2 * q4(I, H) + act(H) + (sub(I) if handoff else B * I * 4),
        "down": q6(H, I) + (sub(I) if handoff else B * I * 4) + ks_down * B * H * 4,
    }
    kinds = {
        "prep_attn": lambda il, L: c.batchPrep(bd.down_parts, bd.ks_f // 2, L.post_ffn_norm, bd.hidden2, L.attn_norm,
                                               bd.hidden, bd.xn, H, B, s.eps, ops=bd.xops),
        "qkv": lambda il, L: c.matmulSegmentsBatchPartial("q4k", bd.xn, [L.wq, L.wk, L.wv],
                                                          [bd.q_parts, bd.k_parts, bd.v_parts], [Q, KV, KV], H, B,
                                                          bd.ks_h, ops=bd.xops),
        # the prologue as a launch of its own: every layer, or (with the
        # one-launch block) the global layers, whose windows the block's
        # in-launch merge does not cover
        "attn_prologue": lambda il, L: (c.pagedAttnPrologue(bd.q_parts, bd.k_parts, bd.v_parts, bd.ks_h, L.q_norm,
                                                            L.k_norm, bd.rope_freqs, bd.q, L.k_cache, L.v_cache,
                                                            bd.page_table, bd.seq_lens, bd.pro_params[il],
                                                            bd.rope_cs[bd.s.is_global(il)], bd.rope_rows)
                                        if s.is_global(il) or not bd.block_attn else "skip"),
        "attn_global": lambda il, L: (c.pagedAttnDecode(bd.q, L.k_cache, L.v_cache, bd.page_table, bd.seq_lens,
                                                        bd.attn, bd.attn_params[il], bd.attn_ws, ops=bd.aops)
                                      if s.is_global(il) else "skip"),
        # the window-512 layers: prologue, attention and merge in one launch
        # (g4_pagedAttnBlock), or the paged decode alone
        "attn_window512": lambda il, L: (("skip" if s.is_global(il) else
                                          c.pagedAttnBlock(bd.q_parts, bd.k_parts, bd.v_parts, bd.ks_h, L.q_norm,
                                                           L.k_norm, bd.rope_freqs, None, L.k_cache, L.v_cache,
                                                           bd.page_table, bd.seq_lens, bd.attn, bd.pro_params[il],
                                                           bd.block_ws, ops=bd.aops,
                                                           rope_cs=bd.rope_cs[False], rope_rows=bd.rope_rows))
                                         if bd.block_attn else
                                         (c.pagedAttnDecode(bd.q, L.k_cache, L.v_cache, bd.page_table, bd.seq_lens,
                                                            bd.attn, bd.attn_params[il], bd.attn_ws, ops=bd.aops)
                                          if not s.is_global(il) else "skip")),
        "o": lambda il, L: c.matmulSegmentsBatchPartial("q4k", bd.attn, [L.wo], [bd.o_parts], [H], Q, B, bd.ks_q,
                                                        ops=bd.aops),
        "prep_ffn": lambda il, L: c.batchPrep(bd.o_parts, bd.ks_q, L.post_attn_norm, bd.hidden, L.pre_ffn_norm,
                                              bd.hidden2, bd.xn, H, B, s.eps, ops=bd.xops),
        "gate_up_gelu": lambda il, L: (c.gateUpGeluBatchOps(bd.xn, bd.xops, L.wgate, L.wup, None, bd.dops, I, H, B)
                                       if handoff else c.gateUpGeluBatch(bd.xn, L.wgate, L.wup, bd.act, I, H, B,
                                                                         ops=bd.xops)),
        "down": lambda il, L: (c.matmulSubBatchPartial(bd.dops, L.wdown, bd.down_parts, H, I, B, ks_down)
                               if handoff else c.matmulSegmentsBatchPartial("q6k", bd.act, [L.wdown],
                                                                            [bd.down_parts], [H], I, B, bd.ks_f)),
    }
    out = {}
    for name, body in kinds.items():
        n = [0]

        def run(body=body):
            for il, L in enumerate(Ls):
                if body(il, L) != "skip":
                    n[0] += 1
        us = graph_us(ctx, run, reps)
        out[name] = {"us_per_launch": round(us / n[0], 2), "per_step_us": round(us, 1), "launches": n[0]}
        if name in nbytes:
            gbps = nbytes[name] / (us / n[0] * 1e-6) / 1e9
            out[name].update({"bytes": nbytes[name], "gbps": round(gbps, 1), "frac": round(gbps / HBM_PEAK_GBPS, 4)})
    us = graph_us(ctx, lambda: c.matmulSegmentsBatchPartial("q6k", bd.xn, [bd.lm_head], [bd.logits], [s.vocab], H,
                                                            B, 1, ops=bd.xops, softcap=s.softcap), max(3, reps // 2))
    nb = s.lm_head_bytes() + act(H) + B * s.vocab * 4
    out["lm_head_softcap"] = {"us_per_launch": round(us, 2), "per_step_us": round(us, 1), "launches": 1, "bytes": nb,
                              "gbps": round(nb / (us * 1e-6) / 1e9, 1),
                              "frac": round(nb / (us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4)}
    return out


def batch_decode(ctx, B, steps, warmup, seed=0, census=False):
    """Aggregate tok/s of the ragged B-sequence step replayed as a HIP graph.
    Context lengths ~ U(128, 8192) (seeded); each replay appends one token
    to every sequence. HBM bytes per step: all weights once, plus every
    sequence's K/V window in every layer."""
    lens = np.random.default_rng(1000 + B).integers(128, 8193, B)
    t0 = time.time()
    bd = BatchDecoder(ctx, lens, E2BShape(), reserve=warmup + steps + 8, seed=seed)
    bd.fill_kv(seed=1)
    ctx.sync()
    s = bd.s
    kv_bytes = bd.kv_bytes_per_step()
    w_bytes = s.layer_weight_bytes() * s.n_layers + s.lm_head_bytes()
    log(f"B={B}: decoder ready in {time.time() - t0:.1f}s, {bd.num_pages} pages, mean context {lens.mean():.0f}")
    g = bd.capture("argmax")
    for _ in range(warmup):
        ctx.graph_launch(g)
    ctx.sync()
    a = ctx.record()
    for _ in range(steps):
        ctx.graph_launch(g)
    b = ctx.record()
    ms = ctx.elapsed_ms(a, b) / steps
    ctx.sync()
    final = bd.seq_lens.download(np.uint32)
    ok = bool(np.array_equal(final, lens + warmup + steps))
    ctx.graph_destroy(g)
    cens = batch_census(ctx, bd) if census else None
    del bd
    res = {"B": B, "tok_s": round(B * 1000.0 / ms, 1), "ms_per_step": round(ms, 4),
           "mean_context": round(float(lens.mean()), 1), "min_context": int(lens.min()),
           "max_context": int(lens.max()), "kv_bytes_per_step": kv_bytes, "weight_bytes_per_step": w_bytes,
           "hbm_gbps_alg": round((kv_bytes + w_bytes) / (ms * 1e-3) / 1e9, 1), "lengths_advanced": ok}
    if cens is not None:
        res["census_us"] = cens
    log(f"B={B}: {res}")
    return res


def decode_rate(ctx, shape, start, steps, warmup, embed=False, warm=True):
    """Single-sequence tok/s of the fused step replayed as a HIP graph from
    position `start` (KV pre-filled up to it). Returns the figures and the
    decoder's launches per token."""
    max_seq = (start + warmup + steps + 64 + 255) // 256 * 256
    t0 = time.time()
    d = Decoder(ctx, shape, max_seq=max_seq, seed=0, embed=embed)
    d.fill_kv(start, seed=1)
    d.set_position(start)
    ctx.sync()
    g = d.capture_fused("argmax", warm=warm)
    for _ in range(warmup):
        ctx.graph_launch(g)
    ctx.sync()
    a = ctx.record()
    for _ in range(steps):
        ctx.graph_launch(g)
    b = ctx.record()
    ms = ctx.elapsed_ms(a, b) / steps
    ctx.sync()
    end = int(d.pos.download(np.uint32)[0])
    ctx.graph_destroy(g)
    s = d.s
    wbytes = s.weight_bytes() + s.lm_head_bytes() + s.ple_bytes()
    res = {"tok_s": round(1000.0 / ms, 1), "us_per_token": round(ms * 1e3, 2), "positions": [start, end],
           "weight_bytes_per_token": wbytes, "launches_per_token": d.launches_per_step_fused(),
           "setup_s": round(time.time() - t0, 1)}
    del d
    return res


def prefill_rate(ctx, shape, T=512, B=64, reps=3):
    """Batched prefill of one T-token prompt from position 0 (B tokens per
    matrix-core step, T / B steps): prompt tokens/s."""
    d = BatchDecoder(ctx, [0] * B, shape, reserve=T + 8, seed=0, shared_pages=True, embed=True)
    ctx.sync()
    toks = np.random.default_rng(5).integers(0, shape.vocab, T)
    d.prefill(toks[:B], 0)  # warm-up
    times = []
    for _ in range(reps):
        a = ctx.record()
        d.prefill(toks, 0)
        b = ctx.record()
        times.append(ctx.elapsed_ms(a, b))
    ms = min(times)
    res = {"tokens": T, "chunk": B, "ms": round(ms, 3), "tok_s": round(T / ms * 1e3, 1),
           "ms_per_chunk": round(ms / (T // B), 3)}
    del d
    return res


def _cpu_threads():
    """Host threads this process may use (the box's CPU share, at most 16)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def node_q4k_gemv(seconds=4.0):
    """Config 0 on the host as a TypeScript host would run it: the builder's
    ES2019 restatement of GGUFParser.dequantizeQ4_K + the f32 dot of
    matmul_quant (oracle/q4k_dot.js) under Node, one core, with the dequant
    inside the timed loop and with the matrix pre-dequantized. Its output is
    checked against the C oracle. None when node is absent."""
    import shutil
    import subprocess
    import tempfile
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    node = shutil.which("node")
    if node is None:
        return None
    M, K = 6144, 1536
    W = O.gen_q4k(12345, M * K // 256)
    x = O.gen_normal_f32(1, K)
    with tempfile.TemporaryDirectory() as td:
        fin, fout = os.path.join(td, "in.bin"), os.path.join(td, "out.bin")
        with open(fin, "wb") as f:
            f.write(np.array([M, K], np.uint32).tobytes())
            f.write(W.tobytes())
            f.write(x.tobytes())
        r = subprocess.run([node, os.path.join(ROOT, "oracle", "q4k_dot.js"), fin, fout, str(seconds)],
                           capture_output=True, text=True, check=True, timeout=20 * seconds + 60)
        res = json.loads(r.stdout.strip().splitlines()[-1])
        y = np.fromfile(fout, np.float32)
    alg = M * K // 256 * 144 + K * 4 + M * 4
    return {"shape": [M, K], "node": res["node"], "cores": 1,
            "ms_dequant_in_loop": round(res["ms_dequant_dot"], 3),
            "gbps_dequant_in_loop": round(alg / (res["ms_dequant_dot"] * 1e-3) / 1e9, 4),
            "ms_predequantized_f32": round(res["ms_dot_predequantized"], 3),
            "gemvs_timed": res["reps_dequant"] + res["reps_dot"],
            "rel_l2_vs_oracle": float(O.rel_l2(y, O.matmul(x, W, M, K, "q4k")))}


def node_step_rate(start=START_POS, steps=100, warmup=10):
    """The fused step from a Node host: gemma4-webgpu_amd/node/bench_step.js
    builds the model of `value` (same shape, weights generated on the device,
    KV filled to `start`) through HipBackend over the N-API addon, captures
    HipBackend.encodeFusedStep once and replays it. None when node or the
    addon is absent."""
    import shutil
    import subprocess
    node = shutil.which("node")
    if node is None or not os.path.exists(os.path.join(ROOT, "gemma4-webgpu_amd", "node", "g4hip.node")):
        return None
    r = subprocess.run([node, os.path.join(ROOT, "gemma4-webgpu_amd", "node", "bench_step.js"), str(start),
                        str(steps), str(warmup)], capture_output=True, text=True, check=True, timeout=600)
    return json.loads(r.stdout.strip().splitlines()[-1])


def torch_attention_cfg3(threads, seconds=0.5):
    """Config 3 on the host: the builder's fp32 torch attention,
    softmax(q k^T) v at scale 1.0 with the sliding-window mask, 8 query heads
    over 1 KV head of dim 256, K/V held in f32 (the reference's cache type)."""
    import torch

    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(3)
    res = {}
    try:
        for L in (512, 4096, 32768):
            K = torch.randn(L, 256, generator=g)
            V = torch.randn(L, 256, generator=g)
            q = torch.randn(8, 256, generator=g)
            for window in (0, 512):
                if window and L <= window:
                    continue
                lo = L - window if window else 0

                def attn():
                    s = q @ K[lo:].T
                    return torch.softmax(s, dim=-1) @ V[lo:]
                attn()
                n, t0 = 0, time.perf_counter()
                while time.perf_counter() - t0 < seconds:
                    attn()
                    n += 1
                us = (time.perf_counter() - t0) / n * 1e6
                l_eff = L - lo
                res[f"ctx{L}_{'window512' if window else 'global'}"] = {
                    "us": round(us, 1), "gbps_f16_equiv": round(l_eff * 1024 / (us * 1e-6) / 1e9, 3)}
    finally:
        torch.set_num_threads(prev)
    return res


def oracle_step_rate(tokens=1):
    """The C oracle (plain C, 1 thread, f64 accumulation) on whole decode
    steps of the benchmark workload: 35 E2B-shaped layers at context
    START_POS + 1 plus the 262144-row Q6_K LM head, softcap and argmax."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    s = E2BShape()
    H, Q, KV, I = s.hidden, s.q_dim, s.kv_dim, s.ffn
    Wq, Wk, Wv = O.gen_q4k(1, Q * H // 256), O.gen_q4k(2, KV * H // 256), O.gen_q4k(3, KV * H // 256)
    Wo, Wg, Wu = O.gen_q4k(4, H * Q // 256), O.gen_q4k(5, I * H // 256), O.gen_q4k(6, I * H // 256)
    Wd = O.gen_q6k(7, H * I // 256)
    Wh = O.gen_q6k(13, s.vocab * H // 256)
    nw = O.gen_normal_f16(8, H, 1.0, 0.1)
    hw = O.gen_normal_f16(9, s.head_dim, 1.0, 0.1)
    L = START_POS + 1
    kc = O.gen_normal_f16(10, (L + 1) * KV)
    vc = O.gen_normal_f16(11, (L + 1) * KV)
    table = np.ones(s.head_dim // 2, np.float16).view(np.uint16)
    x0 = O.gen_normal_f32(12, H)
    t0 = time.perf_counter()
    for _ in range(tokens):
        x = x0
        for il in range(s.n_layers):
            glob = s.is_global(il)
            theta = 1e6 if glob else 1e4
            n = O.rms_norm(x, nw)
            q = O.matmul(n, Wq, Q, H, "q4k")
            k = O.matmul(n, Wk, KV, H, "q4k")
            v = O.per_head_rms_norm_no_weight(O.matmul(n, Wv, KV, H, "q4k"), 1, s.head_dim)
            q = O.fused_per_head_norm_rope(q, hw, s.n_q_heads, s.head_dim, 1e-6, START_POS, theta, 0, table)
            k = O.fused_per_head_norm_rope(k, hw, 1, s.head_dim, 1e-6, START_POS, theta, 0, table)
            O.kv_cache_store_f16(k, v, kc, vc, 1, s.head_dim, START_POS)
            a = O.attention(q, kc, vc, s.n_q_heads, 1, s.head_dim, L, 1.0, 0 if glob else s.window)
            h = O.fused_norm_add(O.matmul(a, Wo, H, Q, "q4k"), nw, x)
            n2 = O.rms_norm(h, nw)
            act = O.gelu_mul(O.matmul(n2, Wg, I, H, "q4k"), O.matmul(n2, Wu, I, H, "q4k"))
            x = O.fused_norm_add(O.matmul(act, Wd, H, I, "q6k"), nw, h)
        lg = O.logit_softcap(O.matmul(O.rms_norm(x, nw), Wh, s.vocab, H, "q6k"))
        O.argmax(lg)
    t = time.perf_counter() - t0
    return {"tok_s": round(tokens / t, 4), "tokens": tokens, "seconds": round(t, 2), "cores": 1}


def cpu_baseline():
    """The host-side baseline: config 0 (Q4_K dequant-dot) in Node on one
    core, config 3 (fp32 torch attention) on one core and on the process's
    host threads, and the C oracle's own step rate. `value` scales the
    one-core figures to the headline unit: one token at batch 1 is 35 layers
    of 22.34 MB of K-quant weights (dequant-dot at the Node rate; Q6_K bytes
    priced like Q4_K) with the attention of the benchmark context (28 layers
    over 512 positions, 7 over 513, torch on one core), plus the 330.3 MB LM
    head."""
    t0 = time.perf_counter()
    g0 = node_q4k_gemv()
    threads = _cpu_threads()
    attn1 = torch_attention_cfg3(1)
    attnT = torch_attention_cfg3(threads)
    orc = oracle_step_rate(1)
    s = E2BShape()
    per_token_us = None
    if g0 is not None:
        bps = g0["gbps_dequant_in_loop"] * 1e9
        w_us = (s.layer_weight_bytes() * s.n_layers + s.lm_head_bytes()) / bps * 1e6
        n_glob = len(s.global_layers)
        a_us = (s.n_layers - n_glob) * attn1["ctx4096_window512"]["us"] + n_glob * attn1["ctx512_global"]["us"]
        per_token_us = w_us + a_us
    value = round(1e6 / per_token_us, 5) if per_token_us else orc["tok_s"]
    return {"value": value, "unit": "tok/s", "cores": 1, "kind": "port",
            "sample": (f"config 0 ({g0['gemvs_timed'] if g0 else 0} Q4_K GEMVs 6144x1536, builder's ES2019 "
                       f"dequantizeQ4_K + f32 dot under Node {g0['node'] if g0 else '(absent)'}, 1 core) and "
                       f"config 3 (fp32 torch attention at 512/4096/32768 positions) scaled to one E2B token; "
                       f"also the C oracle on {orc['tokens']} whole step(s); {time.perf_counter() - t0:.1f} s of "
                       f"CPU work on {_cpu_model()}") if g0 else "node absent: C oracle whole steps only",
            "q4k_gemv_config0_node": g0,
            "attention_config3_torch": {"threads_1": attn1, f"threads_{threads}": attnT, "cpu": _cpu_model(),
                                        "host_threads": threads},
            "oracle_c_step": orc}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--census-reps", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-warm", action="store_true",
                    help="attention launches do not read the next matvecs' weights into L2")
    ap.add_argument("--eager", action="store_true",
                    help="launch the step kernels directly instead of replaying a captured graph "
                         "(for profilers that do not follow graph launches)")
    ap.add_argument("--no-census", action="store_true")
    ap.add_argument("--census-only", action="store_true",
                    help="time only the per-kernel census of the B=1 step (the launches a profiler should see)")
    ap.add_argument("--no-gemv0", action="store_true")
    ap.add_argument("--gemv0-only", action="store_true",
                    help="time only the config-0 GEMV over its rotated copies and the pure-streaming floor "
                         "(the launches a profiler should see for config 0)")
    ap.add_argument("--calib-only", action="store_true",
                    help="one 256 MiB streaming read per cache policy, for the HBM counters' calibration")
    ap.add_argument("--positions", default="4096,32768",
                    help="comma-separated start positions of extra B=1 decode runs ('' to skip)")
    ap.add_argument("--pos-steps", type=int, default=100)
    ap.add_argument("--pos-warmup", type=int, default=10)
    ap.add_argument("--no-real-layout", action="store_true",
                    help="skip the decode runs of Gemma-4-E2B's own layer layout")
    ap.add_argument("--no-prefill", action="store_true", help="skip the batched prefill runs")
    ap.add_argument("--no-node-step", action="store_true",
                    help="skip the fused step's rate from a Node host (gemma4-webgpu_amd/node/bench_step.js)")
    ap.add_argument("--real-eager-only", type=int, default=0, metavar="STEPS",
                    help="run STEPS eager (not captured) fused steps of Gemma-4-E2B's layout with per-layer "
                         "embeddings from position 512 and exit (for the kernel tracer)")
    ap.add_argument("--attn-only", action="store_true",
                    help="time only the decode attention of config 3 (the launches a profiler should see)")
    ap.add_argument("--batch-steps", type=int, default=30)
    ap.add_argument("--batch-warmup", type=int, default=5)
    ap.add_argument("--batch-sweep", default="1,8,32,64",
                    help="comma-separated batch sizes of the ragged step ('' to skip)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); "
              "the multi-GPU layout is described, not built", file=sys.stderr)
        sys.exit(2)
    if int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py runs as a single process on one GPU", file=sys.stderr)
        sys.exit(2)

    ctx = g4hip.Context(0)
    info = ctx.info()
    log(f"device {info}")
    if args.gemv0_only:
        g0, fl = gemv_cfg0(ctx), stream_floor(ctx)
        print(json.dumps({"q4k_gemv_config0": g0, "stream_floor": fl, "q4k_gemv_amortised": gemv_q4k_amortised(ctx)}),
              flush=True)
        return
    if args.calib_only:
        print(json.dumps({"calibration": calibration_reads(ctx)}), flush=True)
        return
    if args.attn_only:
        print(json.dumps({"attention_decode": attention_cfg3(ctx)}), flush=True)
        return
    if args.real_eager_only:
        d = Decoder(ctx, E2BShape.real(), max_seq=1024, seed=0, embed=True)
        d.fill_kv(START_POS, seed=1)
        d.set_position(START_POS)
        ctx.sync()
        a = ctx.record()
        for _ in range(args.real_eager_only):
            d.step_fused("argmax")
        b = ctx.record()
        ctx.sync()
        print(json.dumps({"real_eager": {"steps": args.real_eager_only,
                                         "us_per_step": round(ctx.elapsed_ms(a, b) * 1e3 / args.real_eager_only, 1),
                                         "launches_per_step": d.launches_per_step_fused()}}), flush=True)
        return
    s = E2BShape()
    max_seq = START_POS + args.warmup + args.steps + 64
    max_seq = (max_seq + 255) // 256 * 256
    t0 = time.time()
    dec = Decoder(ctx, s, max_seq=max_seq, seed=0)
    dec.fill_kv(START_POS, seed=1)
    dec.set_position(START_POS)
    ctx.sync()
    log(f"weights + KV ready in {time.time() - t0:.1f}s "
        f"({(s.layer_weight_bytes() * s.n_layers + s.lm_head_bytes()) / 1e9:.3f} GB of weights)")

    if args.census_only:
        census = kernel_census(ctx, dec, args.census_reps)
        print(json.dumps({"kernel_census": census}), flush=True)
        return
    if args.eager:
        def step():
            dec.step_fused("argmax", warm=not args.no_warm)
    else:
        graph = dec.capture_fused("argmax", warm=not args.no_warm)

        def step():
            ctx.graph_launch(graph)
    for _ in range(args.warmup):
        step()
    ctx.sync()
    log(f"warmup {args.warmup} steps done")
    a = ctx.record()
    for _ in range(args.steps):
        step()
    b = ctx.record()
    ms_total = ctx.elapsed_ms(a, b)
    ctx.sync()
    ms_step = ms_total / args.steps
    tok_s = 1000.0 / ms_step
    pos_end = int(dec.pos.download(np.uint32)[0])
    log(f"decode ({'eager' if args.eager else 'graph'}): {ms_step * 1e3:.1f} us/token = {tok_s:.1f} tok/s "
        f"(positions {START_POS}..{pos_end})")
    if not args.eager:
        ctx.graph_destroy(graph)

    # the same step from longer contexts, and Gemma-4-E2B's own layer layout
    # (head dim 512 on the global layers, FFN 12288 and shared KV on layers
    # 15..34) with the embedding lookup of the sampled token in the step
    positions = {}
    for start in [int(x) for x in args.positions.split(",") if x.strip()]:
        positions[f"start{start}"] = decode_rate(ctx, E2BShape(), start, args.pos_steps, args.pos_warmup)
        log(f"decode from position {start}: {positions[f'start{start}']}")
    prefill = {} if args.no_prefill else {"uniform": prefill_rate(ctx, E2BShape())}
    log(f"prefill: {prefill}")
    real = {}
    if not args.no_real_layout:
        for start in (START_POS, 4096):
            real[f"start{start}"] = decode_rate(ctx, E2BShape.real(), start, args.pos_steps, args.pos_warmup,
                                                embed=True)
            log(f"real E2B layout from position {start}: {real[f'start{start}']}")
        # the per-layer embeddings' share: the same step without them
        real[f"start{START_POS}_no_ple"] = decode_rate(ctx, E2BShape.real(ple_dim=0), START_POS, args.pos_steps,
                                                       args.pos_warmup, embed=True)
        log(f"real E2B layout without per-layer embeddings: {real[f'start{START_POS}_no_ple']}")
        if not args.no_prefill:
            prefill["real_e2b_layout"] = prefill_rate(ctx, E2BShape.real())
            log(f"prefill (real layout): {prefill['real_e2b_layout']}")

    node_step = None if args.no_node_step else node_step_rate(START_POS, args.pos_steps, args.pos_warmup)
    log(f"fused step from Node: {node_step}")

    batch = {}
    for B in [int(b) for b in args.batch_sweep.split(",") if b.strip()]:
        batch[f"B={B}"] = batch_decode(ctx, B, args.batch_steps, args.batch_warmup, census=(B == 32 and not
                                                                                              args.no_census))
    if args.no_census:
        print(json.dumps({"value": round(tok_s, 2), "unit": "tok/s", "ms_per_step": ms_step,
                          "decode_from_position": positions, "real_e2b_layout": real,
                          "node_fused_step": node_step, "prefill": prefill, "batch_decode": batch}), flush=True)
        return
    census = kernel_census(ctx, dec, args.census_reps)
    for k, v in census.items():
        log(f"  {k}: {v}")
    # dominant kernel = the launch kind with the largest time per step among
    # those the step issues (per_step > 0)
    per_step = {k: v["us"] * v["per_step"] for k, v in census.items()}
    dom = max((k for k in per_step if census[k]["per_step"] > 0), key=lambda k: per_step[k])
    bytes_launch, us_launch = census[dom]["bytes"], census[dom]["us"]
    achieved = bytes_launch / (us_launch * 1e-6) / 1e9
    traffic = measured_traffic(dom)
    roofline = {"bound": "hbm", "kernel": dom, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                "traffic": None if traffic is None else traffic[0],
                # of which the L2 warming's reads of the next launches' weights
                "traffic_warming": None if traffic is None else traffic[1],
                "bytes_per_launch": bytes_launch, "us_per_launch": round(us_launch, 3)}

    g0 = {} if args.no_gemv0 else gemv_cfg0(ctx)
    if g0:
        g0["stream_floor"] = stream_floor(ctx, wg_list=(648, 2048))
        g0["amortised_262144x1536"] = gemv_q4k_amortised(ctx)
    log(f"config-0 Q4_K GEMV: {g0}")
    attn3 = attention_cfg3(ctx)
    log(f"decode attention: {attn3}")
    head = lm_head_sampling(ctx)
    log(f"LM head + sampling: {head}")

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline()
        log(f"cpu baseline: {cpu}")

    line = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_k/q6_k weights x int8 activation digits (i32 dot), f32 accumulate, f16 KV",
        "data": "synthetic (seeded SplitMix64 weights generated on the device, N(0,1) f16 KV)",
        "config": {"workload": "E2B decode B=1: 35 E2B-shaped layers (Q4_K q/k/v/o/gate/up, Q6_K down, "
                               "H=1536, 8 q heads / 1 kv head x 256, I=6144, local window 512 / 7 global) "
                               "+ tied Q6_K LM head 262144x1536 + softcap + argmax, one HIP-graph replay per "
                               "token",
                   "batch": 1, "start_position": START_POS, "positions": [START_POS, pos_end],
                   "launches_per_token": dec.launches_per_step_fused()},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "q4k_gemv_config0": {k: (round(v, 4) if isinstance(v, float) else
                                 {kk: (round(vv, 4) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                                 if isinstance(v, dict) else v) for k, v in g0.items()},
        "kernel_census": {k: {"us_per_launch": round(v["us"], 3), "launches_per_step": v["per_step"],
                              "us_per_step": round(per_step[k], 2), "bytes_per_launch": v["bytes"],
                              "gbps": None if v["gbps"] is None else round(v["gbps"], 1)}
                          for k, v in census.items()},
        "decode_from_position": positions,
        "real_e2b_layout": real,
        "node_fused_step": node_step,
        "prefill": prefill,
        "batch_decode": batch,
        "attention_decode": attn3,
        "lm_head_sampling": head,
        "device": info["name"],
    }
    print(json.dumps(line), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
