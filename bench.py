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
from g4hip.decoder import Decoder, E2BShape  # noqa: E402

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
    Algorithmic bytes: weights + activations read/written by one launch."""
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

    kinds = {
        # name: (per-layer body, launches per body, algorithmic bytes per launch)
        "qkv_normadd_matvec": (
            lambda il, L: c.normAddMatmulSegments(
                "q4k", dec.down, L.post_ffn_norm, dec.hidden2, L.attn_norm, dec.hidden, [L.wq, L.wk, L.wv],
                [dec.q, dec.k, dec.v], [Q, KV, KV], H, s.eps),
            1, q4(Q + 2 * KV, H) + 5 * H * 4 + (Q + 2 * KV) * 4),
        "attn_fused": (
            lambda il, L: c.attnDecodeFused(dec.q, dec.k, dec.v, L.q_norm, L.k_norm, dec.rope_freqs, L.k_cache,
                                            L.v_cache, dec.attn, dec.attn_params[il], dec.attn_ws, dec.pos),
            1, kv_avg + (Q + 2 * KV) * 4 + Q * 4),
        "o_matvec": (
            lambda il, L: c.matmulQuant(dec.attn, L.wo, dec.o, H, Q),
            1, q4(H, Q) + Q * 4 + H * 4),
        "gateup_gelu": (
            lambda il, L: c.normAddGateUpGelu_q4k(dec.o, L.post_attn_norm, dec.hidden, L.pre_ffn_norm, L.wgate,
                                                  L.wup, dec.hidden2, dec.act, I, H, s.eps),
            1, 2 * q4(I, H) + 4 * H * 4 + I * 4),
        "down_matvec_q6k": (
            lambda il, L: c.matmulQuant(dec.act, L.wdown, dec.down, H, I, "q6k"),
            1, q6(H, I) + I * 4 + H * 4),
    }
    out = {}
    for name, (body, launches, nbytes) in kinds.items():
        ctx.graph_begin()
        try:
            for il, L in enumerate(Ls):
                body(il, L)
        finally:
            g = ctx.graph_end()
        us = time_launches(ctx, lambda _i=0: ctx.graph_launch(g), reps) * 1e3 / nl
        ctx.graph_destroy(g)
        out[name] = {"us": us, "per_step": nl, "bytes": nbytes, "gbps": nbytes / (us * 1e-6) / 1e9}
    # LM head with the final norm-add and softcap (330 MB: larger than the
    # 256 MB last-level cache, so no rotation is needed)
    last = Ls[-1]
    ctx.graph_begin()
    try:
        c.normAddMatmulSegments("q6k", dec.down, last.post_ffn_norm, dec.hidden2, dec.final_norm, dec.hidden,
                                [dec.lm_head], [dec.logits], [V], H, s.eps, softcap=s.softcap)
    finally:
        g = ctx.graph_end()
    us = time_launches(ctx, lambda _i=0: ctx.graph_launch(g), max(5, reps)) * 1e3
    ctx.graph_destroy(g)
    nbytes = s.lm_head_bytes() + 5 * H * 4 + V * 4
    out["lm_head_q6k_softcap"] = {"us": us, "per_step": 1, "bytes": nbytes, "gbps": nbytes / (us * 1e-6) / 1e9}
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
    return None if entry is None else entry["bytes_per_launch"]


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


def cpu_baseline(tokens=5):
    """Times the CPU oracle (plain C, 1 thread, f64 accumulation) on `tokens`
    whole decode steps of the same workload: 35 E2B-shaped layers at context
    START_POS + 1 (local layers windowed, every fifth global) plus the full
    262144-row Q6_K LM head, softcap and argmax. One set of layer weights is
    reused for all layers (the cost does not depend on the values); weight
    generation is outside the timed region."""
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
    return {"value": tokens / t, "unit": "tok/s", "cores": 1, "kind": "port",
            "sample": (f"CPU oracle (plain C, 1 thread, f64 accumulation): {tokens} whole decode steps "
                       f"(35 E2B-shaped layers at context {L} + full 262144-row Q6_K LM head + softcap "
                       f"+ argmax), {t:.1f} s of CPU work")}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--census-reps", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-tokens", type=int, default=5)
    ap.add_argument("--eager", action="store_true",
                    help="launch the step kernels directly instead of replaying a captured graph "
                         "(for profilers that do not follow graph launches)")
    ap.add_argument("--no-census", action="store_true")
    ap.add_argument("--no-gemv0", action="store_true")
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

    if args.eager:
        def step():
            dec.step_fused("argmax")
    else:
        graph = dec.capture_fused("argmax")

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

    if args.no_census:
        print(json.dumps({"value": round(tok_s, 2), "unit": "tok/s", "ms_per_step": ms_step}), flush=True)
        return
    census = kernel_census(ctx, dec, args.census_reps)
    for k, v in census.items():
        log(f"  {k}: {v}")
    # dominant kernel = largest time per step
    per_step = {k: v["us"] * v["per_step"] for k, v in census.items()}
    dom = max(per_step, key=lambda k: per_step[k])
    bytes_launch, us_launch = census[dom]["bytes"], census[dom]["us"]
    achieved = bytes_launch / (us_launch * 1e-6) / 1e9
    roofline = {"bound": "hbm", "kernel": dom, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": measured_traffic(dom),
                "bytes_per_launch": bytes_launch, "us_per_launch": round(us_launch, 3)}

    g0 = {} if args.no_gemv0 else gemv_cfg0(ctx)
    log(f"config-0 Q4_K GEMV: {g0}")

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(tokens=args.cpu_tokens)
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
        "q4k_gemv_config0": {k: (round(v, 4) if isinstance(v, float) else v) for k, v in g0.items()},
        "kernel_census_us": {k: round(per_step[k], 2) for k in per_step},
        "device": info["name"],
    }
    print(json.dumps(line), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
