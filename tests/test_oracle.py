"""Pins the CPU oracle (oracle/g4_oracle.c) before it is trusted as the checker.

Every oracle function is checked against something other than its own
formula: the reference's committed fixtures (HF bf16 activations of
Gemma-4-E2B, tests/golden/ref_fixtures.npz), library routines (numpy IEEE
half, torch's tanh-GELU and softmax attention, transformers' Gemma-4 RoPE and
RMSNorm), an inverse of the Q4_K scale packing written from the byte-layout
description, hand-computed blocks, published SplitMix64 vectors, and an
independent vectorised numpy restatement.
"""
import math
import os
import struct

import numpy as np
import pytest

import oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def fx():
    return np.load(os.path.join(GOLDEN, "ref_fixtures.npz"), allow_pickle=False)


def f16(x) -> int:
    return int(np.array(x, np.float16).view(np.uint16))


# --------------------------------------------------------------------------
# f16 conversions (src/gguf.ts:103-113, 402-473)
# --------------------------------------------------------------------------

def test_f16_to_f32_exhaustive():
    """All 65536 half patterns decode like numpy's IEEE half."""
    hs = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = hs.view(np.float16).astype(np.float32)
    got = np.array([O.f16_to_f32(int(h)) for h in hs], np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_rne_matches_numpy():
    rng = np.random.default_rng(1)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10) ** rng.integers(-9, 6, 20000),
        np.array([0.0, -0.0, 65504, 65519.99, 65520, -65520, 1e30, -1e30, np.inf, -np.inf,
                  2.0 ** -24, 2.0 ** -25, 1.5 * 2.0 ** -25, 2.0 ** -26, 3 * 2.0 ** -26, 2.0 ** -14,
                  2.0 ** -14 * (1 - 2 ** -11), 1e-45], np.float32),
    ]).astype(np.float32)
    got = np.array([O.f32_to_f16_rne(float(v)) for v in vals], np.uint16)
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    assert O.f32_to_f16_rne(float("nan")) & 0x7c00 == 0x7c00


def test_f32_to_f16_trunc_known_answers():
    # 1 + 2^-10 + 2^-11 truncates to 1 + 2^-10 (RNE would round up to 1 + 2^-9)
    assert O.f32_to_f16_trunc(1 + 2 ** -10 + 2 ** -11) == 0x3c01
    assert O.f32_to_f16_rne(1 + 2 ** -10 + 2 ** -11) == 0x3c02
    assert O.f32_to_f16_trunc(1e30) == 0x7c00          # rope_freqs 1e30 -> +Inf
    assert O.f32_to_f16_trunc(1e-40) == 0x0000         # f32 subnormal flushes
    assert O.f32_to_f16_trunc(-2.0) == 0xc000


# --------------------------------------------------------------------------
# Q4_K (src/gguf.ts:157-210)
# --------------------------------------------------------------------------

def pack_q4k_scales(sc, m):
    """Inverse of the 12-byte scale/min packing, from the layout description:
    j<4 -> low 6 bits of s[j] (scale) and s[j+4] (min); j>=4 -> low nibble of
    s[j+4] = scale & 15, high nibble = min & 15, top two bits of s[j-4] =
    scale >> 4, top two bits of s[j] = min >> 4."""
    s = [0] * 12
    for j in range(4):
        s[j] |= sc[j] & 63
        s[j + 4] |= m[j] & 63
    for j in range(4, 8):
        s[j + 4] = (sc[j] & 15) | ((m[j] & 15) << 4)
        s[j - 4] |= (sc[j] >> 4) << 6
        s[j] |= (m[j] >> 4) << 6
    return bytes(s)


def test_q4k_scale_unpack_inverse_exhaustive():
    rng = np.random.default_rng(2)
    for j in range(8):
        for v in range(64):
            for w in range(64):
                sc = list(rng.integers(0, 64, 8))
                m = list(rng.integers(0, 64, 8))
                sc[j], m[j] = v, w
                s = pack_q4k_scales(sc, m)
                assert O.q4k_scale_min(s, j) == (v, w)


def make_q4k_block(d, dmin, sc, m, qs):
    return (struct.pack("<HH", f16(d), f16(dmin)) + pack_q4k_scales(sc, m) + bytes(qs))


def test_q4k_known_answer_block():
    # d=0.5, dmin=0.25, sub-block j has scale j+1 and min 2j; every qs byte 0x21
    # (low nibble 1, high nibble 2): element in sub-block j = 0.5*(j+1)*q - 0.25*2j
    sc = [j + 1 for j in range(8)]
    m = [2 * j for j in range(8)]
    blk = make_q4k_block(0.5, 0.25, sc, m, [0x21] * 128)
    out = O.dequant_q4k(np.frombuffer(blk, np.uint8))
    for j in range(8):
        q = 1 if j % 2 == 0 else 2
        want = 0.5 * (j + 1) * q - 0.25 * 2 * j
        assert np.all(out[32 * j:32 * j + 32] == np.float32(want)), j
    # element order: group g low nibbles -> 64g+l, high nibbles -> 64g+32+l
    qs = list(range(128))
    blk = make_q4k_block(1.0, 0.0, [1] * 8, [0] * 8, [q & 0xff for q in qs])
    out = O.dequant_q4k(np.frombuffer(blk, np.uint8))
    for g in range(4):
        for l in range(32):
            assert out[64 * g + l] == (qs[32 * g + l] & 15)
            assert out[64 * g + 32 + l] == (qs[32 * g + l] >> 4)


def q4k_edge_blocks(rng, n):
    blocks = O.gen_q4k(7, n).reshape(n, 144).copy()
    specials = [0x0000, 0x8000, 0x0001, 0x03ff, 0x0400, 0x7bff, 0xfbff, 0x3c00, 0xbc00, 0x7c00, 0x7e00]
    for i in range(n):
        if i % 3 == 0:
            blocks[i, 0:2] = np.frombuffer(struct.pack("<H", specials[i % len(specials)]), np.uint8)
        if i % 5 == 0:
            blocks[i, 2:4] = np.frombuffer(struct.pack("<H", specials[(i // 5) % len(specials)]), np.uint8)
    return blocks.reshape(-1)


def test_q4k_c_vs_numpy_restatement():
    rng = np.random.default_rng(3)
    b = q4k_edge_blocks(rng, 600)
    a = O.dequant_q4k(b)
    c = O.np_dequant_q4k(b)
    nan = np.isnan(a)
    assert np.array_equal(nan, np.isnan(c))
    assert np.array_equal(a[~nan].view(np.uint32), c[~nan].view(np.uint32))


def test_q4k_f32_single_rounding_equals_f64():
    """The f32 evaluation d1*q - min1 (exact product, one rounding) equals the
    reference's f64 evaluation stored to f32 on every generated block."""
    b = O.gen_q4k(11, 2000).reshape(-1, 144)
    d = O.np_f16_to_f32(b[:, 0:2].copy().view(np.uint16)[:, 0])
    dmin = O.np_f16_to_f32(b[:, 2:4].copy().view(np.uint16)[:, 0])
    sc, m = O.np_q4k_scales(b[:, 4:16])
    qs = b[:, 16:].reshape(-1, 4, 32)
    q = np.empty((b.shape[0], 8, 32), np.float32)
    q[:, 0::2] = qs & 15
    q[:, 1::2] = qs >> 4
    d1 = (d[:, None] * sc.astype(np.float32)).astype(np.float32)
    m1 = (dmin[:, None] * m.astype(np.float32)).astype(np.float32)
    f32 = (d1[:, :, None] * q - m1[:, :, None]).astype(np.float32).reshape(-1)
    assert np.array_equal(f32.view(np.uint32), O.dequant_q4k(b.reshape(-1)).view(np.uint32))


# --------------------------------------------------------------------------
# Q6_K (src/gguf.ts:316-368)
# --------------------------------------------------------------------------

def make_q6k_block(d, q, sc):
    """Packs 256 6-bit values q (0..63, element order) from the layout
    description: per half h and l<32, element 128h + 32k + l takes its low
    nibble from ql[64h + l + 32*(k&1)] (low nibble for k<2, high for k>=2) and
    its top two bits from bits 2k..2k+1 of qh[32h + l]."""
    ql = [0] * 128
    qh = [0] * 64
    for h in range(2):
        for k in range(4):
            for l in range(32):
                v = q[128 * h + 32 * k + l]
                qi = 64 * h + l + 32 * (k & 1)
                if k < 2:
                    ql[qi] |= v & 15
                else:
                    ql[qi] |= (v & 15) << 4
                qh[32 * h + l] |= (v >> 4) << (2 * k)
    return bytes(ql) + bytes(qh) + struct.pack("<16b", *sc) + struct.pack("<H", f16(d))


def test_q6k_known_answer_and_packing():
    rng = np.random.default_rng(4)
    q = rng.integers(0, 64, 256)
    sc = list(rng.integers(-128, 128, 16))
    blk = make_q6k_block(0.125, q, sc)
    out = O.dequant_q6k(np.frombuffer(blk, np.uint8))
    for e in range(256):
        # sub-block of 16 elements e//16 uses scale sc[e // 16]
        assert out[e] == np.float32(0.125 * sc[e // 16] * (int(q[e]) - 32)), e


def test_q6k_c_vs_numpy_restatement():
    b = O.gen_q6k(5, 800).reshape(800, 210).copy()
    b[::7, 208:210] = np.frombuffer(struct.pack("<H", 0x0001), np.uint8)   # subnormal d
    b[1::7, 208:210] = np.frombuffer(struct.pack("<H", 0xbc00), np.uint8)  # d = -1
    b = b.reshape(-1)
    a = O.dequant_q6k(b)
    c = O.np_dequant_q6k(b)
    assert np.array_equal(a.view(np.uint32), c.view(np.uint32))


# --------------------------------------------------------------------------
# matvec
# --------------------------------------------------------------------------

def test_matmul_closed_forms():
    # all weights equal 1: d=1, scale 1, min 0, every nibble 1 -> y_m = sum(x)
    M, N = 5, 512
    blk = make_q4k_block(1.0, 0.0, [1] * 8, [0] * 8, [0x11] * 128)
    W = np.frombuffer(blk * (M * N // 256), np.uint8)
    x = np.random.default_rng(5).standard_normal(N).astype(np.float32)
    y = O.matmul(x, W, M, N, "q4k")
    assert np.allclose(y, x.astype(np.float64).sum(), rtol=1e-6)
    # linearity in x and agreement with dequant @ x
    W = O.gen_q4k(9, 64 * 6)
    x2 = np.random.default_rng(6).standard_normal(1536).astype(np.float32)
    x3 = np.random.default_rng(7).standard_normal(1536).astype(np.float32)
    Wd = O.dequant_q4k(W).reshape(64, 1536).astype(np.float64)
    y2 = O.matmul(x2, W, 64, 1536, "q4k")
    assert np.allclose(y2, Wd @ x2, rtol=1e-6, atol=1e-6)
    y23 = O.matmul((x2 + x3).astype(np.float32), W, 64, 1536, "q4k")
    assert np.allclose(y23, y2 + O.matmul(x3, W, 64, 1536, "q4k"), rtol=1e-5, atol=1e-5)
    W6 = O.gen_q6k(10, 32 * 6)
    Wd6 = O.dequant_q6k(W6).reshape(32, 1536).astype(np.float64)
    assert np.allclose(O.matmul(x2, W6, 32, 1536, "q6k"), Wd6 @ x2, rtol=1e-6, atol=1e-6)


def test_matmul_f16w_closed_forms():
    """The f16-weight matvec (shaders/matmul_quant.wgsl:14,21-54: W is
    array<f16>, f32 accumulate) on weights whose products are known exactly:
    all ones -> sum(x); a permutation matrix -> the permuted x bit for bit;
    powers of two down a diagonal -> x scaled exactly; f16 limits (65504,
    the smallest subnormal) times power-of-two x; and linearity in x."""
    rng = np.random.default_rng(21)
    M, N = 7, 384
    x = rng.standard_normal(N).astype(np.float32)
    ones = np.full(M * N, 0x3C00, np.uint16)
    assert np.allclose(O.matmul(x, ones, M, N, "f16"), x.astype(np.float64).sum(), rtol=1e-7, atol=1e-7)
    perm = rng.permutation(N)
    P = np.zeros((N, N), np.uint16)
    P[np.arange(N), perm] = 0x3C00
    y = O.matmul(x, P.reshape(-1), N, N, "f16")
    assert np.array_equal(y.view(np.uint32), x[perm].view(np.uint32))
    D = np.zeros((N, N), np.float16)
    e = rng.integers(-14, 15, N)
    D[np.arange(N), np.arange(N)] = np.float16(2.0) ** e.astype(np.float16)
    y = O.matmul(x, D.view(np.uint16).reshape(-1), N, N, "f16")
    assert np.array_equal(y, (x.astype(np.float64) * 2.0 ** e).astype(np.float32))
    lim = np.array([0x7BFF, 0x0001, 0x8400, 0x3555], np.uint16)     # 65504, 2^-24, -2^-14, 0.33325...
    xs = np.zeros(4, np.float32)
    for i, h in enumerate(lim):
        xs[:] = 0
        xs[i] = 0.5
        row = lim.reshape(1, 4)
        want = float(np.uint16(h).view(np.float16)) * 0.5
        assert O.matmul(xs, row.reshape(-1), 1, 4, "f16")[0] == np.float32(want)
    # torch's float64 linear on the decoded weights (a library routine)
    import torch
    W = (rng.standard_normal((M, N)) * 0.05).astype(np.float16)
    x2 = rng.standard_normal(N).astype(np.float32)
    ref = torch.nn.functional.linear(torch.from_numpy(x2.astype(np.float64)),
                                     torch.from_numpy(W.astype(np.float64))).numpy()
    got = O.matmul(x2, W.view(np.uint16).reshape(-1), M, N, "f16")
    assert np.allclose(got, ref, rtol=1e-6, atol=1e-7)
    # a transposed operand (W^T x) would fail this
    assert not np.allclose(got, (W.astype(np.float64).T[:M, :M] @ x2[:M]), rtol=1e-2)
    # linearity
    got3 = O.matmul((x2 + x).astype(np.float32), W.view(np.uint16).reshape(-1), M, N, "f16")
    assert np.allclose(got3, got + O.matmul(x, W.view(np.uint16).reshape(-1), M, N, "f16"), rtol=1e-5,
                       atol=1e-6)


# --------------------------------------------------------------------------
# norms, activations, RoPE: fixtures and library routines
# --------------------------------------------------------------------------

def test_v_norm_against_fixture(fx):
    """Weightless per-head RMSNorm of the HF v_proj output reproduces HF's
    v_norm output (bf16 capture => 1e-2 scale tolerance)."""
    v = fx["L0_self_attn__v_proj_output"].astype(np.float32)
    want = fx["L0_self_attn__v_norm_output"].reshape(-1)
    got = O.per_head_rms_norm_no_weight(v, 1, 256, 1e-6)
    assert O.cosine(got, want) > 0.99999
    assert np.max(np.abs(got - want)) < 1.5e-2
    # rms(v) ~ 67: the magnitude that makes v_norm matter
    assert 60 < math.sqrt(float(np.mean(v.astype(np.float64) ** 2))) < 75


def test_gelu_against_fixture_and_torch(fx):
    import torch

    g = fx["L0_mlp__gate_proj_output"].astype(np.float32)
    u = fx["L0_mlp__up_proj_output"].astype(np.float32)
    act = fx["L0_mlp__act_fn_output"]
    down_in = fx["L0_mlp_down_proj_input"]
    ones = np.ones_like(g)
    got_act = O.gelu_mul(g, ones)
    assert np.max(np.abs(got_act - act)) < 2e-2
    assert O.cosine(O.gelu_mul(g, u), down_in) > 0.99999
    # torch's tanh-approximate GELU (a library routine) on a wide range
    x = np.linspace(-40, 40, 20001).astype(np.float32)
    ref = torch.nn.functional.gelu(torch.from_numpy(x).double(), approximate="tanh").numpy()
    got = O.gelu_mul(x, np.ones_like(x))
    assert np.allclose(got, ref, rtol=1e-6, atol=1e-6)
    # and torch's float32 evaluation where tanh saturates: the shader's tanh
    # is an f32, so 1 + tanh(t) is 0 below x ~ -5.5 (f64 would leave ~1e-10)
    ref32 = torch.nn.functional.gelu(torch.from_numpy(x), approximate="tanh").numpy()
    sat = x < -5.5
    assert np.all(got[sat] == 0) and np.all(ref32[sat] == 0)
    near = (x > -5.5) & (x < -3)   # 1 + tanh(t) here is a multiple of 2^-24: within one such step
    assert np.all(np.abs(got[near] - ref32[near]) <= np.abs(x[near]) * 2.0 ** -24 * 1.01)
    assert np.array_equal(O.np_gelu_mul(x, np.ones_like(x)), got)


def test_rms_norm_against_transformers():
    import torch
    from transformers.models.gemma4.modeling_gemma4 import Gemma4RMSNorm

    rng = np.random.default_rng(8)
    x = rng.standard_normal(1536).astype(np.float32) * 3
    w16 = (rng.standard_normal(1536) * 0.1 + 1).astype(np.float16)
    mod = Gemma4RMSNorm(1536, eps=1e-6).double()
    with torch.no_grad():
        mod.weight.copy_(torch.from_numpy(w16.astype(np.float64)))
        want = mod(torch.from_numpy(x.astype(np.float64))).numpy()
    got = O.rms_norm(x, w16.view(np.uint16), 1e-6)
    assert np.allclose(got, want, rtol=2e-6, atol=1e-6)
    res = rng.standard_normal(1536).astype(np.float32)
    assert np.allclose(O.fused_norm_add(x, w16.view(np.uint16), res, 1e-6), res + want, rtol=2e-6, atol=2e-6)
    assert np.allclose(got, O.np_rms_norm(x, w16.view(np.uint16)), rtol=1e-6, atol=1e-7)


def test_rope_against_transformers_rotate_half():
    import torch
    from transformers.models.gemma4.modeling_gemma4 import apply_rotary_pos_emb

    rng = np.random.default_rng(9)
    for hd, theta, pos in [(256, 1e4, 14), (256, 1e4, 511), (512, 1e6, 4095), (256, 1e6, 32767)]:
        x = rng.standard_normal((8, hd)).astype(np.float32)
        w = np.ones(hd, np.float16)
        freqs = np.ones(hd // 2, np.float16)
        got = O.fused_per_head_norm_rope(x.reshape(-1), w.view(np.uint16), 8, hd, 1e-6, pos, theta, 0,
                                         freqs.view(np.uint16)).reshape(8, hd)
        xn = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2, axis=1, keepdims=True) + 1e-6)
        xn = xn.astype(np.float32).astype(np.float64)
        f = np.array([O.rope_freq(theta, i, hd, 0, freqs.view(np.uint16)) for i in range(hd // 2)], np.float32)
        ang = (np.float32(pos) * f).astype(np.float64)        # f32 angle as the shader forms it
        emb = np.concatenate([ang, ang])
        cos = torch.from_numpy(np.cos(emb))[None, None]
        sin = torch.from_numpy(np.sin(emb))[None, None]
        want = apply_rotary_pos_emb(torch.from_numpy(xn)[None], cos, sin, unsqueeze_dim=1)[0].numpy()
        assert np.allclose(got, want, rtol=1e-5, atol=1e-6), (hd, theta, pos)


def _tf_inv_freq():
    """transformers' own RoPE initialisers for Gemma 4 (default rope for the
    sliding layers: theta 1e4, head_dim 256; proportional rope for the full
    layers: theta 1e6, head_dim 512, partial_rotary_factor 0.25), read from
    the rotary module's buffers."""
    from transformers.models.gemma4.configuration_gemma4 import Gemma4TextConfig
    from transformers.models.gemma4.modeling_gemma4 import Gemma4TextRotaryEmbedding

    cfg = Gemma4TextConfig()
    rp = cfg.rope_parameters
    assert rp["sliding_attention"] == {"rope_type": "default", "rope_theta": 10000.0}
    assert rp["full_attention"]["rope_type"] == "proportional"
    assert rp["full_attention"]["partial_rotary_factor"] == 0.25
    assert rp["full_attention"]["rope_theta"] == 1e6
    rot = Gemma4TextRotaryEmbedding(cfg)
    buf = dict(rot.named_buffers())
    return rot, buf["sliding_attention_inv_freq"].numpy(), buf["full_attention_inv_freq"].numpy()


def test_rope_freq_against_transformers_init():
    """Every pair's frequency (src/engine.ts:522-537,
    shaders/fused_per_head_norm_rope.wgsl:50-55) against transformers'
    default and proportional initialisers: 1/theta^(2i/hd) for every pair of
    a sliding layer (hd 256, theta 1e4); for a full layer (hd 512, theta 1e6)
    the first 64 pairs rotate at 1/theta^(2i/512) and the other 192 are
    frozen, which the reference gets from the GGUF rope_freqs divisor table
    (1.0, then 1e30 = +Inf in f16)."""
    _, inv_s, inv_f = _tf_inv_freq()
    assert inv_s.shape == (128,) and inv_f.shape == (256,)
    ones = np.ones(128, np.float16).view(np.uint16)
    got_s = np.array([O.rope_freq(1e4, i, 256, 0, ones) for i in range(128)], np.float32)
    # f64 pow rounded once vs torch's f32 pow: within 2 ulp
    assert np.max(np.abs(got_s.view(np.int32) - inv_s.view(np.int32))) <= 1   # f64 vs f32 pow: 1 ulp
    table = np.where(np.arange(256) < 64, 1.0, 1e30).astype(np.float32)
    table16 = np.array([O.f32_to_f16_trunc(float(t)) for t in table], np.uint16)   # 1e30 -> +Inf
    got_f = np.array([O.rope_freq(1e6, i, 512, 1, table16) for i in range(256)], np.float32)
    assert np.array_equal(got_f[64:], inv_f[64:]) and np.all(inv_f[64:] == 0)
    assert np.max(np.abs(got_f.view(np.int32) - inv_f.view(np.int32))) <= 1
    # a plausible mistake: exponent i/hd instead of 2i/hd fails the check
    wrong = np.array([1.0 / 1e4 ** (i / 256) for i in range(128)], np.float32)
    assert not np.allclose(wrong, inv_s, rtol=1e-3)


def test_rope_rotation_against_transformers_module():
    """The whole per-head norm + RoPE at non-zero positions against
    transformers: its rotary module's cos/sin for each layer type fed to its
    apply_rotary_pos_emb, on the oracle's own normalised vector. torch forms
    each frequency with an f32 pow, which differs from the oracle's by at
    most 1 ulp (checked above); pairs whose frequencies are bit-equal are
    held to 1e-5, the others to the angle difference position * |df| that
    one ulp makes."""
    import torch
    from transformers.models.gemma4.modeling_gemma4 import apply_rotary_pos_emb

    rot, inv_s, inv_f = _tf_inv_freq()
    rng = np.random.default_rng(19)
    for layer_type, hd, theta, div, inv in [("sliding_attention", 256, 1e4, 0, inv_s),
                                            ("full_attention", 512, 1e6, 1, inv_f)]:
        half = hd // 2
        table = np.where(np.arange(half) < 64, 1.0, np.inf).astype(np.float16).view(np.uint16)
        f = np.array([O.rope_freq(theta, i, hd, div, table) for i in range(half)], np.float32)
        df = np.abs(f.astype(np.float64) - inv.astype(np.float64))
        for pos in (1, 14, 511, 4095, 32767):
            x = rng.standard_normal((8, hd)).astype(np.float32)
            w = (rng.standard_normal(hd) * 0.1 + 1).astype(np.float16)
            got = O.fused_per_head_norm_rope(x.reshape(-1), w.view(np.uint16), 8, hd, 1e-6, pos, theta, div,
                                             table).reshape(8, hd)
            xn = np.stack([O.rms_norm(x[h], w.view(np.uint16), 1e-6) for h in range(8)]).astype(np.float64)
            with torch.no_grad():
                cos, sin = rot(torch.zeros(1, 1, hd), torch.tensor([[pos]]), layer_type=layer_type)
                want = apply_rotary_pos_emb(torch.from_numpy(xn)[None], cos.double(), sin.double(),
                                            unsqueeze_dim=1)[0].numpy().reshape(8, hd)
            assert cos.shape[-1] == hd
            pair_mag = np.sqrt(xn[:, :half] ** 2 + xn[:, half:] ** 2)
            tol = np.tile(1e-5 * pair_mag + 3e-6 + 1.01 * pos * df * pair_mag, (1, 2))
            err = np.abs(got - want)
            assert np.all(err <= tol), (layer_type, pos, float(np.max(err - tol)))
            eq = np.tile(df == 0, 2)
            assert np.allclose(got[:, eq], want[:, eq], rtol=1e-5, atol=3e-6), (layer_type, pos)


def test_rope_closed_forms():
    rng = np.random.default_rng(10)
    hd = 256
    x = rng.standard_normal(hd).astype(np.float32)
    w = np.ones(hd, np.float16).view(np.uint16)
    no = np.ones(hd // 2, np.float16).view(np.uint16)
    normed = O.per_head_rms_norm_no_weight(x, 1, hd, 1e-6)
    # position 0: no rotation
    assert np.allclose(O.fused_per_head_norm_rope(x, w, 1, hd, 1e-6, 0, 1e4, 0, no), normed, atol=1e-7)
    # rotation preserves each pair's norm
    y = O.fused_per_head_norm_rope(x, w, 1, hd, 1e-6, 1234, 1e4, 0, no)
    n0 = normed[:128] ** 2 + normed[128:] ** 2
    n1 = y[:128] ** 2 + y[128:] ** 2
    assert np.allclose(n0, n1, rtol=1e-5, atol=1e-6)
    # pair 0 has frequency 1: angle = position exactly
    p = 3
    c, s = math.cos(p), math.sin(p)
    y = O.fused_per_head_norm_rope(x, w, 1, hd, 1e-6, p, 1e4, 0, no)
    assert abs(y[0] - (normed[0] * c - normed[128] * s)) < 1e-6
    # divisor +Inf (the f16 image of 1e30) freezes a pair; 1.0 leaves it alone
    table = np.where(np.arange(hd // 2) < 32, 1.0, np.inf).astype(np.float16).view(np.uint16)
    y = O.fused_per_head_norm_rope(x, w, 1, hd, 1e-6, 777, 1e6, 1, table)
    assert np.array_equal(y[32:128], normed[32:128]) and np.array_equal(y[160:], normed[160:])
    y2 = O.fused_per_head_norm_rope(x, w, 1, hd, 1e-6, 777, 1e6, 0, table)
    assert np.array_equal(y[:32], y2[:32])


# --------------------------------------------------------------------------
# attention: torch softmax attention (library) and the trio
# --------------------------------------------------------------------------

def _attn_inputs(rng, nqh, nkh, hd, L):
    q = rng.standard_normal(nqh * hd).astype(np.float32)
    k = rng.standard_normal(L * nkh * hd).astype(np.float16).view(np.uint16)
    v = rng.standard_normal(L * nkh * hd).astype(np.float16).view(np.uint16)
    return q, k, v


@pytest.mark.parametrize("L,window", [(1, 0), (7, 0), (33, 0), (600, 512), (600, 0)])
def test_attention_against_torch(L, window):
    import torch

    rng = np.random.default_rng(L + window)
    nqh, nkh, hd = 8, 1, 256
    q, k, v = _attn_inputs(rng, nqh, nkh, hd, L)
    got = O.attention(q, k, v, nqh, nkh, hd, L, 1.0, window)
    qt = torch.from_numpy(q.reshape(1, nqh, 1, hd).astype(np.float64))
    kt = torch.from_numpy(k.view(np.float16).astype(np.float64).reshape(1, L, nkh, hd)).transpose(1, 2)
    vt = torch.from_numpy(v.view(np.float16).astype(np.float64).reshape(1, L, nkh, hd)).transpose(1, 2)
    kt = kt.repeat_interleave(nqh // nkh, dim=1)
    vt = vt.repeat_interleave(nqh // nkh, dim=1)
    mask = torch.zeros(1, 1, 1, L, dtype=torch.float64)
    if window:
        mask[..., : max(0, L - window)] = float("-inf")   # keys kv_idx > q_idx - W stay
    want = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, attn_mask=mask, scale=1.0)
    assert np.allclose(got, want.numpy().reshape(-1), rtol=1e-5, atol=1e-6)
    # the per-kernel trio agrees with the fused oracle
    s = O.attn_score(q, k, nqh, nkh, hd, L, 1.0, window)
    p = O.softmax(s, nqh, L)
    trio = O.attn_output(p, v, nqh, nkh, hd, L)
    # the trio stores scores and probabilities as f32 between kernels
    assert O.rel_l2(trio, got) < 1e-5
    if window and L > window:
        assert np.all(s.reshape(nqh, L)[:, : L - window] == np.float32(-1e30))


def test_paged_attention_equals_dense():
    rng = np.random.default_rng(12)
    nqh, nkh, hd, L, P = 8, 1, 256, 77, 16
    q, k, v = _attn_inputs(rng, nqh, nkh, hd, L)
    pages = (L + P - 1) // P
    perm = rng.permutation(pages + 5)[:pages].astype(np.int32)
    kp = np.zeros(((pages + 5) * P, hd), np.uint16)
    vp = np.zeros_like(kp)
    for t in range(L):
        row = perm[t // P] * P + t % P
        kp[row] = k.reshape(L, hd)[t]
        vp[row] = v.reshape(L, hd)[t]
    a = O.attention(q, k, v, nqh, nkh, hd, L)
    b = O.attention_paged(q, kp.reshape(-1), vp.reshape(-1), perm, P, nqh, nkh, hd, L)
    assert np.array_equal(a, b)


# --------------------------------------------------------------------------
# LM head tail: softcap, argmax, topk256 (shaders/argmax.wgsl, topk256.wgsl)
# --------------------------------------------------------------------------

def test_argmax_fixture(fx):
    """The fixture's logits (HF, pos 14) pick token 236777, the reference's greedy token."""
    lg = fx["logits_pos14"]
    assert O.argmax(lg) == 236777 == int(np.argmax(lg))


def bitrev8(c: int) -> int:
    return int(f"{c:08b}"[::-1], 2)


def _rule_argmax(x):
    """Closed form of the shader's tie rule. The tree reduce merges slot t with
    t + stride for stride = 128, 64, ..., 1 and keeps the lower slot on equal
    values, so the last merge (slot 0 vs 1) prefers an even residue class, the
    one before it a class with bit 1 clear, and so on: among the maxima (NaN
    and values <= -1e30 never count) the class c = i mod 256 with the smallest
    bit-reversed c wins, then the smallest index; with no candidate, 0."""
    x = np.asarray(x, np.float32)
    ok = (x > np.float32(-1e30)) & ~np.isnan(x)
    if not ok.any():
        return 0
    mx = x[ok].max()
    idx = np.nonzero(ok & (x == mx))[0]
    return int(min(idx, key=lambda i: (bitrev8(i % 256), i)))


def test_argmax_tie_rule():
    rng = np.random.default_rng(13)
    for trial in range(300):
        n = int(rng.integers(1, 3000))
        x = rng.integers(-3, 4, n).astype(np.float32)   # heavy ties
        if trial % 10 == 0:
            x[rng.integers(0, n, 5)] = np.nan
        if trial % 13 == 0:
            x[:] = -np.inf
        if trial % 17 == 0:
            x[:] = np.float32(-1e30)
        if trial % 19 == 0:
            x[rng.integers(0, n)] = -0.0
        assert O.argmax(x) == _rule_argmax(x), trial


def test_topk256_residue_maxima_and_stable_sort(fx):
    lg = fx["logits_pos14"]
    packed = O.topk256(lg)
    vals = packed[0::2]
    ids = packed[1::2].view(np.uint32)
    # value = max of its residue class, index = first occurrence of it
    grid = lg.reshape(-1, 256)
    assert np.array_equal(vals, grid.max(axis=0))
    first = grid.argmax(axis=0) * 256 + np.arange(256)
    assert np.array_equal(ids, first)
    # the candidate set is not the global top-256 (162/256 overlap on this fixture)
    top = set(np.argsort(-lg, kind="stable")[:256].tolist())
    assert len(top & set(ids.tolist())) == 162
    sid, sval = O.topk_sort(packed)
    # stable descending sort: numpy's stable argsort of -value gives the same order
    order = np.argsort(-vals, kind="stable")
    assert np.array_equal(sid, ids[order]) and np.array_equal(sval, vals[order])
    assert int(np.sum(sval[1:] == sval[:-1])) == 52
    assert sid[0] == 236777


def test_softcap_closed_form():
    x = np.array([0.0, 1.0, -1.0, 30.0, 450.0, 451.0, -1e6, 1e-3], np.float32)
    y = O.logit_softcap(x, 30.0)
    want = np.tanh(np.clip(x.astype(np.float64) / 30.0, -15, 15)) * 30.0
    assert np.allclose(y, want, rtol=1e-6, atol=1e-6)
    assert abs(y[4]) <= 30.0 and y[6] == np.float32(np.tanh(-15.0) * 30.0)


# --------------------------------------------------------------------------
# synthetic generator
# --------------------------------------------------------------------------

def test_splitmix64_published_vectors():
    # SplitMix64 seeded with 1234567 (the widely published reference outputs)
    want = [6457827717110365317, 3203168211198807973, 9817491932198370423,
            4593380528125082431, 16408922859458223821]
    assert [O.splitmix64(1234567, i) for i in range(5)] == want
    assert [int(v) for v in O.np_splitmix64(1234567, np.arange(5))] == want


def test_generators_distribution():
    b = O.gen_q4k(0, 20000).reshape(-1, 144)
    d = O.np_f16_to_f32(b[:, 0:2].copy().view(np.uint16)[:, 0]).astype(np.float64)
    dmin = O.np_f16_to_f32(b[:, 2:4].copy().view(np.uint16)[:, 0]).astype(np.float64)
    # |N(0, s)| has mean s*sqrt(2/pi)
    assert abs(d.mean() / (2e-3 * math.sqrt(2 / math.pi)) - 1) < 0.02
    assert abs(dmin.mean() / (1e-3 * math.sqrt(2 / math.pi)) - 1) < 0.02
    sc, m = O.np_q4k_scales(b[:, 4:16])
    assert sc.min() == 0 and sc.max() == 63 and abs(sc.mean() - 31.5) < 0.3
    b6 = O.gen_q6k(0, 20000).reshape(-1, 210)
    s6 = b6[:, 192:208].view(np.int8)
    assert s6.min() == -32 and s6.max() == 31
    x = O.gen_normal_f32(3, 200000)
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1) < 0.01


def test_embedding_lookup_pinned():
    """shaders/embedding_lookup.wgsl:12 pinned two ways: for H = 1536 against one
    rounding of the exact float64 product (11- by 24-bit significands fit in 53
    bits), and for the perfect square H = 256 where sqrt(H) = 16 exactly."""
    rng = np.random.default_rng(7)
    for H in (1536, 256):
        table = (rng.standard_normal((5, H)) * 0.05).astype(np.float16)
        table[3, :4] = [np.inf, -0.0, 6.1e-5, 65504]
        for tok in (0, 3, 4):
            got = O.embedding_lookup(table, H, tok)
            s = np.float32(np.sqrt(np.float64(H)))  # sqrt correctly rounded to f32
            want = (table[tok].astype(np.float64) * np.float64(s)).astype(np.float32)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
            if H == 256:
                assert np.array_equal(got, table[tok].astype(np.float32) * 16)
    # the row index, not the column, selects the token
    t = np.arange(4 * 16, dtype=np.float16).reshape(4, 16)
    assert O.embedding_lookup(t, 16, 2)[0] == 32 * 4


def test_kv_cache_store_layout():
    """shaders/kv_cache_store.wgsl:1-18: row `position` of [max_seq][nkh][hd],
    K and V each rounded once to f16 (the f16 cache of this build; the
    rounding is NumPy's IEEE half cast), every other row untouched."""
    rng = np.random.default_rng(11)
    nkh, hd, cap, pos = 2, 8, 5, 3
    k = rng.standard_normal(nkh * hd).astype(np.float32)
    v = rng.standard_normal(nkh * hd).astype(np.float32) * 1e3
    kc = rng.integers(0, 1 << 16, cap * nkh * hd).astype(np.uint16)
    vc = kc.copy()
    k0, v0 = kc.copy(), vc.copy()
    O.kv_cache_store_f16(k, v, kc, vc, nkh, hd, pos)
    row = slice(pos * nkh * hd, (pos + 1) * nkh * hd)
    assert np.array_equal(kc[row], k.astype(np.float16).view(np.uint16))
    assert np.array_equal(vc[row], v.astype(np.float16).view(np.uint16))
    other = np.ones(kc.size, bool)
    other[row] = False
    assert np.array_equal(kc[other], k0[other]) and np.array_equal(vc[other], v0[other])


def test_node_q4k_dot_matches_oracle(tmp_path):
    """oracle/q4k_dot.js (the CPU baseline's Node dequant-dot) against the C
    oracle's Q4_K matvec on the same seeded blocks."""
    import shutil
    import subprocess
    node = shutil.which("node")
    if node is None:
        pytest.skip("no node binary")
    M, K = 64, 512
    W = O.gen_q4k(21, M * K // 256)
    x = O.gen_normal_f32(22, K)
    fin, fout = tmp_path / "in.bin", tmp_path / "out.bin"
    fin.write_bytes(np.array([M, K], np.uint32).tobytes() + W.tobytes() + x.tobytes())
    js = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle", "q4k_dot.js")
    subprocess.run([node, js, str(fin), str(fout), "0.01"], check=True, capture_output=True, timeout=60)
    y = np.fromfile(fout, np.float32)
    want = O.matmul(x, W, M, K, "q4k")
    assert O.rel_l2(y, want) < 1e-6


# ---- Q5_K and per-layer embeddings ----------------------------------------------

def _q5k_from_q4k(q4: np.ndarray, qh: np.ndarray) -> np.ndarray:
    """The Q5_K block with a Q4_K block's d, dmin, scales and nibbles and the
    given high-bit bytes (layout: d, dmin, 12 scale bytes, qh[32], qs[128])."""
    q4 = q4.reshape(-1, 144)
    out = np.empty((q4.shape[0], 176), np.uint8)
    out[:, :16] = q4[:, :16]
    out[:, 16:48] = qh.reshape(-1, 32)
    out[:, 48:] = q4[:, 16:]
    return out.reshape(-1)


def test_q5k_without_high_bits_is_q4k():
    """qh = 0: the values are those of the Q4_K block with the same scales and
    nibbles (the Q4_K oracle is pinned above against hand-computed blocks and
    the reference's packing)."""
    q4 = O.gen_q4k(77, 64)
    q5 = _q5k_from_q4k(q4, np.zeros(64 * 32, np.uint8))
    assert np.array_equal(O.dequant_q5k(q5).view(np.uint32), O.dequant_q4k(q4).view(np.uint32))


def test_q5k_high_bit_positions():
    """ggml's Q5_K layout (the one src/gguf.ts:235-255 reads): bit 2g of qh[l]
    adds 16 to value 64g + l, bit 2g + 1 to value 64g + 32 + l. With d = 1,
    every scale 1 and every min 0, a single set bit yields a single 16."""
    blk = np.zeros(176, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    blk[4:8] = 1          # sc(0..3) = 1, m(0..3) = 0
    blk[12:16] = 1        # sc(4..7) = s[8..11] & 15 = 1, m(4..7) = s[8..11] >> 4 = 0
    seen = set()
    for l in range(32):
        for bit in range(8):
            b = blk.copy()
            b[16 + l] = 1 << bit
            v = O.dequant_q5k(b)
            nz = np.flatnonzero(v)
            want = 64 * (bit // 2) + 32 * (bit % 2) + l
            assert nz.tolist() == [want] and v[want] == 16.0, (l, bit)
            seen.add(want)
    assert seen == set(range(256))


def test_q5k_f64_single_rounding():
    """d*sc*q - dmin*m evaluated once in f64 and stored as f32 equals the
    correctly rounded f32 of the exact rational value (fractions), on random
    blocks with d and dmin over the whole f16 range."""
    from fractions import Fraction
    rng = np.random.default_rng(13)
    blk = rng.integers(0, 256, (24, 176), dtype=np.uint8)
    d = np.abs(rng.standard_normal(24) * 10.0 ** rng.integers(-6, 3, 24)).astype(np.float16)
    dm = np.abs(rng.standard_normal(24) * 10.0 ** rng.integers(-6, 3, 24)).astype(np.float16)
    blk[:, 0:2] = d.view(np.uint8).reshape(24, 2)
    blk[:, 2:4] = dm.view(np.uint8).reshape(24, 2)
    got = O.dequant_q5k(blk.reshape(-1)).reshape(24, 256)
    for b in range(24):
        s = bytes(blk[b, 4:16])
        for t in range(0, 256, 7):
            g, hi, l = t // 64, (t // 32) % 2, t % 32
            j = 2 * g + hi
            sc, m = O.q4k_scale_min(s, j)
            q = (blk[b, 48 + 32 * g + l] >> (4 * hi)) & 15
            q += 16 * ((blk[b, 16 + l] >> j) & 1)
            exact = Fraction(float(d[b])) * sc * int(q) - Fraction(float(dm[b])) * m
            assert got[b, t] == np.float32(float(exact)), (b, t)


def _tiny_gemma4(eps):
    import torch
    from transformers.models.gemma4.configuration_gemma4 import Gemma4TextConfig
    from transformers.models.gemma4.modeling_gemma4 import Gemma4TextDecoderLayer, Gemma4TextModel

    cfg = Gemma4TextConfig(vocab_size=64, hidden_size=32, intermediate_size=64, num_hidden_layers=3,
                           num_attention_heads=2, num_key_value_heads=1, head_dim=16, hidden_size_per_layer_input=16,
                           vocab_size_per_layer_input=64, rms_norm_eps=eps)
    torch.manual_seed(0)
    return cfg, Gemma4TextModel(cfg).double(), Gemma4TextDecoderLayer(cfg, 0).double()


def test_ple_stage1_against_transformers():
    """Gemma4TextModel.get_per_layer_inputs + project_per_layer_inputs (the
    token row x sqrt(D), the projection, its RMSNorm, the 1/sqrt(2) blend)
    against the oracle's stage 1 on the same f16 weights. transformers also
    scales the projection by 1/sqrt(H) before the norm, which the reference
    does not: with eps = 0 the norm removes that factor."""
    import torch
    cfg, m, _ = _tiny_gemma4(0.0)
    L, D, H, V = 3, 16, 32, 64
    rng = np.random.default_rng(14)
    proj16 = (rng.standard_normal((L * D, H)) * 0.2).astype(np.float16)
    norm16 = (rng.standard_normal(D) * 0.1 + 1).astype(np.float16)
    table16 = (rng.standard_normal((V, L * D)) * 0.5).astype(np.float16)
    x0 = rng.standard_normal(H).astype(np.float32)
    tok = 37
    with torch.no_grad():
        m.per_layer_model_projection.weight.copy_(torch.from_numpy(proj16.astype(np.float64)))
        m.per_layer_projection_norm.weight.copy_(torch.from_numpy(norm16.astype(np.float64)))
        m.embed_tokens_per_layer.weight.copy_(torch.from_numpy(table16.astype(np.float64)))
        ids = torch.tensor([[tok]])
        pli = m.get_per_layer_inputs(ids, None)
        want = m.project_per_layer_inputs(torch.from_numpy(x0.astype(np.float64))[None, None], pli)
    want = want.numpy().reshape(-1)
    got = O.ple_project(x0, proj16.view(np.uint16), norm16.view(np.uint16), table16[tok].view(np.uint16), L, D, 0.0)
    assert np.allclose(got, want, rtol=1e-5, atol=1e-6), np.abs(got - want).max()


def test_ple_layer_tail_against_transformers():
    """Gemma4TextDecoderLayer.forward with its attention and MLP returning
    zeros (so the residual passes through both, as their norms of zero are
    zero) runs transformers' per-layer-input tail on the input: gate, tanh
    GELU, x per-layer input, projection, RMSNorm, residual add, x layer
    scalar. The oracle's stage 2 must give the same on the same weights."""
    import torch
    cfg, _, lay = _tiny_gemma4(1e-6)

    class Zero(torch.nn.Module):
        def forward(self, hidden_states=None, *a, **k):
            z = torch.zeros_like(hidden_states)
            return (z, None) if k or a else z

    lay.self_attn = Zero()
    lay.mlp = Zero()
    D, H = 16, 32
    rng = np.random.default_rng(15)
    gate16 = (rng.standard_normal((D, H)) * 0.3).astype(np.float16)
    proj16 = (rng.standard_normal((H, D)) * 0.3).astype(np.float16)
    post16 = (rng.standard_normal(H) * 0.1 + 1).astype(np.float16)
    scale16 = np.float16(0.75)
    x = rng.standard_normal(H).astype(np.float32) * 2
    ple = rng.standard_normal(D).astype(np.float32)
    with torch.no_grad():
        lay.per_layer_input_gate.weight.copy_(torch.from_numpy(gate16.astype(np.float64)))
        lay.per_layer_projection.weight.copy_(torch.from_numpy(proj16.astype(np.float64)))
        lay.post_per_layer_input_norm.weight.copy_(torch.from_numpy(post16.astype(np.float64)))
        lay.layer_scalar.copy_(torch.tensor([float(scale16)], dtype=torch.float64))
        want = lay(torch.from_numpy(x.astype(np.float64))[None, None],
                   per_layer_input=torch.from_numpy(ple.astype(np.float64))[None, None]).numpy().reshape(-1)
    got = O.ple_layer_tail(x, gate16.view(np.uint16), proj16.view(np.uint16), post16.view(np.uint16),
                           int(scale16.view(np.uint16)), ple, 1e-6)
    assert np.allclose(got, want, rtol=1e-5, atol=1e-6), np.abs(got - want).max()


def test_ple_stage1_closed_forms():
    """Per-layer slices: a layer's output depends on its own projection slice
    and table slice only; projection zero leaves table * sqrt(D) / sqrt(2);
    with eps 0 a constant slice c normalises to sign(c) * w."""
    L, D = 4, 256
    rng = np.random.default_rng(16)
    w = (rng.standard_normal(D) * 0.1 + 1).astype(np.float16).view(np.uint16)
    row = (rng.standard_normal(L * D) * 0.5).astype(np.float16)
    out = O.ple_stage1(np.zeros(L * D, np.float32), w, row.view(np.uint16), L, D, 1e-6)
    assert np.allclose(out, row.astype(np.float64) * 16 / np.sqrt(2), rtol=1e-6)
    p = np.repeat(np.array([3.0, -0.5, 7.0, -2.0], np.float32), D)
    out = O.ple_stage1(p, w, np.zeros(L * D, np.uint16), L, D, 0.0)
    wf = w.view(np.float16).astype(np.float64)
    for l, sgn in enumerate((1, -1, 1, -1)):
        assert np.allclose(out[l * D:(l + 1) * D], sgn * wf / np.sqrt(2), rtol=1e-6)
    perm = [2, 0, 3, 1]
    pr = rng.standard_normal(L * D).astype(np.float32)
    a = O.ple_stage1(pr, w, row.view(np.uint16), L, D, 1e-6).reshape(L, D)
    b = O.ple_stage1(pr.reshape(L, D)[perm].reshape(-1), w, row.reshape(L, D)[perm].reshape(-1).view(np.uint16), L,
                     D, 1e-6).reshape(L, D)
    assert np.array_equal(a[perm], b)


def test_ple_gelu_mul_and_skip_scale_add():
    rng = np.random.default_rng(17)
    g = rng.standard_normal(256).astype(np.float32)
    ple = rng.standard_normal(3 * 256).astype(np.float32)
    assert np.array_equal(O.ple_gelu_mul(g, ple, 256), O.gelu_mul(g, ple[256:512]))
    h, n = rng.standard_normal(64).astype(np.float32), rng.standard_normal(64).astype(np.float32)
    assert np.array_equal(O.ple_skip_scale_add(h, n, f16(1.0)), (h.astype(np.float64) + n).astype(np.float32))
    assert np.array_equal(O.ple_skip_scale_add(h, n, f16(2.0)), (2 * (h.astype(np.float64) + n)).astype(np.float32))
    assert not np.any(O.ple_skip_scale_add(h, n, f16(0.0)))


def test_q8_0_known_answers():
    """src/gguf.ts:115-131: q * d per 32-value block; known blocks, and the
    int8 sign of every byte value."""
    blk = np.zeros(2 * 34, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)
    blk[2:34] = np.arange(-16, 16, dtype=np.int8).view(np.uint8)
    blk[34:36] = np.frombuffer(np.float16(-3.0).tobytes(), np.uint8)
    blk[36:68] = np.array([-128, 127, 0, 1] * 8, np.int8).view(np.uint8)
    v = O.dequant_q8_0(blk)
    assert np.array_equal(v[:32], np.arange(-16, 16) * 0.5)
    assert np.array_equal(v[32:], np.array([384.0, -381.0, 0.0, -3.0] * 8, np.float32))
    # every q with d = 1: the value is the signed byte
    blocks = np.zeros((8, 34), np.uint8)
    blocks[:, 0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    blocks[:, 2:] = np.arange(256, dtype=np.uint8).reshape(8, 32)
    assert np.array_equal(O.dequant_q8_0(blocks.reshape(-1)), np.arange(256, dtype=np.uint8).view(np.int8))


def test_dequant_f16_rows_per_type():
    """The f16 rows of every tensor type, against the pinned dequants and
    NumPy's IEEE half: F16 unchanged, BF16 through its f32 high half."""
    rng = np.random.default_rng(40)
    f32 = rng.standard_normal(64).astype(np.float32)
    assert np.array_equal(O.dequant_f16_rows(f32.view(np.uint8), 0), f32.astype(np.float16).view(np.uint16))
    h = rng.standard_normal(64).astype(np.float16)
    assert np.array_equal(O.dequant_f16_rows(h.view(np.uint8), 1), h.view(np.uint16))
    bf = (f32.view(np.uint32) >> 16).astype(np.uint16)
    want = (bf.astype(np.uint32) << 16).view(np.float32).astype(np.float16).view(np.uint16)
    assert np.array_equal(O.dequant_f16_rows(bf.view(np.uint8), 30), want)
    q4 = O.gen_q4k(41, 4)
    assert np.array_equal(O.dequant_f16_rows(q4, 12), O.dequant_q4k(q4).astype(np.float16).view(np.uint16))
