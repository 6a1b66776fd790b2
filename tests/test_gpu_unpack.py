"""GPU parity of the hot path's own Q4_K / Q6_K unpack (bit-exact).

`g4_dequantPath` forms the reference's dequantized values
(GGUFParser.dequantizeQ4_K / dequantizeQ6_K, src/gguf.ts:168-210 / :323-368)
from the codes, scales, mins and d exactly as each kernel family extracts
them: path 0 the one-vector matvec's register units (buffer loads, byte
shifts of the 2-byte aligned Q6_K runs), path 1 the units read from blocks
staged in LDS (tile-walking matvec, 2-8 vector matvec), path 2 the
matrix-core operands of the M >= 16 matmul. The blocks cover every 6-bit
scale/min value at every sub-block position, every int8 Q6_K scale at every
position, both Q6_K block alignments, and d/dmin edge values (zero,
subnormal, negative, largest, Inf, NaN)."""
import struct

import numpy as np
import pytest

import oracle as O
from gpu_util import bits_equal

pytestmark = pytest.mark.gpu

F16_EDGES = [0x0000, 0x8000, 0x0001, 0x03ff, 0x0400, 0x7bff, 0xfbff, 0x3c00, 0xbc00, 0x7c00, 0x7e00, 0x3555]


def pack_q4k_scales_np(sc, m):
    """Vectorised inverse of the 12-byte scale/min packing (src/gguf.ts:175-182),
    written from the layout description: [n, 8] scales and mins -> [n, 12]."""
    sc = sc.astype(np.int32)
    m = m.astype(np.int32)
    s = np.zeros((sc.shape[0], 12), np.int32)
    s[:, 0:4] = sc[:, 0:4] & 63
    s[:, 4:8] = m[:, 0:4] & 63
    s[:, 8:12] = (sc[:, 4:8] & 15) | ((m[:, 4:8] & 15) << 4)
    s[:, 0:4] |= (sc[:, 4:8] >> 4) << 6
    s[:, 4:8] |= (m[:, 4:8] >> 4) << 6
    return s.astype(np.uint8)


def q4k_all_scale_blocks(seed=5):
    """8 x 64 x 64 blocks: sub-block j carries every (scale, min) pair, the
    other sub-blocks random values; d and dmin cycle through the f16 edge
    values on some blocks and are random halves elsewhere; qs random."""
    rng = np.random.default_rng(seed)
    n = 8 * 64 * 64
    sc = rng.integers(0, 64, (n, 8))
    m = rng.integers(0, 64, (n, 8))
    idx = np.arange(n)
    j, v, w = idx // 4096, (idx // 64) % 64, idx % 64
    sc[idx, j] = v
    m[idx, j] = w
    b = np.zeros((n, 144), np.uint8)
    d = (np.abs(rng.standard_normal(n)) * 2e-3).astype(np.float16).view(np.uint16)
    dmin = (np.abs(rng.standard_normal(n)) * 1e-3).astype(np.float16).view(np.uint16)
    d[::7] = np.array(F16_EDGES, np.uint16)[(idx[::7] // 7) % len(F16_EDGES)]
    dmin[::11] = np.array(F16_EDGES, np.uint16)[(idx[::11] // 11) % len(F16_EDGES)]
    b[:, 0:2] = d.reshape(-1, 1).view(np.uint8)
    b[:, 2:4] = dmin.reshape(-1, 1).view(np.uint8)
    b[:, 4:16] = pack_q4k_scales_np(sc, m)
    b[:, 16:] = rng.integers(0, 256, (n, 128), dtype=np.uint8)
    return b.reshape(-1), n


def q6k_wide_blocks(seed=6, n=4099):
    """Q6_K blocks whose int8 scales take every value -128..127 at every one of
    the 16 positions (the range real GGUF scales use), random codes, d random
    with f16 edge values on some blocks; n odd so both 4-byte alignments of a
    210-byte block occur and the last block ends off a dword."""
    rng = np.random.default_rng(seed)
    b = O.gen_q6k(seed, n).reshape(n, 210).copy()
    sc = ((np.arange(n)[:, None] * 7 + np.arange(16)[None, :] * 37) % 256 - 128).astype(np.int8)
    b[:, 192:208] = sc.view(np.uint8)
    b[:, :192] = rng.integers(0, 256, (n, 192), dtype=np.uint8)
    d = (np.abs(rng.standard_normal(n)) * 2e-3).astype(np.float16).view(np.uint16)
    d[::5] = np.array(F16_EDGES, np.uint16)[(np.arange(n)[::5] // 5) % len(F16_EDGES)]
    b[:, 208:210] = d.reshape(-1, 1).view(np.uint8)
    return b.reshape(-1), n


def _path(ctx, wtype, path, blocks, n):
    db = ctx.from_numpy(blocks)
    out = ctx.empty(n * 256, np.float32)
    ctx.dequantPath(wtype, path, db, n, out)
    got = out.download(np.float32)
    db.free()
    out.free()
    return got


def test_q4k_scale_patterns_cover_every_pair():
    b, n = q4k_all_scale_blocks()
    sc, m = O.np_q4k_scales(b.reshape(n, 144)[:, 4:16])
    for j in range(8):
        pairs = set(zip(sc[j * 4096:(j + 1) * 4096, j].tolist(), m[j * 4096:(j + 1) * 4096, j].tolist()))
        assert len(pairs) == 4096


@pytest.mark.parametrize("path", [0, 1, 2])
def test_q4k_unpack_paths_bit_exact(ctx, path):
    b, n = q4k_all_scale_blocks()
    print(f"[unpack] q4k path {path}: {n} blocks", flush=True)
    assert bits_equal(_path(ctx, "q4k", path, b, n), O.dequant_q4k(b))


@pytest.mark.parametrize("path", [0, 1])
def test_q6k_unpack_paths_bit_exact(ctx, path):
    b, n = q6k_wide_blocks()
    assert set(b.reshape(n, 210)[:, 192:208].view(np.int8).reshape(-1).tolist()) == set(range(-128, 128))
    print(f"[unpack] q6k path {path}: {n} blocks", flush=True)
    assert bits_equal(_path(ctx, "q6k", path, b, n), O.dequant_q6k(b))


def test_q6k_matrix_core_operand(ctx):
    """The MFMA operand is sc * (q - 32) rounded once to f16: bit-exact
    against that rounding of the oracle's integer product (the oracle's
    dequant with d = 1 gives it exactly), and so equal to the reference
    value wherever |sc * (q - 32)| <= 2048 (every block with |sc| <= 64)."""
    b, n = q6k_wide_blocks()
    got = _path(ctx, "q6k", 2, b, n)
    one = b.reshape(n, 210).copy()
    one[:, 208:210] = np.frombuffer(struct.pack("<H", 0x3C00), np.uint8)
    prod = O.dequant_q6k(one.reshape(-1)).reshape(n, 256)            # exact integers
    assert np.array_equal(prod, np.round(prod)) and np.max(np.abs(prod)) == 128 * 32
    d = O.np_f16_to_f32(b.reshape(n, 210)[:, 208:210].copy().view(np.uint16)[:, 0]).astype(np.float64)
    want = (d[:, None] * prod.astype(np.float16).astype(np.float64)).astype(np.float32)   # exact product
    assert bits_equal(got, want.reshape(-1))
    ref = O.dequant_q6k(b).reshape(n, 256)
    small = np.abs(prod) <= 2048
    g = got.reshape(n, 256)
    assert bits_equal(g[small], ref[small])
    # where the rounding applies it is within half an f16 ulp of 4096 (2^-12 relative)
    fin = ~small & np.isfinite(ref) & (ref != 0)
    assert np.all(np.abs(g[fin].astype(np.float64) / ref[fin] - 1) <= 2.0 ** -11)


def test_dequant_exports_are_path0(ctx):
    """g4_dequant_q4k / q6k run the register units (path 0)."""
    b, n = q6k_wide_blocks(n=257)
    db = ctx.from_numpy(b)
    out = ctx.empty(n * 256, np.float32)
    ctx.dequant_q6k(db, n, out)
    assert bits_equal(out.download(np.float32), _path(ctx, "q6k", 0, b, n))
