"""Seeded K-quant weights shaped like a real model's, for parity tests.

The benchmark's generator (oracle gen_q4k / gen_q6k) draws Q4_K mins
independently of the scales, so its weights have a mean near +0.35 and a
matvec's output scales with the sum of its input; Q6_K scales stay in
[-32, 31]. Real GGUF tensors are near zero-mean (a Q4_K sub-block's min
offsets its codes' middle) and Q6_K scales use the whole int8 range. These
generators produce such blocks (numpy, from the block layouts of
src/gguf.ts:157-210 and :316-368)."""
import numpy as np


def _pack_q4k_scales(sc, m):
    s = np.zeros((sc.shape[0], 12), np.int32)
    s[:, 0:4] = sc[:, 0:4] & 63
    s[:, 4:8] = m[:, 0:4] & 63
    s[:, 8:12] = (sc[:, 4:8] & 15) | ((m[:, 4:8] & 15) << 4)
    s[:, 0:4] |= (sc[:, 4:8] >> 4) << 6
    s[:, 4:8] |= (m[:, 4:8] >> 4) << 6
    return s.astype(np.uint8)


def q4k_centered(seed, nblocks, d_std=2e-3):
    """Q4_K blocks with dmin = 7.5 d and min index = scale index, so each
    sub-block's values are d * sc * (q - 7.5): zero-mean, as in real weights."""
    rng = np.random.default_rng(seed)
    b = np.zeros((nblocks, 144), np.uint8)
    d = np.abs(rng.standard_normal(nblocks) * d_std).astype(np.float16)
    dmin = (d.astype(np.float32) * 7.5).astype(np.float16)
    sc = rng.integers(0, 64, (nblocks, 8))
    b[:, 0:2] = d.view(np.uint16).reshape(-1, 1).view(np.uint8)
    b[:, 2:4] = dmin.view(np.uint16).reshape(-1, 1).view(np.uint8)
    b[:, 4:16] = _pack_q4k_scales(sc, sc)
    b[:, 16:] = rng.integers(0, 256, (nblocks, 128), dtype=np.uint8)
    return b.reshape(-1)


def q6k_wide(seed, nblocks, d_std=5e-4):
    """Q6_K blocks with int8 scales uniform over -128..127 (so |sc * (q - 32)|
    reaches 4096, past the 2048 below which an f16 holds every integer)."""
    rng = np.random.default_rng(seed)
    b = rng.integers(0, 256, (nblocks, 210), dtype=np.uint8)
    b[:, 192:208] = rng.integers(-128, 128, (nblocks, 16)).astype(np.int8).view(np.uint8)
    d = np.abs(rng.standard_normal(nblocks) * d_std).astype(np.float16)
    b[:, 208:210] = d.view(np.uint16).reshape(-1, 1).view(np.uint8)
    return b.reshape(-1)


def make_realistic(dec, seed=900):
    """Replaces a decoder's projection weights (and LM head) with centered
    Q4_K and full-range Q6_K blocks of the same shapes."""
    s = dec.s
    k = 0
    for L in dec.layers:
        for name, M, N in (("wq", s.q_dim, s.hidden), ("wk", s.kv_dim, s.hidden), ("wv", s.kv_dim, s.hidden),
                           ("wo", s.hidden, s.q_dim), ("wgate", s.ffn, s.hidden), ("wup", s.ffn, s.hidden)):
            getattr(L, name).upload(q4k_centered(seed + k, M * N // 256))
            k += 1
        L.wdown.upload(q6k_wide(seed + k, s.hidden * s.ffn // 256))
        k += 1
    if dec.lm_head is not None:
        dec.lm_head.upload(q6k_wide(seed + k, s.vocab * s.hidden // 256))
