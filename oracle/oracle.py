"""CPU oracle for the gemma4 decode hot path — TEST INFRASTRUCTURE ONLY.

Two independent restatements of the reference algorithm live here:

* ``C``: ctypes bindings to ``libg4oracle.so`` (built from ``g4_oracle.c``),
  the primary oracle, f64 accumulation;
* ``np_*``: vectorised numpy restatements written from the reference's byte
  layouts and shader bodies, used to cross-check the C code.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` import this module; the product library never does.

Reference citations are relative to the reference repository root.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libg4oracle.so")

Q4K_BLOCK_BYTES = 144
Q6K_BLOCK_BYTES = 210
Q5K_BLOCK_BYTES = 176
QK = 256


def build() -> str:
    """Compile the C oracle with its Makefile (gcc, no fast-math)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


_P = ctypes.c_void_p
_U32 = ctypes.c_uint32
_U64 = ctypes.c_uint64
_F = ctypes.c_float
_SZ = ctypes.c_size_t


def _declare(L):
    sig = {
        "g4o_f16_to_f32": (_F, [ctypes.c_uint16]),
        "g4o_f32_to_f16_rne": (ctypes.c_uint16, [_F]),
        "g4o_f32_to_f16_trunc": (ctypes.c_uint16, [_F]),
        "g4o_q4k_scale_min": (None, [_P, ctypes.c_int, _P, _P]),
        "g4o_dequant_q4k": (None, [_P, _SZ, _P]),
        "g4o_dequant_q6k": (None, [_P, _SZ, _P]),
        "g4o_dequant_q5k": (None, [_P, _SZ, _P]),
        "g4o_dequant_q8_0": (None, [_P, _SZ, _P]),
        "g4o_ple_stage1": (None, [_P, _P, _P, _P, _U32, _U32, _F]),
        "g4o_ple_skip_scale_add": (None, [_P, _P, ctypes.c_uint16, _U32]),
        "g4o_matmul_f16w": (None, [_P, _P, _P, _U32, _U32]),
        "g4o_matmul_q4k": (None, [_P, _P, _P, _U32, _U32]),
        "g4o_matmul_q6k": (None, [_P, _P, _P, _U32, _U32]),
        "g4o_rms_norm": (None, [_P, _P, _P, _U32, _F]),
        "g4o_fused_norm_add": (None, [_P, _P, _P, _P, _U32, _F]),
        "g4o_gelu_mul": (None, [_P, _P, _P, _U32]),
        "g4o_per_head_rms_norm_no_weight": (None, [_P, _U32, _U32, _F]),
        "g4o_rope_freq": (None, [_F, _U32, _U32, ctypes.c_int, _P, _P]),
        "g4o_fused_per_head_norm_rope": (None, [_P, _P, _U32, _U32, _F, _U32, _F, _U32, _P]),
        "g4o_kv_cache_store_f16": (None, [_P, _P, _P, _P, _U32, _U32, _U32]),
        "g4o_attn_score": (None, [_P, _P, _P, _U32, _U32, _U32, _U32, _F, _U32]),
        "g4o_softmax": (None, [_P, _U32, _U32]),
        "g4o_attn_output": (None, [_P, _P, _P, _U32, _U32, _U32, _U32]),
        "g4o_attention": (None, [_P, _P, _P, _P, _U32, _U32, _U32, _U32, _F, _U32]),
        "g4o_attention_paged": (None, [_P, _P, _P, _P, _U32, _P, _U32, _U32, _U32, _U32, _F, _U32]),
        "g4o_logit_softcap": (None, [_P, _U32, _F]),
        "g4o_argmax": (_U32, [_P, _U32]),
        "g4o_topk256": (None, [_P, _U32, _P]),
        "g4o_topk_sort": (None, [_P, _P, _P]),
        "g4o_splitmix64": (_U64, [_U64, _U64]),
        "g4o_gen_q4k": (None, [_U64, _U64, _P]),
        "g4o_gen_q6k": (None, [_U64, _U64, _P]),
        "g4o_gen_normal_f32": (None, [_U64, _U64, _F, _F, _P]),
        "g4o_gen_normal_f16": (None, [_U64, _U64, _F, _F, _P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle buffers must be C-contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# --------------------------------------------------------------------------
# C oracle wrappers (numpy in, numpy out)
# --------------------------------------------------------------------------

def f16_to_f32(h: int) -> float:
    return lib().g4o_f16_to_f32(int(h))


def f32_to_f16_rne(f: float) -> int:
    return lib().g4o_f32_to_f16_rne(float(f))


def f32_to_f16_trunc(f: float) -> int:
    return lib().g4o_f32_to_f16_trunc(float(f))


def q4k_scale_min(scales12: bytes, j: int):
    s = _c(np.frombuffer(bytes(scales12), dtype=np.uint8), np.uint8)
    sc = ctypes.c_int()
    m = ctypes.c_int()
    lib().g4o_q4k_scale_min(_p(s), j, ctypes.byref(sc), ctypes.byref(m))
    return sc.value, m.value


def dequant_q4k(blocks: np.ndarray) -> np.ndarray:
    b = _c(blocks, np.uint8).reshape(-1)
    assert b.size % Q4K_BLOCK_BYTES == 0
    n = b.size // Q4K_BLOCK_BYTES
    out = np.empty(n * QK, np.float32)
    lib().g4o_dequant_q4k(_p(b), n, _p(out))
    return out


def dequant_q6k(blocks: np.ndarray) -> np.ndarray:
    b = _c(blocks, np.uint8).reshape(-1)
    assert b.size % Q6K_BLOCK_BYTES == 0
    n = b.size // Q6K_BLOCK_BYTES
    out = np.empty(n * QK, np.float32)
    lib().g4o_dequant_q6k(_p(b), n, _p(out))
    return out


def dequant_q5k(blocks: np.ndarray) -> np.ndarray:
    b = _c(blocks, np.uint8).reshape(-1)
    assert b.size % Q5K_BLOCK_BYTES == 0
    n = b.size // Q5K_BLOCK_BYTES
    out = np.empty(n * QK, np.float32)
    lib().g4o_dequant_q5k(_p(b), n, _p(out))
    return out


def dequant_q8_0(blocks: np.ndarray) -> np.ndarray:
    b = _c(blocks, np.uint8).reshape(-1)
    assert b.size % 34 == 0
    n = b.size // 34
    out = np.empty(n * 32, np.float32)
    lib().g4o_dequant_q8_0(_p(b), n, _p(out))
    return out


def dequant_f16_rows(raw: np.ndarray, ggml_type: int) -> np.ndarray:
    """A GGUF tensor's values as the reference uploads them (tensorToF16,
    src/engine.ts:570-579): dequantized to f32 (src/gguf.ts:370-381), then
    f16 bits rounded to nearest even (the Float16Array path)."""
    raw = _c(raw, np.uint8).reshape(-1)
    if ggml_type == 0:
        f = raw.view(np.float32)
    elif ggml_type == 1:
        return raw.view(np.uint16).copy()
    elif ggml_type == 30:
        f = (raw.view(np.uint16).astype(np.uint32) << 16).view(np.float32)
    elif ggml_type == 8:
        f = dequant_q8_0(raw)
    elif ggml_type == 12:
        f = dequant_q4k(raw)
    elif ggml_type == 13:
        f = dequant_q5k(raw)
    elif ggml_type == 14:
        f = dequant_q6k(raw)
    else:
        raise ValueError(f"tensor type {ggml_type}")
    with np.errstate(over="ignore", invalid="ignore"):
        return f.astype(np.float16).view(np.uint16)


def matmul(x: np.ndarray, W: np.ndarray, M: int, N: int, wtype: str) -> np.ndarray:
    """y[M] = W[M, N] . x[N] for wtype in {'f16', 'q4k', 'q6k'}."""
    x = _c(x, np.float32)
    y = np.empty(M, np.float32)
    if wtype == "f16":
        W = _c(W, np.uint16)
        lib().g4o_matmul_f16w(_p(x), _p(W), _p(y), M, N)
    elif wtype == "q4k":
        W = _c(W, np.uint8)
        assert W.size == M * (N // QK) * Q4K_BLOCK_BYTES
        lib().g4o_matmul_q4k(_p(x), _p(W), _p(y), M, N)
    elif wtype == "q6k":
        W = _c(W, np.uint8)
        assert W.size == M * (N // QK) * Q6K_BLOCK_BYTES
        lib().g4o_matmul_q6k(_p(x), _p(W), _p(y), M, N)
    else:
        raise ValueError(wtype)
    return y


def rms_norm(x, w_f16, eps=1e-6):
    x = _c(x, np.float32)
    w = _c(w_f16, np.uint16)
    out = np.empty_like(x)
    lib().g4o_rms_norm(_p(x), _p(w), _p(out), x.size, eps)
    return out


def fused_norm_add(x, w_f16, residual, eps=1e-6):
    x = _c(x, np.float32)
    w = _c(w_f16, np.uint16)
    r = _c(residual, np.float32)
    out = np.empty_like(x)
    lib().g4o_fused_norm_add(_p(x), _p(w), _p(r), _p(out), x.size, eps)
    return out


def gelu_mul(gate, up):
    g = _c(gate, np.float32)
    u = _c(up, np.float32)
    out = np.empty_like(g)
    lib().g4o_gelu_mul(_p(g), _p(u), _p(out), g.size)
    return out


def ple_stage1(projected, norm_w_f16, embed_row_f16, num_layers, dim, eps=1e-6):
    """shaders/ple_stage1_fuse.wgsl for every layer of one token."""
    p = _c(projected, np.float32)
    w = _c(norm_w_f16, np.uint16)
    e = _c(embed_row_f16, np.uint16)
    assert p.size == e.size == num_layers * dim and w.size == dim
    out = np.empty(num_layers * dim, np.float32)
    lib().g4o_ple_stage1(_p(p), _p(w), _p(e), _p(out), num_layers, dim, eps)
    return out


def ple_gelu_mul(gate, ple_inputs, layer_offset):
    """shaders/ple_gelu_mul.wgsl: gelu(gate[i]) * ple_inputs[layer_offset + i]
    (the GELU of gelu_mul)."""
    g = _c(gate, np.float32)
    return gelu_mul(g, _c(ple_inputs, np.float32)[layer_offset:layer_offset + g.size])


def ple_skip_scale_add(hidden, post_normed, scale_f16):
    h = _c(hidden, np.float32).copy()
    n = _c(post_normed, np.float32)
    lib().g4o_ple_skip_scale_add(_p(h), _p(n), int(scale_f16), h.size)
    return h


def ple_project(x0, model_proj_f16, proj_norm_f16, row_f16, num_layers, dim, eps=1e-6):
    """PLE stage 1 for one token (src/engine.ts:1516-1535): the f16
    per_layer_model_proj [L*D x H] times the step's input vector, then
    shaders/ple_stage1_fuse.wgsl per layer with the token's table row (f16)."""
    x0 = _c(x0, np.float32)
    proj = matmul(x0, model_proj_f16, num_layers * dim, x0.size, "f16")
    return ple_stage1(proj, proj_norm_f16, row_f16, num_layers, dim, eps)


def ple_layer_tail(x, gate_f16, proj_f16, post_norm_f16, scale_f16, ple_slice, eps=1e-6):
    """PLE stage 2 of one layer (src/engine.ts:1608-1616): inp_gate,
    gelu * ple_inputs slice, proj, rmsNorm, skip-scale-add."""
    x = _c(x, np.float32)
    D, H = _c(ple_slice, np.float32).size, x.size
    g = matmul(x, gate_f16, D, H, "f16")
    po = matmul(gelu_mul(g, ple_slice), proj_f16, H, D, "f16")
    return ple_skip_scale_add(x, rms_norm(po, post_norm_f16, eps), scale_f16)


def per_head_rms_norm_no_weight(data, num_heads, head_dim, eps=1e-6):
    d = _c(data, np.float32).copy()
    lib().g4o_per_head_rms_norm_no_weight(_p(d), num_heads, head_dim, eps)
    return d


def rope_freq(theta, i, head_dim, apply_divisor, rope_freqs_f16):
    rf = _c(rope_freqs_f16, np.uint16)
    out = ctypes.c_float()
    lib().g4o_rope_freq(theta, i, head_dim, int(apply_divisor), _p(rf), ctypes.byref(out))
    return out.value


def fused_per_head_norm_rope(data, w_f16, num_heads, head_dim, eps, position, theta,
                             apply_divisor, rope_freqs_f16):
    d = _c(data, np.float32).copy()
    w = _c(w_f16, np.uint16)
    rf = _c(rope_freqs_f16, np.uint16)
    lib().g4o_fused_per_head_norm_rope(_p(d), _p(w), num_heads, head_dim, eps, position,
                                       theta, int(apply_divisor), _p(rf))
    return d


def kv_cache_store_f16(k_in, v_in, k_cache, v_cache, num_kv_heads, head_dim, position):
    k_in = _c(k_in, np.float32)
    v_in = _c(v_in, np.float32)
    assert k_cache.dtype == np.uint16 and v_cache.dtype == np.uint16
    lib().g4o_kv_cache_store_f16(_p(k_in), _p(v_in), _p(k_cache), _p(v_cache), num_kv_heads,
                                 head_dim, position)


def attn_score(q, k_cache, nqh, nkh, hd, seq_len, scale=1.0, window=0):
    q = _c(q, np.float32)
    kc = _c(k_cache, np.uint16)
    out = np.empty(nqh * seq_len, np.float32)
    lib().g4o_attn_score(_p(q), _p(kc), _p(out), nqh, nkh, hd, seq_len, scale, window)
    return out


def softmax(scores, num_heads, seq_len):
    s = _c(scores, np.float32).copy()
    lib().g4o_softmax(_p(s), num_heads, seq_len)
    return s


def attn_output(probs, v_cache, nqh, nkh, hd, seq_len):
    p = _c(probs, np.float32)
    vc = _c(v_cache, np.uint16)
    out = np.empty(nqh * hd, np.float32)
    lib().g4o_attn_output(_p(p), _p(vc), _p(out), nqh, nkh, hd, seq_len)
    return out


def attention(q, k_cache, v_cache, nqh, nkh, hd, seq_len, scale=1.0, window=0):
    q = _c(q, np.float32)
    kc = _c(k_cache, np.uint16)
    vc = _c(v_cache, np.uint16)
    out = np.empty(nqh * hd, np.float32)
    lib().g4o_attention(_p(q), _p(kc), _p(vc), _p(out), nqh, nkh, hd, seq_len, scale, window)
    return out


def attention_paged(q, k_pool, v_pool, page_table, page_size, nqh, nkh, hd, seq_len,
                    scale=1.0, window=0):
    q = _c(q, np.float32)
    kp = _c(k_pool, np.uint16)
    vp = _c(v_pool, np.uint16)
    pt = _c(page_table, np.int32)
    out = np.empty(nqh * hd, np.float32)
    lib().g4o_attention_paged(_p(q), _p(kp), _p(vp), _p(pt), page_size, _p(out), nqh, nkh, hd,
                              seq_len, scale, window)
    return out


def embedding_lookup(table_f16, hidden_size, token_id):
    """shaders/embedding_lookup.wgsl:9-13: f32(table[token_id * H + i]) * sqrt(f32(H)).

    Pinned in tests against a float64 product rounded once to f32 (exact here:
    an 11-bit by 24-bit significand product fits in 53 bits) and against
    perfect-square H, where sqrt(H) is exact and each output is f16 * integer.
    """
    t = np.ascontiguousarray(table_f16, dtype=np.float16).reshape(-1, hidden_size)
    return t[token_id].astype(np.float32) * np.sqrt(np.float32(hidden_size))


def logit_softcap(logits, cap=30.0):
    x = _c(logits, np.float32).copy()
    lib().g4o_logit_softcap(_p(x), x.size, cap)
    return x


def argmax(logits) -> int:
    x = _c(logits, np.float32)
    return int(lib().g4o_argmax(_p(x), x.size))


def topk256(logits) -> np.ndarray:
    x = _c(logits, np.float32)
    out = np.empty(512, np.float32)
    lib().g4o_topk256(_p(x), x.size, _p(out))
    return out


def topk_sort(packed512):
    p = _c(packed512, np.float32)
    ids = np.empty(256, np.uint32)
    vals = np.empty(256, np.float32)
    lib().g4o_topk_sort(_p(p), _p(ids), _p(vals))
    return ids, vals


def splitmix64(seed: int, idx: int) -> int:
    return int(lib().g4o_splitmix64(seed, idx))


def gen_q4k(seed: int, nblocks: int) -> np.ndarray:
    out = np.empty(nblocks * Q4K_BLOCK_BYTES, np.uint8)
    lib().g4o_gen_q4k(seed, nblocks, _p(out))
    return out


def gen_q6k(seed: int, nblocks: int) -> np.ndarray:
    out = np.empty(nblocks * Q6K_BLOCK_BYTES, np.uint8)
    lib().g4o_gen_q6k(seed, nblocks, _p(out))
    return out


def gen_normal_f32(seed: int, n: int, mean=0.0, std=1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().g4o_gen_normal_f32(seed, n, mean, std, _p(out))
    return out


def gen_normal_f16(seed: int, n: int, mean=0.0, std=1.0) -> np.ndarray:
    out = np.empty(n, np.uint16)
    lib().g4o_gen_normal_f16(seed, n, mean, std, _p(out))
    return out


def tensor_seed(base_seed: int, tensor_id: int) -> int:
    """Per-tensor stream seed: word `tensor_id` of stream `base_seed`."""
    return splitmix64(base_seed, tensor_id)


# --------------------------------------------------------------------------
# numpy restatements (independent cross-check of the C oracle)
# --------------------------------------------------------------------------

def np_f16_to_f32(h: np.ndarray) -> np.ndarray:
    """src/gguf.ts:103-113 — via numpy's IEEE half, which shares the format."""
    return np.asarray(h, np.uint16).view(np.float16).astype(np.float32)


def np_q4k_scales(scales: np.ndarray):
    """Vectorised getScaleMin (src/gguf.ts:175-182) for every j: [..., 8] sc and m."""
    s = scales.astype(np.int32)
    sc = np.empty(s.shape[:-1] + (8,), np.int32)
    m = np.empty_like(sc)
    sc[..., :4] = s[..., 0:4] & 63
    m[..., :4] = s[..., 4:8] & 63
    sc[..., 4:] = (s[..., 8:12] & 15) | ((s[..., 0:4] >> 6) << 4)
    m[..., 4:] = (s[..., 8:12] >> 4) | ((s[..., 4:8] >> 6) << 4)
    return sc, m


def np_dequant_q4k(blocks: np.ndarray) -> np.ndarray:
    b = np.asarray(blocks, np.uint8).reshape(-1, Q4K_BLOCK_BYTES)
    d = np_f16_to_f32(b[:, 0:2].copy().view(np.uint16)[:, 0]).astype(np.float64)
    dmin = np_f16_to_f32(b[:, 2:4].copy().view(np.uint16)[:, 0]).astype(np.float64)
    sc, m = np_q4k_scales(b[:, 4:16])
    qs = b[:, 16:144].reshape(-1, 4, 32)
    q = np.empty((b.shape[0], 8, 32), np.float64)
    q[:, 0::2, :] = qs & 15
    q[:, 1::2, :] = qs >> 4
    scale = d[:, None] * sc            # [nb, 8], exact
    mins = dmin[:, None] * m
    vals = scale[:, :, None] * q - mins[:, :, None]
    return vals.astype(np.float32).reshape(-1)


def np_dequant_q6k(blocks: np.ndarray) -> np.ndarray:
    b = np.asarray(blocks, np.uint8).reshape(-1, Q6K_BLOCK_BYTES)
    nb = b.shape[0]
    d = np_f16_to_f32(b[:, 208:210].copy().view(np.uint16)[:, 0]).astype(np.float64)
    sc = b[:, 192:208].view(np.int8).astype(np.float64)      # [nb, 16]
    out = np.empty((nb, 2, 4, 32), np.float64)
    for half in range(2):
        ql = b[:, half * 64:half * 64 + 64].astype(np.int32)
        qh = b[:, 128 + half * 32:128 + half * 32 + 32].astype(np.int32)
        q = [
            (ql[:, :32] & 15) | (((qh >> 0) & 3) << 4),
            (ql[:, 32:] & 15) | (((qh >> 2) & 3) << 4),
            (ql[:, :32] >> 4) | (((qh >> 4) & 3) << 4),
            (ql[:, 32:] >> 4) | (((qh >> 6) & 3) << 4),
        ]
        for k in range(4):
            # sub-block of 16: l < 16 uses sc[8*half + 2k], l >= 16 uses sc[8*half + 2k + 1]
            s = np.repeat(sc[:, half * 8 + 2 * k:half * 8 + 2 * k + 2], 16, axis=1)
            out[:, half, k, :] = d[:, None] * s * (q[k] - 32)
    return out.astype(np.float32).reshape(-1)


def np_splitmix64(seed: int, idx: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + (np.asarray(idx, np.uint64) + np.uint64(1)) * np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def np_rms_norm(x, w_f16, eps=1e-6):
    x = np.asarray(x, np.float64)
    w = np_f16_to_f32(w_f16).astype(np.float64)
    return (x * w / np.sqrt(np.mean(x * x) + eps)).astype(np.float32)


def np_gelu_mul(gate, up):
    x = np.asarray(gate, np.float64)
    t = np.clip(0.7978845608028654 * x * (1 + 0.044715 * x * x), -15, 15)
    th = np.tanh(t).astype(np.float32).astype(np.float64)   # the shader's tanh is an f32 value
    return (0.5 * x * (1 + th) * np.asarray(up, np.float64)).astype(np.float32)


def rel_l2(a, b) -> float:
    a = np.asarray(a, np.float64).reshape(-1)
    b = np.asarray(b, np.float64).reshape(-1)
    den = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (den if den > 0 else 1.0))


def cosine(a, b) -> float:
    a = np.asarray(a, np.float64).reshape(-1)
    b = np.asarray(b, np.float64).reshape(-1)
    na, nb = np.linalg.norm(a), np.linalg.norm(b)
    if na == 0 and nb == 0:
        return 1.0
    return float(a @ b / (na * nb))
