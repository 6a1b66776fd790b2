/*
 * g4_oracle.c — CPU restatement of the gemma4 decode hot path (oracle).
 *
 * TEST INFRASTRUCTURE ONLY: this is the checker for the HIP kernels. It is
 * never linked into, loaded by or called from the product library.
 *
 * Conventions
 *  - Reference citations are relative to the reference repository root.
 *  - Sums are carried in double; values are stored as f32 where the
 *    reference stores f32 (every buffer boundary between its kernels).
 *  - Build with -O2 -fno-fast-math -ffp-contract=off: the K-quant unpack is
 *    bit-exact only without reassociation (see g4o_dequant_q4k).
 */
#include "g4_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* f16 conversions                                                           */
/* ------------------------------------------------------------------------ */

/* src/gguf.ts:103-113 (f16ToF32): sign, 5-bit exponent, 10-bit mantissa,
 * subnormals = 2^-14 * mant/1024, exp 31 = Inf/NaN. */
float g4o_f16_to_f32(uint16_t h) {
  const int sign = (h >> 15) & 1;
  const int e = (h >> 10) & 0x1f;
  const int mant = h & 0x3ff;
  double v;
  if (e == 0) {
    if (mant == 0) return sign ? -0.0f : 0.0f;
    v = ldexp((double)mant / 1024.0, -14);
  } else if (e == 31) {
    if (mant == 0) return sign ? -INFINITY : INFINITY;
    return NAN;
  } else {
    v = ldexp(1.0 + (double)mant / 1024.0, e - 15);
  }
  return (float)(sign ? -v : v);
}

/* Round-to-nearest-even f32 -> f16, the conversion a native Float16Array
 * performs (src/gguf.ts:432-436). Subnormal f16 results are produced,
 * overflow goes to +-Inf, NaN stays NaN (quiet). */
uint16_t g4o_f32_to_f16_rne(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t ex = (x >> 23) & 0xffu;
  uint32_t mant = x & 0x7fffffu;
  if (ex == 0xff) return (uint16_t)(sign | 0x7c00u | (mant ? 0x200u : 0u));
  /* unbiased exponent */
  const int e = (int)ex - 127;
  if (e > 15) return (uint16_t)(sign | 0x7c00u);
  if (e >= -14) {
    /* normal f16: keep 10 mantissa bits, round the dropped 13 bits */
    uint32_t h = ((uint32_t)(e + 15) << 10) | (mant >> 13);
    const uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u; /* may carry into exp: ok */
    return (uint16_t)(sign | h);
  }
  if (ex == 0) return (uint16_t)sign; /* f32 subnormal is far below f16 range */
  /* f16 subnormal: value = m * 2^-24 with m = round(|f| * 2^24) */
  mant |= 0x800000u;                 /* 24-bit significand, value = mant * 2^(e-23) */
  const int shift = -e - 14 + 13;    /* bits to drop so the unit is 2^-24 */
  if (shift > 24) return (uint16_t)sign;
  const uint32_t h = mant >> shift;
  const uint32_t rem = mant & ((1u << shift) - 1u);
  const uint32_t half = 1u << (shift - 1);
  uint32_t r = h;
  if (rem > half || (rem == half && (h & 1u))) r += 1u;
  return (uint16_t)(sign | r);
}

/* Truncating fallback of src/gguf.ts:439-471 (used when Float16Array is
 * absent): f32 subnormals flush to 0, mantissa bits are dropped. */
uint16_t g4o_f32_to_f16_trunc(float f) {
  uint32_t bits;
  memcpy(&bits, &f, 4);
  const uint32_t sign = (bits >> 16) & 0x8000u;
  const uint32_t expRaw = (bits >> 23) & 0xffu;
  const uint32_t mant = bits & 0x7fffffu;
  if (expRaw == 0xff) return (uint16_t)(sign | 0x7c00u | (mant ? 0x200u : 0u));
  if (expRaw == 0) return (uint16_t)sign;
  const int newExp = (int)expRaw - 127 + 15;
  if (newExp >= 0x1f) return (uint16_t)(sign | 0x7c00u);
  if (newExp <= 0) {
    if (newExp < -10) return (uint16_t)sign;
    return (uint16_t)(sign | ((mant | 0x800000u) >> (1 - newExp + 13)));
  }
  return (uint16_t)(sign | ((uint32_t)newExp << 10) | (mant >> 13));
}

/* ------------------------------------------------------------------------ */
/* K-quant unpack                                                            */
/* ------------------------------------------------------------------------ */

/* src/gguf.ts:175-182 (getScaleMin): 8 (scale, min) pairs of 6 bits packed in
 * 12 bytes. j<4: low 6 bits of s[j] / s[j+4]; j>=4: a nibble of s[j+4] plus
 * the top 2 bits of s[j-4] (scale) or s[j] (min). */
void g4o_q4k_scale_min(const uint8_t s[12], int j, int* sc, int* m) {
  if (j < 4) {
    *sc = s[j] & 0x3f;
    *m = s[j + 4] & 0x3f;
  } else {
    *sc = (s[j + 4] & 0x0f) | ((s[j - 4] >> 6) << 4);
    *m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
  }
}

static uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* src/gguf.ts:168-210 (dequantizeQ4_K). 144-byte block: f16 d @0, f16 dmin @2,
 * scales[12] @4, qs[128] @16. Group g (0..3) of 32 bytes feeds sub-block 2g
 * (low nibbles -> elements 64g+l) and 2g+1 (high nibbles -> 64g+32+l).
 *
 * The reference evaluates d1*q - min1 in f64 and stores to f32. d*sc and
 * dmin*m carry <= 17 significant bits and d1*q <= 21, all exact in f32, and
 * the difference is exact in f64, so one f32 rounding of (d1*q - min1) is
 * the whole story: the f32 expression below (product exact, one rounded
 * subtraction) reproduces the reference bit for bit. */
void g4o_dequant_q4k(const uint8_t* blocks, size_t nblocks, float* out) {
  for (size_t b = 0; b < nblocks; ++b) {
    const uint8_t* blk = blocks + b * 144;
    const float d = g4o_f16_to_f32(rd16(blk));
    const float dmin = g4o_f16_to_f32(rd16(blk + 2));
    const uint8_t* s = blk + 4;
    const uint8_t* qs = blk + 16;
    float* o = out + b * 256;
    for (int g = 0; g < 4; ++g) {
      int sc1, m1, sc2, m2;
      g4o_q4k_scale_min(s, 2 * g, &sc1, &m1);
      g4o_q4k_scale_min(s, 2 * g + 1, &sc2, &m2);
      const double d1 = (double)d * sc1, min1 = (double)dmin * m1;
      const double d2 = (double)d * sc2, min2 = (double)dmin * m2;
      for (int l = 0; l < 32; ++l) {
        const uint8_t q = qs[32 * g + l];
        o[64 * g + l] = (float)(d1 * (q & 0x0f) - min1);
        o[64 * g + 32 + l] = (float)(d2 * ((q >> 4) & 0x0f) - min2);
      }
    }
  }
}

/* src/gguf.ts:323-368 (dequantizeQ6_K). 210-byte block: ql[128] @0,
 * qh[64] @128, int8 scales[16] @192, f16 d @208. Two halves of 128; for
 * l<32, is=l>>4, four 6-bit values (minus 32) land at l, l+32, l+64, l+96
 * with scales sc[is], sc[is+2], sc[is+4], sc[is+6]. d*sc*q needs <= 23
 * significant bits, so it is exact in any evaluation order. */
void g4o_dequant_q6k(const uint8_t* blocks, size_t nblocks, float* out) {
  for (size_t b = 0; b < nblocks; ++b) {
    const uint8_t* blk = blocks + b * 210;
    const double d = g4o_f16_to_f32(rd16(blk + 208));
    float* o = out + b * 256;
    for (int half = 0; half < 2; ++half) {
      const uint8_t* ql = blk + half * 64;
      const uint8_t* qh = blk + 128 + half * 32;
      const int8_t* sc = (const int8_t*)(blk + 192 + half * 8);
      float* oh = o + half * 128;
      for (int l = 0; l < 32; ++l) {
        const int is = l >> 4;
        const int q1 = ((ql[l] & 0x0f) | (((qh[l] >> 0) & 3) << 4)) - 32;
        const int q2 = ((ql[l + 32] & 0x0f) | (((qh[l] >> 2) & 3) << 4)) - 32;
        const int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
        const int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
        oh[l] = (float)(d * sc[is + 0] * q1);
        oh[l + 32] = (float)(d * sc[is + 2] * q2);
        oh[l + 64] = (float)(d * sc[is + 4] * q3);
        oh[l + 96] = (float)(d * sc[is + 6] * q4);
      }
    }
  }
}

/* src/gguf.ts:115-131 (dequantizeQ8_0): 34-byte blocks, f16 d then 32
 * int8 q; value = q * d (exact in f32: 8 x 11 significant bits). */
void g4o_dequant_q8_0(const uint8_t* blocks, size_t nblocks, float* out) {
  for (size_t b = 0; b < nblocks; ++b) {
    const uint8_t* blk = blocks + b * 34;
    const double d = g4o_f16_to_f32(rd16(blk));
    for (int i = 0; i < 32; ++i) out[b * 32 + i] = (float)((double)(int8_t)blk[2 + i] * d);
  }
}

/* src/gguf.ts:218-257 (decodeQ5_KBlock). 176-byte block: f16 d @0, f16
 * dmin @2, the 12 packed 6-bit scale/min bytes of Q4_K @4, qh[32] @16,
 * qs[128] @48. Group g (values 64g .. 64g+63) uses sub-blocks 2g and 2g+1:
 *   value 64g + l      = d*sc(2g)   * ((qs[32g+l] & 15) + 16*bit(qh[l], 2g))   - dmin*m(2g)
 *   value 64g + 32 + l = d*sc(2g+1) * ((qs[32g+l] >> 4) + 16*bit(qh[l], 2g+1)) - dmin*m(2g+1)
 * evaluated in f64 as the reference's JS numbers and stored as f32. */
void g4o_dequant_q5k(const uint8_t* blocks, size_t nblocks, float* out) {
  for (size_t b = 0; b < nblocks; ++b) {
    const uint8_t* blk = blocks + b * 176;
    const double d = g4o_f16_to_f32(rd16(blk));
    const double dmin = g4o_f16_to_f32(rd16(blk + 2));
    const uint8_t* s = blk + 4;
    const uint8_t* qh = blk + 16;
    const uint8_t* qs = blk + 48;
    float* o = out + b * 256;
    for (int g = 0; g < 4; ++g) {
      int sc1, m1, sc2, m2;
      g4o_q4k_scale_min(s, 2 * g, &sc1, &m1);
      g4o_q4k_scale_min(s, 2 * g + 1, &sc2, &m2);
      const double d1 = d * sc1, min1 = dmin * m1, d2 = d * sc2, min2 = dmin * m2;
      for (int l = 0; l < 32; ++l) {
        const int lo = (qs[32 * g + l] & 0x0f) + (((qh[l] >> (2 * g)) & 1) ? 16 : 0);
        const int hi = (qs[32 * g + l] >> 4) + (((qh[l] >> (2 * g + 1)) & 1) ? 16 : 0);
        o[64 * g + l] = (float)(d1 * lo - min1);
        o[64 * g + 32 + l] = (float)(d2 * hi - min2);
      }
    }
  }
}

/* ------------------------------------------------------------------------ */
/* matvec: y[m] = sum_k W[m,k] * x[k]   (shaders/matmul_quant.wgsl:25-53)    */
/* ------------------------------------------------------------------------ */

/* The reference's own weight format: f16 rows (shaders/matmul_quant.wgsl:14). */
void g4o_matmul_f16w(const float* x, const uint16_t* W, float* y, uint32_t M, uint32_t N) {
  for (uint32_t m = 0; m < M; ++m) {
    const uint16_t* row = W + (size_t)m * N;
    double acc = 0.0;
    for (uint32_t k = 0; k < N; ++k) acc += (double)g4o_f16_to_f32(row[k]) * (double)x[k];
    y[m] = (float)acc;
  }
}

/* Quantized rows: GGUF stores W row-major with the reduction axis fastest,
 * N/256 super-blocks per row. Dequantize a row (bit-exact values), dot in f64. */
void g4o_matmul_q4k(const float* x, const uint8_t* W, float* y, uint32_t M, uint32_t N) {
  const uint32_t bpr = N / 256;
  float* row = (float*)malloc(sizeof(float) * N);
  for (uint32_t m = 0; m < M; ++m) {
    g4o_dequant_q4k(W + (size_t)m * bpr * 144, bpr, row);
    double acc = 0.0;
    for (uint32_t k = 0; k < N; ++k) acc += (double)row[k] * (double)x[k];
    y[m] = (float)acc;
  }
  free(row);
}

void g4o_matmul_q6k(const float* x, const uint8_t* W, float* y, uint32_t M, uint32_t N) {
  const uint32_t bpr = N / 256;
  float* row = (float*)malloc(sizeof(float) * N);
  for (uint32_t m = 0; m < M; ++m) {
    g4o_dequant_q6k(W + (size_t)m * bpr * 210, bpr, row);
    double acc = 0.0;
    for (uint32_t k = 0; k < N; ++k) acc += (double)row[k] * (double)x[k];
    y[m] = (float)acc;
  }
  free(row);
}

/* ------------------------------------------------------------------------ */
/* norms and activations                                                     */
/* ------------------------------------------------------------------------ */

static double mean_sq(const float* v, uint32_t n) {
  double s = 0.0;
  for (uint32_t i = 0; i < n; ++i) s += (double)v[i] * (double)v[i];
  return s / (double)n;
}

/* shaders/rms_norm.wgsl:10-31: out = in * f32(w) / sqrt(mean(in^2) + eps) */
void g4o_rms_norm(const float* in, const uint16_t* w, float* out, uint32_t H, float eps) {
  const double rms = sqrt(mean_sq(in, H) + (double)eps);
  for (uint32_t i = 0; i < H; ++i) out[i] = (float)((double)in[i] * g4o_f16_to_f32(w[i]) / rms);
}

/* shaders/fused_norm_add.wgsl:11-32: out = residual + in * f32(w) / rms(in) */
void g4o_fused_norm_add(const float* in, const uint16_t* w, const float* residual, float* out,
                        uint32_t N, float eps) {
  const double rms = sqrt(mean_sq(in, N) + (double)eps);
  for (uint32_t i = 0; i < N; ++i)
    out[i] = (float)((double)residual[i] + (double)in[i] * g4o_f16_to_f32(w[i]) / rms);
}

/* shaders/gelu_mul.wgsl:1-16: tanh-GELU(gate) * up with the tanh argument
 * clamped to +-15. */
void g4o_gelu_mul(const float* gate, const float* up, float* out, uint32_t n) {
  const double k0 = 0.7978845608028654, k1 = 0.044715;
  for (uint32_t i = 0; i < n; ++i) {
    const double x = gate[i];
    double t = k0 * x * (1.0 + k1 * x * x);
    if (t > 15.0) t = 15.0;
    if (t < -15.0) t = -15.0;
    /* The shader's tanh returns an f32 (shaders/gelu_mul.wgsl:14): carry
     * it as that value (the f64 result rounded once), so that 1 + tanh(t)
     * is exactly 0 where f32 tanh saturates at -1 (x below about -5.5), as
     * in every f32 evaluation, rather than the ~1e-10 an f64 tanh leaves. */
    const double th = (double)(float)tanh(t);
    out[i] = (float)(0.5 * x * (1.0 + th) * (double)up[i]);
  }
}

/* shaders/ple_stage1_fuse.wgsl:14-37 for every layer: with
 * rms_l = sqrt(mean(projected[l*D .. l*D+D)^2) + eps),
 *   ple_inputs[l*D + t] = (projected[l*D+t] / rms_l * f32(norm_w[t])
 *                          + f32(embed_row[l*D+t]) * sqrt(D)) / sqrt(2),
 * embed_row being the token's row of the per-layer table (f16 values). */
void g4o_ple_stage1(const float* projected, const uint16_t* norm_w, const uint16_t* embed_row,
                    float* ple_inputs, uint32_t num_layers, uint32_t dim, float eps) {
  const double sq = sqrt((double)dim), inv2 = 1.0 / sqrt(2.0);
  for (uint32_t l = 0; l < num_layers; ++l) {
    const float* v = projected + (size_t)l * dim;
    const double rms = sqrt(mean_sq(v, dim) + (double)eps);
    for (uint32_t t = 0; t < dim; ++t) {
      const double normed = (double)v[t] / rms * g4o_f16_to_f32(norm_w[t]);
      const double emb = (double)g4o_f16_to_f32(embed_row[(size_t)l * dim + t]) * sq;
      ple_inputs[(size_t)l * dim + t] = (float)((normed + emb) * inv2);
    }
  }
}

/* shaders/ple_skip_scale_add.wgsl:14-20: hidden = (hidden + post_normed) * f32(scale) */
void g4o_ple_skip_scale_add(float* hidden, const float* post_normed, uint16_t scale, uint32_t n) {
  const double s = g4o_f16_to_f32(scale);
  for (uint32_t i = 0; i < n; ++i) hidden[i] = (float)(((double)hidden[i] + (double)post_normed[i]) * s);
}

/* shaders/per_head_rms_norm_no_weight.wgsl:14-37 (v_norm): per head
 * x / sqrt(mean(x^2) + eps), in place. */
void g4o_per_head_rms_norm_no_weight(float* data, uint32_t num_heads, uint32_t head_dim,
                                     float eps) {
  for (uint32_t h = 0; h < num_heads; ++h) {
    float* v = data + (size_t)h * head_dim;
    const double rms = sqrt(mean_sq(v, head_dim) + (double)eps);
    for (uint32_t i = 0; i < head_dim; ++i) v[i] = (float)((double)v[i] / rms);
  }
}

/* RoPE frequency of pair i (shaders/fused_per_head_norm_rope.wgsl:50-54):
 * base = 1/theta^(2i/HD) as the correctly rounded f32, then an f32 division by
 * the f16 divisor table entry when apply_divisor is set (a +Inf entry, which is
 * what 1e30 becomes in f16, gives freq = 0, i.e. no rotation). */
void g4o_rope_freq(float theta, uint32_t i, uint32_t head_dim, int apply_divisor,
                   const uint16_t* rope_freqs, float* freq_out) {
  const double e = (double)(2u * i) / (double)head_dim;
  float f = (float)(1.0 / pow((double)theta, e));
  if (apply_divisor) {
    const float div = g4o_f16_to_f32(rope_freqs[i]);
    f = f / div;
  }
  *freq_out = f;
}

/* shaders/fused_per_head_norm_rope.wgsl:21-63: per head, weighted RMSNorm
 * (stored f32) then rotate-half RoPE over pairs (i, i + HD/2). The angle is
 * the f32 product f32(position) * freq, as in the shader; cos/sin of that f32
 * angle are evaluated in double and rounded to f32. */
void g4o_fused_per_head_norm_rope(float* data, const uint16_t* weight, uint32_t num_heads,
                                  uint32_t head_dim, float eps, uint32_t position, float theta,
                                  uint32_t apply_divisor, const uint16_t* rope_freqs) {
  const uint32_t half = head_dim / 2;
  for (uint32_t h = 0; h < num_heads; ++h) {
    float* v = data + (size_t)h * head_dim;
    const double rms = sqrt(mean_sq(v, head_dim) + (double)eps);
    for (uint32_t i = 0; i < head_dim; ++i)
      v[i] = (float)((double)v[i] * g4o_f16_to_f32(weight[i]) / rms);
    for (uint32_t i = 0; i < half; ++i) {
      float freq;
      g4o_rope_freq(theta, i, head_dim, (int)apply_divisor, rope_freqs, &freq);
      const float angle = (float)position * freq;
      const double c = (float)cos((double)angle), s = (float)sin((double)angle);
      const double x0 = v[i], x1 = v[i + half];
      v[i] = (float)(x0 * c - x1 * s);
      v[i + half] = (float)(x0 * s + x1 * c);
    }
  }
}

/* ------------------------------------------------------------------------ */
/* attention over an f16, position-major KV cache                            */
/* ------------------------------------------------------------------------ */

/* shaders/kv_cache_store.wgsl:9-17: cache[pos*NKH*HD + h*HD + d] = in[h*HD+d];
 * the cache element type is f16 here (round to nearest even). */
void g4o_kv_cache_store_f16(const float* k_in, const float* v_in, uint16_t* k_cache,
                            uint16_t* v_cache, uint32_t num_kv_heads, uint32_t head_dim,
                            uint32_t position) {
  const size_t total = (size_t)num_kv_heads * head_dim;
  for (size_t i = 0; i < total; ++i) {
    k_cache[(size_t)position * total + i] = g4o_f32_to_f16_rne(k_in[i]);
    v_cache[(size_t)position * total + i] = g4o_f32_to_f16_rne(v_in[i]);
  }
}

/* shaders/attn_score.wgsl:23-30: a window W != 0 masks pos < cur+1-W. */
static uint32_t window_start(uint32_t seq_len, uint32_t window) {
  if (window == 0) return 0;
  const uint32_t cur = seq_len - 1;
  return (cur + 1 > window) ? cur + 1 - window : 0;
}

/* shaders/attn_score.wgsl:16-39: scores[h*seq_len + pos] = scale * q_h . K[pos,kvh];
 * kvh = h*NKH/NQH; masked positions get -1e30. */
void g4o_attn_score(const float* q, const uint16_t* k_cache, float* scores, uint32_t nqh,
                    uint32_t nkh, uint32_t hd, uint32_t seq_len, float scale, uint32_t window) {
  const uint32_t ws = window_start(seq_len, window);
  for (uint32_t h = 0; h < nqh; ++h) {
    const uint32_t kvh = h * nkh / nqh;
    for (uint32_t pos = 0; pos < seq_len; ++pos) {
      if (pos < ws) {
        scores[(size_t)h * seq_len + pos] = -1e30f;
        continue;
      }
      const uint16_t* k = k_cache + ((size_t)pos * nkh + kvh) * hd;
      double dot = 0.0;
      for (uint32_t d = 0; d < hd; ++d) dot += (double)q[h * hd + d] * g4o_f16_to_f32(k[d]);
      scores[(size_t)h * seq_len + pos] = (float)(dot * scale);
    }
  }
}

/* shaders/softmax.wgsl:8-45: per head, max (init -1e30), e = exp(s - max) in
 * place, divide by the sum. */
void g4o_softmax(float* scores, uint32_t num_heads, uint32_t seq_len) {
  for (uint32_t h = 0; h < num_heads; ++h) {
    float* s = scores + (size_t)h * seq_len;
    double mx = -1e30;
    for (uint32_t i = 0; i < seq_len; ++i)
      if (s[i] > mx) mx = s[i];
    double sum = 0.0;
    double* e = (double*)malloc(sizeof(double) * (seq_len ? seq_len : 1));
    for (uint32_t i = 0; i < seq_len; ++i) {
      e[i] = exp((double)s[i] - mx);
      sum += e[i];
    }
    for (uint32_t i = 0; i < seq_len; ++i) s[i] = (float)(e[i] / sum);
    free(e);
  }
}

/* shaders/attn_output.wgsl:8-22: out[h*HD+d] = sum_pos p[h,pos] * V[pos,kvh,d]. */
void g4o_attn_output(const float* probs, const uint16_t* v_cache, float* out, uint32_t nqh,
                     uint32_t nkh, uint32_t hd, uint32_t seq_len) {
  for (uint32_t h = 0; h < nqh; ++h) {
    const uint32_t kvh = h * nkh / nqh;
    for (uint32_t d = 0; d < hd; ++d) {
      double acc = 0.0;
      for (uint32_t pos = 0; pos < seq_len; ++pos)
        acc += (double)probs[(size_t)h * seq_len + pos] *
               g4o_f16_to_f32(v_cache[((size_t)pos * nkh + kvh) * hd + d]);
      out[h * hd + d] = (float)acc;
    }
  }
}

static void attention_rows(const float* q, const uint16_t* const* krow, const uint16_t* const* vrow,
                           float* out, uint32_t nqh, uint32_t nkh, uint32_t hd, uint32_t seq_len,
                           float scale, uint32_t window) {
  /* krow[pos] / vrow[pos] point at the NKH*HD f16 row of position pos */
  const uint32_t ws = window_start(seq_len, window);
  double* s = (double*)malloc(sizeof(double) * (seq_len ? seq_len : 1));
  for (uint32_t h = 0; h < nqh; ++h) {
    const uint32_t kvh = h * nkh / nqh;
    double mx = -1e300;
    for (uint32_t pos = ws; pos < seq_len; ++pos) {
      const uint16_t* k = krow[pos] + (size_t)kvh * hd;
      double dot = 0.0;
      for (uint32_t d = 0; d < hd; ++d) dot += (double)q[h * hd + d] * g4o_f16_to_f32(k[d]);
      s[pos] = dot * scale;
      if (s[pos] > mx) mx = s[pos];
    }
    double sum = 0.0;
    for (uint32_t pos = ws; pos < seq_len; ++pos) {
      s[pos] = exp(s[pos] - mx);
      sum += s[pos];
    }
    for (uint32_t d = 0; d < hd; ++d) {
      double acc = 0.0;
      for (uint32_t pos = ws; pos < seq_len; ++pos)
        acc += s[pos] * g4o_f16_to_f32(vrow[pos][(size_t)kvh * hd + d]);
      out[h * hd + d] = (float)(acc / sum);
    }
  }
  free(s);
}

/* score -> softmax -> output with f64 probabilities (the attention oracle the
 * fused split-K kernel is checked against); same masking as the trio. */
void g4o_attention(const float* q, const uint16_t* k_cache, const uint16_t* v_cache, float* out,
                   uint32_t nqh, uint32_t nkh, uint32_t hd, uint32_t seq_len, float scale,
                   uint32_t window) {
  const uint16_t** kr = (const uint16_t**)malloc(sizeof(void*) * (seq_len ? seq_len : 1));
  const uint16_t** vr = (const uint16_t**)malloc(sizeof(void*) * (seq_len ? seq_len : 1));
  for (uint32_t p = 0; p < seq_len; ++p) {
    kr[p] = k_cache + (size_t)p * nkh * hd;
    vr[p] = v_cache + (size_t)p * nkh * hd;
  }
  attention_rows(q, kr, vr, out, nqh, nkh, hd, seq_len, scale, window);
  free(kr);
  free(vr);
}

/* Paged variant: logical position p lives in physical page page_table[p / P],
 * slot p % P; a page holds P rows of NKH*HD f16. */
void g4o_attention_paged(const float* q, const uint16_t* k_pool, const uint16_t* v_pool,
                         const int32_t* page_table, uint32_t page_size, float* out, uint32_t nqh,
                         uint32_t nkh, uint32_t hd, uint32_t seq_len, float scale,
                         uint32_t window) {
  const uint16_t** kr = (const uint16_t**)malloc(sizeof(void*) * (seq_len ? seq_len : 1));
  const uint16_t** vr = (const uint16_t**)malloc(sizeof(void*) * (seq_len ? seq_len : 1));
  for (uint32_t p = 0; p < seq_len; ++p) {
    const size_t row = (size_t)page_table[p / page_size] * page_size + p % page_size;
    kr[p] = k_pool + row * nkh * hd;
    vr[p] = v_pool + row * nkh * hd;
  }
  attention_rows(q, kr, vr, out, nqh, nkh, hd, seq_len, scale, window);
  free(kr);
  free(vr);
}

/* ------------------------------------------------------------------------ */
/* LM head tail                                                              */
/* ------------------------------------------------------------------------ */

/* shaders/logit_softcap.wgsl:10-15: tanh(clamp(x/cap, +-15)) * cap, with the
 * division and the final product in f32. */
void g4o_logit_softcap(float* logits, uint32_t n, float cap) {
  for (uint32_t i = 0; i < n; ++i) {
    float x = logits[i] / cap;
    if (x > 15.0f) x = 15.0f;
    if (x < -15.0f) x = -15.0f;
    logits[i] = (float)tanh((double)x) * cap;
  }
}

/* shaders/argmax.wgsl:8-33. Thread t scans i = t, t+256, ... keeping the
 * first strict '>' maximum (init -1e30, index 0); the tree reduce replaces a
 * slot only on strict '>', so equal maxima resolve to the lowest thread.
 * Restated as that two-stage process. */
uint32_t g4o_argmax(const float* logits, uint32_t n) {
  float bm[256];
  uint32_t bi[256];
  for (uint32_t t = 0; t < 256; ++t) {
    float mx = -1e30f;
    uint32_t idx = 0;
    for (uint32_t i = t; i < n; i += 256) {
      if (logits[i] > mx) {
        mx = logits[i];
        idx = i;
      }
    }
    bm[t] = mx;
    bi[t] = idx;
  }
  for (uint32_t stride = 128; stride > 0; stride >>= 1) {
    for (uint32_t t = 0; t < stride; ++t) {
      if (bm[t + stride] > bm[t]) {
        bm[t] = bm[t + stride];
        bi[t] = bi[t + stride];
      }
    }
  }
  return bi[0];
}

/* shaders/topk256.wgsl:6-20: out[2t] = max over i == t (mod 256) (first
 * strict '>' max, init -1e30), out[2t+1] = bitcast<f32>(its index). */
void g4o_topk256(const float* logits, uint32_t n, float out[512]) {
  for (uint32_t t = 0; t < 256; ++t) {
    float mx = -1e30f;
    uint32_t idx = 0;
    for (uint32_t i = t; i < n; i += 256) {
      if (logits[i] > mx) {
        mx = logits[i];
        idx = i;
      }
    }
    out[2 * t] = mx;
    memcpy(&out[2 * t + 1], &idx, 4);
  }
}

/* src/engine.ts:1795-1811: unpack the 256 (val, id) pairs, then a stable
 * sort by value descending (Array.prototype.sort is stable), so equal values
 * keep ascending residue order. Insertion sort is stable by construction. */
void g4o_topk_sort(const float in[512], uint32_t ids[256], float vals[256]) {
  for (int i = 0; i < 256; ++i) {
    vals[i] = in[2 * i];
    memcpy(&ids[i], &in[2 * i + 1], 4);
  }
  for (int i = 1; i < 256; ++i) {
    const float v = vals[i];
    const uint32_t id = ids[i];
    int j = i - 1;
    while (j >= 0 && vals[j] < v) {
      vals[j + 1] = vals[j];
      ids[j + 1] = ids[j];
      --j;
    }
    vals[j + 1] = v;
    ids[j + 1] = id;
  }
}

/* ------------------------------------------------------------------------ */
/* seeded synthetic inputs                                                   */
/* ------------------------------------------------------------------------ */

/* Counter-based SplitMix64: word idx of stream `seed`. */
uint64_t g4o_splitmix64(uint64_t seed, uint64_t idx) {
  uint64_t z = seed + (idx + 1) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

/* Box-Muller from two words: u1 in (0,1], u2 in [0,1). */
static double normal_from(uint64_t w0, uint64_t w1) {
  const double u1 = (double)((w0 >> 11) + 1) * 0x1.0p-53;
  const double u2 = (double)(w1 >> 11) * 0x1.0p-53;
  return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

static void put16(uint8_t* p, uint16_t v) {
  p[0] = (uint8_t)(v & 0xff);
  p[1] = (uint8_t)(v >> 8);
}

/* Q4_K block b draws words 32b+i: d = f16(|N(0,2e-3)|) from (w0,w1),
 * dmin = f16(|N(0,1e-3)|) from (w2,w3), scales = bytes of w4 and the low
 * half of w5, qs = bytes of w6..w21 (little-endian byte order). */
void g4o_gen_q4k(uint64_t seed, uint64_t nblocks, uint8_t* out) {
  for (uint64_t b = 0; b < nblocks; ++b) {
    uint8_t* blk = out + b * 144;
    uint64_t w[22];
    for (int i = 0; i < 22; ++i) w[i] = g4o_splitmix64(seed, 32 * b + (uint64_t)i);
    put16(blk, g4o_f32_to_f16_rne((float)(fabs(normal_from(w[0], w[1])) * 2e-3)));
    put16(blk + 2, g4o_f32_to_f16_rne((float)(fabs(normal_from(w[2], w[3])) * 1e-3)));
    for (int k = 0; k < 12; ++k) blk[4 + k] = (uint8_t)(w[4 + k / 8] >> (8 * (k % 8)));
    for (int k = 0; k < 128; ++k) blk[16 + k] = (uint8_t)(w[6 + k / 8] >> (8 * (k % 8)));
  }
}

/* Q6_K block b draws words 32b+i: ql = bytes of w0..w15, qh = w16..w23,
 * scales k = (byte k of w24,w25 & 63) - 32 (uniform in -32..31),
 * d = f16(|N(0,2e-3)|) from (w26,w27). */
void g4o_gen_q6k(uint64_t seed, uint64_t nblocks, uint8_t* out) {
  for (uint64_t b = 0; b < nblocks; ++b) {
    uint8_t* blk = out + b * 210;
    uint64_t w[28];
    for (int i = 0; i < 28; ++i) w[i] = g4o_splitmix64(seed, 32 * b + (uint64_t)i);
    for (int k = 0; k < 128; ++k) blk[k] = (uint8_t)(w[k / 8] >> (8 * (k % 8)));
    for (int k = 0; k < 64; ++k) blk[128 + k] = (uint8_t)(w[16 + k / 8] >> (8 * (k % 8)));
    for (int k = 0; k < 16; ++k) {
      const int v = (int)((w[24 + k / 8] >> (8 * (k % 8))) & 63u) - 32;
      blk[192 + k] = (uint8_t)(int8_t)v;
    }
    put16(blk + 208, g4o_f32_to_f16_rne((float)(fabs(normal_from(w[26], w[27])) * 2e-3)));
  }
}

/* element i = f32(mean + std * N(0,1)) from words (2i, 2i+1) */
void g4o_gen_normal_f32(uint64_t seed, uint64_t n, float mean, float std, float* out) {
  for (uint64_t i = 0; i < n; ++i)
    out[i] = (float)((double)mean + (double)std * normal_from(g4o_splitmix64(seed, 2 * i),
                                                              g4o_splitmix64(seed, 2 * i + 1)));
}

void g4o_gen_normal_f16(uint64_t seed, uint64_t n, float mean, float std, uint16_t* out) {
  for (uint64_t i = 0; i < n; ++i)
    out[i] = g4o_f32_to_f16_rne(
        (float)((double)mean + (double)std * normal_from(g4o_splitmix64(seed, 2 * i),
                                                         g4o_splitmix64(seed, 2 * i + 1))));
}
