// k_gemv.hip — quantized matvec for gfx950 (matmulQuant / matmulQuantMR4).
//
// Computes y[m] = sum_k W[m,k] x[k] (shaders/matmul_quant.wgsl:21-54) with W
// kept in its GGUF block form: Q4_K (144 B / 256 weights, src/gguf.ts:157-210)
// or Q6_K (210 B / 256 weights, src/gguf.ts:316-368).
//
// Design (MI355X, wave64):
//  * The activation vector is staged in LDS once per workgroup as a two-digit
//    fixed-point form: per 32-element sub-block a scale s = max|x| / 32512 and
//    x ~= s * (256*hi + lo) with signed 8-bit digits hi, lo. Products with the
//    4/6-bit weight codes are then exact integer dot products
//    (v_dot4_i32_i8, four codes per instruction), so no per-weight
//    conversion or float FMA is needed; the dequant scales are applied once
//    per sub-block. The digit error is <= s/2 = max|x| / 65024.
//  * Weight tiles are streamed straight into registers: a wavefront owns R
//    consecutive rows (a contiguous byte range) and each lane owns one quarter
//    of a super-block per step (Q4_K: one 32-byte group = 64 weights; Q6_K:
//    one 48-byte ql/ql/qh unit = 64 weights), 16 blocks per step, all of a
//    tile's loads issued before the activation prologue so that HBM latency
//    overlaps it.
//  * Per-row sums are folded across the wave with a halving butterfly
//    (R*NV values in log2 steps instead of R*NV full reductions).
#include "g4_internal.hpp"

namespace {

constexpr int NW = 4;          // wavefronts per workgroup
constexpr int NT = NW * 64;    // threads per workgroup
constexpr int XSTRIDE = 288;   // LDS bytes per 256-element block of a digit plane (+32 pad)
constexpr float XQ = 32512.0f; // digit range: |v| <= 32512 keeps both digits in [-128,127]
constexpr size_t kMaxLds = 65536; // LDS bytes one workgroup may claim

typedef uint32_t u32x4a __attribute__((ext_vector_type(4), aligned(4)));

__device__ __forceinline__ uint4 ld16(const uint8_t* p) { return *(const uint4*)p; }
__device__ __forceinline__ u32x4a ld16a4(const uint8_t* p) { return *(const u32x4a*)p; }
__device__ __forceinline__ uint32_t ld4(const uint8_t* p) { return *(const uint32_t*)p; }

__device__ __forceinline__ int plane_off(uint32_t e) { return (int)((e >> 8) * XSTRIDE + (e & 255)); }

// LDS carve-up for NV activation vectors of length K.
struct XView {
  int8_t* hi;     // [NV][nb*XSTRIDE]
  int8_t* lo;     // [NV][nb*XSTRIDE]
  float* s;       // [NV][K/32]
  float* sum;     // [NV][K/32]   sum of x over the sub-block (Q4_K min term)
  int2* c16;      // [NV][K/16]   32*sum(hi), 32*sum(lo) over each 16-run (Q6_K offset)
  float* stage;   // [K]          normalised input (prologue modes 1, 2)
  float* red;     // [16]
  uint32_t K;
  __device__ int plane_bytes() const { return (int)(K / 256) * XSTRIDE; }
};

__host__ __device__ inline size_t xview_bytes(uint32_t K, int NV, bool stage) {
  size_t nb = K / 256;
  size_t b = 2 * (size_t)NV * nb * XSTRIDE;          // hi + lo planes
  b += 2 * (size_t)NV * (K / 32) * sizeof(float);    // s + sum
  b += (size_t)NV * (K / 16) * sizeof(int2);         // c16
  if (stage) b += (size_t)K * sizeof(float);
  b += 16 * sizeof(float);
  return b;
}

__device__ inline XView carve(uint8_t* smem, uint32_t K, int NV, bool stage) {
  XView v;
  v.K = K;
  const size_t nb = K / 256;
  uint8_t* p = smem;
  v.hi = (int8_t*)p;  p += (size_t)NV * nb * XSTRIDE;
  v.lo = (int8_t*)p;  p += (size_t)NV * nb * XSTRIDE;
  v.s = (float*)p;    p += (size_t)NV * (K / 32) * sizeof(float);
  v.sum = (float*)p;  p += (size_t)NV * (K / 32) * sizeof(float);
  v.c16 = (int2*)p;   p += (size_t)NV * (K / 16) * sizeof(int2);
  v.stage = (float*)p; if (stage) p += (size_t)K * sizeof(float);
  v.red = (float*)p;
  return v;
}

// Quantise 4 consecutive elements (one lane of an 8-lane sub-block group).
// e = first element index; all 64 lanes of the wave take part.
__device__ __forceinline__ void digits4(const XView& xv, int vec, uint32_t e, float x0, float x1,
                                        float x2, float x3, bool active) {
  float am = fmaxf(fmaxf(fabsf(x0), fabsf(x1)), fmaxf(fabsf(x2), fabsf(x3)));
  float sm = (x0 + x1) + (x2 + x3);
#pragma unroll
  for (int o = 1; o < 8; o <<= 1) {
    am = fmaxf(am, __shfl_xor(am, o, 64));
    sm += __shfl_xor(sm, o, 64);
  }
  const float inv = am > 0.f ? XQ / am : 0.f;
  const float xs[4] = {x0, x1, x2, x3};
  uint32_t phi = 0, plo = 0;
  int shi = 0, slo = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int v = (int)__builtin_rintf(xs[i] * inv);
    const int lo = ((v + 128) & 255) - 128;
    const int hi = (v - lo) >> 8;
    shi += hi;
    slo += lo;
    phi |= (uint32_t)(hi & 255) << (8 * i);
    plo |= (uint32_t)(lo & 255) << (8 * i);
  }
#pragma unroll
  for (int o = 1; o < 4; o <<= 1) {
    shi += __shfl_xor(shi, o, 64);
    slo += __shfl_xor(slo, o, 64);
  }
  if (active) {
    const int off = vec * xv.plane_bytes() + plane_off(e);
    *(uint32_t*)(xv.hi + off) = phi;
    *(uint32_t*)(xv.lo + off) = plo;
    const int lane8 = threadIdx.x & 7;
    if (lane8 == 0) {
      xv.s[vec * (xv.K / 32) + e / 32] = am * (1.0f / XQ);
      xv.sum[vec * (xv.K / 32) + e / 32] = sm;
    }
    if ((threadIdx.x & 3) == 0) xv.c16[vec * (xv.K / 16) + e / 16] = make_int2(32 * shi, 32 * slo);
  }
}

// Prologue modes: 0 = x from global; 1 = rms_norm(x) * w (shaders/rms_norm.wgsl);
// 2 = h = residual + o*w_post/rms(o), x = h*w_pre/rms(h)
// (shaders/fused_norm_add.wgsl followed by shaders/rms_norm.wgsl).
struct ProArgs {
  const float* x;         // [NV][K] (mode 0/1: input, mode 2: o)
  const uint16_t* w1;     // mode 1: norm weight; mode 2: w_post
  const float* residual;  // mode 2
  const uint16_t* w2;     // mode 2: w_pre
  float* h_out;           // mode 2: written by workgroup 0 when non-null
  float eps;
};

template <int NV, int PRO>
__device__ void prologue(const XView& xv, const ProArgs& a) {
  const uint32_t K = xv.K;
  const int tid = threadIdx.x;
  if constexpr (PRO == 1 || PRO == 2) {
    static_assert(NV == 1, "normalising prologues take one vector");
    float ss = 0.f;
    for (uint32_t i = tid; i < K; i += NT) { const float v = a.x[i]; ss += v * v; }
    ss = g4d::block_sum<NW>(ss, xv.red);
    const float inv1 = 1.0f / sqrtf(ss / (float)K + a.eps);
    if constexpr (PRO == 1) {
      for (uint32_t i = tid; i < K; i += NT) xv.stage[i] = a.x[i] * g4d::f16_bits_to_f32(a.w1[i]) * inv1;
    } else {
      float ss2 = 0.f;
      for (uint32_t i = tid; i < K; i += NT) {
        const float h = a.residual[i] + a.x[i] * g4d::f16_bits_to_f32(a.w1[i]) * inv1;
        xv.stage[i] = h;
        ss2 += h * h;
        if (a.h_out && blockIdx.x == 0) a.h_out[i] = h;
      }
      ss2 = g4d::block_sum<NW>(ss2, xv.red);
      const float inv2 = 1.0f / sqrtf(ss2 / (float)K + a.eps);
      for (uint32_t i = tid; i < K; i += NT) xv.stage[i] = xv.stage[i] * g4d::f16_bits_to_f32(a.w2[i]) * inv2;
    }
    __syncthreads();
  }
  // digit planes: 8 lanes per 32-element sub-block, 4 elements per lane
  const uint32_t nsub = K / 32;
  const uint32_t total = nsub * NV;
  for (uint32_t base = 0; base < total; base += NT / 8) {
    const uint32_t item = base + (uint32_t)(tid >> 3);
    const bool active = item < total;
    const uint32_t vec = active ? item / nsub : 0;
    const uint32_t sub = active ? item % nsub : 0;
    const uint32_t e = sub * 32 + (uint32_t)(tid & 7) * 4;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (active) {
      if constexpr (PRO == 0) v = *(const float4*)(a.x + (size_t)vec * K + e);
      else v = *(const float4*)(xv.stage + e);
    }
    digits4(xv, (int)vec, e, v.x, v.y, v.z, v.w, active);
  }
  __syncthreads();
}

// Q4_K scale/min pair for sub-blocks j = 2g and 2g+1 of one block
// (src/gguf.ts:175-182). S0..S2 are the 12 scale bytes as three words.
__device__ __forceinline__ void q4k_scales(uint32_t S0, uint32_t S1, uint32_t S2, int g, float& sc_lo,
                                           float& sc_hi, float& m_lo, float& m_hi) {
  const int sh = 16 * (g & 1);
  uint32_t scp, mp;
  if (g < 2) {
    scp = (S0 >> sh) & 0x3f3fu;
    mp = (S1 >> sh) & 0x3f3fu;
  } else {
    scp = ((S2 >> sh) & 0x0f0fu) | ((S0 >> (sh + 2)) & 0x3030u);
    mp = ((S2 >> (sh + 4)) & 0x0f0fu) | ((S1 >> (sh + 2)) & 0x3030u);
  }
  sc_lo = (float)(scp & 0xffu);
  sc_hi = (float)(scp >> 8);
  m_lo = (float)(mp & 0xffu);
  m_hi = (float)(mp >> 8);
}

__device__ __forceinline__ int dot8(const uint32_t* q, const uint32_t* x) {
  int acc = 0;
#pragma unroll
  for (int k = 0; k < 8; ++k) acc = __builtin_amdgcn_sdot4((int)q[k], (int)x[k], acc, false);
  return acc;
}

// Halving butterfly: reduces N (power of two) per-lane values across the
// wave. Afterwards lanes with (lane & (64/N - 1)) == 0 hold the sum of value
// index lane / (64/N) in out.
template <int N>
__device__ __forceinline__ float wave_fold(float (&a)[N]) {
  const int lane = threadIdx.x & 63;
  constexpr int LOGN = (N >= 64) ? 6 : (N >= 32) ? 5 : (N >= 16) ? 4 : (N >= 8) ? 3 : (N >= 4) ? 2 : (N >= 2) ? 1 : 0;
  static_assert((1 << LOGN) == N, "power of two");
  int n = N;
#pragma unroll
  for (int step = 0; step < LOGN; ++step) {
    const int o = 32 >> step;
    const bool up = (lane & o) != 0;
    const int half = n >> 1;
#pragma unroll
    for (int i = 0; i < N / 2; ++i) {
      if (i < half) {
        const float mine = up ? a[i + half] : a[i];
        const float send = up ? a[i] : a[i + half];
        a[i] = mine + __shfl_xor(send, o, 64);
      }
    }
    n = half;
  }
  float v = a[0];
#pragma unroll
  for (int o = 32 >> LOGN; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// ---------------------------------------------------------------------------
// Q4_K
// ---------------------------------------------------------------------------

struct GemvSeg {
  const uint8_t* W;
  float* Y;
  uint32_t M;
  uint32_t wg_begin;  // first workgroup of this segment
};
struct GemvSegs {
  GemvSeg s[4];
  int n;
};

template <int BPR, int R>
struct Tile {
  static constexpr int IT = R * BPR / 16;  // steps of 16 blocks
  static_assert((R * BPR) % 16 == 0, "tile must be a whole number of 16-block steps");
  static constexpr int ROWS_WG = R * NW;
};

template <int BPR, int R, int NV>
__device__ __forceinline__ void q4k_tile_compute(const XView& xv, const uint4 (&hd)[Tile<BPR, R>::IT],
                                                 const uint4 (&q0)[Tile<BPR, R>::IT],
                                                 const uint4 (&q1)[Tile<BPR, R>::IT],
                                                 float (&acc)[NV * R]) {
  constexpr int IT = Tile<BPR, R>::IT;
  const int lane = threadIdx.x & 63;
  const int g = lane & 3, bl = lane >> 2;
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int fb = it * 16 + bl;
    const int r = fb / BPR, b = fb % BPR;
    const float d = g4d::f16_bits_to_f32(hd[it].x & 0xffffu);
    const float dmin = g4d::f16_bits_to_f32(hd[it].x >> 16);
    float sc_lo, sc_hi, m_lo, m_hi;
    q4k_scales(hd[it].y, hd[it].z, hd[it].w, g, sc_lo, sc_hi, m_lo, m_hi);
    const float dl = d * sc_lo, dh = d * sc_hi, ml = dmin * m_lo, mh = dmin * m_hi;
    uint32_t nl[8], nh[8];
    const uint32_t qa[8] = {q0[it].x, q0[it].y, q0[it].z, q0[it].w, q1[it].x, q1[it].y, q1[it].z, q1[it].w};
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      nl[k] = qa[k] & 0x0f0f0f0fu;
      nh[k] = (qa[k] >> 4) & 0x0f0f0f0fu;
    }
    const uint32_t e0 = (uint32_t)b * 256 + 64u * g;
    const int sub = (int)(e0 / 32);
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int off = v * xv.plane_bytes() + plane_off(e0);
      uint32_t xh[16], xl[16];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint4 th = *(const uint4*)(xv.hi + off + 16 * c);
        const uint4 tl = *(const uint4*)(xv.lo + off + 16 * c);
        xh[4 * c + 0] = th.x; xh[4 * c + 1] = th.y; xh[4 * c + 2] = th.z; xh[4 * c + 3] = th.w;
        xl[4 * c + 0] = tl.x; xl[4 * c + 1] = tl.y; xl[4 * c + 2] = tl.z; xl[4 * c + 3] = tl.w;
      }
      const int ilo = dot8(nl, xh) * 256 + dot8(nl, xl);
      const int ihi = dot8(nh, xh + 8) * 256 + dot8(nh, xl + 8);
      const float* s = xv.s + v * (xv.K / 32);
      const float* sm = xv.sum + v * (xv.K / 32);
      float part = dl * s[sub] * (float)ilo - ml * sm[sub];
      part += dh * s[sub + 1] * (float)ihi - mh * sm[sub + 1];
      // rows a lane can touch at this step are known at compile time
#pragma unroll
      for (int rr = (it * 16) / BPR; rr <= (it * 16 + 15) / BPR && rr < R; ++rr)
        acc[v * R + rr] += (r == rr) ? part : 0.f;
    }
  }
}

template <int BPR, int R, int NV>
__device__ __forceinline__ void store_rows(float (&acc)[NV * R], float* Y, uint32_t M, uint32_t row0,
                                           uint32_t ldy) {
  constexpr int N = NV * R;
  const float v = wave_fold<N>(acc);
  const int lane = threadIdx.x & 63;
  constexpr int G = 64 / N;
  if ((lane % G) == 0) {
    const int idx = lane / G;
    const int vec = idx / R, rr = idx % R;
    if (row0 + rr < M) Y[(size_t)vec * ldy + row0 + rr] = v;
  }
}

// One workgroup = NW waves x R rows. Segments let one launch cover several
// matrices that share the input vector (e.g. q/k/v projections).
template <int BPR, int R, int NV, int PRO>
__global__ __launch_bounds__(NT) void gemv_q4k_kernel(GemvSegs segs, ProArgs pa, uint32_t ldy) {
  using T = Tile<BPR, R>;
  constexpr int IT = T::IT;
  extern __shared__ __align__(16) uint8_t smem[];
  int si = 0;
#pragma unroll
  for (int i = 1; i < 4; ++i)
    if (i < segs.n && blockIdx.x >= segs.s[i].wg_begin) si = i;
  const GemvSeg sg = segs.s[si];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const uint32_t row0 = ((blockIdx.x - sg.wg_begin) * NW + w) * R;
  const int g = lane & 3, bl = lane >> 2;

  uint4 hd[IT], q0[IT], q1[IT];
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int fb = it * 16 + bl;
    const uint32_t row = row0 + fb / BPR;
    if (row < sg.M) {
      const uint8_t* p = sg.W + ((size_t)row0 * BPR + fb) * 144;
      hd[it] = ld16(p);
      q0[it] = ld16(p + 16 + 32 * g);
      q1[it] = ld16(p + 32 + 32 * g);
    } else {
      hd[it] = make_uint4(0, 0, 0, 0);
      q0[it] = hd[it];
      q1[it] = hd[it];
    }
  }
  const XView xv = carve(smem, BPR * 256, NV, PRO != 0);
  prologue<NV, PRO>(xv, pa);

  float acc[NV * R];
#pragma unroll
  for (int i = 0; i < NV * R; ++i) acc[i] = 0.f;
  q4k_tile_compute<BPR, R, NV>(xv, hd, q0, q1, acc);
  store_rows<BPR, R, NV>(acc, sg.Y, sg.M, row0, ldy);
}

// gate/up pair with the tanh-GELU product epilogue (shaders/gelu_mul.wgsl:10-16):
// out[i] = gelu(gate[i]) * up[i]; both matrices are [M, BPR*256] Q4_K.
__device__ __forceinline__ float gelu_tanh(float x) {
  float t = 0.7978845608028654f * x * (1.0f + 0.044715f * x * x);
  t = fminf(fmaxf(t, -15.0f), 15.0f);
  return 0.5f * x * (1.0f + tanhf(t));
}

template <int BPR, int R, int PRO>
__global__ __launch_bounds__(NT) void gateup_q4k_kernel(const uint8_t* Wg, const uint8_t* Wu, float* out,
                                                        uint32_t M, ProArgs pa) {
  using T = Tile<BPR, R>;
  constexpr int IT = T::IT;
  extern __shared__ __align__(16) uint8_t smem[];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const uint32_t row0 = (blockIdx.x * NW + w) * R;
  const int g = lane & 3, bl = lane >> 2;
  uint4 hg[IT], g0[IT], g1[IT], hu[IT], u0[IT], u1[IT];
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int fb = it * 16 + bl;
    const uint32_t row = row0 + fb / BPR;
    if (row < M) {
      const size_t off = ((size_t)row0 * BPR + fb) * 144;
      hg[it] = ld16(Wg + off);
      g0[it] = ld16(Wg + off + 16 + 32 * g);
      g1[it] = ld16(Wg + off + 32 + 32 * g);
      hu[it] = ld16(Wu + off);
      u0[it] = ld16(Wu + off + 16 + 32 * g);
      u1[it] = ld16(Wu + off + 32 + 32 * g);
    } else {
      hg[it] = g0[it] = g1[it] = hu[it] = u0[it] = u1[it] = make_uint4(0, 0, 0, 0);
    }
  }
  const XView xv = carve(smem, BPR * 256, 1, PRO != 0);
  prologue<1, PRO>(xv, pa);
  float ag[R], au[R];
#pragma unroll
  for (int i = 0; i < R; ++i) ag[i] = au[i] = 0.f;
  q4k_tile_compute<BPR, R, 1>(xv, hg, g0, g1, ag);
  q4k_tile_compute<BPR, R, 1>(xv, hu, u0, u1, au);
  const float vg = wave_fold<R>(ag);
  const float vu = wave_fold<R>(au);
  constexpr int G = 64 / R;
  if ((lane % G) == 0) {
    const uint32_t row = row0 + lane / G;
    if (row < M) out[row] = gelu_tanh(vg) * vu;
  }
}

// ---------------------------------------------------------------------------
// Q6_K
// ---------------------------------------------------------------------------

// 16 bytes at a 2-byte aligned address: an aligned 16-byte word load plus the
// next dword, funnel-shifted by the misalignment (0 or 2 bytes).
struct Piece { u32x4a a; uint32_t e; uint32_t sh; };

__device__ __forceinline__ Piece ld_piece(const uint8_t* p) {
  const uintptr_t ad = (uintptr_t)p;
  const uint8_t* p4 = (const uint8_t*)(ad & ~(uintptr_t)3);
  Piece r;
  r.a = ld16a4(p4);
  r.e = ld4(p4 + 16);
  r.sh = (uint32_t)(ad & 3);
  return r;
}

__device__ __forceinline__ void piece_words(const Piece& p, uint32_t (&w)[4]) {
  w[0] = __builtin_amdgcn_alignbyte(p.a.y, p.a.x, p.sh);
  w[1] = __builtin_amdgcn_alignbyte(p.a.z, p.a.y, p.sh);
  w[2] = __builtin_amdgcn_alignbyte(p.a.w, p.a.z, p.sh);
  w[3] = __builtin_amdgcn_alignbyte(p.e, p.a.w, p.sh);
}

struct Q6Unit {
  Piece A, B, H;
  int sc[4];
  uint32_t d;
};

__device__ __forceinline__ void q6_load(const uint8_t* blk, int u, Q6Unit& q) {
  const int h = u >> 1, l0 = (u & 1) * 16;
  q.A = ld_piece(blk + 64 * h + l0);
  q.B = ld_piece(blk + 64 * h + 32 + l0);
  q.H = ld_piece(blk + 128 + 32 * h + l0);
  const int8_t* sc = (const int8_t*)(blk + 192 + 8 * h + (u & 1));
#pragma unroll
  for (int k = 0; k < 4; ++k) q.sc[k] = sc[2 * k];
  q.d = *(const uint16_t*)(blk + 208);
}

__device__ __forceinline__ void q6_zero(Q6Unit& q) {
  q.A.a = q.B.a = q.H.a = u32x4a{0, 0, 0, 0};
  q.A.e = q.B.e = q.H.e = 0;
  q.A.sh = q.B.sh = q.H.sh = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) q.sc[k] = 0;
  q.d = 0;
}

template <int BPR, int R, int NV>
__device__ __forceinline__ void q6k_tile_compute(const XView& xv, const Q6Unit (&qu)[Tile<BPR, R>::IT],
                                                 float (&acc)[NV * R]) {
  constexpr int IT = Tile<BPR, R>::IT;
  const int lane = threadIdx.x & 63;
  const int u = lane & 3, bl = lane >> 2;
  const int h = u >> 1, l0 = (u & 1) * 16;
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int fb = it * 16 + bl;
    const int r = fb / BPR, b = fb % BPR;
    uint32_t A[4], B[4], H[4];
    piece_words(qu[it].A, A);
    piece_words(qu[it].B, B);
    piece_words(qu[it].H, H);
    // run k covers elements 128h + 32k + l0 + [0,16) (src/gguf.ts:344-361)
    uint32_t q[4][4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      q[0][j] = (A[j] & 0x0f0f0f0fu) | ((H[j] << 4) & 0x30303030u);
      q[1][j] = (B[j] & 0x0f0f0f0fu) | ((H[j] << 2) & 0x30303030u);
      q[2][j] = ((A[j] >> 4) & 0x0f0f0f0fu) | (H[j] & 0x30303030u);
      q[3][j] = ((B[j] >> 4) & 0x0f0f0f0fu) | ((H[j] >> 2) & 0x30303030u);
    }
    const float d = g4d::f16_bits_to_f32(qu[it].d);
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      float part = 0.f;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t e = (uint32_t)b * 256 + 128u * h + 32u * k + l0;
        const int off = v * xv.plane_bytes() + plane_off(e);
        const uint4 th = *(const uint4*)(xv.hi + off);
        const uint4 tl = *(const uint4*)(xv.lo + off);
        int ah = 0, al = 0;
        ah = __builtin_amdgcn_sdot4((int)q[k][0], (int)th.x, ah, false);
        ah = __builtin_amdgcn_sdot4((int)q[k][1], (int)th.y, ah, false);
        ah = __builtin_amdgcn_sdot4((int)q[k][2], (int)th.z, ah, false);
        ah = __builtin_amdgcn_sdot4((int)q[k][3], (int)th.w, ah, false);
        al = __builtin_amdgcn_sdot4((int)q[k][0], (int)tl.x, al, false);
        al = __builtin_amdgcn_sdot4((int)q[k][1], (int)tl.y, al, false);
        al = __builtin_amdgcn_sdot4((int)q[k][2], (int)tl.z, al, false);
        al = __builtin_amdgcn_sdot4((int)q[k][3], (int)tl.w, al, false);
        const int2 c = xv.c16[v * (xv.K / 16) + e / 16];
        const int I = (ah - c.x) * 256 + (al - c.y);
        const float s = xv.s[v * (xv.K / 32) + e / 32];
        part += (float)qu[it].sc[k] * s * (float)I;
      }
      part *= d;
#pragma unroll
      for (int rr = (it * 16) / BPR; rr <= (it * 16 + 15) / BPR && rr < R; ++rr)
        acc[v * R + rr] += (r == rr) ? part : 0.f;
    }
  }
}

template <int BPR, int R, int NV, int PRO>
__global__ __launch_bounds__(NT) void gemv_q6k_kernel(GemvSegs segs, ProArgs pa, uint32_t ldy) {
  using T = Tile<BPR, R>;
  constexpr int IT = T::IT;
  extern __shared__ __align__(16) uint8_t smem[];
  int si = 0;
#pragma unroll
  for (int i = 1; i < 4; ++i)
    if (i < segs.n && blockIdx.x >= segs.s[i].wg_begin) si = i;
  const GemvSeg sg = segs.s[si];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const uint32_t row0 = ((blockIdx.x - sg.wg_begin) * NW + w) * R;
  const int u = lane & 3, bl = lane >> 2;
  Q6Unit qu[IT];
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int fb = it * 16 + bl;
    const uint32_t row = row0 + fb / BPR;
    if (row < sg.M) q6_load(sg.W + ((size_t)row0 * BPR + fb) * 210, u, qu[it]);
    else q6_zero(qu[it]);
  }
  const XView xv = carve(smem, BPR * 256, NV, PRO != 0);
  prologue<NV, PRO>(xv, pa);
  float acc[NV * R];
#pragma unroll
  for (int i = 0; i < NV * R; ++i) acc[i] = 0.f;
  q6k_tile_compute<BPR, R, NV>(xv, qu, acc);
  store_rows<BPR, R, NV>(acc, sg.Y, sg.M, row0, ldy);
}

// ---------------------------------------------------------------------------
// Fallbacks: any N % 256 == 0 (one wave per row, float math) and f16 rows.
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(NT) void gemv_q4k_generic(const float* x, const uint8_t* W, float* y, uint32_t M,
                                                       uint32_t N) {
  const uint32_t row = blockIdx.x * NW + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= M) return;
  const uint32_t bpr = N / 256;
  float acc = 0.f;
  // lane = (block b mod 16, group g)
  for (uint32_t b = lane >> 2; b < bpr; b += 16) {
    const int g = lane & 3;
    const uint8_t* p = W + ((size_t)row * bpr + b) * 144;
    const uint4 hd = ld16(p);
    const float d = g4d::f16_bits_to_f32(hd.x & 0xffffu), dmin = g4d::f16_bits_to_f32(hd.x >> 16);
    float sc_lo, sc_hi, m_lo, m_hi;
    q4k_scales(hd.y, hd.z, hd.w, g, sc_lo, sc_hi, m_lo, m_hi);
    const float* xs = x + b * 256 + 64 * g;
    for (int l = 0; l < 32; ++l) {
      const uint8_t q = p[16 + 32 * g + l];
      acc += (d * sc_lo * (float)(q & 15) - dmin * m_lo) * xs[l];
      acc += (d * sc_hi * (float)(q >> 4) - dmin * m_hi) * xs[32 + l];
    }
  }
  acc = g4d::wave_sum(acc);
  if (lane == 0) y[row] = acc;
}

__global__ __launch_bounds__(NT) void gemv_q6k_generic(const float* x, const uint8_t* W, float* y, uint32_t M,
                                                       uint32_t N) {
  const uint32_t row = blockIdx.x * NW + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= M) return;
  const uint32_t bpr = N / 256;
  float acc = 0.f;
  for (uint32_t b = lane >> 2; b < bpr; b += 16) {
    const int u = lane & 3, h = u >> 1, l0 = (u & 1) * 16;
    const uint8_t* blk = W + ((size_t)row * bpr + b) * 210;
    const float d = g4d::f16_bits_to_f32(*(const uint16_t*)(blk + 208));
    const int8_t* sc = (const int8_t*)(blk + 192 + 8 * h);
    const uint8_t* ql = blk + 64 * h;
    const uint8_t* qh = blk + 128 + 32 * h;
    const float* xs = x + b * 256 + 128 * h;
    for (int i = 0; i < 16; ++i) {
      const int l = l0 + i, is = l >> 4;
      const int q1 = ((ql[l] & 15) | ((qh[l] & 3) << 4)) - 32;
      const int q2 = ((ql[l + 32] & 15) | (((qh[l] >> 2) & 3) << 4)) - 32;
      const int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
      const int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
      acc += d * (float)sc[is] * (float)q1 * xs[l];
      acc += d * (float)sc[is + 2] * (float)q2 * xs[l + 32];
      acc += d * (float)sc[is + 4] * (float)q3 * xs[l + 64];
      acc += d * (float)sc[is + 6] * (float)q4 * xs[l + 96];
    }
  }
  acc = g4d::wave_sum(acc);
  if (lane == 0) y[row] = acc;
}

// f16 rows (the reference's own upload format): R=4 rows per wave, 16-byte
// loads of 8 halves, x staged in LDS as f32.
__global__ __launch_bounds__(NT) void gemv_f16_kernel(const float* x, const uint16_t* W, float* y, uint32_t M,
                                                      uint32_t N) {
  extern __shared__ __align__(16) uint8_t smem[];
  float* xs = (float*)smem;
  for (uint32_t i = threadIdx.x; i < N; i += NT) xs[i] = x[i];
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const uint32_t row0 = (blockIdx.x * NW + (threadIdx.x >> 6)) * 4;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  const bool vec8 = (N % 8) == 0;
  for (uint32_t k = lane * 8; k < N; k += 512) {
    float xv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) xv[i] = (k + i < N) ? xs[k + i] : 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if (row0 + r >= M) continue;
      const uint16_t* wr = W + (size_t)(row0 + r) * N + k;
      if (vec8 && k + 8 <= N) {
        const uint4 wv = *(const uint4*)wr;
        const uint32_t ws[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          acc[r] += g4d::f16_bits_to_f32(ws[i] & 0xffffu) * xv[2 * i];
          acc[r] += g4d::f16_bits_to_f32(ws[i] >> 16) * xv[2 * i + 1];
        }
      } else {
        for (int i = 0; i < 8 && k + i < N; ++i) acc[r] += g4d::f16_bits_to_f32(wr[i]) * xv[i];
      }
    }
  }
  const float v = wave_fold<4>(acc);
  if ((lane & 15) == 0 && row0 + lane / 16 < M) y[row0 + lane / 16] = v;
}

// ---------------------------------------------------------------------------
// Host dispatch
// ---------------------------------------------------------------------------

template <int BPR>
struct RowsFor;  // rows per wave for each supported blocks-per-row
template <> struct RowsFor<4> { static constexpr int R = 8; };
template <> struct RowsFor<6> { static constexpr int R = 8; };
template <> struct RowsFor<8> { static constexpr int R = 4; };
template <> struct RowsFor<12> { static constexpr int R = 4; };
template <> struct RowsFor<16> { static constexpr int R = 2; };
template <> struct RowsFor<24> { static constexpr int R = 2; };
template <> struct RowsFor<32> { static constexpr int R = 1; };
template <> struct RowsFor<48> { static constexpr int R = 1; };

enum class QType { Q4K, Q6K };

struct LaunchReq {
  QType qt;
  const GemvSeg* segs;  // W, Y, M (wg_begin filled here)
  int nseg;
  uint32_t N;
  int nv;
  int pro;
  ProArgs pa;
  uint32_t ldy;
};

template <int BPR, int NV, int PRO>
int launch_fixed(g4_ctx* ctx, const LaunchReq& q) {
  constexpr int R = RowsFor<BPR>::R;
  constexpr int ROWS_WG = R * NW;
  GemvSegs sg{};
  uint32_t wgs = 0;
  for (int i = 0; i < q.nseg; ++i) {
    sg.s[i] = q.segs[i];
    sg.s[i].wg_begin = wgs;
    wgs += ceil_div(q.segs[i].M, ROWS_WG);
  }
  sg.n = q.nseg;
  if (wgs == 0) return G4_OK;
  const size_t lds = xview_bytes(BPR * 256, NV, PRO != 0);
  if (q.qt == QType::Q4K)
    hipLaunchKernelGGL((gemv_q4k_kernel<BPR, R, NV, PRO>), dim3(wgs), dim3(NT), lds, ctx->stream, sg, q.pa, q.ldy);
  else
    hipLaunchKernelGGL((gemv_q6k_kernel<BPR, R, NV, PRO>), dim3(wgs), dim3(NT), lds, ctx->stream, sg, q.pa, q.ldy);
  G4_LAUNCHED(ctx, "gemv");
  return G4_OK;
}

template <int NV, int PRO>
int launch_nv(g4_ctx* ctx, const LaunchReq& q) {
  switch (q.N / 256) {
    case 4: return launch_fixed<4, NV, PRO>(ctx, q);
    case 6: return launch_fixed<6, NV, PRO>(ctx, q);
    case 8: return launch_fixed<8, NV, PRO>(ctx, q);
    case 12: return launch_fixed<12, NV, PRO>(ctx, q);
    case 16: return launch_fixed<16, NV, PRO>(ctx, q);
    case 24: return launch_fixed<24, NV, PRO>(ctx, q);
    case 32: return launch_fixed<32, NV, PRO>(ctx, q);
    case 48: return launch_fixed<48, NV, PRO>(ctx, q);
    default: return G4_ERR_UNSUPPORTED;
  }
}

int launch_gemv(g4_ctx* ctx, const LaunchReq& q) {
  if (q.pro == 1) return launch_nv<1, 1>(ctx, q);
  if (q.pro == 2) return launch_nv<1, 2>(ctx, q);
  switch (q.nv) {
    case 1: return launch_nv<1, 0>(ctx, q);
    case 2: return launch_nv<2, 0>(ctx, q);
    case 4: return launch_nv<4, 0>(ctx, q);
    case 8: return launch_nv<8, 0>(ctx, q);
    default: return G4_ERR_UNSUPPORTED;
  }
}

bool supported_bpr(uint32_t bpr) {
  return bpr == 4 || bpr == 6 || bpr == 8 || bpr == 12 || bpr == 16 || bpr == 24 || bpr == 32 || bpr == 48;
}

int check_mm(const char* fn, const void* in, const void* w, const void* out, g4_matmul_params p) {
  G4_REQUIRE(in && w && out, "%s: null buffer", fn);
  G4_REQUIRE(p.M > 0 && p.N > 0, "%s: empty shape M=%u N=%u", fn, p.M, p.N);
  G4_REQUIRE(p.N % 256 == 0, "%s: N=%u is not a multiple of the 256-weight super-block", fn, p.N);
  G4_REQUIRE(p.N <= 16384, "%s: N=%u exceeds the 16384 activation limit", fn, p.N);
  G4_REQUIRE(((uintptr_t)in & 15) == 0, "%s: input must be 16-byte aligned", fn);
  return G4_OK;
}

int matmul_quant(g4_ctx* ctx, const char* fn, QType qt, const float* in, const void* w, float* out,
                 g4_matmul_params p, uint32_t batch) {
  G4_ENTER(ctx);
  int rc = check_mm(fn, in, w, out, p);
  if (rc) return rc;
  G4_REQUIRE(batch >= 1, "%s: batch must be >= 1", fn);
  if (qt == QType::Q4K) G4_REQUIRE(((uintptr_t)w & 15) == 0, "%s: Q4_K weights must be 16-byte aligned", fn);
  else G4_REQUIRE(((uintptr_t)w & 3) == 0, "%s: Q6_K weights must be 4-byte aligned", fn);
  const uint32_t bpr = p.N / 256;
  if (!supported_bpr(bpr)) {
    if (batch != 1) return g4::set_error(G4_ERR_UNSUPPORTED, "%s: batched N=%u not supported", fn, p.N);
    const dim3 grid(ceil_div(p.M, NW));
    if (qt == QType::Q4K)
      hipLaunchKernelGGL(gemv_q4k_generic, grid, dim3(NT), 0, ctx->stream, in, (const uint8_t*)w, out, p.M, p.N);
    else
      hipLaunchKernelGGL(gemv_q6k_generic, grid, dim3(NT), 0, ctx->stream, in, (const uint8_t*)w, out, p.M, p.N);
    G4_LAUNCHED(ctx, fn);
    return G4_OK;
  }
  int nv_max = 8;
  while (nv_max > 1 && xview_bytes(p.N, nv_max, false) > kMaxLds) nv_max >>= 1;
  uint32_t done = 0;
  while (done < batch) {
    const uint32_t left = batch - done;
    int nv = left >= 8 ? 8 : left >= 4 ? 4 : left >= 2 ? 2 : 1;
    if (nv > nv_max) nv = nv_max;
    GemvSeg s{(const uint8_t*)w, out + (size_t)done * p.M, p.M, 0};
    LaunchReq q{qt, &s, 1, p.N, nv, 0, ProArgs{in + (size_t)done * p.N, nullptr, nullptr, nullptr, nullptr, 0.f},
                p.M};
    rc = launch_gemv(ctx, q);
    if (rc) return rc == G4_ERR_UNSUPPORTED ? g4::set_error(rc, "%s: unsupported shape", fn) : rc;
    done += (uint32_t)nv;
  }
  return G4_OK;
}

size_t gateup_lds(uint32_t N) { return xview_bytes(N, 1, true); }

template <int BPR>
int launch_gateup(g4_ctx* ctx, const uint8_t* wg, const uint8_t* wu, float* out, uint32_t M, const ProArgs& pa) {
  constexpr int R = RowsFor<BPR>::R;
  const dim3 grid(ceil_div(M, R * NW));
  hipLaunchKernelGGL((gateup_q4k_kernel<BPR, R, 2>), grid, dim3(NT), gateup_lds(BPR * 256), ctx->stream, wg, wu,
                     out, M, pa);
  G4_LAUNCHED(ctx, "gateup_q4k");
  return G4_OK;
}

}  // namespace

extern "C" {

int g4_matmulQuant_q4k(g4_ctx* ctx, const float* input, const void* weight, float* output, g4_matmul_params p) {
  return matmul_quant(ctx, __func__, QType::Q4K, input, weight, output, p, 1);
}

int g4_matmulQuantMR4_q4k(g4_ctx* ctx, const float* input, const void* weight, float* output,
                          g4_matmul_params p) {
  return matmul_quant(ctx, __func__, QType::Q4K, input, weight, output, p, 1);
}

int g4_matmulQuant_q6k(g4_ctx* ctx, const float* input, const void* weight, float* output, g4_matmul_params p) {
  return matmul_quant(ctx, __func__, QType::Q6K, input, weight, output, p, 1);
}

int g4_matmulQuantBatch_q4k(g4_ctx* ctx, const float* input, const void* weight, float* output,
                            g4_matmul_params p, uint32_t batch) {
  return matmul_quant(ctx, __func__, QType::Q4K, input, weight, output, p, batch);
}

int g4_matmulQuantBatch_q6k(g4_ctx* ctx, const float* input, const void* weight, float* output,
                            g4_matmul_params p, uint32_t batch) {
  return matmul_quant(ctx, __func__, QType::Q6K, input, weight, output, p, batch);
}

int g4_matmulQuant_f16(g4_ctx* ctx, const float* input, const uint16_t* weight, float* output,
                       g4_matmul_params p) {
  G4_ENTER(ctx);
  G4_REQUIRE(input && weight && output, "g4_matmulQuant_f16: null buffer");
  G4_REQUIRE(p.M > 0 && p.N > 0 && p.N <= 16384, "g4_matmulQuant_f16: bad shape M=%u N=%u", p.M, p.N);
  G4_REQUIRE(((uintptr_t)weight & 15) == 0, "g4_matmulQuant_f16: weights must be 16-byte aligned");
  const dim3 grid(ceil_div(p.M, 4 * NW));
  hipLaunchKernelGGL(gemv_f16_kernel, grid, dim3(NT), p.N * sizeof(float), ctx->stream, input, weight, output,
                     p.M, p.N);
  G4_LAUNCHED(ctx, "gemv_f16");
  return G4_OK;
}

int g4_rmsNormMatmul_q4k(g4_ctx* ctx, const float* x, const uint16_t* norm_w, const void* weight, float* y,
                         g4_matmul_params p, float eps) {
  G4_ENTER(ctx);
  int rc = check_mm(__func__, x, weight, y, p);
  if (rc) return rc;
  G4_REQUIRE(norm_w, "g4_rmsNormMatmul_q4k: null norm weight");
  G4_REQUIRE(((uintptr_t)weight & 15) == 0, "g4_rmsNormMatmul_q4k: weights must be 16-byte aligned");
  G4_REQUIRE(supported_bpr(p.N / 256) && p.N <= 8192, "g4_rmsNormMatmul_q4k: N=%u unsupported", p.N);
  GemvSeg s{(const uint8_t*)weight, y, p.M, 0};
  LaunchReq q{QType::Q4K, &s, 1, p.N, 1, 1, ProArgs{x, norm_w, nullptr, nullptr, nullptr, eps}, p.M};
  return launch_gemv(ctx, q);
}

int g4_normAddGateUpGelu_q4k(g4_ctx* ctx, const float* o, const uint16_t* w_post, const float* residual,
                             const uint16_t* w_pre, const void* w_gate, const void* w_up, float* h_out,
                             float* out, g4_matmul_params p, float eps) {
  G4_ENTER(ctx);
  int rc = check_mm(__func__, o, w_gate, out, p);
  if (rc) return rc;
  G4_REQUIRE(w_post && residual && w_pre && w_up, "g4_normAddGateUpGelu_q4k: null buffer");
  G4_REQUIRE(((uintptr_t)w_gate & 15) == 0 && ((uintptr_t)w_up & 15) == 0,
             "g4_normAddGateUpGelu_q4k: weights must be 16-byte aligned");
  const ProArgs pa{o, w_post, residual, w_pre, h_out, eps};
  switch (p.N / 256) {
    case 6: return launch_gateup<6>(ctx, (const uint8_t*)w_gate, (const uint8_t*)w_up, out, p.M, pa);
    case 8: return launch_gateup<8>(ctx, (const uint8_t*)w_gate, (const uint8_t*)w_up, out, p.M, pa);
    case 16: return launch_gateup<16>(ctx, (const uint8_t*)w_gate, (const uint8_t*)w_up, out, p.M, pa);
    default: return g4::set_error(G4_ERR_UNSUPPORTED, "g4_normAddGateUpGelu_q4k: N=%u unsupported", p.N);
  }
}

}  // extern "C"
