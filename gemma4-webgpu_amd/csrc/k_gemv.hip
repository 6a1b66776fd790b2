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
//  * A wavefront owns R consecutive rows (one contiguous byte range) and each
//    lane one quarter of a super-block (Q4_K: one 32-byte group = 64 weights;
//    Q6_K: one 48-byte ql/ql/qh unit = 64 weights), 16 blocks per step. R is
//    the smallest row count that fills a wave (2 rows at K=1536), so a matrix
//    is spread over many waves and no wave runs a long serial stream.
//  * Order of work in a workgroup: the activation loads are issued first,
//    then every weight load of the tile, then the activation is normalised
//    and digitised in registers while the weights are in flight (loads
//    complete in issue order, so the small activation loads never wait
//    behind the weight stream).
//  * Per-row sums are folded across the wave with a halving butterfly.
//  * Fusions selected by template parameters: RMSNorm (or residual-add +
//    RMSNorm) prologue, softcap epilogue, several matrices sharing one input
//    per launch (q/k/v), gate/up pairs with the GELU product epilogue.
#include "g4_internal.hpp"
#include "mqf_core.hpp"

#include <algorithm>
#include <type_traits>

namespace {

constexpr int NW = 4;             // wavefronts per workgroup
constexpr int NT = NW * 64;       // threads per workgroup
constexpr int XSTRIDE = 288;      // LDS bytes per 256-element block of a digit plane (+32 pad)
constexpr float XQ = 32512.0f;    // digit range: |v| <= 32512 keeps both digits in [-128,127]
constexpr size_t kMaxLds = 65536; // LDS bytes one workgroup may claim

typedef uint32_t u32x4a __attribute__((ext_vector_type(4), aligned(4)));

__device__ __forceinline__ uint4 ld16(const uint8_t* p) { return *(const uint4*)p; }

__device__ __forceinline__ int plane_off(uint32_t e) { return (int)((e >> 8) * XSTRIDE + (e & 255)); }

// ---------------------------------------------------------------------------
// activation digits in LDS
// ---------------------------------------------------------------------------

struct XView {
  int8_t* hi;  // [NV][nb*XSTRIDE]
  int8_t* lo;  // [NV][nb*XSTRIDE]
  float* s;    // [NV][K/32]   scale of each 32-element sub-block
  float* sum;  // [NV][K/32]   sum of x over the sub-block (Q4_K min term)
  int2* c16;   // [NV][K/16]   32*sum(hi), 32*sum(lo) over each 16-run (Q6_K offset)
  float* red;  // [16]         block reductions
  uint32_t K;
  __device__ int plane_bytes() const { return (int)(K / 256) * XSTRIDE; }
};

__host__ __device__ constexpr size_t xview_bytes(uint32_t K, int NV) {
  const size_t nb = K / 256;
  size_t b = 2 * (size_t)NV * nb * XSTRIDE;
  b += 2 * (size_t)NV * (K / 32) * sizeof(float);
  b += (size_t)NV * (K / 16) * sizeof(int2);
  b += 16 * sizeof(float);
  return b;
}

__device__ inline XView carve(uint8_t* smem, uint32_t K, int NV) {
  XView v;
  v.K = K;
  const size_t nb = K / 256;
  uint8_t* p = smem;
  v.hi = (int8_t*)p;  p += (size_t)NV * nb * XSTRIDE;
  v.lo = (int8_t*)p;  p += (size_t)NV * nb * XSTRIDE;
  v.s = (float*)p;    p += (size_t)NV * (K / 32) * sizeof(float);
  v.sum = (float*)p;  p += (size_t)NV * (K / 32) * sizeof(float);
  v.c16 = (int2*)p;   p += (size_t)NV * (K / 16) * sizeof(int2);
  v.red = (float*)p;
  return v;
}

// Quantise 4 consecutive elements; lanes 8j..8j+7 hold one 32-element
// sub-block. All 64 lanes of the wave must call this together.
__device__ __forceinline__ void digits4(const XView& xv, int vec, uint32_t e, float4 x, bool active) {
  float am = fmaxf(fmaxf(fabsf(x.x), fabsf(x.y)), fmaxf(fabsf(x.z), fabsf(x.w)));
  float sm = (x.x + x.y) + (x.z + x.w);
#pragma unroll
  for (int o = 1; o < 8; o <<= 1) {
    am = fmaxf(am, __shfl_xor(am, o, 64));
    sm += __shfl_xor(sm, o, 64);
  }
  const float inv = am > 0.f ? XQ / am : 0.f;
  const float xs[4] = {x.x, x.y, x.z, x.w};
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
    if ((threadIdx.x & 7) == 0) {
      // a NaN or Inf input (sum not finite) makes the sub-block scale NaN,
      // so the products carry it as the reference's f32 matvec does
      xv.s[vec * (xv.K / 32) + e / 32] = __builtin_isfinite(sm) ? am * (1.0f / XQ) : __builtin_nanf("");
      xv.sum[vec * (xv.K / 32) + e / 32] = sm;
    }
    if ((threadIdx.x & 3) == 0) xv.c16[vec * (xv.K / 16) + e / 16] = make_int2(32 * shi, 32 * slo);
  }
}

// Prologue modes: 0 = x from global; 1 = x * w / rms(x) (shaders/rms_norm.wgsl);
// 2 = h = residual + o * w1 / rms(o); x = h * w2 / rms(h)
// (shaders/fused_norm_add.wgsl then shaders/rms_norm.wgsl); h is written to
// h_out by workgroup 0 when h_out is non-null; 3 (one-vector matvec, Q6_K)
// = x already digitised by the launch that produced it (MvD8 block at x);
// 4 (one-vector matvec) = mode 2 with o given as kOShares vectors of K
// (the o projection's shares by group of heads, [kOShares][K] at x),
// added in order.
__host__ __device__ constexpr bool pro_add(int pro) { return pro == 2 || pro == 4; }  // residual-add + norm
// The o projection split by groups of heads (attn_heads_kernel): fewer,
// wider groups trade the chunk partials each of its workgroups reads (8 KB
// per head) against the shares every gate/up workgroup reads ahead of its
// weights (6 KB each at hidden 1536).
constexpr int kHeadsPerWg = 2;
constexpr int kOShares = 8 / kHeadsPerWg;
static_assert(kOShares == G4_O_SHARES, "the ABI states the share count");

struct ProArgs {
  const float* x;         // [NV][K] (mode 2: o)
  const uint16_t* w1;
  const float* residual;
  const uint16_t* w2;
  float* h_out;
  float eps;
  const uint16_t* out_scale;  // mode 2: h = (residual + norm(x)) * f16 scale (NULL: 1)
};

// Thread t owns the float4s at flat element p*1024 + 4t (p < XP) of the
// NV x K activation block.
template <int NV, int K>
struct XRegs {
  static constexpr int XP = (NV * K + 1023) / 1024;
  float4 x[XP];
  float4 r[(NV == 1) ? XP : 1];      // residual (mode 2)
  uint2 w1[(NV == 1) ? XP : 1];      // f16 x4
  uint2 w2[(NV == 1) ? XP : 1];
};

template <int NV, int K, int PRO>
__device__ __forceinline__ void pro_load(XRegs<NV, K>& R, const ProArgs& a) {
  constexpr int XP = XRegs<NV, K>::XP;
#pragma unroll
  for (int p = 0; p < XP; ++p) {
    const uint32_t f = (uint32_t)p * 1024 + 4 * threadIdx.x;
    if (f < (uint32_t)(NV * K)) {
      R.x[p] = *(const float4*)(a.x + f);
      if constexpr (PRO >= 1) R.w1[p] = *(const uint2*)(a.w1 + f);
      if constexpr (PRO == 2) {
        R.r[p] = *(const float4*)(a.residual + f);
        R.w2[p] = *(const uint2*)(a.w2 + f);
      }
    } else {
      R.x[p] = make_float4(0.f, 0.f, 0.f, 0.f);
      if constexpr (PRO >= 1) R.w1[p] = make_uint2(0, 0);
      if constexpr (PRO == 2) {
        R.r[p] = R.x[p];
        R.w2[p] = R.w1[p];
      }
    }
  }
}

__device__ __forceinline__ float4 mul_w(float4 x, uint2 w, float s) {
  return make_float4(x.x * g4d::f16_bits_to_f32(w.x & 0xffffu) * s, x.y * g4d::f16_bits_to_f32(w.x >> 16) * s,
                     x.z * g4d::f16_bits_to_f32(w.y & 0xffffu) * s, x.w * g4d::f16_bits_to_f32(w.y >> 16) * s);
}

__device__ __forceinline__ float sumsq(float4 v) { return (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w); }

template <int NV, int K, int PRO>
__device__ __forceinline__ void pro_finish(XRegs<NV, K>& R, const XView& xv, const ProArgs& a) {
  constexpr int XP = XRegs<NV, K>::XP;
  if constexpr (PRO >= 1) {
    static_assert(NV == 1, "normalising prologues take one vector");
    float ss = 0.f;
#pragma unroll
    for (int p = 0; p < XP; ++p) ss += sumsq(R.x[p]);
    ss = g4d::block_sum<NW>(ss, xv.red);
    const float inv1 = 1.0f / sqrtf(ss / (float)K + a.eps);
    if constexpr (PRO == 1) {
#pragma unroll
      for (int p = 0; p < XP; ++p) R.x[p] = mul_w(R.x[p], R.w1[p], inv1);
    } else {
      float ss2 = 0.f;
      const float sc = a.out_scale ? g4d::f16_bits_to_f32(*a.out_scale) : 1.0f;
#pragma unroll
      for (int p = 0; p < XP; ++p) {
        const float4 t = mul_w(R.x[p], R.w1[p], inv1);
        const float4 h = make_float4((R.r[p].x + t.x) * sc, (R.r[p].y + t.y) * sc, (R.r[p].z + t.z) * sc,
                                     (R.r[p].w + t.w) * sc);
        R.x[p] = h;
        ss2 += sumsq(h);
        const uint32_t f = (uint32_t)p * 1024 + 4 * threadIdx.x;
        if (a.h_out && blockIdx.x == 0 && f < (uint32_t)K) *(float4*)(a.h_out + f) = h;
      }
      ss2 = g4d::block_sum<NW>(ss2, xv.red);
      const float inv2 = 1.0f / sqrtf(ss2 / (float)K + a.eps);
#pragma unroll
      for (int p = 0; p < XP; ++p) R.x[p] = mul_w(R.x[p], R.w2[p], inv2);
    }
  }
#pragma unroll
  for (int p = 0; p < XP; ++p) {
    const uint32_t f = (uint32_t)p * 1024 + 4 * threadIdx.x;
    const bool active = f < (uint32_t)(NV * K);
    const uint32_t fv = active ? f : 0;
    digits4(xv, (int)(fv / K), fv % K, R.x[p], active);
  }
  __syncthreads();
}

// ---------------------------------------------------------------------------
// weight tiles
// ---------------------------------------------------------------------------

// Q4_K scale/min pair for sub-blocks j = 2g and 2g+1 (src/gguf.ts:175-182).
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

// Q4_K 4-bit codes of one 32-bit word of qs (four weights of sub-blocks
// 2g and 2g + 1 of group g, src/gguf.ts:188-207): the low nibbles belong to
// sub-block 2g, the high nibbles to 2g + 1. Every Q4_K unit below extracts
// its codes with these (g4_dequantPath checks them against the oracle).
__device__ __forceinline__ uint32_t q4k_lo_codes(uint32_t w) { return w & 0x0f0f0f0fu; }
__device__ __forceinline__ uint32_t q4k_hi_codes(uint32_t w) { return (w >> 4) & 0x0f0f0f0fu; }

// Q6_K 6-bit codes (0..63, the value is code - 32) of run k of a half
// (elements 128h + 32k + l .. l + 3, src/gguf.ts:344-361) from the words A =
// ql[64h + l..], B = ql[64h + 32 + l..] and H = qh[32h + l..]; k is a
// compile-time constant at every call.
__device__ __forceinline__ uint32_t q6k_codes(int k, uint32_t A, uint32_t B, uint32_t H) {
  if (k == 0) return (A & 0x0f0f0f0fu) | ((H << 4) & 0x30303030u);
  if (k == 1) return (B & 0x0f0f0f0fu) | ((H << 2) & 0x30303030u);
  if (k == 2) return ((A >> 4) & 0x0f0f0f0fu) | (H & 0x30303030u);
  return ((B >> 4) & 0x0f0f0f0fu) | ((H >> 2) & 0x30303030u);
}

__device__ __forceinline__ int dot8(const uint32_t* q, const uint32_t* x) {
  int acc = 0;
#pragma unroll
  for (int k = 0; k < 8; ++k) acc = __builtin_amdgcn_sdot4((int)q[k], (int)x[k], acc, false);
  return acc;
}

// The weight bytes of a workgroup's row tile are one contiguous range. They
// are streamed with coalesced 16-byte loads (lane i of the workgroup takes
// bytes 16i, 16i + 16*NT, ...) into registers, then written to LDS, where
// each lane picks the pieces of the blocks it multiplies.
template <int QT>
struct BlockOf;
template <> struct BlockOf<0> { static constexpr int BYTES = 144; };
template <> struct BlockOf<1> { static constexpr int BYTES = 210; };

// A wave's share of a tile: R rows x BPR blocks, 4 lanes per block, 16
// blocks per step (the last step may be partial). A workgroup tile is the
// NW*R consecutive rows of its waves.
template <int QT, int BPR, int R>
struct Tile {
  static constexpr int BYTES = BlockOf<QT>::BYTES;
  static constexpr int NB = R * BPR;
  static constexpr int IT = (NB + 15) / 16;
  static constexpr int ROWS_WG = R * NW;
  static constexpr uint32_t WAVE_B = (uint32_t)NB * BYTES;  // R rows
  static constexpr uint32_t WG_B = NW * WAVE_B;             // ROWS_WG rows
  static_assert(WG_B == (uint32_t)ROWS_WG * BPR * BYTES, "a tile is ROWS_WG whole rows");
  static constexpr int LPT = (int)((WG_B + 16 * NT - 1) / (16 * NT));  // 16-byte loads per thread
  static constexpr uint32_t LDS_B = (WG_B + 15) / 16 * 16;
};

template <int LPT>
struct Stage {
  u32x4a r[LPT];
};

// Chunk i of a tile of nbytes (nbytes >= 16) is read from and stored to the
// same offset: 16*i, or for the last, partial chunk (and lanes past the end)
// the 16 bytes that end the tile, which overlap the chunk before them with
// identical bytes. The loaded values are only stored, never computed on, and
// the load sits under no branch: any arithmetic on them (or a branch around
// a load) lets the compiler move a wait for the whole weight stream into the
// activation prologue.
__device__ __forceinline__ uint32_t chunk_off(uint32_t off, uint32_t nbytes) {
  return off + 16 <= nbytes ? off : nbytes - 16;
}

// Issues the loads of bytes [0, nbytes) of a tile starting at src (4-byte aligned).
template <class T>
__device__ __forceinline__ void stage_load(const uint8_t* src, uint32_t nbytes, Stage<T::LPT>& st) {
#pragma unroll
  for (int i = 0; i < T::LPT; ++i)
    st.r[i] = *(const u32x4a*)(src + chunk_off((uint32_t)(i * NT + threadIdx.x) * 16u, nbytes));
}

template <class T>
__device__ __forceinline__ void stage_store(uint8_t* lds, uint32_t nbytes, const Stage<T::LPT>& st) {
#pragma unroll
  for (int i = 0; i < T::LPT; ++i) {
    const uint32_t off = (uint32_t)(i * NT + threadIdx.x) * 16u;
    if (off < T::LDS_B) *(u32x4a*)(lds + chunk_off(off, nbytes)) = st.r[i];
  }
}

// 16 bytes at a 2-byte aligned LDS address, from three 8-byte aligned
// reads (wider reads at a weaker alignment stall the LDS pipeline). The
// aligned address is derived from p by pointer arithmetic: a round trip
// through an integer would lose the LDS address space and turn the reads
// into flat loads, which also wait on every global load in flight.
__device__ __forceinline__ void lds_piece(const uint8_t* p, uint32_t (&w)[4]) {
  const uint32_t mis = (uint32_t)(uintptr_t)p & 7u;
  const uint2* p8 = (const uint2*)(p - mis);
  const uint2 b0 = p8[0], b1 = p8[1], b2 = p8[2];
  const bool hi = (mis & 4) != 0;  // skip one dword
  const uint32_t sh = mis & 3;
  const uint32_t a0 = hi ? b0.y : b0.x, a1 = hi ? b1.x : b0.y, a2 = hi ? b1.y : b1.x;
  const uint32_t a3 = hi ? b2.x : b1.y, a4 = hi ? b2.y : b2.x;
  w[0] = __builtin_amdgcn_alignbyte(a1, a0, sh);
  w[1] = __builtin_amdgcn_alignbyte(a2, a1, sh);
  w[2] = __builtin_amdgcn_alignbyte(a3, a2, sh);
  w[3] = __builtin_amdgcn_alignbyte(a4, a3, sh);
}

// Q4_K unit g (a quarter block: sub-blocks 2g, 2g + 1) of a block in LDS:
// the 16-byte header and the unit's 32 quant bytes (qs[32g..32g + 31]).
__device__ __forceinline__ void q4_lds_unit(const uint8_t* blk, int g, uint4& hd, uint32_t (&qa)[8]) {
  hd = *(const uint4*)blk;
  const uint4 q0 = *(const uint4*)(blk + 16 + 32 * g);
  const uint4 q1 = *(const uint4*)(blk + 32 + 32 * g);
  qa[0] = q0.x; qa[1] = q0.y; qa[2] = q0.z; qa[3] = q0.w;
  qa[4] = q1.x; qa[5] = q1.y; qa[6] = q1.z; qa[7] = q1.w;
}

// Q6_K unit g of a block in LDS (half h = g >> 1, l0 = 16 (g & 1)): the
// 16-byte runs ql[64h + l0..], ql[64h + 32 + l0..], qh[32h + l0..], the
// unit's scales sc[8h + (g & 1) + 2k] and d (src/gguf.ts:323-364).
__device__ __forceinline__ void q6_lds_unit(const uint8_t* blk, int g, uint32_t (&A)[4], uint32_t (&B)[4],
                                            uint32_t (&H)[4], int32_t (&scs)[4], float& dd) {
  const int h = g >> 1, l0 = (g & 1) * 16;
  lds_piece(blk + 64 * h + l0, A);
  lds_piece(blk + 64 * h + 32 + l0, B);
  lds_piece(blk + 128 + 32 * h + l0, H);
  const int8_t* scp = (const int8_t*)(blk + 192 + 8 * h + (g & 1));
#pragma unroll
  for (int k = 0; k < 4; ++k) scs[k] = scp[2 * k];
  dd = g4d::f16_bits_to_f32(*(const uint16_t*)(blk + 208));
}

// partial dot of quarter g of the Q4_K block at blk (LDS) with vector v
__device__ __forceinline__ float q4_part(const XView& xv, const uint8_t* blk, int g, uint32_t b, int v) {
  uint4 hd;
  uint32_t qa[8];
  q4_lds_unit(blk, g, hd, qa);
  const float d = g4d::f16_bits_to_f32(hd.x & 0xffffu);
  const float dmin = g4d::f16_bits_to_f32(hd.x >> 16);
  float sc_lo, sc_hi, m_lo, m_hi;
  q4k_scales(hd.y, hd.z, hd.w, g, sc_lo, sc_hi, m_lo, m_hi);
  uint32_t nl[8], nh[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    nl[k] = q4k_lo_codes(qa[k]);
    nh[k] = q4k_hi_codes(qa[k]);
  }
  const uint32_t e0 = b * 256 + 64u * g;
  const int sub = (int)(e0 / 32);
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
  float part = (d * sc_lo) * s[sub] * (float)ilo - (dmin * m_lo) * sm[sub];
  part += (d * sc_hi) * s[sub + 1] * (float)ihi - (dmin * m_hi) * sm[sub + 1];
  return part;
}

// Q6_K quarter u of the block at blk (LDS): h = u >> 1, l0 = 16 (u & 1):
// ql[64h+l0..], ql[64h+32+l0..], qh[32h+l0..] (16 bytes each), scales
// sc[8h + (u&1) + 2k], d.
__device__ __forceinline__ float q6_part(const XView& xv, const uint8_t* blk, int u, uint32_t b, int v) {
  const int h = u >> 1, l0 = (u & 1) * 16;
  uint32_t A[4], B[4], H[4];
  int32_t scs[4];
  float dd;
  q6_lds_unit(blk, u, A, B, H, scs, dd);
  // run k covers elements 128h + 32k + l0 + [0,16) (src/gguf.ts:344-361)
  uint32_t q[4][4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
#pragma unroll
    for (int k = 0; k < 4; ++k) q[k][j] = q6k_codes(k, A[j], B[j], H[j]);
  }
  float part = 0.f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t e = b * 256 + 128u * h + 32u * k + l0;
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
    part += (float)scs[k] * xv.s[v * (xv.K / 32) + e / 32] * (float)I;
  }
  return part * dd;
}

// Multiplies the wave's R rows (at wl in LDS) with the NV activation vectors.
template <int QT, int BPR, int R, int NV>
__device__ __forceinline__ void tile_compute(const XView& xv, const uint8_t* wl, float (&acc)[NV * R]) {
  using T = Tile<QT, BPR, R>;
  const int lane = threadIdx.x & 63;
  const int u = lane & 3, bl = lane >> 2;
#pragma unroll
  for (int it = 0; it < T::IT; ++it) {
    const int fb = it * 16 + bl;
    const bool live = fb < T::NB;
    const int fbc = live ? fb : T::NB - 1;  // idle lanes of a partial step read a valid block
    const int r = fbc / BPR;
    const uint32_t b = (uint32_t)(fbc % BPR);
    const uint8_t* blk = wl + fbc * T::BYTES;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      float part;
      if constexpr (QT == 0) part = q4_part(xv, blk, u, b, v);
      else part = q6_part(xv, blk, u, b, v);
      if (!live) part = 0.f;
      // rows a lane can touch at this step are known at compile time
#pragma unroll
      for (int rr = (it * 16) / BPR; rr <= (it * 16 + 15) / BPR && rr < R; ++rr)
        acc[v * R + rr] += (r == rr) ? part : 0.f;
    }
  }
}

// Halving butterfly: reduces N (power of two) per-lane values across the
// wave; afterwards lane L with L % (64/N) == 0 holds the sum of value L/(64/N).
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

__device__ __forceinline__ float softcap(float y, float cap) {
  const float t = fminf(fmaxf(y / cap, -15.0f), 15.0f);
  return tanhf(t) * cap;
}

struct GemvSeg {
  const uint8_t* W;
  float* Y;
  uint32_t M;
  uint32_t wg_begin;  // first workgroup of this segment
  uint64_t* stage;    // DEV rows: also staged as (1 << 32 | f32 bits) pairs here, [M]
};
struct GemvSegs {
  GemvSeg s[4];
  int n;
  uint32_t rep;     // consecutive row tiles per workgroup
  g4d::Cand* amx;   // mv_kernel, one matrix: per-workgroup argmax candidate of the stored rows, or null
  uint8_t* d8;      // mv_kernel, gate/up pair: the outputs also as an MvD8 block (K = rows), or null
  // mv_kernel, one matrix: per-workgroup top-k candidates (each residue
  // class's first strict maximum among the stored rows), [256][tk_stride], or null
  g4d::Cand* tk;
  uint32_t tk_stride;
};

// EPI: 0 = store y, 1 = store softcap(y) (shaders/logit_softcap.wgsl).
// A workgroup walks `rep` consecutive tiles of NW*R rows with one activation
// prologue, loading the next tile's weights while it computes the current one.
// LDS layout of a workgroup: activation digits, then the weight tile(s).
__host__ __device__ constexpr size_t align16(size_t b) { return (b + 15) / 16 * 16; }

template <int QT, int BPR, int R>
__device__ __forceinline__ uint32_t tile_bytes(uint32_t M, uint32_t t) {
  using T = Tile<QT, BPR, R>;
  const uint64_t total = (uint64_t)M * BPR * T::BYTES;
  const uint64_t o = (uint64_t)t * T::WG_B;
  return o >= total ? 0u : (uint32_t)min((uint64_t)T::WG_B, total - o);
}

// EPI: 0 = store y, 1 = store softcap(y) (shaders/logit_softcap.wgsl).
// A workgroup walks `rep` consecutive tiles of NW*R rows with one activation
// prologue; the next tile's loads are in flight while it computes the current one.
template <int QT, int BPR, int R, int NV, int PRO, int EPI>
__global__ __launch_bounds__(NT) void gemv_kernel(GemvSegs segs, ProArgs pa, uint32_t ldy, float cap) {
  using T = Tile<QT, BPR, R>;
  constexpr int K = BPR * 256;
  extern __shared__ __align__(16) uint8_t smem[];
  int si = 0;
#pragma unroll
  for (int i = 1; i < 4; ++i)
    if (i < segs.n && blockIdx.x >= segs.s[i].wg_begin) si = i;
  const GemvSeg sg = segs.s[si];
  const uint32_t tiles = (sg.M + T::ROWS_WG - 1) / T::ROWS_WG;
  const uint32_t tb = (blockIdx.x - sg.wg_begin) * segs.rep;
  const uint32_t te = min(tiles, tb + segs.rep);
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;

  XRegs<NV, K> xr;
  pro_load<NV, K, PRO>(xr, pa);
  __builtin_amdgcn_sched_barrier(0);
  Stage<T::LPT> st;
  uint32_t nb = tile_bytes<QT, BPR, R>(sg.M, tb);
  stage_load<T>(sg.W + (size_t)tb * T::WG_B, nb, st);
  __builtin_amdgcn_sched_barrier(0);
  const XView xv = carve(smem, K, NV);
  uint8_t* wl = smem + align16(xview_bytes(K, NV));
  pro_finish<NV, K, PRO>(xr, xv, pa);

  for (uint32_t t = tb; t < te; ++t) {
    if (t != tb) __syncthreads();  // every wave is done with the previous tile
    stage_store<T>(wl, nb, st);
    __syncthreads();
    if (t + 1 < te) {
      nb = tile_bytes<QT, BPR, R>(sg.M, t + 1);
      stage_load<T>(sg.W + (size_t)(t + 1) * T::WG_B, nb, st);
    }
    float acc[NV * R];
#pragma unroll
    for (int i = 0; i < NV * R; ++i) acc[i] = 0.f;
    tile_compute<QT, BPR, R, NV>(xv, wl + wave * T::WAVE_B, acc);
    const float y = wave_fold<NV * R>(acc);
    constexpr int G = 64 / (NV * R);
    const uint32_t row0 = t * T::ROWS_WG + wave * R;
    if ((lane % G) == 0) {
      const int idx = lane / G;
      const int vec = idx / R, rr = idx % R;
      if (row0 + rr < sg.M) sg.Y[(size_t)vec * ldy + row0 + rr] = EPI == 1 ? softcap(y, cap) : y;
    }
  }
}

// gate/up pair with the tanh-GELU product epilogue (shaders/gelu_mul.wgsl:10-16):
// out[i] = gelu(gate[i]) * up[i]; both matrices are [M, BPR*256] Q4_K.
using g4d::gelu_tanh;

// ---------------------------------------------------------------------------
// M=1 matvec with register-resident activation digits
// ---------------------------------------------------------------------------
//
// Thread (slot, unit): unit u = 4b + g is one quarter of super-block b, i.e.
// 64 weights of every row. The thread holds the digits of those 64
// activations in registers for the whole launch and multiplies them with the
// matching quarter of the row its slot owns in each tile, reading the
// weight bytes from the tile staged in LDS. Per-row partials meet in an LDS
// buffer, where a group of lanes per row adds them up. The digits are
// computed once per workgroup from coalesced loads, eight lanes per 32-element
// sub-block exchanging their maxima and sums through DPP.

// NWV waves per workgroup; a tile is one row per slot.
template <int BPR, int NWV>
struct MvGeom {
  static constexpr int U = 4 * BPR;                // units per row
  static constexpr int NTH = 64 * NWV;             // threads per workgroup
  static constexpr int SLOTS = NTH / U;            // rows in flight
  static constexpr int NSB = BPR * 8;              // 32-element sub-blocks
  static_assert(SLOTS >= 1 && SLOTS * U == NTH, "slots tile the workgroup exactly");
};

template <int QT, int BPR, int NWV>
struct MvTile {
  using G = MvGeom<BPR, NWV>;
  static constexpr int BYTES = BlockOf<QT>::BYTES;
  static constexpr int TR = G::SLOTS;             // rows per tile
  static constexpr uint32_t RB = BPR * BYTES;     // bytes per row
  static constexpr uint32_t TB = TR * RB;         // bytes per tile
  static constexpr int LPT = (int)((TB + 16 * G::NTH - 1) / (16 * G::NTH));
  static constexpr uint32_t LDS_T = (TB + 15) / 16 * 16;
  static constexpr int RS = G::U + 4;             // reduction row stride (floats)
  // a row's U partials are added by RG lanes of one wave, U / RG each
  static constexpr int RG = (G::U & -G::U) < 64 ? (G::U & -G::U) : 64;
  static_assert(G::U % RG == 0 && 64 % RG == 0, "reduction groups stay inside a wave");
};

// LDS layout: digits | sub-block scales | sums | 16-run offsets | block-sum slots | reductions | tiles
template <int BPR>
struct MvX {
  static constexpr int K = BPR * 256;
  static constexpr int NSB = BPR * 8;
  static constexpr size_t HI = 0, LO = K, S = 2 * (size_t)K, SUM = S + 4 * NSB, C16 = SUM + 4 * NSB,
                          RED8 = C16 + 16 * NSB, END = RED8 + 256;  // a 4-wide block sum of up to 16 waves
};

// Pre-digitised activations ("D8"), the same bytes in global memory and in
// LDS: the two digit planes, then one scale per 8 elements, then 32 x the
// digit sums of each 8 (the Q6_K -32 offset term). A producer that holds 8
// consecutive outputs in one wave (the gate/up launch's GELU rows) writes
// them, so the consumer (the down matvec) skips the per-element prologue.
template <int BPR>
struct MvD8 {
  static constexpr int K = BPR * 256;
  static constexpr size_t HI = 0, LO = K, S = 2 * (size_t)K, C = S + 4 * (size_t)(K / 8), BYTES = C + 8 * (size_t)(K / 8);
};
__host__ __device__ constexpr size_t d8_bytes(uint32_t K) { return 2 * (size_t)K + 12 * (size_t)(K / 8); }

// End of the activation area (and its block-sum slots) for a prologue mode.
template <int BPR, int PRO>
struct MvXA {
  static constexpr size_t RED8 = PRO == 3 ? align16(MvD8<BPR>::BYTES) : MvX<BPR>::RED8;
  static constexpr size_t END = RED8 + 256;
};

// A one-matrix workgroup that walks several tiles (the LM head) reads them
// straight into LDS (global -> LDS loads, no registers) into a ring of
// MvRing::D tile buffers, so that D - 1 tiles are in flight while one is
// multiplied. Lane l of wave w writes the 16-byte chunk 64 w + l of each
// round of NTH chunks, so a buffer spans whole waves' 1024-byte pieces.
// The ring takes as many buffers (3 to 6: two to five tiles in flight) as
// fit next to the activation digits and the row partials in kRingLds bytes
// of LDS (the top-k class table, 2 KB, comes on top).
constexpr uint32_t kRingLds = 152u * 1024u;
template <int QT, int BPR, int NWV>
struct MvRing {
  using T = MvTile<QT, BPR, NWV>;
  static constexpr uint32_t CH = (T::TB + 15) / 16;               // 16-byte chunks of a tile
  static constexpr uint32_t BUF = (CH + 63) / 64 * 1024;          // bytes of one ring buffer
  static constexpr uint32_t FREE = kRingLds - (uint32_t)align16(MvX<BPR>::END) - (uint32_t)align16(T::TR * T::RS * 4);
  static constexpr int D = FREE / BUF < 3 ? 3 : (FREE / BUF > 6 ? 6 : (int)(FREE / BUF));
  static constexpr int LPT = T::LPT;                              // rounds of loads per tile
  static constexpr uint32_t LAST = (uint32_t)(LPT - 1) * 64 * NWV;  // first chunk of the last round
};

// A workgroup with one tile reads its weight units straight into registers;
// one that walks several tiles stages them through LDS (`staged`): the
// ring of MvRing buffers for one matrix, one register-staged tile per
// matrix for a pair.
template <int QT, int BPR, int NWV, int PRO, int NMAT>
__host__ __device__ constexpr size_t mv_lds_bytes(bool staged) {
  using T = MvTile<QT, BPR, NWV>;
  return align16(MvXA<BPR, PRO>::END) + NMAT * align16((size_t)T::TR * T::RS * 4) +
         (staged ? (NMAT == 1 ? MvRing<QT, BPR, NWV>::D * (size_t)MvRing<QT, BPR, NWV>::BUF
                              : NMAT * (size_t)T::LDS_T)
                 : 0);
}

template <class T, int NTH>
__device__ __forceinline__ void mv_stage_load(const uint8_t* src, uint32_t nbytes, Stage<T::LPT>& st) {
#pragma unroll
  for (int i = 0; i < T::LPT; ++i)
    st.r[i] = *(const u32x4a*)(src + chunk_off((uint32_t)(i * NTH + threadIdx.x) * 16u, nbytes));
}

template <class T, int NTH>
__device__ __forceinline__ void mv_stage_store(uint8_t* lds, uint32_t nbytes, const Stage<T::LPT>& st) {
#pragma unroll
  for (int i = 0; i < T::LPT; ++i) {
    const uint32_t off = (uint32_t)(i * NTH + threadIdx.x) * 16u;
    if (off < T::LDS_T) *(u32x4a*)(lds + chunk_off(off, nbytes)) = st.r[i];
  }
}

// Issues the global -> LDS loads of a tile of nbytes at src into the ring
// buffer at buf: round i's chunk 64 w + l of wave w, lane l, goes to byte
// 16 (i NTH + 64 w + l) of the buffer; a chunk past the tile (lanes of the
// last round, or a short last tile) reads the tile's last 16 bytes, which
// land past the bytes any row reads. A wave issues a round only if some of
// its chunks are in the full tile, so it issues the same count for every
// tile (mv_ring_rounds).
template <int QT, int BPR, int NWV>
__device__ __forceinline__ void mv_ring_load(const uint8_t* src, uint32_t nbytes, uint8_t* buf, int w, int l) {
  using R = MvRing<QT, BPR, NWV>;
  constexpr int NTH = 64 * NWV;
#pragma unroll
  for (int i = 0; i < R::LPT; ++i) {
    const uint32_t c0 = (uint32_t)(i * NTH + 64 * w);  // (uniform per wave)
    if (i == R::LPT - 1 && c0 >= R::CH) break;
    const uint32_t off = chunk_off((c0 + (uint32_t)l) * 16u, nbytes);
    // non-temporal: each weight byte is read once per pass (the amortised
    // 262144 x 1536 Q4_K matvec: 45-46 -> 39-40 us, 61-63 -> 72-73 % of HBM)
    __builtin_amdgcn_global_load_lds((const void*)(src + off),
                                     (__attribute__((address_space(3))) void*)(buf + 16u * c0), 16, 0, 2);
  }
}
// Loads one tile issues in wave w: R::LPT, or one less where the last
// round has no chunk of the tile for it.
template <int QT, int BPR, int NWV>
__device__ __forceinline__ bool mv_ring_short(int w) {
  using R = MvRing<QT, BPR, NWV>;
  return R::LAST + 64u * (uint32_t)w >= R::CH;
}
// Workgroup barrier of the LDS ring: waits for this wave's LDS operations
// only. lds_barrier's release fence on LDS also waits for every global ->
// LDS load in flight (they write LDS), which would drain the two tiles the
// ring keeps in flight; the loads of the tile about to be read are waited
// for explicitly (wait_vmcnt) before this barrier. The memory clobber keeps
// the compiler from moving LDS accesses across it.
__device__ __forceinline__ void ring_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// s_waitcnt for vector memory count <= n (the other counters left free).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt field");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
// Waits until at most `ahead` tiles of PER loads each remain in flight
// (ahead < D - 1, a runtime value: one compile-time wait per case).
template <int PER, int D>
__device__ __forceinline__ void wait_tiles(uint32_t ahead) {
  static_assert(D >= 3 && D <= 6, "ring depth");
  switch (ahead) {
    case 0: wait_vmcnt<0>(); break;
    case 1: wait_vmcnt<PER>(); break;
    case 2: if constexpr (D > 3) wait_vmcnt<2 * PER>(); break;
    case 3: if constexpr (D > 4) wait_vmcnt<3 * PER>(); break;
    default: if constexpr (D > 5) wait_vmcnt<4 * PER>(); break;
  }
}

template <int QT, int BPR, int NWV>
__device__ __forceinline__ uint32_t mv_tile_bytes(uint32_t M, uint32_t t) {
  using T = MvTile<QT, BPR, NWV>;
  const uint64_t total = (uint64_t)M * T::RB;
  const uint64_t o = (uint64_t)t * T::TB;
  return o >= total ? 0u : (uint32_t)min((uint64_t)T::TB, total - o);
}

using g4d::dpp;
using g4d::dppi;
using g4d::kDppXor1;
using g4d::kDppXor2;
using g4d::kDppHalfMirror;
using g4d::wave_sum_dpp;

// Sum over the workgroup with one barrier; `red` holds NWV floats not reused
// by another sum before the next barrier.
// Workgroup barrier that orders LDS accesses only: it waits for the wave's
// LDS operations, not for its global loads and stores in flight (a plain
// __syncthreads also waits for every outstanding load, prefetched weights
// included, whenever a global store precedes it).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

template <int NWV>
__device__ __forceinline__ float block_sum_1(float v, float* red) {
  v = wave_sum_dpp(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  lds_barrier();
  float t = 0.f;
#pragma unroll
  for (int i = 0; i < NWV; ++i) t += red[i];
  return t;
}

// Four block-wide sums at once (one barrier); `red` holds >= 4 * NWV floats,
// 16-byte aligned.
template <int NWV>
__device__ __forceinline__ float4 block_sum_4(float4 v, float* red) {
  v.x = wave_sum_dpp(v.x);
  v.y = wave_sum_dpp(v.y);
  v.z = wave_sum_dpp(v.z);
  v.w = wave_sum_dpp(v.w);
  if ((threadIdx.x & 63) == 0) *(float4*)(red + 4 * (threadIdx.x >> 6)) = v;
  lds_barrier();
  float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int i = 0; i < NWV; ++i) {
    const float4 r = *(const float4*)(red + 4 * i);
    t.x += r.x;
    t.y += r.y;
    t.z += r.z;
    t.w += r.w;
  }
  return t;
}

// Activation registers of one prologue thread: the float4 at element
// 4*tid + 4*PTH*p. Eight consecutive lanes hold one 32-element sub-block.
// Only the first PW waves (one per SIMD) load, normalise and digitise the
// vector; the others go straight to the barrier that publishes the digits.
// A SIMD issues one wave64 VALU instruction per 4 cycles whichever wave it
// comes from, and the prologue's per-wave part (block sums, the norm
// scalars) is the same in every wave that runs it, so spreading the vector
// over all waves only multiplies that part on the SIMDs holding two or
// three of them.
template <int BPR, int NWV, int PRO>
struct MvPro {
  static constexpr int K = BPR * 256;
  static constexpr int PW = NWV >= 4 ? 4 : NWV;  // prologue waves
  static constexpr int PTH = 64 * PW;
  static constexpr int XP = (K + 4 * PTH - 1) / (4 * PTH);
  float4 x[XP];
  float4 r[pro_add(PRO) ? XP : 1];
  uint2 w1[PRO >= 1 ? XP : 1];
  uint2 w2[pro_add(PRO) ? XP : 1];
  // Every workgroup reads the whole vector; starting each one at a different
  // sub-block spreads these broadcast reads over the L2 channels instead of
  // all workgroups asking for the same lines at the same moment.
  __device__ static int rot() { return (int)((blockIdx.x * 37u) % (uint32_t)(K / 32)) * 32; }
  __device__ static bool active() { return (int)threadIdx.x < PTH; }  // (wave-uniform)
  __device__ static int slot(int p) { return 4 * (int)threadIdx.x + 4 * PTH * p; }
  __device__ static bool live(int p) { return slot(p) < K; }
  // element held at round p (valid when live(p))
  __device__ static int elem(int p) {
    const int f = slot(p) + rot();
    return f >= K ? f - K : f;
  }
};

template <int BPR, int NWV, int PRO>
__device__ __forceinline__ void mv_pro_load(MvPro<BPR, NWV, PRO>& P, const ProArgs& a) {
  using PP = MvPro<BPR, NWV, PRO>;
  if (!PP::active()) return;
  // Unconditional loads (see chunk_off). Lanes past K read element 0 again;
  // they form whole 8-lane sub-block groups whose digits are never stored,
  // and their squares are masked out of the norms.
#pragma unroll
  for (int p = 0; p < PP::XP; ++p) {
    const int fc = PP::live(p) ? PP::elem(p) : 0;
    if constexpr (PRO == 4) {
      float4 part[kOShares];
#pragma unroll
      for (int i = 0; i < kOShares; ++i) part[i] = *(const float4*)(a.x + (size_t)i * PP::K + fc);
      float4 v = part[0];
#pragma unroll
      for (int i = 1; i < kOShares; ++i) v = make_float4(v.x + part[i].x, v.y + part[i].y, v.z + part[i].z,
                                                         v.w + part[i].w);
      P.x[p] = v;
    } else {
      P.x[p] = *(const float4*)(a.x + fc);
    }
    if constexpr (PRO >= 1) P.w1[p] = *(const uint2*)(a.w1 + fc);
    if constexpr (pro_add(PRO)) {
      P.r[p] = *(const float4*)(a.residual + fc);
      P.w2[p] = *(const uint2*)(a.w2 + fc);
    }
  }
}

// The prologue waves' activations as 8-bit digit pairs, per-sub-block scales,
// sums and 16-run digit sums in LDS.
template <int BPR, int NWV, int PRO>
__device__ __forceinline__ void mv_digitize(const MvPro<BPR, NWV, PRO>& P, uint8_t* smem) {
  using PP = MvPro<BPR, NWV, PRO>;
  using X = MvX<BPR>;
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int p = 0; p < PP::XP; ++p) {
    const int f = PP::elem(p);
    const bool lv = PP::live(p);
    const float4 v = P.x[p];
    float am = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    float sm = (v.x + v.y) + (v.z + v.w);
    am = fmaxf(am, dpp<kDppXor1>(am));
    sm += dpp<kDppXor1>(sm);
    am = fmaxf(am, dpp<kDppXor2>(am));
    sm += dpp<kDppXor2>(sm);
    am = fmaxf(am, dpp<kDppHalfMirror>(am));
    sm += dpp<kDppHalfMirror>(sm);
    // hardware reciprocal (1 ulp): |x * inv| stays below XQ + 0.01, so the
    // rounded digits keep |q| <= XQ
    const float inv = am > 0.f ? XQ * __builtin_amdgcn_rcpf(am) : 0.f;
    const float xs[4] = {v.x, v.y, v.z, v.w};
    uint32_t ph = 0, pl = 0;
    int shi = 0, slo = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int q = (int)__builtin_rintf(xs[e] * inv);
      const int lo = ((q + 128) & 255) - 128;
      const int hi = (q - lo) >> 8;
      shi += hi;
      slo += lo;
      ph |= (uint32_t)(hi & 255) << (8 * e);
      pl |= (uint32_t)(lo & 255) << (8 * e);
    }
    shi += dppi<kDppXor1>(shi);
    slo += dppi<kDppXor1>(slo);
    shi += dppi<kDppXor2>(shi);
    slo += dppi<kDppXor2>(slo);
    if (lv) {
      *(uint32_t*)(smem + X::HI + f) = ph;
      *(uint32_t*)(smem + X::LO + f) = pl;
      if ((lane & 7) == 0) {
        // non-finite input: a NaN scale carries it into every product
        ((float*)(smem + X::S))[f / 32] = __builtin_isfinite(sm) ? am * (1.0f / XQ) : __builtin_nanf("");
        ((float*)(smem + X::SUM))[f / 32] = sm;
      }
      if ((lane & 3) == 0) ((int2*)(smem + X::C16))[f / 16] = make_int2(32 * shi, 32 * slo);
    }
  }
}

// 1 / sqrt(ss / K + eps) with the hardware reciprocal square root (1 ulp).
template <int K>
__device__ __forceinline__ float mv_inv_rms(float ss, float eps) {
  return __builtin_amdgcn_rsqf(ss * (1.0f / (float)K) + eps);
}

// Normalises (PRO 1/2) and digitises the activations into LDS, then barrier.
// Every wave of the workgroup calls it (it holds the barriers); only the
// prologue waves compute.
template <int BPR, int NWV, int PRO>
__device__ __forceinline__ void mv_pro_finish(MvPro<BPR, NWV, PRO>& P, uint8_t* smem, const ProArgs& a) {
  using PP = MvPro<BPR, NWV, PRO>;
  using X = MvX<BPR>;
  float* red8 = (float*)(smem + X::RED8);
  const bool act = PP::active();
  const int wv = (int)threadIdx.x >> 6;
  if constexpr (PRO == 1) {
    if (act) {
      float ss = 0.f;
#pragma unroll
      for (int p = 0; p < PP::XP; ++p) {
        const float q = sumsq(P.x[p]);
        ss += PP::live(p) ? q : 0.f;
      }
      ss = wave_sum_dpp(ss);
      if ((threadIdx.x & 63) == 0) red8[wv] = ss;
    }
    lds_barrier();
    if (act) {
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < PP::PW; ++i) ss += red8[i];
      const float inv1 = mv_inv_rms<X::K>(ss, a.eps);
#pragma unroll
      for (int p = 0; p < PP::XP; ++p) P.x[p] = mul_w(P.x[p], P.w1[p], inv1);
    }
  } else if constexpr (pro_add(PRO)) {
    // h = r + t, t = (o * w1) * inv1. Both norms come out of one block
    // reduction: sum(o^2), and sum(h^2) expanded as
    // sum(r^2) + 2 inv1 sum(r (o w1)) + inv1^2 sum((o w1)^2).
    float4 ow[PP::XP];
    if (act) {
      float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int p = 0; p < PP::XP; ++p) {
        ow[p] = mul_w(P.x[p], P.w1[p], 1.0f);
        const float4 o = P.x[p], r = P.r[p], t = ow[p];
        const float so = sumsq(o), sr = sumsq(r), st = sumsq(t);
        const float rt = (r.x * t.x + r.y * t.y) + (r.z * t.z + r.w * t.w);
        const bool lv = PP::live(p);
        acc.x += lv ? so : 0.f;
        acc.y += lv ? sr : 0.f;
        acc.z += lv ? rt : 0.f;
        acc.w += lv ? st : 0.f;
      }
      acc.x = wave_sum_dpp(acc.x);
      acc.y = wave_sum_dpp(acc.y);
      acc.z = wave_sum_dpp(acc.z);
      acc.w = wave_sum_dpp(acc.w);
      if ((threadIdx.x & 63) == 0) *(float4*)(red8 + 4 * wv) = acc;
    }
    lds_barrier();
    if (act) {
      float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int i = 0; i < PP::PW; ++i) {
        const float4 r = *(const float4*)(red8 + 4 * i);
        acc.x += r.x;
        acc.y += r.y;
        acc.z += r.z;
        acc.w += r.w;
      }
      const float inv1 = mv_inv_rms<X::K>(acc.x, a.eps);
      // with an output scale s, h = s (r + t inv1) and sum(h^2) = s^2 times the above
      const float sc = a.out_scale ? g4d::f16_bits_to_f32(*a.out_scale) : 1.0f;
      const float ss2 = fmaxf(acc.y + 2.0f * inv1 * acc.z + inv1 * inv1 * acc.w, 0.f) * (sc * sc);
      const float inv2 = mv_inv_rms<X::K>(ss2, a.eps);
#pragma unroll
      for (int p = 0; p < PP::XP; ++p) {
        const float4 t = ow[p];
        const float4 h = make_float4((P.r[p].x + t.x * inv1) * sc, (P.r[p].y + t.y * inv1) * sc,
                                     (P.r[p].z + t.z * inv1) * sc, (P.r[p].w + t.w * inv1) * sc);
        if (a.h_out && blockIdx.x == 0 && PP::live(p)) *(float4*)(a.h_out + PP::elem(p)) = h;
        P.x[p] = mul_w(h, P.w2[p], inv2);
      }
    }
  }
  if (act) mv_digitize<BPR, NWV, PRO>(P, smem);
  lds_barrier();
}

// Digits and constants of one unit, held in registers.
template <int QT>
struct MvUnit {
  uint32_t hi[16], lo[16];
  float s[4];   // Q4_K: s[0..1] scales of sub-blocks 2u, 2u+1, s[2..3] their sums; Q6_K: scale of run k
  int2 c[4];    // Q6_K: 32*sum(hi), 32*sum(lo) of run k
};

template <int QT, int BPR>
__device__ __forceinline__ void mv_unit_load(MvUnit<QT>& X, const uint8_t* smem, int u) {
  using XL = MvX<BPR>;
  const float* s = (const float*)(smem + XL::S);
  if constexpr (QT == 0) {
    // elements [64u, 64u + 64): low nibbles -> sub-block 2u, high nibbles -> 2u + 1
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint4 th = *(const uint4*)(smem + XL::HI + 64 * u + 16 * c);
      const uint4 tl = *(const uint4*)(smem + XL::LO + 64 * u + 16 * c);
      X.hi[4 * c] = th.x; X.hi[4 * c + 1] = th.y; X.hi[4 * c + 2] = th.z; X.hi[4 * c + 3] = th.w;
      X.lo[4 * c] = tl.x; X.lo[4 * c + 1] = tl.y; X.lo[4 * c + 2] = tl.z; X.lo[4 * c + 3] = tl.w;
    }
    const float* sum = (const float*)(smem + XL::SUM);
    X.s[0] = s[2 * u];
    X.s[1] = s[2 * u + 1];
    X.s[2] = sum[2 * u];
    X.s[3] = sum[2 * u + 1];
  } else {
    // runs k = 0..3 at element 256b + 128h + 32k + l0 (src/gguf.ts:344-361)
    const int b = u >> 2, g = u & 3, h = g >> 1, l0 = 16 * (g & 1);
    const int4* c16 = (const int4*)(smem + XL::C16);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int e = 256 * b + 128 * h + 32 * k + l0;
      const uint4 th = *(const uint4*)(smem + XL::HI + e);
      const uint4 tl = *(const uint4*)(smem + XL::LO + e);
      X.hi[4 * k] = th.x; X.hi[4 * k + 1] = th.y; X.hi[4 * k + 2] = th.z; X.hi[4 * k + 3] = th.w;
      X.lo[4 * k] = tl.x; X.lo[4 * k + 1] = tl.y; X.lo[4 * k + 2] = tl.z; X.lo[4 * k + 3] = tl.w;
      X.s[k] = s[e / 32];
      const int4 cc = c16[e / 32];
      X.c[k] = (l0 == 0) ? make_int2(cc.x, cc.y) : make_int2(cc.z, cc.w);
    }
  }
}

// Dot product of unit u of one row (block at blk in LDS) with the resident digits.
template <int QT>
__device__ __forceinline__ float mv_unit_dot(const MvUnit<QT>& X, const uint8_t* blk, int g) {
  if constexpr (QT == 0) {
    uint4 hd;
    uint32_t qa[8];
    q4_lds_unit(blk, g, hd, qa);
    float sc_lo, sc_hi, m_lo, m_hi;
    q4k_scales(hd.y, hd.z, hd.w, g, sc_lo, sc_hi, m_lo, m_hi);
    int ah0 = 0, al0 = 0, ah1 = 0, al1 = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t nl = q4k_lo_codes(qa[k]), nh = q4k_hi_codes(qa[k]);
      ah0 = __builtin_amdgcn_sdot4((int)nl, (int)X.hi[k], ah0, false);
      al0 = __builtin_amdgcn_sdot4((int)nl, (int)X.lo[k], al0, false);
      ah1 = __builtin_amdgcn_sdot4((int)nh, (int)X.hi[8 + k], ah1, false);
      al1 = __builtin_amdgcn_sdot4((int)nh, (int)X.lo[8 + k], al1, false);
    }
    const float d = g4d::f16_bits_to_f32(hd.x & 0xffffu);
    const float dmin = g4d::f16_bits_to_f32(hd.x >> 16);
    const float i0 = (float)(ah0 * 256 + al0), i1 = (float)(ah1 * 256 + al1);
    return d * (sc_lo * X.s[0] * i0 + sc_hi * X.s[1] * i1) - dmin * (m_lo * X.s[2] + m_hi * X.s[3]);
  } else {
    uint32_t A[4], B[4], H[4];
    int32_t scs[4];
    float dd;
    q6_lds_unit(blk, g, A, B, H, scs, dd);
    float part = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      int ah = 0, al = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t q = q6k_codes(k, A[j], B[j], H[j]);
        ah = __builtin_amdgcn_sdot4((int)q, (int)X.hi[4 * k + j], ah, false);
        al = __builtin_amdgcn_sdot4((int)q, (int)X.lo[4 * k + j], al, false);
      }
      const int I = (ah - X.c[k].x) * 256 + (al - X.c[k].y);
      part += (float)scs[k] * X.s[k] * (float)I;
    }
    return part * dd;
  }
}

// Q4_K: the 48 bytes unit g of one row-block needs (header, two 16-byte
// quant runs) are 16-byte aligned in global memory (144-byte blocks), so
// each thread loads its own unit straight into registers: no LDS staging and
// no workgroup barrier between the weights' arrival and the products.
struct Q4Unit {
  u32x4a hd, q0, q1;
};
// Weight units are read through a buffer resource over the matrix, with a
// cache policy per kernel shape: POL 2 (non-temporal) measured faster for
// the one-matrix Q4_K launches (o, q/k/v: 0.3 us each), slower where
// neighbouring threads re-read a line (Q6_K runs, the gate/up pair).
typedef uint32_t bu4 __attribute__((ext_vector_type(4)));
template <int POL>
__device__ __forceinline__ u32x4a bl16(__amdgpu_buffer_rsrc_t r, uint32_t o) {
  const bu4 v = __builtin_amdgcn_raw_buffer_load_b128(r, o, 0, POL);
  return u32x4a{v[0], v[1], v[2], v[3]};
}
template <int POL>
__device__ __forceinline__ void q4_unit_load(Q4Unit& w, __amdgpu_buffer_rsrc_t r, uint32_t o, int g) {
  w.hd = bl16<POL>(r, o);
  w.q0 = bl16<POL>(r, o + 16 + 32 * g);
  w.q1 = bl16<POL>(r, o + 32 + 32 * g);
}
// The unit's header and 32 quant bytes as q4_lds_unit gives them.
__device__ __forceinline__ void q4_unit_words(const Q4Unit& w, uint4& hd, uint32_t (&qa)[8]) {
  hd = make_uint4(w.hd[0], w.hd[1], w.hd[2], w.hd[3]);
  qa[0] = w.q0[0]; qa[1] = w.q0[1]; qa[2] = w.q0[2]; qa[3] = w.q0[3];
  qa[4] = w.q1[0]; qa[5] = w.q1[1]; qa[6] = w.q1[2]; qa[7] = w.q1[3];
}
__device__ __forceinline__ float q4_unit_dot(const MvUnit<0>& X, const Q4Unit& w, int g) {
  uint4 hd;
  uint32_t qa[8];
  q4_unit_words(w, hd, qa);
  float sc_lo, sc_hi, m_lo, m_hi;
  q4k_scales(hd.y, hd.z, hd.w, g, sc_lo, sc_hi, m_lo, m_hi);
  int ah0 = 0, al0 = 0, ah1 = 0, al1 = 0;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const uint32_t nl = q4k_lo_codes(qa[k]), nh = q4k_hi_codes(qa[k]);
    ah0 = __builtin_amdgcn_sdot4((int)nl, (int)X.hi[k], ah0, false);
    al0 = __builtin_amdgcn_sdot4((int)nl, (int)X.lo[k], al0, false);
    ah1 = __builtin_amdgcn_sdot4((int)nh, (int)X.hi[8 + k], ah1, false);
    al1 = __builtin_amdgcn_sdot4((int)nh, (int)X.lo[8 + k], al1, false);
  }
  const float d = g4d::f16_bits_to_f32(hd.x & 0xffffu);
  const float dmin = g4d::f16_bits_to_f32(hd.x >> 16);
  const float i0 = (float)(ah0 * 256 + al0), i1 = (float)(ah1 * 256 + al1);
  return d * (sc_lo * X.s[0] * i0 + sc_hi * X.s[1] * i1) - dmin * (m_lo * X.s[2] + m_hi * X.s[3]);
}

// Q6_K: blocks are 210 bytes, so a block starts 4-byte aligned (even block)
// or 2 bytes past a dword (odd block; rows start dword-aligned). Each 16-byte
// run is read as five aligned dwords and shifted into place (the fifth dword
// stays inside the block: runs end at byte 192 at most); the four scales of
// the unit and d are read as single bytes / one half, which never leaves the
// block either.
struct Q6Unit {
  u32x4a a4, b4, h4;
  uint32_t a1, b1, h1, sh;
  uint32_t s0, s1, s2, s3;  // the unit's four int8 scales, as loaded (zero-extended)
  uint32_t d;
};
template <int POL>
__device__ __forceinline__ void q6_unit_load(Q6Unit& w, __amdgpu_buffer_rsrc_t r, uint32_t o, const uint8_t* blk,
                                             int g) {
  const int h = g >> 1, l0 = 16 * (g & 1);
  w.sh = (uint32_t)(uintptr_t)blk & 3u;
  const uint32_t oa = o - w.sh;  // the dword at or before the block
  w.a4 = bl16<POL>(r, oa + 64 * h + l0);
  w.a1 = __builtin_amdgcn_raw_buffer_load_b32(r, oa + 64 * h + l0 + 16, 0, POL);
  w.b4 = bl16<POL>(r, oa + 64 * h + 32 + l0);
  w.b1 = __builtin_amdgcn_raw_buffer_load_b32(r, oa + 64 * h + 32 + l0 + 16, 0, POL);
  w.h4 = bl16<POL>(r, oa + 128 + 32 * h + l0);
  w.h1 = __builtin_amdgcn_raw_buffer_load_b32(r, oa + 128 + 32 * h + l0 + 16, 0, POL);
  // raw bytes only: any arithmetic on a loaded value here would make the
  // compiler wait for it where it is loaded (for the prefetched tile too)
  const uint8_t* scp = blk + 192 + 8 * h + (g & 1);
  w.s0 = scp[0];
  w.s1 = scp[2];
  w.s2 = scp[4];
  w.s3 = scp[6];
  w.d = *(const uint16_t*)(blk + 208);
}
__device__ __forceinline__ void q6_run(const u32x4a& v4, uint32_t v1, uint32_t sh, uint32_t (&o)[4]) {
  o[0] = __builtin_amdgcn_alignbyte(v4[1], v4[0], sh);
  o[1] = __builtin_amdgcn_alignbyte(v4[2], v4[1], sh);
  o[2] = __builtin_amdgcn_alignbyte(v4[3], v4[2], sh);
  o[3] = __builtin_amdgcn_alignbyte(v1, v4[3], sh);
}
// The unit's three runs shifted into place, its four scales and d, as
// q6_lds_unit gives them for a block in LDS.
__device__ __forceinline__ void q6_unit_unpack(const Q6Unit& w, uint32_t (&A)[4], uint32_t (&B)[4],
                                               uint32_t (&H)[4], int32_t (&scs)[4], float& dd) {
  q6_run(w.a4, w.a1, w.sh, A);
  q6_run(w.b4, w.b1, w.sh, B);
  q6_run(w.h4, w.h1, w.sh, H);
  // the empty asm pins the byte extraction here, after the loads' wait
  uint32_t r0 = w.s0, r1 = w.s1, r2 = w.s2, r3 = w.s3, rd = w.d;
  asm volatile("" : "+v"(r0), "+v"(r1), "+v"(r2), "+v"(r3), "+v"(rd));
  scs[0] = (int32_t)(int8_t)r0;
  scs[1] = (int32_t)(int8_t)r1;
  scs[2] = (int32_t)(int8_t)r2;
  scs[3] = (int32_t)(int8_t)r3;
  dd = g4d::f16_bits_to_f32(rd);
}
__device__ __forceinline__ float q6_unit_dot(const MvUnit<1>& X, const Q6Unit& w) {
  uint32_t A[4], B[4], H[4];
  int32_t scs[4];
  float dd;
  q6_unit_unpack(w, A, B, H, scs, dd);
  float part = 0.f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    int ah = 0, al = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t q = q6k_codes(k, A[j], B[j], H[j]);
      ah = __builtin_amdgcn_sdot4((int)q, (int)X.hi[4 * k + j], ah, false);
      al = __builtin_amdgcn_sdot4((int)q, (int)X.lo[4 * k + j], al, false);
    }
    const int I = (ah - X.c[k].x) * 256 + (al - X.c[k].y);
    part += (float)scs[k] * X.s[k] * (float)I;
  }
  return part * dd;
}

// Q6_K unit against D8 digits: each 16-element run (one int8 scale) is two
// 8-element groups, each with its own activation scale and offset.
struct MvUnit8 {
  uint32_t hi[16], lo[16];
  float s[8];
  int2 c[8];
};
template <int BPR>
__device__ __forceinline__ void mv_unit_load8(MvUnit8& X, const uint8_t* smem, int u) {
  using D = MvD8<BPR>;
  const int b = u >> 2, g = u & 3, h = g >> 1, l0 = 16 * (g & 1);
  const float* sc = (const float*)(smem + D::S);
  const int2* cc = (const int2*)(smem + D::C);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int e = 256 * b + 128 * h + 32 * k + l0;  // run k (src/gguf.ts:344-361)
    const uint4 th = *(const uint4*)(smem + D::HI + e);
    const uint4 tl = *(const uint4*)(smem + D::LO + e);
    X.hi[4 * k] = th.x; X.hi[4 * k + 1] = th.y; X.hi[4 * k + 2] = th.z; X.hi[4 * k + 3] = th.w;
    X.lo[4 * k] = tl.x; X.lo[4 * k + 1] = tl.y; X.lo[4 * k + 2] = tl.z; X.lo[4 * k + 3] = tl.w;
    const float2 s2 = *(const float2*)(sc + e / 8);
    const int4 c2 = *(const int4*)(cc + e / 8);
    X.s[2 * k] = s2.x;
    X.s[2 * k + 1] = s2.y;
    X.c[2 * k] = make_int2(c2.x, c2.y);
    X.c[2 * k + 1] = make_int2(c2.z, c2.w);
  }
}
__device__ __forceinline__ float q6_unit_dot8(const MvUnit8& X, const Q6Unit& w) {
  uint32_t A[4], B[4], H[4];
  int32_t scs[4];
  float dd;
  q6_unit_unpack(w, A, B, H, scs, dd);
  float part = 0.f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    int ah[2] = {0, 0}, al[2] = {0, 0};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t q = q6k_codes(k, A[j], B[j], H[j]);
      ah[j >> 1] = __builtin_amdgcn_sdot4((int)q, (int)X.hi[4 * k + j], ah[j >> 1], false);
      al[j >> 1] = __builtin_amdgcn_sdot4((int)q, (int)X.lo[4 * k + j], al[j >> 1], false);
    }
    const int I0 = (ah[0] - X.c[2 * k].x) * 256 + (al[0] - X.c[2 * k].y);
    const int I1 = (ah[1] - X.c[2 * k + 1].x) * 256 + (al[1] - X.c[2 * k + 1].y);
    part += (float)scs[k] * (X.s[2 * k] * (float)I0 + X.s[2 * k + 1] * (float)I1);
  }
  return part * dd;
}

// D8 digits of a gate/up launch's GELU outputs: the 8 rows of a group are
// the 8 rows one wave reduces (8 lanes each, the first of them at lanes 0,
// 8, ..., 56), so the group's maximum and digit sums are wave reductions
// (DPP, no LDS round trip; the digit sums are integers below 2^11, exact in
// f32). `real`: this lane stores a row (the other lanes and rows past the
// output carry 0). Every lane of the wave calls it.
__device__ __forceinline__ void mv_d8_group(float v, bool real, uint32_t row, uint32_t K, uint8_t* d8) {
  const float am = g4d::wave_max_dpp(real ? fabsf(v) : 0.f);
  const float inv = am > 0.f ? XQ * __builtin_amdgcn_rcpf(am) : 0.f;
  const int q = real ? (int)__builtin_rintf(v * inv) : 0;
  const int lo = ((q + 128) & 255) - 128;
  const int hi = (q - lo) >> 8;
  const int shi = (int)g4d::wave_sum_dpp((float)hi), slo = (int)g4d::wave_sum_dpp((float)lo);
  // a NaN or Inf in the group makes its scale NaN (the products carry it)
  const bool bad = __ballot(real && !__builtin_isfinite(v)) != 0;
  if (real) {
    d8[row] = (uint8_t)(hi & 255);
    d8[K + row] = (uint8_t)(lo & 255);
  }
  if (real && (threadIdx.x & 63) == 0) {  // the group's first row
    ((float*)(d8 + 2 * (size_t)K))[row / 8] = bad ? __builtin_nanf("") : am * (1.0f / XQ);
    ((int2*)(d8 + 2 * (size_t)K + 4 * (size_t)(K / 8)))[row / 8] = make_int2(32 * shi, 32 * slo);
  }
}

// Adds each row's U unit partials (RG lanes per row, then a butterfly) and
// stores the tile's rows: y, softcap(y), or gelu(gate) * up for a pair.
// DEV: each row is also staged as a (tag 1, value) pair in one device-scope
// 8-byte store (written through to the point of coherence), for readers in
// other workgroups of the same launch.
template <class T, int NTH, int NMAT, bool DEV = false>
__device__ __forceinline__ void mv_reduce_store(const float* red, const GemvSeg& sg, uint32_t t, int tid, float cap,
                                                bool track, g4d::Cand& best, uint8_t* d8 = nullptr,
                                                g4d::Cand* tkt = nullptr) {
  constexpr int U = NTH / T::TR;
  const int gl = tid % T::RG;
  for (int r = tid / T::RG; r < T::TR; r += NTH / T::RG) {  // uniform within a group
    float y[NMAT];
#pragma unroll
    for (int m = 0; m < NMAT; ++m) {
      const float* rr = red + m * T::TR * T::RS + r * T::RS + gl;
      float a = rr[0];
#pragma unroll
      for (int v = 1; v < U / T::RG; ++v) a += rr[v * T::RG];
      y[m] = g4d::group_sum<T::RG>(a);
    }
    const uint32_t row = t * T::TR + r;
    const bool real = gl == 0 && row < sg.M;
    if constexpr (NMAT == 2) {
      const float v = gelu_tanh(y[0]) * y[1];
      if (real) sg.Y[row] = v;
      // (uniform) every lane of the group's wave is in this iteration: 8
      // rows x 8 lanes fill it, and TR is a multiple of 8 (host-checked)
      if constexpr (T::RG == 8)
        if (d8) mv_d8_group(v, real, row, sg.M, d8);
    } else if (real) {
      const float v = cap > 0.f ? softcap(y[0], cap) : y[0];
      sg.Y[row] = v;
      if constexpr (DEV)
        __hip_atomic_store(sg.stage + row, g4mqf::kStaged | __float_as_uint(v), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      const g4d::Cand d{v, row};
      if (track && g4d::better(d, best)) best = d;
      // top-k classes: a tile's rows are distinct classes (TR <= 256) and
      // tiles come in row order, so a strict '>' keeps the first maximum
      if (tkt && v > tkt[row & 255u].v) tkt[row & 255u] = d;
    }
  }
}

// The workgroup's best candidate over the rows it stored (argmax stage 1 run
// as the matvec's epilogue: the logits are not read back); `sm` holds NWV
// candidates not otherwise in use.
template <int NWV>
__device__ __forceinline__ void mv_argmax_partial(g4d::Cand c, g4d::Cand* sm, g4d::Cand* dst) {
  c = g4d::wave_best(c);
  if ((threadIdx.x & 63) == 0) sm[threadIdx.x >> 6] = c;
  lds_barrier();
  if (threadIdx.x == 0) {
    g4d::Cand b = sm[0];
#pragma unroll
    for (int k = 1; k < NWV; ++k)
      if (g4d::better(sm[k], b)) b = sm[k];
    *dst = b;
  }
}

// The workgroup's top-k class table (the first stage of shaders/topk256.wgsl
// over the rows it stored) to column `wg` of the [256][tk_stride] candidates.
template <int NTH>
__device__ __forceinline__ void mv_topk_partial(const g4d::Cand* tkt, const GemvSegs& segs, uint32_t wg) {
  lds_barrier();
  for (int i = threadIdx.x; i < 256; i += NTH) segs.tk[(size_t)i * segs.tk_stride + wg] = tkt[i];
}

// NMAT = 1: y, or softcap(y) when cap > 0 (shaders/logit_softcap.wgsl), for
// each segment's rows; with `segs.amx`, also the workgroup's argmax
// candidate (shaders/argmax.wgsl order) in segs.amx[blockIdx.x]. NMAT = 2:
// gate/up pair, out = gelu(gate) * up (shaders/gelu_mul.wgsl:10-16).
// STAGED: every workgroup walks several tiles (rep > 1: matrices past two
// tiles per CU, the LM head); the other instances hold the one-tile path
// only. (Bounding the staged instance to two 12-wave workgroups per CU,
// 80 VGPRs, spilled the tile loop to scratch: 199 us instead of 82.)
// One ring step: the loads of tile t + 2 into `nxt` (when `more`), then
// this thread's unit product of tile t from `cur`. The two buffers are
// different ring slots, which the restrict qualifiers tell the compiler, so
// it adds no wait for the new loads before the products' LDS reads (the
// caller waits for tile t's own loads explicitly).
template <int QT, int BPR, int NWV>
__device__ __forceinline__ void mv_ring_step(bool more, const uint8_t* src, uint32_t nbytes, uint8_t* __restrict__ nxt,
                                             const uint8_t* __restrict__ cur, const MvUnit<QT>& X,
                                             float* __restrict__ red, int w, int l, int g) {
  if (more) mv_ring_load<QT, BPR, NWV>(src, nbytes, nxt, w, l);
  *red = mv_unit_dot<QT>(X, cur, g);
}
template <int QT, int BPR, int NWV, int PRO, int NMAT, bool STAGED, bool DEV = false>
__device__ __forceinline__ void mv_body(const GemvSegs& segs, const uint8_t* w_up, const ProArgs& pa, float cap,
                                        uint8_t* smem) {
  using G = MvGeom<BPR, NWV>;
  using T = MvTile<QT, BPR, NWV>;
  constexpr int NTH = G::NTH;
  static_assert(PRO != 3 || (QT == 1 && NMAT == 1), "D8 input: one Q6_K matrix");
  static_assert(!DEV || (!STAGED && NMAT == 1), "device-scope rows: one tile of one matrix");
  int si = 0;
#pragma unroll
  for (int i = 1; i < 4; ++i)
    if (i < segs.n && blockIdx.x >= segs.s[i].wg_begin) si = i;
  const GemvSeg sg = segs.s[si];
  const uint8_t* W[2] = {sg.W, w_up};
  const uint32_t tiles = (sg.M + T::TR - 1) / T::TR;
  const uint32_t tb = (blockIdx.x - sg.wg_begin) * segs.rep;
  const uint32_t te = min(tiles, tb + segs.rep);
  const int tid = threadIdx.x;
  const int slot = tid / G::U, u = tid % G::U;
  // top-k class table past the kernel's other LDS (ordered before its first
  // use by the prologue's barriers)
  g4d::Cand* const tkt =
      (NMAT == 1 && segs.tk) ? (g4d::Cand*)(smem + mv_lds_bytes<QT, BPR, NWV, PRO, NMAT>(STAGED)) : nullptr;
  if (tkt)
    for (int i = tid; i < 256; i += NTH) tkt[i] = g4d::Cand{-1e30f, 0u};
  float* red = (float*)(smem + align16(MvXA<BPR, PRO>::END));
  uint8_t* const d8 = NMAT == 2 ? segs.d8 : nullptr;

  MvPro<BPR, NWV, PRO == 3 ? 0 : PRO> P;
  // D8 input: the block's 16-byte chunks, a few per thread, copied to LDS as is
  constexpr int DN = (int)((MvD8<BPR>::BYTES + 15) / 16), DL = (DN + NTH - 1) / NTH;
  u32x4a dg[PRO == 3 ? DL : 1];
  if constexpr (PRO == 3) {
#pragma unroll
    for (int i = 0; i < DL; ++i)
      dg[i] = *(const u32x4a*)((const uint8_t*)pa.x + 16 * min(tid + i * NTH, DN - 1));
  } else {
    mv_pro_load<BPR, NWV, PRO>(P, pa);
  }
  // Requests leave a CU in issue order across its waves: every wave's
  // activation loads go out before any wave's weight loads, or the last
  // waves' activations queue behind the first waves' weight tiles. A bare
  // s_barrier orders the issue without waiting for any load.
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (!STAGED) {  // one tile per workgroup (host-checked)
    // one tile: each thread's unit straight from global memory into
    // registers; rows past M (a partial tile) read row M - 1, not stored
    using WU = typename std::conditional<QT == 0, Q4Unit, Q6Unit>::type;
    WU wu[NMAT];
#pragma unroll
    for (int m = 0; m < NMAT; ++m) {
      constexpr int POL = (QT == 0 && NMAT == 1) ? 2 : 0;
      const uint32_t row = min(tb * (uint32_t)T::TR + (uint32_t)slot, sg.M - 1);
      const uint32_t off = row * T::RB + (uint32_t)(u >> 2) * T::BYTES;
      const __amdgpu_buffer_rsrc_t rs =
          __builtin_amdgcn_make_buffer_rsrc((void*)W[m], (short)0,
                                            (int)(uint32_t)min((uint64_t)sg.M * T::RB, (uint64_t)0xffffffffu),
                                            0x00020000);
      if constexpr (QT == 0) q4_unit_load<POL>(wu[m], rs, off, u & 3);
      else q6_unit_load<POL>(wu[m], rs, off, W[m] + off, u & 3);
    }
    __builtin_amdgcn_sched_barrier(0);  // every weight load is issued before the activations are used
    if constexpr (PRO == 3) {
#pragma unroll
      for (int i = 0; i < DL; ++i)
        if (tid + i * NTH < DN) *(u32x4a*)(smem + 16 * (tid + i * NTH)) = dg[i];
      lds_barrier();
      MvUnit8 X;
      mv_unit_load8<BPR>(X, smem, u);
      red[slot * T::RS + u] = q6_unit_dot8(X, wu[0]);
    } else {
      mv_pro_finish<BPR, NWV, PRO>(P, smem, pa);
      MvUnit<QT> X;
      mv_unit_load<QT, BPR>(X, smem, u);
#pragma unroll
      for (int m = 0; m < NMAT; ++m) {
        float v;
        if constexpr (QT == 0) v = q4_unit_dot(X, wu[m], u & 3);
        else v = q6_unit_dot(X, wu[m]);
        red[m * T::TR * T::RS + slot * T::RS + u] = v;
      }
    }
    lds_barrier();
    g4d::Cand best{-1e30f, 0u};
    mv_reduce_store<T, NTH, NMAT, DEV>(red, sg, tb, tid, cap, segs.amx != nullptr, best, d8, tkt);
    if constexpr (NMAT == 1)
      if (segs.amx)
        mv_argmax_partial<NWV>(best, (g4d::Cand*)(smem + MvXA<BPR, PRO>::RED8), segs.amx + blockIdx.x);
    if (tkt) mv_topk_partial<NTH>(tkt, segs, blockIdx.x - sg.wg_begin);
    return;
  }
  if constexpr (STAGED && PRO != 3 && NMAT == 1) {
    // several tiles of one matrix: a ring of R::D LDS buffers filled by
    // global -> LDS loads, tiles t + 1 .. t + D - 1 in flight while tile t
    // is multiplied. A wave's loads complete in issue order, so once it has
    // at most the later tiles' loads outstanding (vmcnt <= their count; the
    // row stores among them only make the wait stricter) its share of tile
    // t is in LDS; the barrier that follows makes the whole tile visible.
    // Buffer (t + D - 1) % D held tile t - 1, whose products every wave
    // finished before the barrier ahead of the last reduction.
    using R = MvRing<QT, BPR, NWV>;
    constexpr uint32_t D = (uint32_t)R::D;
    uint8_t* ring = smem + align16(MvXA<BPR, PRO>::END) + align16((size_t)T::TR * T::RS * 4);
    const int w = tid >> 6, l = tid & 63;
    const bool short_wave = mv_ring_short<QT, BPR, NWV>(w);
#pragma unroll
    for (uint32_t k = 0; k + 1 < D; ++k)
      if (tb + k < te)
        mv_ring_load<QT, BPR, NWV>(W[0] + (size_t)(tb + k) * T::TB, mv_tile_bytes<QT, BPR, NWV>(sg.M, tb + k),
                                   ring + k * R::BUF, w, l);
    __builtin_amdgcn_sched_barrier(0);  // every weight load is issued before the activations are used
    mv_pro_finish<BPR, NWV, PRO>(P, smem, pa);
    MvUnit<QT> X;
    mv_unit_load<QT, BPR>(X, smem, u);
    g4d::Cand best{-1e30f, 0u};
    uint32_t cur = 0;  // ring buffer of tile t
    for (uint32_t t = tb; t < te; ++t) {
      const uint32_t ahead = min(D - 2, te - 1 - t);  // (uniform) later tiles in flight
      if (short_wave) wait_tiles<R::LPT - 1, R::D>(ahead);
      else wait_tiles<R::LPT, R::D>(ahead);
      ring_barrier();  // tile t in LDS for every wave; tile t - 1 reduced
      const uint32_t nxt = cur == 0 ? D - 1 : cur - 1;  // tile t - 1's buffer
      mv_ring_step<QT, BPR, NWV>(t + D - 1 < te, W[0] + (size_t)(t + D - 1) * T::TB,
                                 mv_tile_bytes<QT, BPR, NWV>(sg.M, t + D - 1), ring + nxt * R::BUF,
                                 ring + cur * R::BUF + slot * T::RB + (u >> 2) * T::BYTES, X, red + slot * T::RS + u,
                                 w, l, u & 3);
      ring_barrier();
      mv_reduce_store<T, NTH, NMAT>(red, sg, t, tid, cap, segs.amx != nullptr, best, d8, tkt);
      cur = cur + 1 == D ? 0u : cur + 1;
    }
    if (segs.amx) mv_argmax_partial<NWV>(best, (g4d::Cand*)(smem + MvXA<BPR, PRO>::RED8), segs.amx + blockIdx.x);
    if (tkt) mv_topk_partial<NTH>(tkt, segs, blockIdx.x - sg.wg_begin);
  } else if constexpr (STAGED && PRO != 3) {
    // several tiles of a pair: coalesced loads of the next tile into
    // registers while this one is multiplied out of LDS
    uint8_t* tl = smem + align16(MvXA<BPR, PRO>::END) + NMAT * align16((size_t)T::TR * T::RS * 4);
    // (Two tiles in flight per workgroup, in two register sets, measured
    // 85 us for the LM head against 82 with one.)
    Stage<T::LPT> st[NMAT];
    uint32_t nb = mv_tile_bytes<QT, BPR, NWV>(sg.M, tb);
#pragma unroll
    for (int m = 0; m < NMAT; ++m) mv_stage_load<T, NTH>(W[m] + (size_t)tb * T::TB, nb, st[m]);
    __builtin_amdgcn_sched_barrier(0);  // every weight load is issued before the activations are used
    mv_pro_finish<BPR, NWV, PRO>(P, smem, pa);
    MvUnit<QT> X;
    mv_unit_load<QT, BPR>(X, smem, u);
    g4d::Cand best{-1e30f, 0u};
    // The barriers order LDS accesses only: a plain __syncthreads after the
    // row stores would also wait for the next tile's loads.
    for (uint32_t t = tb; t < te; ++t) {
      lds_barrier();  // digits read (first tile) / previous tile reduced
#pragma unroll
      for (int m = 0; m < NMAT; ++m) mv_stage_store<T, NTH>(tl + m * T::LDS_T, nb, st[m]);
      lds_barrier();
      if (t + 1 < te) {
        nb = mv_tile_bytes<QT, BPR, NWV>(sg.M, t + 1);
#pragma unroll
        for (int m = 0; m < NMAT; ++m) mv_stage_load<T, NTH>(W[m] + (size_t)(t + 1) * T::TB, nb, st[m]);
      }
#pragma unroll
      for (int m = 0; m < NMAT; ++m) {
        const uint8_t* blk = tl + m * T::LDS_T + slot * T::RB + (u >> 2) * T::BYTES;
        red[m * T::TR * T::RS + slot * T::RS + u] = mv_unit_dot<QT>(X, blk, u & 3);
      }
      lds_barrier();
      mv_reduce_store<T, NTH, NMAT>(red, sg, t, tid, cap, segs.amx != nullptr, best, d8, tkt);
    }
    if constexpr (NMAT == 1)
      if (segs.amx)
        mv_argmax_partial<NWV>(best, (g4d::Cand*)(smem + MvXA<BPR, PRO>::RED8), segs.amx + blockIdx.x);
    if (tkt) mv_topk_partial<NTH>(tkt, segs, blockIdx.x - sg.wg_begin);
  }
}

template <int QT, int BPR, int NWV, int PRO, int NMAT, bool STAGED>
__global__ __launch_bounds__(64 * NWV) void mv_kernel(GemvSegs segs, const uint8_t* w_up, ProArgs pa, float cap) {
  extern __shared__ __align__(16) uint8_t smem[];
  mv_body<QT, BPR, NWV, PRO, NMAT, STAGED>(segs, w_up, pa, cap, smem);
}

// ---------------------------------------------------------------------------
// Unpack check (the test export g4_dequantPath): weight values as the matvec
// units see them. Each thread takes one unit (a quarter block), loads it
// with the loader of a kernel family, extracts codes, scales, mins and d with
// the same helpers the products use, and forms the reference's dequantized
// value from them: Q4_K (d*sc)*q - dmin*m (src/gguf.ts:184-209), Q6_K
// (d*sc)*(q - 32) (src/gguf.ts:336-364); the products are exact in f32 and
// the result is rounded once, as the reference's f64 value stored to f32.
// PATH 0: register units (q4_unit_load / q6_unit_load through a buffer
// resource, q6_run; the one-tile mv_kernel). PATH 1: units of blocks staged
// in LDS at their byte offsets (q4_lds_unit / q6_lds_unit with lds_piece;
// the tile-walking mv_kernel and gemv_kernel).
// ---------------------------------------------------------------------------
constexpr int UC_BLOCKS = NT / 4;  // blocks per workgroup (4 units each)

__device__ __forceinline__ uint32_t byte_of(uint32_t w, int i) { return (w >> (8 * i)) & 0xffu; }

__device__ __forceinline__ void q4_unit_values(uint4 hd, const uint32_t (&qa)[8], int g, float* out) {
  float sc_lo, sc_hi, m_lo, m_hi;
  q4k_scales(hd.y, hd.z, hd.w, g, sc_lo, sc_hi, m_lo, m_hi);
  const float d = g4d::f16_bits_to_f32(hd.x & 0xffffu), dmin = g4d::f16_bits_to_f32(hd.x >> 16);
  const float d_lo = d * sc_lo, d_hi = d * sc_hi, n_lo = dmin * m_lo, n_hi = dmin * m_hi;  // exact
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const uint32_t lo = q4k_lo_codes(qa[k]), hi = q4k_hi_codes(qa[k]);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[64 * g + 4 * k + i] = d_lo * (float)byte_of(lo, i) - n_lo;
      out[64 * g + 32 + 4 * k + i] = d_hi * (float)byte_of(hi, i) - n_hi;
    }
  }
}

__device__ __forceinline__ void q6_unit_values(const uint32_t (&A)[4], const uint32_t (&B)[4],
                                               const uint32_t (&H)[4], const int32_t (&scs)[4], float dd, int g,
                                               float* out) {
  const int h = g >> 1, l0 = 16 * (g & 1);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float ds = dd * (float)scs[k];  // exact
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t c = q6k_codes(k, A[j], B[j], H[j]);
#pragma unroll
      for (int i = 0; i < 4; ++i) out[128 * h + 32 * k + l0 + 4 * j + i] = ds * (float)((int)byte_of(c, i) - 32);
    }
  }
}

template <int QT, int PATH>
__global__ __launch_bounds__(NT) void unpack_check_kernel(const uint8_t* W, uint32_t nblocks, float* out) {
  constexpr int BY = BlockOf<QT>::BYTES;
  __shared__ __align__(16) uint8_t lds[PATH == 1 ? UC_BLOCKS * BY : 16];
  const uint32_t b0 = blockIdx.x * (uint32_t)UC_BLOCKS;
  const uint32_t b = b0 + threadIdx.x / 4;
  const int g = threadIdx.x & 3;
  float* o = out + (size_t)b * 256;
  if constexpr (PATH == 0) {
    if (b >= nblocks) return;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void*)W, (short)0, (int)(nblocks * (uint32_t)BY), 0x00020000);
    const uint32_t off = b * (uint32_t)BY;
    if constexpr (QT == 0) {
      Q4Unit w;
      q4_unit_load<0>(w, rs, off, g);
      uint4 hd;
      uint32_t qa[8];
      q4_unit_words(w, hd, qa);
      q4_unit_values(hd, qa, g, o);
    } else {
      Q6Unit w;
      q6_unit_load<0>(w, rs, off, W + off, g);
      uint32_t A[4], B[4], H[4];
      int32_t scs[4];
      float dd;
      q6_unit_unpack(w, A, B, H, scs, dd);
      q6_unit_values(A, B, H, scs, dd, g, o);
    }
  } else {
    // the workgroup's blocks, byte for byte at their offsets from the first
    // (16-byte aligned: UC_BLOCKS * BY is a multiple of 16)
    const uint32_t nb = min((uint32_t)UC_BLOCKS, nblocks - b0);
    const uint16_t* src = (const uint16_t*)(W + (size_t)b0 * BY);
    for (uint32_t i = threadIdx.x; i < nb * BY / 2; i += NT) ((uint16_t*)lds)[i] = src[i];
    __syncthreads();
    if (b >= nblocks) return;
    const uint8_t* blk = lds + (threadIdx.x / 4) * BY;
    if constexpr (QT == 0) {
      uint4 hd;
      uint32_t qa[8];
      q4_lds_unit(blk, g, hd, qa);
      q4_unit_values(hd, qa, g, o);
    } else {
      uint32_t A[4], B[4], H[4];
      int32_t scs[4];
      float dd;
      q6_lds_unit(blk, g, A, B, H, scs, dd);
      q6_unit_values(A, B, H, scs, dd, g, o);
    }
  }
}

// Blocks to f16 rows (round to nearest even): each thread's quarter block
// through the register unit of path 0 into LDS, then the workgroup's rows
// leave as 16-byte stores. (The tied embedding table: the LM head reads the
// blocks, the embedding lookup f16 rows, src/engine.ts:570-579.)
template <int QT>
__global__ __launch_bounds__(NT) void unpack_f16_kernel(const uint8_t* W, uint32_t nblocks, uint16_t* out) {
  constexpr int BY = BlockOf<QT>::BYTES;
  __shared__ __align__(16) float vals[UC_BLOCKS * 256];
  const uint32_t b0 = blockIdx.x * (uint32_t)UC_BLOCKS;
  const uint32_t b = b0 + threadIdx.x / 4;
  const int g = threadIdx.x & 3;
  if (b < nblocks) {
    float* o = vals + (threadIdx.x / 4) * 256;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void*)W, (short)0, (int)(nblocks * (uint32_t)BY), 0x00020000);
    const uint32_t off = b * (uint32_t)BY;
    if constexpr (QT == 0) {
      Q4Unit w;
      q4_unit_load<0>(w, rs, off, g);
      uint4 hd;
      uint32_t qa[8];
      q4_unit_words(w, hd, qa);
      q4_unit_values(hd, qa, g, o);
    } else {
      Q6Unit w;
      q6_unit_load<0>(w, rs, off, W + off, g);
      uint32_t A[4], B[4], H[4];
      int32_t scs[4];
      float dd;
      q6_unit_unpack(w, A, B, H, scs, dd);
      q6_unit_values(A, B, H, scs, dd, g, o);
    }
  }
  __syncthreads();
  const uint32_t nb = min((uint32_t)UC_BLOCKS, nblocks - b0);
  for (uint32_t i = threadIdx.x; i < nb * 32; i += NT) {
    const float* v = vals + 8 * i;
    uint32_t h[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      h[j] = (uint32_t)g4d::f32_to_f16_bits(v[2 * j]) | ((uint32_t)g4d::f32_to_f16_bits(v[2 * j + 1]) << 16);
    *(uint4*)(out + (size_t)b0 * 256 + 8 * (size_t)i) = make_uint4(h[0], h[1], h[2], h[3]);
  }
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

// f16 rows (the reference's own upload format): 4 rows per wave, 16-byte
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

// rows per wave: the fewest that fill the 16 block slots of a step
template <int BPR>
struct RowsFor {
  static constexpr int R = BPR >= 12 ? 1 : (BPR >= 6 ? 2 : 4);
};

struct LaunchReq {
  int qt;               // 0 = Q4_K, 1 = Q6_K
  const GemvSeg* segs;  // W, Y, M (wg_begin filled here)
  int nseg;
  uint32_t N;
  int nv;
  int pro;
  int epi;
  float cap;
  ProArgs pa;
  uint32_t ldy;
  g4d::Cand* amx = nullptr;     // one-vector launches: per-workgroup argmax candidates (see GemvSegs)
  uint32_t amx_cap = 0;         // candidates `amx` holds
  uint32_t* wgs_out = nullptr;  // receives the workgroup count
  uint8_t* d8 = nullptr;        // gate/up pair: also write the outputs as an MvD8 block
  g4d::Cand* tk = nullptr;      // one matrix: per-workgroup top-k class candidates [256][workgroups]
  uint32_t tk_cap = 0;          // workgroups `tk` holds candidates for
};

constexpr uint32_t kMaxGemvWgs = 2048;  // beyond this a workgroup walks several row tiles

// Workgroups above 64 KB of LDS must be allowed per kernel.
int claim_lds(const void* kern, g4_ctx* ctx, size_t lds) {
  if (lds > ctx->lds_max)
    return g4::set_error(G4_ERR_UNSUPPORTED, "gemv: %zu bytes of LDS exceed the %zu-byte workgroup limit", lds,
                         ctx->lds_max);
  if (lds > kMaxLds) {
    const hipError_t e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return g4::hip_fail(ctx, e, "hipFuncSetAttribute");
  }
  return G4_OK;
}

// LDS bytes of a plain gemv workgroup (host-side mirror of the kernel layout).
size_t gemv_lds(int qt, uint32_t N, int nv) {
  const uint32_t bpr = N / 256;
  const int R = bpr >= 12 ? 1 : (bpr >= 6 ? 2 : 4);
  return align16(xview_bytes(N, nv)) + align16((size_t)R * NW * bpr * (qt ? 210 : 144));
}

template <int QT, int BPR, int NV, int PRO, int EPI>
int launch_fixed(g4_ctx* ctx, const LaunchReq& q) {
  constexpr int R = RowsFor<BPR>::R;
  constexpr int ROWS_WG = R * NW;
  GemvSegs sg{};
  uint32_t tiles = 0;
  for (int i = 0; i < q.nseg; ++i) tiles += ceil_div(q.segs[i].M, ROWS_WG);
  sg.rep = ceil_div(tiles, kMaxGemvWgs);
  uint32_t wgs = 0;
  for (int i = 0; i < q.nseg; ++i) {
    sg.s[i] = q.segs[i];
    sg.s[i].wg_begin = wgs;
    wgs += ceil_div(ceil_div(q.segs[i].M, ROWS_WG), sg.rep);
  }
  sg.n = q.nseg;
  if (wgs == 0) return G4_OK;
  const size_t lds = align16(xview_bytes(BPR * 256, NV)) + Tile<QT, BPR, R>::LDS_B;
  int rc = claim_lds((const void*)gemv_kernel<QT, BPR, R, NV, PRO, EPI>, ctx, lds);
  if (rc) return rc;
  hipLaunchKernelGGL((gemv_kernel<QT, BPR, R, NV, PRO, EPI>), dim3(wgs), dim3(NT), lds, ctx->stream, sg, q.pa,
                     q.ldy, q.cap);
  G4_LAUNCHED(ctx, "gemv");
  return G4_OK;
}

template <int QT, int NV, int PRO, int EPI>
int launch_bpr(g4_ctx* ctx, const LaunchReq& q) {
  switch (q.N / 256) {
    case 4: return launch_fixed<QT, 4, NV, PRO, EPI>(ctx, q);
    case 6: return launch_fixed<QT, 6, NV, PRO, EPI>(ctx, q);
    case 8: return launch_fixed<QT, 8, NV, PRO, EPI>(ctx, q);
    case 12: return launch_fixed<QT, 12, NV, PRO, EPI>(ctx, q);
    case 16: return launch_fixed<QT, 16, NV, PRO, EPI>(ctx, q);
    case 24: return launch_fixed<QT, 24, NV, PRO, EPI>(ctx, q);
    case 32: return launch_fixed<QT, 32, NV, PRO, EPI>(ctx, q);
    case 48: return launch_fixed<QT, 48, NV, PRO, EPI>(ctx, q);
    default: return G4_ERR_UNSUPPORTED;
  }
}

// Batched activations (NV > 1): staged tiles, digits read from LDS per block.
template <int QT>
int launch_qt(g4_ctx* ctx, const LaunchReq& q) {
  if (q.pro != 0 || q.epi != 0) return G4_ERR_UNSUPPORTED;
  switch (q.nv) {
    case 2: return launch_bpr<QT, 2, 0, 0>(ctx, q);
    case 4: return launch_bpr<QT, 4, 0, 0>(ctx, q);
    case 8: return launch_bpr<QT, 8, 0, 0>(ctx, q);
    default: return G4_ERR_UNSUPPORTED;
  }
}

// One activation vector: register-resident digits (mv_kernel). Each
// workgroup digitises the whole activation vector and walks its tiles one row
// per slot; more waves per workgroup shorten both serial phases. A CU streams
// its tile at a limited rate (measured: a workgroup's weights arrive in time
// proportional to its bytes), so the launch takes the widest workgroup that
// still gives every CU a tile (kMvFullWgs), else the widest of at least
// 6 waves that leaves kMvMinWgs tiles; matrices larger than two workgroups
// per CU are walked tile by tile.
constexpr uint32_t kMvFullWgs = 240, kMvMinWgs = 160;

// Tiles per workgroup: one tile up to two workgroups per CU, else walked
// tile by tile, by one workgroup per CU where the walk fills the LDS ring
// (a 12-wave one-matrix launch: its 131 KB of LDS hold one workgroup per CU,
// and each workgroup pays its prologue and the ring's first tiles once).
__host__ __device__ constexpr uint32_t mv_rep(uint32_t tiles, int num_cus, bool ring) {
  return (tiles + 2u * (uint32_t)num_cus - 1) / (2u * (uint32_t)num_cus) > 1 && ring
             ? (tiles + (uint32_t)num_cus - 1) / (uint32_t)num_cus
             : (tiles + 2u * (uint32_t)num_cus - 1) / (2u * (uint32_t)num_cus);
}

template <int QT, int BPR, int NWV, int PRO, int NMAT>
int mv_launch(g4_ctx* ctx, const LaunchReq& q, const uint8_t* w_up) {
  using T = MvTile<QT, BPR, NWV>;
  static_assert(T::TR == 16 * NWV / BPR, "mv_pick / mv_shape compute the tile rows as 16 NWV / BPR");
  GemvSegs sg{};
  uint32_t tiles = 0;
  for (int i = 0; i < q.nseg; ++i) tiles += ceil_div(q.segs[i].M, T::TR);
  sg.rep = mv_rep(tiles, ctx->num_cus, NWV == 12 && NMAT == 1 && PRO != 3);
  uint32_t wgs = 0;
  for (int i = 0; i < q.nseg; ++i) {
    sg.s[i] = q.segs[i];
    sg.s[i].wg_begin = wgs;
    wgs += ceil_div(ceil_div(q.segs[i].M, T::TR), sg.rep);
  }
  sg.n = q.nseg;
  sg.amx = q.amx;
  sg.d8 = q.d8;
  sg.tk = NMAT == 1 ? q.tk : nullptr;
  if (PRO == 3 && sg.rep != 1)
    return g4::set_error(G4_ERR_UNSUPPORTED, "matvec: digit input needs one tile per workgroup (%u rows)", q.segs[0].M);
  if (q.wgs_out) *q.wgs_out = wgs;
  if (wgs == 0) return G4_OK;
  if (q.amx && wgs > q.amx_cap)
    return g4::set_error(G4_ERR_UNSUPPORTED, "matvec: %u workgroups exceed the %u argmax candidates", wgs, q.amx_cap);
  if (sg.tk && (wgs > q.tk_cap || q.nseg != 1))
    return g4::set_error(G4_ERR_UNSUPPORTED, "matvec: top-k candidates need one matrix and <= %u workgroups (%u)",
                         q.tk_cap, wgs);
  sg.tk_stride = wgs;
  const size_t lds = mv_lds_bytes<QT, BPR, NWV, PRO, NMAT>(sg.rep > 1) + (sg.tk ? 256 * sizeof(g4d::Cand) : 0);
  // rep > 1 means more than 2 * num_cus tiles of the widest workgroup, which
  // mv_pick chooses for at least kMvFullWgs tiles: only the 12-wave
  // instances walk tiles
  if constexpr (NWV == 12 && PRO != 3) {
    if (sg.rep > 1) {
      int rc = claim_lds((const void*)mv_kernel<QT, BPR, NWV, PRO, NMAT, true>, ctx, lds);
      if (rc) return rc;
      hipLaunchKernelGGL((mv_kernel<QT, BPR, NWV, PRO, NMAT, true>), dim3(wgs), dim3(64 * NWV), lds, ctx->stream,
                         sg, w_up, q.pa, q.epi ? q.cap : 0.f);
      G4_LAUNCHED(ctx, "mv");
      return G4_OK;
    }
  }
  if (sg.rep > 1) return g4::set_error(G4_ERR_UNSUPPORTED, "matvec: %d-wave workgroups do not walk tiles", NWV);
  int rc = claim_lds((const void*)mv_kernel<QT, BPR, NWV, PRO, NMAT, false>, ctx, lds);
  if (rc) return rc;
  hipLaunchKernelGGL((mv_kernel<QT, BPR, NWV, PRO, NMAT, false>), dim3(wgs), dim3(64 * NWV), lds, ctx->stream, sg,
                     w_up, q.pa, q.epi ? q.cap : 0.f);
  G4_LAUNCHED(ctx, "mv");
  return G4_OK;
}

// The q/k/v matvec and the attention block in one launch (one sequence,
// one KV head, a window of at most MQF_FAN chunks). Workgroups [0, nmv) are
// the one-tile matvec (Q4_K rows of 1536, MNWV waves: the width the matvec's
// own launch would take, so the rows are the same bit for bit) with its norm
// prologue; each row is also staged, with its tag, in one device-scope
// store.
// Workgroups nmv.. are the attention block's chunk and L2-warming
// workgroups (the first 256 threads; the other two waves end at once).
// A chunk workgroup reads the position and requests its K/V rows at
// once, and polls the staged q/k/v only before its prologue, so the window's
// load overlaps the matvec instead of following a launch boundary. The
// matvec workgroups come first in the grid and wait on nothing: in-order
// dispatch lets them finish whatever the residency, and the wait is bounded.
constexpr int kQkvNwv = 6;  // workgroup width (waves): the wider of the two parts
template <int PRO, int MNWV, bool MERGE>
__global__ __launch_bounds__(64 * kQkvNwv) void qkv_attn_kernel(GemvSegs segs, ProArgs pa, g4mqf::MqfArgs a,
                                                                 uint32_t nmv) {
  static_assert(MNWV <= kQkvNwv && 64 * kQkvNwv >= g4mqf::MQ_NT, "both parts fit the workgroup");
  extern __shared__ __align__(16) uint8_t smem[];
  if (blockIdx.x < nmv) {  // (uniform)
    if (threadIdx.x >= 64u * MNWV) return;  // (uniform per wave)
    mv_body<0, 6, MNWV, PRO, 1, false, true>(segs, nullptr, pa, 0.f, smem);
    return;
  }
  if (threadIdx.x >= (unsigned)g4mqf::MQ_NT) return;  // (uniform per wave)
  g4mqf::mqf_body<false, true, MERGE>(a, blockIdx.x - nmv, 0u, blockIdx.x);
}

// The attention's chunk merge and the o projection, split by head
// (g4_attnHeadsMatmul_q4k). The q/k/v + attention launch without its merge
// leaves per chunk c and head h the partial (m, l, o[256]): the chunk's
// running maximum, its softmax denominator and its unnormalised output.
// Workgroup (tile, group) merges the kHeadsPerWg heads of its group over the
// live chunks (weights exp(m_c - max), as the in-launch merger), digitises
// their outputs exactly as the o matvec's prologue digitises those elements
// (one scale per 32), multiplies them with the group's super-blocks of
// kHeadsRows rows of W_o and writes out[group][row]: that group's share of
// o = sum over groups of out[group]. The next launch (the gate/up prologue,
// PRO 4) adds the kOShares shares in group order. Workgroups also clear the
// staged q/k/v the attention's merger used to clear.
constexpr int kHeadsRows = 32;  // rows per workgroup; 4 units of 64 weights per row and head

struct HeadsArgs {
  const float* ws;       // chunk partials: m [nparts], l [nparts], o [nparts][256]
  uint32_t nparts;       // max_chunks * 8 (one KV head)
  uint32_t max_chunks, chunk;  // chunk length in positions
  uint32_t window, cap;
  const uint32_t* pos_dev;
  const uint8_t* W;      // [M][8 * 256] Q4_K
  float* out;            // [kOShares][M]
  uint32_t M;
  uint64_t* stage;       // staged q/k/v to clear
  uint32_t nstage;
};

__global__ __launch_bounds__(4 * kHeadsRows * kHeadsPerWg) void attn_heads_kernel(HeadsArgs a) {
  constexpr int HPW = kHeadsPerWg, NTH = 4 * kHeadsRows * HPW, U = 4 * HPW;  // U: units per row
  __shared__ __align__(16) uint8_t smem[align16(MvX<HPW>::END)];
  const int tid = threadIdx.x, u = tid % U, slot = tid / U;
  const uint32_t grp = blockIdx.y;
  const uint32_t row = min(blockIdx.x * (uint32_t)kHeadsRows + (uint32_t)slot, a.M - 1);
  // this unit's weights first: 48 bytes of super-block (head) HPW grp + u / 4 of the row
  const uint32_t rb = 8u * 144u;
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)a.W, (short)0, (int)(uint32_t)min((uint64_t)a.M * rb, (uint64_t)0xffffffffu), 0x00020000);
  Q4Unit wu;
  q4_unit_load<2>(wu, rs, row * rb + (HPW * grp + (uint32_t)(u >> 2)) * 144u, u & 3);
  // the staged q/k/v of the attention launch, cleared for the next one
  {
    const uint32_t lin = blockIdx.y * gridDim.x + blockIdx.x, nwg = gridDim.x * gridDim.y;
    for (uint32_t i = lin * (uint32_t)NTH + (uint32_t)tid; i < a.nstage; i += nwg * (uint32_t)NTH)
      a.stage[i] = 0ull;
  }
  using PP = MvPro<HPW, HPW, 0>;  // HPW waves, 4 outputs per lane: the group's 256 HPW outputs
  if (PP::active()) {             // (uniform per wave)
    const uint32_t L = min(*a.pos_dev + 1, a.cap);
    const uint32_t wstart = (a.window != 0 && L > a.window) ? L - a.window : 0;
    const uint32_t nch = (L - wstart + a.chunk - 1) / a.chunk;
    PP P;
    const int e = PP::elem(0);  // this lane's 4 outputs: head HPW grp + e / 256, dims e % 256 ..
    const uint32_t h = HPW * grp + (uint32_t)(e >> 8), d = (uint32_t)(e & 255);
    // every chunk slot is read at a clamped index (a dead chunk's partial
    // is stale) and weighted 0 past the live ones
    float m[g4mqf::MQF_FAN], lv[g4mqf::MQF_FAN];
    float4 o[g4mqf::MQF_FAN];
#pragma unroll
    for (uint32_t c = 0; c < g4mqf::MQF_FAN; ++c) {
      const uint32_t pc = min(c, nch - 1) * 8u + h;
      m[c] = a.ws[pc];
      lv[c] = a.ws[a.nparts + pc];
      o[c] = *(const float4*)(a.ws + 2 * (size_t)a.nparts + (size_t)pc * 256 + d);
    }
    float M = -INFINITY;
#pragma unroll
    for (uint32_t c = 0; c < g4mqf::MQF_FAN; ++c) M = c < nch ? fmaxf(M, m[c]) : M;
    float Ls = 0.f;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (uint32_t c = 0; c < g4mqf::MQF_FAN; ++c) {
      // a stalled chunk's +Inf maximum makes the weights NaN (Inf - Inf)
      const float wc = (c >= nch || m[c] == -INFINITY) ? 0.f : g4mqf::mq_exp(m[c] - M);
      Ls += wc * lv[c];
      acc.x += wc * o[c].x;
      acc.y += wc * o[c].y;
      acc.z += wc * o[c].z;
      acc.w += wc * o[c].w;
    }
    const float li = Ls > 0.f ? 1.0f / Ls : 0.f;  // (NaN stays NaN through acc)
    P.x[0] = make_float4(acc.x * li, acc.y * li, acc.z * li, acc.w * li);
    mv_digitize<HPW, HPW, 0>(P, smem);
  }
  lds_barrier();
  MvUnit<0> X;
  mv_unit_load<0, HPW>(X, smem, u);
  const float v = g4d::group_sum<U>(q4_unit_dot(X, wu, u & 3));
  if (u == 0 && blockIdx.x * (uint32_t)kHeadsRows + (uint32_t)slot < a.M) a.out[(size_t)grp * a.M + row] = v;
}

// workgroup widths in waves for a row of BPR super-blocks (slots must tile it)
struct MvWaveSet {
  int A, B, C, D;
};
constexpr MvWaveSet mv_waves(uint32_t bpr) { return bpr == 32 ? MvWaveSet{12, 8, 6, 4} : MvWaveSet{12, 9, 6, 3}; }
template <int BPR> struct MvWaves {
  static constexpr int A = mv_waves(BPR).A, B = mv_waves(BPR).B, C = mv_waves(BPR).C, D = mv_waves(BPR).D;
};

// The workgroup width of a one-vector launch over row segments of
// 256*bpr-wide rows (the rule stated above kMvFullWgs). Between one and two
// tiles per CU the widest workgroup leaves some CUs two tiles and others
// one: the next width is taken when its tiles spread evenly enough that the
// busiest CU streams fewer bytes (e.g. 2 x 12288 rows of 1536: 384 tiles of
// 12 waves, 128 CUs with two; 512 tiles of 9 waves, two on every CU).
int mv_pick(uint32_t bpr, const GemvSeg* segs, int nseg, int num_cus) {
  const MvWaveSet w = mv_waves(bpr);
  auto tiles = [&](int nwv) {
    const uint32_t slots = (uint32_t)(16 * nwv) / bpr;  // 64 nwv threads over 4 bpr units per row
    uint32_t t = 0;
    for (int i = 0; i < nseg; ++i) t += ceil_div(segs[i].M, slots);
    return t;
  };
  const uint32_t cus = (uint32_t)(num_cus > 0 ? num_cus : 256);
  if (tiles(w.A) >= kMvFullWgs) {
    const uint32_t ta = tiles(w.A), tb = tiles(w.B);
    if (ta > cus && tb <= 2 * cus && ceil_div(tb, cus) * (uint32_t)w.B < ceil_div(ta, cus) * (uint32_t)w.A)
      return w.B;
    return w.A;
  }
  if (tiles(w.B) >= kMvFullWgs) return w.B;
  if (tiles(w.C) >= kMvMinWgs) return w.C;
  return w.D;
}

template <int QT, int BPR, int PRO, int NMAT>
int mv_rows(g4_ctx* ctx, const LaunchReq& q, const uint8_t* w_up) {
  using Wv = MvWaves<BPR>;
  const int nwv = mv_pick(BPR, q.segs, q.nseg, ctx->num_cus);
  if (nwv == Wv::A) return mv_launch<QT, BPR, Wv::A, PRO, NMAT>(ctx, q, w_up);
  if (nwv == Wv::B) return mv_launch<QT, BPR, Wv::B, PRO, NMAT>(ctx, q, w_up);
  if (nwv == Wv::C) return mv_launch<QT, BPR, Wv::C, PRO, NMAT>(ctx, q, w_up);
  return mv_launch<QT, BPR, Wv::D, PRO, NMAT>(ctx, q, w_up);
}

template <int QT, int PRO, int NMAT>
int mv_bpr(g4_ctx* ctx, const LaunchReq& q, const uint8_t* w_up) {
  if constexpr (PRO == 3) {
    // digits come from a GELU product: the FFN width (6144 or 12288)
    switch (q.N / 256) {
      case 24: return mv_rows<QT, 24, PRO, NMAT>(ctx, q, w_up);
      case 48: return mv_rows<QT, 48, PRO, NMAT>(ctx, q, w_up);
      default: return G4_ERR_UNSUPPORTED;
    }
  } else if constexpr (PRO != 0) {
    // the normalising prologues serve the hidden vector (1536 or 2048 wide)
    switch (q.N / 256) {
      case 6: return mv_rows<QT, 6, PRO, NMAT>(ctx, q, w_up);
      case 8: return mv_rows<QT, 8, PRO, NMAT>(ctx, q, w_up);
      default: return G4_ERR_UNSUPPORTED;
    }
  } else {
    switch (q.N / 256) {
      case 4: return mv_rows<QT, 4, PRO, NMAT>(ctx, q, w_up);
      case 6: return mv_rows<QT, 6, PRO, NMAT>(ctx, q, w_up);
      case 8: return mv_rows<QT, 8, PRO, NMAT>(ctx, q, w_up);
      case 12: return mv_rows<QT, 12, PRO, NMAT>(ctx, q, w_up);
      case 16: return mv_rows<QT, 16, PRO, NMAT>(ctx, q, w_up);
      case 24: return mv_rows<QT, 24, PRO, NMAT>(ctx, q, w_up);
      case 32: return mv_rows<QT, 32, PRO, NMAT>(ctx, q, w_up);
      case 48: return mv_rows<QT, 48, PRO, NMAT>(ctx, q, w_up);
      default: return G4_ERR_UNSUPPORTED;
    }
  }
}

template <int QT>
int launch_mv(g4_ctx* ctx, const LaunchReq& q) {
  switch (q.pro) {
    case 0: return mv_bpr<QT, 0, 1>(ctx, q, nullptr);
    case 1: return mv_bpr<QT, 1, 1>(ctx, q, nullptr);
    case 2: return mv_bpr<QT, 2, 1>(ctx, q, nullptr);
    case 3:
      if constexpr (QT == 1) return mv_bpr<QT, 3, 1>(ctx, q, nullptr);
      return G4_ERR_UNSUPPORTED;
    default: return G4_ERR_UNSUPPORTED;
  }
}

int launch_gemv(g4_ctx* ctx, const LaunchReq& q) {
  if (q.nv == 1) return q.qt == 0 ? launch_mv<0>(ctx, q) : launch_mv<1>(ctx, q);
  return q.qt == 0 ? launch_qt<0>(ctx, q) : launch_qt<1>(ctx, q);
}

bool supported_bpr(uint32_t bpr) {
  return bpr == 4 || bpr == 6 || bpr == 8 || bpr == 12 || bpr == 16 || bpr == 24 || bpr == 32 || bpr == 48;
}

int check_mm(const char* fn, const void* in, const void* w, const void* out, g4_matmul_params p) {
  G4_REQUIRE(in && w && out, "%s: null buffer", fn);
  G4_REQUIRE(p.M > 0 && p.N > 0, "%s: empty shape M=%u N=%u", fn, p.M, p.N);
  G4_REQUIRE(p.N % 256 == 0, "%s: N=%u is not a multiple of the 256-weight super-block", fn, p.N);
  G4_REQUIRE(p.N <= 12288, "%s: N=%u exceeds the 12288 activation limit", fn, p.N);
  G4_REQUIRE(((uintptr_t)in & 15) == 0, "%s: input must be 16-byte aligned", fn);
  return G4_OK;
}

int check_w(const char* fn, int qt, const void* w) {
  if (qt == 0) G4_REQUIRE(((uintptr_t)w & 15) == 0, "%s: Q4_K weights must be 16-byte aligned", fn);
  else G4_REQUIRE(((uintptr_t)w & 3) == 0, "%s: Q6_K weights must be 4-byte aligned", fn);
  return G4_OK;
}

int matmul_quant(g4_ctx* ctx, const char* fn, int qt, const float* in, const void* w, float* out, g4_matmul_params p,
                 uint32_t batch) {
  G4_ENTER(ctx);
  int rc = check_mm(fn, in, w, out, p);
  if (rc) return rc;
  rc = check_w(fn, qt, w);
  if (rc) return rc;
  G4_REQUIRE(batch >= 1, "%s: batch must be >= 1", fn);
  const uint32_t bpr = p.N / 256;
  if (!supported_bpr(bpr)) {
    if (batch != 1) return g4::set_error(G4_ERR_UNSUPPORTED, "%s: batched N=%u not supported", fn, p.N);
    const dim3 grid(ceil_div(p.M, NW));
    if (qt == 0)
      hipLaunchKernelGGL(gemv_q4k_generic, grid, dim3(NT), 0, ctx->stream, in, (const uint8_t*)w, out, p.M, p.N);
    else
      hipLaunchKernelGGL(gemv_q6k_generic, grid, dim3(NT), 0, ctx->stream, in, (const uint8_t*)w, out, p.M, p.N);
    G4_LAUNCHED(ctx, fn);
    return G4_OK;
  }
  if (batch >= 16 && batch <= 64) return g4_internal_batch_matmul(ctx, fn, qt, in, w, out, p.M, p.N, batch);
  int nv_max = 8;
  while (nv_max > 1 && gemv_lds(qt, p.N, nv_max) > ctx->lds_max) nv_max >>= 1;
  uint32_t done = 0;
  while (done < batch) {
    const uint32_t left = batch - done;
    int nv = left >= 8 ? 8 : left >= 4 ? 4 : left >= 2 ? 2 : 1;
    if (nv > nv_max) nv = nv_max;
    GemvSeg s{(const uint8_t*)w, out + (size_t)done * p.M, p.M, 0};
    LaunchReq q{qt, &s, 1, p.N, nv, 0, 0, 0.f,
                ProArgs{in + (size_t)done * p.N, nullptr, nullptr, nullptr, nullptr, 0.f}, p.M};
    rc = launch_gemv(ctx, q);
    if (rc) return rc == G4_ERR_UNSUPPORTED ? g4::set_error(rc, "%s: unsupported shape", fn) : rc;
    done += (uint32_t)nv;
  }
  return G4_OK;
}

template <int BPR, int PRO>
int launch_gateup(g4_ctx* ctx, const uint8_t* wg, const uint8_t* wu, float* out, uint32_t M, const ProArgs& pa,
                  uint8_t* d8 = nullptr) {
  const GemvSeg seg{wg, out, M, 0};
  LaunchReq q{0, &seg, 1, BPR * 256, 1, PRO, 0, 0.f, pa, M};
  q.d8 = d8;
  return mv_rows<0, BPR, PRO, 2>(ctx, q, wu);
}

// The one-vector launch's geometry for W [M x 256*bpr] (mv_rows, then
// mv_launch): the workgroup width, the rows a tile holds, the tiles a
// workgroup walks and the workgroup count.
struct MvShape {
  int nwv;
  uint32_t rows_per_tile, rep, wgs;
};
MvShape mv_shape(const g4_ctx* ctx, uint32_t M, uint32_t bpr) {
  const GemvSeg seg{nullptr, nullptr, M, 0};
  MvShape s{};
  s.nwv = mv_pick(bpr, &seg, 1, ctx->num_cus);
  s.rows_per_tile = (uint32_t)(16 * s.nwv) / bpr;
  const uint32_t t = ceil_div(M, s.rows_per_tile);
  s.rep = mv_rep(t, ctx->num_cus, s.nwv == 12);  // as mv_launch for one matrix
  s.wgs = ceil_div(t, s.rep);
  return s;
}

int qkv_attn(g4_ctx* ctx, const char* fn, bool merge, const float* x, const uint16_t* w1, const float* residual,
                              const uint16_t* out_scale, const uint16_t* w2, float* h_out,
                              const void* const* weights, float* const* outputs, int nseg, uint32_t N, float eps,
                              const uint16_t* q_norm_w, const uint16_t* k_norm_w, const uint16_t* rope_freqs,
                              uint16_t* k_cache, uint16_t* v_cache, float* output, g4_attn_fused_params p,
                              void* workspace, size_t workspace_bytes, const uint32_t* position_dev,
                              const g4_warm_region* regions, int nregions, const float* rope_cs,
                              uint32_t rope_rows) {
  G4_ENTER(ctx);
  G4_REQUIRE(nseg == 1 || nseg == 3, "%s: nseg must be 1 (q) or 3 (q, k, v)", fn);
  G4_REQUIRE(weights && outputs, "%s: null buffer", fn);
  const uint32_t rows[3] = {p.num_q_heads * p.head_dim, p.num_kv_heads * p.head_dim, p.num_kv_heads * p.head_dim};
  const float* q_raw = outputs[0];
  const float* k_raw = nseg == 3 ? outputs[1] : nullptr;
  const float* v_raw = nseg == 3 ? outputs[2] : nullptr;
  int rc = g4mqf::mqf_check(ctx, fn, q_raw, k_raw, v_raw, q_norm_w, k_norm_w, rope_freqs,
                            k_cache, v_cache, output, p, workspace, position_dev, regions, nregions, rope_cs,
                            rope_rows);
  if (rc) return rc;
  // the matvec's own checks (g4_normAddScaleMatmulSegments)
  G4_REQUIRE(x && w1, "%s: null buffer", fn);
  G4_REQUIRE(!out_scale || residual, "%s: out_scale needs the residual form", fn);
  G4_REQUIRE(!residual == !w2, "%s: residual and w2 go together", fn);
  G4_REQUIRE(N == 1536 || N == 2048, "%s: N=%u unsupported (1536 or 2048)", fn, N);
  G4_REQUIRE(((uintptr_t)x & 15) == 0 && (!residual || ((uintptr_t)residual & 15) == 0) &&
                 (!h_out || ((uintptr_t)h_out & 15) == 0),
             "%s: activations must be 16-byte aligned", fn);
  G4_REQUIRE(((uintptr_t)w1 & 7) == 0 && ((uintptr_t)w2 & 7) == 0,
             "%s: norm weights must be 8-byte aligned", fn);
  for (int i = 0; i < nseg; ++i) {
    G4_REQUIRE(weights[i] && outputs[i], "%s: segment %d empty", fn, i);
    rc = check_w(fn, 0, weights[i]);
    if (rc) return rc;
  }
  // the one-launch form: q, k and v (a layer reading its producer's cache
  // projects q only, over 256 workgroups of 3 waves that would leave no CU
  // to the attention or its L2 warming: it keeps the two launches), Q4_K
  // rows of 1536 at the width the matvec's own launch takes, one KV head, a
  // window merged in the
  // launch, q/k/v staged in the workspace (at most kMaxStage values)
  GemvSegs sg{};
  for (int i = 0; i < nseg; ++i) sg.s[i] = GemvSeg{(const uint8_t*)weights[i], outputs[i], rows[i], 0};
  const int mnwv = mv_pick(6, sg.s, nseg, ctx->num_cus);
  const uint32_t tr = 16u * (uint32_t)mnwv / 6u;  // rows per tile
  uint32_t nmv = 0;
  for (int i = 0; i < nseg; ++i) {
    sg.s[i].wg_begin = nmv;
    nmv += ceil_div(rows[i], tr);
  }
  bool applies = false;
  g4mqf::MqfLaunch L{};
  if (N == 1536 && mnwv == 6 && nseg == 3 && p.num_kv_heads == 1 && p.head_dim == g4mqf::MQ_HD &&
      rows[0] + 2 * rows[1] <= g4mqf::kMaxStage) {
    rc = g4mqf::mqf_prepare(ctx, q_raw, k_raw, v_raw, q_norm_w, k_norm_w, rope_freqs, k_cache, v_cache, output, p,
                            workspace, workspace_bytes, position_dev, regions, nregions, rope_cs, nmv, applies, L);
    if (rc) return rc;
    applies = applies && !L.partials;
  }
  if (!applies) {  // two launches, the same results
    if (!merge)
      return g4::set_error(G4_ERR_UNSUPPORTED,
                           "%s: the shape does not take the one q/k/v + attention launch with its merge left out", fn);
    rc = g4_normAddScaleMatmulSegments(ctx, 0, x, w1, residual, out_scale, w2, h_out, weights, outputs, rows, nseg,
                                       N, eps, 0.f);
    if (rc) return rc;
    return g4_attnDecodeFusedWarm(ctx, q_raw, k_raw, v_raw, q_norm_w, k_norm_w, rope_freqs, k_cache, v_cache,
                                  output, p, workspace, workspace_bytes, position_dev, regions, nregions, rope_cs,
                                  rope_rows);
  }
  sg.n = nseg;
  sg.rep = 1;
  // staged q/k/v: q at 0, k at nqh * hd, v at (nqh + nkh) * hd
  L.m.nstage = rows[0] + 2 * rows[1];
  for (int i = 0; i < nseg; ++i) sg.s[i].stage = L.m.stage + (i == 0 ? 0 : rows[0] + (size_t)(i - 1) * rows[1]);
  const ProArgs pa{x, w1, residual, w2, h_out, eps, out_scale};
  // g4_test_stage_wait can leave the matvec workgroups out (nothing is
  // staged, so every attention workgroup's bounded wait expires)
  const uint32_t nmv_run = ctx->test_skip_matvec ? 0u : nmv;
  const dim3 grid(nmv_run + L.m.max_chunks + L.m.nwarm), block(64 * kQkvNwv);
  auto launch = [&](auto kern, size_t lds) {
    int r = claim_lds((const void*)kern, ctx, lds);
    if (r) return r;
    hipLaunchKernelGGL(kern, grid, block, lds, ctx->stream, sg, pa, L.m, nmv_run);
    G4_LAUNCHED(ctx, "qkv_attn_fused");
    return G4_OK;
  };
  // (the one launch takes 6-wave matvec workgroups: mnwv == 6 above)
  if (merge) {
    if (residual) return launch(qkv_attn_kernel<2, 6, true>, mv_lds_bytes<0, 6, 6, 2, 1>(false));
    return launch(qkv_attn_kernel<1, 6, true>, mv_lds_bytes<0, 6, 6, 1, 1>(false));
  }
  if (residual) return launch(qkv_attn_kernel<2, 6, false>, mv_lds_bytes<0, 6, 6, 2, 1>(false));
  return launch(qkv_attn_kernel<1, 6, false>, mv_lds_bytes<0, 6, 6, 1, 1>(false));
}

}  // namespace

extern "C" {

int g4_matmulWarmRegion(g4_ctx* ctx, int wtype, uint32_t M, uint32_t N, const void* weight, g4_warm_region* out) {
  G4_ENTER(ctx);
  G4_REQUIRE(out && weight && M > 0, "g4_matmulWarmRegion: null buffer or no rows");
  G4_REQUIRE(wtype == 0 || wtype == 1, "g4_matmulWarmRegion: wtype must be 0 (Q4_K) or 1 (Q6_K)");
  G4_REQUIRE(N % 256 == 0 && supported_bpr(N / 256), "g4_matmulWarmRegion: N=%u has no one-vector launch", N);
  const uint32_t bpr = N / 256;
  const MvShape sh = mv_shape(ctx, M, bpr);
  const uint64_t row_bytes = (uint64_t)bpr * (wtype ? 210 : 144);
  out->base = weight;
  out->total_bytes = (uint64_t)M * row_bytes;
  out->wg_bytes = (uint64_t)sh.rep * sh.rows_per_tile * row_bytes;
  out->nwgs = sh.wgs;
  out->reserved = 0;
  return G4_OK;
}

int g4_matmulQuant_q4k(g4_ctx* ctx, const float* input, const void* weight, float* output, g4_matmul_params p) {
  return matmul_quant(ctx, __func__, 0, input, weight, output, p, 1);
}

int g4_matmulQuantMR4_q4k(g4_ctx* ctx, const float* input, const void* weight, float* output,
                          g4_matmul_params p) {
  return matmul_quant(ctx, __func__, 0, input, weight, output, p, 1);
}

int g4_matmulQuant_q6k(g4_ctx* ctx, const float* input, const void* weight, float* output, g4_matmul_params p) {
  return matmul_quant(ctx, __func__, 1, input, weight, output, p, 1);
}

int g4_matmulQuantBatch_q4k(g4_ctx* ctx, const float* input, const void* weight, float* output,
                            g4_matmul_params p, uint32_t batch) {
  return matmul_quant(ctx, __func__, 0, input, weight, output, p, batch);
}

int g4_matmulQuantBatch_q6k(g4_ctx* ctx, const float* input, const void* weight, float* output,
                            g4_matmul_params p, uint32_t batch) {
  return matmul_quant(ctx, __func__, 1, input, weight, output, p, batch);
}

// g4_dequantPath: values through the unpack of one kernel family. Paths 0
// and 1 (the matvec units) here; path 2 (the matrix-core operands) in
// k_batch.hip. Blocks go in launches of at most 2^24 (the buffer resource
// addresses up to 4 GiB).
int g4_dequantPath(g4_ctx* ctx, int wtype, int path, const void* blocks, uint64_t nblocks, float* out) {
  G4_ENTER(ctx);
  G4_REQUIRE(blocks && out, "g4_dequantPath: null buffer");
  G4_REQUIRE(wtype == 0 || wtype == 1, "g4_dequantPath: wtype must be 0 (Q4_K) or 1 (Q6_K)");
  G4_REQUIRE(path >= 0 && path <= 2, "g4_dequantPath: path must be 0, 1 or 2");
  G4_REQUIRE(((uintptr_t)blocks & 15) == 0, "g4_dequantPath: blocks must be 16-byte aligned");
  if (!nblocks) return G4_OK;
  if (path == 2) return g4_internal_operand_values(ctx, wtype, blocks, nblocks, out);
  const size_t by = wtype == 0 ? 144 : 210;
  constexpr uint64_t kChunk = 1u << 24;
  for (uint64_t b0 = 0; b0 < nblocks; b0 += kChunk) {
    const uint32_t nb = (uint32_t)std::min<uint64_t>(kChunk, nblocks - b0);
    const uint8_t* w = (const uint8_t*)blocks + b0 * by;
    float* o = out + b0 * 256;
    const dim3 grid(ceil_div(nb, UC_BLOCKS));
    if (wtype == 0 && path == 0) hipLaunchKernelGGL((unpack_check_kernel<0, 0>), grid, dim3(NT), 0, ctx->stream, w, nb, o);
    else if (wtype == 0) hipLaunchKernelGGL((unpack_check_kernel<0, 1>), grid, dim3(NT), 0, ctx->stream, w, nb, o);
    else if (path == 0) hipLaunchKernelGGL((unpack_check_kernel<1, 0>), grid, dim3(NT), 0, ctx->stream, w, nb, o);
    else hipLaunchKernelGGL((unpack_check_kernel<1, 1>), grid, dim3(NT), 0, ctx->stream, w, nb, o);
    G4_LAUNCHED(ctx, "unpack_check");
  }
  return G4_OK;
}

int g4_dequantF16(g4_ctx* ctx, int wtype, const void* blocks, uint64_t nblocks, uint16_t* out) {
  G4_ENTER(ctx);
  G4_REQUIRE(blocks && out, "g4_dequantF16: null buffer");
  G4_REQUIRE(wtype >= 0 && wtype <= 3, "g4_dequantF16: wtype must be 0 (Q4_K), 1 (Q6_K), 2 (Q5_K) or 3 (Q8_0)");
  G4_REQUIRE(((uintptr_t)blocks & 15) == 0 && ((uintptr_t)out & 15) == 0,
             "g4_dequantF16: blocks and out must be 16-byte aligned");
  if (!nblocks) return G4_OK;
  if (wtype >= 2) return g4_internal_dequant_f16_q58(ctx, wtype, blocks, nblocks, out);
  const size_t by = wtype == 0 ? 144 : 210;
  constexpr uint64_t kChunk = 1u << 24;
  for (uint64_t b0 = 0; b0 < nblocks; b0 += kChunk) {
    const uint32_t nb = (uint32_t)std::min<uint64_t>(kChunk, nblocks - b0);
    const uint8_t* w = (const uint8_t*)blocks + b0 * by;
    const dim3 grid(ceil_div(nb, UC_BLOCKS));
    if (wtype == 0)
      hipLaunchKernelGGL((unpack_f16_kernel<0>), grid, dim3(NT), 0, ctx->stream, w, nb, out + b0 * 256);
    else
      hipLaunchKernelGGL((unpack_f16_kernel<1>), grid, dim3(NT), 0, ctx->stream, w, nb, out + b0 * 256);
    G4_LAUNCHED(ctx, "unpack_f16");
  }
  return G4_OK;
}

// The dequant debug exports run the one-vector matvec's register units.
int g4_dequant_q4k(g4_ctx* ctx, const void* blocks, uint64_t nblocks, float* out) {
  return g4_dequantPath(ctx, 0, 0, blocks, nblocks, out);
}
int g4_dequant_q6k(g4_ctx* ctx, const void* blocks, uint64_t nblocks, float* out) {
  return g4_dequantPath(ctx, 1, 0, blocks, nblocks, out);
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
  rc = check_w(__func__, 0, weight);
  if (rc) return rc;
  G4_REQUIRE(norm_w && ((uintptr_t)norm_w & 7) == 0, "g4_rmsNormMatmul_q4k: norm weight null or not 8-byte aligned");
  G4_REQUIRE(p.N == 1536 || p.N == 2048, "g4_rmsNormMatmul_q4k: N=%u unsupported (1536 or 2048)", p.N);
  GemvSeg s{(const uint8_t*)weight, y, p.M, 0};
  LaunchReq q{0, &s, 1, p.N, 1, 1, 0, 0.f, ProArgs{x, norm_w, nullptr, nullptr, nullptr, eps}, p.M};
  return launch_gemv(ctx, q);
}

int g4_normAddGateUpGelu_q4k(g4_ctx* ctx, const float* o, const uint16_t* w_post, const float* residual,
                             const uint16_t* w_pre, const void* w_gate, const void* w_up, float* h_out,
                             float* out, g4_matmul_params p, float eps) {
  G4_ENTER(ctx);
  int rc = check_mm(__func__, o, w_gate, out, p);
  if (rc) return rc;
  G4_REQUIRE(w_post && residual && w_pre && w_up, "g4_normAddGateUpGelu_q4k: null buffer");
  G4_REQUIRE(((uintptr_t)w_post & 7) == 0 && ((uintptr_t)w_pre & 7) == 0,
             "g4_normAddGateUpGelu_q4k: norm weights must be 8-byte aligned");
  G4_REQUIRE(((uintptr_t)w_gate & 15) == 0 && ((uintptr_t)w_up & 15) == 0 && ((uintptr_t)residual & 15) == 0,
             "g4_normAddGateUpGelu_q4k: weights and residual must be 16-byte aligned");
  G4_REQUIRE(!h_out || ((uintptr_t)h_out & 15) == 0, "g4_normAddGateUpGelu_q4k: h_out must be 16-byte aligned");
  const ProArgs pa{o, w_post, residual, w_pre, h_out, eps};
  const uint8_t* wg = (const uint8_t*)w_gate;
  const uint8_t* wu = (const uint8_t*)w_up;
  switch (p.N / 256) {
    case 6: return launch_gateup<6, 2>(ctx, wg, wu, out, p.M, pa);
    case 8: return launch_gateup<8, 2>(ctx, wg, wu, out, p.M, pa);
    default:
      return g4::set_error(G4_ERR_UNSUPPORTED, "g4_normAddGateUpGelu_q4k: N=%u unsupported (1536 or 2048)", p.N);
  }
}

int g4_digitsBytes(uint32_t K, size_t* bytes) {
  G4_REQUIRE(bytes && K > 0 && K % 256 == 0, "g4_digitsBytes: K=%u must be a positive multiple of 256", K);
  *bytes = d8_bytes(K);
  return G4_OK;
}

int g4_normAddGateUpGeluDigits_q4k(g4_ctx* ctx, const float* o, const uint16_t* w_post, const float* residual,
                                   const uint16_t* w_pre, const void* w_gate, const void* w_up, float* h_out,
                                   float* out, void* digits, g4_matmul_params p, float eps) {
  G4_ENTER(ctx);
  int rc = check_mm(__func__, o, w_gate, out, p);
  if (rc) return rc;
  G4_REQUIRE(w_post && residual && w_pre && w_up && digits, "g4_normAddGateUpGeluDigits_q4k: null buffer");
  G4_REQUIRE(p.N == 1536, "g4_normAddGateUpGeluDigits_q4k: N=%u unsupported (1536)", p.N);
  G4_REQUIRE(p.M % 256 == 0, "g4_normAddGateUpGeluDigits_q4k: M=%u must be a multiple of 256", p.M);
  G4_REQUIRE(((uintptr_t)w_post & 7) == 0 && ((uintptr_t)w_pre & 7) == 0,
             "g4_normAddGateUpGeluDigits_q4k: norm weights must be 8-byte aligned");
  G4_REQUIRE(((uintptr_t)w_gate & 15) == 0 && ((uintptr_t)w_up & 15) == 0 && ((uintptr_t)residual & 15) == 0 &&
                 ((uintptr_t)digits & 15) == 0 && (!h_out || ((uintptr_t)h_out & 15) == 0),
             "g4_normAddGateUpGeluDigits_q4k: weights, residual, h_out and digits must be 16-byte aligned");
  const ProArgs pa{o, w_post, residual, w_pre, h_out, eps};
  return launch_gateup<6, 2>(ctx, (const uint8_t*)w_gate, (const uint8_t*)w_up, out, p.M, pa, (uint8_t*)digits);
}

int g4_matmulQuantDigits_q6k(g4_ctx* ctx, const void* digits, const void* weight, float* output,
                             g4_matmul_params p) {
  G4_ENTER(ctx);
  G4_REQUIRE(digits && weight && output && p.M > 0, "g4_matmulQuantDigits_q6k: null buffer or no rows");
  G4_REQUIRE(p.N == 6144 || p.N == 12288, "g4_matmulQuantDigits_q6k: N=%u unsupported (6144 or 12288)", p.N);
  G4_REQUIRE(((uintptr_t)digits & 15) == 0, "g4_matmulQuantDigits_q6k: digits must be 16-byte aligned");
  int rc = check_w(__func__, 1, weight);
  if (rc) return rc;
  GemvSeg s{(const uint8_t*)weight, output, p.M, 0};
  LaunchReq q{1, &s, 1, p.N, 1, 3, 0, 0.f, ProArgs{(const float*)digits, nullptr, nullptr, nullptr, nullptr, 0.f},
              p.M};
  return launch_gemv(ctx, q);
}

int g4_normAddMatmulSegments(g4_ctx* ctx, int wtype, const float* x, const uint16_t* w1, const float* residual,
                             const uint16_t* w2, float* h_out, const void* const* weights, float* const* outputs,
                             const uint32_t* rows, int nseg, uint32_t N, float eps, float softcap_cap) {
  return g4_normAddScaleMatmulSegments(ctx, wtype, x, w1, residual, nullptr, w2, h_out, weights, outputs, rows, nseg,
                                       N, eps, softcap_cap);
}

int g4_normAddScaleMatmulSegments(g4_ctx* ctx, int wtype, const float* x, const uint16_t* w1, const float* residual,
                                  const uint16_t* out_scale, const uint16_t* w2, float* h_out,
                                  const void* const* weights, float* const* outputs, const uint32_t* rows, int nseg,
                                  uint32_t N, float eps, float softcap_cap) {
  G4_ENTER(ctx);
  G4_REQUIRE(!out_scale || residual, "g4_normAddScaleMatmulSegments: out_scale needs the residual form");
  G4_REQUIRE(wtype == 0 || wtype == 1, "g4_normAddMatmulSegments: wtype must be 0 (Q4_K) or 1 (Q6_K)");
  G4_REQUIRE(nseg >= 1 && nseg <= 4, "g4_normAddMatmulSegments: 1..4 segments");
  G4_REQUIRE(x && w1 && weights && outputs && rows, "g4_normAddMatmulSegments: null buffer");
  G4_REQUIRE(!residual == !w2, "g4_normAddMatmulSegments: residual and w2 go together");
  G4_REQUIRE(N == 1536 || N == 2048, "g4_normAddMatmulSegments: N=%u unsupported (1536 or 2048)", N);
  G4_REQUIRE(((uintptr_t)x & 15) == 0 && (!residual || ((uintptr_t)residual & 15) == 0) &&
                 (!h_out || ((uintptr_t)h_out & 15) == 0),
             "g4_normAddMatmulSegments: activations must be 16-byte aligned");
  G4_REQUIRE(((uintptr_t)w1 & 7) == 0 && ((uintptr_t)w2 & 7) == 0,
             "g4_normAddMatmulSegments: norm weights must be 8-byte aligned");
  GemvSeg segs[4];
  for (int i = 0; i < nseg; ++i) {
    G4_REQUIRE(weights[i] && outputs[i] && rows[i] > 0, "g4_normAddMatmulSegments: segment %d empty", i);
    int rc = check_w(__func__, wtype, weights[i]);
    if (rc) return rc;
    segs[i] = GemvSeg{(const uint8_t*)weights[i], outputs[i], rows[i], 0};
  }
  const int pro = residual ? 2 : 1;
  LaunchReq q{wtype, segs, nseg, N, 1, pro, softcap_cap != 0.f ? 1 : 0, softcap_cap,
              ProArgs{x, w1, residual, w2, h_out, eps, out_scale}, 0};
  return launch_gemv(ctx, q);
}

int g4_normAddMatmulArgmax(g4_ctx* ctx, int wtype, const float* x, const uint16_t* w1, const float* residual,
                           const uint16_t* w2, float* h_out, const void* weight, float* logits, uint32_t rows,
                           uint32_t N, float eps, float softcap_cap, uint32_t* result, uint32_t* positions,
                           uint32_t delta) {
  G4_ENTER(ctx);
  G4_REQUIRE(wtype == 0 || wtype == 1, "g4_normAddMatmulArgmax: wtype must be 0 (Q4_K) or 1 (Q6_K)");
  G4_REQUIRE(x && w1 && weight && logits && result && rows > 0, "g4_normAddMatmulArgmax: null buffer or no rows");
  G4_REQUIRE(!residual == !w2, "g4_normAddMatmulArgmax: residual and w2 go together");
  G4_REQUIRE(N == 1536 || N == 2048, "g4_normAddMatmulArgmax: N=%u unsupported (1536 or 2048)", N);
  G4_REQUIRE(((uintptr_t)x & 15) == 0 && (!residual || ((uintptr_t)residual & 15) == 0) &&
                 (!h_out || ((uintptr_t)h_out & 15) == 0),
             "g4_normAddMatmulArgmax: activations must be 16-byte aligned");
  G4_REQUIRE(((uintptr_t)w1 & 7) == 0 && ((uintptr_t)w2 & 7) == 0,
             "g4_normAddMatmulArgmax: norm weights must be 8-byte aligned");
  int rc = check_w(__func__, wtype, weight);
  if (rc) return rc;
  // one candidate per workgroup: at most two workgroups per CU for a matrix
  // walked tile by tile, one per tile below that
  const size_t max_parts = 2 * (size_t)ctx->num_cus;
  void* parts = nullptr;
  rc = g4_internal_scratch(ctx, max_parts * sizeof(g4d::Cand), &parts);
  if (rc) return rc;
  GemvSeg seg{(const uint8_t*)weight, logits, rows, 0};
  uint32_t wgs = 0;
  LaunchReq q{wtype, &seg, 1, N, 1, residual ? 2 : 1, softcap_cap != 0.f ? 1 : 0, softcap_cap,
              ProArgs{x, w1, residual, w2, h_out, eps}, 0, (g4d::Cand*)parts, (uint32_t)max_parts, &wgs};
  rc = launch_gemv(ctx, q);
  if (rc) return rc;  // (N is 1536 or 2048: every failure here sets its own message)
  return g4_internal_argmax_final(ctx, parts, (int)wgs, 1, result, positions, delta);
}

int g4_normAddMatmulTopk(g4_ctx* ctx, int wtype, const float* x, const uint16_t* w1, const float* residual,
                         const uint16_t* w2, float* h_out, const void* weight, float* logits, uint32_t rows,
                         uint32_t N, float eps, float softcap_cap, float* result) {
  G4_ENTER(ctx);
  G4_REQUIRE(wtype == 0 || wtype == 1, "g4_normAddMatmulTopk: wtype must be 0 (Q4_K) or 1 (Q6_K)");
  G4_REQUIRE(x && w1 && weight && logits && result && rows > 0, "g4_normAddMatmulTopk: null buffer or no rows");
  G4_REQUIRE(!residual == !w2, "g4_normAddMatmulTopk: residual and w2 go together");
  G4_REQUIRE(N == 1536 || N == 2048, "g4_normAddMatmulTopk: N=%u unsupported (1536 or 2048)", N);
  G4_REQUIRE(((uintptr_t)x & 15) == 0 && (!residual || ((uintptr_t)residual & 15) == 0) &&
                 (!h_out || ((uintptr_t)h_out & 15) == 0),
             "g4_normAddMatmulTopk: activations must be 16-byte aligned");
  G4_REQUIRE(((uintptr_t)w1 & 7) == 0 && ((uintptr_t)w2 & 7) == 0,
             "g4_normAddMatmulTopk: norm weights must be 8-byte aligned");
  int rc = check_w(__func__, wtype, weight);
  if (rc) return rc;
  // 256 candidates per workgroup: at most two workgroups per CU for a
  // matrix walked tile by tile, one per tile below that
  const uint32_t max_parts = 2 * (uint32_t)ctx->num_cus;
  void* parts = nullptr;
  rc = g4_internal_scratch(ctx, (size_t)256 * max_parts * sizeof(g4d::Cand), &parts);
  if (rc) return rc;
  GemvSeg seg{(const uint8_t*)weight, logits, rows, 0};
  uint32_t wgs = 0;
  LaunchReq q{wtype, &seg, 1, N, 1, residual ? 2 : 1, softcap_cap != 0.f ? 1 : 0, softcap_cap,
              ProArgs{x, w1, residual, w2, h_out, eps}, 0, nullptr, 0, &wgs};
  q.tk = (g4d::Cand*)parts;
  q.tk_cap = max_parts;
  rc = launch_gemv(ctx, q);
  if (rc) return rc;
  return g4_internal_topk_final(ctx, parts, (int)wgs, 1, result);
}

int g4_qkvAttnDecodeFusedWarm(g4_ctx* ctx, const float* x, const uint16_t* w1, const float* residual,
                              const uint16_t* out_scale, const uint16_t* w2, float* h_out,
                              const void* const* weights, float* const* outputs, int nseg, uint32_t N, float eps,
                              const uint16_t* q_norm_w, const uint16_t* k_norm_w, const uint16_t* rope_freqs,
                              uint16_t* k_cache, uint16_t* v_cache, float* output, g4_attn_fused_params p,
                              void* workspace, size_t workspace_bytes, const uint32_t* position_dev,
                              const g4_warm_region* regions, int nregions, const float* rope_cs,
                              uint32_t rope_rows) {
  return qkv_attn(ctx, __func__, true, x, w1, residual, out_scale, w2, h_out, weights, outputs, nseg, N, eps, q_norm_w,
                  k_norm_w, rope_freqs, k_cache, v_cache, output, p, workspace, workspace_bytes, position_dev, regions,
                  nregions, rope_cs, rope_rows);
}

int g4_qkvAttnDecodePartials(g4_ctx* ctx, const float* x, const uint16_t* w1, const float* residual,
                             const uint16_t* out_scale, const uint16_t* w2, float* h_out, const void* const* weights,
                             float* const* outputs, int nseg, uint32_t N, float eps, const uint16_t* q_norm_w,
                             const uint16_t* k_norm_w, const uint16_t* rope_freqs, uint16_t* k_cache,
                             uint16_t* v_cache, g4_attn_fused_params p, void* workspace, size_t workspace_bytes,
                             const uint32_t* position_dev, const g4_warm_region* regions, int nregions,
                             const float* rope_cs, uint32_t rope_rows) {
  // (the chunk workgroups write no output: a non-null placeholder for the checks)
  float* no_output = outputs ? outputs[0] : nullptr;
  return qkv_attn(ctx, __func__, false, x, w1, residual, out_scale, w2, h_out, weights, outputs, nseg, N, eps,
                  q_norm_w, k_norm_w, rope_freqs, k_cache, v_cache, no_output, p, workspace, workspace_bytes,
                  position_dev, regions, nregions, rope_cs, rope_rows);
}

int g4_attnHeadsMatmul_q4k(g4_ctx* ctx, void* workspace, size_t workspace_bytes, g4_attn_fused_params p,
                           const uint32_t* position_dev, const void* weight, float* output, uint32_t M) {
  G4_ENTER(ctx);
  G4_REQUIRE(workspace && position_dev && weight && output && M > 0, "g4_attnHeadsMatmul_q4k: null buffer or no rows");
  G4_REQUIRE(p.num_kv_heads == 1 && p.num_q_heads == g4mqf::MQ_G && p.head_dim == g4mqf::MQ_HD,
             "g4_attnHeadsMatmul_q4k: built for 8 query heads of 256 over one KV head");
  G4_REQUIRE(p.max_seq_len > 0, "g4_attnHeadsMatmul_q4k: max_seq_len must be >= 1");
  G4_REQUIRE(((uintptr_t)workspace & 15) == 0 && ((uintptr_t)output & 15) == 0,
             "g4_attnHeadsMatmul_q4k: workspace and output must be 16-byte aligned");
  int rc = check_w(__func__, 0, weight);
  if (rc) return rc;
  bool applies = false;
  g4mqf::MqfLaunch L{};
  uint16_t dummy_w[8] __attribute__((aligned(16))) = {0};  // (plan only: no norm weight is read here)
  rc = g4mqf::mqf_prepare(ctx, nullptr, nullptr, nullptr, dummy_w, nullptr, nullptr, nullptr, nullptr, output, p,
                          workspace, workspace_bytes, position_dev, nullptr, 0, nullptr, 0, applies, L);
  if (rc) return rc;
  G4_REQUIRE(applies && !L.partials && L.m.max_chunks <= g4mqf::MQF_FAN,
             "g4_attnHeadsMatmul_q4k: the window takes the long attention form, whose chunks another launch merges");
  HeadsArgs a{};
  a.ws = L.m.ws;
  a.nparts = L.m.max_chunks * g4mqf::MQ_G;
  a.max_chunks = L.m.max_chunks;
  a.chunk = g4mqf::MQ_STEP * L.m.nstep;
  a.window = p.sliding_window;
  a.cap = p.max_seq_len;
  a.pos_dev = position_dev;
  a.W = (const uint8_t*)weight;
  a.out = output;
  a.M = M;
  a.stage = L.m.stage;
  a.nstage = p.num_q_heads * p.head_dim + 2 * p.num_kv_heads * p.head_dim;
  const dim3 grid(ceil_div(M, (uint32_t)kHeadsRows), p.num_q_heads / kHeadsPerWg);
  hipLaunchKernelGGL(attn_heads_kernel, grid, dim3(4 * kHeadsRows * kHeadsPerWg), 0, ctx->stream, a);
  G4_LAUNCHED(ctx, "attn_heads");
  return G4_OK;
}

int g4_normAddPartsGateUpGeluDigits_q4k(g4_ctx* ctx, const float* o_parts, const uint16_t* w_post,
                                        const float* residual, const uint16_t* w_pre, const void* w_gate,
                                        const void* w_up, float* h_out, float* out, void* digits, g4_matmul_params p,
                                        float eps) {
  G4_ENTER(ctx);
  int rc = check_mm(__func__, o_parts, w_gate, out, p);
  if (rc) return rc;
  G4_REQUIRE(w_post && residual && w_pre && w_up && digits, "g4_normAddPartsGateUpGeluDigits_q4k: null buffer");
  G4_REQUIRE(p.N == 1536, "g4_normAddPartsGateUpGeluDigits_q4k: N=%u unsupported (1536)", p.N);
  G4_REQUIRE(p.M % 256 == 0, "g4_normAddPartsGateUpGeluDigits_q4k: M=%u must be a multiple of 256", p.M);
  G4_REQUIRE(((uintptr_t)w_post & 7) == 0 && ((uintptr_t)w_pre & 7) == 0,
             "g4_normAddPartsGateUpGeluDigits_q4k: norm weights must be 8-byte aligned");
  G4_REQUIRE(((uintptr_t)w_gate & 15) == 0 && ((uintptr_t)w_up & 15) == 0 && ((uintptr_t)residual & 15) == 0 &&
                 ((uintptr_t)digits & 15) == 0 && (!h_out || ((uintptr_t)h_out & 15) == 0),
             "g4_normAddPartsGateUpGeluDigits_q4k: weights, residual, h_out and digits must be 16-byte aligned");
  const ProArgs pa{o_parts, w_post, residual, w_pre, h_out, eps};
  return launch_gateup<6, 4>(ctx, (const uint8_t*)w_gate, (const uint8_t*)w_up, out, p.M, pa, (uint8_t*)digits);
}

}  // extern "C"
