// k_batch.hip — quantized matmul for several activation vectors (ragged
// multi-sequence decode) on the gfx950 matrix cores.
//
// Y[v][m] = sum_k W[m,k] X[v][k] for B vectors (src/engine.ts runs the
// per-token matmulQuant of shaders/matmul_quant.wgsl:21-54 once per sequence;
// here one launch serves all sequences, so each weight byte is read once).
//
//  * quant_kernel turns the B activation vectors into two-digit int8 form
//    (x ~= s * (256*hi + lo) per 32-element sub-block, s = max|x| / 32512),
//    optionally after RMSNorm or residual-add + RMSNorm, into the context
//    scratch buffer. Layout: for sub-block sb, vector v and 8-element group q,
//    16 bytes [hi x8][lo x8] at ((sb*Bp + v)*4 + q)*16; (s, sum) as a float2
//    at [sb*Bp + v]. Bp = 16, 32 or 64 (the MFMA column tiles of a launch).
//  * mm_kernel: a workgroup owns 16 rows; its waves split K by whole
//    super-blocks. Per 32-element sub-block a wave runs
//    v_mfma_i32_16x16x32_i8 with A = 16 rows x 32 weight codes and B = 32
//    digits x 16 vectors (once for hi, once for lo), so the integer products
//    are exact and the sub-block's scales are applied once per output in
//    f32. Q6_K's two 16-element runs of a sub-block sit in lane groups {0,1}
//    and {2,3} of the A operand; two MFMAs with the other half zeroed give
//    each run its own scale. Wave partials meet in LDS.
#include "g4_internal.hpp"

namespace {

constexpr float XQ = 32512.0f;  // |v| <= 32512 keeps both digits in [-128, 127]
constexpr int QNT = 256;        // quant_kernel threads

typedef uint32_t u32x3a __attribute__((ext_vector_type(3), aligned(4)));
typedef int int4v __attribute__((ext_vector_type(4)));

// Vectors are padded to the 16, 32 or 64 columns of the MFMA tiles a launch uses.
__host__ __device__ constexpr uint32_t pad_batch(uint32_t b) { return b <= 16 ? 16 : (b <= 32 ? 32 : 64); }

struct DigitBuf {
  uint8_t* dq;  // [K/32][Bp][4][16] hi/lo bytes
  float2* ds;   // [K/32][Bp] (scale, sum)
  uint32_t Bp;
};

__host__ inline size_t digit_bytes(uint32_t K, uint32_t Bp) {
  return (size_t)2 * K * Bp + (size_t)(K / 32) * Bp * sizeof(float2);
}

// Prologue modes (as the one-vector matvec): 0 = x; 1 = x * w1 / rms(x);
// 2 = h = residual + x * w1 / rms(x) (written to h_out), x' = h * w2 / rms(h).
struct QuantArgs {
  const float* x;  // [B][K]
  const uint16_t* w1;
  const float* residual;  // [B][K]
  const uint16_t* w2;
  float* h_out;  // [B][K]
  float eps;
  DigitBuf d;
};

__device__ __forceinline__ float4 mulw(float4 x, uint2 w, float s) {
  return make_float4(x.x * g4d::f16_bits_to_f32(w.x & 0xffffu) * s, x.y * g4d::f16_bits_to_f32(w.x >> 16) * s,
                     x.z * g4d::f16_bits_to_f32(w.y & 0xffffu) * s, x.w * g4d::f16_bits_to_f32(w.y >> 16) * s);
}
__device__ __forceinline__ float sq4(float4 v) { return (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w); }

// One workgroup per vector; thread t holds the float4 at element 4t + 1024p.
template <int BPR, int PRO>
__global__ __launch_bounds__(QNT) void quant_kernel(QuantArgs a) {
  constexpr int K = BPR * 256;
  constexpr int XP = (K + 4 * QNT - 1) / (4 * QNT);
  __shared__ float red[2 * (QNT / 64)];
  const uint32_t v = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63;
  float4 x[XP], r[PRO == 2 ? XP : 1];
  uint2 w1[PRO >= 1 ? XP : 1], w2[PRO == 2 ? XP : 1];
#pragma unroll
  for (int p = 0; p < XP; ++p) {  // unconditional loads at clamped offsets
    const int f = 4 * tid + 4 * QNT * p, fc = f < K ? f : 0;
    x[p] = *(const float4*)(a.x + (size_t)v * K + fc);
    if constexpr (PRO >= 1) w1[p] = *(const uint2*)(a.w1 + fc);
    if constexpr (PRO == 2) {
      r[p] = *(const float4*)(a.residual + (size_t)v * K + fc);
      w2[p] = *(const uint2*)(a.w2 + fc);
    }
  }
  if constexpr (PRO >= 1) {
    float ss = 0.f;
#pragma unroll
    for (int p = 0; p < XP; ++p) ss += (4 * tid + 4 * QNT * p < K) ? sq4(x[p]) : 0.f;
    ss = g4d::wave_sum_dpp(ss);
    if (lane == 0) red[tid >> 6] = ss;
    __syncthreads();
    float t1 = 0.f;
#pragma unroll
    for (int i = 0; i < QNT / 64; ++i) t1 += red[i];
    const float inv1 = 1.0f / sqrtf(t1 / (float)K + a.eps);
    if constexpr (PRO == 1) {
#pragma unroll
      for (int p = 0; p < XP; ++p) x[p] = mulw(x[p], w1[p], inv1);
    } else {
      float ss2 = 0.f;
#pragma unroll
      for (int p = 0; p < XP; ++p) {
        const int f = 4 * tid + 4 * QNT * p;
        const float4 t = mulw(x[p], w1[p], inv1);
        x[p] = make_float4(r[p].x + t.x, r[p].y + t.y, r[p].z + t.z, r[p].w + t.w);
        ss2 += f < K ? sq4(x[p]) : 0.f;
        if (a.h_out && f < K) *(float4*)(a.h_out + (size_t)v * K + f) = x[p];
      }
      ss2 = g4d::wave_sum_dpp(ss2);
      if (lane == 0) red[QNT / 64 + (tid >> 6)] = ss2;
      __syncthreads();
      float t2 = 0.f;
#pragma unroll
      for (int i = 0; i < QNT / 64; ++i) t2 += red[QNT / 64 + i];
      const float inv2 = 1.0f / sqrtf(t2 / (float)K + a.eps);
#pragma unroll
      for (int p = 0; p < XP; ++p) x[p] = mulw(x[p], w2[p], inv2);
    }
  }
#pragma unroll
  for (int p = 0; p < XP; ++p) {
    const int f = 4 * tid + 4 * QNT * p;
    const float4 xv = x[p];
    float am = fmaxf(fmaxf(fabsf(xv.x), fabsf(xv.y)), fmaxf(fabsf(xv.z), fabsf(xv.w)));
    float sm = (xv.x + xv.y) + (xv.z + xv.w);
    am = g4d::max8(am);
    sm = g4d::sum8(sm);
    const float inv = am > 0.f ? XQ / am : 0.f;
    const float xs[4] = {xv.x, xv.y, xv.z, xv.w};
    uint32_t ph = 0, pl = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int q = (int)__builtin_rintf(xs[e] * inv);
      const int lo = ((q + 128) & 255) - 128;
      const int hi = (q - lo) >> 8;
      ph |= (uint32_t)(hi & 255) << (8 * e);
      pl |= (uint32_t)(lo & 255) << (8 * e);
    }
    if (f < K) {
      const uint32_t sb = (uint32_t)f / 32, e = (uint32_t)f % 32;
      uint8_t* dst = a.d.dq + (((size_t)sb * a.d.Bp + v) * 4 + e / 8) * 16 + (e % 8);
      *(uint32_t*)dst = ph;
      *(uint32_t*)(dst + 8) = pl;
      if ((lane & 7) == 0) a.d.ds[(size_t)sb * a.d.Bp + v] = make_float2(am * (1.0f / XQ), sm);
    }
  }
}

// ---------------------------------------------------------------------------
// matmul
// ---------------------------------------------------------------------------

template <int QT>
struct MmBlock;
template <> struct MmBlock<0> { static constexpr int BYTES = 144; };
template <> struct MmBlock<1> { static constexpr int BYTES = 210; };

// Super-blocks per wave and waves per workgroup for a row of BPR blocks.
template <int BPR>
struct MmGeom {
  static constexpr int BPW = (BPR + 15) / 16;
  static constexpr int NWK = BPR / BPW;
  static_assert(NWK * BPW == BPR && NWK <= 16, "whole blocks per wave");
};

struct MmSeg {
  const uint8_t* W;
  float* Y;  // [B][M]
  uint32_t M;
  uint32_t wg_begin;
};
struct MmArgs {
  MmSeg s[4];
  int n;
  uint32_t B;
  float cap;  // softcap when > 0
  DigitBuf d;
};

// 8 bytes at a 2-byte aligned address: three aligned dwords, funnel-shifted.
__device__ __forceinline__ uint2 ld8_a2(const uint8_t* p) {
  const uintptr_t ad = (uintptr_t)p;
  const u32x3a w = *(const u32x3a*)(p - (ad & 3));
  const uint32_t sh = (uint32_t)(ad & 3);
  return make_uint2(__builtin_amdgcn_alignbyte(w.y, w.x, sh), __builtin_amdgcn_alignbyte(w.z, w.y, sh));
}

__device__ __forceinline__ long as_long(uint2 v) { return (long)(((uint64_t)v.y << 32) | v.x); }

// Q6_K codes minus 32 as signed bytes: c in [0,63] -> c - 32 in two's complement.
__device__ __forceinline__ uint32_t q6_signed(uint32_t c) {
  const uint32_t t = c ^ 0x20202020u;
  const uint32_t neg = t & 0x20202020u;  // bit 5 set <=> c < 32
  return t | (neg << 1) | (neg << 2);
}

template <int QT, int BPR, int NTV>
__global__ __launch_bounds__(64 * MmGeom<BPR>::NWK) void mm_kernel(MmArgs a) {
  using Gm = MmGeom<BPR>;
  constexpr int BPW = Gm::BPW, NWK = Gm::NWK, BY = MmBlock<QT>::BYTES;
  constexpr int SBW = 8 * BPW;  // sub-blocks per wave
  __shared__ float part[NWK][16][16 * NTV];

  int si = 0;
#pragma unroll
  for (int i = 1; i < 4; ++i)
    if (i < a.n && blockIdx.x >= a.s[i].wg_begin) si = i;
  const MmSeg sg = a.s[si];
  const uint32_t row0 = (blockIdx.x - sg.wg_begin) * 16;
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int ra = l & 15, qa = l >> 4;   // A row / C column, k-group
  const uint32_t arow = min(row0 + (uint32_t)ra, sg.M - 1);
  const uint32_t b0 = (uint32_t)w * BPW;  // first super-block of this wave
  const uint8_t* wa = sg.W + ((size_t)arow * BPR + b0) * BY;
  const uint32_t Bp = a.d.Bp;

  // ---- every load of this wave, issued first ----
  // A-side weight pieces (row arow, group qa)
  uint2 qs[BPW][QT == 0 ? 4 : 6];
#pragma unroll
  for (int i = 0; i < BPW; ++i) {
    const uint8_t* blk = wa + (size_t)i * BY;
    if constexpr (QT == 0) {
#pragma unroll
      for (int g = 0; g < 4; ++g) qs[i][g] = *(const uint2*)(blk + 16 + 32 * g + 8 * qa);
    } else {
      // ql[64h + 32c + 8qa..+8] (c = k' & 1) and qh[32h + 8qa..+8]
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        qs[i][2 * h] = ld8_a2(blk + 64 * h + 8 * qa);
        qs[i][2 * h + 1] = ld8_a2(blk + 64 * h + 32 + 8 * qa);
        qs[i][4 + h] = ld8_a2(blk + 128 + 32 * h + 8 * qa);
      }
    }
  }
  // C-side scale data of rows row0 + 4qa + r
  uint4 hd[BPW][4];  // Q4_K: header; Q6_K: sc[16] as 4 dwords (x..w)
  uint32_t dq6[BPW][4];
#pragma unroll
  for (int i = 0; i < BPW; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t crow = min(row0 + 4 * qa + r, sg.M - 1);
      const uint8_t* blk = sg.W + ((size_t)crow * BPR + b0 + i) * BY;
      if constexpr (QT == 0) {
        hd[i][r] = *(const uint4*)blk;
      } else {
        // sc[16] at bytes 192..207 from aligned dwords that stay inside the
        // 210-byte block: four from the dword holding byte 192, and a fifth
        // only needed (and only read past them) when the block is 2 mod 4
        const uintptr_t ad = (uintptr_t)(blk + 192);
        const uint32_t sh = (uint32_t)(ad & 3);
        const uint32_t* p4 = (const uint32_t*)(blk + 192 - sh);
        const uint32_t x0 = p4[0], x1 = p4[1], x2 = p4[2], x3 = p4[3];
        const uint32_t x4 = *(const uint32_t*)((const uint8_t*)p4 + 12 + 2 * sh);  // +16 when sh == 2
        hd[i][r] = make_uint4(__builtin_amdgcn_alignbyte(x1, x0, sh), __builtin_amdgcn_alignbyte(x2, x1, sh),
                              __builtin_amdgcn_alignbyte(x3, x2, sh), __builtin_amdgcn_alignbyte(x4, x3, sh));
        dq6[i][r] = *(const uint16_t*)(blk + 208);
      }
    }
  // B-side digits and scales of this wave's sub-blocks
  uint4 dg[SBW][NTV];
  float2 sc2[SBW][NTV];
#pragma unroll
  for (int s = 0; s < SBW; ++s)
#pragma unroll
    for (int t = 0; t < NTV; ++t) {
      const size_t sb = (size_t)b0 * 8 + s;
      dg[s][t] = *(const uint4*)(a.d.dq + ((sb * Bp + 16 * t + ra) * 4 + qa) * 16);
      sc2[s][t] = a.d.ds[sb * Bp + 16 * t + ra];
    }

  // ---- sub-block products ----
  float acc[NTV][4];
#pragma unroll
  for (int t = 0; t < NTV; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[t][r] = 0.f;

#pragma unroll
  for (int i = 0; i < BPW; ++i) {
    float d[4], dm[4];
    if constexpr (QT == 0) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        d[r] = g4d::f16_bits_to_f32(hd[i][r].x & 0xffffu);
        dm[r] = g4d::f16_bits_to_f32(hd[i][r].x >> 16);
      }
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) d[r] = g4d::f16_bits_to_f32(dq6[i][r]);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int s = i * 8 + j;
      if constexpr (QT == 0) {
        // sub-block j = low (even j) or high (odd j) nibbles of qs group j/2
        const uint2 raw = qs[i][j / 2];
        const uint2 codes = (j & 1) ? make_uint2((raw.x >> 4) & 0x0f0f0f0fu, (raw.y >> 4) & 0x0f0f0f0fu)
                                    : make_uint2(raw.x & 0x0f0f0f0fu, raw.y & 0x0f0f0f0fu);
        const long av = as_long(codes);
        float scr[4], mnr[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          // scale / min of sub-block j (src/gguf.ts:175-182)
          const uint32_t S0 = hd[i][r].y, S1 = hd[i][r].z, S2 = hd[i][r].w;
          const int sh = 8 * (j & 3);
          uint32_t scv, mv;
          if (j < 4) {
            scv = (S0 >> sh) & 63u;
            mv = (S1 >> sh) & 63u;
          } else {
            scv = ((S2 >> sh) & 15u) | (((S0 >> sh) >> 6 & 3u) << 4);
            mv = ((S2 >> sh) >> 4 & 15u) | (((S1 >> sh) >> 6 & 3u) << 4);
          }
          scr[r] = d[r] * (float)scv;
          mnr[r] = dm[r] * (float)mv;
        }
#pragma unroll
        for (int t = 0; t < NTV; ++t) {
          const int4v z = {0, 0, 0, 0};
          const int4v ch = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, as_long(make_uint2(dg[s][t].x, dg[s][t].y)), z,
                                                                  0, 0, 0);
          const int4v cl = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, as_long(make_uint2(dg[s][t].z, dg[s][t].w)), z,
                                                                  0, 0, 0);
          const float2 ss = sc2[s][t];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int I = ch[r] * 256 + cl[r];
            acc[t][r] += scr[r] * ss.x * (float)I - mnr[r] * ss.y;
          }
        }
      } else {
        // sub-block j: half h = j / 4, run pair k' = j % 4 (src/gguf.ts:344-361)
        const int h = j / 4, kp = j % 4;
        const uint2 ql = qs[i][2 * h + (kp & 1)];
        const uint2 qh = qs[i][4 + h];
        const uint32_t lo0 = kp < 2 ? (ql.x & 0x0f0f0f0fu) : ((ql.x >> 4) & 0x0f0f0f0fu);
        const uint32_t lo1 = kp < 2 ? (ql.y & 0x0f0f0f0fu) : ((ql.y >> 4) & 0x0f0f0f0fu);
        const uint32_t hb0 = ((qh.x >> (2 * kp)) & 0x03030303u) << 4;
        const uint32_t hb1 = ((qh.y >> (2 * kp)) & 0x03030303u) << 4;
        const uint2 codes = make_uint2(q6_signed(lo0 | hb0), q6_signed(lo1 | hb1));
        const bool first = qa < 2;  // lanes of the sub-block's first 16-element run
        const long a0 = first ? as_long(codes) : 0l;
        const long a1 = first ? 0l : as_long(codes);
        int sca[4], scb[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          // sc[8h + 2k' + (0|1)] as signed bytes
          const int is = 8 * h + 2 * kp;
          const uint32_t wd = (is < 4) ? hd[i][r].x : (is < 8) ? hd[i][r].y : (is < 12) ? hd[i][r].z : hd[i][r].w;
          sca[r] = (int)(int8_t)((wd >> (8 * (is & 3))) & 0xffu);
          scb[r] = (int)(int8_t)((wd >> (8 * ((is + 1) & 3))) & 0xffu);
        }
#pragma unroll
        for (int t = 0; t < NTV; ++t) {
          const int4v z = {0, 0, 0, 0};
          const long bh = as_long(make_uint2(dg[s][t].x, dg[s][t].y));
          const long bl = as_long(make_uint2(dg[s][t].z, dg[s][t].w));
          const int4v ah = __builtin_amdgcn_mfma_i32_16x16x32_i8(a0, bh, z, 0, 0, 0);
          const int4v al = __builtin_amdgcn_mfma_i32_16x16x32_i8(a0, bl, z, 0, 0, 0);
          const int4v bh2 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a1, bh, z, 0, 0, 0);
          const int4v bl2 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a1, bl, z, 0, 0, 0);
          const float sx = sc2[s][t].x;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int I = (ah[r] * 256 + al[r]) * sca[r] + (bh2[r] * 256 + bl2[r]) * scb[r];
            acc[t][r] += d[r] * sx * (float)I;
          }
        }
      }
    }
  }

  // ---- wave partials -> LDS -> rows ----
#pragma unroll
  for (int t = 0; t < NTV; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) part[w][4 * qa + r][16 * t + ra] = acc[t][r];
  __syncthreads();
  for (int o = threadIdx.x; o < 16 * 16 * NTV; o += 64 * NWK) {
    const int rr = o / (16 * NTV), vv = o % (16 * NTV);
    float y = 0.f;
#pragma unroll
    for (int ww = 0; ww < NWK; ++ww) y += part[ww][rr][vv];
    const uint32_t row = row0 + rr;
    if (row < sg.M && (uint32_t)vv < a.B) {
      if (a.cap > 0.f) {
        const float t = fminf(fmaxf(y / a.cap, -15.0f), 15.0f);
        y = tanhf(t) * a.cap;
      }
      sg.Y[(size_t)vv * sg.M + row] = y;
    }
  }
}

// ---------------------------------------------------------------------------
// host
// ---------------------------------------------------------------------------

template <int BPR>
int quant_bpr(g4_ctx* ctx, int pro, const QuantArgs& q, uint32_t B) {
  const dim3 grid(B);
  if (pro == 0) hipLaunchKernelGGL((quant_kernel<BPR, 0>), grid, dim3(QNT), 0, ctx->stream, q);
  else if (pro == 1) hipLaunchKernelGGL((quant_kernel<BPR, 1>), grid, dim3(QNT), 0, ctx->stream, q);
  else hipLaunchKernelGGL((quant_kernel<BPR, 2>), grid, dim3(QNT), 0, ctx->stream, q);
  G4_LAUNCHED(ctx, "quant");
  return G4_OK;
}

template <int QT, int BPR, int NTV>
int mm_launch(g4_ctx* ctx, MmArgs& a) {
  uint32_t wgs = 0;
  for (int i = 0; i < a.n; ++i) {
    a.s[i].wg_begin = wgs;
    wgs += ceil_div(a.s[i].M, 16);
  }
  hipLaunchKernelGGL((mm_kernel<QT, BPR, NTV>), dim3(wgs), dim3(64 * MmGeom<BPR>::NWK), 0, ctx->stream, a);
  G4_LAUNCHED(ctx, "mm");
  return G4_OK;
}

template <int QT, int BPR>
int mm_ntv(g4_ctx* ctx, MmArgs& a) {  // Bp == 16 * NTV
  if (a.d.Bp == 16) return mm_launch<QT, BPR, 1>(ctx, a);
  if (a.d.Bp == 32) return mm_launch<QT, BPR, 2>(ctx, a);
  return mm_launch<QT, BPR, 4>(ctx, a);
}

bool mm_supported(uint32_t bpr) { return bpr == 4 || bpr == 6 || bpr == 8 || bpr == 12 || bpr == 16 || bpr == 24 || bpr == 32 || bpr == 48; }

template <int QT>
int mm_bpr(g4_ctx* ctx, uint32_t N, MmArgs& a) {
  switch (N / 256) {
    case 4: return mm_ntv<QT, 4>(ctx, a);
    case 6: return mm_ntv<QT, 6>(ctx, a);
    case 8: return mm_ntv<QT, 8>(ctx, a);
    case 12: return mm_ntv<QT, 12>(ctx, a);
    case 16: return mm_ntv<QT, 16>(ctx, a);
    case 24: return mm_ntv<QT, 24>(ctx, a);
    case 32: return mm_ntv<QT, 32>(ctx, a);
    case 48: return mm_ntv<QT, 48>(ctx, a);
    default: return G4_ERR_UNSUPPORTED;
  }
}

int quant_launch(g4_ctx* ctx, uint32_t N, int pro, const QuantArgs& q, uint32_t B) {
  switch (N / 256) {
    case 4: return quant_bpr<4>(ctx, pro, q, B);
    case 6: return quant_bpr<6>(ctx, pro, q, B);
    case 8: return quant_bpr<8>(ctx, pro, q, B);
    case 12: return quant_bpr<12>(ctx, 0, q, B);
    case 16: return quant_bpr<16>(ctx, 0, q, B);
    case 24: return quant_bpr<24>(ctx, 0, q, B);
    case 32: return quant_bpr<32>(ctx, 0, q, B);
    case 48: return quant_bpr<48>(ctx, 0, q, B);
    default: return G4_ERR_UNSUPPORTED;
  }
}

// Digits of B vectors into the context scratch, then one matmul launch over
// up to four matrices sharing the input.
int batch_matmul(g4_ctx* ctx, const char* fn, int qt, int pro, const QuantArgs& q0, const uint8_t* const* W,
                 float* const* Y, const uint32_t* rows, int nseg, uint32_t N, uint32_t B, float cap) {
  G4_REQUIRE(B >= 1 && B <= 64, "%s: batch %u outside 1..64", fn, B);
  G4_REQUIRE(N % 256 == 0 && mm_supported(N / 256), "%s: N=%u unsupported", fn, N);
  G4_REQUIRE(pro == 0 || N == 1536 || N == 2048, "%s: normalising prologue needs N 1536 or 2048", fn);
  const uint32_t Bp = pad_batch(B);
  void* scratch = nullptr;
  int rc = g4_internal_scratch(ctx, digit_bytes(N, Bp), &scratch);
  if (rc) return rc;
  QuantArgs q = q0;
  q.d.dq = (uint8_t*)scratch;
  q.d.ds = (float2*)((uint8_t*)scratch + (size_t)2 * N * Bp);
  q.d.Bp = Bp;
  rc = quant_launch(ctx, N, pro, q, B);
  if (rc) return rc;
  MmArgs a{};
  for (int i = 0; i < nseg; ++i) a.s[i] = MmSeg{W[i], Y[i], rows[i], 0};
  a.n = nseg;
  a.B = B;
  a.cap = cap;
  a.d = q.d;
  rc = qt == 0 ? mm_bpr<0>(ctx, N, a) : mm_bpr<1>(ctx, N, a);
  return rc == G4_ERR_UNSUPPORTED ? g4::set_error(rc, "%s: unsupported shape", fn) : rc;
}

}  // namespace

// Used by k_gemv.hip's batched entry points for batch >= 16.
int g4_internal_batch_matmul(g4_ctx* ctx, const char* fn, int qt, const float* x, const void* w, float* y,
                             uint32_t M, uint32_t N, uint32_t batch) {
  const QuantArgs q{x, nullptr, nullptr, nullptr, nullptr, 0.f, DigitBuf{}};
  const uint8_t* W[1] = {(const uint8_t*)w};
  float* Y[1] = {y};
  const uint32_t rows[1] = {M};
  return batch_matmul(ctx, fn, qt, 0, q, W, Y, rows, 1, N, batch, 0.f);
}

extern "C" {

int g4_normAddMatmulSegmentsBatch(g4_ctx* ctx, int wtype, const float* x, const uint16_t* w1,
                                  const float* residual, const uint16_t* w2, float* h_out,
                                  const void* const* weights, float* const* outputs, const uint32_t* rows, int nseg,
                                  uint32_t N, float eps, float softcap_cap, uint32_t batch) {
  G4_ENTER(ctx);
  G4_REQUIRE(wtype == 0 || wtype == 1, "g4_normAddMatmulSegmentsBatch: wtype must be 0 (Q4_K) or 1 (Q6_K)");
  G4_REQUIRE(nseg >= 1 && nseg <= 4, "g4_normAddMatmulSegmentsBatch: 1..4 segments");
  G4_REQUIRE(x && weights && outputs && rows, "g4_normAddMatmulSegmentsBatch: null buffer");
  G4_REQUIRE(!residual == !w2, "g4_normAddMatmulSegmentsBatch: residual and w2 go together");
  G4_REQUIRE(((uintptr_t)x & 15) == 0 && (!residual || ((uintptr_t)residual & 15) == 0) &&
                 (!h_out || ((uintptr_t)h_out & 15) == 0),
             "g4_normAddMatmulSegmentsBatch: activations must be 16-byte aligned");
  G4_REQUIRE((!w1 || ((uintptr_t)w1 & 7) == 0) && (!w2 || ((uintptr_t)w2 & 7) == 0),
             "g4_normAddMatmulSegmentsBatch: norm weights must be 8-byte aligned");
  const uint8_t* W[4];
  float* Y[4];
  for (int i = 0; i < nseg; ++i) {
    G4_REQUIRE(weights[i] && outputs[i] && rows[i] > 0, "g4_normAddMatmulSegmentsBatch: segment %d empty", i);
    G4_REQUIRE(((uintptr_t)weights[i] & (wtype == 0 ? 15 : 3)) == 0,
               "g4_normAddMatmulSegmentsBatch: weights misaligned (Q4_K 16 B, Q6_K 4 B)");
    W[i] = (const uint8_t*)weights[i];
    Y[i] = outputs[i];
  }
  const int pro = !w1 ? 0 : (residual ? 2 : 1);
  const QuantArgs q{x, w1, residual, w2, h_out, eps, DigitBuf{}};
  return batch_matmul(ctx, __func__, wtype, pro, q, W, Y, rows, nseg, N, batch, softcap_cap);
}

}  // extern "C"
