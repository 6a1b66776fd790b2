// k_batch.hip — quantized matmul for many activation vectors (ragged
// multi-sequence decode) on the gfx950 matrix cores.
//
// Y[v][m] = sum_k W[m,k] X[v][k] for B <= 64 vectors (src/engine.ts runs the
// per-token matmulQuant of shaders/matmul_quant.wgsl:21-54 once per sequence;
// here one launch serves all sequences, so each weight byte is read once).
//
//  * mmf_kernel: a workgroup (4 waves) owns 64 rows (16 per wave) and a chunk
//    of kc super-blocks (256 k each). For each super-block it reads the f32
//    activations of all vectors and builds the MFMA operands in LDS, shared
//    by the four waves: x * 2^e as an f16 pair x_hi + x_lo (2^e a power of
//    two that puts the vector's largest |x| in the super-block in
//    [2^13, 2^14)) and the 32-element sub-block sums as three f16 parts (for
//    the Q4_K min term).
//  * The sub-block scale is folded into the weight operand: each lane turns
//    its 8 weight codes c into f16 sc * q with one byte permutation and one
//    or two packed f16 operations per pair (c | 0x6400 is the f16 1024 + c),
//    exact for Q4_K (sc * q <= 945) and for Q6_K whenever |sc * q| <= 2048
//    (larger products round once, relative error <= 2^-12).
//    v_mfma_f32_16x16x32_f16 against x_hi and x_lo accumulates a whole
//    super-block in the matrix core; the row's d (for Q4_K also dmin times
//    the min-term MFMA) and the vector's 2^-e are applied once per
//    super-block in f32. The next super-block's activations and weights are
//    in flight while the current one is multiplied.
//  * Matrices too small to fill the chip split K into ksplit chunks. Each
//    chunk's products land as partial sums [ksplit][B][M]; whoever reads them
//    next (bprep_kernel, reduce_kernel or the attention prologue) adds the
//    chunks in order, so results do not depend on timing and no workgroup
//    waits for another.
//  * The gate/up pair form gives each workgroup 32 rows of both matrices and
//    writes gelu(gate) * up.
//  * bprep_kernel applies RMSNorm or residual-add + RMSNorm per vector to the
//    (summed) input of a matmul and can also write the operand blocks of the
//    matmul that follows, so that its workgroups copy them instead of each
//    building them again (the LM head's 4096 workgroups read the same
//    activations).
#include <utility>

#include "g4_internal.hpp"

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x3a __attribute__((ext_vector_type(3), aligned(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));  // native vector: stays in registers

constexpr int PNT = 256;   // prep threads
constexpr int MNT = 256;   // matmul threads (4 waves)
constexpr int PMAX = 12;   // partials added per pass of the prep loads (24 measured
                           // slower: passes over fewer chunks load clamped copies)

using g4d::Ops;
using g4d::OpsSub;
using g4d::pad_batch;

__device__ __forceinline__ uint32_t pack_h2(_Float16 a, _Float16 b) {
  h2 v = {a, b};
  return __builtin_bit_cast(uint32_t, v);
}

// ---------------------------------------------------------------------------
// per-vector prologue: out = x' where x = sum of the nparts partials and
//   PRO 0: x' = x;  PRO 1: x' = x * w1 / rms(x);
//   PRO 2: h = residual + x * w1 / rms(x) (written to h_out), x' = h * w2 / rms(h)
// (src/engine.ts:1545 rmsNorm, :1606-1607 fusedNormAdd + rmsNorm)
// ---------------------------------------------------------------------------
struct BPrepArgs {
  const float* x;  // [nparts][B][K]
  uint32_t nparts;
  uint32_t B;
  const uint16_t* w1;
  const float* residual;  // [B][K]
  const uint16_t* w2;
  float* h_out;  // [B][K]
  float* out;    // [B][K]
  float eps;
  uint8_t* ops;  // optional: operand blocks [K/256][Ops::bytes(ntv)]
  int ntv;
  const uint16_t* scale;  // mode 2: h = (residual + norm(x)) * f16 scale (NULL: 1)
};

__device__ __forceinline__ float4 mulw(float4 x, uint2 w, float s) {
  return make_float4(x.x * g4d::f16_bits_to_f32(w.x & 0xffffu) * s, x.y * g4d::f16_bits_to_f32(w.x >> 16) * s,
                     x.z * g4d::f16_bits_to_f32(w.y & 0xffffu) * s, x.w * g4d::f16_bits_to_f32(w.y >> 16) * s);
}
__device__ __forceinline__ float sq4(float4 v) { return (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w); }
__device__ __forceinline__ float4 add4(float4 a, float4 b) {
  return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}

// One workgroup per vector; thread t holds the float4s at 4t + 1024p. The
// partials are read PMAX at a time, all loads of a pass issued together.
template <int BPR, int PRO>
__global__ __launch_bounds__(PNT) void bprep_kernel(BPrepArgs a) {
  constexpr int K = BPR * 256;
  constexpr int XP = (K + 4 * PNT - 1) / (4 * PNT);
  __shared__ float red[2 * (PNT / 64)];
  const uint32_t v = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const size_t vstride = (size_t)a.B * K;
  float4 x[XP], r[PRO == 2 ? XP : 1];
  uint2 w1[PRO >= 1 ? XP : 1], w2[PRO == 2 ? XP : 1];
  // (w2 read unconditionally, from w1 when there is none: a load under a
  // branch is waited for where the branch joins, before the partials below
  // are even requested)
  const uint16_t* const w2p = a.w2 ? a.w2 : a.w1;
  // (likewise the output scale: requested with the rest, not after the first norm)
  const uint16_t scb = PRO == 2 ? (a.scale ? a.scale : a.w1)[0] : (uint16_t)0;
#pragma unroll
  for (int p = 0; p < XP; ++p) {
    const int f = 4 * tid + 4 * PNT * p, fc = f < K ? f : 0;
    x[p] = *(const float4*)(a.x + (size_t)v * K + fc);
    if constexpr (PRO >= 1) w1[p] = *(const uint2*)(a.w1 + fc);
    if constexpr (PRO == 2) {
      r[p] = *(const float4*)(a.residual + (size_t)v * K + fc);
      w2[p] = *(const uint2*)(w2p + fc);
    }
  }
  for (uint32_t c0 = 1; c0 < a.nparts; c0 += PMAX) {  // chunks 1.. in order
    float4 t[PMAX][XP];
#pragma unroll
    for (int i = 0; i < PMAX; ++i) {
      const uint32_t c = min(c0 + i, a.nparts - 1);
#pragma unroll
      for (int p = 0; p < XP; ++p) {
        const int f = 4 * tid + 4 * PNT * p, fc = f < K ? f : 0;
        t[i][p] = *(const float4*)(a.x + c * vstride + (size_t)v * K + fc);
      }
    }
#pragma unroll
    for (int i = 0; i < PMAX; ++i)
      if (c0 + i < a.nparts)
#pragma unroll
        for (int p = 0; p < XP; ++p) x[p] = add4(x[p], t[i][p]);
  }
  if constexpr (PRO >= 1) {
    float ss = 0.f;
#pragma unroll
    for (int p = 0; p < XP; ++p) ss += (4 * tid + 4 * PNT * p < K) ? sq4(x[p]) : 0.f;
    ss = g4d::wave_sum_dpp(ss);
    if (lane == 0) red[w] = ss;
    __syncthreads();
    float t1 = 0.f;
#pragma unroll
    for (int i = 0; i < PNT / 64; ++i) t1 += red[i];
    const float inv1 = __builtin_amdgcn_rsqf(t1 * (1.0f / (float)K) + a.eps);
    if constexpr (PRO == 1) {
#pragma unroll
      for (int p = 0; p < XP; ++p) x[p] = mulw(x[p], w1[p], inv1);
    } else {
      float ss2 = 0.f;
      const float sc = a.scale ? g4d::f16_bits_to_f32(scb) : 1.0f;
#pragma unroll
      for (int p = 0; p < XP; ++p) {
        const int f = 4 * tid + 4 * PNT * p;
        const float4 h = add4(r[p], mulw(x[p], w1[p], inv1));
        x[p] = make_float4(h.x * sc, h.y * sc, h.z * sc, h.w * sc);
        ss2 += f < K ? sq4(x[p]) : 0.f;
        if (a.h_out && f < K) *(float4*)(a.h_out + (size_t)v * K + f) = x[p];
      }
      ss2 = g4d::wave_sum_dpp(ss2);
      if (lane == 0) red[PNT / 64 + w] = ss2;
      __syncthreads();
      float t2 = 0.f;
#pragma unroll
      for (int i = 0; i < PNT / 64; ++i) t2 += red[PNT / 64 + i];
      const float inv2 = __builtin_amdgcn_rsqf(t2 * (1.0f / (float)K) + a.eps);
      if (a.w2)  // (no w2: out = h)
#pragma unroll
        for (int p = 0; p < XP; ++p) x[p] = mulw(x[p], w2[p], inv2);
    }
  }
#pragma unroll
  for (int p = 0; p < XP; ++p) {
    const int f = 4 * tid + 4 * PNT * p;
    if (f < K) *(float4*)(a.out + (size_t)v * K + f) = x[p];
  }
  if (!a.ops) return;
  // operand blocks: wave w of pass p holds super-block 4p + w, lanes 8j .. 8j+7 its sub-block j
  const uint32_t sblk = Ops::bytes(a.ntv);
  const uint32_t t = v / 16, c = v % 16;
  const int s = lane >> 3;        // sub-block within the super-block
  const int kk = (lane & 7) * 4;  // first element within the sub-block
  const int q = kk >> 3;          // 8-element group
#pragma unroll
  for (int p = 0; p < XP; ++p) {
    const uint32_t sb = 4u * p + w;  // uniform over the wave
    if (sb >= (uint32_t)BPR) break;
    const float4 xv = x[p];
    float am = fmaxf(fmaxf(fabsf(xv.x), fabsf(xv.y)), fmaxf(fabsf(xv.z), fabsf(xv.w)));
    am = g4d::wave_max_dpp(am);
    int ex = 0;
    (void)frexpf(am, &ex);
    const int k = am > 0.f ? min(max(14 - ex, -120), 120) : 0;
    const float sc = ldexpf(1.0f, k);
    const float xs[4] = {xv.x * sc, xv.y * sc, xv.z * sc, xv.w * sc};
    _Float16 hi[4], lo[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      hi[e] = (_Float16)xs[e];
      lo[e] = (_Float16)(xs[e] - (float)hi[e]);
    }
    float sum = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) sum += xs[e];
    sum = g4d::sum8(sum) * 0.015625f;  // * 2^-6
    uint8_t* base = a.ops + (size_t)sb * sblk;
    uint8_t* mp = base + t * Ops::MAIN_T + s * 2048 + (c + 16u * q) * 16 + (kk & 7) * 2;
    *(uint2*)mp = make_uint2(pack_h2(hi[0], hi[1]), pack_h2(hi[2], hi[3]));
    *(uint2*)(mp + 1024) = make_uint2(pack_h2(lo[0], lo[1]), pack_h2(lo[2], lo[3]));
    if ((lane & 7) == 0) {
      const _Float16 p0 = (_Float16)sum;
      const float r1 = sum - (float)p0;
      const _Float16 p1 = (_Float16)r1;
      const _Float16 p2 = (_Float16)(r1 - (float)p1);
      *(uint2*)(base + Ops::sums_off(a.ntv) + t * 1024 + (c + 16u * (uint32_t)(s >> 1)) * 16 + (s & 1) * 8) =
          make_uint2(pack_h2(p0, p1), pack_h2(p2, (_Float16)0.f));
    }
    if (lane == 0) *(float*)(base + Ops::scale_off(a.ntv) + t * 64 + c * 4) = ldexpf(1.0f, -k);
  }
}

// Y[v][m] = epilogue(sum_c part[c][v][m]) for a split-K matmul (in chunk order).
__global__ __launch_bounds__(PNT) void reduce_kernel(const float* part, float* Y, uint32_t n, uint32_t nparts,
                                                     float cap) {
  const uint32_t i = blockIdx.x * PNT + threadIdx.x;
  if (i >= n) return;
  float y = part[i];
  for (uint32_t c = 1; c < nparts; ++c) y += part[(size_t)c * n + i];
  if (cap > 0.f) y = tanhf(fminf(fmaxf(y / cap, -15.0f), 15.0f)) * cap;
  Y[i] = y;
}

// ---------------------------------------------------------------------------
// matmul
// ---------------------------------------------------------------------------

template <int QT>
struct Blk;
template <> struct Blk<0> { static constexpr int BYTES = 144; };
template <> struct Blk<1> { static constexpr int BYTES = 210; };

struct MmSeg {
  const uint8_t* W;
  float* Y;  // ksplit == 1: [B][M]; else the partials [ksplit][B][M]
  uint32_t M;
  uint32_t g_begin;  // first row group of the segment
};
struct MmArgs {
  MmSeg s[4];
  int n;
  uint32_t B;
  float cap;       // softcap when > 0 (ksplit == 1)
  const float* x;        // [B][K] activations
  const uint8_t* ops;    // OPK 1: their operand blocks [K/256][Ops::bytes(NTV)]; OPK 2: [K/256][OpsSub::bytes(NTV)]
  uint32_t K;
  uint32_t ksplit, kc;  // K in ksplit chunks of kc super-blocks
  uint8_t* ops_out;     // MODE 1: the product's sub-block-scaled operand blocks (or null)
};

// Weight registers of one 16-row tile and super-block. A side (row lane%16,
// k-group q = lane/16): codes and sub-block scales; D side (rows 4q + i): d
// (Q4_K: d | dmin << 16).
template <int QT>
struct WRegs;
template <> struct WRegs<0> {
  uint2 qs[4];
  uint4 hdr;
  uint32_t dd[4];
};
template <> struct WRegs<1> {
  uint2 ql[4], qh[2];
  uint4 sc;
  uint32_t dd[4];
};

// What load_w leaves in registers: the weights as loaded. Q4_K blocks are
// 16-byte aligned and load straight into WRegs; a Q6_K block (210 bytes) may
// sit 2 bytes off a dword, so its pieces are loaded as the aligned dwords
// around them and shifted into place by w_decode where they are used (a
// shift at the load would wait for the load there, also for the weights of
// a block that is only prefetched).
template <int QT>
struct WLoad;
template <> struct WLoad<0> {
  WRegs<0> r;
};
template <> struct WLoad<1> {
  u32x3a ql[4], qh[2];
  uint32_t s0, s1, s2, s3, s4;  // the dwords around the 16 scale bytes
  uint32_t dd[4];
  uint32_t sh;                  // the block's byte offset within its dword (0 or 2)
};

template <int BPR>
__device__ __forceinline__ void load_w(WLoad<0>& ld, const uint8_t* W, uint32_t M, uint32_t rbase, uint32_t kb,
                                       int l) {
  WRegs<0>& r = ld.r;
  constexpr int BY = 144;
  const int q = l >> 4;
  const uint32_t ra = min(rbase + (uint32_t)(l & 15), M - 1);
  const uint8_t* blk = W + ((size_t)ra * BPR + kb) * BY;
  r.hdr = *(const uint4*)blk;
#pragma unroll
  for (int g = 0; g < 4; ++g) r.qs[g] = *(const uint2*)(blk + 16 + 32 * g + 8 * q);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t rd = min(rbase + 4u * q + i, M - 1);
    r.dd[i] = *(const uint32_t*)(W + ((size_t)rd * BPR + kb) * BY);
  }
}

template <int BPR>
__device__ __forceinline__ void load_w(WLoad<1>& r, const uint8_t* W, uint32_t M, uint32_t rbase, uint32_t kb,
                                       int l) {
  constexpr int BY = 210;
  const int q = l >> 4;
  const uint32_t ra = min(rbase + (uint32_t)(l & 15), M - 1);
  const uint8_t* blk = W + ((size_t)ra * BPR + kb) * BY;
  // every piece sits at a multiple of 8 bytes into the block: one shift for all
  r.sh = (uint32_t)((uintptr_t)blk & 3);
  const uint8_t* b4 = blk - r.sh;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    r.ql[2 * h] = *(const u32x3a*)(b4 + 64 * h + 8 * q);
    r.ql[2 * h + 1] = *(const u32x3a*)(b4 + 64 * h + 32 + 8 * q);
    r.qh[h] = *(const u32x3a*)(b4 + 128 + 32 * h + 8 * q);
  }
  // sc[16] at bytes 192..207: four dwords from the one holding byte 192 and
  // a fifth (bytes 206..209) that only a block at 2 mod 4 needs
  const uint32_t* p4 = (const uint32_t*)(b4 + 192);
  r.s0 = p4[0];
  r.s1 = p4[1];
  r.s2 = p4[2];
  r.s3 = p4[3];
  r.s4 = *(const uint32_t*)((const uint8_t*)p4 + 12 + 2 * r.sh);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t rd = min(rbase + 4u * q + i, M - 1);
    r.dd[i] = *(const uint16_t*)(W + ((size_t)rd * BPR + kb) * BY + 208);
  }
}

__device__ __forceinline__ const WRegs<0>& w_decode(const WLoad<0>& ld) { return ld.r; }
__device__ __forceinline__ WRegs<1> w_decode(const WLoad<1>& ld) {
  WRegs<1> r;
  const uint32_t sh = ld.sh;
  auto piece = [&](const u32x3a& w) {
    return make_uint2(__builtin_amdgcn_alignbyte(w.y, w.x, sh), __builtin_amdgcn_alignbyte(w.z, w.y, sh));
  };
#pragma unroll
  for (int i = 0; i < 4; ++i) r.ql[i] = piece(ld.ql[i]);
#pragma unroll
  for (int h = 0; h < 2; ++h) r.qh[h] = piece(ld.qh[h]);
  r.sc = make_uint4(__builtin_amdgcn_alignbyte(ld.s1, ld.s0, sh), __builtin_amdgcn_alignbyte(ld.s2, ld.s1, sh),
                    __builtin_amdgcn_alignbyte(ld.s3, ld.s2, sh), __builtin_amdgcn_alignbyte(ld.s4, ld.s3, sh));
#pragma unroll
  for (int i = 0; i < 4; ++i) r.dd[i] = ld.dd[i];
  return r;
}

// f16 pairs (1024 + b_i, 1024 + b_j) from two bytes of `codes`: v_perm_b32
// takes selector bytes 0-3 from its second operand and 4-7 from its first.
__device__ __forceinline__ h2 biased_pair(uint32_t codes, uint32_t sel) {
  return __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, codes, sel));
}
constexpr uint32_t kSel01 = 0x04010400u, kSel23 = 0x04030402u;

__device__ __forceinline__ h8 cat(h2 a, h2 b, h2 c, h2 d) { return h8{a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y}; }

// Q4_K 6-bit scale and min of sub-block j (src/gguf.ts:175-182).
__device__ __forceinline__ void q4k_sc_mn(const uint4& hdr, int j, uint32_t& sc, uint32_t& mn) {
  const int sh = 8 * (j & 3);
  if (j < 4) {
    sc = (hdr.y >> sh) & 63u;
    mn = (hdr.z >> sh) & 63u;
  } else {
    sc = ((hdr.w >> sh) & 15u) | (((hdr.y >> sh) >> 6 & 3u) << 4);
    mn = ((hdr.w >> sh) >> 4 & 15u) | (((hdr.z >> sh) >> 6 & 3u) << 4);
  }
}

// Weight operand of sub-block s: 8 f16 values sc * q of row lane%16, k = 8q .. 8q+7.
__device__ __forceinline__ h8 a_operand(const WRegs<0>& r, int s, int) {
  const uint2 raw = r.qs[s >> 1];
  const uint32_t c0 = (s & 1) ? (raw.x >> 4) & 0x0f0f0f0fu : raw.x & 0x0f0f0f0fu;
  const uint32_t c1 = (s & 1) ? (raw.y >> 4) & 0x0f0f0f0fu : raw.y & 0x0f0f0f0fu;
  uint32_t sc, mn;
  q4k_sc_mn(r.hdr, s, sc, mn);
  const _Float16 f = (_Float16)(float)sc;
  const _Float16 fb = (_Float16)(-1024.0f * (float)sc);  // exact: sc <= 63
  const h2 mul = {f, f}, bias = {fb, fb};
  // (1024 + c) * sc - 1024 * sc = c * sc, one rounding of an exact value
  return cat(__builtin_elementwise_fma(biased_pair(c0, kSel01), mul, bias),
             __builtin_elementwise_fma(biased_pair(c0, kSel23), mul, bias),
             __builtin_elementwise_fma(biased_pair(c1, kSel01), mul, bias),
             __builtin_elementwise_fma(biased_pair(c1, kSel23), mul, bias));
}

// Q6_K sub-block s: half h = s/4, run pair k' = s%4 (src/gguf.ts:344-361);
// this lane's 8 codes lie in run q/2 of the sub-block.
__device__ __forceinline__ h8 a_operand(const WRegs<1>& r, int s, int q) {
  const int h = s >> 2, kp = s & 3;
  const uint2 ql = r.ql[2 * h + (kp & 1)];
  const uint2 qh = r.qh[h];
  const uint32_t lo0 = kp < 2 ? (ql.x & 0x0f0f0f0fu) : ((ql.x >> 4) & 0x0f0f0f0fu);
  const uint32_t lo1 = kp < 2 ? (ql.y & 0x0f0f0f0fu) : ((ql.y >> 4) & 0x0f0f0f0fu);
  const uint32_t c0 = lo0 | (((qh.x >> (2 * kp)) & 0x03030303u) << 4);
  const uint32_t c1 = lo1 | (((qh.y >> (2 * kp)) & 0x03030303u) << 4);
  const int is = 8 * h + 2 * kp + (q >> 1);
  const uint32_t wd = (is < 4) ? r.sc.x : (is < 8) ? r.sc.y : (is < 12) ? r.sc.z : r.sc.w;
  const int scv = (int)(int8_t)((wd >> (8 * (is & 3))) & 0xffu);
  const _Float16 f = (_Float16)(float)scv;
  const h2 mul = {f, f};
  const h2 off = {(_Float16)-1056.0f, (_Float16)-1056.0f};
  // (1024 + c) - 1056 = c - 32 exactly, then one rounding of (c - 32) * sc
  return cat((biased_pair(c0, kSel01) + off) * mul, (biased_pair(c0, kSel23) + off) * mul,
             (biased_pair(c1, kSel01) + off) * mul, (biased_pair(c1, kSel23) + off) * mul);
}

// Min operand of a Q4_K super-block: slots 8q .. 8q+3 hold the min of
// sub-block 2q, slots 8q+4 .. +7 that of sub-block 2q+1.
__device__ __forceinline__ h8 min_operand(const WRegs<0>& r, int q) {
  uint32_t sc0, m0, sc1, m1;
  q4k_sc_mn(r.hdr, 2 * q, sc0, m0);
  q4k_sc_mn(r.hdr, 2 * q + 1, sc1, m1);
  const _Float16 a = (_Float16)(float)m0, b = (_Float16)(float)m1;
  return h8{a, a, a, a, b, b, b, b};
}

// Activations of one super-block: item (v, s) = vector v, sub-block s,
// item = tid + MNT * u, v = item / 8, s = item % 8; 8 float4 per item.
template <int NTV>
struct Raw {
  static constexpr int IPT = NTV >= 2 ? NTV / 2 : 1;  // items per thread (Bp * 8 / MNT, at least 1)
  float4 x[IPT][8];
};

template <int NTV>
__device__ __forceinline__ void raw_load(Raw<NTV>& r, const float* x, uint32_t B, uint32_t K, uint32_t kb, int tid) {
#pragma unroll
  for (int u = 0; u < Raw<NTV>::IPT; ++u) {
    const uint32_t it = (uint32_t)(tid + MNT * u), v = it >> 3, s = it & 7;
    const uint32_t vc = v < B ? v : 0;  // padded vectors: read vector 0, zeroed at the store
    const float4* src = (const float4*)(x + (size_t)vc * K + kb * 256 + 32 * s);
#pragma unroll
    for (int j = 0; j < 8; ++j) r.x[u][j] = src[j];
  }
}

// Operand block of the super-block into LDS (see Ops).
template <int NTV>
__device__ __forceinline__ void raw_store(const Raw<NTV>& r, uint8_t* lds, uint32_t B, int tid) {
#pragma unroll
  for (int u = 0; u < Raw<NTV>::IPT; ++u) {
    const uint32_t it = (uint32_t)(tid + MNT * u), v = it >> 3, s = it & 7;
    const bool live = v < B;
    float xs[32];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      xs[4 * j] = live ? r.x[u][j].x : 0.f;
      xs[4 * j + 1] = live ? r.x[u][j].y : 0.f;
      xs[4 * j + 2] = live ? r.x[u][j].z : 0.f;
      xs[4 * j + 3] = live ? r.x[u][j].w : 0.f;
    }
    float am = 0.f;
#pragma unroll
    for (int e = 0; e < 32; ++e) am = fmaxf(am, fabsf(xs[e]));
    am = g4d::max8(am);  // the 8 sub-blocks of vector v sit in 8 consecutive lanes
    int ex = 0;
    (void)frexpf(am, &ex);
    const int k = am > 0.f ? min(max(14 - ex, -120), 120) : 0;
    const float sc = ldexpf(1.0f, k);
    float sum = 0.f;
#pragma unroll
    for (int e = 0; e < 32; ++e) {
      xs[e] *= sc;
      sum += xs[e];
    }
    if (v >= 16u * NTV) continue;  // items past the padded batch (NTV == 1 only)
    const uint32_t t = v >> 4, c = v & 15;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint32_t hw[4], lw[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float a0 = xs[8 * q + 2 * e], a1 = xs[8 * q + 2 * e + 1];
        const _Float16 h0 = (_Float16)a0, h1 = (_Float16)a1;
        hw[e] = pack_h2(h0, h1);
        lw[e] = pack_h2((_Float16)(a0 - (float)h0), (_Float16)(a1 - (float)h1));
      }
      uint8_t* slot = lds + t * Ops::MAIN_T + s * 2048 + (c + 16u * q) * 16;
      *(u32x4*)slot = u32x4{hw[0], hw[1], hw[2], hw[3]};
      *(u32x4*)(slot + 1024) = u32x4{lw[0], lw[1], lw[2], lw[3]};
    }
    sum *= 0.015625f;  // * 2^-6
    const _Float16 p0 = (_Float16)sum;
    const float r1 = sum - (float)p0;
    const _Float16 p1 = (_Float16)r1;
    const _Float16 p2 = (_Float16)(r1 - (float)p1);
    *(u32x2*)(lds + Ops::sums_off(NTV) + t * 1024 + (c + 16u * (s >> 1)) * 16 + (s & 1) * 8) =
        u32x2{pack_h2(p0, p1), pack_h2(p2, (_Float16)0.f)};
    if (s == 0) *(float*)(lds + Ops::scale_off(NTV) + t * 64 + c * 4) = ldexpf(1.0f, -k);
  }
}

// Prebuilt operand block copy, global -> registers -> LDS: N 16-byte pieces,
// piece tid + MNT*i per thread; pieces past N go to the sink slot at N.
template <int NCP, uint32_t N>
__device__ __forceinline__ void cp_load(u32x4 (&cp)[NCP], const u32x4* src, int tid) {
#pragma unroll
  for (int i = 0; i < NCP; ++i) {
    const uint32_t e = (uint32_t)(tid + MNT * i);
    cp[i] = src[e < N ? e : 0];
  }
}
template <int NCP, uint32_t N>
__device__ __forceinline__ void cp_store(const u32x4 (&cp)[NCP], u32x4* lds, int tid) {
#pragma unroll
  for (int i = 0; i < NCP; ++i) {
    const uint32_t e = (uint32_t)(tid + MNT * i);
    lds[e < N ? e : N] = cp[i];
  }
}

// The operand source of one launch: built from f32 activations (OPK 0),
// copied from blocks a prep launch built (OPK 1) or from the sub-block-scaled
// blocks a gate/up launch wrote (OPK 2).
template <int NTV, int OPK>
struct OpSrc;
template <int NTV>
struct OpSrc<NTV, 0> {
  Raw<NTV> r;
  __device__ __forceinline__ void load(const MmArgs& a, uint32_t kb, int tid) { raw_load<NTV>(r, a.x, a.B, a.K, kb, tid); }
  __device__ __forceinline__ void store(uint8_t* lds, const MmArgs& a, int tid) { raw_store<NTV>(r, lds, a.B, tid); }
};
template <int NTV, int OPK>
struct OpSrc {
  static_assert(OPK == 1 || OPK == 2, "copied operand blocks");
  static constexpr uint32_t NPC = (OPK == 1 ? Ops::bytes(NTV) : OpsSub::bytes(NTV)) / 16;
  static constexpr int NCP = (int)((NPC + MNT - 1) / MNT);
  u32x4 cp[NCP];
  __device__ __forceinline__ void load(const MmArgs& a, uint32_t kb, int tid) {
    cp_load<NCP, NPC>(cp, (const u32x4*)a.ops + (size_t)kb * NPC, tid);
  }
  __device__ __forceinline__ void store(uint8_t* lds, const MmArgs&, int tid) {
    cp_store<NCP, NPC>(cp, (u32x4*)lds, tid);
  }
};

using g4d::gelu_tanh;  // shaders/gelu_mul.wgsl:10-16

__device__ __forceinline__ float epilogue(float y, float cap) {
  if (cap > 0.f) {
    const float t = fminf(fmaxf(y / cap, -15.0f), 15.0f);
    return tanhf(t) * cap;
  }
  return y;
}

// Products of one super-block: the weights of this lane's 16-row tile in wr,
// the block's operands in LDS at lds; acc[t] gains the tile's sums for
// vectors 16t .. 16t + 15.
template <int QT, int NTV, int OPK>
__device__ __forceinline__ void mm_block(const WRegs<QT>& wr, const uint8_t* lds, f4 (&acc)[NTV], int l, int q) {
  const u32x4* lv = (const u32x4*)lds;
  f4 C[NTV], Cl[NTV], Cm[NTV];
  if constexpr (OPK == 2) {
    // each sub-block's products scaled by its own 2^-e, then d
    const float* scs = (const float*)(lds + OpsSub::scale_off(NTV));
#pragma unroll
    for (int t = 0; t < NTV; ++t) C[t] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const h8 A = a_operand(wr, s, q);
#pragma unroll
      for (int t = 0; t < NTV; ++t) {
        const u32x4 bh = lv[(t * Ops::MAIN_T + s * 2048) / 16 + l];
        const u32x4 bl = lv[(t * Ops::MAIN_T + s * 2048 + 1024) / 16 + l];
        f4 z = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, __builtin_bit_cast(h8, bh), f4{0.f, 0.f, 0.f, 0.f}, 0, 0,
                                                      0);
        z = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, __builtin_bit_cast(h8, bl), z, 0, 0, 0);
        const float fs = scs[t * 128 + s * 16 + (l & 15)];
#pragma unroll
        for (int i = 0; i < 4; ++i) C[t][i] += fs * z[i];
      }
    }
#pragma unroll
    for (int t = 0; t < NTV; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[t][i] += g4d::f16_bits_to_f32(wr.dd[i]) * C[t][i];
    return;
  }
  // the x_hi and x_lo products accumulate apart: two independent MFMA
  // chains per tile instead of one (a dependent MFMA waits for its
  // predecessor's result; waves of the batched LM head spent 55 % of their
  // cycles waiting to issue with one chain)
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    const h8 A = a_operand(wr, s, q);
#pragma unroll
    for (int t = 0; t < NTV; ++t) {
      const u32x4 bh = lv[(t * Ops::MAIN_T + s * 2048) / 16 + l];
      const u32x4 bl = lv[(t * Ops::MAIN_T + s * 2048 + 1024) / 16 + l];
      const f4 zh = s == 0 ? f4{0.f, 0.f, 0.f, 0.f} : C[t];
      const f4 zl = s == 0 ? f4{0.f, 0.f, 0.f, 0.f} : Cl[t];
      C[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, __builtin_bit_cast(h8, bh), zh, 0, 0, 0);
      Cl[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, __builtin_bit_cast(h8, bl), zl, 0, 0, 0);
    }
  }
#pragma unroll
  for (int t = 0; t < NTV; ++t) C[t] += Cl[t];
  if constexpr (QT == 0) {
    const h8 Am = min_operand(wr, q);
#pragma unroll
    for (int t = 0; t < NTV; ++t) {
      const u32x4 bm = lv[(Ops::sums_off(NTV) + t * 1024) / 16 + l];
      Cm[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(Am, __builtin_bit_cast(h8, bm), f4{0.f, 0.f, 0.f, 0.f}, 0, 0,
                                                      0);
    }
  }
  const float* scl = (const float*)(lds + Ops::scale_off(NTV));
#pragma unroll
  for (int t = 0; t < NTV; ++t) {
    const float fs = scl[t * 16 + (l & 15)];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (QT == 0) {
        const float d = g4d::f16_bits_to_f32(wr.dd[i] & 0xffffu);
        const float dm = g4d::f16_bits_to_f32(wr.dd[i] >> 16) * 64.0f;
        acc[t][i] += fs * (d * C[t][i] - dm * Cm[t][i]);
      } else {
        acc[t][i] += fs * g4d::f16_bits_to_f32(wr.dd[i]) * C[t][i];
      }
    }
  }
}

// Row coordinates of a workgroup: segment, first row of this wave's tile.
struct MmRows {
  int si;
  uint32_t rbase, M;
  const uint8_t* W;
};
template <int MODE>
__device__ __forceinline__ MmRows mm_rows(const MmArgs& a, uint32_t g, int w) {
  MmRows r;
  r.si = 0;
  if constexpr (MODE == 0) {
#pragma unroll
    for (int i = 1; i < 4; ++i)
      if (i < a.n && g >= a.s[i].g_begin) r.si = i;
    r.W = a.s[r.si].W;
    r.M = a.s[r.si].M;
    r.rbase = (g - a.s[r.si].g_begin) * 64 + 16u * w;
  } else {
    r.W = (w >> 1) ? a.s[1].W : a.s[0].W;  // (no dynamic index into the kernel arguments)
    r.M = a.s[0].M;
    r.rbase = g * 32 + 16u * (w & 1);
  }
  return r;
}

// Outputs of a workgroup once every wave's sums are in acc: the sums of
// groups 1 .. KG - 1 go through LDS at x1 into group 0's, then MODE 0 stores rows (or
// partial sums) with the softcap, MODE 1 the gate/up product and its
// operand blocks. lds_all is free scratch for every wave (callers order it
// after their last operand reads with a barrier).
template <int NTV, int MODE, int KG>
__device__ __forceinline__ void mm_epilogue(const MmArgs& a, f4 (&acc)[NTV], uint8_t* lds_all, uint8_t* x1, int kg,
                                            int w, int l, int q, uint32_t g, uint32_t chunk, int si, uint32_t rbase,
                                            uint32_t M) {
  if constexpr (KG > 1) {  // the other groups' sums into group 0's, in group order
    f4* xk = (f4*)x1;
    if (kg > 0) {
#pragma unroll
      for (int t = 0; t < NTV; ++t) xk[(((kg - 1) * 4 + w) * NTV + t) * 64 + l] = acc[t];
    }
    __syncthreads();
    if (kg == 0) {
#pragma unroll
      for (int o = 0; o < KG - 1; ++o)
#pragma unroll
        for (int t = 0; t < NTV; ++t) {
          const f4 v = xk[((o * 4 + w) * NTV + t) * 64 + l];
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[t][i] += v[i];
        }
    }
  }
  const bool out_group = kg == 0;

  // ---- outputs: lane (q, c) holds rows rbase + 4q + i of vectors 16t + c ----
  if constexpr (MODE == 1) {
    // the up waves hand their sums to the gate waves through LDS
    f4* xfer = (f4*)lds_all;
    if (out_group && w >= 2) {
#pragma unroll
      for (int t = 0; t < NTV; ++t) xfer[((w - 2) * NTV + t) * 64 + l] = acc[t];
    }
    __syncthreads();
    f4 y[NTV];  // the product (0 for padded vectors and rows past M)
    if (out_group && w < 2) {
#pragma unroll
      for (int t = 0; t < NTV; ++t) {
        const f4 up = xfer[(w * NTV + t) * 64 + l];
        const uint32_t v = 16u * t + (l & 15);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t row = rbase + 4u * q + i;
          const bool live = row < M && v < a.B;
          y[t][i] = live ? gelu_tanh(acc[t][i]) * up[i] : 0.f;
          if (live && a.s[0].Y) a.s[0].Y[(size_t)v * M + row] = y[t][i];
        }
      }
    }
    if (!a.ops_out) return;  // (uniform)
    // The workgroup's 32 rows are sub-block g % 8 of super-block g / 8 of
    // the product: per vector, the largest |y| over them (lanes of one column
    // in each gate wave, then the two waves) sets its 2^e.
    float* mx = (float*)(lds_all + NTV * 2048);  // [2 waves][NTV][16]
    if (out_group && w < 2) {
#pragma unroll
      for (int t = 0; t < NTV; ++t) {
        float m = fmaxf(fmaxf(fabsf(y[t][0]), fabsf(y[t][1])), fmaxf(fabsf(y[t][2]), fabsf(y[t][3])));
        m = fmaxf(m, __shfl_xor(m, 16, 64));
        m = fmaxf(m, __shfl_xor(m, 32, 64));
        if (q == 0) mx[(w * NTV + t) * 16 + l] = m;
      }
    }
    __syncthreads();
    if (out_group && w < 2) {
      const uint32_t sb = g & 7u, c = (uint32_t)(l & 15);
      uint8_t* base = a.ops_out + (size_t)(g >> 3) * OpsSub::bytes(NTV);
      const uint32_t qq = 2u * (uint32_t)w + (uint32_t)(q >> 1);  // 8-element group of rows 16w + 4q ..
#pragma unroll
      for (int t = 0; t < NTV; ++t) {
        const float am = fmaxf(mx[t * 16 + c], mx[(NTV + t) * 16 + c]);
        int ex = 0;
        (void)frexpf(am, &ex);
        const int k = am > 0.f ? min(max(14 - ex, -120), 120) : 0;
        const float sc = ldexpf(1.0f, k);
        _Float16 hi[4], lo[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float xs = y[t][i] * sc;
          hi[i] = (_Float16)xs;
          lo[i] = (_Float16)(xs - (float)hi[i]);
        }
        uint8_t* slot = base + t * Ops::MAIN_T + sb * 2048 + (c + 16u * qq) * 16 + (q & 1) * 8;
        *(uint2*)slot = make_uint2(pack_h2(hi[0], hi[1]), pack_h2(hi[2], hi[3]));
        *(uint2*)(slot + 1024) = make_uint2(pack_h2(lo[0], lo[1]), pack_h2(lo[2], lo[3]));
        if (w == 0 && q == 0) *(float*)(base + OpsSub::scale_off(NTV) + t * 512 + sb * 64 + c * 4) = ldexpf(1.0f, -k);
      }
    }
    return;
  }
  if (!out_group) return;
  float* Y = a.s[si].Y + (size_t)chunk * a.B * M;
  const float cap = a.ksplit == 1 ? a.cap : 0.f;
#pragma unroll
  for (int t = 0; t < NTV; ++t) {
    const uint32_t v = 16u * t + (l & 15);
    const uint32_t row = rbase + 4u * q;
    if (v >= a.B) continue;
    float* dst = Y + (size_t)v * M + row;
    if ((M & 3) == 0 && row + 3 < M) {
      *(f4*)dst = f4{epilogue(acc[t][0], cap), epilogue(acc[t][1], cap), epilogue(acc[t][2], cap),
                     epilogue(acc[t][3], cap)};
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (row + i < M) dst[i] = epilogue(acc[t][i], cap);
    }
  }
}

template <typename F, int... J>
__device__ __forceinline__ void static_for_seq(F&& f, std::integer_sequence<int, J...>) {
  (f(std::integral_constant<int, J>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_seq(f, std::make_integer_sequence<int, N>{});
}

// MODE 0: a row group is 64 rows of one segment. MODE 1 (gate/up): segments
// 0 and 1 have the same rows; a row group is 32 rows of both, waves 0-1 gate,
// waves 2-3 up, and the output (segment 0's Y) is gelu(gate) * up; with
// ops_out the workgroup also writes its 32 rows of the product as one
// sub-block of the sub-block-scaled operand blocks a Q6_K down projection
// reads (OPK 2).
//
// KG > 1: the workgroup is KG groups of four waves; group g takes blocks
// g, g + KG, ... of the K chunk (kc a multiple of KG), each group through its
// own LDS operand buffer, and the groups add their sums through LDS before
// the epilogue, which group 0 runs (the others pass the same barriers).
//
// NKB > 0: each group walks exactly NKB blocks (kc = KG NKB, host-checked),
// unrolled: the weights of blocks j + 1 and j + 2 are in flight, each in
// registers of its own, while block j is multiplied (a loop that carries
// the next block's weights into the current block's registers waits for
// them at the end of every iteration). NKB = 0: a loop over kc / KG blocks
// with one block in flight.
template <int QT, int BPR, int NTV, int MODE, int OPK, int KG = 1, int NKB = 0>
__global__ __launch_bounds__(MNT * KG)
// (the looping walk over copied operands, one group, as the batched LM head
// takes it: three waves per SIMD with 32-vector tiles, two with 64, rather
// than the two and one its free allocation gives)
__attribute__((amdgpu_waves_per_eu(OPK == 1 && KG == 1 && NKB == 0 ? (NTV <= 2 ? 3 : 2) : 1))) void mmf_kernel(
    MmArgs a) {
  static_assert(OPK != 2 || (QT == 1 && MODE == 0), "sub-block-scaled operands: Q6_K matmuls");
  static_assert(KG >= 1 && KG <= 3, "one to three K groups");
  constexpr uint32_t LB = Ops::bytes(NTV) + 16;  // + the copy's sink slot
  static_assert(KG == 1 || LB >= (uint32_t)(KG - 1) * 4u * NTV * 1024u, "other groups' sums fit in group 1's buffer");
  __shared__ __align__(16) uint8_t lds_all[KG * LB];

  const int kg = KG == 1 ? 0 : (int)(threadIdx.x / MNT);
  uint8_t* const lds = lds_all + kg * LB;
  const int tid = (int)(threadIdx.x % MNT), w = tid >> 6, l = tid & 63, q = l >> 4;
  const uint32_t g = blockIdx.x / a.ksplit, chunk = blockIdx.x % a.ksplit;
  const MmRows rw = mm_rows<MODE>(a, g, w);
  const uint32_t kb0 = chunk * a.kc + (uint32_t)kg;  // this group's blocks: kb0 + KG j

  f4 acc[NTV];
#pragma unroll
  for (int t = 0; t < NTV; ++t) acc[t] = f4{0.f, 0.f, 0.f, 0.f};
  OpSrc<NTV, OPK> src;
  if constexpr (NKB > 0) {
    WLoad<QT> wr[NKB];
    src.load(a, kb0, tid);
    load_w<BPR>(wr[0], rw.W, rw.M, rw.rbase, kb0, l);
    if constexpr (NKB > 1) load_w<BPR>(wr[1], rw.W, rw.M, rw.rbase, kb0 + KG, l);
    src.store(lds, a, tid);
    __syncthreads();
    static_for<NKB>([&](auto jc) {
      constexpr int j = decltype(jc)::value;
      if constexpr (j + 1 < NKB) src.load(a, kb0 + KG * (j + 1), tid);  // the next block's operands
      if constexpr (j + 2 < NKB) load_w<BPR>(wr[j + 2], rw.W, rw.M, rw.rbase, kb0 + KG * (j + 2), l);
      mm_block<QT, NTV, OPK>(w_decode(wr[j]), lds, acc, l, q);
      __syncthreads();  // every wave is done with this block's operands
      if constexpr (j + 1 < NKB) {
        src.store(lds, a, tid);
        __syncthreads();
      }
    });
  } else {
    // two register sets in turn (unrolled by two, so that no copy of the next
    // block's weights waits for them at the end of an iteration)
    const uint32_t nkb = a.kc / KG;
    WLoad<QT> wa, wb;
    src.load(a, kb0, tid);
    load_w<BPR>(wa, rw.W, rw.M, rw.rbase, kb0, l);
    src.store(lds, a, tid);
    __syncthreads();
    auto step = [&](const WLoad<QT>& cur, WLoad<QT>& nxt, uint32_t j) {
      const bool more = j + 1 < nkb;  // (uniform)
      if (more) {  // the next block is in flight during this one
        src.load(a, kb0 + KG * (j + 1), tid);
        load_w<BPR>(nxt, rw.W, rw.M, rw.rbase, kb0 + KG * (j + 1), l);
      }
      mm_block<QT, NTV, OPK>(w_decode(cur), lds, acc, l, q);
      __syncthreads();  // every wave is done with this block's operands
      if (more) {
        src.store(lds, a, tid);
        __syncthreads();
      }
    };
    if constexpr (NTV <= 2) {
      for (uint32_t j = 0; j < nkb; j += 2) {
        step(wa, wb, j);
        if (j + 1 < nkb) step(wb, wa, j + 1);
      }
    } else {
      // 64-vector tiles: one decoded set, the next block's weights decoded
      // into it after this block's products (a second undecoded set costs a
      // wave per SIMD of occupancy here)
      WRegs<QT> wr = w_decode(wa);
      for (uint32_t j = 0; j < nkb; ++j) {
        const bool more = j + 1 < nkb;  // (uniform)
        if (more) {
          src.load(a, kb0 + KG * (j + 1), tid);
          load_w<BPR>(wb, rw.W, rw.M, rw.rbase, kb0 + KG * (j + 1), l);
        }
        mm_block<QT, NTV, OPK>(wr, lds, acc, l, q);
        __syncthreads();  // every wave is done with this block's operands
        if (more) {
          src.store(lds, a, tid);
          __syncthreads();
          wr = w_decode(wb);
        }
      }
    }
  }
  mm_epilogue<NTV, MODE, KG>(a, acc, lds_all, lds_all + LB, kg, w, l, q, g, chunk, rw.si, rw.rbase, rw.M);
}

// ---------------------------------------------------------------------------
// Unpack check of the matrix-core operands (path 2 of the test export
// g4_dequantPath): one wave per 16 blocks, each block a one-block row, lanes
// as in mmf_kernel (row l % 16, k-group q = l / 16) with the weights read by
// load_w. Element 32s + 8q + i of a block gets Q4_K: d * A[i] - dmin * m_s,
// Q6_K: d * A[i], where A = a_operand(s) (f16 sc * q) and m_s the min
// operand of sub-block s; d * A and dmin * m are exact in f32, so for Q4_K
// the value is the reference's (src/gguf.ts:184-209) and for Q6_K it is d
// times the f16 rounding of sc * (q - 32).
// ---------------------------------------------------------------------------
template <int QT>
__global__ __launch_bounds__(64) void operand_check_kernel(const uint8_t* W, uint32_t nblocks, float* out) {
  const int l = threadIdx.x, q = l >> 4;
  const uint32_t rbase = blockIdx.x * 16u;
  WLoad<QT> wl;
  load_w<1>(wl, W, nblocks, rbase, 0, l);
  const auto& wr = w_decode(wl);
  const uint32_t row = rbase + (uint32_t)(l & 15);
  if (row >= nblocks) return;
  float* o = out + (size_t)row * 256;
  float d, dmin = 0.f;
  if constexpr (QT == 0) {
    d = g4d::f16_bits_to_f32(wr.hdr.x & 0xffffu);
    dmin = g4d::f16_bits_to_f32(wr.hdr.x >> 16);
  } else {
    d = g4d::f16_bits_to_f32(*(const uint16_t*)(W + (size_t)row * Blk<QT>::BYTES + 208));
  }
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    const h8 A = a_operand(wr, s, q);
    float mn = 0.f;
    if constexpr (QT == 0) mn = (float)min_operand(wr, s >> 1)[(s & 1) * 4];
#pragma unroll
    for (int i = 0; i < 8; ++i) o[32 * s + 8 * q + i] = d * (float)A[i] - dmin * mn;
  }
}

// ---------------------------------------------------------------------------
// host
// ---------------------------------------------------------------------------

template <int BPR>
int bprep_bpr(g4_ctx* ctx, int pro, const BPrepArgs& p) {
  const dim3 grid(p.B);
  if (pro == 0) hipLaunchKernelGGL((bprep_kernel<BPR, 0>), grid, dim3(PNT), 0, ctx->stream, p);
  else if (pro == 1) hipLaunchKernelGGL((bprep_kernel<BPR, 1>), grid, dim3(PNT), 0, ctx->stream, p);
  else hipLaunchKernelGGL((bprep_kernel<BPR, 2>), grid, dim3(PNT), 0, ctx->stream, p);
  G4_LAUNCHED(ctx, "batch_prep");
  return G4_OK;
}

int bprep_launch(g4_ctx* ctx, uint32_t N, int pro, const BPrepArgs& p) {
  switch (N / 256) {
    case 6: return bprep_bpr<6>(ctx, pro, p);
    case 8: return bprep_bpr<8>(ctx, pro, p);
    default: return G4_ERR_UNSUPPORTED;
  }
}

bool mm_supported(uint32_t bpr) {
  return bpr == 4 || bpr == 6 || bpr == 8 || bpr == 12 || bpr == 16 || bpr == 24 || bpr == 32 || bpr == 48;
}

// Unrolled walks (NKB > 0) for prebuilt operands, where their register sets
// fit without spilling: KG 1 up to 4 blocks (2 with 64-vector tiles), the
// gate/up pair's KG 2 over 3 or 4 (3 with 64-vector tiles), KG 3 over 1 or 2
// (at most 32-vector tiles); anything else, and rebuilt operands, loops.
template <int KG, int OPK, int NTV>
constexpr bool nkb_unrolled(int n) {
  if (OPK == 0) return false;
  if (KG == 1) return n >= 1 && n <= (NTV <= 2 ? 4 : 2);
  if (KG == 2) return n == 3 || (n == 4 && NTV <= 2);
  return NTV <= 2 && (n == 1 || n == 2);
}

template <int QT, int BPR, int NTV, int MODE, int OPK, int KG>
void mm_launch_kg(g4_ctx* ctx, const MmArgs& a, uint32_t groups, bool unroll) {
  const dim3 grid(groups * a.ksplit), block(KG * MNT);
  switch (unroll ? a.kc / KG : 0u) {
#define G4_MM_NKB(n)                                                                                      \
  case n:                                                                                                 \
    if constexpr (BPR % (KG * n) == 0 && nkb_unrolled<KG, OPK, NTV>(n)) {                                 \
      hipLaunchKernelGGL((mmf_kernel<QT, BPR, NTV, MODE, OPK, KG, n>), grid, block, 0, ctx->stream, a); \
      return;                                                                                             \
    }                                                                                                     \
    break;
    G4_MM_NKB(1)
    G4_MM_NKB(2)
    G4_MM_NKB(3)
    G4_MM_NKB(4)
    G4_MM_NKB(6)
#undef G4_MM_NKB
    default:
      break;
  }
  if constexpr (KG == 3) {  // (three groups only unrolled: the loop's registers spill at 12 waves)
    mm_launch_kg<QT, BPR, NTV, MODE, OPK, 1>(ctx, a, groups, false);
  } else {
    hipLaunchKernelGGL((mmf_kernel<QT, BPR, NTV, MODE, OPK, KG, 0>), grid, block, 0, ctx->stream, a);
  }
}

// K groups per workgroup: the gate/up pair (one workgroup per CU, a whole K
// each) takes two; launches of about one workgroup per CU or fewer take
// three where kc allows (a wave per SIMD leaves the latency of every MFMA
// and operand read exposed; 12 waves share one CU's work three ways).
//
// The unrolled walk holds a register set per block: it is taken by launches
// of about one workgroup per CU or fewer (latency-bound), and with 64-vector
// operands only where the walk is short or the gate/up pair's (longer walks
// spill; the batched LM head, 4096 workgroups, keeps its occupancy with the
// loop).
template <int QT, int BPR, int NTV, int MODE, int OPK>
int mm_launch(g4_ctx* ctx, const MmArgs& a, uint32_t groups) {
  const uint32_t cus = (uint32_t)(ctx->num_cus > 0 ? ctx->num_cus : 256);
  const bool few = groups * a.ksplit <= cus;
  if (MODE == 1 && a.kc % 2 == 0) {
    if constexpr (MODE == 1) mm_launch_kg<QT, BPR, NTV, MODE, OPK, 2>(ctx, a, groups, few);
  } else if (NTV <= 2 && few && a.kc % 3 == 0 && (a.kc == 3 || a.kc == 6)) {
    if constexpr (NTV <= 2) mm_launch_kg<QT, BPR, NTV, MODE, OPK, 3>(ctx, a, groups, true);
  } else {
    mm_launch_kg<QT, BPR, NTV, MODE, OPK, 1>(ctx, a, groups, few && (NTV <= 2 || a.kc <= 2));
  }
  G4_LAUNCHED(ctx, "mm");
  return G4_OK;
}

// Prebuilt operands come from the norm prologue (widths 1536 and 2048) and
// from the attention's merge (the q widths 2048 and, head dim 512, 4096).
template <int BPR>
constexpr bool ops_width() { return BPR == 6 || BPR == 8 || BPR == 16; }

template <int QT, int BPR, int MODE>
int mm_ntv(g4_ctx* ctx, const MmArgs& a, uint32_t groups) {
  const uint32_t Bp = pad_batch(a.B);
  if constexpr (ops_width<BPR>()) {
    if (a.ops) {
      if (Bp == 16) return mm_launch<QT, BPR, 1, MODE, 1>(ctx, a, groups);
      if (Bp == 32) return mm_launch<QT, BPR, 2, MODE, 1>(ctx, a, groups);
      return mm_launch<QT, BPR, 4, MODE, 1>(ctx, a, groups);
    }
  }
  if (a.ops) return G4_ERR_UNSUPPORTED;
  if (Bp == 16) return mm_launch<QT, BPR, 1, MODE, 0>(ctx, a, groups);
  if (Bp == 32) return mm_launch<QT, BPR, 2, MODE, 0>(ctx, a, groups);
  return mm_launch<QT, BPR, 4, MODE, 0>(ctx, a, groups);
}
// A Q6_K matmul over sub-block-scaled operand blocks (the FFN widths).
template <int BPR>
int mm_sub_ntv(g4_ctx* ctx, const MmArgs& a, uint32_t groups) {
  const uint32_t Bp = pad_batch(a.B);
  if (Bp == 16) return mm_launch<1, BPR, 1, 0, 2>(ctx, a, groups);
  if (Bp == 32) return mm_launch<1, BPR, 2, 0, 2>(ctx, a, groups);
  return mm_launch<1, BPR, 4, 0, 2>(ctx, a, groups);
}

template <int QT>
int mm_bpr(g4_ctx* ctx, uint32_t N, const MmArgs& a, uint32_t groups) {
  switch (N / 256) {
    case 4: return mm_ntv<QT, 4, 0>(ctx, a, groups);
    case 6: return mm_ntv<QT, 6, 0>(ctx, a, groups);
    case 8: return mm_ntv<QT, 8, 0>(ctx, a, groups);
    case 12: return mm_ntv<QT, 12, 0>(ctx, a, groups);
    case 16: return mm_ntv<QT, 16, 0>(ctx, a, groups);
    case 24: return mm_ntv<QT, 24, 0>(ctx, a, groups);
    case 32: return mm_ntv<QT, 32, 0>(ctx, a, groups);
    case 48: return mm_ntv<QT, 48, 0>(ctx, a, groups);
    default: return G4_ERR_UNSUPPORTED;
  }
}

// Smallest divisor of bpr (at most max_split) that gives about one workgroup per CU.
uint32_t pick_ksplit(const g4_ctx* ctx, uint32_t groups, uint32_t bpr, uint32_t max_split) {
  const uint32_t want = (uint32_t)(ctx->num_cus > 0 ? ctx->num_cus : 256) * 15 / 16;
  uint32_t best = 1;
  for (uint32_t d = 1; d <= bpr && d <= max_split; ++d) {
    if (bpr % d) continue;
    best = d;
    if (groups * d >= want) break;
  }
  return best;
}

int check_x(const char* fn, const float* x, uint32_t N, uint32_t B) {
  G4_REQUIRE(B >= 1 && B <= 64, "%s: batch %u outside 1..64", fn, B);
  G4_REQUIRE(N % 256 == 0 && mm_supported(N / 256), "%s: N=%u unsupported", fn, N);
  G4_REQUIRE(x && ((uintptr_t)x & 15) == 0, "%s: activations must be non-null and 16-byte aligned", fn);
  return G4_OK;
}

// One matmul launch over up to four matrices sharing the input x [B][N] (or
// the gate/up pair). ksplit > 1 leaves partial sums in Y[i] [ksplit][B][rows[i]].
// sub: ops are sub-block-scaled blocks (a Q6_K matmul of width 6144 or
// 12288); ops_out: the gate/up pair also writes its product's blocks.
int mm_run(g4_ctx* ctx, const char* fn, int qt, const float* x, const uint8_t* ops, const uint8_t* const* W,
           float* const* Y, const uint32_t* rows, int nseg, uint32_t N, uint32_t B, float cap, bool gelu,
           uint32_t ksplit, bool sub = false, uint8_t* ops_out = nullptr) {
  const uint32_t bpr = N / 256;
  uint32_t groups = 0;
  MmArgs a{};
  for (int i = 0; i < nseg; ++i) {
    a.s[i] = MmSeg{W[i], Y[i], rows[i], groups};
    if (!gelu) groups += ceil_div(rows[i], 64);
  }
  if (gelu) groups = ceil_div(rows[0], 32);
  a.n = nseg;
  a.B = B;
  a.cap = cap;
  a.x = x;
  a.ops = ops;
  a.K = N;
  a.ksplit = ksplit;
  a.kc = bpr / ksplit;
  a.ops_out = ops_out;
  int rc;
  if (sub) {
    switch (bpr) {
      case 24: rc = mm_sub_ntv<24>(ctx, a, groups); break;
      case 48: rc = mm_sub_ntv<48>(ctx, a, groups); break;
      default: rc = G4_ERR_UNSUPPORTED;
    }
  } else if (gelu) {
    switch (bpr) {
      case 6: rc = mm_ntv<0, 6, 1>(ctx, a, groups); break;
      case 8: rc = mm_ntv<0, 8, 1>(ctx, a, groups); break;
      default: rc = G4_ERR_UNSUPPORTED;
    }
  } else {
    rc = qt == 0 ? mm_bpr<0>(ctx, N, a, groups) : mm_bpr<1>(ctx, N, a, groups);
  }
  return rc == G4_ERR_UNSUPPORTED ? g4::set_error(rc, "%s: unsupported shape", fn) : rc;
}

uint32_t total_groups(const uint32_t* rows, int nseg) {
  uint32_t g = 0;
  for (int i = 0; i < nseg; ++i) g += ceil_div(rows[i], 64);
  return g;
}

// Complete products: [prologue ->] matmul [-> ordered reduction], all
// intermediates in the context scratch.
int batch_matmul(g4_ctx* ctx, const char* fn, int qt, int pro, const BPrepArgs& p0, const uint8_t* const* W,
                 float* const* Y, const uint32_t* rows, int nseg, uint32_t N, uint32_t B, float cap, bool gelu) {
  int rc = check_x(fn, p0.x, N, B);
  if (rc) return rc;
  G4_REQUIRE(pro == 0 || N == 1536 || N == 2048, "%s: normalising prologue needs N 1536 or 2048", fn);
  const uint32_t bpr = N / 256;
  const uint32_t ksplit = gelu ? 1 : pick_ksplit(ctx, total_groups(rows, nseg), bpr, bpr);
  const uint32_t ntv = pad_batch(B) / 16;
  const size_t xbytes = pro ? (size_t)B * N * sizeof(float) + (size_t)bpr * Ops::bytes((int)ntv) : 0;
  size_t part_off[4] = {0, 0, 0, 0}, part_bytes = 0;
  if (ksplit > 1)
    for (int i = 0; i < nseg; ++i) {
      part_off[i] = xbytes + part_bytes;
      part_bytes += (size_t)ksplit * B * rows[i] * sizeof(float);
    }
  void* scratch = nullptr;
  rc = g4_internal_scratch(ctx, xbytes + part_bytes, &scratch);
  if (rc) return rc;
  const float* x = p0.x;
  const uint8_t* ops = nullptr;
  if (pro) {
    BPrepArgs p = p0;
    p.nparts = 1;
    p.B = B;
    p.out = (float*)scratch;
    p.ops = (uint8_t*)scratch + (size_t)B * N * sizeof(float);
    p.ntv = (int)ntv;
    rc = bprep_launch(ctx, N, pro, p);
    if (rc) return rc == G4_ERR_UNSUPPORTED ? g4::set_error(rc, "%s: unsupported shape", fn) : rc;
    x = p.out;
    ops = p.ops;
  }
  float* dst[4];
  for (int i = 0; i < nseg; ++i) dst[i] = ksplit > 1 ? (float*)((uint8_t*)scratch + part_off[i]) : Y[i];
  rc = mm_run(ctx, fn, qt, x, ops, W, dst, rows, nseg, N, B, cap, gelu, ksplit);
  if (rc || ksplit == 1) return rc;
  for (int i = 0; i < nseg; ++i) {
    const uint32_t n = B * rows[i];
    hipLaunchKernelGGL(reduce_kernel, dim3(ceil_div(n, PNT)), dim3(PNT), 0, ctx->stream, dst[i], Y[i], n, ksplit,
                       cap);
    G4_LAUNCHED(ctx, "mm_reduce");
  }
  return G4_OK;
}

int check_norms(const char* fn, const uint16_t* w1, const float* residual, const uint16_t* w2,
                const float* h_out) {
  G4_REQUIRE(!residual == !w2, "%s: residual and w2 go together", fn);
  G4_REQUIRE((!residual || ((uintptr_t)residual & 15) == 0) && (!h_out || ((uintptr_t)h_out & 15) == 0),
             "%s: activations must be 16-byte aligned", fn);
  G4_REQUIRE((!w1 || ((uintptr_t)w1 & 7) == 0) && (!w2 || ((uintptr_t)w2 & 7) == 0),
             "%s: norm weights must be 8-byte aligned", fn);
  return G4_OK;
}

int check_weights(const char* fn, int wtype, const void* const* weights, float* const* outputs,
                  const uint32_t* rows, int nseg) {
  G4_REQUIRE(wtype == 0 || wtype == 1, "%s: wtype must be 0 (Q4_K) or 1 (Q6_K)", fn);
  G4_REQUIRE(nseg >= 1 && nseg <= 4, "%s: 1..4 segments", fn);
  G4_REQUIRE(weights && outputs && rows, "%s: null buffer", fn);
  for (int i = 0; i < nseg; ++i) {
    G4_REQUIRE(weights[i] && outputs[i] && rows[i] > 0, "%s: segment %d empty", fn, i);
    G4_REQUIRE(((uintptr_t)weights[i] & (wtype == 0 ? 15 : 3)) == 0,
               "%s: weights misaligned (Q4_K 16 B, Q6_K 4 B)", fn);
  }
  return G4_OK;
}

}  // namespace

// Used by k_gemv.hip's batched entry points for batch >= 16.
int g4_internal_batch_matmul(g4_ctx* ctx, const char* fn, int qt, const float* x, const void* w, float* y,
                             uint32_t M, uint32_t N, uint32_t batch) {
  BPrepArgs p{};
  p.x = x;
  const uint8_t* W[1] = {(const uint8_t*)w};
  float* Y[1] = {y};
  const uint32_t rows[1] = {M};
  return batch_matmul(ctx, fn, qt, 0, p, W, Y, rows, 1, N, batch, 0.f, false);
}

int g4_internal_operand_values(g4_ctx* ctx, int wtype, const void* blocks, uint64_t nblocks, float* out) {
  G4_REQUIRE(nblocks < (1ull << 32), "g4_dequantPath: path 2 takes fewer than 2^32 blocks");
  const uint32_t nb = (uint32_t)nblocks;
  const dim3 grid((nb + 15) / 16);
  if (wtype == 0)
    hipLaunchKernelGGL(operand_check_kernel<0>, grid, dim3(64), 0, ctx->stream, (const uint8_t*)blocks, nb, out);
  else
    hipLaunchKernelGGL(operand_check_kernel<1>, grid, dim3(64), 0, ctx->stream, (const uint8_t*)blocks, nb, out);
  G4_LAUNCHED(ctx, "operand_check");
  return G4_OK;
}

extern "C" {

int g4_normAddMatmulSegmentsBatch(g4_ctx* ctx, int wtype, const float* x, const uint16_t* w1,
                                  const float* residual, const uint16_t* w2, float* h_out,
                                  const void* const* weights, float* const* outputs, const uint32_t* rows, int nseg,
                                  uint32_t N, float eps, float softcap_cap, uint32_t batch) {
  G4_ENTER(ctx);
  int rc = check_weights(__func__, wtype, weights, outputs, rows, nseg);
  if (!rc) rc = check_norms(__func__, w1, residual, w2, h_out);
  if (rc) return rc;
  const uint8_t* W[4];
  float* Y[4];
  for (int i = 0; i < nseg; ++i) {
    W[i] = (const uint8_t*)weights[i];
    Y[i] = outputs[i];
  }
  const int pro = !w1 ? 0 : (residual ? 2 : 1);
  const BPrepArgs p{x, 1, batch, w1, residual, w2, h_out, nullptr, eps, nullptr, 0};
  return batch_matmul(ctx, __func__, wtype, pro, p, W, Y, rows, nseg, N, batch, softcap_cap, false);
}

int g4_normAddGateUpGeluBatch(g4_ctx* ctx, const float* o, const uint16_t* w_post, const float* residual,
                              const uint16_t* w_pre, const void* w_gate, const void* w_up, float* h_out, float* out,
                              g4_matmul_params p, float eps, uint32_t batch) {
  G4_ENTER(ctx);
  G4_REQUIRE(o && w_post && residual && w_pre && w_gate && w_up && out, "g4_normAddGateUpGeluBatch: null buffer");
  G4_REQUIRE(p.M > 0 && (p.N == 1536 || p.N == 2048), "g4_normAddGateUpGeluBatch: N=%u must be 1536 or 2048",
             p.N);
  G4_REQUIRE(((uintptr_t)w_gate & 15) == 0 && ((uintptr_t)w_up & 15) == 0,
             "g4_normAddGateUpGeluBatch: weights must be 16-byte aligned");
  int rc = check_norms(__func__, w_post, residual, w_pre, h_out);
  if (rc) return rc;
  const uint8_t* W[2] = {(const uint8_t*)w_gate, (const uint8_t*)w_up};
  float* Y[2] = {out, out};
  const uint32_t rows[2] = {p.M, p.M};
  const BPrepArgs pa{o, 1, batch, w_post, residual, w_pre, h_out, nullptr, eps, nullptr, 0};
  return batch_matmul(ctx, __func__, 0, 2, pa, W, Y, rows, 2, p.N, batch, 0.f, true);
}

int g4_batchOperandBytes(uint32_t N, uint32_t batch, size_t* bytes) {
  G4_REQUIRE(bytes && N % 256 == 0 && batch >= 1 && batch <= 64, "g4_batchOperandBytes: bad shape");
  *bytes = (size_t)(N / 256) * Ops::bytes((int)(pad_batch(batch) / 16));
  return G4_OK;
}

int g4_batchPrep(g4_ctx* ctx, const float* x, uint32_t nparts, const uint16_t* w1, const float* residual,
                 const uint16_t* w2, float* h_out, float* out, void* ops, uint32_t N, uint32_t batch, float eps) {
  G4_ENTER(ctx);
  G4_REQUIRE(!residual == !w2, "g4_batchPrep: residual and w2 go together");
  return g4_batchPrepScale(ctx, x, nparts, w1, residual, nullptr, w2, h_out, out, ops, N, batch, eps);
}

int g4_batchPrepScale(g4_ctx* ctx, const float* x, uint32_t nparts, const uint16_t* w1, const float* residual,
                      const uint16_t* out_scale, const uint16_t* w2, float* h_out, float* out, void* ops, uint32_t N,
                      uint32_t batch, float eps) {
  G4_ENTER(ctx);
  G4_REQUIRE(!out_scale || residual, "g4_batchPrepScale: out_scale needs the residual form");
  G4_REQUIRE(!w2 || residual, "g4_batchPrepScale: w2 needs the residual form");
  G4_REQUIRE(x && out && nparts >= 1, "g4_batchPrep: null buffer or no parts");
  G4_REQUIRE(batch >= 1 && batch <= (ops ? 64u : 65535u), "g4_batchPrep: batch %u out of range", batch);
  G4_REQUIRE(N == 1536 || N == 2048, "g4_batchPrep: N=%u must be 1536 or 2048", N);
  G4_REQUIRE(((uintptr_t)x & 15) == 0 && ((uintptr_t)out & 15) == 0 && ((uintptr_t)ops & 15) == 0,
             "g4_batchPrep: buffers must be 16-byte aligned");
  G4_REQUIRE(w1 || !residual, "g4_batchPrep: residual needs w1");
  G4_REQUIRE((!residual || ((uintptr_t)residual & 15) == 0) && (!h_out || ((uintptr_t)h_out & 15) == 0),
             "g4_batchPrep: activations must be 16-byte aligned");
  G4_REQUIRE((!w1 || ((uintptr_t)w1 & 7) == 0) && (!w2 || ((uintptr_t)w2 & 7) == 0),
             "g4_batchPrep: norm weights must be 8-byte aligned");
  const int pro = !w1 ? 0 : (residual ? 2 : 1);
  const BPrepArgs p{x, nparts, batch, w1, residual, w2, h_out, out, eps, (uint8_t*)ops,
                    (int)(pad_batch(batch) / 16), out_scale};
  return bprep_launch(ctx, N, pro, p);
}

int g4_matmulSegmentsBatchPartial(g4_ctx* ctx, int wtype, const float* x, const void* ops,
                                  const void* const* weights, float* const* outputs, const uint32_t* rows, int nseg,
                                  uint32_t N, uint32_t batch, uint32_t max_ksplit, float softcap_cap,
                                  uint32_t* ksplit) {
  G4_ENTER(ctx);
  int rc = check_weights(__func__, wtype, weights, outputs, rows, nseg);
  if (!rc) rc = check_x(__func__, x, N, batch);
  if (rc) return rc;
  G4_REQUIRE(ksplit && max_ksplit >= 1, "g4_matmulSegmentsBatchPartial: null ksplit or max_ksplit 0");
  G4_REQUIRE(softcap_cap <= 0.f || max_ksplit == 1, "g4_matmulSegmentsBatchPartial: softcap needs max_ksplit 1");
  G4_REQUIRE(!ops || ((uintptr_t)ops & 15) == 0, "g4_matmulSegmentsBatchPartial: operands must be 16-byte aligned");
  const uint8_t* W[4];
  float* Y[4];
  for (int i = 0; i < nseg; ++i) {
    W[i] = (const uint8_t*)weights[i];
    Y[i] = outputs[i];
  }
  const uint32_t ks = pick_ksplit(ctx, total_groups(rows, nseg), N / 256, max_ksplit);
  rc = mm_run(ctx, __func__, wtype, x, (const uint8_t*)ops, W, Y, rows, nseg, N, batch, softcap_cap, false, ks);
  if (rc == G4_OK) *ksplit = ks;
  return rc;
}

int g4_gateUpGeluBatch(g4_ctx* ctx, const float* x, const void* ops, const void* w_gate, const void* w_up,
                       float* out, g4_matmul_params p, uint32_t batch) {
  G4_ENTER(ctx);
  G4_REQUIRE(w_gate && w_up && out && p.M > 0, "g4_gateUpGeluBatch: null buffer or empty");
  G4_REQUIRE(p.N == 1536 || p.N == 2048, "g4_gateUpGeluBatch: N=%u must be 1536 or 2048", p.N);
  G4_REQUIRE(((uintptr_t)w_gate & 15) == 0 && ((uintptr_t)w_up & 15) == 0 && ((uintptr_t)ops & 15) == 0,
             "g4_gateUpGeluBatch: weights and operands must be 16-byte aligned");
  int rc = check_x(__func__, x, p.N, batch);
  if (rc) return rc;
  const uint8_t* W[2] = {(const uint8_t*)w_gate, (const uint8_t*)w_up};
  float* Y[2] = {out, out};
  const uint32_t rows[2] = {p.M, p.M};
  return mm_run(ctx, __func__, 0, x, (const uint8_t*)ops, W, Y, rows, 2, p.N, batch, 0.f, true, 1);
}

int g4_batchSubOperandBytes(uint32_t K, uint32_t batch, size_t* bytes) {
  G4_REQUIRE(bytes && (K == 6144 || K == 12288) && batch >= 1 && batch <= 64, "g4_batchSubOperandBytes: bad shape");
  *bytes = (size_t)(K / 256) * OpsSub::bytes((int)(pad_batch(batch) / 16));
  return G4_OK;
}

int g4_gateUpGeluBatchOps(g4_ctx* ctx, const float* x, const void* ops, const void* w_gate, const void* w_up,
                          float* out, void* down_ops, g4_matmul_params p, uint32_t batch) {
  G4_ENTER(ctx);
  G4_REQUIRE(w_gate && w_up && ops && down_ops && p.M > 0, "g4_gateUpGeluBatchOps: null buffer or empty");
  G4_REQUIRE(p.N == 1536 || p.N == 2048, "g4_gateUpGeluBatchOps: N=%u must be 1536 or 2048", p.N);
  G4_REQUIRE(p.M == 6144 || p.M == 12288, "g4_gateUpGeluBatchOps: M=%u must be 6144 or 12288", p.M);
  G4_REQUIRE(((uintptr_t)w_gate & 15) == 0 && ((uintptr_t)w_up & 15) == 0 && ((uintptr_t)ops & 15) == 0 &&
                 ((uintptr_t)down_ops & 15) == 0,
             "g4_gateUpGeluBatchOps: weights and operands must be 16-byte aligned");
  int rc = check_x(__func__, x, p.N, batch);
  if (rc) return rc;
  const uint8_t* W[2] = {(const uint8_t*)w_gate, (const uint8_t*)w_up};
  float* Y[2] = {out, out};
  const uint32_t rows[2] = {p.M, p.M};
  return mm_run(ctx, __func__, 0, x, (const uint8_t*)ops, W, Y, rows, 2, p.N, batch, 0.f, true, 1, false,
                (uint8_t*)down_ops);
}

int g4_matmulSubBatchPartial(g4_ctx* ctx, const void* ops, const void* weight, float* out, uint32_t M, uint32_t K,
                             uint32_t batch, uint32_t max_ksplit, uint32_t* ksplit) {
  G4_ENTER(ctx);
  G4_REQUIRE(ops && weight && out && ksplit && M > 0 && max_ksplit >= 1,
             "g4_matmulSubBatchPartial: null buffer, no rows or max_ksplit 0");
  G4_REQUIRE(K == 6144 || K == 12288, "g4_matmulSubBatchPartial: K=%u must be 6144 or 12288", K);
  G4_REQUIRE(batch >= 1 && batch <= 64, "g4_matmulSubBatchPartial: batch %u outside 1..64", batch);
  G4_REQUIRE(((uintptr_t)ops & 15) == 0 && ((uintptr_t)weight & 3) == 0,
             "g4_matmulSubBatchPartial: operands 16-byte, weights 4-byte aligned");
  const uint8_t* W[1] = {(const uint8_t*)weight};
  float* Y[1] = {out};
  const uint32_t rows[1] = {M};
  const uint32_t ks = pick_ksplit(ctx, total_groups(rows, 1), K / 256, max_ksplit);
  // (x is not read: the operands are the blocks)
  const int rc = mm_run(ctx, __func__, 1, (const float*)ops, (const uint8_t*)ops, W, Y, rows, 1, K, batch, 0.f,
                        false, ks, true);
  if (rc == G4_OK) *ksplit = ks;
  return rc;
}

}  // extern "C"
