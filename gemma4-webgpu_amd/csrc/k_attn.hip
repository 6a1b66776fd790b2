// k_attn.hip — GQA decode attention over an f16 KV cache.
//
// Forms of the same computation (shaders/attn_score.wgsl, shaders/softmax.wgsl,
// shaders/attn_output.wgsl; scale 1.0, sliding window W masks positions
// < seq_len - W):
//  * the per-key trio attnScore -> softmax -> attnOutput, kept so that every
//    reference kernel has a drop-in (scores round-trip through HBM);
//  * split-K flash-decode: workgroup (split, kv head[, sequence]) loads a
//    32/64-row chunk of K/V once for all G = NQH/NKH query heads of that KV
//    head and writes a (max, sum, o) partial per head; a merge kernel
//    combines the splits with a log-sum-exp rescale. The paged form addresses
//    rows through a per-sequence page table (ragged multi-sequence batches).
//  * the fused decode form additionally applies q_norm/k_norm + RoPE and the
//    weightless v_norm and stores the current K/V row
//    (src/engine.ts:1562-1584: perHeadRmsNormNoWeight, fusedPerHeadNormRope
//    q/k, kvCacheStore, attnScore, softmax, attnOutput in two launches).
#include <math.h>

#include <algorithm>

#include "g4_internal.hpp"
#include "mqf_core.hpp"

namespace {

using namespace g4mqf;

constexpr int NT = 256;
constexpr float kMasked = -1e30f;

// ---------------------------------------------------------------------------
// the trio
// ---------------------------------------------------------------------------

// seq_len of a trio launch: the Params value, or with pos_dev (the _dev
// entries) *pos_dev + 1 read on the device, at most the Params value (the
// maximum the grid and the scores buffer were sized for).
__device__ __forceinline__ uint32_t trio_len(uint32_t seq_len, const uint32_t* pos_dev) {
  return pos_dev ? min(*pos_dev + 1u, seq_len) : seq_len;
}

// One wave per position: lanes stride the head dimension (coalesced row
// reads), one wave reduction per query head.
__global__ __launch_bounds__(NT) void attn_score_kernel(const float* q, const uint16_t* kc, float* scores,
                                                        uint32_t nqh, uint32_t nkh, uint32_t hd,
                                                        uint32_t max_len, float scale, uint32_t window,
                                                        const uint32_t* pos_dev) {
  const uint32_t seq_len = trio_len(max_len, pos_dev);
  const int lane = threadIdx.x & 63;
  const uint32_t pos = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (pos >= seq_len) return;
  const uint32_t cur = seq_len - 1;
  const uint32_t ws = (window != 0 && cur + 1 > window) ? cur + 1 - window : 0;
  for (uint32_t h = 0; h < nqh; ++h) {
    float s;
    if (pos < ws) {
      s = kMasked;
    } else {
      const uint32_t kvh = h * nkh / nqh;
      const uint16_t* k = kc + ((size_t)pos * nkh + kvh) * hd;
      float acc = 0.f;
      for (uint32_t d = lane; d < hd; d += 64) acc += q[h * hd + d] * g4d::f16_bits_to_f32(k[d]);
      s = g4d::wave_sum(acc) * scale;
    }
    if (lane == 0) scores[(size_t)h * seq_len + pos] = s;
  }
}

// One workgroup per head: max (init -1e30), exp, sum, normalise.
__global__ __launch_bounds__(NT) void softmax_kernel(float* scores, uint32_t num_heads, uint32_t max_len,
                                                     const uint32_t* pos_dev) {
  const uint32_t seq_len = trio_len(max_len, pos_dev);
  __shared__ float red[4];
  const uint32_t h = blockIdx.x;
  if (h >= num_heads) return;
  float* s = scores + (size_t)h * seq_len;
  float mx = kMasked;
  for (uint32_t i = threadIdx.x; i < seq_len; i += NT) mx = fmaxf(mx, s[i]);
  mx = g4d::wave_max(mx);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  float sum = 0.f;
  for (uint32_t i = threadIdx.x; i < seq_len; i += NT) {
    const float e = expf(s[i] - mx);
    s[i] = e;
    sum += e;
  }
  sum = g4d::block_sum<4>(sum, red);
  const float inv = 1.0f / sum;
  for (uint32_t i = threadIdx.x; i < seq_len; i += NT) s[i] = s[i] * inv;
}

// Thread per (head, d): sum over positions of p * V.
__global__ __launch_bounds__(NT) void attn_output_kernel(const float* probs, const uint16_t* vc, float* out,
                                                         uint32_t nqh, uint32_t nkh, uint32_t hd,
                                                         uint32_t max_len, const uint32_t* pos_dev) {
  const uint32_t seq_len = trio_len(max_len, pos_dev);
  const uint32_t idx = blockIdx.x * NT + threadIdx.x;
  if (idx >= nqh * hd) return;
  const uint32_t h = idx / hd, d = idx % hd;
  const uint32_t kvh = h * nkh / nqh;
  const float* p = probs + (size_t)h * seq_len;
  const uint16_t* v = vc + (size_t)kvh * hd + d;
  const size_t stride = (size_t)nkh * hd;
  float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
  uint32_t pos = 0;
  for (; pos + 4 <= seq_len; pos += 4) {
    a0 += p[pos] * g4d::f16_bits_to_f32(v[(size_t)pos * stride]);
    a1 += p[pos + 1] * g4d::f16_bits_to_f32(v[(size_t)(pos + 1) * stride]);
    a2 += p[pos + 2] * g4d::f16_bits_to_f32(v[(size_t)(pos + 2) * stride]);
    a3 += p[pos + 3] * g4d::f16_bits_to_f32(v[(size_t)(pos + 3) * stride]);
  }
  for (; pos < seq_len; ++pos) a0 += p[pos] * g4d::f16_bits_to_f32(v[(size_t)pos * stride]);
  out[idx] = (a0 + a1) + (a2 + a3);
}

// ---------------------------------------------------------------------------
// split-K flash-decode
// ---------------------------------------------------------------------------
//
// Workgroup (split, kv head, sequence) owns P = 32*CP consecutive positions
// of the window and issues every K and V load of its chunk before any other
// work, so the chunk costs one memory round trip:
//   K: thread t reads row (t/8) of each 32-row block, slice t%8 (HD/8 halves);
//   V: thread t reads column(s) of every row of the chunk (one f16 per row for
//      head_dim 256; head_dim 512 reads two adjacent columns, 128 splits the
//      rows between two threads per column).
// Scores are reduced over the 8 slice lanes, the chunk's softmax statistics
// are formed in LDS, and each thread accumulates o for its own columns, so no
// cross-wave reduction is needed. A partial (m, l, o) per (split, head) goes
// to the workspace and attn_merge_kernel combines the splits.

struct AttnArgs {
  const float* q;            // [num_seqs][nqh][hd] (fused form: raw q projection)
  const uint16_t* kc;        // cache [max_seq][nkh][hd] or pool [rows][nkh][hd]
  uint16_t* vc_w;            // fused form: written at the current row
  uint16_t* kc_w;
  const uint16_t* vc;
  const int32_t* page_table; // paged: [num_seqs][max_pages]
  uint32_t page_size, max_pages, num_pages;
  const uint32_t* seq_lens;  // paged: per sequence
  const uint32_t* pos_dev;   // dense dev forms: seq_len = *pos_dev + 1
  uint32_t seq_len;          // dense: the length (host form) or the cache capacity (dev forms)
  uint32_t cap;              // lengths are clamped to it
  uint32_t nqh, nkh;
  float scale;
  uint32_t window;
  uint32_t chunk;            // positions per split (= 32 * CP)
  uint32_t nsplit;           // splits per (sequence, kv head)
  float* ws;                 // partials: m, l, o
  // fused form
  const float* k_in;         // [num_seqs][nkh][hd] raw k projection
  const float* v_in;         // [num_seqs][nkh][hd] raw v projection
  const uint16_t* q_w;       // q_norm weight f16[hd]
  const uint16_t* k_w;       // k_norm weight f16[hd]
  const uint16_t* rope_freqs;
  float theta;
  uint32_t apply_divisor;
  float eps;
};

__host__ __device__ inline size_t ws_bytes(uint32_t num_seqs, uint32_t nkh, uint32_t nsplit, uint32_t G,
                                          uint32_t hd) {
  return (size_t)num_seqs * nkh * nsplit * G * (hd + 2) * sizeof(float);
}

template <int HD>
struct VMap {  // V columns / row groups per thread
  static constexpr int VD = HD >= 512 ? HD / 256 : 1;   // adjacent columns per thread
  static constexpr int VG = HD >= 256 ? 1 : 256 / HD;   // threads sharing a column (row groups)
};

// Group-of-SL-lanes reductions (SL = 32 or 64, aligned inside a wave): every
// lane gets its group's value.
template <int SL>
__device__ __forceinline__ float group_max(float v) {
  v = g4d::max16(v);
  const float a0 = g4d::lane_value(v, 0), a1 = g4d::lane_value(v, 16);
  const float a2 = g4d::lane_value(v, 32), a3 = g4d::lane_value(v, 48);
  if constexpr (SL == 64) return fmaxf(fmaxf(a0, a1), fmaxf(a2, a3));
  return (threadIdx.x & 32) ? fmaxf(a2, a3) : fmaxf(a0, a1);
}
template <int SL>
__device__ __forceinline__ float group_sum(float v) {
  v = g4d::sum16(v);
  const float a0 = g4d::lane_value(v, 0), a1 = g4d::lane_value(v, 16);
  const float a2 = g4d::lane_value(v, 32), a3 = g4d::lane_value(v, 48);
  if constexpr (SL == 64) return (a0 + a1) + (a2 + a3);
  return (threadIdx.x & 32) ? a2 + a3 : a0 + a1;
}

// Order of work: every load this workgroup needs is issued before any result
// is used, the query side first (all waves, then one s_barrier), then the K
// and V rows of the chunk. Loads are unconditional at clamped positions (rows
// past the chunk are masked in the scores), so no branch or loop surrounds a
// load: the compiler then waits for exactly the loads each step consumes.
template <int G, int HD, int CP, bool PAGED, bool FUSE>
__global__ __launch_bounds__(NT) void attn_kernel(AttnArgs a) {
  constexpr int P = 32 * CP;        // positions of a chunk
  constexpr int KS = HD / 8;        // halves of a K row per slice lane
  constexpr int KW = KS / 8;        // 16-byte words per slice
  constexpr int QS = HD + 32;       // padded q row: 4 floats after each of the 8 slices
  constexpr int VD = VMap<HD>::VD;
  constexpr int VG = VMap<HD>::VG;
  constexpr int VR = P / VG;        // rows of V per thread
  constexpr int QE = (G * HD + NT - 1) / NT;  // q elements per thread (t + NT k)
  constexpr int KE = (HD + NT - 1) / NT;      // k / v elements per thread (fused form)
  static_assert(KS % 8 == 0 && VD <= 2, "layout");
  __shared__ __align__(16) float q_s[G * QS];
  __shared__ __align__(16) float p_s[P * G];     // scores, then probabilities [pos][head]
  __shared__ float stat_s[2 * G];
  __shared__ float2 cs_s[FUSE ? HD / 2 : 1];
  __shared__ float cur_s[FUSE ? 2 * HD : 1];     // current row: k (roped), v; f16-rounded
  __shared__ float red_s[4 * (G + 2)];
  __shared__ float o_s[VG > 1 ? G * HD : 1];

  const uint32_t split = blockIdx.x, kvh = blockIdx.y, seq = blockIdx.z;
  const int tid = threadIdx.x, w = tid >> 6;
  uint32_t L;
  if (PAGED) L = a.seq_lens[seq];
  else L = a.pos_dev ? *a.pos_dev + 1 : a.seq_len;
  L = min(L, a.cap);  // never address rows past the cache / page table
  const uint32_t wstart = (a.window != 0 && L > a.window) ? L - a.window : 0;
  const uint32_t b0 = wstart + split * a.chunk;
  const uint32_t b1 = min(L, b0 + a.chunk);
  const size_t part = (((size_t)seq * a.nkh + kvh) * a.nsplit + split) * G;
  const size_t nparts = (size_t)gridDim.z * a.nkh * a.nsplit * G;
  float* ws_m = a.ws;
  float* ws_l = ws_m + nparts;
  float* ws_o = ws_m + 2 * nparts;
  if (b0 >= b1) {  // a split past the live length (uniform over the workgroup)
    if (tid < G) {
      ws_m[part + tid] = -INFINITY;
      ws_l[part + tid] = 0.f;
    }
    return;
  }

  auto row_of = [&](uint32_t pos) -> size_t {
    if (PAGED) {
      int32_t pg = a.page_table[(size_t)seq * a.max_pages + pos / a.page_size];
      pg = pg < 0 ? 0 : (pg >= (int32_t)a.num_pages ? (int32_t)a.num_pages - 1 : pg);
      return (size_t)pg * a.page_size + pos % a.page_size;
    }
    return pos;
  };

  // ---- 1. query-side loads ----
  const float* qg = a.q + ((size_t)seq * a.nqh + (size_t)kvh * G) * HD;
  float qv[QE];
#pragma unroll
  for (int k = 0; k < QE; ++k) {
    const int i = tid + k * NT;
    qv[k] = qg[i < G * HD ? i : 0];
  }
  float kx[FUSE ? KE : 1], vx[FUSE ? KE : 1], kwt[FUSE ? KE : 1], qwt[FUSE ? QE : 1];
  uint16_t rfb = 0;
  // without k_in the layer reads a cache another layer has already written
  // this position's row into: no row is formed, stored or patched
  const bool own_row = !FUSE || a.k_in != nullptr;
  if constexpr (FUSE) {
#pragma unroll
    for (int k = 0; k < KE; ++k) {
      const int i = tid + k * NT, ic = i < HD ? i : 0;
      kx[k] = own_row ? a.k_in[((size_t)seq * a.nkh + kvh) * HD + ic] : 0.f;
      vx[k] = own_row ? a.v_in[((size_t)seq * a.nkh + kvh) * HD + ic] : 0.f;
      kwt[k] = own_row ? g4d::f16_bits_to_f32(a.k_w[ic]) : 0.f;
    }
#pragma unroll
    for (int k = 0; k < QE; ++k) qwt[k] = g4d::f16_bits_to_f32(a.q_w[(tid + k * NT) % HD]);
    rfb = a.rope_freqs[tid < HD / 2 ? tid : 0];  // valid even without the divisor (host passes q_w)
  }
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();  // every wave's query loads are out before any K/V load
  __builtin_amdgcn_sched_barrier(0);

  // ---- 2. the chunk's K and V rows ----
  const int ks = tid & 7;  // K slice
  uint4 kraw[CP][KW];
#pragma unroll
  for (int c = 0; c < CP; ++c) {
    const uint32_t pos = min(b0 + (uint32_t)(c * 32 + (tid >> 3)), b1 - 1);
    const uint4* kp = (const uint4*)(a.kc + (row_of(pos) * a.nkh + kvh) * HD + ks * KS);
#pragma unroll
    for (int j = 0; j < KW; ++j) kraw[c][j] = kp[j];
  }
  const int vcol = (tid % (HD / VD)) * VD;  // first column of this thread
  const int vgrp = tid / (HD / VD);         // row group (VG > 1 only)
  uint32_t vraw[VR];                        // VD f16 values per row (VD == 2: packed)
#pragma unroll
  for (int r = 0; r < VR; ++r) {
    const uint32_t pos = min(b0 + (uint32_t)(r * VG + vgrp), b1 - 1);
    const uint16_t* vp = a.vc + (row_of(pos) * a.nkh + kvh) * HD + vcol;
    vraw[r] = VD == 2 ? *(const uint32_t*)vp : (uint32_t)*vp;
  }
  __builtin_amdgcn_sched_barrier(0);

  // ---- 3. q (fused: per-head RMSNorm + RoPE, and this position's k/v row) ----
  auto qidx = [](int h, int d) { return h * QS + d + (d / KS) * 4; };
  if constexpr (FUSE) {
    const uint32_t pos = L - 1;  // the position being decoded
    // RoPE for this position: the frequency is the correctly rounded f32 of
    // 1/theta^(2i/HD) and the angle the f32 product, as
    // shaders/fused_per_head_norm_rope.wgsl:50-55 forms them; cos/sin of that
    // angle in f32 (within 2 ulp of the rounded exact values).
    if (tid < HD / 2) cs_s[tid] = rope_cos_sin(a.theta, a.apply_divisor, rfb, tid, HD, pos);
    static_assert((G * HD) % NT == 0 && HD >= 256, "fused form: whole q heads per thread stride");
    const bool owner = b1 == L && own_row;  // this chunk holds the current position and forms its row
    // Where the row is written. Paged: the page id must be in the pool and
    // the length unclamped; otherwise nothing is stored (the attention still
    // uses the row), as g4_pagedKvStore does for a bad table entry.
    bool store = true;
    size_t srow = pos;
    if constexpr (PAGED) {
      const uint32_t lr = a.seq_lens[seq];
      const int32_t pg = a.page_table[(size_t)seq * a.max_pages + pos / a.page_size];
      store = lr <= a.cap && pg >= 0 && pg < (int32_t)a.num_pages;
      srow = (size_t)(store ? pg : 0) * a.page_size + pos % a.page_size;
    }
    uint16_t* kdst = a.kc_w + (srow * a.nkh + kvh) * HD;
    uint16_t* vdst = a.vc_w + (srow * a.nkh + kvh) * HD;
    float ss[G + 2];
#pragma unroll
    for (int h = 0; h < G + 2; ++h) ss[h] = 0.f;
#pragma unroll
    for (int k = 0; k < QE; ++k) ss[(tid + k * NT) / HD] += qv[k] * qv[k];
#pragma unroll
    for (int k = 0; k < KE; ++k) {
      const bool in = tid + k * NT < HD;
      ss[G] += in ? kx[k] * kx[k] : 0.f;
      ss[G + 1] += in ? vx[k] * vx[k] : 0.f;
    }
#pragma unroll
    for (int h = 0; h < G + 2; ++h) {
      const float t = g4d::wave_sum_dpp(ss[h]);
      if ((tid & 63) == 0) red_s[w * (G + 2) + h] = t;
    }
    __syncthreads();
    float inv[G + 2];
#pragma unroll
    for (int h = 0; h < G + 2; ++h) {
      const float tot = red_s[h] + red_s[(G + 2) + h] + red_s[2 * (G + 2) + h] + red_s[3 * (G + 2) + h];
      inv[h] = 1.0f / sqrtf(tot / (float)HD + a.eps);
    }
#pragma unroll
    for (int k = 0; k < QE; ++k) {
      const int i = tid + k * NT, h = i / HD, d = i % HD;
      q_s[qidx(h, d)] = qv[k] * qwt[k] * inv[h];
    }
    if (owner) {
#pragma unroll
      for (int k = 0; k < KE; ++k) {
        const int i = tid + k * NT;
        if (i < HD) {
          cur_s[i] = kx[k] * kwt[k] * inv[G];
          const uint16_t vb = g4d::f32_to_f16_bits(vx[k] * inv[G + 1]);
          cur_s[HD + i] = g4d::f16_bits_to_f32(vb);
          if (store) vdst[i] = vb;
        }
      }
    }
    __syncthreads();
    // rotate-half over pairs (i, i + HD/2): the G q heads, and k in the owner
    for (int j = tid; j < (G + (owner ? 1 : 0)) * HD / 2; j += NT) {
      const int h = j / (HD / 2), i = j % (HD / 2);
      const float2 cs = cs_s[i];
      if (h < G) {
        float* p0 = q_s + qidx(h, i);
        float* p1 = q_s + qidx(h, i + HD / 2);
        const float x0 = *p0, x1 = *p1;
        *p0 = x0 * cs.x - x1 * cs.y;
        *p1 = x0 * cs.y + x1 * cs.x;
      } else {
        const float x0 = cur_s[i], x1 = cur_s[i + HD / 2];
        const uint16_t k0 = g4d::f32_to_f16_bits(x0 * cs.x - x1 * cs.y);
        const uint16_t k1 = g4d::f32_to_f16_bits(x0 * cs.y + x1 * cs.x);
        if (store) {
          kdst[i] = k0;
          kdst[i + HD / 2] = k1;
        }
        cur_s[i] = g4d::f16_bits_to_f32(k0);  // as the cache row will read back
        cur_s[i + HD / 2] = g4d::f16_bits_to_f32(k1);
      }
    }
    __syncthreads();
    // the current row was loaded from the cache before it was written: take it from LDS
    if (owner) {
      const uint32_t pc = pos - b0;
#pragma unroll
      for (int c = 0; c < CP; ++c) {
        if ((uint32_t)(c * 32 + (tid >> 3)) == pc) {
#pragma unroll
          for (int j = 0; j < KW; ++j) {
            uint32_t wd[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int d = ks * KS + 8 * j + 2 * e;
              wd[e] = (uint32_t)g4d::f32_to_f16_bits(cur_s[d]) | ((uint32_t)g4d::f32_to_f16_bits(cur_s[d + 1]) << 16);
            }
            kraw[c][j] = make_uint4(wd[0], wd[1], wd[2], wd[3]);
          }
        }
      }
#pragma unroll
      for (int r = 0; r < VR; ++r) {
        if ((uint32_t)(r * VG + vgrp) == pc) {
          const uint32_t v0 = g4d::f32_to_f16_bits(cur_s[HD + vcol]);
          vraw[r] = VD == 2 ? (v0 | ((uint32_t)g4d::f32_to_f16_bits(cur_s[HD + vcol + 1]) << 16)) : v0;
        }
      }
    }
  } else {
#pragma unroll
    for (int k = 0; k < QE; ++k) {
      const int i = tid + k * NT;
      if (i < G * HD) q_s[qidx(i / HD, i % HD)] = qv[k];
    }
    __syncthreads();
  }

  // ---- 4. scores: 8 slice lanes per row ----
#pragma unroll
  for (int c = 0; c < CP; ++c) {
    float acc[G];
#pragma unroll
    for (int h = 0; h < G; ++h) acc[h] = 0.f;
#pragma unroll
    for (int j = 0; j < KW; ++j) {
      const uint32_t wd[4] = {kraw[c][j].x, kraw[c][j].y, kraw[c][j].z, kraw[c][j].w};
      float kf[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        kf[2 * e] = g4d::f16_bits_to_f32(wd[e] & 0xffffu);
        kf[2 * e + 1] = g4d::f16_bits_to_f32(wd[e] >> 16);
      }
      const int d0 = ks * KS + 8 * j;
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const float4 q0 = *(const float4*)(q_s + qidx(h, d0));
        const float4 q1 = *(const float4*)(q_s + qidx(h, d0 + 4));
        acc[h] += q0.x * kf[0] + q0.y * kf[1] + q0.z * kf[2] + q0.w * kf[3];
        acc[h] += q1.x * kf[4] + q1.y * kf[5] + q1.z * kf[6] + q1.w * kf[7];
      }
    }
    const uint32_t pos = b0 + (uint32_t)(c * 32 + (tid >> 3));
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float v = g4d::sum8(acc[h]);
      acc[h] = pos < b1 ? v * a.scale : -INFINITY;
    }
    if (ks == 0) {
#pragma unroll
      for (int h = 0; h < G; ++h) p_s[(c * 32 + (tid >> 3)) * G + h] = acc[h];
    }
  }
  __syncthreads();

  // ---- 5. chunk softmax statistics per head ----
  constexpr int SL = (NT / G) < 64 ? (NT / G) : 64;
  static_assert(SL == 32 || SL == 64, "head groups of 32 or 64 lanes");
  if (tid < G * SL) {
    const int h = tid / SL, sl = tid % SL;
    float mx = -INFINITY;
#pragma unroll
    for (int i = sl; i < P; i += SL) mx = fmaxf(mx, p_s[i * G + h]);
    mx = group_max<SL>(mx);
    float sum = 0.f;
#pragma unroll
    for (int i = sl; i < P; i += SL) {
      const float e = mq_exp(p_s[i * G + h] - mx);  // rows past the chunk: exp(-inf) = 0
      p_s[i * G + h] = e;
      sum += e;
    }
    sum = group_sum<SL>(sum);
    if (sl == 0) {
      stat_s[h] = mx;
      stat_s[G + h] = sum;
    }
  }
  __syncthreads();

  // ---- 6. o for this thread's columns over the chunk's rows ----
  float o[G][VD];
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int j = 0; j < VD; ++j) o[h][j] = 0.f;
#pragma unroll
  for (int r = 0; r < VR; ++r) {
    const int pi = r * VG + vgrp;
    float vf[VD];
    vf[0] = g4d::f16_bits_to_f32(vraw[r] & 0xffffu);
    if constexpr (VD == 2) vf[1] = g4d::f16_bits_to_f32(vraw[r] >> 16);
    const float4* pp = (const float4*)(p_s + pi * G);
    float pv[G];
#pragma unroll
    for (int h4 = 0; h4 < G / 4; ++h4) {
      const float4 t = pp[h4];
      pv[4 * h4] = t.x; pv[4 * h4 + 1] = t.y; pv[4 * h4 + 2] = t.z; pv[4 * h4 + 3] = t.w;
    }
    if constexpr (G % 4 != 0) {
#pragma unroll
      for (int h = (G / 4) * 4; h < G; ++h) pv[h] = p_s[pi * G + h];
    }
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int j = 0; j < VD; ++j) o[h][j] += pv[h] * vf[j];
  }
  if constexpr (VG > 1) {  // head_dim 128: two row groups per column
    if (vgrp == 1) {
#pragma unroll
      for (int h = 0; h < G; ++h) o_s[h * HD + vcol] = o[h][0];
    }
    __syncthreads();
    if (vgrp != 0) return;
#pragma unroll
    for (int h = 0; h < G; ++h) o[h][0] += o_s[h * HD + vcol];
  }
#pragma unroll
  for (int h = 0; h < G; ++h) {
    float* dst = ws_o + (part + h) * HD + vcol;
#pragma unroll
    for (int j = 0; j < VD; ++j) dst[j] = o[h][j];
  }
  if (tid < G) {
    ws_m[part + tid] = stat_s[tid];
    ws_l[part + tid] = stat_s[G + tid];
  }
}

// Merge the splits of one (sequence, query head):
// O = sum_s o_s e^(m_s - M) / sum_s l_s e^(m_s - M); empty splits (l = 0)
// drop out. MG thread groups of HD threads each take MS splits per pass with
// every load of the pass issued first (unconditional, clamped index); passes
// combine online and the groups combine through LDS at the end.
constexpr int MS = 16;

// Live length of a sequence's attention window (as attn_kernel forms it).
struct LenArgs {
  const uint32_t* seq_lens;  // paged
  const uint32_t* pos_dev;   // dense dev forms
  uint32_t seq_len;          // dense host form
  uint32_t cap, window;
};
__device__ __forceinline__ void live_window(const LenArgs& a, uint32_t seq, uint32_t& start, uint32_t& n) {
  uint32_t L = a.seq_lens ? a.seq_lens[seq] : (a.pos_dev ? *a.pos_dev + 1 : a.seq_len);
  L = min(L, a.cap);
  start = (a.window != 0 && L > a.window) ? L - a.window : 0;
  n = L - start;
}

// Splits past ceil(n / chunk) of a sequence are never read: the matrix-core
// kernel does not launch workgroups for them.
// The merged output of (sequence seq, head hq) also as the matrix-core
// operand blocks of the o projection (g4d::Ops; K = nqh * HD, so the head's
// HD dims are HD / 256 whole super-blocks): per super-block the exponent
// from the block maximum, f16 hi / lo of y * 2^e, the 3-part sub-block sums
// of y * 2^(e-6) and the scale 2^-e, what bprep_kernel writes for the same
// values. Every thread of the workgroup calls it (`live`: a thread of group 0).
template <int HD>
__device__ __forceinline__ void merge_ops(float y, bool live, uint8_t* ops, int ntv, uint32_t seq, uint32_t hq,
                                          uint32_t d) {
  __shared__ float wmax_s[16];
  const uint32_t tid = threadIdx.x;
  const float wm = g4d::wave_max_dpp(fabsf(y));
  if ((tid & 63) == 0) wmax_s[tid >> 6] = wm;
  __syncthreads();
  if (!live) return;
  const uint32_t sbl = d >> 8, e = d & 255u;  // super-block of the head, element in it
  const float am = fmaxf(fmaxf(wmax_s[4 * sbl], wmax_s[4 * sbl + 1]), fmaxf(wmax_s[4 * sbl + 2], wmax_s[4 * sbl + 3]));
  int ex = 0;
  (void)frexpf(am, &ex);
  const int k = am > 0.f ? min(max(14 - ex, -120), 120) : 0;
  const float xs = y * ldexpf(1.0f, k);
  const _Float16 hi = (_Float16)xs, lo = (_Float16)(xs - (float)hi);
  const uint32_t s = e >> 5, p = e & 31u, q = p >> 3, j = p & 7u;
  const uint32_t kb = hq * (uint32_t)(HD / 256) + sbl, t = seq >> 4, c = seq & 15u;
  uint8_t* base = ops + (size_t)kb * g4d::Ops::bytes(ntv);
  uint8_t* mp = base + t * g4d::Ops::MAIN_T + s * 2048 + (c + 16u * q) * 16 + j * 2;
  *(_Float16*)mp = hi;
  *(_Float16*)(mp + 1024) = lo;
  float sum = xs;  // over the sub-block: 32 consecutive lanes
#pragma unroll
  for (int o = 1; o < 32; o <<= 1) sum += __shfl_xor(sum, o, 32);
  if (p == 0) {
    sum *= 0.015625f;  // * 2^-6
    const _Float16 p0 = (_Float16)sum;
    const float r1 = sum - (float)p0;
    const _Float16 p1 = (_Float16)r1;
    const _Float16 p2 = (_Float16)(r1 - (float)p1);
    _Float16* sp = (_Float16*)(base + g4d::Ops::sums_off(ntv) + t * 1024 + (c + 16u * (s >> 1)) * 16 + (s & 1) * 8);
    sp[0] = p0;
    sp[1] = p1;
    sp[2] = p2;
    sp[3] = (_Float16)0.f;
  }
  if (e == 0) *(float*)(base + g4d::Ops::scale_off(ntv) + t * 64 + c * 4) = ldexpf(1.0f, -k);
}

template <int HD>
__global__ __launch_bounds__(1024) void attn_merge_kernel(const float* ws, float* out, uint32_t nqh, uint32_t nkh,
                                                          uint32_t G, uint32_t nsplit, uint32_t num_seqs,
                                                          LenArgs la, uint32_t chunk, uint8_t* ops, int ntv) {
  constexpr int MG = 1024 / HD;  // split groups (thread g*HD + d owns column d of group g)
  __shared__ float gm_s[MG], gl_s[MG];
  __shared__ float go_s[MG > 1 ? (MG - 1) * HD : 1];
  const uint32_t hq = blockIdx.x, seq = blockIdx.y;
  const uint32_t kvh = hq / G, h = hq % G;
  const size_t nparts = (size_t)num_seqs * nkh * nsplit * G;
  const float* ws_m = ws;
  const float* ws_l = ws + nparts;
  const float* ws_o = ws + 2 * nparts;
  const size_t base = ((size_t)seq * nkh + kvh) * nsplit * G + h;
  const uint32_t tid = threadIdx.x, d = tid % HD, grp = tid / HD;
  uint32_t wstart, n;
  live_window(la, seq, wstart, n);
  nsplit = min(nsplit, (n + chunk - 1) / chunk);
  float M = -INFINITY, Ls = 0.f, acc = 0.f;
  for (uint32_t s0 = grp * MS; s0 < nsplit; s0 += MG * MS) {
    float mm[MS], ll[MS], oo[MS];
#pragma unroll
    for (int u = 0; u < MS; ++u) {
      const size_t ps = base + (size_t)min(s0 + u, nsplit - 1) * G;
      mm[u] = ws_m[ps];
      ll[u] = ws_l[ps];
      oo[u] = ws_o[ps * HD + d];
    }
    float mx = -INFINITY;
#pragma unroll
    for (int u = 0; u < MS; ++u) mx = fmaxf(mx, (s0 + u < nsplit && ll[u] > 0.f) ? mm[u] : -INFINITY);
    const float nM = fmaxf(M, mx);
    const float sc = nM == -INFINITY || M == -INFINITY ? 0.f : mq_exp(M - nM);
    acc *= sc;
    Ls *= sc;
#pragma unroll
    for (int u = 0; u < MS; ++u) {
      const float wt = (s0 + u < nsplit && ll[u] > 0.f) ? mq_exp(mm[u] - nM) : 0.f;
      acc += wt * oo[u];
      Ls += wt * ll[u];
    }
    M = nM;
  }
  if (d == 0) {
    gm_s[grp] = M;
    gl_s[grp] = Ls;
  }
  if (grp > 0) go_s[(grp - 1) * HD + d] = acc;
  __syncthreads();
  if (grp != 0 && !ops) return;  // (uniform) the other groups only join the operand block's barrier
  float TM = -INFINITY;
#pragma unroll
  for (int g = 0; g < MG; ++g) TM = fmaxf(TM, gm_s[g]);
  float tl = 0.f, to = 0.f;
#pragma unroll
  for (int g = 0; g < MG; ++g) {
    const float wg = gm_s[g] == -INFINITY ? 0.f : mq_exp(gm_s[g] - TM);
    tl += wg * gl_s[g];
    to += wg * (g == 0 ? acc : go_s[(g - 1) * HD + d]);
  }
  const float y = tl > 0.f ? to / tl : 0.f;
  if (grp == 0) out[((size_t)seq * nqh + hq) * HD + d] = y;
  if (ops) merge_ops<HD>(grp == 0 ? y : 0.f, grp == 0, ops, ntv, seq, hq, d);
}

// Merge of many chunk partials (long contexts): the grid also splits each
// head's dims into slices of MW_D, so a head's partials are read by HD / MW_D
// workgroups at once instead of one. Thread t holds chunk t's (m, l) and
// thread (g, j) the o of dim d0 + j of chunks g, g + MW_G, ...; all of these
// loads are issued together, then the maximum, the weights exp(m - M) (in
// LDS) and the sums are formed, and the MW_G groups are added in LDS.
// Chunks with l == 0 are skipped, as in attn_merge_kernel.
constexpr uint32_t kMaxSplits = 1024;  // merge kernel limit; 64 * 1024 = 65536 positions
constexpr int MW_D = 32;               // dims per workgroup
constexpr int MW_G = 32;               // chunk groups
constexpr int MW_NT = MW_D * MW_G;     // threads: one (m, l) each
constexpr int MW_OU = (int)(kMaxSplits / MW_G);
constexpr uint32_t kMergeWideMin = 64;  // fewer splits merge in attn_merge_kernel
static_assert(MW_NT >= (int)kMaxSplits, "one chunk's (m, l) per thread");
template <int HD>
__global__ __launch_bounds__(MW_NT) void attn_merge_wide_kernel(const float* ws, float* out, uint32_t nqh,
                                                               uint32_t nkh, uint32_t G, uint32_t nsplit,
                                                               uint32_t num_seqs, LenArgs la, uint32_t chunk) {
  __shared__ float w_s[kMaxSplits];  // weight of each chunk
  __shared__ float red_s[2 * (MW_NT / 64)];
  __shared__ float acc_s[MW_G * (MW_D + 1)];
  const uint32_t hq = blockIdx.x, seq = blockIdx.y, d0 = blockIdx.z * MW_D;
  const uint32_t kvh = hq / G, h = hq % G;
  const size_t nparts = (size_t)num_seqs * nkh * nsplit * G;
  const float* ws_m = ws;
  const float* ws_l = ws + nparts;
  const float* ws_o = ws + 2 * nparts;
  const size_t base = ((size_t)seq * nkh + kvh) * nsplit * G + h;
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wv = tid >> 6;
  const uint32_t g = tid / MW_D, j = tid % MW_D;
  // every planned chunk's partial is loaded without waiting for the live
  // length (the workspace holds nsplit chunks); chunks past it are masked
  // afterwards by selection, so stale values never enter a sum
  float mc = -INFINITY, lc = 0.f;
  if (tid < nsplit) {
    mc = ws_m[base + (size_t)tid * G];
    lc = ws_l[base + (size_t)tid * G];
  }
  float ov[MW_OU];
#pragma unroll
  for (int u = 0; u < MW_OU; ++u) {
    const uint32_t c = g + (uint32_t)u * MW_G;
    ov[u] = c < nsplit ? ws_o[(base + (size_t)c * G) * HD + d0 + j] : 0.f;
  }
  uint32_t wstart, n;
  live_window(la, seq, wstart, n);
  const uint32_t ns = min(nsplit, (n + chunk - 1) / chunk);
#pragma unroll
  for (int u = 0; u < MW_OU; ++u)
    if (g + (uint32_t)u * MW_G >= ns) ov[u] = 0.f;
  if (tid >= ns || !(lc > 0.f)) {
    mc = -INFINITY;
    lc = 0.f;
  }
  const float wm = g4d::wave_max_dpp(mc);
  if (lane == 0) red_s[wv] = wm;
  __syncthreads();
  float M = -INFINITY;
#pragma unroll
  for (int w = 0; w < MW_NT / 64; ++w) M = fmaxf(M, red_s[w]);
  const float wt = mc == -INFINITY ? 0.f : mq_exp(mc - M);
  if (tid < kMaxSplits) w_s[tid] = wt;
  const float wl = g4d::wave_sum_dpp(wt * lc);
  if (lane == 0) red_s[MW_NT / 64 + wv] = wl;
  __syncthreads();
  float Ls = 0.f;
#pragma unroll
  for (int w = 0; w < MW_NT / 64; ++w) Ls += red_s[MW_NT / 64 + w];
  float acc = 0.f;
#pragma unroll
  for (int u = 0; u < MW_OU; ++u) acc += w_s[g + u * MW_G] * ov[u];
  acc_s[g * (MW_D + 1) + j] = acc;
  __syncthreads();
  if (g != 0) return;
  float t = 0.f;
#pragma unroll 8
  for (int gg = 0; gg < MW_G; ++gg) t += acc_s[gg * (MW_D + 1) + j];
  out[((size_t)seq * nqh + hq) * HD + d0 + j] = Ls > 0.f ? t / Ls : 0.f;
}

// ---------------------------------------------------------------------------
// matrix-core split-K decode attention: 8 query heads per KV head, head_dim 256
// ---------------------------------------------------------------------------
//
// Workgroup = (chunk of 64 * nstep consecutive positions of one sequence's
// window, KV head); workgroups are numbered over the sequences' live chunks
// only. Each step stages 64 positions of K and V in LDS (rows padded to
// 528 B so that the 16 rows an MFMA operand reads fall on different banks)
// while the next step's rows are loaded; wave w takes positions
// 16w .. 16w+15 of the step:
//  * scores: v_mfma_f32_16x16x32_f16 with A = 16 K rows x 32 dims and
//    B = 16 columns holding q_hi (columns 0-7) and q_lo (8-15) of the 8 heads,
//    so S[pos][h] = D[pos][h] + D[pos][h + 8] (one DPP row rotate by 8).
//  * online softmax per head over the wave's positions (running m, l).
//  * PV: v_mfma_f32_16x16x16_f16 with A = rows (p_hi | p_lo) x 16 positions,
//    which is exactly the layout the score MFMA left p in, and B = 4
//    positions x 16 dims of V; 16 dim tiles.
// At the end the four waves' (m, l, o) are combined in LDS and one partial
// per head is written for attn_merge_kernel.

struct MqArgs {
  const float* q;  // [num_seqs][nqh][256]
  const uint16_t* kc;
  const uint16_t* vc;
  const int32_t* page_table;  // paged: [num_seqs][max_pages]
  uint32_t page_size, max_pages, num_pages;
  LenArgs len;
  uint32_t num_seqs, nqh, nkh;
  float scale;
  uint32_t nstep;       // steps per workgroup
  uint32_t max_chunks;  // partial slots per (sequence, KV head)
  float* ws;
};

constexpr int kMqPages = 96;  // page-table entries of a chunk held in LDS (1024 positions of 16-row pages)

template <bool PAGED>
__global__ __launch_bounds__(NT, 2) void mq_attn_kernel(MqArgs a) {
  __shared__ __align__(16) _Float16 kt[MQ_STEP * MQ_RS];
  __shared__ __align__(16) _Float16 vt[MQ_STEP * MQ_RS];
  __shared__ uint32_t s_seq, s_chunk;
  __shared__ int32_t s_pg[kMqPages];
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, q = l >> 4, c = l & 15;
  const uint32_t kvh = blockIdx.y;
  const uint32_t CH = MQ_STEP * a.nstep;

  // ---- this workgroup's (sequence, chunk) in the order of live chunks ----
  if (w == 0) {
    uint32_t nch = 0;
    if ((uint32_t)l < a.num_seqs) {
      uint32_t st, n;
      live_window(a.len, (uint32_t)l, st, n);
      nch = (n + CH - 1) / CH;
    }
    uint32_t incl = nch;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint32_t t = __shfl_up(incl, o, 64);
      if (l >= o) incl += t;
    }
    const unsigned long long hit = __ballot(incl > blockIdx.x);
    const int sq = hit ? __ffsll(hit) - 1 : 0;
    const uint32_t before = __shfl(incl - nch, sq, 64);
    if (l == 0) {
      s_seq = hit ? (uint32_t)sq : 0xffffffffu;
      s_chunk = blockIdx.x - before;
    }
  }
  __syncthreads();
  const uint32_t seq = s_seq;
  if (seq == 0xffffffffu) return;  // past the last live chunk (uniform)
  const uint32_t chunk = s_chunk;
  uint32_t wstart, n;
  live_window(a.len, seq, wstart, n);
  const uint32_t c0 = chunk * CH;          // chunk start within the window
  const uint32_t cend = min(n, c0 + CH);   // > c0
  const uint32_t last = wstart + cend - 1; // last live position of the chunk
  const uint32_t nst = (cend - c0 + MQ_STEP - 1) / MQ_STEP;

  // PAGED: the chunk's page-table entries, clamped to the pool, in LDS (when
  // they fit), so that a step's row loads do not wait on a page-table load
  const uint32_t fpg = PAGED ? (wstart + c0) / a.page_size : 0u;
  const uint32_t npg = PAGED ? last / a.page_size - fpg + 1 : 0u;
  const bool pg_lds = PAGED && npg <= (uint32_t)kMqPages;  // (uniform)
  if constexpr (PAGED) {
    if (pg_lds && (uint32_t)tid < npg) {
      const int32_t pg = a.page_table[(size_t)seq * a.max_pages + fpg + tid];
      s_pg[tid] = pg < 0 ? 0 : (pg >= (int32_t)a.num_pages ? (int32_t)a.num_pages - 1 : pg);
    }
    __syncthreads();
  }
  auto row_of = [&](uint32_t pos) -> size_t {
    if constexpr (PAGED) {
      int32_t pg;
      if (pg_lds) {
        pg = s_pg[pos / a.page_size - fpg];
      } else {
        pg = a.page_table[(size_t)seq * a.max_pages + pos / a.page_size];
        pg = pg < 0 ? 0 : (pg >= (int32_t)a.num_pages ? (int32_t)a.num_pages - 1 : pg);
      }
      return (size_t)pg * a.page_size + pos % a.page_size;
    }
    return pos;
  };
  // K (pieces 0-7) and V (8-15) of one step: piece tid + 256i covers row
  // (tid + 256i) / 32 % 64, dims 8 * (tid % 32) .. +7; rows past the chunk
  // repeat its last live position (masked in the scores)
  mu4 pf[16];
  auto load_step = [&](uint32_t st) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const uint32_t pc = (uint32_t)tid + 256u * (uint32_t)(i & 7);
      const uint32_t r = pc >> 5, col = (pc & 31) * 8;
      const uint32_t pos = min(wstart + c0 + st * MQ_STEP + r, last);
      const uint16_t* base = i < 8 ? a.kc : a.vc;
      pf[i] = *(const mu4*)(base + (row_of(pos) * a.nkh + kvh) * MQ_HD + col);
    }
  };
  auto store_step = [&]() {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const uint32_t pc = (uint32_t)tid + 256u * (uint32_t)(i & 7);
      const uint32_t r = pc >> 5, col = (pc & 31) * 8;
      _Float16* dst = (i < 8 ? kt : vt) + r * MQ_RS + col;
      *(mu4*)dst = pf[i];
    }
  };

  load_step(0);
  // q as the scores' B operand: column c = (part c/8, head c%8), dims 32j + 8q .. +7
  const float* qg = a.q + ((size_t)seq * a.nqh + kvh * MQ_G + (c & 7)) * MQ_HD;
  float4 qr[16];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    qr[2 * j] = *(const float4*)(qg + 32 * j + 8 * q);
    qr[2 * j + 1] = *(const float4*)(qg + 32 * j + 8 * q + 4);
  }
  mh8 qb[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float xs[8] = {qr[2 * j].x, qr[2 * j].y, qr[2 * j].z, qr[2 * j].w,
                         qr[2 * j + 1].x, qr[2 * j + 1].y, qr[2 * j + 1].z, qr[2 * j + 1].w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const _Float16 hi = (_Float16)xs[e];
      qb[j][e] = c < 8 ? hi : (_Float16)(xs[e] - (float)hi);
    }
  }
  store_step();
  __syncthreads();

  mf4 O[16];
#pragma unroll
  for (int dt = 0; dt < 16; ++dt) O[dt] = mf4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;  // of head c % 8

  for (uint32_t st = 0; st < nst; ++st) {
    const bool more = st + 1 < nst;
    load_step(more ? st + 1 : st);  // the next step's rows are in flight during this one

    // ---- scores of the wave's 16 positions ----
    mf4 S = mf4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const mh8 A = *(const mh8*)(kt + (16 * w + c) * MQ_RS + 32 * j + 8 * q);
      S = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, qb[j], S, 0, 0, 0);
    }
    float sc[4];
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float v = S[i] + g4d::dpp<kDppRor8>(S[i]);  // q_hi + q_lo columns
      const uint32_t off = c0 + st * MQ_STEP + 16u * w + 4u * q + i;
      sc[i] = off < cend ? v * a.scale : -INFINITY;
      mx = fmaxf(mx, sc[i]);
    }
    mx = g4d::xmax16(mx);
    mx = g4d::xmax32(mx);
    const float m_new = fmaxf(m_run, mx);
    const float alpha = m_new == -INFINITY ? 1.f : mq_exp(m_run - m_new);
    float p[4], ps = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      p[i] = sc[i] == -INFINITY ? 0.f : mq_exp(sc[i] - m_new);
      ps += p[i];
    }
    ps = g4d::xsum16(ps);
    ps = g4d::xsum32(ps);
    l_run = l_run * alpha + ps;
    m_run = m_new;
    // rows of O held here: 4q + i = (part, head 4(q&1) + i)
    float ar[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float a0 = g4d::lane_value(alpha, i), a1 = g4d::lane_value(alpha, 4 + i);
      ar[i] = (q & 1) ? a1 : a0;
    }
    mh4 P;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const _Float16 hi = (_Float16)p[i];
      P[i] = c < 8 ? hi : (_Float16)(p[i] - (float)hi);
    }
#pragma unroll
    for (int dt = 0; dt < 16; ++dt) {
      mh4 Bv;
#pragma unroll
      for (int i = 0; i < 4; ++i) Bv[i] = vt[(16 * w + 4 * q + i) * MQ_RS + 16 * dt + c];
      mf4 o = O[dt];
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] *= ar[i];
      O[dt] = __builtin_amdgcn_mfma_f32_16x16x16f16(P, Bv, o, 0, 0, 0);
    }
    __syncthreads();  // every wave is done with this step's rows
    if (more) {
      store_step();
      __syncthreads();
    }
  }

  // ---- combine the hi and lo rows, then the four waves ----
#pragma unroll
  for (int dt = 0; dt < 16; ++dt)
#pragma unroll
    for (int i = 0; i < 4; ++i) O[dt][i] = g4d::xsum32(O[dt][i]);
  float* ow = (float*)kt;                 // [4 waves][8 heads][256]
  float* mw = (float*)vt;                 // [4][8]
  float* lw = mw + 32;                    // [4][8]
  if (q < 2) {
#pragma unroll
    for (int dt = 0; dt < 16; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) ow[(w * MQ_G + 4 * q + i) * MQ_HD + 16 * dt + c] = O[dt][i];
  }
  if (q == 0 && c < MQ_G) {
    mw[w * MQ_G + c] = m_run;
    lw[w * MQ_G + c] = l_run;
  }
  __syncthreads();
  const size_t part = (((size_t)seq * a.nkh + kvh) * a.max_chunks + chunk) * MQ_G;
  const size_t nparts = (size_t)a.num_seqs * a.nkh * a.max_chunks * MQ_G;
  float* ws_m = a.ws;
  float* ws_l = ws_m + nparts;
  float* ws_o = ws_m + 2 * nparts;
#pragma unroll
  for (int h = 0; h < MQ_G; ++h) {
    float M = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < 4; ++ww) M = fmaxf(M, mw[ww * MQ_G + h]);
    float L = 0.f, o = 0.f;
#pragma unroll
    for (int ww = 0; ww < 4; ++ww) {
      const float m = mw[ww * MQ_G + h];
      const float wt = m == -INFINITY ? 0.f : mq_exp(m - M);
      L += wt * lw[ww * MQ_G + h];
      o += wt * ow[(ww * MQ_G + h) * MQ_HD + tid];
    }
    ws_o[(part + h) * MQ_HD + tid] = o;
    if (tid == 0) {
      ws_m[part + h] = M;
      ws_l[part + h] = L;
    }
  }
}

// The paged batch's whole attention block in one launch (g4_pagedAttnBlock):
// workgroup (chunk, sequence, KV head).
__global__ __launch_bounds__(NT, 2) void pmqf_kernel(MqfArgs a) {
  mqf_body<false, false, true, MQ_HD, true>(a, blockIdx.x, blockIdx.z, blockIdx.x, blockIdx.y);
}

// The fused block as a launch of its own (blockIdx.y = KV head), for head
// dim 256 (256 threads) or 512 (512 threads).
template <bool LONG, int HD>
__global__ __launch_bounds__(HD, 512 / HD) void mqf_kernel(MqfArgs a) {
  mqf_body<LONG, false, !LONG, HD>(a, blockIdx.x, blockIdx.y, blockIdx.x);
}


// RoPE table: (cos, sin) of every position and pair, rope_cos_sin's values.
__global__ __launch_bounds__(NT) void rope_table_kernel(float2* out, float theta, uint32_t apply_divisor,
                                                        const uint16_t* rope_freqs, uint32_t hd, uint32_t rows) {
  const uint32_t half = hd / 2;
  const size_t e = (size_t)blockIdx.x * NT + threadIdx.x;
  if (e >= (size_t)rows * half) return;
  const uint32_t i = (uint32_t)(e % half), pos = (uint32_t)(e / half);
  out[e] = rope_cos_sin(theta, apply_divisor, apply_divisor ? rope_freqs[i] : (uint16_t)0, i, hd, pos);
}

// ---------------------------------------------------------------------------
// paged prologue (multi-sequence step): per sequence, the q/k/v projections
// (sums of split-K partials, added in chunk order) through q_norm + RoPE,
// k_norm + RoPE and the weightless v_norm, the f16 K/V row appended to the
// pool (src/engine.ts:1556-1570 per sequence). Workgroup (head, sequence):
// heads [0, nqh) are query heads, [nqh, nqh + nkh) the K/V heads; thread t
// owns the RoPE pair (t, t + hd/2).
// ---------------------------------------------------------------------------
struct ProArgs {
  const float* q;  // [nparts][num_seqs][nqh * hd]
  const float* k;  // [nparts][num_seqs][nkh * hd]
  const float* v;
  uint32_t nparts, num_seqs, nqh, nkh, hd;
  const uint16_t* q_w;
  const uint16_t* k_w;
  const uint16_t* rope_freqs;
  float theta;
  uint32_t apply_divisor;
  float eps;
  float* q_out;  // [num_seqs][nqh * hd]
  uint16_t* kp;
  uint16_t* vp;
  const int32_t* page_table;
  const uint32_t* seq_lens;
  uint32_t page_size, max_pages, num_pages, cap;
  const float2* rope_cs;  // [cap][hd/2] (cos, sin) of every position (g4_ropeTable), or null
};

// Elements i0 and i1 summed over the n partials in chunk order; the loads of
// up to 8 chunks are issued together.
__device__ __forceinline__ float2 sum_parts2(const float* base, size_t stride, uint32_t n, uint32_t i0,
                                             uint32_t i1) {
  float a = 0.f, b = 0.f;
  for (uint32_t c0 = 0; c0 < n; c0 += 8) {
    float ta[8], tb[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const size_t c = min(c0 + (uint32_t)i, n - 1);
      ta[i] = base[c * stride + i0];
      tb[i] = base[c * stride + i1];
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (c0 + i < n) {
        a += ta[i];
        b += tb[i];
      }
  }
  return make_float2(a, b);
}

__global__ __launch_bounds__(NT) void attn_prologue_kernel(ProArgs a) {
  __shared__ float red[8];
  const uint32_t head = blockIdx.x, seq = blockIdx.y;
  const uint32_t t = threadIdx.x, half = a.hd / 2;
  const bool on = t < half;
  const uint32_t tc = on ? t : 0;
  const bool is_q = head < a.nqh;
  const uint32_t kvh = is_q ? 0 : head - a.nqh;
  const uint32_t L = a.seq_lens[seq];
  const uint32_t Lc = min(L, a.cap);
  const uint32_t pos = Lc > 0 ? Lc - 1 : 0;
  float2 x, y = make_float2(0.f, 0.f);
  if (is_q) {
    const size_t stride = (size_t)a.num_seqs * a.nqh * a.hd;
    const float* b = a.q + ((size_t)seq * a.nqh + head) * a.hd;
    x = sum_parts2(b, stride, a.nparts, tc, tc + half);
  } else {
    const size_t stride = (size_t)a.num_seqs * a.nkh * a.hd;
    const size_t off = ((size_t)seq * a.nkh + kvh) * a.hd;
    x = sum_parts2(a.k + off, stride, a.nparts, tc, tc + half);
    y = sum_parts2(a.v + off, stride, a.nparts, tc, tc + half);
  }
  if (!on) x = y = make_float2(0.f, 0.f);
  // sums of squares: x in red[0..3], y in red[4..7]
  const float sx = g4d::wave_sum_dpp(x.x * x.x + x.y * x.y);
  const float sy = g4d::wave_sum_dpp(y.x * y.x + y.y * y.y);
  if ((t & 63) == 0) {
    red[t >> 6] = sx;
    red[4 + (t >> 6)] = sy;
  }
  __syncthreads();
  const float tx = (red[0] + red[1]) + (red[2] + red[3]);
  const float ty = (red[4] + red[5]) + (red[6] + red[7]);
  const float invx = __builtin_amdgcn_rsqf(tx * (1.0f / (float)a.hd) + a.eps);
  const float invy = __builtin_amdgcn_rsqf(ty * (1.0f / (float)a.hd) + a.eps);
  if (!on) return;
  const uint16_t* wn = is_q ? a.q_w : a.k_w;
  float x0 = x.x * g4d::f16_bits_to_f32(wn[t]) * invx;
  float x1 = x.y * g4d::f16_bits_to_f32(wn[t + half]) * invx;
  // RoPE (rope_cos_sin), from the table when there is one
  const float2 cs = a.rope_cs ? a.rope_cs[(size_t)pos * half + t]
                              : rope_cos_sin(a.theta, a.apply_divisor, a.rope_freqs[t], t, a.hd, pos);
  const float cn = cs.x, sn = cs.y;
  const float r0 = x0 * cn - x1 * sn, r1 = x0 * sn + x1 * cn;
  if (is_q) {
    float* o = a.q_out + ((size_t)seq * a.nqh + head) * a.hd;
    o[t] = r0;
    o[t + half] = r1;
    return;
  }
  // append at pos when the length is in range and the page id is in the pool
  if (L == 0 || L > a.cap) return;
  const int32_t pg = a.page_table[(size_t)seq * a.max_pages + pos / a.page_size];
  if (pg < 0 || pg >= (int32_t)a.num_pages) return;
  const size_t row = ((size_t)pg * a.page_size + pos % a.page_size) * a.nkh + kvh;
  uint16_t* kd = a.kp + row * a.hd;
  uint16_t* vd = a.vp + row * a.hd;
  kd[t] = g4d::f32_to_f16_bits(r0);
  kd[t + half] = g4d::f32_to_f16_bits(r1);
  vd[t] = g4d::f32_to_f16_bits(y.x * invy);
  vd[t + half] = g4d::f32_to_f16_bits(y.y * invy);
}

// ---------------------------------------------------------------------------
// paged KV append: row for position seq_lens[s]-1 of each sequence
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(NT) void paged_store_kernel(const float* k_in, const float* v_in, uint16_t* kp,
                                                         uint16_t* vp, const int32_t* page_table,
                                                         const uint32_t* seq_lens, uint32_t total,
                                                         uint32_t page_size, uint32_t max_pages,
                                                         uint32_t num_pages) {
  const uint32_t s = blockIdx.y;
  const uint32_t i = blockIdx.x * NT + threadIdx.x;
  if (i >= total) return;
  const uint32_t L = seq_lens[s];
  if (L == 0 || (L - 1) / page_size >= max_pages) return;
  const uint32_t pos = L - 1;
  const int32_t pg = page_table[(size_t)s * max_pages + pos / page_size];
  if (pg < 0 || pg >= (int32_t)num_pages) return;  // a bad page id writes nothing
  const size_t row = (size_t)pg * page_size + pos % page_size;
  kp[row * total + i] = g4d::f32_to_f16_bits(k_in[(size_t)s * total + i]);
  vp[row * total + i] = g4d::f32_to_f16_bits(v_in[(size_t)s * total + i]);
}

// ---------------------------------------------------------------------------
// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------


struct SplitPlan {
  int cp;           // 32-position blocks per split (1 or 2)
  uint32_t chunk;   // positions per split
  uint32_t nsplit;
};

// 32-position splits up to 16K positions (at most 512 splits), 64-position
// splits beyond.
SplitPlan plan_splits(uint32_t l_eff) {
  SplitPlan p;
  if (l_eff == 0) l_eff = 1;
  p.cp = l_eff <= 16384 ? 1 : 2;
  p.chunk = 32u * (uint32_t)p.cp;
  p.nsplit = ceil_div(l_eff, p.chunk);
  return p;
}

uint32_t eff_len(uint32_t seq_len, uint32_t window) {
  return (window != 0 && seq_len > window) ? window : seq_len;
}

template <int G, int HD, bool PAGED, bool FUSE>
int launch_hd(g4_ctx* ctx, const AttnArgs& a, int cp, dim3 grid) {
  if (cp == 1) hipLaunchKernelGGL((attn_kernel<G, HD, 1, PAGED, FUSE>), grid, dim3(NT), 0, ctx->stream, a);
  else hipLaunchKernelGGL((attn_kernel<G, HD, 2, PAGED, FUSE>), grid, dim3(NT), 0, ctx->stream, a);
  G4_LAUNCHED(ctx, "attn_decode");
  return G4_OK;
}

template <bool PAGED, bool FUSE>
int launch_attn(g4_ctx* ctx, const AttnArgs& a, uint32_t G, uint32_t hd, int cp, dim3 grid) {
#define G4_ATTN_CASE(g, h) \
  if (G == g && hd == h) return launch_hd<g, h, PAGED, FUSE>(ctx, a, cp, grid);
  G4_ATTN_CASE(8, 256)
  G4_ATTN_CASE(8, 512)
  if constexpr (!FUSE) {
    G4_ATTN_CASE(8, 128)
    G4_ATTN_CASE(4, 256)
    G4_ATTN_CASE(4, 512)
    G4_ATTN_CASE(4, 128)
    G4_ATTN_CASE(2, 256)
    G4_ATTN_CASE(2, 128)
    G4_ATTN_CASE(1, 256)
    G4_ATTN_CASE(1, 128)
  }
#undef G4_ATTN_CASE
  return g4::set_error(G4_ERR_UNSUPPORTED, "attention: %u query heads per kv head with head_dim %u not built", G,
                       hd);
}

// Fused single-sequence plan: one 64-position step per workgroup. Up to
// MQF_FAN chunks the last workgroup to arrive merges them in the launch
// (one level of the merge tree); beyond, the workgroups store their
// partials and end, and a merge launch combines them (two dependent
// device-scope round trips per tree level cost more than a launch boundary,
// and the merge launch spreads each head's partials over many workgroups).
// Past kMaxSplits chunks a workgroup takes several steps. The arrival
// counters and the staged q/k/v sit in the first kMqfCnt bytes of the
// workspace, at the same place whatever the plan, so that layers of
// different windows can share one workspace; the chunk partials follow,
// then the group partials.
struct MqfPlan {
  uint32_t nstep, max_chunks;  // 64-position steps per workgroup, workgroups
  bool partials;  // chunk partials + a merge launch
  size_t bytes_ws0, bytes;
};
MqfPlan mqf_plan(const g4_attn_fused_params& p) {
  MqfPlan m{};
  const uint32_t eff = std::max(eff_len(p.max_seq_len, p.sliding_window), 1u);
  m.partials = ceil_div(eff, MQ_STEP) > MQF_FAN;
  // two steps per workgroup past 16K positions (fewer partials to merge;
  // measured 1.2 us faster at 32K)
  m.nstep = m.partials ? std::max(eff > 16384 ? 2u : 1u, ceil_div(eff, MQ_STEP * kMaxSplits)) : 1u;
  m.max_chunks = ceil_div(eff, MQ_STEP * m.nstep);
  const uint32_t hd = p.head_dim == 512 ? 512u : (uint32_t)MQ_HD;
  m.bytes_ws0 = ws_bytes(1, p.num_kv_heads, m.max_chunks, MQ_G, hd);
  m.bytes = kMqfCnt + m.bytes_ws0 + (m.partials ? 0 : ws_bytes(1, p.num_kv_heads, MQF_FAN, MQ_G, hd));
  return m;
}

LenArgs len_args(const AttnArgs& a) { return LenArgs{a.seq_lens, a.pos_dev, a.seq_len, a.cap, a.window}; }

int merge_launch(g4_ctx* ctx, const float* ws, float* out, uint32_t nqh, uint32_t nkh, uint32_t G, uint32_t hd,
                 uint32_t nsplit, uint32_t num_seqs, const LenArgs& la, uint32_t chunk, uint8_t* ops = nullptr) {
  if (!ops && nsplit >= kMergeWideMin && nsplit <= kMaxSplits) {
    const dim3 wg(nqh, num_seqs, hd / MW_D);
    switch (hd) {
      case 128:
        hipLaunchKernelGGL(attn_merge_wide_kernel<128>, wg, dim3(MW_D * MW_G), 0, ctx->stream, ws, out, nqh, nkh, G,
                           nsplit, num_seqs, la, chunk);
        break;
      case 256:
        hipLaunchKernelGGL(attn_merge_wide_kernel<256>, wg, dim3(MW_D * MW_G), 0, ctx->stream, ws, out, nqh, nkh, G,
                           nsplit, num_seqs, la, chunk);
        break;
      default:
        hipLaunchKernelGGL(attn_merge_wide_kernel<512>, wg, dim3(MW_D * MW_G), 0, ctx->stream, ws, out, nqh, nkh, G,
                           nsplit, num_seqs, la, chunk);
        break;
    }
    G4_LAUNCHED(ctx, "attn_merge_wide");
    return G4_OK;
  }
  const int ntv = (int)(g4d::pad_batch(num_seqs) / 16);
  const dim3 mg(nqh, num_seqs);
  switch (hd) {
    case 128:
      hipLaunchKernelGGL(attn_merge_kernel<128>, mg, dim3(1024), 0, ctx->stream, ws, out, nqh, nkh, G, nsplit,
                         num_seqs, la, chunk, ops, ntv);
      break;
    case 256:
      hipLaunchKernelGGL(attn_merge_kernel<256>, mg, dim3(1024), 0, ctx->stream, ws, out, nqh, nkh, G, nsplit,
                         num_seqs, la, chunk, ops, ntv);
      break;
    default:
      hipLaunchKernelGGL(attn_merge_kernel<512>, mg, dim3(1024), 0, ctx->stream, ws, out, nqh, nkh, G, nsplit,
                         num_seqs, la, chunk, ops, ntv);
      break;
  }
  G4_LAUNCHED(ctx, "attn_merge");
  return G4_OK;
}

int merge(g4_ctx* ctx, const AttnArgs& a, float* out, const SplitPlan& sp, uint32_t num_seqs, uint32_t G,
          uint32_t hd, uint8_t* ops = nullptr) {
  return merge_launch(ctx, a.ws, out, a.nqh, a.nkh, G, hd, sp.nsplit, num_seqs, len_args(a), sp.chunk, ops);
}

// The matrix-core kernel serves the paged batch: 8 query heads per KV head at
// head_dim 256 and up to 64 sequences (its chunk numbering runs in one wave).
// One dense sequence takes the VALU form (attn_kernel), measured faster on
// its own at every context of the single-sequence shape (8 query heads,
// 1 KV head x 256: 9.0 against 11.8 us at 512 positions, 11.2 against
// 13.9 at 4096, 20.7 against 21.5 at 32768); in the decode step the fused
// form (mqf_kernel) keeps the matrix cores.
bool mq_fits(uint32_t G, uint32_t hd, uint32_t num_seqs) { return G == 8 && hd == 256 && num_seqs <= 64; }

// Steps per workgroup from the largest window, sized for about four
// workgroups per CU when every sequence is that long.
int mq_decode(g4_ctx* ctx, const char* fn, const AttnArgs& base, uint32_t num_seqs, float* out, size_t ws_len,
              uint8_t* ops = nullptr) {
  const uint32_t eff = eff_len(base.cap, base.window);
  const uint64_t cus = ctx->num_cus > 0 ? (uint64_t)ctx->num_cus : 256;
  const uint64_t want = ((uint64_t)num_seqs * eff + 64 * 4 * cus - 1) / (64 * 4 * cus);
  const uint32_t nstep = (uint32_t)std::min<uint64_t>(std::max<uint64_t>(want, 1), 16);
  const uint32_t chunk = MQ_STEP * nstep;
  const uint32_t max_chunks = ceil_div(eff == 0 ? 1 : eff, chunk);
  const size_t need = ws_bytes(num_seqs, base.nkh, max_chunks, MQ_G, MQ_HD);
  G4_REQUIRE(ws_len >= need, "%s: workspace %zu bytes < %zu required", fn, ws_len, need);
  MqArgs m{};
  m.q = base.q;
  m.kc = base.kc;
  m.vc = base.vc;
  m.page_table = base.page_table;
  m.page_size = base.page_size;
  m.max_pages = base.max_pages;
  m.num_pages = base.num_pages;
  m.len = len_args(base);
  m.num_seqs = num_seqs;
  m.nqh = base.nqh;
  m.nkh = base.nkh;
  m.scale = base.scale;
  m.nstep = nstep;
  m.max_chunks = max_chunks;
  m.ws = base.ws;
  const dim3 grid(num_seqs * max_chunks, base.nkh);
  hipLaunchKernelGGL(mq_attn_kernel<true>, grid, dim3(NT), 0, ctx->stream, m);
  G4_LAUNCHED(ctx, "attn_decode_mfma");
  return merge_launch(ctx, base.ws, out, base.nqh, base.nkh, MQ_G, MQ_HD, max_chunks, num_seqs, m.len, chunk, ops);
}

int check_heads(const char* fn, uint32_t nqh, uint32_t nkh, uint32_t hd) {
  G4_REQUIRE(nqh > 0 && nkh > 0 && nqh % nkh == 0 && nqh / nkh <= 8,
             "%s: num_q_heads %u must be a multiple (<= 8x) of num_kv_heads %u", fn, nqh, nkh);
  G4_REQUIRE(hd == 128 || hd == 256 || hd == 512, "%s: head_dim %u not in {128, 256, 512}", fn, hd);
  return G4_OK;
}

}  // namespace

namespace g4mqf {
int mqf_check(g4_ctx* ctx, const char* fn, const float* q_raw, const float* k_raw, const float* v_raw,
              const uint16_t* q_norm_w, const uint16_t* k_norm_w, const uint16_t* rope_freqs, uint16_t* k_cache,
              uint16_t* v_cache, float* output, const g4_attn_fused_params& p, void* workspace,
              const uint32_t* position_dev, const g4_warm_region* regions, int nregions, const float* rope_cs,
              uint32_t rope_rows) {
  (void)ctx;
  G4_REQUIRE(!rope_cs || rope_rows >= p.max_seq_len, "g4_attnDecodeFusedWarm: RoPE table of %u rows < max_seq_len %u",
             rope_rows, p.max_seq_len);
  G4_REQUIRE(q_raw && q_norm_w && k_cache && v_cache && output && workspace && position_dev,
             "g4_attnDecodeFused: null buffer");
  // k_raw = v_raw = k_norm_w = null: the caches already hold this position's
  // row (a layer reading its producer layer's cache)
  G4_REQUIRE(k_raw ? (v_raw && k_norm_w) : (!v_raw && !k_norm_w),
             "g4_attnDecodeFused: k_raw, v_raw and k_norm_w are all given or all null");
  G4_REQUIRE(nregions >= 0 && nregions <= kMaxWarm && (nregions == 0 || regions),
             "g4_attnDecodeFusedWarm: 0..%d warm regions", kMaxWarm);
  for (int i = 0; i < nregions; ++i) {
    const g4_warm_region& r = regions[i];
    // (below 4 GiB - 4 KiB: the kernel's out-of-range reads use offset 0xfffffff0)
    G4_REQUIRE(r.base && r.total_bytes > 0 && r.total_bytes <= 0xfffff000ull && r.wg_bytes > 0 && r.nwgs > 0 &&
                   r.wg_bytes * (uint64_t)r.nwgs <= 0xfffff000ull,
               "g4_attnDecodeFusedWarm: region %d empty or beyond 4 GiB - 4 KiB", i);
  }
  G4_REQUIRE(!p.apply_divisor || rope_freqs, "g4_attnDecodeFused: apply_divisor needs rope_freqs");
  G4_REQUIRE(((uintptr_t)k_cache & 15) == 0 && ((uintptr_t)v_cache & 15) == 0 && ((uintptr_t)workspace & 15) == 0,
             "g4_attnDecodeFused: KV caches and workspace must be 16-byte aligned");
  int rc = check_heads(fn, p.num_q_heads, p.num_kv_heads, p.head_dim);
  if (rc) return rc;
  G4_REQUIRE(p.max_seq_len > 0, "g4_attnDecodeFused: max_seq_len must be >= 1");
  G4_REQUIRE(p.num_q_heads == 8 * p.num_kv_heads && (p.head_dim == 256 || p.head_dim == 512),
             "g4_attnDecodeFused: built for 8 query heads per kv head and head_dim 256/512");
  return G4_OK;
}

int mqf_prepare(g4_ctx* ctx, const float* q_raw, const float* k_raw, const float* v_raw, const uint16_t* q_norm_w,
                const uint16_t* k_norm_w, const uint16_t* rope_freqs, uint16_t* k_cache, uint16_t* v_cache,
                float* output, const g4_attn_fused_params& p, void* workspace, size_t workspace_bytes,
                const uint32_t* position_dev, const g4_warm_region* regions, int nregions, const float* rope_cs,
                uint32_t busy_extra, bool& applies, MqfLaunch& L) {
  applies = (p.head_dim == 256 || p.head_dim == 512) && p.num_q_heads == MQ_G * p.num_kv_heads &&
            p.num_kv_heads <= kMqfMaxKvHeads &&
            ((uintptr_t)q_norm_w & 15) == 0 && eff_len(p.max_seq_len, p.sliding_window) <= 4 * MQ_STEP * MQF_FAN * MQF_FAN;
  if (!applies) return G4_OK;
  const MqfPlan mp = mqf_plan(p);
  G4_REQUIRE(workspace_bytes >= mp.bytes, "g4_attnDecodeFused: workspace %zu bytes < %zu required", workspace_bytes,
             mp.bytes);
  MqfArgs& m = L.m;
  m = MqfArgs{};
  m.q_raw = q_raw;
  m.k_raw = k_raw;
  m.v_raw = v_raw;
  m.q_w = q_norm_w;
  m.k_w = k_norm_w;
  m.rope_freqs = rope_freqs ? rope_freqs : q_norm_w;  // read unconditionally, used only with the divisor
  m.theta = p.theta;
  m.apply_divisor = p.apply_divisor;
  m.eps = p.eps;
  m.kc = k_cache;
  m.vc = v_cache;
  m.pos_dev = position_dev;
  m.cap = p.max_seq_len;
  m.nqh = p.num_q_heads;
  m.nkh = p.num_kv_heads;
  m.scale = p.scale;
  m.window = p.sliding_window;
  m.nstep = mp.nstep;
  m.max_chunks = mp.max_chunks;
  m.ws = (float*)((uint8_t*)workspace + kMqfCnt);
  m.ws1 = (float*)((uint8_t*)workspace + kMqfCnt + mp.bytes_ws0);
  m.cnt = (uint32_t*)workspace;
  m.out = output;
  m.rope_cs = (const float2*)rope_cs;
  // warming workgroups on the CUs the attention leaves idle, a multiple
  // of 8 so that every XCD gets as many. A launch that warms asks for
  // kWarmLds more LDS per workgroup, so no two of its workgroups share a
  // CU: a warming workgroup next to an attention one slowed it by 1 us.
  const uint32_t busy = mp.max_chunks * p.num_kv_heads + busy_extra;
  const uint32_t idle = (uint32_t)ctx->num_cus > busy ? (uint32_t)ctx->num_cus - busy : 0u;
  m.nwarm = nregions ? idle / 8u * 8u : 0u;
  m.nwarm_regions = m.nwarm ? (uint32_t)nregions : 0u;
  for (int i = 0; i < (int)m.nwarm_regions; ++i) {
    m.wbase[i] = (const uint8_t*)regions[i].base;
    m.wtotal[i] = (uint32_t)regions[i].total_bytes;
    m.wwgb[i] = (uint32_t)regions[i].wg_bytes;
    m.wnwg[i] = regions[i].nwgs;
  }
  m.stage = (uint64_t*)((uint8_t*)workspace + kMqfCntOnly);
  m.nstage = 0;
  m.spin = ctx->test_spin ? ctx->test_spin : kStageSpin;
  m.status = ctx->status_dev;
  m.num_seqs = 1;
  L.partials = mp.partials;
  return G4_OK;
}
}  // namespace g4mqf

namespace {

int check_plan(const char* fn, const SplitPlan& sp) {
  G4_REQUIRE(sp.nsplit <= kMaxSplits, "%s: %u positions exceed the %u-position limit of one decode call", fn,
             sp.nsplit * sp.chunk, kMaxSplits * 64);
  return G4_OK;
}

AttnArgs dense_args(const float* q, const uint16_t* kc, const uint16_t* vc, uint32_t nqh, uint32_t nkh,
                    uint32_t seq_len, float scale, uint32_t window, const SplitPlan& sp, void* ws,
                    const uint32_t* pos_dev) {
  AttnArgs a{};
  a.q = q;
  a.kc = kc;
  a.vc = vc;
  a.pos_dev = pos_dev;
  a.seq_len = seq_len;
  a.cap = seq_len;
  a.nqh = nqh;
  a.nkh = nkh;
  a.scale = scale;
  a.window = window;
  a.chunk = sp.chunk;
  a.nsplit = sp.nsplit;
  a.ws = (float*)ws;
  return a;
}

int dense_decode(g4_ctx* ctx, const char* fn, const float* q, const uint16_t* kc, const uint16_t* vc, float* out,
                 g4_attn_score_params p, void* ws, size_t ws_len, const uint32_t* pos_dev) {
  G4_REQUIRE(q && kc && vc && out && ws, "%s: null buffer", fn);
  G4_REQUIRE(((uintptr_t)kc & 15) == 0 && ((uintptr_t)vc & 15) == 0 && ((uintptr_t)ws & 15) == 0,
             "%s: KV caches and workspace must be 16-byte aligned", fn);
  int rc = check_heads(fn, p.num_q_heads, p.num_kv_heads, p.head_dim);
  if (rc) return rc;
  G4_REQUIRE(p.seq_len > 0, "%s: seq_len must be >= 1", fn);
  const uint32_t G = p.num_q_heads / p.num_kv_heads;
  const SplitPlan sp = plan_splits(eff_len(p.seq_len, p.sliding_window));
  rc = check_plan(fn, sp);
  if (rc) return rc;
  const size_t need = ws_bytes(1, p.num_kv_heads, sp.nsplit, G, p.head_dim);
  G4_REQUIRE(ws_len >= need, "%s: workspace %zu bytes < %zu required", fn, ws_len, need);
  const AttnArgs a = dense_args(q, kc, vc, p.num_q_heads, p.num_kv_heads, p.seq_len, p.scale, p.sliding_window,
                                sp, ws, pos_dev);
  rc = launch_attn<false, false>(ctx, a, G, p.head_dim, sp.cp, dim3(sp.nsplit, p.num_kv_heads, 1));
  if (rc) return rc;
  return merge(ctx, a, out, sp, 1, G, p.head_dim);
}

g4_paged_attn_params fused_attn_part(const g4_paged_attn_fused_params& f) {
  g4_paged_attn_params p{};
  p.num_seqs = f.num_seqs;
  p.num_q_heads = f.num_q_heads;
  p.num_kv_heads = f.num_kv_heads;
  p.head_dim = f.head_dim;
  p.page_size = f.page_size;
  p.max_pages = f.max_pages;
  p.max_seq_len = f.max_seq_len;
  p.num_pages = f.num_pages;
  p.scale = f.scale;
  p.sliding_window = f.sliding_window;
  return p;
}

// Shape checks and the kernel arguments shared by the paged entry points.
int paged_setup(const char* fn, const uint16_t* k_pool, const uint16_t* v_pool, const int32_t* page_table,
                const uint32_t* seq_lens, const g4_paged_attn_params& p, void* ws, size_t ws_len, AttnArgs& a,
                SplitPlan& sp) {
  G4_REQUIRE(((uintptr_t)k_pool & 15) == 0 && ((uintptr_t)v_pool & 15) == 0 && ((uintptr_t)ws & 15) == 0,
             "%s: KV pools and workspace must be 16-byte aligned", fn);
  int rc = check_heads(fn, p.num_q_heads, p.num_kv_heads, p.head_dim);
  if (rc) return rc;
  G4_REQUIRE(p.num_seqs > 0 && p.page_size > 0 && p.max_pages > 0 && p.num_pages > 0,
             "%s: empty batch or pages", fn);
  G4_REQUIRE(p.num_seqs <= 65535, "%s: %u sequences exceed the grid limit 65535", fn, p.num_seqs);
  G4_REQUIRE(p.max_seq_len > 0 && (uint64_t)p.max_seq_len <= (uint64_t)p.page_size * p.max_pages,
             "%s: max_seq_len %u exceeds the page table (%u x %u)", fn, p.max_seq_len, p.max_pages, p.page_size);
  sp = plan_splits(eff_len(p.max_seq_len, p.sliding_window));
  rc = check_plan(fn, sp);
  if (rc) return rc;
  const size_t need = ws_bytes(p.num_seqs, p.num_kv_heads, sp.nsplit, p.num_q_heads / p.num_kv_heads, p.head_dim);
  G4_REQUIRE(ws_len >= need, "%s: workspace %zu bytes < %zu required", fn, ws_len, need);
  a = AttnArgs{};
  a.kc = k_pool;
  a.vc = v_pool;
  a.page_table = page_table;
  a.page_size = p.page_size;
  a.max_pages = p.max_pages;
  a.num_pages = p.num_pages;
  a.cap = p.max_seq_len;
  a.seq_lens = seq_lens;
  a.nqh = p.num_q_heads;
  a.nkh = p.num_kv_heads;
  a.scale = p.scale;
  a.window = p.sliding_window;
  a.chunk = sp.chunk;
  a.nsplit = sp.nsplit;
  a.ws = (float*)ws;
  return G4_OK;
}

// Partials of g4_attnDecode_noalloc: a file-scope device array instead of a
// caller workspace, for callers that cannot allocate (code under graph
// capture, serving loops that forbid hipMalloc). Each GPU the library runs
// on holds its own copy for the life of the process. Host code never passes
// the array's name to a kernel (on the host it is a stand-in, not a device
// address): g4_init looks up the device address on its device and keeps it
// in the context. Every split writes its partial before the merge launch
// reads it, so nothing in the array has to start at zero; calls on one GPU
// share the array, so calls that overlap (other streams) race.
constexpr size_t kNoAllocScratchBytes = 16u << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

}  // namespace

void g4_internal_noalloc_init(g4_ctx* ctx) {
  void* ptr = nullptr;
  const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  ctx->noalloc_status = (int)e;
  ctx->noalloc_scratch = e == hipSuccess ? ptr : nullptr;
  if (e != hipSuccess) (void)hipGetLastError();  // leave no sticky error for the next call
}

extern "C" {

int g4_attnScore_dev(g4_ctx* ctx, const float* q, const uint16_t* k_cache, float* scores, g4_attn_score_params p,
                     const uint32_t* position_dev) {
  G4_ENTER(ctx);
  G4_REQUIRE(q && k_cache && scores, "g4_attnScore: null buffer");
  G4_REQUIRE(p.num_q_heads > 0 && p.num_kv_heads > 0 && p.head_dim > 0, "g4_attnScore: empty shape");
  if (!p.seq_len) return G4_OK;
  hipLaunchKernelGGL(attn_score_kernel, dim3(ceil_div(p.seq_len, 4)), dim3(NT), 0, ctx->stream, q, k_cache, scores,
                     p.num_q_heads, p.num_kv_heads, p.head_dim, p.seq_len, p.scale, p.sliding_window, position_dev);
  G4_LAUNCHED(ctx, "attn_score");
  return G4_OK;
}

int g4_attnScore(g4_ctx* ctx, const float* q, const uint16_t* k_cache, float* scores, g4_attn_score_params p) {
  return g4_attnScore_dev(ctx, q, k_cache, scores, p, nullptr);
}

int g4_softmax_dev(g4_ctx* ctx, float* scores, g4_softmax_params p, const uint32_t* position_dev) {
  G4_ENTER(ctx);
  G4_REQUIRE(scores, "g4_softmax: null buffer");
  if (!p.num_heads || !p.seq_len) return G4_OK;
  hipLaunchKernelGGL(softmax_kernel, dim3(p.num_heads), dim3(NT), 0, ctx->stream, scores, p.num_heads, p.seq_len,
                     position_dev);
  G4_LAUNCHED(ctx, "softmax");
  return G4_OK;
}

int g4_softmax(g4_ctx* ctx, float* scores, g4_softmax_params p) { return g4_softmax_dev(ctx, scores, p, nullptr); }

int g4_attnOutput_dev(g4_ctx* ctx, const float* probs, const uint16_t* v_cache, float* output,
                      g4_attn_output_params p, const uint32_t* position_dev) {
  G4_ENTER(ctx);
  G4_REQUIRE(probs && v_cache && output, "g4_attnOutput: null buffer");
  G4_REQUIRE(p.num_q_heads > 0 && p.num_kv_heads > 0 && p.head_dim > 0, "g4_attnOutput: empty shape");
  hipLaunchKernelGGL(attn_output_kernel, dim3(ceil_div(p.num_q_heads * p.head_dim, NT)), dim3(NT), 0, ctx->stream,
                     probs, v_cache, output, p.num_q_heads, p.num_kv_heads, p.head_dim, p.seq_len, position_dev);
  G4_LAUNCHED(ctx, "attn_output");
  return G4_OK;
}

int g4_attnOutput(g4_ctx* ctx, const float* probs, const uint16_t* v_cache, float* output, g4_attn_output_params p) {
  return g4_attnOutput_dev(ctx, probs, v_cache, output, p, nullptr);
}

int g4_attnDecode_workspace_size(g4_attn_score_params p, size_t* bytes) {
  G4_REQUIRE(bytes, "g4_attnDecode_workspace_size: null out");
  int rc = check_heads(__func__, p.num_q_heads, p.num_kv_heads, p.head_dim);
  if (rc) return rc;
  const SplitPlan sp = plan_splits(eff_len(p.seq_len, p.sliding_window));
  rc = check_plan(__func__, sp);
  if (rc) return rc;
  *bytes = ws_bytes(1, p.num_kv_heads, sp.nsplit, p.num_q_heads / p.num_kv_heads, p.head_dim);
  return G4_OK;
}

int g4_attnDecode(g4_ctx* ctx, const float* q, const uint16_t* k_cache, const uint16_t* v_cache, float* output,
                  g4_attn_score_params p, void* workspace, size_t workspace_bytes) {
  G4_ENTER(ctx);
  return dense_decode(ctx, __func__, q, k_cache, v_cache, output, p, workspace, workspace_bytes, nullptr);
}

int g4_attnDecode_noalloc(g4_ctx* ctx, const float* q, const uint16_t* k_cache, const uint16_t* v_cache,
                          float* output, g4_attn_score_params p) {
  G4_ENTER(ctx);
  if (!ctx->noalloc_scratch)
    return g4::set_error(G4_ERR_HIP, "g4_attnDecode_noalloc: no device address for the static scratch (%s)",
                         hipGetErrorString((hipError_t)ctx->noalloc_status));
  size_t need = 0;
  const int rc = g4_attnDecode_workspace_size(p, &need);
  if (rc) return rc;
  G4_REQUIRE(need <= kNoAllocScratchBytes,
             "g4_attnDecode_noalloc: this shape needs %zu bytes of partials, more than the %zu-byte static "
             "scratch (use g4_attnDecode with a workspace)",
             need, kNoAllocScratchBytes);
  return dense_decode(ctx, __func__, q, k_cache, v_cache, output, p, ctx->noalloc_scratch, kNoAllocScratchBytes,
                      nullptr);
}

int g4_attnDecode_dev(g4_ctx* ctx, const float* q, const uint16_t* k_cache, const uint16_t* v_cache, float* output,
                      g4_attn_score_params p, void* workspace, size_t workspace_bytes, const uint32_t* position_dev) {
  G4_ENTER(ctx);
  G4_REQUIRE(position_dev, "g4_attnDecode_dev: null position");
  // p.seq_len is the capacity; the split plan covers it, and splits past the
  // live length exit after writing an empty partial.
  return dense_decode(ctx, __func__, q, k_cache, v_cache, output, p, workspace, workspace_bytes, position_dev);
}

int g4_ropeTable(g4_ctx* ctx, float theta, uint32_t apply_divisor, const uint16_t* rope_freqs, uint32_t head_dim,
                 uint32_t rows, float* table) {
  G4_ENTER(ctx);
  G4_REQUIRE(table && rows > 0 && head_dim >= 2 && head_dim % 2 == 0 && head_dim <= 1024,
             "g4_ropeTable: null table or bad shape (rows %u, head_dim %u)", rows, head_dim);
  G4_REQUIRE(!apply_divisor || rope_freqs, "g4_ropeTable: apply_divisor needs rope_freqs");
  G4_REQUIRE(((uintptr_t)table & 7) == 0, "g4_ropeTable: table must be 8-byte aligned");
  const size_t n = (size_t)rows * (head_dim / 2);
  hipLaunchKernelGGL(rope_table_kernel, dim3(ceil_div(n, NT)), dim3(NT), 0, ctx->stream, (float2*)table, theta,
                     apply_divisor, rope_freqs, head_dim, rows);
  G4_LAUNCHED(ctx, "rope_table");
  return G4_OK;
}

int g4_attnDecodeFused_workspace_size(g4_attn_fused_params p, size_t* bytes) {
  G4_REQUIRE(bytes, "g4_attnDecodeFused_workspace_size: null out");
  int rc = check_heads(__func__, p.num_q_heads, p.num_kv_heads, p.head_dim);
  if (rc) return rc;
  const SplitPlan sp = plan_splits(eff_len(p.max_seq_len, p.sliding_window));
  rc = check_plan(__func__, sp);
  if (rc) return rc;
  // both forms keep the first kMqfCnt bytes for the one-launch form's
  // counters, so layers of either form can share a workspace
  const size_t old = ws_bytes(1, p.num_kv_heads, sp.nsplit, p.num_q_heads / p.num_kv_heads, p.head_dim);
  *bytes = std::max(kMqfCnt + old, mqf_plan(p).bytes);
  return G4_OK;
}

int g4_attnDecodeFused(g4_ctx* ctx, const float* q_raw, const float* k_raw, const float* v_raw,
                       const uint16_t* q_norm_w, const uint16_t* k_norm_w, const uint16_t* rope_freqs,
                       uint16_t* k_cache, uint16_t* v_cache, float* output, g4_attn_fused_params p, void* workspace,
                       size_t workspace_bytes, const uint32_t* position_dev) {
  return g4_attnDecodeFusedWarm(ctx, q_raw, k_raw, v_raw, q_norm_w, k_norm_w, rope_freqs, k_cache, v_cache, output, p,
                                workspace, workspace_bytes, position_dev, nullptr, 0, nullptr, 0);
}

int g4_attnDecodeFusedWarm(g4_ctx* ctx, const float* q_raw, const float* k_raw, const float* v_raw,
                           const uint16_t* q_norm_w, const uint16_t* k_norm_w, const uint16_t* rope_freqs,
                           uint16_t* k_cache, uint16_t* v_cache, float* output, g4_attn_fused_params p,
                           void* workspace, size_t workspace_bytes, const uint32_t* position_dev,
                           const g4_warm_region* regions, int nregions, const float* rope_cs,
                           uint32_t rope_rows) {
  G4_ENTER(ctx);
  int rc = mqf_check(ctx, "g4_attnDecodeFusedWarm", q_raw, k_raw, v_raw, q_norm_w, k_norm_w, rope_freqs, k_cache,
                     v_cache, output, p, workspace, position_dev, regions, nregions, rope_cs, rope_rows);
  if (rc) return rc;
  const uint32_t G = p.num_q_heads / p.num_kv_heads;
  bool one_launch = false;
  MqfLaunch L{};
  rc = mqf_prepare(ctx, q_raw, k_raw, v_raw, q_norm_w, k_norm_w, rope_freqs, k_cache, v_cache, output, p, workspace,
                   workspace_bytes, position_dev, regions, nregions, rope_cs, 0, one_launch, L);
  if (rc) return rc;
  if (one_launch) {
    const MqfArgs& m = L.m;
    const dim3 grid(m.max_chunks + m.nwarm, p.num_kv_heads);
    if (p.head_dim == 512) {  // (its LDS already keeps one workgroup per CU)
      if (L.partials) hipLaunchKernelGGL((mqf_kernel<true, 512>), grid, dim3(512), 0, ctx->stream, m);
      else hipLaunchKernelGGL((mqf_kernel<false, 512>), grid, dim3(512), 0, ctx->stream, m);
    } else {
      const size_t lds = m.nwarm ? kWarmLds : 0;
      if (L.partials) hipLaunchKernelGGL((mqf_kernel<true, 256>), grid, dim3(NT), lds, ctx->stream, m);
      else hipLaunchKernelGGL((mqf_kernel<false, 256>), grid, dim3(NT), lds, ctx->stream, m);
    }
    G4_LAUNCHED(ctx, "attn_decode_fused_mfma");
    if (!L.partials) return G4_OK;
    const LenArgs la{nullptr, position_dev, p.max_seq_len, p.max_seq_len, p.sliding_window};
    return merge_launch(ctx, m.ws, output, p.num_q_heads, p.num_kv_heads, MQ_G, p.head_dim, m.max_chunks, 1, la,
                        MQ_STEP * m.nstep);
  }
  // (the two-launch form computes the RoPE per call: a table is not needed)
  const SplitPlan sp = plan_splits(eff_len(p.max_seq_len, p.sliding_window));
  rc = check_plan(__func__, sp);
  if (rc) return rc;
  const size_t need = kMqfCnt + ws_bytes(1, p.num_kv_heads, sp.nsplit, G, p.head_dim);
  G4_REQUIRE(workspace_bytes >= need, "g4_attnDecodeFused: workspace %zu bytes < %zu required", workspace_bytes,
             need);
  AttnArgs a = dense_args(q_raw, k_cache, v_cache, p.num_q_heads, p.num_kv_heads, p.max_seq_len, p.scale,
                          p.sliding_window, sp, (uint8_t*)workspace + kMqfCnt, position_dev);
  a.kc_w = k_cache;
  a.vc_w = v_cache;
  a.k_in = k_raw;
  a.v_in = v_raw;
  a.q_w = q_norm_w;
  a.k_w = k_norm_w;
  // the kernel reads the table unconditionally; without the divisor any
  // valid buffer of >= head_dim/2 halves serves (the value is unused)
  a.rope_freqs = rope_freqs ? rope_freqs : q_norm_w;
  a.theta = p.theta;
  a.apply_divisor = p.apply_divisor;
  a.eps = p.eps;
  rc = launch_attn<false, true>(ctx, a, G, p.head_dim, sp.cp, dim3(sp.nsplit, p.num_kv_heads, 1));
  if (rc) return rc;
  return merge(ctx, a, output, sp, 1, G, p.head_dim);
}

int g4_pagedAttnDecode_workspace_size(g4_paged_attn_params p, size_t* bytes) {
  G4_REQUIRE(bytes, "g4_pagedAttnDecode_workspace_size: null out");
  int rc = check_heads(__func__, p.num_q_heads, p.num_kv_heads, p.head_dim);
  if (rc) return rc;
  const SplitPlan sp = plan_splits(eff_len(p.max_seq_len, p.sliding_window));
  rc = check_plan(__func__, sp);
  if (rc) return rc;
  *bytes = ws_bytes(p.num_seqs, p.num_kv_heads, sp.nsplit, p.num_q_heads / p.num_kv_heads, p.head_dim);
  return G4_OK;
}

int g4_pagedAttnDecodeOps(g4_ctx* ctx, const float* q, const uint16_t* k_pool, const uint16_t* v_pool,
                          const int32_t* page_table, const uint32_t* seq_lens, float* output,
                          g4_paged_attn_params p, void* workspace, size_t workspace_bytes, void* ops) {
  G4_ENTER(ctx);
  G4_REQUIRE(q && k_pool && v_pool && page_table && seq_lens && output && workspace,
             "g4_pagedAttnDecode: null buffer");
  G4_REQUIRE(!ops || (p.head_dim % 256 == 0 && p.num_seqs <= 64 && ((uintptr_t)ops & 15) == 0),
             "g4_pagedAttnDecodeOps: operand blocks need head_dim a multiple of 256, <= 64 sequences and a "
             "16-byte aligned buffer");
  AttnArgs a{};
  SplitPlan sp{};
  int rc = paged_setup(__func__, k_pool, v_pool, page_table, seq_lens, p, workspace, workspace_bytes, a, sp);
  if (rc) return rc;
  a.q = q;
  if (mq_fits(p.num_q_heads / p.num_kv_heads, p.head_dim, p.num_seqs))
    return mq_decode(ctx, __func__, a, p.num_seqs, output, workspace_bytes, (uint8_t*)ops);
  rc = launch_attn<true, false>(ctx, a, p.num_q_heads / p.num_kv_heads, p.head_dim, sp.cp,
                                dim3(sp.nsplit, p.num_kv_heads, p.num_seqs));
  if (rc) return rc;
  return merge(ctx, a, output, sp, p.num_seqs, p.num_q_heads / p.num_kv_heads, p.head_dim, (uint8_t*)ops);
}

int g4_pagedAttnDecode(g4_ctx* ctx, const float* q, const uint16_t* k_pool, const uint16_t* v_pool,
                       const int32_t* page_table, const uint32_t* seq_lens, float* output, g4_paged_attn_params p,
                       void* workspace, size_t workspace_bytes) {
  return g4_pagedAttnDecodeOps(ctx, q, k_pool, v_pool, page_table, seq_lens, output, p, workspace, workspace_bytes,
                               nullptr);
}

int g4_pagedAttnDecodeFused_workspace_size(g4_paged_attn_fused_params p, size_t* bytes) {
  return g4_pagedAttnDecode_workspace_size(fused_attn_part(p), bytes);
}

int g4_pagedAttnDecodeFused(g4_ctx* ctx, const float* q_raw, const float* k_raw, const float* v_raw,
                            const uint16_t* q_norm_w, const uint16_t* k_norm_w, const uint16_t* rope_freqs,
                            uint16_t* k_pool, uint16_t* v_pool, const int32_t* page_table, const uint32_t* seq_lens,
                            float* output, g4_paged_attn_fused_params p, void* workspace, size_t workspace_bytes) {
  G4_ENTER(ctx);
  G4_REQUIRE(q_raw && q_norm_w && k_pool && v_pool && page_table && seq_lens && output && workspace,
             "g4_pagedAttnDecodeFused: null buffer");
  G4_REQUIRE(k_raw ? (v_raw && k_norm_w) : (!v_raw && !k_norm_w),
             "g4_pagedAttnDecodeFused: k_raw, v_raw and k_norm_w are all given or all null");
  G4_REQUIRE(!p.apply_divisor || rope_freqs, "g4_pagedAttnDecodeFused: apply_divisor needs rope_freqs");
  const g4_paged_attn_params ap = fused_attn_part(p);
  AttnArgs a{};
  SplitPlan sp{};
  int rc = paged_setup(__func__, k_pool, v_pool, page_table, seq_lens, ap, workspace, workspace_bytes, a, sp);
  if (rc) return rc;
  const uint32_t G = p.num_q_heads / p.num_kv_heads;
  G4_REQUIRE(G == 8 && (p.head_dim == 256 || p.head_dim == 512),
             "g4_pagedAttnDecodeFused: built for 8 query heads per kv head and head_dim 256/512");
  a.q = q_raw;
  a.kc_w = k_pool;
  a.vc_w = v_pool;
  a.k_in = k_raw;
  a.v_in = v_raw;
  a.q_w = q_norm_w;
  a.k_w = k_norm_w;
  a.rope_freqs = rope_freqs ? rope_freqs : q_norm_w;  // read unconditionally, used only with the divisor
  a.theta = p.theta;
  a.apply_divisor = p.apply_divisor;
  a.eps = p.eps;
  rc = launch_attn<true, true>(ctx, a, G, p.head_dim, sp.cp, dim3(sp.nsplit, p.num_kv_heads, p.num_seqs));
  if (rc) return rc;
  return merge(ctx, a, output, sp, p.num_seqs, G, p.head_dim);
}

int g4_pagedAttnPrologue(g4_ctx* ctx, const float* q_parts, const float* k_parts, const float* v_parts,
                         uint32_t nparts, const uint16_t* q_norm_w, const uint16_t* k_norm_w,
                         const uint16_t* rope_freqs, float* q_out, uint16_t* k_pool, uint16_t* v_pool,
                         const int32_t* page_table, const uint32_t* seq_lens, g4_paged_attn_fused_params p,
                         const float* rope_cs, uint32_t rope_rows) {
  G4_ENTER(ctx);
  G4_REQUIRE(!rope_cs || rope_rows >= p.max_seq_len, "g4_pagedAttnPrologue: RoPE table of %u rows < max_seq_len %u",
             rope_rows, p.max_seq_len);
  G4_REQUIRE(q_parts && q_norm_w && q_out && page_table && seq_lens && nparts >= 1,
             "g4_pagedAttnPrologue: null buffer or no parts");
  // k_parts = v_parts = null: q only (a layer reading its producer layer's
  // pool appends no row); the pools and k_norm_w are then not used
  const bool kv = k_parts != nullptr;
  G4_REQUIRE(kv ? (v_parts && k_norm_w && k_pool && v_pool) : !v_parts,
             "g4_pagedAttnPrologue: k_parts, v_parts, k_norm_w and the pools go together");
  G4_REQUIRE(((uintptr_t)rope_cs & 7) == 0, "g4_pagedAttnPrologue: rope_cs must be 8-byte aligned");
  G4_REQUIRE(!p.apply_divisor || rope_freqs, "g4_pagedAttnPrologue: apply_divisor needs rope_freqs");
  G4_REQUIRE(p.num_seqs > 0 && p.num_seqs <= 65535 && p.num_q_heads > 0 && p.num_kv_heads > 0,
             "g4_pagedAttnPrologue: empty batch or heads");
  G4_REQUIRE(p.head_dim >= 2 && p.head_dim <= 2 * NT && p.head_dim % 2 == 0,
             "g4_pagedAttnPrologue: head_dim %u must be even and <= %d", p.head_dim, 2 * NT);
  G4_REQUIRE(p.page_size > 0 && p.max_pages > 0 && p.num_pages > 0 && p.max_seq_len > 0 &&
                 (uint64_t)p.max_seq_len <= (uint64_t)p.page_size * p.max_pages,
             "g4_pagedAttnPrologue: max_seq_len %u exceeds the page table (%u x %u)", p.max_seq_len, p.max_pages,
             p.page_size);
  ProArgs a{};
  a.q = q_parts;
  a.k = k_parts;
  a.v = v_parts;
  a.nparts = nparts;
  a.num_seqs = p.num_seqs;
  a.nqh = p.num_q_heads;
  a.nkh = p.num_kv_heads;
  a.hd = p.head_dim;
  a.q_w = q_norm_w;
  a.k_w = k_norm_w;
  a.rope_freqs = rope_freqs ? rope_freqs : q_norm_w;
  a.theta = p.theta;
  a.apply_divisor = p.apply_divisor;
  a.eps = p.eps;
  a.q_out = q_out;
  a.kp = k_pool;
  a.vp = v_pool;
  a.page_table = page_table;
  a.seq_lens = seq_lens;
  a.page_size = p.page_size;
  a.max_pages = p.max_pages;
  a.num_pages = p.num_pages;
  a.cap = p.max_seq_len;
  a.rope_cs = (const float2*)rope_cs;
  hipLaunchKernelGGL(attn_prologue_kernel, dim3(p.num_q_heads + (kv ? p.num_kv_heads : 0u), p.num_seqs), dim3(NT), 0,
                     ctx->stream, a);
  G4_LAUNCHED(ctx, "attn_prologue");
  return G4_OK;
}

// g4_pagedAttnBlock: the one-launch plan (pmqf_kernel) when the window takes
// at most MQF_FAN chunks of MQ_STEP positions at head dim 256, else
// g4_pagedAttnPrologue then g4_pagedAttnDecodeOps. Workspace: the arrival
// counters [num_seqs][nkh][MQF_CNT] (zero between calls), then the chunk
// partials, or q_out (when the caller gives none) and the decode's
// workspace.
namespace {
size_t block_cnt_bytes(const g4_paged_attn_fused_params& p) {
  return ((size_t)p.num_seqs * p.num_kv_heads * g4mqf::MQF_CNT * sizeof(uint32_t) + 255) / 256 * 256;
}
bool block_one_launch(const g4_paged_attn_fused_params& p, uint32_t nparts) {
  const uint32_t eff = std::max(eff_len(p.max_seq_len, p.sliding_window), 1u);
  return p.head_dim == MQ_HD && p.num_q_heads == MQ_G * p.num_kv_heads && p.num_seqs <= 64 &&
         nparts <= (uint32_t)g4mqf::kMaxParts && ceil_div(eff, MQ_STEP) <= g4mqf::MQF_FAN;
}
}  // namespace

int g4_pagedAttnBlock_workspace_size(g4_paged_attn_fused_params p, uint32_t nparts, size_t* bytes) {
  G4_REQUIRE(bytes, "g4_pagedAttnBlock_workspace_size: null out");
  size_t dec = 0;
  int rc = g4_pagedAttnDecode_workspace_size(fused_attn_part(p), &dec);
  if (rc) return rc;
  const size_t qo = ((size_t)p.num_seqs * p.num_q_heads * p.head_dim * sizeof(float) + 255) / 256 * 256;
  size_t body = qo + dec;
  if (block_one_launch(p, nparts)) {
    const uint32_t eff = std::max(eff_len(p.max_seq_len, p.sliding_window), 1u);
    body = std::max(body, ws_bytes(p.num_seqs, p.num_kv_heads, ceil_div(eff, MQ_STEP), MQ_G, MQ_HD));
  }
  *bytes = block_cnt_bytes(p) + body;
  return G4_OK;
}

int g4_pagedAttnBlock(g4_ctx* ctx, const float* q_parts, const float* k_parts, const float* v_parts, uint32_t nparts,
                      const uint16_t* q_norm_w, const uint16_t* k_norm_w, const uint16_t* rope_freqs, float* q_out,
                      uint16_t* k_pool, uint16_t* v_pool, const int32_t* page_table, const uint32_t* seq_lens,
                      float* output, void* ops, g4_paged_attn_fused_params p, void* workspace,
                      size_t workspace_bytes, const float* rope_cs, uint32_t rope_rows) {
  G4_ENTER(ctx);
  G4_REQUIRE(output && workspace && k_pool && v_pool, "g4_pagedAttnBlock: null buffer");
  G4_REQUIRE(((uintptr_t)workspace & 15) == 0, "g4_pagedAttnBlock: the workspace must be 16-byte aligned");
  G4_REQUIRE(!ops || (p.head_dim % 256 == 0 && p.num_seqs <= 64 && ((uintptr_t)ops & 15) == 0),
             "g4_pagedAttnBlock: operand blocks need head_dim a multiple of 256, <= 64 sequences and a 16-byte "
             "aligned buffer");
  size_t need = 0;
  int rc = g4_pagedAttnBlock_workspace_size(p, nparts, &need);
  if (rc) return rc;
  G4_REQUIRE(workspace_bytes >= need, "g4_pagedAttnBlock: workspace %zu bytes < %zu required", workspace_bytes, need);
  const size_t cb = block_cnt_bytes(p);
  uint8_t* body = (uint8_t*)workspace + cb;
  if (!block_one_launch(p, nparts) || ((uintptr_t)q_norm_w & 15) != 0) {
    float* qo = q_out;
    size_t used = 0;
    if (!qo) {
      qo = (float*)body;
      used = ((size_t)p.num_seqs * p.num_q_heads * p.head_dim * sizeof(float) + 255) / 256 * 256;
    }
    rc = g4_pagedAttnPrologue(ctx, q_parts, k_parts, v_parts, nparts, q_norm_w, k_norm_w, rope_freqs, qo, k_pool,
                              v_pool, page_table, seq_lens, p, rope_cs, rope_rows);
    if (rc) return rc;
    return g4_pagedAttnDecodeOps(ctx, qo, k_pool, v_pool, page_table, seq_lens, output, fused_attn_part(p),
                                 body + used, workspace_bytes - cb - used, ops);
  }
  // the prologue's argument rules, then the one launch
  G4_REQUIRE(!rope_cs || rope_rows >= p.max_seq_len, "g4_pagedAttnBlock: RoPE table of %u rows < max_seq_len %u",
             rope_rows, p.max_seq_len);
  G4_REQUIRE(q_parts && q_norm_w && page_table && seq_lens && nparts >= 1, "g4_pagedAttnBlock: null buffer or no parts");
  const bool kv = k_parts != nullptr;
  G4_REQUIRE(kv ? (v_parts && k_norm_w) : !v_parts, "g4_pagedAttnBlock: k_parts, v_parts and k_norm_w go together");
  G4_REQUIRE(((uintptr_t)rope_cs & 7) == 0, "g4_pagedAttnBlock: rope_cs must be 8-byte aligned");
  G4_REQUIRE(!p.apply_divisor || rope_freqs, "g4_pagedAttnBlock: apply_divisor needs rope_freqs");
  G4_REQUIRE(p.num_seqs > 0 && p.page_size > 0 && p.max_pages > 0 && p.num_pages > 0 && p.max_seq_len > 0 &&
                 (uint64_t)p.max_seq_len <= (uint64_t)p.page_size * p.max_pages,
             "g4_pagedAttnBlock: max_seq_len %u exceeds the page table (%u x %u)", p.max_seq_len, p.max_pages,
             p.page_size);
  G4_REQUIRE(((uintptr_t)q_parts & 15) == 0 && ((uintptr_t)k_pool & 15) == 0 && ((uintptr_t)v_pool & 15) == 0,
             "g4_pagedAttnBlock: q partials and pools must be 16-byte aligned");
  const uint32_t eff = std::max(eff_len(p.max_seq_len, p.sliding_window), 1u);
  MqfArgs m{};
  m.q_raw = q_parts;
  m.k_raw = k_parts;
  m.v_raw = v_parts;
  m.q_w = q_norm_w;
  m.k_w = k_norm_w;
  m.rope_freqs = rope_freqs ? rope_freqs : q_norm_w;  // read unconditionally, used only with the divisor
  m.theta = p.theta;
  m.apply_divisor = p.apply_divisor;
  m.eps = p.eps;
  m.kc = k_pool;
  m.vc = v_pool;
  m.cap = p.max_seq_len;
  m.nqh = p.num_q_heads;
  m.nkh = p.num_kv_heads;
  m.scale = p.scale;
  m.window = p.sliding_window;
  m.nstep = 1;
  m.max_chunks = ceil_div(eff, MQ_STEP);
  m.ws = (float*)body;
  m.cnt = (uint32_t*)workspace;
  m.out = output;
  m.rope_cs = (const float2*)rope_cs;
  m.status = ctx->status_dev;
  m.page_table = page_table;
  m.seq_lens = seq_lens;
  m.page_size = p.page_size;
  m.max_pages = p.max_pages;
  m.num_pages = p.num_pages;
  m.num_seqs = p.num_seqs;
  m.nparts = nparts;
  m.q_out = q_out;
  m.ops = (uint8_t*)ops;
  m.ntv = (int)(g4d::pad_batch(p.num_seqs) / 16);
  hipLaunchKernelGGL(pmqf_kernel, dim3(m.max_chunks, p.num_seqs, p.num_kv_heads), dim3(NT), 0, ctx->stream, m);
  G4_LAUNCHED(ctx, "paged_attn_block");
  return G4_OK;
}

int g4_pagedKvStore(g4_ctx* ctx, const float* k_in, const float* v_in, uint16_t* k_pool, uint16_t* v_pool,
                    const int32_t* page_table, const uint32_t* seq_lens, g4_paged_attn_params p) {
  G4_ENTER(ctx);
  G4_REQUIRE(k_in && v_in && k_pool && v_pool && page_table && seq_lens, "g4_pagedKvStore: null buffer");
  G4_REQUIRE(p.num_seqs > 0 && p.page_size > 0, "g4_pagedKvStore: empty batch");
  const uint32_t total = p.num_kv_heads * p.head_dim;
  if (!total) return G4_OK;
  G4_REQUIRE(p.num_pages > 0, "g4_pagedKvStore: empty pool");
  hipLaunchKernelGGL(paged_store_kernel, dim3(ceil_div(total, NT), p.num_seqs), dim3(NT), 0, ctx->stream, k_in, v_in,
                     k_pool, v_pool, page_table, seq_lens, total, p.page_size, p.max_pages, p.num_pages);
  G4_LAUNCHED(ctx, "paged_kv_store");
  return G4_OK;
}

}  // extern "C"
