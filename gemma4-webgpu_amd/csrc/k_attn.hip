// k_attn.hip — GQA decode attention over an f16 KV cache.
//
// Two forms of the same computation (shaders/attn_score.wgsl,
// shaders/softmax.wgsl, shaders/attn_output.wgsl; scale 1.0, sliding window
// W masks positions < seq_len - W):
//  * the per-key trio attnScore -> softmax -> attnOutput, kept so that every
//    reference kernel has a drop-in (scores round-trip through HBM);
//  * split-K flash-decode: workgroup (split, kv head[, sequence]) streams a
//    chunk of K/V rows once for all G = NQH/NKH query heads of that KV head,
//    keeps a running (max, sum, o) per head, and a combine kernel merges the
//    splits with a log-sum-exp rescale. The paged form addresses rows through
//    a per-sequence page table (ragged multi-sequence batches).
#include <math.h>

#include "g4_internal.hpp"

namespace {

constexpr int NT = 256;
constexpr float kMasked = -1e30f;

// ---------------------------------------------------------------------------
// the trio
// ---------------------------------------------------------------------------

// One wave per position: lanes stride the head dimension (coalesced row
// reads), one wave reduction per query head.
__global__ __launch_bounds__(NT) void attn_score_kernel(const float* q, const uint16_t* kc, float* scores,
                                                        uint32_t nqh, uint32_t nkh, uint32_t hd,
                                                        uint32_t seq_len, float scale, uint32_t window) {
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
__global__ __launch_bounds__(NT) void softmax_kernel(float* scores, uint32_t num_heads, uint32_t seq_len) {
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

// Thread per (head, d); the position loop is split across blockIdx.y slabs
// whose partial sums are added in a fixed order by the last pass.
__global__ __launch_bounds__(NT) void attn_output_kernel(const float* probs, const uint16_t* vc, float* out,
                                                         uint32_t nqh, uint32_t nkh, uint32_t hd,
                                                         uint32_t seq_len) {
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

struct AttnArgs {
  const float* q;            // [num_seqs][nqh][hd]
  const uint16_t* kc;        // cache [max_seq][nkh][hd] or pool [rows][nkh][hd]
  const uint16_t* vc;
  const int32_t* page_table; // paged: [num_seqs][max_pages]
  uint32_t page_size, max_pages, num_pages;
  const uint32_t* seq_lens;  // paged: per sequence
  const uint32_t* pos_dev;   // dense dev variant: seq_len = *pos_dev + 1
  uint32_t seq_len;          // dense: the length (host variant) or the cache capacity (dev variant)
  uint32_t cap;              // positions addressable (lengths are clamped to it)
  uint32_t nqh, nkh;
  float scale;
  uint32_t window;
  uint32_t chunk;            // positions per split (multiple of the pass size)
  uint32_t nsplit;           // splits per (sequence, kv head)
  float* ws;                 // partials
};

// workspace: m, l then o, indexed by (seq, kvh, split, head-in-group)
__host__ __device__ inline size_t ws_floats(uint32_t num_seqs, uint32_t nkh, uint32_t nsplit, uint32_t G,
                                           uint32_t hd) {
  return (size_t)num_seqs * nkh * nsplit * G * (hd + 2);
}

template <int G, int HD, int PPL, bool PAGED>
__global__ __launch_bounds__(NT) void attn_split_kernel(AttnArgs a) {
  constexpr int CH = 64 * PPL;             // positions per pass
  constexpr int DPL = HD / 4;              // halves of a row per lane in the score phase
  constexpr int QS = HD + HD / 16;         // padded q row (4 floats of pad per 64)
  constexpr int DPV = HD / 64;             // dims per lane in the PV phase
  __shared__ __align__(16) float q_s[G * QS];
  __shared__ __align__(16) float p_s[CH * G];      // [pos][head]
  __shared__ __align__(16) float o_s[2 * G * HD];  // cross-wave fold
  __shared__ float stat_s[2 * G];                  // pass max / sum per head

  const uint32_t split = blockIdx.x, kvh = blockIdx.y, seq = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
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
  float* ws_l = a.ws + nparts;
  float* ws_o = a.ws + 2 * nparts;
  if (b0 >= b1) {
    if (tid < G) {
      ws_m[part + tid] = -INFINITY;
      ws_l[part + tid] = 0.f;
    }
    return;
  }

  // stage q (G heads of this kv head) with a 16-byte pad every 64 floats
  const float* qg = a.q + ((size_t)seq * a.nqh + (size_t)kvh * G) * HD;
  for (int i = tid; i < G * HD; i += NT) {
    const int h = i / HD, d = i % HD;
    q_s[h * QS + d + (d >> 6) * 4] = qg[i];
  }

  auto row_ptr = [&](const uint16_t* base, uint32_t pos) -> const uint16_t* {
    size_t row;
    if (PAGED) {
      int32_t pg = a.page_table[(size_t)seq * a.max_pages + pos / a.page_size];
      pg = pg < 0 ? 0 : (pg >= (int32_t)a.num_pages ? (int32_t)a.num_pages - 1 : pg);
      row = (size_t)pg * a.page_size + pos % a.page_size;
    } else {
      row = pos;
    }
    return base + (row * a.nkh + kvh) * HD;
  };

  float m_run[G], l_run[G];
  float o[G][DPV];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    m_run[h] = -INFINITY;
    l_run[h] = 0.f;
#pragma unroll
    for (int j = 0; j < DPV; ++j) o[h][j] = 0.f;
  }
  __syncthreads();

  const int qd = lane & 3;   // quarter of the head dimension
  const int pl = lane >> 2;  // position slot within the wave
  for (uint32_t pass0 = b0; pass0 < b1; pass0 += CH) {
    // ---- scores: lane = (position, quarter); PPL positions per lane ----
    float acc[PPL][G];
    uint32_t pos[PPL];
    bool valid[PPL];
#pragma unroll
    for (int j = 0; j < PPL; ++j) {
      pos[j] = pass0 + (uint32_t)(j * 64 + w * 16 + pl);
      valid[j] = pos[j] < b1;
#pragma unroll
      for (int h = 0; h < G; ++h) acc[j][h] = 0.f;
    }
#pragma unroll
    for (int db = 0; db < DPL / 32; ++db) {
      float kf[PPL][32];
#pragma unroll
      for (int j = 0; j < PPL; ++j) {
        if (valid[j]) {
          const uint4* kp = (const uint4*)(row_ptr(a.kc, pos[j]) + qd * DPL + db * 32);
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const uint4 t = kp[c];
            const uint32_t wd[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              kf[j][8 * c + 2 * i] = g4d::f16_bits_to_f32(wd[i] & 0xffffu);
              kf[j][8 * c + 2 * i + 1] = g4d::f16_bits_to_f32(wd[i] >> 16);
            }
          }
        } else {
#pragma unroll
          for (int i = 0; i < 32; ++i) kf[j][i] = 0.f;
        }
      }
      const int dbase = qd * DPL + db * 32;
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const float* qr = q_s + h * QS + dbase + (dbase >> 6) * 4;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          const float4 qv = *(const float4*)(qr + 4 * c);
#pragma unroll
          for (int j = 0; j < PPL; ++j) {
            acc[j][h] += qv.x * kf[j][4 * c] + qv.y * kf[j][4 * c + 1];
            acc[j][h] += qv.z * kf[j][4 * c + 2] + qv.w * kf[j][4 * c + 3];
          }
        }
      }
    }
#pragma unroll
    for (int j = 0; j < PPL; ++j) {
#pragma unroll
      for (int h = 0; h < G; ++h) {
        float v = acc[j][h];
        v += __shfl_xor(v, 1, 64);
        v += __shfl_xor(v, 2, 64);
        acc[j][h] = valid[j] ? v * a.scale : -INFINITY;
      }
      if (qd == 0) {
        const int pi = j * 64 + w * 16 + pl;
#pragma unroll
        for (int h = 0; h < G; ++h) p_s[pi * G + h] = acc[j][h];
      }
    }
    __syncthreads();
    // ---- pass max per head, online rescale, probabilities ----
    // thread -> (head, slot): G heads x SL slots over CH positions; SL <= 64
    // so a head's slots sit in one wave and whole waves are idle or busy.
    constexpr int SL = (NT / G) < 64 ? (NT / G) : 64;
    if (tid < G * SL) {
      const int h = tid / SL, sl = tid % SL;
      float mx = -INFINITY;
      for (int i = sl; i < CH; i += SL) mx = fmaxf(mx, p_s[i * G + h]);
#pragma unroll
      for (int off = SL / 2; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
      if (sl == 0) stat_s[h] = mx;
    }
    __syncthreads();
    float alpha[G];
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float m_new = fmaxf(m_run[h], stat_s[h]);
      alpha[h] = expf(m_run[h] - m_new);  // 0 on the first pass (m_run = -inf)
      m_run[h] = m_new;
    }
    if (tid < G * SL) {
      const int h = tid / SL, sl = tid % SL;
      float sum = 0.f;
      for (int i = sl; i < CH; i += SL) {
        const float e = expf(p_s[i * G + h] - m_run[h]);  // masked: exp(-inf) = 0
        p_s[i * G + h] = e;
        sum += e;
      }
#pragma unroll
      for (int off = SL / 2; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
      if (sl == 0) stat_s[G + h] = sum;
    }
    __syncthreads();
#pragma unroll
    for (int h = 0; h < G; ++h) {
      l_run[h] = l_run[h] * alpha[h] + stat_s[G + h];
#pragma unroll
      for (int j = 0; j < DPV; ++j) o[h][j] *= alpha[h];
    }
    // ---- PV: lane owns DPV dims, wave w takes positions w, w+4, ... ----
    const int npos = (b1 - pass0) < (uint32_t)CH ? (int)(b1 - pass0) : CH;
    for (int i = w; i < npos; i += 4) {
      const uint16_t* vp = row_ptr(a.vc, pass0 + (uint32_t)i) + lane * DPV;
      float vf[DPV];
      if constexpr (DPV == 4) {
        const uint2 t = *(const uint2*)vp;
        vf[0] = g4d::f16_bits_to_f32(t.x & 0xffffu);
        vf[1] = g4d::f16_bits_to_f32(t.x >> 16);
        vf[2] = g4d::f16_bits_to_f32(t.y & 0xffffu);
        vf[3] = g4d::f16_bits_to_f32(t.y >> 16);
      } else {
#pragma unroll
        for (int c = 0; c < DPV / 8; ++c) {
          const uint4 t = *(const uint4*)(vp + 8 * c);
          const uint32_t wd[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            vf[8 * c + 2 * k] = g4d::f16_bits_to_f32(wd[k] & 0xffffu);
            vf[8 * c + 2 * k + 1] = g4d::f16_bits_to_f32(wd[k] >> 16);
          }
        }
      }
      const float* pp = p_s + i * G;
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const float pv = pp[h];
#pragma unroll
        for (int j = 0; j < DPV; ++j) o[h][j] += pv * vf[j];
      }
    }
    __syncthreads();  // p_s is rewritten by the next pass
  }

  // ---- fold the 4 waves' o (fixed order: (w2+w0) + (w3+w1), then + ) ----
  if (w >= 2) {
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int j = 0; j < DPV; ++j) o_s[((w - 2) * G + h) * HD + lane * DPV + j] = o[h][j];
  }
  __syncthreads();
  if (w < 2) {
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int j = 0; j < DPV; ++j) o[h][j] += o_s[(w * G + h) * HD + lane * DPV + j];
  }
  __syncthreads();
  if (w == 1) {
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int j = 0; j < DPV; ++j) o_s[h * HD + lane * DPV + j] = o[h][j];
  }
  __syncthreads();
  if (w == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float* dst = ws_o + (part + h) * HD + lane * DPV;
#pragma unroll
      for (int j = 0; j < DPV; ++j) dst[j] = o[h][j] + o_s[h * HD + lane * DPV + j];
    }
    if (lane < G) {
      ws_m[part + lane] = m_run[lane];
      ws_l[part + lane] = l_run[lane];
    }
  }
}

// Merge the splits of one (sequence, query head): O = sum_s o_s e^(m_s - M) /
// sum_s l_s e^(m_s - M); empty splits (l = 0) are skipped.
__global__ __launch_bounds__(NT) void attn_combine_kernel(const float* ws, float* out, uint32_t nqh, uint32_t nkh,
                                                          uint32_t G, uint32_t hd, uint32_t nsplit,
                                                          uint32_t num_seqs) {
  const uint32_t hq = blockIdx.x, seq = blockIdx.y;
  const uint32_t kvh = hq / G, h = hq % G;
  const size_t nparts = (size_t)num_seqs * nkh * nsplit * G;
  const float* ws_m = ws;
  const float* ws_l = ws + nparts;
  const float* ws_o = ws + 2 * nparts;
  const size_t base = ((size_t)seq * nkh + kvh) * nsplit * G + h;
  float M = -INFINITY;
  for (uint32_t s = 0; s < nsplit; ++s)
    if (ws_l[base + (size_t)s * G] > 0.f) M = fmaxf(M, ws_m[base + (size_t)s * G]);
  float Lsum = 0.f;
  float acc0 = 0.f, acc1 = 0.f;
  const uint32_t d0 = threadIdx.x, d1 = threadIdx.x + NT;
  for (uint32_t s = 0; s < nsplit; ++s) {
    const size_t pi = base + (size_t)s * G;
    const float l = ws_l[pi];
    if (!(l > 0.f)) continue;
    const float wgt = expf(ws_m[pi] - M);
    Lsum += l * wgt;
    const float* op = ws_o + pi * hd;
    if (d0 < hd) acc0 += op[d0] * wgt;
    if (d1 < hd) acc1 += op[d1] * wgt;
  }
  const float inv = Lsum > 0.f ? 1.0f / Lsum : 0.f;
  float* dst = out + ((size_t)seq * nqh + hq) * hd;
  if (d0 < hd) dst[d0] = acc0 * inv;
  if (d1 < hd) dst[d1] = acc1 * inv;
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
// host side
// ---------------------------------------------------------------------------

struct SplitPlan {
  int ppl;
  uint32_t chunk;
  uint32_t nsplit;
};

// Pass size 64 (one position per lane) up to 64 splits, then 128-position
// passes with as many passes per split as keep the grid near 256 splits.
SplitPlan plan_splits(uint32_t l_eff) {
  SplitPlan p;
  if (l_eff == 0) l_eff = 1;
  if (l_eff <= 64 * 64) {
    p.ppl = 1;
    p.chunk = 64;
  } else {
    p.ppl = 2;
    const uint32_t passes = ceil_div(ceil_div(l_eff, 128), 256);
    p.chunk = 128 * passes;
  }
  p.nsplit = ceil_div(l_eff, p.chunk);
  return p;
}

uint32_t eff_len(uint32_t seq_len, uint32_t window) {
  return (window != 0 && seq_len > window) ? window : seq_len;
}

template <int G, int HD, bool PAGED>
int launch_split_hd(g4_ctx* ctx, const AttnArgs& a, int ppl, dim3 grid) {
  if (ppl == 1) hipLaunchKernelGGL((attn_split_kernel<G, HD, 1, PAGED>), grid, dim3(NT), 0, ctx->stream, a);
  else hipLaunchKernelGGL((attn_split_kernel<G, HD, 2, PAGED>), grid, dim3(NT), 0, ctx->stream, a);
  G4_LAUNCHED(ctx, "attn_split");
  return G4_OK;
}

template <bool PAGED>
int launch_split(g4_ctx* ctx, const AttnArgs& a, uint32_t G, uint32_t hd, int ppl, dim3 grid) {
#define G4_ATTN_CASE(g, h) \
  if (G == g && hd == h) return launch_split_hd<g, h, PAGED>(ctx, a, ppl, grid);
  G4_ATTN_CASE(8, 256)
  G4_ATTN_CASE(8, 512)
  G4_ATTN_CASE(8, 128)
  G4_ATTN_CASE(4, 256)
  G4_ATTN_CASE(4, 512)
  G4_ATTN_CASE(4, 128)
  G4_ATTN_CASE(2, 256)
  G4_ATTN_CASE(2, 128)
  G4_ATTN_CASE(1, 256)
  G4_ATTN_CASE(1, 128)
#undef G4_ATTN_CASE
  return g4::set_error(G4_ERR_UNSUPPORTED, "attention: %u query heads per kv head with head_dim %u not built", G,
                       hd);
}

int check_heads(const char* fn, uint32_t nqh, uint32_t nkh, uint32_t hd) {
  G4_REQUIRE(nqh > 0 && nkh > 0 && nqh % nkh == 0 && nqh / nkh <= 8,
             "%s: num_q_heads %u must be a multiple (<= 8x) of num_kv_heads %u", fn, nqh, nkh);
  G4_REQUIRE(hd == 128 || hd == 256 || hd == 512, "%s: head_dim %u not in {128, 256, 512}", fn, hd);
  return G4_OK;
}

int dense_decode(g4_ctx* ctx, const char* fn, const float* q, const uint16_t* kc, const uint16_t* vc, float* out,
                 g4_attn_score_params p, void* ws, size_t ws_bytes, const uint32_t* pos_dev) {
  G4_REQUIRE(q && kc && vc && out && ws, "%s: null buffer", fn);
  G4_REQUIRE(((uintptr_t)kc & 15) == 0 && ((uintptr_t)vc & 15) == 0, "%s: KV caches must be 16-byte aligned", fn);
  int rc = check_heads(fn, p.num_q_heads, p.num_kv_heads, p.head_dim);
  if (rc) return rc;
  G4_REQUIRE(p.seq_len > 0, "%s: seq_len must be >= 1", fn);
  const uint32_t G = p.num_q_heads / p.num_kv_heads;
  const SplitPlan sp = plan_splits(eff_len(p.seq_len, p.sliding_window));
  const size_t need = ws_floats(1, p.num_kv_heads, sp.nsplit, G, p.head_dim) * sizeof(float);
  G4_REQUIRE(ws_bytes >= need, "%s: workspace %zu bytes < %zu required", fn, ws_bytes, need);
  AttnArgs a{};
  a.q = q;
  a.kc = kc;
  a.vc = vc;
  a.pos_dev = pos_dev;
  a.seq_len = p.seq_len;
  a.cap = p.seq_len;
  a.nqh = p.num_q_heads;
  a.nkh = p.num_kv_heads;
  a.scale = p.scale;
  a.window = p.sliding_window;
  a.chunk = sp.chunk;
  a.nsplit = sp.nsplit;
  a.ws = (float*)ws;
  rc = launch_split<false>(ctx, a, G, p.head_dim, sp.ppl, dim3(sp.nsplit, p.num_kv_heads, 1));
  if (rc) return rc;
  hipLaunchKernelGGL(attn_combine_kernel, dim3(p.num_q_heads, 1), dim3(NT), 0, ctx->stream, (const float*)ws, out,
                     p.num_q_heads, p.num_kv_heads, G, p.head_dim, sp.nsplit, 1u);
  G4_LAUNCHED(ctx, "attn_combine");
  return G4_OK;
}

}  // namespace

extern "C" {

int g4_attnScore(g4_ctx* ctx, const float* q, const uint16_t* k_cache, float* scores, g4_attn_score_params p) {
  G4_ENTER(ctx);
  G4_REQUIRE(q && k_cache && scores, "g4_attnScore: null buffer");
  G4_REQUIRE(p.num_q_heads > 0 && p.num_kv_heads > 0 && p.head_dim > 0, "g4_attnScore: empty shape");
  if (!p.seq_len) return G4_OK;
  hipLaunchKernelGGL(attn_score_kernel, dim3(ceil_div(p.seq_len, 4)), dim3(NT), 0, ctx->stream, q, k_cache, scores,
                     p.num_q_heads, p.num_kv_heads, p.head_dim, p.seq_len, p.scale, p.sliding_window);
  G4_LAUNCHED(ctx, "attn_score");
  return G4_OK;
}

int g4_softmax(g4_ctx* ctx, float* scores, g4_softmax_params p) {
  G4_ENTER(ctx);
  G4_REQUIRE(scores, "g4_softmax: null buffer");
  if (!p.num_heads || !p.seq_len) return G4_OK;
  hipLaunchKernelGGL(softmax_kernel, dim3(p.num_heads), dim3(NT), 0, ctx->stream, scores, p.num_heads, p.seq_len);
  G4_LAUNCHED(ctx, "softmax");
  return G4_OK;
}

int g4_attnOutput(g4_ctx* ctx, const float* probs, const uint16_t* v_cache, float* output, g4_attn_output_params p) {
  G4_ENTER(ctx);
  G4_REQUIRE(probs && v_cache && output, "g4_attnOutput: null buffer");
  G4_REQUIRE(p.num_q_heads > 0 && p.num_kv_heads > 0 && p.head_dim > 0, "g4_attnOutput: empty shape");
  hipLaunchKernelGGL(attn_output_kernel, dim3(ceil_div(p.num_q_heads * p.head_dim, NT)), dim3(NT), 0, ctx->stream,
                     probs, v_cache, output, p.num_q_heads, p.num_kv_heads, p.head_dim, p.seq_len);
  G4_LAUNCHED(ctx, "attn_output");
  return G4_OK;
}

int g4_attnDecode_workspace_size(g4_attn_score_params p, size_t* bytes) {
  G4_REQUIRE(bytes, "g4_attnDecode_workspace_size: null out");
  int rc = check_heads(__func__, p.num_q_heads, p.num_kv_heads, p.head_dim);
  if (rc) return rc;
  const SplitPlan sp = plan_splits(eff_len(p.seq_len, p.sliding_window));
  *bytes = ws_floats(1, p.num_kv_heads, sp.nsplit, p.num_q_heads / p.num_kv_heads, p.head_dim) * sizeof(float);
  return G4_OK;
}

int g4_attnDecode(g4_ctx* ctx, const float* q, const uint16_t* k_cache, const uint16_t* v_cache, float* output,
                  g4_attn_score_params p, void* workspace, size_t workspace_bytes) {
  G4_ENTER(ctx);
  return dense_decode(ctx, __func__, q, k_cache, v_cache, output, p, workspace, workspace_bytes, nullptr);
}

int g4_attnDecode_dev(g4_ctx* ctx, const float* q, const uint16_t* k_cache, const uint16_t* v_cache, float* output,
                      g4_attn_score_params p, void* workspace, size_t workspace_bytes, const uint32_t* position_dev) {
  G4_ENTER(ctx);
  G4_REQUIRE(position_dev, "g4_attnDecode_dev: null position");
  // p.seq_len is the capacity; the split plan covers it, and splits past the
  // live length exit after writing an empty partial.
  return dense_decode(ctx, __func__, q, k_cache, v_cache, output, p, workspace, workspace_bytes, position_dev);
}

int g4_pagedAttnDecode_workspace_size(g4_paged_attn_params p, size_t* bytes) {
  G4_REQUIRE(bytes, "g4_pagedAttnDecode_workspace_size: null out");
  int rc = check_heads(__func__, p.num_q_heads, p.num_kv_heads, p.head_dim);
  if (rc) return rc;
  const SplitPlan sp = plan_splits(eff_len(p.max_seq_len, p.sliding_window));
  *bytes = ws_floats(p.num_seqs, p.num_kv_heads, sp.nsplit, p.num_q_heads / p.num_kv_heads, p.head_dim) *
           sizeof(float);
  return G4_OK;
}

int g4_pagedAttnDecode(g4_ctx* ctx, const float* q, const uint16_t* k_pool, const uint16_t* v_pool,
                       const int32_t* page_table, const uint32_t* seq_lens, float* output, g4_paged_attn_params p,
                       void* workspace, size_t workspace_bytes) {
  G4_ENTER(ctx);
  G4_REQUIRE(q && k_pool && v_pool && page_table && seq_lens && output && workspace,
             "g4_pagedAttnDecode: null buffer");
  G4_REQUIRE(((uintptr_t)k_pool & 15) == 0 && ((uintptr_t)v_pool & 15) == 0,
             "g4_pagedAttnDecode: KV pools must be 16-byte aligned");
  int rc = check_heads(__func__, p.num_q_heads, p.num_kv_heads, p.head_dim);
  if (rc) return rc;
  G4_REQUIRE(p.num_seqs > 0 && p.page_size > 0 && p.max_pages > 0 && p.num_pages > 0,
             "g4_pagedAttnDecode: empty batch or pages");
  G4_REQUIRE(p.max_seq_len > 0 && p.max_seq_len <= p.page_size * p.max_pages,
             "g4_pagedAttnDecode: max_seq_len %u exceeds the page table (%u x %u)", p.max_seq_len, p.max_pages,
             p.page_size);
  const uint32_t G = p.num_q_heads / p.num_kv_heads;
  const SplitPlan sp = plan_splits(eff_len(p.max_seq_len, p.sliding_window));
  const size_t need = ws_floats(p.num_seqs, p.num_kv_heads, sp.nsplit, G, p.head_dim) * sizeof(float);
  G4_REQUIRE(workspace_bytes >= need, "g4_pagedAttnDecode: workspace %zu bytes < %zu required", workspace_bytes,
             need);
  AttnArgs a{};
  a.q = q;
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
  a.ws = (float*)workspace;
  rc = launch_split<true>(ctx, a, G, p.head_dim, sp.ppl, dim3(sp.nsplit, p.num_kv_heads, p.num_seqs));
  if (rc) return rc;
  hipLaunchKernelGGL(attn_combine_kernel, dim3(p.num_q_heads, p.num_seqs), dim3(NT), 0, ctx->stream,
                     (const float*)workspace, output, p.num_q_heads, p.num_kv_heads, G, p.head_dim, sp.nsplit,
                     p.num_seqs);
  G4_LAUNCHED(ctx, "attn_combine");
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
