// mqf_core.hpp — the fused single-sequence decode attention block on the
// matrix cores (q/k norm + RoPE, v_norm, KV row store, split-K attention and
// its in-launch merge), shared by k_attn.hip (g4_attnDecodeFused*) and
// k_gemv.hip (the launch that also runs the q/k/v matvec).
#pragma once
#include "g4_internal.hpp"

namespace g4mqf {


constexpr int MQ_NT = 256;  // threads of an attention workgroup

// exp(x) = 2^(x log2 e) on the hardware exp2 (v_exp_f32, 1 ulp): the
// softmax and merge weights are exponents of differences <= 0, where the
// product's rounding (|x| ulp of log2 e) stays below 1e-5 relative; a
// library expf is some 15 instructions on the merge's critical path.
__device__ __forceinline__ float mq_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504f); }

// RoPE of position `pos` for the pair (i, i + hd/2): the frequency is the
// correctly rounded f32 of 1/theta^(2i/hd) (divided in f32 by the f16
// divisor when apply_divisor), the angle the f32 product, as
// shaders/fused_per_head_norm_rope.wgsl:50-55 forms them; cos/sin of that
// angle in f32 (within 2 ulp of the rounded exact values). The table kernel
// and the in-launch path share it, so a precomputed table is bit-identical.
__device__ __forceinline__ float2 rope_cos_sin(float theta, uint32_t apply_divisor, uint16_t divisor_bits, uint32_t i,
                                               uint32_t hd, uint32_t pos) {
  float f = (float)(1.0 / pow((double)theta, (double)(2 * i) / (double)hd));
  if (apply_divisor) f = f / g4d::f16_bits_to_f32(divisor_bits);
  const float ang = (float)pos * f;
  float sn, cn;
  sincosf(ang, &sn, &cn);
  return make_float2(cn, sn);
}

typedef _Float16 mh8 __attribute__((ext_vector_type(8)));
typedef _Float16 mh4 __attribute__((ext_vector_type(4)));
typedef float mf4 __attribute__((ext_vector_type(4)));
typedef uint32_t mu4 __attribute__((ext_vector_type(4)));

constexpr int MQ_STEP = 64;  // positions per step (head dim 256)
constexpr int MQ_RS = 264;   // LDS row stride in halves (528 B)
constexpr int MQ_G = 8, MQ_HD = 256;
constexpr int kDppRor8 = 0x128;  // row_ror:8 within 16 lanes

// The block's shape per head dim: one thread per dim of a K/V row, so
// 256 threads (4 waves) at head dim 256 and 512 (8 waves) at 512. A step is
// 64 positions in 16-position row tiles; wave w takes row tile w % 4 and the
// 256 dims from 256 (w / 4) on, so every wave multiplies 16 positions x 256
// dims at either head dim. In the prologue and the merge a head's values
// are spread over HD / 8 threads, 4 dims of each RoPE half per thread.
template <int HD>
struct MqShape {
  static_assert(HD == 256 || HD == 512, "head dim 256 or 512");
  static constexpr int NT = HD;        // threads
  static constexpr int NW = NT / 64;   // waves
  static constexpr int NH = HD / 256;  // 256-dim halves of a row
  static constexpr int RS = HD + 8;    // K/V row stride in LDS (halves)
  static constexpr int QS = HD + 8;    // q column stride in LDS (halves)
  static constexpr int TPH = HD / 8;   // threads per head in the prologue and the merge
};

// Fused single-sequence form over a dense cache (the one-token decode step),
// the whole attention block of src/engine.ts:1556-1584 in one launch:
//  * every workgroup applies q_norm + RoPE to q once, cooperatively (thread t
//    owns head t / 32 and the RoPE pairs (d, d + 128), d = 4 (t % 32) + 0..3),
//    and stages the MFMA B operand (q hi / lo columns) in LDS;
//  * the workgroup that owns the current position forms that position's K/V
//    row (k_norm + RoPE, weightless v_norm), writes it to the caches and
//    patches it into its LDS tile;
//  * each workgroup writes one (m, l, o) partial per head; the last one to
//    arrive (arrival counter per KV head, reset for the next call) merges
//    the chunks in chunk order.
// With one sequence the grid is a few dozen workgroups, so latency is the
// instruction count of one wave's path: the per-thread work outside the
// MFMA loop is kept to a handful of vector operations.
constexpr int kMaxWarm = 4;
// Dynamic LDS a warming launch adds to each workgroup's static ~75 KB: past
// half of the CU's 160 KB, so one workgroup per CU (unused otherwise).
constexpr size_t kWarmLds = 16384;
struct MqfArgs {
  const float* q_raw;  // [nqh][head dim]
  const float* k_raw;  // [nkh][head dim]
  const float* v_raw;
  const uint16_t* q_w;
  const uint16_t* k_w;
  const uint16_t* rope_freqs;
  float theta;
  uint32_t apply_divisor;
  float eps;
  uint16_t* kc;  // [cap][nkh][head dim]
  uint16_t* vc;
  const uint32_t* pos_dev;
  uint32_t cap, nqh, nkh;
  float scale;
  uint32_t window;
  uint32_t nstep, max_chunks;  // steps per chunk (of the head dim's step), chunks
  float* ws;      // chunk partials [nkh][max_chunks][8] (m, l, o)
  float* ws1;     // group partials [nkh][MQF_FAN][8] (m, l, o)
  uint32_t* cnt;  // [nkh][MQF_CNT] arrivals (groups, then the top), zero between calls
  float* out;     // [nqh][head dim]
  // L2 warming: workgroups max_chunks.. of row 0 read the weights of the
  // launches that follow (see mqf_warm)
  const uint8_t* wbase[kMaxWarm];
  uint32_t wtotal[kMaxWarm];  // bytes of the matrix (reads past it return 0)
  uint32_t wwgb[kMaxWarm];    // bytes each consuming workgroup reads
  uint32_t wnwg[kMaxWarm];    // consuming workgroups
  uint32_t nwarm_regions, nwarm;  // regions; warming workgroups (a multiple of 8)
  const float2* rope_cs;          // [cap][head dim / 2] (cos, sin) of every position (g4_ropeTable), or null
  // the launch that also runs the q/k/v matvec (mqf_body<false, true>):
  // q, k and v staged as (tag << 32 | f32 bits) pairs, tag 1 once the matvec
  // stored the value, reset to 0 by the merger ([nqh][256] q, [nkh][256] k,
  // then v)
  uint64_t* stage;
  uint32_t nstage;
  uint32_t spin;       // polls before the wait for the staged values gives up
  uint32_t* status;    // the context's kernel status word (pinned host memory)
  // the paged batch (mqf_body<..., PAGED>, sequence `seq`): q_raw / k_raw /
  // v_raw are the q/k/v projections' nparts split-K partial sums
  // ([nparts][num_seqs][heads * 256], added in chunk order), the K/V rows
  // live in pages of the pools, the lengths (already advanced) in seq_lens;
  // out is [num_seqs][nqh][256]; q_out (or null) receives q after q_norm +
  // RoPE, ops (or null) the output as the o projection's operand blocks
  const int32_t* page_table;
  const uint32_t* seq_lens;
  uint32_t page_size, max_pages, num_pages;
  uint32_t num_seqs, nparts;  // (num_seqs 1 for the dense forms)
  float* q_out;
  uint8_t* ops;
  int ntv;
};

constexpr int MQF_QS = 264;  // LDS stride of a q column (halves)
constexpr int kMaxParts = 8;  // split-K partials the paged block adds (the hidden width's super-blocks)

// Device-scope (agent) loads and stores through a buffer resource: written
// through / read past the XCD-local L2, so they are coherent across XCDs
// without a write-back or invalidation of the whole L2. Offsets in bytes.
typedef float mqf_f4 __attribute__((ext_vector_type(4)));
constexpr int kScDevice = 16;  // cache policy operand: sc1 (device scope)
// Merge tree: chunk partials are merged in groups of up to MQF_FAN by the
// last workgroup of each group to arrive; with more than one group, the last
// group merger merges the group partials (two levels: MQF_FAN^2 chunks). The
// plan uses the tree for windows of up to MQF_FAN chunks (one level); longer
// windows end in the merge launch (mqf_kernel<true>).
constexpr uint32_t MQF_FAN = 16, MQF_CNT = 32;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t dev_rsrc(float* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(base, (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ void st_dev(__amdgpu_buffer_rsrc_t r, uint32_t off, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, off, 0, kScDevice);
}
__device__ __forceinline__ void st_dev4(__amdgpu_buffer_rsrc_t r, uint32_t off, const float4& v) {
  __builtin_amdgcn_raw_buffer_store_b128(mqf_f4{v.x, v.y, v.z, v.w}, r, off, 0, kScDevice);
}
__device__ __forceinline__ float ld_dev(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, kScDevice));
}
__device__ __forceinline__ float4 ld_dev4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const mqf_f4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kScDevice);
  return make_float4(v.x, v.y, v.z, v.w);
}

// The staged q/k/v of a launch that also runs the matvec. A value and its
// tag travel in one 8-byte device-scope store and load, so a pair read with
// tag 1 holds the stored value: the attention polls the values it needs
// until every one carries the tag, with no separate flag to wait for. The
// wait is bounded (kStageSpin polls, each a device-scope round trip, about
// 0.1 s in all) so that every workgroup ends even if a value never comes;
// the matvec workgroups precede the attention ones in the grid and wait on
// nothing, so in-order dispatch always lets them finish. A wait that
// expires is not silent: the workgroup takes NaN for every value, stores a
// partial whose maximum is +Inf (so every merge that includes it yields NaN
// whatever the order), and sets the kernel status word, which the host
// reports as G4_ERR_STALLED.
constexpr uint32_t kStageSpin = 1u << 16;
constexpr uint32_t kStatusStageWait = 1u;  // status bit: the q/k/v hand-off wait expired
constexpr uint32_t kMaxStage = 4096;  // staged values: nqh * 256 + 2 * nkh * 256
constexpr uint64_t kStaged = 1ull << 32;
__device__ __forceinline__ uint64_t stage_ld(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float stage_val(uint64_t e) { return __uint_as_float((uint32_t)e); }
// The MQ_NT threads (4 waves; a wider launch's other waves have ended) each
// poll their 8 q values and (own_row) one k and one v value; the vote goes
// through LDS, one word per wave. Returns true (uniform over the
// workgroup) when the wait expired, with every value NaN.
__device__ __forceinline__ bool mqf_wait_stage(const MqfArgs& a, int tid, size_t qoff, uint32_t kvh, bool own_row,
                                               float4& q0, float4& q1, float& kx, float& vx) {
  __shared__ uint32_t s_ok[MQ_NT / 64];
  const uint64_t* sq = a.stage + qoff;
  const uint64_t* sk = a.stage + (size_t)a.nqh * MQ_HD + (size_t)kvh * MQ_HD + tid;
  const uint64_t* sv = sk + (size_t)a.nkh * MQ_HD;
  for (uint32_t it = 0;; ++it) {
    uint64_t e[10];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      e[i] = stage_ld(sq + i);
      e[4 + i] = stage_ld(sq + MQ_HD / 2 + i);
    }
    e[8] = own_row ? stage_ld(sk) : kStaged;
    e[9] = own_row ? stage_ld(sv) : kStaged;
    bool set = true;
#pragma unroll
    for (int i = 0; i < 10; ++i) set = set && (e[i] >> 32) == 1u;
    const uint64_t votes = __ballot(set);
    if ((tid & 63) == 0) s_ok[tid >> 6] = votes == ~0ull ? 1u : 0u;
    __syncthreads();
    bool all = true;
#pragma unroll
    for (int w = 0; w < MQ_NT / 64; ++w) all = all && s_ok[w] != 0u;
    __syncthreads();  // every wave has read the votes before the next round writes them
    if (all) {
      q0 = make_float4(stage_val(e[0]), stage_val(e[1]), stage_val(e[2]), stage_val(e[3]));
      q1 = make_float4(stage_val(e[4]), stage_val(e[5]), stage_val(e[6]), stage_val(e[7]));
      kx = own_row ? stage_val(e[8]) : 0.f;
      vx = own_row ? stage_val(e[9]) : 0.f;
      return false;
    }
    if (it >= a.spin) {  // (uniform) expired: poison, and report it to the host
      const float nan = __builtin_nanf("");
      q0 = make_float4(nan, nan, nan, nan);
      q1 = q0;
      kx = nan;
      vx = nan;
      if (tid == 0) __hip_atomic_store(a.status, kStatusStageWait, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      return true;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}
__device__ __forceinline__ void mqf_clear_stage(const MqfArgs& a, int tid) {
  for (uint32_t i = (uint32_t)tid; i < a.nstage; i += MQ_NT)
    __hip_atomic_store(a.stage + i, (uint64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Workspace head: the arrival counters ([kv head][MQF_CNT]), then the staged
// q/k/v; zero between calls.
constexpr uint32_t kMqfMaxKvHeads = 64;
constexpr size_t kMqfCntOnly = (size_t)kMqfMaxKvHeads * MQF_CNT * sizeof(uint32_t);
constexpr size_t kMqfCnt = kMqfCntOnly + kMaxStage * sizeof(uint64_t);

struct MqfLaunch {
  MqfArgs m;
  bool partials;  // chunk partials + the merge launch
};
// Host side (k_attn.hip). mqf_check: the argument checks of
// g4_attnDecodeFusedWarm (messages name `fn`).
int mqf_check(g4_ctx* ctx, const char* fn, const float* q_raw, const float* k_raw, const float* v_raw,
              const uint16_t* q_norm_w, const uint16_t* k_norm_w, const uint16_t* rope_freqs, uint16_t* k_cache,
              uint16_t* v_cache, float* output, const g4_attn_fused_params& p, void* workspace,
              const uint32_t* position_dev, const g4_warm_region* regions, int nregions, const float* rope_cs,
              uint32_t rope_rows);
// mqf_prepare: after those checks, sets
// `applies` when the one-launch matrix-core form serves p and then fills L
// (workspace plan, warming workgroups on the CUs left idle by the attention
// and `busy_extra` other workgroups of the same launch). m.stage points at
// the workspace's staged q/k/v, m.nstage is 0.
int mqf_prepare(g4_ctx* ctx, const float* q_raw, const float* k_raw, const float* v_raw, const uint16_t* q_norm_w,
                const uint16_t* k_norm_w, const uint16_t* rope_freqs, uint16_t* k_cache, uint16_t* v_cache,
                float* output, const g4_attn_fused_params& p, void* workspace, size_t workspace_bytes,
                const uint32_t* position_dev, const g4_warm_region* regions, int nregions, const float* rope_cs,
                uint32_t busy_extra, bool& applies, MqfLaunch& L);

// Brings the weights of the launches that follow into the L2 of the XCD
// that will read them. Workgroups are dispatched to the 8 XCDs in turn
// (linear id mod 8), in this launch and in the consuming ones, so consuming
// workgroup j reads through the L2 of XCD j % 8: warming workgroup p (at
// linear id max_chunks + p, XCD c) reads the tiles of consuming workgroups
// j = c + 8 (p / 8 + R i), R = nwarm / 8. These workgroups run on the CUs
// the attention leaves idle; the loads go through a buffer resource sized to
// each matrix, so a partial last tile reads zeros past its end.
template <int NT = MQ_NT>
__device__ __forceinline__ void mqf_warm(const MqfArgs& a, uint32_t p, uint32_t c) {
  const uint32_t r = p >> 3, R = a.nwarm >> 3;
  const uint32_t t = threadIdx.x;
  // regions past nwarm_regions have no records (their loads return 0)
  __amdgpu_buffer_rsrc_t rs[kMaxWarm];
  uint32_t wgb[kMaxWarm], nwg[kMaxWarm], maxwg = 0;
#pragma unroll
  for (int g = 0; g < kMaxWarm; ++g) {
    const bool on = (uint32_t)g < a.nwarm_regions;
    rs[g] = __builtin_amdgcn_make_buffer_rsrc((void*)a.wbase[g], (short)0, on ? (int)a.wtotal[g] : 0, 0x00020000);
    wgb[g] = on ? a.wwgb[g] : 0u;
    nwg[g] = on ? a.wnwg[g] : 0u;
    maxwg = max(maxwg, nwg[g]);
  }
  constexpr uint32_t kStep = 64u * NT * 8u;  // bytes one round of 8 loads covers
  uint32_t acc = 0;
  // one region's round at a time, the workgroups' first rounds staggered:
  // a burst of every region at once queued ahead of the attention's own
  // memory traffic and slowed it by 1 us
  for (uint32_t k = 0; k < (p & 3u); ++k) __builtin_amdgcn_s_sleep(16);
  for (uint32_t j = c + 8u * r; j < maxwg; j += 8u * R) {
#pragma unroll
    for (int g = 0; g < kMaxWarm; ++g) {
      for (uint32_t o = 0; o < wgb[g]; o += kStep) {
        uint32_t v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          // one dword per 64-byte line brings the line into the cache
          const uint32_t off = o + (64u * NT) * (uint32_t)k + 64u * t;
          const bool in = j < nwg[g] && off < wgb[g];
          v[k] = __builtin_amdgcn_raw_buffer_load_b32(rs[g], in ? j * wgb[g] + off : 0xfffffff0u, 0, 0);
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) acc ^= v[k];
      }
    }
  }
  asm volatile("" ::"v"(acc));
}

// The paged merger's output as the o projection's matrix-core operand
// blocks (the layout g4d::Ops and merge_ops write: per super-block of K and
// tile of 16 vectors, the f16 hi / lo of y * 2^k with k from the largest
// |y| of the super-block, the 3-part f16 sums of each 32-value sub-block
// times 2^-6, and 2^-k). Thread (head th, dims td.. and 128 + td..) holds
// ov[0] and ov[1] of head hq = 8 kvh + th; head dim 256, so one head is one
// super-block.
__device__ __forceinline__ void mqf_write_ops(uint8_t* ops, int ntv, uint32_t seq, uint32_t hq, int td,
                                              const float4& y0, const float4& y1) {
  float am = fmaxf(fmaxf(fmaxf(fabsf(y0.x), fabsf(y0.y)), fmaxf(fabsf(y0.z), fabsf(y0.w))),
                   fmaxf(fmaxf(fabsf(y1.x), fabsf(y1.y)), fmaxf(fabsf(y1.z), fabsf(y1.w))));
  am = g4d::max16(am);
  am = g4d::xmax16(am);  // the head's 32 threads
  int ex = 0;
  (void)frexpf(am, &ex);
  const int k = am > 0.f ? min(max(14 - ex, -120), 120) : 0;
  const float sc = ldexpf(1.0f, k);
  const uint32_t t = seq >> 4, c = seq & 15u;
  uint8_t* base = ops + (size_t)hq * g4d::Ops::bytes(ntv);
  const float ys[8] = {y0.x, y0.y, y0.z, y0.w, y1.x, y1.y, y1.z, y1.w};
  float part[2] = {0.f, 0.f};
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    // dims e .. e + 3 (e a multiple of 4): four consecutive f16 of one lane's
    // 16 bytes, one 8-byte store for the hi plane and one for the lo
    const uint32_t e = (uint32_t)(h * 128 + td);
    const uint32_t sb = e >> 5, p = e & 31u, q = p >> 3, j = p & 7u;
    mh4 hi, lo;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float xs = ys[4 * h + i] * sc;
      hi[i] = (_Float16)xs;
      lo[i] = (_Float16)(xs - (float)hi[i]);
      part[h] += xs;
    }
    uint8_t* mp = base + t * g4d::Ops::MAIN_T + sb * 2048 + (c + 16u * q) * 16 + j * 2;
    *(mh4*)mp = hi;
    *(mh4*)(mp + 1024) = lo;
  }
  // a sub-block's 32 values are 8 consecutive threads' 4 (per half)
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const float sum = g4d::sum8(part[h]) * 0.015625f;  // * 2^-6
    const uint32_t sb = (uint32_t)(h * 4) + ((uint32_t)td >> 5);
    if ((td & 31) == 0) {
      const _Float16 p0 = (_Float16)sum;
      const float r1 = sum - (float)p0;
      const _Float16 p1 = (_Float16)r1;
      const _Float16 p2 = (_Float16)(r1 - (float)p1);
      _Float16* sp =
          (_Float16*)(base + g4d::Ops::sums_off(ntv) + t * 1024 + (c + 16u * (sb >> 1)) * 16 + (sb & 1) * 8);
      sp[0] = p0;
      sp[1] = p1;
      sp[2] = p2;
      sp[3] = (_Float16)0.f;
    }
  }
  if (td == 0) *(float*)(base + g4d::Ops::scale_off(ntv) + t * 64 + c * 4) = ldexpf(1.0f, -k);
}

// LONG (windows past MQF_FAN chunks): K/V rows are loaded non-temporally
// (read once, measured faster at 32K positions) and the workgroups end after
// storing their partials, which the merge launch that follows combines.
// FUSED && !MERGE: the launch that also runs the q/k/v matvec, whose
// workgroups end after storing their partials; the o projection's launch
// merges them per head (attn_heads_kernel) and clears the staged q/k/v.
// HD: the head dim (MqShape: HD threads); the matvec hand-off is built for 256.
// PAGED: sequence `seq` of a paged batch (the MqfArgs fields above), its
// q/k/v from split-K partial sums, merged in the launch.
template <bool LONG, bool FUSED, bool MERGE = !LONG, int HD = MQ_HD, bool PAGED = false>
__device__ __forceinline__ void mqf_body(const MqfArgs& a, uint32_t bx, uint32_t kvh, uint32_t lin,
                                         uint32_t seq = 0) {
  static_assert(!(LONG && FUSED), "the fused matvec form merges in the launch or in the o projection");
  static_assert(!(LONG && MERGE), "the long form merges in a launch of its own");
  static_assert(!FUSED || HD == MQ_HD, "the q/k/v hand-off is built for head dim 256");
  static_assert(!PAGED || (HD == MQ_HD && MERGE && !FUSED && !LONG), "the paged block: head dim 256, merged");
  using Sh = MqShape<HD>;
  constexpr int NT = Sh::NT, NW = Sh::NW, RS = Sh::RS, QS = Sh::QS, TPH = Sh::TPH;
  constexpr int PR = HD / 8;  // 16-byte pieces of a K/V row
  if (bx >= a.max_chunks) {  // (uniform) L2 warming workgroups
    if (kvh == 0) mqf_warm<NT>(a, bx - a.max_chunks, lin & 7u);
    return;
  }
  // K and V tiles; after the last step, the waves' o rows [NW waves][256 dims][16 rows]
  __shared__ __align__(16) _Float16 kvt[2 * MQ_STEP * RS];
  static_assert(2 * MQ_STEP * RS * 2 >= NW * 256 * 16 * 4, "the o rows fit in the K/V tiles");
  // B operand: column c = head c % 8, hi (c < 8) / lo; once the waves hold
  // it in registers, the space takes their partial scores (head dim 512)
  __shared__ __align__(16) _Float16 qs[16 * QS];
  static_assert(16 * QS * 2 >= NW * 64 * 16, "the scores fit in the q operand's space");
  __shared__ float2 cs_s[HD / 2];
  __shared__ float red_s[2 * NW];
  __shared__ float kn_s[HD];
  __shared__ __align__(16) uint16_t cur_s[2 * HD];  // the current row: k (roped), v; f16
  __shared__ float ml_s[2 * NW * MQ_G];             // per (wave, head) m, then l
  __shared__ __align__(16) float wt_s[4 * MQ_G];    // per (row tile, head) weight
  __shared__ uint32_t s_last;
  _Float16* const kt = kvt;
  _Float16* const vt = kvt + MQ_STEP * RS;
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, q = l >> 4, c = l & 15;
  const int rt = w & 3, dh = w >> 2;  // this wave's row tile and 256-dim half
  const uint32_t chunk = bx;
  const uint32_t CH = MQ_STEP * a.nstep;
  const uint32_t L = PAGED ? min(a.seq_lens[seq], a.cap) : min(*a.pos_dev + 1, a.cap);
  const uint32_t pos = L - 1;  // the position being decoded (PAGED: L == 0 has no chunk)
  const uint32_t wstart = (a.window != 0 && L > a.window) ? L - a.window : 0;
  const uint32_t n = L - wstart;
  const uint32_t nch = (n + CH - 1) / CH;
  if (chunk >= nch) return;  // (uniform) past the live chunks
  const uint32_t c0 = chunk * CH, cend = min(n, c0 + CH), last = wstart + cend - 1;
  const uint32_t nst = (cend - c0 + MQ_STEP - 1) / MQ_STEP;
  // this chunk ends at the current position and forms its row (without
  // k_raw the layer reads a cache another layer has already written the
  // row into: nothing is formed, stored or patched)
  const bool own_row = a.k_raw != nullptr;
  const bool owner = cend == n && own_row;
  // thread -> (head, 4 dims of each RoPE half) for q, the partial and the merge
  const int th = tid / TPH, td = 4 * (tid % TPH);
  // the cache row of position p (PAGED: its page, clamped to the pool)
  auto crow = [&](uint32_t p) -> size_t {
    if constexpr (PAGED) {
      int32_t pg = a.page_table[(size_t)seq * a.max_pages + p / a.page_size];
      pg = pg < 0 ? 0 : (pg >= (int32_t)a.num_pages ? (int32_t)a.num_pages - 1 : pg);
      return (size_t)pg * a.page_size + p % a.page_size;
    }
    return p;
  };

  // a step's K rows, then its V rows: piece pc = tid + NT (i % 8) is row
  // pc / PR, 16 bytes at column 8 (pc % PR)
  mu4 pf[16];
  // PAGED: the page of each row this thread loads in the first step,
  // requested before any other load of the launch (the rows' loads wait for
  // it; the q/k/v partials, issued after it, then arrive meanwhile)
  int32_t pg0[8];
  if constexpr (PAGED) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t r = ((uint32_t)tid + (uint32_t)NT * (uint32_t)i) / PR;
      const uint32_t p = min(wstart + c0 + r, last);
      pg0[i] = a.page_table[(size_t)seq * a.max_pages + p / a.page_size];
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  auto load_step = [&](uint32_t st) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const uint32_t pc = (uint32_t)tid + (uint32_t)NT * (uint32_t)(i & 7);
      const uint32_t r = pc / PR, col = (pc % PR) * 8;
      const uint32_t p = min(wstart + c0 + st * MQ_STEP + r, last);
      size_t row;
      if (PAGED && st == 0) {
        const int32_t pg = pg0[i & 7];
        row = (size_t)(pg < 0 ? 0 : (pg >= (int32_t)a.num_pages ? (int32_t)a.num_pages - 1 : pg)) * a.page_size +
              p % a.page_size;
      } else {
        row = crow(p);
      }
      const uint16_t* base = i < 8 ? a.kc : a.vc;
      const mu4* src = (const mu4*)(base + (row * a.nkh + kvh) * HD + col);
      pf[i] = LONG ? __builtin_nontemporal_load(src) : *src;
    }
  };
  auto store_step = [&]() {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const uint32_t pc = (uint32_t)tid + (uint32_t)NT * (uint32_t)(i & 7);
      const uint32_t r = pc / PR, col = (pc % PR) * 8;
      *(mu4*)((i < 8 ? kt : vt) + r * RS + col) = pf[i];
    }
  };
  // the owner's last step: rows from the current position on (the clamped
  // rows repeat it) take the row formed here, not the cache's stale one
  auto patch = [&](uint32_t st) {
    const uint32_t r0 = last - (wstart + c0 + st * MQ_STEP);
    for (uint32_t e = (uint32_t)tid; e < (MQ_STEP - r0) * PR; e += NT) {
      const uint32_t r = r0 + e / PR, col = (e % PR) * 8;
      *(mu4*)(kt + r * RS + col) = *(const mu4*)(cur_s + col);
      *(mu4*)(vt + r * RS + col) = *(const mu4*)(cur_s + HD + col);
    }
  };

  // ---- every load of the prologue, then the first step's rows ----
  // (FUSED: q, k and v come from the matvec workgroups of the same launch;
  // the K/V rows and the weights are requested first, then the staged q/k/v
  // are polled until every value this thread needs is there)
  const size_t qoff = (size_t)(kvh * MQ_G + th) * HD + td;
  float4 q0, q1;
  float kx, vx;
  bool stalled = false;  // (uniform) FUSED: the wait for q/k/v expired
  // PAGED: the split-K partial sums (up to kMaxParts partials), added in
  // chunk order once the first step's rows are requested
  float4 u[PAGED ? kMaxParts : 1], v[PAGED ? kMaxParts : 1];
  float ku[PAGED ? kMaxParts : 1], vu[PAGED ? kMaxParts : 1];
  if constexpr (PAGED) {
    const size_t qs_stride = (size_t)a.num_seqs * a.nqh * HD;
    const float* qg = a.q_raw + (size_t)seq * a.nqh * HD + qoff;
#pragma unroll
    for (int k = 0; k < kMaxParts; ++k) {
      const size_t o = (size_t)min((uint32_t)k, a.nparts - 1) * qs_stride;
      u[k] = *(const float4*)(qg + o);
      v[k] = *(const float4*)(qg + o + HD / 2);
    }
  } else if constexpr (!FUSED) {
    const float* qg = a.q_raw + qoff;
    q0 = *(const float4*)qg;
    q1 = *(const float4*)(qg + HD / 2);
  }
  const uint2 w0 = *(const uint2*)(a.q_w + td), w1 = *(const uint2*)(a.q_w + HD / 2 + td);
  // The k/v loads are unconditional (from the q input, no smaller, when the
  // layer forms no row) and selected only where they are used: a load under
  // a branch is waited for where the branch joins, and with it every load
  // issued before it.
  const float* const kr = own_row ? a.k_raw : a.q_raw;
  const float* const vr = own_row ? a.v_raw : a.q_raw;
  if constexpr (PAGED) {
    const size_t kv_stride = (size_t)a.num_seqs * a.nkh * HD;
    const size_t ko = ((size_t)seq * a.nkh + kvh) * HD + tid;
#pragma unroll
    for (int k = 0; k < kMaxParts; ++k) {
      const size_t o = (size_t)min((uint32_t)k, a.nparts - 1) * kv_stride + ko;
      ku[k] = kr[o];
      vu[k] = vr[o];
    }
  } else if constexpr (!FUSED) {
    kx = kr[(size_t)kvh * HD + tid];
    vx = vr[(size_t)kvh * HD + tid];
  }
  // (raw bits, from the q norm's weights when there is no row: converting
  // here would wait for every load issued so far)
  const uint16_t kwb = (own_row ? a.k_w : a.q_w)[tid];
  const uint16_t rfb = a.rope_freqs[tid & (HD / 2 - 1)];
  // the table row through a buffer resource of no records when there is no
  // table: the load stays unconditional (reads past a resource return 0;
  // the value is then unused) and a plain global load, not a flat one
  const __amdgpu_buffer_rsrc_t csr =
      __builtin_amdgcn_make_buffer_rsrc((void*)a.rope_cs, (short)0, a.rope_cs ? (int)0xffffffff : 0, 0x00020000);
  const auto csw = __builtin_amdgcn_raw_buffer_load_b64(
      csr, (uint32_t)(((size_t)pos * (HD / 2) + (tid & (HD / 2 - 1))) * sizeof(float2)), 0, 0);
  const float2 cst = make_float2(__uint_as_float(csw[0]), __uint_as_float(csw[1]));
  __builtin_amdgcn_sched_barrier(0);
  load_step(0);
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (FUSED) stalled = mqf_wait_stage(a, tid, qoff, kvh, own_row, q0, q1, kx, vx);
  if constexpr (PAGED) {
    q0 = make_float4(0.f, 0.f, 0.f, 0.f);
    q1 = q0;
    kx = 0.f;
    vx = 0.f;
#pragma unroll
    for (int k = 0; k < kMaxParts; ++k)
      if ((uint32_t)k < a.nparts) {
        q0.x += u[k].x; q0.y += u[k].y; q0.z += u[k].z; q0.w += u[k].w;
        q1.x += v[k].x; q1.y += v[k].y; q1.z += v[k].z; q1.w += v[k].w;
        kx += ku[k];
        vx += vu[k];
      }
  }
  if constexpr (!FUSED) {
    if (!own_row) {
      kx = 0.f;
      vx = 0.f;
    }
  }

  // RoPE of this position (rope_cos_sin), from the table when there is one:
  // the frequency's f64 pow and a large-argument sincos are some 380 VALU
  // instructions of the prologue's critical path
  if (tid < HD / 2) cs_s[tid] = a.rope_cs ? cst : rope_cos_sin(a.theta, a.apply_divisor, rfb, tid, HD, pos);
  const float sk = g4d::wave_sum_dpp(kx * kx), sv = g4d::wave_sum_dpp(vx * vx);
  if (l == 0) {
    red_s[w] = sk;
    red_s[NW + w] = sv;
  }
  // q: the head's sum of squares over its TPH threads (DPP rows, then the
  // half-wave swap, then at head dim 512 the wave's two halves)
  float qss = (q0.x * q0.x + q0.y * q0.y) + (q0.z * q0.z + q0.w * q0.w) + (q1.x * q1.x + q1.y * q1.y) +
              (q1.z * q1.z + q1.w * q1.w);
  qss = g4d::sum16(qss);
  qss = g4d::xsum16(qss);
  if constexpr (TPH == 64) qss = g4d::xsum32(qss);
  const float invq = __builtin_amdgcn_rsqf(qss * (1.0f / (float)HD) + a.eps);
  __syncthreads();
  float skk = (red_s[0] + red_s[1]) + (red_s[2] + red_s[3]), svv = (red_s[NW] + red_s[NW + 1]) + (red_s[NW + 2] + red_s[NW + 3]);
  if constexpr (NW == 8) {
    skk += (red_s[4] + red_s[5]) + (red_s[6] + red_s[7]);
    svv += (red_s[12] + red_s[13]) + (red_s[14] + red_s[15]);
  }
  const float invk = __builtin_amdgcn_rsqf(skk * (1.0f / (float)HD) + a.eps);
  const float invv = __builtin_amdgcn_rsqf(svv * (1.0f / (float)HD) + a.eps);
  kn_s[tid] = own_row ? kx * g4d::f16_bits_to_f32(kwb) * invk : 0.f;
  cur_s[HD + tid] = g4d::f32_to_f16_bits(vx * invv);
  {
    const float x0[4] = {q0.x, q0.y, q0.z, q0.w}, x1[4] = {q1.x, q1.y, q1.z, q1.w};
    const uint32_t wa[4] = {w0.x & 0xffffu, w0.x >> 16, w0.y & 0xffffu, w0.y >> 16};
    const uint32_t wb[4] = {w1.x & 0xffffu, w1.x >> 16, w1.y & 0xffffu, w1.y >> 16};
    mh4 h0, l0, h1, l1;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float2 cs = cs_s[td + e];
      const float y0 = x0[e] * g4d::f16_bits_to_f32(wa[e]) * invq;
      const float y1 = x1[e] * g4d::f16_bits_to_f32(wb[e]) * invq;
      const float r0 = y0 * cs.x - y1 * cs.y, r1 = y0 * cs.y + y1 * cs.x;
      h0[e] = (_Float16)r0;
      l0[e] = (_Float16)(r0 - (float)h0[e]);
      h1[e] = (_Float16)r1;
      l1[e] = (_Float16)(r1 - (float)h1[e]);
      if constexpr (PAGED) {  // the roped q, as g4_pagedAttnPrologue writes it (chunk 0's copy)
        if (a.q_out && chunk == 0) {
          float* qo = a.q_out + ((size_t)seq * a.nqh + kvh * MQ_G + th) * HD + td + e;
          qo[0] = r0;
          qo[HD / 2] = r1;
        }
      }
    }
    *(mh4*)(qs + th * QS + td) = h0;
    *(mh4*)(qs + (th + 8) * QS + td) = l0;
    *(mh4*)(qs + th * QS + HD / 2 + td) = h1;
    *(mh4*)(qs + (th + 8) * QS + HD / 2 + td) = l1;
  }
  __syncthreads();
  if (tid < HD / 2) {
    const float2 cs = cs_s[tid];
    const float x0 = kn_s[tid], x1 = kn_s[tid + HD / 2];
    cur_s[tid] = g4d::f32_to_f16_bits(x0 * cs.x - x1 * cs.y);
    cur_s[tid + HD / 2] = g4d::f32_to_f16_bits(x0 * cs.y + x1 * cs.x);
  }
  store_step();
  __syncthreads();
  if (owner) {
    bool store = true;
    if constexpr (PAGED) {  // as the prologue: only into a page of the pool
      const int32_t pg = a.page_table[(size_t)seq * a.max_pages + pos / a.page_size];
      store = pg >= 0 && pg < (int32_t)a.num_pages;
    }
    if (store) {
      a.kc[(crow(pos) * a.nkh + kvh) * HD + tid] = cur_s[tid];
      a.vc[(crow(pos) * a.nkh + kvh) * HD + tid] = cur_s[HD + tid];
    }
    if (nst == 1) patch(0);
  }
  mh8 qb[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) qb[j] = *(const mh8*)(qs + c * QS + 256 * dh + 32 * j + 8 * q);
  __syncthreads();
  float* const sx = (float*)qs;  // (head dim 512) the waves' partial scores

  mf4 O[16];
#pragma unroll
  for (int dt = 0; dt < 16; ++dt) O[dt] = mf4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;  // of head c % 8

  for (uint32_t st = 0; st < nst; ++st) {
    const bool more = st + 1 < nst;
    if (more) load_step(st + 1);
    mf4 S = mf4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const mh8 A = *(const mh8*)(kt + (16 * rt + c) * RS + 256 * dh + 32 * j + 8 * q);
      S = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, qb[j], S, 0, 0, 0);
    }
    if constexpr (NW == 8) {
      // a row tile's scores over its two dim halves, added in the same order
      // in both of its waves (so both hold the same scores)
      *(mf4*)(sx + (w * 64 + l) * 4) = S;
      __syncthreads();
      const mf4 s0 = *(const mf4*)(sx + (rt * 64 + l) * 4), s1 = *(const mf4*)(sx + ((4 + rt) * 64 + l) * 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) S[i] = s0[i] + s1[i];
    }
    float sc[4];
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float v = S[i] + g4d::dpp<kDppRor8>(S[i]);
      const uint32_t off = c0 + st * MQ_STEP + 16u * rt + 4u * q + i;
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
      for (int i = 0; i < 4; ++i) Bv[i] = vt[(16 * rt + 4 * q + i) * RS + 256 * dh + 16 * dt + c];
      mf4 o = O[dt];
      if (st > 0) {  // (uniform) the first step's O is zero
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] *= ar[i];
      }
      O[dt] = __builtin_amdgcn_mfma_f32_16x16x16f16(P, Bv, o, 0, 0, 0);
    }
    __syncthreads();
    if (more) {
      store_step();
      if (owner && st + 2 == nst) {  // (uniform) the patched rows are stored rows: order the two writes
        __syncthreads();
        patch(st + 1);
      }
      __syncthreads();
    }
  }

  // ---- the waves, then this chunk's partial ----
  // O row 4q + i of lane (q, c) is head (4q + i) % 8 (the p_hi rows for
  // q < 2, the p_lo rows for q >= 2) at dim 256 dh + 16 dt + c; wave w's
  // 256 dims go to block w of ow.
  float* ow = (float*)kvt;
#pragma unroll
  for (int dt = 0; dt < 16; ++dt) *(mf4*)(ow + ((w * 256) + 16 * dt + c) * 16 + 4 * q) = O[dt];
  if (q == 0 && c < MQ_G) {
    ml_s[w * MQ_G + c] = m_run;
    ml_s[NW * MQ_G + w * MQ_G + c] = l_run;
  }
  __syncthreads();
  const size_t nparts = (size_t)a.num_seqs * a.nkh * a.max_chunks * MQ_G;
  // chunk partials: m [nparts], l [nparts], o [nparts][HD] (f32)
  const __amdgpu_buffer_rsrc_t r0 = dev_rsrc(a.ws, (uint32_t)(nparts * (HD + 2) * sizeof(float)));
  const size_t skh = (size_t)seq * a.nkh + kvh;  // (sequence, KV head)
  const size_t part0 = (skh * a.max_chunks + chunk) * MQ_G;
  if (tid < MQ_G) {  // thread h: the head's weight per row tile and the chunk's (m, l)
    float m4[4], M = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < 4; ++ww) {
      m4[ww] = ml_s[ww * MQ_G + tid];
      M = fmaxf(M, m4[ww]);
    }
    float Ls = 0.f;
#pragma unroll
    for (int ww = 0; ww < 4; ++ww) {
      const float wt = m4[ww] == -INFINITY ? 0.f : mq_exp(m4[ww] - M);
      wt_s[ww * MQ_G + tid] = wt;
      Ls += wt * ml_s[NW * MQ_G + ww * MQ_G + tid];
    }
    // a stalled chunk's +Inf maximum turns every merge that includes it into NaN
    st_dev(r0, (uint32_t)(part0 + tid) * 4u, stalled ? INFINITY : M);
    st_dev(r0, (uint32_t)(nparts + part0 + tid) * 4u, Ls);
  }
  __syncthreads();
  {  // thread = dim: o[h] = sum over row tiles of wt * (hi row + lo row)
    float o[MQ_G];
#pragma unroll
    for (int h = 0; h < MQ_G; ++h) o[h] = 0.f;
    const int e = tid >> 8, d = tid & 255;  // dim half, dim within it
#pragma unroll
    for (int ww = 0; ww < 4; ++ww) {
      const float* r = ow + ((e * 4 + ww) * 256 + d) * 16;
      const mf4 h03 = *(const mf4*)r, h47 = *(const mf4*)(r + 4), l03 = *(const mf4*)(r + 8),
                l47 = *(const mf4*)(r + 12);
      const mf4 w03 = *(const mf4*)(wt_s + ww * MQ_G), w47 = *(const mf4*)(wt_s + ww * MQ_G + 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        o[i] += w03[i] * (h03[i] + l03[i]);
        o[4 + i] += w47[i] * (h47[i] + l47[i]);
      }
    }
#pragma unroll
    for (int h = 0; h < MQ_G; ++h) st_dev(r0, (uint32_t)(2 * nparts + (part0 + h) * HD + tid) * 4u, o[h]);
  }
  if constexpr (!MERGE) return;  // a later launch combines the chunks

  // ---- merge tree: the last arriver of each group merges it in chunk order ----
  // thread (head th, dims td.. and HD / 2 + td..): one pass with a running maximum
  auto merge = [&](__amdgpu_buffer_rsrc_t r, size_t stride, size_t first, uint32_t count, float& M, float& Ls,
                   float4& o0, float4& o1) {
    M = -INFINITY;
    Ls = 0.f;
    o0 = make_float4(0.f, 0.f, 0.f, 0.f);
    o1 = o0;
#pragma unroll 4
    for (uint32_t s2 = 0; s2 < count; ++s2) {
      const size_t pp = first + (size_t)s2 * MQ_G + th;
      const float m = ld_dev(r, (uint32_t)pp * 4u), lv = ld_dev(r, (uint32_t)(stride + pp) * 4u);
      const uint32_t ob = (uint32_t)(2 * stride + pp * HD + td) * 4u;
      const float4 a0 = ld_dev4(r, ob);
      const float4 a1 = ld_dev4(r, ob + HD / 2 * 4u);
      const float Mn = fmaxf(M, m);
      const float fo = M == -INFINITY ? 0.f : mq_exp(M - Mn);
      const float fn = m == -INFINITY ? 0.f : mq_exp(m - Mn);
      Ls = Ls * fo + lv * fn;
      o0.x = o0.x * fo + a0.x * fn; o0.y = o0.y * fo + a0.y * fn;
      o0.z = o0.z * fo + a0.z * fn; o0.w = o0.w * fo + a0.w * fn;
      o1.x = o1.x * fo + a1.x * fn; o1.y = o1.y * fo + a1.y * fn;
      o1.z = o1.z * fo + a1.z * fn; o1.w = o1.w * fo + a1.w * fn;
      M = Mn;
    }
  };
  // The partials are written and read with device-scope accesses (written
  // through / read past the XCD-local L2), so an arrival needs only its own
  // stores complete, not a write-back or invalidation of the whole L2.
  auto arrive = [&](uint32_t* cp, uint32_t fanin) -> bool {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_s_waitcnt(0);  // every store of this thread has completed
    __syncthreads();
    if (tid == 0)
      s_last = __hip_atomic_fetch_add(cp, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == fanin - 1 ? 1u : 0u;
    __syncthreads();
    if (!s_last) return false;
    if (tid == 0) __hip_atomic_store(cp, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // all arrivals are in
    return true;
  };
  auto write_out = [&](float Ls, const float4& o0, const float4& o1) {
    const float li = Ls > 0.f ? 1.0f / Ls : 0.f;
    float* dst = a.out + (skh * MQ_G + th) * HD + td;
    const float4 y0 = make_float4(o0.x * li, o0.y * li, o0.z * li, o0.w * li);
    const float4 y1 = make_float4(o1.x * li, o1.y * li, o1.z * li, o1.w * li);
    *(float4*)dst = y0;
    *(float4*)(dst + HD / 2) = y1;
    if constexpr (PAGED)
      if (a.ops) mqf_write_ops(a.ops, a.ntv, seq, (uint32_t)(kvh * MQ_G + th), td, y0, y1);
  };
  uint32_t* cnt = a.cnt + skh * MQF_CNT;
  const uint32_t ng = (nch + MQF_FAN - 1) / MQF_FAN, g = chunk / MQF_FAN;
  if (!arrive(cnt + g, min(MQF_FAN, nch - g * MQF_FAN))) return;
  float M, Ls;
  float4 o0, o1;
  merge(r0, nparts, (skh * a.max_chunks + g * MQF_FAN) * MQ_G, min(MQF_FAN, nch - g * MQF_FAN), M, Ls, o0, o1);
  if (ng == 1) {
    if constexpr (FUSED) mqf_clear_stage(a, tid);
    write_out(Ls, o0, o1);
    return;
  }
  if constexpr (PAGED) return;  // (the host keeps the paged block to one merge level)
  const size_t nparts1 = (size_t)a.nkh * MQF_FAN * MQ_G;
  const __amdgpu_buffer_rsrc_t r1 = dev_rsrc(a.ws1, (uint32_t)(nparts1 * (HD + 2) * sizeof(float)));
  {
    const size_t pp = ((size_t)kvh * MQF_FAN + g) * MQ_G + th;
    if ((tid % TPH) == 0) {
      st_dev(r1, (uint32_t)pp * 4u, M);
      st_dev(r1, (uint32_t)(nparts1 + pp) * 4u, Ls);
    }
    const uint32_t ob = (uint32_t)(2 * nparts1 + pp * HD + td) * 4u;
    st_dev4(r1, ob, o0);
    st_dev4(r1, ob + HD / 2 * 4u, o1);
  }
  if (!arrive(cnt + MQF_CNT - 1, ng)) return;
  merge(r1, nparts1, (size_t)kvh * MQF_FAN * MQ_G, ng, M, Ls, o0, o1);
  if constexpr (FUSED) mqf_clear_stage(a, tid);
  write_out(Ls, o0, o1);
}

}  // namespace g4mqf
