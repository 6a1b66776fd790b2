// k_ple.hip — Gemma 4 per-layer embeddings (PLE) on gfx950.
//
// The reference runs PLE as one f16 matmul and one single-workgroup
// dispatch per layer before the layers (src/engine.ts:1516-1535) and five
// passes inside every layer (src/engine.ts:1608-1616). Here:
//  * stage 1 is one launch for every layer and every row of a batch: the
//    per-layer table stays in its Q5_K blocks (176 B per 256 values, one
//    block per (token, layer)); each workgroup unpacks its block, rounds the
//    values to f16 as the reference's f16 upload does (src/engine.ts:626-700),
//    and fuses the projection's RMSNorm and the 1/sqrt(2) blend;
//  * the f16 matvecs (per_layer_model_proj, inp_gate, proj) keep the
//    weights in registers, one wave per row, while the vectors (up to 8 at a
//    time) are read from LDS as f32, so B vectors cost one weight read;
//  * the inp_gate launch takes the post-FFN norm-add as its prologue (one
//    vector) and gelu(gate) * ple_inputs as its epilogue; the tail's rmsNorm
//    + skip-scale-add is the next launch's prologue (the scaled norm-add of
//    g4_normAddScaleMatmulSegments / g4_batchPrepScale).
#include "g4_internal.hpp"

namespace {

constexpr int PT = 256;       // threads per workgroup
constexpr int PW = PT / 64;   // waves per workgroup
constexpr uint32_t kQ5Bytes = 176;

// vectors staged in LDS per workgroup (at most 48 KB of f32)
template <int N>
constexpr int vectors_per_pass() { return N <= 1536 ? 8 : N <= 2048 ? 4 : N <= 4096 ? 2 : 1; }
inline uint32_t vectors_per_pass_of(uint32_t N) { return N <= 1536 ? 8 : N <= 2048 ? 4 : N <= 4096 ? 2 : 1; }

// Q5_K value t (0..255) of one block (src/gguf.ts:218-257): group g = t/64
// uses sub-block j = 2g + (t/32 odd); q = 4 bits of qs[32g + l] (low nibble
// for the first 32, high for the second) + 16 * bit j of qh[l], l = t % 32;
// value = d*sc(j)*q - dmin*m(j) with the Q4_K scale/min packing. d*sc*q has
// at most 22 significant bits, so the fma rounds the exact value once, as
// the reference's f64 evaluation stored to f32 does; as_f32 keeps that f32
// rounding when the caller rounds on to f16.
__device__ __forceinline__ float q5k_value(const uint8_t* blk, int t) {
  const int g = t >> 6, hi = (t >> 5) & 1, l = t & 31, j = 2 * g + hi;
  const uint32_t dd = *(const uint32_t*)blk;
  const uint8_t* s = blk + 4;
  int sc, m;
  if (j < 4) {
    sc = s[j] & 63;
    m = s[j + 4] & 63;
  } else {
    sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4);
    m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
  }
  const int qs = blk[48 + 32 * g + l];
  const int q = (hi ? (qs >> 4) : (qs & 15)) + (((blk[16 + l] >> j) & 1) << 4);
  const float d = g4d::f16_bits_to_f32(dd & 0xffffu) * (float)sc;
  const float mn = g4d::f16_bits_to_f32(dd >> 16) * (float)m;
  return g4d::as_f32(__builtin_fmaf(d, (float)q, -mn));
}

__device__ __forceinline__ float f16_round(float v) { return g4d::f16_bits_to_f32(g4d::f32_to_f16_bits(v)); }

struct Stage1Args {
  const float* projected;  // [count][L * 256]
  const uint16_t* norm_w;  // [256]
  const uint8_t* table;    // Q5_K blocks [rows][L]
  const uint32_t* tokens;  // [count] (NULL: token)
  uint32_t token, rows, L;
  float* out;              // [count][L * 256]
  float eps;
};

// shaders/ple_stage1_fuse.wgsl:14-37 for layer blockIdx.x of row blockIdx.y.
// A token past the table reads as a zero row (the embedding lookup's rule).
__global__ __launch_bounds__(PT) void ple_stage1_kernel(Stage1Args a) {
  __shared__ float red[PW];
  const uint32_t il = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
  const uint32_t tok = a.tokens ? a.tokens[b] : a.token;
  const size_t base = ((size_t)b * a.L + il) * 256;
  const float v = a.projected[base + t];
  const float w = g4d::f16_bits_to_f32(a.norm_w[t]);
  // the table value first: its loads wait on the token, the norm's do not
  const float e = tok < a.rows ? f16_round(q5k_value(a.table + ((size_t)tok * a.L + il) * kQ5Bytes, (int)t)) : 0.f;
  const float ss = g4d::block_sum<PW>(v * v, red);
  const float rms = sqrtf(ss * (1.0f / 256.0f) + a.eps);
  const float normed = (v / rms) * w;
  a.out[base + t] = (normed + e * 16.0f) * 0.70710678118654752f;  // sqrt(256) = 16
}

// Q5_K blocks to f16 (the reference's table values, src/engine.ts:626-700).
__global__ __launch_bounds__(PT) void q5k_f16_kernel(const uint8_t* W, uint64_t nblocks, uint16_t* out) {
  const uint64_t b = blockIdx.x;
  if (b >= nblocks) return;
  out[b * 256 + threadIdx.x] = g4d::f32_to_f16_bits(q5k_value(W + b * kQ5Bytes, (int)threadIdx.x));
}

// Q8_0 blocks (34 B: f16 d, 32 int8) to f16 (src/gguf.ts:115-131: q * d,
// exact in f32, then rounded to f16 as the reference's upload does); thread
// t of a workgroup takes value t of its 8 blocks.
__global__ __launch_bounds__(PT) void q8_0_f16_kernel(const uint8_t* W, uint64_t nblocks, uint16_t* out) {
  const uint64_t e = (uint64_t)blockIdx.x * PT + threadIdx.x, b = e / 32;
  if (b >= nblocks) return;
  const uint8_t* blk = W + b * 34;
  const uint32_t dbits = (uint32_t)blk[0] | ((uint32_t)blk[1] << 8);
  const int32_t q = (int8_t)blk[2 + e % 32];
  // The product is exact in f32; one rounding to f16. The compiler turns
  // the multiply into fma(d, q, +0), which loses the sign of a zero product
  // (d = 0, q < 0 gives -0 in the reference's f64 product), so the sign is
  // set from the operands.
  const uint16_t h = g4d::f32_to_f16_bits(g4d::f16_bits_to_f32(dbits) * (float)q);
  out[e] = (uint16_t)((h & 0x7fffu) | (((dbits >> 15) ^ (uint32_t)(q < 0)) << 15));
}

// shaders/ple_gelu_mul.wgsl:11-20
__global__ __launch_bounds__(PT) void ple_gelu_mul_kernel(const float* gate, const float* ple, float* out,
                                                          uint32_t n) {
  const uint32_t i = blockIdx.x * PT + threadIdx.x;
  if (i < n) out[i] = g4d::gelu_tanh(gate[i]) * ple[i];
}

// shaders/ple_skip_scale_add.wgsl:14-20
__global__ __launch_bounds__(PT) void ple_skip_scale_add_kernel(float* hidden, const float* post, const uint16_t* scale,
                                                                uint32_t n) {
  const uint32_t i = blockIdx.x * PT + threadIdx.x;
  if (i < n) hidden[i] = (hidden[i] + post[i]) * g4d::f16_bits_to_f32(scale[0]);
}

// ---------------------------------------------------------------------------
// f16 rows x f32 vectors
// ---------------------------------------------------------------------------

struct HmvArgs {
  const uint16_t* W;  // [M][N] f16
  uint32_t M;
  const float* x;     // [B][N] (PRO 1: the post-FFN down vector)
  uint32_t B;
  float* y;           // [B][M]
  // PRO 1 (B == 1): h = residual + x * w1 / rms(x) is the vector (h_out by workgroup 0)
  const uint16_t* w1;
  const float* residual;
  float* h_out;
  float eps;
  // EPI 1: y = gelu(y) * ple[b * ple_stride + m]
  const float* ple;
  uint32_t ple_stride;
};

// One wave per row (rows blockIdx.x * PW + wave, then + gridDim.x * PW):
// lane l holds row elements 8l + 512i (N = 1536: 3 x 16 B) or 4l (N = 256:
// 8 B) in registers and multiplies them with each of the up to HB vectors
// of its workgroup row (blockIdx.y), staged in LDS; the 64 lane partials
// meet through DPP and lane v stores vector v's result. Every global load a result waits on is issued before
// the first wait: the wave's first row and the next one (prefetched while a
// row is multiplied), the prologue's vector, residual and norm weights, and
// the epilogue's ple_inputs values.
template <int N>
struct HmvRow {
  static constexpr int EPL = N == 256 ? 4 : 8;   // f16 per lane per load
  static constexpr int NL = N == 256 ? 1 : N / 512;
  uint4 u[NL];
  __device__ void load(const uint16_t* W, uint32_t m, int lane) {
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      if constexpr (EPL == 8) {
        u[i] = *(const uint4*)(W + (size_t)m * N + 512 * i + 8 * lane);
      } else {
        const uint2 v = *(const uint2*)(W + (size_t)m * N + 4 * lane);
        u[i] = make_uint4(v.x, v.y, 0u, 0u);
      }
    }
  }
  // row . xv (the lane's elements), f32 products and sums
  __device__ float dot(const float* xv, int lane) const {
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const float* xe = xv + (EPL == 8 ? 512 * i + 8 * lane : 4 * lane);
      const float4 p = *(const float4*)xe;
      acc += g4d::f16_bits_to_f32(u[i].x & 0xffffu) * p.x + g4d::f16_bits_to_f32(u[i].x >> 16) * p.y +
             g4d::f16_bits_to_f32(u[i].y & 0xffffu) * p.z + g4d::f16_bits_to_f32(u[i].y >> 16) * p.w;
      if constexpr (EPL == 8) {
        const float4 q = *(const float4*)(xe + 4);
        acc += g4d::f16_bits_to_f32(u[i].z & 0xffffu) * q.x + g4d::f16_bits_to_f32(u[i].z >> 16) * q.y +
               g4d::f16_bits_to_f32(u[i].w & 0xffffu) * q.z + g4d::f16_bits_to_f32(u[i].w >> 16) * q.w;
      }
    }
    return acc;
  }
};

template <int N, int PRO, int EPI>
__global__ __launch_bounds__(PT) void hmv_kernel(HmvArgs a) {
  static_assert(N == 256 || N % 512 == 0, "row width");
  static_assert(PRO == 0 || N % PT == 0, "prologue width");
  constexpr int HB = vectors_per_pass<N>();
  constexpr int PE = PRO == 1 ? N / PT : 1;  // prologue elements per thread
  __shared__ __align__(16) float xs[HB * N];
  __shared__ float red[2 * PW];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const uint32_t step = gridDim.x * PW, m_first = blockIdx.x * PW;
  if (m_first >= a.M) return;  // (uniform)
  HmvRow<N> row, next;
  // workgroup row blockIdx.y takes vectors HB * blockIdx.y .. + HB (one pass:
  // the vector groups run side by side, each reading the rows it needs)
  const uint32_t b0 = blockIdx.y * (uint32_t)HB;
  const uint32_t nb = min((uint32_t)HB, a.B - b0);
  row.load(a.W, min(m_first + wv, a.M - 1), lane);  // (a wave past M reads row M - 1, stores nothing)
  if constexpr (PRO == 1) {
    // the one vector: h = residual + x * w1 / rms(x)
    float xr[PE], rr[PE], wr[PE];
#pragma unroll
    for (int k = 0; k < PE; ++k) {
      xr[k] = a.x[tid + PT * k];
      rr[k] = a.residual[tid + PT * k];
      wr[k] = g4d::f16_bits_to_f32(a.w1[tid + PT * k]);
    }
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < PE; ++k) ss += xr[k] * xr[k];
    ss = g4d::block_sum<PW>(ss, red);
    const float inv = __builtin_amdgcn_rsqf(ss * (1.0f / (float)N) + a.eps);
#pragma unroll
    for (int k = 0; k < PE; ++k) {
      const float h = rr[k] + xr[k] * wr[k] * inv;
      xs[tid + PT * k] = h;
      if (a.h_out && blockIdx.x == 0) a.h_out[tid + PT * k] = h;
    }
  } else {
    for (uint32_t i = tid; i < nb * N / 4; i += PT) ((float4*)xs)[i] = ((const float4*)(a.x + (size_t)b0 * N))[i];
  }
  __syncthreads();
  for (uint32_t m0 = m_first; m0 < a.M; m0 += step) {
    const uint32_t m = m0 + wv;
    const bool live = m < a.M;
    // (rows past 4096 wide are not prefetched: two of them would not fit the registers)
    if (N <= 4096 && m0 + step < a.M) next.load(a.W, min(m0 + step + wv, a.M - 1), lane);
    // lane v's epilogue input, for vector b0 + v of this row
    float pv = 0.f;
    if (EPI == 1 && live && (uint32_t)lane < nb) pv = a.ple[(size_t)(b0 + lane) * a.ple_stride + m];
    float mine = 0.f;
    for (uint32_t v = 0; v < nb; ++v) {
      const float r = g4d::wave_sum_dpp(row.dot(xs + v * N, lane));
      if ((uint32_t)lane == v) mine = r;
    }
    if (live && (uint32_t)lane < nb) {
      float r = mine;
      if constexpr (EPI == 1) r = g4d::gelu_tanh(mine) * pv;
      a.y[(size_t)(b0 + lane) * a.M + m] = r;
    }
    if constexpr (N <= 4096) {
      row = next;
    } else if (m0 + step < a.M) {
      row.load(a.W, min(m0 + step + wv, a.M - 1), lane);
    }
  }
}

template <int PRO, int EPI>
int hmv_launch(g4_ctx* ctx, const HmvArgs& a, uint32_t N) {
  // about four workgroups per CU over the rows, times the vector groups
  const uint32_t cus = (uint32_t)(ctx->num_cus > 0 ? ctx->num_cus : 256);
  const dim3 grid(std::min<uint32_t>(4 * cus, ceil_div(a.M, (uint32_t)PW)), ceil_div(a.B, vectors_per_pass_of(N)));
  switch (N) {
    case 256: hipLaunchKernelGGL((hmv_kernel<256, PRO, EPI>), grid, dim3(PT), 0, ctx->stream, a); break;
    case 1536: hipLaunchKernelGGL((hmv_kernel<1536, PRO, EPI>), grid, dim3(PT), 0, ctx->stream, a); break;
    case 2048: hipLaunchKernelGGL((hmv_kernel<2048, PRO, EPI>), grid, dim3(PT), 0, ctx->stream, a); break;
    case 4096: hipLaunchKernelGGL((hmv_kernel<4096, PRO, EPI>), grid, dim3(PT), 0, ctx->stream, a); break;
    case 6144: hipLaunchKernelGGL((hmv_kernel<6144, PRO, EPI>), grid, dim3(PT), 0, ctx->stream, a); break;
    case 12288: hipLaunchKernelGGL((hmv_kernel<12288, PRO, EPI>), grid, dim3(PT), 0, ctx->stream, a); break;
    default: return g4::set_error(G4_ERR_UNSUPPORTED, "f16 matvec: N=%u (256, 1536, 2048, 4096, 6144, 12288)", N);
  }
  G4_LAUNCHED(ctx, "hmv");
  return G4_OK;
}

int check_hmv(const char* fn, const float* x, const uint16_t* w, const float* y, uint32_t M, uint32_t N,
              uint32_t batch) {
  G4_REQUIRE(x && w && y, "%s: null buffer", fn);
  G4_REQUIRE(M > 0 && batch >= 1 && batch <= 65535, "%s: shape M=%u batch=%u (batch 1..65535)", fn, M, batch);
  G4_REQUIRE(N == 256 || N == 1536 || N == 2048 || N == 4096 || N == 6144 || N == 12288,
             "%s: N=%u (256, 1536, 2048, 4096, 6144 or 12288)", fn, N);
  G4_REQUIRE(((uintptr_t)x & 15) == 0 && ((uintptr_t)w & 15) == 0, "%s: x and weights must be 16-byte aligned", fn);
  return G4_OK;
}

}  // namespace

// Q5_K (wtype 2) and Q8_0 (wtype 3) blocks to f16 for g4_dequantF16
// (k_gemv.hip handles Q4_K and Q6_K): nblocks blocks of 256 (Q5_K) or 32
// (Q8_0) values.
int g4_internal_dequant_f16_q58(g4_ctx* ctx, int wtype, const void* blocks, uint64_t nblocks, uint16_t* out) {
  constexpr uint64_t kChunk = 1u << 22;  // workgroups per launch
  if (wtype == 2) {
    for (uint64_t b0 = 0; b0 < nblocks; b0 += kChunk) {
      const uint64_t nb = std::min<uint64_t>(kChunk, nblocks - b0);
      hipLaunchKernelGGL(q5k_f16_kernel, dim3((uint32_t)nb), dim3(PT), 0, ctx->stream,
                         (const uint8_t*)blocks + b0 * kQ5Bytes, nb, out + b0 * 256);
      G4_LAUNCHED(ctx, "q5k_f16");
    }
    return G4_OK;
  }
  // Q8_0: 8 blocks (256 values) per workgroup
  const uint64_t groups = (nblocks + 7) / 8;
  for (uint64_t g0 = 0; g0 < groups; g0 += kChunk) {
    const uint64_t ng = std::min<uint64_t>(kChunk, groups - g0);
    const uint64_t nb = std::min<uint64_t>(ng * 8, nblocks - g0 * 8);
    hipLaunchKernelGGL(q8_0_f16_kernel, dim3((uint32_t)ng), dim3(PT), 0, ctx->stream,
                       (const uint8_t*)blocks + g0 * 8 * 34, nb, out + g0 * 8 * 32);
    G4_LAUNCHED(ctx, "q8_0_f16");
  }
  return G4_OK;
}

extern "C" {

int g4_pleStage1Fuse(g4_ctx* ctx, const float* projected, const uint16_t* norm_w, const void* table_q5k,
                     uint32_t table_rows, uint32_t token, const uint32_t* tokens_dev, float* ple_inputs,
                     uint32_t num_layers, uint32_t per_layer_dim, float eps, uint32_t count) {
  G4_ENTER(ctx);
  G4_REQUIRE(projected && norm_w && table_q5k && ple_inputs, "g4_pleStage1Fuse: null buffer");
  G4_REQUIRE(per_layer_dim == 256, "g4_pleStage1Fuse: per_layer_dim %u (one Q5_K block per layer: 256)",
             per_layer_dim);
  G4_REQUIRE(num_layers >= 1 && num_layers <= 65535 && count >= 1 && count <= 65535,
             "g4_pleStage1Fuse: %u layers, %u rows", num_layers, count);
  G4_REQUIRE(tokens_dev || count == 1, "g4_pleStage1Fuse: several rows need tokens_dev");
  G4_REQUIRE(tokens_dev || token < table_rows, "g4_pleStage1Fuse: token %u >= %u rows", token, table_rows);
  G4_REQUIRE(((uintptr_t)table_q5k & 15) == 0, "g4_pleStage1Fuse: the table must be 16-byte aligned");
  const Stage1Args a{projected, norm_w, (const uint8_t*)table_q5k, tokens_dev, token, table_rows, num_layers,
                     ple_inputs, eps};
  hipLaunchKernelGGL(ple_stage1_kernel, dim3(num_layers, count), dim3(PT), 0, ctx->stream, a);
  G4_LAUNCHED(ctx, "ple_stage1");
  return G4_OK;
}

int g4_pleGeluMul(g4_ctx* ctx, const float* gate, const float* ple_inputs, float* output, uint32_t layer_offset,
                  uint32_t size) {
  G4_ENTER(ctx);
  G4_REQUIRE(gate && ple_inputs && output, "g4_pleGeluMul: null buffer");
  if (!size) return G4_OK;
  hipLaunchKernelGGL(ple_gelu_mul_kernel, dim3(ceil_div(size, (uint32_t)PT)), dim3(PT), 0, ctx->stream, gate,
                     ple_inputs + layer_offset, output, size);
  G4_LAUNCHED(ctx, "ple_gelu_mul");
  return G4_OK;
}

int g4_pleSkipScaleAdd(g4_ctx* ctx, float* hidden, const float* post_normed, const uint16_t* scale, uint32_t size) {
  G4_ENTER(ctx);
  G4_REQUIRE(hidden && post_normed && scale, "g4_pleSkipScaleAdd: null buffer");
  if (!size) return G4_OK;
  hipLaunchKernelGGL(ple_skip_scale_add_kernel, dim3(ceil_div(size, (uint32_t)PT)), dim3(PT), 0, ctx->stream,
                     hidden, post_normed, scale, size);
  G4_LAUNCHED(ctx, "ple_skip_scale_add");
  return G4_OK;
}

int g4_matmulF16(g4_ctx* ctx, const float* x, const uint16_t* weight, float* y, uint32_t M, uint32_t N,
                 uint32_t batch) {
  G4_ENTER(ctx);
  int rc = check_hmv(__func__, x, weight, y, M, N, batch);
  if (rc) return rc;
  HmvArgs a{};
  a.W = weight;
  a.M = M;
  a.x = x;
  a.B = batch;
  a.y = y;
  return hmv_launch<0, 0>(ctx, a, N);
}

int g4_pleGate(g4_ctx* ctx, const float* x, const uint16_t* w1, const float* residual, float* h_out,
               const uint16_t* w_gate, const float* ple_inputs, uint32_t ple_stride, uint32_t layer_offset,
               float* out, uint32_t M, uint32_t N, float eps, uint32_t batch) {
  G4_ENTER(ctx);
  int rc = check_hmv(__func__, x, w_gate, out, M, N, batch);
  if (rc) return rc;
  G4_REQUIRE(ple_inputs, "g4_pleGate: null ple_inputs");
  G4_REQUIRE(!w1 == !residual, "g4_pleGate: w1 and residual go together");
  G4_REQUIRE(!w1 || batch == 1, "g4_pleGate: the norm-add prologue takes one vector");
  G4_REQUIRE(!w1 || N == 1536 || N == 2048, "g4_pleGate: the norm-add prologue is over the hidden width");
  HmvArgs a{};
  a.W = w_gate;
  a.M = M;
  a.x = x;
  a.B = batch;
  a.y = out;
  a.w1 = w1;
  a.residual = residual;
  a.h_out = h_out;
  a.eps = eps;
  a.ple = ple_inputs + layer_offset;
  a.ple_stride = ple_stride;
  return w1 ? hmv_launch<1, 1>(ctx, a, N) : hmv_launch<0, 1>(ctx, a, N);
}

}  // extern "C"
