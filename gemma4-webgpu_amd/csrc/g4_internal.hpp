// g4_internal.hpp — shared host/device helpers of libg4hip (not installed).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "g4hip.h"

struct g4_ctx {
  int device = 0;
  hipStream_t own_stream = nullptr;
  hipStream_t stream = nullptr;  // the stream every entry point enqueues on
  bool lost = false;
  int num_cus = 0;
  size_t hbm_bytes = 0;
  size_t lds_max = 65536;  // LDS bytes one workgroup may use (160 KB on gfx950)
  char name[128] = {0};
  bool capturing = false;
  // Device buffer for the partials of two-stage reductions (argmax, topk256)
  // and the activation digits of batched matmuls, allocated once at g4_init
  // so that no entry point allocates. Calls use it in stream order.
  void* scratch = nullptr;
  size_t scratch_bytes = 0;
  // Device address, on this context's device, of the static partials array
  // of g4_attnDecode_noalloc (k_attn.hip), looked up once at g4_init; null
  // (with the lookup's status in noalloc_status) when the lookup failed.
  void* noalloc_scratch = nullptr;
  int noalloc_status = 0;
  // Kernel status word in pinned host memory that kernels write through its
  // device address: nonzero once a bounded in-kernel wait of a launch on
  // this context expired (that launch's outputs are NaN). Checked by every
  // entry point and after every synchronisation; cleared by g4_clear_stall.
  volatile uint32_t* status = nullptr;
  uint32_t* status_dev = nullptr;
  // g4_test_stage_wait: poll limit of the q/k/v hand-off (0 = the built-in
  // one) and whether the q/k/v + attention launch leaves out its matvec
  uint32_t test_spin = 0;
  bool test_skip_matvec = false;
};

// Looks up the device address of g4_attnDecode_noalloc's static partials
// array on the current device (k_attn.hip); called by g4_init.
void g4_internal_noalloc_init(g4_ctx* ctx);

// Returns the context scratch buffer if it holds `bytes`.
int g4_internal_scratch(g4_ctx* ctx, size_t bytes, void** out);

// Second argmax stage (k_elem.hip): reduces `nparts` (value, index)
// candidates per row, writes the winning index of row r to result[r] and,
// with `adv` non-null, adds `delta` to adv[r].
int g4_internal_argmax_final(g4_ctx* ctx, const void* parts, int nparts, uint32_t batch, uint32_t* result,
                             uint32_t* adv, uint32_t delta);

// Weight values through the matrix-core operands (k_batch.hip; the path 2
// of g4_dequantPath).
int g4_internal_operand_values(g4_ctx* ctx, int wtype, const void* blocks, uint64_t nblocks, float* out);
// Q5_K (wtype 2) / Q8_0 (wtype 3) blocks to f16 (k_ple.hip), for g4_dequantF16.
int g4_internal_dequant_f16_q58(g4_ctx* ctx, int wtype, const void* blocks, uint64_t nblocks, uint16_t* out);

// Second top-k stage (k_elem.hip): per batch row, each of the 256 residue
// classes takes the best of its `nparts` candidates (Cand, laid out
// [batch][256][nparts]) and result[r][512] receives (value, index bits).
int g4_internal_topk_final(g4_ctx* ctx, const void* parts, int nparts, uint32_t batch, float* result);

// Matrix-core matmul of `batch` activation vectors (k_batch.hip).
int g4_internal_batch_matmul(g4_ctx* ctx, const char* fn, int qt, const float* x, const void* w, float* y,
                             uint32_t M, uint32_t N, uint32_t batch);

struct g4_event {
  hipEvent_t ev = nullptr;
  int device = 0;
  const volatile uint32_t* status = nullptr;  // the recording context's kernel status word
};

struct g4_graph {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
};

namespace g4 {

// Thread-local message of the last failure (g4_last_error).
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Maps a HIP status to a g4 status; a device fault marks the context lost.
int hip_fail(g4_ctx* ctx, hipError_t e, const char* what);
// Common prologue of every entry point: null / lost checks, set the device.
int enter(g4_ctx* ctx, const char* fn);
// Checks the launch that was just enqueued.
int check_launch(g4_ctx* ctx, const char* kernel);
// G4_ERR_STALLED when a kernel status word reports an expired wait.
int check_status(const volatile uint32_t* status, const char* fn);

}  // namespace g4

#define G4_ENTER(ctx)                              \
  do {                                             \
    int _rc = g4::enter((ctx), __func__);          \
    if (_rc != G4_OK) return _rc;                  \
  } while (0)

#define G4_REQUIRE(cond, ...)                                      \
  do {                                                             \
    if (!(cond)) return g4::set_error(G4_ERR_INVALID, __VA_ARGS__); \
  } while (0)

#define G4_HIP(ctx, call)                                    \
  do {                                                       \
    hipError_t _e = (call);                                  \
    if (_e != hipSuccess) return g4::hip_fail((ctx), _e, #call); \
  } while (0)

#define G4_LAUNCHED(ctx, name)                      \
  do {                                              \
    int _rc = g4::check_launch((ctx), (name));      \
    if (_rc != G4_OK) return _rc;                   \
  } while (0)

// ---------------------------------------------------------------------------
// device helpers
// ---------------------------------------------------------------------------

namespace g4d {

constexpr int kWave = 64;

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  _Float16 v = __builtin_bit_cast(_Float16, (uint16_t)h);
  return (float)v;
}

// Round to nearest even f32 -> f16 bits (the hardware conversion).
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// v as an f32 register value. The empty asm keeps the compiler from fusing
// the fma that produced v with a later f32 -> f16 conversion into one
// mixed-precision fma that rounds once: the reference rounds to f32 first
// (a Float32Array store) and then to f16, and the two can differ by one f16
// ulp.
__device__ __forceinline__ float as_f32(float v) {
  asm volatile("" : "+v"(v));
  return v;
}

// tanh-GELU with the tanh argument clamped to +-15 (shaders/gelu_mul.wgsl:10-16).
// tanh(t) = 2 / (1 + e^(-2t)) - 1: the quotient carries the few-ulp error of
// the hardware exp and reciprocal relative to itself, so the final f32
// subtraction rounds to the correctly rounded tanh except within ~1e-11 of
// a rounding boundary; 1 + tanh(t) is then formed in f32 as the shader forms
// it (exactly 0, or a multiple of 2^-24, where tanh is near -1). The
// library tanhf's exact evaluation cost the gate/up epilogue more than a
// microsecond per launch.
__device__ __forceinline__ float gelu_tanh(float x) {
  float t = 0.7978845608028654f * x * (1.0f + 0.044715f * x * x);
  t = fminf(fmaxf(t, -15.0f), 15.0f);
  const float th = 2.0f * __builtin_amdgcn_rcpf(1.0f + __expf(-2.0f * t)) - 1.0f;
  return 0.5f * x * (1.0f + th);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

// DPP lane exchanges inside a row of 16 lanes (VALU; no LDS round trip as
// __shfl_xor's ds_bpermute has).
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
template <int CTRL>
__device__ __forceinline__ int dppi(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
}
constexpr int kDppXor1 = 0xb1;         // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4e;         // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;  // lane i <-> 7 - i within 8 lanes
constexpr int kDppMirror = 0x140;      // lane i <-> 15 - i within 16 lanes

// Sum / max over each aligned group of 8 lanes; every lane gets its group's value.
__device__ __forceinline__ float sum8(float v) {
  v += dpp<kDppXor1>(v);
  v += dpp<kDppXor2>(v);
  return v + dpp<kDppHalfMirror>(v);
}
__device__ __forceinline__ float max8(float v) {
  v = fmaxf(v, dpp<kDppXor1>(v));
  v = fmaxf(v, dpp<kDppXor2>(v));
  return fmaxf(v, dpp<kDppHalfMirror>(v));
}
// ... over each 16-lane row
__device__ __forceinline__ float sum16(float v) { v = sum8(v); return v + dpp<kDppMirror>(v); }
__device__ __forceinline__ float max16(float v) { v = max8(v); return fmaxf(v, dpp<kDppMirror>(v)); }

// Combine with lane l ^ 16 / l ^ 32 through the gfx950 row / half-wave
// swaps (v_permlane16_swap / v_permlane32_swap on two copies of v give, in
// every lane, the pair's lower and upper values): VALU, no ds_bpermute.
__device__ __forceinline__ float xsum16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xmax16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xsum32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xmax32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// Sum over each aligned group of RG lanes (RG a power of two <= 64); every
// lane of the group gets it.
template <int RG>
__device__ __forceinline__ float group_sum(float a) {
  if constexpr (RG >= 2) a += dpp<kDppXor1>(a);
  if constexpr (RG >= 4) a += dpp<kDppXor2>(a);
  if constexpr (RG >= 8) a += dpp<kDppHalfMirror>(a);
  if constexpr (RG >= 16) a += dpp<kDppMirror>(a);
  if constexpr (RG >= 32) a = xsum16(a);
  if constexpr (RG >= 64) a = xsum32(a);
  return a;
}

__device__ __forceinline__ float lane_value(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
// Wave-wide sum / max, wave-uniform result.
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v = sum16(v);
  return (lane_value(v, 0) + lane_value(v, 16)) + (lane_value(v, 32) + lane_value(v, 48));
}
__device__ __forceinline__ float wave_max_dpp(float v) {
  v = max16(v);
  return fmaxf(fmaxf(lane_value(v, 0), lane_value(v, 16)), fmaxf(lane_value(v, 32), lane_value(v, 48)));
}

// Block-wide sum for blockDim.x == 64 * nwaves; `red` holds >= nwaves floats.
// Every thread gets the total. Contains __syncthreads.
template <int NWAVES>
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum_dpp(v);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (lane == 0) red[w] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int i = 0; i < NWAVES; ++i) t += red[i];
  __syncthreads();
  return t;
}

// argmax candidates (shaders/argmax.wgsl:12-33). The reference keeps, per
// residue class c = i mod 256, the first strict '>' maximum (init -1e30,
// index 0), then merges slot t with slot t + stride for stride = 128, 64,
// ..., 1, keeping the lower slot on equal values. The last merge (slot 0 vs
// 1) therefore prefers an even class, the one before it a class with bit 1
// clear, and so on: among equal maxima the class with the smallest
// bit-reversed 8-bit id wins, then the lowest index. NaN and values <= -1e30
// never win; with no candidate the answer is 0. `better` encodes exactly that
// order, so any partition of the index range reduces to the same answer.
struct Cand {
  float v;
  uint32_t i;
};

__device__ __forceinline__ bool better(const Cand& a, const Cand& b) {
  if (a.v > b.v) return true;
  if (a.v < b.v || !(a.v == b.v)) return false;
  const uint32_t ra = __brev(a.i & 255u), rb = __brev(b.i & 255u);
  if (ra != rb) return ra < rb;
  return a.i < b.i;
}

// The wave's best candidate, wave-uniform (every lane active): DPP steps
// inside each 16-lane row, then the four rows' winners by readlane (no
// ds_bpermute round trips).
template <int CTRL>
__device__ __forceinline__ void cand_step(Cand& c) {
  Cand d;
  d.v = dpp<CTRL>(c.v);
  d.i = (uint32_t)dppi<CTRL>((int)c.i);
  if (better(d, c)) c = d;
}
__device__ __forceinline__ Cand wave_best(Cand c) {
  cand_step<kDppXor1>(c);
  cand_step<kDppXor2>(c);
  cand_step<kDppHalfMirror>(c);
  cand_step<kDppMirror>(c);
  Cand b{lane_value(c.v, 0), (uint32_t)__builtin_amdgcn_readlane((int)c.i, 0)};
#pragma unroll
  for (int r = 16; r < 64; r += 16) {
    const Cand d{lane_value(c.v, r), (uint32_t)__builtin_amdgcn_readlane((int)c.i, r)};
    if (better(d, b)) b = d;
  }
  return b;
}

// Counter-based SplitMix64 (same definition as the host g4_splitmix64).
__host__ __device__ __forceinline__ uint64_t splitmix64(uint64_t seed, uint64_t idx) {
  uint64_t z = seed + (idx + 1) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// Matrix-core operand blocks of the M >= 16 matmul (k_batch.hip), one per
// super-block of K. Vectors are padded to the 16, 32 or 64 columns of the
// MFMA tiles a launch uses (NTV tiles of 16 vectors):
//   main  [t][s][h][lane] 16 B: f16 x 8 of vector 16t + lane%16 at
//         k = 32s + 8(lane/16) .. +7; h = 0: x_hi, 1: x_lo of x * 2^e
//   sums  [t][lane] 16 B: f16 slots 8(lane/16) .. +7 of vector 16t + lane%16;
//         slot j is part j%4 of the sum over sub-block j/4 of x * 2^(e-6)
//         (parts 0..2, part 3 zero)
//   scale [t][16] f32: 2^-e per vector
// where 2^e puts the vector's largest |x| in the super-block in [2^13, 2^14).
__host__ __device__ constexpr uint32_t pad_batch(uint32_t b) { return b <= 16 ? 16 : (b <= 32 ? 32 : 64); }
struct Ops {
  static constexpr uint32_t MAIN_T = 8 * 2 * 1024;
  __host__ __device__ static constexpr uint32_t sums_off(int ntv) { return (uint32_t)ntv * MAIN_T; }
  __host__ __device__ static constexpr uint32_t scale_off(int ntv) { return (uint32_t)ntv * (MAIN_T + 1024); }
  __host__ __device__ static constexpr uint32_t bytes(int ntv) { return (uint32_t)ntv * (MAIN_T + 1024 + 64); }
};
// Sub-block-scaled operand blocks (the gate/up launch's product, written for
// a Q6_K down projection): main as above, but every 32-element sub-block has
// its own 2^e (largest |x| of the vector's sub-block in [2^13, 2^14)), so
// the workgroup that owns 32 rows of the product can write them alone; no
// sums (Q6_K has no min term).
//   scale [t][s][16] f32: 2^-e of vector 16t + lane%16, sub-block s
struct OpsSub {
  static constexpr uint32_t MAIN_T = Ops::MAIN_T;
  __host__ __device__ static constexpr uint32_t scale_off(int ntv) { return (uint32_t)ntv * MAIN_T; }
  __host__ __device__ static constexpr uint32_t bytes(int ntv) { return (uint32_t)ntv * (MAIN_T + 512); }
};

}  // namespace g4d

inline unsigned ceil_div(uint64_t a, uint64_t b) { return (unsigned)((a + b - 1) / b); }
