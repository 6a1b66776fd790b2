/*
 * g4hip.h — C ABI of libg4hip.so, the MI355X (gfx950) drop-in for the WebGPU
 * decode hot path of gemma4-webgpu.
 *
 * The reference dispatches one WGSL compute shader per kernel key
 * (src/shaders.ts:34-56) with storage buffers bound in order and a `Params`
 * uniform (src/engine.ts:412-430). Each g4_<key> entry below takes the same
 * buffers, in the same binding order, as device pointers, followed by a
 * Params struct passed by value whose fields match the WGSL struct field for
 * field. Grid geometry is internal to the library (the reference's caller-side
 * dispatchMatmul, src/engine.ts:332-341, has no counterpart here).
 *
 * Conventions
 *  - Every call returns an int status: G4_OK (0) or a negative G4_ERR_*.
 *    g4_last_error() returns a thread-local message for the last failure.
 *  - A device fault makes the context sticky-lost: every later call on it
 *    returns G4_ERR_DEVICE_LOST (mirrors `device.lost`, src/engine.ts:385-388).
 *  - A launch whose workgroups hand values to each other inside the launch
 *    (g4_qkvAttnDecodeFusedWarm) waits for them a bounded number of polls.
 *    If a wait expires, the launch still ends, its outputs are NaN, and the
 *    context's kernel status word is set: every later call, and the
 *    synchronisation that follows the launch (g4_stream_sync, g4_download,
 *    g4_event_wait / g4_event_query), returns G4_ERR_STALLED until
 *    g4_clear_stall. The reference has no in-launch hand-off and so no
 *    counterpart; it is reported as device loss is, at the next call.
 *  - Kernels are enqueued on the context's stream and return immediately;
 *    they never allocate (callers own every buffer, src/engine.ts:1001-1064).
 *  - Weights are raw GGUF block bytes (Q4_K: 144 B / 256 weights, Q6_K: 210 B /
 *    256 weights), rows of N/256 blocks, instead of the f16 rows the reference
 *    expands them to at load (src/engine.ts:828-841). An f16 entry point is
 *    kept for hosts that still upload f16.
 *  - The KV cache element type is f16 (the reference's is f32,
 *    src/engine.ts:1053-1063); layout is unchanged: position-major,
 *    [max_seq][num_kv_heads][head_dim].
 *  - `_dev` variants read the per-forward dynamic field (position; seq_len is
 *    position + 1) from device memory, so a captured graph can be replayed
 *    and the sampled token can stay on the GPU (src/engine.ts:1487-1504,
 *    1724-1727).
 */
#ifndef G4HIP_H
#define G4HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define G4_OK 0
#define G4_ERR_INVALID (-1)      /* bad argument / shape / null pointer */
#define G4_ERR_HIP (-2)          /* a HIP runtime call failed */
#define G4_ERR_DEVICE_LOST (-3)  /* sticky: the context is unusable */
#define G4_ERR_OOM (-4)          /* device allocation failed */
#define G4_ERR_UNSUPPORTED (-5)  /* shape the kernels do not handle */
#define G4_ERR_NO_DEVICE (-6)    /* no HIP device / wrong architecture */
#define G4_ERR_STALLED (-7)      /* sticky until g4_clear_stall: a bounded wait inside a
                                    kernel expired, and that launch wrote NaN outputs */

typedef struct g4_ctx g4_ctx;
typedef struct g4_event g4_event;
typedef struct g4_graph g4_graph;

/* ------------------------------------------------------------------------ */
/* Lifecycle, memory, synchronisation                                        */
/* (replaces initWebGPU / createF16Buffer / writeBuffer / mapAsync:          */
/*  src/engine.ts:354-389, 553-567, 313-316, 1772-1787)                      */
/* ------------------------------------------------------------------------ */

const char* g4_last_error(void);
int g4_version(void); /* ABI version, currently 1 */

int g4_init(int device, g4_ctx** out);
int g4_destroy(g4_ctx* ctx);
/* Use an external HIP stream (hipStream_t as void*); NULL restores the
 * context's own stream. */
int g4_set_stream(g4_ctx* ctx, void* hip_stream);
void* g4_get_stream(g4_ctx* ctx);
int g4_device_info(g4_ctx* ctx, char* name, size_t name_len, int* num_cus, size_t* hbm_bytes);

int g4_alloc(g4_ctx* ctx, size_t bytes, void** dptr);
int g4_free(g4_ctx* ctx, void* dptr);
int g4_memset(g4_ctx* ctx, void* dptr, int value, size_t bytes);
/* host -> device, complete when the call returns (writeBuffer semantics) */
int g4_upload(g4_ctx* ctx, void* dst, const void* src, size_t bytes, size_t dst_offset);
/* device -> host, blocking */
int g4_download(g4_ctx* ctx, void* dst, const void* src, size_t bytes, size_t src_offset);
/* device -> host, completes asynchronously; poll or wait on the event.
 * dst must stay valid until the event completes. */
int g4_download_async(g4_ctx* ctx, void* dst, const void* src, size_t bytes, size_t src_offset,
                      g4_event** ev);
int g4_copy_d2d(g4_ctx* ctx, void* dst, const void* src, size_t bytes);
/* Pinned (page-locked) host memory, the destination g4_download_async needs
 * to complete without blocking the caller (the mapAsync staging buffer of
 * src/engine.ts:1772-1787). g4_host_free takes what g4_host_alloc returned. */
int g4_host_alloc(g4_ctx* ctx, size_t bytes, void** host);
int g4_host_free(void* host);
int g4_stream_sync(g4_ctx* ctx);
/* Clears the kernel status word after a G4_ERR_STALLED (no counterpart in
 * the reference, see Conventions). The launch that stalled may still have
 * left staged values in its attention workspace: zero that workspace
 * (g4_memset) before the next g4_qkvAttnDecodeFusedWarm on it. */
int g4_clear_stall(g4_ctx* ctx);

/* An event reports its context's G4_ERR_STALLED once complete, so it is
 * destroyed before the context that recorded it. */
int g4_event_record(g4_ctx* ctx, g4_event** ev);
int g4_event_query(g4_event* ev); /* 1 = complete, 0 = pending, <0 error */
int g4_event_wait(g4_event* ev);
int g4_event_elapsed_ms(g4_event* start, g4_event* end, float* ms);
int g4_event_destroy(g4_event* ev);

/* Graph capture of everything enqueued on the context stream between begin
 * and end; launch replays it on the context stream. While capturing,
 * g4_memset, g4_upload, g4_download(_async) and g4_stream_sync return
 * G4_ERR_INVALID (a memset node or a synchronisation has no place in a
 * replayed graph). */
int g4_graph_begin(g4_ctx* ctx);
int g4_graph_end(g4_ctx* ctx, g4_graph** graph);
int g4_graph_launch(g4_ctx* ctx, g4_graph* graph);
int g4_graph_destroy(g4_graph* graph);
/* Kernel nodes of a captured graph (diagnostics, no reference counterpart:
 * the launches one replay issues). */
int g4_graph_kernel_nodes(g4_graph* graph, size_t* count);

/* ------------------------------------------------------------------------ */
/* Kernel entry points (one per SHADERS key, src/shaders.ts:34-56)           */
/* ------------------------------------------------------------------------ */

/* shaders/matmul_quant.wgsl:12 — Params { M: out rows, N: reduction }. */
typedef struct { uint32_t M, N; } g4_matmul_params;

/* y[M] = W[M,N] . x[N].  shaders/matmul_quant.wgsl:21-54 (matmulQuant);
 * W is raw Q4_K blocks, N % 256 == 0. */
int g4_matmulQuant_q4k(g4_ctx* ctx, const float* input, const void* weight, float* output,
                       g4_matmul_params p);
/* Same contract with W as raw Q6_K blocks (ffn down, tied LM head). */
int g4_matmulQuant_q6k(g4_ctx* ctx, const float* input, const void* weight, float* output,
                       g4_matmul_params p);
/* Same contract with the reference's own f16 rows (shaders/matmul_quant.wgsl:14). */
int g4_matmulQuant_f16(g4_ctx* ctx, const float* input, const uint16_t* weight, float* output,
                       g4_matmul_params p);
/* shaders/matmul_quant_mr4.wgsl:17-88 (matmulQuantMR4): same bindings and
 * Params; rows per wavefront are internal, so this is the same kernel. */
int g4_matmulQuantMR4_q4k(g4_ctx* ctx, const float* input, const void* weight, float* output,
                          g4_matmul_params p);
/* Batched variant (LM head at M=8, ragged batch): Y[b][M] = W . X[b] for
 * b < batch; X is [batch][N] f32, Y is [batch][M] f32. batch <= 8 uses the
 * vector path, batch >= 16 the MFMA path. */
int g4_matmulQuantBatch_q4k(g4_ctx* ctx, const float* input, const void* weight, float* output,
                            g4_matmul_params p, uint32_t batch);
int g4_matmulQuantBatch_q6k(g4_ctx* ctx, const float* input, const void* weight, float* output,
                            g4_matmul_params p, uint32_t batch);

/* shaders/kv_cache_store.wgsl:1 — Params {num_kv_heads, head_dim, position, max_seq_len}.
 * Writes k_in/v_in (f32) as f16 into row `position` of the caches. */
typedef struct { uint32_t num_kv_heads, head_dim, position, max_seq_len; } g4_kv_store_params;
int g4_kvCacheStore(g4_ctx* ctx, const float* k_in, const float* v_in, uint16_t* k_cache,
                    uint16_t* v_cache, g4_kv_store_params p);
int g4_kvCacheStore_dev(g4_ctx* ctx, const float* k_in, const float* v_in, uint16_t* k_cache,
                        uint16_t* v_cache, g4_kv_store_params p, const uint32_t* position_dev);

/* shaders/attn_score.wgsl:9 — Params {num_q_heads, num_kv_heads, head_dim,
 * seq_len, scale, sliding_window}; scores is [num_q_heads][seq_len]. */
typedef struct {
  uint32_t num_q_heads, num_kv_heads, head_dim, seq_len;
  float scale;
  uint32_t sliding_window;
} g4_attn_score_params;
int g4_attnScore(g4_ctx* ctx, const float* q, const uint16_t* k_cache, float* scores,
                 g4_attn_score_params p);

/* shaders/softmax.wgsl:1 — Params {num_heads, seq_len}; in place. */
typedef struct { uint32_t num_heads, seq_len; } g4_softmax_params;
int g4_softmax(g4_ctx* ctx, float* scores, g4_softmax_params p);

/* shaders/attn_output.wgsl:1 — Params {num_q_heads, num_kv_heads, head_dim, seq_len}. */
typedef struct { uint32_t num_q_heads, num_kv_heads, head_dim, seq_len; } g4_attn_output_params;
int g4_attnOutput(g4_ctx* ctx, const float* probs, const uint16_t* v_cache, float* output,
                  g4_attn_output_params p);
/* The trio with seq_len = *position_dev + 1 read on the device (the per-forward
 * seq_len patches of src/engine.ts:1496-1504, so the per-key sequence can be
 * captured once and replayed): p.seq_len is the maximum the grid and the
 * scores buffer were sized for, and the device value is clamped to it. The
 * scores rows keep the reference's stride seq_len (the device value). */
int g4_attnScore_dev(g4_ctx* ctx, const float* q, const uint16_t* k_cache, float* scores,
                     g4_attn_score_params p, const uint32_t* position_dev);
int g4_softmax_dev(g4_ctx* ctx, float* scores, g4_softmax_params p, const uint32_t* position_dev);
int g4_attnOutput_dev(g4_ctx* ctx, const float* probs, const uint16_t* v_cache, float* output,
                      g4_attn_output_params p, const uint32_t* position_dev);

/* Fused split-K flash-decode: the attnScore -> softmax -> attnOutput trio in
 * one pass over the KV cache (same inputs and masking as the trio,
 * src/engine.ts:1582-1584). `workspace` holds the per-split partials; its
 * size comes from g4_attnDecode_workspace_size. Calls that share a workspace
 * must not overlap. */
int g4_attnDecode_workspace_size(g4_attn_score_params p, size_t* bytes);
int g4_attnDecode(g4_ctx* ctx, const float* q, const uint16_t* k_cache, const uint16_t* v_cache,
                  float* output, g4_attn_score_params p, void* workspace, size_t workspace_bytes);
/* g4_attnDecode without a workspace: the split-K partials go to a static
 * 16 MiB device array of the library (each GPU holds one until the process
 * ends), and the call allocates nothing. No counterpart in the reference; it
 * is for callers that cannot allocate (code under graph capture, serving
 * loops that forbid hipMalloc). Shapes whose g4_attnDecode_workspace_size
 * exceeds 16 MiB (e.g. head_dim 512 beyond 32768 positions) return
 * G4_ERR_INVALID. All calls on one GPU share the array: calls that overlap
 * (on other streams) race. */
int g4_attnDecode_noalloc(g4_ctx* ctx, const float* q, const uint16_t* k_cache,
                          const uint16_t* v_cache, float* output, g4_attn_score_params p);
/* seq_len = *position_dev + 1 read on the device; p.seq_len is the maximum
 * the workspace was sized for. */
int g4_attnDecode_dev(g4_ctx* ctx, const float* q, const uint16_t* k_cache,
                      const uint16_t* v_cache, float* output, g4_attn_score_params p,
                      void* workspace, size_t workspace_bytes, const uint32_t* position_dev);

/* The per-layer attention block of a decode step in one launch
 * (src/engine.ts:1562-1584): q_norm + RoPE on the raw q projection, k_norm +
 * RoPE on k and the weightless v_norm on v, the K/V row stored (f16) at
 * position *position_dev, then split-K decode attention over positions
 * [0, *position_dev] with the window. q_raw is [num_q_heads][head_dim] and is
 * not modified; k_raw/v_raw are [num_kv_heads][head_dim]; caches hold
 * max_seq_len rows. The workspace (g4_attnDecodeFused_workspace_size bytes)
 * keeps arrival counters in its first 8 KB and partials after them: it
 * must be zeroed (g4_memset) before its first use, every call leaves the
 * counters zero, and one workspace may serve calls of different windows and
 * lengths (the layers of a step) as long as they do not overlap and no other
 * entry point writes into it in between.
 * A layer that reads another layer's KV cache (the consumer layers of
 * src/engine.ts:1541-1583, which compute only q and attend over their
 * producer's cache, src/engine.ts:1149-1152) passes k_raw = v_raw =
 * k_norm_w = NULL and that cache: no row is formed or stored, and the row
 * at *position_dev is read from the cache like every other. */
typedef struct {
  uint32_t num_q_heads, num_kv_heads, head_dim, max_seq_len;
  float scale;
  uint32_t sliding_window;
  float eps, theta;
  uint32_t apply_divisor;
} g4_attn_fused_params;
int g4_attnDecodeFused_workspace_size(g4_attn_fused_params p, size_t* bytes);
int g4_attnDecodeFused(g4_ctx* ctx, const float* q_raw, const float* k_raw, const float* v_raw,
                       const uint16_t* q_norm_w, const uint16_t* k_norm_w, const uint16_t* rope_freqs,
                       uint16_t* k_cache, uint16_t* v_cache, float* output, g4_attn_fused_params p,
                       void* workspace, size_t workspace_bytes, const uint32_t* position_dev);

/* L2 warming (an MI355X scheduling aid with no counterpart in the
 * reference, for hosts that issue a fixed launch sequence such as the decode
 * step). A one-vector matvec launch over W [M x N] has workgroup j read the
 * bytes [j * wg_bytes, (j + 1) * wg_bytes) of W (of each matrix of a gate/up
 * pair); g4_matmulWarmRegion describes that for the launch
 * g4_matmulQuant_* / g4_normAddGateUpGelu_q4k would make. */
typedef struct {
  const void* base;
  uint64_t total_bytes; /* bytes of the matrix; at most 4 GiB - 1 */
  uint64_t wg_bytes;
  uint32_t nwgs;
  uint32_t reserved;
} g4_warm_region;
int g4_matmulWarmRegion(g4_ctx* ctx, int wtype, uint32_t M, uint32_t N, const void* weight,
                        g4_warm_region* out);
/* g4_attnDecodeFused, whose launch also reads up to 4 regions (the weights
 * of the matvecs that follow it) into the L2 cache of the XCD each
 * consuming workgroup will run on, using the CUs the attention leaves idle,
 * and, with rope_cs non-NULL, takes the RoPE cos/sin of the position from a
 * table g4_ropeTable wrote for this theta / divisor, of rope_rows >=
 * max_seq_len rows (the per-call frequency pow and sincos cost the prologue
 * about 0.3 us). Results are those of g4_attnDecodeFused, bit for bit. */
int g4_attnDecodeFusedWarm(g4_ctx* ctx, const float* q_raw, const float* k_raw, const float* v_raw,
                           const uint16_t* q_norm_w, const uint16_t* k_norm_w,
                           const uint16_t* rope_freqs, uint16_t* k_cache, uint16_t* v_cache,
                           float* output, g4_attn_fused_params p, void* workspace,
                           size_t workspace_bytes, const uint32_t* position_dev,
                           const g4_warm_region* regions, int nregions, const float* rope_cs,
                           uint32_t rope_rows);
/* The q/k/v projections and the attention block of one layer
 * (src/engine.ts:1550-1584: the Q4_K q/k/v matvecs over the attention
 * rmsNorm of the residual stream, then the block g4_attnDecodeFusedWarm
 * runs): g4_normAddScaleMatmulSegments(wtype Q4_K, x .. eps, weights,
 * outputs, rows = q_dim / kv_dim / kv_dim, nseg, no softcap) followed by
 * g4_attnDecodeFusedWarm(outputs[0], outputs[1], outputs[2] (null when
 * nseg = 1, a layer reading its producer's cache), ...). Results are those
 * of the two calls, bit for bit; outputs[] receive q/k/v as well.
 * When N = 1536, one KV head and a window of at most 1024 positions, both
 * run as one launch: the attention workgroups load their K/V rows while the
 * matvec workgroups run, and poll q/k/v, which the matvec also stages with
 * a tag in the workspace (an MI355X fusion with no reference counterpart);
 * other shapes make the two launches. The workspace is g4_attnDecodeFused's, zeroed before its first
 * use; calls that share a workspace must not overlap. The attention
 * workgroups of the one launch poll for q/k/v at most 2^16 times (about
 * 0.1 s); if that expires, the launch writes NaN to `output` (and to the
 * K/V row it stores) and the call's stall is reported as G4_ERR_STALLED
 * (Conventions). */
int g4_qkvAttnDecodeFusedWarm(g4_ctx* ctx, const float* x, const uint16_t* w1, const float* residual,
                              const uint16_t* out_scale, const uint16_t* w2, float* h_out,
                              const void* const* weights, float* const* outputs, int nseg, uint32_t N, float eps,
                              const uint16_t* q_norm_w, const uint16_t* k_norm_w, const uint16_t* rope_freqs,
                              uint16_t* k_cache, uint16_t* v_cache, float* output, g4_attn_fused_params p,
                              void* workspace, size_t workspace_bytes, const uint32_t* position_dev,
                              const g4_warm_region* regions, int nregions, const float* rope_cs,
                              uint32_t rope_rows);
/* g4_qkvAttnDecodeFusedWarm's one launch with the attention's chunk merge
 * left out: the attention workgroups end after storing their chunk partials
 * (m, l, o) in the workspace, and g4_attnHeadsMatmul_q4k merges them in the
 * o projection's launch. Only shapes that take the one launch (N = 1536,
 * Q4_K q/k/v, one KV head of 256, a window of at most 1024 positions);
 * others return G4_ERR_UNSUPPORTED. Leaves the staged q/k/v in the
 * workspace: the next call on it must be g4_attnHeadsMatmul_q4k, which
 * clears them. An MI355X split of src/engine.ts:1550-1584 with no reference
 * counterpart. */
int g4_qkvAttnDecodePartials(g4_ctx* ctx, const float* x, const uint16_t* w1, const float* residual,
                             const uint16_t* out_scale, const uint16_t* w2, float* h_out, const void* const* weights,
                             float* const* outputs, int nseg, uint32_t N, float eps, const uint16_t* q_norm_w,
                             const uint16_t* k_norm_w, const uint16_t* rope_freqs, uint16_t* k_cache,
                             uint16_t* v_cache, g4_attn_fused_params p, void* workspace, size_t workspace_bytes,
                             const uint32_t* position_dev, const g4_warm_region* regions, int nregions,
                             const float* rope_cs, uint32_t rope_rows);
/* The attention output projection of src/engine.ts:1585-1589
 * (matmulQuant of attn_output by W_o, Q4_K [M][8 * 256]) over the chunk
 * partials g4_qkvAttnDecodePartials left in the workspace, split into
 * G4_O_SHARES groups of 8 / G4_O_SHARES heads:
 * output[g][M] = sum over the group's heads h of W_o[:, 256 h .. 256 h + 255] . o_h,
 * o_h the attention output of head h (its chunks merged as attn_output.wgsl
 * sums over all positions). o = sum over g of output[g], which
 * g4_normAddPartsGateUpGeluDigits_q4k adds in group order. Also clears the
 * workspace's staged q/k/v. */
#define G4_O_SHARES 4
int g4_attnHeadsMatmul_q4k(g4_ctx* ctx, void* workspace, size_t workspace_bytes, g4_attn_fused_params p,
                           const uint32_t* position_dev, const void* weight, float* output, uint32_t M);
/* g4_normAddGateUpGeluDigits_q4k with o given as G4_O_SHARES shares
 * o_parts[G4_O_SHARES][N] (g4_attnHeadsMatmul_q4k's output), added in order
 * before the post-attention norm-add (src/engine.ts:1590-1602). */
int g4_normAddPartsGateUpGeluDigits_q4k(g4_ctx* ctx, const float* o_parts, const uint16_t* w_post,
                                        const float* residual, const uint16_t* w_pre, const void* w_gate,
                                        const void* w_up, float* h_out, float* out, void* digits, g4_matmul_params p,
                                        float eps);
/* Test hook with no reference counterpart, for tests of the stall report:
 * the following one-launch g4_qkvAttnDecodeFusedWarm calls on this context
 * poll at most `spin_limit` times (0 restores the built-in limit) and, when
 * skip_matvec is nonzero, launch no matvec workgroups, so that nothing
 * stages q/k/v and every attention workgroup's wait expires (every kernel
 * still ends). (0, 0) restores normal operation. */
int g4_test_stage_wait(g4_ctx* ctx, uint32_t spin_limit, int skip_matvec);
/* RoPE table of shaders/fused_per_head_norm_rope.wgsl:50-55: for position
 * t < rows and pair i < head_dim/2, table[2 (t head_dim/2 + i)] = cos and
 * [.. + 1] = sin of t * freq_i, freq_i = 1/theta^(2i/head_dim) (divided by
 * rope_freqs[i] when apply_divisor), the values the fused attention
 * computes per call. An MI355X aid with no reference counterpart (the
 * reference recomputes them in every fusedPerHeadNormRope dispatch). */
int g4_ropeTable(g4_ctx* ctx, float theta, uint32_t apply_divisor, const uint16_t* rope_freqs,
                 uint32_t head_dim, uint32_t rows, float* table);

/* Ragged multi-sequence decode attention over a paged f16 KV pool: sequence
 * s has seq_lens[s] positions; its logical position t lives in page
 * page_table[s * max_pages + t / page_size], slot t % page_size, of a pool
 * of num_pages pages of page_size rows [num_kv_heads][head_dim]. q is
 * [num_seqs][num_q_heads][head_dim], output likewise. Lengths are clamped to
 * max_seq_len and page ids to [0, num_pages), so a bad table cannot address
 * memory outside the pool. */
typedef struct {
  uint32_t num_seqs, num_q_heads, num_kv_heads, head_dim;
  uint32_t page_size, max_pages, max_seq_len, num_pages;
  float scale;
  uint32_t sliding_window;
} g4_paged_attn_params;
int g4_pagedAttnDecode_workspace_size(g4_paged_attn_params p, size_t* bytes);
int g4_pagedAttnDecode(g4_ctx* ctx, const float* q, const uint16_t* k_pool, const uint16_t* v_pool,
                       const int32_t* page_table, const uint32_t* seq_lens, float* output,
                       g4_paged_attn_params p, void* workspace, size_t workspace_bytes);
/* g4_pagedAttnDecode that also writes its output as the matrix-core operand
 * blocks of the o projection (ops: g4_batchOperandBytes(num_q_heads *
 * head_dim, num_seqs) bytes, 16-byte aligned), which g4_matmulSegmentsBatch-
 * Partial takes so that its workgroups need not rebuild them (an MI355X
 * hand-off with no reference counterpart). head_dim a multiple of 256,
 * num_seqs <= 64; ops == NULL is g4_pagedAttnDecode. */
int g4_pagedAttnDecodeOps(g4_ctx* ctx, const float* q, const uint16_t* k_pool, const uint16_t* v_pool,
                          const int32_t* page_table, const uint32_t* seq_lens, float* output,
                          g4_paged_attn_params p, void* workspace, size_t workspace_bytes, void* ops);
/* The per-layer attention block of a multi-sequence decode step in one launch
 * (per sequence, the block src/engine.ts:1562-1584 runs for one token):
 * sequence s decodes position seq_lens[s] - 1 (seq_lens already advanced,
 * g4_advanceSeqLens). q_norm + RoPE on q_raw [num_seqs][num_q_heads][head_dim]
 * (not modified), k_norm + RoPE on k_raw and the weightless v_norm on v_raw
 * ([num_seqs][num_kv_heads][head_dim]), the f16 K/V row stored in the pool
 * page the table names (a page id outside [0, num_pages) stores nothing),
 * then split-K decode attention over the sequence's window. The workspace is
 * sized by g4_pagedAttnDecodeFused_workspace_size; calls that share it must
 * not overlap. k_raw = v_raw = k_norm_w = NULL: a consumer layer over its
 * producer's pool, as for g4_attnDecodeFused. */
typedef struct {
  uint32_t num_seqs, num_q_heads, num_kv_heads, head_dim;
  uint32_t page_size, max_pages, max_seq_len, num_pages;
  float scale;
  uint32_t sliding_window;
  float eps, theta;
  uint32_t apply_divisor;
} g4_paged_attn_fused_params;
int g4_pagedAttnDecodeFused_workspace_size(g4_paged_attn_fused_params p, size_t* bytes);
int g4_pagedAttnDecodeFused(g4_ctx* ctx, const float* q_raw, const float* k_raw, const float* v_raw,
                            const uint16_t* q_norm_w, const uint16_t* k_norm_w, const uint16_t* rope_freqs,
                            uint16_t* k_pool, uint16_t* v_pool, const int32_t* page_table,
                            const uint32_t* seq_lens, float* output, g4_paged_attn_fused_params p,
                            void* workspace, size_t workspace_bytes);
/* The same block before the attention, as a launch of its own over the
 * split-K partial sums of the q/k/v projections (q_parts [nparts][num_seqs]
 * [num_q_heads*head_dim], k_parts / v_parts [nparts][num_seqs]
 * [num_kv_heads*head_dim], added in chunk order): q_out [num_seqs]
 * [num_q_heads][head_dim] receives q after q_norm + RoPE, and the f16 K/V
 * row is appended to the pool as g4_pagedAttnDecodeFused does;
 * g4_pagedAttnDecode then attends. p.scale and p.sliding_window are unused.
 * rope_cs: a g4_ropeTable table for p.theta / p.apply_divisor of
 * rope_rows >= p.max_seq_len rows, or NULL to compute the RoPE angles per
 * call (same values). k_parts = v_parts = NULL: q only, for a consumer layer
 * (src/engine.ts:1547-1574 skip the k/v projections, k_norm, v_norm and the
 * store there); k_norm_w and the pools are then not read and may be NULL. */
int g4_pagedAttnPrologue(g4_ctx* ctx, const float* q_parts, const float* k_parts,
                         const float* v_parts, uint32_t nparts, const uint16_t* q_norm_w,
                         const uint16_t* k_norm_w, const uint16_t* rope_freqs, float* q_out,
                         uint16_t* k_pool, uint16_t* v_pool, const int32_t* page_table,
                         const uint32_t* seq_lens, g4_paged_attn_fused_params p,
                         const float* rope_cs, uint32_t rope_rows);
/* g4_pagedAttnPrologue followed by g4_pagedAttnDecodeOps (the per-layer
 * attention block of a multi-sequence step, src/engine.ts:1556-1584 per
 * sequence) in one launch where the window takes at most 16 chunks of 64
 * positions (sliding windows up to 1024, or a cache of at most 1024
 * positions), head_dim 256, 8 query heads per KV head, <= 64 sequences and
 * nparts <= 8: every workgroup sums its sequence's q (and k/v) partials,
 * forms q_norm + RoPE, the chunk that ends at the sequence's position forms
 * and appends its K/V row, each chunk attends, and the last chunk of each
 * sequence to arrive merges them and writes the output (and, with ops, the
 * o projection's operand blocks). Other shapes make the two calls. q_out
 * (or NULL) receives q after q_norm + RoPE as the prologue writes it. The
 * row a sequence appends is read by that sequence only in this launch: a
 * batch whose rows share pages (the rows of one prompt, a batched prefill)
 * takes the two calls, whose first appends every row before the second
 * reads any. workspace: g4_pagedAttnBlock_workspace_size bytes, 16-byte
 * aligned, zero before the first call (calls leave its arrival counters
 * zero; calls sharing it must not overlap). An MI355X launch fusion with
 * no counterpart in the reference. */
int g4_pagedAttnBlock_workspace_size(g4_paged_attn_fused_params p, uint32_t nparts, size_t* bytes);
int g4_pagedAttnBlock(g4_ctx* ctx, const float* q_parts, const float* k_parts, const float* v_parts, uint32_t nparts,
                      const uint16_t* q_norm_w, const uint16_t* k_norm_w, const uint16_t* rope_freqs, float* q_out,
                      uint16_t* k_pool, uint16_t* v_pool, const int32_t* page_table, const uint32_t* seq_lens,
                      float* output, void* ops, g4_paged_attn_fused_params p, void* workspace,
                      size_t workspace_bytes, const float* rope_cs, uint32_t rope_rows);
/* seq_lens[s] += delta for s < num_seqs, on the stream (the device-side
 * length counters a captured multi-sequence step replays with). */
int g4_advanceSeqLens(g4_ctx* ctx, uint32_t* seq_lens, uint32_t num_seqs, uint32_t delta);
/* Append one row per sequence at position seq_lens[s] - 1 (after the host or
 * a previous kernel advanced seq_lens). k_in/v_in are [num_seqs][nkh*hd] f32. */
int g4_pagedKvStore(g4_ctx* ctx, const float* k_in, const float* v_in, uint16_t* k_pool,
                    uint16_t* v_pool, const int32_t* page_table, const uint32_t* seq_lens,
                    g4_paged_attn_params p);

/* shaders/per_head_rms_norm_no_weight.wgsl:8 — Params {num_heads, head_dim, eps, pad}; in place. */
typedef struct { uint32_t num_heads, head_dim; float eps; uint32_t pad; } g4_per_head_norm_params;
int g4_perHeadRmsNormNoWeight(g4_ctx* ctx, float* data, g4_per_head_norm_params p);

/* shaders/fused_per_head_norm_rope.wgsl:13 — Params {num_heads, head_dim, eps,
 * position, theta, apply_divisor}; bindings data (rw), weight f16[head_dim],
 * params, rope_freqs f16[head_dim/2]. */
typedef struct {
  uint32_t num_heads, head_dim;
  float eps;
  uint32_t position;
  float theta;
  uint32_t apply_divisor;
} g4_norm_rope_params;
int g4_fusedPerHeadNormRope(g4_ctx* ctx, float* data, const uint16_t* weight,
                            g4_norm_rope_params p, const uint16_t* rope_freqs);
int g4_fusedPerHeadNormRope_dev(g4_ctx* ctx, float* data, const uint16_t* weight,
                                g4_norm_rope_params p, const uint16_t* rope_freqs,
                                const uint32_t* position_dev);

/* shaders/rms_norm.wgsl:2 — Params {hidden_size, eps}. */
typedef struct { uint32_t hidden_size; float eps; } g4_rms_norm_params;
int g4_rmsNorm(g4_ctx* ctx, const float* input, const uint16_t* weight, float* output,
               g4_rms_norm_params p);

/* shaders/fused_norm_add.wgsl:2 — Params {size, eps}; out = residual + norm(in)*w. */
typedef struct { uint32_t size; float eps; } g4_norm_add_params;
int g4_fusedNormAdd(g4_ctx* ctx, const float* input, const uint16_t* weight, const float* residual,
                    float* output, g4_norm_add_params p);

/* shaders/gelu_mul.wgsl:7 — uniform size. */
int g4_geluMul(g4_ctx* ctx, const float* gate, const float* up, float* output, uint32_t size);

/* shaders/logit_softcap.wgsl:5 — Params {size, cap}; in place. */
typedef struct { uint32_t size; float cap; } g4_softcap_params;
int g4_logitSoftcap(g4_ctx* ctx, float* logits, g4_softcap_params p);

/* shaders/embedding_lookup.wgsl:2,12 — Params {hidden_size, token_id};
 * out[i] = f32(embedding[token_id * hidden_size + i]) * sqrt(f32(hidden_size)),
 * the first dispatch of a forward (src/engine.ts:1488,1511-1514). `embedding`
 * is the f16 table [num_rows][hidden_size]; num_rows bounds token_id (the
 * shader has no bound): a token_id >= num_rows is G4_ERR_ARG. */
typedef struct { uint32_t hidden_size; uint32_t token_id; } g4_embedding_params;
int g4_embeddingLookup(g4_ctx* ctx, const uint16_t* embedding, uint32_t num_rows, float* output,
                       g4_embedding_params p);
/* As g4_embeddingLookup with the token read from device memory (the argmax
 * result that the reference copies into this uniform, src/engine.ts:1724-1727);
 * p.token_id is ignored. A device token >= num_rows writes a zero row. */
int g4_embeddingLookup_dev(g4_ctx* ctx, const uint16_t* embedding, uint32_t num_rows, float* output,
                           g4_embedding_params p, const uint32_t* token_dev);

/* `count` lookups at once: output row r [hidden_size] from tokens_dev[r] (a
 * token >= num_rows writes a zero row). The embedding of every row of a
 * multi-sequence step, or of every prompt token of a batched prefill
 * (src/engine.ts:1923-1938 runs one embedding lookup per prompt token);
 * count <= 65535. */
int g4_embeddingLookupBatch(g4_ctx* ctx, const uint16_t* embedding, uint32_t num_rows, float* output,
                            uint32_t hidden_size, const uint32_t* tokens_dev, uint32_t count);

/* *position_dev += delta on the stream: the device-side step counter that lets
 * a captured decode graph be replayed token after token (the role of the
 * per-forward uniform patches, src/engine.ts:1487-1504). */
int g4_advancePosition(g4_ctx* ctx, uint32_t* position_dev, uint32_t delta);

/* shaders/argmax.wgsl:1-3 — result u32[1]; size = vocabulary. */
int g4_argmax(g4_ctx* ctx, const float* logits, uint32_t* result, uint32_t size);
/* shaders/topk256.wgsl:1-3 — result f32[512] = (max, bitcast idx) per residue class. */
int g4_topk256(g4_ctx* ctx, const float* logits, float* result, uint32_t size);
/* The same per row of `batch` rows of `size` logits each (sampling at M > 1):
 * result[r] is row r's argmax / result[512 r .. 512 r + 511] its top-k pairs,
 * each equal to what the one-row call returns for that row. batch <= 1024. */
int g4_argmaxBatch(g4_ctx* ctx, const float* logits, uint32_t* result, uint32_t size, uint32_t batch);
int g4_topk256Batch(g4_ctx* ctx, const float* logits, float* result, uint32_t size, uint32_t batch);
/* g4_argmaxBatch, then positions[r] += delta for every row, in the same
 * launch: the greedy sample (shaders/argmax.wgsl) and the position step the
 * host takes after it (src/engine.ts:1724-1727) at the end of a captured
 * decode step. */
int g4_argmaxAdvance(g4_ctx* ctx, const float* logits, uint32_t* result, uint32_t size, uint32_t batch,
                     uint32_t* positions, uint32_t delta);

/* ------------------------------------------------------------------------ */
/* Fused step kernels (the MI355X decode path; each is equivalent to a run   */
/* of the per-key kernels above, named in its comment)                       */
/* ------------------------------------------------------------------------ */

/* rmsNorm -> matmulQuant: y = W . (x * w / rms(x)). src/engine.ts:1546-1547.
 * p.N (the hidden width) is 1536 or 2048. */
int g4_rmsNormMatmul_q4k(g4_ctx* ctx, const float* x, const uint16_t* norm_w, const void* weight,
                         float* y, g4_matmul_params p, float eps);
/* fusedNormAdd -> rmsNorm -> matmulQuant gate/up -> geluMul:
 *   h = residual + o * w_post / rms(o)   (written to h_out when non-NULL)
 *   x = h * w_pre / rms(h)
 *   out = gelu(W_gate . x) * (W_up . x)
 * src/engine.ts:1587-1604. Gate and up are separate raw Q4_K tensors of
 * [I, N]; p.M = I, p.N = N (the hidden width, 1536 or 2048). */
int g4_normAddGateUpGelu_q4k(g4_ctx* ctx, const float* o, const uint16_t* w_post,
                             const float* residual, const uint16_t* w_pre, const void* w_gate,
                             const void* w_up, float* h_out, float* out, g4_matmul_params p,
                             float eps);

/* The FFN of g4_normAddGateUpGelu_q4k and the down projection with the
 * activation handed over pre-digitised (an MI355X form of the gelu_mul ->
 * matmulQuant down hand-off, src/engine.ts:1604-1605; no reference
 * counterpart for the digit block itself). The gate/up launch also writes
 * its outputs as a digit block (two 8-bit digit planes, a scale per 8
 * elements and the digit sums: g4_digitsBytes(K) bytes, K = the FFN width),
 * and the down launch reads that block instead of digitising the f32
 * vector itself. g4_normAddGateUpGeluDigits_q4k: p.N = 1536, p.M a multiple
 * of 256; g4_matmulQuantDigits_q6k: p.N (= the FFN width) 6144 or 12288. */
int g4_digitsBytes(uint32_t K, size_t* bytes);
int g4_normAddGateUpGeluDigits_q4k(g4_ctx* ctx, const float* o, const uint16_t* w_post,
                                   const float* residual, const uint16_t* w_pre,
                                   const void* w_gate, const void* w_up, float* h_out, float* out,
                                   void* digits, g4_matmul_params p, float eps);
int g4_matmulQuantDigits_q6k(g4_ctx* ctx, const void* digits, const void* weight, float* output,
                             g4_matmul_params p);

/* [fusedNormAdd ->] rmsNorm -> matmulQuant over up to 4 matrices that share
 * the input (src/engine.ts:1546-1554 for q/k/v, :1606 + :1621-1625 + :1686-1701
 * for the post-FFN add, final norm, LM head and softcap):
 *   residual == NULL:  x' = x * w1 / rms(x)
 *   residual != NULL:  h = residual + x * w1 / rms(x)   (written to h_out if non-NULL)
 *                      x' = h * w2 / rms(h)
 *   outputs[i] = weights[i] . x'  (rows[i] x N), then tanh(y/cap)*cap if
 *   softcap_cap != 0.
 * wtype 0 = Q4_K, 1 = Q6_K; N (the hidden width) is 1536 or 2048; norm
 * weights are f16[N]. */
int g4_normAddMatmulSegments(g4_ctx* ctx, int wtype, const float* x, const uint16_t* w1,
                             const float* residual, const uint16_t* w2, float* h_out,
                             const void* const* weights, float* const* outputs,
                             const uint32_t* rows, int nseg, uint32_t N, float eps,
                             float softcap_cap);
/* The same with the residual form's sum scaled by the f16 scalar at
 * out_scale before it is written to h_out and normalised by w2:
 *   h = (residual + x * w1 / rms(x)) * out_scale[0];  x' = h * w2 / rms(h)
 * (src/engine.ts:1611-1616: the per-layer-embedding tail's rmsNorm +
 * pleSkipScaleAdd, shaders/ple_skip_scale_add.wgsl, ahead of the next
 * layer's attention rmsNorm). out_scale NULL is g4_normAddMatmulSegments. */
int g4_normAddScaleMatmulSegments(g4_ctx* ctx, int wtype, const float* x, const uint16_t* w1,
                                  const float* residual, const uint16_t* out_scale, const uint16_t* w2,
                                  float* h_out, const void* const* weights, float* const* outputs,
                                  const uint32_t* rows, int nseg, uint32_t N, float eps,
                                  float softcap_cap);
/* The LM head with greedy sampling in two launches: g4_normAddMatmulSegments
 * over one matrix (logits[rows], softcapped when softcap_cap != 0), whose
 * workgroups also keep the argmax candidate of the rows they store, then the
 * reduction of those candidates: *result = g4_argmax(logits, rows), ties
 * and NaN as shaders/argmax.wgsl:12-33, without reading the logits back;
 * with `positions` non-NULL, *positions += delta (the GPU-written position
 * of src/engine.ts:1724-1727). Replaces src/engine.ts:1686-1717 (final norm,
 * LM head, softcap, argmax). */
int g4_normAddMatmulArgmax(g4_ctx* ctx, int wtype, const float* x, const uint16_t* w1,
                           const float* residual, const uint16_t* w2, float* h_out,
                           const void* weight, float* logits, uint32_t rows, uint32_t N, float eps,
                           float softcap_cap, uint32_t* result, uint32_t* positions,
                           uint32_t delta);

/* The LM head with top-k sampling in two launches: g4_normAddMatmulSegments
 * over one matrix (logits[rows], softcapped when softcap_cap != 0), whose
 * workgroups also keep, for each residue class i mod 256, the first strict
 * maximum among the rows they store, then the reduction of those candidates:
 * result f32[512] = g4_topk256(logits, rows) (per class (max, bitcast index),
 * ties, NaN and the (-1e30, 0) default as shaders/topk256.wgsl:8-20), without
 * reading the logits back. Replaces src/engine.ts:1686-1701 + 1735-1740
 * (final norm, LM head, softcap, topk256). */
int g4_normAddMatmulTopk(g4_ctx* ctx, int wtype, const float* x, const uint16_t* w1,
                         const float* residual, const uint16_t* w2, float* h_out,
                         const void* weight, float* logits, uint32_t rows, uint32_t N, float eps,
                         float softcap_cap, float* result);

/* The same over `batch` activation vectors at once (ragged multi-sequence
 * decode: src/engine.ts:1546-1554 run once per sequence). x, residual and
 * h_out are [batch][N]; outputs[i] is [batch][rows[i]]. w1 == NULL skips the
 * norms (plain matmul). 1 <= batch <= 64. Runs on the matrix cores; the
 * activation operands live in the context scratch between its two launches. */
int g4_normAddMatmulSegmentsBatch(g4_ctx* ctx, int wtype, const float* x, const uint16_t* w1,
                                  const float* residual, const uint16_t* w2, float* h_out,
                                  const void* const* weights, float* const* outputs,
                                  const uint32_t* rows, int nseg, uint32_t N, float eps,
                                  float softcap_cap, uint32_t batch);
/* g4_normAddGateUpGelu_q4k over `batch` vectors (1..64): o, residual, h_out
 * are [batch][N], out is [batch][p.M]. */
int g4_normAddGateUpGeluBatch(g4_ctx* ctx, const float* o, const uint16_t* w_post,
                              const float* residual, const uint16_t* w_pre, const void* w_gate,
                              const void* w_up, float* h_out, float* out, g4_matmul_params p,
                              float eps, uint32_t batch);

/* The pieces of a multi-sequence step, for callers that chain them without
 * an intermediate reduction (src/engine.ts:1545-1625 per sequence, for many
 * sequences at once).
 *
 * g4_batchPrep: x = the sum of the nparts chunks of x_parts
 * [nparts][batch][N] (added in chunk order); then w1 == NULL: out = x;
 * residual == NULL: out = x * w1 / rms(x) (rmsNorm); else
 * h = residual + x * w1 / rms(x) (written to h_out when non-NULL) and
 * out = h * w2 / rms(h) (fusedNormAdd -> rmsNorm). N is 1536 or 2048. When
 * `ops` is non-NULL (batch <= 64) it also receives the matrix-core operand
 * blocks of `out` (g4_batchOperandBytes bytes), which the matmul entries
 * below take so that their workgroups need not rebuild them from `out`. */
int g4_batchOperandBytes(uint32_t N, uint32_t batch, size_t* bytes);
int g4_batchPrep(g4_ctx* ctx, const float* x_parts, uint32_t nparts, const uint16_t* w1,
                 const float* residual, const uint16_t* w2, float* h_out, float* out, void* ops,
                 uint32_t N, uint32_t batch, float eps);
/* g4_batchPrep with the residual form's sum scaled by the f16 scalar at
 * out_scale (NULL: 1) before it is written to h_out and normalised:
 * h = (residual + x * w1 / rms(x)) * out_scale[0] (the per-layer-embedding
 * tail, src/engine.ts:1614-1616); and with w2 == NULL, out = h (no second
 * norm: the input of the per-layer-embedding gate, src/engine.ts:1612). */
int g4_batchPrepScale(g4_ctx* ctx, const float* x_parts, uint32_t nparts, const uint16_t* w1,
                      const float* residual, const uint16_t* out_scale, const uint16_t* w2, float* h_out,
                      float* out, void* ops, uint32_t N, uint32_t batch, float eps);
/* x [batch][N] f32 (with `ops` from g4_batchPrep of the same x, or NULL)
 * times up to 4 matrices on the matrix cores, K split into
 * *ksplit <= max_ksplit chunks (chosen to fill the device); outputs[i]
 * receives [*ksplit][batch][rows[i]] partial sums (one chunk each) and must
 * hold max_ksplit * batch * rows[i] floats. The consumer adds the chunks in
 * order: g4_batchPrep, g4_pagedAttnPrologue. softcap_cap > 0 (tanh softcap
 * of the outputs) needs max_ksplit == 1. Prebuilt `ops` are taken for N
 * 1536, 2048 and 4096 (the norm prologue's and the attention merge's
 * widths); other widths with ops are G4_ERR_UNSUPPORTED. */
int g4_matmulSegmentsBatchPartial(g4_ctx* ctx, int wtype, const float* x, const void* ops,
                                  const void* const* weights, float* const* outputs,
                                  const uint32_t* rows, int nseg, uint32_t N, uint32_t batch,
                                  uint32_t max_ksplit, float softcap_cap, uint32_t* ksplit);
/* out = gelu(W_gate . x) * (W_up . x) for x [batch][p.N] (already
 * normalised; `ops` as above). */
int g4_gateUpGeluBatch(g4_ctx* ctx, const float* x, const void* ops, const void* w_gate,
                       const void* w_up, float* out, g4_matmul_params p, uint32_t batch);
/* The FFN's hand-off at batch sizes 1..64 (the batched counterpart of
 * g4_normAddGateUpGeluDigits_q4k; src/engine.ts:1594-1601 runs gate, up,
 * geluMul and down as four dispatches per token): g4_gateUpGeluBatch (Q4_K
 * gate and up, p.M 6144 or 12288; `out` may be NULL) that also writes its
 * product as sub-block-scaled operand blocks (down_ops,
 * g4_batchSubOperandBytes(p.M, batch) bytes: each 32 consecutive values of
 * a vector scaled by their own power of two, split into f16 hi + lo), which
 * g4_matmulSubBatchPartial multiplies by a Q6_K down projection
 * (shaders/matmul_quant.wgsl over Q6_K, src/gguf.ts:323-368) without
 * rebuilding them from f32 values: out [*ksplit][batch][M] partial sums as
 * g4_matmulSegmentsBatchPartial's (max_ksplit * batch * M floats). */
int g4_batchSubOperandBytes(uint32_t K, uint32_t batch, size_t* bytes);
int g4_gateUpGeluBatchOps(g4_ctx* ctx, const float* x, const void* ops, const void* w_gate,
                          const void* w_up, float* out, void* down_ops, g4_matmul_params p, uint32_t batch);
int g4_matmulSubBatchPartial(g4_ctx* ctx, const void* ops, const void* weight, float* out, uint32_t M,
                             uint32_t K, uint32_t batch, uint32_t max_ksplit, uint32_t* ksplit);

/* ------------------------------------------------------------------------ */
/* Debug / test exports                                                      */
/* ------------------------------------------------------------------------ */

/* Dequantize nblocks raw blocks to f32 (bit-exact vs src/gguf.ts:168-210 / :323-368),
 * through the unpack of the one-vector matvec's register units (path 0 below). */
int g4_dequant_q4k(g4_ctx* ctx, const void* blocks, uint64_t nblocks, float* out);
int g4_dequant_q6k(g4_ctx* ctx, const void* blocks, uint64_t nblocks, float* out);
/* The weight values as one kernel family of the hot path unpacks them
 * (GGUFParser.dequantizeQ4_K / dequantizeQ6_K, src/gguf.ts:168-210 / :323-368,
 * restated with the family's own loads and code/scale extraction; blocks is
 * 16-byte aligned, one-block rows, wtype 0 = Q4_K, 1 = Q6_K):
 *   path 0: register units of the one-vector matvec (buffer loads, byte shifts);
 *   path 1: units read from blocks staged in LDS (the tile-walking matvec and
 *           the 2-8 vector matvec);
 *   path 2: the matrix-core operands of the M >= 16 matmul: Q4_K d*(sc*q) -
 *           dmin*m as the reference; Q6_K d times sc*(q-32) rounded once to
 *           f16 (exact for |sc*(q-32)| <= 2048).
 * Paths 0 and 1 are bit-exact with the reference's f32 values. */
int g4_dequantPath(g4_ctx* ctx, int wtype, int path, const void* blocks, uint64_t nblocks, float* out);

/* Blocks to f16 values, each the reference's f32 dequantized value rounded
 * to nearest even (tensorToF16, src/engine.ts:570-579): wtype 0 Q4_K and 1
 * Q6_K (the f32 values of g4_dequantPath's path 0; the tied token table the
 * lookup reads), 2 Q5_K (src/gguf.ts:218-257; the per-layer table's values
 * and Q5_K matrices), 3 Q8_0 (src/gguf.ts:115-131; nblocks of 32 values).
 * blocks and out 16-byte aligned; out holds nblocks * 256 values (Q8_0:
 * nblocks * 32). */
int g4_dequantF16(g4_ctx* ctx, int wtype, const void* blocks, uint64_t nblocks, uint16_t* out);

/* Measurement probe: reads bytes of src once with 16-byte loads (nwgs
 * workgroups of 256 threads, 4 loads in flight per thread) under a cache
 * policy (0 plain, 1 non-temporal as the one-matrix Q4_K matvec reads its
 * weights, 2 device scope as the attention's partials are read) and writes
 * one word per workgroup to sink[nwgs]. It times the pure-streaming floor of
 * a launch and calibrates the HBM byte counters. */
int g4_streamRead(g4_ctx* ctx, const void* src, uint64_t bytes, int policy, uint32_t nwgs, uint32_t* sink);

/* ---- per-layer embeddings (Gemma 4 PLE) ----
 *
 * g4_pleStage1Fuse: shaders/ple_stage1_fuse.wgsl for every layer of `count`
 * rows in one launch (replaces the per-layer dispatches of
 * src/engine.ts:1529-1535). projected [count][num_layers*256] is
 * per_layer_model_proj . embedding; table_q5k holds the per_layer_token_embd
 * Q5_K blocks, table_rows x num_layers of them (row = token, one block =
 * one layer's 256 values, src/engine.ts:626-700); each value is rounded to
 * f16 as the reference's upload does. Row b's token is tokens_dev[b] (NULL:
 * `token`, count 1); a token past the table reads a zero row.
 *   ple_inputs[b][l*256 + t] = (p/rms_l * f32(norm_w[t]) + f16(table) * 16) / sqrt(2)
 * per_layer_dim must be 256. */
int g4_pleStage1Fuse(g4_ctx* ctx, const float* projected, const uint16_t* norm_w, const void* table_q5k,
                     uint32_t table_rows, uint32_t token, const uint32_t* tokens_dev, float* ple_inputs,
                     uint32_t num_layers, uint32_t per_layer_dim, float eps, uint32_t count);
/* shaders/ple_gelu_mul.wgsl: output[i] = gelu(gate[i]) * ple_inputs[layer_offset + i]. */
int g4_pleGeluMul(g4_ctx* ctx, const float* gate, const float* ple_inputs, float* output, uint32_t layer_offset,
                  uint32_t size);
/* shaders/ple_skip_scale_add.wgsl: hidden[i] = (hidden[i] + post_normed[i]) * f32(scale[0]). */
int g4_pleSkipScaleAdd(g4_ctx* ctx, float* hidden, const float* post_normed, const uint16_t* scale,
                       uint32_t size);
/* y[b][m] = W[m] . x[b] for f16 rows W [M][N] (N 256, 1536, 2048, 4096, 6144
 * or 12288) and
 * `batch` f32 vectors: the reference's matmulQuant on its f16 weights
 * (shaders/matmul_quant.wgsl), as PLE runs it for per_layer_model_proj,
 * inp_gate and proj (src/engine.ts:1521-1524, 1611, 1613). */
int g4_matmulF16(g4_ctx* ctx, const float* x, const uint16_t* weight, float* y, uint32_t M, uint32_t N,
                 uint32_t batch);
/* The PLE gate (src/engine.ts:1606 + 1611-1612): with w1 (batch 1) the
 * vector is h = residual + x * w1 / rms(x) (fusedNormAdd; written to h_out
 * when non-NULL, which must not alias x or residual), else x [batch][N];
 * out[b][m] = gelu(w_gate[m] . h_b) * ple_inputs[b * ple_stride +
 * layer_offset + m]. */
int g4_pleGate(g4_ctx* ctx, const float* x, const uint16_t* w1, const float* residual, float* h_out,
               const uint16_t* w_gate, const float* ple_inputs, uint32_t ple_stride, uint32_t layer_offset,
               float* out, uint32_t M, uint32_t N, float eps, uint32_t batch);

/* GGUF v2/v3 model files (replaces GGUFParser, src/gguf.ts:75-101 header,
 * :103-134 key/values, :136-160 tensor infos and data offset, :385-395 tensor
 * sizes). The file is memory-mapped (g4_gguf_open) or read from caller memory
 * that outlives the handle (g4_gguf_open_memory); only the header is parsed,
 * every read bounds-checked: a malformed or truncated file is G4_ERR_INVALID
 * with the reason in g4_last_error. The data section starts at the header's
 * end rounded up to general.alignment (32 when absent, as src/gguf.ts:97).
 * Value types are GGUF's (0 u8 ... 12 f64; 8 string, 9 array). Tensor types
 * with known sizes: 0 F32, 1 F16, 8 Q8_0, 12 Q4_K, 13 Q5_K, 14 Q6_K, 30 BF16;
 * other types parse (nbytes 0) but have no data access. Strings returned are
 * not NUL-terminated (use len); key and tensor names are. Returned pointers
 * live until g4_gguf_close. The handle is read-only and may be shared by
 * threads. */
typedef struct g4_gguf g4_gguf;
int g4_gguf_open(const char* path, g4_gguf** out);
int g4_gguf_open_memory(const void* data, size_t bytes, g4_gguf** out);
int g4_gguf_close(g4_gguf* g);
int g4_gguf_info(const g4_gguf* g, uint32_t* version, uint64_t* tensor_count, uint64_t* kv_count,
                 uint64_t* data_offset, uint32_t* alignment);
/* *index = -1 when absent. */
int g4_gguf_find_key(const g4_gguf* g, const char* key, int64_t* index);
/* type = the value type; for arrays arr_type = the element type and count
 * the element count (1 and 0 for scalars). */
int g4_gguf_kv(const g4_gguf* g, uint64_t index, const char** key, uint32_t* type, uint32_t* arr_type,
               uint64_t* count);
/* A numeric scalar (element 0) or array element, as f64, i64 and u64. */
int g4_gguf_kv_number(const g4_gguf* g, uint64_t index, uint64_t element, double* f, int64_t* i,
                      uint64_t* u);
/* A string (element 0) or string-array element. */
int g4_gguf_kv_string(const g4_gguf* g, uint64_t index, uint64_t element, const char** s, uint64_t* len);
int g4_gguf_find_tensor(const g4_gguf* g, const char* name, int64_t* index);
/* dims[4] (GGUF order, dims[0] the contiguous one; unused dims 1); offset is
 * relative to the data section. */
int g4_gguf_tensor(const g4_gguf* g, uint64_t index, const char** name, uint32_t* n_dims, uint64_t* dims,
                   uint32_t* type, uint64_t* offset, uint64_t* nbytes);
/* Host address of the tensor's bytes inside the mapping. */
int g4_gguf_tensor_data(const g4_gguf* g, uint64_t index, const void** data);
/* Copies the tensor's GGUF bytes unchanged to device memory (the quantized
 * blocks are what the matvecs read; the reference instead dequantizes every
 * tensor to f16 at upload, src/engine.ts:570-593). Synchronous; not during
 * graph capture. */
int g4_gguf_upload(g4_ctx* ctx, const g4_gguf* g, uint64_t index, void* dst, size_t dst_bytes);
/* An F32, F16 or BF16 tensor to f16 on the device, rounded to nearest even
 * (src/engine.ts:570-579 for the norm weights, rope_freqs and other f32
 * tensors). */
int g4_gguf_upload_f16(g4_ctx* ctx, const g4_gguf* g, uint64_t index, uint16_t* dst, size_t dst_elems);

/* Seeded synthetic inputs, generated on the device (counter-based SplitMix64;
 * block b of a stream draws words 32b.., element i of a normal stream words
 * 2i and 2i+1; Box-Muller in f64). */
uint64_t g4_splitmix64(uint64_t seed, uint64_t idx);
int g4_fill_q4k(g4_ctx* ctx, void* dst, uint64_t nblocks, uint64_t seed);
int g4_fill_q6k(g4_ctx* ctx, void* dst, uint64_t nblocks, uint64_t seed);
int g4_fill_q5k(g4_ctx* ctx, void* dst, uint64_t nblocks, uint64_t seed);
int g4_fill_normal_f32(g4_ctx* ctx, float* dst, uint64_t n, uint64_t seed, float mean, float std);
int g4_fill_normal_f16(g4_ctx* ctx, uint16_t* dst, uint64_t n, uint64_t seed, float mean,
                       float std);

#ifdef __cplusplus
}
#endif
#endif /* G4HIP_H */
