/*
 * g4_oracle.h — CPU oracle for the gemma4 decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker that the HIP path is
 * compared against; it is loaded only by tests/, by the smoke() check and by
 * the cpu_baseline leg of bench.py. No product code links or calls it.
 *
 * Every function restates one piece of the reference's algorithm and cites the
 * reference file:line it follows. Accumulations are carried in double so that
 * the oracle is at least as accurate as the reference's f32 shaders; values
 * are stored as f32 at the same points where the reference stores f32.
 */
#ifndef G4_ORACLE_H
#define G4_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- f16 conversions (src/gguf.ts:103-113, :402-473) ---- */
float g4o_f16_to_f32(uint16_t h);
uint16_t g4o_f32_to_f16_rne(float f);   /* Float16Array path, src/gguf.ts:432-436 */
uint16_t g4o_f32_to_f16_trunc(float f); /* manual fallback, src/gguf.ts:439-471 */

/* ---- K-quant unpack (src/gguf.ts:157-210, :316-368) ---- */
void g4o_q4k_scale_min(const uint8_t scales12[12], int j, int* sc, int* m);
void g4o_dequant_q4k(const uint8_t* blocks, size_t nblocks, float* out);
void g4o_dequant_q6k(const uint8_t* blocks, size_t nblocks, float* out);
void g4o_dequant_q5k(const uint8_t* blocks, size_t nblocks, float* out); /* src/gguf.ts:218-257 */
void g4o_dequant_q8_0(const uint8_t* blocks, size_t nblocks, float* out); /* src/gguf.ts:115-131 */

/* ---- matvec (shaders/matmul_quant.wgsl:12-54; rows M, reduction N) ---- */
void g4o_matmul_f16w(const float* x, const uint16_t* W, float* y, uint32_t M, uint32_t N);
void g4o_matmul_q4k(const float* x, const uint8_t* W, float* y, uint32_t M, uint32_t N);
void g4o_matmul_q6k(const float* x, const uint8_t* W, float* y, uint32_t M, uint32_t N);

/* ---- norms / activations ---- */
void g4o_rms_norm(const float* in, const uint16_t* w, float* out, uint32_t H, float eps);
void g4o_fused_norm_add(const float* in, const uint16_t* w, const float* residual, float* out,
                        uint32_t N, float eps);
void g4o_gelu_mul(const float* gate, const float* up, float* out, uint32_t n);
void g4o_per_head_rms_norm_no_weight(float* data, uint32_t num_heads, uint32_t head_dim, float eps);
void g4o_rope_freq(float theta, uint32_t i, uint32_t head_dim, int apply_divisor,
                   const uint16_t* rope_freqs, float* freq_out);
void g4o_fused_per_head_norm_rope(float* data, const uint16_t* weight, uint32_t num_heads,
                                  uint32_t head_dim, float eps, uint32_t position, float theta,
                                  uint32_t apply_divisor, const uint16_t* rope_freqs);

/* ---- attention over an f16 position-major KV cache ---- */
void g4o_kv_cache_store_f16(const float* k_in, const float* v_in, uint16_t* k_cache,
                            uint16_t* v_cache, uint32_t num_kv_heads, uint32_t head_dim,
                            uint32_t position);
void g4o_attn_score(const float* q, const uint16_t* k_cache, float* scores, uint32_t nqh,
                    uint32_t nkh, uint32_t hd, uint32_t seq_len, float scale, uint32_t window);
void g4o_softmax(float* scores, uint32_t num_heads, uint32_t seq_len);
void g4o_attn_output(const float* probs, const uint16_t* v_cache, float* out, uint32_t nqh,
                     uint32_t nkh, uint32_t hd, uint32_t seq_len);
/* score -> softmax -> output in one call, f64 throughout (the attention oracle) */
void g4o_attention(const float* q, const uint16_t* k_cache, const uint16_t* v_cache, float* out,
                   uint32_t nqh, uint32_t nkh, uint32_t hd, uint32_t seq_len, float scale,
                   uint32_t window);
/* same, with K/V rows fetched through a page table of `page_size`-token pages */
void g4o_attention_paged(const float* q, const uint16_t* k_pool, const uint16_t* v_pool,
                         const int32_t* page_table, uint32_t page_size, float* out, uint32_t nqh,
                         uint32_t nkh, uint32_t hd, uint32_t seq_len, float scale,
                         uint32_t window);

/* ---- per-layer embeddings (shaders/ple_*.wgsl) ---- */
void g4o_ple_stage1(const float* projected, const uint16_t* norm_w, const uint16_t* embed_row,
                    float* ple_inputs, uint32_t num_layers, uint32_t dim, float eps);
void g4o_ple_skip_scale_add(float* hidden, const float* post_normed, uint16_t scale, uint32_t n);

/* ---- LM head tail ---- */
void g4o_logit_softcap(float* logits, uint32_t n, float cap);
uint32_t g4o_argmax(const float* logits, uint32_t n);
void g4o_topk256(const float* logits, uint32_t n, float out512[512]);
void g4o_topk_sort(const float in512[512], uint32_t ids_out[256], float vals_out[256]);

/* ---- seeded synthetic inputs (SplitMix64, counter based) ---- */
uint64_t g4o_splitmix64(uint64_t seed, uint64_t idx);
void g4o_gen_q4k(uint64_t seed, uint64_t nblocks, uint8_t* out);
void g4o_gen_q6k(uint64_t seed, uint64_t nblocks, uint8_t* out);
void g4o_gen_normal_f32(uint64_t seed, uint64_t n, float mean, float std, float* out);
void g4o_gen_normal_f16(uint64_t seed, uint64_t n, float mean, float std, uint16_t* out);

#ifdef __cplusplus
}
#endif
#endif
