/*
 * kanso_oracle.h — CPU restatement of kanso-infer's attention-path arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker the parity tests,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg compare the HIP
 * library against. No product code links, loads or calls it.
 *
 * The reference is Rust (kanso-infer; no toolchain for it exists in this
 * environment), so each function restates the cited Rust source line by line:
 * the same loop order, the same f32 operations, no fused multiply-add (the
 * library is compiled with -ffp-contract=off, as Rust never contracts).
 *
 * Pinning (what checks each function besides the HIP comparison) is recorded in
 * the tests under tests/test_oracle_*.py. Unpinned: the Q4_K quantizer's byte
 * choice (candle's QTensor::quantize is not available, see
 * oracle_quantize_row_q4_k), and byte parity of the FP8 encoder with the float8
 * 0.7.0 crate (not vendored; the encoder here is pinned to round-to-nearest-even
 * by brute force, see oracle_f32_to_e4m3).
 */
#ifndef KANSO_ORACLE_H
#define KANSO_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#include "../include/kanso_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- attention ---------------------------------------------------------- */

/* cpu_paged_attention (src/metal/paged_attention.rs:84-178), F32 pool. */
void oracle_paged_attention(const float* q, const float* k_cache, const float* v_cache,
                            const uint32_t* block_tables, const uint32_t* context_lens,
                            const kanso_paged_attention_params* p, float* out);

/* Mixed-batch attention of forward_batch_rows (src/model.rs:1689-1714): per
 * sequence, gather the context (dequantized for INT8 / Q8_0 pools exactly as
 * gather_dequantized_blocks, quantized_storage.rs:284-383), then per query head
 * and row: scores with the offset causal limit (model.rs:1510-1527), max, exp,
 * sum, 1/sum, weighted V — the arithmetic of cpu_paged_attention. nthreads > 1
 * runs sequences x heads on OpenMP threads (results do not depend on it).
 * Returns 0, or -1 for an empty / inconsistent sequence (model.rs:1488-1493). */
int oracle_ragged_attention(const float* q, const void* k_pool, const void* v_pool,
                            const void* k_scales, const void* v_scales,
                            const uint32_t* block_tables, const int32_t* cu_seqlens,
                            const uint32_t* context_lens,
                            const kanso_ragged_attention_params* p, float* out,
                            int nthreads);

/* ---- packing ------------------------------------------------------------ */

/* Host packing loop of Engine::step (src/engine.rs:376-402) plus
 * PaddedDecodeTables::new (src/model.rs:71-111). Outputs as kanso_packed_step but
 * host arrays. *max_blocks_out receives the padded width. Returns 0, -1 if a
 * position has no block (engine.rs:387-394). */
int oracle_pack_step(const kanso_seq_plan* plan, uint32_t num_seqs,
                     const uint32_t* token_arena, const uint32_t* table_arena,
                     uint32_t block_size, int32_t* cu_seqlens, int32_t* seq_of_query,
                     int32_t* positions, int64_t* slot_mapping, uint32_t* tokens,
                     uint32_t* block_tables, uint32_t* context_lens,
                     uint32_t* max_blocks_out);

/* ---- KV append / quantization ------------------------------------------ */

/* quantize_head_slice, INT8 arm (src/kv_cache/quantized_storage.rs:452-469). */
float oracle_quantize_head_int8(const float* x, uint32_t n, int8_t* q);
/* Host memory bandwidth, STREAM triad a = b + s c over n doubles per array with
 * nthreads OpenMP threads (first-touch initialisation by the same threads): best
 * of `reps` in GB/s, counting 24 bytes per element (src/hardware.rs:436-459). */
double oracle_stream_triad(uint64_t n, int nthreads, int reps);
float oracle_quantize_head_fp8(const float* x, uint32_t n, uint8_t* q);
uint8_t oracle_f32_to_e4m3(float x);
float oracle_e4m3_to_f32(uint8_t b);

/* BlockQ8_0::from_f32_slice (src/quant/q8_0.rs:13-32) on 32 values; returns d (f32). */
float oracle_quantize_q8_0_block(const float* x, int8_t* qs);

/* IEEE binary16 conversions (round to nearest even), used for GGUF scales. */
uint16_t oracle_f32_to_f16(float x);
float oracle_f16_to_f32(uint16_t h);

/* write_kv_slots for every pool kind (src/kv_cache/kind.rs:348-374). Returns 0,
 * -1 when a slot is outside the pool (kind.rs:130-137; nothing is written then). */
int oracle_kv_append(uint32_t kv_dtype, const float* k, const float* v,
                     const int64_t* slot_mapping, uint32_t num_tokens, uint32_t num_blocks,
                     uint32_t block_size, uint32_t num_kv_heads, uint32_t head_dim,
                     void* k_pool, void* v_pool, void* k_scales, void* v_scales);

/* ---- quantized GEMV ---------------------------------------------------- */

/* scalar_gemv_q8_0 (src/quant/q8_0.rs:69-93) on GGUF blocks {f16 d; i8 qs[32]}
 * (34 B) and on the reference's own blocks {f32 d; i8 qs[32]} (36 B). batch rows
 * of x are independent GEMVs. */
void oracle_gemv_q8_0(const void* w, const float* x, float* y, uint32_t rows,
                      uint32_t cols, uint32_t batch, int nthreads);
void oracle_gemv_q8_0_f32d(const void* w, const float* x, float* y, uint32_t rows,
                           uint32_t cols, uint32_t batch);

/* BlockQ4_K::dequantize (src/quant/q4_k.rs:30-55) on a GGUF block {f16 d; f16 dmin;
 * u8 scales[12]; u8 qs[128]} (144 B) and on the reference block with f32 d/dmin
 * (148 B). */
void oracle_dequant_q4_k(const void* blk, float* out256);
void oracle_dequant_q4_k_f32d(const void* blk, float* out256);
void oracle_get_scale_min_k4(uint32_t j, const uint8_t* scales12, uint8_t* sc, uint8_t* m);

/* scalar_gemv_q4_k (src/quant/q4_k.rs:162-186) on GGUF / reference blocks. */
void oracle_gemv_q4_k(const void* w, const float* x, float* y, uint32_t rows,
                      uint32_t cols, uint32_t batch, int nthreads);
void oracle_gemv_q4_k_f32d(const void* w, const float* x, float* y, uint32_t rows,
                           uint32_t cols, uint32_t batch);

/* Row quantizers used to build synthetic weights (GGUF layouts). Q8_0 is the
 * q8_0.rs:13-32 rule with d stored as f16. Q4_K is this build's own quantizer
 * (per 32-element sub-block: min/max to 6-bit scale/min, nibble = round((x+m)/s)),
 * because the reference takes Q4_K bytes from candle's QTensor::quantize, which is
 * not available here: its bytes are "parity unpinned"; only dequantization and the
 * GEMV over given bytes are pinned. */
void oracle_quantize_row_q8_0(const float* x, uint32_t n, void* blocks);
/* BlockQ8_0::dequantize (src/quant/q8_0.rs:35-39) over n elements of GGUF blocks. */
void oracle_dequant_row_q8_0(const void* blocks, uint32_t n, float* out);
void oracle_quantize_row_q4_k(const float* x, uint32_t n, void* blocks);

/* ---- decoder glue (config 5) -------------------------------------------- */

/* kanso_model_init_random restated (include/kanso_hip.h): splitmix64 (the
 * published output function), the Irwin-Hall(4) draw of one hash times
 * c = oracle_randn_scale(std), then oracle_quantize_row_q8_0 per row. Writes GGUF
 * Q8_0 bytes [rows][cols/32]. */
uint64_t oracle_splitmix64(uint64_t x);
float oracle_randn_scale(float std_dev);
int oracle_init_random_q8_0(uint64_t stream_seed, uint32_t rows, uint32_t cols, float c, void* gguf_out);

/* Model::rmsnorm (src/model.rs:653-659): x / sqrt(mean(x^2) + eps) * w, rows of n. */
void oracle_rmsnorm(const float* x, const float* w, float* y, uint32_t rows, uint32_t n,
                    float eps);
/* build_rope_table (src/model.rs:698-718): cos/sin [len][head_dim/2]. */
void oracle_rope_table(uint32_t len, uint32_t head_dim, float theta, float* cos_t,
                       float* sin_t);
/* rope_apply (src/model.rs:720-737), in place on [rows][heads][head_dim] with the
 * table rows of positions[rows]. */
void oracle_rope_apply(float* x, uint32_t rows, uint32_t heads, uint32_t head_dim,
                       const int32_t* positions, const float* cos_t, const float* sin_t);
/* silu(gate) * up (src/model.rs:375-378; metal/ops.rs cpu_silu_gate_multiply). */
void oracle_silu_mul(const float* gate, const float* up, float* y, uint32_t n);
/* greedy_token (src/sampler.rs:7-17): first maximum wins. */
uint32_t oracle_greedy(const float* logits, uint32_t n);
/* fnv1a_64 (src/bench.rs:20-29): one XOR per u32 token widened to u64. */
uint64_t oracle_fnv1a_64(const uint32_t* tokens, size_t n);

/* ---- batched llama forward (config 5), kanso_oracle_model.cpp ------------ */

/* weight_format: 0 = GGUF Q8_0 matrices; 1 = F32 row-major [rows][in] matrices and
 * embedding (the F32 LinearWeight of the reference's mock models, src/model.rs:509-587,
 * computed as x @ W^T in f32 with a sequential sum). */
typedef struct {
    uint32_t hidden, num_heads, num_kv_heads, head_dim, num_layers, intermediate, vocab;
    float eps, rope_theta;
    uint32_t weight_format;
    uint32_t kv_dtype; /* KANSO_KV_* of the pools passed to the forward */
    /* Granite multipliers (src/weights.rs:395-406), 0 = absent: embedding rows x
     * embedding_scale (model.rs:424-430); attention_scale replaces 1/sqrt(head_dim)
     * (:755-760); attention / FFN outputs x residual_scale before each residual add
     * (:739-744); logits x (1 / logit_scale) (:747-752). Each multiplies f32 values by
     * the f64 factor rounded to f32, as candle's affine does. */
    float embedding_scale, attention_scale, residual_scale, logit_scale;
} oracle_model_config;

/* Matrices in the config's weight_format and f32 norm weights; per-layer
 * fields are arrays of num_layers pointers. lm_head may alias embed (tied). */
typedef struct {
    const void* embed;
    const void* lm_head;
    const float* final_norm;
    const void* const* wq;
    const void* const* wk;
    const void* const* wv;
    const void* const* wo;
    const void* const* w_gate;
    const void* const* w_up;
    const void* const* w_down;
    const float* const* attn_norm;
    const float* const* ffn_norm;
    /* Q8_0 weights only: the GGUF type of each projection, [num_layers][7] in the
     * order wq, wk, wv, wo, w_gate, w_up, w_down (8 = Q8_0, 12 = Q4_K); NULL = all
     * Q8_0. */
    const uint32_t* formats;
} oracle_model_weights;

/* Model::forward_batch_rows with RowSelection::LastPerSequence (src/model.rs:
 * 1418-1739), the mixed-batch arm: embed, per layer RMSNorm -> Q/K/V -> RoPE ->
 * write_kv_slots into the per-layer F32 pools -> ragged attention with the offset
 * causal mask -> O + residual -> RMSNorm -> SwiGLU MLP + residual; final RMSNorm
 * of each sequence's last row and lm_head. logits [S][vocab]. Returns 0 or -1. */
int oracle_forward_batch(const oracle_model_config* cfg, const oracle_model_weights* w,
                         const uint32_t* tokens, const int32_t* positions,
                         const int64_t* slot_mapping, uint32_t T, float* const* k_pools,
                         float* const* v_pools, uint32_t num_blocks, uint32_t block_size,
                         const uint32_t* block_tables, uint32_t max_blocks,
                         const int32_t* cu_seqlens, const uint32_t* context_lens, uint32_t S,
                         float* logits, int nthreads);

/* The shared body of forward_batch / forward_batch_all_rows (src/model.rs:1382-1410,
 * RowSelection): all_rows = 0 gives logits [S][vocab] of each sequence's last row,
 * all_rows = 1 logits [T][vocab] of every new token (the speculative verifier's rows).
 * The pools are of cfg->kv_dtype (k_scales / v_scales per layer for the 1-byte
 * kinds, NULL for F32): new rows go through oracle_kv_append of that kind. */
int oracle_forward_batch_rows(const oracle_model_config* cfg, const oracle_model_weights* w,
                              const uint32_t* tokens, const int32_t* positions,
                              const int64_t* slot_mapping, uint32_t T, void* const* k_pools,
                              void* const* v_pools, void* const* k_scales, void* const* v_scales,
                              uint32_t num_blocks, uint32_t block_size,
                              const uint32_t* block_tables, uint32_t max_blocks,
                              const int32_t* cu_seqlens, const uint32_t* context_lens, uint32_t S,
                              int all_rows, float* logits, int nthreads);

#ifdef __cplusplus
}
#endif
#endif
