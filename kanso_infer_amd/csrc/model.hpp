// model.hpp — the device-resident llama decoder (weights, paged F32 KV pool,
// activation buffers) and its batched forward, shared by model.hip and the engine.
#pragma once

#include <vector>

#include "common.hpp"

namespace kanso {

// Fused decoder ops (decoder.hip).
int op_embed(kanso_ctx* ctx, const void* table, uint32_t vocab, uint32_t hidden, const uint32_t* tokens,
             uint32_t T, float* out, hipStream_t s, bool tiled, float scale);
int op_qkv_rope_append(kanso_ctx* ctx, const kanso_qkv_params* p, const void* w, const float* x,
                       const float* norm_w, const int32_t* positions, const int64_t* slots, const float* cos_t,
                       const float* sin_t, float* q, float* k_pool, float* v_pool, hipStream_t s, bool tiled,
                       bool q4k);
int op_qkv_rope_quant(kanso_ctx* ctx, const kanso_qkv_params* p, const void* w, const float* x, const float* norm_w,
                      const int32_t* positions, const int64_t* slots, const float* cos_t, const float* sin_t,
                      float* q, uint32_t kv_dtype, void* k_pool, void* v_pool, void* k_scales, void* v_scales,
                      hipStream_t s, bool tiled, bool q4k);
int op_gemm_residual(const void* w, const float* x, float* y, uint32_t out, uint32_t in, uint32_t T,
                     hipStream_t s, bool tiled, bool q4k, float scale);
int op_gate_up_swiglu(const void* w, const float* x, const float* norm_w, float eps, uint32_t T,
                      uint32_t hidden, uint32_t inter, float* h, hipStream_t s, bool tiled, bool q4k);
int op_lm_head_argmax(kanso_ctx* ctx, const void* w, const float* x, const int32_t* rows, const float* norm_w,
                      float eps, uint32_t S, uint32_t hidden, uint32_t vocab, float* logits, uint32_t* tokens,
                      hipStream_t s, bool tiled, float logit_mul);
// The ragged attention with its output in the tiled activation order (the O
// projection's input) when out_tiled is set (attention.hip).
// work: an optional work list (kanso_ragged_build_work): n_work decode items, then
// n_work_chunk chunk items, kanso_ragged_work_item_words words each.
int op_ragged_attention(kanso_ctx* ctx, const kanso_ragged_attention_params* p, const float* q, const void* k_pool,
                        const void* v_pool, const void* k_scales, const void* v_scales, const uint32_t* block_tables,
                        const int32_t* cu_seqlens, const uint32_t* context_lens, float* out, hipStream_t s,
                        bool out_tiled, const uint32_t* work = nullptr, uint32_t n_work = 0,
                        uint32_t n_work_chunk = 0);
constexpr uint32_t kanso_ragged_work_item_words = KANSO_RAGGED_WORK_ITEM_WORDS;  // 60 block ids + 4 header words
bool ragged_work_supported(const kanso_ragged_attention_params* p);

// One step as the scheduler hands it over: the compact plan plus the token and
// block-table arenas kanso_pack_step reads (host memory).
struct HostStep {
    std::vector<kanso_seq_plan> plan;
    std::vector<uint32_t> token_arena;
    std::vector<uint32_t> table_arena;
};

}  // namespace kanso

struct kanso_model {
    kanso_ctx* ctx = nullptr;
    kanso_model_config cfg{};
    struct Layer {
        uint8_t* qkv = nullptr;      // packed [Wq; Wk; Wv]
        uint8_t* o = nullptr;        // packed Wo
        uint8_t* gate_up = nullptr;  // packed, gate / up groups interleaved
        uint8_t* down = nullptr;     // packed Wdown
        float* attn_norm = nullptr;
        float* ffn_norm = nullptr;
        // GGUF Q4_K storage (kanso_model_set_weight_q4_k): [Wq; Wk; Wv] rows, gate / up
        // rows interleaved by 16-row groups, Wo, Wdown; null while that matrix is Q8_0.
        // q4k_parts: bit per kind (1 << (kind - KANSO_W_Q)) uploaded as Q4_K.
        uint8_t* qkv_q4k = nullptr;
        uint8_t* gate_up_q4k = nullptr;
        uint8_t* o_q4k = nullptr;
        uint8_t* down_q4k = nullptr;
        uint32_t q4k_parts = 0;
    };
    std::vector<Layer> layers;
    uint8_t* embed = nullptr;    // packed [vocab][hidden]
    uint8_t* lm_head = nullptr;  // packed; == embed when tied
    float* final_norm = nullptr;
    float* cos_t = nullptr;  // [max_position][head_dim / 2]
    float* sin_t = nullptr;
    std::vector<void*> allocations;  // every device buffer above, freed at destroy
    // KV pool: [layers][num_blocks][block_size][kv_heads][head_dim], K and V, of kind
    // kv_dtype: f32 elements, or 1-byte elements with per-row scales (INT8 / FP8: one
    // f32 per token-head row; Q8_0: one f16 per 32 elements) in k_scales / v_scales.
    float* k_pool = nullptr;  // (bytes for the 1-byte kinds)
    float* v_pool = nullptr;
    uint32_t kv_dtype = 0;
    uint8_t* k_scales = nullptr;
    uint8_t* v_scales = nullptr;
    uint32_t num_blocks = 0, block_size = 0;
    size_t layer_pool_elems = 0;   // elements of one layer's K (or V) pool
    size_t layer_pool_bytes = 0;
    size_t layer_scale_bytes = 0;
    // Step buffers sized for max_tokens rows / max_seqs sequences (grow-only).
    uint32_t cap_tokens = 0, cap_seqs = 0, cap_tables = 0, cap_arena = 0;
    float *hidden = nullptr, *q = nullptr, *attn = nullptr, *act = nullptr;
    void* d_stage = nullptr;   // plan | token arena | table arena | last rows (device)
    void* h_stage = nullptr;   // pinned host mirror
    size_t stage_bytes = 0;
    int32_t *cu = nullptr, *seq_of_query = nullptr, *positions = nullptr;
    int64_t* slots = nullptr;
    uint32_t *tokens = nullptr, *tables = nullptr, *ctx_lens = nullptr, *next = nullptr;
    uint32_t* h_next = nullptr;  // pinned
    uint32_t* d_reset = nullptr; // blocks to erase this step
    uint32_t cap_reset = 0;
    uint64_t forward_calls = 0;
};

namespace kanso {

// The model's vocabulary size (token ids must be below it).
uint32_t kanso_model_vocab(const kanso_model* m);

// Erases blocks (host list) of every layer's K and V pool (allocate_zeroed,
// src/kv_cache/mod.rs:25-35).
int model_reset_blocks(kanso_model* m, const uint32_t* blocks, uint32_t n, hipStream_t s);
// One batched forward; next[s] = greedy token of sequence s's last row. logits
// (device, [S][vocab]) is written when non-null.
int model_forward(kanso_model* m, const HostStep& step, float* logits, uint32_t* next, hipStream_t s,
                  bool all_rows = false);

}  // namespace kanso
