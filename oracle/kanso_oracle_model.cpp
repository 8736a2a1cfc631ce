// kanso_oracle_model.cpp — CPU restatement of kanso-infer's batched llama forward
// (Model::forward_batch_rows, src/model.rs:1418-1739) over Q8_0 weights and an F32
// paged KV pool.
//
// TEST INFRASTRUCTURE ONLY: the checker of the GPU decoder forward and of the
// greedy token streams; nothing in the product links or loads it.
//
// Each step restates the reference op in the reference's order, using the
// restated primitives of kanso_oracle.cpp (rmsnorm, Q8_0 GEMV, RoPE, the ragged
// attention with the offset causal mask, SiLU gating, greedy argmax).

#include <cmath>
#include <cstring>
#include <vector>

#include "kanso_oracle.h"

extern "C" {

uint64_t oracle_splitmix64(uint64_t x) {
    // splitmix64's output function for state x + golden gamma (Steele, Lea & Flood,
    // "Fast splittable pseudorandom number generators", OOPSLA 2014)
    x += 0x9e3779b97f4a7c15ull;
    x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ull;
    x = (x ^ (x >> 27)) * 0x94d049bb133111ebull;
    return x ^ (x >> 31);
}

float oracle_randn_scale(float std_dev) {
    return static_cast<float>(static_cast<double>(std_dev) * 1.7320508075688772 / 65536.0);
}

int oracle_init_random_q8_0(uint64_t stream_seed, uint32_t rows, uint32_t cols, float c, void* gguf_out) {
    // kanso_model_init_random's matrix: element i = (sum of the four 16-bit fields of
    // splitmix64(seed ^ i * 0xd1342543de82ef95) - 131070) * c, then Q8_0 per row.
    if (cols % 32 != 0) return -1;
    std::vector<float> row(cols);
    uint8_t* out = static_cast<uint8_t*>(gguf_out);
    for (uint32_t r = 0; r < rows; ++r) {
        for (uint32_t k = 0; k < cols; ++k) {
            const uint64_t i = static_cast<uint64_t>(r) * cols + k;
            const uint64_t h = oracle_splitmix64(stream_seed ^ (i * 0xd1342543de82ef95ull));
            const int32_t s = static_cast<int32_t>((h & 0xffff) + ((h >> 16) & 0xffff) + ((h >> 32) & 0xffff) +
                                                   (h >> 48)) -
                              131070;
            row[k] = static_cast<float>(s) * c;
        }
        oracle_quantize_row_q8_0(row.data(), cols, out + static_cast<size_t>(r) * (cols / 32) * 34);
    }
    return 0;
}

int oracle_forward_batch_rows(const oracle_model_config* cfg, const oracle_model_weights* w,
                              const uint32_t* tokens, const int32_t* positions,
                              const int64_t* slot_mapping, uint32_t T, void* const* k_pools,
                              void* const* v_pools, void* const* k_scales, void* const* v_scales,
                              uint32_t num_blocks, uint32_t block_size,
                              const uint32_t* block_tables, uint32_t max_blocks,
                              const int32_t* cu_seqlens, const uint32_t* context_lens, uint32_t S,
                              int all_rows, float* logits, int nthreads) {
    const uint32_t Hd = cfg->hidden, H = cfg->num_heads, HKV = cfg->num_kv_heads;
    const uint32_t D = cfg->head_dim, I = cfg->intermediate, V = cfg->vocab;
    const bool f32w = cfg->weight_format == 1;
    if (cfg->weight_format > 1) return -1;
    if (T == 0 || S == 0 || H % HKV != 0 || D % 2 != 0) return -1;
    if (!f32w && (Hd % 32 != 0 || I % 32 != 0)) return -1;
    if (static_cast<uint32_t>(cu_seqlens[S]) != T) return -1;
    // y[t] = x[t] @ W^T for every token (LinearWeight::forward, src/weights.rs:43-45);
    // fmt: the GGUF type of a quantized matrix (8 = Q8_0, 12 = Q4_K)
    const auto linear = [&](const void* m, const float* x, float* y, uint32_t rows, uint32_t cols, uint32_t fmt) {
        if (!f32w) {
            if (fmt == 12)
                oracle_gemv_q4_k(m, x, y, rows, cols, T, nthreads);
            else
                oracle_gemv_q8_0(m, x, y, rows, cols, T, nthreads);
            return;
        }
        const float* wm = static_cast<const float*>(m);
        for (uint32_t t = 0; t < T; ++t)
            for (uint32_t r = 0; r < rows; ++r) {
                float acc = 0.f;
                for (uint32_t c = 0; c < cols; ++c)
                    acc += x[static_cast<size_t>(t) * cols + c] * wm[static_cast<size_t>(r) * cols + c];
                y[static_cast<size_t>(t) * rows + r] = acc;
            }
    };
    // Model::embed (src/model.rs:425-431): table rows (dequantized for Q8_0), times
    // the Granite embedding scale when present.
    std::vector<float> hidden(static_cast<size_t>(T) * Hd);
    for (uint32_t t = 0; t < T; ++t) {
        if (tokens[t] >= V) return -1;
        if (f32w) {
            std::memcpy(&hidden[static_cast<size_t>(t) * Hd],
                        static_cast<const float*>(w->embed) + static_cast<size_t>(tokens[t]) * Hd, Hd * sizeof(float));
            continue;
        }
        const uint8_t* blocks = static_cast<const uint8_t*>(w->embed) + static_cast<size_t>(tokens[t]) * (Hd / 32) * 34;
        oracle_dequant_row_q8_0(blocks, Hd, &hidden[static_cast<size_t>(t) * Hd]);
    }
    if (cfg->embedding_scale != 0.f)
        for (float& v : hidden) v = v * cfg->embedding_scale;
    // rope_cos_sin (src/model.rs:667-696): rows of a table grown in 1024 steps; a
    // row depends only on its position.
    int32_t max_pos = 0;
    for (uint32_t t = 0; t < T; ++t) max_pos = std::max(max_pos, positions[t]);
    const uint32_t rope_len = (static_cast<uint32_t>(max_pos) + 1 + 1023) / 1024 * 1024;
    std::vector<float> cos_t(static_cast<size_t>(rope_len) * D / 2), sin_t(cos_t.size());
    oracle_rope_table(rope_len, D, cfg->rope_theta, cos_t.data(), sin_t.data());

    std::vector<float> normed(static_cast<size_t>(T) * Hd);
    std::vector<float> q(static_cast<size_t>(T) * H * D), k(static_cast<size_t>(T) * HKV * D),
        v(static_cast<size_t>(T) * HKV * D), attn(static_cast<size_t>(T) * H * D);
    std::vector<float> proj(static_cast<size_t>(T) * Hd);
    std::vector<float> gate(static_cast<size_t>(T) * I), up(static_cast<size_t>(T) * I),
        act(static_cast<size_t>(T) * I);
    kanso_ragged_attention_params ap;
    ap.num_seqs = S;
    ap.num_heads = H;
    ap.num_kv_heads = HKV;
    ap.head_dim = D;
    ap.block_size = block_size;
    ap.max_num_blocks_per_seq = max_blocks;
    // attention_scale: 1 / sqrt(head_dim) (src/model.rs:757-762), applied in f32.
    ap.scale = cfg->attention_scale != 0.f ? cfg->attention_scale
                                           : static_cast<float>(1.0 / std::sqrt(static_cast<double>(D)));
    ap.total_q = T;
    ap.kv_dtype = cfg->kv_dtype;
    if (cfg->kv_dtype > KANSO_KV_FP8 || (cfg->kv_dtype != KANSO_KV_F32 && (!k_scales || !v_scales))) return -1;
    ap.num_blocks = num_blocks;
    ap.max_q_len = 0;
    ap.pool_layout = KANSO_POOL_TOKEN_MAJOR;

    const float res_mul = cfg->residual_scale;
    const auto fmt = [&](uint32_t l, uint32_t j) -> uint32_t { return w->formats ? w->formats[l * 7 + j] : 8u; };
    for (uint32_t l = 0; l < cfg->num_layers; ++l) {
        oracle_rmsnorm(hidden.data(), w->attn_norm[l], normed.data(), T, Hd, cfg->eps);
        linear(w->wq[l], normed.data(), q.data(), H * D, Hd, fmt(l, 0));
        linear(w->wk[l], normed.data(), k.data(), HKV * D, Hd, fmt(l, 1));
        linear(w->wv[l], normed.data(), v.data(), HKV * D, Hd, fmt(l, 2));
        oracle_rope_apply(q.data(), T, H, D, positions, cos_t.data(), sin_t.data());
        oracle_rope_apply(k.data(), T, HKV, D, positions, cos_t.data(), sin_t.data());
        // write_kv_slots (src/model.rs:1673; storage.rs:219-254)
        void* ks = cfg->kv_dtype != KANSO_KV_F32 ? k_scales[l] : nullptr;
        void* vs = cfg->kv_dtype != KANSO_KV_F32 ? v_scales[l] : nullptr;
        if (oracle_kv_append(cfg->kv_dtype, k.data(), v.data(), slot_mapping, T, num_blocks, block_size, HKV, D,
                             k_pools[l], v_pools[l], ks, vs) != 0)
            return -1;
        if (oracle_ragged_attention(q.data(), k_pools[l], v_pools[l], ks, vs, block_tables, cu_seqlens,
                                    context_lens, &ap, attn.data(), nthreads) != 0)
            return -1;
        // hidden = hidden + attn_output(attn) (src/model.rs:1716-1717)
        linear(w->wo[l], attn.data(), proj.data(), Hd, H * D, fmt(l, 3));
        if (res_mul != 0.f)  // Granite: scale_residual (src/model.rs:739-744)
            for (float& p : proj) p = p * res_mul;
        for (size_t i = 0; i < hidden.size(); ++i) hidden[i] = hidden[i] + proj[i];
        // ffn: rmsnorm, gate/up, silu * up, down, residual (src/model.rs:1719-1721, 367-380)
        oracle_rmsnorm(hidden.data(), w->ffn_norm[l], normed.data(), T, Hd, cfg->eps);
        linear(w->w_gate[l], normed.data(), gate.data(), I, Hd, fmt(l, 4));
        linear(w->w_up[l], normed.data(), up.data(), I, Hd, fmt(l, 5));
        oracle_silu_mul(gate.data(), up.data(), act.data(), T * I);
        linear(w->w_down[l], act.data(), proj.data(), Hd, I, fmt(l, 6));
        if (res_mul != 0.f)
            for (float& p : proj) p = p * res_mul;
        for (size_t i = 0; i < hidden.size(); ++i) hidden[i] = hidden[i] + proj[i];
    }
    // final norm, then lm_head on every row (RowSelection::EveryToken) or on each
    // sequence's last row (LastPerSequence), src/model.rs:1726-1738. The norm is per
    // row, so normalising only the selected rows gives the same values.
    const uint32_t R = all_rows ? T : S;
    std::vector<float> last(static_cast<size_t>(R) * Hd);
    for (uint32_t r = 0; r < R; ++r) {
        const size_t src = all_rows ? r : static_cast<size_t>(cu_seqlens[r + 1] - 1);
        std::memcpy(&last[static_cast<size_t>(r) * Hd], &hidden[src * Hd], Hd * sizeof(float));
    }
    std::vector<float> last_normed(last.size());
    oracle_rmsnorm(last.data(), w->final_norm, last_normed.data(), R, Hd, cfg->eps);
    if (f32w) {
        const float* wm = static_cast<const float*>(w->lm_head);
        for (uint32_t r = 0; r < R; ++r)
            for (uint32_t o = 0; o < V; ++o) {
                float acc = 0.f;
                for (uint32_t c = 0; c < Hd; ++c)
                    acc += last_normed[static_cast<size_t>(r) * Hd + c] * wm[static_cast<size_t>(o) * Hd + c];
                logits[static_cast<size_t>(r) * V + o] = acc;
            }
    } else {
        oracle_gemv_q8_0(w->lm_head, last_normed.data(), logits, V, Hd, R, nthreads);
    }
    if (cfg->logit_scale != 0.f) {  // Granite: scale_logits (src/model.rs:747-752)
        const float mul = static_cast<float>(1.0 / static_cast<double>(cfg->logit_scale));
        for (size_t i = 0; i < static_cast<size_t>(R) * V; ++i) logits[i] = logits[i] * mul;
    }
    return 0;
}

int oracle_forward_batch(const oracle_model_config* cfg, const oracle_model_weights* w,
                         const uint32_t* tokens, const int32_t* positions,
                         const int64_t* slot_mapping, uint32_t T, float* const* k_pools,
                         float* const* v_pools, uint32_t num_blocks, uint32_t block_size,
                         const uint32_t* block_tables, uint32_t max_blocks,
                         const int32_t* cu_seqlens, const uint32_t* context_lens, uint32_t S,
                         float* logits, int nthreads) {
    oracle_model_config f32 = *cfg;
    f32.kv_dtype = KANSO_KV_F32;
    return oracle_forward_batch_rows(&f32, w, tokens, positions, slot_mapping, T,
                                     reinterpret_cast<void* const*>(k_pools),
                                     reinterpret_cast<void* const*>(v_pools), nullptr, nullptr,
                                     num_blocks, block_size, block_tables, max_blocks, cu_seqlens,
                                     context_lens, S, 0, logits, nthreads);
}

}  // extern "C"
