// decoder.hip — the fused llama-layer operations around the attention kernel:
// embedding lookup, RMSNorm + Q/K/V + RoPE + KV write, O / down projections with
// the residual add, RMSNorm + gate/up + SwiGLU, and the final RMSNorm + lm_head +
// greedy argmax. All weights are packed Q8_0 (q8_gemm.hpp).
//
// Reference: the per-layer body of Model::forward_batch_rows (src/model.rs:1569-
// 1739): rmsnorm (:653-659), project_qkv (:437-475), rope_apply (:720-737),
// write_kv_slots (src/kv_cache/storage.rs:219-254), attention, attn_output +
// residual, ffn rmsnorm, SwiGLU MLP (:367-380) + residual, final norm, lm_head on
// each sequence's last row (:1729-1738) and greedy_token (src/sampler.rs:7-17).
#include "q8_gemm.hpp"

namespace kanso {
namespace {

// out[m][k] = d * q of token tokens[m]'s row in a packed Q8_0 table
// (BlockQ8_0::dequantize, src/quant/q8_0.rs:35-39: d * q, exact in f32).
__global__ __launch_bounds__(256) void embed_q8_0_kernel(const uint8_t* __restrict__ table, uint32_t vocab,
                                                         uint32_t hidden, const uint32_t* __restrict__ tokens,
                                                         uint32_t T, float* __restrict__ out, uint32_t* status,
                                                         uint32_t tiled, float scale) {
    const uint32_t nb = hidden / 32;
    const uint64_t total = static_cast<uint64_t>(T) * hidden / 8;
    for (uint64_t e = blockIdx.x * 256ull + threadIdx.x; e < total; e += static_cast<uint64_t>(gridDim.x) * 256) {
        const uint32_t m = static_cast<uint32_t>(e / (hidden / 8));
        const uint32_t k = static_cast<uint32_t>(e % (hidden / 8)) * 8;
        uint32_t tok = tokens[m];
        if (tok >= vocab) {
            if (k == 0) raise_status(status, KANSO_DEV_TOKEN_OOB);
            tok = 0;
        }
        const uint32_t g = tok / 16, rr = tok % 16, b = k / 32, kq = (k % 32) / 8;
        const uint8_t* tile = table + (static_cast<size_t>(g) * nb + b) * kPackedTileBytes;
        const uint64_t q = *reinterpret_cast<const uint64_t*>(tile + 8 * (16 * kq + rr));
        const float d = f16_bits_to_f32(*reinterpret_cast<const uint16_t*>(tile + 512 + 2 * rr));
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = d * static_cast<float>(static_cast<int8_t>((q >> (8 * j)) & 0xff)) * scale;
        float* o0 = tiled ? out + act_tile_off(m, k, nb) : out + static_cast<size_t>(m) * hidden + k;
        float* o1 = tiled ? out + act_tile_off(m, k + 4, nb) : o0 + 4;
        *reinterpret_cast<float4*>(o0) = make_float4(v[0], v[1], v[2], v[3]);
        *reinterpret_cast<float4*>(o1) = make_float4(v[4], v[5], v[6], v[7]);
    }
}

// One workgroup per token: the maximum of its per-pair keys (max is order-free,
// so the token does not depend on the reduction order); key 0 = no finite logit.
__global__ __launch_bounds__(256) void argmax_finish_kernel(const unsigned long long* keys, uint32_t pairs,
                                                            uint32_t* tokens) {
    __shared__ unsigned long long s_best[256 / kWave];
    const unsigned long long* row = keys + static_cast<size_t>(blockIdx.x) * pairs;
    unsigned long long best = 0;
    for (uint32_t i = threadIdx.x; i < pairs; i += 256) best = max(best, row[i]);
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) best = max(best, static_cast<unsigned long long>(__shfl_xor(best, o, kWave)));
    if ((threadIdx.x & (kWave - 1)) == 0) s_best[threadIdx.x / kWave] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 256 / kWave; ++w) best = max(best, s_best[w]);
        tokens[blockIdx.x] = best ? 0xffffffffu - static_cast<uint32_t>(best & 0xffffffffu) : 0u;
    }
}

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

}  // namespace

// Internal entry points shared with the model forward (model.hip).
int op_embed(kanso_ctx* ctx, const void* table, uint32_t vocab, uint32_t hidden, const uint32_t* tokens,
             uint32_t T, float* out, hipStream_t s, bool tiled, float scale) {
    if (T == 0) return KANSO_OK;
    const uint64_t total = static_cast<uint64_t>(T) * hidden / 8;
    const uint32_t grid = static_cast<uint32_t>(std::min<uint64_t>((total + 255) / 256, 4096));
    hipLaunchKernelGGL(embed_q8_0_kernel, dim3(grid), dim3(256), 0, s, static_cast<const uint8_t*>(table), vocab,
                       hidden, tokens, T, out, ctx->status, tiled ? 1u : 0u, scale);
    KANSO_LAUNCH_CHECK();
    return KANSO_OK;
}

int op_qkv_rope_append(kanso_ctx* ctx, const kanso_qkv_params* p, const void* w, const float* x,
                       const float* norm_w, const int32_t* positions, const int64_t* slots, const float* cos_t,
                       const float* sin_t, float* q, float* k_pool, float* v_pool, hipStream_t s, bool tiled,
                       bool q4k) {
    XIn xa{x, nullptr, norm_w, p->eps, p->hidden, p->num_tokens, p->hidden, tiled ? 1u : 0u};
    EpiQkvRope epi;
    epi.q = q;
    epi.k_pool = k_pool;
    epi.v_pool = v_pool;
    epi.positions = positions;
    epi.slots = slots;
    epi.cos_t = cos_t;
    epi.sin_t = sin_t;
    epi.status = ctx->status;
    epi.num_heads = p->num_heads;
    epi.num_kv_heads = p->num_kv_heads;
    epi.max_pos = p->max_pos;
    epi.num_slots = static_cast<int64_t>(p->num_blocks) * p->block_size;
    const uint32_t pairs = 2 * (p->num_heads + 2 * p->num_kv_heads);
    if (q4k)
        return launch_q8_gemm(WQ4K{static_cast<const uint8_t*>(w), p->hidden / 256, 32 * pairs}, xa, epi, pairs, s);
    return launch_q8_gemm(WPacked{static_cast<const uint8_t*>(w), p->hidden / 32}, xa, epi, pairs, s);
}

template <int KVT>
int qkv_rope_quant(kanso_ctx* ctx, const kanso_qkv_params* p, const void* w, const XIn& xa, const int32_t* positions,
                   const int64_t* slots, const float* cos_t, const float* sin_t, float* q, void* k_pool, void* v_pool,
                   void* k_scales, void* v_scales, hipStream_t s, bool q4k) {
    EpiQkvRopeQ<KVT> epi;
    epi.q = q;
    epi.k_pool = static_cast<uint8_t*>(k_pool);
    epi.v_pool = static_cast<uint8_t*>(v_pool);
    epi.k_scales = k_scales;
    epi.v_scales = v_scales;
    epi.positions = positions;
    epi.slots = slots;
    epi.cos_t = cos_t;
    epi.sin_t = sin_t;
    epi.status = ctx->status;
    epi.num_heads = p->num_heads;
    epi.num_kv_heads = p->num_kv_heads;
    epi.max_pos = p->max_pos;
    epi.num_slots = static_cast<int64_t>(p->num_blocks) * p->block_size;
    const uint32_t pairs = 2 * (p->num_heads + 2 * p->num_kv_heads);
    if (q4k)
        return launch_q8_gemm_paired(WQ4K{static_cast<const uint8_t*>(w), p->hidden / 256, 32 * pairs}, xa, epi,
                                     pairs, s);
    return launch_q8_gemm_paired(WPacked{static_cast<const uint8_t*>(w), p->hidden / 32}, xa, epi, pairs, s);
}

// The QKV product with RoPE whose K / V rows are quantized into a 1-byte pool in its
// epilogue (one kernel: the f32 path's op_qkv_rope_append plus kanso_kv_append).
int op_qkv_rope_quant(kanso_ctx* ctx, const kanso_qkv_params* p, const void* w, const float* x, const float* norm_w,
                      const int32_t* positions, const int64_t* slots, const float* cos_t, const float* sin_t,
                      float* q, uint32_t kv_dtype, void* k_pool, void* v_pool, void* k_scales, void* v_scales,
                      hipStream_t s, bool tiled, bool q4k) {
    XIn xa{x, nullptr, norm_w, p->eps, p->hidden, p->num_tokens, p->hidden, tiled ? 1u : 0u};
    switch (kv_dtype) {
        case KANSO_KV_INT8:
            return qkv_rope_quant<KANSO_KV_INT8>(ctx, p, w, xa, positions, slots, cos_t, sin_t, q, k_pool, v_pool,
                                                 k_scales, v_scales, s, q4k);
        case KANSO_KV_FP8:
            return qkv_rope_quant<KANSO_KV_FP8>(ctx, p, w, xa, positions, slots, cos_t, sin_t, q, k_pool, v_pool,
                                                k_scales, v_scales, s, q4k);
        case KANSO_KV_Q8_0:
            return qkv_rope_quant<KANSO_KV_Q8_0>(ctx, p, w, xa, positions, slots, cos_t, sin_t, q, k_pool, v_pool,
                                                 k_scales, v_scales, s, q4k);
        default:
            set_error("qkv_rope_quant: kv dtype %u is not a 1-byte pool", kv_dtype);
            return KANSO_E_INVALID_ARG;
    }
}

int op_gemm_residual(const void* w, const float* x, float* y, uint32_t out, uint32_t in, uint32_t T,
                     hipStream_t s, bool tiled, bool q4k, float scale) {
    XIn xa{x, nullptr, nullptr, 0.f, in, T, in, tiled ? 1u : 0u};
    EpiStore<true> epi{y, out, out, tiled ? 1u : 0u, scale};
    if (q4k) return launch_q8_gemm(WQ4K{static_cast<const uint8_t*>(w), in / 256, out}, xa, epi, (out + 31) / 32, s);
    return launch_q8_gemm(WPacked{static_cast<const uint8_t*>(w), in / 32}, xa, epi, (out + 31) / 32, s);
}

int op_gate_up_swiglu(const void* w, const float* x, const float* norm_w, float eps, uint32_t T,
                      uint32_t hidden, uint32_t inter, float* h, hipStream_t s, bool tiled, bool q4k) {
    XIn xa{x, nullptr, norm_w, eps, hidden, T, hidden, tiled ? 1u : 0u};
    EpiSwiGLU epi{h, inter, inter, tiled ? 1u : 0u};
    if (q4k) return launch_q8_gemm(WQ4K{static_cast<const uint8_t*>(w), hidden / 256, 2 * inter}, xa, epi, inter / 16, s);
    return launch_q8_gemm(WPacked{static_cast<const uint8_t*>(w), hidden / 32}, xa, epi, inter / 16, s);
}

int op_lm_head_argmax(kanso_ctx* ctx, const void* w, const float* x, const int32_t* rows, const float* norm_w,
                      float eps, uint32_t S, uint32_t hidden, uint32_t vocab, float* logits, uint32_t* tokens,
                      hipStream_t s, bool tiled, float logit_mul) {
    if (S == 0) return KANSO_OK;
    const uint32_t pairs = (vocab + 31) / 32;
    int rc = ensure_keys(ctx, static_cast<size_t>(S) * pairs * sizeof(unsigned long long));
    if (rc) return rc;
    auto* keys = static_cast<unsigned long long*>(ctx->keys);
    WPacked wl{static_cast<const uint8_t*>(w), hidden / 32};
    XIn xa{x, rows, norm_w, eps, hidden, S, hidden, tiled ? 1u : 0u};
    EpiArgmax epi{logits, vocab, vocab, keys, pairs, logit_mul};
    if ((rc = launch_q8_gemm(wl, xa, epi, pairs, s))) return rc;
    hipLaunchKernelGGL(argmax_finish_kernel, dim3(S), dim3(256), 0, s, keys, pairs, tokens);
    KANSO_LAUNCH_CHECK();
    return KANSO_OK;
}

}  // namespace kanso

using namespace kanso;

extern "C" {

int kanso_embed_q8_0(kanso_ctx* ctx, const void* packed_table, uint32_t vocab, uint32_t hidden,
                     const uint32_t* tokens, uint32_t num_tokens, float* out, kanso_stream_t stream) {
    if (!ctx || !packed_table || !tokens || !out) {
        set_error("kanso_embed_q8_0: null argument");
        return KANSO_E_INVALID_ARG;
    }
    if (vocab == 0 || hidden == 0 || hidden % 32 != 0 || !aligned16(out)) {
        set_error("kanso_embed_q8_0: vocab %u / hidden %u (multiple of 32, out 16-byte aligned)", vocab, hidden);
        return KANSO_E_INVALID_SHAPE;
    }
    return op_embed(ctx, packed_table, vocab, hidden, tokens, num_tokens, out, as_stream(stream), false, 1.f);
}

int kanso_qkv_rope_append(kanso_ctx* ctx, const kanso_qkv_params* p, const void* packed_qkv, const float* x,
                          const float* norm_w, const int32_t* positions, const int64_t* slot_mapping,
                          const float* cos_table, const float* sin_table, float* q_out, float* k_pool,
                          float* v_pool, kanso_stream_t stream) {
    if (!ctx || !p || !packed_qkv || !x || !norm_w || !positions || !slot_mapping || !cos_table || !sin_table ||
        !q_out || !k_pool || !v_pool) {
        set_error("kanso_qkv_rope_append: null argument");
        return KANSO_E_INVALID_ARG;
    }
    if (p->head_dim != 64) {
        set_error("kanso_qkv_rope_append: head_dim %u (this kernel handles 64)", p->head_dim);
        return KANSO_E_INVALID_SHAPE;
    }
    if (p->num_tokens == 0 || p->hidden == 0 || p->hidden % 32 != 0 || p->num_heads == 0 ||
        p->num_kv_heads == 0 || p->max_pos == 0 || p->block_size == 0 || !aligned16(x)) {
        set_error("kanso_qkv_rope_append: bad shape (tokens %u, hidden %u, heads %u/%u, max_pos %u)",
                  p->num_tokens, p->hidden, p->num_heads, p->num_kv_heads, p->max_pos);
        return KANSO_E_INVALID_SHAPE;
    }
    return op_qkv_rope_append(ctx, p, packed_qkv, x, norm_w, positions, slot_mapping, cos_table, sin_table, q_out,
                              k_pool, v_pool, as_stream(stream), false, false);
}

int kanso_qkv_rope_append_quant(kanso_ctx* ctx, const kanso_qkv_params* p, const void* packed_qkv, const float* x,
                                const float* norm_w, const int32_t* positions, const int64_t* slot_mapping,
                                const float* cos_table, const float* sin_table, float* q_out, uint32_t kv_dtype,
                                void* k_pool, void* v_pool, void* k_scales, void* v_scales, kanso_stream_t stream) {
    if (!ctx || !p || !packed_qkv || !x || !norm_w || !positions || !slot_mapping || !cos_table || !sin_table ||
        !q_out || !k_pool || !v_pool || !k_scales || !v_scales) {
        set_error("kanso_qkv_rope_append_quant: null argument");
        return KANSO_E_INVALID_ARG;
    }
    if (p->head_dim != 64) {
        set_error("kanso_qkv_rope_append_quant: head_dim %u (this kernel handles 64)", p->head_dim);
        return KANSO_E_INVALID_SHAPE;
    }
    if (p->num_tokens == 0 || p->hidden == 0 || p->hidden % 32 != 0 || p->num_heads == 0 ||
        p->num_kv_heads == 0 || p->max_pos == 0 || p->block_size == 0 || !aligned16(x)) {
        set_error("kanso_qkv_rope_append_quant: bad shape (tokens %u, hidden %u, heads %u/%u, max_pos %u)",
                  p->num_tokens, p->hidden, p->num_heads, p->num_kv_heads, p->max_pos);
        return KANSO_E_INVALID_SHAPE;
    }
    return op_qkv_rope_quant(ctx, p, packed_qkv, x, norm_w, positions, slot_mapping, cos_table, sin_table, q_out,
                             kv_dtype, k_pool, v_pool, k_scales, v_scales, as_stream(stream), false, false);
}

int kanso_gemm_q8_0_residual(kanso_ctx* ctx, const void* packed, const float* x, float* y, uint32_t out_features,
                             uint32_t in_features, uint32_t num_tokens, kanso_stream_t stream) {
    if (!ctx || !packed || !x || !y) {
        set_error("kanso_gemm_q8_0_residual: null argument");
        return KANSO_E_INVALID_ARG;
    }
    if (out_features == 0 || in_features == 0 || in_features % 32 != 0 || num_tokens == 0 || !aligned16(x)) {
        set_error("kanso_gemm_q8_0_residual: bad shape (out %u, in %u, tokens %u)", out_features, in_features,
                  num_tokens);
        return KANSO_E_INVALID_SHAPE;
    }
    return op_gemm_residual(packed, x, y, out_features, in_features, num_tokens, as_stream(stream), false, false,
                            1.f);
}

int kanso_gate_up_swiglu(kanso_ctx* ctx, const void* packed_gate_up, const float* x, const float* norm_w,
                         float eps, uint32_t num_tokens, uint32_t hidden, uint32_t intermediate, float* h,
                         kanso_stream_t stream) {
    if (!ctx || !packed_gate_up || !x || !norm_w || !h) {
        set_error("kanso_gate_up_swiglu: null argument");
        return KANSO_E_INVALID_ARG;
    }
    if (num_tokens == 0 || hidden == 0 || hidden % 32 != 0 || intermediate == 0 || intermediate % 16 != 0 ||
        !aligned16(x)) {
        set_error("kanso_gate_up_swiglu: bad shape (tokens %u, hidden %u, intermediate %u multiple of 16)",
                  num_tokens, hidden, intermediate);
        return KANSO_E_INVALID_SHAPE;
    }
    return op_gate_up_swiglu(packed_gate_up, x, norm_w, eps, num_tokens, hidden, intermediate, h,
                             as_stream(stream), false, false);
}

int kanso_lm_head_argmax(kanso_ctx* ctx, const void* packed, const float* x, const int32_t* rows,
                         const float* norm_w, float eps, uint32_t num_rows, uint32_t hidden, uint32_t vocab,
                         float* logits, uint32_t* tokens, kanso_stream_t stream) {
    if (!ctx || !packed || !x || !tokens) {
        set_error("kanso_lm_head_argmax: null argument");
        return KANSO_E_INVALID_ARG;
    }
    if (num_rows == 0 || hidden == 0 || hidden % 32 != 0 || vocab == 0 || !aligned16(x)) {
        set_error("kanso_lm_head_argmax: bad shape (rows %u, hidden %u, vocab %u)", num_rows, hidden, vocab);
        return KANSO_E_INVALID_SHAPE;
    }
    return op_lm_head_argmax(ctx, packed, x, rows, norm_w, eps, num_rows, hidden, vocab, logits, tokens,
                             as_stream(stream), false, 1.f);
}

}  // extern "C"
