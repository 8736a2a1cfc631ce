// model.hip — the device-resident llama decoder: weight upload / random init,
// the paged F32 KV pool, and one batched forward per engine step.
//
// Reference: Model (src/model.rs:177-194) and forward_batch_rows (:1418-1739) on
// the mixed-batch arm, with every per-layer op replaced by the fused kernels of
// decoder.hip and the ragged attention of attention.hip. A step is:
//   pack (kanso_pack_step) -> embed -> per layer [RMSNorm+QKV+RoPE+KV write ->
//   ragged attention -> O + residual -> RMSNorm+gate/up+SwiGLU -> down + residual]
//   -> final RMSNorm + lm_head + greedy argmax on each sequence's last row.
// All step inputs travel in one host-to-device copy from a pinned staging buffer;
// the S sampled tokens come back in one device-to-host copy.
#include <cmath>
#include <cstring>

#include "model.hpp"

namespace kanso {
namespace {

__device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
    x += 0x9e3779b97f4a7c15ull;
    x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ull;
    x = (x ^ (x >> 27)) * 0x94d049bb133111ebull;
    return x ^ (x >> 31);
}

// Random-init value i of a stream: four 16-bit fields of one splitmix64 hash summed
// (an Irwin-Hall(4) variate: mean 0, bell-shaped, within +-3.46 standard
// deviations) and scaled by c = std * sqrt(3) / 65536. The sum is an exact integer
// (|s| <= 131070) and the scale is one IEEE multiply, so the host restatement
// computes every value bit for bit (a Box-Muller draw would depend on the device's
// log / cos, which differ from the host's in the last bits).
__global__ void randn_kernel(float* out, uint64_t n, uint64_t seed, float c) {
    for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < n; i += static_cast<uint64_t>(gridDim.x) * 256) {
        const uint64_t h = splitmix64(seed ^ (i * 0xd1342543de82ef95ull));
        const int32_t s = static_cast<int32_t>((h & 0xffff) + ((h >> 16) & 0xffff) + ((h >> 32) & 0xffff) + (h >> 48)) -
                          131070;
        out[i] = static_cast<float>(s) * c;
    }
}

// Scale of randn_kernel for a standard deviation (host f64 arithmetic, one rounding).
float randn_scale(float std) { return static_cast<float>(static_cast<double>(std) * 1.7320508075688772 / 65536.0); }

// One thread per (group, block, lane) of a packed matrix: the inverse of
// kanso_q8_0_pack (GGUF [rows][in/32] blocks from the packed tiles).
__global__ __launch_bounds__(256) void unpack_q8_0_kernel(const uint8_t* __restrict__ src, uint32_t rows,
                                                          uint32_t nb, uint8_t* __restrict__ dst, uint32_t stride,
                                                          uint32_t offset) {
    const uint64_t total = static_cast<uint64_t>((rows + 15) / 16) * nb * 64;
    for (uint64_t e = blockIdx.x * 256ull + threadIdx.x; e < total; e += static_cast<uint64_t>(gridDim.x) * 256) {
        const uint32_t lane = static_cast<uint32_t>(e % 64);
        const uint32_t b = static_cast<uint32_t>((e / 64) % nb);
        const uint32_t g = static_cast<uint32_t>(e / (64ull * nb));
        const uint32_t row = g * 16 + (lane & 15);
        if (row >= rows) continue;
        const uint8_t* tile = src + (static_cast<size_t>(g * stride + offset) * nb + b) * 544;
        uint8_t* blk = dst + (static_cast<size_t>(row) * nb + b) * 34;
        for (int j = 0; j < 8; ++j) blk[2 + 8 * (lane >> 4) + j] = tile[8 * lane + j];
        if (lane < 16) {
            blk[0] = tile[512 + 2 * lane];
            blk[1] = tile[512 + 2 * lane + 1];
        }
    }
}

// BlockQ8_0::from_f32_slice (src/quant/q8_0.rs:13-32), one thread per block:
// amax, d = amax / 127, id = 1 / d (0 when d == 0), q = round(x * id) clamped,
// d stored as f16 (round to nearest even). Every step is one IEEE operation, so
// the bytes equal the CPU rule's.
__global__ void quantize_q8_0_kernel(const float* __restrict__ x, uint64_t nblocks, uint8_t* __restrict__ out) {
    for (uint64_t b = blockIdx.x * 256ull + threadIdx.x; b < nblocks; b += static_cast<uint64_t>(gridDim.x) * 256) {
        const float* xb = x + b * 32;
        float amax = 0.f;
        for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(xb[i]));
        const float d = amax / 127.0f;
        const float id = d != 0.f ? 1.0f / d : 0.f;
        uint8_t* ob = out + b * 34;
        const uint16_t dh = __half_as_ushort(__float2half_rn(d));
        ob[0] = static_cast<uint8_t>(dh & 0xff);
        ob[1] = static_cast<uint8_t>(dh >> 8);
        for (int i = 0; i < 32; ++i) {
            const float r = roundf(xb[i] * id);
            ob[2 + i] = static_cast<uint8_t>(static_cast<int8_t>(fminf(fmaxf(r, -128.0f), 127.0f)));
        }
    }
}

__global__ void fill_f32_kernel(float* p, uint64_t n, float v) {
    for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < n; i += static_cast<uint64_t>(gridDim.x) * 256) p[i] = v;
}

// Zeroes block blocks[i] of every layer's K and V pool: one float4 per thread.
__global__ void reset_blocks_kernel(float* k, float* v, const uint32_t* blocks, uint32_t n, uint32_t layers,
                                    size_t layer_elems, uint32_t block_elems, uint32_t num_blocks) {
    const uint64_t per_block = block_elems / 4;
    const uint64_t total = static_cast<uint64_t>(n) * layers * per_block;
    for (uint64_t e = blockIdx.x * 256ull + threadIdx.x; e < total; e += static_cast<uint64_t>(gridDim.x) * 256) {
        const uint32_t i = static_cast<uint32_t>(e / (layers * per_block));
        const uint32_t l = static_cast<uint32_t>((e / per_block) % layers);
        const uint64_t c = e % per_block;
        const uint32_t blk = blocks[i];
        if (blk >= num_blocks) continue;
        const size_t off = l * layer_elems + static_cast<size_t>(blk) * block_elems + 4 * c;
        *reinterpret_cast<float4*>(k + off) = make_float4(0.f, 0.f, 0.f, 0.f);
        *reinterpret_cast<float4*>(v + off) = make_float4(0.f, 0.f, 0.f, 0.f);
    }
}

uint32_t grid_for(uint64_t n) { return static_cast<uint32_t>(std::min<uint64_t>((n + 255) / 256, 8192)); }

// Allocates a device buffer owned by the model. A buffer that *p already holds is
// replaced: freed and dropped from the model's list (callers that grow a buffer
// synchronise the device first, so no queued kernel still reads it).
template <class T>
int dev_alloc(kanso_model* m, T** p, size_t bytes) {
    void* q = nullptr;
    KANSO_HIP_TRY(hipMalloc(&q, std::max<size_t>(bytes, 256)));
    if (*p) {
        void* old = static_cast<void*>(*p);
        for (size_t i = 0; i < m->allocations.size(); ++i)
            if (m->allocations[i] == old) {
                m->allocations[i] = m->allocations.back();
                m->allocations.pop_back();
                (void)hipFree(old);
                break;
            }
    }
    m->allocations.push_back(q);
    *p = static_cast<T*>(q);
    return KANSO_OK;
}

// Activation rows are padded to whole 16-token tiles (the tiled activation order).
size_t tile_rows(uint32_t t) { return (static_cast<size_t>(t) + 15) / 16 * 16; }

int model_check(kanso_model* m, const char* who) {
    if (!m) {
        set_error("%s: null model", who);
        return KANSO_E_INVALID_ARG;
    }
    return KANSO_OK;
}

// Packed buffer of the fused Q/K/V matrix.
size_t qkv_rows(const kanso_model_config& c) { return static_cast<size_t>(c.num_heads + 2 * c.num_kv_heads) * 64; }

int alloc_weights(kanso_model* m) {
    const kanso_model_config& c = m->cfg;
    int rc;
    m->layers.resize(c.num_layers);
    for (auto& L : m->layers) {
        if ((rc = dev_alloc(m, &L.qkv, kanso_q8_0_packed_bytes(qkv_rows(c), c.hidden)))) return rc;
        if ((rc = dev_alloc(m, &L.o, kanso_q8_0_packed_bytes(c.hidden, c.num_heads * 64)))) return rc;
        if ((rc = dev_alloc(m, &L.gate_up, kanso_q8_0_packed_bytes(2 * c.intermediate, c.hidden)))) return rc;
        if ((rc = dev_alloc(m, &L.down, kanso_q8_0_packed_bytes(c.hidden, c.intermediate)))) return rc;
        if ((rc = dev_alloc(m, &L.attn_norm, c.hidden * sizeof(float)))) return rc;
        if ((rc = dev_alloc(m, &L.ffn_norm, c.hidden * sizeof(float)))) return rc;
        KANSO_HIP_TRY(hipMemset(L.qkv, 0, kanso_q8_0_packed_bytes(qkv_rows(c), c.hidden)));
        KANSO_HIP_TRY(hipMemset(L.gate_up, 0, kanso_q8_0_packed_bytes(2 * c.intermediate, c.hidden)));
    }
    if ((rc = dev_alloc(m, &m->embed, kanso_q8_0_packed_bytes(c.vocab, c.hidden)))) return rc;
    if (c.tied_embeddings) {
        m->lm_head = m->embed;
    } else if ((rc = dev_alloc(m, &m->lm_head, kanso_q8_0_packed_bytes(c.vocab, c.hidden)))) {
        return rc;
    }
    if ((rc = dev_alloc(m, &m->final_norm, c.hidden * sizeof(float)))) return rc;
    // RoPE table on the host with the reference's f32 arithmetic (build_rope_table,
    // src/model.rs:698-718): theta_j = base^(-2j/D), angle = pos * theta_j.
    const uint32_t half = c.head_dim / 2;
    std::vector<float> theta(half), cs(static_cast<size_t>(c.max_position) * half), sn(cs.size());
    for (uint32_t j = 0; j < half; ++j)
        theta[j] = std::pow(c.rope_theta, -2.0f * static_cast<float>(j) / static_cast<float>(c.head_dim));
    for (uint32_t p = 0; p < c.max_position; ++p)
        for (uint32_t j = 0; j < half; ++j) {
            const float a = static_cast<float>(p) * theta[j];
            cs[static_cast<size_t>(p) * half + j] = std::cos(a);
            sn[static_cast<size_t>(p) * half + j] = std::sin(a);
        }
    if ((rc = dev_alloc(m, &m->cos_t, cs.size() * sizeof(float)))) return rc;
    if ((rc = dev_alloc(m, &m->sin_t, sn.size() * sizeof(float)))) return rc;
    KANSO_HIP_TRY(hipMemcpy(m->cos_t, cs.data(), cs.size() * sizeof(float), hipMemcpyHostToDevice));
    KANSO_HIP_TRY(hipMemcpy(m->sin_t, sn.data(), sn.size() * sizeof(float), hipMemcpyHostToDevice));
    return KANSO_OK;
}

// Destination of a matrix kind: packed buffer, rows, in-features, group stride and
// offset in that buffer.
struct MatrixSlot {
    uint8_t* dst;
    uint32_t rows, in, stride, offset;
};

bool matrix_slot(kanso_model* m, uint32_t kind, uint32_t layer, MatrixSlot& ms) {
    const kanso_model_config& c = m->cfg;
    if (kind == KANSO_W_EMBED) {
        ms = {m->embed, c.vocab, c.hidden, 1, 0};
        return true;
    }
    if (kind == KANSO_W_LM_HEAD) {
        ms = {m->lm_head, c.vocab, c.hidden, 1, 0};
        return true;
    }
    if (layer >= c.num_layers) return false;
    auto& L = m->layers[layer];
    switch (kind) {
        case KANSO_W_Q: ms = {L.qkv, c.num_heads * 64, c.hidden, 1, 0}; return true;
        case KANSO_W_K: ms = {L.qkv, c.num_kv_heads * 64, c.hidden, 1, 4 * c.num_heads}; return true;
        case KANSO_W_V:
            ms = {L.qkv, c.num_kv_heads * 64, c.hidden, 1, 4 * (c.num_heads + c.num_kv_heads)};
            return true;
        case KANSO_W_O: ms = {L.o, c.hidden, c.num_heads * 64, 1, 0}; return true;
        case KANSO_W_GATE: ms = {L.gate_up, c.intermediate, c.hidden, 2, 0}; return true;
        case KANSO_W_UP: ms = {L.gate_up, c.intermediate, c.hidden, 2, 1}; return true;
        case KANSO_W_DOWN: ms = {L.down, c.hidden, c.intermediate, 1, 0}; return true;
        default: return false;
    }
}

float* norm_slot(kanso_model* m, uint32_t kind, uint32_t layer) {
    if (kind == KANSO_W_FINAL_NORM) return m->final_norm;
    if (layer >= m->cfg.num_layers) return nullptr;
    if (kind == KANSO_W_ATTN_NORM) return m->layers[layer].attn_norm;
    if (kind == KANSO_W_FFN_NORM) return m->layers[layer].ffn_norm;
    return nullptr;
}

int ensure_step_buffers(kanso_model* m, uint32_t T, uint32_t S, uint32_t tables, uint32_t arena,
                        size_t work_bytes = 0) {
    const kanso_model_config& c = m->cfg;
    int rc;
    if (T > m->cap_tokens || S > m->cap_seqs) {
        // grow with headroom, so a caller whose batch creeps up step by step does
        // not reallocate on every step; the old buffers may still be in use by
        // queued work, so wait for it before they are replaced
        KANSO_HIP_TRY(hipDeviceSynchronize());
        const uint32_t t = T > m->cap_tokens ? std::max(T, m->cap_tokens + m->cap_tokens / 2) : m->cap_tokens;
        const uint32_t sq = S > m->cap_seqs ? std::max(S, m->cap_seqs + m->cap_seqs / 2) : m->cap_seqs;
        const size_t tr = tile_rows(t);
        if ((rc = dev_alloc(m, &m->hidden, tr * c.hidden * 4))) return rc;
        if ((rc = dev_alloc(m, &m->q, static_cast<size_t>(t) * c.num_heads * 64 * 4))) return rc;
        if ((rc = dev_alloc(m, &m->attn, tr * c.num_heads * 64 * 4))) return rc;
        if ((rc = dev_alloc(m, &m->act, tr * c.intermediate * 4))) return rc;
        if ((rc = dev_alloc(m, &m->cu, (sq + 1) * 4ull))) return rc;
        if ((rc = dev_alloc(m, &m->seq_of_query, t * 4ull))) return rc;
        if ((rc = dev_alloc(m, &m->positions, t * 4ull))) return rc;
        if ((rc = dev_alloc(m, &m->slots, t * 8ull))) return rc;
        if ((rc = dev_alloc(m, &m->tokens, t * 4ull))) return rc;
        if ((rc = dev_alloc(m, &m->ctx_lens, sq * 4ull))) return rc;
        if ((rc = dev_alloc(m, &m->next, sq * 4ull))) return rc;
        void* h = nullptr;
        KANSO_HIP_TRY(hipHostMalloc(&h, (sq + 1) * 4ull));  // + the status word
        if (m->h_next) (void)hipHostFree(m->h_next);
        m->h_next = static_cast<uint32_t*>(h);
        m->cap_tokens = t;
        m->cap_seqs = sq;
        // per-pair argmax keys of the lm_head for every sampled row
        if ((rc = ensure_keys(m->ctx, static_cast<size_t>(sq) * ((c.vocab + 31) / 32) * 8))) return rc;
    }
    if (tables > m->cap_tables) {
        KANSO_HIP_TRY(hipDeviceSynchronize());
        const uint32_t want = std::max(tables, m->cap_tables + m->cap_tables / 2);
        if ((rc = dev_alloc(m, &m->tables, static_cast<size_t>(want) * 4))) return rc;
        m->cap_tables = want;
    }
    const size_t need = align_up(static_cast<size_t>(S) * sizeof(kanso_seq_plan), 256) +
                        align_up(static_cast<size_t>(arena) * 4, 256) + align_up(static_cast<size_t>(S) * 4, 256) +
                        work_bytes;
    if (need > m->stage_bytes) {
        const size_t want = align_up(need + need / 2, 1 << 16);
        KANSO_HIP_TRY(hipDeviceSynchronize());
        if ((rc = dev_alloc(m, &m->d_stage, want))) return rc;
        void* h = nullptr;
        KANSO_HIP_TRY(hipHostMalloc(&h, want));
        if (m->h_stage) (void)hipHostFree(m->h_stage);
        m->h_stage = h;
        m->stage_bytes = want;
    }
    return KANSO_OK;
}

}  // namespace

int model_reset_blocks(kanso_model* m, const uint32_t* blocks, uint32_t n, hipStream_t s) {
    if (n == 0) return KANSO_OK;
    if (!m->k_pool) {
        set_error("kanso_model_reset_blocks: KV pool not allocated");
        return KANSO_E_INVALID_ARG;
    }
    int rc;
    const uint32_t L = m->cfg.num_layers;
    const uint32_t need = m->kv_dtype == KANSO_KV_F32 ? n : n * L;
    if (need > m->cap_reset) {
        KANSO_HIP_TRY(hipDeviceSynchronize());
        const uint32_t want = std::max(need, m->cap_reset + m->cap_reset / 2);
        if ((rc = dev_alloc(m, &m->d_reset, want * 4ull))) return rc;
        m->cap_reset = want;
    }
    if (m->kv_dtype != KANSO_KV_F32) {
        // Every layer's pool is the next num_blocks blocks of one pool of L x num_blocks
        // blocks, so one erase of the blocks b + l * num_blocks covers all layers
        // (bytes to 0, scales to their empty value).
        // (Ids outside the pool are skipped, as in the F32 erase.)
        std::vector<uint32_t> all;
        all.reserve(need);
        for (uint32_t l = 0; l < L; ++l)
            for (uint32_t i = 0; i < n; ++i)
                if (blocks[i] < m->num_blocks) all.push_back(blocks[i] + l * m->num_blocks);
        if (all.empty()) return KANSO_OK;
        const uint32_t cnt = static_cast<uint32_t>(all.size());
        KANSO_HIP_TRY(hipMemcpyAsync(m->d_reset, all.data(), cnt * 4ull, hipMemcpyHostToDevice, s));
        if ((rc = kanso_kv_reset_blocks(m->ctx, m->kv_dtype, m->d_reset, cnt, m->num_blocks * L, m->block_size,
                                        m->cfg.num_kv_heads, m->cfg.head_dim, m->k_pool, m->v_pool, m->k_scales,
                                        m->v_scales, reinterpret_cast<kanso_stream_t>(s))))
            return rc;
        KANSO_HIP_TRY(hipStreamSynchronize(s));
        return KANSO_OK;
    }
    // The list is tiny; a synchronous copy keeps the host array's lifetime simple.
    KANSO_HIP_TRY(hipMemcpyAsync(m->d_reset, blocks, n * 4ull, hipMemcpyHostToDevice, s));
    const uint32_t block_elems = m->block_size * m->cfg.num_kv_heads * m->cfg.head_dim;
    const uint64_t total = static_cast<uint64_t>(n) * m->cfg.num_layers * (block_elems / 4);
    hipLaunchKernelGGL(reset_blocks_kernel, dim3(grid_for(total)), dim3(256), 0, s, m->k_pool, m->v_pool,
                       m->d_reset, n, m->cfg.num_layers, m->layer_pool_elems, block_elems, m->num_blocks);
    KANSO_LAUNCH_CHECK();
    KANSO_HIP_TRY(hipStreamSynchronize(s));
    return KANSO_OK;
}

// all_rows: RowSelection::EveryToken (src/model.rs:1382-1410): the lm_head and the
// greedy argmax run on every new token (next / logits have T rows), not only on each
// sequence's last one.
int model_forward(kanso_model* m, const HostStep& step, float* logits, uint32_t* next, hipStream_t s,
                  bool all_rows) {
    const kanso_model_config& c = m->cfg;
    const uint32_t S = static_cast<uint32_t>(step.plan.size());
    if (S == 0) {
        set_error("forward_batch: empty batch");
        return KANSO_E_INVALID_SHAPE;
    }
    if (!m->k_pool) {
        set_error("forward_batch: KV pool not allocated (kanso_model_alloc_kv)");
        return KANSO_E_INVALID_ARG;
    }
    for (uint32_t l = 0; l < c.num_layers; ++l) {
        // a fused product needs all its matrices in one format
        const uint32_t parts = m->layers[l].q4k_parts;
        const uint32_t qkv = parts & 7u, gu = (parts >> (KANSO_W_GATE - KANSO_W_Q)) & 3u;
        if ((qkv != 0 && qkv != 7u) || (gu != 0 && gu != 3u)) {
            set_error("forward_batch: layer %u mixes Q4_K and Q8_0 in its Q/K/V or gate/up matrices", l);
            return KANSO_E_INVALID_ARG;
        }
    }
    // Shapes from the plan (PaddedDecodeTables::new, src/model.rs:84-88).
    uint32_t T = 0, max_blocks = 1, max_q = 0;
    for (const auto& p : step.plan) {
        if (p.q_len == 0) {
            set_error("forward_batch: a sequence has query_len 0");
            return KANSO_E_INVALID_SHAPE;
        }
        T += p.q_len;
        max_q = std::max(max_q, p.q_len);
        const uint32_t ctx = p.start_pos + p.q_len;
        if (ctx > c.max_position) {
            set_error("forward_batch: context %u beyond the RoPE table (%u positions)", ctx, c.max_position);
            return KANSO_E_OUT_OF_BOUNDS;
        }
        max_blocks = std::max(max_blocks, std::max((ctx + m->block_size - 1) / m->block_size, 1u));
    }
    const uint32_t R = all_rows ? T : S;  // rows through the lm_head
    kanso_ragged_attention_params ap{};
    ap.num_seqs = S;
    ap.num_heads = c.num_heads;
    ap.num_kv_heads = c.num_kv_heads;
    ap.head_dim = c.head_dim;
    ap.block_size = m->block_size;
    ap.max_num_blocks_per_seq = max_blocks;
    ap.scale = c.attention_scale != 0.f ? c.attention_scale
                                        : static_cast<float>(1.0 / std::sqrt(static_cast<double>(c.head_dim)));  // src/model.rs:757-762
    ap.total_q = T;
    ap.kv_dtype = m->kv_dtype;
    ap.num_blocks = m->num_blocks;
    ap.max_q_len = max_q;
    // The split-K partition from the step's planned lengths (the attention library
    // alone only sees the table capacity). Measured on config 5: 10.96 k tok/s with
    // the capacity-based choice, 11.2 k with the planned lengths.
    std::vector<uint32_t> ql(S), cl(S);
    for (uint32_t i = 0; i < S; ++i) {
        ql[i] = step.plan[i].q_len;
        cl[i] = step.plan[i].start_pos + step.plan[i].q_len;
    }
    ap.partition_size = kanso_ragged_partition_size(m->ctx, &ap, ql.data(), cl.data());
    ap.chunk_partition_size = kanso_ragged_chunk_partition_size(m->ctx, &ap, ql.data(), cl.data());
    // The attention takes the work-list path (kanso_ragged_build_work): the items
    // with their block ids come from the host's plan in the same upload as the plan,
    // so an attention wave's first load is its item and its second its keys (no
    // sequence table, no block-table round trip).
    uint32_t n_chunk_items = 0;
    const uint32_t n_items = kanso_ragged_work_items(&ap, ql.data(), cl.data(), &n_chunk_items);
    const bool use_work = n_items != 0;
    int rc = ensure_step_buffers(m, T, std::max(S, R), S * max_blocks,
                                 static_cast<uint32_t>(step.token_arena.size() + step.table_arena.size()),
                                 static_cast<size_t>(n_items) * kanso_ragged_work_item_words * 4);
    if (rc) return rc;
    // Stage: plan | token arena + table arena | last rows.
    char* h = static_cast<char*>(m->h_stage);
    const size_t off_arena = align_up(S * sizeof(kanso_seq_plan), 256);
    const size_t arena_n = step.token_arena.size() + step.table_arena.size();
    const size_t off_last = off_arena + align_up(arena_n * 4, 256);
    std::memcpy(h, step.plan.data(), S * sizeof(kanso_seq_plan));
    std::memcpy(h + off_arena, step.token_arena.data(), step.token_arena.size() * 4);
    std::memcpy(h + off_arena + step.token_arena.size() * 4, step.table_arena.data(), step.table_arena.size() * 4);
    int32_t* last = reinterpret_cast<int32_t*>(h + off_last);
    if (all_rows) {
        for (uint32_t i = 0; i < T; ++i) last[i] = static_cast<int32_t>(i);
    } else {
        int32_t run = 0;
        for (uint32_t i = 0; i < S; ++i) {
            run += static_cast<int32_t>(step.plan[i].q_len);
            last[i] = run - 1;
        }
    }
    const size_t off_work = align_up(off_last + R * 4ull, 256);
    size_t stage_n = off_last + R * 4ull;
    if (use_work) {
        // the step's tables padded to [S][max_blocks] as the device holds them
        // (PaddedDecodeTables: the last needed block repeats)
        std::vector<uint32_t> tabs(static_cast<size_t>(S) * max_blocks, 0u);
        for (uint32_t i = 0; i < S; ++i) {
            const kanso_seq_plan& p = step.plan[i];
            const uint32_t* t = step.table_arena.data() + p.table_offset;
            for (uint32_t j = 0; j < max_blocks; ++j)
                tabs[static_cast<size_t>(i) * max_blocks + j] = p.table_len ? t[std::min(j, p.table_len - 1)] : 0u;
        }
        if ((rc = kanso_ragged_build_work(&ap, ql.data(), cl.data(), tabs.data(),
                                          reinterpret_cast<uint32_t*>(h + off_work), n_items)))
            return rc;
        stage_n = off_work + static_cast<size_t>(n_items) * kanso_ragged_work_item_words * 4;
    }
    KANSO_HIP_TRY(hipMemcpyAsync(m->d_stage, h, stage_n, hipMemcpyHostToDevice, s));
    char* d = static_cast<char*>(m->d_stage);
    const auto* d_plan = reinterpret_cast<const kanso_seq_plan*>(d);
    const auto* d_tok_arena = reinterpret_cast<const uint32_t*>(d + off_arena);
    const auto* d_tab_arena = d_tok_arena + step.token_arena.size();
    const auto* d_last = reinterpret_cast<const int32_t*>(d + off_last);
    const auto* d_work = use_work ? reinterpret_cast<const uint32_t*>(d + off_work) : nullptr;

    kanso_packed_step packed{m->cu, m->seq_of_query, m->positions, m->slots, m->tokens, m->tables, m->ctx_lens};
    if ((rc = kanso_pack_step(m->ctx, d_plan, S, d_tok_arena, d_tab_arena, m->block_size, max_blocks, T, &packed,
                              reinterpret_cast<kanso_stream_t>(s))))
        return rc;
    // hidden, attn and act are in the tiled activation order (act_tile_off): the
    // products read them as contiguous 1 KB slices
    // Granite multipliers: the reference multiplies by the f64 scale on f32 tensors,
    // i.e. by the scale rounded to f32 (src/model.rs:424-430, 739-760)
    const float emb_mul = c.embedding_scale != 0.f ? c.embedding_scale : 1.f;
    const float res_mul = c.residual_scale != 0.f ? c.residual_scale : 1.f;
    const float logit_mul = c.logit_scale != 0.f ? static_cast<float>(1.0 / static_cast<double>(c.logit_scale)) : 1.f;
    if ((rc = op_embed(m->ctx, m->embed, c.vocab, c.hidden, m->tokens, T, m->hidden, s, true, emb_mul))) return rc;

    kanso_qkv_params qp{T, c.hidden, c.num_heads, c.num_kv_heads, 64, c.max_position, c.eps, m->num_blocks,
                        m->block_size};
    const uint32_t qd = c.num_heads * 64;
    const bool quant = m->kv_dtype != KANSO_KV_F32;
    // 1-byte pools: the QKV epilogue quantizes each K / V row into its pool slot
    // (write_kv_slots of the quantized storage) with no f32 staging rows.
    for (uint32_t l = 0; l < c.num_layers; ++l) {
        const auto& L = m->layers[l];
        const uint32_t bits = L.q4k_parts;
        const bool qkv4 = (bits & 7u) == 7u, gu4 = ((bits >> (KANSO_W_GATE - KANSO_W_Q)) & 3u) == 3u;
        const bool o4 = (bits >> (KANSO_W_O - KANSO_W_Q)) & 1u, down4 = (bits >> (KANSO_W_DOWN - KANSO_W_Q)) & 1u;
        uint8_t* kp = reinterpret_cast<uint8_t*>(m->k_pool) + l * m->layer_pool_bytes;
        uint8_t* vp = reinterpret_cast<uint8_t*>(m->v_pool) + l * m->layer_pool_bytes;
        uint8_t* ks = quant ? m->k_scales + l * m->layer_scale_bytes : nullptr;
        uint8_t* vs = quant ? m->v_scales + l * m->layer_scale_bytes : nullptr;
        if (!quant) {
            if ((rc = op_qkv_rope_append(m->ctx, &qp, qkv4 ? L.qkv_q4k : L.qkv, m->hidden, L.attn_norm, m->positions,
                                         m->slots, m->cos_t, m->sin_t, m->q, reinterpret_cast<float*>(kp),
                                         reinterpret_cast<float*>(vp), s, true, qkv4)))
                return rc;
        } else if ((rc = op_qkv_rope_quant(m->ctx, &qp, qkv4 ? L.qkv_q4k : L.qkv, m->hidden, L.attn_norm,
                                           m->positions, m->slots, m->cos_t, m->sin_t, m->q, m->kv_dtype, kp, vp, ks,
                                           vs, s, true, qkv4))) {
            return rc;
        }
        if ((rc = op_ragged_attention(m->ctx, &ap, m->q, kp, vp, ks, vs, m->tables, m->cu, m->ctx_lens, m->attn, s,
                                      true, d_work, n_items - n_chunk_items, n_chunk_items)))
            return rc;
        if ((rc = op_gemm_residual(o4 ? L.o_q4k : L.o, m->attn, m->hidden, c.hidden, qd, T, s, true, o4, res_mul)))
            return rc;
        if ((rc = op_gate_up_swiglu(gu4 ? L.gate_up_q4k : L.gate_up, m->hidden, L.ffn_norm, c.eps, T, c.hidden,
                                    c.intermediate, m->act, s, true, gu4)))
            return rc;
        if ((rc = op_gemm_residual(down4 ? L.down_q4k : L.down, m->act, m->hidden, c.hidden, c.intermediate, T, s,
                                   true, down4, res_mul)))
            return rc;
    }
    if ((rc = op_lm_head_argmax(m->ctx, m->lm_head, m->hidden, d_last, m->final_norm, c.eps, R, c.hidden, c.vocab,
                                logits, m->next, s, true, logit_mul)))
        return rc;
    // the sampled tokens and the device status word come back at the same sync: a
    // flag raised by any kernel of the step (slot, block, position, token bounds)
    // fails the step instead of passing wrong tokens on
    KANSO_HIP_TRY(hipMemcpyAsync(m->h_next, m->next, R * 4ull, hipMemcpyDeviceToHost, s));
    KANSO_HIP_TRY(hipMemcpyAsync(m->h_next + m->cap_seqs, m->ctx->status, 4, hipMemcpyDeviceToHost, s));
    KANSO_HIP_TRY(hipStreamSynchronize(s));
    if (m->h_next[m->cap_seqs]) return kanso_check_device_status(m->ctx, reinterpret_cast<kanso_stream_t>(s), nullptr);
    std::memcpy(next, m->h_next, R * 4ull);
    ++m->forward_calls;
    return KANSO_OK;
}

uint32_t kanso_model_vocab(const kanso_model* m) { return m ? m->cfg.vocab : 0; }

}  // namespace kanso

using namespace kanso;

extern "C" {

int kanso_quantize_q8_0(kanso_ctx* ctx, const float* x, uint64_t n, void* gguf_out, kanso_stream_t stream) {
    if (!ctx || !x || !gguf_out) {
        set_error("kanso_quantize_q8_0: null argument");
        return KANSO_E_INVALID_ARG;
    }
    if (n == 0 || n % 32 != 0) {
        set_error("kanso_quantize_q8_0: n %llu must be a non-zero multiple of 32", static_cast<unsigned long long>(n));
        return KANSO_E_INVALID_SHAPE;
    }
    hipLaunchKernelGGL(quantize_q8_0_kernel, dim3(grid_for(n / 32)), dim3(256), 0, as_stream(stream), x, n / 32,
                       static_cast<uint8_t*>(gguf_out));
    KANSO_LAUNCH_CHECK();
    return KANSO_OK;
}

int kanso_model_create(kanso_ctx* ctx, const kanso_model_config* cfg, kanso_model** out) {
    if (!ctx || !cfg || !out) {
        set_error("kanso_model_create: null argument");
        return KANSO_E_INVALID_ARG;
    }
    *out = nullptr;
    const kanso_model_config& c = *cfg;
    if (c.head_dim != 64 || c.num_heads == 0 || c.num_kv_heads == 0 || c.num_heads % c.num_kv_heads != 0 ||
        c.num_heads / c.num_kv_heads > 8 || c.hidden == 0 || c.hidden % 32 != 0 || c.intermediate == 0 ||
        c.intermediate % 32 != 0 || c.vocab == 0 || c.num_layers == 0 || c.max_position == 0) {
        set_error("kanso_model_create: unsupported shape (head_dim %u must be 64; hidden %u and intermediate %u "
                  "multiples of 32; heads %u / kv heads %u with group <= 8)",
                  c.head_dim, c.hidden, c.intermediate, c.num_heads, c.num_kv_heads);
        return KANSO_E_INVALID_SHAPE;
    }
    for (float v : {c.embedding_scale, c.attention_scale, c.residual_scale, c.logit_scale})
        if (!std::isfinite(v) || v < 0.f) {
            set_error("kanso_model_create: Granite multipliers must be finite and >= 0 (0 = absent)");
            return KANSO_E_INVALID_SHAPE;
        }
    KANSO_HIP_TRY(hipSetDevice(ctx->device));
    auto* m = new kanso_model();
    m->ctx = ctx;
    m->cfg = c;
    int rc = alloc_weights(m);
    if (rc) {
        kanso_model_destroy(m);
        return rc;
    }
    *out = m;
    return KANSO_OK;
}

int kanso_model_destroy(kanso_model* m) {
    if (!m) return KANSO_OK;
    (void)hipDeviceSynchronize();
    for (void* p : m->allocations) (void)hipFree(p);
    if (m->h_stage) (void)hipHostFree(m->h_stage);
    if (m->h_next) (void)hipHostFree(m->h_next);
    delete m;
    return KANSO_OK;
}

int kanso_model_set_weight(kanso_model* m, uint32_t kind, uint32_t layer, const void* host_data, size_t bytes) {
    int rc = model_check(m, "kanso_model_set_weight");
    if (rc) return rc;
    if (!host_data) {
        set_error("kanso_model_set_weight: null data");
        return KANSO_E_INVALID_ARG;
    }
    if (float* nw = norm_slot(m, kind, layer)) {
        if (bytes != m->cfg.hidden * sizeof(float)) {
            set_error("kanso_model_set_weight: norm of %zu bytes, expected %zu", bytes, m->cfg.hidden * sizeof(float));
            return KANSO_E_INVALID_SHAPE;
        }
        KANSO_HIP_TRY(hipMemcpy(nw, host_data, bytes, hipMemcpyHostToDevice));
        return KANSO_OK;
    }
    MatrixSlot ms;
    if ((kind == KANSO_W_LM_HEAD && m->cfg.tied_embeddings) || !matrix_slot(m, kind, layer, ms)) {
        set_error("kanso_model_set_weight: kind %u / layer %u not a weight of this model", kind, layer);
        return KANSO_E_INVALID_ARG;
    }
    const size_t want = static_cast<size_t>(ms.rows) * (ms.in / 32) * 34;
    if (bytes != want) {
        set_error("kanso_model_set_weight: kind %u has %zu bytes, expected %zu (GGUF Q8_0 [%u][%u])", kind, bytes,
                  want, ms.rows, ms.in);
        return KANSO_E_INVALID_SHAPE;
    }
    if (kind >= KANSO_W_Q && kind <= KANSO_W_DOWN) m->layers[layer].q4k_parts &= ~(1u << (kind - KANSO_W_Q));
    void* tmp = nullptr;
    KANSO_HIP_TRY(hipMalloc(&tmp, bytes));
    hipError_t e = hipMemcpy(tmp, host_data, bytes, hipMemcpyHostToDevice);
    if (e == hipSuccess) {
        rc = kanso_q8_0_pack(m->ctx, tmp, ms.rows, ms.in, ms.dst, ms.stride, ms.offset, nullptr);
        e = hipDeviceSynchronize();
    }
    (void)hipFree(tmp);
    if (e != hipSuccess) {
        set_error("kanso_model_set_weight: %s", hipGetErrorString(e));
        return KANSO_E_HIP;
    }
    return rc;
}

int kanso_model_set_weight_q4_k(kanso_model* m, uint32_t kind, uint32_t layer, const void* host_data, size_t bytes) {
    int rc = model_check(m, "kanso_model_set_weight_q4_k");
    if (rc) return rc;
    const kanso_model_config& c = m->cfg;
    if (!host_data || kind < KANSO_W_Q || kind > KANSO_W_DOWN || layer >= c.num_layers) {
        set_error("kanso_model_set_weight_q4_k: kind %u / layer %u is not a projection of this model", kind, layer);
        return KANSO_E_INVALID_ARG;
    }
    MatrixSlot ms;
    matrix_slot(m, kind, layer, ms);
    if (ms.in % 256 != 0) {
        set_error("kanso_model_set_weight_q4_k: in_features %u is not a multiple of 256 (Q4_K super-blocks)", ms.in);
        return KANSO_E_INVALID_SHAPE;
    }
    const size_t row_bytes = static_cast<size_t>(ms.in / 256) * 144;
    if (bytes != ms.rows * row_bytes) {
        set_error("kanso_model_set_weight_q4_k: kind %u has %zu bytes, expected %zu (GGUF Q4_K [%u][%u])", kind, bytes,
                  ms.rows * row_bytes, ms.rows, ms.in);
        return KANSO_E_INVALID_SHAPE;
    }
    auto& L = m->layers[layer];
    const auto alloc = [&](uint8_t*& buf, size_t rows) -> int {
        if (buf) return KANSO_OK;
        void* p = nullptr;
        KANSO_HIP_TRY(hipMalloc(&p, rows * row_bytes));
        m->allocations.push_back(p);
        buf = static_cast<uint8_t*>(p);
        return KANSO_OK;
    };
    const char* src = static_cast<const char*>(host_data);
    switch (kind) {
        case KANSO_W_Q:
        case KANSO_W_K:
        case KANSO_W_V: {
            // rows of [Wq; Wk; Wv], as the packed layout concatenates them
            if ((rc = alloc(L.qkv_q4k, qkv_rows(c)))) return rc;
            const size_t row0 = kind == KANSO_W_Q ? 0 : kind == KANSO_W_K ? c.num_heads * 64ull
                                                                            : (c.num_heads + c.num_kv_heads) * 64ull;
            KANSO_HIP_TRY(hipMemcpy(L.qkv_q4k + row0 * row_bytes, src, bytes, hipMemcpyHostToDevice));
            break;
        }
        case KANSO_W_GATE:
        case KANSO_W_UP: {
            // 16-row groups interleaved: gate rows 16j.. at 32j, up rows 16j.. at 32j + 16
            if ((rc = alloc(L.gate_up_q4k, 2ull * c.intermediate))) return rc;
            const size_t off = kind == KANSO_W_GATE ? 0 : 16 * row_bytes;
            KANSO_HIP_TRY(hipMemcpy2D(L.gate_up_q4k + off, 32 * row_bytes, src, 16 * row_bytes, 16 * row_bytes,
                                      c.intermediate / 16, hipMemcpyHostToDevice));
            break;
        }
        case KANSO_W_O:
            if ((rc = alloc(L.o_q4k, c.hidden))) return rc;
            KANSO_HIP_TRY(hipMemcpy(L.o_q4k, src, bytes, hipMemcpyHostToDevice));
            break;
        default:
            if ((rc = alloc(L.down_q4k, c.hidden))) return rc;
            KANSO_HIP_TRY(hipMemcpy(L.down_q4k, src, bytes, hipMemcpyHostToDevice));
            break;
    }
    L.q4k_parts |= 1u << (kind - KANSO_W_Q);
    return KANSO_OK;
}

int kanso_model_init_random(kanso_model* m, uint64_t seed, float std) {
    int rc = model_check(m, "kanso_model_init_random");
    if (rc) return rc;
    const kanso_model_config& c = m->cfg;
    size_t max_elems = static_cast<size_t>(c.vocab) * c.hidden;
    max_elems = std::max(max_elems, static_cast<size_t>(c.intermediate) * c.hidden);
    float* f = nullptr;
    uint8_t* g = nullptr;
    KANSO_HIP_TRY(hipMalloc(&f, max_elems * 4));
    if (hipMalloc(&g, max_elems / 32 * 34) != hipSuccess) {
        (void)hipFree(f);
        set_error("kanso_model_init_random: out of device memory");
        return KANSO_E_HIP;
    }
    uint64_t stream_id = 0;
    for (auto& L : m->layers) L.q4k_parts = 0;  // every matrix Q8_0
    auto one = [&](uint32_t kind, uint32_t layer) -> int {
        MatrixSlot ms;
        if (!matrix_slot(m, kind, layer, ms)) return KANSO_E_INVALID_ARG;
        const uint64_t n = static_cast<uint64_t>(ms.rows) * ms.in;
        const uint64_t sd = seed * 0x100000001b3ull + (++stream_id) * 0x9e3779b97f4a7c15ull;
        hipLaunchKernelGGL(randn_kernel, dim3(grid_for(n)), dim3(256), 0, nullptr, f, n, sd, randn_scale(std));
        hipLaunchKernelGGL(quantize_q8_0_kernel, dim3(grid_for(n / 32)), dim3(256), 0, nullptr, f, n / 32, g);
        KANSO_LAUNCH_CHECK();
        return kanso_q8_0_pack(m->ctx, g, ms.rows, ms.in, ms.dst, ms.stride, ms.offset, nullptr);
    };
    rc = one(KANSO_W_EMBED, 0);
    if (!rc && !c.tied_embeddings) rc = one(KANSO_W_LM_HEAD, 0);
    for (uint32_t l = 0; l < c.num_layers && !rc; ++l)
        for (uint32_t kind : {KANSO_W_Q, KANSO_W_K, KANSO_W_V, KANSO_W_O, KANSO_W_GATE, KANSO_W_UP, KANSO_W_DOWN})
            if (!rc) rc = one(kind, l);
    if (!rc) {
        auto ones = [&](float* p) {
            hipLaunchKernelGGL(fill_f32_kernel, dim3(grid_for(c.hidden)), dim3(256), 0, nullptr, p,
                               static_cast<uint64_t>(c.hidden), 1.0f);
        };
        ones(m->final_norm);
        for (auto& L : m->layers) {
            ones(L.attn_norm);
            ones(L.ffn_norm);
        }
    }
    const hipError_t e = hipDeviceSynchronize();
    (void)hipFree(f);
    (void)hipFree(g);
    if (!rc && e != hipSuccess) {
        set_error("kanso_model_init_random: %s", hipGetErrorString(e));
        return KANSO_E_HIP;
    }
    return rc;
}

int kanso_model_get_weight(kanso_model* m, uint32_t kind, uint32_t layer, void* host_out, size_t bytes) {
    int rc = model_check(m, "kanso_model_get_weight");
    if (rc) return rc;
    if (!host_out) {
        set_error("kanso_model_get_weight: null output");
        return KANSO_E_INVALID_ARG;
    }
    if (float* nw = norm_slot(m, kind, layer)) {
        if (bytes != m->cfg.hidden * sizeof(float)) {
            set_error("kanso_model_get_weight: norm of %zu bytes, expected %zu", bytes, m->cfg.hidden * sizeof(float));
            return KANSO_E_INVALID_SHAPE;
        }
        KANSO_HIP_TRY(hipMemcpy(host_out, nw, bytes, hipMemcpyDeviceToHost));
        return KANSO_OK;
    }
    MatrixSlot ms;
    if ((kind == KANSO_W_LM_HEAD && m->cfg.tied_embeddings) || !matrix_slot(m, kind, layer, ms)) {
        set_error("kanso_model_get_weight: kind %u / layer %u not a weight of this model", kind, layer);
        return KANSO_E_INVALID_ARG;
    }
    if (kind >= KANSO_W_Q && kind <= KANSO_W_DOWN && (m->layers[layer].q4k_parts >> (kind - KANSO_W_Q) & 1u)) {
        set_error("kanso_model_get_weight: kind %u of layer %u is stored as Q4_K", kind, layer);
        return KANSO_E_INVALID_ARG;
    }
    const size_t want = static_cast<size_t>(ms.rows) * (ms.in / 32) * 34;
    if (bytes != want) {
        set_error("kanso_model_get_weight: kind %u has %zu bytes, expected %zu", kind, want, bytes);
        return KANSO_E_INVALID_SHAPE;
    }
    void* tmp = nullptr;
    KANSO_HIP_TRY(hipMalloc(&tmp, bytes));
    const uint64_t total = static_cast<uint64_t>((ms.rows + 15) / 16) * (ms.in / 32) * 64;
    hipLaunchKernelGGL(unpack_q8_0_kernel, dim3(grid_for(total)), dim3(256), 0, nullptr, ms.dst, ms.rows, ms.in / 32,
                       static_cast<uint8_t*>(tmp), ms.stride, ms.offset);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess) e = hipMemcpy(host_out, tmp, bytes, hipMemcpyDeviceToHost);
    (void)hipFree(tmp);
    if (e != hipSuccess) {
        set_error("kanso_model_get_weight: %s", hipGetErrorString(e));
        return KANSO_E_HIP;
    }
    return KANSO_OK;
}

int kanso_model_alloc_kv_quant(kanso_model* m, uint32_t num_blocks, uint32_t block_size, uint32_t max_tokens,
                               uint32_t max_seqs, uint32_t kv_dtype) {
    int rc = model_check(m, "kanso_model_alloc_kv");
    if (rc) return rc;
    if (m->k_pool) {
        set_error("kanso_model_alloc_kv: KV pool already allocated");
        return KANSO_E_INVALID_ARG;
    }
    if (num_blocks == 0 || block_size == 0 || (block_size & (block_size - 1)) != 0 || max_tokens == 0 ||
        max_seqs == 0) {
        set_error("kanso_model_alloc_kv: num_blocks %u, block_size %u (power of two), max_tokens %u, max_seqs %u",
                  num_blocks, block_size, max_tokens, max_seqs);
        return KANSO_E_INVALID_SHAPE;
    }
    if (kv_dtype > KANSO_KV_FP8) {
        set_error("kanso_model_alloc_kv: unknown kv_dtype %u", kv_dtype);
        return KANSO_E_INVALID_ARG;
    }
    const uint64_t rows = static_cast<uint64_t>(num_blocks) * block_size * m->cfg.num_kv_heads;
    if (static_cast<uint64_t>(num_blocks) * m->cfg.num_layers >= (1ull << 32)) {
        set_error("kanso_model_alloc_kv: %u blocks x %u layers too many", num_blocks, m->cfg.num_layers);
        return KANSO_E_INVALID_SHAPE;
    }
    m->num_blocks = num_blocks;
    m->block_size = block_size;
    m->kv_dtype = kv_dtype;
    m->layer_pool_elems = rows * m->cfg.head_dim;
    m->layer_pool_bytes = m->layer_pool_elems * (kv_dtype == KANSO_KV_F32 ? 4 : 1);
    m->layer_scale_bytes = kv_dtype == KANSO_KV_INT8 || kv_dtype == KANSO_KV_FP8 ? rows * 4
                           : kv_dtype == KANSO_KV_Q8_0                          ? rows * (m->cfg.head_dim / 32) * 2
                                                                                : 0;
    const size_t bytes = m->layer_pool_bytes * m->cfg.num_layers;
    if ((rc = dev_alloc(m, &m->k_pool, bytes))) return rc;
    if ((rc = dev_alloc(m, &m->v_pool, bytes))) return rc;
    KANSO_HIP_TRY(hipMemset(m->k_pool, 0, bytes));
    KANSO_HIP_TRY(hipMemset(m->v_pool, 0, bytes));
    if (m->layer_scale_bytes) {
        const size_t sb = m->layer_scale_bytes * m->cfg.num_layers;
        if ((rc = dev_alloc(m, &m->k_scales, sb))) return rc;
        if ((rc = dev_alloc(m, &m->v_scales, sb))) return rc;
        if (kv_dtype == KANSO_KV_Q8_0) {
            KANSO_HIP_TRY(hipMemset(m->k_scales, 0, sb));
            KANSO_HIP_TRY(hipMemset(m->v_scales, 0, sb));
        } else {  // an empty INT8 / FP8 row has scale 1 (quantized_storage.rs:35-40)
            const uint64_t n = sb / 4;
            hipLaunchKernelGGL(fill_f32_kernel, dim3(grid_for(n)), dim3(256), 0, 0,
                               reinterpret_cast<float*>(m->k_scales), n, 1.0f);
            hipLaunchKernelGGL(fill_f32_kernel, dim3(grid_for(n)), dim3(256), 0, 0,
                               reinterpret_cast<float*>(m->v_scales), n, 1.0f);
            KANSO_LAUNCH_CHECK();
            KANSO_HIP_TRY(hipDeviceSynchronize());
        }
    }
    return ensure_step_buffers(m, max_tokens, max_seqs, max_seqs * 64, max_tokens + max_seqs * 64);
}

int kanso_model_alloc_kv(kanso_model* m, uint32_t num_blocks, uint32_t block_size, uint32_t max_tokens,
                         uint32_t max_seqs) {
    return kanso_model_alloc_kv_quant(m, num_blocks, block_size, max_tokens, max_seqs, KANSO_KV_F32);
}

int kanso_model_kv_pool(kanso_model* m, uint32_t layer, float** k_pool, float** v_pool) {
    int rc = model_check(m, "kanso_model_kv_pool");
    if (rc) return rc;
    if (!m->k_pool || layer >= m->cfg.num_layers || m->kv_dtype != KANSO_KV_F32) {
        set_error("kanso_model_kv_pool: no F32 pool for layer %u", layer);
        return KANSO_E_INVALID_ARG;
    }
    if (k_pool) *k_pool = m->k_pool + layer * m->layer_pool_elems;
    if (v_pool) *v_pool = m->v_pool + layer * m->layer_pool_elems;
    return KANSO_OK;
}

int kanso_model_read_kv_rows(kanso_model* m, uint32_t layer, const uint64_t* slots, uint32_t n, float* k_out,
                             float* v_out) {
    int rc = model_check(m, "kanso_model_read_kv_rows");
    if (rc) return rc;
    if (!m->k_pool || layer >= m->cfg.num_layers || m->kv_dtype != KANSO_KV_F32 ||
        (n && (!slots || !k_out || !v_out))) {
        set_error("kanso_model_read_kv_rows: no F32 pool for layer %u or null argument", layer);
        return KANSO_E_INVALID_ARG;
    }
    const size_t row = static_cast<size_t>(m->cfg.num_kv_heads) * m->cfg.head_dim;
    const uint64_t num_slots = static_cast<uint64_t>(m->num_blocks) * m->block_size;
    KANSO_HIP_TRY(hipDeviceSynchronize());
    for (uint32_t i = 0; i < n; ++i) {
        if (slots[i] >= num_slots) {
            set_error("kanso_model_read_kv_rows: slot %llu outside %llu slots",
                      static_cast<unsigned long long>(slots[i]), static_cast<unsigned long long>(num_slots));
            return KANSO_E_OUT_OF_BOUNDS;
        }
        const size_t off = layer * m->layer_pool_elems + slots[i] * row;
        KANSO_HIP_TRY(hipMemcpy(k_out + i * row, m->k_pool + off, row * 4, hipMemcpyDeviceToHost));
        KANSO_HIP_TRY(hipMemcpy(v_out + i * row, m->v_pool + off, row * 4, hipMemcpyDeviceToHost));
    }
    return KANSO_OK;
}

int kanso_model_reset_blocks(kanso_model* m, const uint32_t* blocks, uint32_t n, kanso_stream_t stream) {
    int rc = model_check(m, "kanso_model_reset_blocks");
    if (rc) return rc;
    if (n && !blocks) {
        set_error("kanso_model_reset_blocks: null block list");
        return KANSO_E_INVALID_ARG;
    }
    return model_reset_blocks(m, blocks, n, as_stream(stream));
}

namespace {

int model_forward_entry(kanso_model* m, const char* name, const kanso_seq_plan* plan, uint32_t num_seqs,
                        const uint32_t* token_arena, uint32_t token_arena_len, const uint32_t* table_arena,
                        uint32_t table_arena_len, float* logits, uint32_t* next_tokens, kanso_stream_t stream,
                        bool all_rows) {
    int rc = model_check(m, name);
    if (rc) return rc;
    if (!plan || !token_arena || !table_arena || !next_tokens || num_seqs == 0) {
        set_error("%s: null argument or empty plan", name);
        return KANSO_E_INVALID_ARG;
    }
    HostStep hs;
    hs.plan.assign(plan, plan + num_seqs);
    hs.token_arena.assign(token_arena, token_arena + token_arena_len);
    hs.table_arena.assign(table_arena, table_arena + table_arena_len);
    for (const auto& p : hs.plan) {
        if (static_cast<uint64_t>(p.table_offset) + p.table_len > table_arena_len) {
            set_error("%s: table range outside the table arena", name);
            return KANSO_E_OUT_OF_BOUNDS;
        }
        for (uint32_t i = 0; i < p.q_len; ++i) {
            const uint32_t at = static_cast<uint32_t>(p.token_offset + p.start_pos + i);
            if (at >= token_arena_len) {
                set_error("%s: token outside the token arena", name);
                return KANSO_E_OUT_OF_BOUNDS;
            }
            if (token_arena[at] >= m->cfg.vocab) {
                set_error("%s: token id %u outside the vocabulary (%u)", name, token_arena[at], m->cfg.vocab);
                return KANSO_E_INVALID_ARG;
            }
        }
    }
    return model_forward(m, hs, logits, next_tokens, as_stream(stream), all_rows);
}

}  // namespace

int kanso_model_forward(kanso_model* m, const kanso_seq_plan* plan, uint32_t num_seqs, const uint32_t* token_arena,
                        uint32_t token_arena_len, const uint32_t* table_arena, uint32_t table_arena_len,
                        float* logits, uint32_t* next_tokens, kanso_stream_t stream) {
    return model_forward_entry(m, "kanso_model_forward", plan, num_seqs, token_arena, token_arena_len, table_arena,
                               table_arena_len, logits, next_tokens, stream, false);
}

int kanso_model_forward_all_rows(kanso_model* m, const kanso_seq_plan* plan, uint32_t num_seqs,
                                 const uint32_t* token_arena, uint32_t token_arena_len, const uint32_t* table_arena,
                                 uint32_t table_arena_len, float* logits, uint32_t* next_tokens,
                                 kanso_stream_t stream) {
    return model_forward_entry(m, "kanso_model_forward_all_rows", plan, num_seqs, token_arena, token_arena_len,
                               table_arena, table_arena_len, logits, next_tokens, stream, true);
}

}  // extern "C"
