// attention.hip — ragged paged attention (PagedAttention-v2 shape: split-K over
// context partitions + a reduce pass) for gfx950.
//
// Reference semantics: cpu_paged_attention (src/metal/paged_attention.rs:84-178) for
// a decode row, and the offset causal mask of forward_batch_rows (src/model.rs:
// 1510-1527) for a prefill-chunk row. The Metal kernel's structure
// (paged_attention_v2.metal:32-205: partitions, (m, d) stats, merge) is kept as a
// contract; the mapping onto the hardware is this file's own:
//
//  * One work item = (query row, context partition, KV head). A 256-thread
//    workgroup (4 wave64s) owns one item at a time and walks a device-built work
//    list in a grid-stride loop, so no host knowledge of context lengths is needed.
//  * Inside a wave, LPT = head_dim/4 lanes share one token: each lane loads one
//    float4 (16 B) of K and of V, so a load instruction moves 64 x 16 B = 1 KB of
//    fully used, coalesced bytes (four 256 B rows at head_dim 64). A lane loads
//    NL = 8 tokens per tile, K and V together, before any arithmetic, so 16
//    independent 16 B loads per lane are in flight.
//  * Every query head of the GQA group is served from the same K/V registers, so
//    K/V bytes are read once per (token, KV head), not once per query head.
//  * Scores live in the log2 domain (scale * log2(e) folded into one multiply) and
//    the online softmax runs per tile: one max / sum butterfly per tile and head
//    instead of one per token.
//  * The four waves of a workgroup split the partition into interleaved tiles and
//    merge their (m, l, acc) through LDS before one partial is written.
//  * Quantized pools (INT8 per token-head scale, Q8_0 per-32 f16 scale) are
//    dequantized in registers with the reference's own product (q as f32) * scale.
//
// Decode is a bandwidth-bound GEMV-like walk over K/V; it uses no MFMA.
#include <cmath>

#include "common.hpp"

namespace kanso {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr float kLog2e = 1.4426950408889634f;

struct AttnArgs {
    const float* q;
    const void* k_pool;
    const void* v_pool;
    const void* k_scales;
    const void* v_scales;
    const uint32_t* tables;
    const int32_t* cu;
    const uint32_t* ctx_lens;
    float* part_out;   // [T][H][max_parts][D]
    float2* part_stats;  // [T][H][max_parts] (m in log2 units, l)
    float* out;        // [T][H][D]
    const int4* items; // {row, part, limit, seq}
    const uint32_t* n_items;
    uint32_t* status;
    uint32_t num_seqs, num_heads, num_kv_heads, group, block_size, bs_shift;
    uint32_t max_blocks, num_blocks, part_size, max_parts, total_q, capacity;
    float scale_log2;
};

// Key limit of row i of a sequence: keys 0..=ctx-q_len+i, clamped to what the table
// can address (the Metal kernel clamps the same way, paged_attention_v2.metal:86-89).
__device__ __forceinline__ uint32_t row_limit(int32_t ctx, int32_t q_len, int32_t i, uint32_t cap) {
    int32_t lim = ctx - q_len + i + 1;
    if (lim < 0) lim = 0;
    return min(static_cast<uint32_t>(lim), cap);
}

// Single workgroup: validates every sequence, counts its (row, partition) items,
// scans the counts and writes the work list. Sequences are split into contiguous
// ranges, one per thread.
__global__ __launch_bounds__(kThreads) void build_worklist(AttnArgs a, int4* items, uint32_t* n_items) {
    __shared__ uint32_t scan[kThreads];
    const uint32_t tid = threadIdx.x;
    const uint32_t per = (a.num_seqs + kThreads - 1) / kThreads;
    const uint32_t s0 = min(tid * per, a.num_seqs), s1 = min(s0 + per, a.num_seqs);
    const uint32_t P = a.part_size;
    uint32_t count = 0, flags = 0;
    for (uint32_t s = s0; s < s1; ++s) {
        const int32_t ql = a.cu[s + 1] - a.cu[s];
        const int32_t ctx = static_cast<int32_t>(a.ctx_lens[s]);
        if (ctx == 0) flags |= KANSO_DEV_EMPTY_CONTEXT;
        if (static_cast<uint32_t>(ctx) > a.capacity) flags |= KANSO_DEV_CONTEXT_OVERFLOW;
        if (ql > ctx) flags |= KANSO_DEV_QUERY_OVERFLOW;
        for (int32_t i = 0; i < ql; ++i) count += (row_limit(ctx, ql, i, a.capacity) + P - 1) / P;
    }
    if (flags) raise_status(a.status, flags);
    scan[tid] = count;
    __syncthreads();
    for (uint32_t off = 1; off < kThreads; off <<= 1) {
        const uint32_t v = tid >= off ? scan[tid - off] : 0;
        __syncthreads();
        scan[tid] += v;
        __syncthreads();
    }
    uint32_t pos = scan[tid] - count;
    for (uint32_t s = s0; s < s1; ++s) {
        const int32_t ql = a.cu[s + 1] - a.cu[s];
        const int32_t ctx = static_cast<int32_t>(a.ctx_lens[s]);
        for (int32_t i = 0; i < ql; ++i) {
            const uint32_t lim = row_limit(ctx, ql, i, a.capacity);
            const uint32_t np = (lim + P - 1) / P;
            for (uint32_t p = 0; p < np; ++p)
                items[pos++] = make_int4(a.cu[s] + i, static_cast<int>(p), static_cast<int>(lim), static_cast<int>(s));
        }
    }
    if (tid == kThreads - 1) *n_items = scan[tid];
}

template <int KVT>
struct KvLoader;

// F32 pool: one float4 per lane.
template <>
struct KvLoader<KANSO_KV_F32> {
    __device__ __forceinline__ static float4 load(const void* pool, const void*, size_t row, int D, int dl) {
        return *reinterpret_cast<const float4*>(static_cast<const float*>(pool) + row * D + dl * 4);
    }
};

// INT8 pool with one f32 scale per (token, KV head): (q as f32) * scale.
template <>
struct KvLoader<KANSO_KV_INT8> {
    __device__ __forceinline__ static float4 load(const void* pool, const void* scales, size_t row, int D, int dl) {
        const char4 q = *reinterpret_cast<const char4*>(static_cast<const int8_t*>(pool) + row * D + dl * 4);
        const float sc = static_cast<const float*>(scales)[row];
        return make_float4(static_cast<float>(q.x) * sc, static_cast<float>(q.y) * sc,
                           static_cast<float>(q.z) * sc, static_cast<float>(q.w) * sc);
    }
};

// Q8_0 pool with one f16 scale per 32 elements: d * (q as f32).
template <>
struct KvLoader<KANSO_KV_Q8_0> {
    __device__ __forceinline__ static float4 load(const void* pool, const void* scales, size_t row, int D, int dl) {
        const char4 q = *reinterpret_cast<const char4*>(static_cast<const int8_t*>(pool) + row * D + dl * 4);
        const __half h = static_cast<const __half*>(scales)[row * (D / 32) + (dl * 4) / 32];
        const float d = __half2float(h);
        return make_float4(d * static_cast<float>(q.x), d * static_cast<float>(q.y),
                           d * static_cast<float>(q.z), d * static_cast<float>(q.w));
    }
};

__device__ __forceinline__ float dot4(float4 a, float4 b) {
    return a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w;
}

template <int D, int GMAX, int KVT>
__global__ __launch_bounds__(kThreads) void attn_stage1(AttnArgs a) {
    constexpr int LPT = D / 4;          // lanes per token
    constexpr int TPI = kWave / LPT;    // tokens per load instruction
    constexpr int NL = 8;               // tokens per lane per tile
    constexpr int TT = TPI * NL;        // tokens per wave tile
    __shared__ float sm_acc[kWaves][GMAX][D];
    __shared__ float sm_m[kWaves][GMAX];
    __shared__ float sm_l[kWaves][GMAX];

    const int lane = threadIdx.x & (kWave - 1);
    const int wv = threadIdx.x / kWave;
    const int ts = lane / LPT;
    const int dl = lane % LPT;
    const uint32_t G = a.group;
    const uint32_t n_work = *a.n_items * a.num_kv_heads;

    for (uint32_t w = blockIdx.x; w < n_work; w += gridDim.x) {
        const int4 it = a.items[w / a.num_kv_heads];
        const uint32_t kvh = w % a.num_kv_heads;
        const uint32_t row = static_cast<uint32_t>(it.x), part = static_cast<uint32_t>(it.y);
        const uint32_t limit = static_cast<uint32_t>(it.z), seq = static_cast<uint32_t>(it.w);
        const uint32_t t_begin = part * a.part_size;
        const uint32_t t_end = min(t_begin + a.part_size, limit);

        float4 qv[GMAX], acc[GMAX];
        float m[GMAX], l[GMAX];
#pragma unroll
        for (int g = 0; g < GMAX; ++g) {
            qv[g] = make_float4(0.f, 0.f, 0.f, 0.f);
            acc[g] = make_float4(0.f, 0.f, 0.f, 0.f);
            m[g] = -INFINITY;
            l[g] = 0.f;
            if (g < static_cast<int>(G))
                qv[g] = *reinterpret_cast<const float4*>(
                    a.q + (static_cast<size_t>(row) * a.num_heads + kvh * G + g) * D + dl * 4);
        }
        const uint32_t* table = a.tables + static_cast<size_t>(seq) * a.max_blocks;

        for (uint32_t tile0 = t_begin + wv * TT; tile0 < t_end; tile0 += kWaves * TT) {
            float4 kx[NL], vx[NL];
            bool ok[NL];
#pragma unroll
            for (int i = 0; i < NL; ++i) {
                const uint32_t t = tile0 + i * TPI + ts;
                ok[i] = t < t_end;
                kx[i] = make_float4(0.f, 0.f, 0.f, 0.f);
                vx[i] = kx[i];
                if (ok[i]) {
                    const uint32_t blk = a.bs_shift < 32 ? (t >> a.bs_shift) : t / a.block_size;
                    const uint32_t off = t - blk * a.block_size;
                    uint32_t phys = table[blk];
                    if (phys >= a.num_blocks) {
                        raise_status(a.status, KANSO_DEV_BLOCK_OOB);
                        phys = 0;
                    }
                    const size_t r = (static_cast<size_t>(phys) * a.block_size + off) * a.num_kv_heads + kvh;
                    kx[i] = KvLoader<KVT>::load(a.k_pool, a.k_scales, r, D, dl);
                    vx[i] = KvLoader<KVT>::load(a.v_pool, a.v_scales, r, D, dl);
                }
            }
#pragma unroll
            for (int g = 0; g < GMAX; ++g) {
                if (g >= static_cast<int>(G)) break;
                float sc[NL];
                float mt = -INFINITY;
#pragma unroll
                for (int i = 0; i < NL; ++i) {
                    float d = dot4(qv[g], kx[i]);
#pragma unroll
                    for (int o = 1; o < LPT; o <<= 1) d += wave_xor(d, o);
                    sc[i] = ok[i] ? d * a.scale_log2 : -INFINITY;
                    mt = fmaxf(mt, sc[i]);
                }
#pragma unroll
                for (int o = LPT; o < kWave; o <<= 1) mt = fmaxf(mt, wave_xor(mt, o));
                const float mn = fmaxf(m[g], mt);
                const float alpha = exp2f(m[g] - mn);
                float ps = 0.f;
                float4 pv = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
                for (int i = 0; i < NL; ++i) {
                    const float p = exp2f(sc[i] - mn);
                    ps += p;
                    pv.x += p * vx[i].x;
                    pv.y += p * vx[i].y;
                    pv.z += p * vx[i].z;
                    pv.w += p * vx[i].w;
                }
#pragma unroll
                for (int o = LPT; o < kWave; o <<= 1) ps += wave_xor(ps, o);
                l[g] = l[g] * alpha + ps;
                acc[g].x = acc[g].x * alpha + pv.x;
                acc[g].y = acc[g].y * alpha + pv.y;
                acc[g].z = acc[g].z * alpha + pv.z;
                acc[g].w = acc[g].w * alpha + pv.w;
                m[g] = mn;
            }
        }

        // Sum the token groups of the wave; lanes of group 0 then hold the wave's acc.
#pragma unroll
        for (int g = 0; g < GMAX; ++g) {
            if (g >= static_cast<int>(G)) break;
#pragma unroll
            for (int o = LPT; o < kWave; o <<= 1) {
                acc[g].x += wave_xor(acc[g].x, o);
                acc[g].y += wave_xor(acc[g].y, o);
                acc[g].z += wave_xor(acc[g].z, o);
                acc[g].w += wave_xor(acc[g].w, o);
            }
            if (ts == 0) *reinterpret_cast<float4*>(&sm_acc[wv][g][dl * 4]) = acc[g];
            if (lane == 0) {
                sm_m[wv][g] = m[g];
                sm_l[wv][g] = l[g];
            }
        }
        __syncthreads();
        for (uint32_t e = threadIdx.x; e < G * D; e += kThreads) {
            const uint32_t g = e / D, d = e % D;
            float M = -INFINITY;
#pragma unroll
            for (int x = 0; x < kWaves; ++x) M = fmaxf(M, sm_m[x][g]);
            float o = 0.f, L = 0.f;
#pragma unroll
            for (int x = 0; x < kWaves; ++x) {
                const float f = exp2f(sm_m[x][g] - M);  // 0 for a wave with no tile
                o += sm_acc[x][g][d] * f;
                L += sm_l[x][g] * f;
            }
            const size_t slot = (static_cast<size_t>(row) * a.num_heads + kvh * G + g) * a.max_parts + part;
            a.part_out[slot * D + d] = o;
            if (d == 0) a.part_stats[slot] = make_float2(M, L);
        }
        __syncthreads();
    }
}

// One wave per (row, query head): merge the row's partitions,
// out = sum_p acc_p 2^(m_p - M) / sum_p l_p 2^(m_p - M)
// (paged_attention_v2.metal:154-205), 1/denominator = 0 for an empty row.
template <int D>
__global__ __launch_bounds__(kThreads) void attn_reduce(AttnArgs a) {
    constexpr int PER = (D + kWave - 1) / kWave;
    const int lane = threadIdx.x & (kWave - 1);
    const uint32_t gw = blockIdx.x * kWaves + threadIdx.x / kWave;
    if (gw >= a.total_q * a.num_heads) return;
    const uint32_t row = gw / a.num_heads, h = gw % a.num_heads;
    // Sequence of this row: last s with cu[s] <= row.
    uint32_t lo = 0, hi = a.num_seqs;
    while (hi - lo > 1) {
        const uint32_t mid = (lo + hi) / 2;
        if (static_cast<uint32_t>(a.cu[mid]) <= row) lo = mid;
        else hi = mid;
    }
    const int32_t ql = a.cu[lo + 1] - a.cu[lo];
    const uint32_t lim = row_limit(static_cast<int32_t>(a.ctx_lens[lo]), ql,
                                   static_cast<int32_t>(row) - a.cu[lo], a.capacity);
    const uint32_t np = (lim + a.part_size - 1) / a.part_size;
    const size_t base = (static_cast<size_t>(row) * a.num_heads + h) * a.max_parts;
    float M = -INFINITY;
    for (uint32_t p = 0; p < np; ++p) M = fmaxf(M, a.part_stats[base + p].x);
    float o[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) o[k] = 0.f;
    float L = 0.f;
    for (uint32_t p = 0; p < np; ++p) {
        const float2 st = a.part_stats[base + p];
        const float f = exp2f(st.x - M);
        L += st.y * f;
        const float* src = a.part_out + (base + p) * D;
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            const int d = lane + k * kWave;
            if (d < D) o[k] += src[d] * f;
        }
    }
    const float inv = L > 0.f ? 1.0f / L : 0.f;
    float* dst = a.out + (static_cast<size_t>(row) * a.num_heads + h) * D;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const int d = lane + k * kWave;
        if (d < D) dst[d] = o[k] * inv;
    }
}

__global__ void iota_cu(int32_t* cu, uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i <= n) cu[i] = static_cast<int32_t>(i);
}

using Stage1Fn = void (*)(AttnArgs);

template <int D, int KVT>
Stage1Fn pick_group(uint32_t G) {
    return G <= 4 ? attn_stage1<D, 4, KVT> : attn_stage1<D, 8, KVT>;
}

template <int KVT>
Stage1Fn pick_stage1(uint32_t D, uint32_t G) {
    switch (D) {
        case 4: return KVT == KANSO_KV_F32 || KVT == KANSO_KV_INT8 ? pick_group<4, KVT>(G) : nullptr;
        case 8: return KVT == KANSO_KV_F32 || KVT == KANSO_KV_INT8 ? pick_group<8, KVT>(G) : nullptr;
        case 16: return KVT == KANSO_KV_F32 || KVT == KANSO_KV_INT8 ? pick_group<16, KVT>(G) : nullptr;
        case 32: return pick_group<32, KVT>(G);
        case 64: return pick_group<64, KVT>(G);
        case 128: return pick_group<128, KVT>(G);
        case 256: return pick_group<256, KVT>(G);
        default: return nullptr;
    }
}

Stage1Fn pick_stage1_kv(uint32_t kv, uint32_t D, uint32_t G) {
    if (kv == KANSO_KV_F32) return pick_stage1<KANSO_KV_F32>(D, G);
    if (kv == KANSO_KV_INT8) return pick_stage1<KANSO_KV_INT8>(D, G);
    if (kv == KANSO_KV_Q8_0) return pick_stage1<KANSO_KV_Q8_0>(D, G);
    return nullptr;
}

using ReduceFn = void (*)(AttnArgs);
ReduceFn pick_reduce(uint32_t D) {
    switch (D) {
        case 4: return attn_reduce<4>;
        case 8: return attn_reduce<8>;
        case 16: return attn_reduce<16>;
        case 32: return attn_reduce<32>;
        case 64: return attn_reduce<64>;
        case 128: return attn_reduce<128>;
        case 256: return attn_reduce<256>;
        default: return nullptr;
    }
}

constexpr uint32_t kMaxGroup = 8;
constexpr uint32_t kMaxHeadDim = 256;
constexpr uint32_t kRefPartition = 256;  // PARTITION_SIZE, paged_attention.rs:6

bool head_dim_supported(uint32_t d) {
    return d == 4 || d == 8 || d == 16 || d == 32 || d == 64 || d == 128 || d == 256;
}

// Partition size: 256 tokens (the reference's PARTITION_SIZE) unless that leaves
// too few work items to fill the chip, then halved down to 64.
uint32_t choose_partition(const kanso_ctx* ctx, uint32_t rows, uint32_t kv_heads, uint32_t capacity) {
    uint32_t P = kRefPartition;
    const uint64_t target = static_cast<uint64_t>(ctx->num_cus) * 4;
    while (P > 64 && static_cast<uint64_t>(rows) * kv_heads * ((capacity + P - 1) / P) < target) P /= 2;
    return P;
}

int run_ragged(kanso_ctx* ctx, const kanso_ragged_attention_params* p, const float* q,
               const void* kp, const void* vp, const void* ks, const void* vs,
               const uint32_t* tables, const int32_t* cu, const uint32_t* ctx_lens, float* out,
               hipStream_t stream, const char* who) {
    const uint32_t S = p->num_seqs, H = p->num_heads, HKV = p->num_kv_heads, D = p->head_dim;
    if (!q || !kp || !vp || !tables || !cu || !ctx_lens || !out) {
        set_error("%s: null buffer", who);
        return KANSO_E_INVALID_ARG;
    }
    if (S == 0 || H == 0 || HKV == 0 || p->total_q == 0) {
        set_error("%s: empty shape (seqs %u, heads %u, kv heads %u, rows %u)", who, S, H, HKV, p->total_q);
        return KANSO_E_INVALID_SHAPE;
    }
    if (H % HKV != 0) {
        set_error("%s: num_heads %u not divisible by num_kv_heads %u", who, H, HKV);
        return KANSO_E_INVALID_SHAPE;
    }
    const uint32_t G = H / HKV;
    if (G > kMaxGroup) {
        set_error("%s: GQA group size %u exceeds kernel limit %u", who, G, kMaxGroup);
        return KANSO_E_INVALID_SHAPE;
    }
    if (!head_dim_supported(D)) {
        set_error("%s: head_dim %u outside kernel range (powers of two 4..=%u)", who, D, kMaxHeadDim);
        return KANSO_E_INVALID_SHAPE;
    }
    if (p->block_size == 0 || p->max_num_blocks_per_seq == 0) {
        set_error("%s: block_size %u / max_num_blocks_per_seq %u must be non-zero", who,
                  p->block_size, p->max_num_blocks_per_seq);
        return KANSO_E_INVALID_SHAPE;
    }
    if (p->kv_dtype > KANSO_KV_Q8_0) {
        set_error("%s: unknown kv_dtype %u", who, p->kv_dtype);
        return KANSO_E_INVALID_ARG;
    }
    if (p->kv_dtype != KANSO_KV_F32 && (!ks || !vs)) {
        set_error("%s: quantized pool needs k_scales and v_scales", who);
        return KANSO_E_INVALID_ARG;
    }
    if (p->kv_dtype == KANSO_KV_Q8_0 && D % 32 != 0) {
        set_error("%s: Q8_0 KV needs head_dim %% 32 == 0 (got %u)", who, D);
        return KANSO_E_INVALID_SHAPE;
    }
    const uint64_t cap64 = static_cast<uint64_t>(p->max_num_blocks_per_seq) * p->block_size;
    if (cap64 > (1u << 30)) {
        set_error("%s: table capacity %llu tokens too large", who, static_cast<unsigned long long>(cap64));
        return KANSO_E_INVALID_SHAPE;
    }
    const uint32_t capacity = static_cast<uint32_t>(cap64);
    const uint32_t T = p->total_q;
    const uint32_t P = choose_partition(ctx, T, HKV, capacity);
    const uint32_t max_parts = (capacity + P - 1) / P;
    const uint64_t partial_elems = static_cast<uint64_t>(T) * H * max_parts * D;
    if (partial_elems > (1ull << 31)) {
        set_error("%s: %llu partial elements exceed the scratch limit", who,
                  static_cast<unsigned long long>(partial_elems));
        return KANSO_E_INVALID_SHAPE;
    }

    // Scratch: [n_items][items T*max_parts int4][stats T*H*max_parts float2][partials].
    const size_t off_items = 256;
    const size_t off_stats = align_up(off_items + static_cast<size_t>(T) * max_parts * sizeof(int4), 256);
    const size_t off_part = align_up(off_stats + static_cast<size_t>(T) * H * max_parts * sizeof(float2), 256);
    const size_t total = off_part + partial_elems * sizeof(float);
    int rc = ensure_scratch(ctx, total);
    if (rc) return rc;
    char* base = static_cast<char*>(ctx->scratch);

    AttnArgs a;
    a.q = q;
    a.k_pool = kp;
    a.v_pool = vp;
    a.k_scales = ks;
    a.v_scales = vs;
    a.tables = tables;
    a.cu = cu;
    a.ctx_lens = ctx_lens;
    a.part_out = reinterpret_cast<float*>(base + off_part);
    a.part_stats = reinterpret_cast<float2*>(base + off_stats);
    a.out = out;
    a.items = reinterpret_cast<const int4*>(base + off_items);
    a.n_items = reinterpret_cast<const uint32_t*>(base);
    a.status = ctx->status;
    a.num_seqs = S;
    a.num_heads = H;
    a.num_kv_heads = HKV;
    a.group = G;
    a.block_size = p->block_size;
    a.bs_shift = 32;
    for (uint32_t sh = 0; sh < 31; ++sh)
        if ((1u << sh) == p->block_size) a.bs_shift = sh;
    a.max_blocks = p->max_num_blocks_per_seq;
    a.num_blocks = p->num_blocks ? p->num_blocks : 0xffffffffu;
    a.part_size = P;
    a.max_parts = max_parts;
    a.total_q = T;
    a.capacity = capacity;
    a.scale_log2 = p->scale * kLog2e;

    Stage1Fn stage1 = pick_stage1_kv(p->kv_dtype, D, G);
    ReduceFn reduce = pick_reduce(D);
    if (!stage1 || !reduce) {
        set_error("%s: no kernel for head_dim %u / kv_dtype %u", who, D, p->kv_dtype);
        return KANSO_E_INVALID_SHAPE;
    }

    hipEvent_t ev;
    hipLaunchKernelGGL(build_worklist, dim3(1), dim3(kThreads), 0, stream, a,
                       reinterpret_cast<int4*>(base + off_items), reinterpret_cast<uint32_t*>(base));
    KANSO_LAUNCH_CHECK();
    const uint64_t max_work = static_cast<uint64_t>(T) * max_parts * HKV;
    const uint32_t grid = static_cast<uint32_t>(std::min<uint64_t>(max_work, static_cast<uint64_t>(ctx->num_cus) * 4));
    if ((rc = prof_begin(ctx, "attention", stream, &ev))) return rc;
    hipLaunchKernelGGL(stage1, dim3(grid), dim3(kThreads), 0, stream, a);
    KANSO_LAUNCH_CHECK();
    if ((rc = prof_end(ctx, "attention", stream, ev))) return rc;
    const uint32_t rgrid = (T * H + kWaves - 1) / kWaves;
    if ((rc = prof_begin(ctx, "reduce", stream, &ev))) return rc;
    hipLaunchKernelGGL(reduce, dim3(rgrid), dim3(kThreads), 0, stream, a);
    KANSO_LAUNCH_CHECK();
    return prof_end(ctx, "reduce", stream, ev);
}

}  // namespace
}  // namespace kanso

using namespace kanso;

extern "C" {

uint32_t kanso_paged_attention_num_partitions(const kanso_paged_attention_params* p) {
    if (!p) return 1;
    const uint64_t capacity = static_cast<uint64_t>(p->max_num_blocks_per_seq) * p->block_size;
    const uint64_t parts = (std::min<uint64_t>(capacity, 0xffffffffu) + kRefPartition - 1) / kRefPartition;
    return static_cast<uint32_t>(std::max<uint64_t>(parts, 1));
}

int kanso_validate_paged_attention_params(const kanso_paged_attention_params* p) {
    if (!p) {
        set_error("paged attention: null params");
        return KANSO_E_INVALID_ARG;
    }
    if (p->num_seqs == 0 || p->num_heads == 0 || p->num_kv_heads == 0) {
        set_error("paged attention: empty shape (seqs %u, heads %u, kv heads %u)", p->num_seqs,
                  p->num_heads, p->num_kv_heads);
        return KANSO_E_INVALID_SHAPE;
    }
    if (p->num_heads % p->num_kv_heads != 0) {
        set_error("paged attention: num_heads %u not divisible by num_kv_heads %u", p->num_heads,
                  p->num_kv_heads);
        return KANSO_E_INVALID_SHAPE;
    }
    const uint32_t group = p->num_heads / p->num_kv_heads;
    if (group > kMaxGroup) {
        set_error("paged attention: GQA group size %u exceeds kernel limit %u", group, kMaxGroup);
        return KANSO_E_INVALID_SHAPE;
    }
    if (!head_dim_supported(p->head_dim)) {
        set_error("paged attention: head_dim %u outside kernel range (powers of two 4..=%u)",
                  p->head_dim, kMaxHeadDim);
        return KANSO_E_INVALID_SHAPE;
    }
    if (p->block_size == 0 || p->max_num_blocks_per_seq == 0) {
        set_error("paged attention: block_size %u / max_num_blocks_per_seq %u must be non-zero",
                  p->block_size, p->max_num_blocks_per_seq);
        return KANSO_E_INVALID_SHAPE;
    }
    const uint64_t partial = static_cast<uint64_t>(p->num_seqs) * p->num_heads *
                             kanso_paged_attention_num_partitions(p) * p->head_dim;
    if (partial > (1ull << 31)) {
        set_error("paged attention: %llu partial elements exceed 32-bit kernel indexing",
                  static_cast<unsigned long long>(partial));
        return KANSO_E_INVALID_SHAPE;
    }
    return KANSO_OK;
}

int kanso_paged_attention_v2(kanso_ctx* ctx, const kanso_paged_attention_params* p,
                             const float* q, const float* k_cache, const float* v_cache,
                             const uint32_t* block_tables, const uint32_t* context_lens,
                             float* out, kanso_stream_t stream) {
    if (!ctx) {
        set_error("kanso_paged_attention_v2: null context");
        return KANSO_E_INVALID_ARG;
    }
    int rc = kanso_validate_paged_attention_params(p);
    if (rc) return rc;
    hipStream_t s = as_stream(stream);
    // One query row per sequence: cu_seqlens = 0..=num_seqs in the context's
    // auxiliary buffer (kept apart from scratch, which run_ragged may grow).
    rc = ensure_aux(ctx, (static_cast<size_t>(p->num_seqs) + 1) * sizeof(int32_t));
    if (rc) return rc;
    int32_t* cu_buf = static_cast<int32_t*>(ctx->aux);
    hipLaunchKernelGGL(iota_cu, dim3((p->num_seqs + 256) / 256), dim3(256), 0, s, cu_buf, p->num_seqs);
    KANSO_LAUNCH_CHECK();
    kanso_ragged_attention_params rp;
    rp.num_seqs = p->num_seqs;
    rp.num_heads = p->num_heads;
    rp.num_kv_heads = p->num_kv_heads;
    rp.head_dim = p->head_dim;
    rp.block_size = p->block_size;
    rp.max_num_blocks_per_seq = p->max_num_blocks_per_seq;
    rp.scale = p->scale;
    rp.total_q = p->num_seqs;
    rp.kv_dtype = KANSO_KV_F32;
    rp.num_blocks = 0;  // the reference call carries no pool size
    rp.max_q_len = 1;
    return run_ragged(ctx, &rp, q, k_cache, v_cache, nullptr, nullptr, block_tables, cu_buf,
                      context_lens, out, s, "kanso_paged_attention_v2");
}

int kanso_ragged_paged_attention(kanso_ctx* ctx, const kanso_ragged_attention_params* p,
                                 const float* q, const void* k_pool, const void* v_pool,
                                 const void* k_scales, const void* v_scales,
                                 const uint32_t* block_tables, const int32_t* cu_seqlens,
                                 const uint32_t* context_lens, float* out,
                                 kanso_stream_t stream) {
    if (!ctx || !p) {
        set_error("kanso_ragged_paged_attention: null context or params");
        return KANSO_E_INVALID_ARG;
    }
    return run_ragged(ctx, p, q, k_pool, v_pool, k_scales, v_scales, block_tables, cu_seqlens,
                      context_lens, out, as_stream(stream), "kanso_ragged_paged_attention");
}

}  // extern "C"
