// attention.hip — ragged paged attention (PagedAttention-v2 shape: split-K over
// context partitions + a reduce pass) for gfx950.
//
// Reference semantics: cpu_paged_attention (src/metal/paged_attention.rs:84-178) for
// a decode row, and the offset causal mask of forward_batch_rows (src/model.rs:
// 1510-1527) for the rows of a prefill chunk: row i of a sequence with q_len rows
// and context c attends keys 0..=c-q_len+i. The Metal kernel's contract
// (paged_attention_v2.metal:32-205: partitions, per-partition (m, d) statistics,
// a merge) is kept; the mapping onto CDNA4 is this file's own:
//
//  * One persistent launch, two 4-wave workgroups per CU. No work list is
//    materialised: each workgroup copies cu_seqlens / context_lens into LDS and
//    scans the per-sequence item counts; a wave maps a work index to a sequence
//    by binary search. Prefill-chunk items (64 rows x partition x KV head) go to
//    the first workgroups, decode items (one row x partition x KV head) to every
//    wave of the others, so matrix-core and bandwidth-bound work share the chip.
//  * Decode rows, F32 pool: LPT = head_dim/4 lanes share a token, each lane loads
//    one 16 B float4 of K and of V, so a load instruction moves 1 KB of fully used
//    bytes. A ring of two tiles of NL tokens per lane keeps one tile's loads in
//    flight while the other is scored. Every query head of the GQA group is
//    served from the same K/V registers: K/V bytes are read once per (token, KV
//    head).
//  * Decode rows, INT8 / Q8_0 / FP8 pool: 8 bytes per lane (one b64 load), tiles kept
//    raw and dequantized when scored, row scales folded into score and
//    probability.
//  * Prefill-chunk rows: 16 rows x G heads per wave on the bf16 matrix cores with
//    a hi / lo split of every f32 operand (v_mfma_f32_16x16x32_bf16, three
//    products per pair, f32 accumulation). A 32-key K/V tile is staged once per
//    workgroup in LDS in operand order. S^T = K Q^T puts the scores in exactly
//    the B-operand layout of O^T = V^T P^T, so probabilities never leave
//    registers and each query's softmax statistics live in that query's lanes.
//  * Block tables: the <= 64 table entries a partition touches are loaded once
//    into one register per lane; token -> physical block is a lane shuffle.
//  * Scores live in the log2 domain (scale * log2(e) folded into one multiply);
//    the online softmax rescales once per tile, not once per token.
//  * A row whose context fits one partition is normalised and written directly;
//    only rows split over several partitions go through the reduce kernel.
//  * Quantized pools (INT8 and FP8 E4M3 per token-head scale, Q8_0 per-32 f16
//    scale) use the reference's products, (q as f32) * scale, reordered only by
//    the scale folds.
#include <cmath>
#include <cstdlib>

#include "common.hpp"
#include "model.hpp"

namespace kanso {
namespace {

// Split-K scratch of kanso_ragged_paged_attention_noalloc: a fixed array in device
// memory (each GPU holds its own copy for the life of the process). Host code
// never passes the array's name to a kernel (on the host it is only a stand-in
// for the symbol): its device address is resolved once per context by
// noalloc_scratch_init and the kernels take that pointer.
constexpr size_t kNoAllocScratchBytes = 64ull << 20;
__device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kChunkBlockRows = 64;  // query rows per MFMA chunk workgroup item (4 waves x 16)

struct AttnArgs {
    const float* q;
    const void* k_pool;
    const void* v_pool;
    const void* k_scales;
    const void* v_scales;
    const uint32_t* tables;
    const int32_t* cu;
    const uint32_t* ctx_lens;
    float* part_out;     // [T][H][max_parts][D]
    float2* part_stats;  // [T][H][max_parts] (m in log2 units, l)
    uint32_t* row_np;    // [T] partitions of each query row (0: no key), for the merge
    float* out;          // [T][H][D]
    uint32_t* status;
    uint32_t num_seqs, num_heads, num_kv_heads, group, block_size, bs_shift;
    uint32_t max_blocks, num_blocks, part_size, max_parts, total_q, capacity;
    uint32_t chunk_part;  // partition size of MFMA chunk rows (>= part_size)
    uint32_t use_mfma;
    uint32_t head_major;  // pool rows [block][kv head][offset] instead of [block][offset][kv head]
    uint32_t pool_bytes, scale_bytes;  // per pool tensor, for buffer resources (< 4 GiB)
    float scale_log2;
    uint32_t out_nbk;  // 0: out is row-major [T][H][D]; else the tiled activation order, K / 32
    // Optional work list built by the caller that planned the step: n_work decode
    // items of kWorkWords words (row, partition: words 0 .. kWorkBlocks-1 the
    // partition's physical block ids, the last four row, first key, end key, the
    // row's key count), then n_work_chunk chunk items (64-row block, partition: the
    // block ids, then first row, rows, key position of the first row, partition).
    // Null: items come from the sequence tables.
    const uint32_t* work;
    uint32_t n_work;        // decode items (first in the list)
    uint32_t n_work_chunk;  // MFMA chunk items after them: 64 rows x partition each
};

constexpr uint32_t kWorkWords = kanso_ragged_work_item_words;
constexpr uint32_t kXcds = 8;  // MI355X: workgroup b of a launch runs on XCD b % 8
constexpr uint32_t kWorkBlocks = kWorkWords - 4;

// Output of query row `head / H`, head `head % H`, dims d .. (up to 4 consecutive
// floats starting at a multiple of 4: contiguous in both orders).
__device__ __forceinline__ float* out_at(const AttnArgs& a, size_t head, uint32_t D, uint32_t d) {
    if (!a.out_nbk) return a.out + head * D + d;
    const uint32_t row = static_cast<uint32_t>(head / a.num_heads);
    const uint32_t col = static_cast<uint32_t>(head % a.num_heads) * D + d;
    return a.out + act_tile_off(row, col, a.out_nbk);
}

// Key limit of row i of a sequence: keys 0..=ctx-q_len+i, clamped to what the table
// can address (the Metal kernel clamps the same way, paged_attention_v2.metal:86-89).
__device__ __forceinline__ uint32_t row_limit(int32_t ctx, int32_t q_len, int32_t i, uint32_t cap) {
    int32_t lim = ctx - q_len + i + 1;
    if (lim < 0) lim = 0;
    return min(static_cast<uint32_t>(lim), cap);
}

__device__ __forceinline__ uint32_t ceil_div(uint32_t a, uint32_t b) { return (a + b - 1) / b; }

// ---------------------------------------------------------------- work mapping
//
// No work list is materialised. Each workgroup copies cu_seqlens / context_lens
// into LDS and scans the per-sequence item counts of its kernel (chunk items for
// the MFMA kernel, decode items for the other); a wave maps its work index to a
// sequence by binary search over that prefix and to (rows, partition) by walking
// the sequence's rows or 16-row tiles.

constexpr uint32_t kMaxSeqs = 2048;  // sequences per call (LDS-resident tables)

struct SeqTable {
    int32_t cu[kMaxSeqs + 1];
    int32_t ctx[kMaxSeqs];
    uint32_t pre[kMaxSeqs + 1];  // exclusive prefix of this kernel's item counts
    uint32_t part_sums[kThreads];
};

__device__ __forceinline__ bool is_chunk_seq(const AttnArgs& a, int32_t ql) { return a.use_mfma && ql > 1; }

// Partition size of a sequence's rows: MFMA chunk rows use their own partition
// (their work items are already 64 rows wide), decode rows the split-K partition.
__device__ __forceinline__ uint32_t part_of(const AttnArgs& a, int32_t ql, uint32_t P) {
    return is_chunk_seq(a, ql) ? a.chunk_part : P;
}

// Items of one sequence for this kernel: per 64-row tile (chunk) or per row
// (decode), ceil(limit / P) partitions of the tile's last row / the row.
__device__ uint32_t seq_items(const AttnArgs& a, int32_t ql, int32_t ctx, bool chunk, uint32_t P) {
    uint32_t n = 0;
    if (chunk) {
        for (int32_t i0 = 0; i0 < ql; i0 += kChunkBlockRows)
            n += ceil_div(row_limit(ctx, ql, min(i0 + kChunkBlockRows, ql) - 1, a.capacity), P);
    } else {
        for (int32_t i = 0; i < ql; ++i) n += ceil_div(row_limit(ctx, ql, i, a.capacity), P);
    }
    return n;
}

// Fills the workgroup's SeqTable (all threads participate). Workgroup 0 also
// raises the input-validation flags.
template <bool CHUNK>
__device__ void load_seq_table(const AttnArgs& a, SeqTable& st) {
    const uint32_t tid = threadIdx.x, S = a.num_seqs;
    for (uint32_t s = tid; s <= S; s += kThreads) {
        st.cu[s] = a.cu ? a.cu[s] : static_cast<int32_t>(s);  // null: one row per sequence
        if (s < S) st.ctx[s] = static_cast<int32_t>(a.ctx_lens[s]);
    }
    __syncthreads();
    const uint32_t seg = ceil_div(S, kThreads);
    const uint32_t s0 = min(tid * seg, S), s1 = min(s0 + seg, S);
    uint32_t run = 0, flags = 0;
    for (uint32_t s = s0; s < s1; ++s) {
        const int32_t ql = st.cu[s + 1] - st.cu[s], ctx = st.ctx[s];
        if (ctx == 0) flags |= KANSO_DEV_EMPTY_CONTEXT;
        if (static_cast<uint32_t>(ctx) > a.capacity) flags |= KANSO_DEV_CONTEXT_OVERFLOW;
        if (ql > ctx) flags |= KANSO_DEV_QUERY_OVERFLOW;
        const bool chunk = is_chunk_seq(a, ql);
        run += chunk == CHUNK ? seq_items(a, ql, ctx, chunk, CHUNK ? a.chunk_part : a.part_size) : 0u;
        st.pre[s + 1] = run;  // inclusive within this thread's segment
    }
    // workgroup 0 reports: it loads the chunk table when the batch has chunk items
    // (and may then stop before the decode table), else the decode table
    if (flags && blockIdx.x == 0 && (CHUNK || !a.use_mfma)) raise_status(a.status, flags);
    // exclusive prefix of the per-thread totals: a shuffle scan inside each wave,
    // then the wave totals through LDS (one barrier instead of two per step)
    const uint32_t lane = tid & (kWave - 1), wv = tid / kWave;
    uint32_t incl = run;
#pragma unroll
    for (uint32_t off = 1; off < kWave; off <<= 1) {
        const uint32_t v = __shfl_up(incl, off, kWave);
        if (lane >= off) incl += v;
    }
    if (lane == kWave - 1) st.part_sums[wv] = incl;
    __syncthreads();
    uint32_t base = incl - run;
    for (uint32_t w = 0; w < wv; ++w) base += st.part_sums[w];
    for (uint32_t s = s0; s < s1; ++s) st.pre[s + 1] += base;
    if (tid == 0) st.pre[0] = 0;
    __syncthreads();
}

// Sequence owning item `idx`: the s with pre[s] <= idx < pre[s + 1].
__device__ __forceinline__ uint32_t find_seq(const SeqTable& st, uint32_t S, uint32_t idx) {
    uint32_t lo = 0, hi = S;
    while (hi - lo > 1) {
        const uint32_t mid = (lo + hi) >> 1;
        if (st.pre[mid] <= idx) lo = mid;
        else hi = mid;
    }
    return lo;
}

// ---------------------------------------------------------------- KV loads

template <int KVT>
struct KvLoader;

// F32 pool: one float4 per lane.
template <>
struct KvLoader<KANSO_KV_F32> {
    __device__ __forceinline__ static float4 load(const void* pool, const void*, size_t row, int D, int d0) {
        return *reinterpret_cast<const float4*>(static_cast<const float*>(pool) + row * D + d0);
    }
};

// INT8 pool with one f32 scale per (token, KV head): (q as f32) * scale.
template <>
struct KvLoader<KANSO_KV_INT8> {
    __device__ __forceinline__ static float4 load(const void* pool, const void* scales, size_t row, int D, int d0) {
        const char4 q = *reinterpret_cast<const char4*>(static_cast<const int8_t*>(pool) + row * D + d0);
        const float sc = static_cast<const float*>(scales)[row];
        return make_float4(static_cast<float>(q.x) * sc, static_cast<float>(q.y) * sc,
                           static_cast<float>(q.z) * sc, static_cast<float>(q.w) * sc);
    }
};

// FP8 pool (E4M3 bytes) with one f32 scale per (token, KV head): fp8_to_f32(q) * scale.
template <>
struct KvLoader<KANSO_KV_FP8> {
    __device__ __forceinline__ static float4 load(const void* pool, const void* scales, size_t row, int D, int d0) {
        const uint32_t w = *reinterpret_cast<const uint32_t*>(static_cast<const uint8_t*>(pool) + row * D + d0);
        const float sc = static_cast<const float*>(scales)[row];
        float x0, x1, x2, x3;
        e4m3x4_to_f32(w, x0, x1, x2, x3);
        return make_float4(x0 * sc, x1 * sc, x2 * sc, x3 * sc);
    }
};

// Q8_0 pool with one f16 scale per 32 elements: d * (q as f32).
template <>
struct KvLoader<KANSO_KV_Q8_0> {
    __device__ __forceinline__ static float4 load(const void* pool, const void* scales, size_t row, int D, int d0) {
        const char4 q = *reinterpret_cast<const char4*>(static_cast<const int8_t*>(pool) + row * D + d0);
        const float d = __half2float(static_cast<const __half*>(scales)[row * (D / 32) + d0 / 32]);
        return make_float4(d * static_cast<float>(q.x), d * static_cast<float>(q.y),
                           d * static_cast<float>(q.z), d * static_cast<float>(q.w));
    }
};

// Buffer-resource loads: the pool base and size live in scalar registers, a lane
// only carries a 32-bit byte offset (one VGPR shared by K and V), and an offset
// past the pool returns zeros without touching memory, which is how masked tokens
// are skipped. Used when every pool tensor is below 4 GiB.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
constexpr uint32_t kOffNone = 0xffffffffu;  // out of range: the load returns 0

struct PoolRsrc {
    __amdgpu_buffer_rsrc_t k, v, ks, vs;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), static_cast<short>(0),
                                             static_cast<int>(bytes), 0x00020000);
}

// Cache policy of the decode rows' F32 K/V loads: nt (non-temporal). A decode item's
// keys are read once per call and by no other item, so its lines are marked to be
// the first replaced instead of displacing what other loads reuse (the block ids,
// the keys that a prefill chunk's row blocks share in L2). Measured on the mixed
// Sarathi batch: 67.3 -> 62.0 us per call, 0.548 -> 0.595 of HBM peak; the sc1 bit
// alone changed nothing. The 1-byte pools' decode loads and the chunk rows' loads
// were slower with it (config 3 FP8 26.2 -> 29.3 us) and keep the default.
constexpr int kStream = 2;

template <int KVT>
struct KvBuf;

template <>
struct KvBuf<KANSO_KV_F32> {
    template <int CPOL = 0>
    __device__ __forceinline__ static float4 load(__amdgpu_buffer_rsrc_t pool, __amdgpu_buffer_rsrc_t, uint32_t row,
                                                  bool ok, int D, int d0) {
        const uint32_t off = ok ? (row * D + d0) * 4u : kOffNone;
        return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(pool, off, 0, CPOL));
    }
};

template <>
struct KvBuf<KANSO_KV_INT8> {
    template <int CPOL = 0>
    __device__ __forceinline__ static float4 load(__amdgpu_buffer_rsrc_t pool, __amdgpu_buffer_rsrc_t scales,
                                                  uint32_t row, bool ok, int D, int d0) {
        const uint32_t w = __builtin_amdgcn_raw_buffer_load_b32(pool, ok ? row * D + d0 : kOffNone, 0, CPOL);
        const float sc = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(scales, ok ? row * 4u : kOffNone, 0, 0));
        const char4 q = __builtin_bit_cast(char4, w);
        return make_float4(static_cast<float>(q.x) * sc, static_cast<float>(q.y) * sc,
                           static_cast<float>(q.z) * sc, static_cast<float>(q.w) * sc);
    }
};

template <>
struct KvBuf<KANSO_KV_FP8> {
    template <int CPOL = 0>
    __device__ __forceinline__ static float4 load(__amdgpu_buffer_rsrc_t pool, __amdgpu_buffer_rsrc_t scales,
                                                  uint32_t row, bool ok, int D, int d0) {
        const uint32_t w = __builtin_amdgcn_raw_buffer_load_b32(pool, ok ? row * D + d0 : kOffNone, 0, CPOL);
        const float sc = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(scales, ok ? row * 4u : kOffNone, 0, 0));
        float x0, x1, x2, x3;
        e4m3x4_to_f32(w, x0, x1, x2, x3);
        return make_float4(x0 * sc, x1 * sc, x2 * sc, x3 * sc);
    }
};

template <>
struct KvBuf<KANSO_KV_Q8_0> {
    template <int CPOL = 0>
    __device__ __forceinline__ static float4 load(__amdgpu_buffer_rsrc_t pool, __amdgpu_buffer_rsrc_t scales,
                                                  uint32_t row, bool ok, int D, int d0) {
        const uint32_t w = __builtin_amdgcn_raw_buffer_load_b32(pool, ok ? row * D + d0 : kOffNone, 0, CPOL);
        const uint16_t hb = __builtin_amdgcn_raw_buffer_load_b16(
            scales, ok ? (row * (D / 32) + d0 / 32) * 2u : kOffNone, 0, 0);
        const float d = __half2float(__ushort_as_half(hb));
        const char4 q = __builtin_bit_cast(char4, w);
        return make_float4(d * static_cast<float>(q.x), d * static_cast<float>(q.y),
                           d * static_cast<float>(q.z), d * static_cast<float>(q.w));
    }
};

// The decode arithmetic spells out its fused multiply-adds: left to the compiler,
// whether a product and a sum fuse depends on where the scheduler puts them, so two
// instantiations of one formula (buffer or global loads) could round differently.
__device__ __forceinline__ float dot4(float4 a, float4 b) {
    return fmaf(a.w, b.w, fmaf(a.z, b.z, fmaf(a.y, b.y, a.x * b.x)));
}

// Merge of `np` partials of one (row, head) by the LPG lanes of its group:
// out = sum_p acc_p 2^(m_p - M) / sum_p l_p 2^(m_p - M) (paged_attention_v2.metal:
// 154-205), 1/denominator = 0 for an empty row. LPT lanes cover a partial row
// (lane `sub` holds elements [4*N4*sub, 4*N4*(sub+1))); the R = LPG / LPT lane
// sets take partitions r, r + R, ..., and each issues U partial loads at once, so
// a round requests R*U partials. LPG = 64 (R = 4 at head_dim 64) serves rows split
// into many partitions; LPG = LPT packs several short merges into one wave.
template <int D, int LPG>
__device__ __forceinline__ void merge_partials(const AttnArgs& a, size_t head, uint32_t np, int lane) {
    constexpr int LPT = D / 4 < LPG ? D / 4 : LPG;
    constexpr int N4 = D / 4 / LPT;
    constexpr int R = LPG / LPT;
    constexpr int U = N4 >= 4 ? 2 : 8 / N4;
    const size_t base = head * a.max_parts;
    const uint32_t gl = static_cast<uint32_t>(lane) % LPG;  // lane within the group
    const uint32_t r = gl / LPT, sub = gl % LPT;
    const uint32_t d0 = sub * 4 * N4;
    float4 v[U][N4];
    float2 st[U];
    bool ok[U];
    const auto load_round = [&](uint32_t p0) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t p = p0 + r + R * u;
            ok[u] = p < np;
            const uint32_t pp = ok[u] ? p : 0;
            st[u] = a.part_stats[base + pp];
            const float4* src = reinterpret_cast<const float4*>(a.part_out + (base + pp) * D + d0);
#pragma unroll
            for (int k = 0; k < N4; ++k) v[u][k] = src[k];
        }
    };
    // the first round's partials are requested together with the statistics the
    // maximum needs, so a row of up to R*U partitions costs one memory latency
    load_round(0);
    float M = -INFINITY;
    for (uint32_t p = gl; p < np; p += LPG) M = fmaxf(M, a.part_stats[base + p].x);
    M = group_max<LPG>(M);
    float4 o[N4];
#pragma unroll
    for (int k = 0; k < N4; ++k) o[k] = make_float4(0.f, 0.f, 0.f, 0.f);
    float L = 0.f;  // counted once per partition: by the lane with sub == 0
    for (uint32_t p0 = 0;;) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const float f = ok[u] ? fast_exp2(st[u].x - M) : 0.f;
            if (sub == 0) L += st[u].y * f;
#pragma unroll
            for (int k = 0; k < N4; ++k) {
                o[k].x += v[u][k].x * f;
                o[k].y += v[u][k].y * f;
                o[k].z += v[u][k].z * f;
                o[k].w += v[u][k].w * f;
            }
        }
        p0 += R * U;
        if (p0 >= np) break;
        load_round(p0);
    }
    L = group_sum<LPG>(L);
#pragma unroll
    for (int k = 0; k < N4; ++k)
#pragma unroll
        for (int m = LPT; m < LPG; m <<= 1) {
            o[k].x += wave_xor(o[k].x, m);
            o[k].y += wave_xor(o[k].y, m);
            o[k].z += wave_xor(o[k].z, m);
            o[k].w += wave_xor(o[k].w, m);
        }
    const float inv = L > 0.f ? 1.0f / L : 0.f;
    if (r == 0)
#pragma unroll
        for (int k = 0; k < N4; ++k)
            *reinterpret_cast<float4*>(out_at(a, head, D, d0 + 4 * k)) =
                make_float4(o[k].x * inv, o[k].y * inv, o[k].z * inv, o[k].w * inv);
}

__device__ __forceinline__ float comp(const float4& v, int i) {
    return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// Partition geometry of one (row set, partition): keys [t_begin, t_end), the block
// ids they touch loaded one per lane (lane j holds table[blk0 + j]).
struct PartView {
    uint32_t t_begin, t_end, blk0;
    int tab;
    uint32_t kvh = 0;  // the item's KV head (chunk items)
};

__device__ __forceinline__ uint32_t block_of(const AttnArgs& a, uint32_t t) {
    return a.bs_shift < 32 ? (t >> a.bs_shift) : t / a.block_size;
}

__device__ __forceinline__ PartView load_part(const AttnArgs& a, uint32_t seq, uint32_t t_begin,
                                              uint32_t t_end, int lane) {
    PartView pv;
    pv.t_begin = t_begin;
    pv.t_end = t_end;
    pv.blk0 = block_of(a, t_begin);
    const uint32_t nblk = block_of(a, t_end - 1) - pv.blk0 + 1;  // <= 64 by choice of P
    uint32_t phys = 0;
    if (static_cast<uint32_t>(lane) < nblk) {
        phys = a.tables[static_cast<size_t>(seq) * a.max_blocks + pv.blk0 + lane];
        if (phys >= a.num_blocks) {
            raise_status(a.status, KANSO_DEV_BLOCK_OOB);
            phys = 0;
        }
    }
    pv.tab = static_cast<int>(phys);
    return pv;
}

// Pool row (block * bs + offset) * Hkv + kv_head of token t (t inside the view).
__device__ __forceinline__ size_t pool_row(const AttnArgs& a, const PartView& pv, uint32_t t, uint32_t kvh) {
    const uint32_t blk = block_of(a, t);
    const uint32_t phys = static_cast<uint32_t>(__shfl(pv.tab, static_cast<int>(blk - pv.blk0), kWave));
    const uint32_t off = t - blk * a.block_size;
    if (a.head_major) return (static_cast<size_t>(phys) * a.num_kv_heads + kvh) * a.block_size + off;
    return (static_cast<size_t>(phys) * a.block_size + off) * a.num_kv_heads + kvh;
}

// ---------------------------------------------------------------- decode rows

template <int D, int KVT, int NL>
struct DecodeTile {
    float4 k[NL], v[NL];
};

template <int D, int KVT, int NL, bool BUF>
__device__ __forceinline__ void decode_load(const AttnArgs& a, const PoolRsrc& rs, const PartView& pv,
                                            uint32_t tile0, uint32_t kvh, int ts, int dl,
                                            DecodeTile<D, KVT, NL>& tl) {
    constexpr int TPI = kWave / (D / 4);
#pragma unroll
    for (int i = 0; i < NL; ++i) {
        const uint32_t t = tile0 + i * TPI + ts;
        const bool ok = t < pv.t_end;
        if constexpr (BUF) {
            const uint32_t r = static_cast<uint32_t>(pool_row(a, pv, ok ? t : tile0, kvh));
            tl.k[i] = KvBuf<KVT>::template load<(KVT == KANSO_KV_F32 ? kStream : 0)>(rs.k, rs.ks, r, ok, D, dl * 4);
            tl.v[i] = KvBuf<KVT>::template load<(KVT == KANSO_KV_F32 ? kStream : 0)>(rs.v, rs.vs, r, ok, D, dl * 4);
        } else {
            const size_t r = pool_row(a, pv, ok ? t : tile0, kvh);  // masked: re-read a valid row
            tl.k[i] = KvLoader<KVT>::load(a.k_pool, a.k_scales, r, D, dl * 4);
            tl.v[i] = KvLoader<KVT>::load(a.v_pool, a.v_scales, r, D, dl * 4);
        }
    }
}

template <int D, int GMAX, int KVT, int NL>
__device__ __forceinline__ void decode_compute(const AttnArgs& a, const PartView& pv, uint32_t tile0,
                                               int ts, const float4 (&qv)[GMAX], float4 (&acc)[GMAX],
                                               float (&m)[GMAX], float (&l)[GMAX],
                                               const DecodeTile<D, KVT, NL>& tl) {
    constexpr int LPT = D / 4;
    constexpr int TPI = kWave / LPT;
    const uint32_t G = a.group;
#pragma unroll
    for (int g = 0; g < GMAX; ++g) {
        if (g >= static_cast<int>(G)) break;
        float sc[NL];
        float mt = -INFINITY;
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const float d = group_sum<LPT>(dot4(qv[g], tl.k[i]));
            const bool ok = tile0 + i * TPI + ts < pv.t_end;
            sc[i] = ok ? d * a.scale_log2 : -INFINITY;
            mt = fmaxf(mt, sc[i]);
        }
#pragma unroll
        for (int o = LPT; o < kWave; o <<= 1) mt = fmaxf(mt, wave_xor(mt, o));
        const float mn = fmaxf(m[g], mt);  // finite: every tile holds a live token
        const float alpha = fast_exp2(m[g] - mn);
        float ps = 0.f;
        float4 pv4 = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const float p = fast_exp2(sc[i] - mn);
            ps += p;
            pv4.x = fmaf(p, tl.v[i].x, pv4.x);
            pv4.y = fmaf(p, tl.v[i].y, pv4.y);
            pv4.z = fmaf(p, tl.v[i].z, pv4.z);
            pv4.w = fmaf(p, tl.v[i].w, pv4.w);
        }
#pragma unroll
        for (int o = LPT; o < kWave; o <<= 1) ps += wave_xor(ps, o);
        l[g] = fmaf(l[g], alpha, ps);
        acc[g].x = fmaf(acc[g].x, alpha, pv4.x);
        acc[g].y = fmaf(acc[g].y, alpha, pv4.y);
        acc[g].z = fmaf(acc[g].z, alpha, pv4.z);
        acc[g].w = fmaf(acc[g].w, alpha, pv4.w);
        m[g] = mn;
    }
}

// One decode item: query row `row`, KV head kvh, keys [pv.t_begin, pv.t_end) of the
// row's `limit` keys, the partition's block ids in pv.
template <int D, int GMAX, int KVT, int NL, int NB, bool BUF>
__device__ void decode_body(const AttnArgs& a, const PoolRsrc& rs, uint32_t row, uint32_t kvh, uint32_t limit,
                            const PartView& pv, int lane) {
    constexpr int LPT = D / 4;
    constexpr int TT = (kWave / LPT) * NL;
    const int ts = lane / LPT, dl = lane % LPT;
    const uint32_t G = a.group;
    const uint32_t t_begin = pv.t_begin, t_end = pv.t_end;
    const uint32_t part = t_begin / a.part_size;

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

    // A ring of NB tiles: while one tile is scored, the loads of the next NB - 1
    // are in flight. The ring is walked NB tiles per iteration so every buffer
    // index is a compile-time constant (registers, never scratch).
    DecodeTile<D, KVT, NL> ring[NB];
#pragma unroll
    for (int j = 0; j + 1 < NB; ++j)
        if (t_begin + j * TT < t_end) decode_load<D, KVT, NL, BUF>(a, rs, pv, t_begin + j * TT, kvh, ts, dl, ring[j]);
    for (uint32_t t0 = t_begin; t0 < t_end; t0 += NB * TT) {
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const uint32_t tj = t0 + j * TT;
            if (tj >= t_end) break;
            const uint32_t nxt = tj + (NB - 1) * TT;
            // The next tile's loads sit under a branch, so the compiler waits for every
            // load in flight (vmcnt(0)) before scoring the current tile: a wave then has
            // about one tile in flight. Issued unconditionally (keys past the partition
            // read out of range), two overlap and one wave streams 25% faster alone
            // (240 items of 512 keys: 51.9 -> 39.0 us), but with the chip full the
            // headline is unchanged and config 3 is 5% slower, so the branch stays.
            if (nxt < t_end) decode_load<D, KVT, NL, BUF>(a, rs, pv, nxt, kvh, ts, dl, ring[(j + NB - 1) % NB]);
            decode_compute<D, GMAX, KVT, NL>(a, pv, tj, ts, qv, acc, m, l, ring[j]);
        }
    }

    const bool single = t_begin == 0 && t_end == limit;  // whole context in this partition
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
        const size_t head = static_cast<size_t>(row) * a.num_heads + kvh * G + g;
        if (single) {
            const float inv = l[g] > 0.f ? 1.0f / l[g] : 0.f;
            if (ts == 0)
                *reinterpret_cast<float4*>(out_at(a, head, D, dl * 4)) =
                    make_float4(acc[g].x * inv, acc[g].y * inv, acc[g].z * inv, acc[g].w * inv);
            continue;
        }
        const size_t slot = head * a.max_parts + part;
        if (ts == 0) *reinterpret_cast<float4*>(a.part_out + slot * D + dl * 4) = acc[g];
        if (lane == 0) a.part_stats[slot] = make_float2(m[g], l[g]);
    }
}

template <int D, int GMAX, int KVT, int NL, int NB, bool BUF>
__device__ void decode_item(const AttnArgs& a, const SeqTable& st, const PoolRsrc& rs, uint32_t row, uint32_t part,
                            uint32_t P, uint32_t seq, uint32_t kvh, int lane) {
    const int32_t ql = st.cu[seq + 1] - st.cu[seq];
    const uint32_t limit = row_limit(st.ctx[seq], ql, static_cast<int32_t>(row) - st.cu[seq], a.capacity);
    const uint32_t t_begin = part * P;
    const PartView pv = load_part(a, seq, t_begin, min(t_begin + P, limit), lane);
    decode_body<D, GMAX, KVT, NL, NB, BUF>(a, rs, row, kvh, limit, pv, lane);
}

// ---------------------------------------------------------------- decode rows, 1-byte pools
//
// INT8 / Q8_0 / FP8 pools keep their tiles raw: a lane loads QE = 8 elements (8 bytes,
// one b64 buffer load) of a token row plus that row's scale, and dequantizes only
// when the tile is scored. A tile of NL rows per lane then carries twice the bytes
// of the float path in fewer registers. The per-row scale of K folds into the
// score (s = scale_k * sum q k) and that of V into the probability (p * scale_v),
// one multiply each instead of one per element; the reference dequantizes each
// element first ((q as f32) * scale, src/kv_cache/quantized_storage.rs:284-357),
// which only reorders
// the same products. (A lane's 8 elements always sit in one Q8_0 block, so the
// scale is applied to each lane's partial sum before the lanes are added.)
constexpr int kQE = 8;

template <int NL>
struct DecodeTileQ {
    uint2 k[NL], v[NL];
    float ks[NL], vs[NL];
};

template <int KVT>
__device__ __forceinline__ float load_row_scale(__amdgpu_buffer_rsrc_t sc, uint32_t row, bool ok, int D, int d0) {
    if constexpr (KVT == KANSO_KV_INT8 || KVT == KANSO_KV_FP8) {
        return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(sc, ok ? row * 4u : kOffNone, 0, 0));
    } else {
        const uint16_t hb = __builtin_amdgcn_raw_buffer_load_b16(
            sc, ok ? (row * static_cast<uint32_t>(D / 32) + static_cast<uint32_t>(d0 / 32)) * 2u : kOffNone, 0, 0);
        return __half2float(__ushort_as_half(hb));
    }
}

// 8 pool bytes -> f32: int8 (INT8, Q8_0) or E4M3 (FP8) values, before the scale.
template <int KVT>
__device__ __forceinline__ void bytes8_to_f32(uint2 w, float (&f)[kQE]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        if constexpr (KVT == KANSO_KV_FP8) {
            if (j == 0) {
                e4m3x4_to_f32(w.x, f[0], f[1], f[2], f[3]);
                e4m3x4_to_f32(w.y, f[4], f[5], f[6], f[7]);
            }
        } else {
            f[j] = static_cast<float>(static_cast<int8_t>((w.x >> (8 * j)) & 0xff));
            f[4 + j] = static_cast<float>(static_cast<int8_t>((w.y >> (8 * j)) & 0xff));
        }
    }
}

template <int D, int KVT, int NL>
__device__ __forceinline__ void decode_load_q(const AttnArgs& a, const PoolRsrc& rs, const PartView& pv,
                                              uint32_t tile0, uint32_t kvh, int ts, int dl, DecodeTileQ<NL>& tl) {
    constexpr int TPI = kWave / (D / kQE);
#pragma unroll
    for (int i = 0; i < NL; ++i) {
        const uint32_t t = tile0 + i * TPI + ts;
        const bool ok = t < pv.t_end;
        const uint32_t r = static_cast<uint32_t>(pool_row(a, pv, ok ? t : tile0, kvh));
        const uint32_t off = ok ? r * D + static_cast<uint32_t>(dl * kQE) : kOffNone;
        tl.k[i] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rs.k, off, 0, 0));
        tl.v[i] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rs.v, off, 0, 0));
        tl.ks[i] = load_row_scale<KVT>(rs.ks, r, ok, D, dl * kQE);
        tl.vs[i] = load_row_scale<KVT>(rs.vs, r, ok, D, dl * kQE);
    }
}

// q is pre-multiplied by scale * log2(e), so the score is sum over lanes of
// ks * sum(q k) in log2 units.
template <int D, int GMAX, int KVT, int NL>
__device__ __forceinline__ void decode_compute_q(const AttnArgs& a, const PartView& pv, uint32_t tile0, int ts,
                                                 const float (&q)[GMAX][kQE], float (&acc)[GMAX][kQE],
                                                 float (&m)[GMAX], float (&l)[GMAX], const DecodeTileQ<NL>& tl) {
    constexpr int LPT = D / kQE;
    constexpr int TPI = kWave / LPT;
    const uint32_t G = a.group;
    float sc[GMAX][NL];
#pragma unroll
    for (int i = 0; i < NL; ++i) {
        float kf[kQE];
        bytes8_to_f32<KVT>(tl.k[i], kf);
        const bool ok = tile0 + i * TPI + ts < pv.t_end;
#pragma unroll
        for (int g = 0; g < GMAX; ++g) {
            if (g >= static_cast<int>(G)) break;
            float d = 0.f;
#pragma unroll
            for (int j = 0; j < kQE; ++j) d += q[g][j] * kf[j];
            // the scale before the sum: a Q8_0 row has one scale per 32 elements
            d = group_sum<LPT>(d * tl.ks[i]);
            sc[g][i] = ok ? d : -INFINITY;
        }
    }
    float alpha[GMAX];
#pragma unroll
    for (int g = 0; g < GMAX; ++g) {
        if (g >= static_cast<int>(G)) break;
        float mt = -INFINITY;
#pragma unroll
        for (int i = 0; i < NL; ++i) mt = fmaxf(mt, sc[g][i]);
#pragma unroll
        for (int o = LPT; o < kWave; o <<= 1) mt = fmaxf(mt, wave_xor(mt, o));
        const float mn = fmaxf(m[g], mt);  // finite: every tile holds a live token
        alpha[g] = fast_exp2(m[g] - mn);
        m[g] = mn;
        float ps = 0.f;
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            sc[g][i] = fast_exp2(sc[g][i] - mn);
            ps += sc[g][i];
        }
#pragma unroll
        for (int o = LPT; o < kWave; o <<= 1) ps += wave_xor(ps, o);
        l[g] = l[g] * alpha[g] + ps;
#pragma unroll
        for (int j = 0; j < kQE; ++j) acc[g][j] *= alpha[g];
    }
#pragma unroll
    for (int i = 0; i < NL; ++i) {
        float vf[kQE];
        bytes8_to_f32<KVT>(tl.v[i], vf);
#pragma unroll
        for (int g = 0; g < GMAX; ++g) {
            if (g >= static_cast<int>(G)) break;
            const float pv_ = sc[g][i] * tl.vs[i];
#pragma unroll
            for (int j = 0; j < kQE; ++j) acc[g][j] += pv_ * vf[j];
        }
    }
}

template <int D, int GMAX, int KVT, int NL, int NB>
__device__ void decode_body_q(const AttnArgs& a, const PoolRsrc& rs, uint32_t row, uint32_t kvh, uint32_t limit,
                              const PartView& pv, int lane) {
    constexpr int LPT = D / kQE;
    constexpr int TT = (kWave / LPT) * NL;
    const int ts = lane / LPT, dl = lane % LPT;
    const uint32_t G = a.group;
    const uint32_t t_begin = pv.t_begin, t_end = pv.t_end;
    const uint32_t part = t_begin / a.part_size;

    float q[GMAX][kQE], acc[GMAX][kQE], m[GMAX], l[GMAX];
#pragma unroll
    for (int g = 0; g < GMAX; ++g) {
        m[g] = -INFINITY;
        l[g] = 0.f;
#pragma unroll
        for (int j = 0; j < kQE; ++j) q[g][j] = acc[g][j] = 0.f;
        if (g < static_cast<int>(G)) {
            const float4* src = reinterpret_cast<const float4*>(
                a.q + (static_cast<size_t>(row) * a.num_heads + kvh * G + g) * D + dl * kQE);
            const float4 x0 = src[0], x1 = src[1];
            const float xs[kQE] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int j = 0; j < kQE; ++j) q[g][j] = xs[j] * a.scale_log2;
        }
    }

    DecodeTileQ<NL> ring[NB];
#pragma unroll
    for (int j = 0; j + 1 < NB; ++j)
        if (t_begin + j * TT < t_end) decode_load_q<D, KVT, NL>(a, rs, pv, t_begin + j * TT, kvh, ts, dl, ring[j]);
    for (uint32_t t0 = t_begin; t0 < t_end; t0 += NB * TT) {
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const uint32_t tj = t0 + j * TT;
            if (tj >= t_end) break;
            const uint32_t nxt = tj + (NB - 1) * TT;
            if (nxt < t_end) decode_load_q<D, KVT, NL>(a, rs, pv, nxt, kvh, ts, dl, ring[(j + NB - 1) % NB]);
            decode_compute_q<D, GMAX, KVT, NL>(a, pv, tj, ts, q, acc, m, l, ring[j]);
        }
    }

    const bool single = t_begin == 0 && t_end == limit;
#pragma unroll
    for (int g = 0; g < GMAX; ++g) {
        if (g >= static_cast<int>(G)) break;
#pragma unroll
        for (int j = 0; j < kQE; ++j)
#pragma unroll
            for (int o = LPT; o < kWave; o <<= 1) acc[g][j] += wave_xor(acc[g][j], o);
        const size_t head = static_cast<size_t>(row) * a.num_heads + kvh * G + g;
        if (single) {
            const float inv = l[g] > 0.f ? 1.0f / l[g] : 0.f;
            if (ts == 0) {
                static_assert(kQE == 8, "two float4 per lane");
                *reinterpret_cast<float4*>(out_at(a, head, D, dl * kQE)) =
                    make_float4(acc[g][0] * inv, acc[g][1] * inv, acc[g][2] * inv, acc[g][3] * inv);
                *reinterpret_cast<float4*>(out_at(a, head, D, dl * kQE + 4)) =
                    make_float4(acc[g][4] * inv, acc[g][5] * inv, acc[g][6] * inv, acc[g][7] * inv);
            }
            continue;
        }
        const size_t slot = head * a.max_parts + part;
        if (ts == 0) {
            float4* d4 = reinterpret_cast<float4*>(a.part_out + slot * D + dl * kQE);
            d4[0] = make_float4(acc[g][0], acc[g][1], acc[g][2], acc[g][3]);
            d4[1] = make_float4(acc[g][4], acc[g][5], acc[g][6], acc[g][7]);
        }
        if (lane == 0) a.part_stats[slot] = make_float2(m[g], l[g]);
    }
}

template <int D, int GMAX, int KVT, int NL, int NB>
__device__ void decode_item_q(const AttnArgs& a, const SeqTable& st, const PoolRsrc& rs, uint32_t row,
                              uint32_t part, uint32_t P, uint32_t seq, uint32_t kvh, int lane) {
    const int32_t ql = st.cu[seq + 1] - st.cu[seq];
    const uint32_t limit = row_limit(st.ctx[seq], ql, static_cast<int32_t>(row) - st.cu[seq], a.capacity);
    const uint32_t t_begin = part * P;
    const PartView pv = load_part(a, seq, t_begin, min(t_begin + P, limit), lane);
    decode_body_q<D, GMAX, KVT, NL, NB>(a, rs, row, kvh, limit, pv, lane);
}

// ---------------------------------------------------------------- chunk rows (MFMA)

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// Split of f32 values into bf16 hi + lo (x - hi is exact in f32): a product is
// then ah*bh + ah*bl + al*bh on the bf16 matrix cores with f32 accumulation, about
// 2^-16 relative error per product against the exact f32 product.
struct Bf16Split {
    bf16x8 hi, lo;
};

__device__ __forceinline__ Bf16Split split8(const float (&x)[8]) {
    Bf16Split r;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const __bf16 h = static_cast<__bf16>(x[j]);
        r.hi[j] = h;
        r.lo[j] = static_cast<__bf16>(x[j] - static_cast<float>(h));
    }
    return r;
}

__device__ __forceinline__ floatx4 mfma3(const Bf16Split& a, const Bf16Split& b, floatx4 c) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.hi, b.hi, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.hi, b.lo, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.lo, b.hi, c, 0, 0, 0);
    return c;
}

// ---------------------------------------------------------------- decode rows, 1-byte pools, S on MFMA
//
// head_dim 64, GQA groups of at most 4 heads: S = Q K^T of a decode row runs on
// v_mfma_f32_16x16x32_bf16. Q (query heads x 32 dims, split into bf16 hi + lo) is
// the A operand, built once per item; K^T (32 dims x 16 keys) is the B operand, and
// lane l's share of it is exactly one 8-byte load of its key's row (key l % 16,
// dims 8 (l / 16) .. +7 of a 32-dim half): int8 and E4M3 values are exact in bf16, so
// K is not split. C lands as S[head 4 (l / 16) + r][key l % 16]: the 16 lanes of the
// first row hold every head's score of their key, so the softmax runs once per key,
// not once per lane of a key. P V stays on the vector ALU: lane l accumulates its
// key's V row (16 of the dims) with that key's probabilities, fetched from the
// first-row lane of the key by one shuffle per head and 16-key group; the 16 keys of
// a row are summed once per item. Scales as in the vector path: the K scale of a
// key (per 32-dim half for Q8_0) multiplies its score, the V scale its probability.
// Used for FP8 pools, whose byte conversion made the vector path instruction-bound
// (config 3: 38.0 -> 33.7 us); INT8 and Q8_0 pools measured slower here (32.0 -> 34.1
// and 33.1 -> 37.5 us: their cost is the chain of dependent loads, not the ALU), so
// they keep the vector path.
constexpr int kMqGroups = 3;  // 16-key groups per tile (4 spills with FP8 and Q8_0)

template <int NG>
struct MqTile {
    uint2 k[NG][2], v[NG][2];     // [group][32-dim half]: 8 bytes of key (16 gi + l % 16)
    float ks[NG][2], vs[NG][2];   // row scales ([gi][0] only for INT8 / FP8)
};

template <int KVT, int NG>
__device__ __forceinline__ void mq_load(const AttnArgs& a, const PoolRsrc& rs, const PartView& pv, uint32_t tile0,
                                        uint32_t kvh, int c, int j, MqTile<NG>& tl) {
#pragma unroll
    for (int gi = 0; gi < NG; ++gi) {
        const uint32_t key = tile0 + 16 * gi + c;
        const bool ok = key < pv.t_end;
        const uint32_t r = static_cast<uint32_t>(pool_row(a, pv, ok ? key : tile0, kvh));
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t off = ok ? r * 64u + static_cast<uint32_t>(32 * h + 8 * j) : kOffNone;
            tl.k[gi][h] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rs.k, off, 0, 0));
            tl.v[gi][h] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rs.v, off, 0, 0));
            if (KVT == KANSO_KV_Q8_0 || h == 0) {
                tl.ks[gi][h] = load_row_scale<KVT>(rs.ks, r, ok, 64, 32 * h);
                tl.vs[gi][h] = load_row_scale<KVT>(rs.vs, r, ok, 64, 32 * h);
            }
        }
    }
}

template <int KVT>
__device__ __forceinline__ bf16x8 bytes8_to_bf16(uint2 w) {
    float f[kQE];
    bytes8_to_f32<KVT>(w, f);
    bf16x8 r;
#pragma unroll
    for (int e = 0; e < kQE; ++e) r[e] = static_cast<__bf16>(f[e]);  // exact: 8 significant bits at most
    return r;
}

template <int GMAX, int KVT, int NG>
__device__ __forceinline__ void mq_compute(const AttnArgs& a, const PartView& pv, uint32_t tile0, int lane,
                                           const Bf16Split (&qa)[2], float (&acc)[GMAX][2][kQE],
                                           float (&m)[GMAX], float (&l)[GMAX], const MqTile<NG>& tl) {
    const int c = lane & 15;
    const uint32_t G = a.group;
    float sc[NG][4];  // S[head r][key 16 gi + c] (first row of lanes)
#pragma unroll
    for (int gi = 0; gi < NG; ++gi) {
        const bf16x8 k0 = bytes8_to_bf16<KVT>(tl.k[gi][0]), k1 = bytes8_to_bf16<KVT>(tl.k[gi][1]);
        const floatx4 z = {0.f, 0.f, 0.f, 0.f};
        floatx4 s0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa[0].hi, k0, z, 0, 0, 0);
        s0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa[0].lo, k0, s0, 0, 0, 0);
        floatx4 s1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa[1].hi, k1, z, 0, 0, 0);
        s1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa[1].lo, k1, s1, 0, 0, 0);
        const bool ok = tile0 + 16 * gi + c < pv.t_end;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float sv = KVT == KANSO_KV_Q8_0 ? s0[r] * tl.ks[gi][0] + s1[r] * tl.ks[gi][1]
                                                  : (s0[r] + s1[r]) * tl.ks[gi][0];
            sc[gi][r] = ok ? sv : -INFINITY;
        }
    }
    float alpha[GMAX];
#pragma unroll
    for (int g = 0; g < GMAX; ++g) {
        if (g >= static_cast<int>(G)) break;
        float mt = -INFINITY;
#pragma unroll
        for (int gi = 0; gi < NG; ++gi) mt = fmaxf(mt, sc[gi][g]);
        mt = __shfl(group_max<16>(mt), 0, kWave);  // the first row holds the heads
        const float mn = fmaxf(m[g], mt);          // finite: every tile holds a live key
        alpha[g] = fast_exp2(m[g] - mn);
        m[g] = mn;
        float ps = 0.f;
#pragma unroll
        for (int gi = 0; gi < NG; ++gi) {
            sc[gi][g] = fast_exp2(sc[gi][g] - mn);
            ps += sc[gi][g];
        }
        ps = __shfl(group_sum<16>(ps), 0, kWave);
        l[g] = l[g] * alpha[g] + ps;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int e = 0; e < kQE; ++e) acc[g][h][e] *= alpha[g];
    }
#pragma unroll
    for (int gi = 0; gi < NG; ++gi) {
        float v0[kQE], v1[kQE];
        bytes8_to_f32<KVT>(tl.v[gi][0], v0);
        bytes8_to_f32<KVT>(tl.v[gi][1], v1);
#pragma unroll
        for (int g = 0; g < GMAX; ++g) {
            if (g >= static_cast<int>(G)) break;
            const float p = __shfl(sc[gi][g], c, kWave);  // key c's probability for head g
            const float p0 = p * tl.vs[gi][0];
            const float p1 = KVT == KANSO_KV_Q8_0 ? p * tl.vs[gi][1] : p0;
#pragma unroll
            for (int e = 0; e < kQE; ++e) {
                acc[g][0][e] += p0 * v0[e];
                acc[g][1][e] += p1 * v1[e];
            }
        }
    }
}

template <int GMAX, int KVT, int NB>
__device__ void decode_item_mq(const AttnArgs& a, const SeqTable& st, const PoolRsrc& rs, uint32_t row,
                               uint32_t part, uint32_t P, uint32_t seq, uint32_t kvh, int lane) {
    constexpr int NG = kMqGroups;
    constexpr int TT = 16 * NG;
    const int c = lane & 15, j = lane >> 4;
    const uint32_t G = a.group;
    const int32_t ql = st.cu[seq + 1] - st.cu[seq];
    const uint32_t limit = row_limit(st.ctx[seq], ql, static_cast<int32_t>(row) - st.cu[seq], a.capacity);
    const uint32_t t_begin = part * P;
    const uint32_t t_end = min(t_begin + P, limit);
    const PartView pv = load_part(a, seq, t_begin, t_end, lane);

    Bf16Split qa[2];  // A operand: head c, dims 32 h + 8 j .. +7 (zero rows past the group)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        float x[kQE] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        if (c < static_cast<int>(G)) {
            const float4* src = reinterpret_cast<const float4*>(
                a.q + (static_cast<size_t>(row) * a.num_heads + kvh * G + c) * 64 + 32 * h + 8 * j);
            const float4 x0 = src[0], x1 = src[1];
            const float xs[kQE] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int e = 0; e < kQE; ++e) x[e] = xs[e] * a.scale_log2;
        }
        qa[h] = split8(x);
    }
    float acc[GMAX][2][kQE], m[GMAX], l[GMAX];
#pragma unroll
    for (int g = 0; g < GMAX; ++g) {
        m[g] = -INFINITY;
        l[g] = 0.f;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int e = 0; e < kQE; ++e) acc[g][h][e] = 0.f;
    }

    MqTile<NG> ring[NB];
#pragma unroll
    for (int i = 0; i + 1 < NB; ++i)
        if (t_begin + i * TT < t_end) mq_load<KVT, NG>(a, rs, pv, t_begin + i * TT, kvh, c, j, ring[i]);
    for (uint32_t t0 = t_begin; t0 < t_end; t0 += NB * TT) {
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            const uint32_t ti = t0 + i * TT;
            if (ti >= t_end) break;
            const uint32_t nxt = ti + (NB - 1) * TT;
            if (nxt < t_end) mq_load<KVT, NG>(a, rs, pv, nxt, kvh, c, j, ring[(i + NB - 1) % NB]);
            mq_compute<GMAX, KVT, NG>(a, pv, ti, lane, qa, acc, m, l, ring[i]);
        }
    }

    // sum the 16 keys of each row; lane c == 0 of row j then holds dims 32 h + 8 j .. +7
    const bool single = t_begin == 0 && t_end == limit;
#pragma unroll
    for (int g = 0; g < GMAX; ++g) {
        if (g >= static_cast<int>(G)) break;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int e = 0; e < kQE; ++e) acc[g][h][e] = group_sum<16>(acc[g][h][e]);
        const size_t head = static_cast<size_t>(row) * a.num_heads + kvh * G + g;
        if (single) {
            const float inv = l[g] > 0.f ? 1.0f / l[g] : 0.f;
            if (c == 0)
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    *reinterpret_cast<float4*>(out_at(a, head, 64, 32 * h + 8 * j)) =
                        make_float4(acc[g][h][0] * inv, acc[g][h][1] * inv, acc[g][h][2] * inv, acc[g][h][3] * inv);
                    *reinterpret_cast<float4*>(out_at(a, head, 64, 32 * h + 8 * j + 4)) =
                        make_float4(acc[g][h][4] * inv, acc[g][h][5] * inv, acc[g][h][6] * inv, acc[g][h][7] * inv);
                }
            continue;
        }
        const size_t slot = head * a.max_parts + part;
        if (c == 0)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                float4* d4 = reinterpret_cast<float4*>(a.part_out + slot * 64 + 32 * h + 8 * j);
                d4[0] = make_float4(acc[g][h][0], acc[g][h][1], acc[g][h][2], acc[g][h][3]);
                d4[1] = make_float4(acc[g][h][4], acc[g][h][5], acc[g][h][6], acc[g][h][7]);
            }
        if (lane == 0) a.part_stats[slot] = make_float2(m[g], l[g]);
    }
}

// ---- chunk workgroup: 4 waves x 16 query rows share every K/V tile
//
// A 32-key tile is loaded once per workgroup with coalesced 16 B loads (each
// thread: 2 float4 of K, 2 of V), split to bf16 hi / lo once, and stored in LDS
// already in MFMA operand order, so a wave fetches an operand with one
// ds_read_b128 per plane. Raw tiles are prefetched two ahead in registers.
constexpr int kChunkWaveRows = 16;
static_assert(kChunkBlockRows == kChunkWaveRows * kWaves, "one 16-row slice per wave");
constexpr int kChunkKeys = 32;

// LDS image of one tile. K: [b][sd][kq][m] holds K[key 16b + m][d = 32sd + 8kq .. +7]
// (A operand of S^T); V: [nb][kq][m] holds V[key 16b + 4kq + r][d = 4m + nb] at
// element j = 4b + r (A operand of O^T). hi and lo planes each.
struct ChunkStage {
    bf16x8 k_hi[2][2][4][16], k_lo[2][2][4][16];
    bf16x8 v_hi[4][4][16], v_lo[4][4][16];
};

struct RawTile {
    float4 k[2], v[2];  // float4 f = tid + 256 j: key f / 16, d0 = 4 (f % 16)
};

template <int KVT>
__device__ __forceinline__ void chunk_load_raw(const AttnArgs& a, const PoolRsrc& rs, const PartView& pv,
                                               uint32_t t0, uint32_t kvh, RawTile& rt) {
    constexpr int D = 64;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const uint32_t f = threadIdx.x + kThreads * j;
        const uint32_t t = t0 + f / 16;
        const bool ok = t < pv.t_end;
        const uint32_t r = static_cast<uint32_t>(pool_row(a, pv, ok ? t : t0, kvh));
        rt.k[j] = KvBuf<KVT>::load(rs.k, rs.ks, r, ok, D, 4 * (f % 16));
        rt.v[j] = KvBuf<KVT>::load(rs.v, rs.vs, r, ok, D, 4 * (f % 16));
    }
}

__device__ __forceinline__ void chunk_store(const RawTile& rt, ChunkStage& st) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const uint32_t f = threadIdx.x + kThreads * j;
        const uint32_t key = f / 16, d0 = 4 * (f % 16);
        // K: 4 consecutive d of one key -> half of a 16 B operand entry.
        {
            const uint32_t b = key / 16, m = key % 16, sd = d0 / 32, kq = (d0 % 32) / 8, j0 = d0 % 8;
            const float x[4] = {rt.k[j].x, rt.k[j].y, rt.k[j].z, rt.k[j].w};
            __bf16* hi = reinterpret_cast<__bf16*>(&st.k_hi[b][sd][kq][m]) + j0;
            __bf16* lo = reinterpret_cast<__bf16*>(&st.k_lo[b][sd][kq][m]) + j0;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const __bf16 h = static_cast<__bf16>(x[c]);
                hi[c] = h;
                lo[c] = static_cast<__bf16>(x[c] - static_cast<float>(h));
            }
        }
        // V: the 4 values land in the 4 d-blocks nb = c (transpose to d-major).
        {
            const uint32_t b = key / 16, kq = (key % 16) / 4, r = key % 4, m = d0 / 4;
            const float x[4] = {rt.v[j].x, rt.v[j].y, rt.v[j].z, rt.v[j].w};
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const __bf16 h = static_cast<__bf16>(x[c]);
                reinterpret_cast<__bf16*>(&st.v_hi[c][kq][m])[4 * b + r] = h;
                reinterpret_cast<__bf16*>(&st.v_lo[c][kq][m])[4 * b + r] =
                    static_cast<__bf16>(x[c] - static_cast<float>(h));
            }
        }
    }
}

// One tile for this wave's 16 rows x G heads. Operands are fetched from LDS one key
// block (S^T) or one d-block (O^T) at a time, so only the scores / probabilities of
// the G heads stay live across the tile.
template <int G>
__device__ __forceinline__ void chunk_compute(const AttnArgs& a, const ChunkStage& st, uint32_t t0,
                                              uint32_t t_end, int lane, uint32_t lim,
                                              const Bf16Split (&qs)[G][2], floatx4 (&o)[G][4],
                                              float (&m)[G], float (&l)[G]) {
    const int kq = lane >> 4, mm = lane & 15;
    const uint32_t kbase = t0 + 4 * kq;  // key of score (b, r) is kbase + 16b + r
    float sc[G][8];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        Bf16Split k0, k1;
        k0.hi = st.k_hi[b][0][kq][mm];
        k0.lo = st.k_lo[b][0][kq][mm];
        k1.hi = st.k_hi[b][1][kq][mm];
        k1.lo = st.k_lo[b][1][kq][mm];
#pragma unroll
        for (int g = 0; g < G; ++g) {
            floatx4 s4 = {0.f, 0.f, 0.f, 0.f};
            s4 = mfma3(k0, qs[g][0], s4);
            s4 = mfma3(k1, qs[g][1], s4);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t key = kbase + 16 * b + r;
                sc[g][4 * b + r] = (key < lim && key < t_end) ? s4[r] * a.scale_log2 : -INFINITY;
            }
        }
    }
    Bf16Split pp[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        float mt = -INFINITY;
#pragma unroll
        for (int j = 0; j < 8; ++j) mt = fmaxf(mt, sc[g][j]);
        mt = fmaxf(mt, wave_xor(mt, 16));
        mt = fmaxf(mt, wave_xor(mt, 32));
        const float mn = fmaxf(m[g], mt);
        const bool live = mn != -INFINITY;
        const float alpha = live ? fast_exp2(m[g] - mn) : 1.0f;
        float ps = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            sc[g][j] = live ? fast_exp2(sc[g][j] - mn) : 0.f;
            ps += sc[g][j];
        }
        ps += wave_xor(ps, 16);
        ps += wave_xor(ps, 32);
        l[g] = l[g] * alpha + ps;
        m[g] = mn;
        pp[g] = split8(sc[g]);
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) o[g][nb] *= alpha;
    }
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
        Bf16Split v;
        v.hi = st.v_hi[nb][kq][mm];
        v.lo = st.v_lo[nb][kq][mm];
#pragma unroll
        for (int g = 0; g < G; ++g) o[g][nb] = mfma3(v, pp[g], o[g][nb]);
    }
}

// One workgroup item: 64 query rows (wave w: rows 16w .. 16w + 15 of the block) of
// one sequence, one key partition, one KV head.
template <int G, int KVT>
__device__ void chunk_body(const AttnArgs& a, const PoolRsrc& rs, ChunkStage (&stage)[2], uint32_t row0,
                           uint32_t part, int nrows_blk, int32_t pos0, const PartView& pv) {
    // pos0: key position of the block's first row (ctx - q_len + its index in the
    // sequence); row j of the block attends keys 0 ..= pos0 + j (row_limit)
    constexpr int D = 64;
    const int lane = threadIdx.x & (kWave - 1), wv = threadIdx.x / kWave;
    const uint32_t kvh = pv.kvh;
    const int nrows = min(kChunkWaveRows, nrows_blk - kChunkWaveRows * wv);  // this wave's rows (may be <= 0)
    const int qi = lane & 15;
    const bool qlive = qi < nrows;
    const uint32_t wrow0 = row0 + kChunkWaveRows * wv;
    const uint32_t lim = qlive ? row_limit(pos0 + 1, 1, kChunkWaveRows * wv + qi, a.capacity) : 0;
    const uint32_t t_begin = pv.t_begin, t_end = pv.t_end;

    Bf16Split qs[G][2];  // Q[query qi][d = 32 sd + 8 kq + j] as bf16 hi / lo (B operand of S^T)
    floatx4 o[G][4];
    float m[G], l[G];
    const uint32_t qrow = wrow0 + (qlive ? qi : 0);
#pragma unroll
    for (int g = 0; g < G; ++g) {
        m[g] = -INFINITY;
        l[g] = 0.f;
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) o[g][nb] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int sd = 0; sd < 2; ++sd) {
            float x[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            if (qlive) {
                const float* src = a.q + (static_cast<size_t>(qrow) * a.num_heads + kvh * G + g) * D +
                                   32 * sd + 8 * (lane >> 4);
                const float4 x0 = *reinterpret_cast<const float4*>(src);
                const float4 x1 = *reinterpret_cast<const float4*>(src + 4);
                x[0] = x0.x; x[1] = x0.y; x[2] = x0.z; x[3] = x0.w;
                x[4] = x1.x; x[5] = x1.y; x[6] = x1.z; x[7] = x1.w;
            }
            qs[g][sd] = split8(x);
        }
    }

    // Two raw tiles ping-pong in fixed registers (the loop is unrolled by two, so no
    // register copy waits on a load in flight), and every load is issued without a
    // branch: keys past the partition read out of range (zeros, no traffic). Tile
    // i + 2 is then in flight while tile i is scored and tile i + 1 is staged,
    // instead of every iteration waiting for all outstanding loads.
    const uint32_t n_tiles = ceil_div(t_end - t_begin, kChunkKeys);
    RawTile ra, rb;
    chunk_load_raw<KVT>(a, rs, pv, t_begin, kvh, ra);
    chunk_load_raw<KVT>(a, rs, pv, t_begin + kChunkKeys, kvh, rb);
    chunk_store(ra, stage[0]);
    __syncthreads();
    for (uint32_t i = 0; i < n_tiles; i += 2) {
        chunk_load_raw<KVT>(a, rs, pv, t_begin + kChunkKeys * (i + 2), kvh, ra);
        if (nrows > 0) chunk_compute<G>(a, stage[0], t_begin + kChunkKeys * i, t_end, lane, lim, qs, o, m, l);
        chunk_store(rb, stage[1]);
        __syncthreads();
        if (i + 1 >= n_tiles) break;
        chunk_load_raw<KVT>(a, rs, pv, t_begin + kChunkKeys * (i + 3), kvh, rb);
        if (nrows > 0)
            chunk_compute<G>(a, stage[1], t_begin + kChunkKeys * (i + 1), t_end, lane, lim, qs, o, m, l);
        chunk_store(ra, stage[0]);
        __syncthreads();
    }

    // Lane holds O^T[d = 16(lane/16) + 4r + nb][query qi] in o[g][nb][r].
    const uint32_t np = ceil_div(lim, a.chunk_part);
    const bool writer = qlive && part < np;
    const bool single = np == 1;
    const int qq = lane >> 4;
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const size_t head = static_cast<size_t>(qrow) * a.num_heads + kvh * G + g;
        if (writer) {
            const float inv = single ? (l[g] > 0.f ? 1.0f / l[g] : 0.f) : 1.0f;
            float* dst = a.part_out + (head * a.max_parts + part) * D;
#pragma unroll
            for (int r = 0; r < 4; ++r)
                *reinterpret_cast<float4*>(single ? out_at(a, head, D, 16 * qq + 4 * r) : dst + 16 * qq + 4 * r) =
                    make_float4(o[g][0][r] * inv, o[g][1][r] * inv, o[g][2][r] * inv, o[g][3][r] * inv);
            if (!single && qq == 0) a.part_stats[head * a.max_parts + part] = make_float2(m[g], l[g]);
        }
    }
}

template <int G, int KVT>
__device__ void chunk_block(const AttnArgs& a, const SeqTable& st, const PoolRsrc& rs, ChunkStage (&stage)[2],
                            uint32_t row0, uint32_t part, int nrows_blk, uint32_t seq, uint32_t kvh) {
    const int lane = threadIdx.x & (kWave - 1);
    const int32_t ql = st.cu[seq + 1] - st.cu[seq];
    const int32_t pos0 = st.ctx[seq] - ql + (static_cast<int32_t>(row0) - st.cu[seq]);
    const uint32_t lim_max = row_limit(pos0 + 1, 1, nrows_blk - 1, a.capacity);  // last row of the block
    const uint32_t t_begin = part * a.chunk_part;
    PartView pv = load_part(a, seq, t_begin, min(t_begin + a.chunk_part, lim_max), lane);
    pv.kvh = kvh;
    chunk_body<G, KVT>(a, rs, stage, row0, part, nrows_blk, pos0, pv);
}

// Decode items from the caller's work list: one load per wave gives the item's row,
// keys and block ids (no sequence table, no block-table round trip), then the same
// item body as the table-driven path.
template <int D, int GMAX, int KVT, bool BUF, int NL, int NB>
__device__ void decode_work(const AttnArgs& a, const PoolRsrc& rs, uint32_t first_wg) {
    const int lane = threadIdx.x & (kWave - 1);
    const uint32_t wave = (blockIdx.x - first_wg) * kWaves + threadIdx.x / kWave;
    const uint32_t n_waves = (gridDim.x - first_wg) * kWaves;
    const uint32_t n = a.n_work * a.num_kv_heads;
    for (uint32_t w = wave; w < n; w += n_waves) {
        const uint32_t item = w / a.num_kv_heads, kvh = w % a.num_kv_heads;
        const uint32_t word = a.work[static_cast<size_t>(item) * kWorkWords + lane];
        const uint32_t row = __builtin_amdgcn_readlane(word, kWorkBlocks);
        const uint32_t limit = __builtin_amdgcn_readlane(word, kWorkBlocks + 3);
        PartView pv;
        pv.t_begin = __builtin_amdgcn_readlane(word, kWorkBlocks + 1);
        pv.t_end = __builtin_amdgcn_readlane(word, kWorkBlocks + 2);
        pv.blk0 = block_of(a, pv.t_begin);
        const uint32_t nblk = block_of(a, pv.t_end - 1) - pv.blk0 + 1;  // <= kWorkBlocks (host-checked)
        uint32_t phys = static_cast<uint32_t>(lane) < nblk ? word : 0u;
        if (phys >= a.num_blocks) {
            raise_status(a.status, KANSO_DEV_BLOCK_OOB);
            phys = 0;
        }
        pv.tab = static_cast<int>(phys);
        if (pv.t_begin == 0 && kvh == 0 && lane == 0) a.row_np[row] = ceil_div(limit, a.part_size);
        if constexpr (KVT != KANSO_KV_F32 && BUF && D >= kQE)
            decode_body_q<D, GMAX, KVT, (GMAX <= 4 ? 8 : 4), 2>(a, rs, row, kvh, limit, pv, lane);
        else
            decode_body<D, GMAX, KVT, NL, NB, BUF>(a, rs, row, kvh, limit, pv, lane);
    }
}

// ---------------------------------------------------------------- kernels

// Rows with no key (an empty context, or more query rows than context) get zeros,
// cpu_paged_attention's output for an empty context. Grid-stride over sequences,
// by the workgroups from first_wg on (the ones that run the decode phase).
__device__ void zero_empty_rows(const AttnArgs& a, const SeqTable& st, uint32_t D, uint32_t first_wg) {
    const uint32_t n_threads = (gridDim.x - first_wg) * kThreads;
    for (uint32_t s = (blockIdx.x - first_wg) * kThreads + threadIdx.x; s < a.num_seqs; s += n_threads) {
        const int32_t ql = st.cu[s + 1] - st.cu[s];
        for (int32_t i = 0; i < ql; ++i)
            if (row_limit(st.ctx[s], ql, i, a.capacity) == 0) {
                a.row_np[st.cu[s] + i] = 0;
                const size_t head0 = static_cast<size_t>(st.cu[s] + i) * a.num_heads;
                for (uint32_t e = 0; e < a.num_heads * D; e += 4)
                    *reinterpret_cast<float4*>(out_at(a, head0 + e / D, D, e % D)) = make_float4(0.f, 0.f, 0.f, 0.f);
            }
    }
}

// The attention kernel: one persistent launch. Workgroups [0, n_chunk_wg) take the
// prefill-chunk items (64 rows x partition x KV head, grid-stride over those
// workgroups); the waves of the other workgroups take the decode items (one row x
// partition x KV head) round-robin. Compute-bound MFMA work and bandwidth-bound
// decode work therefore run side by side on different CUs. With no chunk items (or
// more chunk items than workgroups) every wave also takes decode items.
template <int D, int GMAX, int KVT, bool BUF, int GC, int NL = 8, int NB = 2>
__global__ __launch_bounds__(kThreads, 2) void attn_main(AttnArgs a) {
    __shared__ SeqTable st;
    PoolRsrc rs;
    if constexpr (BUF) {
        rs.k = make_rsrc(a.k_pool, a.pool_bytes);
        rs.v = make_rsrc(a.v_pool, a.pool_bytes);
        rs.ks = make_rsrc(a.k_scales, a.scale_bytes);
        rs.vs = make_rsrc(a.v_scales, a.scale_bytes);
    }
    if constexpr (GC == 0) {
        if (a.work) {
            decode_work<D, GMAX, KVT, BUF, NL, NB>(a, rs, 0);
            return;
        }
    }
    uint32_t n_chunk_wg = 0;
    if constexpr (GC > 0) {
        __shared__ ChunkStage stage[2];
        if (a.use_mfma && a.work) {  // chunk and decode items from the caller's list
            // Chunk work index L = kv_head * items + item, the list holding the row
            // blocks of one (sequence, partition) next to each other; with a
            // workgroup per item, the workgroups of XCD x (workgroup b runs on XCD
            // b % 8) take the contiguous run of L from x * per, so the row blocks that
            // read the same keys share an L2 rather than each fetching them from HBM.
            const uint32_t n_chunk = a.n_work_chunk * a.num_kv_heads;
            const uint32_t per = (n_chunk + kXcds - 1) / kXcds;
            n_chunk_wg = per * kXcds < gridDim.x ? per * kXcds : 0u;
            const uint32_t stride = n_chunk_wg ? n_chunk_wg : gridDim.x;
            if (n_chunk_wg == 0 || blockIdx.x < n_chunk_wg) {
                const int lane = threadIdx.x & (kWave - 1);
                for (uint32_t b = blockIdx.x; b < (n_chunk_wg ? n_chunk_wg : n_chunk); b += stride) {
                    const uint32_t w = n_chunk_wg ? (b % kXcds) * per + b / kXcds : b;
                    if (w >= n_chunk) continue;  // the round-up's idle workgroups
                    const uint32_t item = w % a.n_work_chunk, kvh_w = w / a.n_work_chunk;
                    const uint32_t word =
                        a.work[static_cast<size_t>(a.n_work + item) * kWorkWords + static_cast<uint32_t>(lane)];
                    const uint32_t row0 = __builtin_amdgcn_readlane(word, kWorkBlocks);
                    const int nrows = static_cast<int>(__builtin_amdgcn_readlane(word, kWorkBlocks + 1));
                    const int32_t pos0 = static_cast<int32_t>(__builtin_amdgcn_readlane(word, kWorkBlocks + 2));
                    const uint32_t part = __builtin_amdgcn_readlane(word, kWorkBlocks + 3);
                    PartView pv;
                    pv.kvh = kvh_w;
                    pv.t_begin = part * a.chunk_part;
                    pv.t_end = min(pv.t_begin + a.chunk_part, row_limit(pos0 + 1, 1, nrows - 1, a.capacity));
                    pv.blk0 = block_of(a, pv.t_begin);
                    const uint32_t nblk = block_of(a, pv.t_end - 1) - pv.blk0 + 1;  // <= kWorkBlocks (host-checked)
                    uint32_t phys = static_cast<uint32_t>(lane) < nblk ? word : 0u;
                    if (phys >= a.num_blocks) {
                        raise_status(a.status, KANSO_DEV_BLOCK_OOB);
                        phys = 0;
                    }
                    pv.tab = static_cast<int>(phys);
                    if (part == 0 && pv.kvh == 0 && static_cast<int>(threadIdx.x) < nrows)
                        a.row_np[row0 + threadIdx.x] =
                            ceil_div(row_limit(pos0 + 1, 1, static_cast<int32_t>(threadIdx.x), a.capacity),
                                     a.chunk_part);
                    chunk_body<GC, KVT>(a, rs, stage, row0, part, nrows, pos0, pv);
                    __syncthreads();  // the next item's prologue reuses the stages
                }
                if (n_chunk_wg) return;  // chunk workgroup: done
            }
            decode_work<D, GMAX, KVT, BUF, NL, NB>(a, rs, n_chunk_wg);
            return;
        }
        if (a.use_mfma) {
            load_seq_table<true>(a, st);
            const uint32_t n_chunk = st.pre[a.num_seqs] * a.num_kv_heads;
            n_chunk_wg = n_chunk < gridDim.x ? n_chunk : 0u;  // 0: all workgroups do both
            const uint32_t stride = n_chunk_wg ? n_chunk_wg : gridDim.x;
            if (n_chunk_wg == 0 || blockIdx.x < n_chunk_wg) {
                for (uint32_t w = blockIdx.x; w < n_chunk; w += stride) {
                    const uint32_t item = w / a.num_kv_heads, kvh = w % a.num_kv_heads;
                    const uint32_t s = find_seq(st, a.num_seqs, item);
                    uint32_t local = item - st.pre[s];
                    const int32_t ql = st.cu[s + 1] - st.cu[s];
                    int32_t i0 = 0;
                    for (; i0 < ql; i0 += kChunkBlockRows) {
                        const int32_t last = min(i0 + kChunkBlockRows, ql) - 1;
                        const uint32_t np = ceil_div(row_limit(st.ctx[s], ql, last, a.capacity), a.chunk_part);
                        if (local < np) break;
                        local -= np;
                    }
                    if (local == 0 && kvh == 0 && static_cast<int32_t>(threadIdx.x) < min(kChunkBlockRows, ql - i0))
                        a.row_np[st.cu[s] + i0 + threadIdx.x] =
                            ceil_div(row_limit(st.ctx[s], ql, i0 + threadIdx.x, a.capacity), a.chunk_part);
                    chunk_block<GC, KVT>(a, st, rs, stage, static_cast<uint32_t>(st.cu[s] + i0), local,
                                         min(kChunkBlockRows, ql - i0), s, kvh);
                    __syncthreads();  // the next item's prologue reuses the stages
                }
                if (n_chunk_wg) return;  // chunk workgroup: done
            }
            __syncthreads();  // the decode tables below overwrite the chunk tables
        }
    }
    load_seq_table<false>(a, st);
    zero_empty_rows(a, st, D, n_chunk_wg);
    const int lane = threadIdx.x & (kWave - 1);
    const uint32_t wave = (blockIdx.x - n_chunk_wg) * kWaves + threadIdx.x / kWave;
    const uint32_t n_waves = (gridDim.x - n_chunk_wg) * kWaves;
    const uint32_t n_work = st.pre[a.num_seqs] * a.num_kv_heads;
    for (uint32_t w = wave; w < n_work; w += n_waves) {
        const uint32_t item = w / a.num_kv_heads, kvh = w % a.num_kv_heads;
        const uint32_t s = find_seq(st, a.num_seqs, item);
        uint32_t local = item - st.pre[s];
        const int32_t ql = st.cu[s + 1] - st.cu[s];
        int32_t i = 0;
        if (ql > 1) {  // rows of a multi-row sequence without the MFMA path
            for (; i < ql; ++i) {
                const uint32_t np = ceil_div(row_limit(st.ctx[s], ql, i, a.capacity), a.part_size);
                if (local < np) break;
                local -= np;
            }
        }
        const uint32_t row = static_cast<uint32_t>(st.cu[s] + i);
        if (local == 0 && kvh == 0 && lane == 0)
            a.row_np[row] = ceil_div(row_limit(st.ctx[s], ql, i, a.capacity), a.part_size);
        if constexpr (KVT == KANSO_KV_FP8 && BUF && D == 64 && GMAX <= 4)
            decode_item_mq<GMAX, KVT, 2>(a, st, rs, row, local, a.part_size, s, kvh, lane);
        else if constexpr (KVT != KANSO_KV_F32 && BUF && D >= kQE)
            decode_item_q<D, GMAX, KVT, (GMAX <= 4 ? 8 : 4), 2>(a, st, rs, row, local, a.part_size, s, kvh, lane);
        else
            decode_item<D, GMAX, KVT, NL, NB, BUF>(a, st, rs, row, local, a.part_size, s, kvh, lane);
    }
}

// One group of LPG lanes per (row, query head) in a grid-stride loop: rows split
// over several partitions are merged (a kernel boundary orders them after every
// partial); single-partition rows were written by stage 1. Each row's partition
// count comes from the main kernel (row_np), so no sequence table is built here:
// the first loads are the row's statistics.
template <int D, int LPG>
__global__ __launch_bounds__(kThreads) void attn_reduce(AttnArgs a) {
    const int lane = threadIdx.x & (kWave - 1);
    constexpr uint32_t kGroups = kThreads / LPG;
    const uint32_t n_groups = gridDim.x * kGroups;
    const uint32_t n_work = a.total_q * a.num_heads;
    for (uint32_t w = blockIdx.x * kGroups + threadIdx.x / LPG; w < n_work; w += n_groups) {
        const uint32_t row = w / a.num_heads, h = w % a.num_heads;
        // written by the main kernel for every row the call's items cover; a work list
        // without a row's items leaves a stale count, which must not index past the
        // row's partials
        uint32_t np = a.row_np[row];
        if (np > a.max_parts) {
            if (h == 0) raise_status(a.status, KANSO_DEV_PARTS_OOB);
            np = 0;
        }
        if (np > 1) merge_partials<D, LPG>(a, static_cast<size_t>(row) * a.num_heads + h, np, lane);
    }
}

using Stage1Fn = void (*)(AttnArgs);

// Batches with prefill chunks get the kernel with the MFMA chunk path (it needs
// the exact group size); all-decode batches the one without it (fewer registers).
template <int D, int GMAX, int KVT, bool BUF>
Stage1Fn pick_main_g(uint32_t G, bool mfma) {
    if constexpr (D == 64 && BUF) {
        if (mfma) switch (G) {
            case 1: return attn_main<D, GMAX, KVT, BUF, 1>;
            case 2: return attn_main<D, GMAX, KVT, BUF, 2>;
            case 3: return attn_main<D, GMAX, KVT, BUF, 3>;
            case 4: return attn_main<D, GMAX, KVT, BUF, 4>;
            default: break;
        }
    }
    return attn_main<D, GMAX, KVT, BUF, 0>;
}

template <int D, int KVT>
Stage1Fn pick_group(uint32_t G, bool buf, bool mfma) {
    if (D == 64 && G == 3)  // SmolLM2 (15 / 5 heads)
        return buf ? pick_main_g<D, 3, KVT, true>(G, mfma) : pick_main_g<D, 3, KVT, false>(G, mfma);
    if (G <= 4) return buf ? pick_main_g<D, 4, KVT, true>(G, mfma) : pick_main_g<D, 4, KVT, false>(G, mfma);
    return buf ? pick_main_g<D, 8, KVT, true>(G, mfma) : pick_main_g<D, 8, KVT, false>(G, mfma);
}

template <int KVT>
Stage1Fn pick_decode(uint32_t D, uint32_t G, bool buf, bool mfma) {
    switch (D) {
        case 4: return KVT != KANSO_KV_Q8_0 ? pick_group<4, KVT>(G, buf, mfma) : nullptr;
        case 8: return KVT != KANSO_KV_Q8_0 ? pick_group<8, KVT>(G, buf, mfma) : nullptr;
        case 16: return KVT != KANSO_KV_Q8_0 ? pick_group<16, KVT>(G, buf, mfma) : nullptr;
        case 32: return pick_group<32, KVT>(G, buf, mfma);
        case 64: return pick_group<64, KVT>(G, buf, mfma);
        case 128: return pick_group<128, KVT>(G, buf, mfma);
        case 256: return pick_group<256, KVT>(G, buf, mfma);
        default: return nullptr;
    }
}

Stage1Fn pick_main_kv(uint32_t kv, uint32_t D, uint32_t G, bool buf, bool mfma) {
    if (kv == KANSO_KV_F32) return pick_decode<KANSO_KV_F32>(D, G, buf, mfma);
    if (kv == KANSO_KV_INT8) return pick_decode<KANSO_KV_INT8>(D, G, buf, mfma);
    if (kv == KANSO_KV_Q8_0) return pick_decode<KANSO_KV_Q8_0>(D, G, buf, mfma);
    if (kv == KANSO_KV_FP8) return pick_decode<KANSO_KV_FP8>(D, G, buf, mfma);
    return nullptr;
}

// Lanes per merge: a whole wave when a row may have more partitions than a
// 16-lane group covers in two rounds, else the head's natural lane count.
template <int D>
Stage1Fn pick_reduce_d(bool wide) {
    constexpr int narrow = D / 4 < kWave ? (D / 4 < 16 ? 16 : D / 4) : kWave;
    return wide ? attn_reduce<D, kWave> : attn_reduce<D, narrow>;
}

Stage1Fn pick_reduce(uint32_t D, bool wide) {
    switch (D) {
        case 4: return pick_reduce_d<4>(wide);
        case 8: return pick_reduce_d<8>(wide);
        case 16: return pick_reduce_d<16>(wide);
        case 32: return pick_reduce_d<32>(wide);
        case 64: return pick_reduce_d<64>(wide);
        case 128: return pick_reduce_d<128>(wide);
        case 256: return pick_reduce_d<256>(wide);
        default: return nullptr;
    }
}

constexpr uint32_t kMaxGroup = 8;
constexpr uint32_t kMaxHeadDim = 256;
constexpr uint32_t kRefPartition = 256;  // PARTITION_SIZE, paged_attention.rs:6

bool head_dim_supported(uint32_t d) {
    return d == 4 || d == 8 || d == 16 || d == 32 || d == 64 || d == 128 || d == 256;
}

// Decode partition. Every partial a row is split into costs a write, a read and a
// merge, so partitions are as long as the occupancy allows: the largest of 512,
// 256, 128, 64 tokens for which the decode items (sequences x KV heads x
// partitions of a context assumed to be half the table capacity, the only context
// size known on the host without reading device data) still reach one per
// resident wave of one workgroup per CU, times four for 1-byte pools (whose items
// move a quarter of the bytes). Calibrated on the benchmark batches (config 2: 512
// beats 256 by 5%; config 1: 64; config 3: 128). A device-side choice from the
// actual contexts was measured too: its extra pass cost more than it saved.
// Capped so a partition touches at most 62 table entries (one register lane each).
uint32_t choose_partition(const kanso_ctx* ctx, uint32_t seqs, uint32_t kv_heads, uint32_t capacity,
                          uint32_t block_size, uint32_t elem_bytes) {
    uint32_t P = 2 * kRefPartition;
    const uint64_t target = static_cast<uint64_t>(ctx->num_cus) * kWaves * (elem_bytes >= 4 ? 1 : 4);
    const uint32_t half_ctx = std::max(capacity / 2, 1u);
    while (P > 64 && static_cast<uint64_t>(seqs) * kv_heads * ((half_ctx + P - 1) / P) < target) P /= 2;
    while (P > 32 && P > 62u * block_size) P /= 2;
    return P;
}

// Launch geometry shared by run_ragged and the host partition helper.
bool pool_fits_rsrc(const kanso_ragged_attention_params* p) {
    const uint64_t elem = p->kv_dtype == KANSO_KV_F32 ? 4 : 1;
    const uint64_t rows = static_cast<uint64_t>(p->num_blocks) * p->block_size * p->num_kv_heads;
    return p->num_blocks != 0 && rows * p->head_dim * elem < (1ull << 32);
}

// Whether a batch takes the kernel with the MFMA chunk path: some sequence has more
// than one query row, head_dim 64, GQA groups up to 4, the pool within buffer range.
bool use_mfma_path(const kanso_ragged_attention_params* p, uint32_t max_q) {
    const uint32_t G = p->num_heads / p->num_kv_heads;
    return p->head_dim == 64 && G <= 4 && max_q > 1 && pool_fits_rsrc(p);
}

// Chunk items are 64 rows wide: their partition stays long (at least 512 keys, within
// 62 table entries), so small decode partitions do not multiply them.
uint32_t chunk_partition(uint32_t P, uint32_t block_size) {
    return std::max(P, std::min(512u, 62u * block_size / 32u * 32u));
}

// One persistent launch: two workgroups (eight waves) per CU, plus half a CU's worth
// for batches with chunk items (chunk workgroups hold their slots only briefly; the
// extra decode workgroups are dispatched into the slots they free).
uint32_t main_grid(const kanso_ctx* ctx, uint64_t T, uint32_t max_parts, uint32_t HKV, bool mfma) {
    const uint64_t max_waves = (T * max_parts * HKV + kWaves - 1) / kWaves;
    uint32_t grid = static_cast<uint32_t>(std::max<uint64_t>(
        1, std::min<uint64_t>(std::max<uint64_t>(max_waves, mfma ? ctx->num_cus : 1),
                              static_cast<uint64_t>(ctx->num_cus) * 2)));
    if (mfma) grid += ctx->num_cus / 2;
    return grid;
}

uint32_t host_row_limit(uint32_t ctx_len, uint32_t q_len, uint32_t i, uint32_t cap) {
    const int64_t lim = static_cast<int64_t>(ctx_len) - q_len + i + 1;
    return static_cast<uint32_t>(std::min<int64_t>(std::max<int64_t>(lim, 0), cap));
}

// fixed_scratch: the device address of the fixed scratch array (no allocation, no
// profiling events); null: the context's grow-only scratch.
int run_ragged(kanso_ctx* ctx, const kanso_ragged_attention_params* p, const float* q,
               const void* kp, const void* vp, const void* ks, const void* vs,
               const uint32_t* tables, const int32_t* cu, const uint32_t* ctx_lens, float* out,
               hipStream_t stream, const char* who, bool out_tiled = false, void* fixed_scratch = nullptr,
               const uint32_t* work = nullptr, uint32_t n_work = 0, uint32_t n_work_chunk = 0) {
    const uint32_t S = p->num_seqs, H = p->num_heads, HKV = p->num_kv_heads, D = p->head_dim;
    const bool one_row_each = p->total_q == S && p->max_q_len == 1;
    if (!q || !kp || !vp || !tables || (!cu && !one_row_each) || !ctx_lens || !out) {
        set_error("%s: null buffer", who);
        return KANSO_E_INVALID_ARG;
    }
    if (S > kMaxSeqs) {
        set_error("%s: %u sequences exceed the per-call limit %u", who, S, kMaxSeqs);
        return KANSO_E_INVALID_SHAPE;
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
    if (p->kv_dtype > KANSO_KV_FP8) {
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
    const auto bad_partition = [&](uint32_t v) {
        return v && (v < 32 || v > 992 || v % 32 != 0 || v > 62u * p->block_size);
    };
    if (bad_partition(p->partition_size) || bad_partition(p->chunk_partition_size)) {
        set_error("%s: partition_size %u / chunk_partition_size %u must be 0 or a multiple of 32 in "
                  "[32, min(992, 62 * block_size)]",
                  who, p->partition_size, p->chunk_partition_size);
        return KANSO_E_INVALID_SHAPE;
    }
    const uint32_t P = p->partition_size ? p->partition_size
                                         : choose_partition(ctx, S, HKV, capacity, p->block_size,
                                                            p->kv_dtype == KANSO_KV_F32 ? 4 : 1);
    const uint32_t CP = p->chunk_partition_size ? p->chunk_partition_size : chunk_partition(P, p->block_size);
    // partials are indexed by partition: the shorter of the two partitions sets the count
    const uint32_t max_parts = (capacity + std::min(P, CP) - 1) / std::min(P, CP);
    const uint64_t partial_elems = static_cast<uint64_t>(T) * H * max_parts * D;
    if (partial_elems > (1ull << 31)) {
        set_error("%s: %llu partial elements exceed the scratch limit", who,
                  static_cast<unsigned long long>(partial_elems));
        return KANSO_E_INVALID_SHAPE;
    }

    // Scratch: [stats T*H*max_parts float2][partials T*H*max_parts*D f32].
    const size_t off_stats = 0;
    const size_t off_part = align_up(static_cast<size_t>(T) * H * max_parts * sizeof(float2), 256);
    const size_t off_np = align_up(off_part + partial_elems * sizeof(float), 256);
    const size_t total = off_np + static_cast<size_t>(T) * sizeof(uint32_t);
    int rc = KANSO_OK;
    char* base = nullptr;
    if (fixed_scratch) {
        if (total > kNoAllocScratchBytes) {
            set_error("%s: this call needs %zu bytes of split-K scratch, above the fixed %zu (fewer rows or "
                      "partitions, or the allocating entry point)",
                      who, total, kNoAllocScratchBytes);
            return KANSO_E_INVALID_SHAPE;
        }
        base = static_cast<char*>(fixed_scratch);
    } else {
        if ((rc = ensure_scratch(ctx, total))) return rc;
        base = static_cast<char*>(ctx->scratch);
    }
    const bool prof = fixed_scratch == nullptr;  // profiling events come from a pool that grows

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
    a.row_np = reinterpret_cast<uint32_t*>(base + off_np);
    a.out = out;
    a.out_nbk = out_tiled ? H * D / 32 : 0u;
    a.work = nullptr;
    a.n_work = 0;
    a.n_work_chunk = 0;
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
    a.chunk_part = CP;
    a.max_parts = max_parts;
    a.total_q = T;
    a.capacity = capacity;
    a.scale_log2 = p->scale * kLog2e;

    // Buffer-resource loads need the pool size and every pool tensor below 4 GiB.
    const uint64_t elem = p->kv_dtype == KANSO_KV_F32 ? 4 : 1;
    const uint64_t rows = static_cast<uint64_t>(p->num_blocks) * p->block_size * HKV;
    const uint64_t pool_bytes = rows * D * elem;
    const uint64_t scale_bytes = p->kv_dtype == KANSO_KV_INT8 || p->kv_dtype == KANSO_KV_FP8 ? rows * 4
                                 : p->kv_dtype == KANSO_KV_Q8_0 ? rows * (D / 32) * 2 : 0;
    const bool buf = pool_fits_rsrc(p);
    a.pool_bytes = buf ? static_cast<uint32_t>(pool_bytes) : 0u;
    a.scale_bytes = buf ? static_cast<uint32_t>(scale_bytes) : 0u;
    // MFMA chunk items exist only when some sequence has more than one query row; the
    // chunk kernel reads the pool through buffer resources (pool below 4 GiB).
    const uint32_t max_q = p->max_q_len ? p->max_q_len : T;
    a.use_mfma = use_mfma_path(p, max_q) ? 1u : 0u;
    a.head_major = p->pool_layout == KANSO_POOL_HEAD_MAJOR ? 1u : 0u;
    Stage1Fn main_fn = pick_main_kv(p->kv_dtype, D, G, buf, a.use_mfma != 0);
    if (work) {
        // the work-list path (kanso_ragged_build_work): decode rows from the list,
        // MFMA chunk rows (if any) from the sequence tables
        if (!ragged_work_supported(p) || n_work + n_work_chunk == 0 || (n_work_chunk && !a.use_mfma) ||
            CP > kWorkBlocks * p->block_size) {
            set_error("%s: work list given for a batch it cannot serve", who);
            return KANSO_E_INVALID_ARG;
        }
        a.work = work;
        a.n_work = n_work;
        a.n_work_chunk = n_work_chunk;
    }
    const bool wide_merge = max_parts > 16;
    Stage1Fn reduce = pick_reduce(D, wide_merge);
    if (!main_fn || !reduce) {
        set_error("%s: no kernel for head_dim %u / kv_dtype %u", who, D, p->kv_dtype);
        return KANSO_E_INVALID_SHAPE;
    }

    // nothing in the grid depends on device data
    hipEvent_t ev = nullptr;
    const uint32_t grid = main_grid(ctx, T, max_parts, HKV, a.use_mfma != 0);
    if (prof && (rc = prof_begin(ctx, "attention", stream, &ev))) return rc;
    hipLaunchKernelGGL(main_fn, dim3(grid), dim3(kThreads), 0, stream, a);
    KANSO_LAUNCH_CHECK();
    if (prof && (rc = prof_end(ctx, "attention", stream, ev))) return rc;
    const uint64_t merges_per_wg = wide_merge ? kWaves : kThreads / std::max<uint32_t>(16, std::min<uint32_t>(D / 4, kWave));
    const uint32_t rgrid = static_cast<uint32_t>(std::max<uint64_t>(
        1, std::min<uint64_t>((static_cast<uint64_t>(T) * H + merges_per_wg - 1) / merges_per_wg, ctx->num_cus * 8)));
    if (prof && (rc = prof_begin(ctx, "reduce", stream, &ev))) return rc;
    hipLaunchKernelGGL(reduce, dim3(rgrid), dim3(kThreads), 0, stream, a);
    KANSO_LAUNCH_CHECK();
    return prof ? prof_end(ctx, "reduce", stream, ev) : KANSO_OK;
}

}  // namespace

bool ragged_work_supported(const kanso_ragged_attention_params* p) {
    return p->kv_dtype != KANSO_KV_FP8 && p->partition_size != 0 && p->partition_size % 32 == 0 &&
           p->partition_size <= std::min(992u, kWorkBlocks * p->block_size) && p->block_size != 0 &&
           pool_fits_rsrc(p) && p->pool_layout == KANSO_POOL_TOKEN_MAJOR && p->num_kv_heads != 0 &&
           p->num_heads % p->num_kv_heads == 0;
}

// The work list of a batch: decode items (every row outside the MFMA chunk path, per
// partition) in row order, then chunk items (each 64-row block of a multi-row
// sequence on the MFMA path, per chunk partition). Returns false when the batch
// cannot take a list (a row without keys, or parameters the list path does not
// serve); fills `work` when given, and the two counts.
bool ragged_work(const kanso_ragged_attention_params* p, const uint32_t* q_lens, const uint32_t* context_lens,
                 const uint32_t* block_tables, uint32_t* work, uint64_t* n_decode, uint64_t* n_chunk) {
    *n_decode = *n_chunk = 0;
    if (!ragged_work_supported(p)) return false;
    const uint32_t S = p->num_seqs, P = p->partition_size, bs = p->block_size;
    const uint64_t cap64 = static_cast<uint64_t>(p->max_num_blocks_per_seq) * bs;
    const uint32_t cap = static_cast<uint32_t>(std::min<uint64_t>(cap64, 0xffffffffu));
    uint64_t T = 0;
    uint32_t max_q = 0;
    for (uint32_t s = 0; s < S; ++s) {
        T += q_lens[s];
        max_q = std::max(max_q, q_lens[s]);
    }
    if (T != p->total_q || T == 0) return false;
    const bool mfma = use_mfma_path(p, p->max_q_len ? p->max_q_len : max_q);
    const uint32_t CP = p->chunk_partition_size ? p->chunk_partition_size : chunk_partition(P, bs);
    if (mfma && CP > kWorkBlocks * bs) return false;
    // the item's block ids: keys [t0, t1) of sequence s
    const auto blocks = [&](uint32_t* w, uint32_t s, uint32_t t0, uint32_t t1) {
        const uint32_t b0 = t0 / bs, nb = (t1 - 1) / bs - b0 + 1;
        const uint32_t* tab = block_tables + static_cast<size_t>(s) * p->max_num_blocks_per_seq;
        for (uint32_t j = 0; j < kWorkBlocks; ++j) w[j] = j < nb ? tab[b0 + j] : 0u;
    };
    uint64_t nd = 0, nc = 0;
    for (int pass = 0; pass < (work ? 2 : 1); ++pass) {
        uint64_t di = 0, ci = 0;  // items written so far of each kind
        uint32_t row = 0;
        for (uint32_t s = 0; s < S; ++s) {
            const uint32_t ql = q_lens[s], c = context_lens[s];
            if (mfma && ql > 1) {
                if (host_row_limit(c, ql, 0, cap) == 0) return false;  // rows without keys: table path
                // partition-major: the row blocks that read the same keys are adjacent
                const uint32_t np_max = (host_row_limit(c, ql, ql - 1, cap) + CP - 1) / CP;
                for (uint32_t part = 0; part < np_max; ++part)
                    for (uint32_t i0 = 0; i0 < ql; i0 += kChunkBlockRows) {
                        const uint32_t nrows = std::min<uint32_t>(kChunkBlockRows, ql - i0);
                        const uint32_t lim_max = host_row_limit(c, ql, i0 + nrows - 1, cap);
                        const uint32_t t0 = part * CP;
                        if (t0 >= lim_max) continue;  // this block's rows end before the partition
                        if (pass == 1) {
                            uint32_t* w = work + (nd + ci) * kWorkWords;
                            blocks(w, s, t0, std::min(t0 + CP, lim_max));
                            w[kWorkBlocks] = row + i0;
                            w[kWorkBlocks + 1] = nrows;
                            w[kWorkBlocks + 2] = c - ql + i0;  // key position of the block's first row
                            w[kWorkBlocks + 3] = part;
                        }
                        ++ci;
                    }
                row += ql;
                continue;
            }
            for (uint32_t i = 0; i < ql; ++i, ++row) {
                const uint32_t limit = host_row_limit(c, ql, i, cap);
                if (limit == 0) return false;
                for (uint32_t t0 = 0; t0 < limit; t0 += P, ++di) {
                    if (pass == 0) continue;
                    uint32_t* w = work + di * kWorkWords;
                    const uint32_t t1 = std::min(t0 + P, limit);
                    blocks(w, s, t0, t1);
                    w[kWorkBlocks] = row;
                    w[kWorkBlocks + 1] = t0;
                    w[kWorkBlocks + 2] = t1;
                    w[kWorkBlocks + 3] = limit;
                }
            }
        }
        nd = di;
        nc = ci;
    }
    *n_decode = nd;
    *n_chunk = nc;
    return nd + nc > 0;
}

int op_ragged_attention(kanso_ctx* ctx, const kanso_ragged_attention_params* p, const float* q, const void* k_pool,
                        const void* v_pool, const void* k_scales, const void* v_scales, const uint32_t* block_tables,
                        const int32_t* cu_seqlens, const uint32_t* context_lens, float* out, hipStream_t s,
                        bool out_tiled, const uint32_t* work, uint32_t n_work, uint32_t n_work_chunk) {
    if (out_tiled && (p->num_heads * p->head_dim) % 32 != 0) {
        set_error("ragged attention: tiled output needs heads x head_dim (%u) to be a multiple of 32",
                  p->num_heads * p->head_dim);
        return KANSO_E_INVALID_SHAPE;
    }
    return run_ragged(ctx, p, q, k_pool, v_pool, k_scales, v_scales, block_tables, cu_seqlens, context_lens, out, s,
                      "ragged attention", out_tiled, nullptr, work, n_work, n_work_chunk);
}

int noalloc_scratch_init(void** ptr) {
    *ptr = nullptr;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
        set_error("kanso_create: no device address for the fixed attention scratch: %s", hipGetErrorString(e));
        return KANSO_E_HIP;
    }
    *ptr = p;
    return KANSO_OK;
}

}  // namespace kanso

using namespace kanso;

extern "C" {

uint32_t kanso_paged_attention_num_partitions(const kanso_paged_attention_params* p) {
    if (!p) return 1;
    const uint64_t capacity = static_cast<uint64_t>(p->max_num_blocks_per_seq) * p->block_size;
    const uint64_t parts = (std::min<uint64_t>(capacity, 0xffffffffu) + kRefPartition - 1) / kRefPartition;
    return static_cast<uint32_t>(std::max<uint64_t>(parts, 1));
}

uint32_t kanso_ragged_partition_size(const kanso_ctx* ctx, const kanso_ragged_attention_params* p,
                                     const uint32_t* q_lens, const uint32_t* context_lens) {
    // The smallest partition (a multiple of 32) whose decode items (row x KV head x
    // partition) all get a resident wave of their own in one pass: shorter items
    // finish sooner, while items beyond the resident waves would run in a second
    // round. Chunk items (64 rows, their own partition of at least 512) hold one
    // resident workgroup each; a partition that gives them every one is not taken.
    // Measured on the benchmark batches: the optimum of a sweep over multiples of 32
    // is where the decode items just fit (config 2: 448; 48 decodes alone: 320;
    // config 1: 32; config 3: 160-192).
    if (!ctx || !p || !q_lens || !context_lens || p->num_seqs == 0 || p->num_kv_heads == 0 ||
        p->num_heads % p->num_kv_heads != 0 || p->block_size == 0)
        return 0;
    const uint32_t S = p->num_seqs, HKV = p->num_kv_heads;
    const uint64_t cap64 = static_cast<uint64_t>(p->max_num_blocks_per_seq) * p->block_size;
    const uint32_t cap = static_cast<uint32_t>(std::min<uint64_t>(cap64, 1u << 30));
    uint64_t T = 0;
    uint32_t max_q = 0;
    for (uint32_t s = 0; s < S; ++s) {
        T += q_lens[s];
        max_q = std::max(max_q, q_lens[s]);
    }
    if (T == 0 || cap == 0) return 0;
    const bool mfma = use_mfma_path(p, max_q);
    const uint32_t p_max = std::max(32u, std::min(512u, 62u * p->block_size / 32u * 32u));
    uint32_t best = p_max;
    for (uint32_t P = p_max; P >= 32; P -= 32) {
        const uint32_t cp = chunk_partition(P, p->block_size);
        uint64_t n_chunk = 0, items = 0;
        for (uint32_t s = 0; s < S; ++s) {
            const uint32_t ql = q_lens[s], c = context_lens[s];
            if (mfma && ql > 1) {
                for (uint32_t i0 = 0; i0 < ql; i0 += 64)
                    n_chunk += (host_row_limit(c, ql, std::min(i0 + 64, ql) - 1, cap) + cp - 1) / cp * HKV;
            } else {
                for (uint32_t i = 0; i < ql; ++i) items += (host_row_limit(c, ql, i, cap) + P - 1) / P * HKV;
            }
        }
        // resident: two workgroups per CU (the kernel's register budget); chunk
        // workgroups hold some of them, the extra workgroups of the grid wait
        const uint64_t resident = std::min<uint64_t>(main_grid(ctx, T, (cap + P - 1) / P, HKV, mfma),
                                                     2ull * ctx->num_cus);
        if (n_chunk >= resident) break;
        if (items > (resident - n_chunk) * kWaves) break;
        best = P;
    }
    return best;
}

uint32_t kanso_ragged_chunk_partition_size(const kanso_ctx* ctx, const kanso_ragged_attention_params* p,
                                           const uint32_t* q_lens, const uint32_t* context_lens) {
    // Only batches without decode rows shorten their chunk partitions: the chunk
    // items then have the machine to themselves, and an item's tiles run one after
    // another (latency-bound), so more, shorter items finish sooner. Measured on
    // config 2's four prefill chunks alone: 44.9 us at 512 keys, 28.8 at 96-128.
    if (!ctx || !p || !q_lens || !context_lens || p->num_seqs == 0 || p->num_kv_heads == 0 ||
        p->num_heads % p->num_kv_heads != 0 || p->block_size == 0)
        return 0;
    const uint32_t S = p->num_seqs, HKV = p->num_kv_heads;
    const uint64_t cap64 = static_cast<uint64_t>(p->max_num_blocks_per_seq) * p->block_size;
    const uint32_t cap = static_cast<uint32_t>(std::min<uint64_t>(cap64, 1u << 30));
    uint64_t T = 0;
    uint32_t max_q = 0;
    for (uint32_t s = 0; s < S; ++s) {
        if (q_lens[s] == 1) return 0;
        T += q_lens[s];
        max_q = std::max(max_q, q_lens[s]);
    }
    if (T == 0 || cap == 0 || !use_mfma_path(p, max_q)) return 0;
    const uint32_t p_max = std::max(32u, std::min(512u, 62u * p->block_size / 32u * 32u));
    for (uint32_t cp = std::min(64u, p_max); cp <= p_max; cp += 32) {
        // the launch's grid for this partition (its partial count sizes it), at most
        // two workgroups per CU resident
        const uint64_t resident =
            std::min<uint64_t>(main_grid(ctx, T, (cap + cp - 1) / cp, HKV, true), 2ull * ctx->num_cus);
        uint64_t n_chunk = 0;
        for (uint32_t s = 0; s < S; ++s) {
            const uint32_t ql = q_lens[s], c = context_lens[s];
            for (uint32_t i0 = 0; i0 < ql; i0 += 64)
                n_chunk += (host_row_limit(c, ql, std::min(i0 + 64, ql) - 1, cap) + cp - 1) / cp * HKV;
        }
        if (n_chunk <= resident) return cp;
    }
    return p_max;
}

uint32_t kanso_ragged_work_items(const kanso_ragged_attention_params* p, const uint32_t* q_lens,
                                 const uint32_t* context_lens, uint32_t* n_chunk_items) {
    if (n_chunk_items) *n_chunk_items = 0;
    if (!p || !q_lens || !context_lens || p->num_seqs == 0) return 0;
    uint64_t nd = 0, nc = 0;
    if (!ragged_work(p, q_lens, context_lens, nullptr, nullptr, &nd, &nc) || nd + nc > 0xffffffffu) return 0;
    if (n_chunk_items) *n_chunk_items = static_cast<uint32_t>(nc);
    return static_cast<uint32_t>(nd + nc);
}

int kanso_ragged_build_work(const kanso_ragged_attention_params* p, const uint32_t* q_lens,
                            const uint32_t* context_lens, const uint32_t* block_tables, uint32_t* work,
                            uint32_t n_items) {
    if (!p || !q_lens || !context_lens || !block_tables || !work || p->num_seqs == 0) {
        set_error("kanso_ragged_build_work: null argument");
        return KANSO_E_INVALID_ARG;
    }
    uint64_t nd = 0, nc = 0;
    if (!ragged_work(p, q_lens, context_lens, nullptr, nullptr, &nd, &nc) || nd + nc != n_items) {
        set_error("kanso_ragged_build_work: the batch has %llu work items, the buffer %u",
                  static_cast<unsigned long long>(nd + nc), n_items);
        return KANSO_E_INVALID_SHAPE;
    }
    ragged_work(p, q_lens, context_lens, block_tables, work, &nd, &nc);
    return KANSO_OK;
}

int kanso_ragged_paged_attention_work(kanso_ctx* ctx, const kanso_ragged_attention_params* p, const float* q,
                                      const void* k_pool, const void* v_pool, const void* k_scales,
                                      const void* v_scales, const uint32_t* block_tables,
                                      const int32_t* cu_seqlens, const uint32_t* context_lens, float* out,
                                      const uint32_t* work, uint32_t n_items, uint32_t n_chunk_items,
                                      kanso_stream_t stream) {
    if (!ctx) {
        set_error("kanso_ragged_paged_attention_work: null context");
        return KANSO_E_INVALID_ARG;
    }
    if (!work || n_items == 0 || n_chunk_items > n_items) {
        set_error("kanso_ragged_paged_attention_work: empty work list or %u chunk items of %u", n_chunk_items,
                  n_items);
        return KANSO_E_INVALID_ARG;
    }
    return run_ragged(ctx, p, q, k_pool, v_pool, k_scales, v_scales, block_tables, cu_seqlens, context_lens, out,
                      as_stream(stream), "kanso_ragged_paged_attention_work", false, nullptr, work,
                      n_items - n_chunk_items, n_chunk_items);
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
    // One query row per sequence: the kernel reads a null cu_seqlens as 0..=num_seqs
    // (no extra launch to write it).
    kanso_ragged_attention_params rp{};
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
    rp.pool_layout = KANSO_POOL_TOKEN_MAJOR;
    return run_ragged(ctx, &rp, q, k_cache, v_cache, nullptr, nullptr, block_tables, nullptr,
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

int kanso_ragged_paged_attention_noalloc(kanso_ctx* ctx, const kanso_ragged_attention_params* p, const float* q,
                                         const void* k_pool, const void* v_pool, const void* k_scales,
                                         const void* v_scales, const uint32_t* block_tables,
                                         const int32_t* cu_seqlens, const uint32_t* context_lens, float* out,
                                         kanso_stream_t stream) {
    if (!ctx || !p) {
        set_error("kanso_ragged_paged_attention_noalloc: null context or params");
        return KANSO_E_INVALID_ARG;
    }
    if (!ctx->noalloc_scratch) {
        set_error("kanso_ragged_paged_attention_noalloc: context has no fixed scratch");
        return KANSO_E_INVALID_ARG;
    }
    return run_ragged(ctx, p, q, k_pool, v_pool, k_scales, v_scales, block_tables, cu_seqlens, context_lens, out,
                      as_stream(stream), "kanso_ragged_paged_attention_noalloc", false, ctx->noalloc_scratch);
}

}  // extern "C"
