// pack.hip — scheduler-to-device packing of one step.
//
// Reference: the host loop of Engine::step (src/engine.rs:376-402), which walks the
// planned sequences in plan order (decodes first, then prefill chunks) and builds
// tokens / positions / slot_mapping / block_tables / context_lens / query_lens, and
// PaddedDecodeTables::new (src/model.rs:71-111), which pads every table to the
// batch's widest by repeating the last block the sequence needs.
//
// Here the host ships only the compact plan (kanso_seq_plan per sequence) and the
// device builds the flat arrays. Every workgroup redundantly scans the S query
// lengths into LDS (S is at most a few thousand), then takes a grid-stride share of
// the T query rows and of the S x max_blocks table entries. All outputs are
// integer copies, so they are bit-exact by construction.
#include "common.hpp"

namespace kanso {
namespace {

constexpr int kPackThreads = 1024;
constexpr uint32_t kMaxPackSeqs = 8192;

__global__ __launch_bounds__(kPackThreads) void pack_step_kernel(
    const kanso_seq_plan* __restrict__ plan, uint32_t S, const uint32_t* __restrict__ token_arena,
    const uint32_t* __restrict__ table_arena, uint32_t bs, uint32_t max_blocks, uint32_t T,
    kanso_packed_step out, uint32_t* status) {
    __shared__ int32_t cu[kMaxPackSeqs + 1];
    __shared__ int32_t part[kPackThreads];
    const uint32_t tid = threadIdx.x;
    // Block-wide exclusive scan of q_len: contiguous ranges per thread, then a
    // Hillis-Steele scan of the per-thread sums.
    const uint32_t per = (S + kPackThreads - 1) / kPackThreads;
    const uint32_t s0 = min(tid * per, S), s1 = min(s0 + per, S);
    int32_t local = 0;
    for (uint32_t s = s0; s < s1; ++s) local += static_cast<int32_t>(plan[s].q_len);
    part[tid] = local;
    __syncthreads();
    for (uint32_t off = 1; off < kPackThreads; off <<= 1) {
        const int32_t v = tid >= off ? part[tid - off] : 0;
        __syncthreads();
        part[tid] += v;
        __syncthreads();
    }
    int32_t run = part[tid] - local;
    for (uint32_t s = s0; s < s1; ++s) {
        cu[s] = run;
        run += static_cast<int32_t>(plan[s].q_len);
    }
    if (tid == kPackThreads - 1) cu[S] = part[tid];
    __syncthreads();

    const uint32_t stride = gridDim.x * kPackThreads;
    const uint32_t gtid = blockIdx.x * kPackThreads + tid;
    if (blockIdx.x == 0) {
        for (uint32_t s = tid; s <= S; s += kPackThreads) out.cu_seqlens[s] = cu[s];
    }
    // Per-sequence scalars and padded tables.
    for (uint32_t s = gtid; s < S; s += stride) out.context_lens[s] = plan[s].start_pos + plan[s].q_len;
    uint32_t flags = 0;
    const uint32_t n_tab = S * max_blocks;
    for (uint32_t e = gtid; e < n_tab; e += stride) {
        const uint32_t s = e / max_blocks, b = e % max_blocks;
        const kanso_seq_plan pl = plan[s];
        const uint32_t ctx = pl.start_pos + pl.q_len;
        const uint32_t needed = max((ctx + bs - 1) / bs, 1u);
        uint32_t idx = min(b, needed - 1);
        if (pl.table_len < needed) {  // src/model.rs:92-100
            flags |= KANSO_DEV_TABLE_SHORT;
            idx = pl.table_len ? min(idx, pl.table_len - 1) : 0;
        }
        out.block_tables[e] = pl.table_len ? table_arena[pl.table_offset + idx] : 0u;
    }
    // Per-query rows, in plan order.
    for (uint32_t n = gtid; n < T; n += stride) {
        uint32_t lo = 0, hi = S;  // last s with cu[s] <= n
        while (hi - lo > 1) {
            const uint32_t mid = (lo + hi) / 2;
            if (static_cast<uint32_t>(cu[mid]) <= n) lo = mid;
            else hi = mid;
        }
        const kanso_seq_plan pl = plan[lo];
        const uint32_t pos = pl.start_pos + (n - static_cast<uint32_t>(cu[lo]));
        const uint32_t blk_idx = pos / bs;
        out.tokens[n] = token_arena[pl.token_offset + pos];
        out.positions[n] = static_cast<int32_t>(pos);
        out.seq_of_query[n] = static_cast<int32_t>(lo);
        if (blk_idx < pl.table_len) {
            out.slot_mapping[n] = static_cast<int64_t>(table_arena[pl.table_offset + blk_idx]) * bs + pos % bs;
        } else {  // src/engine.rs:387-394
            flags |= KANSO_DEV_TABLE_SHORT;
            out.slot_mapping[n] = -1;
        }
    }
    if (flags) raise_status(status, flags);
}

}  // namespace
}  // namespace kanso

using namespace kanso;

extern "C" int kanso_pack_step(kanso_ctx* ctx, const kanso_seq_plan* plan, uint32_t num_seqs,
                               const uint32_t* token_arena, const uint32_t* table_arena,
                               uint32_t block_size, uint32_t max_blocks, uint32_t total_q,
                               const kanso_packed_step* out, kanso_stream_t stream) {
    if (!ctx || !plan || !token_arena || !table_arena || !out) {
        set_error("kanso_pack_step: null argument");
        return KANSO_E_INVALID_ARG;
    }
    if (!out->cu_seqlens || !out->seq_of_query || !out->positions || !out->slot_mapping ||
        !out->tokens || !out->block_tables || !out->context_lens) {
        set_error("kanso_pack_step: null output buffer");
        return KANSO_E_INVALID_ARG;
    }
    if (num_seqs == 0 || num_seqs > kMaxPackSeqs) {
        set_error("kanso_pack_step: num_seqs %u outside 1..=%u", num_seqs, kMaxPackSeqs);
        return KANSO_E_INVALID_SHAPE;
    }
    if (block_size == 0 || max_blocks == 0 || total_q == 0) {
        set_error("kanso_pack_step: block_size %u, max_blocks %u, total_q %u must be non-zero",
                  block_size, max_blocks, total_q);
        return KANSO_E_INVALID_SHAPE;
    }
    hipStream_t s = as_stream(stream);
    const uint64_t work = std::max<uint64_t>(total_q, static_cast<uint64_t>(num_seqs) * max_blocks);
    const uint32_t grid = static_cast<uint32_t>(std::min<uint64_t>((work + kPackThreads - 1) / kPackThreads, 64));
    hipEvent_t ev;
    int rc = prof_begin(ctx, "pack", s, &ev);
    if (rc) return rc;
    hipLaunchKernelGGL(pack_step_kernel, dim3(grid), dim3(kPackThreads), 0, s, plan, num_seqs,
                       token_arena, table_arena, block_size, max_blocks, total_q, *out, ctx->status);
    KANSO_LAUNCH_CHECK();
    return prof_end(ctx, "pack", s, ev);
}
