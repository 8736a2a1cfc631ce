// q8_gemm.hpp — dequant-on-the-fly Q8_0 (and Q4_K) matrix products on the bf16
// matrix cores, with the fused prologues / epilogues the decoder layer needs.
//
// Arithmetic. Y[t][r] = sum_b d[r][b] * sum_{i<32} q[r][32b+i] * x[t][32b+i]
// (scalar_gemv_q8_0, src/quant/q8_0.rs:51-93). One v_mfma_f32_16x16x32_bf16 has
// K = 32, exactly one Q8_0 block, so the per-block scale is applied to the MFMA
// result before it joins the f32 accumulator — the reference's own order. The
// int8 weights are exact in bf16; x is split into bf16 hi + lo (x - hi is exact in
// f32), so sum q*x = MFMA(hi, q) + MFMA(lo, q) leaves only the ~2^-17 relative
// residue of the split. Results do not depend on the batch size: a token's
// output is computed in the same order whatever else is in the batch.
//
// Operand layouts (16x16x32 bf16): lane l holds A[m = l%16][k = 8(l/16) .. +7]
// (x of token m), B[k = 8(l/16) .. +7][n = l%16] (weights of row n), and the
// accumulator C[m = 4(l/16) + r][n = l%16], r = 0..3. So a lane's output row is
// the row whose weights it loaded, and the block scale is a per-lane scalar.
//
// Work mapping. Output rows come in pairs of 16-row weight groups (32 rows,
// chosen by the epilogue); a workgroup owns one pair and 16, 32 or 64 tokens and
// splits K over its waves (see q8_gemm_kernel).
//
// Weight layouts:
//   GGUF   : [rows][in/32] blocks {f16 d; i8 qs[32]} (34 B), the format the
//            reference reads (src/quant/mod.rs:1-17);
//   Q4_K   : GGUF block_q4_K rows (WQ4K: one 32-element sub-block per k-block, an
//            affine block d q - m, the m term from a product against ones);
//   packed : [groups][in/32] tiles of 544 B, one per (16-row group, block):
//            qs[kq][row][8] (512 B: lane l's 8 bytes are at 8l) then d[16] f16.
//            Rows past the matrix are zero. Produced by kanso_q8_0_pack; the
//            bytes are the GGUF bytes, re-laid so a wave's operand is one
//            coalesced 512 B load.
#pragma once

#include <atomic>
#include <type_traits>

#include "common.hpp"

namespace kanso {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr uint32_t kPackedTileBytes = 544;  // 16 rows x (32 qs + 2 d)

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) { return __half2float(__ushort_as_half(h)); }

// 8 int8 (little-endian in q) -> 8 bf16 (exact: |q| <= 128 needs 8 bits). Each
// byte converts to f32 (sign-extended byte select); one byte permute then takes
// the upper halves of two floats, which are their bf16 values (exact, no rounding).
__device__ __forceinline__ bf16x8 i8x8_to_bf16(uint64_t q) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float f0 = static_cast<float>(static_cast<int8_t>((q >> (16 * i)) & 0xff));
        const float f1 = static_cast<float>(static_cast<int8_t>((q >> (16 * i + 8)) & 0xff));
        // bytes 2,3 of f0 -> 0,1 and bytes 2,3 of f1 -> 2,3
        w[i] = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, f1), __builtin_bit_cast(uint32_t, f0), 0x07060302u);
    }
    return __builtin_bit_cast(bf16x8, w);
}

__device__ __forceinline__ bf16x8 bf16_ones() {
    const uint32_t one2 = 0x3f803f80u;  // two bf16 1.0
    const uint32_t w[4] = {one2, one2, one2, one2};
    return __builtin_bit_cast(bf16x8, w);
}

struct Bf16Pair {
    bf16x8 hi, lo;
};

__device__ __forceinline__ Bf16Pair split_bf16(const float (&x)[8]) {
    Bf16Pair r;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const __bf16 h = static_cast<__bf16>(x[j]);
        r.hi[j] = h;
        r.lo[j] = static_cast<__bf16>(x[j] - static_cast<float>(h));
    }
    return r;
}

// ---------------------------------------------------------------- weight loaders

// A loader splits into load() (raw bytes only: every load of a round is issued
// before any of them is used) and decode() (after the round's loads are in
// flight). Converting the f16 scale inside load() made the compiler wait for each
// block's loads before issuing the next block's, one memory round trip per block.
struct RawQ8 {
    uint64_t q;
    uint32_t d;  // f16 bits
};

// at(g, lane) resolves a lane's row of 16-row group g once per kernel; load()
// then adds a 32-bit block offset (the 64-bit address arithmetic per block cost
// more instructions than the conversion of the block's weights).
struct WPacked {
    const uint8_t* w;
    uint32_t nb;  // in / 32
    static constexpr bool kHasMin = false;
    using Raw = RawQ8;
    struct Ptr {
        const uint8_t* q;  // lane's 8 bytes of block 0
        const uint8_t* d;  // lane's row scale of block 0
    };
    __device__ __forceinline__ Ptr at(uint32_t g, int lane) const {
        const uint8_t* t = w + static_cast<size_t>(g) * nb * kPackedTileBytes;
        return {t + 8 * lane, t + 512 + 2 * (lane & 15)};
    }
    __device__ __forceinline__ void load(const Ptr& p, uint32_t b, Raw& r) const {
        const uint32_t off = b * kPackedTileBytes;
        r.q = *reinterpret_cast<const uint64_t*>(p.q + off);
        r.d = *reinterpret_cast<const uint16_t*>(p.d + off);
    }
    __device__ __forceinline__ void decode(const Raw& r, uint32_t, uint64_t& q, float& d, float& m) const {
        q = r.q;
        d = f16_bits_to_f32(static_cast<uint16_t>(r.d));
        m = 0.f;
    }
};

struct WGguf {
    const uint8_t* w;
    uint32_t nb;
    uint32_t rows;
    static constexpr bool kHasMin = false;
    using Raw = RawQ8;
    struct Ptr {
        const uint8_t* blk;  // the lane's row, block 0
        uint32_t kq;         // byte offset of the lane's 8 quants in a block
    };
    __device__ __forceinline__ Ptr at(uint32_t g, int lane) const {
        // rows past the matrix read row 0 and are zeroed in decode()
        uint32_t row = g * 16 + (lane & 15);
        row = row < rows ? row : 0;
        return {w + static_cast<size_t>(row) * nb * 34, 2u + 8u * static_cast<uint32_t>(lane >> 4)};
    }
    __device__ __forceinline__ void load(const Ptr& p, uint32_t b, Raw& r) const {
        // Blocks are 34 B, so qs is only 2-byte aligned; gfx950 serves an unaligned
        // 8-byte global load as one instruction (global_load_dwordx2).
        const uint8_t* blk = p.blk + b * 34;
        r.d = *reinterpret_cast<const uint16_t*>(blk);
        __builtin_memcpy(&r.q, __builtin_assume_aligned(blk + p.kq, 2), 8);
    }
    __device__ __forceinline__ void decode(const Raw& r, uint32_t row, uint64_t& q, float& d, float& m) const {
        const bool ok = row < rows;
        q = ok ? r.q : 0;
        d = ok ? f16_bits_to_f32(static_cast<uint16_t>(r.d)) : 0.f;
        m = 0.f;
    }
};

// GGUF block_q4_K rows ([rows][in/256] x 144 B: f16 d, f16 dmin, 12 packed 6-bit
// scale/min bytes, 128 nibble bytes). k-block b is 32-element sub-block b % 8 of
// super-block b / 8: weights d * sc * q - dmin * m (BlockQ4_K::dequantize,
// src/quant/q4_k.rs:30-55, with get_scale_min_k4, :16-26). Sub-blocks 2j and 2j+1
// share the 32 bytes qs[32j ..): low nibbles for 2j, high for 2j+1.
struct WQ4K {
    static constexpr bool kHasMin = true;
    const uint8_t* w;
    uint32_t nsb;  // in / 256
    uint32_t rows;
    struct Raw {
        uint64_t q;
        uint32_t dd, s0, s1, s2;
        uint32_t sub;
    };
    struct Ptr {
        const uint8_t* row;  // the lane's row
        uint32_t kq;         // byte offset of the lane's 8 bytes in a 32-byte qs slice
    };
    __device__ __forceinline__ Ptr at(uint32_t g, int lane) const {
        uint32_t row = g * 16 + (lane & 15);
        row = row < rows ? row : 0;
        return {w + static_cast<size_t>(row) * nsb * 144, 8u * static_cast<uint32_t>(lane >> 4)};
    }
    __device__ __forceinline__ void load(const Ptr& p, uint32_t b, Raw& r) const {
        const uint8_t* blk = p.row + (b / 8) * 144;
        r.sub = b % 8;
        r.dd = *reinterpret_cast<const uint32_t*>(blk);
        r.s0 = *reinterpret_cast<const uint32_t*>(blk + 4);
        r.s1 = *reinterpret_cast<const uint32_t*>(blk + 8);
        r.s2 = *reinterpret_cast<const uint32_t*>(blk + 12);
        r.q = *reinterpret_cast<const uint64_t*>(blk + 16 + 32 * (r.sub / 2) + p.kq);
    }
    __device__ __forceinline__ void decode(const Raw& r, uint32_t row, uint64_t& q, float& d, float& m) const {
        const uint32_t sub = r.sub;
        const auto byte = [&](uint32_t i) -> uint32_t {
            const uint32_t word = i < 4 ? r.s0 : (i < 8 ? r.s1 : r.s2);
            return (word >> (8 * (i % 4))) & 0xff;
        };
        uint32_t sc, mn;
        if (sub < 4) {
            sc = byte(sub) & 63;
            mn = byte(sub + 4) & 63;
        } else {
            sc = (byte(sub + 4) & 0xF) | ((byte(sub - 4) >> 6) << 4);
            mn = (byte(sub + 4) >> 4) | ((byte(sub) >> 6) << 4);
        }
        const bool ok = row < rows;
        d = ok ? f16_bits_to_f32(static_cast<uint16_t>(r.dd & 0xffff)) * static_cast<float>(sc) : 0.f;
        m = ok ? f16_bits_to_f32(static_cast<uint16_t>(r.dd >> 16)) * static_cast<float>(mn) : 0.f;
        q = ok ? ((sub & 1) ? ((r.q >> 4) & 0x0f0f0f0f0f0f0f0full) : (r.q & 0x0f0f0f0f0f0f0f0full)) : 0;
    }
};

// ---------------------------------------------------------------- activations

// x rows: token m reads row (rows ? rows[m] : m) of a [*, ldx] f32 matrix, or, with
// tiled set, of the tiled activation order (act_tile_off, K = in). With norm_w set,
// the row is RMS-normalised first: x / sqrt(mean(x^2) + eps) * w
// (Model::rmsnorm, src/model.rs:653-659).
struct XIn {
    const float* x;
    const int32_t* rows;
    const float* norm_w;
    float eps;
    uint32_t ldx;
    uint32_t T;
    uint32_t in;
    uint32_t tiled = 0;
    // lane's pointer to columns 8 kq .. of token m, block 0; block b adds b *
    // bstride(), the second half of the 8 columns hoff()
    __device__ __forceinline__ const float* lane_ptr(uint32_t m, int kq) const {
        const uint32_t r = rows ? static_cast<uint32_t>(rows[m]) : m;
        if (tiled) return x + act_tile_off(r, 8u * kq, in / 32);
        return x + static_cast<size_t>(r) * ldx + 8 * kq;
    }
    __device__ __forceinline__ uint32_t bstride() const { return tiled ? 512u : 32u; }
    __device__ __forceinline__ uint32_t hoff() const { return tiled ? 256u : 4u; }
};

// ---------------------------------------------------------------- the kernel

// Every epilogue provides
//   kGroups: 16-row weight groups per epilogue unit, 2 (a pair) or 1;
//   groups(p, g0, g1): the weight groups of unit p (kGroups = 1: g0 = p);
//   pre(p, lane, m0, T): its own operands for outputs of unit p, tokens m0 .. m0+3,
//     requested before the main loop;
//   apply(p, lane, m0, T, v0, v1, pre): outputs of rows g0*16 + lane%16 (v0) and
//     g1*16 + lane%16 (v1, unused when kGroups = 1) for tokens m0 .. m0+3 (skip
//     m >= T).
//
// A workgroup of KS waves owns NU epilogue units (NG = NU * kGroups weight groups)
// and 16*MT tokens; wave w takes k-blocks w, w + KS, ... and issues the loads of U
// such blocks (weights of every group, x, norm weights) before any arithmetic, so
// a matrix is requested in one or a few rounds: at decode sizes the time is load
// latency, not bandwidth. Each x load feeds the products of all NG groups, so
// wider workgroups (NU > 1) re-read x from L2 less often, at the cost of fewer
// workgroups. The KS partial sums meet in LDS in a fixed order: a token's result
// does not depend on T, MT or NU.
//
// RMSNorm prologue folded into the product: RMSNorm(x) W = (1 / rms) ((x * w) W),
// and the sum of squares of each token row is accumulated from the very x values
// the waves load, so no pass over x precedes the main loop. The division by rms
// happens on the reduced outputs.
//
// The loads of a round are branch-free (a block past the row is replaced by the
// last block, its scale forced to 0; a unit past `units` by the workgroup's first
// unit, never stored): a branch around them would make the compiler wait for each
// block's loads at the join, serialising the round.
// An epilogue with kPairedUnits = true takes the outputs of units u0 and u0 + 1
// (even u0, NU = 2) in one wave: apply_pair(u0, lane, m0, T, v[4], pre) with v[n]
// the rows of weight group g[n] (unit u0: g[0], g[1]; unit u0 + 1: g[2], g[3]), for
// epilogues that need a whole row of outputs at once (a quantized KV row's scale).
template <class E, class = void>
struct PairedUnits : std::false_type {};
template <class E>
struct PairedUnits<E, std::void_t<decltype(E::kPairedUnits)>> : std::bool_constant<E::kPairedUnits> {};

template <int KS, int U, int MT, int NU, bool NORM, class WL, class Epi>
__global__ __launch_bounds__(KS * kWave) void q8_gemm_kernel(WL wl, XIn xa, Epi epi, uint32_t units) {
    constexpr int EG = Epi::kGroups;
    constexpr int NG = NU * EG;
    constexpr bool PU = PairedUnits<Epi>::value;
    static_assert(!PU || (NU == 2 && EG == 2), "paired units: two units of two groups per workgroup");
    constexpr int NC = PU ? MT : MT * NU;  // (token tile, unit) combinations of the epilogue
    static_assert(NG * MT <= 8 && NC <= KS, "partial sums must fit 64 KB of LDS");
    __shared__ floatx4 s_part[KS][NG][MT][kWave];
    __shared__ float s_ss[KS][MT][16];
    // the wave index is uniform: keep it (and every block index) in scalar registers
    const int lane = threadIdx.x & (kWave - 1), wv = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int kq = lane >> 4, mm = lane & 15;
    const uint32_t u0 = blockIdx.x * NU;
    const uint32_t t0 = blockIdx.y * 16 * MT;
    const uint32_t nb = xa.in / 32;
    constexpr bool norm = NORM;
    uint32_t g[NG];
#pragma unroll
    for (int j = 0; j < NU; ++j) {
        uint32_t ga, gb;
        epi.groups(u0 + j < units ? u0 + j : u0, ga, gb);
        g[EG * j] = ga;
        if constexpr (EG == 2) g[EG * j + 1] = gb;
    }
    typename WL::Ptr wp[NG];
#pragma unroll
    for (int n = 0; n < NG; ++n) wp[n] = wl.at(g[n], lane);
    // a lane's x row (tokens past T repeat the tile's first token: their products
    // land in accumulator rows that are never stored) at its k-chunk
    const float* xr[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) {
        const uint32_t m = t0 + 16 * i + mm;
        xr[i] = xa.lane_ptr(m < xa.T ? m : t0, kq);
    }
    const float* nr = NORM ? xa.norm_w + 8 * kq : nullptr;
    const uint32_t xbs = xa.bstride(), xho = xa.hoff();
    // wave c < NC stores combination c = (tile c % MT, unit c / MT); the epilogue's
    // own operands (residual rows, RoPE tables, slots) are requested now, so their
    // latency hides under the main loop
    const int ci = wv % MT, cj = wv / MT;
    const uint32_t cunit = u0 + cj;
    const bool cstore = wv < NC && cunit < units;
    typename Epi::Pre pre{};
    if (cstore) pre = epi.pre(cunit, lane, t0 + 16 * ci + 4 * kq, xa.T);
    floatx4 acc[NG][MT];
    float ss[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) {
#pragma unroll
        for (int n = 0; n < NG; ++n) acc[n][i] = floatx4{0.f, 0.f, 0.f, 0.f};
        ss[i] = 0.f;
    }
    for (uint32_t b0 = wv; b0 < nb; b0 += KS * U) {
        typename WL::Raw raw[NG][U];
        float4 xv[U][MT][2], nv[U][2];
        bool live[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            live[u] = b0 + u * KS < nb;
            const uint32_t b = live[u] ? b0 + u * KS : nb - 1;
#pragma unroll
            for (int n = 0; n < NG; ++n) wl.load(wp[n], b, raw[n][u]);
            const uint32_t k = 32 * b;
#pragma unroll
            for (int i = 0; i < MT; ++i) {
                xv[u][i][0] = *reinterpret_cast<const float4*>(xr[i] + b * xbs);
                xv[u][i][1] = *reinterpret_cast<const float4*>(xr[i] + b * xbs + xho);
            }
            if constexpr (NORM) {
                nv[u][0] = *reinterpret_cast<const float4*>(nr + k);
                nv[u][1] = *reinterpret_cast<const float4*>(nr + k + 4);
            } else {
                nv[u][0] = nv[u][1] = make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
        // keep every load of the round ahead of the arithmetic: the scheduler would
        // otherwise sink later blocks' loads below earlier blocks' products
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            // a repeated block contributes nothing: zero scale and min, no squares
            bf16x8 w[NG];
            float d[NG], mn[NG];
#pragma unroll
            for (int n = 0; n < NG; ++n) {
                uint64_t qb;
                wl.decode(raw[n][u], g[n] * 16 + mm, qb, d[n], mn[n]);
                d[n] = live[u] ? d[n] : 0.f;
                mn[n] = live[u] ? mn[n] : 0.f;
                w[n] = i8x8_to_bf16(qb);
            }
            const float sq = live[u] ? 1.f : 0.f;
            const float nw[8] = {nv[u][0].x, nv[u][0].y, nv[u][0].z, nv[u][0].w,
                                 nv[u][1].x, nv[u][1].y, nv[u][1].z, nv[u][1].w};
#pragma unroll
            for (int i = 0; i < MT; ++i) {
                float xs[8] = {xv[u][i][0].x, xv[u][i][0].y, xv[u][i][0].z, xv[u][i][0].w,
                               xv[u][i][1].x, xv[u][i][1].y, xv[u][i][1].z, xv[u][i][1].w};
                if constexpr (NORM) {
                    float s2 = 0.f;
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        s2 += xs[j] * xs[j];
                        xs[j] *= nw[j];
                    }
                    ss[i] += sq * s2;
                }
                const Bf16Pair a = split_bf16(xs);
                const floatx4 z = {0.f, 0.f, 0.f, 0.f};
                floatx4 sx = z;
                if constexpr (WL::kHasMin) {
                    // block-wise affine weights w = d q - m: sum w x = d (sum q x) - m (sum x);
                    // sum x per token comes out of one more product, against ones, already
                    // in the accumulator layout.
                    sx = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.hi, bf16_ones(), z, 0, 0, 0);
                    sx = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.lo, bf16_ones(), sx, 0, 0, 0);
                }
#pragma unroll
                for (int n = 0; n < NG; ++n) {
                    floatx4 t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.hi, w[n], z, 0, 0, 0);
                    t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.lo, w[n], t, 0, 0, 0);
                    if constexpr (WL::kHasMin)
                        acc[n][i] += d[n] * t - mn[n] * sx;
                    else
                        acc[n][i] += d[n] * t;
                }
            }
        }
    }
#pragma unroll
    for (int i = 0; i < MT; ++i) {
#pragma unroll
        for (int n = 0; n < NG; ++n) s_part[wv][n][i][lane] = acc[n][i];
        if (norm) {
            // the four lanes holding a token's k-chunks: lane ^ 16, lane ^ 32
            float s = ss[i] + wave_xor(ss[i], 16);
            s += wave_xor(s, 32);
            if (kq == 0) s_ss[wv][i][mm] = s;
        }
    }
    __syncthreads();
    if constexpr (PU) {
        if (cstore) {
            floatx4 v[4];
#pragma unroll
            for (int n = 0; n < 4; ++n) {
                v[n] = s_part[0][n][ci][lane];
#pragma unroll
                for (int w = 1; w < KS; ++w) v[n] += s_part[w][n][ci][lane];
            }
            if (norm) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    float s = s_ss[0][ci][4 * kq + r];
#pragma unroll
                    for (int w = 1; w < KS; ++w) s += s_ss[w][ci][4 * kq + r];
                    const float rms = sqrtf(s / static_cast<float>(xa.in) + xa.eps);
#pragma unroll
                    for (int n = 0; n < 4; ++n) v[n][r] /= rms;
                }
            }
            epi.apply_pair(cunit, lane, t0 + 16 * ci + 4 * kq, xa.T, v, pre);
        }
    } else if (cstore) {
        const int ga = EG * cj, gb = EG * cj + EG - 1;
        floatx4 v0 = s_part[0][ga][ci][lane], v1 = {0.f, 0.f, 0.f, 0.f};
        if constexpr (EG == 2) v1 = s_part[0][gb][ci][lane];
#pragma unroll
        for (int w = 1; w < KS; ++w) {
            v0 += s_part[w][ga][ci][lane];
            if constexpr (EG == 2) v1 += s_part[w][gb][ci][lane];
        }
        if (norm) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float s = s_ss[0][ci][4 * kq + r];
#pragma unroll
                for (int w = 1; w < KS; ++w) s += s_ss[w][ci][4 * kq + r];
                const float rms = sqrtf(s / static_cast<float>(xa.in) + xa.eps);
                v0[r] /= rms;
                v1[r] /= rms;
            }
        }
        epi.apply(cunit, lane, t0 + 16 * ci + 4 * kq, xa.T, v0, v1, pre);
    }
}

// ---------------------------------------------------------------- epilogues

// y[m][row] (= or +=) for rows < rows. NG = 2: pair p = groups 2p, 2p+1; NG = 1:
// workgroup p owns group p alone (twice the workgroups, half the bytes each).
// tiled: y is in the tiled activation order with K = rows (a multiple of 32).
template <bool ADD, int NG = 2>
struct EpiStore {
    static constexpr int kGroups = NG;
    float* y;
    uint32_t ldy;
    uint32_t rows;
    uint32_t tiled = 0;
    float scale = 1.f;  // products x scale before the store / add (Granite residual_scale)
    __device__ __forceinline__ size_t at(uint32_t m, uint32_t r) const {
        return tiled ? act_tile_off(m, r, rows / 32) : static_cast<size_t>(m) * ldy + r;
    }
    __device__ __forceinline__ void groups(uint32_t p, uint32_t& g0, uint32_t& g1) const {
        g0 = NG * p;
        g1 = NG * p + 1;
    }
    struct Pre {
        float a0[4], a1[4];  // residual values (ADD)
    };
    __device__ __forceinline__ Pre pre(uint32_t p, int lane, uint32_t m0, uint32_t T) const {
        Pre r{};
        if constexpr (ADD) {
            const uint32_t r0 = 16 * NG * p + (lane & 15), r1 = r0 + 16;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t m = m0 + i;
                if (m >= T) break;
                if (r0 < rows) r.a0[i] = y[at(m, r0)];
                if (NG == 2 && r1 < rows) r.a1[i] = y[at(m, r1)];
            }
        }
        return r;
    }
    __device__ __forceinline__ void apply(uint32_t p, int lane, uint32_t m0, uint32_t T, const floatx4& v0,
                                          const floatx4& v1, const Pre& pr) const {
        const uint32_t r0 = 16 * NG * p + (lane & 15), r1 = r0 + 16;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t m = m0 + r;
            if (m >= T) break;
            if (r0 < rows) y[at(m, r0)] = ADD ? pr.a0[r] + v0[r] * scale : v0[r] * scale;
            if (NG == 2 && r1 < rows) y[at(m, r1)] = ADD ? pr.a1[r] + v1[r] * scale : v1[r] * scale;
        }
    }
};

// Gate and up projections packed as interleaved groups (2j: gate rows 16j..,
// 2j+1: up rows 16j..): h[m][16p + lane%16] = silu(gate) * up, silu(g) =
// g / (1 + exp(-g)) (src/model.rs:375-378).
struct EpiSwiGLU {
    static constexpr int kGroups = 2;
    float* h;
    uint32_t ldh;
    uint32_t inter;
    uint32_t tiled = 0;  // h in the tiled activation order (K = inter, a multiple of 32)
    __device__ __forceinline__ void groups(uint32_t p, uint32_t& g0, uint32_t& g1) const {
        g0 = 2 * p;
        g1 = 2 * p + 1;
    }
    struct Pre {};
    __device__ __forceinline__ Pre pre(uint32_t, int, uint32_t, uint32_t) const { return {}; }
    __device__ __forceinline__ void apply(uint32_t p, int lane, uint32_t m0, uint32_t T, const floatx4& g,
                                          const floatx4& u, const Pre&) const {
        const uint32_t j = 16 * p + (lane & 15);
        if (j >= inter) return;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t m = m0 + r;
            if (m >= T) break;
            const size_t at = tiled ? act_tile_off(m, j, inter / 32) : static_cast<size_t>(m) * ldh + j;
            h[at] = g[r] / (1.0f + expf(-g[r])) * u[r];
        }
    }
};

// Rotate-half RoPE of one dim pair (d, d + 32): [a cos - b sin, a sin + b cos]
// (rope_apply, src/model.rs:720-737), each product rounded before the sum as in the
// reference (no fused multiply-add: otherwise the compiler's choice of which product
// to fuse may differ between kernels that inline this).
__device__ __forceinline__ void rope_rotate(float& a, float& b, float c, float s) {
#pragma clang fp contract(off)
    const float ra = a * c - b * s;
    const float rb = a * s + b * c;
    a = ra;
    b = rb;
}

// Fused Q/K/V projection epilogue for head_dim 64: weights are the row
// concatenation [Wq; Wk; Wv] (heads of 64 rows = 4 groups). Pair p = (head p/2,
// half p%2) takes groups 4h + half and 4h + half + 2, i.e. dims d and d + 32 of
// the head, the two halves rotate-half RoPE mixes (src/model.rs:720-737):
//   [x1 cos - x2 sin, x1 sin + x2 cos] with cos/sin rows of the token's position.
// Q heads go to q[m][h][64]; K heads (rotated) and V heads go straight into the
// F32 pool row slot_mapping[m] (write_kv_slots, src/kv_cache/storage.rs:219-254).
struct EpiQkvRope {
    static constexpr int kGroups = 2;
    float* q;
    float* k_pool;
    float* v_pool;
    const int32_t* positions;
    const int64_t* slots;
    const float* cos_t;  // [max_pos][32]
    const float* sin_t;
    uint32_t* status;
    uint32_t num_heads, num_kv_heads, max_pos;
    int64_t num_slots;
    __device__ __forceinline__ void groups(uint32_t p, uint32_t& g0, uint32_t& g1) const {
        g0 = 4 * (p / 2) + (p % 2);
        g1 = g0 + 2;
    }
    struct Pre {
        float c[4], s[4];  // RoPE cos / sin at the token's position (Q and K heads)
        int64_t slot[4];   // pool row (K and V heads)
    };
    __device__ __forceinline__ Pre pre(uint32_t p, int lane, uint32_t m0, uint32_t T) const {
        Pre r{};
        const uint32_t head = p / 2;
        const uint32_t d = 16 * (p % 2) + (lane & 15);
        const bool is_q = head < num_heads, is_v = head >= num_heads + num_kv_heads;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t m = m0 + i;
            if (m >= T) break;
            if (!is_v) {
                uint32_t pos = static_cast<uint32_t>(positions[m]);
                if (pos >= max_pos) {
                    raise_status(status, KANSO_DEV_POSITION_OOB);
                    pos = max_pos - 1;
                }
                r.c[i] = cos_t[static_cast<size_t>(pos) * 32 + d];
                r.s[i] = sin_t[static_cast<size_t>(pos) * 32 + d];
            }
            if (!is_q) r.slot[i] = slots[m];
        }
        return r;
    }
    __device__ __forceinline__ void apply(uint32_t p, int lane, uint32_t m0, uint32_t T, const floatx4& x1,
                                          const floatx4& x2, const Pre& pr) const {
        const uint32_t head = p / 2;
        const uint32_t d = 16 * (p % 2) + (lane & 15);
        const bool is_q = head < num_heads, is_v = head >= num_heads + num_kv_heads;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t m = m0 + r;
            if (m >= T) break;
            float a = x1[r], b = x2[r];
            if (!is_v) rope_rotate(a, b, pr.c[r], pr.s[r]);
            if (is_q) {
                float* qr = q + (static_cast<size_t>(m) * num_heads + head) * 64;
                qr[d] = a;
                qr[d + 32] = b;
                continue;
            }
            const int64_t slot = pr.slot[r];
            if (slot < 0 || slot >= num_slots) {
                raise_status(status, KANSO_DEV_SLOT_OOB);
                continue;
            }
            const uint32_t kvh = is_v ? head - num_heads - num_kv_heads : head - num_heads;
            float* dst = (is_v ? v_pool : k_pool) + (static_cast<size_t>(slot) * num_kv_heads + kvh) * 64;
            dst[d] = a;
            dst[d + 32] = b;
        }
    }
};

// EpiQkvRope for a 1-byte pool (INT8, FP8 or Q8_0 rows): the two halves of a head
// (units 2h, 2h + 1) meet in one wave, so each K / V row of 64 values is rotated,
// quantized and stored straight into its pool slot with its scale, in the bytes the
// append kernel writes (quantize_head_slice, quantized_storage.rs:452-486;
// BlockQ8_0::from_f32_slice, src/quant/q8_0.rs:13-32): no f32 staging rows and no
// second kernel. Lane l holds dims l % 16 + {0, 32} (v[0], v[1]) and 16 + l % 16 +
// {0, 32} (v[2], v[3]) of tokens m0 .. m0 + 3; a row's maximum is one 16-lane
// reduction. Q rows go to q[m][h][64] as f32.
template <int KVT>
struct EpiQkvRopeQ {
    static constexpr int kGroups = 2;
    static constexpr bool kPairedUnits = true;
    float* q;
    uint8_t* k_pool;
    uint8_t* v_pool;
    void* k_scales;
    void* v_scales;
    const int32_t* positions;
    const int64_t* slots;
    const float* cos_t;  // [max_pos][32]
    const float* sin_t;
    uint32_t* status;
    uint32_t num_heads, num_kv_heads, max_pos;
    int64_t num_slots;
    __device__ __forceinline__ void groups(uint32_t p, uint32_t& g0, uint32_t& g1) const {
        g0 = 4 * (p / 2) + (p % 2);
        g1 = g0 + 2;
    }
    struct Pre {
        float c[2][4], s[2][4];  // RoPE cos / sin of dims l % 16 and 16 + l % 16
        int64_t slot[4];
    };
    __device__ __forceinline__ Pre pre(uint32_t p, int lane, uint32_t m0, uint32_t T) const {
        Pre r{};
        const uint32_t head = p / 2;
        const uint32_t d = lane & 15;
        const bool is_q = head < num_heads, is_v = head >= num_heads + num_kv_heads;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t m = m0 + i;
            if (m >= T) break;
            if (!is_v) {
                uint32_t pos = static_cast<uint32_t>(positions[m]);
                if (pos >= max_pos) {
                    raise_status(status, KANSO_DEV_POSITION_OOB);
                    pos = max_pos - 1;
                }
                r.c[0][i] = cos_t[static_cast<size_t>(pos) * 32 + d];
                r.s[0][i] = sin_t[static_cast<size_t>(pos) * 32 + d];
                r.c[1][i] = cos_t[static_cast<size_t>(pos) * 32 + 16 + d];
                r.s[1][i] = sin_t[static_cast<size_t>(pos) * 32 + 16 + d];
            }
            if (!is_q) r.slot[i] = slots[m];
        }
        return r;
    }
    __device__ __forceinline__ void apply_pair(uint32_t p, int lane, uint32_t m0, uint32_t T, const floatx4 (&v)[4],
                                               const Pre& pr) const {
        const uint32_t head = p / 2;
        const uint32_t d = lane & 15;
        const bool is_q = head < num_heads, is_v = head >= num_heads + num_kv_heads;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            // every lane runs every token (the 16-lane reductions below need the
            // whole group); tokens past T store nothing
            const uint32_t m = m0 + r;
            const bool live = m < T;
            float x[4] = {v[0][r], v[1][r], v[2][r], v[3][r]};  // dims d, d + 32, 16 + d, 48 + d
            if (!is_v) {
                rope_rotate(x[0], x[1], pr.c[0][r], pr.s[0][r]);
                rope_rotate(x[2], x[3], pr.c[1][r], pr.s[1][r]);
            }
            if (is_q) {
                if (live) {
                    float* qr = q + (static_cast<size_t>(m) * num_heads + head) * 64;
                    qr[d] = x[0];
                    qr[d + 32] = x[1];
                    qr[d + 16] = x[2];
                    qr[d + 48] = x[3];
                }
                continue;
            }
            const int64_t slot = pr.slot[r];
            const bool ok = live && slot >= 0 && slot < num_slots;
            if (live && !ok) raise_status(status, KANSO_DEV_SLOT_OOB);
            const uint32_t kvh = is_v ? head - num_heads - num_kv_heads : head - num_heads;
            const size_t row = static_cast<size_t>(ok ? slot : 0) * num_kv_heads + kvh;
            uint8_t* dst = (is_v ? v_pool : k_pool) + row * 64;
            int8_t qv[4];
            if constexpr (KVT == KANSO_KV_Q8_0) {
                // blocks of 32: dims 0..31 are x[0], x[2]; dims 32..63 x[1], x[3]
                const float a0 = group_max<16>(fmaxf(fabsf(x[0]), fabsf(x[2])));
                const float a1 = group_max<16>(fmaxf(fabsf(x[1]), fabsf(x[3])));
                const float d0 = a0 / 127.0f, d1 = a1 / 127.0f;
                const float i0 = d0 != 0.f ? 1.0f / d0 : 0.f, i1 = d1 != 0.f ? 1.0f / d1 : 0.f;
                qv[0] = quant_i8(x[0], i0, -128.0f);
                qv[2] = quant_i8(x[2], i0, -128.0f);
                qv[1] = quant_i8(x[1], i1, -128.0f);
                qv[3] = quant_i8(x[3], i1, -128.0f);
                if (ok && d == 0) {
                    __half* sc = static_cast<__half*>(is_v ? v_scales : k_scales) + row * 2;
                    sc[0] = __float2half_rn(d0);
                    sc[1] = __float2half_rn(d1);
                }
            } else {
                const float amax =
                    group_max<16>(fmaxf(fmaxf(fabsf(x[0]), fabsf(x[1])), fmaxf(fabsf(x[2]), fabsf(x[3]))));
                const float scale = KVT == KANSO_KV_FP8 ? fp8_row_scale(amax) : int8_row_scale(amax);
                const float inv = 1.0f / scale;
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    qv[j] = KVT == KANSO_KV_FP8 ? static_cast<int8_t>(f32_to_e4m3(x[j] * inv))
                                                : quant_i8(x[j], inv, -127.0f);
                if (ok && d == 0) static_cast<float*>(is_v ? v_scales : k_scales)[row] = scale;
            }
            if (ok) {
                dst[d] = static_cast<uint8_t>(qv[0]);
                dst[d + 32] = static_cast<uint8_t>(qv[1]);
                dst[d + 16] = static_cast<uint8_t>(qv[2]);
                dst[d + 48] = static_cast<uint8_t>(qv[3]);
            }
        }
    }
};

// Orderable key of (value, index): larger value wins, then the smaller index
// (greedy_token keeps the first maximum, src/sampler.rs:7-17). NaN never wins.
__device__ __forceinline__ unsigned long long argmax_key(float v, uint32_t idx) {
    const uint32_t b = __builtin_bit_cast(uint32_t, v);
    const uint32_t ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return (static_cast<unsigned long long>(ord) << 32) | (0xffffffffu - idx);
}

// lm_head: optional logits store, and the best key of this pair's 32 rows for
// each token stored to keys[m][p] (plain stores: a device-wide atomic per
// workgroup and token serialises on the token's address); a second kernel takes
// the maximum over the pairs.
struct EpiArgmax {
    static constexpr int kGroups = 2;
    float* logits;  // may be null
    uint32_t ld;
    uint32_t rows;
    unsigned long long* keys;  // [T][pairs]
    uint32_t pairs;
    float scale = 1.f;  // logits x scale (Granite: 1 / logit_scale)
    __device__ __forceinline__ void groups(uint32_t p, uint32_t& g0, uint32_t& g1) const {
        g0 = 2 * p;
        g1 = 2 * p + 1;
    }
    struct Pre {};
    __device__ __forceinline__ Pre pre(uint32_t, int, uint32_t, uint32_t) const { return {}; }
    __device__ __forceinline__ void apply(uint32_t p, int lane, uint32_t m0, uint32_t T, const floatx4& u0,
                                          const floatx4& u1, const Pre&) const {
        const uint32_t r0 = 32 * p + (lane & 15), r1 = r0 + 16;
        const floatx4 v0 = u0 * scale, v1 = u1 * scale;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t m = m0 + r;
            const bool live = m < T;
            unsigned long long key = 0;
            if (live && r0 < rows && !(v0[r] != v0[r])) key = argmax_key(v0[r], r0);
            if (live && r1 < rows && !(v1[r] != v1[r])) key = max(key, argmax_key(v1[r], r1));
            if (live && logits) {
                float* lr = logits + static_cast<size_t>(m) * ld;
                if (r0 < rows) lr[r0] = v0[r];
                if (r1 < rows) lr[r1] = v1[r];
            }
            // max over the 16 lanes that hold this token (same lane / 16)
#pragma unroll
            for (int o = 1; o < 16; o <<= 1) {
                const unsigned long long other = __shfl_xor(key, o, kWave);
                key = max(key, other);
            }
            if (live && (lane & 15) == 0) keys[static_cast<size_t>(m) * pairs + p] = key;
        }
    }
};

// Launch helper: K split over 8 waves (so a token's result never depends on the
// batch size), U blocks of loads in flight per wave so that a whole row (960 or
// 2560 wide) is requested in one round where the registers allow. Up to 256
// tokens a workgroup takes 16 of them (MT = 1): at decode sizes more workgroups
// in flight beat the weight reuse of wider token tiles (re-reads hit L2 / MALL);
// above, 32 (MT = 2, launch_mt2).
template <int U, int MT, int NU, bool NORM, class WL, class Epi>
inline void launch_u(const WL& wl, const XIn& xa, const Epi& epi, uint32_t units, hipStream_t s) {
    const dim3 grid((units + NU - 1) / NU, (xa.T + 16 * MT - 1) / (16 * MT));
    hipLaunchKernelGGL((q8_gemm_kernel<8, U, MT, NU, NORM, WL, Epi>), grid, dim3(8 * kWave), 0, s, wl, xa, epi,
                       units);
}

template <int MT, int NU, bool NORM, class WL, class Epi>
inline void launch_mt(const WL& wl, const XIn& xa, const Epi& epi, uint32_t units, uint32_t nb, hipStream_t s) {
    constexpr int NG = NU * Epi::kGroups;
    if constexpr (MT >= 2)  // 32-64 tokens of x per block already fill the registers
        launch_u<2, MT, NU, NORM>(wl, xa, epi, units, s);
    else if constexpr (NG >= 8)
        launch_u<2, MT, NU, NORM>(wl, xa, epi, units, s);
    else if (nb <= 32)
        launch_u<4, MT, NU, NORM>(wl, xa, epi, units, s);
    else if (NORM || nb <= 40 || NG > 2)  // (the norm weights of 10 blocks would not fit the registers)
        launch_u<5, MT, NU, NORM>(wl, xa, epi, units, s);
    else if constexpr (!NORM && NG <= 2)  // 2560-wide rows (the down projection) in one round
        launch_u<10, MT, NU, NORM>(wl, xa, epi, units, s);
}

// Plain stores need no partner group: with 16-token tiles a unit is one 16-row
// group, so narrow products get twice the workgroups (960 rows: 30 pairs would
// keep 30 CUs busy at batch 1, each pulling a whole pair's weights).
template <class Epi>
struct SingleGroup {
    static constexpr bool kOk = false;
};
template <bool ADD>
struct SingleGroup<EpiStore<ADD, 2>> {
    static constexpr bool kOk = true;
    static EpiStore<ADD, 1> make(const EpiStore<ADD, 2>& e) { return {e.y, e.ldy, e.rows, e.tiled, e.scale}; }
};

// Units per workgroup for 16-token tiles. At these sizes a product's time follows
// the bytes its workgroups pull through their CUs (x once per workgroup, the
// weights once per token tile), and a CU holding two of them takes twice as long:
// the smallest NU that keeps to one workgroup per CU, else the widest. Measured on
// the SmolLM2 shapes at 16-256 tokens: within 5% of the best NU in 31 of 32 cases
// (e.g. gate/up at 80 tokens 10.4 us against 17.4 with NU = 1, down 10.1 against
// 16.5).
inline uint32_t device_cus() {
    static std::atomic<int> cached[64] = {};  // per device; 0 = not queried yet
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int n = cached[dev].load(std::memory_order_relaxed);
    if (n == 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cached[dev].store(n, std::memory_order_relaxed);
    }
    return static_cast<uint32_t>(n);
}

inline uint32_t pick_nu(uint32_t units, uint32_t tiles) {
    const uint64_t cus = device_cus();
    for (uint32_t nu = 1; nu < 4; nu *= 2)
        if (static_cast<uint64_t>((units + nu - 1) / nu) * tiles <= cus) return nu;
    return 4;
}

template <bool NORM, class WL, class Epi>
inline void launch_mt1(const WL& wl, const XIn& xa, const Epi& epi, uint32_t units, uint32_t nb, hipStream_t s) {
    const uint32_t nu = pick_nu(units, (xa.T + 15) / 16);
    if (nu >= 4)
        launch_mt<1, 4, NORM>(wl, xa, epi, units, nb, s);
    else if (nu == 2)
        launch_mt<1, 2, NORM>(wl, xa, epi, units, nb, s);
    else
        launch_mt<1, 1, NORM>(wl, xa, epi, units, nb, s);
}

// Above 256 tokens: 32-token tiles and up to two units (four 16-row groups) per
// workgroup, so each x load feeds 4 groups and each weight load 32 tokens (bytes
// per output (4 MT + 1.06 NG) / (MT NG): 1.53 at MT = 2, NG = 4 against 2.26 for
// 64-token tiles of one pair). Four units would halve the x traffic again but need
// 128 KB of LDS for the partial sums (one workgroup per CU) and measured slower:
// gate/up at 512 tokens 38.5 us (NU = 2), 52.4 (NU = 4), 60 (64-token tiles).
template <bool NORM, class WL, class Epi>
inline void launch_mt2(const WL& wl, const XIn& xa, const Epi& epi, uint32_t units, uint32_t nb, hipStream_t s) {
    if (pick_nu(units, (xa.T + 31) / 32) >= 2)
        launch_mt<2, 2, NORM>(wl, xa, epi, units, nb, s);
    else
        launch_mt<2, 1, NORM>(wl, xa, epi, units, nb, s);
}

template <bool NORM, class WL, class Epi>
inline void launch_norm(const WL& wl, const XIn& xa, const Epi& epi, uint32_t pairs, uint32_t nb, hipStream_t s) {
    // Paired epilogues (gate/up, QKV, the lm_head) switch to 32-token tiles as soon
    // as 16-token tiles would need more than four workgroups per CU: the lm_head at
    // 49 tokens 68 -> 53 us, gate/up at 128 tokens 17.7 -> 16.4. Plain stores keep
    // their single-group units up to 256 tokens (down at 49 tokens: 9.5 us against
    // 13.5 with 32-token tiles of pairs).
    const bool wide = !SingleGroup<Epi>::kOk && xa.T > 16 &&
                      static_cast<uint64_t>(pairs) * ((xa.T + 15) / 16) >= 4ull * device_cus();
    if (xa.T > 256 || wide)
        launch_mt2<NORM>(wl, xa, epi, pairs, nb, s);
    else if constexpr (SingleGroup<Epi>::kOk)
        launch_mt1<NORM>(wl, xa, SingleGroup<Epi>::make(epi), (epi.rows + 15) / 16, nb, s);
    else
        launch_mt1<NORM>(wl, xa, epi, pairs, nb, s);
}

// Paired-unit epilogues (a whole 64-row head per wave): two units per workgroup,
// 32-token tiles under the same rule as the other paired epilogues.
template <class WL, class Epi>
inline int launch_q8_gemm_paired(const WL& wl, const XIn& xa, const Epi& epi, uint32_t units, hipStream_t s) {
    if (xa.T == 0 || units == 0) return KANSO_OK;
    if (!xa.norm_w || units % 2 != 0) {
        set_error("paired-unit product: needs the RMSNorm prologue and an even unit count");
        return KANSO_E_INVALID_ARG;
    }
    const uint32_t nb = xa.in / 32;
    const bool wide = xa.T > 16 && static_cast<uint64_t>(units / 2) * ((xa.T + 15) / 16) >= 4ull * device_cus();
    if (xa.T > 256 || wide)
        launch_mt<2, 2, true>(wl, xa, epi, units, nb, s);
    else
        launch_mt<1, 2, true>(wl, xa, epi, units, nb, s);
    KANSO_LAUNCH_CHECK();
    return KANSO_OK;
}

template <class WL, class Epi>
inline int launch_q8_gemm(const WL& wl, const XIn& xa, const Epi& epi, uint32_t pairs, hipStream_t s) {
    if (xa.T == 0 || pairs == 0) return KANSO_OK;
    const uint32_t nb = xa.in / 32;
    if (xa.norm_w)
        launch_norm<true>(wl, xa, epi, pairs, nb, s);
    else
        launch_norm<false>(wl, xa, epi, pairs, nb, s);
    KANSO_LAUNCH_CHECK();
    return KANSO_OK;
}

}  // namespace kanso
