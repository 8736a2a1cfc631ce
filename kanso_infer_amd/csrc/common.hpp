// common.hpp — shared plumbing of libkanso_hip.so: the context, error reporting,
// scratch management and wave64 helpers for the gfx950 kernels.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>
#include <vector>

#include "../../include/kanso_hip.h"

namespace kanso {

// ---------------------------------------------------------------- host side

void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));

struct ProfileRecord {
    std::string name;
    hipEvent_t start, stop;
};

struct ProfileTotal {
    double ms = 0.0;
    uint64_t launches = 0;
};

}  // namespace kanso

struct kanso_ctx {
    int device = 0;
    int num_cus = 256;
    uint32_t* status = nullptr;  // device status word (KANSO_DEV_* bits)
    // Grow-only scratch: split-K partials, work list, small index arrays.
    void* scratch = nullptr;
    size_t scratch_bytes = 0;
    // Events reused by the profiling hooks.
    std::vector<hipEvent_t> event_pool;
    // Grow-only buffer of 64-bit argmax keys (lm_head epilogue).
    void* keys = nullptr;
    size_t keys_bytes = 0;
    // Device address of this device's copy of attention.hip's fixed scratch array
    // (kanso_ragged_paged_attention_noalloc), resolved once at kanso_create.
    void* noalloc_scratch = nullptr;
    bool profiling = false;
    std::vector<kanso::ProfileRecord> pending;
    std::vector<std::pair<std::string, kanso::ProfileTotal>> totals;
};

namespace kanso {

#define KANSO_HIP_TRY(expr)                                                             \
    do {                                                                                \
        hipError_t _e = (expr);                                                         \
        if (_e != hipSuccess) {                                                         \
            ::kanso::set_error("%s failed: %s (%s:%d)", #expr, hipGetErrorString(_e),   \
                               __FILE__, __LINE__);                                     \
            return KANSO_E_HIP;                                                         \
        }                                                                               \
    } while (0)

// Makes ctx->scratch at least `bytes` large. Scratch may still be read by work
// enqueued earlier, so growth waits for the device before freeing the old buffer.
int ensure_scratch(kanso_ctx* ctx, size_t bytes);
// Resolves the device address of the fixed attention scratch array on the current
// device (attention.hip); called once per context by kanso_create.
int noalloc_scratch_init(void** ptr);
int ensure_keys(kanso_ctx* ctx, size_t bytes);

// Profiling hooks around one kernel launch (no-ops unless ctx->profiling).
int prof_begin(kanso_ctx* ctx, const char* name, hipStream_t stream, hipEvent_t* start);
int prof_end(kanso_ctx* ctx, const char* name, hipStream_t stream, hipEvent_t start);

inline hipStream_t as_stream(kanso_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// Launch check: a bad configuration surfaces here instead of as a later fault.
#define KANSO_LAUNCH_CHECK()                                                            \
    do {                                                                                \
        hipError_t _e = hipGetLastError();                                              \
        if (_e != hipSuccess) {                                                         \
            ::kanso::set_error("kernel launch failed: %s (%s:%d)", hipGetErrorString(_e), \
                               __FILE__, __LINE__);                                     \
            return KANSO_E_HIP;                                                         \
        }                                                                               \
    } while (0)

// ---------------------------------------------------------------- device side

constexpr int kWave = 64;

// v of lane (this lane ^ mask). Masks 16 and 32 use gfx950's lane swaps
// (v_permlane16_swap / v_permlane32_swap: a VALU op that hands each lane the values
// of both lanes of its pair, no LDS round trip); other masks a lane permute
// through LDS (ds_bpermute). Same values either way.
__device__ __forceinline__ float wave_xor(float v, int mask) {
    const uint32_t u = __float_as_uint(v);
    if (mask == 32) {
        const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);  // {lane & ~32, lane | 32}
        return __uint_as_float((__lane_id() & 32) ? r[0] : r[1]);
    }
    if (mask == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);  // {lane & ~16, lane | 16}
        return __uint_as_float((__lane_id() & 16) ? r[0] : r[1]);
    }
    return __shfl_xor(v, mask, kWave);
}

// DPP lane permutations inside a 16-lane row (no LDS traffic, no address registers).
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xf, 0xf, true));
}
constexpr int kDppQuadSwap1 = 0xB1;   // quad_perm [1,0,3,2]: lane ^ 1
constexpr int kDppQuadSwap2 = 0x4E;   // quad_perm [2,3,0,1]: lane ^ 2
constexpr int kDppHalfMirror = 0x141;  // lane i <-> 7 - i within 8 lanes
constexpr int kDppRowMirror = 0x140;   // lane i <-> 15 - i within 16 lanes

// Sum over aligned groups of N lanes (N = 1, 2, 4, 8, 16, 32, 64); every lane of a
// group ends with the group's total. Within a row the partners are lane ^ 1,
// lane ^ 2, the mirror of 8 and the mirror of 16 (a butterfly whose pairings span
// the group); across rows a lane shuffle.
template <int N>
__device__ __forceinline__ float group_sum(float v) {
    if constexpr (N >= 2) v += dpp<kDppQuadSwap1>(v);
    if constexpr (N >= 4) v += dpp<kDppQuadSwap2>(v);
    if constexpr (N >= 8) v += dpp<kDppHalfMirror>(v);
    if constexpr (N >= 16) v += dpp<kDppRowMirror>(v);
    if constexpr (N >= 32) v += wave_xor(v, 16);
    if constexpr (N >= 64) v += wave_xor(v, 32);
    return v;
}

// Maximum over aligned groups of N lanes, like group_sum.
template <int N>
__device__ __forceinline__ float group_max(float v) {
    if constexpr (N >= 2) v = fmaxf(v, dpp<kDppQuadSwap1>(v));
    if constexpr (N >= 4) v = fmaxf(v, dpp<kDppQuadSwap2>(v));
    if constexpr (N >= 8) v = fmaxf(v, dpp<kDppHalfMirror>(v));
    if constexpr (N >= 16) v = fmaxf(v, dpp<kDppRowMirror>(v));
    if constexpr (N >= 32) v = fmaxf(v, wave_xor(v, 16));
    if constexpr (N >= 64) v = fmaxf(v, wave_xor(v, 32));
    return v;
}

// Tiled activation order: the decoder's activation matrices [tokens][K] (K a
// multiple of 32) laid out in the order the bf16 matrix cores take their A operand
// (lane l = 16 kq + mm holds token mm, columns 32 b + 8 kq .. + 7). Token m, column
// k lives in 16-token tile m / 16, 32-column block k / 32, half (k % 8) / 4, at lane
// 16 ((k % 32) / 8) + m % 16, element k % 4:
//   ((tile * nbk + block) * 2 + half) * 256 + lane * 4 + k % 4   (nbk = K / 32).
// So one wave reads a (tile, block, half) slice as one contiguous 1 KB load, where
// the row-major order makes each load touch 16 rows; four consecutive columns
// (k % 4 == 0) stay contiguous, so float4 stores of a row keep working.
__host__ __device__ __forceinline__ size_t act_tile_off(uint32_t m, uint32_t k, uint32_t nbk) {
    return ((static_cast<size_t>(m >> 4) * nbk + (k >> 5)) * 2 + ((k >> 2) & 1)) * 256 +
           (((k >> 3) & 3) * 16 + (m & 15)) * 4 + (k & 3);
}

// 2^x on the transcendental unit (v_exp_f32); results below the f32 normal range
// flush to 0, which only ever affects probabilities that are already negligible.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ void raise_status(uint32_t* status, uint32_t bits) {
    atomicOr(status, bits);
}

// OCP FP8 E4M3FN (bias 7, 3 mantissa bits, subnormal step 2^-9, no infinities,
// NaN = S.1111.111, largest finite 448). Encode: round to nearest, ties to even;
// 464 and above saturate to 448 (the KV quantizer never reaches them).
__device__ __forceinline__ uint32_t f32_to_e4m3(float x) {
    const uint32_t u = __float_as_uint(x);
    const uint32_t sign = (u >> 24) & 0x80u;
    const uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return sign | 0x7fu;
    if (a >= 0x43e80000u) return sign | 0x7eu;
    if (a >= 0x3c800000u) return sign | (((a + 0x7ffffu + ((a >> 20) & 1u)) >> 20) - (120u << 3));
    return sign | static_cast<uint32_t>(__builtin_rintf(__uint_as_float(a) * 512.0f));
}

// Row scales of the 1-byte KV quantizers, shared by the append kernel and the QKV
// epilogue so both write the same bytes. quantize_head_slice
// (quantized_storage.rs:452-486): INT8 scale = amax > 0 ? amax / 127 : 1, q =
// round(x / scale) clamped to +-127; FP8 scale = 2^ceil(log2(amax / 64)) (1 for
// amax = 0), q = E4M3(x / scale). BlockQ8_0::from_f32_slice (src/quant/q8_0.rs:13-32):
// d = amax / 127, q = round(x / d) clamped to [-128, 127] (0 for d = 0). All steps
// are IEEE-exact or correctly rounded: this library is built with correctly rounded
// division, roundf rounds half away from zero like Rust's f32::round.
__device__ __forceinline__ float int8_row_scale(float amax) { return amax > 0.f ? amax / 127.0f : 1.0f; }
__device__ __forceinline__ float fp8_row_scale(float amax) {
    float scale = 1.0f;
    if (amax > 0.f) {
        int e2;
        const float fr = frexpf(amax / 64.0f, &e2);
        scale = ldexpf(1.0f, fr == 0.5f ? e2 - 1 : e2);
    }
    return scale;
}
__device__ __forceinline__ int8_t quant_i8(float x, float inv, float lo) {
    return static_cast<int8_t>(fminf(fmaxf(roundf(x * inv), lo), 127.0f));
}

// Four E4M3 bytes of a word -> f32 with gfx950's packed conversion
// (v_cvt_pk_f32_fp8: OCP E4M3FN on CDNA4), two bytes per instruction.
__device__ __forceinline__ void e4m3x4_to_f32(uint32_t w, float& a, float& b, float& c, float& d) {
    const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w), false);
    const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w), true);
    a = lo[0];
    b = lo[1];
    c = hi[0];
    d = hi[1];
}

__device__ __forceinline__ float e4m3_to_f32(uint32_t b) {
    const uint32_t e = (b >> 3) & 0xfu, m = b & 7u;
    float v = e ? __uint_as_float(((e + 120u) << 23) | (m << 20)) : static_cast<float>(m) * 0.001953125f;
    v = (b & 0x7fu) == 0x7fu ? __uint_as_float(0x7fc00000u) : v;
    return (b & 0x80u) ? -v : v;
}

}  // namespace kanso
