// kv_append.hip — fused KV append (+ quantize) into the paged pool, and block reset.
//
// Reference: KvStorageKind::write_kv_slots (src/kv_cache/kind.rs:348-374) — an F32
// scatter of [T, Hkv, D] rows into pool row `slot` (storage.rs:219-254), or per
// token and KV head quantize_head_slice (quantized_storage.rs:452-486) for INT8 and FP8;
// Q8_0 rows use BlockQ8_0::from_f32_slice (src/quant/q8_0.rs:13-32) per 32 values
// with d stored as f16.
//
// Bit-exactness: the quantizers use only IEEE-exact steps — |x| and max are exact,
// amax / 127 and 1 / scale are correctly rounded divisions (this library is built
// with -fhip-fp32-correctly-rounded-divide-sqrt), x * inv is one rounded multiply,
// roundf rounds half away from zero like Rust's f32::round, and the clamp makes the
// i8 conversion exact. f16 conversion is round-to-nearest-even.
//
// Mapping: one wave64 per (token, KV head) row; lane i holds elements i, i+64, ...
// so the row's amax is one wave butterfly (INT8) or one butterfly per 32-lane half
// (Q8_0: a 32-element block is exactly half a wave).
#include <cmath>

#include "common.hpp"

namespace kanso {
namespace {

constexpr int kAppendThreads = 256;
constexpr int kAppendWaves = kAppendThreads / kWave;

__global__ __launch_bounds__(kAppendThreads) void append_f32(
    const float4* __restrict__ k, const float4* __restrict__ v, const int64_t* __restrict__ slots,
    uint32_t T, uint32_t row4, int64_t num_slots, float4* __restrict__ kp, float4* __restrict__ vp,
    uint32_t* status) {
    const uint64_t total = static_cast<uint64_t>(T) * row4;
    for (uint64_t e = blockIdx.x * static_cast<uint64_t>(kAppendThreads) + threadIdx.x; e < total;
         e += static_cast<uint64_t>(gridDim.x) * kAppendThreads) {
        const uint32_t t = static_cast<uint32_t>(e / row4), c = static_cast<uint32_t>(e % row4);
        const int64_t slot = slots[t];
        if (slot < 0 || slot >= num_slots) {
            if (c == 0) raise_status(status, KANSO_DEV_SLOT_OOB);
            continue;
        }
        kp[static_cast<size_t>(slot) * row4 + c] = k[e];
        vp[static_cast<size_t>(slot) * row4 + c] = v[e];
    }
}

__device__ __forceinline__ float wave_max_all(float v) {
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) v = fmaxf(v, wave_xor(v, o));
    return v;
}

__device__ __forceinline__ float half_wave_max(float v) {
#pragma unroll
    for (int o = 1; o < 32; o <<= 1) v = fmaxf(v, wave_xor(v, o));
    return v;
}

// quantize_head_slice, INT8 arm: scale = amax > 0 ? amax / 127 : 1; inv = 1 / scale;
// q = round(x * inv).clamp(-127, 127).
template <int PER>
__device__ void quant_row_int8(const float* __restrict__ x, uint32_t D, int lane, int8_t* __restrict__ q,
                               float* __restrict__ scale_out) {
    float vals[PER];
    float amax = 0.f;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const uint32_t d = lane + k * kWave;
        vals[k] = d < D ? x[d] : 0.f;
        amax = fmaxf(amax, fabsf(vals[k]));
    }
    amax = wave_max_all(amax);
    const float scale = int8_row_scale(amax);
    const float inv = 1.0f / scale;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const uint32_t d = lane + k * kWave;
        if (d < D) q[d] = quant_i8(vals[k], inv, -127.0f);
    }
    if (lane == 0) *scale_out = scale;
}

// quantize_head_slice, FP8 arm (quantized_storage.rs:470-486): scale =
// 2^ceil(log2(amax / 64)) (1 for amax = 0), q = E4M3(x * (1 / scale)). ceil(log2)
// is exact here (frexp of amax / 64), scale and 1 / scale are powers of two, and
// the E4M3 encode rounds to nearest even.
template <int PER>
__device__ void quant_row_fp8(const float* __restrict__ x, uint32_t D, int lane, uint8_t* __restrict__ q,
                              float* __restrict__ scale_out) {
    float vals[PER];
    float amax = 0.f;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const uint32_t d = lane + k * kWave;
        vals[k] = d < D ? x[d] : 0.f;
        amax = fmaxf(amax, fabsf(vals[k]));
    }
    amax = wave_max_all(amax);
    const float scale = fp8_row_scale(amax);
    const float inv = 1.0f / scale;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const uint32_t d = lane + k * kWave;
        if (d < D) q[d] = static_cast<uint8_t>(f32_to_e4m3(vals[k] * inv));
    }
    if (lane == 0) *scale_out = scale;
}

// BlockQ8_0::from_f32_slice per 32 elements: d = amax / 127; id = d != 0 ? 1 / d : 0;
// q = round(x * id).clamp(-128, 127); d stored as f16 (round to nearest even).
template <int PER>
__device__ void quant_row_q8_0(const float* __restrict__ x, uint32_t D, int lane, int8_t* __restrict__ q,
                               __half* __restrict__ d_out) {
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const uint32_t d = lane + k * kWave;  // D % 32 == 0, so a half-wave is one block
        const bool in = d < D;
        const float val = in ? x[d] : 0.f;
        const float amax = half_wave_max(fabsf(val));
        const float sc = amax / 127.0f;
        const float id = sc != 0.f ? 1.0f / sc : 0.f;
        if (in) {
            q[d] = quant_i8(val, id, -128.0f);
            if ((d & 31) == 0) d_out[d / 32] = __float2half_rn(sc);
        }
    }
}

template <int PER, int KVT>
__global__ __launch_bounds__(kAppendThreads) void append_quant(
    const float* __restrict__ k, const float* __restrict__ v, const int64_t* __restrict__ slots,
    uint32_t T, uint32_t HKV, uint32_t D, int64_t num_slots, int8_t* __restrict__ kq,
    int8_t* __restrict__ vq, void* __restrict__ ks, void* __restrict__ vs, uint32_t* status) {
    const int lane = threadIdx.x & (kWave - 1);
    const uint64_t rows = static_cast<uint64_t>(T) * HKV;
    for (uint64_t r = blockIdx.x * static_cast<uint64_t>(kAppendWaves) + threadIdx.x / kWave; r < rows;
         r += static_cast<uint64_t>(gridDim.x) * kAppendWaves) {
        const uint32_t t = static_cast<uint32_t>(r / HKV), h = static_cast<uint32_t>(r % HKV);
        const int64_t slot = slots[t];
        if (slot < 0 || slot >= num_slots) {
            if (lane == 0 && h == 0) raise_status(status, KANSO_DEV_SLOT_OOB);
            continue;
        }
        const size_t dst_row = static_cast<size_t>(slot) * HKV + h;  // (block*bs + off)*Hkv + h
        const float* ksrc = k + r * D;
        const float* vsrc = v + r * D;
        if (KVT == KANSO_KV_INT8) {
            quant_row_int8<PER>(ksrc, D, lane, kq + dst_row * D, static_cast<float*>(ks) + dst_row);
            quant_row_int8<PER>(vsrc, D, lane, vq + dst_row * D, static_cast<float*>(vs) + dst_row);
        } else if (KVT == KANSO_KV_FP8) {
            quant_row_fp8<PER>(ksrc, D, lane, reinterpret_cast<uint8_t*>(kq) + dst_row * D,
                               static_cast<float*>(ks) + dst_row);
            quant_row_fp8<PER>(vsrc, D, lane, reinterpret_cast<uint8_t*>(vq) + dst_row * D,
                               static_cast<float*>(vs) + dst_row);
        } else {
            quant_row_q8_0<PER>(ksrc, D, lane, kq + dst_row * D, static_cast<__half*>(ks) + dst_row * (D / 32));
            quant_row_q8_0<PER>(vsrc, D, lane, vq + dst_row * D, static_cast<__half*>(vs) + dst_row * (D / 32));
        }
    }
}

// Erase blocks: quant / f32 bytes -> 0, INT8 / FP8 scales -> 1.0 (QuantizedKvBlock::reset,
// quantized_storage.rs:35-40), Q8_0 scales -> 0.
__global__ __launch_bounds__(kAppendThreads) void reset_blocks_kernel(
    const uint32_t* __restrict__ blocks, uint32_t n, uint32_t num_blocks, uint32_t block_bytes,
    uint32_t scale_elems, uint32_t kv_dtype, uint8_t* kp, uint8_t* vp, void* ks, void* vs,
    uint32_t* status) {
    for (uint32_t b = blockIdx.x; b < n; b += gridDim.x) {
        const uint32_t blk = blocks[b];
        if (blk >= num_blocks) {
            if (threadIdx.x == 0) raise_status(status, KANSO_DEV_BLOCK_OOB);
            continue;
        }
        uint32_t* kw = reinterpret_cast<uint32_t*>(kp + static_cast<size_t>(blk) * block_bytes);
        uint32_t* vw = reinterpret_cast<uint32_t*>(vp + static_cast<size_t>(blk) * block_bytes);
        for (uint32_t i = threadIdx.x; i < block_bytes / 4; i += kAppendThreads) {
            kw[i] = 0u;
            vw[i] = 0u;
        }
        if (kv_dtype == KANSO_KV_INT8 || kv_dtype == KANSO_KV_FP8) {
            float* ksf = static_cast<float*>(ks) + static_cast<size_t>(blk) * scale_elems;
            float* vsf = static_cast<float*>(vs) + static_cast<size_t>(blk) * scale_elems;
            for (uint32_t i = threadIdx.x; i < scale_elems; i += kAppendThreads) {
                ksf[i] = 1.0f;
                vsf[i] = 1.0f;
            }
        } else if (kv_dtype == KANSO_KV_Q8_0) {
            uint16_t* ksh = static_cast<uint16_t*>(ks) + static_cast<size_t>(blk) * scale_elems;
            uint16_t* vsh = static_cast<uint16_t*>(vs) + static_cast<size_t>(blk) * scale_elems;
            for (uint32_t i = threadIdx.x; i < scale_elems; i += kAppendThreads) {
                ksh[i] = 0;
                vsh[i] = 0;
            }
        }
    }
}

using QuantFn = void (*)(const float*, const float*, const int64_t*, uint32_t, uint32_t, uint32_t,
                         int64_t, int8_t*, int8_t*, void*, void*, uint32_t*);

template <int KVT>
QuantFn pick_quant(uint32_t D) {
    if (D <= 64) return append_quant<1, KVT>;
    if (D <= 128) return append_quant<2, KVT>;
    return append_quant<4, KVT>;
}

int check_common(uint32_t kv_dtype, uint32_t num_blocks, uint32_t block_size, uint32_t hkv,
                 uint32_t head_dim, const void* kp, const void* vp, const void* ks, const void* vs,
                 const char* who) {
    if (!kp || !vp) {
        set_error("%s: null pool", who);
        return KANSO_E_INVALID_ARG;
    }
    if (kv_dtype > KANSO_KV_FP8) {
        set_error("%s: unknown kv_dtype %u", who, kv_dtype);
        return KANSO_E_INVALID_ARG;
    }
    if (kv_dtype != KANSO_KV_F32 && (!ks || !vs)) {
        set_error("%s: quantized pool needs k_scales and v_scales", who);
        return KANSO_E_INVALID_ARG;
    }
    if (num_blocks == 0 || block_size == 0 || hkv == 0 || head_dim == 0 || head_dim > 256) {
        set_error("%s: bad pool geometry (blocks %u, block_size %u, kv heads %u, head_dim %u)", who,
                  num_blocks, block_size, hkv, head_dim);
        return KANSO_E_INVALID_SHAPE;
    }
    if (head_dim % 4 != 0 || (kv_dtype == KANSO_KV_Q8_0 && head_dim % 32 != 0)) {
        set_error("%s: head_dim %u not supported for kv_dtype %u", who, head_dim, kv_dtype);
        return KANSO_E_INVALID_SHAPE;
    }
    return KANSO_OK;
}

}  // namespace
}  // namespace kanso

using namespace kanso;

extern "C" {

int kanso_kv_append(kanso_ctx* ctx, uint32_t kv_dtype, const float* k, const float* v,
                    const int64_t* slot_mapping, uint32_t num_tokens, uint32_t num_blocks,
                    uint32_t block_size, uint32_t num_kv_heads, uint32_t head_dim, void* k_pool,
                    void* v_pool, void* k_scales, void* v_scales, kanso_stream_t stream) {
    if (!ctx || !k || !v || !slot_mapping) {
        set_error("kanso_kv_append: null argument");
        return KANSO_E_INVALID_ARG;
    }
    int rc = check_common(kv_dtype, num_blocks, block_size, num_kv_heads, head_dim, k_pool, v_pool,
                          k_scales, v_scales, "kanso_kv_append");
    if (rc) return rc;
    if (num_tokens == 0) return KANSO_OK;
    hipStream_t s = as_stream(stream);
    const int64_t num_slots = static_cast<int64_t>(num_blocks) * block_size;
    hipEvent_t ev;
    if ((rc = prof_begin(ctx, "append", s, &ev))) return rc;
    if (kv_dtype == KANSO_KV_F32) {
        const uint32_t row4 = num_kv_heads * head_dim / 4;
        const uint64_t total = static_cast<uint64_t>(num_tokens) * row4;
        const uint32_t grid = static_cast<uint32_t>(std::min<uint64_t>((total + kAppendThreads - 1) / kAppendThreads, 4096));
        hipLaunchKernelGGL(append_f32, dim3(grid), dim3(kAppendThreads), 0, s,
                           reinterpret_cast<const float4*>(k), reinterpret_cast<const float4*>(v),
                           slot_mapping, num_tokens, row4, num_slots, static_cast<float4*>(k_pool),
                           static_cast<float4*>(v_pool), ctx->status);
    } else {
        QuantFn fn = kv_dtype == KANSO_KV_INT8  ? pick_quant<KANSO_KV_INT8>(head_dim)
                     : kv_dtype == KANSO_KV_FP8 ? pick_quant<KANSO_KV_FP8>(head_dim)
                                                : pick_quant<KANSO_KV_Q8_0>(head_dim);
        const uint64_t rows = static_cast<uint64_t>(num_tokens) * num_kv_heads;
        const uint32_t grid = static_cast<uint32_t>(std::min<uint64_t>((rows + kAppendWaves - 1) / kAppendWaves, 4096));
        hipLaunchKernelGGL(fn, dim3(grid), dim3(kAppendThreads), 0, s, k, v, slot_mapping, num_tokens,
                           num_kv_heads, head_dim, num_slots, static_cast<int8_t*>(k_pool),
                           static_cast<int8_t*>(v_pool), k_scales, v_scales, ctx->status);
    }
    KANSO_LAUNCH_CHECK();
    return prof_end(ctx, "append", s, ev);
}

int kanso_kv_reset_blocks(kanso_ctx* ctx, uint32_t kv_dtype, const uint32_t* blocks,
                          uint32_t num_reset, uint32_t num_blocks, uint32_t block_size,
                          uint32_t num_kv_heads, uint32_t head_dim, void* k_pool, void* v_pool,
                          void* k_scales, void* v_scales, kanso_stream_t stream) {
    if (!ctx || (!blocks && num_reset)) {
        set_error("kanso_kv_reset_blocks: null argument");
        return KANSO_E_INVALID_ARG;
    }
    int rc = check_common(kv_dtype, num_blocks, block_size, num_kv_heads, head_dim, k_pool, v_pool,
                          k_scales, v_scales, "kanso_kv_reset_blocks");
    if (rc) return rc;
    if (num_reset == 0) return KANSO_OK;
    const uint32_t elems = block_size * num_kv_heads * head_dim;
    const uint32_t block_bytes = kv_dtype == KANSO_KV_F32 ? elems * 4 : elems;
    const uint32_t scale_elems = kv_dtype == KANSO_KV_INT8 || kv_dtype == KANSO_KV_FP8 ? block_size * num_kv_heads
                                 : kv_dtype == KANSO_KV_Q8_0 ? block_size * num_kv_heads * (head_dim / 32)
                                                             : 0;
    hipStream_t s = as_stream(stream);
    hipLaunchKernelGGL(reset_blocks_kernel, dim3(std::min<uint32_t>(num_reset, 4096)), dim3(kAppendThreads), 0, s,
                       blocks, num_reset, num_blocks, block_bytes, scale_elems, kv_dtype,
                       static_cast<uint8_t*>(k_pool), static_cast<uint8_t*>(v_pool), k_scales, v_scales,
                       ctx->status);
    KANSO_LAUNCH_CHECK();
    return KANSO_OK;
}

}  // extern "C"
