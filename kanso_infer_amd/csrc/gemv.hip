// gemv.hip — dequant-on-the-fly GEMV / small GEMM over GGUF Q4_K weights (the
// Q8_0 products live in gemm.hip).
//
// Reference: scalar_gemv_q4_k (src/quant/q4_k.rs:162-186): out[r] = sum over
// blocks of the dequantized weights times x, f32 accumulation; a batch of b
// activation rows is b GEMVs. Production reads candle's GGUF blocks (f16 d / dmin:
// 144 B), which is what this kernel consumes (src/quant/mod.rs:1-17).
//
// Mapping: 16 lanes share one weight row and stride over its blocks, 4 rows per
// wave64, 16 rows per 256-thread workgroup. The 16 partial sums of a row meet in a
// 4-step butterfly. The batch is processed in chunks of up to 8 activation rows
// held in registers, so weights stream from HBM once per chunk (batch <= 8: once).
// Activations are small (b x in x 4 B <= 320 KB) and stay in L2.
#include "common.hpp"

namespace kanso {
namespace {

constexpr int kGemvThreads = 256;
constexpr int kLanesPerRow = 16;
constexpr int kRowsPerBlock = kGemvThreads / kLanesPerRow;
constexpr int kBatchChunk = 8;

__device__ __forceinline__ float row_sum16(float v) {
#pragma unroll
    for (int o = 1; o < kLanesPerRow; o <<= 1) v += wave_xor(v, o);
    return v;
}

// get_scale_min_k4 (src/quant/q4_k.rs:16-26) on the 12 packed scale bytes.
__device__ __forceinline__ void scale_min_k4(uint32_t j, const uint8_t* q, float& sc, float& m) {
    if (j < 4) {
        sc = static_cast<float>(q[j] & 63);
        m = static_cast<float>(q[j + 4] & 63);
    } else {
        sc = static_cast<float>((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        m = static_cast<float>((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

// One unit = one 64-element chunk of a 256-element Q4_K block: 32 qs bytes whose low
// nibbles are sub-block 2c and high nibbles sub-block 2c+1 (q4_k.rs:127-146).
template <int BC>
__global__ __launch_bounds__(kGemvThreads) void gemv_q4_k_kernel(
    const uint8_t* __restrict__ w, const float* __restrict__ x, float* __restrict__ y, uint32_t rows,
    uint32_t in, uint32_t b0, uint32_t bn) {
    const uint32_t row = blockIdx.x * kRowsPerBlock + threadIdx.x / kLanesPerRow;
    const uint32_t sub = threadIdx.x % kLanesPerRow;
    const uint32_t nb = in / 256;
    const uint32_t units = nb * 4;
    const bool live = row < rows;
    const uint8_t* wr = w + static_cast<size_t>(live ? row : 0) * nb * 144;
    float acc[BC];
#pragma unroll
    for (int j = 0; j < BC; ++j) acc[j] = 0.f;
    if (live) {
        for (uint32_t u = sub; u < units; u += kLanesPerRow) {
            const uint32_t blk = u / 4, c = u % 4;
            const uint8_t* bp = wr + static_cast<size_t>(blk) * 144;
            const uint32_t dd = *reinterpret_cast<const uint32_t*>(bp);
            const float d = __half2float(__ushort_as_half(static_cast<uint16_t>(dd & 0xffff)));
            const float dmin = __half2float(__ushort_as_half(static_cast<uint16_t>(dd >> 16)));
            uint8_t scales[12];
            const uint32_t* sw = reinterpret_cast<const uint32_t*>(bp + 4);
#pragma unroll
            for (int i = 0; i < 3; ++i) {
                const uint32_t v = sw[i];
                scales[4 * i] = v & 0xff;
                scales[4 * i + 1] = (v >> 8) & 0xff;
                scales[4 * i + 2] = (v >> 16) & 0xff;
                scales[4 * i + 3] = v >> 24;
            }
            float sc1, m1, sc2, m2;
            scale_min_k4(2 * c, scales, sc1, m1);
            scale_min_k4(2 * c + 1, scales, sc2, m2);
            const float d1 = d * sc1, min1 = dmin * m1, d2 = d * sc2, min2 = dmin * m2;
            float lo[32], hi[32];
            const uint32_t* qw = reinterpret_cast<const uint32_t*>(bp + 16 + 32 * c);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t v = qw[i];
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    const uint32_t byte = (v >> (8 * b)) & 0xff;
                    lo[4 * i + b] = d1 * static_cast<float>(byte & 0xF) - min1;
                    hi[4 * i + b] = d2 * static_cast<float>(byte >> 4) - min2;
                }
            }
#pragma unroll
            for (int j = 0; j < BC; ++j) {
                if (j >= static_cast<int>(bn)) break;
                const float4* xv = reinterpret_cast<const float4*>(x + static_cast<size_t>(b0 + j) * in + blk * 256 + c * 64);
                float s = 0.f;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const float4 xl = xv[i], xh = xv[8 + i];
                    s += lo[4 * i] * xl.x + lo[4 * i + 1] * xl.y + lo[4 * i + 2] * xl.z + lo[4 * i + 3] * xl.w;
                    s += hi[4 * i] * xh.x + hi[4 * i + 1] * xh.y + hi[4 * i + 2] * xh.z + hi[4 * i + 3] * xh.w;
                }
                acc[j] += s;
            }
        }
    }
#pragma unroll
    for (int j = 0; j < BC; ++j) {
        if (j >= static_cast<int>(bn)) break;
        const float r = row_sum16(acc[j]);
        if (live && sub == 0) y[static_cast<size_t>(b0 + j) * rows + row] = r;
    }
}

constexpr uint32_t kMaxBatch = 64;

int check_gemv(kanso_ctx* ctx, const void* w, const float* x, float* y, uint32_t out_f, uint32_t in_f,
               uint32_t batch, uint32_t block, const char* who) {
    if (!ctx || !w || !x || !y) {
        set_error("%s: null argument", who);
        return KANSO_E_INVALID_ARG;
    }
    if (out_f == 0 || in_f == 0 || in_f % block != 0) {
        set_error("%s: in_features %u must be a non-zero multiple of %u (out_features %u)", who, in_f,
                  block, out_f);
        return KANSO_E_INVALID_SHAPE;
    }
    if (batch == 0 || batch > kMaxBatch) {
        set_error("%s: batch %u outside 1..=%u", who, batch, kMaxBatch);
        return KANSO_E_INVALID_SHAPE;
    }
    if (reinterpret_cast<uintptr_t>(x) % 16 != 0 || reinterpret_cast<uintptr_t>(w) % 4 != 0) {
        set_error("%s: x must be 16-byte and w 4-byte aligned", who);
        return KANSO_E_INVALID_ARG;
    }
    return KANSO_OK;
}

}  // namespace
}  // namespace kanso

using namespace kanso;

extern "C" {

int kanso_gemv_q4_k(kanso_ctx* ctx, const void* w, const float* x, float* y, uint32_t out_features,
                    uint32_t in_features, uint32_t batch, kanso_stream_t stream) {
    int rc = check_gemv(ctx, w, x, y, out_features, in_features, batch, 256, "kanso_gemv_q4_k");
    if (rc) return rc;
    hipStream_t s = as_stream(stream);
    const uint32_t grid = (out_features + kRowsPerBlock - 1) / kRowsPerBlock;
    hipEvent_t ev;
    if ((rc = prof_begin(ctx, "gemv", s, &ev))) return rc;
    for (uint32_t b0 = 0; b0 < batch; b0 += kBatchChunk) {
        const uint32_t bn = std::min<uint32_t>(kBatchChunk, batch - b0);
        if (bn <= 1)
            hipLaunchKernelGGL(gemv_q4_k_kernel<1>, dim3(grid), dim3(kGemvThreads), 0, s,
                               static_cast<const uint8_t*>(w), x, y, out_features, in_features, b0, bn);
        else if (bn <= 4)
            hipLaunchKernelGGL(gemv_q4_k_kernel<4>, dim3(grid), dim3(kGemvThreads), 0, s,
                               static_cast<const uint8_t*>(w), x, y, out_features, in_features, b0, bn);
        else
            hipLaunchKernelGGL(gemv_q4_k_kernel<8>, dim3(grid), dim3(kGemvThreads), 0, s,
                               static_cast<const uint8_t*>(w), x, y, out_features, in_features, b0, bn);
        KANSO_LAUNCH_CHECK();
    }
    return prof_end(ctx, "gemv", s, ev);
}

}  // extern "C"
