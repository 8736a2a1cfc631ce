// gemm.hip — Q8_0 weight products: the reference-format GEMV (GGUF blocks), the
// packed-weight GEMM the decoder uses, and the GGUF -> packed re-layout.
//
// Reference: scalar_gemv_q8_0 / scalar_dot_q8_0 (src/quant/q8_0.rs:51-93) behind
// LinearWeight::forward (src/weights.rs:43-45). The kernel and its arithmetic are
// described in q8_gemm.hpp.
#include "q8_gemm.hpp"

namespace kanso {
namespace {

// One thread per (destination group, block, lane): copies lane l's 8 qs bytes
// (row l%16, k = 8(l/16)) and, for lanes < 16, the row's d.
__global__ __launch_bounds__(256) void pack_q8_0_kernel(const uint8_t* __restrict__ src, uint32_t rows,
                                                        uint32_t nb, uint8_t* __restrict__ dst,
                                                        uint32_t src_groups, uint32_t group_stride,
                                                        uint32_t group_offset) {
    const uint64_t total = static_cast<uint64_t>(src_groups) * nb * kWave;
    for (uint64_t e = blockIdx.x * 256ull + threadIdx.x; e < total; e += static_cast<uint64_t>(gridDim.x) * 256) {
        const uint32_t lane = static_cast<uint32_t>(e % kWave);
        const uint32_t b = static_cast<uint32_t>((e / kWave) % nb);
        const uint32_t g = static_cast<uint32_t>(e / (static_cast<uint64_t>(kWave) * nb));
        const uint32_t row = g * 16 + (lane & 15);
        uint8_t* tile = dst + (static_cast<size_t>(g * group_stride + group_offset) * nb + b) * kPackedTileBytes;
        uint8_t qs[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        uint16_t d = 0;
        if (row < rows) {
            const uint8_t* blk = src + (static_cast<size_t>(row) * nb + b) * 34;
            d = static_cast<uint16_t>(blk[0] | (blk[1] << 8));
#pragma unroll
            for (int j = 0; j < 8; ++j) qs[j] = blk[2 + 8 * (lane >> 4) + j];
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) tile[8 * lane + j] = qs[j];
        if (lane < 16) {
            tile[512 + 2 * lane] = static_cast<uint8_t>(d & 0xff);
            tile[512 + 2 * lane + 1] = static_cast<uint8_t>(d >> 8);
        }
    }
}

int check_q8(kanso_ctx* ctx, const void* w, const float* x, float* y, uint32_t out_f, uint32_t in_f,
             uint32_t batch, const char* who) {
    if (!ctx || !w || !x || !y) {
        set_error("%s: null argument", who);
        return KANSO_E_INVALID_ARG;
    }
    if (out_f == 0 || in_f == 0 || in_f % 32 != 0) {
        set_error("%s: in_features %u must be a non-zero multiple of 32 (out_features %u)", who, in_f, out_f);
        return KANSO_E_INVALID_SHAPE;
    }
    if (batch == 0) {
        set_error("%s: batch must be >= 1", who);
        return KANSO_E_INVALID_SHAPE;
    }
    if (reinterpret_cast<uintptr_t>(x) % 16 != 0) {
        set_error("%s: x must be 16-byte aligned", who);
        return KANSO_E_INVALID_ARG;
    }
    return KANSO_OK;
}

}  // namespace
}  // namespace kanso

using namespace kanso;

extern "C" {

size_t kanso_q8_0_packed_bytes(uint32_t rows, uint32_t in_features) {
    const size_t groups = (static_cast<size_t>(rows) + 31) / 32 * 2;
    return groups * (in_features / 32) * kPackedTileBytes;
}

int kanso_q8_0_pack(kanso_ctx* ctx, const void* gguf, uint32_t rows, uint32_t in_features, void* packed,
                    uint32_t group_stride, uint32_t group_offset, kanso_stream_t stream) {
    if (!ctx || !gguf || !packed) {
        set_error("kanso_q8_0_pack: null argument");
        return KANSO_E_INVALID_ARG;
    }
    if (rows == 0 || in_features == 0 || in_features % 32 != 0 || group_stride == 0) {
        set_error("kanso_q8_0_pack: rows %u / in_features %u (multiple of 32) / group_stride %u", rows,
                  in_features, group_stride);
        return KANSO_E_INVALID_SHAPE;
    }
    const uint32_t nb = in_features / 32;
    const uint32_t groups = (rows + 15) / 16;
    const uint64_t total = static_cast<uint64_t>(groups) * nb * kWave;
    const uint32_t grid = static_cast<uint32_t>(std::min<uint64_t>((total + 255) / 256, 65536));
    hipLaunchKernelGGL(pack_q8_0_kernel, dim3(grid), dim3(256), 0, as_stream(stream),
                       static_cast<const uint8_t*>(gguf), rows, nb, static_cast<uint8_t*>(packed), groups,
                       group_stride, group_offset);
    KANSO_LAUNCH_CHECK();
    return KANSO_OK;
}

int kanso_gemm_q8_0(kanso_ctx* ctx, const void* packed, const float* x, float* y, uint32_t out_features,
                    uint32_t in_features, uint32_t num_tokens, kanso_stream_t stream) {
    int rc = check_q8(ctx, packed, x, y, out_features, in_features, num_tokens, "kanso_gemm_q8_0");
    if (rc) return rc;
    hipStream_t s = as_stream(stream);
    WPacked wl{static_cast<const uint8_t*>(packed), in_features / 32};
    XIn xa{x, nullptr, nullptr, 0.f, in_features, num_tokens, in_features};
    EpiStore<false> epi{y, out_features, out_features};
    hipEvent_t ev;
    if ((rc = prof_begin(ctx, "gemv", s, &ev))) return rc;
    if ((rc = launch_q8_gemm(wl, xa, epi, (out_features + 31) / 32, s))) return rc;
    return prof_end(ctx, "gemv", s, ev);
}

int kanso_gemv_q8_0(kanso_ctx* ctx, const void* w, const float* x, float* y, uint32_t out_features,
                    uint32_t in_features, uint32_t batch, kanso_stream_t stream) {
    int rc = check_q8(ctx, w, x, y, out_features, in_features, batch, "kanso_gemv_q8_0");
    if (rc) return rc;
    hipStream_t s = as_stream(stream);
    WGguf wl{static_cast<const uint8_t*>(w), in_features / 32, out_features};
    XIn xa{x, nullptr, nullptr, 0.f, in_features, batch, in_features};
    EpiStore<false> epi{y, out_features, out_features};
    hipEvent_t ev;
    if ((rc = prof_begin(ctx, "gemv", s, &ev))) return rc;
    if ((rc = launch_q8_gemm(wl, xa, epi, (out_features + 31) / 32, s))) return rc;
    return prof_end(ctx, "gemv", s, ev);
}

}  // extern "C"
