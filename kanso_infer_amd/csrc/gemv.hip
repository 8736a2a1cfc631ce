// gemv.hip — dequant-on-the-fly GEMV / small GEMM over GGUF Q4_K weights (the
// Q8_0 products live in gemm.hip; both run the matrix-core kernel of q8_gemm.hpp).
//
// Reference: scalar_gemv_q4_k (src/quant/q4_k.rs:162-186): out[r] = sum over
// blocks of the dequantized weights times x, f32 accumulation; a batch of b
// activation rows is b GEMVs. Production reads candle's GGUF blocks (f16 d / dmin:
// 144 B), which is what this kernel consumes (src/quant/mod.rs:1-17).
//
// Arithmetic: a 32-element sub-block has weights d1 * q - m1 with q a nibble, so
// sum w x = d1 (sum q x) - m1 (sum x): nibbles are exact in bf16 and both sums come
// from the bf16 hi / lo products of q8_gemm_kernel (WQ4K loader).
#include "q8_gemm.hpp"

namespace kanso {
namespace {

int check_q4k(kanso_ctx* ctx, const void* w, const float* x, float* y, uint32_t out_f, uint32_t in_f,
              uint32_t batch) {
    if (!ctx || !w || !x || !y) {
        set_error("kanso_gemv_q4_k: null argument");
        return KANSO_E_INVALID_ARG;
    }
    if (out_f == 0 || in_f == 0 || in_f % 256 != 0) {
        set_error("kanso_gemv_q4_k: in_features %u must be a non-zero multiple of 256 (out_features %u)", in_f,
                  out_f);
        return KANSO_E_INVALID_SHAPE;
    }
    if (batch == 0) {
        set_error("kanso_gemv_q4_k: batch must be >= 1");
        return KANSO_E_INVALID_SHAPE;
    }
    if (reinterpret_cast<uintptr_t>(x) % 16 != 0 || reinterpret_cast<uintptr_t>(w) % 16 != 0) {
        set_error("kanso_gemv_q4_k: x and w must be 16-byte aligned");
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
    int rc = check_q4k(ctx, w, x, y, out_features, in_features, batch);
    if (rc) return rc;
    hipStream_t s = as_stream(stream);
    WQ4K wl{static_cast<const uint8_t*>(w), in_features / 256, out_features};
    XIn xa{x, nullptr, nullptr, 0.f, in_features, batch, in_features};
    EpiStore<false> epi{y, out_features, out_features};
    hipEvent_t ev;
    if ((rc = prof_begin(ctx, "gemv", s, &ev))) return rc;
    if ((rc = launch_q8_gemm(wl, xa, epi, (out_features + 31) / 32, s))) return rc;
    return prof_end(ctx, "gemv", s, ev);
}

}  // extern "C"
