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
    // Grow-only auxiliary buffer for small per-call index arrays.
    void* aux = nullptr;
    size_t aux_bytes = 0;
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
int ensure_aux(kanso_ctx* ctx, size_t bytes);

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

__device__ __forceinline__ float wave_xor(float v, int mask) { return __shfl_xor(v, mask, kWave); }

__device__ __forceinline__ void raise_status(uint32_t* status, uint32_t bits) {
    atomicOr(status, bits);
}

}  // namespace kanso
