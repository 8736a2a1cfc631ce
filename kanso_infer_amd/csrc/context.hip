// context.hip — kanso_ctx lifetime, error reporting, scratch, status word and
// kernel timing (HIP events on the launch stream).
#include <cstdarg>
#include <cstring>

#include "common.hpp"

namespace kanso {

static thread_local std::string g_last_error;

void set_error(const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
}

int ensure_scratch(kanso_ctx* ctx, size_t bytes) {
    if (bytes <= ctx->scratch_bytes) return KANSO_OK;
    size_t want = align_up(bytes + bytes / 2, 1 << 20);
    if (ctx->scratch) {
        KANSO_HIP_TRY(hipDeviceSynchronize());
        KANSO_HIP_TRY(hipFree(ctx->scratch));
        ctx->scratch = nullptr;
        ctx->scratch_bytes = 0;
    }
    KANSO_HIP_TRY(hipMalloc(&ctx->scratch, want));
    ctx->scratch_bytes = want;
    return KANSO_OK;
}

int ensure_keys(kanso_ctx* ctx, size_t bytes) {
    if (bytes <= ctx->keys_bytes) return KANSO_OK;
    size_t want = align_up(bytes + bytes / 2, 1 << 16);
    if (ctx->keys) {
        KANSO_HIP_TRY(hipDeviceSynchronize());
        KANSO_HIP_TRY(hipFree(ctx->keys));
        ctx->keys = nullptr;
        ctx->keys_bytes = 0;
    }
    KANSO_HIP_TRY(hipMalloc(&ctx->keys, want));
    ctx->keys_bytes = want;
    return KANSO_OK;
}

static int pooled_event(kanso_ctx* ctx, hipEvent_t* ev) {
    if (!ctx->event_pool.empty()) {
        *ev = ctx->event_pool.back();
        ctx->event_pool.pop_back();
        return KANSO_OK;
    }
    KANSO_HIP_TRY(hipEventCreate(ev));
    return KANSO_OK;
}

int prof_begin(kanso_ctx* ctx, const char* name, hipStream_t stream, hipEvent_t* start) {
    (void)name;
    *start = nullptr;
    if (!ctx->profiling) return KANSO_OK;
    int rc = pooled_event(ctx, start);
    if (rc) return rc;
    KANSO_HIP_TRY(hipEventRecord(*start, stream));
    return KANSO_OK;
}

int prof_end(kanso_ctx* ctx, const char* name, hipStream_t stream, hipEvent_t start) {
    if (!ctx->profiling || !start) return KANSO_OK;
    hipEvent_t stop;
    int rc = pooled_event(ctx, &stop);
    if (rc) return rc;
    KANSO_HIP_TRY(hipEventRecord(stop, stream));
    ctx->pending.push_back(ProfileRecord{name, start, stop});
    return KANSO_OK;
}

static int resolve_profiles(kanso_ctx* ctx) {
    for (auto& rec : ctx->pending) {
        KANSO_HIP_TRY(hipEventSynchronize(rec.stop));
        float ms = 0.0f;
        KANSO_HIP_TRY(hipEventElapsedTime(&ms, rec.start, rec.stop));
        ProfileTotal* tot = nullptr;
        for (auto& kv : ctx->totals)
            if (kv.first == rec.name) tot = &kv.second;
        if (!tot) {
            ctx->totals.emplace_back(rec.name, ProfileTotal{});
            tot = &ctx->totals.back().second;
        }
        tot->ms += ms;
        tot->launches += 1;
        ctx->event_pool.push_back(rec.start);
        ctx->event_pool.push_back(rec.stop);
    }
    ctx->pending.clear();
    return KANSO_OK;
}

}  // namespace kanso

using namespace kanso;

extern "C" {

const char* kanso_last_error(void) { return g_last_error.c_str(); }

int kanso_create(int device, kanso_ctx** out) {
    if (!out) {
        set_error("kanso_create: out is null");
        return KANSO_E_INVALID_ARG;
    }
    *out = nullptr;
    int count = 0;
    KANSO_HIP_TRY(hipGetDeviceCount(&count));
    if (device < 0 || device >= count) {
        set_error("kanso_create: device %d not present (%d devices)", device, count);
        return KANSO_E_INVALID_ARG;
    }
    KANSO_HIP_TRY(hipSetDevice(device));
    kanso_ctx* ctx = new kanso_ctx();
    ctx->device = device;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) == hipSuccess && prop.multiProcessorCount > 0)
        ctx->num_cus = prop.multiProcessorCount;
    if (hipMalloc(&ctx->status, sizeof(uint32_t)) != hipSuccess ||
        hipMemset(ctx->status, 0, sizeof(uint32_t)) != hipSuccess) {
        set_error("kanso_create: status word allocation failed");
        delete ctx;
        return KANSO_E_HIP;
    }
    if (int rc = noalloc_scratch_init(&ctx->noalloc_scratch)) {
        (void)hipFree(ctx->status);
        delete ctx;
        return rc;
    }

    *out = ctx;
    return KANSO_OK;
}

int kanso_destroy(kanso_ctx* ctx) {
    if (!ctx) return KANSO_OK;
    // Teardown: errors here have no caller to report to, so they are dropped.
    (void)hipDeviceSynchronize();
    for (auto& rec : ctx->pending) {
        (void)hipEventDestroy(rec.start);
        (void)hipEventDestroy(rec.stop);
    }
    if (ctx->scratch) (void)hipFree(ctx->scratch);
    if (ctx->keys) (void)hipFree(ctx->keys);
    if (ctx->status) (void)hipFree(ctx->status);
    for (hipEvent_t e : ctx->event_pool) (void)hipEventDestroy(e);

    delete ctx;
    return KANSO_OK;
}

int kanso_check_device_status(kanso_ctx* ctx, kanso_stream_t stream, uint32_t* flags) {
    if (!ctx) {
        set_error("kanso_check_device_status: null context");
        return KANSO_E_INVALID_ARG;
    }
    uint32_t host = 0;
    hipStream_t s = as_stream(stream);
    KANSO_HIP_TRY(hipMemcpyAsync(&host, ctx->status, sizeof(uint32_t), hipMemcpyDeviceToHost, s));
    KANSO_HIP_TRY(hipStreamSynchronize(s));
    if (flags) *flags = host;
    if (host) {
        KANSO_HIP_TRY(hipMemsetAsync(ctx->status, 0, sizeof(uint32_t), s));
        KANSO_HIP_TRY(hipStreamSynchronize(s));
        std::string msg = "device check failed:";
        if (host & KANSO_DEV_EMPTY_CONTEXT) msg += " context_len must be non-zero;";
        if (host & KANSO_DEV_CONTEXT_OVERFLOW) msg += " context_len exceeds block table capacity;";
        if (host & KANSO_DEV_QUERY_OVERFLOW) msg += " query rows exceed context_len;";
        if (host & KANSO_DEV_TABLE_SHORT) msg += " block table shorter than a position needs;";
        if (host & KANSO_DEV_SLOT_OOB) msg += " slot outside the KV pool;";
        if (host & KANSO_DEV_BLOCK_OOB) msg += " physical block id outside the pool;";
        if (host & KANSO_DEV_POSITION_OOB) msg += " position beyond the RoPE table;";
        if (host & KANSO_DEV_TOKEN_OOB) msg += " token id beyond the vocabulary;";
        if (host & KANSO_DEV_PARTS_OOB) msg += " partition count beyond the partials (work list without a row's items);";
        set_error("%s", msg.c_str());
        return KANSO_E_DEVICE_CHECK;
    }
    return KANSO_OK;
}

int kanso_set_profiling(kanso_ctx* ctx, int enabled) {
    if (!ctx) {
        set_error("kanso_set_profiling: null context");
        return KANSO_E_INVALID_ARG;
    }
    int rc = resolve_profiles(ctx);
    if (rc) return rc;
    ctx->profiling = enabled != 0;
    ctx->totals.clear();
    return KANSO_OK;
}

int kanso_get_kernel_time(kanso_ctx* ctx, const char* name, double* total_ms,
                          uint64_t* launches) {
    if (!ctx || !name) {
        set_error("kanso_get_kernel_time: null argument");
        return KANSO_E_INVALID_ARG;
    }
    int rc = resolve_profiles(ctx);
    if (rc) return rc;
    double ms = 0.0;
    uint64_t n = 0;
    for (auto& kv : ctx->totals)
        if (kv.first == name) {
            ms = kv.second.ms;
            n = kv.second.launches;
        }
    if (total_ms) *total_ms = ms;
    if (launches) *launches = n;
    return KANSO_OK;
}

}  // extern "C"
