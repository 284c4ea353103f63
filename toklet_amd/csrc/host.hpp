// host.hpp - host-side internals shared by the C ABI translation units:
// error reporting in the reference's check order, the context and the KV
// owner objects behind the opaque handles of include/tokhip.h.
#pragma once
#include <hip/hip_runtime.h>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "../../include/tokhip.h"
#include "device.hpp"

namespace tkh_host {

inline constexpr int kSlots = 16;
inline constexpr int kSlotProblems = 1024;

// ---------------------------------------------------------------- errors

inline uint32_t fail(tkh_error *err, uint32_t code, const char *tensor, uint64_t index,
              uint64_t expected, uint64_t actual, const char *fmt, ...) {
    if (err) {
        err->code = code;
        err->index = index;
        err->expected = expected;
        err->actual = actual;
        std::snprintf(err->tensor, sizeof err->tensor, "%s", tensor ? tensor : "");
        va_list ap;
        va_start(ap, fmt);
        std::vsnprintf(err->message, sizeof err->message, fmt, ap);
        va_end(ap);
    }
    return code;
}

inline uint32_t ok(tkh_error *err) {
    if (err) {
        std::memset(err, 0, sizeof *err);
    }
    return TKH_OK;
}

#define TRY(expr)                          \
    do {                                   \
        uint32_t _rc = (expr);             \
        if (_rc != TKH_OK) return _rc;     \
    } while (0)

// src/cpu/mod.rs:84-114 restated for the C ABI.
inline uint32_t nonzero(uint64_t value, const char *name, tkh_error *err) {
    if (value == 0) return fail(err, TKH_ZERO_DIMENSION, name, 0, 0, 0, "%s must be nonzero", name);
    return TKH_OK;
}
inline uint32_t product(uint64_t a, uint64_t b, uint64_t *out, tkh_error *err) {
    if (__builtin_mul_overflow(a, b, out))
        return fail(err, TKH_SIZE_OVERFLOW, nullptr, 0, 0, 0, "tensor size arithmetic overflow");
    return TKH_OK;
}
inline uint32_t add(uint64_t a, uint64_t b, uint64_t *out, tkh_error *err) {
    if (__builtin_add_overflow(a, b, out))
        return fail(err, TKH_SIZE_OVERFLOW, nullptr, 0, 0, 0, "tensor size arithmetic overflow");
    return TKH_OK;
}
inline uint32_t length(const char *tensor, uint64_t actual, uint64_t expected, tkh_error *err) {
    if (actual != expected)
        return fail(err, TKH_LENGTH, tensor, 0, expected, actual, "%s length is %llu, expected %llu",
                    tensor, (unsigned long long)actual, (unsigned long long)expected);
    return TKH_OK;
}
inline uint32_t invalid(const char *what, tkh_error *err) {
    return fail(err, TKH_INVALID_PARAMETER, what, 0, 0, 0, "invalid parameter: %s", what);
}
inline uint32_t device_error(hipError_t e, const char *where, tkh_error *err) {
    return fail(err, TKH_DEVICE, where, 0, 0, 0, "%s: %s", where, hipGetErrorString(e));
}

#define HIP_TRY(call, where)                                  \
    do {                                                      \
        hipError_t _e = (call);                               \
        if (_e != hipSuccess) return device_error(_e, where, err); \
    } while (0)

inline int esize(tkh_dtype dt) { return dt == TKH_F32 ? 4 : 2; }
inline bool valid_dtype(uint32_t dt) { return dt <= TKH_BF16; }

inline int env_int(const char *name, int fallback) {
    const char *v = std::getenv(name);
    return v && *v ? std::atoi(v) : fallback;
}

}  // namespace tkh_host
using namespace tkh_host;

// ---------------------------------------------------------------- context

struct tkh_context {
    int device = 0;
    hipStream_t stream = nullptr;
    bool synchronous = true;
    uint32_t *status_dev = nullptr;
    uint32_t *status_host = nullptr;
    uint8_t *workspace = nullptr;
    size_t workspace_bytes = 0;
    tkh::Problem *ring_dev = nullptr;
    tkh::Problem *ring_host = nullptr;
    tkh::Problem *batch_store = nullptr;  // kSlotProblems: the batched entry points' plans
    hipEvent_t ring_events[kSlots] = {};
    bool ring_used[kSlots] = {};
    int ring_next = 0;
    int split_keys_override = 0;
    int force_generic = 0;
    int decode_waves = 8;        // waves per decode workgroup
    int decode_keys_per_lane = 4;  // keys each lane holds per streamed block
    int cus = 256;               // compute units of the device
    int decode_groups = 256;     // target decode workgroups per launch (little work)
    int decode_bulk_groups = 2048;  // ... when the launch has much work of mixed lengths
    int decode_even_groups = 256;   // ... when the launch has much work of even length
    int decode_bulk_waves = 4;   // waves per decode workgroup when the launch has much work
    int decode_even_waves = 8;   // ... much work of even length
    int decode_even_keys_per_lane = 2;  // keys per lane per block, much work of even length
    int decode_bulk_keys = 2048; // keys x KV heads per CU from which a launch has much work
    int decode_stream_nt = -1;   // nontemporal K/V loads: -1 with much work only, 0 never, 1 always
    int decode_max_splits = 64;  // cap on key splits per KV head (bounds the merge)
    int decode_disable = 0;
    bool decode_merge_launch = true;  // single-problem, latency-bound decode: combine in a second launch
    bool decode_merge_batch = false;  // compact-batch decode: combine in a second launch
    uint32_t epoch = 0;          // last decode split-K epoch handed out
    uint64_t split_wait_ticks = 50000000;  // bound of a decode merge's wait for its splits
    bool test_flag_skew = false; // test hook: merges wait for a flag value no split stores
    int prefill_groups = 128;    // below this many row-block workgroups (128-row units), split the keys
    int prefill_fill_groups = 512;  // row-block workgroups (128-row units) from which eight-wave ones fill the device
    int prefill_max_splits = 16;
    int prefill_min_keys = 64;   // keys per split at least
    int prefill_waves = 0;       // waves per prefill workgroup: 0 = chosen per launch, 4 or 8
    bool prefill_compact = true; // chunks of one shape carried in the kernel arguments (no upload)
    int prefill16 = 1;           // four-wave launches at head_dim 128/256 on the 16-row kernel (0: never)
    int prefill16_groups = 64;   // split target of the 16-row kernel's launches (in 128-row workgroups)
    int prefill16_waves = 4;     // 16-row waves per workgroup: 4 (64-row blocks) or 8 (128-row blocks)
    // profiling: per launch, start/stop of the attention kernel and of the combine kernel
    bool profiling = false;
    std::vector<hipEvent_t> prof_events;
    std::vector<char> prof_has_combine;
    size_t prof_used = 0;
    uint64_t prof_launches = 0;
    double prof_attention_ms = 0, prof_combine_ms = 0;
};

// The workspace halves: split-K partials of the prefill and generic kernels
// in the lower half, the decode kernel's tagged partials in the upper half
// (kept apart so no other kernel's bits can pass for a decode tag).
inline size_t split_region_bytes(const tkh_context *ctx) { return ctx->workspace_bytes / 2; }
inline size_t decode_region_offset(const tkh_context *ctx) {
    return (ctx->workspace_bytes / 2 + 255) / 256 * 256;
}
inline uint8_t *decode_region(const tkh_context *ctx) { return ctx->workspace + decode_region_offset(ctx); }
inline size_t decode_region_bytes(const tkh_context *ctx) {
    const size_t off = decode_region_offset(ctx);
    return off < ctx->workspace_bytes ? (ctx->workspace_bytes - off) / 8 * 8 : 0;
}

struct tkh_kv {
    tkh_context *ctx = nullptr;
    int device = 0;
    uint64_t heads = 0, dims = 0, capacity = 0, max_positions = 0;
    bool has_window = false;
    uint64_t window = 0;
    tkh_dtype storage = TKH_BF16;
    void *k = nullptr;
    void *v = nullptr;
    uint64_t offset = 0, generation = 0, owner = 0;
    uint64_t allocated_bytes = 0;
};

namespace tkh_host {
// attention_cached of one token with the producer folded into the decode
// kernel (api.cpp); used by the session for decode steps.
uint32_t attention_cached_fused(tkh_context *ctx, const tkh_cached_shape *shape, tkh_dtype dtype,
                                const void *k, const void *v, float *context,
                                const tkh::FusedDecode &fused, tkh_error *err);
// span_attention of one token (the last key of the view) with the producer
// folded into the decode kernel: the session's decode steps of layers with a
// score scale, softcap or window, and of ring caches (the new K/V row goes to
// the layer's staging row, fused.new_row 0).
uint32_t span_attention_fused(tkh_context *ctx, const tkh_span_shape *shape, tkh_dtype dtype,
                              const tkh_segment segments[3], float *context,
                              const tkh::FusedDecode &fused, tkh_error *err);
// tkh_kv_commit_batch with an optional device gate (api.cpp).
uint32_t commit_frames(tkh_kv *const *kvs, const tkh_kv_frame *frames, uint64_t count,
                       const uint32_t *gate, uint64_t *committed, uint64_t committed_value,
                       tkh_error *err);
}  // namespace tkh_host
