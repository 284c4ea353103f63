// Host-allocation and device-memory check of a session's steady state, the
// sequence of the reference's admitted_prefill_decode_and_reuse_allocate_no_buffers
// (tests/session.rs:715-744) run through the C ABI: after tkh_session_create,
// set_tokens + evaluate twice, eight decode steps (append one token + evaluate),
// append + discard_pending, set_tokens + evaluate, reset, append + evaluate.
//
// This program interposes malloc, calloc, realloc and every operator new, and
// counts the calls whose caller is code of libtokhip.so (the HIP runtime's own
// allocations are not the library's).  It runs the sequence on a synchronous
// and on a queued context (two layers: a full one and a ring of window 4), after
// one warm-up pass per context on a separate session (the runtime's lazy device
// allocations), and reports the counted calls, the session's memory accounting
// and the device's free memory (hipMemGetInfo) before and after.  Exit status 0:
// no counted allocation and nothing changed.  Test infrastructure: pytest runs it
// as a child process on the GPU box.
#include <dlfcn.h>
#include <link.h>
#include <hip/hip_runtime_api.h>

#include <atomic>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <new>
#include <vector>

#include "tokhip.h"

extern "C" void *__libc_malloc(size_t);
extern "C" void *__libc_calloc(size_t, size_t);
extern "C" void *__libc_realloc(void *, size_t);
extern "C" void *__libc_memalign(size_t, size_t);

namespace {

struct Range {
    uintptr_t lo, hi;
};
Range g_text[8];
int g_ntext = 0;
std::atomic<bool> g_track{false};
std::atomic<int> g_count{0};
void *g_sites[32];

inline void note(void *caller) {
    if (!g_track.load(std::memory_order_relaxed)) return;
    const uintptr_t a = reinterpret_cast<uintptr_t>(caller);
    for (int i = 0; i < g_ntext; ++i) {
        if (a >= g_text[i].lo && a < g_text[i].hi) {
            const int n = g_count.fetch_add(1);
            if (n < 32) g_sites[n] = caller;
            return;
        }
    }
}

// The executable segments of the shared object that holds `symbol`.
int find_text(ElfW(Addr) base) {
    struct Ctx {
        ElfW(Addr) base;
    } ctx{base};
    dl_iterate_phdr(
        [](struct dl_phdr_info *info, size_t, void *p) -> int {
            auto *c = static_cast<Ctx *>(p);
            if (info->dlpi_addr != c->base) return 0;
            for (int i = 0; i < info->dlpi_phnum && g_ntext < 8; ++i) {
                const ElfW(Phdr) &ph = info->dlpi_phdr[i];
                if (ph.p_type == PT_LOAD && (ph.p_flags & PF_X))
                    g_text[g_ntext++] = {info->dlpi_addr + ph.p_vaddr,
                                         info->dlpi_addr + ph.p_vaddr + ph.p_memsz};
            }
            return 1;
        },
        &ctx);
    return g_ntext;
}

}  // namespace

extern "C" void *malloc(size_t n) {
    note(__builtin_return_address(0));
    return __libc_malloc(n);
}
extern "C" void *calloc(size_t n, size_t m) {
    note(__builtin_return_address(0));
    return __libc_calloc(n, m);
}
extern "C" void *realloc(void *p, size_t n) {
    note(__builtin_return_address(0));
    return __libc_realloc(p, n);
}
void *operator new(size_t n) {
    note(__builtin_return_address(0));
    if (void *p = __libc_malloc(n ? n : 1)) return p;
    throw std::bad_alloc();
}
void *operator new[](size_t n) {
    note(__builtin_return_address(0));
    if (void *p = __libc_malloc(n ? n : 1)) return p;
    throw std::bad_alloc();
}
void *operator new(size_t n, const std::nothrow_t &) noexcept {
    note(__builtin_return_address(0));
    return __libc_malloc(n ? n : 1);
}
void *operator new[](size_t n, const std::nothrow_t &) noexcept {
    note(__builtin_return_address(0));
    return __libc_malloc(n ? n : 1);
}
void *operator new(size_t n, std::align_val_t a) {
    note(__builtin_return_address(0));
    if (void *p = __libc_memalign((size_t)a, n ? n : 1)) return p;
    throw std::bad_alloc();
}
void *operator new[](size_t n, std::align_val_t a) {
    note(__builtin_return_address(0));
    if (void *p = __libc_memalign((size_t)a, n ? n : 1)) return p;
    throw std::bad_alloc();
}
void operator delete(void *p) noexcept { free(p); }
void operator delete[](void *p) noexcept { free(p); }
void operator delete(void *p, size_t) noexcept { free(p); }
void operator delete[](void *p, size_t) noexcept { free(p); }
void operator delete(void *p, std::align_val_t) noexcept { free(p); }
void operator delete[](void *p, std::align_val_t) noexcept { free(p); }
void operator delete(void *p, size_t, std::align_val_t) noexcept { free(p); }
void operator delete[](void *p, size_t, std::align_val_t) noexcept { free(p); }

namespace {

constexpr uint64_t kCap = 32, kChunk = 3, kLayers = 2, kHq = 4, kHkv = 2, kD = 64;

bool ok(uint32_t rc, const tkh_error &e, const char *what) {
    if (rc == TKH_OK) return true;
    std::printf("FAIL %s: code %u %s: %s\n", what, rc, e.tensor, e.message);
    return false;
}

struct Inputs {
    float *proj[kLayers][3] = {};
    float *context[kLayers] = {};
    tkh_layer_io io[kLayers];
};

bool make_inputs(Inputs &in) {
    const uint64_t heads[3] = {kHq, kHkv, kHkv};
    std::vector<float> host(kCap * kHq * kD);
    for (uint64_t l = 0; l < kLayers; ++l) {
        for (int k = 0; k < 3; ++k) {
            const size_t n = kCap * heads[k] * kD;
            for (size_t i = 0; i < n; ++i)
                host[i] = (float)((int)((i * 7 + l * 13 + k * 5) % 29) - 14) / 16.0f;
            if (hipMalloc(&in.proj[l][k], n * sizeof(float)) != hipSuccess) return false;
            if (hipMemcpy(in.proj[l][k], host.data(), n * sizeof(float), hipMemcpyHostToDevice) != hipSuccess)
                return false;
        }
        if (hipMalloc(&in.context[l], kCap * kHq * kD * sizeof(float)) != hipSuccess) return false;
        in.io[l] = tkh_layer_io{in.proj[l][0], in.proj[l][1], in.proj[l][2], nullptr, nullptr, in.context[l]};
    }
    return true;
}

tkh_session_options options() {
    tkh_session_options o{};
    o.capacity = kCap;
    o.prefill_chunk_size = kChunk;
    o.vocab_size = 64;
    o.layers = kLayers;
    o.query_heads = kHq;
    o.kv_heads = kHkv;
    o.head_dim = kD;
    o.storage = TKH_BF16;
    o.score_scale = 0.125f;
    o.norm_epsilon = 1e-6f;
    o.rotary = TKH_ROTARY_SPLIT_HALF;
    o.theta = 10000.0f;
    o.factor = 1.0f;
    o.low_freq_factor = 1.0f;
    o.high_freq_factor = 4.0f;
    o.original_max_positions = 8192;
    return o;
}

// The reference test's sequence (tokens of its tiny vocabulary; the decode
// steps append fixed tokens where the reference appends its greedy pick).
bool sequence(tkh_session *s, const Inputs &in, bool queued) {
    tkh_error e{};
    uint64_t done = 0;
    const uint32_t prompt[4] = {1, 7, 13, 3};
    const uint32_t two[2] = {1, 7}, eleven[1] = {11}, three[3] = {7, 13, 3};
    if (!ok(tkh_session_set_tokens(s, prompt, 4, &e), e, "set_tokens")) return false;
    if (!ok(tkh_session_evaluate(s, in.io, kChunk, &done, &e), e, "evaluate")) return false;
    if (!ok(tkh_session_set_tokens(s, prompt, 4, &e), e, "set_tokens again")) return false;
    if (!ok(tkh_session_evaluate(s, in.io, kChunk, &done, &e), e, "evaluate again")) return false;
    for (uint32_t i = 0; i < 8; ++i) {
        const uint32_t token = 2 + i;
        if (!ok(tkh_session_append(s, &token, 1, &e), e, "append")) return false;
        if (!ok(tkh_session_evaluate(s, in.io, kChunk, &done, &e), e, "decode step")) return false;
    }
    if (!ok(tkh_session_append(s, two, 2, &e), e, "append pending")) return false;
    tkh_session_discard_pending(s);
    if (!ok(tkh_session_set_tokens(s, eleven, 1, &e), e, "set_tokens short")) return false;
    if (!ok(tkh_session_evaluate(s, in.io, kChunk, &done, &e), e, "evaluate short")) return false;
    tkh_session_reset(s);
    if (!ok(tkh_session_append(s, three, 3, &e), e, "append after reset")) return false;
    if (!ok(tkh_session_evaluate(s, in.io, kChunk, &done, &e), e, "evaluate after reset")) return false;
    if (queued && !ok(tkh_session_synchronize(s, &e), e, "synchronize")) return false;
    tkh_session_state st{};
    tkh_session_state_get(s, &st);
    if (st.evaluated_len != 3 || st.pending_len != 0) {
        std::printf("FAIL state: evaluated %llu pending %llu\n", (unsigned long long)st.evaluated_len,
                    (unsigned long long)st.pending_len);
        return false;
    }
    return true;
}

bool run(bool queued, const Inputs &in) {
    const char *label = queued ? "queued" : "synchronous";
    tkh_error e{};
    tkh_context *ctx = nullptr;
    if (!ok(tkh_context_create(0, nullptr, 0, queued ? 0 : 1, &ctx, &e), e, "context")) return false;
    const tkh_session_options o = options();
    const uint64_t windows[kLayers] = {0, 4};
    {
        tkh_session *warm = nullptr;
        if (!ok(tkh_session_create(ctx, &o, windows, &warm, &e), e, "warm-up session")) return false;
        const bool good = sequence(warm, in, queued);
        tkh_session_destroy(warm);
        if (!good) return false;
    }
    tkh_session *s = nullptr;
    if (!ok(tkh_session_create(ctx, &o, windows, &s, &e), e, "session")) return false;
    tkh_session_state before{}, after{};
    tkh_session_state_get(s, &before);
    if (hipDeviceSynchronize() != hipSuccess) return false;
    size_t free0 = 0, free1 = 0, total = 0;
    if (hipMemGetInfo(&free0, &total) != hipSuccess) return false;
    g_count = 0;
    g_track = true;
    const bool good = sequence(s, in, queued);
    g_track = false;
    if (hipDeviceSynchronize() != hipSuccess) return false;
    if (hipMemGetInfo(&free1, &total) != hipSuccess) return false;
    tkh_session_state_get(s, &after);
    const int counted = g_count.load();
    std::printf("%s: %d host allocations by libtokhip, device free memory %zu -> %zu bytes, session "
                "memory %llu+%llu -> %llu+%llu bytes\n",
                label, counted, free0, free1, (unsigned long long)before.kv_bytes,
                (unsigned long long)before.scratch_bytes, (unsigned long long)after.kv_bytes,
                (unsigned long long)after.scratch_bytes);
    for (int i = 0; i < counted && i < 32; ++i) {
        Dl_info info{};
        dladdr(g_sites[i], &info);
        std::printf("  allocation from %s+%#lx\n", info.dli_sname ? info.dli_sname : "?",
                    (unsigned long)((uintptr_t)g_sites[i] - (uintptr_t)(info.dli_saddr ? info.dli_saddr : info.dli_fbase)));
    }
    tkh_session_destroy(s);
    tkh_context_destroy(ctx);
    return good && counted == 0 && free0 == free1 && before.kv_bytes == after.kv_bytes &&
           before.scratch_bytes == after.scratch_bytes;
}

}  // namespace

int main() {
    Dl_info info{};
    if (!dladdr(reinterpret_cast<void *>(&tkh_abi_version), &info) ||
        find_text(reinterpret_cast<ElfW(Addr)>(info.dli_fbase)) == 0) {
        std::printf("FAIL: libtokhip's code segments not found\n");
        return 2;
    }
    std::printf("libtokhip: %s (ABI %u)\n", info.dli_fname, tkh_abi_version());
    Inputs in;
    if (!make_inputs(in)) {
        std::printf("FAIL: device inputs\n");
        return 2;
    }
    const bool a = run(false, in);
    const bool b = run(true, in);
    std::printf("%s\n", a && b ? "OK: no allocation in the steady state" : "FAIL");
    return a && b ? 0 : 1;
}
