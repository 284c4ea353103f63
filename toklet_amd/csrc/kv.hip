// kv.hip - device KV ownership kernels and small elementwise operators.
//
//  * kv_append: token-major new rows [tokens, heads, D] (any dtype) into
//    head-major cache rows [offset, offset+tokens) in the storage dtype,
//    rounding to nearest even and flagging non-finite input
//    (LayerKv::append, src/model/cache.rs:64-85).
//  * kv_copy_batch: the ring commits of WindowKvCache::commit_validated
//    (src/model/window_cache.rs:298-321), every sliding layer of a chunk in
//    one launch: up to two contiguous row runs per head from the staged
//    chunk [heads, tokens, D] into ring slots.
//  * check_finite: finiteness scan of a staged chunk (the device half of
//    WindowKvCache::prepare's finite() checks, src/model/window_cache.rs:193-212).
//  * logit_softcap: cap * tanh(x / cap) in FP64, rounded once to FP32
//    (src/cpu/softcap.rs:16-29).
//  * convert: FP32 -> storage dtype rounding for callers that hold FP32 rows.
#include <algorithm>

#include "device.hpp"

namespace tkh {

template <int DT> __device__ __forceinline__ void store_elem(void *base, int64_t i, float x);
template <> __device__ __forceinline__ void store_elem<F32>(void *base, int64_t i, float x) {
    reinterpret_cast<float *>(base)[i] = x;
}
template <> __device__ __forceinline__ void store_elem<F16>(void *base, int64_t i, float x) {
    reinterpret_cast<_Float16 *>(base)[i] = (_Float16)x;
}
template <> __device__ __forceinline__ void store_elem<BF16>(void *base, int64_t i, float x) {
    reinterpret_cast<uint16_t *>(base)[i] = f32_to_bf16_bits(x);
}

__device__ __forceinline__ void flag(uint32_t *status, bool bad, uint32_t bit) {
    uint64_t m = __ballot(bad);
    if (m != 0 && (threadIdx.x & 63) == (int)__builtin_ctzll(m)) atomicOr(status, bit);
}

template <int SRC, int DST>
__global__ __launch_bounds__(256) void kv_append(const void *k, const void *v, void *kc, void *vc,
                                                 int64_t tokens, int32_t heads, int32_t dims,
                                                 int64_t capacity, int64_t offset,
                                                 uint32_t *status) {
    const int64_t total = tokens * heads * dims;
    bool bad = false;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        int64_t f = i % dims;
        int64_t hd = (i / dims) % heads;
        int64_t t = i / ((int64_t)dims * heads);
        int64_t dst = (hd * capacity + offset + t) * dims + f;
        float a = load_elem<SRC>(k, i), b = load_elem<SRC>(v, i);
        bad |= !is_finite_f(a) || !is_finite_f(b);
        store_elem<DST>(kc, dst, a);
        store_elem<DST>(vc, dst, b);
    }
    flag(status, bad, ST_NONFINITE_INPUT);
}

// The ring commits of one chunk in one launch, WindowKvCache::commit_validated
// (src/model/window_cache.rs:298-321) for every sliding layer: blockIdx.y is
// the entry, whose staged rows [heads, tokens, row] go to up to two runs of
// ring slots, runs {source row, slot, rows}.  A thread copies one UNIT-byte
// piece of a row (16 when every row is whole 16-byte pieces, else 2), with
// 32-bit index arithmetic when the pieces fit.  Gated commit (queued
// sessions): the status word is read together with the rows, and nothing is
// stored when it reports a failure in this or an earlier chunk, so either
// every entry is copied or none is; otherwise the session's device-side
// committed length moves to the end of this chunk.  (The first form copied
// 2-byte elements with 64-bit divisions per element and read the gate before
// the rows: 4.1 us per commit at configs[3].)
template <int UNIT> struct Piece;
template <> struct Piece<16> { using T = u32x4; };
template <> struct Piece<2> { using T = uint16_t; };

// The gate of ungated commits: a zero word, so that the gate is always read
// through a valid pointer and waited for only at the stores.
__device__ const uint32_t kv_open_gate = 0u;

constexpr int COPY_THREADS = 256;  // kv_copy_batch's workgroup size

template <int UNIT>
__global__ __launch_bounds__(COPY_THREADS) void kv_copy_batch(CopyBatch b) {
    using T = typename Piece<UNIT>::T;
    // Every argument field the copy needs, read before the first use of any:
    // left to itself the compiler read them in several dependent batches
    // (gate pointer, entry, run bounds), each a wait on a kernel-argument line.
    // The grid size (a hidden argument on a line of its own) joins the batch.
    CopyRunsEntry e = b.e[blockIdx.y];
    const uint32_t *gate = b.gate ? b.gate : &kv_open_gate;
    uint64_t *committed = b.committed;
    uint64_t committed_value = b.committed_value;
    uint32_t nblocks = gridDim.x;
    pin_args(e.src_k, e.src_v, e.dst_k, e.dst_v, e.tokens, e.row_bytes, e.capacity, e.runs[0], e.runs[1],
             e.runs[2], e.runs[3], e.runs[4], e.runs[5], e.heads, gate, committed, committed_value, nblocks);
    // Written by earlier launches on the stream (visible at this launch's
    // start).  The compiler tests it once, before the copy loop.
    const uint32_t g = *gate;
    const int64_t per_row = e.row_bytes / UNIT;
    const int64_t r0_rows = e.runs[2], rows = e.runs[2] + e.runs[5];
    const int64_t total = (int64_t)e.heads * rows * per_row;
    const bool narrow = total <= 0x7fffffff;
    for (int64_t i = (int64_t)blockIdx.x * COPY_THREADS + threadIdx.x; i < total;
         i += (int64_t)nblocks * COPY_THREADS) {
        int64_t c, r, h;
        if (narrow) {
            const uint32_t i32 = (uint32_t)i, pr = (uint32_t)per_row, rs = (uint32_t)rows;
            const uint32_t row = i32 / pr;
            c = i32 - row * pr;
            h = row / rs;
            r = row - (uint32_t)h * rs;
        } else {
            const int64_t row = i / per_row;
            c = i - row * per_row;
            h = row / rows;
            r = row - h * rows;
        }
        const int64_t srow = r < r0_rows ? e.runs[0] + r : e.runs[3] + (r - r0_rows);
        const int64_t slot = r < r0_rows ? e.runs[1] + r : e.runs[4] + (r - r0_rows);
        const int64_t s = (h * e.tokens + srow) * per_row + c;
        const int64_t d = (h * e.capacity + slot) * per_row + c;
        const T kx = reinterpret_cast<const T *>(e.src_k)[s];
        const T vx = reinterpret_cast<const T *>(e.src_v)[s];
        if (g == 0) {
            reinterpret_cast<T *>(e.dst_k)[d] = kx;
            reinterpret_cast<T *>(e.dst_v)[d] = vx;
        }
    }
    if (committed && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0 && g == 0)
        *committed = committed_value;
}

template <int DT>
__global__ __launch_bounds__(256) void check_finite(const void *a, const void *b, int64_t n,
                                                    uint32_t *status) {
    bool bad = false;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        bad |= !is_finite_f(load_elem<DT>(a, i)) || !is_finite_f(load_elem<DT>(b, i));
    flag(status, bad, ST_NONFINITE_INPUT);
}

// Single block: the whole input is checked (block-wide OR) before any write,
// as the reference checks finiteness before writing (src/cpu/softcap.rs:20-23).
__global__ __launch_bounds__(256) void logit_softcap(float *x, int64_t n, float cap,
                                                     uint32_t *status) {
    const double c = (double)cap;
    int bad = 0;
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) bad |= !is_finite_f(x[i]);
    bad = __syncthreads_or(bad);
    if (bad) {
        if (threadIdx.x == 0) atomicOr(status, (uint32_t)ST_NONFINITE_INPUT);
        return;
    }
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x)
        x[i] = (float)(tanh((double)x[i] / c) * c);
}

template <int DT>
__global__ __launch_bounds__(256) void convert_from_f32(const float *src, void *dst, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        store_elem<DT>(dst, i, src[i]);
}

__global__ void fill_u32(uint32_t *p, uint32_t v) { *p = v; }
__global__ void fill_u64(uint64_t *p, uint64_t v) { *p = v; }
__global__ __launch_bounds__(256) void zero_u64(uint64_t *p, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        p[i] = 0;
}

}  // namespace tkh

using namespace tkh;

static unsigned grid_for(int64_t n) {
    int64_t g = (n + 255) / 256;
    if (g < 1) g = 1;
    if (g > 8192) g = 8192;
    return (unsigned)g;
}

extern "C" hipError_t tkh_launch_kv_append(int src, int dst, const void *k, const void *v,
                                           void *kc, void *vc, int64_t tokens, int heads,
                                           int dims, int64_t capacity, int64_t offset,
                                           uint32_t *status, hipStream_t stream) {
    dim3 grid(grid_for(tokens * heads * dims)), block(256);
#define TKH_APPEND(S, D)                                                                      \
    if (src == S && dst == D) {                                                               \
        hipLaunchKernelGGL((kv_append<S, D>), grid, block, 0, stream, k, v, kc, vc, tokens,   \
                           heads, dims, capacity, offset, status);                            \
        return hipGetLastError();                                                             \
    }
    TKH_APPEND(F32, F32) TKH_APPEND(F32, F16) TKH_APPEND(F32, BF16)
    TKH_APPEND(F16, F16) TKH_APPEND(BF16, BF16)
#undef TKH_APPEND
    return hipErrorInvalidValue;
}

extern "C" hipError_t tkh_launch_copy_batch(const tkh::CopyBatch *b, hipStream_t stream) {
    using namespace tkh;
    if (b->count < 1 || b->count > COPY_BATCH_MAX) return hipErrorInvalidValue;
    // 16-byte pieces when every row and base allows them.
    bool vec = true;
    for (int i = 0; i < b->count; ++i) {
        const auto &e = b->e[i];
        const uintptr_t bases = (uintptr_t)e.src_k | (uintptr_t)e.src_v | (uintptr_t)e.dst_k |
                                (uintptr_t)e.dst_v;
        vec = vec && e.row_bytes % 16 == 0 && bases % 16 == 0;
    }
    const int64_t unit = vec ? 16 : 2;
    int64_t most = 1;
    for (int i = 0; i < b->count; ++i) {
        const auto &e = b->e[i];
        most = std::max<int64_t>(most, (int64_t)e.heads * (e.runs[2] + e.runs[5]) * (e.row_bytes / unit));
    }
    dim3 grid(grid_for(most), (unsigned)b->count), block(COPY_THREADS);
    if (vec) hipLaunchKernelGGL(kv_copy_batch<16>, grid, block, 0, stream, *b);
    else hipLaunchKernelGGL(kv_copy_batch<2>, grid, block, 0, stream, *b);
    return hipGetLastError();
}

extern "C" hipError_t tkh_launch_check_finite(int dtype, const void *a, const void *b, int64_t n,
                                              uint32_t *status, hipStream_t stream) {
    dim3 grid(grid_for(n)), block(256);
    if (dtype == F32) hipLaunchKernelGGL((check_finite<F32>), grid, block, 0, stream, a, b, n, status);
    else if (dtype == F16) hipLaunchKernelGGL((check_finite<F16>), grid, block, 0, stream, a, b, n, status);
    else if (dtype == BF16) hipLaunchKernelGGL((check_finite<BF16>), grid, block, 0, stream, a, b, n, status);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

extern "C" hipError_t tkh_launch_softcap(float *x, int64_t n, float cap, uint32_t *status,
                                         hipStream_t stream) {
    hipLaunchKernelGGL(logit_softcap, dim3(1), dim3(256), 0, stream, x, n, cap, status);
    return hipGetLastError();
}

extern "C" hipError_t tkh_launch_convert(int dtype, const float *src, void *dst, int64_t n,
                                         hipStream_t stream) {
    dim3 grid(grid_for(n)), block(256);
    if (dtype == F16) hipLaunchKernelGGL((convert_from_f32<F16>), grid, block, 0, stream, src, dst, n);
    else if (dtype == BF16) hipLaunchKernelGGL((convert_from_f32<BF16>), grid, block, 0, stream, src, dst, n);
    else if (dtype == F32) hipLaunchKernelGGL((convert_from_f32<F32>), grid, block, 0, stream, src, dst, n);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

extern "C" hipError_t tkh_launch_fill_u64(uint64_t *p, uint64_t v, hipStream_t stream) {
    hipLaunchKernelGGL(fill_u64, dim3(1), dim3(1), 0, stream, p, v);
    return hipGetLastError();
}

// Zero `words` 8-byte words (a kernel rather than a memset node, so the
// clear also behaves inside a captured graph).
extern "C" hipError_t tkh_launch_zero_u64(uint64_t *p, int64_t words, hipStream_t stream) {
    if (words <= 0) return hipSuccess;
    const int64_t blocks = std::min<int64_t>((words + 255) / 256, 4096);
    hipLaunchKernelGGL(zero_u64, dim3((unsigned)blocks), dim3(256), 0, stream, p, words);
    return hipGetLastError();
}

extern "C" hipError_t tkh_launch_fill_u32(uint32_t *p, uint32_t v, hipStream_t stream) {
    hipLaunchKernelGGL(fill_u32, dim3(1), dim3(1), 0, stream, p, v);
    return hipGetLastError();
}
