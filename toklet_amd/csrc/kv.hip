// kv.hip - device KV ownership kernels and small elementwise operators.
//
//  * kv_append: token-major new rows [tokens, heads, D] (any dtype) into
//    head-major cache rows [offset, offset+tokens) in the storage dtype,
//    rounding to nearest even and flagging non-finite input
//    (LayerKv::append, src/model/cache.rs:64-85).
//  * kv_copy_runs: the ring commit of WindowKvCache::commit_validated
//    (src/model/window_cache.rs:298-321): up to two contiguous row runs per
//    head from the staged chunk [heads, tokens, D] into ring slots.
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

// Element-size generic row copy: runs[r] = {source_row, slot, rows}.
__global__ __launch_bounds__(256) void kv_copy_runs(const uint8_t *src_k, const uint8_t *src_v,
                                                    uint8_t *dst_k, uint8_t *dst_v,
                                                    int64_t tokens, int32_t heads,
                                                    int64_t row_bytes, int64_t capacity,
                                                    int64_t r0_src, int64_t r0_slot,
                                                    int64_t r0_rows, int64_t r1_src,
                                                    int64_t r1_slot, int64_t r1_rows,
                                                    const uint32_t *gate, uint64_t *committed,
                                                    uint64_t committed_value) {
    // Gated commit (queued sessions): nothing is copied once the status word
    // reports a failure in this or an earlier chunk; otherwise the session's
    // device-side committed length moves to the end of this chunk.
    if (gate && *(volatile const uint32_t *)gate != 0) return;
    if (committed && blockIdx.x == 0 && threadIdx.x == 0) *committed = committed_value;
    const int64_t words = row_bytes / 2;  // rows are whole 2-byte units
    const int64_t rows = r0_rows + r1_rows;
    const int64_t total = (int64_t)heads * rows * words;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        int64_t w = i % words;
        int64_t r = (i / words) % rows;
        int64_t h = i / (words * rows);
        int64_t srow = r < r0_rows ? r0_src + r : r1_src + (r - r0_rows);
        int64_t slot = r < r0_rows ? r0_slot + r : r1_slot + (r - r0_rows);
        int64_t s = ((h * tokens + srow) * row_bytes) / 2 + w;
        int64_t d = ((h * capacity + slot) * row_bytes) / 2 + w;
        reinterpret_cast<uint16_t *>(dst_k)[d] = reinterpret_cast<const uint16_t *>(src_k)[s];
        reinterpret_cast<uint16_t *>(dst_v)[d] = reinterpret_cast<const uint16_t *>(src_v)[s];
    }
}

// kv_copy_runs for several rings at once: blockIdx.y is the entry.  The gate
// is read once per workgroup before any copy, so either every entry is
// copied or none is, as with one launch per ring in a row.
__global__ __launch_bounds__(256) void kv_copy_batch(CopyBatch b) {
    if (b.gate && *(volatile const uint32_t *)b.gate != 0) return;
    if (b.committed && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0)
        *b.committed = b.committed_value;
    const CopyRunsEntry &e = b.e[blockIdx.y];
    const int64_t words = e.row_bytes / 2;
    const int64_t r0_rows = e.runs[2], rows = e.runs[2] + e.runs[5];
    const int64_t total = (int64_t)e.heads * rows * words;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t w = i % words;
        const int64_t r = (i / words) % rows;
        const int64_t h = i / (words * rows);
        const int64_t srow = r < r0_rows ? e.runs[0] + r : e.runs[3] + (r - r0_rows);
        const int64_t slot = r < r0_rows ? e.runs[1] + r : e.runs[4] + (r - r0_rows);
        const int64_t sidx = ((h * e.tokens + srow) * e.row_bytes) / 2 + w;
        const int64_t didx = ((h * e.capacity + slot) * e.row_bytes) / 2 + w;
        reinterpret_cast<uint16_t *>(e.dst_k)[didx] = reinterpret_cast<const uint16_t *>(e.src_k)[sidx];
        reinterpret_cast<uint16_t *>(e.dst_v)[didx] = reinterpret_cast<const uint16_t *>(e.src_v)[sidx];
    }
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

extern "C" hipError_t tkh_launch_copy_runs(const void *src_k, const void *src_v, void *dst_k,
                                           void *dst_v, int64_t tokens, int heads,
                                           int64_t row_bytes, int64_t capacity,
                                           const int64_t runs[6], const uint32_t *gate,
                                           uint64_t *committed, uint64_t committed_value,
                                           hipStream_t stream) {
    const int64_t rows = runs[2] + runs[5];
    if (rows == 0 && !committed) return hipSuccess;
    dim3 grid(rows ? grid_for(heads * rows * (row_bytes / 2)) : 1), block(256);
    hipLaunchKernelGGL(kv_copy_runs, grid, block, 0, stream, (const uint8_t *)src_k,
                       (const uint8_t *)src_v, (uint8_t *)dst_k, (uint8_t *)dst_v, tokens, heads,
                       row_bytes, capacity, runs[0], runs[1], runs[2], runs[3], runs[4], runs[5],
                       gate, committed, committed_value);
    return hipGetLastError();
}

extern "C" hipError_t tkh_launch_copy_batch(const tkh::CopyBatch *b, hipStream_t stream) {
    using namespace tkh;
    if (b->count < 1 || b->count > COPY_BATCH_MAX) return hipErrorInvalidValue;
    int64_t most = 1;
    for (int i = 0; i < b->count; ++i) {
        const auto &e = b->e[i];
        most = std::max<int64_t>(most, (int64_t)e.heads * (e.runs[2] + e.runs[5]) * (e.row_bytes / 2));
    }
    dim3 grid(grid_for(most), (unsigned)b->count), block(256);
    hipLaunchKernelGGL(kv_copy_batch, grid, block, 0, stream, *b);
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
