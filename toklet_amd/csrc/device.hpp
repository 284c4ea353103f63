// device.hpp - shared device-side types of the gfx950 attention kernels.
//
// One "problem" is one causal/sliding GQA attention call: a block of query
// tokens at consecutive absolute positions attending to a logical key range
// made of up to three segments (the reference's AttentionKvSegment triple,
// src/cpu/span_attention.rs:9-16).  A launch covers an array of problems
// (independent sessions) through a flat tile space; each problem records the
// first tile it owns so a wave finds its problem by binary search.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tkh {

enum Dtype : int32_t { F32 = 0, F16 = 1, BF16 = 2 };

// Status bits OR-ed into the per-context device status word.
enum StatusBits : uint32_t {
    ST_NONFINITE_INPUT = 1u,   // a visible score, or a partial context, is not finite
    ST_BAD_MASS = 2u,          // softmax mass not finite or not positive
    ST_NONFINITE_OUTPUT = 4u,  // combined context not finite
};

struct Segment {
    const void *k;
    const void *v;
    int64_t head_stride;  // elements between KV heads
    int64_t row_stride;   // elements between consecutive keys
    int64_t keys;         // rows in this segment
    int64_t start;        // logical index of its first key
};

struct Problem {
    const void *q;        // [queries, Hq, D] (row stride q_row_stride elements)
    float *out;           // [queries, Hq, D] FP32 context
    int64_t q_row_stride;
    int64_t q_pos0;       // absolute position of query 0
    int64_t k_pos0;       // absolute position of logical key 0
    int64_t keys;         // logical keys
    int32_t queries;
    int32_t nseg;
    Segment seg[3];
    int32_t splits;       // key splits
    int32_t split_keys;   // keys per split (multiple of the key tile)
    int32_t row_blocks;   // row blocks per KV head (MFMA path)
    int32_t pad0;
    int64_t tile_base;    // first global tile of this problem
    int64_t part_base;    // first output row (rows are query*Hq + head)
    int64_t slot_base;    // first split-K partial slot (row-major [rows, splits])
};

struct Params {
    const Problem *problems;
    int32_t nproblems;
    int32_t query_heads;
    int32_t kv_heads;
    int32_t head_dim;
    int32_t group;          // query_heads / kv_heads
    int32_t has_window;
    int64_t window;
    float scale_log2;       // scale * log2(e): scores live in the exp2 domain
    float scale;
    float softcap;          // 0 disables cap*tanh(score/cap)
    int32_t pad1;
    int64_t total_tiles;
    // split-K partials
    float *part_o;          // [rows, splits, D]
    float *part_ml;         // [rows, splits, 2] (max in log2 units, mass)
    uint32_t *status;
    // optional diagnostics (generic kernel only)
    float *scores;
    float *probs;
    int32_t diag_mode;      // 0 none, 1 full [Hq, queries, keys], 2 last row [keys]
    int32_t pad2;
    Problem single;         // the problem itself when nproblems == 1 (no descriptor upload)
};

__device__ __forceinline__ int find_problem(const Params &p, int64_t tile) {
    int lo = 0, hi = p.nproblems - 1;
    while (lo < hi) {
        int mid = (lo + hi + 1) >> 1;
        if (p.problems[mid].tile_base <= tile) lo = mid; else hi = mid - 1;
    }
    return lo;
}

__device__ __forceinline__ const Problem &tile_problem(const Params &p, int64_t tile) {
    if (p.nproblems == 1) return p.single;
    return p.problems[find_problem(p, tile)];
}

// Load one K or V element (any dtype) as float.
template <int DT> __device__ __forceinline__ float load_elem(const void *base, int64_t i);
template <> __device__ __forceinline__ float load_elem<F32>(const void *base, int64_t i) {
    return reinterpret_cast<const float *>(base)[i];
}
template <> __device__ __forceinline__ float load_elem<F16>(const void *base, int64_t i) {
    return (float)reinterpret_cast<const _Float16 *>(base)[i];
}
template <> __device__ __forceinline__ float load_elem<BF16>(const void *base, int64_t i) {
    uint32_t bits = (uint32_t)reinterpret_cast<const uint16_t *>(base)[i] << 16;
    return __builtin_bit_cast(float, bits);
}

template <int DT> struct ElemSize;
template <> struct ElemSize<F32> { static constexpr int value = 4; };
template <> struct ElemSize<F16> { static constexpr int value = 2; };
template <> struct ElemSize<BF16> { static constexpr int value = 2; };

// Round-to-nearest-even FP32 -> bf16 bits (NaN stays NaN).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float x) {
    uint32_t u = __builtin_bit_cast(uint32_t, x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

__device__ __forceinline__ bool is_finite_f(float x) {
    return __builtin_isfinite(x);
}

// Position of logical key `key` inside the problem's segments.
__device__ __forceinline__ int64_t seg_offset(const Problem &pr, int64_t key, int kvh,
                                              int *which) {
    int s = 0;
    if (pr.nseg > 1 && key >= pr.seg[1].start) s = 1;
    if (pr.nseg > 2 && key >= pr.seg[2].start) s = 2;
    *which = s;
    const Segment &g = pr.seg[s];
    return (int64_t)kvh * g.head_stride + (key - g.start) * g.row_stride;
}

}  // namespace tkh
