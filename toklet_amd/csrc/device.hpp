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
#include <hip/hip_ext.h>
#include <stdint.h>

namespace tkh {

enum Dtype : int32_t { F32 = 0, F16 = 1, BF16 = 2 };

// Status bits OR-ed into the per-context device status word.
enum StatusBits : uint32_t {
    ST_NONFINITE_INPUT = 1u,   // a visible score, or a partial context, is not finite
    ST_BAD_MASS = 2u,          // softmax mass not finite or not positive
    ST_NONFINITE_OUTPUT = 4u,  // combined context not finite
    ST_SPLIT_TIMEOUT = 8u,     // a decode merge gave up waiting for the other key splits
    // 16u: unused (a value-range refusal the chunk kernel no longer makes)
    ST_NONFINITE_LOGIT = 32u,  // a projected logit is not finite (project.hip)
};

// The o-projection and greedy pick (project.hip).
struct ProjectParams {
    const float *context;  // [rows, hidden] FP32
    const float *weights;  // [vocab, hidden] FP32
    float *logits;         // [rows, vocab] or null
    uint64_t *pairs;       // [rows, vblocks]: each workgroup's best (key << 32 | ~id)
    uint32_t *tokens;      // [rows]
    int64_t rows, hidden, vocab;
    int32_t vblocks;       // workgroups along the vocabulary
    uint32_t *status;
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
    int32_t group_base;   // first split-K arrival counter (decode path: one per KV head)
    int64_t tile_base;    // first global tile of this problem
    int64_t part_base;    // first output row (rows are query*Hq + head)
    int64_t slot_base;    // first split-K partial slot (row-major [rows, splits])
    int64_t vis_lo;       // logical key range visible to at least one query row
    int64_t vis_hi;
    int32_t seg_splits[3];  // decode path: key splits inside each segment (splits never
    int32_t pad1;           // straddle a segment boundary)
};

// Producer launch (produce.hip): per-head RMSNorm, rotary, cache rounding.
// Rotary position embedding of the producer: kind 0 none, 1 split-half
// (theta), 2 proportional (base in theta, rotated_dims, factor), 3 Llama 3
// wavelength bands (theta, factor, low/high frequency factors, original
// context length).
struct RotarySpec {
    int32_t kind;
    int32_t rotated_dims;
    float theta, factor, low, high;
    double original;
};

struct ProduceParams {
    const float *q, *k, *v;   // [T, Hq, D], [T, Hkv, D], [T, Hkv, D] FP32, token-major
    const float *q_norm;      // [D] or null (no norm)
    const float *k_norm;
    void *q_out;              // [T, Hq, D] in the cache dtype
    void *k_out, *v_out;      // element (h, t, d) at h * out_head_stride + t * D + d
    int64_t out_head_stride;
    int64_t tokens;
    int64_t position;         // absolute rotary position of token 0
    int32_t hq, hkv, d;
    RotarySpec rot;
    float eps;
    uint32_t *status;
    // Optional precomputed (cos, sin) per (position, pair), rows from absolute
    // position rope_pos0, `pairs` entries per row (the same FP64 formulas,
    // evaluated once per session); null: computed in the kernel.
    const float *rope;
    int64_t rope_pos0;
};

// Decode steps of a session with the producer folded in: one new token whose
// Q/K/V projections are normalised, rotated and rounded inside the decode
// kernel (every workgroup makes the Q rows it needs; the workgroup whose key
// split holds the new key makes that K/V row, uses it, and stores it into
// cache row `new_row`: the row of key `new_key` in a linear cache, or a ring
// layer's staging row, which the gated commit copies into the ring).
struct FusedDecode {
    const float *q_proj;   // [Hq, D] FP32
    const float *k_proj;   // [Hkv, D]
    const float *v_proj;   // [Hkv, D]
    const float *q_norm;   // [D] or null
    const float *k_norm;
    const float *rope;     // (cos, sin) of the token's position, `pairs` entries, or null
    int32_t pairs;
    float eps;
    void *k_cache;         // cache bases; element (h, key, d) at h * head_stride + key * D + d
    void *v_cache;
    int64_t head_stride;
    int64_t new_key;       // logical key index of the new token
    int64_t new_row;       // cache row its K/V go to (new_key for a linear cache, 0 for a ring's stage)
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
    float softcap_inv;      // 1 / softcap (0 when disabled)
    float softcap_y;        // scale / softcap: raw dot -> tanh argument (0 when disabled)
    float softcap_log2;     // softcap * log2(e): tanh units -> log2 units
    int64_t total_tiles;
    // split-K partials
    float *part_o;          // per slot: [rows, D] (generic kernel), [D, rows] (chunk kernel)
    float *part_ml;         // [rows, splits, 2] (max in log2 units, mass)
    uint32_t *status;
    // optional diagnostics (generic kernel only)
    float *scores;
    float *probs;
    int32_t diag_mode;      // 0 none, 1 full [Hq, queries, keys], 2 last row [keys]
    int32_t stream_nt;      // decode: K/V stream read with nontemporal loads (1) or plain (0)
    uint32_t *flags;        // decode split-K completion flags, one per partial slot
    uint32_t epoch;         // decode split-K: this launch's flag value (never 0; flags start at 0)
    uint32_t wait_epoch;    // the flag value the merging split waits for (= epoch)
    uint64_t split_wait_ticks;  // bound of that wait, s_memrealtime ticks
    int32_t merge_launch;   // decode split-K: every split stores its partial; attn_decode_merge combines
    FusedDecode fused;      // decode kernel built with FUSED only
    Problem single;         // the problem itself when nproblems == 1 (no descriptor upload)
};

// The ring commits of one chunk (one per sliding layer) in a single launch:
// entry i copies its staged rows [heads, tokens, row_bytes] into up to two
// runs of ring slots, runs {source row, slot, rows} (kv_copy_batch).
constexpr int COPY_BATCH_MAX = 16;
struct CopyRunsEntry {
    const uint8_t *src_k, *src_v;
    uint8_t *dst_k, *dst_v;
    int64_t tokens, row_bytes, capacity;
    int64_t runs[6];
    int32_t heads;
};
struct CopyBatch {
    CopyRunsEntry e[COPY_BATCH_MAX];
    int32_t count;
    const uint32_t *gate;
    uint64_t *committed;
    uint64_t committed_value;
};

// A batch of single-segment, single-token decode problems (tkh_decode_batch of
// at most DECODE_BATCH_MAX sessions) carried in the decode kernel's own
// arguments, so the launch needs no descriptor upload: the upload is a copy
// ordered after the previous kernel on the stream, about 20 us of idle device
// time per launch.  Session i reads Q row i and writes context row i; its K/V
// cache starts kv_offset elements from k/v.
constexpr int DECODE_BATCH_MAX = 64;
struct DecodeBatchEntry {
    int64_t kv_offset;     // elements from k / v to the session's cache
    uint32_t head_stride;  // elements between its KV heads
    uint32_t keys;         // its keys (the query sits at position keys - 1)
    uint32_t tile_base;    // its first workgroup, which is also its first partial slot
    uint32_t splits;       // its key splits per KV head
};
struct DecodeBatch {
    const void *q;         // [count, Hq, D] in the cache dtype
    float *out;            // [count, Hq, D]
    const void *k, *v;
    int32_t count;         // 0: the launch describes its problems in Params
    int32_t split_keys;
    DecodeBatchEntry e[DECODE_BATCH_MAX];
};

// The decode kernel's one argument: the launch parameters, then the compact
// batch (count 0 when unused).
struct DecodeArgs {
    Params p;
    DecodeBatch b;
};

// Chunks of one shape (tkh_prefill_batch: equal query counts, one K/V segment
// from key 0 each, no window, no key splits; at most PREFILL_BATCH_MAX) carried
// in the prefill kernel's own arguments, so the launch needs no descriptor
// upload (a copy ordered after the previous kernel: about 4 us plus the gaps
// around it per launch).  Chunk i reads Q and writes context from q_step * i
// elements past q / out; its K/V cache starts kv_offset elements from k / v
// (the same offset for both), and its first query sits at key `position`.
constexpr int PREFILL_BATCH_MAX = 64;
struct PrefillBatchEntry {
    int64_t kv_offset;
    int64_t head_stride;  // elements between its KV heads
    int64_t position;
    int64_t tile_base;    // its first workgroup
};
struct PrefillBatch {
    const void *q;        // chunk 0's Q in the cache dtype, [tokens, Hq, D]
    float *out;           // chunk 0's context
    const void *k, *v;
    int64_t q_step;       // elements between consecutive chunks' Q (and contexts)
    int32_t count;        // 0: the launch describes its problems in Params
    int32_t tokens;       // query tokens per chunk
    int32_t row_blocks;   // row blocks per KV head
    int32_t split_keys;
    PrefillBatchEntry e[PREFILL_BATCH_MAX];
};
struct PrefillArgs {
    Params p;             // first: the single-problem path reads it at the kernel-argument base
    PrefillBatch b;
};
static_assert(sizeof(PrefillArgs) <= 4096, "kernel arguments");
static_assert(sizeof(DecodeArgs) <= 4096, "kernel arguments");

// Address-space qualified views: the problem descriptors are read-only for a
// launch (scalar loads through the constant space), tensors are global.
template <class T> using const_ptr = const __attribute__((address_space(4))) T *;
template <class T> using global_ptr = __attribute__((address_space(1))) T *;
template <class T> using global_cptr = const __attribute__((address_space(1))) T *;

template <class T> __device__ __forceinline__ global_cptr<T> gload_ptr(const void *p) {
    return (global_cptr<T>)p;
}
template <class T> __device__ __forceinline__ global_ptr<T> gstore_ptr(void *p) {
    return (global_ptr<T>)p;
}

__device__ __forceinline__ int find_problem(const Params &p, int64_t tile) {
    const_ptr<Problem> probs = (const_ptr<Problem>)p.problems;
    int lo = 0, hi = p.nproblems - 1;
    while (lo < hi) {
        int mid = (lo + hi + 1) >> 1;
        if (probs[mid].tile_base <= tile) lo = mid; else hi = mid - 1;
    }
    return lo;
}

// The same search by a whole wave: each lane tests one candidate, a ballot
// picks the interval, so up to 64 problems take one round trip of loads and up
// to 4096 two (the scalar binary search above is a chain of log2(n) dependent
// loads).  Every lane of the wave must be active.
__device__ __forceinline__ int find_problem_wave(const Problem *problems, int n, int64_t tile) {
    const int lane = threadIdx.x & 63;
    int lo = 0, count = n;
    while (count > 1) {
        const int stride = (count + 63) >> 6;
        const int off = lane * stride;
        const bool le = off < count && gload_ptr<Problem>(problems + lo + off)->tile_base <= tile;
        const uint64_t m = __ballot(le);  // bit 0 is set: problems[lo] starts at or before tile
        const int k = 63 - __builtin_clzll(m);
        lo += k * stride;
        count = count - k * stride < stride ? count - k * stride : stride;
    }
    return __builtin_amdgcn_readfirstlane(lo);
}

// The problem owning global tile `tile`, as a constant-space pointer: either
// the copy inside the kernel arguments (Params must be the kernel's first
// argument) or an entry of the uploaded descriptor array.  Its fields are
// uniform and load through the scalar cache.  Call with the whole wave active.
// Bring the first NL 64-byte lines of the kernel arguments, and the line at
// byte EXTRA (the hidden arguments after them: the grid size), into the
// scalar cache at once: one scalar load per line, all in flight together,
// then one wait.  A kernel's descriptor fields are read by chains of
// dependent scalar loads (a count decides which fields come next, a field
// indexes the next one), each of which would otherwise miss the cache on its
// own line in turn; after this they hit.  The loaded words are discarded;
// the destinations are early-clobber, so none of them shares a register with
// the base address that a later load of the same block still reads.
template <int NL, int EXTRA> __device__ __forceinline__ void warm_kernarg() {
    static_assert(NL >= 1 && NL <= 11, "kernel-argument lines");
    static_assert(EXTRA >= 0 && EXTRA % 4 == 0, "a dword offset");
    const auto kp = __builtin_amdgcn_kernarg_segment_ptr();
    constexpr int L = 64;
    uint32_t d0, d1, d2, d3, d4, d5, d6, d7, d8, d9, d10, d11;
    asm volatile(
        "s_load_dword %0, %12, %13\n\t"
        "s_load_dword %1, %12, %14\n\t"
        "s_load_dword %2, %12, %15\n\t"
        "s_load_dword %3, %12, %16\n\t"
        "s_load_dword %4, %12, %17\n\t"
        "s_load_dword %5, %12, %18\n\t"
        "s_load_dword %6, %12, %19\n\t"
        "s_load_dword %7, %12, %20\n\t"
        "s_load_dword %8, %12, %21\n\t"
        "s_load_dword %9, %12, %22\n\t"
        "s_load_dword %10, %12, %23\n\t"
        "s_load_dword %11, %12, %24\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&s"(d0), "=&s"(d1), "=&s"(d2), "=&s"(d3), "=&s"(d4), "=&s"(d5), "=&s"(d6), "=&s"(d7),
          "=&s"(d8), "=&s"(d9), "=&s"(d10), "=&s"(d11)
        : "s"(kp), "i"(0), "i"(NL > 1 ? L : 0), "i"(NL > 2 ? 2 * L : 0), "i"(NL > 3 ? 3 * L : 0),
          "i"(NL > 4 ? 4 * L : 0), "i"(NL > 5 ? 5 * L : 0), "i"(NL > 6 ? 6 * L : 0),
          "i"(NL > 7 ? 7 * L : 0), "i"(NL > 8 ? 8 * L : 0), "i"(NL > 9 ? 9 * L : 0),
          "i"(NL > 10 ? 10 * L : 0), "i"(EXTRA));
}
// Hold wave-uniform values (kernel-argument fields) in scalar registers from
// here on: each needs its load complete, so loads read before a call are all
// issued before its first wait.
template <class T> __device__ __forceinline__ void pin_arg(T &x) { asm volatile("" : "+s"(x)); }
template <class... T> __device__ __forceinline__ void pin_args(T &...x) { (pin_arg(x), ...); }
// warm_kernarg, then the kernel-argument pointer offset by a zero the
// compiler cannot see through.  Argument fields are invariant loads, which
// the compiler may move above the warm-up (and wait for them there, a miss of
// their own); read through this pointer they depend on it, so they issue
// after its one wait and hit the scalar cache.
template <class T, int NL, int EXTRA> __device__ __forceinline__ const_ptr<T> warm_kernarg_ptr() {
    warm_kernarg<NL, EXTRA>();
    uint32_t z;
    asm volatile("s_mov_b32 %0, 0" : "=s"(z));
    return (const_ptr<T>)((const_ptr<char>)__builtin_amdgcn_kernarg_segment_ptr() + z);
}

__device__ __forceinline__ const_ptr<Problem> problem_ptr(const Params &p, int64_t tile) {
    if (p.nproblems == 1) {
        const_ptr<Params> args = (const_ptr<Params>)__builtin_amdgcn_kernarg_segment_ptr();
        return &args->single;
    }
    return (const_ptr<Problem>)p.problems + find_problem_wave(p.problems, p.nproblems, tile);
}

// Generic reference form used by the VALU and MFMA kernels.
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

// K/V addresses of logical key `key` by per-lane selects over the three
// segments (constant indices only, so the descriptors stay in scalar
// registers).  Returns the element offset inside the selected segment.
__device__ __forceinline__ int64_t seg_select(const_ptr<Problem> pr, int64_t key, int kvh,
                                              const void **k, const void **v) {
    const auto &s0 = pr->seg[0], &s1 = pr->seg[1], &s2 = pr->seg[2];
    const bool in1 = pr->nseg > 1 && key >= s1.start;
    const bool in2 = pr->nseg > 2 && key >= s2.start;
    const int64_t hs = in2 ? s2.head_stride : (in1 ? s1.head_stride : s0.head_stride);
    const int64_t rs = in2 ? s2.row_stride : (in1 ? s1.row_stride : s0.row_stride);
    const int64_t st = in2 ? s2.start : (in1 ? s1.start : s0.start);
    *k = in2 ? s2.k : (in1 ? s1.k : s0.k);
    *v = in2 ? s2.v : (in1 ? s1.v : s0.v);
    return (int64_t)kvh * hs + (key - st) * rs;
}

// ---------------------------------------------------------------------------
// Helpers shared by the attention kernels
// ---------------------------------------------------------------------------

using f32x4 = float __attribute__((ext_vector_type(4)));
using u32x4 = uint32_t __attribute__((ext_vector_type(4)));
using f32x2 = float __attribute__((ext_vector_type(2)));
using bf16x2 = __bf16 __attribute__((ext_vector_type(2)));
using f16x2 = _Float16 __attribute__((ext_vector_type(2)));
using bf16x8 = __bf16 __attribute__((ext_vector_type(8)));
using f16x8 = _Float16 __attribute__((ext_vector_type(8)));

constexpr float LOG2E = 1.4426950408889634f;
constexpr float NEG_INF = -__builtin_inff();

__device__ __forceinline__ float xor_max(float x, int mask) { return fmaxf(x, __shfl_xor(x, mask, 64)); }
__device__ __forceinline__ float xor_sum(float x, int mask) { return x + __shfl_xor(x, mask, 64); }

// Sum over the wave by the xor butterfly x + x[lane ^ m], m = 32, 16, ..., 1,
// in FP64: every lane ends with the same, fixed association.  The partner
// values move in registers (lane swaps for 32 and 16, a DPP row rotate for 8,
// a swizzle for 4, DPP quad permutes for 2 and 1), not through LDS.
__device__ __forceinline__ double wave_sum_f64(double x) {
    auto halves = [](double v, uint32_t &lo, uint32_t &hi) {
        const uint64_t u = __builtin_bit_cast(uint64_t, v);
        lo = (uint32_t)u;
        hi = (uint32_t)(u >> 32);
    };
    auto join = [](uint32_t lo, uint32_t hi) {
        return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
    };
    uint32_t lo, hi;
    {
        halves(x, lo, hi);
        const auto l = __builtin_amdgcn_permlane32_swap(lo, lo, false, false);
        const auto h = __builtin_amdgcn_permlane32_swap(hi, hi, false, false);
        x = join(l[0], h[0]) + join(l[1], h[1]);
    }
    {
        halves(x, lo, hi);
        const auto l = __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
        const auto h = __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
        x = join(l[0], h[0]) + join(l[1], h[1]);
    }
    halves(x, lo, hi);
    x += join((uint32_t)__builtin_amdgcn_update_dpp(0, (int)lo, 0x128, 0xF, 0xF, false),
              (uint32_t)__builtin_amdgcn_update_dpp(0, (int)hi, 0x128, 0xF, 0xF, false));
    halves(x, lo, hi);
    x += join((uint32_t)__builtin_amdgcn_ds_swizzle((int)lo, 0x101F),
              (uint32_t)__builtin_amdgcn_ds_swizzle((int)hi, 0x101F));
    halves(x, lo, hi);
    x += join((uint32_t)__builtin_amdgcn_update_dpp(0, (int)lo, 0x4E, 0xF, 0xF, false),
              (uint32_t)__builtin_amdgcn_update_dpp(0, (int)hi, 0x4E, 0xF, 0xF, false));
    halves(x, lo, hi);
    x += join((uint32_t)__builtin_amdgcn_update_dpp(0, (int)lo, 0xB1, 0xF, 0xF, false),
              (uint32_t)__builtin_amdgcn_update_dpp(0, (int)hi, 0xB1, 0xF, 0xF, false));
    return x;
}

__device__ __forceinline__ float wave_max(float x) {
    for (int m = 32; m >= 1; m >>= 1) x = xor_max(x, m);
    return x;
}
__device__ __forceinline__ float wave_sum(float x) {
    for (int m = 32; m >= 1; m >>= 1) x = xor_sum(x, m);
    return x;
}

// cap * tanh(x / cap), FP32.  tanh(y) = sign(y) (1 - 2 / (exp(2|y|) + 1)), with a
// short odd Taylor series near zero where the subtraction would cancel.
__device__ __forceinline__ float softcap_f(float x, float cap) {
    float y = x / cap;
    float a = fabsf(y);
    float t;
    if (a < 0.0625f) {
        float y2 = y * y;
        t = y * (1.0f + y2 * (-1.0f / 3.0f + y2 * (2.0f / 15.0f + y2 * (-17.0f / 315.0f))));
    } else {
        float e = __builtin_amdgcn_exp2f(fminf(2.0f * LOG2E * a, 126.0f));
        t = copysignf(1.0f - 2.0f / (e + 1.0f), y);
    }
    return cap * t;
}

// tanh(y) = sign(y) (1 - 2 / (e^(2|y|) + 1)) in six vector instructions, for
// the kernels' inner loops (no division, no branch).  Its absolute error stays
// below about 2e-7 (for small |y| the subtraction cancels, but only absolute
// error reaches the softmax: the capped score is t * cap in natural units, an
// exponent).  NaN propagates; |y| large gives e = inf and exactly +-1.
__device__ __forceinline__ float tanh_fast(float y) {
    const float e = __builtin_amdgcn_exp2f(2.0f * LOG2E * __builtin_fabsf(y));
    const float t = __builtin_fmaf(-2.0f, __builtin_amdgcn_rcpf(e + 1.0f), 1.0f);
    return __builtin_copysignf(t, y);
}

// Visible key range [lo, hi) (logical indices) of a query at absolute `pos`.
__device__ __forceinline__ void visible_range(bool has_window, int64_t window, int64_t k_pos0,
                                              int64_t keys, int64_t pos, int64_t *lo, int64_t *hi) {
    int64_t h = pos - k_pos0 + 1;
    *hi = h < keys ? h : keys;
    int64_t l = 0;
    if (has_window) {
        int64_t first = pos - (window - 1) - k_pos0;
        l = first > 0 ? first : 0;
    }
    *lo = l;
}
__device__ __forceinline__ void visible_range(const Params &p, int64_t k_pos0, int64_t keys,
                                              int64_t pos, int64_t *lo, int64_t *hi) {
    visible_range(p.has_window != 0, p.window, k_pos0, keys, pos, lo, hi);
}
__device__ __forceinline__ void visible_range(const Params &p, const Problem &pr, int64_t pos,
                                              int64_t *lo, int64_t *hi) {
    visible_range(p, pr.k_pos0, pr.keys, pos, lo, hi);
}

__device__ __forceinline__ void raise_status(uint32_t *status, bool bad, uint32_t bit) {
    if (__builtin_amdgcn_read_exec() != 0) {
        uint64_t m = __ballot(bad);
        if (m != 0 && (threadIdx.x & 63) == (int)__builtin_ctzll(m)) atomicOr(status, bit);
    }
}
__device__ __forceinline__ void raise_status(const Params &p, bool bad, uint32_t bit) {
    raise_status(p.status, bad, bit);
}

}  // namespace tkh
