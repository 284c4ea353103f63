// decode_kernel.hpp - gfx950 streaming decode attention (few query rows per KV head).
//
// attn_decode<DT, D, R> handles every call whose query rows per KV head
// (tokens x query heads of the GQA group) fit in R <= 8: single-token decode
// of one session or of a batch of sessions, and short chunks.  The work is
// HBM-bound (about 2 FLOP per byte of K/V), so the kernel is organised
// around the K/V stream, not the matrix cores:
//
//  * One workgroup per (problem, KV head, key split); the waves of the
//    workgroup take interleaved blocks of keys inside the split.
//  * Eight lanes share one key row: lane s of the eight reads the 16-byte
//    chunks at byte offsets 128*c + 16*s of the row, so each load
//    instruction of a wave covers eight whole 128-byte lines.  The query
//    rows are held in registers in the same element order.
//  * Q.K is a packed bf16/f16 dot2 (v_dot2_f32_*) over the lane's chunks
//    followed by a three-step DPP sum across the eight lanes; P.V is FP32 FMA
//    after widening V.  The next block of K/V is in flight while the current
//    one is consumed (register double buffering).
//  * Online softmax runs per lane over the keys it sees (exp2 domain).  The
//    rescale of the running context is skipped for a block unless some
//    lane's running maximum moved, which after the first blocks is rare.
//  * At the end the eight key lanes merge by lane swaps, the waves merge
//    through LDS, and a split either writes the context directly (one split)
//    or writes an unnormalised partial and a completion flag; the last split
//    of a KV head (its highest block index) waits for the other flags, merges
//    the partials and writes the context.  No atomics, one launch per call.
#pragma once

#include <type_traits>

#include "device.hpp"

namespace tkh {

namespace {

// DPP sums inside groups of eight lanes (quad xor 1, quad xor 2, half-row mirror).
__device__ __forceinline__ float dpp_sum8(float x) {
    int v = __builtin_bit_cast(int, x);
    x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false));
    v = __builtin_bit_cast(int, x);
    x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false));
    v = __builtin_bit_cast(int, x);
    x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false));
    return x;
}

// The value of lane i and of lane i ^ MASK (MASK 8: DPP row rotate by 8 inside
// 16-lane rows; 16 / 32: v_permlane16/32_swap, which hand back the pair
// {x[i & ~MASK], x[i | MASK]}).  Every merge below is symmetric in the pair, so
// both lanes of a pair compute the same result.
template <int MASK> __device__ __forceinline__ void lane_pair(float x, float &a, float &b) {
    const uint32_t u = __builtin_bit_cast(uint32_t, x);
    if constexpr (MASK == 8) {
        a = x;
        b = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, (int)u, 0x128, 0xF, 0xF, false));
    } else if constexpr (MASK == 16) {
        const auto p = __builtin_amdgcn_permlane16_swap(u, u, false, false);
        const uint32_t p0 = p[0], p1 = p[1];
        a = __builtin_bit_cast(float, p0);
        b = __builtin_bit_cast(float, p1);
    } else {
        static_assert(MASK == 32, "lane_pair masks are 8, 16, 32");
        const auto p = __builtin_amdgcn_permlane32_swap(u, u, false, false);
        const uint32_t p0 = p[0], p1 = p[1];
        a = __builtin_bit_cast(float, p0);
        b = __builtin_bit_cast(float, p1);
    }
}

template <int DT> struct Elem;
template <> struct Elem<F32> { static constexpr int size = 4; };
template <> struct Elem<F16> { static constexpr int size = 2; };
template <> struct Elem<BF16> { static constexpr int size = 2; };

// Element j of a 16-byte chunk as a scalar.  Every reinterpretation below
// goes through this copy: with this ROCm clang, __builtin_bit_cast applied
// directly to a vector element (v[j]) reads element 0 for every j.
__device__ __forceinline__ uint32_t word(u32x4 v, int j) {
    const uint32_t w = v[j];
    return w;
}

// Partial dot product of one 16-byte chunk of K with the same chunk of Q.
template <int DT> __device__ __forceinline__ float chunk_dot(u32x4 k, u32x4 q, float acc);
template <> __device__ __forceinline__ float chunk_dot<BF16>(u32x4 k, u32x4 q, float acc) {
    for (int j = 0; j < 4; ++j) {
        const uint32_t kw = word(k, j), qw = word(q, j);
        acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, kw),
                                              __builtin_bit_cast(bf16x2, qw), acc, false);
    }
    return acc;
}
template <> __device__ __forceinline__ float chunk_dot<F16>(u32x4 k, u32x4 q, float acc) {
    for (int j = 0; j < 4; ++j) {
        const uint32_t kw = word(k, j), qw = word(q, j);
        acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, kw), __builtin_bit_cast(f16x2, qw),
                                     acc, false);
    }
    return acc;
}
template <> __device__ __forceinline__ float chunk_dot<F32>(u32x4 k, u32x4 q, float acc) {
    for (int j = 0; j < 4; ++j) {
        const uint32_t kw = word(k, j), qw = word(q, j);
        acc = __builtin_fmaf(__builtin_bit_cast(float, kw), __builtin_bit_cast(float, qw), acc);
    }
    return acc;
}

// Widen the elements of one 16-byte chunk to FP32.
template <int DT> __device__ __forceinline__ void widen(u32x4 w, float *out);
template <> __device__ __forceinline__ void widen<BF16>(u32x4 w, float *out) {
    for (int j = 0; j < 4; ++j) {
        const uint32_t x = word(w, j);
        out[2 * j] = __builtin_bit_cast(float, x << 16);
        out[2 * j + 1] = __builtin_bit_cast(float, x & 0xffff0000u);
    }
}
template <> __device__ __forceinline__ void widen<F16>(u32x4 w, float *out) {
    for (int j = 0; j < 4; ++j) {
        const uint32_t x = word(w, j);
        const f16x2 h = __builtin_bit_cast(f16x2, x);
        out[2 * j] = (float)h[0];
        out[2 * j + 1] = (float)h[1];
    }
}
template <> __device__ __forceinline__ void widen<F32>(u32x4 w, float *out) {
    for (int j = 0; j < 4; ++j) {
        const uint32_t x = word(w, j);
        out[j] = __builtin_bit_cast(float, x);
    }
}

__device__ __forceinline__ u32x4 load16(const uint8_t *p) { return *gload_ptr<u32x4>(p); }
// The K/V stream of a launch with much work: each line is read once, so the
// loads can be marked nontemporal (global_load_dwordx4 ... nt).  A plain read
// stream of 0.5-1 GiB measured 6.1-6.3 TB/s on MI355X, the nontemporal form
// 6.9-7.2 TB/s.
__device__ __forceinline__ u32x4 load16_stream(const uint8_t *p) {
    return __builtin_nontemporal_load(gload_ptr<u32x4>(p));
}

// Round a chunk's worth of FP32 values to the storage dtype (RNE) and pack them.
template <int DT> __device__ __forceinline__ u32x4 pack_chunk(const float *x);
template <> __device__ __forceinline__ u32x4 pack_chunk<BF16>(const float *x) {
    u32x4 w;
    for (int j = 0; j < 4; ++j) {
        const f32x2 v = {x[2 * j], x[2 * j + 1]};
        w[j] = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
    }
    return w;
}
template <> __device__ __forceinline__ u32x4 pack_chunk<F16>(const float *x) {
    u32x4 w;
    for (int j = 0; j < 4; ++j) {
        const f32x2 v = {x[2 * j], x[2 * j + 1]};
        w[j] = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
    }
    return w;
}
template <> __device__ __forceinline__ u32x4 pack_chunk<F32>(const float *x) {
    u32x4 w;
    for (int j = 0; j < 4; ++j) w[j] = __builtin_bit_cast(uint32_t, x[j]);
    return w;
}

// The producer for one head row, by one whole wave, in produce_qkv's own
// arithmetic and order (so both give the same bits): lane l holds elements
// l, l + 64, ...; per-head RMSNorm with the squares summed in FP64 per lane
// (in element order) and then by the same xor butterfly (wave_sum_f64), the
// reciprocal root in FP64 and value = f32(x * inv * w) in FP64; then the
// rotary of pair j (elements j and j + D/2) with the row's (cos, sin) from the
// session's table and FP32 products and sums rounded separately.  Every load
// (the row, the weights, the (cos, sin) pairs) is issued before any
// arithmetic, and the row stays in registers: with D = 128 a lane holds both
// elements of its pair, with D = 256 both elements of two pairs (j = l and
// l + 64), with D = 64 the partner comes by a lane swap.  Returns the lane's
// D/64 finished values.
template <int D>
__device__ __forceinline__ void wave_produce_row(const float *src, const float *w, float eps,
                                                 const float *rope, int pairs, int lane,
                                                 float (&y)[D / 64], bool &bad) {
#pragma clang fp contract(off)
    static_assert(D == 64 || D == 128 || D == 256, "the fused producer covers head sizes 64, 128, 256");
    constexpr int K = D / 64, half = D / 2;
    constexpr int NP = K >= 2 ? K / 2 : 1;  // rotary pairs a lane computes
    float x[K], wv[K];
    f32x2 cs[NP];
    bool rotated[NP];
    for (int k = 0; k < K; ++k) {
        x[k] = src[lane + 64 * k];
        wv[k] = w ? w[lane + 64 * k] : 1.0f;
    }
    for (int q = 0; q < NP; ++q) {
        const int j = K >= 2 ? lane + 64 * q : lane % half;  // the pair of element x[q]
        cs[q] = f32x2{1.0f, 0.0f};
        rotated[q] = rope && j < pairs;
        if (rotated[q]) cs[q] = *gload_ptr<f32x2>(rope + 2 * j);
    }
    for (int k = 0; k < K; ++k) bad |= !is_finite_f(x[k]);
    if (w) {
        double ss = 0.0;
        for (int k = 0; k < K; ++k) ss += (double)x[k] * (double)x[k];
        ss = wave_sum_f64(ss);
        const double inv = 1.0 / sqrt(ss / (double)D + (double)eps);
        for (int k = 0; k < K; ++k) {
            x[k] = (float)((double)x[k] * inv * (double)wv[k]);
            bad |= !is_finite_f(x[k]) || !is_finite_f(wv[k]);
        }
    }
    if (rope) {
        for (int q = 0; q < NP; ++q) {
            // a = element j, b = element j + half: with D >= 128 x[q] and
            // x[q + K/2] of this lane; with D = 64 this lane's x[0] and the
            // one of lane ^ 32.
            float a, b;
            if constexpr (K >= 2) {
                a = x[q];
                b = x[q + K / 2];
            } else {
                float lo, hi;
                lane_pair<32>(x[0], lo, hi);
                a = lo;
                b = hi;
            }
            if (rotated[q]) {
                const float c = cs[q][0], sn = cs[q][1];
                const float ac = a * c, bs = b * sn, bc = b * c, as = a * sn;
                const float ra = ac - bs, rb = bc + as;
                bad |= !is_finite_f(ra) || !is_finite_f(rb);
                a = ra;
                b = rb;
            }
            if constexpr (K >= 2) {
                x[q] = a;
                x[q + K / 2] = b;
            } else {
                x[0] = lane < half ? a : b;
            }
        }
    }
    for (int k = 0; k < K; ++k) y[k] = x[k];
}

// Split-K partials and completion flags: agent-scope accesses, which on
// gfx950 are sc1 stores and loads (the merge reads partials with sc1 buffer
// loads).  They bypass the CU's vector L1 (a
// workgroup-scope sc0 load may be served from it, so a poll with one can read
// a stale line for ever) and are coherent across the XCDs.  A partial is read
// only after its writer's stores were acknowledged and its flag seen: a line
// read while a store to it is still on its way can stay stale in the reader's
// caches for microseconds.
__device__ __forceinline__ void split_store(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void flag_store(uint32_t *p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t flag_load(const uint32_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Buffer resource word 3 for raw 32-bit-element buffers on gfx9, the cache
// policy operand of a buffer load that makes it an sc1 (device-coherent),
// non-temporal load (the partials are read once), and an offset past every
// buffer range (the load returns zeros).
constexpr int BUFFER_RSRC_WORD3 = 0x00020000;
constexpr int CPOL_SC1_NT = 16 | 2;
constexpr uint32_t OUT_OF_RANGE = 0x80000000u;

}  // namespace

// A key segment's fields the decode kernel reads (Segment minus nothing it
// needs), and the problem fields its first K/V and Q loads depend on.
struct DecodeSegment {
    const void *k, *v;
    int64_t head_stride, row_stride, keys, start;
};
struct DecodeView {
    int64_t tile_base, vis_lo, vis_hi, k_pos0, keys, q_pos0, q_row_stride;
    const void *q;
    int32_t splits, split_keys, seg_splits0, seg_splits1, queries;
    DecodeSegment seg0;
};
__device__ __forceinline__ DecodeSegment decode_segment(const_ptr<Problem> pr, int s) {
    const auto &g = pr->seg[s];
    return DecodeSegment{g.k, g.v, g.head_stride, g.row_stride, g.keys, g.start};
}
// Held in scalar registers at this point: an empty asm that reads and
// "writes" the value keeps its load ahead of what follows.
template <class T> __device__ __forceinline__ void pin_scalar(T &x) { asm volatile("" : "+s"(x)); }
__device__ __forceinline__ void pin_view(DecodeView &v) {
    pin_scalar(v.tile_base);
    pin_scalar(v.vis_lo);
    pin_scalar(v.vis_hi);
    pin_scalar(v.k_pos0);
    pin_scalar(v.keys);
    pin_scalar(v.q_pos0);
    pin_scalar(v.q_row_stride);
    pin_scalar(v.q);
    pin_scalar(v.splits);
    pin_scalar(v.split_keys);
    pin_scalar(v.seg_splits0);
    pin_scalar(v.seg_splits1);
    pin_scalar(v.queries);
    pin_scalar(v.seg0.k);
    pin_scalar(v.seg0.v);
    pin_scalar(v.seg0.head_stride);
    pin_scalar(v.seg0.row_stride);
    pin_scalar(v.seg0.keys);
    pin_scalar(v.seg0.start);
}
__device__ __forceinline__ DecodeView decode_view(const_ptr<Problem> pr) {
    DecodeView v;
    v.tile_base = pr->tile_base;
    v.vis_lo = pr->vis_lo;
    v.vis_hi = pr->vis_hi;
    v.k_pos0 = pr->k_pos0;
    v.keys = pr->keys;
    v.q_pos0 = pr->q_pos0;
    v.q_row_stride = pr->q_row_stride;
    v.q = pr->q;
    v.splits = pr->splits;
    v.split_keys = pr->split_keys;
    v.seg_splits0 = pr->seg_splits[0];
    v.seg_splits1 = pr->seg_splits[1];
    v.queries = pr->queries;
    v.seg0 = decode_segment(pr, 0);
    return v;
}

constexpr int DECODE_MAX_SPLITS = 64;  // key splits per KV head (bounds the merge)

// Waves per workgroup the kernel is built for: eight when the rows and the
// row size leave room in the register file (256 VGPRs per lane), else four.
constexpr int decode_waves_for(int row_bytes, int rows) { return rows <= 2 && row_bytes <= 512 ? 8 : 4; }

// The session of global workgroup `tile` in a compact batch, by the whole
// wave: lane i tests entry i, a ballot picks the last entry that starts at or
// before the tile.
__device__ __forceinline__ int find_batch_entry(const_ptr<DecodeBatch> b, int count, uint32_t tile) {
    const int lane = threadIdx.x & 63;
    const bool le = lane < count && b->e[lane].tile_base <= tile;
    const uint64_t m = __ballot(le);  // bit 0 is set: entry 0 starts at tile 0
    return __builtin_amdgcn_readfirstlane(63 - __builtin_clzll(m));
}

template <int DT, int D, int R, int U, bool CAP, bool FUSED>
__global__ __launch_bounds__(64 * decode_waves_for(D * Elem<DT>::size, R)) void attn_decode(DecodeArgs kargs) {
    const Params &p = kargs.p;
    constexpr int ES = Elem<DT>::size;
    constexpr int NWMAX = decode_waves_for(D * ES, R);
    constexpr int ROWB = D * ES;            // bytes per K/V row
    constexpr int CPL = ROWB / 128;         // 16-byte chunks per lane per key
    constexpr int EPC = 16 / ES;            // elements per chunk
    constexpr int EPL = CPL * EPC;          // elements per lane
    constexpr int KPB = 8 * U;              // keys per wave block (U keys per lane)
    static_assert(CPL >= 1, "head rows must be at least 128 bytes");

    __shared__ float lds_o[NWMAX * R * D];
    __shared__ float lds_ml[NWMAX * R * 2];
    // The merging split's own partial (context, (max, mass) per row) and its
    // flag-wait outcome.
    __shared__ __attribute__((aligned(16))) float lds_own[R * D + 2 * R + 1];
    // Fused producer: the new K/V rows and the Q rows in 16-byte chunks
    // (chunk 8 c + sub is lane sub's chunk c), and one staging row per wave.
    __shared__ u32x4 lds_new[FUSED ? 2 * CPL * 8 : 1];
    __shared__ u32x4 lds_q[FUSED ? R * CPL * 8 : 1];
    __shared__ float lds_prow[FUSED ? NWMAX * D : 1];

    const int nw = blockDim.x >> 6;
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int sub = lane & 7;   // which chunks of the row
    const int kg = lane >> 3;   // which key of the block

    // The scalars the first K/V load depends on arrive in one batch: the
    // problem inside the kernel arguments is read together with the problem
    // count (a single-problem launch needs nothing else), and a batched launch
    // then finds its problem by a wave-parallel search and reads it again.
    // Segments past the first load only when the split lies in one (rings).
    const_ptr<DecodeArgs> dargs = (const_ptr<DecodeArgs>)__builtin_amdgcn_kernarg_segment_ptr();
    const_ptr<Params> args = &dargs->p;
    const_ptr<DecodeBatch> batch = &dargs->b;
    const_ptr<Problem> pr = &args->single;
    // Every kernel-argument field the prologue and the stream need, read
    // before the first use of any (the pins below then cost one wait): the
    // problem view, the launch fields and the fused producer's descriptor.  A
    // field first read after that wait is another round trip to L2.
    DecodeView pv = decode_view(pr);
    int64_t slot_base = pr->slot_base;
    float *out = pr->out;
    int nproblems = args->nproblems;
    int bcount = batch->count;
    int G = args->group, Hq = args->query_heads, has_window = args->has_window;
    int64_t window = args->window;
    float scale_log2 = args->scale_log2;
    // Capped score in log2 units: tanh(raw * scale / cap) * cap * log2(e).
    float ycap = args->softcap_y, caplog2 = args->softcap_log2;
    int stream_nt = args->stream_nt;
    FusedDecode fz{};
    if constexpr (FUSED) {
        const auto &fa = args->fused;
        fz.q_proj = fa.q_proj;
        fz.k_proj = fa.k_proj;
        fz.v_proj = fa.v_proj;
        fz.q_norm = fa.q_norm;
        fz.k_norm = fa.k_norm;
        fz.rope = fa.rope;
        fz.pairs = fa.pairs;
        fz.eps = fa.eps;
        fz.k_cache = fa.k_cache;
        fz.v_cache = fa.v_cache;
        fz.head_stride = fa.head_stride;
        fz.new_key = fa.new_key;
        fz.new_row = fa.new_row;
    }
    pin_scalar(nproblems);
    pin_scalar(bcount);
    pin_scalar(slot_base);
    pin_scalar(out);
    pin_view(pv);
    pin_scalar(G);
    pin_scalar(Hq);
    pin_scalar(has_window);
    pin_scalar(window);
    pin_scalar(scale_log2);
    pin_scalar(ycap);
    pin_scalar(caplog2);
    pin_scalar(stream_nt);
    if constexpr (FUSED) {
        pin_scalar(fz.q_proj);
        pin_scalar(fz.k_proj);
        pin_scalar(fz.v_proj);
        pin_scalar(fz.q_norm);
        pin_scalar(fz.k_norm);
        pin_scalar(fz.rope);
        pin_scalar(fz.pairs);
        pin_scalar(fz.eps);
        pin_scalar(fz.k_cache);
        pin_scalar(fz.v_cache);
        pin_scalar(fz.head_stride);
        pin_scalar(fz.new_key);
        pin_scalar(fz.new_row);
    }
    if (bcount > 0) {
        // A compact batch: one segment, one query token at the last key.
        const int i = find_batch_entry(batch, bcount, blockIdx.x);
        const auto &e = batch->e[i];
        const int64_t kv_offset = e.kv_offset;
        const uint32_t keys = e.keys, tile_base = e.tile_base, splits = e.splits;
        const uint32_t head_stride = e.head_stride;
        const int64_t row = (int64_t)Hq * D;
        pv.tile_base = tile_base;
        pv.vis_lo = 0;
        pv.vis_hi = keys;
        pv.k_pos0 = 0;
        pv.keys = keys;
        pv.q_pos0 = (int64_t)keys - 1;
        pv.q_row_stride = row;
        pv.q = reinterpret_cast<const uint8_t *>(batch->q) + (int64_t)i * row * ES;
        pv.splits = (int32_t)splits;
        pv.split_keys = batch->split_keys;
        pv.seg_splits0 = (int32_t)splits;
        pv.seg_splits1 = 0;
        pv.queries = 1;
        pv.seg0 = DecodeSegment{reinterpret_cast<const uint8_t *>(batch->k) + kv_offset * ES,
                                reinterpret_cast<const uint8_t *>(batch->v) + kv_offset * ES,
                                (int64_t)head_stride, D, (int64_t)keys, 0};
        slot_base = tile_base;
        out = batch->out + (int64_t)i * row;
    } else if (nproblems != 1) {
        pr = (const_ptr<Problem>)p.problems + find_problem_wave(p.problems, p.nproblems, blockIdx.x);
        pv = decode_view(pr);
        slot_base = pr->slot_base;
        out = pr->out;
    }
    const uint32_t local = blockIdx.x - (uint32_t)pv.tile_base;
    const int split = (int)(local % (uint32_t)pv.splits);
    const int kvh = (int)(local / (uint32_t)pv.splits);
    const int nrows = pv.queries * G;

    // This split's segment and logical key range [a, b): splits are laid out
    // segment by segment and never straddle a boundary, so the segment's base
    // pointers and strides are uniform for the workgroup.
    int sidx = split;
    DecodeSegment sg = pv.seg0;
    if (sidx >= pv.seg_splits0) {
        sidx -= pv.seg_splits0;
        int which = 1;
        if (sidx >= pv.seg_splits1) {
            sidx -= pv.seg_splits1;
            which = 2;
        }
        sg = decode_segment(pr, which);
    }
    const int64_t seg_lo = sg.start > pv.vis_lo ? sg.start : pv.vis_lo;
    const int64_t seg_end = sg.start + sg.keys;
    const int64_t seg_hi = seg_end < pv.vis_hi ? seg_end : pv.vis_hi;
    const int64_t a = seg_lo + (int64_t)sidx * pv.split_keys;
    int64_t b = a + pv.split_keys;
    if (b > seg_hi) b = seg_hi;
    const int span = (int)(b - a);
    // Row r of key a + rel starts at kbase/vbase + rel * row_bytes.
    const int64_t seg_first = (int64_t)kvh * sg.head_stride + (a - sg.start) * sg.row_stride;
    const uint8_t *kseg = reinterpret_cast<const uint8_t *>(sg.k) + seg_first * ES + 16 * sub;
    const uint8_t *vseg = reinterpret_cast<const uint8_t *>(sg.v) + seg_first * ES + 16 * sub;
    const int64_t row_bytes = sg.row_stride * ES;

    bool bad = false;
    // Rows: visible range relative to a, and the query chunks in registers.
    int rlo[R], rhi[R];
    u32x4 q[R][CPL];
    const uint8_t *qbase = reinterpret_cast<const uint8_t *>(pv.q);
    for (int r = 0; r < R; ++r) {
        rlo[r] = 0;
        rhi[r] = 0;
        for (int c = 0; c < CPL; ++c) q[r][c] = u32x4{0, 0, 0, 0};
        if (r < nrows) {
            // r and the group are non-negative: unsigned divisions.
            const int t = (int)((uint32_t)r / (uint32_t)G), h = kvh * G + (int)((uint32_t)r % (uint32_t)G);
            int64_t lo, hi;
            visible_range(has_window != 0, window, pv.k_pos0, pv.keys, pv.q_pos0 + t, &lo, &hi);
            lo -= a;
            hi -= a;
            rlo[r] = (int)(lo < 0 ? 0 : (lo > span ? span : lo));
            rhi[r] = (int)(hi < 0 ? 0 : (hi > span ? span : hi));
            if constexpr (!FUSED) {
                const uint8_t *qrow = qbase + ((int64_t)t * pv.q_row_stride + (int64_t)h * D) * ES;
                for (int c = 0; c < CPL; ++c) q[r][c] = load16(qrow + 128 * c + 16 * sub);
            }
        }
    }
    // Fused producer: the new key is the last of the visible range, so it
    // falls in the last split.  Wave 0 of that workgroup makes its K/V row,
    // stores it into the cache, keeps a copy in LDS, and scores it after the
    // stream of the older keys (which the stream below leaves out).
    int rel_new = -1;
    int stream_span = span;
    if constexpr (FUSED) {
        const int64_t rn = fz.new_key - a;
        if (rn >= 0 && rn < span) {
            rel_new = (int)rn;
            stream_span = rel_new;  // keys after the new one: none (it is the last)
        }
    }
    // The producer's work, after the first K/V block is in flight (below):
    // one wave per row (the Q rows of this KV head and, in the workgroup
    // holding the new key, its K and V rows), packed to the cache dtype in
    // 16-byte chunks; Q rows go to LDS for every wave, the K/V rows to the
    // cache and to LDS for the scoring of the new key after the stream.
    auto produce = [&]() {
        if constexpr (FUSED) {
            const FusedDecode &f = fz;
            const int jobs = nrows + (rel_new >= 0 ? 2 : 0);
            float *row = lds_prow + wave * D;
            for (int job = wave; job < jobs; job += nw) {
                const bool is_q = job < nrows, is_k = job == nrows;
                const float *src = is_q ? f.q_proj + (int64_t)(kvh * G + job % G) * D
                                        : (is_k ? f.k_proj : f.v_proj) + (int64_t)kvh * D;
                const float *wn = is_q ? f.q_norm : (is_k ? f.k_norm : nullptr);
                float y[D / 64];
                wave_produce_row<D>(src, wn, f.eps, is_q || is_k ? f.rope : nullptr, f.pairs, lane, y,
                                    bad);
                // Regroup into 16-byte chunks of the cache dtype through LDS.
                for (int k = 0; k < D / 64; ++k) row[lane + 64 * k] = y[k];
                if (lane < ROWB / 16) {
                    const u32x4 chunk = pack_chunk<DT>(row + lane * EPC);
                    if (is_q) {
                        lds_q[job * CPL * 8 + lane] = chunk;
                    } else {
                        lds_new[(is_k ? 0 : CPL * 8) + lane] = chunk;
                        void *cache = is_k ? f.k_cache : f.v_cache;
                        const int64_t row0 = ((int64_t)kvh * f.head_stride + f.new_row * D) * ES;
                        *gstore_ptr<u32x4>(reinterpret_cast<uint8_t *>(cache) + row0 + 16 * lane) = chunk;
                    }
                }
            }
            __syncthreads();
            for (int r = 0; r < R; ++r)
                for (int c = 0; c < CPL; ++c)
                    q[r][c] = r < nrows ? lds_q[r * CPL * 8 + 8 * c + sub] : u32x4{0, 0, 0, 0};
        }
    };

    float m[R], l[R], acc[R][EPL];
    for (int r = 0; r < R; ++r) {
        m[r] = NEG_INF;
        l[r] = 0.0f;
        for (int e = 0; e < EPL; ++e) acc[r][e] = 0.0f;
    }

    const int nblk = (stream_span + KPB - 1) / KPB;

    // Every load of a block is issued, with no branch: a key past the stream
    // (in the block's tail) reads the stream's last row instead, which is in
    // bounds and which consume() masks (its rel lies past every rhi).  The
    // compiler then knows how many loads follow a block's, so consuming it
    // waits for that block only, not for the next one issued just before
    // (with loads under per-key branches it had to wait for all of them).
    auto load_block_as = [&](auto nt_tag, int blk, u32x4 (&kb)[U][CPL], u32x4 (&vb)[U][CPL]) {
        constexpr bool NT = decltype(nt_tag)::value;
        for (int u = 0; u < U; ++u) {
            const int rel = blk * KPB + kg + 8 * u;
            const int row = rel < stream_span ? rel : stream_span - 1;
            const uint8_t *kp = kseg + row * row_bytes;
            const uint8_t *vp = vseg + row * row_bytes;
            for (int c = 0; c < CPL; ++c) kb[u][c] = NT ? load16_stream(kp + 128 * c) : load16(kp + 128 * c);
            for (int c = 0; c < CPL; ++c) vb[u][c] = NT ? load16_stream(vp + 128 * c) : load16(vp + 128 * c);
        }
    };

    auto consume = [&](int blk, const u32x4 (&kb)[U][CPL], const u32x4 (&vb)[U][CPL]) {
        float s[U][R];
        for (int u = 0; u < U; ++u) {
            const int rel = blk * KPB + kg + 8 * u;
            for (int r = 0; r < R; ++r) {
                float dot = 0.0f;
                for (int c = 0; c < CPL; ++c) dot = chunk_dot<DT>(kb[u][c], q[r][c], dot);
                dot = dpp_sum8(dot);
                float x;
                if constexpr (CAP) x = tanh_fast(dot * ycap) * caplog2;
                else x = dot * scale_log2;
                const bool vis = rel >= rlo[r] && rel < rhi[r];
                bad |= vis && !is_finite_f(x);
                s[u][r] = vis ? x : NEG_INF;
            }
        }
        float m_use[R];
        bool moved = false;
        for (int r = 0; r < R; ++r) {
            float mt = s[0][r];
            for (int u = 1; u < U; ++u) mt = fmaxf(mt, s[u][r]);
            const float m_new = fmaxf(m[r], mt);
            moved |= m_new != m[r];
            m_use[r] = m_new;
        }
        if (__ballot(moved) != 0) {
            for (int r = 0; r < R; ++r) {
                const float base = m_use[r] == NEG_INF ? 0.0f : m_use[r];
                const float corr = __builtin_amdgcn_exp2f(m[r] - base);
                l[r] *= corr;
                for (int e = 0; e < EPL; ++e) acc[r][e] *= corr;
                m[r] = m_use[r];
            }
        }
        float pr_[U][R];
        for (int r = 0; r < R; ++r) {
            const float base = m[r] == NEG_INF ? 0.0f : m[r];
            for (int u = 0; u < U; ++u) {
                pr_[u][r] = __builtin_amdgcn_exp2f(s[u][r] - base);
                l[r] += pr_[u][r];
            }
        }
        for (int u = 0; u < U; ++u) {
            float vf[EPL];
            for (int c = 0; c < CPL; ++c) widen<DT>(vb[u][c], vf + c * EPC);
            for (int r = 0; r < R; ++r)
                for (int e = 0; e < EPL; ++e) acc[r][e] = __builtin_fmaf(pr_[u][r], vf[e], acc[r][e]);
        }
    };

    // The stream covers keys [0, stream_span): keys past it are never visible
    // to it (their K/V are not loaded).
    int rhi_all[R];
    for (int r = 0; r < R; ++r) {
        rhi_all[r] = rhi[r];
        if (rhi[r] > stream_span) rhi[r] = stream_span;
    }

    // Block blk + nw streams in while block blk is consumed; the last block
    // is consumed after the loop, so inside it the next block's loads are
    // always issued.  The load form (nontemporal or not) is uniform per
    // launch, so the whole stream is built once per form rather than
    // branching per block.
    auto stream = [&](auto nt_tag) {
        int blk = wave;
        u32x4 kc[U][CPL], vc[U][CPL];
        if (blk < nblk) load_block_as(nt_tag, blk, kc, vc);
        produce();
        if (blk >= nblk) return;
        for (; blk + nw < nblk; blk += nw) {
            u32x4 kn[U][CPL], vn[U][CPL];
            load_block_as(nt_tag, blk + nw, kn, vn);
            consume(blk, kc, vc);
            for (int u = 0; u < U; ++u)
                for (int c = 0; c < CPL; ++c) {
                    kc[u][c] = kn[u][c];
                    vc[u][c] = vn[u][c];
                }
        }
        consume(blk, kc, vc);
    };
    if (stream_nt) stream(std::true_type{});
    else stream(std::false_type{});

    // Fused producer: wave 0 of the workgroup holding the new key scores it
    // (lanes kg == 0 hold its chunks; the other key lanes add nothing).
    if constexpr (FUSED) {
        if (rel_new >= 0 && wave == 0) {
            u32x4 kb[U][CPL], vb[U][CPL];
            for (int u = 0; u < U; ++u)
                for (int c = 0; c < CPL; ++c) {
                    kb[u][c] = u == 0 && kg == 0 ? lds_new[(0 * CPL + c) * 8 + sub] : u32x4{0, 0, 0, 0};
                    vb[u][c] = u == 0 && kg == 0 ? lds_new[(1 * CPL + c) * 8 + sub] : u32x4{0, 0, 0, 0};
                }
            // A block index whose lane kg == 0, u == 0 key is rel_new: the
            // consume() key of (kg, u) is blk * KPB + kg + 8 u, so shift the
            // visibility bounds instead of the block.
            const int shift = rel_new;
            for (int r = 0; r < R; ++r) {
                rlo[r] -= shift;
                rhi[r] = rhi_all[r] - shift;
            }
            for (int r = 0; r < R; ++r)
                if (kg != 0) rhi[r] = rlo[r];  // only the key lanes that hold the row
            consume(0, kb, vb);
        }
    }

    // Merge the eight key lanes (lanes that hold the same chunks): reduce the
    // row maximum and mass to every lane, rescale each lane's context to the
    // maximum once, then reduce-scatter the context.  One v_permlane16_swap of
    // elements e and e + EPL/2 hands each lane its partner's copy of the half
    // it keeps (lanes 16 apart), one v_permlane32_swap does the same for the
    // quarters (lanes 32 apart), and a DPP sum adds the lanes 8 apart.  Lane
    // kg then holds elements e + (EPL/4)(kg >> 2) + (EPL/2)((kg >> 1) & 1),
    // e < EPL/4, of the row, and the lanes of even kg store them: 16 lane
    // exchanges per row at EPL 16 instead of 48 for an all-reduce.
    auto pair_max = [](auto mask_tag, float x) {
        float a, b;
        lane_pair<decltype(mask_tag)::value>(x, a, b);
        return fmaxf(a, b);
    };
    auto pair_sum = [](auto mask_tag, float x) {
        float a, b;
        lane_pair<decltype(mask_tag)::value>(x, a, b);
        return a + b;
    };
    using M8 = std::integral_constant<int, 8>;
    using M16 = std::integral_constant<int, 16>;
    using M32 = std::integral_constant<int, 32>;
    for (int r = 0; r < R; ++r) {
        float mx = pair_max(M8{}, m[r]);
        mx = pair_max(M16{}, mx);
        mx = pair_max(M32{}, mx);
        const float base = mx == NEG_INF ? 0.0f : mx;
        const float c = __builtin_amdgcn_exp2f(m[r] - base);
        m[r] = mx;
        float lr = l[r] * c;
        lr = pair_sum(M8{}, lr);
        lr = pair_sum(M16{}, lr);
        l[r] = pair_sum(M32{}, lr);
        constexpr int H1 = EPL / 2, H2 = EPL / 4;
        static_assert(EPL % 4 == 0, "the context reduce-scatter splits a lane's elements in quarters");
        float half[H1];
        for (int e = 0; e < H1; ++e) {
            const auto p16 = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, acc[r][e] * c),
                                                              __builtin_bit_cast(uint32_t, acc[r][e + H1] * c),
                                                              false, false);
            const uint32_t a = p16[0], b = p16[1];
            half[e] = __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
        }
        for (int e = 0; e < H2; ++e) {
            const auto p32 = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, half[e]),
                                                              __builtin_bit_cast(uint32_t, half[e + H2]),
                                                              false, false);
            const uint32_t a = p32[0], b = p32[1];
            acc[r][e] = pair_sum(M8{}, __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b));
        }
    }
    if ((kg & 1) == 0) {
        constexpr int H1 = EPL / 2, H2 = EPL / 4;
        const int first = H2 * (kg >> 2) + H1 * ((kg >> 1) & 1);
        for (int r = 0; r < R; ++r) {
            float *dst = lds_o + (wave * R + r) * D;
            for (int e = 0; e < H2; ++e) {
                const int idx = first + e, c = idx / EPC, j = idx - c * EPC;
                dst[(128 * c + 16 * sub) / ES + j] = acc[r][e];
            }
            if (kg == 0 && sub == 0) {
                lds_ml[(wave * R + r) * 2 + 0] = m[r];
                lds_ml[(wave * R + r) * 2 + 1] = l[r];
            }
        }
    }
    __syncthreads();

    // Merge the waves: one thread per (row, feature).
    const bool single = pv.splits == 1;
    const int64_t slot = slot_base + (int64_t)kvh * pv.splits + split;
    bool bad_mass = false, bad_out = false;
    for (int i = threadIdx.x; i < R * D; i += blockDim.x) {
        const int r = i / D, d = i - r * D;
        if (r >= nrows) continue;
        float M = NEG_INF;
        for (int w = 0; w < nw; ++w) M = fmaxf(M, lds_ml[(w * R + r) * 2]);
        const float base = M == NEG_INF ? 0.0f : M;
        float L = 0.0f, O = 0.0f;
        for (int w = 0; w < nw; ++w) {
            const float cw = __builtin_amdgcn_exp2f(lds_ml[(w * R + r) * 2] - base);
            L += cw * lds_ml[(w * R + r) * 2 + 1];
            O += cw * lds_o[(w * R + r) * D + d];
        }
        bad |= !is_finite_f(O);
        if (single) {
            const int t = r / G, h = kvh * G + r % G;
            bad_mass |= !(L > 0.0f) || !is_finite_f(L);
            const float v = O / L;
            bad_out |= !is_finite_f(v);
            gstore_ptr<float>(out)[((int64_t)t * Hq + h) * D + d] = v;
        } else if (p.merge_launch) {
            // Combined by attn_decode_merge after this kernel: the kernel
            // boundary orders the stores, so they are plain.
            p.part_o[(slot * R + r) * D + d] = O;
            if (d == 0) {
                p.part_ml[(slot * R + r) * 2 + 0] = M;
                p.part_ml[(slot * R + r) * 2 + 1] = L;
            }
        } else if (split == pv.splits - 1) {
            lds_own[r * D + d] = O;
            if (d == 0) {
                lds_own[R * D + 2 * r] = M;
                lds_own[R * D + 2 * r + 1] = L;
            }
        } else {
            split_store(p.part_o + (slot * R + r) * D + d, O);
            if (d == 0) {
                split_store(p.part_ml + (slot * R + r) * 2 + 0, M);
                split_store(p.part_ml + (slot * R + r) * 2 + 1, L);
            }
        }
    }
    raise_status(p, bad, ST_NONFINITE_INPUT);
    if (single) {
        raise_status(p, bad_mass, ST_BAD_MASS);
        raise_status(p, bad_out, ST_NONFINITE_OUTPUT);
        return;
    }
    if (p.merge_launch) return;

    // Split-K completion without atomics: every split but the last stores its
    // partial, waits until the stores are acknowledged, and then stores this
    // launch's epoch into its flag.  The last split of the KV head (its block
    // index is the head's highest, so every other split was dispatched before
    // it) keeps its own partial in LDS, waits for the other flags (bounded)
    // and merges.
    const int S = pv.splits;
    const uint32_t epoch = p.epoch;
    if (split != S - 1) {
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (threadIdx.x == 0) flag_store(p.flags + slot, epoch);
        return;
    }
    const int64_t slot0 = slot_base + (int64_t)kvh * S;
    if (wave == 0) {
        const uint64_t t_start = __builtin_amdgcn_s_memrealtime();
        bool arrived = false;
        for (;;) {
            const uint32_t f = lane < S - 1 ? flag_load(p.flags + slot0 + lane) : p.wait_epoch;
            if (__ballot(f != p.wait_epoch) == 0) {
                arrived = true;
                break;
            }
            // Bounded (p.split_wait_ticks of the 100 MHz clock, half a second
            // unless a test shortens it): then ST_SPLIT_TIMEOUT, not a hang.
            if (__builtin_amdgcn_s_memrealtime() - t_start > p.split_wait_ticks) break;
            __builtin_amdgcn_s_sleep(1);
        }
        // Every flag was seen: clear them, so no later launch that carries
        // the same epoch (a replayed graph of this launch) can take them for
        // its own.  The next launch starts after this one has ended.
        if (arrived && lane < S - 1) flag_store(p.flags + slot0 + lane, 0u);
        if (lane == 0) lds_own[R * D + 2 * R] = arrived ? 1.0f : 0.0f;
    }
    __syncthreads();
    const bool timed_out = lds_own[R * D + 2 * R] == 0.0f;
    // One wave per 64 outputs of one row (D is a multiple of 64).  Lane
    // (g4, q4) = (lane / 16, lane % 16) reads, for splits 4 g + g4, the four
    // outputs d0 + 4 q4 .. + 3 (16-byte buffer loads, sc1) and the split's
    // (max, mass); lanes past the other splits read out of the buffer's range,
    // which returns zeros and touches no memory, so the loads are issued in
    // straight runs with no branches and no repeated address: every split's
    // (max, mass) at once, then the outputs of four split groups per run (the
    // merge's registers stay below the stream's: one run over all sixteen
    // groups held 64 more).  Then: the row maximum, per-split weights, the
    // weighted sums over the lane's splits, and lane swaps over the four
    // split groups.
    const __amdgpu_buffer_rsrc_t prs =
        __builtin_amdgcn_make_buffer_rsrc(p.part_ml, 0, 0x7FFFFFFF, BUFFER_RSRC_WORD3);
    const uint32_t o_base = (uint32_t)(reinterpret_cast<const char *>(p.part_o) -
                                       reinterpret_cast<const char *>(p.part_ml));
    const int g4 = lane >> 4, q4 = lane & 15;
    const int ng = (S + 3) >> 2;
    const int chunks = R * D / 64;
    constexpr int GRUN = 4;  // split groups per run of output loads
    for (int c = wave; c < chunks && !timed_out; c += nw) {
        const int r = c * 64 / D, d = c * 64 - r * D + 4 * q4;
        if (r >= nrows) continue;  // uniform over the wave
        const uint32_t ml0 = (uint32_t)((slot0 * R + r) * 2) * 4u, ml_step = (uint32_t)R * 8u;
        const uint32_t o0 = o_base + (uint32_t)((slot0 * R + r) * D + d) * 4u, o_step = (uint32_t)(R * D) * 4u;
        f32x2 mv[DECODE_MAX_SPLITS / 4];
        for (int g = 0; g < DECODE_MAX_SPLITS / 4; ++g) {
            if (g < ng) {
                const int sp = 4 * g + g4;
                const bool theirs = sp < S - 1;
                mv[g] = __builtin_amdgcn_raw_buffer_load_b64(prs, theirs ? ml0 + (uint32_t)sp * ml_step : OUT_OF_RANGE, 0, CPOL_SC1_NT);
            }
        }
        const f32x4 own_o = *reinterpret_cast<const f32x4 *>(lds_own + r * D + d);
        const f32x2 own_ml = {lds_own[R * D + 2 * r], lds_own[R * D + 2 * r + 1]};
        float mmax = NEG_INF;
        for (int g = 0; g < DECODE_MAX_SPLITS / 4; ++g) {
            if (g < ng) {
                const int sp = 4 * g + g4;
                if (sp == S - 1) {
                    mv[g] = own_ml;
                } else if (sp >= S) {
                    mv[g][0] = NEG_INF;
                }
                mmax = fmaxf(mmax, mv[g][0]);
            }
        }
        // The lanes of one split group (same g4) read the same (max, mass)
        // words, so the row's maximum and mass need only the four groups:
        // the lanes 16 and 32 apart.
        float pa, pb;
        lane_pair<16>(mmax, pa, pb);
        lane_pair<32>(fmaxf(pa, pb), pa, pb);
        const float M = fmaxf(pa, pb);
        const float base = M == NEG_INF ? 0.0f : M;
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
        float lsum = 0.0f;
        for (int g = 0; g < DECODE_MAX_SPLITS / 4; ++g) {
            if (g < ng) lsum = __builtin_fmaf(__builtin_amdgcn_exp2f(mv[g][0] - base), mv[g][1], lsum);
        }
        for (int g0 = 0; g0 < DECODE_MAX_SPLITS / 4; g0 += GRUN) {
            if (g0 >= ng) break;  // uniform over the wave
            f32x4 ov[GRUN];
            for (int j = 0; j < GRUN; ++j) {
                const int sp = 4 * (g0 + j) + g4;
                const bool theirs = g0 + j < ng && sp < S - 1;
                ov[j] = __builtin_amdgcn_raw_buffer_load_b128(prs, theirs ? o0 + (uint32_t)sp * o_step : OUT_OF_RANGE, 0, CPOL_SC1_NT);
            }
            for (int j = 0; j < GRUN; ++j) {
                const int g = g0 + j;
                if (g < ng) {
                    const int sp = 4 * g + g4;
                    if (sp == S - 1) ov[j] = own_o;
                    const float wgt = __builtin_amdgcn_exp2f(mv[g][0] - base);
                    for (int k = 0; k < 4; ++k) acc[k] = __builtin_fmaf(wgt, ov[j][k], acc[k]);
                }
            }
        }
        lane_pair<16>(lsum, pa, pb);
        lane_pair<32>(pa + pb, pa, pb);
        const float L = pa + pb;
        for (int k = 0; k < 4; ++k) {
            float a, b;
            lane_pair<16>(acc[k], a, b);
            lane_pair<32>(a + b, a, b);
            acc[k] = a + b;
        }
        const int t = r / G, h = kvh * G + r % G;
        bad_mass |= !(L > 0.0f) || !is_finite_f(L);
        if (g4 == 0) {
            f32x4 v;
            for (int k = 0; k < 4; ++k) {
                v[k] = acc[k] / L;
                bad_out |= !is_finite_f(v[k]);
            }
            *gstore_ptr<f32x4>(out + ((int64_t)t * Hq + h) * D + d) = v;
        }
    }
    raise_status(p, timed_out, ST_SPLIT_TIMEOUT);
    raise_status(p, bad_mass, ST_BAD_MASS);
    raise_status(p, bad_out, ST_NONFINITE_OUTPUT);
}

}  // namespace tkh

namespace tkh {

// Launch of one attn_decode geometry: the softcap and fused-producer variants.
// The producer is folded in for bf16/f16 rows (head_dim 64 to 256) and, with
// the score softcap, for head_dim 256 (Gemma's sliding and global layers).
template <int DT, int DD, int RR, int UU>
hipError_t decode_launch_variant(const DecodeArgs *a, int fused, dim3 grid, dim3 block,
                                 hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
    if (fused) {
        if constexpr (DT != F32 && DD * Elem<DT>::size <= 512) {
            if (a->p.softcap != 0.0f) {
                if constexpr (DD == 256) {
                    hipExtLaunchKernelGGL((attn_decode<DT, DD, RR, UU, true, true>), grid, block, 0,
                                          stream, start, stop, 0, *a);
                    return hipGetLastError();
                }
                return hipErrorInvalidValue;
            }
            hipExtLaunchKernelGGL((attn_decode<DT, DD, RR, UU, false, true>), grid, block, 0, stream,
                                  start, stop, 0, *a);
            return hipGetLastError();
        } else {
            return hipErrorInvalidValue;
        }
    }
    if (a->p.softcap != 0.0f)
        hipExtLaunchKernelGGL((attn_decode<DT, DD, RR, UU, true, false>), grid, block, 0, stream,
                              start, stop, 0, *a);
    else
        hipExtLaunchKernelGGL((attn_decode<DT, DD, RR, UU, false, false>), grid, block, 0, stream,
                              start, stop, 0, *a);
    return hipGetLastError();
}

// Every (rows, keys per lane) build of one (dtype, head_dim): rows up to 8
// with 2 or 4 keys per lane for rows of at most 256 bytes, up to 4 with 1 or
// 2 keys for 512-byte rows, up to 2 with 1 key for 1024-byte rows.
template <int DT, int DD>
hipError_t decode_launch_unit(const DecodeArgs *p, int rows, int keys_per_lane, int fused, dim3 grid,
                              dim3 block, hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
    constexpr int ROWB = DD * Elem<DT>::size;
    constexpr int UMAX = ROWB <= 256 ? 4 : (ROWB <= 512 ? 2 : 1);
    constexpr int UMIN = UMAX > 1 ? UMAX / 2 : 1;
    constexpr int RMAX = ROWB <= 256 ? 8 : (ROWB <= 512 ? 4 : 2);
    hipError_t e = hipErrorInvalidValue;
    bool done = false;
    auto one = [&](auto r_tag, auto u_tag) {
        constexpr int R = decltype(r_tag)::value, U = decltype(u_tag)::value;
        if constexpr (R <= RMAX) {
            if (!done && rows <= R && keys_per_lane == U) {
                e = decode_launch_variant<DT, DD, R, U>(p, fused, grid, block, stream, start, stop);
                done = true;
            }
        }
    };
    auto rows_of = [&](auto u_tag) {
        one(std::integral_constant<int, 1>{}, u_tag);
        one(std::integral_constant<int, 2>{}, u_tag);
        one(std::integral_constant<int, 4>{}, u_tag);
        one(std::integral_constant<int, 8>{}, u_tag);
    };
    rows_of(std::integral_constant<int, UMIN>{});
    if constexpr (UMAX != UMIN) rows_of(std::integral_constant<int, UMAX>{});
    return e;
}

}  // namespace tkh

// One translation unit per (dtype, head_dim) instantiates its builds (they
// compile in parallel); decode.hip dispatches to them.
#define TKH_DECODE_UNIT(DT, DD, NAME)                                                          \
    hipError_t tkh_decode_launch_##NAME(const tkh::DecodeArgs *p, int rows, int keys_per_lane, \
                                        int fused, dim3 grid, dim3 block, hipStream_t stream,   \
                                        hipEvent_t start, hipEvent_t stop) {                    \
        return tkh::decode_launch_unit<tkh::DT, DD>(p, rows, keys_per_lane, fused, grid, block, \
                                                    stream, start, stop);                       \
    }
