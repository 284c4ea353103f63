// decode.hip - gfx950 streaming decode attention (few query rows per KV head).
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
//  * At the end the eight key lanes merge by xor shuffles, the waves merge
//    through LDS, and a split either writes the context directly (one split)
//    or writes an unnormalised partial; the last workgroup of a KV head to
//    arrive (device-scope counter) merges the partials and writes the
//    context, then resets the counter.  One launch per call.
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

// The producer for one head row, in this kernel's lane layout: lane `sub` of
// an eight-lane group holds the 16-byte chunks at byte offsets 128 c + 16 sub,
// i.e. elements c * (128 / ES) + sub * EPC + i.  Loading (produce_load) is
// separate from the arithmetic (produce_row) so a caller can put every load
// in flight first.  Per-head RMSNorm (FP64 sum over the eight lanes, FP64
// scaling by the reciprocal root and the weight, rounded to FP32), then the
// rotary of pair j (elements j and j + D/2) with the given (cos, sin) and FP32
// products and sums rounded separately, then rounding to the cache dtype.
// Matches produce_qkv element for element.
template <int DT, int D> struct ProduceLayout {
    static constexpr int ES = Elem<DT>::size;
    static constexpr int CPL = D * ES / 128;
    static constexpr int EPC = 16 / ES;
    static constexpr int EPL = CPL * EPC;
    static constexpr int CE = 128 / ES;  // elements per chunk column
    // (cos, sin) floats per lane: two per first-half slot (with one chunk per
    // lane every slot of the lane is a first-half slot of its pair).
    static constexpr int CS = 2 * (CPL >= 2 ? CPL / 2 : 1) * EPC;
    // Pair index of element slot (c, i) of lane `sub` for the rotary's first
    // half; the second half's slots hold the partners.
    __device__ static int pair_of(int sub, int c, int i) {
        return CPL >= 2 ? c * CE + sub * EPC + i : (sub & 3) * EPC + i;
    }
};

// This lane's elements of a row (EPL floats).
template <int DT, int D> __device__ __forceinline__ void produce_load(const float *src, int sub, float *x) {
    using PL = ProduceLayout<DT, D>;
    for (int c = 0; c < PL::CPL; ++c)
        for (int i = 0; i < PL::EPC; i += 4) {
            const f32x4 v = *gload_ptr<f32x4>(src + c * PL::CE + sub * PL::EPC + i);
            for (int e = 0; e < 4; ++e) x[c * PL::EPC + i + e] = v[e];
        }
}
// This lane's (cos, sin) pairs, in the order produce_row consumes them
// (ProduceLayout::CS floats).
template <int DT, int D> __device__ __forceinline__ void produce_load_rope(const float *rope, int sub, float *cs) {
    using PL = ProduceLayout<DT, D>;
    constexpr int SLOTS = PL::CPL >= 2 ? PL::CPL / 2 : 1;
    for (int c = 0; c < SLOTS; ++c)
        for (int i = 0; i < PL::EPC; i += 2) {
            const f32x4 v = *gload_ptr<f32x4>(rope + 2 * PL::pair_of(sub, c, i));
            for (int e = 0; e < 4; ++e) cs[2 * (c * PL::EPC + i) + e] = v[e];
        }
}

template <int DT, int D>
__device__ __forceinline__ void produce_row(float *x, bool norm, const float *w, float eps,
                                            bool rotate, const float *cs, int pairs, int sub,
                                            u32x4 *out, bool &bad) {
#pragma clang fp contract(off)
    using PL = ProduceLayout<DT, D>;
    constexpr int CPL = PL::CPL, EPC = PL::EPC, EPL = PL::EPL;
    for (int e = 0; e < EPL; ++e) bad |= !is_finite_f(x[e]);
    if (norm) {
        double ss = 0.0;
        for (int e = 0; e < EPL; ++e) {
            const double d = (double)x[e];
            ss += d * d;
        }
        for (int m = 1; m < 8; m <<= 1) ss += __shfl_xor(ss, m, 64);
        const double inv = 1.0 / sqrt(ss / (double)D + (double)eps);
        for (int e = 0; e < EPL; ++e) {
            const float y = (float)((double)x[e] * inv * (double)w[e]);
            bad |= !is_finite_f(y) || !is_finite_f(w[e]);
            x[e] = y;
        }
    }
    if (rotate && pairs > 0) {
        if constexpr (CPL >= 2) {
            // Pair partner in the same lane, CPL / 2 chunks on.
            for (int c = 0; c < CPL / 2; ++c)
                for (int i = 0; i < EPC; ++i) {
                    if (PL::pair_of(sub, c, i) < pairs) {
                        const float co = cs[2 * (c * EPC + i)], sn = cs[2 * (c * EPC + i) + 1];
                        const float a = x[c * EPC + i], b = x[(c + CPL / 2) * EPC + i];
                        const float ac = a * co, bs = b * sn, bc = b * co, as = a * sn;
                        x[c * EPC + i] = ac - bs;
                        x[(c + CPL / 2) * EPC + i] = bc + as;
                        bad |= !is_finite_f(ac - bs) || !is_finite_f(bc + as);
                    }
                }
        } else {
            // One chunk per lane: element e pairs with e + D/2 in lane sub ^ 4.
            for (int i = 0; i < EPC; ++i) {
                const float mine = x[i];
                const float other = __shfl_xor(mine, 4, 64);
                const bool first = sub < 4;
                if (PL::pair_of(sub, 0, i) < pairs) {
                    const float co = cs[2 * i], sn = cs[2 * i + 1];
                    const float a = first ? mine : other, b = first ? other : mine;
                    const float ac = a * co, bs = b * sn, bc = b * co, as = a * sn;
                    x[i] = first ? ac - bs : bc + as;
                    bad |= !is_finite_f(x[i]);
                }
            }
        }
    }
    for (int c = 0; c < CPL; ++c) out[c] = pack_chunk<DT>(x + c * EPC);
}

// Device-coherent (agent scope) store and load of split-K partials: sc1
// write-through stores and sc1 loads, visible across the XCDs' L2 caches.
__device__ __forceinline__ void coherent_store(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float coherent_load(const float *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

constexpr int DECODE_MAX_SPLITS = 64;  // key splits per KV head (bounds the merge)

// Waves per workgroup the kernel is built for: eight when the rows and the
// row size leave room in the register file (256 VGPRs per lane), else four.
constexpr int decode_waves_for(int row_bytes, int rows) { return rows <= 2 && row_bytes <= 512 ? 8 : 4; }

template <int DT, int D, int R, int U, bool CAP, bool FUSED>
__global__ __launch_bounds__(64 * decode_waves_for(D * Elem<DT>::size, R)) void attn_decode(Params p) {
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
    __shared__ float lds_w[DECODE_MAX_SPLITS * R];
    __shared__ float lds_l[DECODE_MAX_SPLITS * R];
    __shared__ float lds_mass[R];
    __shared__ int lds_last;
    __shared__ u32x4 lds_new[FUSED ? 2 * CPL * 8 : 1];  // fused: the new K/V row (chunk c of lane sub)

    const int nw = blockDim.x >> 6;
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int sub = lane & 7;   // which chunks of the row
    const int kg = lane >> 3;   // which key of the block

    const_ptr<Problem> pr = problem_ptr(p, blockIdx.x);
    const int64_t local = (int64_t)blockIdx.x - pr->tile_base;
    const int split = (int)(local % pr->splits);
    const int kvh = (int)(local / pr->splits);
    const int G = p.group;
    const int Hq = p.query_heads;
    const int nrows = pr->queries * G;

    // This split's segment and logical key range [a, b): splits are laid out
    // segment by segment and never straddle a boundary, so the segment's base
    // pointers and strides are uniform for the workgroup.
    int seg = 0, sidx = split;
    if (sidx >= pr->seg_splits[0]) {
        sidx -= pr->seg_splits[0];
        seg = 1;
        if (sidx >= pr->seg_splits[1]) {
            sidx -= pr->seg_splits[1];
            seg = 2;
        }
    }
    const int64_t seg_lo = pr->seg[seg].start > pr->vis_lo ? pr->seg[seg].start : pr->vis_lo;
    const int64_t seg_end = pr->seg[seg].start + pr->seg[seg].keys;
    const int64_t seg_hi = seg_end < pr->vis_hi ? seg_end : pr->vis_hi;
    const int64_t a = seg_lo + (int64_t)sidx * pr->split_keys;
    int64_t b = a + pr->split_keys;
    if (b > seg_hi) b = seg_hi;
    const int span = (int)(b - a);
    // Row r of key a + rel starts at kbase/vbase + rel * row_bytes.
    const int64_t seg_first = (int64_t)kvh * pr->seg[seg].head_stride +
                              (a - pr->seg[seg].start) * pr->seg[seg].row_stride;
    const uint8_t *kseg = reinterpret_cast<const uint8_t *>(pr->seg[seg].k) + seg_first * ES + 16 * sub;
    const uint8_t *vseg = reinterpret_cast<const uint8_t *>(pr->seg[seg].v) + seg_first * ES + 16 * sub;
    const int64_t row_bytes = pr->seg[seg].row_stride * ES;

    bool bad = false;
    // Rows: visible range relative to a, and the query chunks in registers.
    int rlo[R], rhi[R];
    u32x4 q[R][CPL];
    const uint8_t *qbase = reinterpret_cast<const uint8_t *>(pr->q);
    for (int r = 0; r < R; ++r) {
        rlo[r] = 0;
        rhi[r] = 0;
        for (int c = 0; c < CPL; ++c) q[r][c] = u32x4{0, 0, 0, 0};
        if (r < nrows) {
            const int t = r / G, h = kvh * G + r % G;
            int64_t lo, hi;
            visible_range(p, pr->k_pos0, pr->keys, pr->q_pos0 + t, &lo, &hi);
            lo -= a;
            hi -= a;
            rlo[r] = (int)(lo < 0 ? 0 : (lo > span ? span : lo));
            rhi[r] = (int)(hi < 0 ? 0 : (hi > span ? span : hi));
            if constexpr (!FUSED) {
                const uint8_t *qrow = qbase + ((int64_t)t * pr->q_row_stride + (int64_t)h * D) * ES;
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
        const int64_t rn = p.fused.new_key - a;
        if (rn >= 0 && rn < span) {
            rel_new = (int)rn;
            stream_span = rel_new;  // keys after the new one: none (it is the last)
        }
    }
    // The producer's work, after the first K/V block is in flight (below).
    auto produce = [&]() {
        if constexpr (FUSED) {
            // Every load first (Q rows, and for wave 0 of the workgroup holding
            // the new key its K and V rows), then the arithmetic.
            const FusedDecode &f = p.fused;
            const bool make_kv = rel_new >= 0 && wave == 0;
            float xq[R][EPL], wq[EPL], cs[ProduceLayout<DT, D>::CS], xk[EPL], wk[EPL], xv[EPL];
            for (int r = 0; r < R; ++r)
                if (r < nrows) produce_load<DT, D>(f.q_proj + (int64_t)(kvh * G + r % G) * D, sub, xq[r]);
            if (f.q_norm) produce_load<DT, D>(f.q_norm, sub, wq);
            if (f.rope) produce_load_rope<DT, D>(f.rope, sub, cs);
            if (make_kv) {
                produce_load<DT, D>(f.k_proj + (int64_t)kvh * D, sub, xk);
                produce_load<DT, D>(f.v_proj + (int64_t)kvh * D, sub, xv);
                if (f.k_norm) produce_load<DT, D>(f.k_norm, sub, wk);
            }
            const bool rot = f.rope != nullptr;
            for (int r = 0; r < R; ++r)
                if (r < nrows)
                    produce_row<DT, D>(xq[r], f.q_norm != nullptr, wq, f.eps, rot, cs, f.pairs, sub,
                                       q[r], bad);
            if (make_kv) {
                u32x4 knew[CPL], vnew[CPL];
                produce_row<DT, D>(xk, f.k_norm != nullptr, wk, f.eps, rot, cs, f.pairs, sub, knew, bad);
                produce_row<DT, D>(xv, false, wk, 0.0f, false, cs, 0, sub, vnew, bad);
                if (kg == 0) {
                    const int64_t row0 = ((int64_t)kvh * f.head_stride + f.new_key * D) * ES;
                    for (int c = 0; c < CPL; ++c) {
                        *gstore_ptr<u32x4>(reinterpret_cast<uint8_t *>(f.k_cache) + row0 + 128 * c + 16 * sub) = knew[c];
                        *gstore_ptr<u32x4>(reinterpret_cast<uint8_t *>(f.v_cache) + row0 + 128 * c + 16 * sub) = vnew[c];
                        lds_new[(0 * CPL + c) * 8 + sub] = knew[c];
                        lds_new[(1 * CPL + c) * 8 + sub] = vnew[c];
                    }
                }
            }
        }
    };

    float m[R], l[R], acc[R][EPL];
    for (int r = 0; r < R; ++r) {
        m[r] = NEG_INF;
        l[r] = 0.0f;
        for (int e = 0; e < EPL; ++e) acc[r][e] = 0.0f;
    }
    const float scale_log2 = p.scale_log2;
    const float scale = p.scale;
    const float softcap = p.softcap, softcap_inv = p.softcap_inv;

    const int nblk = (stream_span + KPB - 1) / KPB;

    auto load_block = [&](int blk, u32x4 (&kb)[U][CPL], u32x4 (&vb)[U][CPL]) {
        for (int u = 0; u < U; ++u) {
            const int rel = blk * KPB + kg + 8 * u;
            if (rel < stream_span) {
                const uint8_t *kp = kseg + rel * row_bytes;
                const uint8_t *vp = vseg + rel * row_bytes;
                for (int c = 0; c < CPL; ++c) kb[u][c] = load16(kp + 128 * c);
                for (int c = 0; c < CPL; ++c) vb[u][c] = load16(vp + 128 * c);
            } else {
                for (int c = 0; c < CPL; ++c) {
                    kb[u][c] = u32x4{0, 0, 0, 0};
                    vb[u][c] = u32x4{0, 0, 0, 0};
                }
            }
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
                if constexpr (CAP) x = softcap_fast(dot * scale, softcap, softcap_inv) * LOG2E;
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

    // Block blk + nw streams in while block blk is consumed.
    int blk = wave;
    u32x4 kc[U][CPL], vc[U][CPL];
    if (blk < nblk) load_block(blk, kc, vc);
    produce();
    if (blk < nblk) {
        for (;;) {
            const bool more = blk + nw < nblk;
            u32x4 kn[U][CPL], vn[U][CPL];
            if (more) load_block(blk + nw, kn, vn);
            consume(blk, kc, vc);
            if (!more) break;
            for (int u = 0; u < U; ++u)
                for (int c = 0; c < CPL; ++c) {
                    kc[u][c] = kn[u][c];
                    vc[u][c] = vn[u][c];
                }
            blk += nw;
        }
    }

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
    // row maximum, rescale each lane's state to it once, then sum-reduce.
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
        for (int e = 0; e < EPL; ++e) {
            float x = acc[r][e] * c;
            x = pair_sum(M8{}, x);
            x = pair_sum(M16{}, x);
            acc[r][e] = pair_sum(M32{}, x);
        }
    }
    if (kg == 0) {
        for (int r = 0; r < R; ++r) {
            float *dst = lds_o + (wave * R + r) * D;
            for (int c = 0; c < CPL; ++c)
                for (int j = 0; j < EPC; ++j) dst[(128 * c + 16 * sub) / ES + j] = acc[r][c * EPC + j];
            if (sub == 0) {
                lds_ml[(wave * R + r) * 2 + 0] = m[r];
                lds_ml[(wave * R + r) * 2 + 1] = l[r];
            }
        }
    }
    __syncthreads();

    // Merge the waves: one thread per (row, feature).
    const bool single = pr->splits == 1;
    const int64_t slot = pr->slot_base + (int64_t)kvh * pr->splits + split;
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
            gstore_ptr<float>(pr->out)[((int64_t)t * Hq + h) * D + d] = v;
        } else {
            coherent_store(p.part_o + (slot * R + r) * D + d, O);
            if (d == 0) {
                coherent_store(p.part_ml + (slot * R + r) * 2 + 0, M);
                coherent_store(p.part_ml + (slot * R + r) * 2 + 1, L);
            }
        }
    }
    raise_status(p, bad, ST_NONFINITE_INPUT);
    if (single) {
        raise_status(p, bad_mass, ST_BAD_MASS);
        raise_status(p, bad_out, ST_NONFINITE_OUTPUT);
        return;
    }

    // Split-K: the last workgroup of this KV head to arrive merges the partials.
    // The partials went out as device-coherent (write-through) stores; once
    // they are acknowledged (vmcnt 0) and the workgroup has synchronised, one
    // lane counts the arrival.  The merging workgroup reads them with
    // device-coherent loads.  No L2-wide write-back/invalidate is needed.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    uint32_t *counter = p.counters + pr->group_base + kvh;
    if (threadIdx.x == 0)
        lds_last = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                   (uint32_t)(pr->splits - 1);
    __syncthreads();
    if (!lds_last) return;
    const int64_t slot0 = pr->slot_base + (int64_t)kvh * pr->splits;
    const int S = pr->splits;
    const int OUT = R * D;
    const int nt = blockDim.x;
    // Threads per output when the workgroup is wider than the output (P > 1,
    // a power of two): thread (k, o) handles splits k, k + P, ...
    const int P = nt >= OUT ? nt / OUT : 1;
    const int o0 = threadIdx.x % OUT, k0 = nt >= OUT ? threadIdx.x / OUT : 0;
    constexpr int VB = 32;  // partial loads per thread issued together
    // One round trip: (max, mass) of every (split, row) into LDS, and this
    // thread's first VB partial contexts into registers.
    for (int i = threadIdx.x; i < S * R; i += nt) {
        lds_w[i] = coherent_load(p.part_ml + (slot0 * R + i) * 2);
        lds_l[i] = coherent_load(p.part_ml + (slot0 * R + i) * 2 + 1);
    }
    float v0[VB];
    {
        const int r = o0 / D;
        for (int j = 0; j < VB; ++j) {
            const int sp = k0 + j * P;
            v0[j] = (nt >= OUT && r < nrows && sp < S)
                        ? coherent_load(p.part_o + ((slot0 + sp) * R) * D + o0) : 0.0f;
        }
    }
    __syncthreads();
    // Per row (one wave each): global maximum, split weights 2^(m_s - M), total mass.
    for (int r = wave; r < R; r += nw) {
        float M = NEG_INF;
        for (int sp = lane; sp < S; sp += 64) M = fmaxf(M, lds_w[sp * R + r]);
        M = wave_max(M);
        const float base = M == NEG_INF ? 0.0f : M;
        float L = 0.0f;
        for (int sp = lane; sp < S; sp += 64) {
            const float w = __builtin_amdgcn_exp2f(lds_w[sp * R + r] - base);
            lds_w[sp * R + r] = w;
            L += w * lds_l[sp * R + r];
        }
        L = wave_sum(L);
        if (lane == 0) lds_mass[r] = L;
    }
    __syncthreads();
    if (nt >= OUT) {
        // Weighted sum of this thread's splits, then the P shares through LDS.
        const int r = o0 / D;
        float O = 0.0f;
        if (r < nrows) {
            for (int j = 0; j < VB; ++j) {
                const int sp = k0 + j * P;
                if (sp < S) O = __builtin_fmaf(lds_w[sp * R + r], v0[j], O);
            }
            for (int base = VB * P; base < S; base += VB * P) {
                float v[VB];
                for (int j = 0; j < VB; ++j) {
                    const int sp = base + k0 + j * P;
                    v[j] = sp < S ? coherent_load(p.part_o + ((slot0 + sp) * R) * D + o0) : 0.0f;
                }
                for (int j = 0; j < VB; ++j) {
                    const int sp = base + k0 + j * P;
                    if (sp < S) O = __builtin_fmaf(lds_w[sp * R + r], v[j], O);
                }
            }
        }
        lds_o[k0 * OUT + o0] = O;
        __syncthreads();
        if (k0 == 0 && r < nrows) {
            float total = 0.0f;
            for (int k = 0; k < P; ++k) total += lds_o[k * OUT + o0];
            const float L = lds_mass[r];
            const int d = o0 - r * D;
            const int t = r / G, h = kvh * G + r % G;
            bad_mass |= !(L > 0.0f) || !is_finite_f(L);
            const float v = total / L;
            bad_out |= !is_finite_f(v);
            gstore_ptr<float>(pr->out)[((int64_t)t * Hq + h) * D + d] = v;
        }
    } else {
        // More outputs than threads: each thread loops over outputs.
        for (int i = threadIdx.x; i < OUT; i += nt) {
            const int r = i / D, d = i - r * D;
            if (r >= nrows) continue;
            float O = 0.0f;
            int sp = 0;
            for (; sp + VB <= S; sp += VB) {
                float v[VB];
                for (int j = 0; j < VB; ++j) v[j] = coherent_load(p.part_o + ((slot0 + sp + j) * R + r) * D + d);
                for (int j = 0; j < VB; ++j) O = __builtin_fmaf(lds_w[(sp + j) * R + r], v[j], O);
            }
            for (; sp < S; ++sp)
                O = __builtin_fmaf(lds_w[sp * R + r], coherent_load(p.part_o + ((slot0 + sp) * R + r) * D + d), O);
            const float L = lds_mass[r];
            const int t = r / G, h = kvh * G + r % G;
            bad_mass |= !(L > 0.0f) || !is_finite_f(L);
            const float v = O / L;
            bad_out |= !is_finite_f(v);
            gstore_ptr<float>(pr->out)[((int64_t)t * Hq + h) * D + d] = v;
        }
    }
    if (threadIdx.x == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    raise_status(p, bad_mass, ST_BAD_MASS);
    raise_status(p, bad_out, ST_NONFINITE_OUTPUT);
}

}  // namespace tkh

// Rows per KV head the decode kernel handles for a head_dim / dtype (0: none).
extern "C" int tkh_decode_max_rows(int dtype, int head_dim) {
    const int rowb = head_dim * (dtype == tkh::F32 ? 4 : 2);
    if (head_dim != 64 && head_dim != 128 && head_dim != 256) return 0;
    return rowb <= 256 ? 8 : (rowb <= 512 ? 4 : 2);
}

// Keys per lane per block the kernel is built with for this row size, given
// the caller's preference `want` (the largest available value not above it).
extern "C" int tkh_decode_keys_per_lane(int dtype, int head_dim, int want) {
    const int rowb = head_dim * (dtype == tkh::F32 ? 4 : 2);
    const int top = rowb <= 256 ? 4 : (rowb <= 512 ? 2 : 1);
    int u = 1;
    while (u * 2 <= top && u * 2 <= want) u *= 2;
    return u;
}

extern "C" int tkh_decode_max_waves(int dtype, int head_dim, int rows) {
    return tkh::decode_waves_for(head_dim * (dtype == tkh::F32 ? 4 : 2), rows);
}
extern "C" int tkh_decode_max_splits(void) { return tkh::DECODE_MAX_SPLITS; }

namespace {
// The softcap and fused-producer variants of one geometry.  The producer is
// folded in only for rows of at most 256 bytes (its per-lane row copy fits the
// register budget there).
template <int DT, int DD, int RR, int UU>
hipError_t launch_variant(const tkh::Params *p, int fused, dim3 grid, dim3 block,
                          hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
    using namespace tkh;
    if (fused) {
        if constexpr (DD * Elem<DT>::size <= 256) {
            if (p->softcap != 0.0f) return hipErrorInvalidValue;
            hipExtLaunchKernelGGL((attn_decode<DT, DD, RR, UU, false, true>), grid, block, 0, stream,
                                  start, stop, 0, *p);
            return hipGetLastError();
        } else {
            return hipErrorInvalidValue;
        }
    }
    if (p->softcap != 0.0f)
        hipExtLaunchKernelGGL((attn_decode<DT, DD, RR, UU, true, false>), grid, block, 0, stream,
                              start, stop, 0, *p);
    else
        hipExtLaunchKernelGGL((attn_decode<DT, DD, RR, UU, false, false>), grid, block, 0, stream,
                              start, stop, 0, *p);
    return hipGetLastError();
}
}  // namespace

extern "C" hipError_t tkh_launch_decode(const tkh::Params *p, int dtype, int head_dim, int rows,
                                        int keys_per_lane, int waves, int64_t groups, int fused,
                                        hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
    using namespace tkh;
    if (waves < 1 || waves > tkh_decode_max_waves(dtype, head_dim, rows)) return hipErrorInvalidValue;
    dim3 grid((unsigned)groups), block(64 * waves);
#define TKH_DEC(DT, DD, RR, UU)                                                             \
    if (dtype == DT && head_dim == DD && rows <= RR && keys_per_lane == UU) {               \
        return launch_variant<DT, DD, RR, UU>(p, fused, grid, block, stream, start, stop); \
    }
#define TKH_DEC_R(DT, DD, UU) TKH_DEC(DT, DD, 1, UU) TKH_DEC(DT, DD, 2, UU) TKH_DEC(DT, DD, 4, UU) TKH_DEC(DT, DD, 8, UU)
#define TKH_DEC_R4(DT, DD, UU) TKH_DEC(DT, DD, 1, UU) TKH_DEC(DT, DD, 2, UU) TKH_DEC(DT, DD, 4, UU)
    // 128- and 256-byte rows: 2 or 4 keys per lane.
    TKH_DEC_R(BF16, 64, 2) TKH_DEC_R(BF16, 64, 4) TKH_DEC_R(BF16, 128, 2) TKH_DEC_R(BF16, 128, 4)
    TKH_DEC_R(F16, 64, 2) TKH_DEC_R(F16, 64, 4) TKH_DEC_R(F16, 128, 2) TKH_DEC_R(F16, 128, 4)
    TKH_DEC_R(F32, 64, 2) TKH_DEC_R(F32, 64, 4)
    // 512-byte rows: 1 or 2 keys per lane.
    TKH_DEC_R4(BF16, 256, 1) TKH_DEC_R4(BF16, 256, 2) TKH_DEC_R4(F16, 256, 1) TKH_DEC_R4(F16, 256, 2)
    TKH_DEC_R4(F32, 128, 1) TKH_DEC_R4(F32, 128, 2)
    // 1024-byte rows.
    TKH_DEC(F32, 256, 1, 1) TKH_DEC(F32, 256, 2, 1)
#undef TKH_DEC_R4
#undef TKH_DEC_R
#undef TKH_DEC
    return hipErrorInvalidValue;
}
