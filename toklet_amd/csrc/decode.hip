// decode.hip - host-visible queries and launch dispatch of the gfx950 decode
// kernel (decode_kernel.hpp); the kernel builds live in decode_<dtype>_<D>.hip.
#include "decode_kernel.hpp"

hipError_t tkh_decode_launch_bf16_64(const tkh::DecodeArgs *, int, int, int, dim3, dim3, hipStream_t, hipEvent_t, hipEvent_t);
hipError_t tkh_decode_launch_bf16_128(const tkh::DecodeArgs *, int, int, int, dim3, dim3, hipStream_t, hipEvent_t, hipEvent_t);
hipError_t tkh_decode_launch_bf16_256(const tkh::DecodeArgs *, int, int, int, dim3, dim3, hipStream_t, hipEvent_t, hipEvent_t);
hipError_t tkh_decode_launch_f16_64(const tkh::DecodeArgs *, int, int, int, dim3, dim3, hipStream_t, hipEvent_t, hipEvent_t);
hipError_t tkh_decode_launch_f16_128(const tkh::DecodeArgs *, int, int, int, dim3, dim3, hipStream_t, hipEvent_t, hipEvent_t);
hipError_t tkh_decode_launch_f16_256(const tkh::DecodeArgs *, int, int, int, dim3, dim3, hipStream_t, hipEvent_t, hipEvent_t);
hipError_t tkh_decode_launch_f32_64(const tkh::DecodeArgs *, int, int, int, dim3, dim3, hipStream_t, hipEvent_t, hipEvent_t);
hipError_t tkh_decode_launch_f32_128(const tkh::DecodeArgs *, int, int, int, dim3, dim3, hipStream_t, hipEvent_t, hipEvent_t);
hipError_t tkh_decode_launch_f32_256(const tkh::DecodeArgs *, int, int, int, dim3, dim3, hipStream_t, hipEvent_t, hipEvent_t);

// Rows per KV head the decode kernel handles for a head_dim / dtype (0: none).
extern "C" int tkh_decode_max_rows(int dtype, int head_dim) {
    const int rowb = head_dim * (dtype == tkh::F32 ? 4 : 2);
    if (head_dim != 64 && head_dim != 128 && head_dim != 256) return 0;
    return rowb <= 256 ? 8 : (rowb <= 512 ? 4 : 2);
}

// Keys per lane per block the kernel is built with for this row size and
// rows per KV head, given the caller's preference `want` (the largest
// available value not above it).  512-byte rows take two keys per lane only
// for one row: with two rows the K/V blocks, Q and the context exceed 256
// registers and the build spills (configs[3] decode, fused: 96.7 -> 94.6 us
// per token; unfused 125 -> 114 us).
extern "C" int tkh_decode_keys_per_lane(int dtype, int head_dim, int rows, int want) {
    const int rowb = head_dim * (dtype == tkh::F32 ? 4 : 2);
    const int top = rowb <= 256 ? 4 : (rowb <= 512 ? (rows <= 1 ? 2 : 1) : 1);
    int u = 1;
    while (u * 2 <= top && u * 2 <= want) u *= 2;
    return u;
}

extern "C" int tkh_decode_max_waves(int dtype, int head_dim, int rows) {
    return tkh::decode_waves_for(head_dim * (dtype == tkh::F32 ? 4 : 2), rows);
}
extern "C" int tkh_decode_max_splits(void) { return tkh::DECODE_MAX_SPLITS; }

extern "C" hipError_t tkh_launch_decode(const tkh::DecodeArgs *p, int dtype, int head_dim, int rows,
                                        int keys_per_lane, int waves, int64_t groups, int fused,
                                        hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
    if (waves < 1 || waves > tkh_decode_max_waves(dtype, head_dim, rows)) return hipErrorInvalidValue;
    const dim3 grid((unsigned)groups), block(64 * waves);
    if (dtype == tkh::BF16 && head_dim == 64) return tkh_decode_launch_bf16_64(p, rows, keys_per_lane, fused, grid, block, stream, start, stop);
    if (dtype == tkh::BF16 && head_dim == 128) return tkh_decode_launch_bf16_128(p, rows, keys_per_lane, fused, grid, block, stream, start, stop);
    if (dtype == tkh::BF16 && head_dim == 256) return tkh_decode_launch_bf16_256(p, rows, keys_per_lane, fused, grid, block, stream, start, stop);
    if (dtype == tkh::F16 && head_dim == 64) return tkh_decode_launch_f16_64(p, rows, keys_per_lane, fused, grid, block, stream, start, stop);
    if (dtype == tkh::F16 && head_dim == 128) return tkh_decode_launch_f16_128(p, rows, keys_per_lane, fused, grid, block, stream, start, stop);
    if (dtype == tkh::F16 && head_dim == 256) return tkh_decode_launch_f16_256(p, rows, keys_per_lane, fused, grid, block, stream, start, stop);
    if (dtype == tkh::F32 && head_dim == 64) return tkh_decode_launch_f32_64(p, rows, keys_per_lane, fused, grid, block, stream, start, stop);
    if (dtype == tkh::F32 && head_dim == 128) return tkh_decode_launch_f32_128(p, rows, keys_per_lane, fused, grid, block, stream, start, stop);
    if (dtype == tkh::F32 && head_dim == 256) return tkh_decode_launch_f32_256(p, rows, keys_per_lane, fused, grid, block, stream, start, stop);
    return hipErrorInvalidValue;
}

namespace tkh {
// Split-K combine of a single-problem decode launch, as a second kernel: one
// wave per 64 outputs of one row of one KV head.  Lane (g4, q4) = (lane / 16,
// lane % 16) reads, for splits 4 g + g4, the four outputs d0 + 4 q4 .. + 3
// (16-byte buffer loads) and the split's (max, mass); lanes past the last
// split read beyond the buffer range, which returns zeros, so every load is
// issued in one straight run.  The partial slot of split s is slot_base +
// kvh * S + s with `rows` rows (the decode build's R).  Weights 2^(m_s - M)
// in the kernel's log2 units; the context is divided by the mass.
// One wave's share of the combine: 64 outputs of row r of KV head kvh of a
// problem with S splits whose partials start at slot_base.
// The launch fields the combine reads (from Params, passed on so that a
// kernel can load and pin them all before the first use).
struct MergeFields {
    int G, Hq;
    float *part_ml, *part_o;
    uint32_t *status;
};
template <int D>
__device__ __forceinline__ void merge_chunk(const MergeFields &mf, int rows, int S, int64_t slot_base,
                                            float *out, int kvh, int r, int c) {
    const int G = mf.G, Hq = mf.Hq;
    const int lane = threadIdx.x, g4 = lane >> 4, q4 = lane & 15;
    const int d = 64 * c + 4 * q4;
    const int64_t slot0 = slot_base + (int64_t)kvh * S;
    const __amdgpu_buffer_rsrc_t prs =
        __builtin_amdgcn_make_buffer_rsrc(mf.part_ml, 0, 0x7FFFFFFF, BUFFER_RSRC_WORD3);
    const uint32_t o_base = (uint32_t)(reinterpret_cast<const char *>(mf.part_o) -
                                       reinterpret_cast<const char *>(mf.part_ml));
    const uint32_t ml0 = (uint32_t)((slot0 * rows + r) * 2) * 4u, ml_step = (uint32_t)rows * 8u;
    const uint32_t o0 = o_base + (uint32_t)((slot0 * rows + r) * D + d) * 4u,
                   o_step = (uint32_t)(rows * D) * 4u;
    constexpr int NG = DECODE_MAX_SPLITS / 4;
    f32x4 ov[NG];
    f32x2 mv[NG];
#pragma unroll
    for (int g = 0; g < NG; ++g) {
        const int sp = 4 * g + g4;
        const bool in = sp < S;
        ov[g] = __builtin_amdgcn_raw_buffer_load_b128(prs, in ? o0 + (uint32_t)sp * o_step : OUT_OF_RANGE, 0, 0);
        mv[g] = __builtin_amdgcn_raw_buffer_load_b64(prs, in ? ml0 + (uint32_t)sp * ml_step : OUT_OF_RANGE, 0, 0);
    }
    // Every load is issued before the first use: left to itself the scheduler
    // interleaves the maximum's chain with the loads, and the waits for the
    // early loads then hold back the later ones (more than one memory trip).
    __builtin_amdgcn_sched_barrier(0);
    float mmax = NEG_INF;
#pragma unroll
    for (int g = 0; g < NG; ++g) {
        if (4 * g + g4 >= S) mv[g][0] = NEG_INF;
        mmax = fmaxf(mmax, mv[g][0]);
    }
    float pa, pb;
    lane_pair<16>(mmax, pa, pb);
    lane_pair<32>(fmaxf(pa, pb), pa, pb);
    const float M = fmaxf(pa, pb);
    const float base = M == NEG_INF ? 0.0f : M;
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    float lsum = 0.0f;
#pragma unroll
    for (int g = 0; g < NG; ++g) {
        const float w = __builtin_amdgcn_exp2f(mv[g][0] - base);
        for (int k = 0; k < 4; ++k) acc[k] = __builtin_fmaf(w, ov[g][k], acc[k]);
        lsum = __builtin_fmaf(w, mv[g][1], lsum);
    }
    lane_pair<16>(lsum, pa, pb);
    lane_pair<32>(pa + pb, pa, pb);
    const float L = pa + pb;
    for (int k = 0; k < 4; ++k) {
        float x, y;
        lane_pair<16>(acc[k], x, y);
        lane_pair<32>(x + y, x, y);
        acc[k] = x + y;
    }
    const bool bad_mass = !(L > 0.0f) || !is_finite_f(L);
    bool bad_out = false;
    if (g4 == 0) {
        f32x4 v;
        for (int k = 0; k < 4; ++k) {
            v[k] = acc[k] / L;
            bad_out |= !is_finite_f(v[k]);
        }
        const int t = r / G, h = kvh * G + r % G;
        *gstore_ptr<f32x4>(out + ((int64_t)t * Hq + h) * D + d) = v;
    }
    raise_status(mf.status, bad_mass, ST_BAD_MASS);
    raise_status(mf.status, bad_out, ST_NONFINITE_OUTPUT);
}

// Split-K combine of a single-problem decode launch, as a second kernel: one
// wave per 64 outputs of one row of one KV head.  Lane (g4, q4) = (lane / 16,
// lane % 16) reads, for splits 4 g + g4, the four outputs d0 + 4 q4 .. + 3
// (16-byte buffer loads) and the split's (max, mass); lanes past the last
// split read beyond the buffer range, which returns zeros, so every load is
// issued in one straight run.  The partial slot of split s is slot_base +
// kvh * S + s with `rows` rows (the decode build's R).  Weights 2^(m_s - M)
// in the kernel's log2 units; the context is divided by the mass.
template <int D>
__global__ __launch_bounds__(64) void attn_decode_merge(Params p, int rows) {
    constexpr int CH = D / 64;  // 64-output chunks per row
    // The argument fields span several lines, which the compiler read in two
    // dependent batches (the second missing on a line of its own): every line
    // is brought in at once, and the fields are read after that, as hits.
    const_ptr<Params> args = warm_kernarg_ptr<Params, (sizeof(Params) + sizeof(int) + 63) / 64, 0>();
    (void)p;
    rows = *(const_ptr<int>)((const_ptr<char>)args + sizeof(Params));
    const MergeFields mf{args->group, args->query_heads, args->part_ml, args->part_o, args->status};
    const int queries = args->single.queries, splits = args->single.splits;
    const int64_t slot_base = args->single.slot_base;
    float *out = args->single.out;
    const uint32_t nrows = (uint32_t)(queries * mf.G);
    const uint32_t b = blockIdx.x;  // non-negative: unsigned divisions
    const int c = (int)(b % CH), r = (int)((b / CH) % nrows), kvh = (int)(b / (CH * nrows));
    merge_chunk<D>(mf, rows, splits, slot_base, out, kvh, r, c);
}

// The same for a compact batch (one query token per session): the sessions
// share Hkv, the GQA group and D, so wave b serves session b / (Hkv G D/64);
// sessions with one split wrote their context themselves.
template <int D>
__global__ __launch_bounds__(64) void attn_decode_merge_batch(Params p, DecodeBatch bt, int rows) {
    constexpr int CH = D / 64;
    const int G = p.group;
    const int per = p.kv_heads * G * CH;
    const int i = blockIdx.x / per, b = blockIdx.x % per;
    const DecodeBatchEntry &e = bt.e[i];
    const int S = (int)e.splits;
    if (S <= 1) return;
    const int c = b % CH, r = (b / CH) % G, kvh = b / (CH * G);
    const MergeFields mf{p.group, p.query_heads, p.part_ml, p.part_o, p.status};
    merge_chunk<D>(mf, rows, S, (int64_t)e.tile_base, bt.out + (int64_t)i * p.query_heads * D, kvh, r, c);
}
}  // namespace tkh

extern "C" hipError_t tkh_launch_decode_merge_batch(const tkh::DecodeArgs *a, int head_dim, int rows,
                                                     hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
    using namespace tkh;
    const dim3 grid((unsigned)(a->b.count * a->p.kv_heads * a->p.group * (head_dim / 64))), block(64);
    if (head_dim == 64) hipExtLaunchKernelGGL(attn_decode_merge_batch<64>, grid, block, 0, stream, start, stop, 0, a->p, a->b, rows);
    else if (head_dim == 128) hipExtLaunchKernelGGL(attn_decode_merge_batch<128>, grid, block, 0, stream, start, stop, 0, a->p, a->b, rows);
    else if (head_dim == 256) hipExtLaunchKernelGGL(attn_decode_merge_batch<256>, grid, block, 0, stream, start, stop, 0, a->p, a->b, rows);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

extern "C" hipError_t tkh_launch_decode_merge(const tkh::Params *p, int head_dim, int rows, int kv_heads,
                                               hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
    using namespace tkh;
    const int nrows = p->single.queries * p->group;
    const dim3 grid((unsigned)(kv_heads * nrows * (head_dim / 64))), block(64);
    if (head_dim == 64) hipExtLaunchKernelGGL(attn_decode_merge<64>, grid, block, 0, stream, start, stop, 0, *p, rows);
    else if (head_dim == 128) hipExtLaunchKernelGGL(attn_decode_merge<128>, grid, block, 0, stream, start, stop, 0, *p, rows);
    else if (head_dim == 256) hipExtLaunchKernelGGL(attn_decode_merge<256>, grid, block, 0, stream, start, stop, 0, *p, rows);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}
