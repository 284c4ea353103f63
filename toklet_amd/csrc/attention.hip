// attention.hip - generic attention kernels of the session path.
//
//  * attn_generic<DT>: one wave per (query, query head) with FP32 VALU math;
//    any head_dim <= 512, FP32 storage, and the optional score/probability
//    diagnostics the reference operators can return.  bf16/f16 chunks and
//    decode at head_dim 64/128/256 take the MFMA prefill and streaming decode
//    kernels instead.
//  * attn_combine: merges split-K partials (max, mass, unnormalised context)
//    and publishes FP32 context only when the status word is clean.
//
// Scores are kept in the exp2 domain (score * scale * log2 e) so the softmax
// uses v_exp_f32 directly.  Masked keys contribute exactly zero.
#include "device.hpp"

namespace tkh {

// ---------------------------------------------------------------------------
// Generic VALU kernel: one wave per (problem query, query head)
// ---------------------------------------------------------------------------

template <int DT>
__global__ __launch_bounds__(64) void attn_generic(Params p) {
    __shared__ float qs[512];
    const int lane = threadIdx.x;
    const int64_t tile = blockIdx.x;
    if (tile >= p.total_tiles) return;
    const Problem &pr = tile_problem(p, tile);
    const int Hq = p.query_heads, D = p.head_dim;
    const int64_t local = tile - pr.tile_base;
    const int t = (int)(local / Hq), h = (int)(local % Hq);
    const int kvh = h / p.group;
    const int64_t pos = pr.q_pos0 + t;
    int64_t lo, hi;
    visible_range(p, pr, pos, &lo, &hi);

    for (int d = lane; d < D; d += 64)
        qs[d] = load_elem<DT>(pr.q, (int64_t)t * pr.q_row_stride + (int64_t)h * D + d);
    __syncthreads();

    auto score_of = [&](int64_t key, bool *finite_ok) -> float {
        int which;
        int64_t off = seg_offset(pr, key, kvh, &which);
        const void *kbase = pr.seg[which].k;
        float dot = 0.0f;
        for (int d = 0; d < D; ++d) dot += qs[d] * load_elem<DT>(kbase, off + d);
        float x = dot * p.scale;
        if (p.softcap != 0.0f) x = softcap_f(x, p.softcap);
        *finite_ok = is_finite_f(x);
        return x;
    };

    float acc[8];
    for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
    float m = NEG_INF, l = 0.0f;
    bool bad = false;
    for (int64_t j0 = lo; j0 < hi; j0 += 64) {
        int64_t key = j0 + lane;
        float s2 = NEG_INF;
        if (key < hi) {
            bool ok;
            float x = score_of(key, &ok);
            bad |= !ok;
            s2 = x * LOG2E;
        }
        float m_new = fmaxf(m, wave_max(s2));
        float m_use = m_new == NEG_INF ? 0.0f : m_new;
        float corr = __builtin_amdgcn_exp2f(m - m_use);
        float e = __builtin_amdgcn_exp2f(s2 - m_use);
        l = l * corr + wave_sum(e);
        m = m_new;
        for (int i = 0; i < 8; ++i) acc[i] *= corr;
        int n = (int)min<int64_t>(64, hi - j0);
        for (int jj = 0; jj < n; ++jj) {
            float pj = __shfl(e, jj, 64);
            int which;
            int64_t off = seg_offset(pr, j0 + jj, kvh, &which);
            const void *vbase = pr.seg[which].v;
            for (int i = 0; i < 8; ++i) {
                int d = lane + 64 * i;
                if (d < D) acc[i] += pj * load_elem<DT>(vbase, off + d);
            }
        }
    }

    // Diagnostics: raw scores and normalised probabilities in the reference layouts.
    const bool last_row = (h == Hq - 1) && (t == pr.queries - 1);
    if (p.diag_mode == 1 || (p.diag_mode == 2 && last_row)) {
        int64_t d_lo = p.diag_mode == 1 ? 0 : lo;
        int64_t d_hi = p.diag_mode == 1 ? pr.keys : hi;
        int64_t row = p.diag_mode == 1 ? ((int64_t)h * pr.queries + t) * pr.keys : 0;
        float inv = 1.0f / l;
        for (int64_t j0 = d_lo; j0 < d_hi; j0 += 64) {
            int64_t key = j0 + lane;
            if (key >= d_hi) continue;
            bool ok;
            float x = score_of(key, &ok);
            float pr_v = (key >= lo && key < hi) ? __builtin_amdgcn_exp2f(x * LOG2E - m) * inv : 0.0f;
            if (p.scores) p.scores[row + key] = x;
            if (p.probs) p.probs[row + key] = pr_v;
        }
    }

    const int64_t prow = pr.slot_base + ((int64_t)t * Hq + h) * pr.splits;
    for (int i = 0; i < 8; ++i) {
        int d = lane + 64 * i;
        if (d < D) {
            bad |= !is_finite_f(acc[i]);
            p.part_o[prow * D + d] = acc[i];
        }
    }
    if (lane == 0) {
        p.part_ml[prow * 2 + 0] = m;
        p.part_ml[prow * 2 + 1] = l;
    }
    raise_status(p, bad, ST_NONFINITE_INPUT);
}

// ---------------------------------------------------------------------------
// Split-K combine + gated publish: one wave per output row
// ---------------------------------------------------------------------------

__device__ __forceinline__ int find_row_problem(const Params &p, int64_t row) {
    int lo = 0, hi = p.nproblems - 1;
    while (lo < hi) {
        int mid = (lo + hi + 1) >> 1;
        if (p.problems[mid].part_base <= row) lo = mid; else hi = mid - 1;
    }
    return lo;
}

__global__ __launch_bounds__(256) void attn_combine(Params p, int64_t total_rows) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= total_rows) return;
    if (__atomic_load_n(p.status, __ATOMIC_RELAXED) != 0) return;  // never publish after bad input
    const Problem &pr = p.nproblems == 1 ? p.single : p.problems[find_row_problem(p, row)];
    const int D = p.head_dim, Hq = p.query_heads;
    const int64_t local = row - pr.part_base;
    const int t = (int)(local / Hq), h = (int)(local % Hq);
    const int S = pr.splits;
    const int64_t base = pr.slot_base + local * S;
    // Lanes over splits: global max, then weights 2^(m_s - M) and the total mass.
    float M = NEG_INF;
    for (int s0 = 0; s0 < S; s0 += 64) {
        int s = s0 + lane;
        M = fmaxf(M, s < S ? p.part_ml[(base + s) * 2] : NEG_INF);
    }
    M = wave_max(M);
    float L = 0.0f;
    for (int s0 = 0; s0 < S; s0 += 64) {
        int s = s0 + lane;
        if (s < S) {
            float ms = p.part_ml[(base + s) * 2];
            float ws = ms == NEG_INF ? 0.0f : __builtin_amdgcn_exp2f(ms - M);
            L += ws * p.part_ml[(base + s) * 2 + 1];
        }
    }
    L = wave_sum(L);
    bool bad_mass = !(L > 0.0f) || !is_finite_f(L);
    float inv = 1.0f / L;
    float o[8];
    for (int i = 0; i < 8; ++i) o[i] = 0.0f;
    for (int s0 = 0; s0 < S; s0 += 64) {
        int s = s0 + lane;
        float ws = 0.0f;
        if (s < S) {
            float ms = p.part_ml[(base + s) * 2];
            ws = ms == NEG_INF ? 0.0f : __builtin_amdgcn_exp2f(ms - M);
        }
        int n = S - s0 < 64 ? S - s0 : 64;
        for (int j = 0; j < n; ++j) {
            float wj = __shfl(ws, j, 64);
            if (wj == 0.0f) continue;
            const float *src = p.part_o + (base + s0 + j) * D;
            for (int i = 0; i < 8; ++i) {
                int d = lane + 64 * i;
                if (d < D) o[i] += wj * src[d];
            }
        }
    }
    bool bad_out = false;
    float *out = pr.out + (int64_t)t * Hq * D + (int64_t)h * D;
    for (int i = 0; i < 8; ++i) {
        int d = lane + 64 * i;
        if (d < D) {
            float v = o[i] * inv;
            bad_out |= !is_finite_f(v);
            out[d] = v;
        }
    }
    raise_status(p, bad_mass, ST_BAD_MASS);
    raise_status(p, bad_out, ST_NONFINITE_OUTPUT);
}

// ---------------------------------------------------------------------------
// Launch helpers (host side, same translation unit)
// ---------------------------------------------------------------------------

}  // namespace tkh

// start/stop, when not null, are recorded around the kernel by the dispatch
// itself (hipExtLaunchKernelGGL), so profiled durations exclude the host gap
// that separate hipEventRecord calls would add.
extern "C" hipError_t tkh_launch_generic(const tkh::Params *p, int dtype, hipStream_t stream,
                                         hipEvent_t start, hipEvent_t stop) {
    using namespace tkh;
    dim3 grid((unsigned)p->total_tiles), block(64);
    if (dtype == F32)
        hipExtLaunchKernelGGL((attn_generic<F32>), grid, block, 0, stream, start, stop, 0, *p);
    else if (dtype == F16)
        hipExtLaunchKernelGGL((attn_generic<F16>), grid, block, 0, stream, start, stop, 0, *p);
    else if (dtype == BF16)
        hipExtLaunchKernelGGL((attn_generic<BF16>), grid, block, 0, stream, start, stop, 0, *p);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

extern "C" hipError_t tkh_launch_combine(const tkh::Params *p, int64_t total_rows,
                                         hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
    using namespace tkh;
    dim3 grid((unsigned)((total_rows + 3) / 4)), block(256);
    hipExtLaunchKernelGGL(attn_combine, grid, block, 0, stream, start, stop, 0, *p, total_rows);
    return hipGetLastError();
}
