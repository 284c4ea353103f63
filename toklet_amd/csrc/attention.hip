// attention.hip - gfx950 attention kernels of the session path.
//
//  * attn_mfma<DT, D, NRB>: flash-style GQA attention on bf16/f16 MFMA with
//    FP32 accumulation.  One wave owns NRB*16 packed query rows (rows are
//    (token, query head of the KV head's group) pairs) and one split of the
//    key range; waves never synchronise with each other.  Scores are formed
//    transposed, S^T = K Q^T, so each lane holds one query row and eight keys
//    of every 32-key tile.  That puts the row's softmax state in one lane
//    (two cross-lane steps per tile instead of four) and makes the
//    probabilities already sit in the B-operand layout of O^T = V^T P^T.  V
//    is transposed through a wave-private LDS tile.
//  * attn_generic<DT>: one wave per (query, query head) with FP32 VALU math;
//    any head_dim <= 512, FP32 storage, and the optional score/probability
//    diagnostics the reference operators can return.
//  * attn_combine: merges split-K partials (max, mass, unnormalised context)
//    and publishes FP32 context only when the status word is clean.
//
// Scores are kept in the exp2 domain (score * scale * log2 e) so the softmax
// uses v_exp_f32 directly.  Masked keys contribute exactly zero.
#include "device.hpp"

namespace tkh {

template <int DT>
__device__ __forceinline__ f32x4 mfma_16x16x32(u32x4 a, u32x4 b, f32x4 c);
template <>
__device__ __forceinline__ f32x4 mfma_16x16x32<BF16>(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x4 mfma_16x16x32<F16>(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// Round two floats to the storage dtype (round to nearest even), packed.
template <int DT> __device__ __forceinline__ uint32_t pack2(float a, float b);
template <> __device__ __forceinline__ uint32_t pack2<BF16>(float a, float b) {
    f32x2 v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}
template <> __device__ __forceinline__ uint32_t pack2<F16>(float a, float b) {
    f32x2 v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
}
// Widen the low/high half of a packed pair.
template <int DT> __device__ __forceinline__ float lo_f(uint32_t w);
template <int DT> __device__ __forceinline__ float hi_f(uint32_t w);
template <> __device__ __forceinline__ float lo_f<BF16>(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
template <> __device__ __forceinline__ float hi_f<BF16>(uint32_t w) { return __builtin_bit_cast(float, w & 0xffff0000u); }
template <> __device__ __forceinline__ float lo_f<F16>(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu));
}
template <> __device__ __forceinline__ float hi_f<F16>(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
}

// ---------------------------------------------------------------------------
// MFMA flash kernel
// ---------------------------------------------------------------------------

template <int DT, int D, int NRB>
__global__ __launch_bounds__(256) void attn_mfma(Params p) {
    constexpr int KT = 32;                 // keys per tile
    constexpr int KS = D / 32;             // QK k-steps
    constexpr int DB = D / 16;             // PV d-blocks
    constexpr int PITCH = D * 2 + 8;       // LDS bytes per V row (bank-spread)
    constexpr int VCH = D / 16;            // 16-byte V chunks per lane per tile
    __shared__ __attribute__((aligned(16))) uint8_t lds_all[4][KT * PITCH];

    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int g4 = lane >> 4;
    const int l16 = lane & 15;
    const int64_t tile = (int64_t)blockIdx.x * 4 + wave;
    if (tile >= p.total_tiles) return;
    uint8_t *lds = lds_all[wave];

    const Problem &pr = tile_problem(p, tile);
    int64_t local = tile - pr.tile_base;
    const int rb = (int)(local % pr.row_blocks);
    local /= pr.row_blocks;
    const int split = (int)(local % pr.splits);
    const int kvh = (int)(local / pr.splits);
    const int G = p.group;
    const int Hq = p.query_heads;
    const int m_kv = pr.queries * G;
    const int row0 = rb * 16 * NRB;
    const int row_last = min(row0 + 16 * NRB, m_kv) - 1;

    // Query rows of this lane and their B operands (Q^T k-blocks).
    int64_t pos[NRB];
    bool rvalid[NRB];
    u32x4 qb[NRB][KS];
    const uint8_t *qbase = reinterpret_cast<const uint8_t *>(pr.q);
    for (int b = 0; b < NRB; ++b) {
        int r = row0 + b * 16 + l16;
        rvalid[b] = r < m_kv;
        int rr = rvalid[b] ? r : row_last;
        int t = rr / G, h = kvh * G + rr % G;
        pos[b] = pr.q_pos0 + t;
        const uint8_t *qrow = qbase + ((int64_t)t * pr.q_row_stride + (int64_t)h * D) * 2;
        for (int ks = 0; ks < KS; ++ks) {
            u32x4 v = {0, 0, 0, 0};
            if (rvalid[b]) v = *reinterpret_cast<const u32x4 *>(qrow + (32 * ks + 8 * g4) * 2);
            qb[b][ks] = v;
        }
    }

    // Key range shared by every row of the wave, clipped to this split.
    const int64_t pos_min = pr.q_pos0 + row0 / G;
    const int64_t pos_max = pr.q_pos0 + row_last / G;
    int64_t lo_min, hi_dummy, lo_dummy, hi_max;
    visible_range(p, pr, pos_min, &lo_min, &hi_dummy);
    visible_range(p, pr, pos_max, &lo_dummy, &hi_max);
    int64_t kb = (int64_t)split * pr.split_keys;
    int64_t ke = kb + pr.split_keys;
    if (ke > pr.keys) ke = pr.keys;
    if (kb < lo_min) kb = lo_min;
    if (ke > hi_max) ke = hi_max;

    float m_run[NRB], l_run[NRB];
    f32x4 acc[NRB][DB];
    for (int b = 0; b < NRB; ++b) {
        m_run[b] = NEG_INF;
        l_run[b] = 0.0f;
        for (int db = 0; db < DB; ++db) acc[b][db] = f32x4{0, 0, 0, 0};
    }
    bool bad = false;
    const float scale_log2 = p.scale_log2;
    const float softcap = p.softcap;

    for (int64_t j0 = kb & ~(int64_t)(KT - 1); j0 < ke; j0 += KT) {
        // ---- K tile as A operands: MFMA row m of block mb is key 8(m/4)+4mb+(m%4)
        u32x4 ka[2][KS];
        for (int mb = 0; mb < 2; ++mb) {
            int64_t key = j0 + 8 * (l16 >> 2) + 4 * mb + (l16 & 3);
            bool ok = key < ke && key >= kb;
            int which;
            int64_t off = ok ? seg_offset(pr, key, kvh, &which) : 0;
            const uint8_t *kp = reinterpret_cast<const uint8_t *>(pr.seg[ok ? which : 0].k) + off * 2;
            for (int ks = 0; ks < KS; ++ks) {
                u32x4 v = {0, 0, 0, 0};
                if (ok) v = *reinterpret_cast<const u32x4 *>(kp + (32 * ks + 8 * g4) * 2);
                ka[mb][ks] = v;
            }
        }
        // ---- V tile rows j0..j0+31 into LDS (row-major, padded pitch)
        for (int c = 0; c < VCH; ++c) {
            int e = (c * 64 + lane) * 8;  // element index within the 32 x D tile
            int row = e / D, col = e % D;
            int64_t key = j0 + row;
            u32x4 v = {0, 0, 0, 0};
            if (key < ke && key >= kb) {
                int which;
                int64_t off = seg_offset(pr, key, kvh, &which);
                v = *reinterpret_cast<const u32x4 *>(
                    reinterpret_cast<const uint8_t *>(pr.seg[which].v) + (off + col) * 2);
            }
            *reinterpret_cast<u32x4 *>(lds + row * PITCH + col * 2) = v;
        }

        // ---- S^T = K Q^T per row block
        f32x4 st[NRB][2];
        for (int b = 0; b < NRB; ++b)
            for (int mb = 0; mb < 2; ++mb) {
                f32x4 c = {0, 0, 0, 0};
                for (int ks = 0; ks < KS; ++ks) c = mfma_16x16x32<DT>(ka[mb][ks], qb[b][ks], c);
                st[b][mb] = c;
            }

        // ---- mask, online softmax, probabilities as PV B operands
        const bool tile_full = (j0 >= kb) && (j0 + KT <= ke) &&
                               (pr.k_pos0 + j0 + KT - 1 <= pos_min) &&
                               (!p.has_window || pos_max - (pr.k_pos0 + j0) < p.window);
        u32x4 pb[NRB], pl[NRB];
        for (int b = 0; b < NRB; ++b) {
            float s[8];
            for (int mb = 0; mb < 2; ++mb)
                for (int i = 0; i < 4; ++i) {
                    float x = st[b][mb][i];
                    x = softcap != 0.0f ? softcap_f(x * p.scale, softcap) * LOG2E : x * scale_log2;
                    int64_t key = j0 + 8 * g4 + 4 * mb + i;
                    bool vis = rvalid[b];
                    if (!tile_full) {
                        int64_t kp = pr.k_pos0 + key;
                        vis = vis && key < ke && key >= kb && kp <= pos[b] &&
                              (!p.has_window || pos[b] - kp < p.window);
                    }
                    bad |= vis && !is_finite_f(x);
                    s[4 * mb + i] = vis ? x : NEG_INF;
                }
            float mt = s[0];
            for (int j = 1; j < 8; ++j) mt = fmaxf(mt, s[j]);
            mt = xor_max(mt, 16);
            mt = xor_max(mt, 32);
            float m_new = fmaxf(m_run[b], mt);
            float m_use = m_new == NEG_INF ? 0.0f : m_new;
            float corr = __builtin_amdgcn_exp2f(m_run[b] - m_use);
            m_run[b] = m_new;
            float e[8];
            float sum = 0.0f;
            for (int j = 0; j < 8; ++j) {
                e[j] = __builtin_amdgcn_exp2f(s[j] - m_use);
            }
            uint32_t w[4], wl[4];
            for (int j = 0; j < 4; ++j) {
                w[j] = pack2<DT>(e[2 * j], e[2 * j + 1]);
                if constexpr (DT == BF16) {
                    float r0 = e[2 * j] - lo_f<DT>(w[j]);
                    float r1 = e[2 * j + 1] - hi_f<DT>(w[j]);
                    wl[j] = pack2<DT>(r0, r1);
                    sum += (lo_f<DT>(w[j]) + lo_f<DT>(wl[j])) + (hi_f<DT>(w[j]) + hi_f<DT>(wl[j]));
                } else {
                    sum += lo_f<DT>(w[j]) + hi_f<DT>(w[j]);
                }
            }
            l_run[b] = l_run[b] * corr + sum;
            for (int db = 0; db < DB; ++db) acc[b][db] *= corr;
            pb[b] = u32x4{w[0], w[1], w[2], w[3]};
            if constexpr (DT == BF16) pl[b] = u32x4{wl[0], wl[1], wl[2], wl[3]};
        }

        // ---- O^T += V^T P^T; V^T operand: lane holds V[8*g4 + j][16*db + l16]
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        for (int db = 0; db < DB; ++db) {
            const uint8_t *col = lds + (8 * g4) * PITCH + (16 * db + l16) * 2;
            uint32_t w[4];
            for (int j = 0; j < 4; ++j) {
                uint32_t a = *reinterpret_cast<const uint16_t *>(col + (2 * j) * PITCH);
                uint32_t c = *reinterpret_cast<const uint16_t *>(col + (2 * j + 1) * PITCH);
                w[j] = a | (c << 16);
            }
            u32x4 va = {w[0], w[1], w[2], w[3]};
            for (int b = 0; b < NRB; ++b) {
                acc[b][db] = mfma_16x16x32<DT>(va, pb[b], acc[b][db]);
                if constexpr (DT == BF16) acc[b][db] = mfma_16x16x32<DT>(va, pl[b], acc[b][db]);
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }

    // ---- partials: (max, mass, unnormalised context) per row
    for (int b = 0; b < NRB; ++b) {
        float l = l_run[b];
        l = xor_sum(l, 16);
        l = xor_sum(l, 32);
        if (!rvalid[b]) continue;
        int r = row0 + b * 16 + l16;
        int t = r / G, h = kvh * G + r % G;
        int64_t prow = pr.slot_base + ((int64_t)t * Hq + h) * pr.splits + split;
        float *po = p.part_o + prow * D;
        for (int db = 0; db < DB; ++db) {
            f32x4 v = acc[b][db];
            bad |= !(is_finite_f(v[0]) && is_finite_f(v[1]) && is_finite_f(v[2]) && is_finite_f(v[3]));
            *reinterpret_cast<f32x4 *>(po + 16 * db + 4 * g4) = v;
        }
        if (g4 == 0) {
            p.part_ml[prow * 2 + 0] = m_run[b];
            p.part_ml[prow * 2 + 1] = l;
        }
    }
    raise_status(p, bad, ST_NONFINITE_INPUT);
}

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

extern "C" hipError_t tkh_launch_mfma(const tkh::Params *p, int dtype, int head_dim, int nrb,
                                      hipStream_t stream) {
    using namespace tkh;
    dim3 grid((unsigned)((p->total_tiles + 3) / 4)), block(256);
#define TKH_MFMA_CASE(DT, DD, NR)                                                   \
    if (dtype == DT && head_dim == DD && nrb == NR) {                               \
        hipLaunchKernelGGL((attn_mfma<DT, DD, NR>), grid, block, 0, stream, *p);    \
        return hipGetLastError();                                                   \
    }
    TKH_MFMA_CASE(BF16, 64, 1) TKH_MFMA_CASE(BF16, 64, 2)
    TKH_MFMA_CASE(BF16, 128, 1) TKH_MFMA_CASE(BF16, 128, 2)
    TKH_MFMA_CASE(BF16, 256, 1)
    TKH_MFMA_CASE(F16, 64, 1) TKH_MFMA_CASE(F16, 64, 2)
    TKH_MFMA_CASE(F16, 128, 1) TKH_MFMA_CASE(F16, 128, 2)
    TKH_MFMA_CASE(F16, 256, 1)
#undef TKH_MFMA_CASE
    return hipErrorInvalidValue;
}

extern "C" hipError_t tkh_launch_generic(const tkh::Params *p, int dtype, hipStream_t stream) {
    using namespace tkh;
    dim3 grid((unsigned)p->total_tiles), block(64);
    if (dtype == F32) hipLaunchKernelGGL((attn_generic<F32>), grid, block, 0, stream, *p);
    else if (dtype == F16) hipLaunchKernelGGL((attn_generic<F16>), grid, block, 0, stream, *p);
    else if (dtype == BF16) hipLaunchKernelGGL((attn_generic<BF16>), grid, block, 0, stream, *p);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

extern "C" hipError_t tkh_launch_combine(const tkh::Params *p, int64_t total_rows,
                                         hipStream_t stream) {
    using namespace tkh;
    dim3 grid((unsigned)((total_rows + 3) / 4)), block(256);
    hipLaunchKernelGGL(attn_combine, grid, block, 0, stream, *p, total_rows);
    return hipGetLastError();
}
