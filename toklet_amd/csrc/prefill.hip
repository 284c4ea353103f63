// prefill.hip - gfx950 flash attention for chunks (many query rows per KV head).
//
// attn_prefill<DT, D> handles bf16/f16 calls whose query rows per KV head
// (tokens x query heads of the GQA group, "packed rows") exceed what the
// streaming decode kernel holds.  It is MFMA-bound:
//
//  * One workgroup = four waves = 128 packed rows of one (problem, KV head),
//    optionally one key split of it.  Each wave owns 32 rows.
//  * K and V tiles of 32 keys are copied once per workgroup into padded LDS
//    (double buffered: the next tile's global loads are in flight while the
//    current tile is consumed) and read by all four waves.
//  * Scores are formed transposed, S^T = K Q^T, on v_mfma_f32_32x32x16: lane
//    l holds query row l % 32 and sixteen keys of the tile, so the row's
//    softmax state lives in one lane pair (one cross-lane step per tile).
//    Q stays in registers as the B operand for the whole key range.
//  * O^T = V^T P^T on the same MFMA.  The V^T operand comes from LDS with
//    ds_read_b64_tr_b16 (each 16-lane group reads 4 keys x 16 features and
//    receives them transposed); P^T is already in B-operand layout.  For
//    bf16 the probabilities are split into a bf16 head and a bf16 remainder
//    (two MFMAs) because a single bf16 rounding of P can move the output by
//    more than 2e-3; f16 probabilities are rounded once.
//  * The online-softmax rescale of O is skipped for a tile unless some
//    row's running maximum moved.
//  * Workgroups are mapped XCD-major (dispatch slot b runs on XCD b % 8) so
//    the row blocks of one (problem, KV head) sit on one XCD and share its
//    L2 for the K/V stream.
//  * Split-K partials (max, mass, unnormalised context) use device-coherent
//    stores; the last workgroup of a row block to arrive merges them.
#include <type_traits>

#include "device.hpp"

namespace tkh {

namespace {

using f32x16 = float __attribute__((ext_vector_type(16)));
using u32x2 = uint32_t __attribute__((ext_vector_type(2)));
using i16x4 = short __attribute__((ext_vector_type(4)));
template <class T> using lds_ptr = __attribute__((address_space(3))) T *;

template <int DT> __device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c);
template <> __device__ __forceinline__ f32x16 mfma32<BF16>(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
template <> __device__ __forceinline__ f32x16 mfma32<F16>(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// Round two floats to the storage dtype (RNE) and pack them.
template <int DT> __device__ __forceinline__ uint32_t pack2(float a, float b);
template <> __device__ __forceinline__ uint32_t pack2<BF16>(float a, float b) {
    const f32x2 v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}
template <> __device__ __forceinline__ uint32_t pack2<F16>(float a, float b) {
    const f32x2 v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
}
// Widen the two halves of a packed pair.
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

__device__ __forceinline__ u32x2 read_tr(lds_ptr<uint8_t> p) {
    const i16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_ptr<i16x4>)p);
    return __builtin_bit_cast(u32x2, r);
}

__device__ __forceinline__ void coherent_store(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float coherent_load(const float *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

constexpr int PF_WAVES = 4;
constexpr int PF_ROWS = 32 * PF_WAVES;  // packed rows per workgroup
constexpr int PF_KT = 32;               // keys per tile

template <int D> struct PrefillLds {
    static constexpr int pitch = D * 2 + 16;            // bytes per staged row (bank spread)
    static constexpr int tile = PF_KT * pitch;          // one K or V tile
    static constexpr int stage = 2 * tile;              // K + V
    static constexpr int bytes = 2 * stage;             // double buffered
};

template <int DT, int D>
__global__ __launch_bounds__(64 * PF_WAVES) void attn_prefill(Params p) {
    constexpr int KS = D / 16;        // QK k-steps (16 features each)
    constexpr int MB = D / 32;        // PV M-blocks (32 features each)
    constexpr int CH = D * 2 / 16;    // 16-byte chunks per staged row
    constexpr int PITCH = PrefillLds<D>::pitch;
    constexpr bool SPLIT_P = DT == BF16;
    static_assert(D % 32 == 0, "head_dim must be a multiple of 32");

    __shared__ __attribute__((aligned(16))) uint8_t lds_raw[PrefillLds<D>::bytes];
    __shared__ int lds_last;
    lds_ptr<uint8_t> lds = (lds_ptr<uint8_t>)lds_raw;

    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int j = lane & 31;   // query row of this lane inside the wave
    const int h = lane >> 5;   // which half of the k-slots / key quads

    // XCD-major tile order: dispatch slot b runs on XCD b % 8; give each XCD
    // a contiguous range of logical tiles.
    int64_t tile;
    {
        const int64_t nb = gridDim.x;
        const int64_t per = (nb + 7) / 8;
        const int64_t x = blockIdx.x % 8, k = blockIdx.x / 8;
        const int64_t full = nb % 8 == 0 ? 8 : nb % 8;  // XCDs that receive `per` blocks
        tile = x < full ? x * per + k : full * per + (x - full) * (per - 1) + k;
    }
    const_ptr<Problem> pr = problem_ptr(p, tile);
    int64_t local = tile - pr->tile_base;
    const int rb = (int)(local % pr->row_blocks);
    local /= pr->row_blocks;
    const int split = (int)(local % pr->splits);
    const int kvh = (int)(local / pr->splits);
    const int G = p.group;
    const int Hq = p.query_heads;
    const int m_kv = pr->queries * G;

    // This lane's query row.
    const int row = rb * PF_ROWS + wave * 32 + j;
    const bool rvalid = row < m_kv;
    const int rrow = rvalid ? row : m_kv - 1;
    const int t_row = rrow / G, h_row = kvh * G + rrow % G;
    const int64_t pos = pr->q_pos0 + t_row;
    int64_t r_lo, r_hi;
    visible_range(p, pr->k_pos0, pr->keys, pos, &r_lo, &r_hi);
    if (!rvalid) r_hi = r_lo;  // no visible keys: never contributes, never stored

    // Key range of the workgroup: the union over its rows, clipped to the split.
    const int wg_row_first = rb * PF_ROWS;
    const int wg_row_last = min(wg_row_first + PF_ROWS, m_kv) - 1;
    int64_t k_lo, k_hi, tmp;
    visible_range(p, pr->k_pos0, pr->keys, pr->q_pos0 + wg_row_first / G, &k_lo, &tmp);
    visible_range(p, pr->k_pos0, pr->keys, pr->q_pos0 + wg_row_last / G, &tmp, &k_hi);
    {
        const int64_t s_lo = pr->vis_lo + (int64_t)split * pr->split_keys;
        const int64_t s_hi = s_lo + pr->split_keys;
        if (k_lo < s_lo) k_lo = s_lo;
        if (k_hi > s_hi) k_hi = s_hi;
        if (k_hi < k_lo) k_hi = k_lo;
    }
    // Keys the whole wave sees (tiles inside this need no mask).
    const int w_first = min(wg_row_first + wave * 32, m_kv - 1);
    const int w_last = min(wg_row_first + wave * 32 + 31, m_kv - 1);
    int64_t wfull_lo, wfull_hi;
    {
        int64_t a, b;
        visible_range(p, pr->k_pos0, pr->keys, pr->q_pos0 + w_first / G, &a, &wfull_hi);
        visible_range(p, pr->k_pos0, pr->keys, pr->q_pos0 + w_last / G, &wfull_lo, &b);
    }

    // Q^T B operands: lane holds row j, features 16 ks + 8 h .. + 7.
    u32x4 qb[KS];
    {
        const uint8_t *qrow = reinterpret_cast<const uint8_t *>(pr->q) +
                              ((int64_t)t_row * pr->q_row_stride + (int64_t)h_row * D) * 2;
        for (int ks = 0; ks < KS; ++ks)
            qb[ks] = *gload_ptr<u32x4>(qrow + 32 * ks + 16 * h);
    }

    f32x16 acc[MB];
    for (int mb = 0; mb < MB; ++mb)
        for (int i = 0; i < 16; ++i) acc[mb][i] = 0.0f;
    float m_run = NEG_INF, l_run = 0.0f;
    bool bad = false;
    const float scale_log2 = p.scale_log2, scale = p.scale, softcap = p.softcap;

    // ---- staging: each thread moves CPT 16-byte chunks of K and of V per tile
    constexpr int CPT = (PF_KT * CH) / (64 * PF_WAVES);
    static_assert(CPT >= 1 && (PF_KT * CH) % (64 * PF_WAVES) == 0, "tile/thread mismatch");
    u32x4 stage_k[CPT], stage_v[CPT];

    // Segment pieces of [k_lo, k_hi): tiles never straddle a segment.
    int seg = 0;
    int64_t tile_key = k_lo;  // first logical key of the next tile to load
    auto seg_end = [&](int s) { return pr->seg[s].start + pr->seg[s].keys; };
    auto advance_seg = [&]() {
        while (seg < pr->nseg - 1 && tile_key >= seg_end(seg)) ++seg;
    };
    advance_seg();

    // Load the tile starting at `key0` (inside segment `s`) into registers.
    auto load_tile = [&](int64_t key0, int s) {
        const int64_t key_end = min(k_hi, seg_end(s));
        const auto &sg = pr->seg[s];
        const uint8_t *kb = reinterpret_cast<const uint8_t *>(sg.k);
        const uint8_t *vb = reinterpret_cast<const uint8_t *>(sg.v);
        const int64_t base = (int64_t)kvh * sg.head_stride + (key0 - sg.start) * sg.row_stride;
        for (int c = 0; c < CPT; ++c) {
            const int idx = threadIdx.x + c * 64 * PF_WAVES;
            const int r = idx / CH, col = idx % CH;
            u32x4 kv = {0, 0, 0, 0}, vv = {0, 0, 0, 0};
            if (key0 + r < key_end) {
                const int64_t off = (base + (int64_t)r * sg.row_stride) * 2 + col * 16;
                kv = *gload_ptr<u32x4>(kb + off);
                vv = *gload_ptr<u32x4>(vb + off);
            }
            stage_k[c] = kv;
            stage_v[c] = vv;
        }
    };
    auto store_tile = [&](int buf) {
        lds_ptr<uint8_t> kt = lds + buf * PrefillLds<D>::stage;
        lds_ptr<uint8_t> vt = kt + PrefillLds<D>::tile;
        for (int c = 0; c < CPT; ++c) {
            const int idx = threadIdx.x + c * 64 * PF_WAVES;
            const int r = idx / CH, col = idx % CH;
            *(lds_ptr<u32x4>)(kt + r * PITCH + col * 16) = stage_k[c];
            *(lds_ptr<u32x4>)(vt + r * PITCH + col * 16) = stage_v[c];
        }
    };

    // Tile list: walk the pieces; `cur_*` describe the tile in LDS buffer `buf`.
    int buf = 0;
    bool have = tile_key < k_hi;
    int64_t cur_key = tile_key, cur_end = 0;
    if (have) {
        load_tile(tile_key, seg);
        cur_end = min(k_hi, seg_end(seg));
        tile_key = min(tile_key + PF_KT, cur_end);
        store_tile(0);
    }
    __syncthreads();
    int cur_seg = seg;
    (void)cur_seg;

    while (have) {
        // Next tile (if any) streams in while this one is consumed.
        int64_t nxt_key = tile_key;
        if (nxt_key >= cur_end) {  // this piece is done: move to the next segment
            advance_seg();
        }
        const bool more = nxt_key < k_hi;
        int64_t nxt_end = 0;
        if (more) {
            load_tile(nxt_key, seg);
            nxt_end = min(k_hi, seg_end(seg));
        }

        lds_ptr<uint8_t> kt = lds + buf * PrefillLds<D>::stage;
        lds_ptr<uint8_t> vt = kt + PrefillLds<D>::tile;
        const int nkeys = (int)min<int64_t>(PF_KT, cur_end - cur_key);

        // ---- S^T = K Q^T (32 keys x 32 rows)
        f32x16 st;
        for (int i = 0; i < 16; ++i) st[i] = 0.0f;
        for (int ks = 0; ks < KS; ++ks) {
            const u32x4 ka = *(lds_ptr<u32x4>)(kt + j * PITCH + 32 * ks + 16 * h);
            st = mfma32<DT>(ka, qb[ks], st);
        }

        // ---- scores, mask, online softmax (lane: row j, keys 8q + 4h + r)
        const bool full = nkeys == PF_KT && cur_key >= wfull_lo && cur_key + PF_KT <= wfull_hi;
        float s[16];
        float mt = NEG_INF;
        for (int i = 0; i < 16; ++i) {
            const int kk = 8 * (i >> 2) + 4 * h + (i & 3);
            float x = softcap != 0.0f ? softcap_f(st[i] * scale, softcap) * LOG2E : st[i] * scale_log2;
            bool vis = true;
            if (!full) {
                const int64_t key = cur_key + kk;
                vis = kk < nkeys && key >= r_lo && key < r_hi;
            }
            bad |= vis && !is_finite_f(x);
            x = vis ? x : NEG_INF;
            s[i] = x;
            mt = fmaxf(mt, x);
        }
        {
            const uint32_t u = __builtin_bit_cast(uint32_t, mt);
            const auto pr32 = __builtin_amdgcn_permlane32_swap(u, u, false, false);
            const uint32_t a0 = pr32[0], a1 = pr32[1];
            mt = fmaxf(__builtin_bit_cast(float, a0), __builtin_bit_cast(float, a1));
        }
        const float m_new = fmaxf(m_run, mt);
        if (__ballot(m_new != m_run) != 0) {
            const float base = m_new == NEG_INF ? 0.0f : m_new;
            const float corr = __builtin_amdgcn_exp2f(m_run - base);
            l_run *= corr;
            for (int mb = 0; mb < MB; ++mb)
                for (int i = 0; i < 16; ++i) acc[mb][i] *= corr;
            m_run = m_new;
        }
        const float base = m_run == NEG_INF ? 0.0f : m_run;
        uint32_t ph[8], pl[8];
        for (int i = 0; i < 8; ++i) {
            const float e0 = __builtin_amdgcn_exp2f(s[2 * i] - base);
            const float e1 = __builtin_amdgcn_exp2f(s[2 * i + 1] - base);
            ph[i] = pack2<DT>(e0, e1);
            if constexpr (SPLIT_P) {
                const float r0 = e0 - lo_f<DT>(ph[i]);
                const float r1 = e1 - hi_f<DT>(ph[i]);
                pl[i] = pack2<DT>(r0, r1);
                l_run += (lo_f<DT>(ph[i]) + lo_f<DT>(pl[i])) + (hi_f<DT>(ph[i]) + hi_f<DT>(pl[i]));
            } else {
                l_run += lo_f<DT>(ph[i]) + hi_f<DT>(ph[i]);
            }
        }

        // ---- O^T += V^T P^T, two 16-key steps.  B slots 8h..8h+7 of step st
        // are keys {16 st + 4h + 0..3, 16 st + 8 + 4h + 0..3} = acc quads 2st, 2st+1.
        const int gi = lane >> 4, si = lane & 15;
        for (int stp = 0; stp < 2; ++stp) {
            const u32x4 bh = {ph[4 * stp], ph[4 * stp + 1], ph[4 * stp + 2], ph[4 * stp + 3]};
            u32x4 bl = {0, 0, 0, 0};
            if constexpr (SPLIT_P) bl = u32x4{pl[4 * stp], pl[4 * stp + 1], pl[4 * stp + 2], pl[4 * stp + 3]};
            // Transposed reads: group gi covers features dbase + 0..15 of keys kb..kb+3;
            // source lane si supplies row kb + si/4, features dbase + 4 (si % 4).
            const int kb1 = 16 * stp + 4 * (gi >> 1);
            const int dsub = 16 * (gi & 1) + 4 * (si & 3);
            for (int mb = 0; mb < MB; ++mb) {
                const int dcol = (32 * mb + dsub) * 2;
                const u32x2 r1 = read_tr(vt + (kb1 + (si >> 2)) * PITCH + dcol);
                const u32x2 r2 = read_tr(vt + (kb1 + 8 + (si >> 2)) * PITCH + dcol);
                const u32x4 va = {r1[0], r1[1], r2[0], r2[1]};
                acc[mb] = mfma32<DT>(va, bh, acc[mb]);
                if constexpr (SPLIT_P) acc[mb] = mfma32<DT>(va, bl, acc[mb]);
            }
        }

        if (more) store_tile(buf ^ 1);
        __syncthreads();
        buf ^= 1;
        have = more;
        cur_key = nxt_key;
        cur_end = nxt_end;
        tile_key = min(nxt_key + PF_KT, nxt_end);
    }

    // ---- the two key halves of each row (lanes j and j + 32) share m_run; add l.
    {
        const uint32_t u = __builtin_bit_cast(uint32_t, l_run);
        const auto pr32 = __builtin_amdgcn_permlane32_swap(u, u, false, false);
        const uint32_t a0 = pr32[0], a1 = pr32[1];
        l_run = __builtin_bit_cast(float, a0) + __builtin_bit_cast(float, a1);
    }
    for (int mb = 0; mb < MB; ++mb)
        for (int i = 0; i < 16; ++i) bad |= !is_finite_f(acc[mb][i]);

    // O^T lane layout: row j, features 32 mb + 8 q + 4 h + r (register 4 q + r).
    const bool single = pr->splits == 1;
    bool bad_mass = false, bad_out = false;
    if (single) {
        if (rvalid) {
            const float inv = 1.0f / l_run;
            bad_mass |= !(l_run > 0.0f) || !is_finite_f(l_run);
            float *orow = pr->out + ((int64_t)t_row * Hq + h_row) * D;
            for (int mb = 0; mb < MB; ++mb)
                for (int q = 0; q < 4; ++q) {
                    f32x4 v;
                    for (int r = 0; r < 4; ++r) {
                        v[r] = acc[mb][4 * q + r] * inv;
                        bad_out |= !is_finite_f(v[r]);
                    }
                    *gstore_ptr<f32x4>(orow + 32 * mb + 8 * q + 4 * h) = v;
                }
        }
        raise_status(p, bad, ST_NONFINITE_INPUT);
        raise_status(p, bad_mass, ST_BAD_MASS);
        raise_status(p, bad_out, ST_NONFINITE_OUTPUT);
        return;
    }

    // ---- split-K partial: slot (row block, split) holds PF_ROWS x (D + 2)
    const int64_t group = (int64_t)kvh * pr->row_blocks + rb;
    const int64_t slot = pr->slot_base + group * pr->splits + split;
    {
        float *po = p.part_o + (slot * PF_ROWS + wave * 32 + j) * D;
        for (int mb = 0; mb < MB; ++mb)
            for (int q = 0; q < 4; ++q)
                for (int r = 0; r < 4; ++r) coherent_store(po + 32 * mb + 8 * q + 4 * h + r, acc[mb][4 * q + r]);
        if (h == 0) {
            coherent_store(p.part_ml + (slot * PF_ROWS + wave * 32 + j) * 2, m_run);
            coherent_store(p.part_ml + (slot * PF_ROWS + wave * 32 + j) * 2 + 1, l_run);
        }
    }
    raise_status(p, bad, ST_NONFINITE_INPUT);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    uint32_t *counter = p.counters + pr->group_base + group;
    if (threadIdx.x == 0)
        lds_last = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                   (uint32_t)(pr->splits - 1);
    __syncthreads();
    if (!lds_last) return;

    // ---- merge: thread per (row, 4 features); splits read in batches.
    const int S = pr->splits;
    const int64_t slot0 = pr->slot_base + group * pr->splits;
    constexpr int F4 = D / 4;
    for (int i = threadIdx.x; i < PF_ROWS * F4; i += 64 * PF_WAVES) {
        const int r = i / F4, f = (i % F4) * 4;
        const int prow = rb * PF_ROWS + r;
        if (prow >= m_kv) continue;
        float M = NEG_INF;
        for (int sp = 0; sp < S; ++sp) M = fmaxf(M, coherent_load(p.part_ml + ((slot0 + sp) * PF_ROWS + r) * 2));
        const float mbase = M == NEG_INF ? 0.0f : M;
        float L = 0.0f, o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int sp = 0; sp < S; ++sp) {
            const int64_t srow = (slot0 + sp) * PF_ROWS + r;
            const float w = __builtin_amdgcn_exp2f(coherent_load(p.part_ml + srow * 2) - mbase);
            L += w * coherent_load(p.part_ml + srow * 2 + 1);
            for (int e = 0; e < 4; ++e) o[e] += w * coherent_load(p.part_o + srow * D + f + e);
        }
        bad_mass |= !(L > 0.0f) || !is_finite_f(L);
        const int t = prow / G, hh = kvh * G + prow % G;
        f32x4 v;
        for (int e = 0; e < 4; ++e) {
            v[e] = o[e] / L;
            bad_out |= !is_finite_f(v[e]);
        }
        *gstore_ptr<f32x4>(pr->out + ((int64_t)t * Hq + hh) * D + f) = v;
    }
    if (threadIdx.x == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    raise_status(p, bad_mass, ST_BAD_MASS);
    raise_status(p, bad_out, ST_NONFINITE_OUTPUT);
}

}  // namespace tkh

extern "C" int tkh_prefill_rows_per_group(void) { return tkh::PF_ROWS; }

extern "C" hipError_t tkh_launch_prefill(const tkh::Params *p, int dtype, int head_dim,
                                         int64_t groups, hipStream_t stream) {
    using namespace tkh;
    dim3 grid((unsigned)groups), block(64 * PF_WAVES);
#define TKH_PF(DT, DD)                                                            \
    if (dtype == DT && head_dim == DD) {                                          \
        hipLaunchKernelGGL((attn_prefill<DT, DD>), grid, block, 0, stream, *p);   \
        return hipGetLastError();                                                 \
    }
    TKH_PF(BF16, 64) TKH_PF(BF16, 128) TKH_PF(BF16, 256)
    TKH_PF(F16, 64) TKH_PF(F16, 128) TKH_PF(F16, 256)
#undef TKH_PF
    return hipErrorInvalidValue;
}
