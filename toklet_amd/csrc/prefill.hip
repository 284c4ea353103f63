// prefill.hip - gfx950 flash attention for chunks (many query rows per KV head).
//
// attn_prefill<DT, D> handles bf16/f16 calls whose query rows per KV head
// (tokens x query heads of the GQA group, "packed rows") exceed what the
// streaming decode kernel holds.  It is MFMA-bound:
//
//  * One workgroup = four waves = 128 packed rows of one (problem, KV head),
//    optionally one key split of it.  Each wave owns 32 rows.
//  * K and V tiles of 32 keys are copied once per workgroup into an LDS ring
//    by direct global->LDS loads, two tiles ahead of the two in use, and read
//    by all four waves.  The scores of tile t + 1 are formed while the
//    softmax and P.V of tile t run (software pipeline).
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
//  * Split-K partials (max, mass, unnormalised context) go to the workspace
//    and a second, fully parallel kernel (attn_prefill_merge) combines them,
//    so no single workgroup reads a whole row block's partials.
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

// Direct global->LDS 16-byte load for each lane: lane i's 16 bytes land at
// LDS address `l` + 16 i.  Issued as inline assembly so that the compiler,
// which cannot prove these LDS writes apart from the tile being read, does not
// put a full vmcnt(0) wait before every LDS read; ring_sync() orders them.
__device__ __forceinline__ void dma16(const void *g, lds_ptr<uint8_t> l) {
    const uint32_t m = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)l);  // wave-uniform
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(m) : "memory", "m0");
}

__device__ __forceinline__ int64_t uniform64(int64_t x) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)x);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)x >> 32));
    return (int64_t)(((uint64_t)hi << 32) | lo);
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

// LDS ring of K/V tiles.  Rows are unpadded (2D bytes) with the 16-byte
// chunks XOR-swizzled by row, so the K-operand and transposed V reads spread
// over the banks; direct global->LDS loads fill whole 1 KiB runs per wave
// instruction.  Three tiles are in flight ahead of the one being consumed
// (two for head_dim 256, where a stage is 32 KiB).
template <int D> struct PrefillLds {
    static constexpr int row = D * 2;                      // bytes per staged row
    static constexpr int chunks = row / 16;                // 16-byte chunks per row
    // Chunk swizzle of row r: XOR with (2r + r/4) mod 8.  Eight consecutive
    // rows (a K-operand read) get eight distinct 16-byte bank groups, and the
    // four rows of a transposed V read keep their two-chunk pairs disjoint.
    __device__ static constexpr int swz(int r) { return (2 * r + (r >> 2)) & 7; }
    static constexpr int tile = PF_KT * row;               // one K or V tile
    static constexpr int stage = 2 * tile;                 // K + V
    static constexpr int stages = D >= 256 ? 3 : 4;
    static constexpr int bytes = stages * stage;
    static constexpr int runs = tile / 1024;               // 1 KiB runs per tile
    static constexpr int runs_per_wave = runs / PF_WAVES;
    static_assert(runs % PF_WAVES == 0, "tile runs must split evenly over the waves");
    // Byte offset of chunk `c` of row `r` inside a tile.
    __device__ static constexpr int at(int r, int c) { return r * row + ((c ^ swz(r)) << 4); }
};

// Wait until at most `ahead` later tiles' direct loads of this wave are in
// flight, then synchronise the workgroup.  Direct global->LDS loads count in
// vmcnt; the compiler neither tracks nor orders them, hence the explicit wait
// and the compiler fences around the barrier.
template <int LPT> __device__ __forceinline__ void ring_sync(int ahead) {
    static_assert(LPT * 2 < 64, "vmcnt field");
    auto wait = [](auto n_tag) {
        constexpr int n = decltype(n_tag)::value;
        // gfx9 s_waitcnt: vmcnt in [3:0] and [15:14], expcnt [6:4], lgkmcnt [11:8].
        __builtin_amdgcn_s_waitcnt((n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8));
    };
    if (ahead >= 2) wait(std::integral_constant<int, 2 * LPT>{});
    else if (ahead == 1) wait(std::integral_constant<int, LPT>{});
    else wait(std::integral_constant<int, 0>{});
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
}

template <int DT, int D, bool CAP>
__global__ __launch_bounds__(64 * PF_WAVES) __attribute__((amdgpu_waves_per_eu(2))) void attn_prefill(Params p) {
    constexpr int KS = D / 16;        // QK k-steps (16 features each)
    constexpr int MB = D / 32;        // PV M-blocks (32 features each)
    constexpr bool SPLIT_P = DT == BF16;
    static_assert(D % 32 == 0, "head_dim must be a multiple of 32");

    __shared__ __attribute__((aligned(16))) uint8_t lds_raw[PrefillLds<D>::bytes];
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
        // Wave-uniform by construction; say so, so the full-tile test is a scalar branch.
        wfull_lo = uniform64(wfull_lo);
        wfull_hi = uniform64(wfull_hi);
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
    // Raw-score extremes over the visible range: +/-inf inputs show up here,
    // NaN propagates into the mass and the context.
    float raw_max = NEG_INF, raw_min = -NEG_INF;
    const float scale = p.scale, softcap = p.softcap, softcap_inv = p.softcap_inv;
    const float tmul = CAP ? 1.0f : p.scale_log2;  // t units -> log2 units

    // ---- tiles: walk [k_lo, k_hi) segment by segment in steps of PF_KT keys.
    using L = PrefillLds<D>;
    constexpr int NS = L::stages;
    constexpr int LPT = 2 * L::runs_per_wave;  // direct loads per wave per tile (K + V)

    // The segment piece tiles are issued from, cached in scalars.
    int iseg = 0;
    const uint8_t *pk = nullptr, *pv = nullptr;  // row of logical key `pstart`, this KV head
    int64_t pstart = 0, pend = 0;
    int prow = 0;                                // bytes between consecutive keys
    auto enter_piece = [&](int64_t key) {
        while (iseg < pr->nseg - 1 && key >= pr->seg[iseg].start + pr->seg[iseg].keys) ++iseg;
        const auto &sg = pr->seg[iseg];
        pstart = sg.start;
        pend = min(k_hi, sg.start + sg.keys);
        prow = (int)(sg.row_stride * 2);
        pk = reinterpret_cast<const uint8_t *>(sg.k) + (int64_t)kvh * sg.head_stride * 2;
        pv = reinterpret_cast<const uint8_t *>(sg.v) + (int64_t)kvh * sg.head_stride * 2;
    };
    int64_t ikey = k_lo;  // first key of the next tile to issue
    if (ikey < k_hi) enter_piece(ikey);

    // Per-lane part of the direct-load addresses (row in the tile, swizzled chunk).
    int run_row[L::runs_per_wave], run_col[L::runs_per_wave];
    for (int i = 0; i < L::runs_per_wave; ++i) {
        const int pos = (wave * L::runs_per_wave + i) * 1024 + lane * 16;
        run_row[i] = pos / L::row;
        run_col[i] = (((pos % L::row) >> 4) ^ L::swz(run_row[i])) * 16;
    }
    // Issue the tile at `ikey` into stage `st`; returns its key count.
    auto issue = [&](int st) -> int {
        const int nk = (int)min<int64_t>(PF_KT, pend - ikey);
        const int64_t first = (ikey - pstart) * prow;
        const uint8_t *kb = pk + first, *vb = pv + first;
        lds_ptr<uint8_t> kt = lds + st * L::stage;
        for (int i = 0; i < L::runs_per_wave; ++i) {
            const int run = wave * L::runs_per_wave + i;
            const int re = run_row[i] < nk ? run_row[i] : nk - 1;  // past the keys: repeat a valid row
            const uint32_t off = (uint32_t)(re * prow + run_col[i]);
            dma16(kb + off, kt + run * 1024);
            dma16(vb + off, kt + L::tile + run * 1024);
        }
        ikey += nk;
        if (ikey >= pend && ikey < k_hi) enter_piece(ikey);
        return nk;
    };

    // Queue of issued tiles (first key, key count), oldest first.
    int64_t qk[NS - 1];
    int qn[NS - 1];
    int queued = 0;
    for (int i = 0; i < NS - 1; ++i) {
        qk[i] = ikey;
        qn[i] = 0;
        if (ikey < k_hi) {
            qn[i] = issue(i);
            ++queued;
        }
    }
    // LDS offsets of this lane's operand reads (tile-relative).
    int k_off[KS];
    for (int ks = 0; ks < KS; ++ks) k_off[ks] = L::at(j, 2 * ks + h);
    const int gi = lane >> 4, si = lane & 15;
    int v_off[2][2][MB];
    for (int stp = 0; stp < 2; ++stp) {
        const int kr1 = 16 * stp + 4 * (gi >> 1) + (si >> 2);
        const int dsub = 16 * (gi & 1) + 4 * (si & 3);
        for (int mb = 0; mb < MB; ++mb) {
            const int db = (32 * mb + dsub) * 2;  // byte offset of the 4 features in a row
            v_off[stp][0][mb] = L::at(kr1, db >> 4) + (db & 15);
            v_off[stp][1][mb] = L::at(kr1 + 8, db >> 4) + (db & 15);
        }
    }

    // S^T = K Q^T of the tile in stage `stg` (32 keys x 32 rows); lane: row j,
    // keys 8q + 4h + r.
    auto scores_of = [&](int stg) {
        lds_ptr<uint8_t> kt = lds + stg * L::stage;
        f32x16 sc;
        for (int i = 0; i < 16; ++i) sc[i] = 0.0f;
        for (int ks = 0; ks < KS; ++ks)
            sc = mfma32<DT>(*(lds_ptr<u32x4>)(kt + k_off[ks]), qb[ks], sc);
        return sc;
    };

    // Software pipeline: iteration t forms the scores of tile t + 1 while it
    // runs the softmax and P.V of tile t, so the matrix cores have independent
    // work while the vector unit computes probabilities.
    int stage = 0;
    f32x16 st;
    if (queued > 0) {
        ring_sync<LPT>(queued - 1);
        st = scores_of(0);
    }
    while (queued > 0) {
        const int64_t cur_key = qk[0];
        const int nkeys = qn[0];
        const bool next = queued > 1;
        f32x16 st_next;
        const int stage_next = stage + 1 == NS ? 0 : stage + 1;
        lds_ptr<uint8_t> vt = lds + stage * L::stage + L::tile;
        lds_ptr<uint8_t> kn = lds + stage_next * L::stage;
        const int stage_free = stage == 0 ? NS - 1 : stage - 1;
        stage = stage_next;

        // ---- scores, mask, online softmax.  t = raw dot (or, with the softcap,
        // the capped score in log2 units); p = 2^(t * tmul - m * tmul), where
        // both transforms are increasing so the tile maximum follows from the
        // raw maximum.
        float t[16];
        for (int i = 0; i < 16; ++i) {
            if constexpr (CAP) t[i] = softcap_fast(st[i] * scale, softcap, softcap_inv) * LOG2E;
            else t[i] = st[i];
        }
        const bool full = nkeys == PF_KT && cur_key >= wfull_lo && cur_key + PF_KT <= wfull_hi;
        float hi, lo;
        if (full) {
            hi = fmaxf(fmaxf(st[0], st[1]), st[2]);
            lo = fminf(fminf(st[0], st[1]), st[2]);
            for (int i = 3; i < 16; ++i) {
                hi = fmaxf(hi, st[i]);
                lo = fminf(lo, st[i]);
            }
        } else {
            // Visible keys of this row inside the tile: [lo_rel, hi_rel).
            const int64_t a = r_lo - cur_key, b = min(r_hi, cur_key + nkeys) - cur_key;
            const int lo_rel = (int)(a < 0 ? 0 : (a > PF_KT ? PF_KT : a));
            const int hi_rel = (int)(b < 0 ? 0 : (b > PF_KT ? PF_KT : b));
            hi = NEG_INF;
            lo = -NEG_INF;
            for (int i = 0; i < 16; ++i) {
                const int kk = 8 * (i >> 2) + 4 * h + (i & 3);
                const bool vis = kk >= lo_rel && kk < hi_rel;
                hi = fmaxf(hi, vis ? st[i] : NEG_INF);
                lo = fminf(lo, vis ? st[i] : -NEG_INF);
                t[i] = vis ? t[i] : NEG_INF;
            }
        }
        raw_max = fmaxf(raw_max, hi);
        raw_min = fminf(raw_min, lo);
        float mt;
        if constexpr (CAP) mt = hi == NEG_INF ? NEG_INF : softcap_fast(hi * scale, softcap, softcap_inv) * LOG2E;
        else mt = hi;
        {
            const uint32_t u = __builtin_bit_cast(uint32_t, mt);
            const auto pr32 = __builtin_amdgcn_permlane32_swap(u, u, false, false);
            const uint32_t a0 = pr32[0], a1 = pr32[1];
            mt = fmaxf(__builtin_bit_cast(float, a0), __builtin_bit_cast(float, a1));
        }
        const float m_new = fmaxf(m_run, mt);
        if (__ballot(m_new != m_run) != 0) {
            const float corr = m_new == NEG_INF ? 1.0f : __builtin_amdgcn_exp2f((m_run - m_new) * tmul);
            l_run *= corr;
            for (int mb = 0; mb < MB; ++mb)
                for (int i = 0; i < 16; ++i) acc[mb][i] *= corr;
            m_run = m_new;
        }
        const float nbase = m_run == NEG_INF ? 0.0f : -m_run * tmul;

        if (next) {
            // Tile t + 1 resident; everyone is done with tile t - 1, whose stage
            // takes the next load.
            ring_sync<LPT>(queued - 2);
            const int64_t new_key = ikey;
            int new_n = 0;
            if (ikey < k_hi) new_n = issue(stage_free);
            for (int i = 0; i < NS - 2; ++i) {
                qk[i] = qk[i + 1];
                qn[i] = qn[i + 1];
            }
            qk[NS - 2] = new_key;
            qn[NS - 2] = new_n;
            queued = queued - 1 + (new_n > 0 ? 1 : 0);
        } else {
            queued = 0;
        }

        // Scores of tile t + 1 interleaved with the probabilities of tile t:
        // each QK MFMA (its K operand read one step ahead) is followed by a
        // share of the exp/pack work, the order fixed by scheduling fences so
        // the vector unit runs while the matrix core works.  With no next tile
        // the stage holds stale data and the result is unused.
        uint32_t ph[8], pl[8];
        for (int i = 0; i < 16; ++i) st_next[i] = 0.0f;
        u32x4 kop = *(lds_ptr<u32x4>)(kn + k_off[0]);
        for (int ks = 0; ks < KS; ++ks) {
            const u32x4 kcur = kop;
            if (ks + 1 < KS) kop = *(lds_ptr<u32x4>)(kn + k_off[ks + 1]);
            st_next = mfma32<DT>(kcur, qb[ks], st_next);
            __builtin_amdgcn_sched_barrier(0);
            for (int i = 8 * ks / KS; i < 8 * (ks + 1) / KS; ++i) {
                const float e0 = __builtin_amdgcn_exp2f(__builtin_fmaf(t[2 * i], tmul, nbase));
                const float e1 = __builtin_amdgcn_exp2f(__builtin_fmaf(t[2 * i + 1], tmul, nbase));
                ph[i] = pack2<DT>(e0, e1);
                if constexpr (SPLIT_P) pl[i] = pack2<DT>(e0 - lo_f<DT>(ph[i]), e1 - hi_f<DT>(ph[i]));
                l_run += e0 + e1;
            }
            __builtin_amdgcn_sched_barrier(0);
        }

        // ---- O^T += V^T P^T, two 16-key steps.  B slots 8h..8h+7 of step st
        // are keys {16 st + 4h + 0..3, 16 st + 8 + 4h + 0..3} = acc quads 2st, 2st+1.
        // V^T rows come transposed from LDS: group gi of 16 lanes reads features
        // 32 mb + 16 (gi & 1) + 0..15 of keys kb..kb+3; source lane si supplies row
        // kb + si / 4, features + 4 (si % 4).
        for (int stp = 0; stp < 2; ++stp) {
            const u32x4 bh = {ph[4 * stp], ph[4 * stp + 1], ph[4 * stp + 2], ph[4 * stp + 3]};
            u32x4 bl = {0, 0, 0, 0};
            if constexpr (SPLIT_P) bl = u32x4{pl[4 * stp], pl[4 * stp + 1], pl[4 * stp + 2], pl[4 * stp + 3]};
            for (int mb = 0; mb < MB; ++mb) {
                const u32x2 r1 = read_tr(vt + v_off[stp][0][mb]);
                const u32x2 r2 = read_tr(vt + v_off[stp][1][mb]);
                const u32x4 va = {r1[0], r1[1], r2[0], r2[1]};
                acc[mb] = mfma32<DT>(va, bh, acc[mb]);
                if constexpr (SPLIT_P) acc[mb] = mfma32<DT>(va, bl, acc[mb]);
            }
        }
        if (next) st = st_next;
    }
    bool bad = raw_max == -NEG_INF || raw_min == NEG_INF;  // an infinite visible score

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
    // floats, merged by attn_prefill_merge after this kernel.
    raise_status(p, bad, ST_NONFINITE_INPUT);
    const int64_t group = (int64_t)kvh * pr->row_blocks + rb;
    const int64_t slot = pr->slot_base + group * pr->splits + split;
    float *po = p.part_o + (slot * PF_ROWS + wave * 32 + j) * D;
    for (int mb = 0; mb < MB; ++mb)
        for (int q = 0; q < 4; ++q) {
            const f32x4 v = {acc[mb][4 * q], acc[mb][4 * q + 1], acc[mb][4 * q + 2], acc[mb][4 * q + 3]};
            *gstore_ptr<f32x4>(po + 32 * mb + 8 * q + 4 * h) = v;
        }
    if (h == 0) {
        const f32x2 ml = {m_run, l_run};
        *gstore_ptr<f32x2>(p.part_ml + (slot * PF_ROWS + wave * 32 + j) * 2) = ml;
    }
}

// Merge of the split-K partials of attn_prefill.  Merge block b covers
// PF_MERGE_ROWS packed rows of one (problem, KV head, row block); each thread
// owns four features of one row and reads the S partials of its row at once
// (one round trip): m and l of every split, then the weighted sum of the
// unnormalised contexts.  Problem::part_base is the problem's first merge block.
template <int D>
__global__ __launch_bounds__(256) void attn_prefill_merge(Params p, int64_t blocks) {
    constexpr int TPR = D / 4;                  // threads per row
    constexpr int RPB = 256 / TPR;              // rows per merge block
    constexpr int MAXS = 16;
    const int64_t b = blockIdx.x;
    if (b >= blocks) return;
    const_ptr<Problem> pr;
    if (p.nproblems == 1) {
        pr = &((const_ptr<Params>)__builtin_amdgcn_kernarg_segment_ptr())->single;
    } else {
        const_ptr<Problem> probs = (const_ptr<Problem>)p.problems;
        int lo = 0, hi = p.nproblems - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (probs[mid].part_base <= b) lo = mid; else hi = mid - 1;
        }
        pr = probs + lo;
    }
    const int G = p.group, Hq = p.query_heads;
    const int m_kv = pr->queries * G;
    const int64_t local = b - pr->part_base;
    const int blocks_per_rb = PF_ROWS / RPB;
    const int64_t group = local / blocks_per_rb;          // kvh * row_blocks + rb
    const int kvh = (int)(group / pr->row_blocks), rb = (int)(group % pr->row_blocks);
    const int r = (int)(local % blocks_per_rb) * RPB + (int)(threadIdx.x / TPR);
    const int f = (int)(threadIdx.x % TPR) * 4;
    const int prow = rb * PF_ROWS + r;
    if (prow >= m_kv) return;
    const int S = pr->splits;
    const int64_t slot0 = pr->slot_base + group * S;

    f32x2 ml[MAXS];
    f32x4 po[MAXS];
#pragma unroll
    for (int sp = 0; sp < MAXS; ++sp) {
        if (sp < S) {
            const int64_t srow = (slot0 + sp) * PF_ROWS + r;
            ml[sp] = *gload_ptr<f32x2>(p.part_ml + srow * 2);
            po[sp] = *gload_ptr<f32x4>(p.part_o + srow * D + f);
        }
    }
    float M = NEG_INF;
#pragma unroll
    for (int sp = 0; sp < MAXS; ++sp)
        if (sp < S) M = fmaxf(M, ml[sp][0]);
    const float mbase = M == NEG_INF ? 0.0f : M;
    const float tmul = p.softcap != 0.0f ? 1.0f : p.scale_log2;
    float L = 0.0f;
    f32x4 o = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int sp = 0; sp < MAXS; ++sp) {
        if (sp < S) {
            const float w = ml[sp][0] == NEG_INF ? 0.0f : __builtin_amdgcn_exp2f((ml[sp][0] - mbase) * tmul);
            L += w * ml[sp][1];
            for (int e = 0; e < 4; ++e) o[e] += w * po[sp][e];
        }
    }
    const bool bad_mass = !(L > 0.0f) || !is_finite_f(L);
    const float inv = 1.0f / L;
    bool bad_out = false;
    f32x4 v;
    for (int e = 0; e < 4; ++e) {
        v[e] = o[e] * inv;
        bad_out |= !is_finite_f(v[e]);
    }
    const int t = prow / G, hh = kvh * G + prow % G;
    *gstore_ptr<f32x4>(pr->out + ((int64_t)t * Hq + hh) * D + f) = v;
    raise_status(p, bad_mass, ST_BAD_MASS);
    raise_status(p, bad_out, ST_NONFINITE_OUTPUT);
}

}  // namespace tkh

extern "C" int tkh_prefill_rows_per_group(void) { return tkh::PF_ROWS; }
extern "C" int tkh_prefill_max_splits(void) { return 16; }
extern "C" int tkh_prefill_merge_rows_per_block(int head_dim) { return 256 / (head_dim / 4); }

extern "C" hipError_t tkh_launch_prefill_merge(const tkh::Params *p, int head_dim, int64_t blocks,
                                               hipStream_t stream, hipEvent_t start,
                                               hipEvent_t stop) {
    using namespace tkh;
    dim3 grid((unsigned)blocks), block(256);
    if (head_dim == 64)
        hipExtLaunchKernelGGL((attn_prefill_merge<64>), grid, block, 0, stream, start, stop, 0, *p, blocks);
    else if (head_dim == 128)
        hipExtLaunchKernelGGL((attn_prefill_merge<128>), grid, block, 0, stream, start, stop, 0, *p, blocks);
    else if (head_dim == 256)
        hipExtLaunchKernelGGL((attn_prefill_merge<256>), grid, block, 0, stream, start, stop, 0, *p, blocks);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

extern "C" hipError_t tkh_launch_prefill(const tkh::Params *p, int dtype, int head_dim,
                                         int64_t groups, hipStream_t stream, hipEvent_t start,
                                         hipEvent_t stop) {
    using namespace tkh;
    dim3 grid((unsigned)groups), block(64 * PF_WAVES);
#define TKH_PF(DT, DD)                                                                  \
    if (dtype == DT && head_dim == DD) {                                                \
        if (p->softcap != 0.0f)                                                         \
            hipExtLaunchKernelGGL((attn_prefill<DT, DD, true>), grid, block, 0, stream, start, stop, 0, *p);  \
        else                                                                            \
            hipExtLaunchKernelGGL((attn_prefill<DT, DD, false>), grid, block, 0, stream, start, stop, 0, *p); \
        return hipGetLastError();                                                       \
    }
    TKH_PF(BF16, 64) TKH_PF(BF16, 128) TKH_PF(BF16, 256)
    TKH_PF(F16, 64) TKH_PF(F16, 128) TKH_PF(F16, 256)
#undef TKH_PF
    return hipErrorInvalidValue;
}
