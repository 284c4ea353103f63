// prefill.hip - gfx950 flash attention for chunks (many query rows per KV head).
//
// attn_prefill<DT, D> handles bf16/f16 calls whose query rows per KV head
// (tokens x query heads of the GQA group, "packed rows") exceed what the
// streaming decode kernel holds.  It is MFMA-bound:
//
//  * One workgroup = W waves of 32 packed rows each (W = 8 at head_dim 128
//    when the row blocks fill the device, 4 otherwise) of one (problem, KV
//    head), optionally one key split of it.
//  * K and V tiles of 32 keys are copied once per workgroup into an LDS ring
//    by direct global->LDS loads, two tiles ahead of the two in use, and read
//    by all waves.  The scores of tile t + 1 are formed while the
//    softmax and P.V of tile t run (software pipeline).
//  * Scores are formed transposed, S^T = K Q^T, on v_mfma_f32_32x32x16: lane
//    l holds query row l % 32 and sixteen keys of the tile, so the row's
//    softmax state lives in one lane pair (one cross-lane step per tile).
//    Q stays in registers as the B operand for the whole key range.
//  * O^T = V^T P^T on the same MFMA.  Each V tile is transposed once per
//    workgroup (ds_read_b64_tr_b16: a 16-lane group reads 4 keys x 16
//    features and receives them transposed) into a V^T buffer laid out in
//    the A operand's key order, which every wave then reads with 16-byte
//    loads; P^T is already in B-operand layout.  P is
//    rounded once to f16 for both dtypes (a single bf16 rounding of P can
//    move the output by more than 2e-3), and the row mass is summed from the
//    same rounded values (one v_dot2 with (1, 1) per pair).  For bf16 the
//    transposing pass also converts V to f16 (exact for every bf16 value from
//    2^-14 up to 65280, the largest bf16 below f16's overflow; smaller ones
//    lose at most 2^-25 absolute).  A wave whose V tile held a larger finite
//    value recomputes its rows on the vector unit in FP32 after the loop.
//  * The softmax maximum is lazy: a tile's probabilities are formed against
//    the row's base without computing the tile's own maximum, and only a
//    wave in which some row's tile mass exceeds 2^15 (a score about 15 log2
//    units above the base, a non-finite score, or a row's first tile)
//    computes the tile maximum, rescales O and forms the tile again.  A
//    max-of-magnitudes chain over the scores checks their finiteness.
//  * Workgroups are mapped XCD-major (dispatch slot b runs on XCD b % 8) so
//    the row blocks of one (problem, KV head) sit on one XCD and share its
//    L2 for the K/V stream.
//  * Split-K partials (max, mass, unnormalised context) go to the workspace
//    and a second, fully parallel kernel (attn_prefill_merge) combines them,
//    so no single workgroup reads a whole row block's partials.
//
// attn_prefill16<DT, D, CAP, W> is the same algorithm with 16 packed rows per
// wave on v_mfma_f32_16x16x32, for launches whose row blocks do not fill the
// device (session chunks, small batches) at head_dim 128 and 256.  Four waves
// make 64-row blocks (the default: twice a chunk's workgroups at the same
// partial volume), eight the 32-row kernel's 128-row block.  At head_dim 256
// a 32-row wave needs a whole SIMD's registers and a 16-row wave about half.
#include <cstddef>
#include <type_traits>
#include <utility>

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

// l + a + b for the f16 pair (a, b) packed in `w`, in one instruction.  The
// row mass is summed from the same rounded probabilities that weight V.
__device__ __forceinline__ float add_pair(uint32_t w, float l) {
    const f16x2 ones = {(_Float16)1.0f, (_Float16)1.0f};
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, w), ones, l, false);
}

// Maximum and minimum with IEEE 754-2019 maximum/minimum semantics: a NaN
// operand gives NaN.  A NaN score makes its row's probabilities, and with
// them the context, NaN, which is reported as a non-finite input whatever the
// row maximum became.  Chains of these compile to v_maximum3_f32 /
// v_minimum3_f32 (two operands per instruction) with no canonicalising moves,
// which fmaxf/fminf chains need, and no hazard padding, which the same chains
// written as inline assembly get.
__device__ __forceinline__ float maxn(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ float minn(float a, float b) { return __builtin_elementwise_minimum(a, b); }

__device__ __forceinline__ u32x2 read_tr(lds_ptr<uint8_t> p) {
    const i16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_ptr<i16x4>)p);
    return __builtin_bit_cast(u32x2, r);
}

// Direct global->LDS 16-byte load for each lane: lane i's 16 bytes land at
// LDS address `l` + 16 i.  Issued as inline assembly so that the compiler,
// which cannot prove these LDS writes apart from the tile being read, does not
// put a full vmcnt(0) wait before every LDS read; ring_sync() orders them.
// The address is a scalar base plus this lane's 32-bit offset; `m` is the
// wave-uniform LDS destination.
__device__ __forceinline__ void dma16(const void *base, uint32_t off, uint32_t m) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(m)
                 : "memory", "m0");
}

// f(std::integral_constant<int, 0>{}), ..., f(std::integral_constant<int, N - 1>{}).
template <class F, int... I>
__device__ __forceinline__ void static_for_impl(F &f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F> __device__ __forceinline__ void static_for(F &&f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
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

// Waves per workgroup (32 packed rows each).  Four, or eight at head_dim 128,
// where the registers still allow two waves per SIMD, so the V conversion and
// the tile loads, which the workgroup shares, cost each wave half as much (a
// head_dim 64 tile is only four 1 KiB load runs, and at head_dim 256 one wave
// fills a SIMD's registers).  The host takes eight only for launches whose
// row blocks fill the device: smaller ones want more, smaller workgroups.
constexpr int PF_WAVES_NARROW = 4;
__host__ __device__ constexpr int pf_wide_waves(int D) { return D == 128 ? 8 : PF_WAVES_NARROW; }
constexpr int PF_KT = 32;               // keys per tile

// LDS ring of K/V tiles.  Rows are unpadded (2D bytes) with the 16-byte
// chunks XOR-swizzled by row, so the K-operand and transposed V reads spread
// over the banks; direct global->LDS loads fill whole 1 KiB runs per wave
// instruction.  The ring has NS stages: the tile being consumed, the next
// one, and NS - 2 in flight; four (three for head_dim 256, where a stage is
// 32 KiB).  Deeper rings measured slower on the 32-session 4096-key batch
// (five stages 2%, six 3%, eight 6% with eight-wave workgroups): more tiles
// in flight per CU only add L2 pressure.
template <int D, int W> struct PrefillLds {
    static constexpr int row = D * 2;                      // bytes per staged row
    static constexpr int chunks = row / 16;                // 16-byte chunks per row
    // Chunk swizzle of row r.  Rows of 256 bytes or more (head_dim 128, 256)
    // XOR with 5r mod 16: measured on gfx950 with four waves reading a
    // K-operand pattern (row j = lane % 32, one chunk per half-wave), a
    // ds_read_b128 takes 34.6 cycles per wave, as fast as contiguous reads,
    // against 43-52 for (2r + r/4) mod 8, the earlier choice, which leaves two
    // rows of each 16-row half-wave on one bank group.  128-byte rows (head_dim
    // 64) keep (2r + r/4) mod 8, the fastest of the 3-bit swizzles measured
    // there.  The transposing V reads (ds_read_b64_tr_b16) measured the same
    // for every swizzle tried.
    __device__ static constexpr int swz(int r) {
        return D >= 128 ? (5 * r) & 15 : (2 * r + (r >> 2)) & 7;
    }
    static constexpr int tile = PF_KT * row;               // one K or V tile
    static constexpr int stages = D >= 256 ? 3 : 4;
    // Layout: the transposed V buffers, then the K tiles of the ring, then its
    // raw V tiles.  The buffers every wave reads each tile (V^T and K) come
    // first, so at head_dim 128 their offsets fit the 16-bit immediate of the
    // LDS instructions; raw V is read only by the transposing pass.
    //
    // Transposed f16 V tiles, the A operand of the P.V MFMAs, in vt_bufs
    // buffers (tile t in buffer t % vt_bufs).  Row f (a feature)
    // holds the tile's 32 keys as four 16-byte chunks: chunk c = 2 stp + h holds
    // keys 16 stp + 4 h + 0..3 and 16 stp + 8 + 4 h + 0..3, the key order of the
    // MFMA's k slots, and sits at chunk c ^ ((f / 4) % 4), so 16 consecutive rows
    // at one chunk (a 16-lane access) hit 16 distinct bank groups.
    static constexpr int vt_row = PF_KT * 2;
    static constexpr int vt_bytes = D * vt_row;
    static constexpr int vt_bufs = stages % 2 == 0 ? 2 : stages;
    static constexpr int vt_base = 0;
    static constexpr int k_base = vt_base + vt_bufs * vt_bytes;
    static constexpr int v_base = k_base + stages * tile;
    static constexpr int bytes = v_base + stages * tile;
    static constexpr int k_at(int s) { return k_base + s * tile; }   // K tile of stage s
    static constexpr int v_at(int s) { return v_base + s * tile; }   // raw V tile of stage s
    __device__ static constexpr int vt_at(int f, int c) { return f * vt_row + ((c ^ ((f >> 2) & 3)) << 4); }
    static constexpr int runs = tile / 1024;               // 1 KiB runs per tile
    static constexpr int runs_per_wave = runs / W;
    static_assert(runs % W == 0, "tile runs must split evenly over the waves");
    // Byte offset of chunk `c` of row `r` inside a tile.
    __device__ static constexpr int at(int r, int c) { return r * row + ((c ^ swz(r)) << 4); }
};

// One V tile (PF_KT keys x D as staged by the direct loads) to its transposed
// f16 form (PrefillLds::vt_at), by the whole workgroup: each thread builds
// `per` 16-byte chunks.  A 16-lane group reads four keys x 16 features with
// ds_read_b64_tr_b16 (lane j receives the four keys of feature fb + j), twice
// for the chunk's two key quads; for bf16 each pair is then widened (a shift
// and a mask) and rounded to f16 in one v_cvt_pk_f16_f32, which is exact for
// bf16 values up to 65280 and gives inf above.  Split in a read half and a
// write half so a caller can put MFMAs between.  K16: the key order of
// attn_prefill16's P.V operands (chunk c holds keys 4c .. 4c + 3 and
// 16 + 4c .. 16 + 4c + 3) instead of attn_prefill's.
template <int D, int W, bool CONV, bool K16 = false> struct VTranspose {
    using L = PrefillLds<D, W>;
    static constexpr int threads = 64 * W;
    static constexpr int per = D * 4 / threads;  // chunks per thread
    static_assert(per >= 1 && D * 4 % threads == 0, "chunks must split evenly over the threads");
    int src1[per], src2[per], dst[per];  // LDS offsets: the two key quads' reads, the write
    u32x2 a[per], b[per];
    __device__ explicit VTranspose(int tid) {
        for (int n = 0; n < per; ++n) {
            const int q = n * threads + tid;
            const int g = q >> 4, jj = q & 15;  // 16-lane group, lane in it
            const int c = g & 3, fb = 16 * (g >> 2);
            const int row = K16 ? 4 * c + (jj >> 2) : 16 * (c >> 1) + 4 * (c & 1) + (jj >> 2);
            const int fbyte = (fb + 4 * (jj & 3)) * 2;
            src1[n] = L::at(row, fbyte >> 4) + (fbyte & 15);
            src2[n] = L::at(row + (K16 ? 16 : 8), fbyte >> 4) + (fbyte & 15);
            dst[n] = L::vt_at(fb + jj, c);
        }
    }
    __device__ void read(lds_ptr<uint8_t> v) {
        for (int n = 0; n < per; ++n) {
            a[n] = read_tr(v + src1[n]);
            b[n] = read_tr(v + src2[n]);
        }
    }
    __device__ void write(lds_ptr<uint8_t> vt) {
        for (int n = 0; n < per; ++n) {
            u32x4 o = {a[n][0], a[n][1], b[n][0], b[n][1]};
            if constexpr (CONV)
                for (int j = 0; j < 4; ++j) {
                    const uint32_t w = o[j];
                    const f32x2 v = {__builtin_bit_cast(float, w << 16),
                                     __builtin_bit_cast(float, w & 0xffff0000u)};
                    o[j] = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
                }
            *(lds_ptr<u32x4>)(vt + dst[n]) = o;
        }
    }
};

// Wait until at most `ahead` later tiles' direct loads of this wave are in
// flight, then synchronise the workgroup.  Direct global->LDS loads count in
// vmcnt; the compiler neither tracks nor orders them, hence the explicit wait
// and the compiler fences around the barrier.
template <int LPT, int MAXA> __device__ __forceinline__ void ring_sync(int ahead) {
    static_assert(LPT * MAXA < 64, "vmcnt field");
    // One exact wait per possible `ahead` (a wave-uniform value): the waits
    // take immediates.
    static_for<MAXA + 1>([&](auto a_tag) {
        constexpr int a = decltype(a_tag)::value;
        constexpr int n = a * LPT;
        // gfx9 s_waitcnt: vmcnt in [3:0] and [15:14], expcnt [6:4], lgkmcnt [11:8].
        if (ahead == a || (a == MAXA && ahead > MAXA))
            __builtin_amdgcn_s_waitcnt((n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8));
    });
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
}
// ring_sync for a compile-time `ahead`: one wait, no selection.
template <int LPT, int A> __device__ __forceinline__ void ring_sync_fixed() {
    constexpr int n = A * LPT;
    static_assert(n < 64, "vmcnt field");
    __builtin_amdgcn_s_waitcnt((n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8));
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
}

// The running maximum of a row (the exp base) is moved, and O and l
// rescaled, only when a tile's mass against it exceeds MASS_LIMIT = 2^15:
// until then probabilities up to 2^15 are accumulated against the stale
// base, which f16 P (largest finite 65504) and the FP32 accumulators hold.
// The base is always a score the row has seen, so its mass stays at least 1,
// and every key within 14 log2 units of the row's maximum is a normal f16.
// (Moving the base above the maximum would send fewer tiles here but leaves
// keys a few units below a dominant one subnormal in f16.)  The final
// division by l is unchanged, so the result is the same softmax.
constexpr float MASS_LIMIT = 0x1p15f;
// The exp base of a row that has seen no score: finite (a masked score of
// -inf gives 2^-inf = 0, not NaN) and large enough that any finite visible
// score exceeds MASS_LIMIT, which sends the row's first tile to the exact path.
constexpr float BASE_NONE = 0x1p100f;

__device__ __forceinline__ int uniform32(int x) { return __builtin_amdgcn_readfirstlane(x); }

// The fields of a problem the prefill kernel reads, with the segment of the
// workgroup's split: from the problem descriptors, or built from a compact
// batch entry (one segment from key 0, causal, no splits).
struct PfView {
    const void *q;
    float *out;
    int64_t q_row_stride, q_pos0, k_pos0, keys, vis_lo, vis_hi, tile_base, slot_base;
    int32_t queries, row_blocks, splits, split_keys;
    Segment sg;
};

// The entry of a compact prefill batch that holds global workgroup `tile`, by
// the whole wave: lane i tests entry i, a ballot picks the last entry that
// starts at or before the tile.
__device__ __forceinline__ int find_prefill_entry(const_ptr<PrefillBatch> b, int count, int64_t tile) {
    const int lane = threadIdx.x & 63;
    const bool le = lane < count && b->e[lane].tile_base <= tile;
    const uint64_t m = __ballot(le);  // bit 0 is set: entry 0 starts at tile 0
    return __builtin_amdgcn_readfirstlane(63 - __builtin_clzll(m));
}

// The workgroup's logical tile and what it covers: its problem (from the
// descriptors, or built from a compact batch entry), row block, key split,
// KV head and the split's index inside its segment.
template <int D>
__device__ __forceinline__ void pf_locate(const Params &p, PfView &pv, int &rb, int &split, int &kvh, int &sidx) {
    // XCD-major tile order: dispatch slot b runs on XCD b % 8; give each XCD
    // a contiguous range of logical tiles.
    int64_t tile;
    {
        const uint32_t nb = gridDim.x;
        const uint32_t per = (nb + 7) / 8;
        const uint32_t x = blockIdx.x % 8, k = blockIdx.x / 8;
        const uint32_t full = nb % 8 == 0 ? 8 : nb % 8;  // XCDs that receive `per` blocks
        tile = (int64_t)(x < full ? x * per + k : full * per + (x - full) * (per - 1) + k);
    }
    const int Hq = p.query_heads;
    {
        const_ptr<PrefillArgs> args = (const_ptr<PrefillArgs>)__builtin_amdgcn_kernarg_segment_ptr();
        const_ptr<PrefillBatch> batch = &args->b;
        const int bcount = batch->count;
        if (bcount > 0) {
            // A compact batch: one segment from key 0, no key splits.
            const int i = find_prefill_entry(batch, bcount, tile);
            const auto &e = batch->e[i];
            const int64_t tokens = batch->tokens, position = e.position;
            const int64_t step = batch->q_step * i;
            pv.q = reinterpret_cast<const uint8_t *>(batch->q) + step * 2;
            pv.out = batch->out + step;
            pv.q_row_stride = (int64_t)Hq * D;
            pv.q_pos0 = position;
            pv.k_pos0 = 0;
            pv.keys = position + tokens;
            pv.vis_lo = 0;
            pv.vis_hi = position + tokens;
            pv.tile_base = e.tile_base;
            pv.slot_base = 0;
            pv.queries = (int32_t)tokens;
            pv.row_blocks = batch->row_blocks;
            pv.splits = 1;
            pv.split_keys = batch->split_keys;
            pv.sg = Segment{reinterpret_cast<const uint8_t *>(batch->k) + e.kv_offset * 2,
                            reinterpret_cast<const uint8_t *>(batch->v) + e.kv_offset * 2,
                            e.head_stride, D, position + tokens, 0};
            // 32-bit: a launch has fewer than 2^31 workgroups.
            const uint32_t local = (uint32_t)(tile - pv.tile_base), nrb = (uint32_t)pv.row_blocks;
            rb = (int)(local % nrb);
            kvh = (int)(local / nrb);
            split = 0;
            sidx = 0;
        } else {
            const_ptr<Problem> pr = problem_ptr(p, tile);
            pv.q = pr->q;
            pv.out = pr->out;
            pv.q_row_stride = pr->q_row_stride;
            pv.q_pos0 = pr->q_pos0;
            pv.k_pos0 = pr->k_pos0;
            pv.keys = pr->keys;
            pv.vis_lo = pr->vis_lo;
            pv.vis_hi = pr->vis_hi;
            pv.tile_base = pr->tile_base;
            pv.slot_base = pr->slot_base;
            pv.queries = pr->queries;
            pv.row_blocks = pr->row_blocks;
            pv.splits = pr->splits;
            pv.split_keys = pr->split_keys;
            uint32_t local = (uint32_t)(tile - pv.tile_base);
            const uint32_t nrb = (uint32_t)pv.row_blocks, ns = (uint32_t)pv.splits;
            rb = (int)(local % nrb);
            local /= nrb;
            split = (int)(local % ns);
            kvh = (int)(local / ns);
            // This split's segment: splits are laid out segment by segment over
            // the visible range and never straddle a boundary, so one base
            // pointer and row stride serve every tile of the workgroup.
            int seg = 0;
            sidx = split;
            if (sidx >= pr->seg_splits[0]) {
                sidx -= pr->seg_splits[0];
                seg = 1;
                if (sidx >= pr->seg_splits[1]) {
                    sidx -= pr->seg_splits[1];
                    seg = 2;
                }
            }
            const auto &sgp = pr->seg[seg];
            pv.sg = Segment{sgp.k, sgp.v, sgp.head_stride, sgp.row_stride, sgp.keys, sgp.start};
        }
    }
}

// One lane's query row and its workgroup's key range inside the split.
struct PfRows {
    int m_kv;              // packed rows of the (problem, KV head)
    int t_row, h_row;      // this lane's token and query head (a valid row's)
    bool rvalid;           // the lane's row exists
    int64_t k_lo;          // first key of the workgroup's range (absolute)
    int nkeys, ntiles, nlast;  // keys, tiles and keys of the last tile
    int tf_lo, tf_hi;      // tiles [tf_lo, tf_hi) are visible to every row of the wave
    int rlo0, rhi0;        // this row's visible keys relative to k_lo
};

// The rows of workgroup row block `rb` (ROWS rows, RW per wave): lane row j of
// `wave`, the union of the rows' visible keys clipped to split `sidx`, and
// the tiles no row of the wave masks.
template <int ROWS, int RW>
__device__ __forceinline__ PfRows pf_rows(const Params &p, const PfView &pv, int rb, int kvh, int sidx,
                                          int wave, int j) {
    PfRows r;
    const int G = p.group;
    r.m_kv = pv.queries * G;
    const int m_kv = r.m_kv;
    const int64_t seg_start = pv.sg.start;
    const int64_t seg_end = seg_start + pv.sg.keys;
    const int64_t seg_lo = seg_start > pv.vis_lo ? seg_start : pv.vis_lo;
    const int64_t seg_hi = seg_end < pv.vis_hi ? seg_end : pv.vis_hi;
    const int64_t s_lo = seg_lo + (int64_t)sidx * pv.split_keys;
    const int64_t s_hi = s_lo + pv.split_keys < seg_hi ? s_lo + pv.split_keys : seg_hi;

    // This lane's query row.
    const int row = rb * ROWS + wave * RW + j;
    r.rvalid = row < m_kv;
    const int rrow = r.rvalid ? row : m_kv - 1;
    // Rows and the group are non-negative: unsigned divisions (shorter sequences).
    const uint32_t ug = (uint32_t)G;
    r.t_row = (int)((uint32_t)rrow / ug);
    r.h_row = kvh * G + (int)((uint32_t)rrow % ug);
    int64_t r_lo, r_hi;
    visible_range(p, pv.k_pos0, pv.keys, pv.q_pos0 + r.t_row, &r_lo, &r_hi);
    if (!r.rvalid) r_hi = r_lo;  // no visible keys: never contributes, never stored

    // Key range of the workgroup: the union over its rows, clipped to the split.
    const int wg_row_first = rb * ROWS;
    const int wg_row_last = min(wg_row_first + ROWS, m_kv) - 1;
    int64_t k_lo, k_hi, tmp;
    visible_range(p, pv.k_pos0, pv.keys, pv.q_pos0 + (uint32_t)wg_row_first / ug, &k_lo, &tmp);
    visible_range(p, pv.k_pos0, pv.keys, pv.q_pos0 + (uint32_t)wg_row_last / ug, &tmp, &k_hi);
    if (k_lo < s_lo) k_lo = s_lo;
    if (k_hi > s_hi) k_hi = s_hi;
    if (k_hi < k_lo) k_hi = k_lo;
    r.k_lo = k_lo;
    const int nkeys = uniform32((int)(k_hi - k_lo));
    const int ntiles = (nkeys + PF_KT - 1) / PF_KT;
    const int nlast = nkeys - (ntiles - 1) * PF_KT;
    r.nkeys = nkeys;
    r.ntiles = ntiles;
    r.nlast = nlast;
    {
        const int w_first = min(wg_row_first + wave * RW, m_kv - 1);
        const int w_last = min(wg_row_first + wave * RW + RW - 1, m_kv - 1);
        int64_t a, b, full_lo, full_hi;
        visible_range(p, pv.k_pos0, pv.keys, pv.q_pos0 + (uint32_t)w_first / ug, &a, &full_hi);
        visible_range(p, pv.k_pos0, pv.keys, pv.q_pos0 + (uint32_t)w_last / ug, &full_lo, &b);
        int64_t lo_t = full_lo - k_lo;
        lo_t = lo_t <= 0 ? 0 : (lo_t + PF_KT - 1) / PF_KT;
        int64_t hi_t = full_hi - k_lo;
        hi_t = hi_t <= 0 ? 0 : hi_t / PF_KT;
        if (hi_t > ntiles - (nlast < PF_KT ? 1 : 0)) hi_t = ntiles - (nlast < PF_KT ? 1 : 0);
        r.tf_lo = uniform32((int)(lo_t < ntiles ? lo_t : ntiles));
        r.tf_hi = uniform32((int)hi_t);
    }
    {
        int64_t x = r_lo - k_lo, y = r_hi - k_lo;
        r.rlo0 = (int)(x < 0 ? 0 : (x > nkeys ? nkeys : x));
        r.rhi0 = (int)(y < 0 ? 0 : (y > nkeys ? nkeys : y));
    }
    return r;
}

// The ring's direct loads: K/V tiles of PF_KT keys into stages of LDS layout
// L, RPW 1 KiB runs per wave and tile.  Rows past the last tile's keys repeat
// a valid row.
template <class L> struct PfRing {
    static constexpr int RPW = L::runs_per_wave;
    const uint8_t *k_next, *v_next;  // the next tile's first rows
    int64_t first;                   // element offset of the range's first row
    int prow;                        // bytes between keys
    int ntiles, t_next;
    uint32_t run0;                   // this wave's first run inside a tile (scalar)
    int off_full[RPW], off_last[RPW];
    __device__ __forceinline__ PfRing(const PfView &pv, int kvh, const PfRows &r, int wave, int lane) {
        prow = uniform32((int)(pv.sg.row_stride * 2));
        first = (int64_t)kvh * pv.sg.head_stride + (r.k_lo - pv.sg.start) * pv.sg.row_stride;
        k_next = reinterpret_cast<const uint8_t *>(pv.sg.k) + uniform64(first * 2);
        v_next = reinterpret_cast<const uint8_t *>(pv.sg.v) + uniform64(first * 2);
        for (int i = 0; i < RPW; ++i) {
            const int pos = (wave * RPW + i) * 1024 + lane * 16;
            const int rr = pos / L::row;
            const int cc = (((pos % L::row) >> 4) ^ L::swz(rr)) * 16;
            off_full[i] = rr * prow + cc;
            off_last[i] = (rr < r.nlast ? rr : r.nlast - 1) * prow + cc;
        }
        ntiles = r.ntiles;
        t_next = 0;
        run0 = (uint32_t)uniform32(wave) * (RPW * 1024);
    }
    // Issue the next tile into stage STG (a compile-time stage: the LDS
    // destinations are scalar constants plus run0).  FULL: the caller knows
    // this is not the last tile.
    template <int STG, bool FULL> __device__ __forceinline__ void issue(lds_ptr<uint8_t> lds) {
        const uint32_t mk = (uint32_t)(uintptr_t)(lds + L::k_at(STG)) + run0;
        const uint32_t mv = (uint32_t)(uintptr_t)(lds + L::v_at(STG)) + run0;
        if (!FULL && t_next == ntiles - 1) {
            for (int i = 0; i < RPW; ++i) {
                dma16(k_next, (uint32_t)off_last[i], mk + i * 1024);
                dma16(v_next, (uint32_t)off_last[i], mv + i * 1024);
            }
        } else {
            for (int i = 0; i < RPW; ++i) {
                dma16(k_next, (uint32_t)off_full[i], mk + i * 1024);
                dma16(v_next, (uint32_t)off_full[i], mv + i * 1024);
            }
        }
        k_next += PF_KT * prow;
        v_next += PF_KT * prow;
        ++t_next;
    }
    // Wait for tile `t` (issued earlier) and synchronise the workgroup.
    __device__ __forceinline__ void wait(int t) {
        const int ahead = t_next - 1 - t;  // later tiles still allowed in flight
        ring_sync<2 * RPW, L::stages - 2>(ahead);
    }
};

// bf16 V rows [0, nkeys) of the range: any non-finite value, any of magnitude
// 2^16 or more (beyond what the f16 P.V operands hold), by the whole wave.
__device__ __forceinline__ void pf_scan_v(const uint8_t *vrows, int nkeys, int prow, int D, int lane,
                                          bool &nonfinite, bool &big) {
    const int cpr = D * 2 / 16;  // 16-byte chunks per row
    const int rpi = 64 / cpr;    // rows per wave iteration
    nonfinite = false;
    big = false;
    for (int r0 = 0; r0 < nkeys; r0 += rpi) {
        const int r = r0 + lane / cpr;
        if (r < nkeys) {
            const u32x4 w = *gload_ptr<u32x4>(vrows + (int64_t)r * prow + 16 * (lane % cpr));
            for (int e = 0; e < 4; ++e) {
                const uint32_t x = w[e];
                const uint32_t lo = x & 0x7fffu, hi = (x >> 16) & 0x7fffu;
                nonfinite |= lo >= 0x7f80u || hi >= 0x7f80u;  // bf16 inf / NaN
                big |= lo >= 0x4780u || hi >= 0x4780u;        // |v| >= 65536
            }
        }
    }
}

template <int DT, int D, bool CAP, int W>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(2))) void attn_prefill(PrefillArgs a) {
    // The problem's fields are read by dependent scalar loads (the batch
    // count, then the problem, then its segment); with their lines already in
    // the scalar cache the chain costs one memory round trip, not one per
    // line (chunk launches: about 0.7 us less before the first tile).
    warm_kernarg<(offsetof(PrefillArgs, b) + offsetof(PrefillBatch, e) + 63) / 64, sizeof(PrefillArgs)>();
    const Params &p = a.p;
    constexpr int ROWS = 32 * W;  // packed rows per workgroup
    constexpr int KS = D / 16;        // QK k-steps (16 features each)
    constexpr int MB = D / 32;        // PV M-blocks (32 features each)
    constexpr int PDT = F16;          // P and V^T operand type of the P.V MFMAs
    constexpr bool VCONV = DT == BF16;  // V tiles converted to f16 in LDS
    static_assert(D % 32 == 0, "head_dim must be a multiple of 32");
    using L = PrefillLds<D, W>;
    constexpr int NS = L::stages;
    constexpr int RPW = L::runs_per_wave;
    constexpr int LPT = 2 * RPW;      // direct loads per wave per tile (K + V)

    __shared__ __attribute__((aligned(16))) uint8_t lds_raw[L::bytes];
    lds_ptr<uint8_t> lds = (lds_ptr<uint8_t>)lds_raw;

    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int j = lane & 31;   // query row of this lane inside the wave
    const int h = lane >> 5;   // which half of the k-slots / key quads

    const int G = p.group;
    const int Hq = p.query_heads;
    PfView pv;
    int rb, split, kvh, sidx;
    pf_locate<D>(p, pv, rb, split, kvh, sidx);
    const PfRows rows = pf_rows<ROWS, 32>(p, pv, rb, kvh, sidx, wave, j);
    const int t_row = rows.t_row, h_row = rows.h_row;
    const bool rvalid = rows.rvalid;
    const int nkeys = rows.nkeys, ntiles = rows.ntiles;
    const int tf_lo = rows.tf_lo, tf_hi = rows.tf_hi, rlo0 = rows.rlo0, rhi0 = rows.rhi0;
    // Fully visible tiles as a width, for one unsigned test per tile (none
    // when hi < lo, which happens for waves that see no whole tile).
    const unsigned tf_n = tf_hi > tf_lo ? (unsigned)(tf_hi - tf_lo) : 0u;

    // Q^T B operands: lane holds row j, features 16 ks + 8 h .. + 7.
    u32x4 qb[KS];
    {
        const uint8_t *qrow = reinterpret_cast<const uint8_t *>(pv.q) +
                              ((int64_t)t_row * pv.q_row_stride + (int64_t)h_row * D) * 2;
        for (int ks = 0; ks < KS; ++ks)
            qb[ks] = *gload_ptr<u32x4>(qrow + 32 * ks + 16 * h);
        // Complete the Q loads before the first direct K/V load.  The compiler
        // counts only the loads it sees (not the direct loads issued as inline
        // assembly); with Q still pending on its books it would place
        // vmcnt(7..3) waits before the QK MFMAs of every tile, which in
        // hardware also wait for the K/V tiles just issued.
        __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8));  // vmcnt(0)
    }

    f32x16 acc[MB];
    for (int mb = 0; mb < MB; ++mb)
        for (int i = 0; i < 16; ++i) acc[mb][i] = 0.0f;
    // m_run: the row's exp base in t units (a score it has seen; -inf before
    // the first), nbase_run = -m_run * tmul (BASE_NONE before the first).
    float m_run = NEG_INF, l_run = 0.0f, nbase_run = BASE_NONE;
    // The largest |score| of fully visible tiles: not below +inf exactly when
    // one of them was not finite (masked tiles check their visible scores
    // themselves).
    float amax_run = 0.0f;
    bool bad = false;  // a non-finite visible score
    // With the softcap a score is kept as t = tanh(raw * scale / cap), whose
    // log2-unit value is t * cap * log2(e): the cap's factor rides on the
    // exp's multiplier instead of a multiply per score.
    const float ycap = p.softcap_y;
    const float tmul = CAP ? p.softcap_log2 : p.scale_log2;  // t units -> log2 units
    // A row maximum of 2^10 or more in log2 units (natural-log logits above
    // about 700) makes the rounding of m * tmul worth a large part of an
    // exponent, so 2^(t * tmul - round(m * tmul)) would lose the mass.  A wave
    // holding such a row subtracts the maximum in raw units first (wave-uniform,
    // decided whenever a maximum moves).
    bool huge = false;

    // ---- K/V tiles: PF_KT keys each, issued into an NS-stage LDS ring.
    PfRing<L> ring(pv, kvh, rows, wave, lane);
    const int prow = ring.prow;
    const int64_t first = ring.first;
    int &t_next = ring.t_next;
    auto issue = [&](auto stg_tag, auto full_tag) {
        ring.template issue<decltype(stg_tag)::value, decltype(full_tag)::value>(lds);
    };
    auto wait_tile = [&](int t) { ring.wait(t); };

    // LDS offsets of this lane's operand reads (tile-relative).
    int k_off[KS];
    for (int ks = 0; ks < KS; ++ks) k_off[ks] = L::at(j, 2 * ks + h);
    // V^T operand of M-block mb, key step stp: row 32 mb + j, chunk 2 stp + h
    // (the swizzle depends on j only, so mb adds a constant).
    int vt_off[2];
    for (int stp = 0; stp < 2; ++stp) vt_off[stp] = L::vt_at(j, 2 * stp + h);

    // Software pipeline.  Iteration t:
    //   1. P.V of tile t - 1 on the matrix cores, with the statistics of tile
    //      t's scores (mask, maximum, rescale decision) and the first half of
    //      its probabilities on the vector unit between those MFMAs;
    //   2. wait for tile t + 1 and hand the stage of tile t - 1 to a new load;
    //   3. the scores of tile t + 1 (QK MFMAs) with the second half of tile t's
    //      probabilities and the reads of tile t's V^T operands (for step 1 of
    //      the next iteration) between them.
    // Scheduling fences keep that interleave; every MFMA slot is a compile-time
    // position.  In iteration 0 step 1 multiplies zero operands, and after the
    // last tile step 3 scores stale LDS data (of a stage that holds an earlier
    // tile) that is never used.
    constexpr int NPV = 2 * MB;  // P.V MFMAs per tile
    static_assert(NPV == KS, "one V^T operand read per Q.K k-step");
    // head_dim 256: the V^T operands of a tile are read just before its P.V
    // MFMAs, VPF ahead, instead of a whole Q.K chain ahead: 16 operands held
    // across an iteration (64 registers) made the compiler spill in the loop.
    constexpr bool VLATE = D >= 256;
    constexpr int VPF = 4;
    // head_dim 256 (one wave per SIMD): steps 1 and 3 run as one phase after
    // the ring wait, P.V and Q.K MFMAs alternating (the merged body below).
    constexpr bool MERGED = D >= 256;
    static_assert(!MERGED || (VLATE && L::vt_bufs == NS && NS >= 3),
                  "the merged phase writes tile t + 1's V^T while it reads tile t - 1's");
    auto vt_buf = [&](int tile_stage) { return lds + L::vt_base + (tile_stage % L::vt_bufs) * L::vt_bytes; };
    auto vt_operand = [&](lds_ptr<uint8_t> buf, int k) {
        return *(lds_ptr<u32x4>)(buf + vt_off[k / MB] + (k % MB) * 32 * L::vt_row);
    };
    static_for<NS - 1>([&](auto stg) {
        if (decltype(stg)::value < ntiles) issue(stg, std::false_type{});
    });
    f32x16 st;
    for (int i = 0; i < 16; ++i) st[i] = 0.0f;
    VTranspose<D, W, VCONV> vtr(threadIdx.x);
    if (ntiles > 0) {
        if constexpr (VLATE) {
            // Iteration 0's P.V reads the buffer of "tile -1" (stage NS - 1):
            // zeros, which the zero probabilities of iteration 0 multiply.
            lds_ptr<uint8_t> z = vt_buf(NS - 1);
            for (int i = threadIdx.x; i < L::vt_bytes / 16; i += 64 * W)
                *(lds_ptr<u32x4>)(z + 16 * i) = u32x4{0, 0, 0, 0};
        }
        wait_tile(0);
        for (int ks = 0; ks < KS; ++ks)
            st = mfma32<DT>(*(lds_ptr<u32x4>)(lds + L::k_at(0) + k_off[ks]), qb[ks], st);
        vtr.read(lds + L::v_at(0));
        vtr.write(lds + L::vt_base);
        // Tile 0's V^T is read at the end of iteration 0, after the barrier of
        // its step 2, which a single tile does not have (the merged form opens
        // every iteration with a barrier and needs none here).
        if (!MERGED && ntiles == 1) __syncthreads();
    }
    // V^T operands of the tile whose P.V is pending (read ahead unless VLATE).
    u32x4 vop[VLATE ? 1 : 2][VLATE ? 1 : MB];
    uint32_t ph[8];                    // its probabilities (f16 pairs)
    for (int stp = 0; stp < (VLATE ? 1 : 2); ++stp)
        for (int mb = 0; mb < (VLATE ? 1 : MB); ++mb) vop[stp][mb] = u32x4{0, 0, 0, 0};
    for (int i = 0; i < 8; ++i) {
        ph[i] = 0u;
    }
    int t = 0;
    // Tile t sits in stage t % NS.  The loop is unrolled by NS, so every
    // stage, and with it every LDS offset, is a compile-time constant, and the
    // two score registers swap roles (a copy per round only for an odd NS).
    f32x16 st_b;
    // bulk: the round of NS iterations starting at t is steady-state: every
    // tile t' of it is visible to all rows of the wave, tile t' + 1 and the
    // tile it issues (t' + NS - 1) come before the last.  Such an iteration
    // skips the visibility test, takes a fixed ring wait and issues and
    // converts unconditionally.
    bool bulk = false;
    // Close tile t's softmax step: st holds its scores (masked, capped, shifted
    // by `shift` in raw units), ph its probabilities against the row's base
    // and lt their mass in this lane.
    auto close_tile = [&](f32x16 &st, float shift, float &lt) {
        // ---- the exact path, rare: some row's tile mass exceeds MASS_LIMIT
        // (a score about 15 log2 units above its base, the row's first
        // visible tile, or a non-finite score).  The wave moves
        // each such row's base to the tile maximum, rescales O (which holds
        // tiles up to t - 1) and l, and forms tile t's probabilities again.
        if (__ballot(!(lt <= MASS_LIMIT)) != 0) {
            float hi = st[0];
            for (int i = 1; i < 16; ++i) hi = maxn(hi, st[i]);
            {
                const uint32_t u = __builtin_bit_cast(uint32_t, hi);
                const auto pr32 = __builtin_amdgcn_permlane32_swap(u, u, false, false);
                // Copied to scalars first: a bit_cast of a vector element reads
                // element 0 whatever the index.
                const uint32_t a0 = pr32[0], a1 = pr32[1];
                hi = maxn(__builtin_bit_cast(float, a0), __builtin_bit_cast(float, a1));
            }
            hi += shift;  // raw units (st of a huge row was shifted)
            // A NaN maximum leaves the base (the row already reports a
            // non-finite score).
            const float m_new = fmaxf(m_run, hi);
            if (m_new > m_run) {
                const float corr = m_run == NEG_INF ? 0.0f : __builtin_amdgcn_exp2f((m_run - m_new) * tmul);
                l_run *= corr;
                for (int mb = 0; mb < MB; ++mb)
                    for (int i = 0; i < 16; ++i) acc[mb][i] *= corr;
                m_run = m_new;
            }
            if constexpr (!CAP)
                huge = __ballot(m_run != NEG_INF && fabsf(m_run * tmul) >= 1024.0f) != 0;
            nbase_run = m_run == NEG_INF ? BASE_NONE : -m_run * tmul;
            // Tile t against the new base, in the units st holds.
            const float delta = m_run == NEG_INF ? 0.0f : m_run - shift;
            const float nb = -delta * tmul;
            lt = 0.0f;
            for (int i = 0; i < 8; ++i) {
                float y0, y1;
                if (!CAP && huge) {
                    y0 = (st[2 * i] - delta) * tmul;
                    y1 = (st[2 * i + 1] - delta) * tmul;
                } else {
                    y0 = __builtin_fmaf(st[2 * i], tmul, nb);
                    y1 = __builtin_fmaf(st[2 * i + 1], tmul, nb);
                }
                ph[i] = pack2<PDT>(__builtin_amdgcn_exp2f(y0), __builtin_amdgcn_exp2f(y1));
                lt = add_pair(ph[i], lt);
            }
        }
        l_run += lt;
    };

    auto body = [&](auto stg_tag, f32x16 &st, f32x16 &st_next) {
        constexpr int STG = decltype(stg_tag)::value;
        constexpr int STG_NEXT = (STG + 1) % NS;
        __builtin_amdgcn_sched_barrier(0);
        lds_ptr<uint8_t> vt = lds + L::vt_base + (STG % L::vt_bufs) * L::vt_bytes;
        lds_ptr<uint8_t> kn = lds + L::k_at(STG_NEXT);

        // ---- step 1.  t = raw dot (or, with the softcap, tanh(raw * scale /
        // cap)); p = 2^(t * tmul + nbase) against the row's current base,
        // with no tile maximum (the check after step 3 catches a base that is
        // too low).
        float nbase = nbase_run;
        float shift = 0.0f;      // subtracted from st in raw units (huge rows)
        float lt = 0.0f;         // this lane's mass of the tile
        uint32_t nh[4];
        u32x4 vq[VLATE ? VPF : 1];
        lds_ptr<uint8_t> vtp = vt_buf((STG + NS - 1) % NS);  // tile t - 1's V^T
        if constexpr (VLATE)
            for (int i = 0; i < VPF; ++i) vq[i] = vt_operand(vtp, i);
#pragma unroll
        for (int k = 0; k < NPV; ++k) {
            {
                const int stp = k / MB, mb = k % MB;
                const u32x4 bv = u32x4{ph[4 * stp], ph[4 * stp + 1], ph[4 * stp + 2], ph[4 * stp + 3]};
                if constexpr (VLATE) {
                    const u32x4 a = vq[k % VPF];
                    if (k + VPF < NPV) vq[k % VPF] = vt_operand(vtp, k + VPF);
                    acc[mb] = mfma32<PDT>(a, bv, acc[mb]);
                } else {
                    acc[mb] = mfma32<PDT>(vop[stp][mb], bv, acc[mb]);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            if (k == 0) {
                if (bulk || (unsigned)(t - tf_lo) < tf_n) {  // t in [tf_lo, tf_hi)
                    float a = amax_run;
                    for (int i = 0; i < 16; ++i) a = maxn(a, __builtin_fabsf(st[i]));
                    amax_run = a;
                    // With the softcap the tanh values replace the raw scores
                    // in place, which keeps 16 registers free.
                    if constexpr (CAP)
                        for (int i = 0; i < 16; ++i) st[i] = tanh_fast(st[i] * ycap);
                } else {
                    // Visible keys of this row inside the tile: [lo_rel, hi_rel).
                    const int lo_rel = min(max(rlo0 - t * PF_KT, 0), PF_KT);
                    const int hi_rel = min(max(rhi0 - t * PF_KT, 0), PF_KT);
                    for (int i = 0; i < 16; ++i) {
                        const int kk = 8 * (i >> 2) + 4 * h + (i & 3);
                        const bool vis = kk >= lo_rel && kk < hi_rel;
                        bad |= vis && !(__builtin_fabsf(st[i]) < -NEG_INF);
                        // masked (and capped) in place: no copy of the scores
                        if constexpr (CAP) st[i] = vis ? tanh_fast(st[i] * ycap) : NEG_INF;
                        else st[i] = vis ? st[i] : NEG_INF;
                    }
                }
            }
            if (k == (NPV > 1 ? 1 : 0)) {
                if constexpr (!CAP) {
                    if (huge) {
                        // Rows with no base yet keep BASE_NONE (their first
                        // visible tile takes the exact path).
                        shift = m_run == NEG_INF ? 0.0f : m_run;
                        for (int i = 0; i < 16; ++i) st[i] -= shift;
                        nbase = m_run == NEG_INF ? BASE_NONE : 0.0f;
                    }
                }
            }
            // First half of tile t's probabilities (tile t - 1's are still being read).
            for (int i = 0; i < 4; ++i) {
                if (k == (NPV > 2 ? 2 + (i * (NPV - 2)) / 4 : NPV - 1)) {
                    const float e0 = __builtin_amdgcn_exp2f(__builtin_fmaf(st[2 * i], tmul, nbase));
                    const float e1 = __builtin_amdgcn_exp2f(__builtin_fmaf(st[2 * i + 1], tmul, nbase));
                    nh[i] = pack2<PDT>(e0, e1);
                    lt = add_pair(nh[i], lt);
                    // Pin the pair here: the compiler would otherwise sink it to
                    // its use after step 1, out of the MFMA shadow.
                    asm volatile("" : "+v"(nh[i]), "+v"(lt));
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        for (int i = 0; i < 4; ++i) {
            ph[i] = nh[i];
        }

        // ---- step 2: tile t + 1 resident; everyone is done with tile t - 1,
        // whose stage takes the next load.
        if (bulk) {
            // t_next == t + NS - 1: NS - 3 later tiles may stay in flight.
            ring_sync_fixed<LPT, NS - 3>();
            issue(std::integral_constant<int, (STG + NS - 1) % NS>{}, std::true_type{});
        } else if (t + 1 < ntiles) {
            wait_tile(t + 1);
            if (t_next < ntiles) issue(std::integral_constant<int, (STG + NS - 1) % NS>{}, std::false_type{});
        } else if (t > 0) {
            // The last tile: its transposed V was written by the whole
            // workgroup in the previous iteration's step 3, and no step-2
            // barrier follows that here; step 3 reads it.
            __syncthreads();
        }

        // ---- step 3: scores of tile t + 1 (K operands read KPRE steps ahead),
        // second half of tile t's probabilities.
        constexpr int KPRE = CAP ? 2 : 3;
        for (int i = 0; i < 16; ++i) st_next[i] = 0.0f;
        u32x4 kq[KPRE];
        for (int i = 0; i < KPRE && i < KS; ++i) kq[i] = *(lds_ptr<u32x4>)(kn + k_off[i]);
        // Tile t + 1's V, resident since step 2, transposed (bf16: converted)
        // between these MFMAs; the barrier of the next step 2 precedes its V^T
        // reads.  After the last tile this transposes a stale stage into a
        // buffer nobody reads again (the buffers of tiles t and t - 1 differ
        // from it, and every read of its previous tile preceded this
        // iteration's step-2 barrier), which costs less than the branch.
        lds_ptr<uint8_t> vn = lds + L::v_at(STG_NEXT);
        lds_ptr<uint8_t> vtn = lds + L::vt_base + (STG_NEXT % L::vt_bufs) * L::vt_bytes;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const u32x4 kcur = kq[ks % KPRE];
            if (ks + KPRE < KS) kq[ks % KPRE] = *(lds_ptr<u32x4>)(kn + k_off[ks + KPRE]);
            // Tile t's V^T operands (for step 1 of the next iteration), one
            // per k-step: resident since the step-2 barrier, and a whole Q.K
            // chain ahead of their use.  B slots 8h..8h+7 of step stp are keys
            // {16 stp + 4h + 0..3, 16 stp + 8 + 4h + 0..3}, the order in which
            // the transposed tile stores them.  (2 MB == KS.)
            if constexpr (!VLATE) vop[ks / MB][ks % MB] = vt_operand(vt, ks);
            // The two waves of a SIMD leave the step-2 barrier together and
            // would contend for the matrix core and the vector unit in
            // lockstep.  A raised priority over the first half of the Q.K
            // chain lets whichever wave gets there first keep its MFMAs
            // issuing while the other one's exp/pack work fills the gaps
            // (configs[4]: 388 -> 377 us mean of three alternating runs;
            // the whole chain or a quarter of it measured no gain).
            st_next = mfma32<DT>(kcur, qb[ks], st_next);
            if (ks == 0) __builtin_amdgcn_s_setprio(1);
            if (ks == KS / 2) __builtin_amdgcn_s_setprio(0);
            __builtin_amdgcn_sched_barrier(0);
            if (ks == 0) vtr.read(vn);
            if (ks == KS / 2) vtr.write(vtn);
            for (int i = 4 + 4 * ks / KS; i < 4 + 4 * (ks + 1) / KS; ++i) {
                const float e0 = __builtin_amdgcn_exp2f(__builtin_fmaf(st[2 * i], tmul, nbase));
                const float e1 = __builtin_amdgcn_exp2f(__builtin_fmaf(st[2 * i + 1], tmul, nbase));
                ph[i] = pack2<PDT>(e0, e1);
                lt = add_pair(ph[i], lt);
                asm volatile("" : "+v"(ph[i]), "+v"(lt));
            }
            __builtin_amdgcn_sched_barrier(0);
        }

        close_tile(st, shift, lt);

        __builtin_amdgcn_sched_barrier(0);
    };
    // The merged form of iteration t (head_dim 256, where each SIMD runs one
    // wave and nothing hides a phase's LDS reads or vector work but the same
    // wave's MFMAs):
    //   1. wait for tile t + 1 and hand the stage of tile t - 1 to a new load;
    //   2. one phase of 2 KS MFMA slots: P.V of tile t - 1 in the even slots,
    //      the scores of tile t + 1 in the odd ones, with the statistics and
    //      the probabilities of tile t, tile t + 1's V transposition and both
    //      chains' LDS operand reads between them.
    // Tile t - 1's V^T (read here), tile t's (written in iteration t - 1, read
    // in t + 1) and tile t + 1's (written here) need three buffers, one per
    // ring stage; the buffer written in iteration t last held tile
    // t + 1 - NS, read in iteration t + 2 - NS <= t - 1, before this
    // iteration's barrier.  In iteration 0 the phase multiplies the zeroed
    // buffer of "tile -1"; after the last tile it scores and transposes a
    // stale stage into a buffer nobody reads again.
    auto body_mg = [&](auto stg_tag, f32x16 &st, f32x16 &st_next) {
        constexpr int STG = decltype(stg_tag)::value;
        constexpr int STG_NEXT = (STG + 1) % NS;
        __builtin_amdgcn_sched_barrier(0);
        if (bulk) {
            ring_sync_fixed<LPT, NS - 3>();
            issue(std::integral_constant<int, (STG + NS - 1) % NS>{}, std::true_type{});
        } else if (t + 1 < ntiles) {
            wait_tile(t + 1);
            if (t_next < ntiles) issue(std::integral_constant<int, (STG + NS - 1) % NS>{}, std::false_type{});
        } else {
            // The last tile: the V^T buffer its phase writes held tile
            // t + 1 - NS, which a slower wave may still be reading.
            __syncthreads();
        }
        __builtin_amdgcn_sched_barrier(0);

        lds_ptr<uint8_t> vtp = vt_buf((STG + NS - 1) % NS);  // tile t - 1's V^T
        lds_ptr<uint8_t> kn = lds + L::k_at(STG_NEXT);
        lds_ptr<uint8_t> vn = lds + L::v_at(STG_NEXT);
        lds_ptr<uint8_t> vtn = vt_buf(STG_NEXT);
        float nbase = nbase_run;
        float shift = 0.0f;  // subtracted from st in raw units (huge rows)
        float lt = 0.0f;     // this lane's mass of the tile
        uint32_t pn[8];      // tile t's probabilities (ph holds tile t - 1's until the phase ends)
        constexpr int KPRE = CAP ? 2 : 3;
        constexpr int SLOTS = NPV + KS;
        u32x4 vq[VPF];
        for (int i = 0; i < VPF; ++i) vq[i] = vt_operand(vtp, i);
        u32x4 kq[KPRE];
        for (int i = 0; i < KPRE; ++i) kq[i] = *(lds_ptr<u32x4>)(kn + k_off[i]);
        for (int i = 0; i < 16; ++i) st_next[i] = 0.0f;
#pragma unroll
        for (int k = 0; k < SLOTS; ++k) {
            const int m = k / 2;
            if (k % 2 == 0) {
                const int stp = m / MB, mb = m % MB;
                const u32x4 bv = u32x4{ph[4 * stp], ph[4 * stp + 1], ph[4 * stp + 2], ph[4 * stp + 3]};
                const u32x4 a = vq[m % VPF];
                if (m + VPF < NPV) vq[m % VPF] = vt_operand(vtp, m + VPF);
                acc[mb] = mfma32<PDT>(a, bv, acc[mb]);
            } else {
                const u32x4 kcur = kq[m % KPRE];
                if (m + KPRE < KS) kq[m % KPRE] = *(lds_ptr<u32x4>)(kn + k_off[m + KPRE]);
                st_next = mfma32<DT>(kcur, qb[m], st_next);
            }
            // Raised priority over the first half of the phase, as in the
            // two-wave form; without these two instructions the compiler
            // stops unrolling the softcapped phase (dynamic register indexing
            // and scratch, 3.6x slower on the configs[3] session).
            if (k == 1) __builtin_amdgcn_s_setprio(1);
            if (k == SLOTS / 2) __builtin_amdgcn_s_setprio(0);
            __builtin_amdgcn_sched_barrier(0);
            if (k == 0) {
                if (bulk || (unsigned)(t - tf_lo) < tf_n) {  // t in [tf_lo, tf_hi)
                    float a = amax_run;
                    for (int i = 0; i < 16; ++i) a = maxn(a, __builtin_fabsf(st[i]));
                    amax_run = a;
                    if constexpr (CAP)
                        for (int i = 0; i < 16; ++i) st[i] = tanh_fast(st[i] * ycap);
                } else {
                    const int lo_rel = min(max(rlo0 - t * PF_KT, 0), PF_KT);
                    const int hi_rel = min(max(rhi0 - t * PF_KT, 0), PF_KT);
                    for (int i = 0; i < 16; ++i) {
                        const int kk = 8 * (i >> 2) + 4 * h + (i & 3);
                        const bool vis = kk >= lo_rel && kk < hi_rel;
                        bad |= vis && !(__builtin_fabsf(st[i]) < -NEG_INF);
                        if constexpr (CAP) st[i] = vis ? tanh_fast(st[i] * ycap) : NEG_INF;
                        else st[i] = vis ? st[i] : NEG_INF;
                    }
                }
            }
            if constexpr (!CAP) {
                if (k == 1 && huge) {
                    shift = m_run == NEG_INF ? 0.0f : m_run;
                    for (int i = 0; i < 16; ++i) st[i] -= shift;
                    nbase = m_run == NEG_INF ? BASE_NONE : 0.0f;
                }
            }
            // Tile t + 1's V, resident since the ring wait, transposed
            // (bf16: converted) for the phase of iteration t + 2.
            if (k == 1) vtr.read(vn);
            if (k == SLOTS / 2) vtr.write(vtn);
            for (int i = 0; i < 8; ++i) {
                if (k == 2 + (i * (SLOTS - 2)) / 8) {
                    const float e0 = __builtin_amdgcn_exp2f(__builtin_fmaf(st[2 * i], tmul, nbase));
                    const float e1 = __builtin_amdgcn_exp2f(__builtin_fmaf(st[2 * i + 1], tmul, nbase));
                    pn[i] = pack2<PDT>(e0, e1);
                    lt = add_pair(pn[i], lt);
                    // Pin the pair here: the compiler would otherwise sink it
                    // to its use after the phase, out of the MFMA shadow.
                    asm volatile("" : "+v"(pn[i]), "+v"(lt));
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        for (int i = 0; i < 8; ++i) ph[i] = pn[i];
        close_tile(st, shift, lt);

        __builtin_amdgcn_sched_barrier(0);
    };
    while (t < ntiles) {
        // A round of NS steady-state iterations when all of them qualify
        // (t is a multiple of NS here, so stage K is tile t + K's).  Once t
        // reaches ntiles the remaining iterations of the round do nothing.
        bulk = t >= tf_lo && t + NS <= tf_hi && t + 2 * NS - 1 < ntiles && t_next == t + NS - 1;
        static_for<NS>([&](auto k) {
            constexpr int K = decltype(k)::value;
            if (t >= ntiles) return;
            if constexpr (MERGED) {
                if constexpr (K % 2 == 0) body_mg(std::integral_constant<int, K>{}, st, st_b);
                else body_mg(std::integral_constant<int, K>{}, st_b, st);
            } else {
                if constexpr (K % 2 == 0) body(std::integral_constant<int, K>{}, st, st_b);
                else body(std::integral_constant<int, K>{}, st_b, st);
            }
            ++t;
        });
        // An odd ring leaves the next scores in st_b.
        if constexpr (NS % 2 == 1) st = st_b;
    }
    // P.V of the last tile.
    if (ntiles > 0) {
        lds_ptr<uint8_t> vtl = vt_buf((ntiles - 1) % NS);
#pragma unroll
        for (int k = 0; k < NPV; ++k) {
            const int stp = k / MB, mb = k % MB;
            const u32x4 bv = u32x4{ph[4 * stp], ph[4 * stp + 1], ph[4 * stp + 2], ph[4 * stp + 3]};
            if constexpr (VLATE) acc[mb] = mfma32<PDT>(vt_operand(vtl, k), bv, acc[mb]);
            else acc[mb] = mfma32<PDT>(vop[stp][mb], bv, acc[mb]);
        }
    }
    bad |= !(amax_run < -NEG_INF);
    // ---- the two key halves of each row (lanes j and j + 32) share m_run; add l.
    {
        const uint32_t u = __builtin_bit_cast(uint32_t, l_run);
        const auto pr32 = __builtin_amdgcn_permlane32_swap(u, u, false, false);
        const uint32_t a0 = pr32[0], a1 = pr32[1];
        l_run = __builtin_bit_cast(float, a0) + __builtin_bit_cast(float, a1);
    }
    bool bad_acc = false;
    for (int mb = 0; mb < MB; ++mb)
        for (int i = 0; i < 16; ++i) bad_acc |= !is_finite_f(acc[mb][i]);
    // bf16: the P.V products took V as f16, which overflows for finite values
    // above 65280.  Only a wave whose context is not finite while its scores
    // were reads the workgroup's V rows again, to tell a non-finite input
    // (ST_NONFINITE_INPUT) from such a value.  For the latter the wave forms
    // its rows again on the vector unit in FP32 (scores, probabilities against
    // the same base, context and mass), which is slow and exact for every
    // finite value.
    if constexpr (VCONV) {
        if (__ballot(bad_acc && !bad) != 0) {
            const uint8_t *vrows = reinterpret_cast<const uint8_t *>(pv.sg.v) + first * 2;
            const uint8_t *krows = reinterpret_cast<const uint8_t *>(pv.sg.k) + first * 2;
            bool nonfinite, big;
            pf_scan_v(vrows, nkeys, prow, D, lane, nonfinite, big);
            if (__ballot(nonfinite) == 0 && __ballot(big) != 0) {
                // Lane (j, h) holds Q features 16 ks + 8 h .. + 7 and context
                // features 32 mb + 8 q + 4 h .. + 3 of row j; a score is the
                // lane pair's two partial dots added.
                for (int mb = 0; mb < MB; ++mb)
                    for (int i = 0; i < 16; ++i) acc[mb][i] = 0.0f;
                float l = 0.0f;
                const bool any = m_run != NEG_INF;
                for (int kk = 0; kk < nkeys; ++kk) {
                    const uint8_t *kr = krows + (int64_t)kk * prow;
                    float d = 0.0f;
                    for (int ks = 0; ks < KS; ++ks) {
                        const u32x4 kw = *gload_ptr<u32x4>(kr + 32 * ks + 16 * h);
                        for (int e = 0; e < 4; ++e) {
                            const uint32_t qw = qb[ks][e], kx = kw[e];
                            d = __builtin_fmaf(lo_f<BF16>(qw), lo_f<BF16>(kx), d);
                            d = __builtin_fmaf(hi_f<BF16>(qw), hi_f<BF16>(kx), d);
                        }
                    }
                    {
                        const uint32_t u = __builtin_bit_cast(uint32_t, d);
                        const auto pr32 = __builtin_amdgcn_permlane32_swap(u, u, false, false);
                        const uint32_t a0 = pr32[0], a1 = pr32[1];
                        d = __builtin_bit_cast(float, a0) + __builtin_bit_cast(float, a1);
                    }
                    float y;
                    if constexpr (CAP) y = (tanh_fast(d * ycap) - m_run) * tmul;
                    else y = (d - m_run) * tmul;
                    const bool vis = any && kk >= rlo0 && kk < rhi0;
                    const float pk = vis ? __builtin_amdgcn_exp2f(y) : 0.0f;
                    l += pk;
                    const uint8_t *vr = vrows + (int64_t)kk * prow;
                    for (int mb = 0; mb < MB; ++mb)
                        for (int q = 0; q < 4; ++q) {
                            const u32x2 vw = *gload_ptr<u32x2>(vr + (32 * mb + 8 * q + 4 * h) * 2);
                            const uint32_t v0 = vw[0], v1 = vw[1];
                            acc[mb][4 * q + 0] = __builtin_fmaf(pk, lo_f<BF16>(v0), acc[mb][4 * q + 0]);
                            acc[mb][4 * q + 1] = __builtin_fmaf(pk, hi_f<BF16>(v0), acc[mb][4 * q + 1]);
                            acc[mb][4 * q + 2] = __builtin_fmaf(pk, lo_f<BF16>(v1), acc[mb][4 * q + 2]);
                            acc[mb][4 * q + 3] = __builtin_fmaf(pk, hi_f<BF16>(v1), acc[mb][4 * q + 3]);
                        }
                }
                l_run = l;  // both lanes of the pair summed every key
                bad_acc = false;
                for (int mb = 0; mb < MB; ++mb)
                    for (int i = 0; i < 16; ++i) bad_acc |= !is_finite_f(acc[mb][i]);
            }
        }
    }
    bad |= bad_acc;

    // O^T lane layout: row j, features 32 mb + 8 q + 4 h + r (register 4 q + r).
    const bool single = pv.splits == 1;
    bool bad_mass = false, bad_out = false;
    if (single) {
        if (rvalid) {
            const float inv = 1.0f / l_run;
            bad_mass |= !(l_run > 0.0f) || !is_finite_f(l_run);
            float *orow = pv.out + ((int64_t)t_row * Hq + h_row) * D;
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

    // ---- split-K partial: slot (row block, split) holds the unnormalised
    // context feature-major, D x ROWS floats (the rows of a feature
    // contiguous), and (max, mass) per row; attn_prefill_merge combines the
    // slots after this kernel.  Feature-major stores are one dword per lane:
    // the 32 rows of each lane half fill one 128-byte line, so a store writes
    // two whole lines, where a row-major 16-byte store touched 32 lines (its
    // stores took 3.5 instead of 1.4 us per workgroup at head_dim 256).
    raise_status(p, bad, ST_NONFINITE_INPUT);
    const int64_t group = (int64_t)kvh * pv.row_blocks + rb;
    const int64_t slot = pv.slot_base + group * pv.splits + split;
    float *pf = p.part_o + slot * ROWS * D + wave * 32 + j;
    for (int mb = 0; mb < MB; ++mb)
        for (int q = 0; q < 4; ++q)
            for (int r = 0; r < 4; ++r)
                *gstore_ptr<float>(pf + (int64_t)(32 * mb + 8 * q + 4 * h + r) * ROWS) =
                    acc[mb][4 * q + r];
    if (h == 0) {
        const f32x2 ml = {m_run, l_run};
        *gstore_ptr<f32x2>(p.part_ml + (slot * ROWS + wave * 32 + j) * 2) = ml;
    }
}

// ---------------------------------------------------------------------------
// attn_prefill16: the same flash loop with sixteen packed rows per wave, on
// v_mfma_f32_16x16x32, for launches of few row blocks (session chunks).  A
// wave does half the MFMAs and half the softmax work of a 32-row wave per
// tile, and at head_dim 256 needs about half its registers.  Four-wave
// workgroups (64-row blocks) give a chunk twice the workgroups of 128-row
// blocks with the same split partials; eight-wave ones cover a 128-row block
// (attn_prefill<..., 4>'s grid and workspace slots).
//
// Lane (j, g) = (lane % 16, lane / 16):
//  * S^T = K Q^T per 16-key block kb: A = K (lane: key 16 kb + j, features
//    32 ks + 8 g .. + 7), B = Q^T (lane: row j, the same features), D: row j,
//    keys 16 kb + 4 g + r (register r).
//  * O^T = V^T P^T: B = P^T in the MFMA's k order k = 8 g + 4 kb + r for key
//    16 kb + 4 g + r, which is where the scores already sit; A = V^T row
//    16 fb + j, chunk g (keys 4 g .. + 3 and 16 + 4 g .. + 3); D: row j,
//    features 16 fb + 4 g + r.
// A row's 32 keys of a tile are spread over the four lanes j, j + 16, j + 32,
// j + 48 (8 each); its statistics are reduced across them where the 32-row
// kernel reduces across a lane pair.
template <int DT> __device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c);
template <> __device__ __forceinline__ f32x4 mfma16<BF16>(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
template <> __device__ __forceinline__ f32x4 mfma16<F16>(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}
// Sum and maximum over the four lanes of a row (j, j + 16, j + 32, j + 48);
// every lane of the row gets the same bits.
__device__ __forceinline__ float row4_sum(float x) {
    x += __shfl_xor(x, 16);
    return x + __shfl_xor(x, 32);
}
__device__ __forceinline__ float row4_max(float x) {
    x = maxn(x, __shfl_xor(x, 16));
    return maxn(x, __shfl_xor(x, 32));
}

// W 16-row waves per workgroup: eight make the four-wave 32-row kernel's
// 128-row block; four make 64-row blocks.
template <int DT, int D, bool CAP, int W>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(2))) void attn_prefill16(PrefillArgs a) {
    warm_kernarg<(offsetof(PrefillArgs, b) + offsetof(PrefillBatch, e) + 63) / 64, sizeof(PrefillArgs)>();
    const Params &p = a.p;
    constexpr int RW = 16;            // packed rows per wave
    constexpr int ROWS = RW * W;      // packed rows per workgroup
    constexpr int KS = D / 32;        // Q.K k-steps (32 features each) per 16-key block
    constexpr int NQK = 2 * KS;       // Q.K MFMAs per tile (two 16-key blocks)
    constexpr int FB = D / 16;        // P.V MFMAs per tile (16-feature blocks)
    constexpr int PDT = F16;
    constexpr bool VCONV = DT == BF16;
    static_assert(D == 128 || D == 256, "16-row form: head_dim 128 or 256");
    using L = PrefillLds<D, W>;
    constexpr int NS = L::stages;
    constexpr int RPW = L::runs_per_wave;
    constexpr int LPT = 2 * RPW;
    // The last iteration's Q.K pass transposes a stale stage into the buffer
    // after tile t's; with two buffers that is tile t - 1's, which step 1 of
    // the same iteration reads, so the last iteration always takes the step-2
    // barrier below.
    static_assert(L::vt_bufs >= 2, "V^T buffers");

    __shared__ __attribute__((aligned(16))) uint8_t lds_raw[L::bytes];
    lds_ptr<uint8_t> lds = (lds_ptr<uint8_t>)lds_raw;

    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int j = lane & 15;   // query row of this lane inside the wave
    const int g = lane >> 4;   // its key quad (scores) and feature quad (context)

    const int G = p.group;
    const int Hq = p.query_heads;
    PfView pv;
    int rb, split, kvh, sidx;
    pf_locate<D>(p, pv, rb, split, kvh, sidx);
    const PfRows rows = pf_rows<ROWS, RW>(p, pv, rb, kvh, sidx, wave, j);
    const int t_row = rows.t_row, h_row = rows.h_row;
    const bool rvalid = rows.rvalid;
    const int nkeys = rows.nkeys, ntiles = rows.ntiles;
    const int tf_lo = rows.tf_lo, tf_hi = rows.tf_hi, rlo0 = rows.rlo0, rhi0 = rows.rhi0;
    const unsigned tf_n = tf_hi > tf_lo ? (unsigned)(tf_hi - tf_lo) : 0u;

    // Q^T B operands: lane holds row j, features 32 ks + 8 g .. + 7.
    u32x4 qb[KS];
    {
        const uint8_t *qrow = reinterpret_cast<const uint8_t *>(pv.q) +
                              ((int64_t)t_row * pv.q_row_stride + (int64_t)h_row * D) * 2;
        for (int ks = 0; ks < KS; ++ks)
            qb[ks] = *gload_ptr<u32x4>(qrow + 64 * ks + 16 * g);
        __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8));  // vmcnt(0), as in attn_prefill
    }

    f32x4 acc[FB];
    for (int fb = 0; fb < FB; ++fb)
        for (int i = 0; i < 4; ++i) acc[fb][i] = 0.0f;
    float m_run = NEG_INF, l_run = 0.0f, nbase_run = BASE_NONE;
    float amax_run = 0.0f;
    bool bad = false;
    const float ycap = p.softcap_y;
    const float tmul = CAP ? p.softcap_log2 : p.scale_log2;
    bool huge = false;

    PfRing<L> ring(pv, kvh, rows, wave, lane);
    const int prow = ring.prow;
    const int64_t first = ring.first;
    int &t_next = ring.t_next;
    auto issue = [&](auto stg_tag, auto full_tag) {
        ring.template issue<decltype(stg_tag)::value, decltype(full_tag)::value>(lds);
    };
    auto wait_tile = [&](int t) { ring.wait(t); };

    // K operand of k-step ks: key row j of a 16-key block (the swizzle of row
    // 16 kb + j equals row j's at these row sizes), chunk 4 ks + g.
    static_assert(L::swz(16) == L::swz(0) && L::swz(17) == L::swz(1), "16-key blocks share the swizzle");
    int k_off[KS];
    for (int ks = 0; ks < KS; ++ks) k_off[ks] = L::at(j, 4 * ks + g);
    constexpr int KB_BYTES = 16 * L::row;  // second 16-key block
    // V^T operand of feature block fb: row 16 fb + j, chunk g (the swizzle
    // depends on (row / 4) % 4 = (j / 4) % 4 only).
    const int vt_off = L::vt_at(j, g);
    constexpr int VPF = 4;
    auto vt_buf = [&](int tile_stage) { return lds + L::vt_base + (tile_stage % L::vt_bufs) * L::vt_bytes; };
    auto vt_operand = [&](lds_ptr<uint8_t> buf, int fb) {
        return *(lds_ptr<u32x4>)(buf + vt_off + fb * 16 * L::vt_row);
    };
    auto k_operand = [&](lds_ptr<uint8_t> kt, int m) {  // MFMA m: block m % 2, k-step m / 2
        return *(lds_ptr<u32x4>)(kt + (m % 2) * KB_BYTES + k_off[m / 2]);
    };
    static_for<NS - 1>([&](auto stg) {
        if (decltype(stg)::value < ntiles) issue(stg, std::false_type{});
    });
    f32x4 st[2];
    for (int kb = 0; kb < 2; ++kb)
        for (int i = 0; i < 4; ++i) st[kb][i] = 0.0f;
    VTranspose<D, W, VCONV, true> vtr(threadIdx.x);
    if (ntiles > 0) {
        // Iteration 0's P.V reads the buffer of "tile -1": zeros, which the
        // zero probabilities of iteration 0 multiply.
        lds_ptr<uint8_t> z = vt_buf(NS - 1);
        for (int i = threadIdx.x; i < L::vt_bytes / 16; i += 64 * W)
            *(lds_ptr<u32x4>)(z + 16 * i) = u32x4{0, 0, 0, 0};
        wait_tile(0);
        for (int m = 0; m < NQK; ++m)
            st[m % 2] = mfma16<DT>(k_operand(lds + L::k_at(0), m), qb[m / 2], st[m % 2]);
        vtr.read(lds + L::v_at(0));
        vtr.write(lds + L::vt_base);
    }
    uint32_t ph[4];  // the probabilities of the tile whose P.V is pending (f16 pairs)
    for (int i = 0; i < 4; ++i) ph[i] = 0u;
    int t = 0;
    f32x4 st_b[2];
    bool bulk = false;
    // The exact path, rare (as in attn_prefill): some lane's tile mass exceeds
    // MASS_LIMIT.  The wave moves each such row's base to the tile maximum,
    // rescales O (tiles up to t - 1) and l, and forms tile t's probabilities
    // again.
    auto close_tile = [&](f32x4 (&st)[2], float shift, float &lt) {
        if (__ballot(!(lt <= MASS_LIMIT)) != 0) {
            float hi = st[0][0];
            for (int kb = 0; kb < 2; ++kb)
                for (int i = 0; i < 4; ++i) hi = maxn(hi, st[kb][i]);
            hi = row4_max(hi) + shift;
            const float m_new = fmaxf(m_run, hi);
            if (m_new > m_run) {
                const float corr = m_run == NEG_INF ? 0.0f : __builtin_amdgcn_exp2f((m_run - m_new) * tmul);
                l_run *= corr;
                for (int fb = 0; fb < FB; ++fb)
                    for (int i = 0; i < 4; ++i) acc[fb][i] *= corr;
                m_run = m_new;
            }
            if constexpr (!CAP)
                huge = __ballot(m_run != NEG_INF && fabsf(m_run * tmul) >= 1024.0f) != 0;
            nbase_run = m_run == NEG_INF ? BASE_NONE : -m_run * tmul;
            const float delta = m_run == NEG_INF ? 0.0f : m_run - shift;
            const float nb = -delta * tmul;
            lt = 0.0f;
            for (int i = 0; i < 4; ++i) {
                const int kb = i >> 1, r = 2 * (i & 1);
                float y0, y1;
                if (!CAP && huge) {
                    y0 = (st[kb][r] - delta) * tmul;
                    y1 = (st[kb][r + 1] - delta) * tmul;
                } else {
                    y0 = __builtin_fmaf(st[kb][r], tmul, nb);
                    y1 = __builtin_fmaf(st[kb][r + 1], tmul, nb);
                }
                ph[i] = pack2<PDT>(__builtin_amdgcn_exp2f(y0), __builtin_amdgcn_exp2f(y1));
                lt = add_pair(ph[i], lt);
            }
        }
        l_run += lt;
    };
    // Iteration t: (1) P.V of tile t - 1 with tile t's statistics and first
    // two probability pairs between the MFMAs; (2) wait for tile t + 1 and hand
    // the stage of tile t - 1 to a new load; (3) the scores of tile t + 1 with
    // tile t's last two pairs and tile t + 1's V transposition between them.
    auto body = [&](auto stg_tag, f32x4 (&st)[2], f32x4 (&st_next)[2]) {
        constexpr int STG = decltype(stg_tag)::value;
        constexpr int STG_NEXT = (STG + 1) % NS;
        __builtin_amdgcn_sched_barrier(0);
        lds_ptr<uint8_t> vtp = vt_buf((STG + NS - 1) % NS);  // tile t - 1's V^T
        lds_ptr<uint8_t> kn = lds + L::k_at(STG_NEXT);
        float nbase = nbase_run;
        float shift = 0.0f;
        float lt = 0.0f;
        uint32_t nh[2];
        u32x4 vq[VPF];
        for (int i = 0; i < VPF; ++i) vq[i] = vt_operand(vtp, i);
        const u32x4 bv = u32x4{ph[0], ph[1], ph[2], ph[3]};
#pragma unroll
        for (int k = 0; k < FB; ++k) {
            const u32x4 a = vq[k % VPF];
            if (k + VPF < FB) vq[k % VPF] = vt_operand(vtp, k + VPF);
            acc[k] = mfma16<PDT>(a, bv, acc[k]);
            __builtin_amdgcn_sched_barrier(0);
            if (k == 0) {
                if (bulk || (unsigned)(t - tf_lo) < tf_n) {  // t in [tf_lo, tf_hi)
                    float am = amax_run;
                    for (int kb = 0; kb < 2; ++kb)
                        for (int i = 0; i < 4; ++i) am = maxn(am, __builtin_fabsf(st[kb][i]));
                    amax_run = am;
                    if constexpr (CAP)
                        for (int kb = 0; kb < 2; ++kb)
                            for (int i = 0; i < 4; ++i) st[kb][i] = tanh_fast(st[kb][i] * ycap);
                } else {
                    const int lo_rel = min(max(rlo0 - t * PF_KT, 0), PF_KT);
                    const int hi_rel = min(max(rhi0 - t * PF_KT, 0), PF_KT);
                    for (int kb = 0; kb < 2; ++kb)
                        for (int i = 0; i < 4; ++i) {
                            const int kk = 16 * kb + 4 * g + i;
                            const bool vis = kk >= lo_rel && kk < hi_rel;
                            bad |= vis && !(__builtin_fabsf(st[kb][i]) < -NEG_INF);
                            if constexpr (CAP) st[kb][i] = vis ? tanh_fast(st[kb][i] * ycap) : NEG_INF;
                            else st[kb][i] = vis ? st[kb][i] : NEG_INF;
                        }
                }
            }
            if constexpr (!CAP) {
                if (k == 1 && huge) {
                    shift = m_run == NEG_INF ? 0.0f : m_run;
                    for (int kb = 0; kb < 2; ++kb)
                        for (int i = 0; i < 4; ++i) st[kb][i] -= shift;
                    nbase = m_run == NEG_INF ? BASE_NONE : 0.0f;
                }
            }
            // Tile t's first two pairs (tile t - 1's are still being read).
            for (int i = 0; i < 2; ++i) {
                if (k == 2 + (i * (FB - 2)) / 2) {
                    const int kb = i >> 1, r = 2 * (i & 1);
                    const float e0 = __builtin_amdgcn_exp2f(__builtin_fmaf(st[kb][r], tmul, nbase));
                    const float e1 = __builtin_amdgcn_exp2f(__builtin_fmaf(st[kb][r + 1], tmul, nbase));
                    nh[i] = pack2<PDT>(e0, e1);
                    lt = add_pair(nh[i], lt);
                    asm volatile("" : "+v"(nh[i]), "+v"(lt));
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        ph[0] = nh[0];
        ph[1] = nh[1];

        if (bulk) {
            ring_sync_fixed<LPT, NS - 3>();
            issue(std::integral_constant<int, (STG + NS - 1) % NS>{}, std::true_type{});
        } else if (t + 1 < ntiles) {
            wait_tile(t + 1);
            if (t_next < ntiles) issue(std::integral_constant<int, (STG + NS - 1) % NS>{}, std::false_type{});
        } else {
            __syncthreads();
        }

        constexpr int KPRE = 3;
        for (int kb = 0; kb < 2; ++kb)
            for (int i = 0; i < 4; ++i) st_next[kb][i] = 0.0f;
        u32x4 kq[KPRE];
        for (int i = 0; i < KPRE; ++i) kq[i] = k_operand(kn, i);
        lds_ptr<uint8_t> vn = lds + L::v_at(STG_NEXT);
        lds_ptr<uint8_t> vtn = vt_buf(STG_NEXT);
#pragma unroll
        for (int m = 0; m < NQK; ++m) {
            const u32x4 kcur = kq[m % KPRE];
            if (m + KPRE < NQK) kq[m % KPRE] = k_operand(kn, m + KPRE);
            st_next[m % 2] = mfma16<DT>(kcur, qb[m / 2], st_next[m % 2]);
            if (m == 0) __builtin_amdgcn_s_setprio(1);
            if (m == NQK / 2) __builtin_amdgcn_s_setprio(0);
            __builtin_amdgcn_sched_barrier(0);
            if (m == 0) vtr.read(vn);
            if (m == NQK / 2) vtr.write(vtn);
            for (int i = 2; i < 4; ++i) {
                if (m == 1 + ((i - 2) * (NQK - 2)) / 2) {
                    const int kb = i >> 1, r = 2 * (i & 1);
                    const float e0 = __builtin_amdgcn_exp2f(__builtin_fmaf(st[kb][r], tmul, nbase));
                    const float e1 = __builtin_amdgcn_exp2f(__builtin_fmaf(st[kb][r + 1], tmul, nbase));
                    ph[i] = pack2<PDT>(e0, e1);
                    lt = add_pair(ph[i], lt);
                    asm volatile("" : "+v"(ph[i]), "+v"(lt));
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        close_tile(st, shift, lt);
        __builtin_amdgcn_sched_barrier(0);
    };
    while (t < ntiles) {
        bulk = t >= tf_lo && t + NS <= tf_hi && t + 2 * NS - 1 < ntiles && t_next == t + NS - 1;
        static_for<NS>([&](auto k) {
            constexpr int K = decltype(k)::value;
            if (t >= ntiles) return;
            if constexpr (K % 2 == 0) body(std::integral_constant<int, K>{}, st, st_b);
            else body(std::integral_constant<int, K>{}, st_b, st);
            ++t;
        });
        if constexpr (NS % 2 == 1) {
            st[0] = st_b[0];
            st[1] = st_b[1];
        }
    }
    // P.V of the last tile.
    if (ntiles > 0) {
        lds_ptr<uint8_t> vtl = vt_buf((ntiles - 1) % NS);
        const u32x4 bv = u32x4{ph[0], ph[1], ph[2], ph[3]};
#pragma unroll
        for (int fb = 0; fb < FB; ++fb) acc[fb] = mfma16<PDT>(vt_operand(vtl, fb), bv, acc[fb]);
    }
    bad |= !(amax_run < -NEG_INF);
    l_run = row4_sum(l_run);
    bool bad_acc = false;
    for (int fb = 0; fb < FB; ++fb)
        for (int i = 0; i < 4; ++i) bad_acc |= !is_finite_f(acc[fb][i]);
    // bf16 V above f16's range: the rows again on the vector unit in FP32, as
    // in attn_prefill (lane (j, g) holds Q features 32 ks + 8 g .. + 7 and
    // context features 16 fb + 4 g .. + 3 of row j; a score is the four lanes'
    // partial dots added).
    if constexpr (VCONV) {
        if (__ballot(bad_acc && !bad) != 0) {
            const uint8_t *vrows = reinterpret_cast<const uint8_t *>(pv.sg.v) + first * 2;
            const uint8_t *krows = reinterpret_cast<const uint8_t *>(pv.sg.k) + first * 2;
            bool nonfinite, big;
            pf_scan_v(vrows, nkeys, prow, D, lane, nonfinite, big);
            if (__ballot(nonfinite) == 0 && __ballot(big) != 0) {
                for (int fb = 0; fb < FB; ++fb)
                    for (int i = 0; i < 4; ++i) acc[fb][i] = 0.0f;
                float l = 0.0f;
                const bool any = m_run != NEG_INF;
                for (int kk = 0; kk < nkeys; ++kk) {
                    const uint8_t *kr = krows + (int64_t)kk * prow;
                    float d = 0.0f;
                    for (int ks = 0; ks < KS; ++ks) {
                        const u32x4 kw = *gload_ptr<u32x4>(kr + 64 * ks + 16 * g);
                        for (int e = 0; e < 4; ++e) {
                            const uint32_t qw = qb[ks][e], kx = kw[e];
                            d = __builtin_fmaf(lo_f<BF16>(qw), lo_f<BF16>(kx), d);
                            d = __builtin_fmaf(hi_f<BF16>(qw), hi_f<BF16>(kx), d);
                        }
                    }
                    d = row4_sum(d);
                    float y;
                    if constexpr (CAP) y = (tanh_fast(d * ycap) - m_run) * tmul;
                    else y = (d - m_run) * tmul;
                    const bool vis = any && kk >= rlo0 && kk < rhi0;
                    const float pk = vis ? __builtin_amdgcn_exp2f(y) : 0.0f;
                    l += pk;
                    const uint8_t *vr = vrows + (int64_t)kk * prow;
                    for (int fb = 0; fb < FB; ++fb) {
                        const u32x2 vw = *gload_ptr<u32x2>(vr + (16 * fb + 4 * g) * 2);
                        const uint32_t v0 = vw[0], v1 = vw[1];
                        acc[fb][0] = __builtin_fmaf(pk, lo_f<BF16>(v0), acc[fb][0]);
                        acc[fb][1] = __builtin_fmaf(pk, hi_f<BF16>(v0), acc[fb][1]);
                        acc[fb][2] = __builtin_fmaf(pk, lo_f<BF16>(v1), acc[fb][2]);
                        acc[fb][3] = __builtin_fmaf(pk, hi_f<BF16>(v1), acc[fb][3]);
                    }
                }
                l_run = l;  // every lane of the row summed every key
                bad_acc = false;
                for (int fb = 0; fb < FB; ++fb)
                    for (int i = 0; i < 4; ++i) bad_acc |= !is_finite_f(acc[fb][i]);
            }
        }
    }
    bad |= bad_acc;

    const bool single = pv.splits == 1;
    bool bad_mass = false, bad_out = false;
    if (single) {
        if (rvalid) {
            const float inv = 1.0f / l_run;
            bad_mass |= !(l_run > 0.0f) || !is_finite_f(l_run);
            float *orow = pv.out + ((int64_t)t_row * Hq + h_row) * D;
            for (int fb = 0; fb < FB; ++fb) {
                f32x4 v;
                for (int r = 0; r < 4; ++r) {
                    v[r] = acc[fb][r] * inv;
                    bad_out |= !is_finite_f(v[r]);
                }
                *gstore_ptr<f32x4>(orow + 16 * fb + 4 * g) = v;
            }
        }
        raise_status(p, bad, ST_NONFINITE_INPUT);
        raise_status(p, bad_mass, ST_BAD_MASS);
        raise_status(p, bad_out, ST_NONFINITE_OUTPUT);
        return;
    }
    // Split-K partial in attn_prefill's slot format (feature-major context,
    // (max, mass) per row): lanes j of a feature store 16 consecutive rows.
    raise_status(p, bad, ST_NONFINITE_INPUT);
    const int64_t group = (int64_t)kvh * pv.row_blocks + rb;
    const int64_t slot = pv.slot_base + group * pv.splits + split;
    float *pf = p.part_o + slot * ROWS * D + wave * RW + j;
    for (int fb = 0; fb < FB; ++fb)
        for (int r = 0; r < 4; ++r)
            *gstore_ptr<float>(pf + (int64_t)(16 * fb + 4 * g + r) * ROWS) = acc[fb][r];
    if (g == 0) {
        const f32x2 ml = {m_run, l_run};
        *gstore_ptr<f32x2>(p.part_ml + (slot * ROWS + wave * RW + j) * 2) = ml;
    }
}

// Merge of the split-K partials of attn_prefill.  Merge block b covers 64
// packed rows and 16 features of one (problem, KV head, row block); each
// thread owns four features of one row and reads the S partials of its row at
// once (one round trip): m and l of every split, then the weighted sum of the
// unnormalised contexts.  Problem::part_base is the problem's first merge block.
template <int D, int ROWS>
__global__ __launch_bounds__(256) void attn_prefill_merge(Params p, int64_t blocks) {
    // The fields below arrive through dependent scalar loads (the block
    // count, the problem count, the problem): their lines are brought in
    // together first (Params, `blocks` and the hidden arguments after them).
    warm_kernarg<(sizeof(Params) + sizeof(int64_t) + 63) / 64, 0>();
    constexpr int FB = D / 16;                  // 16-feature blocks per row
    constexpr int RC = ROWS / 64;               // 64-row chunks per row block
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
    const int64_t group = local / (RC * FB);              // kvh * row_blocks + rb
    const int within = (int)(local % (RC * FB));
    const int kvh = (int)(group / pr->row_blocks), rb = (int)(group % pr->row_blocks);
    // Thread (fq, rr) = (threadIdx.x / 64, threadIdx.x % 64): row rr of the
    // block's 64, features 4 fq .. 4 fq + 3 of its 16, so each dword load of
    // a wave reads 64 consecutive rows of one feature.
    const int r = (within / FB) * 64 + (int)(threadIdx.x & 63);
    const int f = (within % FB) * 16 + (int)(threadIdx.x >> 6) * 4;
    const int prow = rb * ROWS + r;
    if (prow >= m_kv) return;
    const int S = pr->splits;
    const int64_t slot0 = pr->slot_base + group * S;

    f32x2 ml[MAXS];
    f32x4 po[MAXS];
#pragma unroll
    for (int sp = 0; sp < MAXS; ++sp) {
        if (sp < S) {
            ml[sp] = *gload_ptr<f32x2>(p.part_ml + ((slot0 + sp) * ROWS + r) * 2);
            const float *col = p.part_o + ((slot0 + sp) * D + f) * ROWS + r;
            for (int e = 0; e < 4; ++e) po[sp][e] = *gload_ptr<float>(col + (int64_t)e * ROWS);
        }
    }
    float M = NEG_INF;
#pragma unroll
    for (int sp = 0; sp < MAXS; ++sp)
        if (sp < S) M = fmaxf(M, ml[sp][0]);
    const float mbase = M == NEG_INF ? 0.0f : M;
    const float tmul = p.softcap != 0.0f ? p.softcap_log2 : p.scale_log2;  // the chunk kernel's units
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

extern "C" int tkh_prefill_waves(int head_dim, int wide) {
    return wide ? tkh::pf_wide_waves(head_dim) : tkh::PF_WAVES_NARROW;
}
extern "C" int tkh_prefill_max_splits(void) { return 16; }
extern "C" int tkh_prefill_merge_blocks_per_row_block(int head_dim, int rows) {
    return (rows / 64) * (head_dim / 16);
}

extern "C" hipError_t tkh_launch_prefill_merge(const tkh::Params *p, int head_dim, int rows,
                                               int64_t blocks, hipStream_t stream,
                                               hipEvent_t start, hipEvent_t stop) {
    using namespace tkh;
    dim3 grid((unsigned)blocks), block(256);
#define TKH_PM(DD, RR)                                                                           \
    if (head_dim == DD && rows == RR) {                                                          \
        hipExtLaunchKernelGGL((attn_prefill_merge<DD, RR>), grid, block, 0, stream, start, stop, 0, \
                              *p, blocks);                                                       \
        return hipGetLastError();                                                                \
    }
    TKH_PM(64, 128) TKH_PM(128, 128) TKH_PM(128, 256) TKH_PM(256, 128) TKH_PM(128, 64) TKH_PM(256, 64)
#undef TKH_PM
    return hipErrorInvalidValue;
}

extern "C" hipError_t tkh_launch_prefill(const tkh::PrefillArgs *p, int dtype, int head_dim, int waves,
                                         int64_t groups, hipStream_t stream, hipEvent_t start,
                                         hipEvent_t stop) {
    using namespace tkh;
    dim3 grid((unsigned)groups), block(64 * waves);
#define TKH_PF(DT, DD, WW)                                                              \
    if (dtype == DT && head_dim == DD && waves == WW) {                                 \
        if (p->p.softcap != 0.0f)                                                       \
            hipExtLaunchKernelGGL((attn_prefill<DT, DD, true, WW>), grid, block, 0, stream, start, stop, 0, *p);  \
        else                                                                            \
            hipExtLaunchKernelGGL((attn_prefill<DT, DD, false, WW>), grid, block, 0, stream, start, stop, 0, *p); \
        return hipGetLastError();                                                       \
    }
    TKH_PF(BF16, 64, 4) TKH_PF(BF16, 128, 4) TKH_PF(BF16, 128, 8) TKH_PF(BF16, 256, 4)
    TKH_PF(F16, 64, 4) TKH_PF(F16, 128, 4) TKH_PF(F16, 128, 8) TKH_PF(F16, 256, 4)
#undef TKH_PF
    return hipErrorInvalidValue;
}

// The 16-row kernel: `waves` 16-row waves per workgroup (8: the four-wave
// 32-row kernel's 128-row blocks, grid and workspace; 4: 64-row blocks).
extern "C" hipError_t tkh_launch_prefill16(const tkh::PrefillArgs *p, int dtype, int head_dim, int waves,
                                           int64_t groups, hipStream_t stream, hipEvent_t start,
                                           hipEvent_t stop) {
    using namespace tkh;
    dim3 grid((unsigned)groups), block(64 * waves);
#define TKH_PF16(DT, DD, WW)                                                            \
    if (dtype == DT && head_dim == DD && waves == WW) {                                 \
        if (p->p.softcap != 0.0f)                                                       \
            hipExtLaunchKernelGGL((attn_prefill16<DT, DD, true, WW>), grid, block, 0, stream, start, stop, 0, *p);  \
        else                                                                            \
            hipExtLaunchKernelGGL((attn_prefill16<DT, DD, false, WW>), grid, block, 0, stream, start, stop, 0, *p); \
        return hipGetLastError();                                                       \
    }
    TKH_PF16(BF16, 128, 8) TKH_PF16(BF16, 256, 8) TKH_PF16(F16, 128, 8) TKH_PF16(F16, 256, 8)
    TKH_PF16(BF16, 128, 4) TKH_PF16(BF16, 256, 4) TKH_PF16(F16, 128, 4) TKH_PF16(F16, 256, 4)
#undef TKH_PF16
    return hipErrorInvalidValue;
}
