// project.hip - the step after attention: the FP32 o-projection of context
// rows onto a vocabulary and the greedy token of each row, on the device.
//
// logits[r, v] = sum_d context[r, d] * weights[v, d], formed exactly as the
// reference's FP32 matmul forms it (src/cpu/mod.rs:208-247): one running FP32
// sum per (row, output), products and additions each rounded, in feature
// order.  One lane owns one (row, vocab) sum for the whole feature range, so
// the logits are the reference's bit for bit, and the greedy choice
// (src/sampling.rs:5-18: the largest logit, the lowest id on ties, +0 and -0
// equal) follows from them exactly.
//
// The weights are read once per block of context rows, which makes a decode
// step (one row) a stream over [vocab, hidden] FP32: HBM-bound.
//
//  * project_logits: a workgroup owns 256 vocabulary rows (one per lane) and
//    R context rows.  Feature tiles of 32 stage the 256 weight rows through
//    LDS with coalesced 16-byte loads (rows padded to 36 floats, so a lane's
//    16-byte reads of its own row hit distinct bank groups within each
//    16-lane phase) while the context tile is read by every lane at once (a
//    broadcast); the next tile's loads are in flight while a tile is
//    multiplied.  At the end the workgroup reduces, per row, the best
//    (key, id) pair of its 256 candidates and stores it.
//  * project_pick: one wave per row reduces those pairs to the token.
//
// Keys order finite floats as unsigned integers (the sign-folded bit
// pattern, both zeros mapped to one key); a pair is (key << 32) | ~id, so
// the largest pair has the largest logit and, among equal ones, the lowest
// id.  A non-finite logit raises the status word and never becomes a
// candidate.
#include "device.hpp"

namespace tkh {

namespace {

constexpr int PJ_V = 256;   // vocabulary rows per workgroup, one per lane
// 32 features per tile keep a workgroup's LDS at 37 KiB, so four fit on a CU
// and a one-row launch over a 151,936-row vocabulary (594 workgroups) runs
// in one round; 64-feature tiles (70 KiB, two per CU) left 82 workgroups to
// a second round on an otherwise idle device.
constexpr int PJ_D = 32;    // features per staged tile
constexpr int PJ_CPR = PJ_D / 4;  // 16-byte chunks per staged row
constexpr int PJ_PAD = 36;  // staged row stride in floats

__device__ __forceinline__ uint32_t order_key(float x) {
    const uint32_t b = __builtin_bit_cast(uint32_t, x);
    if ((b & 0x7fffffffu) == 0) return 0x80000000u;  // +0 and -0
    return (b & 0x80000000u) ? ~b : (b ^ 0x80000000u);
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t x) {
    for (int m = 32; m >= 1; m >>= 1) {
        const uint32_t lo = __shfl_xor((uint32_t)x, m, 64);
        const uint32_t hi = __shfl_xor((uint32_t)(x >> 32), m, 64);
        const uint64_t y = ((uint64_t)hi << 32) | lo;
        x = y > x ? y : x;
    }
    return x;
}

}  // namespace

template <int R, bool VEC>
__global__ __launch_bounds__(256) void project_logits(ProjectParams p) {
#pragma clang fp contract(off)
    __shared__ __attribute__((aligned(16))) float wt[PJ_V * PJ_PAD];
    __shared__ __attribute__((aligned(16))) float ct[R * PJ_D];
    __shared__ uint64_t best_lds[R * 4];
    const int t = threadIdx.x;
    const int64_t v0 = (int64_t)blockIdx.x * PJ_V;
    const int64_t r0 = (int64_t)blockIdx.y * R;
    const int64_t H = p.hidden;
    const int nr = (int)(p.rows - r0 < R ? p.rows - r0 : R);
    float acc[R];
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;

    // Features past the end of the range are zeros in both tiles: adding
    // their +-0 products leaves every sum unchanged (a sum that starts at +0
    // is never -0).
    auto compute = [&]() {
        for (int q = 0; q < PJ_D / 4; ++q) {
            const f32x4 w = *reinterpret_cast<const f32x4 *>(wt + t * PJ_PAD + 4 * q);
            for (int r = 0; r < R; ++r) {
                const f32x4 c = *reinterpret_cast<const f32x4 *>(ct + r * PJ_D + 4 * q);
                float s = acc[r];
                s = s + c[0] * w[0];
                s = s + c[1] * w[1];
                s = s + c[2] * w[2];
                s = s + c[3] * w[3];
                acc[r] = s;
            }
        }
    };

    if constexpr (VEC) {
        // Thread t stages chunks i = t + 256 n (n < PJ_CPR) of the tile: row
        // i / PJ_CPR, features 4 (i % PJ_CPR) ..+3; the context tile's
        // R x PJ_CPR chunks likewise.
        // A tile's loads are all issued at once, and later tiles' go out
        // before the current one is multiplied: one tile ahead, or two for a
        // single context row, whose launch is a bare stream of the weights
        // (two register sets; the two sets alternate, unrolled by two, so no
        // set is copied).
        constexpr int NW = PJ_V * PJ_CPR / 256;            // weight chunks per thread
        constexpr int NC = (R * PJ_CPR + 255) / 256;       // context chunks per thread
        constexpr int AHEAD = R == 1 ? 2 : 1;              // tiles in flight
        f32x4 wb[2][NW], cb[2][NC];
        auto load = [&](int64_t d0, f32x4 (&w)[NW], f32x4 (&cx)[NC]) {
            const int dn = (int)(H - d0 < PJ_D ? H - d0 : PJ_D);
#pragma unroll
            for (int n = 0; n < NW; ++n) {
                const int i = t + 256 * n, row = i / PJ_CPR, c = i % PJ_CPR;
                const int64_t v = v0 + row;
                w[n] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                if (v < p.vocab && 4 * c < dn)
                    w[n] = __builtin_nontemporal_load(gload_ptr<f32x4>(p.weights + v * H + d0 + 4 * c));
            }
#pragma unroll
            for (int n = 0; n < NC; ++n) {
                const int i = t + 256 * n, r = i / PJ_CPR, c = i % PJ_CPR;
                cx[n] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                if (i < R * PJ_CPR && r < nr && 4 * c < dn)
                    cx[n] = *gload_ptr<f32x4>(p.context + (r0 + r) * H + d0 + 4 * c);
            }
        };
        auto stage = [&](const f32x4 (&w)[NW], const f32x4 (&cx)[NC]) {
            __syncthreads();  // the previous tile is no longer read
#pragma unroll
            for (int n = 0; n < NW; ++n) {
                const int i = t + 256 * n;
                *reinterpret_cast<f32x4 *>(wt + (i / PJ_CPR) * PJ_PAD + 4 * (i % PJ_CPR)) = w[n];
            }
#pragma unroll
            for (int n = 0; n < NC; ++n) {
                const int i = t + 256 * n;
                if (i < R * PJ_CPR) *reinterpret_cast<f32x4 *>(ct + (i / PJ_CPR) * PJ_D + 4 * (i % PJ_CPR)) = cx[n];
            }
            __syncthreads();
        };
        if constexpr (AHEAD == 1) {
            load(0, wb[0], cb[0]);
            for (int64_t d0 = 0; d0 < H; d0 += PJ_D) {
                stage(wb[0], cb[0]);
                if (d0 + PJ_D < H) load(d0 + PJ_D, wb[0], cb[0]);
                compute();
            }
        } else {
            load(0, wb[0], cb[0]);
            if (PJ_D < H) load(PJ_D, wb[1], cb[1]);
            for (int64_t d0 = 0; d0 < H; d0 += 2 * PJ_D) {
                stage(wb[0], cb[0]);
                if (d0 + 2 * PJ_D < H) load(d0 + 2 * PJ_D, wb[0], cb[0]);
                compute();
                if (d0 + PJ_D >= H) break;
                stage(wb[1], cb[1]);
                if (d0 + 3 * PJ_D < H) load(d0 + 3 * PJ_D, wb[1], cb[1]);
                compute();
            }
        }
    } else {
        for (int64_t d0 = 0; d0 < H; d0 += PJ_D) {
            const int dn = (int)(H - d0 < PJ_D ? H - d0 : PJ_D);
            __syncthreads();
            for (int i = t; i < PJ_V * PJ_D; i += 256) {
                const int row = i / PJ_D, c = i % PJ_D;
                const int64_t v = v0 + row;
                wt[row * PJ_PAD + c] = v < p.vocab && c < dn ? p.weights[v * H + d0 + c] : 0.0f;
            }
            for (int i = t; i < R * PJ_D; i += 256) {
                const int r = i / PJ_D, c = i % PJ_D;
                ct[i] = r < nr && c < dn ? p.context[(r0 + r) * H + d0 + c] : 0.0f;
            }
            __syncthreads();
            compute();
        }
    }

    const int64_t v = v0 + t;
    const bool valid = v < p.vocab;
    bool bad = false;
    const int wave = t >> 6, lane = t & 63;
    for (int r = 0; r < R; ++r) {
        if (r >= nr) break;
        const float x = acc[r];
        const bool finite = is_finite_f(x);
        bad |= valid && !finite;
        if (p.logits && valid) p.logits[(r0 + r) * p.vocab + v] = x;
        const uint64_t pair = valid && finite ? ((uint64_t)order_key(x) << 32) | (uint32_t)~(uint32_t)v : 0;
        const uint64_t m = wave_max_u64(pair);
        if (lane == 0) best_lds[r * 4 + wave] = m;
    }
    __syncthreads();
    if (t < nr) {
        uint64_t m = best_lds[t * 4];
        for (int w = 1; w < 4; ++w) m = best_lds[t * 4 + w] > m ? best_lds[t * 4 + w] : m;
        p.pairs[(r0 + t) * p.vblocks + blockIdx.x] = m;
    }
    raise_status(p.status, bad, ST_NONFINITE_LOGIT);
}

__global__ __launch_bounds__(64) void project_pick(ProjectParams p) {
    const int64_t row = blockIdx.x;
    const int lane = threadIdx.x;
    uint64_t m = 0;
    for (int i = lane; i < p.vblocks; i += 64) {
        const uint64_t x = p.pairs[row * p.vblocks + i];
        m = x > m ? x : m;
    }
    m = wave_max_u64(m);
    if (lane == 0) p.tokens[row] = m == 0 ? 0xffffffffu : ~(uint32_t)m;
}

}  // namespace tkh

extern "C" int tkh_project_vocab_per_block(void) { return tkh::PJ_V; }

extern "C" hipError_t tkh_launch_project(const tkh::ProjectParams *p, hipStream_t stream,
                                         hipEvent_t start, hipEvent_t stop) {
    using namespace tkh;
    const bool vec = p->hidden % 4 == 0 && (reinterpret_cast<uintptr_t>(p->weights) & 15) == 0;
    const int R = p->rows <= 1 ? 1 : (p->rows <= 4 ? 4 : 16);
    const dim3 grid((unsigned)p->vblocks, (unsigned)((p->rows + R - 1) / R)), block(256);
#define TKH_PJ(RR, VV)                                                                           \
    if (R == RR && vec == VV) {                                                                  \
        hipExtLaunchKernelGGL((project_logits<RR, VV>), grid, block, 0, stream, start, nullptr, 0, \
                              *p);                                                               \
    }
    TKH_PJ(1, true) TKH_PJ(1, false) TKH_PJ(4, true) TKH_PJ(4, false) TKH_PJ(16, true)
    TKH_PJ(16, false)
#undef TKH_PJ
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipExtLaunchKernelGGL(project_pick, dim3((unsigned)p->rows), dim3(64), 0, stream, nullptr, stop,
                          0, *p);
    return hipGetLastError();
}
