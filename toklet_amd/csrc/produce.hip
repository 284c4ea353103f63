// produce.hip - the step before attention on the session path: per-head
// RMSNorm of Q and K, rotary position embedding, rounding to the cache dtype,
// and the K/V append into head-major rows, in one launch.
//
// Order and arithmetic follow Model::run (src/model/mod.rs:611-662):
//  * rmsnorm (src/cpu/reductions.rs:8-49): squares and their sum in FP64,
//    denominator sqrt(sum / D + eps) in FP64, value = f32(x * (1 / den) * w) in
//    FP64 (the reference divides by den; the reciprocal form can move the FP64
//    value by an ulp, which changes the FP32 result only at a rounding tie);
//  * rotary (src/cpu/attention.rs:10-64): frequency theta^(-2j/D), angle =
//    position * frequency and sine/cosine in FP64, rounded to FP32; rotation
//    a*c - b*s, b*c + a*s in FP32 with separate roundings (no contraction);
//  * proportional rotary (src/cpu/proportional_rotary.rs:32-91): inverse
//    frequency base^(-2j/D) / factor for pairs j < rotated_dims / 2, other
//    features copied;
//  * Llama 3 rotary (src/cpu/llama3_rotary.rs:44-61, 87-146): the ordinary
//    frequency theta^(-2j/D) kept for wavelengths below original/high, divided
//    by factor above original/low, blended linearly in original/wavelength in
//    between, all in FP64; angle and rotation as for split-half;
//  * LayerKv::append (src/model/cache.rs:64-85): token-major new rows into
//    head-major cache rows, here rounded once to the cache dtype.
// The FP64 sum runs in a different order than the reference's sequential one;
// the denominator can differ in its last FP64 bit, which reaches an FP32
// result only at a rounding tie.
//
// One wave per (token, head slot): slots [0, Hq) are query heads, [Hq,
// Hq + Hkv) key heads, the rest value heads.  Non-finite inputs or results set
// the device status word (the reference returns Error::NonFinite).
#include "device.hpp"

namespace tkh {


namespace {

__host__ __device__ __forceinline__ int rotary_pairs(int kind, int D, int rotated_dims) {
    return (kind == 1 || kind == 3) ? D / 2 : (kind == 2 ? rotated_dims / 2 : 0);
}

// Inverse frequency of pair j in FP64: theta^(-2j/D), divided by factor for
// the proportional form (src/cpu/proportional_rotary.rs:68-70), or scaled by
// wavelength band for Llama 3 (Llama3Scaling::inverse_frequency,
// src/cpu/llama3_rotary.rs:44-61; 6.283185307179586 is 2*pi rounded to FP64).
__device__ __forceinline__ double inverse_frequency(const RotarySpec &r, int D, int j) {
#pragma clang fp contract(off)
    const double ordinary = pow((double)r.theta, -(2.0 * (double)j) / (double)D);
    if (r.kind == 2) return ordinary / (double)r.factor;
    if (r.kind != 3) return ordinary;
    const double factor = r.factor, low = r.low, high = r.high;
    const double wavelength = 6.283185307179586 / ordinary;
    if (factor == 1.0 || wavelength < r.original / high) return ordinary;
    if (wavelength > r.original / low) return ordinary / factor;
    const double smooth = (r.original / wavelength - low) / (high - low);
    return (1.0 - smooth) * ordinary / factor + smooth * ordinary;
}

// Rotation of pair j at absolute position pos: angle and sine/cosine in FP64,
// rounded once to FP32 (src/cpu/attention.rs:41-46,
// src/cpu/proportional_rotary.rs:68-74, src/cpu/llama3_rotary.rs:126-128).
__device__ __forceinline__ void rotary_cos_sin(const RotarySpec &r, int D, int64_t pos, int j,
                                               float *c, float *s) {
#pragma clang fp contract(off)
    const double angle = (double)pos * inverse_frequency(r, D, j);
    *s = (float)sin(angle);
    *c = (float)cos(angle);
}

template <int DT> __device__ __forceinline__ void store_out(void *base, int64_t i, float x);
template <> __device__ __forceinline__ void store_out<F32>(void *base, int64_t i, float x) {
    reinterpret_cast<float *>(base)[i] = x;
}
template <> __device__ __forceinline__ void store_out<F16>(void *base, int64_t i, float x) {
    reinterpret_cast<_Float16 *>(base)[i] = (_Float16)x;
}
template <> __device__ __forceinline__ void store_out<BF16>(void *base, int64_t i, float x) {
    reinterpret_cast<__bf16 *>(base)[i] = (__bf16)x;  // round to nearest even
}


}  // namespace

// TABLE: (cos, sin) come from p.rope.  Without it the kernel carries the FP64
// pow/sin/cos of rotary_cos_sin, which takes its register count to 129: three
// waves per SIMD instead of four, so a session chunk's 4096 waves
// needed a second round (launch span 6.7 us, the last waves starting 3.9 us
// late).  Sessions always pass the table.
template <int DT, bool TABLE>
__global__ __launch_bounds__(64) void produce_qkv(ProduceParams p) {
#pragma clang fp contract(off)
    // Its fields arrive through dependent scalar loads: their lines (and the
    // hidden arguments' start) first, in one round trip.
    warm_kernarg<(sizeof(ProduceParams) + 63) / 64, 0>();
    __shared__ float row[512];
    const int lane = threadIdx.x;
    const int D = p.d;
    const int slots = p.hq + 2 * p.hkv;
    const int64_t t = blockIdx.x / slots;
    const int slot = (int)(blockIdx.x % slots);
    if (t >= p.tokens) return;
    const int kind = slot < p.hq ? 0 : (slot < p.hq + p.hkv ? 1 : 2);  // q, k, v
    const int h = kind == 0 ? slot : (kind == 1 ? slot - p.hq : slot - p.hq - p.hkv);
    const int heads = kind == 0 ? p.hq : p.hkv;
    const float *src = (kind == 0 ? p.q : (kind == 1 ? p.k : p.v)) + (t * heads + h) * D;
    void *dst = kind == 0 ? p.q_out : (kind == 1 ? p.k_out : p.v_out);
    const int64_t dst0 = kind == 0 ? (t * p.hq + h) * D : h * p.out_head_stride + t * D;

    // Every load first (the row, the norm weights, the rotary pairs), then the
    // arithmetic: one memory round trip per launch instead of three.
    constexpr int KMAX = 8;  // elements per lane, D <= 512
    const float *w = kind == 0 ? p.q_norm : (kind == 1 ? p.k_norm : nullptr);
    const int half = D / 2;
    const int pairs = kind == 2 ? 0 : rotary_pairs(p.rot.kind, D, p.rot.rotated_dims);
    float xv[KMAX], wv[KMAX], cv[KMAX / 2], sv[KMAX / 2];
    for (int k = 0; k < KMAX; ++k) {
        const int i = lane + 64 * k;
        xv[k] = i < D ? src[i] : 0.0f;
        wv[k] = w && i < D ? w[i] : 0.0f;
    }
    for (int k = 0; k < KMAX / 2; ++k) {
        const int j = lane + 64 * k;
        cv[k] = 1.0f;
        sv[k] = 0.0f;
        if (j < half && j < pairs) {
            if constexpr (TABLE) {
                const float *cs = p.rope + 2 * ((p.position + t - p.rope_pos0) * pairs + j);
                cv[k] = cs[0];
                sv[k] = cs[1];
            } else {
                rotary_cos_sin(p.rot, D, p.position + t, j, &cv[k], &sv[k]);
            }
        }
    }

    bool bad = false;
    for (int k = 0; k < KMAX; ++k)
        if (lane + 64 * k < D) bad |= !is_finite_f(xv[k]);
    if (kind == 2) {
        for (int k = 0; k < KMAX; ++k)
            if (lane + 64 * k < D) store_out<DT>(dst, dst0 + lane + 64 * k, xv[k]);
        raise_status(p.status, bad, ST_NONFINITE_INPUT);
        return;
    }
    if (w) {
        double ss = 0.0;
        for (int k = 0; k < KMAX; ++k)
            if (lane + 64 * k < D) {
                const double x = (double)xv[k];
                ss += x * x;
            }
        ss = wave_sum_f64(ss);
        const double inv = 1.0 / sqrt(ss / (double)D + (double)p.eps);
        for (int k = 0; k < KMAX; ++k)
            if (lane + 64 * k < D) {
                const float y = (float)((double)xv[k] * inv * (double)wv[k]);
                bad |= !is_finite_f(y) || !is_finite_f(wv[k]);
                xv[k] = y;
            }
    }
    // The rotary pairs elements j and j + D/2, which may sit in other lanes:
    // through LDS (one wave, whose LDS accesses complete in order).
    for (int k = 0; k < KMAX; ++k)
        if (lane + 64 * k < D) row[lane + 64 * k] = xv[k];
    __syncthreads();
    for (int k = 0; k < KMAX / 2; ++k) {
        const int j = lane + 64 * k;
        if (j >= half) break;
        const float a = row[j], b = row[j + half];
        float x = a, y = b;
        if (j < pairs) {
            const float c = cv[k], sn = sv[k];
            const float ac = a * c, bs = b * sn, bc = b * c, as = a * sn;
            x = ac - bs;
            y = bc + as;
            bad |= !is_finite_f(x) || !is_finite_f(y);
        }
        store_out<DT>(dst, dst0 + j, x);
        store_out<DT>(dst, dst0 + j + half, y);
    }
    raise_status(p.status, bad, ST_NONFINITE_INPUT);
}

// (cos, sin) of every (position, pair) for rows [pos0, pos0 + rows): the
// producer's table, filled once per session with the same FP64 formulas.
__global__ __launch_bounds__(256) void rotary_table(float *out, int64_t pos0, int64_t rows,
                                                    int pairs, RotarySpec rot, int D) {
#pragma clang fp contract(off)
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * pairs) return;
    const int64_t r = i / pairs;
    const int j = (int)(i % pairs);
    float c, s;
    rotary_cos_sin(rot, D, pos0 + r, j, &c, &s);
    out[2 * i] = c;
    out[2 * i + 1] = s;
}

}  // namespace tkh

extern "C" int tkh_rotary_pairs(int rotary, int head_dim, int rotated_dims) {
    return tkh::rotary_pairs(rotary, head_dim, rotated_dims);
}

extern "C" hipError_t tkh_launch_rotary_table(float *out, int64_t pos0, int64_t rows,
                                              const tkh::RotarySpec *rot, int head_dim,
                                              hipStream_t stream) {
    using namespace tkh;
    const int pairs = rotary_pairs(rot->kind, head_dim, rot->rotated_dims);
    const int64_t n = rows * pairs;
    if (n <= 0) return hipSuccess;
    dim3 grid((unsigned)((n + 255) / 256)), block(256);
    hipLaunchKernelGGL(rotary_table, grid, block, 0, stream, out, pos0, rows, pairs, *rot,
                       head_dim);
    return hipGetLastError();
}

extern "C" hipError_t tkh_launch_produce(const tkh::ProduceParams *p, int dtype, hipStream_t stream) {
    using namespace tkh;
    const int64_t blocks = p->tokens * (p->hq + 2 * p->hkv);
    if (blocks <= 0 || p->d > 512 || p->d % 2) return hipErrorInvalidValue;
    dim3 grid((unsigned)blocks), block(64);
    const bool table = p->rope != nullptr;
    if (dtype == F32) {
        if (table) hipLaunchKernelGGL((produce_qkv<F32, true>), grid, block, 0, stream, *p);
        else hipLaunchKernelGGL((produce_qkv<F32, false>), grid, block, 0, stream, *p);
    } else if (dtype == F16) {
        if (table) hipLaunchKernelGGL((produce_qkv<F16, true>), grid, block, 0, stream, *p);
        else hipLaunchKernelGGL((produce_qkv<F16, false>), grid, block, 0, stream, *p);
    } else if (dtype == BF16) {
        if (table) hipLaunchKernelGGL((produce_qkv<BF16, true>), grid, block, 0, stream, *p);
        else hipLaunchKernelGGL((produce_qkv<BF16, false>), grid, block, 0, stream, *p);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}
