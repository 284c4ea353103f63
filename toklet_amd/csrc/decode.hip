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
