// decode_f32_256.hip - attn_decode builds for f32 K/V at head_dim 256.
#include "decode_kernel.hpp"

TKH_DECODE_UNIT(F32, 256, f32_256)
