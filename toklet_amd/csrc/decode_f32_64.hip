// decode_f32_64.hip - attn_decode builds for f32 K/V at head_dim 64.
#include "decode_kernel.hpp"

TKH_DECODE_UNIT(F32, 64, f32_64)
