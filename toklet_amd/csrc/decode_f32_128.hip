// decode_f32_128.hip - attn_decode builds for f32 K/V at head_dim 128.
#include "decode_kernel.hpp"

TKH_DECODE_UNIT(F32, 128, f32_128)
