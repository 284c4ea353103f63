// decode_f16_128.hip - attn_decode builds for f16 K/V at head_dim 128.
#include "decode_kernel.hpp"

TKH_DECODE_UNIT(F16, 128, f16_128)
