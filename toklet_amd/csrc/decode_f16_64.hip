// decode_f16_64.hip - attn_decode builds for f16 K/V at head_dim 64.
#include "decode_kernel.hpp"

TKH_DECODE_UNIT(F16, 64, f16_64)
