// decode_f16_256.hip - attn_decode builds for f16 K/V at head_dim 256.
#include "decode_kernel.hpp"

TKH_DECODE_UNIT(F16, 256, f16_256)
