// decode_bf16_256.hip - attn_decode builds for bf16 K/V at head_dim 256.
#include "decode_kernel.hpp"

TKH_DECODE_UNIT(BF16, 256, bf16_256)
