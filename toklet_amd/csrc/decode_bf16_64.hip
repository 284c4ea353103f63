// decode_bf16_64.hip - attn_decode builds for bf16 K/V at head_dim 64.
#include "decode_kernel.hpp"

TKH_DECODE_UNIT(BF16, 64, bf16_64)
