// decode_bf16_128.hip - attn_decode builds for bf16 K/V at head_dim 128.
#include "decode_kernel.hpp"

TKH_DECODE_UNIT(BF16, 128, bf16_128)
