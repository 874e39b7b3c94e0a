// probe.hip -- the rounding probe of herbert-metal-probe `round`
// (src/bin/herbert-metal-probe.rs:7-11): chunk c (state[0], 0..255) of every
// f32 bit pattern, pattern (c << 24) | i, rounded to bf16 by the kernels'
// integer form (f32_to_bf16, the epilogues' rounding) into out_int[i], and
// by the compiler's conversion to __bf16 (gfx950's v_cvt_pk_bf16_f32) into
// out_hw[i].  Bindings: state, out_int (u16[2^24]), out_hw (u16[2^24]).
#include "hb_common.h"

extern "C" __global__ __launch_bounds__(256) void HB_NAME(const u32* __restrict__ state,
                                                           u16* __restrict__ out_int,
                                                           u16* __restrict__ out_hw, u32 m) {
    (void)m;
    const u32 i = blockIdx.x * 256u + threadIdx.x;
    const u32 bits = (state[0] << 24) | i;
    const float f = __builtin_bit_cast(float, bits);
    out_int[i] = (u16)f32_to_bf16(f);
    out_hw[i] = __builtin_bit_cast(u16, (__bf16)f);
}
