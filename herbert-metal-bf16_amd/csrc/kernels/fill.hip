// fill.hip -- zero `words` 16-byte words (hb_zero), a kernel rather than a
// memset so that it can sit in a captured HIP graph.
#include "hb_common.h"

extern "C" __global__ __launch_bounds__(256) void HB_NAME(u32x4* __restrict__ p, u64 words) {
    const u64 i = (u64)blockIdx.x * 256u + threadIdx.x;
    if (i < words) p[i] = u32x4{0u, 0u, 0u, 0u};
}
