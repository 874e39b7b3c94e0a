// fill.hip -- zero the bytes [p, p + n) (hb_zero), a kernel rather than a
// memset or a copy so that it can sit in a captured HIP graph.  Thread t
// owns the 16-byte-aligned word t of the range's span: whole words by one
// 16-byte store, the ragged first and last words byte by byte, so the wide
// stores only ever see 16-byte-aligned addresses.
#include "hb_common.h"

extern "C" __global__ __launch_bounds__(256) void HB_NAME(unsigned char* __restrict__ p, u64 n) {
    const u64 start = (u64)p, end = start + n, base = start & ~15ull;
    const u64 i = (u64)blockIdx.x * 256u + threadIdx.x;
    const u64 a = base + 16 * i;
    if (a >= end) return;
    if (a >= start && a + 16 <= end) {
        *(u32x4*)a = u32x4{0u, 0u, 0u, 0u};
    } else {
        for (u64 b = a < start ? start : a; b < a + 16 && b < end; b++) *(unsigned char*)b = 0;
    }
}
