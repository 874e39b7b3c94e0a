// hb_common.h -- shared device helpers of the HIP kernel sources.  These
// sources are compiled by hiprtc at load for gfx950 with every shape baked in
// as -D constants (the role the reference's MSL emission at load plays,
// src/msl/mod.rs:1-27); the build embeds them in libherbert_hip.so.
#pragma once

typedef unsigned int u32;
typedef unsigned short u16;
typedef unsigned long long u64;
typedef u32 u32x2 __attribute__((ext_vector_type(2)));
typedef u32 u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

#define HB_DEV __device__ __attribute__((always_inline)) inline

// src/core/bf16.rs:7-9: exact widening.
HB_DEV float bf16_to_f32(u32 h) { return __builtin_bit_cast(float, h << 16); }
HB_DEV float bf16_lo(u32 w) { return __builtin_bit_cast(float, w << 16); }
HB_DEV float bf16_hi(u32 w) { return __builtin_bit_cast(float, w & 0xffff0000u); }

// src/core/bf16.rs:13-23, src/msl/mod.rs:1333-1347: (bits + 0x7fff + lsb) >> 16.
HB_DEV u32 f32_to_bf16(float f) {
    u32 b = __builtin_bit_cast(u32, f);
    return (b + 0x7fffu + ((b >> 16) & 1u)) >> 16;
}
HB_DEV float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }
HB_DEV u32 pack_bf16x2(float lo, float hi) { return f32_to_bf16(lo) | (f32_to_bf16(hi) << 16); }

// exp of f32: Cody-Waite reduction by ln 2 and the minimax polynomial of
// Moshier's Cephes expf, every step an explicit fma, so that the CPU checker
// built with the same steps gives the same bits.
HB_DEV float hb_expf(float x) {
    if (x > 88.72283905206835f) return __builtin_inff();
    if (x < -103.278929903431851103f) return 0.0f;
    if (x != x) return x;
    float n = __builtin_floorf(__builtin_fmaf(x, 1.44269504088896341f, 0.5f));
    float r = __builtin_fmaf(n, -0.693359375f, x);
    r = __builtin_fmaf(n, 2.12194440e-4f, r);
    float z = r * r;
    float p = 1.9875691500e-4f;
    p = __builtin_fmaf(p, r, 1.3981999507e-3f);
    p = __builtin_fmaf(p, r, 8.3334519073e-3f);
    p = __builtin_fmaf(p, r, 4.1665795894e-2f);
    p = __builtin_fmaf(p, r, 1.6666665459e-1f);
    p = __builtin_fmaf(p, r, 5.0000001201e-1f);
    p = __builtin_fmaf(p, z, r);
    p = p + 1.0f;
    int e = (int)n;
    int e1 = e / 2, e2 = e - e / 2;
    float s1 = __builtin_bit_cast(float, (u32)(e1 + 127) << 23);
    float s2 = __builtin_bit_cast(float, (u32)(e2 + 127) << 23);
    return (p * s1) * s2;
}

// src/msl/mod.rs:885-890: 1 / (1 + e^-x), an IEEE division.
HB_DEV float hb_sigmoid(float x) { return 1.0f / (1.0f + hb_expf(-x)); }

// The row count of a block: state[3] as the reference's kernels read it
// (src/metal/kernels.rs:15, prefill.rs:21-24), never more than the rows the
// launch was sized for.
#define STATE_ROWS 3
HB_DEV u32 rows_of_state(const u32* state, u32 m_launch) {
    u32 m = state[STATE_ROWS];
    return m < m_launch ? m : m_launch;
}

// The workgroups a launch of `groups` spreads over the 8 XCDs round robin
// (workgroup g runs on XCD g % 8): the logical index that gives each XCD a
// contiguous range of tiles, so that tiles sharing a panel of W or X share
// that XCD's L2.
HB_DEV u32 xcd_remap(u32 g, u32 groups) {
    const u32 x = g & 7u, i = g >> 3;
    const u32 q = groups >> 3, r = groups & 7u;
    return x * q + (x < r ? x : r) + i;
}

// The kernel's symbol: the emitted name (gemm_mma_2560x4608_..., set with
// -DHB_NAME by the library), so profiles tell the variants apart.
#ifndef HB_NAME
#define HB_NAME hb_kernel
#endif
