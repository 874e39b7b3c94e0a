// gemm_splitk.hip -- the second kernel of a split-K GEMM: the parts' f32
// sums added in part order and written as Out says.
//
// Reference: src/metal/kernels.rs:223-236 (the Out epilogue: Bf16 rounds
// once, F32 stores the sum, Residual adds the rounded sum to Y's bf16 and
// rounds again); the fold of partial sums in a fixed order follows
// matvec_split's (src/metal/kernels.rs:917-950), whose split-K parts are
// added in simdgroup order.
//
// The GEMM (gemm_mfma.hip with HB_KSPLIT = s) wrote slab p = the f32 sums of
// Y[m][N] over part p's K range, slabs [m_launch][N] apart.  Here each
// thread takes 4 consecutive outputs per step: acc = slab 0, then + slab 1,
// ..., + slab s-1 (f32, in that order, so the bits do not depend on the
// launch), then one rounding.  The GEMM's launch ends before this one
// starts (same stream), so no fence is needed between the two.
//
// Compile-time constants (-D): HB_N, HB_OUT (0 bf16, 1 f32, 2 residual),
// HB_KSPLIT (the parts), HB_NAME.
// Bindings: state (u32[4], state[3] = rows), P (the slabs), Y; then the
// rows the launch was sized for (m_launch).
#include "hb_common.h"

constexpr u32 N = HB_N, KSP = HB_KSPLIT;
constexpr int OUT = HB_OUT;
static_assert(N % 4 == 0 && KSP >= 2 && KSP <= 16, "N a multiple of 4, 2..16 parts");

extern "C" __global__ __launch_bounds__(256) void HB_NAME(const u32* __restrict__ state,
                                                         const float* __restrict__ P,
                                                         void* __restrict__ Yv, u32 m_launch) {
    const u32 m = rows_of_state(state, m_launch);
    const u64 quads = (u64)m * (N / 4), slab = (u64)m_launch * (N / 4);
    const f32x4* p4 = (const f32x4*)P;
    for (u64 i = (u64)blockIdx.x * 256 + threadIdx.x; i < quads; i += (u64)gridDim.x * 256) {
        f32x4 parts[KSP];
#pragma unroll
        for (u32 p = 0; p < KSP; p++) parts[p] = __builtin_nontemporal_load(&p4[p * slab + i]);
        f32x4 a = parts[0];
#pragma unroll
        for (u32 p = 1; p < KSP; p++) a = a + parts[p];
        if constexpr (OUT == 1) {
            ((f32x4*)Yv)[i] = a;
        } else {
            u32x2* y = (u32x2*)Yv + i;
            u32x2 o;
            if constexpr (OUT == 2) {
                const u32x2 old = *y;
                o.x = pack_bf16x2(bf16_lo(old.x) + round_bf16(a.x), bf16_hi(old.x) + round_bf16(a.y));
                o.y = pack_bf16x2(bf16_lo(old.y) + round_bf16(a.z), bf16_hi(old.y) + round_bf16(a.w));
            } else {
                o.x = pack_bf16x2(a.x, a.y);
                o.y = pack_bf16x2(a.z, a.w);
            }
            *y = o;
        }
    }
}
