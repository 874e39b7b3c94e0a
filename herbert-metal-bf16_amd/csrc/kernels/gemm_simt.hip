// gemm_simt.hip -- the prefill GEMM on the vector ALUs (gemm.mma=0):
// Y[m][N] = X[m][K] . W[N][K]^T with each output summed by one thread in
// increasing k, f32 fma of exact bf16 products: the CPU contract's order, so
// its outputs equal the scalar oracle's bit for bit.
//
// Reference: src/metal/prefill.rs:121-307 (gemm_simt: a 64 x 64 tile per
// group of 256 threads, 4 x 4 accumulators per thread, K staged by 16 as
// f32, rows past m or N clamped on read and not stored; groups
// gemm_simt_groups = ceil(m/64) * ceil(N/64)).
// Constants: HB_K, HB_N, HB_OUT, HB_MFIRST.  Bindings: state, W, X, Y, and
// two unused ones (the expert GEMMs' list and tiles); then m.
#include "hb_common.h"

constexpr u32 K = HB_K, N = HB_N, T = 64, KB = 16;
constexpr int OUT = HB_OUT;
constexpr u32 NTILES = (N + T - 1) / T;
static_assert(K % KB == 0, "K a multiple of 16");

HB_DEV void store1(void* Yv, u64 at, float v) {
    if constexpr (OUT == 1) {
        ((float*)Yv)[at] = v;
    } else if constexpr (OUT == 2) {
        u16* p = (u16*)Yv + at;
        *p = (u16)f32_to_bf16(bf16_to_f32(*p) + round_bf16(v));
    } else {
        ((u16*)Yv)[at] = (u16)f32_to_bf16(v);
    }
}

extern "C" __global__ __launch_bounds__(256) void HB_NAME(
    const u32* __restrict__ state, const u16* __restrict__ W, const u16* __restrict__ X,
    void* __restrict__ Yv, const u32* __restrict__ unused0, const u32* __restrict__ unused1,
    u32 m_launch) {
    __shared__ float sX[KB][T + 1], sW[KB][T + 1];  // K-major, padded
    const u32 m = rows_of_state(state, m_launch);
    const u32 mb = (m + T - 1) / T;
    const u32 g = blockIdx.x;
    u32 gm, gn;
    if (HB_MFIRST) { gm = g % mb; gn = g / mb; }
    else { gn = g % NTILES; gm = g / NTILES; }
    if (gm >= mb || gn >= NTILES) return;
    const u32 m0 = gm * T, n0 = gn * T, tid = threadIdx.x;
    const u32 tx = tid % 16, ty = tid / 16;  // outputs rows ty*4.., cols tx*4..
    // Loader: thread t stages row t/4, k (t%4)*4..+3 of each tile.
    const u32 lr = tid / 4, lk = (tid % 4) * 4;
    const u32 xr = m0 + lr < m ? m0 + lr : m - 1;
    const u32 wr = n0 + lr < N ? n0 + lr : N - 1;
    const u16* xp = X + (u64)xr * K + lk;
    const u16* wp = W + (u64)wr * K + lk;
    float acc[4][4];
#pragma unroll
    for (u32 i = 0; i < 4; i++)
#pragma unroll
        for (u32 j = 0; j < 4; j++) acc[i][j] = 0.0f;
    for (u32 k0 = 0; k0 < K; k0 += KB) {
        const u32x2 xv = *(const u32x2*)(xp + k0), wv = *(const u32x2*)(wp + k0);
        __syncthreads();
        sX[lk][lr] = bf16_lo(xv.x);
        sX[lk + 1][lr] = bf16_hi(xv.x);
        sX[lk + 2][lr] = bf16_lo(xv.y);
        sX[lk + 3][lr] = bf16_hi(xv.y);
        sW[lk][lr] = bf16_lo(wv.x);
        sW[lk + 1][lr] = bf16_hi(wv.x);
        sW[lk + 2][lr] = bf16_lo(wv.y);
        sW[lk + 3][lr] = bf16_hi(wv.y);
        __syncthreads();
#pragma unroll
        for (u32 kk = 0; kk < KB; kk++) {
            float a[4], b[4];
#pragma unroll
            for (u32 i = 0; i < 4; i++) a[i] = sX[kk][ty * 4 + i];
#pragma unroll
            for (u32 j = 0; j < 4; j++) b[j] = sW[kk][tx * 4 + j];
#pragma unroll
            for (u32 i = 0; i < 4; i++)
#pragma unroll
                for (u32 j = 0; j < 4; j++) acc[i][j] = __builtin_fmaf(a[i], b[j], acc[i][j]);
        }
    }
#pragma unroll
    for (u32 i = 0; i < 4; i++) {
        const u32 r = m0 + ty * 4 + i;
        if (r >= m) continue;
#pragma unroll
        for (u32 j = 0; j < 4; j++) {
            const u32 n = n0 + tx * 4 + j;
            if (n < N) store1(Yv, (u64)r * N + n, acc[i][j]);
        }
    }
}
