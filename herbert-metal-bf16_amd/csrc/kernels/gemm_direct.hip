// gemm_direct.hip -- the prefill GEMM with the MFMA operands read straight
// from memory, no LDS staging (gemm.mma=2): a tile of TM rows of X by TN
// rows of W per workgroup, one 16 x 16 output block per wavefront
// ((TM/16) x (TN/16) wavefronts), v_mfma_f32_16x16x32_bf16 over all of K;
// the wavefronts of a workgroup share the tile's rows through the caches.
//
// Reference: src/metal/prefill.rs:442-569 (gemm_mm2d / gemm_mm2d_rows: one
// tm x tn tile, 16/32/64 each, over the whole K read from device memory, the
// epilogue of Out; groups gemm_mm2d_groups = ceil(m/tm) * ceil(N/tn)).
// Constants: HB_K, HB_N, HB_OUT, HB_BM (= tm), HB_BN (= tn), HB_MFIRST.
// Bindings: state, W, X, Y, two unused; then m.
#include "hb_common.h"

constexpr u32 K = HB_K, N = HB_N, TM = HB_BM, TN = HB_BN;
constexpr int OUT = HB_OUT;
constexpr u32 WM = TM / 16, WN = TN / 16, NT = 64 * WM * WN;
constexpr u32 NTILES = (N + TN - 1) / TN;
constexpr u32 U = 4;  // K steps of 32 in flight, each its own accumulator
static_assert(TM % 16 == 0 && TN % 16 == 0 && NT <= 1024, "tiles of 16..64");
static_assert(K % 32 == 0, "K a multiple of 32");

HB_DEV void store4(void* Yv, u64 at, float v0, float v1, float v2, float v3) {
    if constexpr (OUT == 1) {
        *(f32x4*)((float*)Yv + at) = f32x4{v0, v1, v2, v3};
    } else if constexpr (OUT == 2) {
        u32x2* p = (u32x2*)((u16*)Yv + at);
        u32x2 old = *p, o;
        o.x = pack_bf16x2(bf16_lo(old.x) + round_bf16(v0), bf16_hi(old.x) + round_bf16(v1));
        o.y = pack_bf16x2(bf16_lo(old.y) + round_bf16(v2), bf16_hi(old.y) + round_bf16(v3));
        *p = o;
    } else {
        *(u32x2*)((u16*)Yv + at) = u32x2{pack_bf16x2(v0, v1), pack_bf16x2(v2, v3)};
    }
}

extern "C" __global__ __launch_bounds__(NT) void HB_NAME(
    const u32* __restrict__ state, const u16* __restrict__ W, const u16* __restrict__ X,
    void* __restrict__ Yv, const u32* __restrict__ unused0, const u32* __restrict__ unused1,
    u32 m_launch) {
    const u32 m = rows_of_state(state, m_launch);
    const u32 mb = (m + TM - 1) / TM;
    const u32 g = blockIdx.x;
    u32 gm, gn;
    if (HB_MFIRST) { gm = g % mb; gn = g / mb; }
    else { gn = g % NTILES; gm = g / NTILES; }
    if (gm >= mb || gn >= NTILES) return;
    const u32 lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const u32 wm = wave % WM, wn = wave / WM;
    const u32 r = lane & 15u, q = lane >> 4;
    u32 xr = gm * TM + wm * 16 + r, wr = gn * TN + wn * 16 + r;
    xr = xr < m ? xr : m - 1;
    wr = wr < N ? wr : N - 1;
    // Lane (r, q) holds elements q*8.. of each 32-K step (A: W row, B: X row).
    const u16* wp = W + (u64)wr * K + q * 8;
    const u16* xp = X + (u64)xr * K + q * 8;
    f32x4 acc[U];
#pragma unroll
    for (u32 u = 0; u < U; u++) acc[u] = f32x4{0.f, 0.f, 0.f, 0.f};
    u32 k0 = 0;
    for (; k0 + 32 * U <= K; k0 += 32 * U) {
        u32x4 a[U], b[U];
#pragma unroll
        for (u32 u = 0; u < U; u++) {
            a[u] = *(const u32x4*)(wp + k0 + 32 * u);
            b[u] = *(const u32x4*)(xp + k0 + 32 * u);
        }
#pragma unroll
        for (u32 u = 0; u < U; u++)
            acc[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a[u]),
                                                             __builtin_bit_cast(bf16x8, b[u]),
                                                             acc[u], 0, 0, 0);
    }
    for (; k0 < K; k0 += 32) {
        const u32x4 a = *(const u32x4*)(wp + k0), b = *(const u32x4*)(xp + k0);
        acc[0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                         __builtin_bit_cast(bf16x8, b), acc[0],
                                                         0, 0, 0);
    }
#pragma unroll
    for (u32 u = 1; u < U; u++) acc[0] += acc[u];
    // Lane (r, q): rows 4q..4q+3 of the block's W rows for X row r.
    const u32 row = gm * TM + wm * 16 + r;
    const u32 n = gn * TN + wn * 16 + 4 * q;
    if (row < m && n < N) store4(Yv, (u64)row * N + n, acc[0][0], acc[0][1], acc[0][2], acc[0][3]);
}
