// gemm_epi.h -- the dense GEMM's epilogue through LDS: the tile's outputs
// rounded to bf16 into LDS, then written to Y in 16-byte chunks along whole
// tile rows.  Out::Bf16 and Out::Residual (src/metal/kernels.rs:223-236);
// the same bits as the direct stores, whose pattern (each store
// instruction: 16 rows x 32 bytes) left the L2 merging partial lines and
// measured 5-15% of a 2048 x 18432 x 2560 GEMM.
//
// Included after the kernel's constants: BM, BN (rows of X and of W per
// tile), TM, TN (per wave), IM, IN (MFMA blocks per wave), FM (16 | 32), N,
// OUT, NT (threads) and the accumulator type acc_t.
#pragma once

// HB_EPI_NT 1 (the including kernel's choice): the output chunks are
// written with non-temporal stores, which do not displace the operands other
// tiles still read from the caches (measured in the ping-pong GEMM: the M=2048
// layer step 352-357 -> 335 us, every GEMM of it faster; 8192^3 +5%).
#ifndef HB_EPI_NT
#define HB_EPI_NT 0
#endif

// Bytes per staged tile row: the 16 bytes of padding move consecutive rows
// four banks apart.
constexpr u32 EPI_ROW = BN * 2 + 16;
// Bf16 and Residual outputs whose rows are whole 16-byte chunks.
constexpr bool EPI_LDS = OUT != 1 && N % 8 == 0 && BN % 8 == 0;
// u32x4 of LDS the staging needs (0: direct stores).
constexpr u32 EPI_CHUNKS = EPI_LDS ? BM * EPI_ROW / 16 : 0;

// The tile at (row0, n0) of `rows` valid rows: lane (fr, fc) of wave (wm,
// wn) holds, per MFMA block (i, j), runs of 4 columns of one row.  Every
// wave must be past its last LDS read of the main loop (the barrier here
// sees to it) and `lds` must hold EPI_CHUNKS.
HB_DEV void epilogue_lds(u32x4* lds, const acc_t (&acc)[IN][IM], u32 tid, u32 wm, u32 wn, u32 fr,
                         u32 fc, u32 row0, u32 rows, u32 n0, void* Yv) {
    __syncthreads();
    u16* t = (u16*)lds;
#pragma unroll
    for (u32 j = 0; j < IM; j++) {
#pragma unroll
        for (u32 i = 0; i < IN; i++) {
#pragma unroll
            for (u32 q = 0; q < FM * FM / 256; q++) {
                const u32 r = wm * TM + j * FM + fr, c = wn * TN + i * FM + q * 8 + 4 * fc;
                const acc_t& v = acc[i][j];
                u32x2 o;
                o.x = pack_bf16x2(v[4 * q], v[4 * q + 1]);
                o.y = pack_bf16x2(v[4 * q + 2], v[4 * q + 3]);
                *(u32x2*)(t + r * (EPI_ROW / 2) + c) = o;
            }
        }
    }
    __syncthreads();
    constexpr u32 CPR = BN / 8;  // 16-byte chunks per tile row
    for (u32 c = tid; c < BM * CPR; c += NT) {
        const u32 r = c / CPR, n = n0 + (c % CPR) * 8;
        if (r >= rows || n >= N) continue;
        u32x4 v = *(const u32x4*)(t + r * (EPI_ROW / 2) + (c % CPR) * 8);
        u32x4* dst = (u32x4*)((u16*)Yv + (u64)(row0 + r) * N + n);
        if constexpr (OUT == 2) {
            // y = rne(f(y) + f(rne(acc))): the staged value is rne(acc).
            const u32x4 old = *dst;
#pragma unroll
            for (u32 e = 0; e < 4; e++)
                v[e] = pack_bf16x2(bf16_lo(old[e]) + bf16_lo(v[e]), bf16_hi(old[e]) + bf16_hi(v[e]));
        }
        if constexpr (HB_EPI_NT)
            __builtin_nontemporal_store(v, dst);
        else
            *dst = v;
    }
}
