// gemm_mfma.hip -- the prefill block GEMM and the grouped expert GEMM on
// gfx950's matrix cores: Y[m][N] = X[m][K] . W[N][K]^T, bf16 operands, f32
// accumulators, one rounding at the output as Out says.
//
// Reference: src/metal/prefill.rs:838-1307 (gemm_mma_rows / gemm_mma_impl:
// the tile staged in threadgroup memory, the clamped rows, the epilogue of
// Out at :1200-1230, the expert rows of MmaRows at :317-338 and :1004-1048).
//
// The MI355X design (not a translation of the MSL):
//  - A workgroup of WM x WN wavefronts (64 lanes) computes a BN x BM tile
//    of Y^T: the MFMA's A operand is a fragment of W, its B operand a
//    fragment of X, so each lane ends with runs of 4 consecutive columns n
//    of one row m and the epilogue stores 8 bytes (bf16) per lane.
//  - v_mfma_f32_16x16x32_bf16 or v_mfma_f32_32x32x16_bf16 (HB_MFMA).
//  - X and W tiles of BK along K are staged in LDS as 16-byte chunks with an
//    XOR swizzle of the chunk index by (row >> SWZ), so that the ds_read_b128
//    of a fragment (16 or 32 rows at one chunk) hits distinct banks; the
//    global loads are 128-bit and coalesced (CH consecutive lanes read one
//    row's BK elements).
//  - HB_DBUF: two LDS stages, the next K tile's global loads in flight while
//    the current one is multiplied, one barrier per K tile.
//  - HB_ORDER 1: the workgroup index remapped so each XCD works on a
//    contiguous range of tiles (its own L2 keeps their panels).
//
// Compile-time constants (-D): HB_K, HB_N, HB_OUT (0 bf16, 1 f32, 2
// residual), HB_ROWS (0 dense, 1 gather, 2 scatter), HB_TOPK, HB_BM, HB_BN,
// HB_BK, HB_WM, HB_WN, HB_MFMA (16|32), HB_DBUF, HB_SWZ, HB_ORDER, HB_MFIRST.
//
// Bindings: state (u32[4], state[3] = rows), W, X, Y, list, tiles; then the
// rows the launch was sized for (m_launch).  Dense: rows past m read the
// last valid row and are not stored.  Experts: tile t of the table is
// (expert, first sorted row, rows); groups past tiles[0] return.
#include "hb_common.h"

constexpr u32 K = HB_K, N = HB_N;
constexpr int OUT = HB_OUT, ROWS = HB_ROWS;
constexpr u32 TOPK = HB_TOPK;
constexpr u32 BM = HB_BM, BN = HB_BN, BK = HB_BK;
constexpr u32 WM = HB_WM, WN = HB_WN, NT = 64 * WM * WN;
constexpr u32 FM = HB_MFMA;
constexpr u32 TM = BM / WM, TN = BN / WN;
constexpr u32 IM = TM / FM, IN = TN / FM;
constexpr u32 CH = BK / 8;                 // 16-byte chunks of a staged row
constexpr u32 KS = FM == 16 ? 32 : 16;     // K of one MFMA
constexpr u32 KT = K / BK;
constexpr u32 NTILES = (N + BN - 1) / BN;
constexpr u32 XCH = BM * CH, WCH = BN * CH; // chunks per stage
constexpr u32 X_LD = (XCH + NT - 1) / NT, W_LD = (WCH + NT - 1) / NT;
constexpr u32 NBUF = HB_DBUF ? 2 : 1;

static_assert(K % BK == 0, "K a multiple of the K step");
static_assert(N % 4 == 0, "N a multiple of 4");
static_assert(TM % FM == 0 && TN % FM == 0, "wave tile a multiple of the MFMA block");
static_assert(BK % KS == 0 && (CH & (CH - 1)) == 0, "K step");
static_assert(NT % CH == 0, "threads a multiple of the chunks of a row");

typedef __attribute__((ext_vector_type(FM == 16 ? 4 : 16))) float acc_t;

HB_DEV u32 lpos(u32 r, u32 c) { return r * CH + (c ^ ((r >> HB_SWZ) & (CH - 1))); }

HB_DEV acc_t mfma(bf16x8 a, bf16x8 b, acc_t c) {
#if HB_MFMA == 16
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
#else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
#endif
}

// Four consecutive outputs (columns n..n+3 of row `yrow`), as Out says
// (src/metal/kernels.rs:223-236).
HB_DEV void store4(void* Yv, u64 at, float v0, float v1, float v2, float v3) {
    if constexpr (OUT == 1) {
        f32x4 o = {v0, v1, v2, v3};
        *(f32x4*)((float*)Yv + at) = o;
    } else if constexpr (OUT == 2) {
        u32x2* p = (u32x2*)((u16*)Yv + at);
        u32x2 old = *p;
        u32x2 o;
        o.x = pack_bf16x2(bf16_lo(old.x) + round_bf16(v0), bf16_hi(old.x) + round_bf16(v1));
        o.y = pack_bf16x2(bf16_lo(old.y) + round_bf16(v2), bf16_hi(old.y) + round_bf16(v3));
        *p = o;
    } else {
        u32x2 o;
        o.x = pack_bf16x2(v0, v1);
        o.y = pack_bf16x2(v2, v3);
        *(u32x2*)((u16*)Yv + at) = o;
    }
}

extern "C" __global__ __launch_bounds__(NT) void hb_kernel(
    const u32* __restrict__ state, const u16* __restrict__ W, const u16* __restrict__ X,
    void* __restrict__ Yv, const u32* __restrict__ list, const u32* __restrict__ tiles,
    u32 m_launch) {
    __shared__ u32x4 sX[NBUF][XCH];
    __shared__ u32x4 sW[NBUF][WCH];

    const u32 tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const u32 wm = wave % WM, wn = wave / WM;
    u32 g = blockIdx.x;
    if (HB_ORDER == 1) g = xcd_remap(g, gridDim.x);

    // The tile: its first row (dense row or sorted pair), its rows, its
    // column tile and its expert.
    u32 row0, rows, gn, expert = 0;
    u32 m = m_launch;
    if constexpr (ROWS == 0) {
        m = rows_of_state(state, m_launch);
        const u32 mb = (m + BM - 1) / BM;
        u32 gm;
        if (HB_MFIRST) { gm = g % mb; gn = g / mb; }
        else { gn = g % NTILES; gm = g / NTILES; }
        if (gm >= mb || gn >= NTILES) return;
        row0 = gm * BM;
        rows = m - row0 < BM ? m - row0 : BM;
    } else {
        const u32 tmax = gridDim.x / NTILES;
        u32 t;
        if (HB_MFIRST) { t = g % tmax; gn = g / tmax; }
        else { gn = g % NTILES; t = g / NTILES; }
        if (t >= tiles[0]) return;
        expert = tiles[1 + 3 * t];
        row0 = tiles[2 + 3 * t];
        rows = tiles[3 + 3 * t];
    }
    const u32 pairs = m_launch * TOPK;  // experts: sorted rows of the block
    const u32 n0 = gn * BN;

    // Global element offsets of this thread's chunks (row clamped to the
    // last valid one), per K tile advanced by BK.
    const u32 c = tid % CH;
    u32 xoff[X_LD], woff[W_LD];
#pragma unroll
    for (u32 q = 0; q < X_LD; q++) {
        u32 r = tid / CH + q * (NT / CH);
        if (r >= BM) r = BM - 1;
        u32 rr = r < rows ? r : rows - 1;
        u32 xrow;
        if constexpr (ROWS == 1) {
            u32 pr = list[row0 + rr] / TOPK;
            xrow = pr < m_launch ? pr : m_launch - 1;
        } else if constexpr (ROWS == 2) {
            u32 p = row0 + rr;
            xrow = p < pairs ? p : pairs - 1;
        } else {
            xrow = row0 + rr;
        }
        xoff[q] = xrow * K + c * 8;
    }
#pragma unroll
    for (u32 q = 0; q < W_LD; q++) {
        u32 r = tid / CH + q * (NT / CH);
        if (r >= BN) r = BN - 1;
        u32 n = n0 + r;
        if (n >= N) n = N - 1;
        woff[q] = (expert * N + n) * K + c * 8;
    }

    u32x4 rx[X_LD], rw[W_LD];
    auto load = [&](u32 kt) {
#pragma unroll
        for (u32 q = 0; q < X_LD; q++) rx[q] = *(const u32x4*)(X + xoff[q] + kt * BK);
#pragma unroll
        for (u32 q = 0; q < W_LD; q++) rw[q] = *(const u32x4*)(W + (u64)woff[q] + kt * BK);
    };
    auto stage = [&](u32 buf) {
#pragma unroll
        for (u32 q = 0; q < X_LD; q++) {
            u32 id = tid + q * NT;
            if (XCH % NT == 0 || id < XCH) sX[buf][lpos(id / CH, id % CH)] = rx[q];
        }
#pragma unroll
        for (u32 q = 0; q < W_LD; q++) {
            u32 id = tid + q * NT;
            if (WCH % NT == 0 || id < WCH) sW[buf][lpos(id / CH, id % CH)] = rw[q];
        }
    };

    acc_t acc[IN][IM];
#pragma unroll
    for (u32 i = 0; i < IN; i++)
#pragma unroll
        for (u32 j = 0; j < IM; j++) acc[i][j] = acc_t{};

    const u32 fr = lane % FM, fc = lane / FM;
    auto multiply = [&](u32 buf) {
#pragma unroll
        for (u32 s = 0; s < BK / KS; s++) {
            const u32 ch = s * (KS / 8) + fc;
            bf16x8 a[IN], b[IM];
#pragma unroll
            for (u32 i = 0; i < IN; i++)
                a[i] = __builtin_bit_cast(bf16x8, sW[buf][lpos(wn * TN + i * FM + fr, ch)]);
#pragma unroll
            for (u32 j = 0; j < IM; j++)
                b[j] = __builtin_bit_cast(bf16x8, sX[buf][lpos(wm * TM + j * FM + fr, ch)]);
#pragma unroll
            for (u32 i = 0; i < IN; i++)
#pragma unroll
                for (u32 j = 0; j < IM; j++) acc[i][j] = mfma(a[i], b[j], acc[i][j]);
        }
    };

    load(0);
    stage(0);
    __syncthreads();
    for (u32 kt = 0; kt < KT; kt++) {
        const u32 cur = NBUF == 2 ? (kt & 1u) : 0u;
        if (kt + 1 < KT) load(kt + 1);
        multiply(cur);
        if constexpr (NBUF == 2) {
            if (kt + 1 < KT) stage(cur ^ 1u);
            __syncthreads();
        } else {
            __syncthreads();
            if (kt + 1 < KT) {
                stage(0);
                __syncthreads();
            }
        }
    }

    // Epilogue: lane holds, per MFMA block, runs of 4 columns of one row.
#pragma unroll
    for (u32 j = 0; j < IM; j++) {
        const u32 ml = wm * TM + j * FM + fr;
        if (ml >= rows) continue;
        u32 yrow;
        if constexpr (ROWS == 2) {
            u32 s = list[row0 + ml];
            yrow = s < pairs ? s : pairs - 1;
        } else {
            yrow = row0 + ml;
        }
#pragma unroll
        for (u32 i = 0; i < IN; i++) {
#pragma unroll
            for (u32 q = 0; q < FM * FM / 256; q++) {
                // FM 16: one run, columns 4*fc..+3 of the block; FM 32: four
                // runs, columns q*8 + 4*fc..+3.
                const u32 nl = wn * TN + i * FM + q * 8 + 4 * fc;
                const u32 n = n0 + nl;
                if (n < N) {
                    const acc_t& v = acc[i][j];
                    store4(Yv, (u64)yrow * N + n, v[4 * q], v[4 * q + 1], v[4 * q + 2],
                           v[4 * q + 3]);
                }
            }
        }
    }
}
