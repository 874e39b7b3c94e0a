// gemm_pp.hip -- the prefill block GEMM with its K loop software-pipelined
// across or within wavefronts: Y[m][N] = X[m][K] . W[N][K]^T, bf16 operands,
// f32 accumulators, one rounding at the output as Out says.  Two schedules
// (HB_SCHED): 1, two groups of four wavefronts that take turns on the matrix
// cores ("ping-pong"); 3, four wavefronts, one per SIMD, each issuing its
// next K tile's LDS reads between its MFMAs (larger wave tiles: fewer LDS
// bytes per flop).
//
// Reference: src/metal/prefill.rs:838-1307 (gemm_mma_rows / gemm_mma_impl:
// the staged K loop at :1177-1192, the clamped rows, the epilogue of Out at
// :1200-1230), src/metal/prefill.rs:615-631 (nax_tile_order, the band order).
//
// Why a second schedule.  In the lock-step form (gemm_mfma.hip) every wave
// of a workgroup waits for the same stage at the same barrier, so a stage
// that lands late idles all four matrix cores at once, and the kernel's time
// came out near the sum of its MFMA time and its load time.  Here the eight
// wavefronts of a workgroup are two groups of four, one wave of each group on
// every SIMD, and each group alternates a memory phase and a compute phase,
// half a period apart from the other:
//
//   barrier | group A: MEM(k)   | group B: COMP(k-1) | barrier
//   barrier | group A: COMP(k)  | group B: MEM(k)    | barrier
//
//  - MEM(k): issue this wave's share of the direct-to-LDS loads (gfx950's
//    buffer_load_dwordx4 ... lds) of K tile k + NS - 1 into the stage K tile
//    k - 1 used; read the wave's MFMA fragments of K tile k from LDS into
//    registers; wait until its own loads of K tile k + 1 have landed and its
//    LDS reads are done.
//  - COMP(k): the MFMAs of K tile k on those registers, at raised wave
//    priority.
//  Each SIMD then always has one wave issuing MFMAs while the other waits on
//  memory; a barrier is where the roles swap.  The loads of a K tile are
//  issued NS - 1 tiles ahead (three with four stages), so the L2/HBM latency
//  is covered by about 2 * (NS - 1) phases of MFMA work.
//
// HB_SCHED 3 (four waves, wave tiles of TM x TN, two fragment register sets):
//   barrier B_k | loads of K tile k + NS into stage k % NS;
//               | MFMAs of tile k (fragments in set k % 2) interleaved with
//               |   the LDS reads of tile k + 1's fragments into set 1 - k % 2;
//               | own loads of tile k + 2 landed, LDS reads done | B_{k+1}
//  Stage k % NS is free at B_k: tile k's fragments were read during step k-1
//  and every wave waited for those reads before B_k.  Tile k + 1 is visible
//  at B_k: every wave waited for its own loads of it at the end of step k-1.
//  Loads run NS - 1 steps ahead of the barrier that needs them.
//
// Ordering (phase p = the span between two barriers; A runs MEM(k) in phase
// 2k and COMP(k) in 2k+1, B one phase later):
//  - the stage MEM(k) loads into was last read in MEM(k-1), i.e. by A in
//    phase 2k-2 and by B in phase 2k-1, each wave waiting for its LDS reads
//    before the barrier that closes the phase; A loads in phase 2k, B in
//    2k+1: both after every read.
//  - K tile k+1 is read by A in phase 2k+2; every wave waited for its own
//    loads of it by the end of phase 2k+1 (A in phase 2k, B in 2k+1), and
//    direct-to-LDS data is in LDS once the wave's vmcnt says so.
//
// Layout and staging follow gemm_mfma.hip: 16-byte chunks of BK elements per
// row, XOR-swizzled by (row >> SWZ) so fragment reads are conflict-free; the
// MFMA's A operand is a W fragment and its B operand an X fragment, so a
// lane holds runs of 4 consecutive columns of one row and stores 8 bytes.
// Rows past m load from past the buffer range (zeros, no memory access) and
// are not stored; W rows past N are clamped and not stored.
//
// Compile-time constants (-D): HB_K, HB_N, HB_OUT (0 bf16, 1 f32, 2
// residual), HB_BM, HB_BN, HB_BK, HB_WM, HB_WN (WM * WN = 8), HB_MFMA (16|32),
// HB_STAGES (3|4), HB_SWZ, HB_ORDER, HB_MFIRST, HB_BAND, HB_SCHED (1 | 3),
// HB_GRP (ping-pong: which waves form a group: 0 waves 0-3 / 4-7, 1 even /
// odd waves), HB_KSPLIT (s > 1: K cut into s parts, part p's f32 sums into
// slab p of Y, [m_launch][N] floats each, as in gemm_mfma.hip; a second
// kernel adds the slabs).
//
// Bindings: state (u32[4], state[3] = rows), W, X, Y, list, tiles (unused:
// dense rows); then the rows the launch was sized for (m_launch).
#include "hb_common.h"

constexpr u32 K = HB_K, N = HB_N;
constexpr int OUT = HB_OUT;
constexpr u32 BM = HB_BM, BN = HB_BN, BK = HB_BK;
#ifndef HB_SCHED
#define HB_SCHED 1
#endif
constexpr bool PP = HB_SCHED == 1;
constexpr u32 WM = HB_WM, WN = HB_WN, NWV = PP ? 8 : 4, NT = 64 * NWV;
constexpr u32 FM = HB_MFMA;
constexpr u32 TM = BM / WM, TN = BN / WN;
constexpr u32 IM = TM / FM, IN = TN / FM;
constexpr u32 CH = BK / 8;                 // 16-byte chunks of a staged row
constexpr u32 KS = FM == 16 ? 32 : 16;     // K of one MFMA
constexpr u32 S = BK / KS;                 // MFMA steps per K tile
#ifndef HB_KSPLIT
#define HB_KSPLIT 1
#endif
constexpr u32 KSP = HB_KSPLIT;
constexpr u32 KT = K / BK / KSP;           // K tiles of one part
constexpr u32 NS = HB_STAGES;
constexpr u32 NTILES = (N + BN - 1) / BN;
constexpr u32 XST = BM * CH, WST = BN * CH;  // chunks per stage
// Wave-loads (64 chunks, 1 KiB) per stage of each operand, shared out over
// the NWV waves: wave w issues the operand's wave-loads w, w + NWV, ...; when
// a count is not a multiple of NWV the first waves issue one more.
constexpr u32 NXL = XST / 64, NWL = WST / 64;
constexpr u32 XLMAX = (NXL + NWV - 1) / NWV, WLMAX = (NWL + NWV - 1) / NWV;
constexpr u32 LMIN = NXL / NWV + NWL / NWV;  // loads per stage of every wave
#ifndef HB_BAND
#define HB_BAND 0
#endif
#ifndef HB_GRP
#define HB_GRP 0
#endif

static_assert(HB_SCHED == 1 || HB_SCHED == 3, "schedule 1 or 3");
static_assert(WM * WN == NWV, "eight wavefronts (ping-pong) or four");
static_assert(K % (BK * KSP) == 0, "K a multiple of the K step times the parts");
static_assert(KSP == 1 || OUT == 1, "split K: f32 partial sums");
static_assert(N % 4 == 0, "N a multiple of 4");
static_assert(TM % FM == 0 && TN % FM == 0, "wave tile a multiple of the MFMA block");
static_assert(BK % KS == 0 && (CH & (CH - 1)) == 0, "K step");
static_assert(XST % 64 == 0 && WST % 64 == 0, "whole wave-loads per stage");
static_assert(NS >= 3 && NS <= 4, "3 or 4 stages");
static_assert(PP || KT % 2 == 0, "four-wave schedule: an even count of K tiles");
static_assert(LMIN >= 1, "every wave loads");

typedef __attribute__((ext_vector_type(FM == 16 ? 4 : 16))) float acc_t;

HB_DEV acc_t mfma(bf16x8 a, bf16x8 b, acc_t c) {
#if HB_MFMA == 16
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
#else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
#endif
}

// s_waitcnt vmcnt(n), the other counters left alone (gfx9 encoding).
#define WAIT_VM(n) __builtin_amdgcn_s_waitcnt((((n) & 15) | (((n) >> 4) << 14) | (7 << 4) | (15 << 8)))
// This wave's LDS reads done, then the workgroup barrier; the "memory"
// clobber keeps the compiler from moving LDS accesses across it.
#define PHASE_END_LDS() asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory")
#define PHASE_END() asm volatile("s_barrier" ::: "memory")

// Four consecutive outputs (columns n..n+3 of one row), as Out says
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

#define HB_EPI_NT 1  // non-temporal output stores
#include "gemm_epi.h"

#define HB_INLINE __attribute__((always_inline))
template <bool B> struct bconst { static constexpr bool value = B; };

extern "C" __global__ __launch_bounds__(NT) void HB_NAME(
    const u32* __restrict__ state, const u16* __restrict__ W, const u16* __restrict__ X,
    void* __restrict__ Yv, const u32* __restrict__ list, const u32* __restrict__ tiles,
    u32 m_launch) {
    (void)list;
    (void)tiles;
    // The stages, X's then W's; after the K loop the epilogue's staging.
    constexpr u32 STG = NS * (XST + WST);
    __shared__ u32x4 lds[STG > EPI_CHUNKS ? STG : EPI_CHUNKS];
    u32x4* const sXa = lds;
    u32x4* const sWa = lds + NS * XST;

    const u32 tid = threadIdx.x, lane = tid & 63u;
    const u32 wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const u32 grp = HB_GRP ? (wave & 1u) : (wave >> 2);
    const u32 wm = wave % WM, wn = wave / WM;

    // The tile (dense rows): XCD-contiguous order, then the m_first walk or
    // bands of row tiles (nax_tile_order).
    u32 g = blockIdx.x;
    if (HB_ORDER == 1) g = xcd_remap(g, gridDim.x);
    // Split K: part = the slow index; g the tile within the part.
    const u32 part = KSP > 1 ? g / (gridDim.x / KSP) : 0;
    if constexpr (KSP > 1) g -= part * (gridDim.x / KSP);
    const u32 m = rows_of_state(state, m_launch);
    const u32 mb = (m + BM - 1) / BM;
    u32 gm, gn;
    if constexpr (HB_BAND > 0) {
        constexpr u32 PER = HB_BAND * NTILES;
        const u32 full = mb / HB_BAND;
        if (g < full * PER) {
            const u32 idx = g % PER;
            gm = (g / PER) * HB_BAND + idx % HB_BAND;
            gn = idx / HB_BAND;
        } else {
            const u32 rem = mb - full * HB_BAND, idx = g - full * PER;
            if (rem == 0) return;
            gm = full * HB_BAND + idx % rem;
            gn = idx / rem;
        }
    } else if (HB_MFIRST) { gm = g % mb; gn = g / mb; }
    else { gn = g % NTILES; gm = g / NTILES; }
    // Uniform over the workgroup: every wave returns here or none does.
    if (gm >= mb || gn >= NTILES) return;
    const u32 row0 = gm * BM;
    const u32 rows = m - row0 < BM ? m - row0 : BM;
    const u32 n0 = gn * BN;

    // This wave's wave-loads of a stage: LDS slot p = q*64 + lane of the
    // operand's stage holds (row p / CH, chunk (p % CH) ^ swizzle(row));
    // the lane loads that chunk.  Byte offsets; rows past m at an offset
    // past the buffer resource's range (0x7fffffff bytes): the load writes
    // zeros to LDS without a memory access.
    u32 xoff[XLMAX], woff[WLMAX];
#pragma unroll
    for (u32 i = 0; i < XLMAX; i++) {
        const u32 p = (wave + NWV * i) * 64 + lane, r = p / CH;
        const u32 cc = (p % CH) ^ ((r >> HB_SWZ) & (CH - 1));
        xoff[i] = r < rows && r < BM ? ((row0 + r) * K + part * (KT * BK) + cc * 8) * 2 : 0x80000000u;
    }
#pragma unroll
    for (u32 i = 0; i < WLMAX; i++) {
        const u32 p = (wave + NWV * i) * 64 + lane, r = p / CH;
        const u32 cc = (p % CH) ^ ((r >> HB_SWZ) & (CH - 1));
        const u32 n = n0 + r;
        woff[i] = ((n < N ? n : N - 1) * K + part * (KT * BK) + cc * 8) * 2;
    }

    const __amdgpu_buffer_rsrc_t rX =
        __builtin_amdgcn_make_buffer_rsrc((void*)X, (short)0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t rW =
        __builtin_amdgcn_make_buffer_rsrc((void*)W, (short)0, 0x7fffffff, 0x00020000);
    typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
    auto lds_addr = [&](u32x4* p) HB_INLINE -> u32 { return (u32)(u64)(lds_u32x4*)p; };
    // This wave's loads of K tile kt into stage st (the branches are
    // wave-uniform and only where a count is not a multiple of NWV).
    auto load_tile = [&](u32 kt, u32 st) HB_INLINE {
        const u32 kb = kt * BK * 2;
#pragma unroll
        for (u32 i = 0; i < XLMAX; i++) {
            if (NXL % NWV && wave + NWV * i >= NXL) continue;
            asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                         :: "s"(lds_addr(&sXa[st * XST + (wave + NWV * i) * 64])), "v"(xoff[i]),
                            "s"(rX), "s"(kb) : "memory");
        }
#pragma unroll
        for (u32 i = 0; i < WLMAX; i++) {
            if (NWL % NWV && wave + NWV * i >= NWL) continue;
            asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                         :: "s"(lds_addr(&sWa[st * WST + (wave + NWV * i) * 64])), "v"(woff[i]),
                            "s"(rW), "s"(kb) : "memory");
        }
    };

    acc_t acc[IN][IM];
#pragma unroll
    for (u32 i = 0; i < IN; i++)
#pragma unroll
        for (u32 j = 0; j < IM; j++) acc[i][j] = acc_t{};

    // Fragment addressing as in gemm_mfma.hip: lane (fr, fc) reads rows
    // base + i*FM + fr at chunk s*(KS/8) + fc, XORed by its own swizzle.
    const u32 fr = lane % FM, fc = lane / FM;
    static_assert(((FM >> HB_SWZ) % CH) == 0 && ((TN >> HB_SWZ) % CH) == 0 &&
                      ((TM >> HB_SWZ) % CH) == 0,
                  "fragment rows keep the lane's swizzle");
    const u32 fsw = (fr >> HB_SWZ) & (CH - 1);
    const u32 wbase = (wn * TN + fr) * CH, xbase = (wm * TM + fr) * CH;
    constexpr u32 NF = PP ? 1 : 2;  // fragment register sets
    bf16x8 a[NF][S][IN], b[NF][S][IM];
    auto read_frags = [&](u32 st, u32 h) HB_INLINE {
        const u32x4* sW = sWa + st * WST;
        const u32x4* sX = sXa + st * XST;
#pragma unroll
        for (u32 s = 0; s < S; s++) {
            const u32 ch = (s * (KS / 8) + fc) ^ fsw;
#pragma unroll
            for (u32 i = 0; i < IN; i++)
                a[h][s][i] = __builtin_bit_cast(bf16x8, sW[wbase + ch + i * FM * CH]);
#pragma unroll
            for (u32 j = 0; j < IM; j++)
                b[h][s][j] = __builtin_bit_cast(bf16x8, sX[xbase + ch + j * FM * CH]);
        }
    };
    auto compute = [&](u32 h) HB_INLINE {
#pragma unroll
        for (u32 s = 0; s < S; s++)
#pragma unroll
            for (u32 i = 0; i < IN; i++)
#pragma unroll
                for (u32 j = 0; j < IM; j++) acc[i][j] = mfma(a[h][s][i], b[h][s][j], acc[i][j]);
    };

    if constexpr (PP) {
    // Prologue: K tiles 0..NS-2 in flight, this wave's share of tile 0
    // landed, then the barrier that publishes tile 0.
#pragma unroll
    for (u32 t = 0; t + 1 < NS; t++)
        if (t < KT) load_tile(t, t);
    if (KT >= NS - 1) WAIT_VM((NS - 2) * LMIN);
    else WAIT_VM(0);
    PHASE_END();
    // Group B starts half a period later: one phase with nothing to do.
    if (grp == 1) PHASE_END();

    // K tile kt in stage st: MEM then COMP, each closed by a barrier.
    auto step = [&](u32 kt, u32 st) HB_INLINE {
        __builtin_amdgcn_sched_barrier(0);
        const bool more = kt + NS - 1 < KT;
        if (more) load_tile(kt + NS - 1, st == 0 ? NS - 1 : st - 1);
        read_frags(st, 0);
        // Own loads of K tile kt + 1 landed: at most the later tiles' loads
        // (LMIN or more each) still in flight.
        if (more) WAIT_VM((NS - 2) * LMIN);
        else WAIT_VM(0);
        PHASE_END_LDS();
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(1);
        compute(0);
        __builtin_amdgcn_s_setprio(0);
        __builtin_amdgcn_sched_barrier(0);
        PHASE_END();
    };
    if constexpr (KT % NS == 0) {
        for (u32 kt0 = 0; kt0 < KT; kt0 += NS) {
#pragma unroll
            for (u32 bi = 0; bi < NS; bi++) step(kt0 + bi, bi);
        }
    } else {
        u32 st = 0;
        for (u32 kt = 0; kt < KT; kt++) {
            step(kt, st);
            st = st + 1 == NS ? 0 : st + 1;
        }
    }
    // Group A meets group B's last barrier: equal barrier counts.
    if (grp == 0) PHASE_END();
    } else {
    // Four waves.  Prologue: every stage's K tile in flight, tile 0 landed
    // and published, its fragments read, tile 1 landed and published (B_0).
#pragma unroll
    for (u32 t = 0; t < NS; t++)
        if (t < KT) load_tile(t, t);
    if (KT >= NS) WAIT_VM((NS - 1) * LMIN);
    else WAIT_VM(0);
    PHASE_END();
    read_frags(0, 0);
    if (KT >= NS) WAIT_VM((NS - 2) * LMIN);
    else WAIT_VM(0);
    PHASE_END_LDS();
    // Step kt (stage st, fragment set h): one LDS read, then a few MFMAs,
    // in turn (scheduling groups), the loads first.  `next`: a K tile
    // follows (its fragments are read during this step).
    auto step = [&](u32 kt, u32 st, u32 h, auto next) HB_INLINE {
        __builtin_amdgcn_sched_barrier(0);
        const bool more = kt + NS < KT;
        if (more) load_tile(kt + NS, st);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (decltype(next)::value) {
            read_frags(st + 1 == NS ? 0 : st + 1, 1 - h);
            compute(h);
            constexpr u32 NR = S * (IN + IM), NM = S * IN * IM, PER = NM / NR ? NM / NR : 1;
#pragma unroll
            for (u32 q = 0; q < NR; q++) {
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
                __builtin_amdgcn_sched_group_barrier(0x008, PER, 0);  // MFMA
            }
        } else {
            compute(h);
        }
        __builtin_amdgcn_sched_barrier(0);
        // Own loads of tile kt + 2 landed: at most NS - 2 later tiles' loads
        // still in flight.
        if (more) WAIT_VM((NS - 2) * LMIN);
        else WAIT_VM(0);
        PHASE_END_LDS();
    };
    // K tiles in pairs (fragment sets 0, 1), the last pair apart: its second
    // step reads no next tile.
    u32 st = 0;
    for (u32 kt = 0; kt + 2 < KT; kt += 2) {
        step(kt, st, 0, bconst<true>{});
        st = st + 1 == NS ? 0 : st + 1;
        step(kt + 1, st, 1, bconst<true>{});
        st = st + 1 == NS ? 0 : st + 1;
    }
    step(KT - 2, st, 0, bconst<true>{});
    st = st + 1 == NS ? 0 : st + 1;
    step(KT - 1, st, 1, bconst<false>{});
    }

    if constexpr (KSP > 1) Yv = (float*)Yv + (u64)part * m_launch * N;  // this part's slab
    if constexpr (EPI_LDS) {
        epilogue_lds(lds, acc, tid, wm, wn, fr, fc, row0, rows, n0, Yv);
        return;
    }
    // Epilogue (F32, or N not a multiple of 8): per MFMA block, runs of 4
    // columns of one row.
#pragma unroll
    for (u32 j = 0; j < IM; j++) {
        const u32 ml = wm * TM + j * FM + fr;
        if (ml >= rows) continue;
        const u32 yrow = row0 + ml;
#pragma unroll
        for (u32 i = 0; i < IN; i++) {
#pragma unroll
            for (u32 q = 0; q < FM * FM / 256; q++) {
                const u32 n = n0 + wn * TN + i * FM + q * 8 + 4 * fc;
                if (n < N) {
                    const acc_t& v = acc[i][j];
                    store4(Yv, (u64)yrow * N + n, v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
                }
            }
        }
    }
}
