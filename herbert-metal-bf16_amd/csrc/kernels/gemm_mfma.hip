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
//  - HB_DMA 1: the tiles go straight from global memory into LDS (gfx950's
//    buffer_load_dwordx4 ... lds) through HB_STAGES stages: the loads of K tile
//    kt + STAGES - 1 are issued while tile kt is multiplied, so the memory
//    latency is covered by STAGES - 1 tiles of MFMA work; the barrier that
//    publishes tile kt + 1 sits inside the last MFMA step of tile kt, so the
//    first fragments of tile kt + 1 are read while those MFMAs run.
//    HB_DMA 0: staging through registers (global_load, ds_write), one or two
//    stages; the form for tiles whose chunk count is not a multiple of the
//    workgroup's lanes.
//  - Within a stage, the fragments of MFMA step s+1 are read while step s's
//    MFMAs run, interleaved by scheduling groups.
//  - HB_ORDER 1: the workgroup index remapped so each XCD works on a
//    contiguous range of tiles (its own L2 keeps their panels).
//
// Compile-time constants (-D): HB_K, HB_N, HB_OUT (0 bf16, 1 f32, 2
// residual), HB_ROWS (0 dense, 1 gather, 2 scatter, 3 sorted: row p of X
// and of Y, the rows a gather put in sorted order), HB_TOPK, HB_BM, HB_BN,
// HB_BK, HB_WM, HB_WN, HB_MFMA (16|32), HB_STAGES (1..4), HB_SWZ, HB_ORDER,
// HB_MFIRST, HB_DMA, HB_SWIGLU, HB_BAND (the tile order band), HB_KSPLIT.
//
// HB_KSPLIT s > 1 (dense rows, f32 out): K cut into s equal parts; the
// launch holds s workgroups per tile (part = the slow index of the tile
// walk, so each XCD's contiguous range is mostly one part's tiles), and part
// p writes its f32 sums over K tiles p*KT .. p*KT + KT - 1 to slab p of Y,
// [m_launch][N] floats each.  A second kernel (gemm_splitk.hip) adds the
// slabs and applies Out.
//
// HB_SWIGLU 1 (dense or gathered rows, Bf16): the [gate | up] projection and
// the SwiGLU in one (prefill.rs:755-824, gemm_nax_swiglu; for the experts,
// the grouped gate|up and swiglu_slots, qwen_kernels.rs:2087-2117).  N is the
// feature count nf and W holds 2*nf rows per expert (gate rows, then their
// up rows); a tile covers BN/2
// features: each wave's W fragments 0..IN/2-1 are gate rows and fragments
// IN/2.. the up rows of the same features, so a lane holds the gate and the
// up sums of the same outputs and writes h = rne(g * sigmoid(g) * u) with g,
// u the bf16-rounded sums -- the bits of the unfused GEMM (same tile form)
// followed by swiglu_rows, since each sum runs the same MFMA sequence.
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
constexpr u32 CH = BK / 8;                  // 16-byte chunks of a staged row
constexpr u32 KS = FM == 16 ? 32 : 16;      // K of one MFMA
constexpr u32 S = BK / KS;                  // MFMA steps per staged tile
#ifndef HB_KSPLIT
#define HB_KSPLIT 1
#endif
constexpr u32 KSP = HB_KSPLIT;
constexpr u32 KT = K / BK / KSP;            // K tiles of one part
#ifndef HB_SWIGLU
#define HB_SWIGLU 0
#endif
#ifndef HB_BAND
#define HB_BAND 0
#endif

constexpr bool SWI = HB_SWIGLU != 0;
constexpr u32 BF = SWI ? BN / 2 : BN;       // output columns of a tile
constexpr u32 NTILES = (N + BF - 1) / BF;
constexpr u32 XCH = BM * CH, WCH = BN * CH;  // chunks per stage
constexpr u32 X_LD = (XCH + NT - 1) / NT, W_LD = (WCH + NT - 1) / NT;
// Direct-to-LDS staging writes whole wavefronts of chunks: the stage is
// padded to a multiple of the workgroup's lanes (the padding holds copies of
// the tile's last row, never read), so every wave issues the same loads.
constexpr u32 XCHP = HB_DMA ? X_LD * NT : XCH, WCHP = HB_DMA ? W_LD * NT : WCH;
constexpr u32 NS = HB_STAGES;

static_assert(K % (BK * KSP) == 0, "K a multiple of the K step times the parts");
static_assert(KSP == 1 || (ROWS == 0 && OUT == 1 && HB_SWIGLU == 0),
              "split K: dense rows, f32 partial sums");
static_assert(N % 4 == 0, "N a multiple of 4");
static_assert(TM % FM == 0 && TN % FM == 0, "wave tile a multiple of the MFMA block");
static_assert(BK % KS == 0 && (CH & (CH - 1)) == 0, "K step");
static_assert(NT % CH == 0, "threads a multiple of the chunks of a row");
static_assert(NS >= 1 && NS <= 4, "1 to 4 stages");
static_assert(HB_DMA || NS <= 2, "register staging: 1 or 2 stages");
static_assert(!SWI || (IN % 2 == 0 && OUT == 0 && ROWS != 2),
              "fused SwiGLU: dense or gathered rows, bf16 out, an even count of W fragments per wave");

typedef __attribute__((ext_vector_type(FM == 16 ? 4 : 16))) float acc_t;

HB_DEV u32 lpos(u32 r, u32 c) { return r * CH + (c ^ ((r >> HB_SWZ) & (CH - 1))); }

// HB_W_NT 1: W's direct-to-LDS loads non-temporal (W read by one tile).
#if defined(HB_W_NT) && HB_W_NT
#define HB_W_CPOL " nt"
#else
#define HB_W_CPOL ""
#endif

HB_DEV acc_t mfma(bf16x8 a, bf16x8 b, acc_t c) {
#if HB_MFMA == 16
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
#else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
#endif
}

// s_waitcnt with vmcnt(n) and the other counters left alone (gfx9
// encoding: vmcnt[3:0] bits 3:0, vmcnt[5:4] bits 15:14, expcnt 6:4,
// lgkmcnt 11:8).
#define WAIT_VM(n) __builtin_amdgcn_s_waitcnt((((n) & 15) | (((n) >> 4) << 14) | (7 << 4) | (15 << 8)))
// The workgroup barrier of the staged pipeline: this wave's LDS reads done
// and (by a WAIT_VM before it) its tile's direct-to-LDS loads landed, then
// s_barrier.  Not __syncthreads(): its release fence would also wait for
// the later stages' loads still in flight.  The "memory" clobber keeps the
// compiler from moving LDS accesses across it.
#define STAGE_BARRIER() asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory")

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

#include "gemm_epi.h"
// Dense rows through direct-to-LDS stages: the epilogue through LDS.
constexpr bool EPI_VIA_LDS = EPI_LDS && HB_DMA && ROWS == 0 && !SWI;

#define HB_INLINE __attribute__((always_inline))

extern "C" __global__ __launch_bounds__(NT) void HB_NAME(
    const u32* __restrict__ state, const u16* __restrict__ W, const u16* __restrict__ X,
    void* __restrict__ Yv, const u32* __restrict__ list, const u32* __restrict__ tiles,
    u32 m_launch) {
#if HB_DMA
    // The stages, one after another in one LDS array per operand; the stage
    // in use is a scalar index, so any count of K tiles runs one loop body.
    constexpr u32 STG = NS * (XCHP + WCHP), EPC = EPI_VIA_LDS ? EPI_CHUNKS : 0;
    __shared__ u32x4 lds[STG > EPC ? STG : EPC];
    u32x4* const sXa = lds;
    u32x4* const sWa = lds + NS * XCHP;
#else
    // Register staging: the stages as distinct LDS objects, so that the
    // compiler sees that one stage's stores never alias the other's reads.
    __shared__ u32x4 sX0[XCHP], sW0[WCHP];
    __shared__ u32x4 sX1[NS > 1 ? XCHP : 1], sW1[NS > 1 ? WCHP : 1];
#endif

    const u32 tid = threadIdx.x, lane = tid & 63u;
    const u32 wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar
    const u32 wm = wave % WM, wn = wave / WM;
    u32 g = blockIdx.x;
    if constexpr (HB_ORDER == 1 && ROWS != 0) {
        // Experts: only the table's tiles[0] row tiles are real, so the XCD
        // ranges split those (total groups), not the launch: XCD x takes
        // groups x*per .. x*per + per - 1; the rest of its groups return.
        const u32 total = tiles[0] * NTILES, per = (total + 7) / 8;
        const u32 i = g >> 3;
        g = i < per ? (g & 7u) * per + i : 0xffffffffu;
    } else if (HB_ORDER == 1) {
        g = xcd_remap(g, gridDim.x);
    }
    // Split K: part = the slow index; g the tile within the part.
    const u32 part = KSP > 1 ? g / (gridDim.x / KSP) : 0;
    if constexpr (KSP > 1) g -= part * (gridDim.x / KSP);

    // The tile: its first row (dense row or sorted pair), its rows, its
    // column tile and its expert.
    u32 row0, rows, gn, expert = 0;
    if constexpr (ROWS == 0) {
        const u32 m = rows_of_state(state, m_launch);
        const u32 mb = (m + BM - 1) / BM;
        u32 gm;
        if constexpr (HB_BAND > 0) {
            // nax_tile_order (prefill.rs:615-631): bands of HB_BAND row
            // tiles, each walked over every column tile, its row tiles
            // interleaved; the last band holds the rest.
            constexpr u32 PER = HB_BAND * NTILES;
            const u32 full = mb / HB_BAND;
            if (g < full * PER) {
                const u32 idx = g % PER;
                gm = (g / PER) * HB_BAND + idx % HB_BAND;
                gn = idx / HB_BAND;
            } else {
                const u32 rem = mb - full * HB_BAND, idx = g - full * PER;
                if (rem == 0) return;  // groups past m's tiles
                gm = full * HB_BAND + idx % rem;
                gn = idx / rem;
            }
        } else if (HB_MFIRST) { gm = g % mb; gn = g / mb; }
        else { gn = g % NTILES; gm = g / NTILES; }
        if (gm >= mb || gn >= NTILES) return;
        row0 = gm * BM;
        rows = m - row0 < BM ? m - row0 : BM;
    } else {
        // The row-tile count walked: the table's (XCD-balanced order) or the
        // launch's.
        const u32 tmax = HB_ORDER == 1 ? tiles[0] : gridDim.x / NTILES;
        if (g == 0xffffffffu || tmax == 0) return;
        u32 t;
        if (HB_MFIRST) { t = g % tmax; gn = g / tmax; }
        else { gn = g % NTILES; t = g / NTILES; }
        if (t >= tiles[0]) return;
        expert = tiles[1 + 3 * t];
        row0 = tiles[2 + 3 * t];
        rows = tiles[3 + 3 * t];
    }
    const u32 pairs = m_launch * TOPK;  // experts: sorted rows of the block
    const u32 n0 = gn * BF;

    // Global element offsets of this thread's chunks (row clamped to the
    // last valid one), advanced by BK per K tile.  Register staging: chunk
    // id = tid + q*NT is (row id/CH, chunk id%CH), written to its swizzled
    // place.  Direct-to-LDS staging: lane l of a wave writes LDS slot base +
    // l, so slot p = tid + q*NT holds (row p/CH, chunk (p%CH) ^
    // swizzle(row)) and the lane loads that chunk.
    auto x_row = [&](u32 r) HB_INLINE -> u32 {
        if (r >= BM) r = BM - 1;
        u32 rr = r < rows ? r : rows - 1;
        if constexpr (ROWS == 1) {
            u32 pr = list[row0 + rr] / TOPK;
            return pr < m_launch ? pr : m_launch - 1;
        } else if constexpr (ROWS == 2 || ROWS == 3) {
            u32 p = row0 + rr;
            return p < pairs ? p : pairs - 1;
        } else {
            return row0 + rr;
        }
    };
    auto w_row = [&](u32 r) HB_INLINE -> u32 {
        if (r >= BN) r = BN - 1;
        if constexpr (SWI) {
            // Tile row r: wave r / TN, its fragment i; gate rows for i <
            // IN/2, else the up rows of fragment i - IN/2's features.
            const u32 t = r % TN, i = t / FM, up = i >= IN / 2 ? 1u : 0u;
            u32 f = n0 + (r / TN) * (TN / 2) + (i - up * (IN / 2)) * FM + t % FM;
            f = f < N ? f : N - 1;
            return (expert * 2 + up) * N + f;  // an expert's [gate | up] rows
        }
        u32 n = n0 + r;
        return expert * N + (n < N ? n : N - 1);
    };
    u32 xoff[X_LD], woff[W_LD];
#pragma unroll
    for (u32 q = 0; q < X_LD; q++) {
        const u32 p = tid + q * NT, r = p / CH;
        const u32 cc = HB_DMA ? ((p % CH) ^ ((r >> HB_SWZ) & (CH - 1))) : p % CH;
        xoff[q] = x_row(r) * K + part * (KT * BK) + cc * 8;
        // Direct-to-LDS: rows past the tile's (never stored) at a byte
        // offset past the buffer resource's range (0x7fffffff bytes), so
        // the load writes zeros to LDS without a memory access.
        if (HB_DMA && r >= rows) xoff[q] = 0x40000000u;
    }
#pragma unroll
    for (u32 q = 0; q < W_LD; q++) {
        const u32 p = tid + q * NT, r = p / CH;
        const u32 cc = HB_DMA ? ((p % CH) ^ ((r >> HB_SWZ) & (CH - 1))) : p % CH;
        woff[q] = w_row(r) * K + part * (KT * BK) + cc * 8;
    }

    acc_t acc[IN][IM];
#pragma unroll
    for (u32 i = 0; i < IN; i++)
#pragma unroll
        for (u32 j = 0; j < IM; j++) acc[i][j] = acc_t{};

    const u32 fr = lane % FM, fc = lane / FM;
    // Fragment addressing: lane (fr, fc) reads rows base + i*FM + fr at
    // chunk s*(KS/8) + fc of every step s.  The swizzle term of those rows is
    // the lane's own ((fr >> SWZ) & (CH-1)) whatever i and the wave (the row
    // offsets are multiples of CH << SWZ), so each read is a per-lane base
    // plus a per-step chunk plus a constant: few live address registers.
    static_assert(((FM >> HB_SWZ) % CH) == 0 && ((TN >> HB_SWZ) % CH) == 0 &&
                      ((TM >> HB_SWZ) % CH) == 0,
                  "fragment rows keep the lane's swizzle");
    const u32 fsw = (fr >> HB_SWZ) & (CH - 1);
    const u32 wbase = (wn * TN + fr) * CH, xbase = (wm * TM + fr) * CH;
    bf16x8 a[2][IN], b[2][IM];
    auto frag = [&](bf16x8& dst, const u32x4* p) HB_INLINE {
        dst = __builtin_bit_cast(bf16x8, *p);
    };
    // Step s's fragments of a stage into a[h], b[h]: IN of W (A operand), IM
    // of X (B operand).
    auto read_frags = [&](const u32x4* sX, const u32x4* sW, u32 s, u32 h) HB_INLINE {
        const u32 ch = (s * (KS / 8) + fc) ^ fsw;
#pragma unroll
        for (u32 i = 0; i < IN; i++)
            frag(a[h][i], &sW[wbase + ch + i * FM * CH]);
#pragma unroll
        for (u32 j = 0; j < IM; j++)
            frag(b[h][j], &sX[xbase + ch + j * FM * CH]);
    };
    auto mfmas = [&](u32 h) HB_INLINE {
#pragma unroll
        for (u32 i = 0; i < IN; i++)
#pragma unroll
            for (u32 j = 0; j < IM; j++) acc[i][j] = mfma(a[h][i], b[h][j], acc[i][j]);
    };
    // One LDS read, then IN*IM/(IN+IM) MFMAs, in turn.
    auto interleave = [&]() HB_INLINE {
        constexpr u32 NR = IN + IM, NM = IN * IM, PER = NM / NR ? NM / NR : 1;
#pragma unroll
        for (u32 q = 0; q < NR; q++) {
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
            __builtin_amdgcn_sched_group_barrier(0x008, PER, 0);  // MFMA
        }
    };
    // Steps 0..S-2 of a stage whose step-0 fragments are in a[0], b[0].
    auto steps = [&](const u32x4* sX, const u32x4* sW) HB_INLINE {
#pragma unroll
        for (u32 s = 0; s + 1 < S; s++) {
            __builtin_amdgcn_sched_barrier(0);
            read_frags(sX, sW, s + 1, (s + 1) & 1);
            mfmas(s & 1);
            interleave();
        }
        __builtin_amdgcn_sched_barrier(0);
    };

#if HB_DMA
    // Buffer loads straight into LDS: the base in a scalar resource, one
    // 32-bit byte offset per chunk, the K tile's advance as scalar offset,
    // the wave's LDS slot in m0.  Issued as inline asm so that the compiler's
    // wait-count pass, which cannot tell the stages apart, does not wait for
    // every stage in flight before each LDS read; the waits are the
    // pipeline's own (WAIT_VM / STAGE_BARRIER).
    const __amdgpu_buffer_rsrc_t rX =
        __builtin_amdgcn_make_buffer_rsrc((void*)X, (short)0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t rW =
        __builtin_amdgcn_make_buffer_rsrc((void*)W, (short)0, 0x7fffffff, 0x00020000);
    typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
    auto lds_addr = [&](u32x4* p) HB_INLINE -> u32 {
        return (u32)(u64)(lds_u32x4*)p;
    };
    // Load q of K tile kt's stage: q < X_LD an X chunk, else a W chunk.
    auto load_one = [&](u32 kt, u32x4* sX, u32x4* sW, u32 q) HB_INLINE {
        const u32 kb = kt * BK * 2;
        if (q < X_LD)
            asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                         :: "s"(lds_addr(&sX[q * NT + wave * 64])), "v"(xoff[q] * 2), "s"(rX),
                            "s"(kb) : "memory");
        else
            asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen" HB_W_CPOL " lds"
                         :: "s"(lds_addr(&sW[(q - X_LD) * NT + wave * 64])),
                            "v"(woff[q - X_LD] * 2), "s"(rW), "s"(kb) : "memory");
    };
    constexpr u32 LDT = X_LD + W_LD;  // load instructions per tile per lane
    auto load_stage = [&](u32 kt, u32x4* sX, u32x4* sW) HB_INLINE {
#pragma unroll
        for (u32 q = 0; q < LDT; q++) load_one(kt, sX, sW, q);
    };
    auto stx = [&](u32 i) HB_INLINE -> u32x4* { return sXa + i * XCHP; };
    auto stw = [&](u32 i) HB_INLINE -> u32x4* { return sWa + i * WCHP; };
    // Prologue: tiles 0..NS-2 in flight, tile 0 landed and published.
#pragma unroll
    for (u32 t = 0; t + 1 < NS; t++)
        if (t < KT) load_stage(t, stx(t), stw(t));
    if (NS == 1) load_stage(0, stx(0), stw(0));
    if (NS > 2 && KT > NS - 2) WAIT_VM((NS - 2) * LDT);
    else WAIT_VM(0);
    STAGE_BARRIER();
    read_frags(stx(0), stw(0), 0, 0);

    // The stage step of K tile kt, whose stage is `cur` (next: `nxt`, the
    // one to load: `ld`).  Past the last tile the "next" fragments are read
    // from a stale stage and never used.
    auto tile_step = [&](u32 kt, u32 cur, u32 nxt, u32 ld) HB_INLINE {
        if constexpr (NS > 1) {
            // Tile kt + NS - 1 into the stage tile kt - 1 used; every wave
            // passed the barrier after its last read of it.
            const bool more = kt + NS - 1 < KT;
            if (more) load_stage(kt + NS - 1, stx(ld), stw(ld));
            steps(stx(cur), stw(cur));
            // Tile kt + 1 landed (its loads are the oldest in flight),
            // published, and its first fragments read under the last MFMAs
            // of tile kt.
            if (more) WAIT_VM((NS - 2) * LDT);
            else WAIT_VM(0);
            STAGE_BARRIER();
            read_frags(stx(nxt), stw(nxt), 0, S & 1);
            mfmas((S - 1) & 1);
            interleave();
            __builtin_amdgcn_sched_barrier(0);
        } else {
            steps(stx(0), stw(0));
            // One stage: every wave done with it, then the next tile.
            STAGE_BARRIER();
            if (kt + 1 < KT) load_stage(kt + 1, stx(0), stw(0));
            WAIT_VM(0);
            STAGE_BARRIER();
            read_frags(stx(0), stw(0), 0, S & 1);
            mfmas((S - 1) & 1);
        }
        // The next tile's step 0 is in a[S & 1]; steps() expects a[0].
        if constexpr (S & 1) {
#pragma unroll
            for (u32 i = 0; i < IN; i++) a[0][i] = a[1][i];
#pragma unroll
            for (u32 j = 0; j < IM; j++) b[0][j] = b[1][j];
        }
    };
    // One MFMA site per step keeps the accumulators in registers: a K tile
    // count that is a multiple of the stages runs the loop unrolled by NS
    // (every stage at a constant LDS offset), any other one loop body with
    // the stage as a scalar index.
    if constexpr (KT % NS == 0) {
        for (u32 kt0 = 0; kt0 < KT; kt0 += NS) {
#pragma unroll
            for (u32 bi = 0; bi < NS; bi++)
                tile_step(kt0 + bi, bi, (bi + 1) % NS, (bi + NS - 1) % NS);
        }
    } else {
        u32 cur = 0;
        for (u32 kt = 0; kt < KT; kt++) {
            const u32 nxt = cur + 1 == NS ? 0 : cur + 1;
            tile_step(kt, cur, nxt, cur == 0 ? NS - 1 : cur - 1);
            cur = nxt;
        }
    }
#else
    u32x4 rx[X_LD], rw[W_LD];
    auto load = [&](u32 kt) HB_INLINE {
#pragma unroll
        for (u32 q = 0; q < X_LD; q++)
            if (XCH % NT == 0 || tid + q * NT < XCH) rx[q] = *(const u32x4*)(X + xoff[q] + kt * BK);
#pragma unroll
        for (u32 q = 0; q < W_LD; q++)
            if (WCH % NT == 0 || tid + q * NT < WCH) rw[q] = *(const u32x4*)(W + (u64)woff[q] + kt * BK);
    };
    auto stage = [&](u32x4* sX, u32x4* sW) HB_INLINE {
#pragma unroll
        for (u32 q = 0; q < X_LD; q++) {
            u32 id = tid + q * NT;
            if (XCH % NT == 0 || id < XCH) sX[lpos(id / CH, id % CH)] = rx[q];
        }
#pragma unroll
        for (u32 q = 0; q < W_LD; q++) {
            u32 id = tid + q * NT;
            if (WCH % NT == 0 || id < WCH) sW[lpos(id / CH, id % CH)] = rw[q];
        }
    };
    auto tile = [&](u32 kt, u32x4* cx, u32x4* cw, u32x4* nx, u32x4* nw) HB_INLINE {
        if (kt + 1 < KT) load(kt + 1);
        // Keep the next tile's loads ahead of the multiplies (the scheduler
        // would otherwise sink them next to their LDS stores).
        __builtin_amdgcn_sched_barrier(0);
        read_frags(cx, cw, 0, 0);
        steps(cx, cw);
        mfmas((S - 1) & 1);
        if (NS == 1) __syncthreads();
        if (kt + 1 < KT) stage(nx, nw);
        __syncthreads();
    };
    load(0);
    stage(sX0, sW0);
    __syncthreads();
    if constexpr (NS == 2) {
        for (u32 kt = 0; kt < KT; kt += 2) {
            tile(kt, sX0, sW0, sX1, sW1);
            if (kt + 1 < KT) tile(kt + 1, sX1, sW1, sX0, sW0);
        }
    } else {
        for (u32 kt = 0; kt < KT; kt++) tile(kt, sX0, sW0, sX0, sW0);
    }
#endif

    if constexpr (KSP > 1) Yv = (float*)Yv + (u64)part * m_launch * N;  // this part's slab
#if HB_DMA
    if constexpr (EPI_VIA_LDS) {
        epilogue_lds(lds, acc, tid, wm, wn, fr, fc, row0, rows, n0, Yv);
        return;
    }
#endif
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
        if constexpr (SWI) {
#pragma unroll
            for (u32 i = 0; i < IN / 2; i++) {
#pragma unroll
                for (u32 q = 0; q < FM * FM / 256; q++) {
                    const u32 f = n0 + wn * (TN / 2) + i * FM + q * 8 + 4 * fc;
                    if (f < N) {
                        const acc_t& g = acc[i][j];
                        const acc_t& u = acc[i + IN / 2][j];
                        float h[4];
#pragma unroll
                        for (u32 e = 0; e < 4; e++) {
                            const float gr = round_bf16(g[4 * q + e]), ur = round_bf16(u[4 * q + e]);
                            h[e] = (gr * hb_sigmoid(gr)) * ur;
                        }
                        store4(Yv, (u64)yrow * N + f, h[0], h[1], h[2], h[3]);
                    }
                }
            }
            continue;
        }
#pragma unroll
        for (u32 i = 0; i < IN; i++) {
#pragma unroll
            for (u32 q = 0; q < FM * FM / 256; q++) {
                // FM 16: one run, columns 4*fc..+3 of the block; FM 32: four
                // runs, columns q*8 + 4*fc..+3.
                const u32 n = n0 + wn * TN + i * FM + q * 8 + 4 * fc;
                if (n < N) {
                    const acc_t& v = acc[i][j];
                    store4(Yv, (u64)yrow * N + n, v[4 * q], v[4 * q + 1], v[4 * q + 2],
                           v[4 * q + 3]);
                }
            }
        }
    }
}
