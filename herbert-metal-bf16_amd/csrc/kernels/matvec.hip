// matvec.hip -- the decode projection y[m][N] = x[m][K] . W[N][K]^T for the
// few rows m of a decode step (m <= MV_M), bf16 operands, f32 sums, Out's
// epilogue.  HBM-bound: W is streamed once per launch.
//
// Reference: src/metal/kernels.rs:146-220 (matvec: a simdgroup per `rows`
// rows, lanes striding K by 8 bf16, an fma chain per lane, the simdgroup
// sum), :502-519 and :640-975 (matvec_split: `split` simdgroups sharing a
// row's K, partials folded in simdgroup order, persistent groups), :223-236
// (store).  The reference decodes one row; m up to MV_M is this build's
// extension (one W read serves every row).
//
// Four forms (HB_FORM):
//  0 (VALU, the reference's arithmetic layout): a wavefront computes ROWS
//    consecutive rows of W over its K range; lane l takes the 16-byte
//    chunks l, l+64, ... of it, UNROLL chunks per row in flight; then a
//    sum over the 64 lanes (DPP lane moves, wave_sum_rows).
//  2 (dot2): form 0's layout, each pair of products added by one
//    v_dot2_f32_bf16 (bf16 operands straight from the loaded words, f32
//    sum): half the VALU instructions of form 0 and no conversions -- the
//    form for 4-8 rows, where form 0 runs out of VALU issue before HBM.
//  1 (MFMA): a wavefront computes 16 rows of W with
//    v_mfma_f32_16x16x32_bf16, W the A operand (the lane's 16-byte chunks
//    loaded straight from memory as the operand, no conversion), x the B
//    operand (rows past m are zeros).  Lane (r, q) holds row r's elements
//    (u*4 + q)*8 .. +7 of step u of a UNROLL-step block, so one load
//    instruction reads 64 contiguous bytes of each of the 16 rows (whole
//    64-byte segments) and a block 64*UNROLL bytes of each row; x uses the
//    same K mapping.
//    Up to 4 independent accumulators, summed at the end.
//  3 (MFMA, W through LDS): form 1's MFMAs and x, with W loaded in row
//    order (512 B or 1 KB of one row per load instruction, as the VALU
//    forms read it) and turned into the A operand through a wave-private
//    LDS tile: the MFMA's arithmetic with the VALU forms' HBM access; its
//    x (the B operand) from memory, or staged in LDS once per workgroup.
//  4 (MFMA 4x4x4, 16 blocks): a wavefront computes ROWS (4, 8, 16) rows
//    of W, in groups of 4, with
//    v_mfma_f32_4x4x4_16b_bf16, its 16 blocks 16 slices of K: lane
//    (b, j) = 4b + j loads W row j's elements 128c + 8b .. +7 (one load
//    instruction reads 256 contiguous bytes of each of the 4 rows, whole
//    128-byte lines) and holds x row j (and 4 + j) at the same elements, as
//    the MFMA's B and A operands, the low and high 4 elements in two
//    MFMAs: no LDS and no VALU arithmetic in the K loop.  The wave's x
//    stays in registers for its K range; with PERSIST the next row block's
//    W loads are issued before this one's MFMAs.  The 16 blocks' sums are
//    added by DPP within each 16 lanes and two lane swaps across them.
// Both: SPLIT wavefronts of a workgroup share a row block's K (contiguous
// ranges); their partials are added in wave order through LDS.  PERSIST
// > 0: that many workgroups loop over the row blocks.
//
// Decode fusions (VALU forms, src/metal/kernels.rs:236-290, 640-975):
// HB_XSRC 1 (XSrc::Swiglu): x holds [gate (K) | up (K)] per row, x =
// bf16(g*sigmoid(g)*u) computed where it is loaded; HB_XSRC 2 (XSrc::Norm):
// x is the residual stream, its RMSNorm (HB_EPS the epsilon's bits, HB_PLUS1)
// computed into LDS first, the norm weights the 4th binding; HB_OUT 3
// (Out::Swiglu): W holds [gate | up] rows, y = bf16(g*sigmoid(g)*u) of the
// bf16-rounded sums, N/2 wide.
//
// Constants: HB_K, HB_N, HB_OUT, HB_MV_M, HB_FORM, HB_ROWS (form 0),
// HB_SPLIT, HB_PERSIST, HB_UNROLL, HB_XSRC, HB_EPS, HB_PLUS1, HB_XLDS,
// HB_WAVES (wavefronts per workgroup: 4, 8 or 16).  Bindings: W,
// x, y[, norm weights]; then m (<= MV_M).
#include "hb_common.h"

// The MFMA forms: 1 (W loaded as the A operand) and 3 (W through LDS).
#define HB_MMA (HB_FORM == 1 || HB_FORM == 3)

constexpr u32 K = HB_K, N = HB_N, MV = HB_MV_M;
constexpr int OUT = HB_OUT;
constexpr u32 SPLIT = HB_SPLIT, U = HB_UNROLL;
#ifndef HB_WAVES
#define HB_WAVES 4
#endif
constexpr u32 WAVES = HB_WAVES, NT = 64 * WAVES;
static_assert(WAVES == 4 || WAVES == 8 || WAVES == 16, "4, 8 or 16 waves");
constexpr u32 GROUPS_PER_WG = WAVES / SPLIT;  // row blocks per workgroup
#if !HB_MMA && HB_FORM != 4
constexpr u32 RB = HB_ROWS;                   // rows per row block
#elif HB_FORM == 3
constexpr u32 RB = HB_ROWS == 32 ? 32 : 16;   // one or two 16-row MFMA tiles
#elif HB_FORM == 4
constexpr u32 RB = HB_ROWS;                   // 4, 8 or 16: groups of the MFMA's 4 W rows
static_assert(RB == 4 || RB == 8 || RB == 16, "MFMA 4x4x4 form: 4, 8 or 16 rows per wave");
#else
constexpr u32 RB = 16;
#endif
#ifndef HB_XSRC
#define HB_XSRC 0
#endif
#ifndef HB_XLDS
#define HB_XLDS 0
#endif
// x rows in LDS: XSrc::Norm's normed rows, or (HB_XLDS) the plain or
// swiglu'd rows staged once per workgroup.
#define HB_XIN_LDS (HB_XSRC == 2 || HB_XLDS)
#ifndef HB_EPS
#define HB_EPS 0
#endif
#ifndef HB_PLUS1
#define HB_PLUS1 0
#endif
// Out::Swiglu (HB_OUT 3): W's rows are [gate (N/2) | up (N/2)]; a row
// block's RB rows are RB/2 gate rows and the same rows' up rows, and it
// writes RB/2 outputs.
constexpr u32 T = RB / 16;  // MFMA forms: 16-row tiles per wave (2 only in form 3)
constexpr bool SWO = OUT == 3;
constexpr u32 NOUT = SWO ? N / 2 : N;         // output rows
constexpr u32 RO = SWO ? RB / 2 : RB;         // output rows per row block
constexpr u32 NBLK = (NOUT + RO - 1) / RO;
constexpr u32 KS = K / SPLIT;                 // K of one wave's range
static_assert(!SWO || (RB % 2 == 0 && N % 2 == 0 && !HB_MMA), "Out::Swiglu: VALU forms, even rows");
static_assert(HB_XSRC == 0 || !HB_MMA, "XSrc fusions: VALU forms");
static_assert(HB_XSRC != 2 || WAVES == 4, "XSrc::Norm: 4 waves");
static_assert(!HB_XIN_LDS || (HB_FORM != 1 && MV * K * 2 <= (WAVES == 4 ? 65536u : 147456u)),
              "x in LDS: VALU forms and form 3, m*K*2 <= 64 KiB (144 KiB with 8 or 16 waves)");
// x rows in LDS, in 16-byte chunks: form 3 reads the B operand of 16 lanes
// (x rows 0..15) at one K offset, so its rows are one chunk longer (each row
// four banks on from the last: no conflicts); the VALU forms read one row.
constexpr u32 XST = HB_FORM == 3 ? K / 8 + 1 : K / 8;

static_assert(WAVES % SPLIT == 0, "split divides the waves");
static_assert(K % (8 * SPLIT) == 0 && KS % 8 == 0, "K split in whole chunks");
static_assert(!HB_MMA || (MV <= 16 && KS % 32 == 0), "MFMA form: m <= 16, K steps of 32");
static_assert(HB_FORM != 4 || (MV <= 8 && KS % 128 == 0 && HB_XSRC == 0 && !SWO && !HB_XLDS),
              "MFMA 4x4x4 form: m <= 8, K/split a multiple of 128, no fusions, x in registers");

// bf16(g * sigmoid(g) * u) as f32: swiglu's arithmetic (the SwiGLU kernels'
// own expression, kernels.rs:256-261).
HB_DEV float swiglu1(float g, float u) { return round_bf16((g * hb_sigmoid(g)) * u); }

HB_DEV void store_out(void* y, u64 at, float v) {
    if constexpr (OUT == 1) {
        ((float*)y)[at] = v;
    } else if constexpr (OUT == 2) {
        u16* p = (u16*)y + at;
        *p = (u16)f32_to_bf16(bf16_to_f32(*p) + round_bf16(v));
    } else {
        ((u16*)y)[at] = (u16)f32_to_bf16(v);
    }
}

struct HbTrue { static constexpr bool value = true; };
struct HbFalse { static constexpr bool value = false; };
#define HB_INLINE2 __attribute__((always_inline))

HB_DEV float wave_sum(float v) {
    // Butterfly over the 64 lanes (xor 32, 16, ..., 1).
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) v += __shfl_xor(v, s, 64);
    return v;
}

// The 64 lanes' sum of the matvec's row sums without the LDS crossbar:
// pairs (quad_perm 1,0,3,2), quads (2,3,0,1), then the half-row and row
// mirrors (once each 4- and 8-lane group is uniform, the mirrored lane
// holds the other group's value), the 16-lane halves of each 32 by a
// swizzle (xor 16), and the two 32-lane halves read as scalars.  Every
// lane ends with the same value; the association is this tree's.
template <int CTRL>
HB_DEV float dpp_add(float v) {
    return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                                      0xf, 0xf, true));
}
HB_DEV float wave_sum_rows(float v) {
    v = dpp_add<0xB1>(v);   // quad_perm [1,0,3,2]
    v = dpp_add<0x4E>(v);   // quad_perm [2,3,0,1]
    v = dpp_add<0x141>(v);  // row_half_mirror
    v = dpp_add<0x140>(v);  // row_mirror
    v += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0)) +
           __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
}

extern "C" __global__ __launch_bounds__(NT) void HB_NAME(const u16* __restrict__ W,
                                                           const u16* __restrict__ x,
                                                           void* __restrict__ y,
#if HB_XSRC == 2
                                                           const u16* __restrict__ wn,
#endif
                                                           u32 m_launch) {
    __shared__ float part[SPLIT > 1 ? WAVES * RB * 16 : 1];
#if HB_FORM == 3
    static_assert((U == 4 || U == 8 || U == 16) && WAVES * U * T <= 64, "W through LDS: unroll 4, 8 or 16, WAVES*U*T KiB of tile");
    __shared__ u32x4 wtile[WAVES * RB * 4 * U];
#endif
    const u32 tid = threadIdx.x, lane = tid & 63u;
    const u32 wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const u32 gi = wave / SPLIT, sp = wave % SPLIT;  // row block in the group, K part
    const u32 m = m_launch < MV ? m_launch : MV;
#if HB_XIN_LDS
    __shared__ u32x4 xn4[MV * XST];
#endif
#if HB_XSRC == 2
    // XSrc::Norm (kernels.rs:355-440, rmsnorm :48-103): each x row's RMSNorm
    // into LDS as bf16 before the matvec.  ss = sum of x^2: thread t's fma
    // chain over elements t, t+256, ..., the 64 lanes' butterfly, then the 4
    // waves' sums in wave order; m = ss * (1/K) + eps; inv = 1/sqrt(m)
    // (correctly rounded); x' = bf16((x * inv) * w) with w + 1 for plus_one.
    static_assert(K % 256 == 0, "XSrc::Norm: K a multiple of 256");
    __shared__ float nred[WAVES * MV];
    auto prologue = [&]() HB_INLINE2 {
        constexpr u32 PER = K / 256;
#pragma unroll
        for (u32 j = 0; j < MV; j++) {
            const u32 jj = j < m ? j : m - 1;
            float a = 0.0f;
            for (u32 i = 0; i < PER; i++) {
                const float v = bf16_to_f32(x[(u64)jj * K + tid + i * 256]);
                a = __builtin_fmaf(v, v, a);
            }
            a = wave_sum(a);
            if (lane == 0) nred[wave * MV + j] = a;
        }
        __syncthreads();
        const float inv_d = 1.0f / (float)K, eps = __uint_as_float((u32)HB_EPS);
        u16* xn = (u16*)xn4;
#pragma unroll
        for (u32 j = 0; j < MV; j++) {
            const u32 jj = j < m ? j : m - 1;
            float ss = nred[j];
#pragma unroll
            for (u32 w = 1; w < WAVES; w++) ss = ss + nred[w * MV + j];
            const float mm = ss * inv_d + eps;  // -ffp-contract=off: a mul, then an add
            const float inv = __fdiv_rn(1.0f, __fsqrt_rn(mm));
            for (u32 i = 0; i < PER; i++) {
                const u32 c = tid + i * 256;
                float wf = bf16_to_f32(wn[c]);
                if (HB_PLUS1) wf = wf + 1.0f;
                xn[j * K + c] = (u16)f32_to_bf16((bf16_to_f32(x[(u64)jj * K + c]) * inv) * wf);
            }
        }
        __syncthreads();
    };
#endif
    // 8 bf16 of x row jj at element `off` from memory (XSrc: plain, swiglu'd).
    auto xmem = [&](u32 jj, u32 off) HB_INLINE2 -> u32x4 {
#if HB_XSRC == 1
        const u32x4 g = *(const u32x4*)(x + (u64)jj * 2 * K + off);
        const u32x4 u = *(const u32x4*)(x + (u64)jj * 2 * K + K + off);
        u32x4 h;
#pragma unroll
        for (u32 e = 0; e < 4; e++)
            h[e] = pack_bf16x2(swiglu1(bf16_lo(g[e]), bf16_lo(u[e])), swiglu1(bf16_hi(g[e]), bf16_hi(u[e])));
        return h;
#else
        return *(const u32x4*)(x + (u64)jj * K + off);
#endif
    };
#if HB_XLDS && HB_XSRC != 2
    // Every x row's 16-byte chunks into LDS once (rows past m repeat row
    // m-1, as the loads below would).
    auto prologue = [&]() HB_INLINE2 {
        for (u32 c = tid; c < MV * K / 8; c += NT) {
            const u32 j = c / (K / 8), jj = j < m ? j : m - 1;
            xn4[j * XST + c % (K / 8)] = xmem(jj, (c % (K / 8)) * 8);
        }
        __syncthreads();
    };
#endif
    // x in LDS: the prologue fills it once per workgroup.  XSrc::Norm's
    // (two passes over x, a reduction) without persistent workgroups runs
    // after the first W block's loads are issued, whose HBM latency then
    // covers it; otherwise first (measured: hoisting the short staging of
    // plain x, or a prologue a persistent workgroup amortises, lost 1-15%).
    // Form 1 reads x from memory; form 3 from memory, or with HB_XLDS from
    // LDS (the B operand: one x load per workgroup instead of one per row
    // block).
    constexpr bool HOIST = HB_XSRC == 2 && HB_PERSIST == 0;
    bool pending = HB_XIN_LDS && !HB_MMA && HOIST;
    (void)pending;
#if HB_XIN_LDS
    if constexpr (!HOIST) prologue();
#endif
    auto xload = [&](u32 jj, u32 off) HB_INLINE2 -> u32x4 {
#if HB_XIN_LDS
        return xn4[jj * XST + off / 8];
#else
        return xmem(jj, off);
#endif
    };
    const u32 k0 = sp * KS;
    const u32 nwg = (NBLK + GROUPS_PER_WG - 1) / GROUPS_PER_WG;
    const u32 step = HB_PERSIST ? gridDim.x : nwg;

#if HB_FORM == 4
    constexpr u32 MQ = (MV + 3) / 4;  // quads of x rows
    constexpr u32 TG = RB / 4;        // groups of 4 W rows per row block
    constexpr u32 LI = KS / 128;      // load instructions per group
    const u32 jr = lane & 3u, kb = (lane >> 2) * 8;
    // x: lane (b, j) holds x row 4q + j, elements k0 + 128c + 8b .. +7: the
    // A operand of quad q (A row i = lane % 4).  Rows past m read row m-1:
    // they only reach D's rows past m, which are never stored.
    u32x4 xr[MQ][LI];
#pragma unroll
    for (u32 q = 0; q < MQ; q++) {
        const u32 row = 4 * q + jr < m ? 4 * q + jr : m - 1;
        const u16* xp = x + (u64)row * K + k0 + kb;
#pragma unroll
        for (u32 c = 0; c < LI; c++) xr[q][c] = *(const u32x4*)(xp + 128 * c);
    }
    // W rows n0 + 4t + j (rows past N read row N-1; their sums are never
    // stored).
    auto wload = [&](u32x4 (&v)[TG][LI], u32 wg) HB_INLINE2 {
#pragma unroll
        for (u32 t = 0; t < TG; t++) {
            const u32 n = (wg * GROUPS_PER_WG + gi) * RB + 4 * t + jr;
            const u16* wr = W + (u64)(n < N ? n : N - 1) * K + k0 + kb;
#pragma unroll
            for (u32 c = 0; c < LI; c++) v[t][c] = __builtin_nontemporal_load((const u32x4*)(wr + 128 * c));
        }
    };
    typedef __attribute__((ext_vector_type(4))) short s16x4;
    auto lo4 = [](u32x4 v) HB_INLINE2 { return __builtin_bit_cast(s16x4, u32x2{v.x, v.y}); };
    auto hi4 = [](u32x4 v) HB_INLINE2 { return __builtin_bit_cast(s16x4, u32x2{v.z, v.w}); };
    auto block4 = [&](const u32x4 (&v)[TG][LI], u32 wg) HB_INLINE2 {
        const u32 n0 = (wg * GROUPS_PER_WG + gi) * RB;
        // D of block b: lane 4b + j, register i = the sum of x row 4q + i and
        // W row n0 + 4t + j over block b's elements.
        f32x4 acc[TG][MQ][2];
#pragma unroll
        for (u32 t = 0; t < TG; t++)
#pragma unroll
            for (u32 q = 0; q < MQ; q++) acc[t][q][0] = acc[t][q][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (u32 c = 0; c < LI; c++)
#pragma unroll
            for (u32 t = 0; t < TG; t++)
#pragma unroll
                for (u32 q = 0; q < MQ; q++) {
                    acc[t][q][0] =
                        __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(lo4(xr[q][c]), lo4(v[t][c]), acc[t][q][0], 0, 0, 0);
                    acc[t][q][1] =
                        __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(hi4(xr[q][c]), hi4(v[t][c]), acc[t][q][1], 0, 0, 0);
                }
        // The 16 blocks' sum: the 4 of each 16 lanes by DPP (row rotations
        // by 4 and 8), then lane (r, i, j) keeps register i and the 4 rows of
        // 16 lanes are added (xor 16, xor 32).  Lane l < 16 * MQ ends with
        // x row 4 * (l / 16) + (l / 4) % 4, W row n0 + 4t + l % 4.
        const u32 qd = (lane >> 2) & 3u;
        float mine[TG];
#pragma unroll
        for (u32 t = 0; t < TG; t++) {
            mine[t] = 0.0f;
#pragma unroll
            for (u32 q = 0; q < MQ; q++) {
                const f32x4 a = acc[t][q][0] + acc[t][q][1];
                float r = 0.0f;
#pragma unroll
                for (u32 i = 0; i < 4; i++) {
                    float v1 = dpp_add<0x124>(a[i]);  // row_ror:4
                    v1 = dpp_add<0x128>(v1);          // row_ror:8
                    r = qd == i ? v1 : r;
                }
                r += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, r), 0x401F));
                r += __shfl_xor(r, 32, 64);
                if (lane >> 4 == q) mine[t] = r;
            }
        }
        const bool owner = lane < 16 * MQ;
        if constexpr (SPLIT > 1) {
            if (owner)
#pragma unroll
                for (u32 t = 0; t < TG; t++) part[(wave * TG + t) * 32 + lane] = mine[t];
            __syncthreads();
            if (sp == 0 && owner) {
#pragma unroll
                for (u32 t = 0; t < TG; t++) {
                    float s = 0.0f;
#pragma unroll
                    for (u32 q = 0; q < SPLIT; q++) s += part[((gi * SPLIT + q) * TG + t) * 32 + lane];
                    mine[t] = s;
                }
            }
        }
        const u32 mr = 4 * (lane >> 4) + qd;
        if (sp == 0 && owner && mr < m)
#pragma unroll
            for (u32 t = 0; t < TG; t++) {
                const u32 nn = n0 + 4 * t + jr;
                if (nn < N) store_out(y, (u64)mr * N + nn, mine[t]);
            }
        if constexpr (SPLIT > 1) __syncthreads();  // part[] reused by the next block
    };
    u32x4 va[TG][LI];
    u32 wg = blockIdx.x;
    if (wg < nwg) wload(va, wg);
    if constexpr (HB_PERSIST == 0) {
        if (wg < nwg) block4(va, wg);
    } else while (wg < nwg) {
        u32x4 vb[TG][LI];
        const u32 w2 = wg + step;
        if (w2 < nwg) wload(vb, w2);
        block4(va, wg);
        if (w2 >= nwg) break;
        const u32 w3 = w2 + step;
        if (w3 < nwg) wload(va, w3);
        block4(vb, w2);
        wg = w3;
    }
#else
    for (u32 wg = blockIdx.x; wg < nwg; wg += step) {
        const u32 blk = wg * GROUPS_PER_WG + gi;
        const u32 n0 = blk * RO;  // first output row
#if !HB_MMA
        // ---- VALU: ROWS rows, lanes over 16-byte chunks ----
        float acc[RB][MV];
#pragma unroll
        for (u32 r = 0; r < RB; r++)
#pragma unroll
            for (u32 j = 0; j < MV; j++) acc[r][j] = 0.0f;
        const u16* wr[RB];
#pragma unroll
        for (u32 r = 0; r < RB; r++) {
            // Out::Swiglu: rows RO.. are the up rows of rows 0..RO-1.
            const u32 q = SWO && r >= RO ? r - RO : r;
            u32 n = n0 + q;
            n = n < NOUT ? n : NOUT - 1;
            if (SWO && r >= RO) n += NOUT;
            wr[r] = W + (u64)n * K;
        }
        // Blocks of 64*U chunks: lane l takes chunks l, l+64, ..., all U
        // loads of every row issued before the first fma; the last block
        // (K not a multiple of the block) predicated per chunk, its loads
        // still issued together.
        constexpr u32 CHUNKS = KS / 8, BLK = 64 * U;
        constexpr u32 NFULL = CHUNKS / BLK, REM = CHUNKS % BLK;
        auto block = [&](u32 c0, auto full) HB_INLINE2 {
            u32x4 wv[U][RB];
#pragma unroll
            for (u32 u = 0; u < U; u++) {
                if (!decltype(full)::value && u * 64 >= REM) break;  // no lane has this chunk
                const bool on = decltype(full)::value || (u * 64 + 64 <= REM) || (c0 + 64 * u < CHUNKS);
#pragma unroll
                for (u32 r = 0; r < RB; r++)
                    wv[u][r] = on ? __builtin_nontemporal_load((const u32x4*)(wr[r] + k0 + (c0 + 64 * u) * 8))
                                  : u32x4{0u, 0u, 0u, 0u};
            }
#if HB_XIN_LDS
            if (HOIST && pending) {
                prologue();
                pending = false;
            }
#endif
#pragma unroll
            for (u32 u = 0; u < U; u++) {
                if (!decltype(full)::value && u * 64 >= REM) break;  // no lane has this chunk
                const bool on = decltype(full)::value || (u * 64 + 64 <= REM) || (c0 + 64 * u < CHUNKS);
                // Every x row's chunk loaded before the first sum (rows past
                // m read row m-1, their sums never stored): one wait per
                // chunk instead of one per x row.
                u32x4 xs[MV];
#pragma unroll
                for (u32 j = 0; j < MV; j++) {
                    const u32 jj = j < m ? j : m - 1;
                    xs[j] = on ? xload(jj, k0 + (c0 + 64 * u) * 8) : u32x4{0u, 0u, 0u, 0u};
                }
#if HB_FORM == 2
                // Inline asm: the builtin on words extracted from these
                // vectors was miscompiled (every e got e=0's operands) by
                // this image's compiler.  The asm keeps its order, so the
                // word index e is outermost: consecutive dot2s update
                // different sums (each sum still takes e = 0..3 in turn)
                // instead of one dependent chain of four.
                float t[RB][MV];  // the sums as locals (asm operands)
#pragma unroll
                for (u32 r = 0; r < RB; r++)
#pragma unroll
                    for (u32 j = 0; j < MV; j++) t[r][j] = acc[r][j];
#pragma unroll
                for (u32 e = 0; e < 4; e++)
#pragma unroll
                    for (u32 j = 0; j < MV; j++)
#pragma unroll
                        for (u32 r = 0; r < RB; r++)
                            asm volatile("v_dot2c_f32_bf16 %0, %1, %2"
                                         : "+v"(t[r][j])
                                         : "v"(wv[u][r][e]), "v"(xs[j][e]));
#pragma unroll
                for (u32 r = 0; r < RB; r++)
#pragma unroll
                    for (u32 j = 0; j < MV; j++) acc[r][j] = t[r][j];
#else
#pragma unroll
                for (u32 j = 0; j < MV; j++) {
                    const u32x4 xv = xs[j];
#pragma unroll
                    for (u32 r = 0; r < RB; r++) {
                        float a = acc[r][j];
#pragma unroll
                        for (u32 e = 0; e < 4; e++) {
                            a = __builtin_fmaf(bf16_lo(wv[u][r][e]), bf16_lo(xv[e]), a);
                            a = __builtin_fmaf(bf16_hi(wv[u][r][e]), bf16_hi(xv[e]), a);
                        }
                        acc[r][j] = a;
                    }
                }
#endif
            }
        };
        for (u32 bi = 0; bi < NFULL; bi++) block(bi * BLK + lane, HbTrue{});
        if constexpr (REM != 0) block(NFULL * BLK + lane, HbFalse{});
#if HB_FORM == 2
        // The sums' last writers are asm statements, which the compiler's
        // wait-state padding before a DPP read of their results may not
        // count: two wait states here, and every sum passed through an asm
        // after them, so no DPP read is scheduled above the s_nop.
        asm volatile("s_nop 1");
#pragma unroll
        for (u32 r = 0; r < RB; r++)
#pragma unroll
            for (u32 j = 0; j < MV; j++) asm volatile("" : "+v"(acc[r][j]));
#endif
#pragma unroll
        for (u32 r = 0; r < RB; r++)
#pragma unroll
            for (u32 j = 0; j < MV; j++) acc[r][j] = wave_sum_rows(acc[r][j]);
        // Lane r*MV + j owns (row r, x row j).
        float mine = 0.0f;
#pragma unroll
        for (u32 r = 0; r < RB; r++)
#pragma unroll
            for (u32 j = 0; j < MV; j++)
                if (lane == r * MV + j) mine = acc[r][j];
        const u32 own_r = lane / MV, own_j = lane % MV;
        const bool owner = lane < RB * MV;
        // Out::Swiglu: the owner of gate row r also takes up row r + RO.
        float mine_u = 0.0f;
        if constexpr (SWO) {
#pragma unroll
            for (u32 r = 0; r < RO; r++)
#pragma unroll
                for (u32 j = 0; j < MV; j++)
                    if (lane == r * MV + j) mine_u = acc[r + RO][j];
        }
#else
        // ---- MFMA: T tiles of 16 rows x (m <= 16) columns per wave ----
        const u32 fr = lane & 15u, fq = lane >> 4;
        const bool xon = fr < m;
        const u16* xrow = x + (u64)(xon ? fr : 0) * K + k0;
        // The B operand's 8 bf16 of x row fr at element k0 + off (zeros for
        // rows past m): from memory, or (form 3 with x in LDS) from LDS.
        auto xfrag = [&](u32 off) HB_INLINE2 -> u32x4 {
            if (!xon) return u32x4{0u, 0u, 0u, 0u};
#if HB_XIN_LDS
            return xn4[fr * XST + (k0 + off) / 8];
#else
            return *(const u32x4*)(xrow + off);
#endif
        };
        const u16* wrow[T];  // the A operand's row (fr) of each tile
#pragma unroll
        for (u32 t = 0; t < T; t++) {
            const u32 n = n0 + 16 * t + fr;
            wrow[t] = W + (u64)(n < N ? n : N - 1) * K + k0;
        }
        constexpr u32 NA = U < 4 ? U : 4;  // independent accumulators per tile
        f32x4 acc[T][NA];
#pragma unroll
        for (u32 t = 0; t < T; t++)
#pragma unroll
            for (u32 u = 0; u < NA; u++) acc[t][u] = f32x4{0.f, 0.f, 0.f, 0.f};
        constexpr u32 BLOCK = 32 * U;  // K per unrolled block
        u32 kk = 0;
#if HB_FORM == 3
        // W through a wave-private LDS tile: a block's 16*T rows x 32*U K
        // are T*U load instructions of 16-byte chunks in row order
        // (instruction i, lane l: row i*RPI + l/CPR, chunk l%CPR; 256 B,
        // 512 B or 1 KB of one row per 16, 32 or 64 lanes), written to the
        // tile with the chunk index XORed by the row, then read back as the
        // A operands (lane (fr, fq): row 16t + fr, chunk 4u + fq; 16 lanes
        // of one chunk column hit 16 distinct 16-byte bank groups).  Each x
        // fragment serves the T tiles.  The next block's loads are issued
        // before this block's LDS writes and MFMAs.
        constexpr u32 CPR = 4 * U;  // chunks per row per block
        constexpr u32 LI = T * U;   // load instructions per block
        u32x4* tile = wtile + wave * (16 * T * CPR);
        constexpr u32 RPI = 64 / CPR;  // rows per load instruction
        const u32 lr = lane / CPR, lc = lane % CPR;
        // The last workgroup's waves past the last row block have n0 >= N:
        // their base is row N-1 (their sums are never stored).
        const u32 nb0 = n0 < N ? n0 : N - 1;
        const u16* wrow0 = W + (u64)nb0 * K + k0 + lc * 8;
        auto wload = [&](u32x4 (&v)[LI], u32 at) HB_INLINE2 {
#pragma unroll
            for (u32 i = 0; i < LI; i++) {
                const u32 r = i * RPI + lr;
                const u32 rr = nb0 + r < N ? r : N - 1 - nb0;  // rows past N read row N-1
                v[i] = __builtin_nontemporal_load((const u32x4*)(wrow0 + at + rr * K));
            }
        };
        auto wstep = [&](u32x4 (&v)[LI], u32 at) HB_INLINE2 {
#pragma unroll
            for (u32 i = 0; i < LI; i++) {
                const u32 r = i * RPI + lr;
                tile[r * CPR + (lc ^ (r & (CPR - 1)))] = v[i];
            }
            u32x4 xv[U];
#pragma unroll
            for (u32 u = 0; u < U; u++)
                xv[u] = xfrag(at + (u * 4 + fq) * 8);
#pragma unroll
            for (u32 u = 0; u < U; u++)
#pragma unroll
                for (u32 t = 0; t < T; t++) {
                    const u32 r = 16 * t + fr;
                    const u32x4 a = tile[r * CPR + ((u * 4 + fq) ^ (r & (CPR - 1)))];
                    acc[t][u % NA] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        __builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, xv[u]), acc[t][u % NA], 0, 0, 0);
                }
        };
        constexpr u32 NB = KS / BLOCK;  // whole blocks
        if constexpr (NB > 0) {
            u32x4 va[LI], vb[LI];
            wload(va, 0);
            for (u32 b = 0; b < NB; b += 2) {
                if (b + 1 < NB) wload(vb, (b + 1) * BLOCK);
                wstep(va, b * BLOCK);
                if (b + 1 < NB) {
                    if (b + 2 < NB) wload(va, (b + 2) * BLOCK);
                    wstep(vb, (b + 1) * BLOCK);
                }
            }
            kk = NB * BLOCK;
        }
#else
        for (; kk + BLOCK <= KS; kk += BLOCK) {
            u32x4 wv[U], xv[U];
#pragma unroll
            for (u32 u = 0; u < U; u++)
                wv[u] = __builtin_nontemporal_load((const u32x4*)(wrow[0] + kk + (u * 4 + fq) * 8));
#pragma unroll
            for (u32 u = 0; u < U; u++)
                xv[u] = xfrag(kk + (u * 4 + fq) * 8);
#pragma unroll
            for (u32 u = 0; u < U; u++)
                acc[0][u % NA] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, wv[u]),
                                                                         __builtin_bit_cast(bf16x8, xv[u]),
                                                                         acc[0][u % NA], 0, 0, 0);
        }
#endif
        for (; kk < KS; kk += 32) {
            const u32x4 xv = xfrag(kk + fq * 8);
#pragma unroll
            for (u32 t = 0; t < T; t++) {
                const u32x4 wv = *(const u32x4*)(wrow[t] + kk + fq * 8);
                acc[t][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, wv),
                                                                    __builtin_bit_cast(bf16x8, xv), acc[t][0],
                                                                    0, 0, 0);
            }
        }
#pragma unroll
        for (u32 t = 0; t < T; t++)
#pragma unroll
            for (u32 u = 1; u < NA; u++) acc[t][0] += acc[t][u];
        // Lane (fr, fq) holds rows 16t + 4*fq..+3 of the block for x row fr.
#endif

        // ---- fold the SPLIT partials in wave order, then Out ----
#if !HB_MMA
        if constexpr (SPLIT > 1) {
            if (owner) part[(wave * RB + own_r) * 16 + own_j] = mine;
            __syncthreads();
            if (sp == 0 && owner) {
                float s = 0.0f, su = 0.0f;
#pragma unroll
                for (u32 q = 0; q < SPLIT; q++) {
                    s += part[((gi * SPLIT + q) * RB + own_r) * 16 + own_j];
                    if (SWO && own_r < RO) su += part[((gi * SPLIT + q) * RB + own_r + RO) * 16 + own_j];
                }
                mine = s;
                mine_u = su;
            }
        }
        if constexpr (SWO) {
            // swiglu's bits: the gate and up sums as bf16, then bf16(g*sigmoid(g)*u)
            // (kernels.rs:935-945).
            if (sp == 0 && owner && own_r < RO && own_j < m && n0 + own_r < NOUT)
                ((u16*)y)[(u64)own_j * NOUT + n0 + own_r] =
                    (u16)f32_to_bf16(swiglu1(round_bf16(mine), round_bf16(mine_u)));
        } else if (sp == 0 && owner && own_j < m && n0 + own_r < N) {
            store_out(y, (u64)own_j * N + n0 + own_r, mine);
        }
#else
        if constexpr (SPLIT > 1) {
#pragma unroll
            for (u32 t = 0; t < T; t++)
#pragma unroll
                for (u32 i = 0; i < 4; i++) part[(wave * RB + 16 * t + 4 * fq + i) * 16 + fr] = acc[t][0][i];
            __syncthreads();
            if (sp == 0) {
#pragma unroll
                for (u32 t = 0; t < T; t++)
#pragma unroll
                    for (u32 i = 0; i < 4; i++) {
                        float s = 0.0f;
#pragma unroll
                        for (u32 q = 0; q < SPLIT; q++)
                            s += part[((gi * SPLIT + q) * RB + 16 * t + 4 * fq + i) * 16 + fr];
                        acc[t][0][i] = s;
                    }
            }
        }
        if (sp == 0 && fr < m) {
#pragma unroll
            for (u32 t = 0; t < T; t++)
#pragma unroll
                for (u32 i = 0; i < 4; i++) {
                    const u32 nn = n0 + 16 * t + 4 * fq + i;
                    if (nn < N) store_out(y, (u64)fr * N + nn, acc[t][0][i]);
                }
        }
#endif
        if constexpr (SPLIT > 1) __syncthreads();  // part[] reused by the next block
    }
#endif
}
