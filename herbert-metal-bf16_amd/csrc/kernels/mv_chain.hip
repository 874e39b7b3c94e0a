// mv_chain.hip -- a decode step's projections in one launch: NPH matvec
// phases y_p[m][N_p] = x_p[m][K_p] . W_p[N_p][K_p]^T (bf16 operands, f32
// sums, Out's epilogue), each phase starting only after every output of the
// one before it is written, as consecutive kernels in stream order would.
//
// What it replaces: the reference records a decode step as one command
// buffer of matvec dispatches (QwenEngine::step, src/metal/qwen.rs:3177;
// each dispatch src/metal/kernels.rs:146-236, 502-519); on this GPU every
// kernel boundary costs a drain, a dispatch and a fresh HBM ramp, while the
// projections' W streams are independent of the data that orders them.
// Here one persistent workgroup per CU (a cooperative launch: every
// workgroup resident) runs the phases in turn; between two phases each
// workgroup, once its outputs are written, issues the loads of its first W
// block of the next phase and only then waits for the others (a counter per
// phase), so that W is already on its way when the phase's x is ready.
//
// Per phase (shapes constants: HB_PH_K, HB_PH_N, HB_PH_OUT lists): x's m
// rows are staged in LDS (m*K*2 bytes); each wavefront takes blocks of RB
// consecutive W rows (RB = as many rows as fit CPL 16-byte chunks per lane,
// at most 4), lanes striding K by 16-byte chunks (a load instruction reads 1
// KiB of one row), the products added by v_dot2_f32_bf16, then the sum over
// the 64 lanes (DPP); blocks go round the grid's wavefronts.  Out: 0 Bf16,
// 1 F32, 2 Residual (y = bf16(y + bf16(acc))).
//
// Ordering between phases (device scope, across the XCDs' L2s): outputs are
// written with agent-scope stores (write-through, visible device-wide once
// complete); a workgroup waits for its stores (s_waitcnt vmcnt(0)), then
// adds 1 to the phase's counter (agent-scope atomic); a waiting workgroup
// polls the counter with agent-scope loads until it reaches the grid size
// (bounded: after ~2^20 polls it records an error word and goes on, so the
// launch always ends), then an agent-scope acquire fence (invalidating the
// CU's and the XCD's non-coherent cached lines) before it reads x.  The
// last workgroup to finish the last phase sets every counter back to 0 for
// the next launch.
//
// Constants: HB_MV_M (rows, <= 8), HB_NPH, HB_PH_K / HB_PH_N / HB_PH_OUT
// (comma lists, K a multiple of 512), HB_CPL (the largest K/512), HB_WAVES.
// Bindings: table (per phase: W, x, y device addresses), sync (NPH + 1
// words: the phase counters, the last one the done counter; then the error
// word); then m.
#include "hb_common.h"

constexpr u32 MV = HB_MV_M, NPH = HB_NPH, CPLMAX = HB_CPL;
#ifndef HB_WAVES
#define HB_WAVES 8
#endif
constexpr u32 WAVES = HB_WAVES, NT = 64 * WAVES;
constexpr u32 PK[NPH] = {HB_PH_K};
constexpr u32 PN[NPH] = {HB_PH_N};
constexpr u32 PO[NPH] = {HB_PH_OUT};
static_assert(MV >= 1 && MV <= 8, "1 to 8 rows");

constexpr u32 kmax() {
    u32 k = 0;
    for (u32 p = 0; p < NPH; p++) k = PK[p] > k ? PK[p] : k;
    return k;
}
constexpr u32 KMAX = kmax();
static_assert(KMAX / 512 == CPLMAX, "HB_CPL = the largest K / 512");
static_assert(MV * KMAX * 2 <= 160 * 1024 - 256, "x rows in LDS");
constexpr u32 cpl_of(u32 p) { return PK[p] / 512; }
constexpr u32 rb_of(u32 p) {
    const u32 r = CPLMAX / cpl_of(p);
    return r < 1 ? 1 : (r > 4 ? 4 : r);
}
constexpr u32 nb_of(u32 p) { return (PN[p] + rb_of(p) - 1) / rb_of(p); }
constexpr bool shapes_ok() {
    for (u32 p = 0; p < NPH; p++)
        if (PK[p] % 512 != 0 || PK[p] == 0 || PN[p] == 0 || PO[p] > 2) return false;
    return true;
}
static_assert(shapes_ok(), "K a multiple of 512, Out 0..2");

struct Phase {
    const u16* w;
    const u16* x;
    void* y;
};

#define HB_INLINE2 __attribute__((always_inline))

template <int CTRL>
HB_DEV float dpp_add(float v) {
    return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                                      0xf, 0xf, true));
}
// The 64 lanes' sum (every lane ends with it): quad swaps, the half-row and
// row mirrors, a 16-lane swizzle, the two 32-lane halves as scalars.
HB_DEV float wave_sum_rows(float v) {
    v = dpp_add<0xB1>(v);
    v = dpp_add<0x4E>(v);
    v = dpp_add<0x141>(v);
    v = dpp_add<0x140>(v);
    v += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0)) +
           __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
}

struct Ctx {
    const Phase* tab;
    u32* sync;
    u32 m, lane, wave, tid, gw, gwaves, groups;
    u32x4* xs;  // LDS: x rows of the current phase
};

// The W rows of block b of phase P into w: w[r * CPL + i] = row n0 + r's
// chunk lane + 64 i (rows past N read row N-1; their sums are not stored).
template <u32 P>
HB_DEV void wload(const Ctx& c, u32x4 (&w)[CPLMAX], u32 b) {
    constexpr u32 K = PK[P], N = PN[P], CPL = cpl_of(P), RB = rb_of(P);
    const u16* W = c.tab[P].w;
#pragma unroll
    for (u32 r = 0; r < RB; r++) {
        u32 n = b * RB + r;
        n = n < N ? n : N - 1;
        const u16* row = W + (u64)n * K + c.lane * 8;
#pragma unroll
        for (u32 i = 0; i < CPL; i++) w[r * CPL + i] = __builtin_nontemporal_load((const u32x4*)(row + i * 512));
    }
}

// Waits until every workgroup has added itself to counter q (bounded).
HB_DEV void wait_for(const Ctx& c, u32 q) {
    if (c.tid == 0) {
        u32 polls = 0;
        while (__hip_atomic_load(&c.sync[q], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < c.groups) {
            if (++polls > (1u << 20)) {
                __hip_atomic_store(&c.sync[NPH], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
    }
    __syncthreads();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
}

// This workgroup's outputs of the phase are written: counter q += 1.
HB_DEV void arrive(const Ctx& c, u32 q) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (c.tid == 0) __hip_atomic_fetch_add(&c.sync[q], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <u32 P>
HB_DEV void phase(const Ctx& c, u32x4 (&w)[CPLMAX]) {
    constexpr u32 K = PK[P], N = PN[P], OUT = PO[P], CPL = cpl_of(P), RB = rb_of(P), NB = nb_of(P);
    constexpr u32 KC = K / 8;  // 16-byte chunks of a row
    // x rows into LDS (rows past m repeat row m-1).
    {
        const u16* x = c.tab[P].x;
        for (u32 q = c.tid; q < MV * KC; q += NT) {
            const u32 j = q / KC, jj = j < c.m ? j : c.m - 1;
            c.xs[q] = *(const u32x4*)(x + (u64)jj * K + (q % KC) * 8);
        }
    }
    __syncthreads();
    void* y = c.tab[P].y;
    for (u32 b = c.gw; b < NB; b += c.gwaves) {
        if (b != c.gw) wload<P>(c, w, b);  // the first block was loaded ahead
        float acc[RB][MV];
#pragma unroll
        for (u32 r = 0; r < RB; r++)
#pragma unroll
            for (u32 j = 0; j < MV; j++) acc[r][j] = 0.0f;
#pragma unroll
        for (u32 i = 0; i < CPL; i++) {
            u32x4 xv[MV];
#pragma unroll
            for (u32 j = 0; j < MV; j++) xv[j] = c.xs[j * KC + c.lane + 64 * i];
            // Word e outermost: consecutive dot2s update different sums.
#pragma unroll
            for (u32 e = 0; e < 4; e++)
#pragma unroll
                for (u32 j = 0; j < MV; j++)
#pragma unroll
                    for (u32 r = 0; r < RB; r++)
                        asm volatile("v_dot2c_f32_bf16 %0, %1, %2"
                                     : "+v"(acc[r][j])
                                     : "v"(w[r * CPL + i][e]), "v"(xv[j][e]));
        }
        // The sums' last writers are asm: two wait states before a DPP read,
        // and every sum through an asm after them.
        asm volatile("s_nop 1");
#pragma unroll
        for (u32 r = 0; r < RB; r++)
#pragma unroll
            for (u32 j = 0; j < MV; j++) asm volatile("" : "+v"(acc[r][j]));
        float mine = 0.0f;
#pragma unroll
        for (u32 r = 0; r < RB; r++)
#pragma unroll
            for (u32 j = 0; j < MV; j++) {
                const float s = wave_sum_rows(acc[r][j]);
                if (c.lane == r * MV + j) mine = s;
            }
        const u32 r = c.lane / MV, j = c.lane % MV, n = b * RB + r;
        if (c.lane < RB * MV && n < N && j < c.m) {
            const u64 at = (u64)j * N + n;
            if constexpr (OUT == 1) {
                __hip_atomic_store((float*)y + at, mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            } else if constexpr (OUT == 2) {
                u16* p = (u16*)y + at;
                const u16 v = (u16)f32_to_bf16(bf16_to_f32(*p) + round_bf16(mine));
                __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            } else {
                __hip_atomic_store((u16*)y + at, (u16)f32_to_bf16(mine), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
    if constexpr (P + 1 < NPH) {
        arrive(c, P);
        // The next phase's first block on its way before the wait.
        if (c.gw < nb_of(P + 1)) wload<P + 1>(c, w, c.gw);
        wait_for(c, P);
    }
}

template <u32 P>
HB_DEV void phases_from(const Ctx& c, u32x4 (&w)[CPLMAX]) {
    phase<P>(c, w);
    if constexpr (P + 1 < NPH) phases_from<P + 1>(c, w);
}

extern "C" __global__ __launch_bounds__(NT) void HB_NAME(const Phase* __restrict__ tab, u32* __restrict__ sync,
                                                           u32 m_launch) {
    __shared__ u32x4 xs[MV * KMAX / 8];
    Ctx c;
    c.tab = tab;
    c.sync = sync;
    c.m = m_launch < MV ? (m_launch ? m_launch : 1) : MV;
    c.tid = threadIdx.x;
    c.lane = c.tid & 63u;
    c.wave = __builtin_amdgcn_readfirstlane(c.tid >> 6);
    c.groups = gridDim.x;
    c.gwaves = gridDim.x * WAVES;
    c.gw = blockIdx.x * WAVES + c.wave;
    c.xs = xs;
    u32x4 w[CPLMAX];
    if (c.gw < nb_of(0)) wload<0>(c, w, c.gw);
    phases_from<0>(c, w);
    // Done: the last workgroup out resets the counters for the next launch.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (c.tid == 0) {
        const u32 before = __hip_atomic_fetch_add(&sync[NPH - 1], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (before == c.groups - 1)
            for (u32 q = 0; q < NPH; q++) __hip_atomic_store(&sync[q], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}
