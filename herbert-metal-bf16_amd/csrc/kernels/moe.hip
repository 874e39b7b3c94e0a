// moe.hip -- the MoE layer's kernels around the grouped expert GEMM: the
// route, the sort of (row, slot) pairs by expert and its tile table, the
// gather of X rows in sorted order, the SwiGLU over [gate | up] rows and the
// weighted combine back to tokens.  HB_OP selects one:
//   1 route   (src/metal/qwen_kernels.rs:1802-1884, route_qwen)
//   2 sort    (src/metal/prefill.rs:1315-1448, moe_sort: pairs of an expert
//             in increasing pair order)
//   3 sort_atomic (src/metal/prefill.rs:1450-1531: any order within an expert)
//   4 gather  (src/metal/prefill.rs:579-610, moe_gather)
//   5 swiglu  (src/metal/qwen_kernels.rs:2087-2117, swiglu_slots)
//   6 combine (src/metal/qwen_kernels.rs:2119-2165, moe_combine)
//   7 moe_out (src/metal/qwen_kernels.rs:2163-2214: the shared expert's
//             gate, the experts' and shared sums, the residual add)
//   8 rmsnorm (src/metal/kernels.rs:48-103: the block's input norm)
// Constants: HB_OP, HB_E (experts), HB_TOPK, HB_BM (rows per expert tile),
// HB_TILES (table capacity), HB_D (row width: hidden, or n of SwiGLU),
// HB_RMAX (sort: rows of the largest block).
#include "hb_common.h"

#ifndef HB_EPS
#define HB_EPS 0
#endif
#ifndef HB_PLUS1
#define HB_PLUS1 0
#endif
constexpr u32 E = HB_E, TOPK = HB_TOPK, D = HB_D;

#if HB_OP == 1
// ---- route: one wavefront per row, E/64 experts per lane ----
// p = softmax in f32 of the bf16 scores: max, e = exp(s - max), the sum in
// the halving-tree order over the expert index (v[i] += v[i + h] for h =
// E/2, ..., 1: first within the lane, then across lanes by xor shuffles,
// whose lane-0 value is that tree), p = e / sum.  Top-k by repeated argmax,
// the lowest expert on a tie; the k weights divided by their sum (added from
// the best down), rounded to bf16, written in increasing expert order:
// route[r][s] = expert, route[r][k + s] = the f32 bits of the bf16 weight.
static_assert(E % 64 == 0 && E <= 1024 && TOPK <= 64, "route: experts a multiple of 64");
constexpr u32 P = E / 64;

// The wave's maximum, and its argmax (the largest value, the lowest index on
// a tie): within each 16 lanes by DPP (quad swaps, then row rotations by 4
// and 8), then the four rows' results read as scalars.  Both are the same for
// any order of combination (a max; a total order on (value, -index)), so
// they equal the xor-butterfly's results without its LDS-crossbar round
// trips, which made the top-k loop a chain of 96 shuffles.
template <int CTRL>
HB_DEV u32 dpp_u32(u32 v) {
    return (u32)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, true);
}
template <int CTRL>
HB_DEV float dpp_f32(float v) {
    return __builtin_bit_cast(float, dpp_u32<CTRL>(__builtin_bit_cast(u32, v)));
}
HB_DEV float lane_f32(float v, u32 l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
HB_DEV float wave_max(float v) {
    float o;
    o = dpp_f32<0xB1>(v);  v = o > v ? o : v;   // quad_perm [1,0,3,2]
    o = dpp_f32<0x4E>(v);  v = o > v ? o : v;   // quad_perm [2,3,0,1]
    o = dpp_f32<0x124>(v); v = o > v ? o : v;   // row_ror:4
    o = dpp_f32<0x128>(v); v = o > v ? o : v;   // row_ror:8
    float m = lane_f32(v, 0);
#pragma unroll
    for (u32 r = 1; r < 4; r++) {
        o = lane_f32(v, 16 * r);
        m = o > m ? o : m;
    }
    return m;
}
HB_DEV void wave_argmax(float& best, u32& idx) {
    auto take = [&](float ob, u32 oi) {
        if (ob > best || (ob == best && oi < idx)) { best = ob; idx = oi; }
    };
    take(dpp_f32<0xB1>(best), dpp_u32<0xB1>(idx));
    take(dpp_f32<0x4E>(best), dpp_u32<0x4E>(idx));
    take(dpp_f32<0x124>(best), dpp_u32<0x124>(idx));
    take(dpp_f32<0x128>(best), dpp_u32<0x128>(idx));
    float b = lane_f32(best, 0);
    u32 i = __builtin_amdgcn_readlane(idx, 0);
#pragma unroll
    for (u32 r = 1; r < 4; r++) {
        const float ob = lane_f32(best, 16 * r);
        const u32 oi = __builtin_amdgcn_readlane(idx, 16 * r);
        if (ob > b || (ob == b && oi < i)) { b = ob; i = oi; }
    }
    best = b;
    idx = i;
}

extern "C" __global__ __launch_bounds__(256) void HB_NAME(const u16* __restrict__ scores,
                                                            u32* __restrict__ route, u32 rows) {
    const u32 lane = threadIdx.x & 63u;
    const u32 r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    const u16* s = scores + (u64)r * E;
    float v[P];
#pragma unroll
    for (u32 p = 0; p < P; p++) v[p] = bf16_to_f32(s[lane + 64 * p]);
    float mx = v[0];
#pragma unroll
    for (u32 p = 1; p < P; p++) mx = v[p] > mx ? v[p] : mx;
    mx = wave_max(mx);
    float e[P], t[P];
#pragma unroll
    for (u32 p = 0; p < P; p++) e[p] = t[p] = hb_expf(v[p] - mx);
#pragma unroll
    for (u32 h = P / 2; h >= 1; h /= 2)
#pragma unroll
        for (u32 p = 0; p < h; p++) t[p] = t[p] + t[p + h];
    float sum = t[0];
#pragma unroll
    for (int sh = 32; sh >= 1; sh >>= 1) sum = sum + __shfl_xor(sum, sh, 64);
    sum = __shfl(sum, 0, 64);  // lane 0 holds the tree's value
    float pr[P];
#pragma unroll
    for (u32 p = 0; p < P; p++) pr[p] = e[p] / sum;

    u32 chosen[TOPK];
    float vals[TOPK];
#pragma unroll
    for (u32 i = 0; i < TOPK; i++) {
        float best = -2.0f;
        u32 idx = 0;
#pragma unroll
        for (u32 p = 0; p < P; p++)
            if (pr[p] > best) { best = pr[p]; idx = lane + 64 * p; }
        wave_argmax(best, idx);
        chosen[i] = idx;
        vals[i] = best;
#pragma unroll
        for (u32 p = 0; p < P; p++)
            if (lane + 64 * p == idx) pr[p] = -1.0f;
    }
    float total = 0.0f;
#pragma unroll
    for (u32 i = 0; i < TOPK; i++) total = total + vals[i];
    if (lane < TOPK) {
        u32 mine = 0;
        float wv = 0.0f;
#pragma unroll
        for (u32 i = 0; i < TOPK; i++)
            if (i == lane) { mine = chosen[i]; wv = vals[i]; }
        u32 rank = 0;
#pragma unroll
        for (u32 j = 0; j < TOPK; j++) rank += chosen[j] < mine ? 1u : 0u;
        const float w = round_bf16(wv / total);
        u32* o = route + (u64)r * 2 * TOPK;
        o[rank] = mine;
        o[TOPK + rank] = __builtin_bit_cast(u32, w);
    }
}

#elif HB_OP == 2 || HB_OP == 3
// ---- sort: one workgroup of 1024 threads (16 wavefronts) ----
// list[p] = pair row*TOPK + slot grouped by expert, experts ascending;
// tiles[0] = tile count, tile t = tiles[1+3t..] = (expert, first sorted
// row, rows <= BM).  Rows = state[3], at most the launch's m.
// A thread's pairs: scan form, wave w's contiguous range [lo, hi) with lane
// l taking lo + l + 64k (the pairs of an expert then land in pair order);
// atomic form, tid + 1024k.  Up to 32 per thread (HB_RMAX * TOPK <= 32768
// pairs) their experts are read once, all loads issued together, and kept
// in registers for both passes; beyond that they are read in each pass.
static_assert(E <= 1024, "sort: at most 1024 experts");
constexpr u32 BM = HB_BM, NW = 16;
// Histograms in use: one per wave (scan form), one shared (atomic form).
constexpr u32 NH = HB_OP == 2 ? NW : 1;
constexpr u32 PMAX = HB_RMAX * TOPK, PER = (PMAX + 1023) / 1024;
constexpr bool HOLD = PER <= 32;
constexpr u32 EPL = (E + 63) / 64;  // experts per lane of the scans

extern "C" __global__ __launch_bounds__(1024) void HB_NAME(const u32* __restrict__ state,
                                                             const u32* __restrict__ route,
                                                             u32* __restrict__ list,
                                                             u32* __restrict__ tiles, u32 m_launch) {
    __shared__ u32 hist[NH][E];  // per wave (or shared) per expert: count, then the cursor
    __shared__ u32 start[E], tstart[E + 1], cnt[E];
    const u32 tid = threadIdx.x, lane = tid & 63u, w = tid >> 6;
    const u32 m = rows_of_state(state, m_launch);
    const u32 pairs = m * TOPK;
    auto expert_of = [&](u32 i) -> u32 {
        u32 x = route[(i / TOPK) * 2 * TOPK + i % TOPK];
        return x < E ? x : E - 1;
    };
#if HB_OP == 2
    const u32 cp = (pairs + NW - 1) / NW;
    const u32 lo = w * cp < pairs ? w * cp : pairs, hi = lo + cp < pairs ? lo + cp : pairs;
    auto pair_k = [&](u32 k) -> u32 { return lo + lane + 64 * k; };
    auto in_k = [&](u32 k) -> bool { return pair_k(k) < hi; };
    u32* const myhist = hist[w];
#else
    auto pair_k = [&](u32 k) -> u32 { return tid + 1024 * k; };
    auto in_k = [&](u32 k) -> bool { return pair_k(k) < pairs; };
    u32* const myhist = hist[0];
#endif
    u32 ex[HOLD ? PER : 1];
    if constexpr (HOLD) {
#pragma unroll
        for (u32 k = 0; k < PER; k++) ex[k] = in_k(k) ? expert_of(pair_k(k)) : E;
    }
    for (u32 i = tid; i < NH * E; i += 1024) (&hist[0][0])[i] = 0;
    __syncthreads();
    if constexpr (HOLD) {
#pragma unroll
        for (u32 k = 0; k < PER; k++)
            if (ex[k] < E) atomicAdd(&myhist[ex[k]], 1u);
    } else {
        for (u32 k = 0; in_k(k); k++) atomicAdd(&myhist[expert_of(pair_k(k))], 1u);
    }
    __syncthreads();
    // Per expert: its count, and each wave's offset inside the expert.
    for (u32 x = tid; x < E; x += 1024) {
        u32 s = 0;
        for (u32 q = 0; q < NH; q++) {
            u32 c = hist[q][x];
            hist[q][x] = s;
            s += c;
        }
        cnt[x] = s;
    }
    __syncthreads();
    // Expert starts and tile starts: exclusive scans in expert order, by
    // wave 0 (lane l sums experts l*EPL .., then a prefix over the lanes).
    if (w == 0) {
        u32 a = 0, t = 0;
#pragma unroll
        for (u32 j = 0; j < EPL; j++) {
            const u32 x = lane * EPL + j;
            if (x < E) {
                a += cnt[x];
                t += (cnt[x] + BM - 1) / BM;
            }
        }
        u32 ia = a, it = t;
#pragma unroll
        for (u32 sh = 1; sh < 64; sh <<= 1) {
            const u32 va = __shfl_up(ia, sh, 64), vt = __shfl_up(it, sh, 64);
            if (lane >= sh) {
                ia += va;
                it += vt;
            }
        }
        u32 ea = ia - a, et = it - t;
#pragma unroll
        for (u32 j = 0; j < EPL; j++) {
            const u32 x = lane * EPL + j;
            if (x < E) {
                start[x] = ea;
                tstart[x] = et;
                ea += cnt[x];
                et += (cnt[x] + BM - 1) / BM;
            }
        }
        if (lane == 63) {
            tstart[E] = it;
            tiles[0] = it;
        }
    }
    __syncthreads();
    for (u32 x = tid; x < E; x += 1024) {
        const u32 c = cnt[x], t0 = tstart[x];
        for (u32 j = 0; j * BM < c; j++) {
            u32* t = tiles + 1 + 3 * (t0 + j);
            t[0] = x;
            t[1] = start[x] + j * BM;
            t[2] = c - j * BM < BM ? c - j * BM : BM;
        }
#pragma unroll 1
        for (u32 q = 0; q < NH; q++) hist[q][x] += start[x];
    }
    __syncthreads();
#if HB_OP == 2
    // Place the wave's pairs chunk by chunk: a lane's rank among the earlier
    // lanes of the same expert (ballots over the expert's bits).
    auto place = [&](u32 k, u32 x) {
        const u32 i = pair_k(k);
        const bool on = i < hi;
        if (!on) x = E;  // matches no real expert
        u64 same = __ballot(on);
#pragma unroll
        for (u32 b = 0; b < 11; b++) {
            const u64 bal = __ballot(((x >> b) & 1u) != 0u);
            same &= ((x >> b) & 1u) ? bal : ~bal;
        }
        const u64 lower = same & ((1ull << lane) - 1ull);
        if (on) {
            const u32 pos = hist[w][x] + (u32)__popcll(lower);
            list[pos] = i;
        }
        // The group's first lane advances the wave's cursor after every
        // lane has read it: only the LDS accesses are ordered (lgkmcnt 0;
        // the list stores are not waited for).
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_wave_barrier();
        if (on && lower == 0) hist[w][x] += (u32)__popcll(same);
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_wave_barrier();
    };
    if constexpr (HOLD) {
#pragma unroll
        for (u32 k = 0; k < PER; k++)
            if (lo + 64 * k < hi) place(k, ex[k]);
    } else {
        for (u32 k = 0; lo + 64 * k < hi; k++) place(k, pair_k(k) < hi ? expert_of(pair_k(k)) : E);
    }
#else
    if constexpr (HOLD) {
#pragma unroll
        for (u32 k = 0; k < PER; k++)
            if (ex[k] < E) list[atomicAdd(&hist[0][ex[k]], 1u)] = pair_k(k);
    } else {
        for (u32 k = 0; in_k(k); k++) {
            const u32 i = pair_k(k);
            list[atomicAdd(&hist[0][expert_of(i)], 1u)] = i;
        }
    }
#endif
}

#elif HB_OP == 4
// ---- gather: XS[p] = X[list[p] / TOPK], 16 bytes per thread ----
static_assert(D % 8 == 0, "gather: hidden a multiple of 8");
constexpr u32 CELLS = D / 8;

extern "C" __global__ __launch_bounds__(256) void HB_NAME(const u32* __restrict__ state,
                                                            const u32* __restrict__ list,
                                                            const u32x4* __restrict__ X,
                                                            u32x4* __restrict__ XS, u32 m_launch) {
    const u32 m = rows_of_state(state, m_launch);
    const u64 total = (u64)m * TOPK * CELLS;
    const u64 i = (u64)blockIdx.x * 256 + threadIdx.x;
    if (i >= total) return;
    const u32 p = (u32)(i / CELLS), c = (u32)(i % CELLS);
    u32 row = list[p] / TOPK;
    row = row < m ? row : m - 1;
    XS[i] = X[(u64)row * CELLS + c];
}

#elif HB_OP == 5
// ---- SwiGLU over rows of [gate (D) | up (D)]: h = rne(g * sigmoid(g) * u) ----
static_assert(D % 8 == 0, "swiglu: n a multiple of 8");
constexpr u32 CELLS = D / 8;

extern "C" __global__ __launch_bounds__(256) void HB_NAME(const u32x4* __restrict__ gu,
                                                            u32x4* __restrict__ h, u32 rows) {
    const u64 i = (u64)blockIdx.x * 256 + threadIdx.x;
    if (i >= (u64)rows * CELLS) return;
    const u32 s = (u32)(i / CELLS), c = (u32)(i % CELLS);
    const u32x4 g = gu[(u64)s * 2 * CELLS + c], u = gu[(u64)s * 2 * CELLS + CELLS + c];
    u32x4 o;
#pragma unroll
    for (u32 e = 0; e < 4; e++) {
        const float g0 = bf16_lo(g[e]), g1 = bf16_hi(g[e]);
        const float u0 = bf16_lo(u[e]), u1 = bf16_hi(u[e]);
        const float h0 = (g0 * hb_sigmoid(g0)) * u0;
        const float h1 = (g1 * hb_sigmoid(g1)) * u1;
        o[e] = pack_bf16x2(h0, h1);
    }
    h[i] = o;
}

#elif HB_OP == 6
// ---- combine: out[r] = the slots added in route order, each rounding as
// index_add_ into a bf16 zero vector: acc = rne(acc + rne(y * w)) ----
static_assert(D % 8 == 0 && TOPK <= 16, "combine: hidden a multiple of 8, top_k <= 16");
constexpr u32 CELLS = D / 8;

extern "C" __global__ __launch_bounds__(256) void HB_NAME(const u32x4* __restrict__ y,
                                                            const u32* __restrict__ route,
                                                            u32x4* __restrict__ out, u32 rows) {
    const u64 i = (u64)blockIdx.x * 256 + threadIdx.x;
    if (i >= (u64)rows * CELLS) return;
    const u32 r = (u32)(i / CELLS), c = (u32)(i % CELLS);
    float acc[8];
#pragma unroll
    for (u32 e = 0; e < 8; e++) acc[e] = 0.0f;
    // Every slot's row chunk and weight loaded before the first sum (one
    // memory latency, not TOPK), then the sums in slot order.
    u32x4 vs[TOPK];
    float ws[TOPK];
#pragma unroll
    for (u32 s = 0; s < TOPK; s++) {
        vs[s] = y[((u64)r * TOPK + s) * CELLS + c];
        ws[s] = __builtin_bit_cast(float, route[(u64)r * 2 * TOPK + TOPK + s]);
    }
#pragma unroll
    for (u32 s = 0; s < TOPK; s++) {
        const u32x4 v = vs[s];
        const float w = ws[s];
#pragma unroll
        for (u32 e = 0; e < 4; e++) {
            acc[2 * e] = round_bf16(acc[2 * e] + round_bf16(bf16_lo(v[e]) * w));
            acc[2 * e + 1] = round_bf16(acc[2 * e + 1] + round_bf16(bf16_hi(v[e]) * w));
        }
    }
    u32x4 o;
#pragma unroll
    for (u32 e = 0; e < 4; e++) o[e] = pack_bf16x2(acc[2 * e], acc[2 * e + 1]);
    out[i] = o;
}

#elif HB_OP == 7
// ---- moe_out (qwen_kernels.rs:2163-2214): the end of the sparse MoE block
// and the residual add, a workgroup per row: g = bf16(sigmoid(bf16(gate .
// xn))), x = bf16(x + bf16(experts + bf16(g * shared))).  The dot: thread
// t's fma chain over elements t, t+256, ..., the 64 lanes' butterfly, the 4
// waves' sums in wave order (the oracle restates this order). ----
static_assert(D % 256 == 0, "moe_out: d a multiple of 256");

extern "C" __global__ __launch_bounds__(256) void HB_NAME(const u16* __restrict__ xn,
                                                            const u16* __restrict__ gate,
                                                            const u16* __restrict__ ex,
                                                            const u16* __restrict__ sh,
                                                            u16* __restrict__ x, u32 rows) {
    __shared__ float red[4];
    const u32 r = blockIdx.x, t = threadIdx.x, lane = t & 63u;
    if (r >= rows) return;
    const u64 base = (u64)r * D;
    float a = 0.0f;
#pragma unroll
    for (u32 i = t; i < D; i += 256) a = __builtin_fmaf(bf16_to_f32(xn[base + i]), bf16_to_f32(gate[i]), a);
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) a += __shfl_xor(a, s, 64);
    if (lane == 0) red[t >> 6] = a;
    __syncthreads();
    const float dot = ((red[0] + red[1]) + red[2]) + red[3];
    const float g = round_bf16(hb_sigmoid(round_bf16(dot)));
#pragma unroll
    for (u32 i = t; i < D; i += 256) {
        const float s = round_bf16(g * bf16_to_f32(sh[base + i]));
        const float o = round_bf16(bf16_to_f32(ex[base + i]) + s);
        x[base + i] = (u16)f32_to_bf16(bf16_to_f32(x[base + i]) + o);
    }
}

#elif HB_OP == 8
// ---- rmsnorm (kernels.rs:48-103), a workgroup per row: ss = sum of x^2
// (thread t's fma chain over t, t+256, ..., the 64-lane butterfly, the 4
// waves in order), m = ss * f32(1/D) + eps, inv = 1/sqrt(m) correctly
// rounded, y = bf16((x * inv) * w) with w + 1 for plus_one -- the same
// arithmetic as the matvec's fused XSrc::Norm. ----
static_assert(D % 256 == 0, "rmsnorm: d a multiple of 256");

extern "C" __global__ __launch_bounds__(256) void HB_NAME(const u16* __restrict__ x,
                                                            const u16* __restrict__ w,
                                                            u16* __restrict__ y, u32 rows) {
    __shared__ float red[4];
    const u32 r = blockIdx.x, t = threadIdx.x, lane = t & 63u;
    if (r >= rows) return;
    const u64 base = (u64)r * D;
    float a = 0.0f;
#pragma unroll
    for (u32 i = t; i < D; i += 256) {
        const float v = bf16_to_f32(x[base + i]);
        a = __builtin_fmaf(v, v, a);
    }
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) a += __shfl_xor(a, s, 64);
    if (lane == 0) red[t >> 6] = a;
    __syncthreads();
    const float ss = ((red[0] + red[1]) + red[2]) + red[3];
    const float inv_d = 1.0f / (float)D, eps = __uint_as_float((u32)HB_EPS);
    const float inv = __fdiv_rn(1.0f, __fsqrt_rn(ss * inv_d + eps));
#pragma unroll
    for (u32 i = t; i < D; i += 256) {
        float wf = bf16_to_f32(w[i]);
        if (HB_PLUS1) wf = wf + 1.0f;
        y[base + i] = (u16)f32_to_bf16((bf16_to_f32(x[base + i]) * inv) * wf);
    }
}
#endif
