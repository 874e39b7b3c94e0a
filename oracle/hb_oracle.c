/*
 * hb_oracle.c -- CPU restatement of herbert-metal-bf16's bf16
 * matrix-multiplication path.  TEST INFRASTRUCTURE ONLY: the checker the
 * parity tests, smoke() and bench.py's cpu_baseline leg compare the HIP
 * library against.  Nothing in the product path links, loads or calls it.
 *
 * Every function cites the reference file:line (under src/ of
 * xigh/herbert-metal-bf16) whose arithmetic it restates.  The reference is
 * Rust emitting Metal Shading Language at load; it cannot be compiled or run
 * here (no cargo, no Metal), so the restatement is pinned by the checks the
 * test suite runs:
 *   - hbo_f32_to_bf16: exhaustively over all 2^32 f32 patterns against the
 *     integer closed form and the branchy form of core/bf16.rs:13-23;
 *   - hbo_gemm / hbo_experts_gemm: f64 brute force at K where every
 *     summation order is exact, identity and permutation W, linearity, and
 *     committed fixtures;
 *   - hbo_rmsnorm_rows: closed forms (constant rows: x' = w exactly; one
 *     nonzero element), its two summation orders against each other, and
 *     an f64 restatement within one bf16 ulp;
 *   - hbo_moe_out: closed forms (zero gate weights: g = bf16(sigmoid(0)) =
 *     0.5; shared = 0: x + experts) and an f64 restatement;
 *   - hbo_route / hbo_moe_sort: brute-force restatements in numpy (argsort
 *     with ties, set invariants, tile cover), and hbo_expf against libm
 *     within 2 ulp over a dense sweep;
 *   - hbo_swiglu: closed forms (g = 0 or u = 0: 0; g >= 20: sigmoid = 1 in
 *     f32, h = bf16(g*u); g <= -104: 0) and one rounding of the f64 value
 *     g*sigmoid(g)*u wherever that value is clear of a rounding boundary;
 *   - hbo_combine: exact-term sums (f64), top_k 1 with weight 1 (identity),
 *     and two hand-worked cases that fix the slot order, the rounding of
 *     each partial sum and the rounding of each product;
 *   - hbo_gather_rows: X rows that carry their own index; the identity list
 *     repeats each row top_k times (np.repeat), top_k = 1 is a row
 *     permutation (np.take), and each token's top_k pairs read its row;
 *   and the swiglu / combine / gather checks are shown to fail on builds of this
 *   file with one deliberate error each (tests/test_oracle_mutants.py).
 *
 * Numerical contract: bf16 operands widened
 * exactly, products exact in f32, sums in f32 in increasing k order, one
 * round-to-nearest-even to bf16 at the output.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off -pthread -shared).
 * -ffp-contract=off keeps every a*b+c of the MoE helpers two roundings, as
 * the HIP kernels (compiled with the same flag) compute them.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define HBO_OUT_BF16 0
#define HBO_OUT_F32 1
#define HBO_OUT_RESIDUAL 2

/* ---- a1: bf16 <-> f32 ------------------------------------------------- */

/* core/bf16.rs:7-9: exact widening, the 16 bits become the high half. */
float hbo_bf16_to_f32(uint16_t h) {
    uint32_t b = (uint32_t)h << 16;
    float f;
    memcpy(&f, &b, 4);
    return f;
}

/* core/bf16.rs:13-23 (and msl/mod.rs:1333-1347): round to nearest even in
 * integers, (bits + 0x7fff + lsb) >> 16; NaN/Inf go through the same
 * expression (a NaN whose low bits carry can overflow into the sign). */
uint16_t hbo_f32_to_bf16(float v) {
    uint32_t b;
    memcpy(&b, &v, 4);
    return (uint16_t)((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}

/* msl/mod.rs:1361 `round_bf16`: the value rounded to bf16, kept as f32. */
float hbo_round_bf16(float v) { return hbo_bf16_to_f32(hbo_f32_to_bf16(v)); }

/* Bulk form for the exhaustive test: n f32 bit patterns starting at `first`. */
void hbo_f32_to_bf16_range(uint32_t first, uint32_t n, uint16_t *out) {
    for (uint32_t i = 0; i < n; i++) {
        uint32_t b = first + i;
        float f;
        memcpy(&f, &b, 4);
        out[i] = hbo_f32_to_bf16(f);
    }
}

/* ---- a2/a3/a7: the GEMM contract --------------------------------------- */

/* One output of the contract: f32 sum of exact products in increasing k,
 * prefill.rs:413 (bf16 x bf16 is exact in f32), kernels.rs:146-220. */
static float dot_f32(const uint16_t *x, const uint16_t *w, int k) {
    float acc = 0.0f;
    for (int i = 0; i < k; i++) acc += hbo_bf16_to_f32(x[i]) * hbo_bf16_to_f32(w[i]);
    return acc;
}

/* kernels.rs:30-43 (`Out`) and 223-236 (`store`), prefill.rs:1200-1230
 * (`emit_out`): Bf16 y = rne(acc); F32 y = acc; Residual y = rne(y + rne(acc)). */
static void store_out(void *y, size_t at, float acc, int out) {
    if (out == HBO_OUT_F32) {
        ((float *)y)[at] = acc;
    } else if (out == HBO_OUT_RESIDUAL) {
        uint16_t *yy = (uint16_t *)y;
        float s = hbo_bf16_to_f32(yy[at]) + hbo_round_bf16(acc);
        yy[at] = hbo_f32_to_bf16(s);
    } else {
        ((uint16_t *)y)[at] = hbo_f32_to_bf16(acc);
    }
}

/* Rows of a GEMM job: output row r reads X row xrow(r), W rows from wbase,
 * writes Y row yrow(r).  Dense: identity maps. */
typedef struct {
    const uint16_t *x, *w;
    void *y;
    int k, n, out;
    const int64_t *xrow, *yrow; /* per job row; NULL = identity */
    const int64_t *wrow0;       /* per job row: first W row (expert offset); NULL = 0 */
    int64_t rows;
    int64_t next;               /* work counter */
    pthread_mutex_t mu;
} gemm_job;

/* Eight outputs of one row at once: eight independent sums, each still
 * in increasing k (the same bits as dot_f32 eight times, faster). */
static void dot8_f32(const uint16_t *x, const uint16_t *w, size_t ws, int k, float *acc) {
    float a[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int i = 0; i < k; i++) {
        float xv = hbo_bf16_to_f32(x[i]);
        for (int j = 0; j < 8; j++) a[j] += xv * hbo_bf16_to_f32(w[j * ws + i]);
    }
    for (int j = 0; j < 8; j++) acc[j] = a[j];
}

static void gemm_row(gemm_job *j, int64_t r) {
    int64_t xr = j->xrow ? j->xrow[r] : r;
    int64_t yr = j->yrow ? j->yrow[r] : r;
    int64_t w0 = j->wrow0 ? j->wrow0[r] : 0;
    const uint16_t *xp = j->x + (size_t)xr * j->k;
    int c = 0;
    for (; c + 8 <= j->n; c += 8) {
        float acc[8];
        dot8_f32(xp, j->w + (size_t)(w0 + c) * j->k, (size_t)j->k, j->k, acc);
        for (int i = 0; i < 8; i++) store_out(j->y, (size_t)yr * j->n + c + i, acc[i], j->out);
    }
    for (; c < j->n; c++) {
        const uint16_t *wp = j->w + (size_t)(w0 + c) * j->k;
        store_out(j->y, (size_t)yr * j->n + c, dot_f32(xp, wp, j->k), j->out);
    }
}

static void *gemm_worker(void *arg) {
    gemm_job *j = (gemm_job *)arg;
    for (;;) {
        pthread_mutex_lock(&j->mu);
        int64_t r = j->next++;
        pthread_mutex_unlock(&j->mu);
        if (r >= j->rows) break;
        gemm_row(j, r);
    }
    return NULL;
}

static void run_job(gemm_job *j, int threads) {
    if (threads <= 1 || j->rows <= 1) {
        for (int64_t r = 0; r < j->rows; r++) gemm_row(j, r);
        return;
    }
    if (threads > 256) threads = 256;
    pthread_t t[256];
    pthread_mutex_init(&j->mu, NULL);
    j->next = 0;
    for (int i = 0; i < threads; i++) pthread_create(&t[i], NULL, gemm_worker, j);
    for (int i = 0; i < threads; i++) pthread_join(t[i], NULL);
    pthread_mutex_destroy(&j->mu);
}

/* prefill.rs:838-1307 (gemm_mma_rows, Dense) and kernels.rs:146-236
 * (matvec): Y[m][n] = X[m][k] . W[n][k]^T as `out` says.  The decode matvec
 * is this with m in {1, 4, 8}.  Rows are split over `threads` host threads;
 * each output is computed alone, so the result does not depend on them. */
void hbo_gemm(const uint16_t *x, const uint16_t *w, void *y, int m, int k, int n, int out,
              int threads) {
    gemm_job j;
    memset(&j, 0, sizeof j);
    j.x = x; j.w = w; j.y = y; j.k = k; j.n = n; j.out = out; j.rows = m;
    run_job(&j, threads);
}

/* prefill.rs:317-338 (MmaRows), 1004-1048 and 1200-1211 (expert rows):
 * the grouped expert GEMM over the tile table of hbo_moe_sort.
 * mode 1 (Gather, the experts' [gate|up]): sorted row p reads X row
 *   list[p] / top_k, W rows e*n.., writes Y[p].
 * mode 2 (Scatter, the experts' down): sorted row p reads X[p], W rows
 *   e*n.., writes Y[list[p]] (the slot row row*top_k + slot).
 * W is [experts*n][k].  Rows no tile covers are not written. */
void hbo_experts_gemm(const uint16_t *x, const uint16_t *w, void *y, const uint32_t *list,
                      const uint32_t *tiles, int k, int n, int mode, int top_k, int out,
                      int threads) {
    uint32_t nt = tiles[0];
    int64_t rows = 0;
    for (uint32_t t = 0; t < nt; t++) rows += tiles[1 + 3 * t + 2];
    int64_t *xr = (int64_t *)malloc(sizeof(int64_t) * (rows ? rows : 1));
    int64_t *yr = (int64_t *)malloc(sizeof(int64_t) * (rows ? rows : 1));
    int64_t *wr = (int64_t *)malloc(sizeof(int64_t) * (rows ? rows : 1));
    int64_t r = 0;
    for (uint32_t t = 0; t < nt; t++) {
        uint32_t e = tiles[1 + 3 * t], start = tiles[2 + 3 * t], cnt = tiles[3 + 3 * t];
        for (uint32_t i = 0; i < cnt; i++, r++) {
            uint32_t p = start + i;
            if (mode == 1) {
                xr[r] = list[p] / (uint32_t)top_k;
                yr[r] = p;
            } else {
                xr[r] = p;
                yr[r] = list[p];
            }
            wr[r] = (int64_t)e * n;
        }
    }
    gemm_job j;
    memset(&j, 0, sizeof j);
    j.x = x; j.w = w; j.y = y; j.k = k; j.n = n; j.out = out; j.rows = rows;
    j.xrow = xr; j.yrow = yr; j.wrow0 = wr;
    run_job(&j, threads);
    free(xr); free(yr); free(wr);
}

/* ---- a8: the route --------------------------------------------------- */

/* exp of f32: Cody-Waite range reduction by ln 2 and the degree-7 minimax
 * polynomial of S. L. Moshier's Cephes `expf` (Cephes Mathematical Library,
 * expf.c), every step an explicit fmaf so that the HIP kernels, which run
 * the same steps, give the same bits.  Within 2 ulp of libm's expf over the
 * range the route and SwiGLU use (checked by the tests). */
float hbo_expf(float x) {
    if (x > 88.72283905206835f) return INFINITY;
    if (x < -103.278929903431851103f) return 0.0f;
    if (x != x) return x;
    float n = floorf(fmaf(x, 1.44269504088896341f, 0.5f));
    float r = fmaf(n, -0.693359375f, x);
    r = fmaf(n, 2.12194440e-4f, r);
    float z = r * r;
    float p = 1.9875691500e-4f;
    p = fmaf(p, r, 1.3981999507e-3f);
    p = fmaf(p, r, 8.3334519073e-3f);
    p = fmaf(p, r, 4.1665795894e-2f);
    p = fmaf(p, r, 1.6666665459e-1f);
    p = fmaf(p, r, 5.0000001201e-1f);
    p = fmaf(p, z, r);
    p = p + 1.0f;
    int e = (int)n;
    /* p * 2^e in two exact power-of-two steps (e in [-150, 128]). */
    int e1 = e / 2, e2 = e - e / 2;
    uint32_t b1 = (uint32_t)(e1 + 127) << 23, b2 = (uint32_t)(e2 + 127) << 23;
    float s1, s2;
    memcpy(&s1, &b1, 4);
    memcpy(&s2, &b2, 4);
    return (p * s1) * s2;
}

/* The sum of 256 per-expert values in the order the route kernel adds them:
 * v[i] += v[i+128], then v[i] += v[i+64], ... down to v[0] += v[1]
 * (a halving tree over the index range).  n a power of two. */
static float tree_sum(float *v, int n) {
    for (int h = n / 2; h >= 1; h /= 2)
        for (int i = 0; i < h; i++) v[i] = v[i] + v[i + h];
    return v[0];
}

/* qwen_kernels.rs:1802-1884 (route_qwen): per row, p = softmax in f32 of the
 * bf16 scores (max, exp(s - max), sum, divide); the top_k best by repeated
 * argmax (`>`: the lowest expert on a tie), removed by setting -1; each
 * divided by their sum (summed from the best down), rounded to bf16, and
 * written in increasing expert order: route[r][s] = expert, route[r][k+s] =
 * the f32 bits of the bf16 weight.  experts a power of two <= 1024. */
void hbo_route(const uint16_t *scores, int rows, int experts, int top_k, uint32_t *route) {
    float p[1024], t[1024];
    for (int r = 0; r < rows; r++) {
        const uint16_t *s = scores + (size_t)r * experts;
        float mx = -INFINITY;
        for (int e = 0; e < experts; e++) {
            float v = hbo_bf16_to_f32(s[e]);
            if (v > mx) mx = v;
        }
        for (int e = 0; e < experts; e++) t[e] = hbo_expf(hbo_bf16_to_f32(s[e]) - mx);
        memcpy(p, t, sizeof(float) * experts);
        float sum = tree_sum(t, experts);
        for (int e = 0; e < experts; e++) p[e] = p[e] / sum;
        int chosen[64];
        float vals[64];
        for (int i = 0; i < top_k; i++) {
            float best = -2.0f;
            int idx = 0;
            for (int e = 0; e < experts; e++)
                if (p[e] > best) { best = p[e]; idx = e; }
            p[idx] = -1.0f;
            chosen[i] = idx;
            vals[i] = best;
        }
        float total = 0.0f;
        for (int i = 0; i < top_k; i++) total = total + vals[i];
        uint32_t *o = route + (size_t)r * 2 * top_k;
        for (int i = 0; i < top_k; i++) {
            float wv = hbo_round_bf16(vals[i] / total);
            int rank = 0;
            for (int j = 0; j < top_k; j++)
                if (j != i && chosen[j] < chosen[i]) rank++;
            uint32_t bits;
            memcpy(&bits, &wv, 4);
            o[rank] = (uint32_t)chosen[i];
            o[top_k + rank] = bits;
        }
    }
}

/* ---- a9: the sort and the tile table ---------------------------------- */

/* prefill.rs:1315-1448 (moe_sort, the scan form) with the table of
 * prefill.rs:1390-1420: list[p] = pair row*top_k + slot, the pairs of an
 * expert together in increasing pair order, experts in increasing order;
 * tiles[0] = the number of tiles, tile t = tiles[1+3t..] = (expert, first
 * sorted row, rows <= bm).  Returns the tile count. */
uint32_t hbo_moe_sort(const uint32_t *route, int rows, int top_k, int experts, int bm,
                      uint32_t *list, uint32_t *tiles) {
    uint32_t pairs = (uint32_t)rows * top_k;
    uint32_t *cnt = (uint32_t *)calloc(experts, sizeof(uint32_t));
    uint32_t *off = (uint32_t *)calloc(experts, sizeof(uint32_t));
    for (uint32_t i = 0; i < pairs; i++) cnt[route[(i / top_k) * 2 * top_k + i % top_k]]++;
    uint32_t total = 0, nt = 0;
    for (int e = 0; e < experts; e++) {
        off[e] = total;
        for (uint32_t j = 0; j < cnt[e]; j += bm) {
            uint32_t left = cnt[e] - j;
            tiles[1 + 3 * nt] = e;
            tiles[2 + 3 * nt] = total + j;
            tiles[3 + 3 * nt] = left < (uint32_t)bm ? left : (uint32_t)bm;
            nt++;
        }
        total += cnt[e];
    }
    tiles[0] = nt;
    for (uint32_t i = 0; i < pairs; i++) {
        uint32_t e = route[(i / top_k) * 2 * top_k + i % top_k];
        list[off[e]++] = i;
    }
    free(cnt);
    free(off);
    return nt;
}

/* prefill.rs:832-835 (moe_tiles): the most tiles a block can need. */
uint32_t hbo_moe_tiles(int rows, int top_k, int experts, int bm) {
    return ((uint32_t)rows * top_k + bm - 1) / bm + experts;
}

/* ---- a10, a12, a13: gather, SwiGLU, combine --------------------------- */

/* prefill.rs:579-610 (moe_gather): XS[p] = X[list[p] / top_k]. */
void hbo_gather_rows(const uint16_t *x, const uint32_t *list, int pairs, int top_k, int hidden,
                     uint16_t *xs) {
    for (int p = 0; p < pairs; p++)
        memcpy(xs + (size_t)p * hidden, x + (size_t)(list[p] / top_k) * hidden, 2 * (size_t)hidden);
}

/* msl/mod.rs:885-890: sigmoid = 1 / (1 + exp(-x)). */
static float sigmoid(float x) { return 1.0f / (1.0f + hbo_expf(-x)); }

/* qwen_kernels.rs:2087-2117 (swiglu_slots) = prefill.rs:2790 (swiglu_rows):
 * over rows of [gate (n) | up (n)], h = rne(g * sigmoid(g) * u). */
void hbo_swiglu(const uint16_t *gu, int slots, int n, uint16_t *h) {
    for (int s = 0; s < slots; s++)
        for (int i = 0; i < n; i++) {
            float g = hbo_bf16_to_f32(gu[(size_t)s * 2 * n + i]);
            float u = hbo_bf16_to_f32(gu[(size_t)s * 2 * n + n + i]);
            float gs = g * sigmoid(g);
            h[(size_t)s * n + i] = hbo_f32_to_bf16(gs * u);
        }
}

/* prefill.rs:746-750, 755-824 (gemm_nax_swiglu): the fused [gate|up] GEMM
 * whose output is SwiGLU of the two bf16-rounded sums: h = rne(rg *
 * sigmoid(rg) * ru), rg = rne(g), ru = rne(u); bit-equal to the GEMM (Out
 * Bf16) then hbo_swiglu.  W is [2*inter][k] = [gate | up]. */
void hbo_gemm_swiglu(const uint16_t *x, const uint16_t *w, uint16_t *h, int m, int k, int inter,
                     int threads) {
    uint16_t *gu = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)m * 2 * inter);
    hbo_gemm(x, w, gu, m, k, 2 * inter, HBO_OUT_BF16, threads);
    hbo_swiglu(gu, m, inter, h);
    free(gu);
}

/* ---- decode fusion XSrc::Norm (kernels.rs:48-103 rmsnorm, 355-440
 * norm_into, 640-975 matvec_split_impl) ----------------------------------
 * Each row of the residual stream x [m][k] normed: ss = sum of x^2, m =
 * ss * f32(1/k) + eps (a multiply, then an add), inv = 1 / sqrt(m), x' =
 * bf16((x * inv) * w') with w' = w (+ 1 for plus_one).  order 0 sums ss as
 * the HIP kernel does (256 threads: thread t's fma chain over t, t+256, ...;
 * the 64 lanes of each wave by the xor butterfly 32, 16, ..., 1; the 4
 * waves' results added in wave order); order 1 sums in increasing index
 * (one fma chain).  The reference's own order is Apple's simd_sum tree
 * inside a threadgroup (parity with its bits unpinned). */
void hbo_rmsnorm_rows(const uint16_t *x, const uint16_t *w, int m, int k, float eps, int plus_one,
                      int order, uint16_t *out) {
    const float inv_d = 1.0f / (float)k;
    for (int j = 0; j < m; j++) {
        const uint16_t *xr = x + (size_t)j * k;
        float ss = 0.0f;
        if (order == 1) {
            for (int i = 0; i < k; i++) {
                float v = hbo_bf16_to_f32(xr[i]);
                ss = fmaf(v, v, ss);
            }
        } else {
            float t[256], wave[4];
            for (int th = 0; th < 256; th++) {
                float a = 0.0f;
                for (int i = th; i < k; i += 256) {
                    float v = hbo_bf16_to_f32(xr[i]);
                    a = fmaf(v, v, a);
                }
                t[th] = a;
            }
            for (int wv = 0; wv < 4; wv++) {
                float l[64];
                memcpy(l, t + 64 * wv, sizeof l);
                for (int sh = 32; sh >= 1; sh >>= 1) {
                    float nl[64];
                    for (int i = 0; i < 64; i++) nl[i] = l[i] + l[i ^ sh];
                    memcpy(l, nl, sizeof l);
                }
                wave[wv] = l[0];
            }
            ss = wave[0];
            for (int wv = 1; wv < 4; wv++) ss = ss + wave[wv];
        }
        float mm = ss * inv_d;
        mm = mm + eps;
        float inv = 1.0f / sqrtf(mm);
        for (int i = 0; i < k; i++) {
            float wf = hbo_bf16_to_f32(w[i]);
            if (plus_one) wf = wf + 1.0f;
            out[(size_t)j * k + i] = hbo_f32_to_bf16((hbo_bf16_to_f32(xr[i]) * inv) * wf);
        }
    }
}

/* qwen_kernels.rs:2163-2214 (moe_out): per row, g = bf16(sigmoid(bf16(gate .
 * xn))), x = bf16(x + bf16(experts + bf16(g * shared))) in place.  order 0
 * sums the dot as the HIP kernel does (256 threads' fma chains over t, t+256,
 * ..., the 64-lane butterfly, the 4 waves in order); order 1 in increasing
 * index.  The reference's own order is Apple's threadgroup reduction (parity
 * with its bits unpinned). */
void hbo_moe_out(const uint16_t *xn, const uint16_t *gate, const uint16_t *ex, const uint16_t *sh,
                 uint16_t *x, int rows, int d, int order) {
    for (int r = 0; r < rows; r++) {
        const uint16_t *xr = xn + (size_t)r * d;
        float dot = 0.0f;
        if (order == 1) {
            for (int i = 0; i < d; i++) dot = fmaf(hbo_bf16_to_f32(xr[i]), hbo_bf16_to_f32(gate[i]), dot);
        } else {
            float t[256], wave[4];
            for (int th = 0; th < 256; th++) {
                float a = 0.0f;
                for (int i = th; i < d; i += 256) a = fmaf(hbo_bf16_to_f32(xr[i]), hbo_bf16_to_f32(gate[i]), a);
                t[th] = a;
            }
            for (int wv = 0; wv < 4; wv++) {
                float l[64];
                memcpy(l, t + 64 * wv, sizeof l);
                for (int s = 32; s >= 1; s >>= 1) {
                    float nl[64];
                    for (int i = 0; i < 64; i++) nl[i] = l[i] + l[i ^ s];
                    memcpy(l, nl, sizeof l);
                }
                wave[wv] = l[0];
            }
            dot = ((wave[0] + wave[1]) + wave[2]) + wave[3];
        }
        float g = hbo_round_bf16(sigmoid(hbo_round_bf16(dot)));
        for (int i = 0; i < d; i++) {
            size_t at = (size_t)r * d + i;
            float s = hbo_round_bf16(g * hbo_bf16_to_f32(sh[at]));
            float o = hbo_round_bf16(hbo_bf16_to_f32(ex[at]) + s);
            x[at] = hbo_f32_to_bf16(hbo_bf16_to_f32(x[at]) + o);
        }
    }
}

/* qwen_kernels.rs:2119-2165 (moe_combine): per token row, acc = 0, then for
 * each slot s in the route's (increasing expert) order
 * acc = rne(acc + rne(y[row][s] * w_s)); out = rne(acc). */
void hbo_combine(const uint16_t *y, const uint32_t *route, int rows, int top_k, int d,
                 uint16_t *out) {
    for (int r = 0; r < rows; r++)
        for (int i = 0; i < d; i++) {
            float acc = 0.0f;
            for (int s = 0; s < top_k; s++) {
                float yf = hbo_bf16_to_f32(y[((size_t)r * top_k + s) * d + i]);
                uint32_t wb = route[(size_t)r * 2 * top_k + top_k + s];
                float wf;
                memcpy(&wf, &wb, 4);
                acc = hbo_round_bf16(acc + hbo_round_bf16(yf * wf));
            }
            out[(size_t)r * d + i] = hbo_f32_to_bf16(acc);
        }
}
