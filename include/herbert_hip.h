/*
 * herbert_hip.h -- C ABI of the MI355X (gfx950) bf16 matrix-multiplication
 * path of herbert-metal-bf16: the prefill block GEMM, the decode matvec and
 * the MoE expert grouped GEMM with its route, sort, gather, SwiGLU and
 * combine.  Plain pointers, sizes and integer status codes; no C++ or torch
 * types cross it.  One context per device; a context is used by one host
 * thread at a time (the reference's `Gpu` is not Send either), and work is
 * ordered on the context's one HIP stream.
 *
 * Every entry point cites the reference interface it replaces, as
 * path:line under src/ of xigh/herbert-metal-bf16.
 */
#ifndef HERBERT_HIP_H
#define HERBERT_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes (the reference's HerbertError, core/error.rs:9-27) ---- */
#define HB_OK 0
#define HB_ERR_INVALID (-1)     /* bad argument: HerbertError::Config-like     */
#define HB_ERR_HIP (-2)         /* HIP runtime failure: HerbertError::Backend  */
#define HB_ERR_COMPILE (-3)     /* hiprtc failure: pipeline "not built"        */
#define HB_ERR_UNSUPPORTED (-4) /* descriptor the kernels do not implement     */
#define HB_ERR_NO_DEVICE (-5)   /* no HIP device                               */

/* The message of the last failing call on this thread
 * (HerbertError::Backend(String), core/error.rs:9-27). */
const char *hb_last_error(void);

/* ---- context: Gpu::open / summary / drop (metal/gpu.rs:22-124) ---- */
typedef struct hb_gpu hb_gpu;

/* Gpu::open (metal/gpu.rs:70): the HIP device `device`, its stream, its
 * kernel cache. */
int hb_open(int device, hb_gpu **gpu);
/* Drop of Gpu: every buffer and module of the context freed. */
void hb_close(hb_gpu *gpu);
/* Gpu::summary (metal/gpu.rs:108): "name, CUs, memory, arch". */
const char *hb_device_summary(hb_gpu *gpu);

/* ---- memory: Gpu::alloc / alloc_with, Buffer, Range (metal/gpu.rs:59-67,
 * 150-157).  The context owns every buffer until hb_free or hb_close. ---- */
typedef uint32_t hb_buf;

typedef struct hb_range { /* Range {buf, offset, size} (metal/gpu.rs:40-57) */
    hb_buf buf;
    uint32_t reserved;
    uint64_t offset; /* bytes */
    uint64_t size;   /* bytes; 0 = to the end of the buffer */
} hb_range;

int hb_alloc(hb_gpu *gpu, uint64_t bytes, hb_buf *out);
int hb_free(hb_gpu *gpu, hb_buf buf);
int hb_upload(hb_gpu *gpu, hb_buf buf, uint64_t offset, const void *src, uint64_t bytes);
int hb_download(hb_gpu *gpu, hb_buf buf, uint64_t offset, void *dst, uint64_t bytes);
/* Zero `bytes` at `offset` with a fill kernel on the context's stream. */
int hb_zero(hb_gpu *gpu, hb_buf buf, uint64_t offset, uint64_t bytes);
/* Device-to-device copy of `src` into `dst` (equal sizes, no overlap) on the
 * context's stream, by HIP's copy kernel.  No counterpart in the reference,
 * whose buffers are shared with the CPU; for callers that stage device
 * buffers, and the plain copy that calibrates the traffic counters. */
int hb_copy(hb_gpu *gpu, hb_range dst, hb_range src);
/* Device address of a buffer (for callers that bring their own kernels). */
int hb_buffer_ptr(hb_gpu *gpu, hb_buf buf, void **ptr);

/* ---- kernel descriptors: the emitter functions of the reference
 * (prefill.rs, kernels.rs, qwen_kernels.rs) as one shape-keyed struct ---- */
enum hb_kind {
    HB_KIND_GEMM = 0,        /* gemm_mma_rows / gemm_mma_form (prefill.rs:418-431, 838-1307) */
    HB_KIND_GEMM_SIMT = 1,   /* gemm_simt (prefill.rs:121-307) */
    HB_KIND_GEMM_DIRECT = 2, /* gemm_mm2d / gemm_mm2d_rows (prefill.rs:442-569) */
    HB_KIND_GEMM_SWIGLU = 3, /* gemm_nax_swiglu (prefill.rs:755-824) */
    HB_KIND_MATVEC = 4,      /* matvec / matvec_split (kernels.rs:146-220, 502-519, 640-975) */
    HB_KIND_ROUTE = 5,       /* route_qwen (qwen_kernels.rs:1802-1884) */
    HB_KIND_SORT = 6,        /* moe_sort (prefill.rs:1315-1448) */
    HB_KIND_SORT_ATOMIC = 7, /* moe_sort_atomic (prefill.rs:1450-1531) */
    HB_KIND_GATHER = 8,      /* moe_gather (prefill.rs:579-610) */
    HB_KIND_SWIGLU = 9,      /* swiglu_slots / swiglu_rows (qwen_kernels.rs:2087-2117) */
    HB_KIND_COMBINE = 10,    /* moe_combine (qwen_kernels.rs:2119-2165) */
    HB_KIND_ROUND_PROBE = 11, /* herbert-metal-probe round (bin/herbert-metal-probe.rs:7-11) */
    HB_KIND_MOE_OUT = 12,    /* moe_out (qwen_kernels.rs:2163-2214): the MoE block's end */
    HB_KIND_RMSNORM = 13     /* rmsnorm (kernels.rs:48-103): the block's input norm, rows of n */
};

enum hb_out { /* Out (kernels.rs:30-43) */
    HB_OUT_BF16 = 0,
    HB_OUT_F32 = 1,
    HB_OUT_RESIDUAL = 2,
    /* matvec only: W holds [gate (n/2 rows) | up (n/2 rows)] and y[j] =
     * bf16(g*sigmoid(g)*u) of the bf16-rounded gate and up sums, n/2 wide
     * (Out::Swiglu, kernels.rs:655-660, 935-945) */
    HB_OUT_SWIGLU = 3
};

enum hb_xsrc { /* XSrc (kernels.rs:236-256): what a matvec's x binding holds */
    HB_XSRC_PLAIN = 0,  /* x [m][k] */
    HB_XSRC_SWIGLU = 1, /* [gate (k) | up (k)] per row: x = bf16(g*sigmoid(g)*u) on load */
    HB_XSRC_NORM = 2    /* the residual stream [m][k]: x = its RMSNorm (eps, plus_one, the
                         * norm weights [k] at binding 3), computed into LDS first */
};

enum hb_rows { /* MmaRows (prefill.rs:317-338) */
    HB_ROWS_DENSE = 0,
    HB_ROWS_GATHER = 1,
    HB_ROWS_SCATTER = 2,
    /* sorted row p reads X[p] and writes Y[p] with its tile's expert: the
     * [gate|up] GEMM after moe_gather (the gather+mm2d candidate of
     * expert_pipes, qwen.rs:2358) */
    HB_ROWS_SORTED = 3
};

typedef struct hb_desc {
    uint32_t kind;    /* enum hb_kind */
    uint32_t k, n;    /* K and N (per expert for the grouped GEMM); route: experts in n */
    uint32_t out;     /* enum hb_out */
    uint32_t rows_of; /* enum hb_rows (GEMM kinds) */
    uint32_t m_first; /* tile_of (prefill.rs:31-43): walk row tiles first */
    /* GEMM tile: bm rows of X x bn rows of W per workgroup, K by bk,
     * wm x wn wavefronts, MFMA block 16 or 32, dbuf = LDS stages - 1 (0..3),
     * LDS swizzle (0 = conflict-free for the K step, s + 1 = shift s), tile
     * order (0 plain, 1 XCD-contiguous). 0 = the kind's default. */
    uint32_t bm, bn, bk, wm, wn, mfma, dbuf, swz, order;
    /* matvec: rows of x (1..16); waves sharing a row block's K (split: 1,
     * 2, 4; 8 and 16 with at least as many mv_waves); persistent workgroups
     * (0 = one per row block); W rows per wave (VALU forms 1..8; form 3: 16
     * or 32); form: 0 VALU lanes-stride-K, 1 MFMA, 2 the VALU layout with
     * v_dot2_f32_bf16 (two products added per instruction, no conversion),
     * 3 MFMA with W loaded in row order and turned into the A operand
     * through a per-wave LDS tile (unroll 4, 8 or 16; rows 32: two 16-row
     * MFMA tiles sharing each x fragment), 4 v_mfma_f32_4x4x4_16b_bf16 with
     * 4 W rows per wave, its 16 blocks slices of K, W loaded straight into
     * the operand (m <= 8, K/split a multiple of 128, no fusions). */
    uint32_t mv_m, split, persist, rows, form;
    /* MoE: slots per row (top_k), experts, the tile table's capacity
     * (moe_tiles, prefill.rs:832-835), rows of the largest block. */
    uint32_t top_k, experts, tiles, rows_max;
    /* GEMM staging: 0 through registers (global_load + ds_write), 1 straight
     * into LDS (gfx950 global_load_lds_dwordx4). */
    uint32_t lds_dma;
    /* matvec: 16-byte chunks (VALU form) or 32-K MFMA steps (MFMA form)
     * each lane keeps in flight per row (1..8; MFMA form 1..16); 0 = 4. */
    uint32_t unroll;
    /* GEMM tile order band (nax_tile_order, prefill.rs:615-631): 0 the
     * m_first walk; b > 0: consecutive workgroups walk every column tile of
     * b row tiles, those row tiles interleaved (the last band holds what is
     * left).  Dense rows only. */
    uint32_t band;
    /* matvec: enum hb_xsrc; XSrc::Norm's epsilon (the f32's bits) and
     * plus_one (weights used as w + 1). */
    uint32_t xsrc, eps_bits, plus_one;
    /* matvec (VALU forms): 1 = the x rows (plain, or XSrc::Swiglu's h) are
     * staged once per workgroup into LDS (m*k*2 <= 64 KiB; 144 KiB with
     * 8 or 16 mv_waves) and every row
     * block reads them from there; XSrc::Norm always does. */
    uint32_t x_lds;
    /* MFMA GEMM, direct-to-LDS: 1 = W's loads marked non-temporal (nt), for
     * W read by one tile only (the experts' weights): measured +6-8% on the
     * grouped GEMMs, slower where tiles share W through L2. */
    uint32_t w_nt;
    /* matvec (plain x or XSrc::Swiglu): wavefronts per workgroup, 0 or 4
     * (256 threads), 8 or 16.  With x_lds, 8 and 16 waves stage up to
     * 144 KiB of x (one workgroup per CU, x staged once per CU), against
     * 64 KiB for 4. */
    uint32_t mv_waves;
    /* MFMA GEMM (dense rows, direct-to-LDS): the K loop's schedule.  0: every
     * wave loads and multiplies in lock step (wm x wn waves); 1: eight waves
     * in two groups of four, one of each on every SIMD, taking turns between
     * a memory phase and an MFMA phase (a "ping-pong"; wm * wn = 8, 3 or 4
     * stages); 2: as 1 with the groups formed by even and odd waves; 3: four
     * waves (wm * wn = 4), one per SIMD, each reading its next K tile's
     * fragments from LDS between its MFMAs (3 or 4 stages, an even count of
     * K tiles). */
    uint32_t sched;
    /* MFMA GEMM (dense rows, direct-to-LDS, any sched), 0 or 1 = no split:
     * K cut into `ksplit` equal parts, one workgroup per (tile, part) writing
     * its f32 sums to a workspace the context owns, then a second kernel
     * adding the parts in order 0..ksplit-1 and applying Out -- for shapes
     * whose tiles fill less than a round of the CUs.  Each part must hold a
     * whole number of K tiles (sched 3: an even number), and N must be a
     * multiple of 4 (the second kernel's vector width).  One launch handle:
     * hb_launch / hb_time run both kernels.  The workspace grows on the
     * first launch over more rows than any before it on the context: that
     * launch synchronizes the stream and calls hipFree / hipMalloc (not
     * allowed under stream capture), so launch a split kernel once at its
     * largest rows before capturing it. */
    uint32_t ksplit;
} hb_desc;

/* Gpu::pipeline(&Emitted) (metal/gpu.rs:127-148) for the kernel the
 * descriptor names: HIP C++ compiled by hiprtc for gfx950 with the shape as
 * constants, cached by name in the context (QwenEngine::get, qwen.rs:1156-1166)
 * and on disk by source hash.  *kernel is the pipeline's index. */
int hb_kernel_build(hb_gpu *gpu, const hb_desc *desc, int32_t *kernel);
/* No counterpart in the reference (Metal compiles its MSL at load and keeps
 * its own pipeline cache): the kernel `desc` names compiled for gfx950 into
 * the disk cache, with no GPU and no context -- build.py warms the cache for
 * the kernels a manifest lists, so a fresh box does not spend minutes in
 * hiprtc at load.  HB_OK, or the error that building it gives. */
int hb_kernel_precompile(const hb_desc *desc);
/* Emitted::name: the descriptor in the reference's naming
 * (gemm_mma_{K}x{N}_{bf16|f32|res}..., prefill.rs:1295-1300). */
const char *hb_kernel_name(hb_gpu *gpu, int32_t kernel);
/* The xxx_groups grid functions (gemm_mma_groups prefill.rs:406,
 * gemm_mma_expert_groups :826, matvec_groups kernels.rs:1456, ...): the
 * workgroups of a launch over `m` rows. */
uint32_t hb_kernel_groups(hb_gpu *gpu, int32_t kernel, uint32_t m);
/* Bindings the kernel takes, in order (Emitted::bindings). */
uint32_t hb_kernel_bindings(hb_gpu *gpu, int32_t kernel);
/* The kernel's descriptor kind (enum hb_kind; 0 for no such kernel): the
 * Rust side keeps its pipelines' kinds itself; here it tells a caller of
 * hb_engine_experts whether the gate|up kernel writes the SwiGLU. */
uint32_t hb_kernel_kind(hb_gpu *gpu, int32_t kernel);
/* Seconds spent compiling so far ([metal] line, qwen.rs:1069). */
double hb_compile_seconds(hb_gpu *gpu);

/* Gpu::dispatch (metal/gpu.rs:166-201) of one kernel over `m` rows on the
 * context's stream: the bindings' sizes are checked against the descriptor
 * and m before anything runs.  Bindings per kind:
 *   GEMM, GEMM_DIRECT, GEMM_SIMT, GEMM_SWIGLU: state, W, X, Y[, list, tiles]
 *   MATVEC: W, x, y[, norm weights (XSrc::Norm)]          ROUTE: scores, route
 *   SORT, SORT_ATOMIC: state, route, list, tiles
 *   GATHER: state, list, X, XS        SWIGLU: gate_up, h
 *   COMBINE: y, route, out    ROUND_PROBE: state (state[0] = chunk), out_int, out_hw
 *   MOE_OUT: xn, shared_gate, experts, shared, x (x updated in place)
 *   RMSNORM: x, w, y (eps_bits, plus_one of the descriptor)
 * `m` is the rows of the block (the kernels read state[3], never beyond m).
 * A split-K GEMM (ksplit > 1) launched over more rows than any earlier
 * split launch on this context first grows the context's workspace: the
 * stream is synchronized and the workspace reallocated. */
int hb_launch(hb_gpu *gpu, int32_t kernel, const hb_range *bindings, uint32_t nbind, uint32_t m);

typedef struct hb_op { /* Op {pipe, ranges, groups} (qwen.rs:650-655) */
    int32_t kernel;
    uint32_t m;
    uint32_t nbind;
    uint32_t reserved;
    hb_range bind[8];
} hb_op;

/* time_ops (qwen.rs:2593): `reps` runs of `ops` in order on the stream,
 * timed by two HIP events on that stream; *seconds = the GPU time of all. */
int hb_time(hb_gpu *gpu, const hb_op *ops, uint32_t nops, uint32_t reps, double *seconds);
/* hb_time with an event recorded after every launch on the same stream:
 * op_seconds[i] = the mean duration of op i over the reps (the
 * time_ops-per-pipe breakdown of the reference's --profile, qwen.rs:2593),
 * *seconds the whole run. */
int hb_time_each(hb_gpu *gpu, const hb_op *ops, uint32_t nops, uint32_t reps, double *seconds,
                 double *op_seconds);

/* A recorded op sequence: the reference encodes a decode step's ops into one
 * command buffer and submits it (QwenEngine::step, qwen.rs:3177); here the
 * ops are captured from the context's stream into a HIP graph (kernel nodes
 * only, no memset nodes) and instantiated once, checked as hb_time checks
 * them.  The bindings are fixed at record time (the buffers' contents may
 * change between replays).  While a graph lives, the context's split-K
 * workspace cannot grow (a launch that would need it to returns
 * HB_ERR_INVALID). */
typedef struct hb_graph hb_graph;
int hb_graph_record(hb_gpu *gpu, const hb_op *ops, uint32_t nops, hb_graph **graph);
/* `reps` replays on the context's stream (asynchronous, as hb_launch). */
int hb_graph_launch(hb_graph *graph, uint32_t reps);
/* GPU seconds of `reps` replays, events at the ends only. */
int hb_graph_time(hb_graph *graph, uint32_t reps, double *seconds);
void hb_graph_free(hb_graph *graph);
/* submit_wait (metal/gpu.rs:209-221): wait for the stream. */
int hb_sync(hb_gpu *gpu);

/* ---- synthetic inputs (host side, no GPU) ---- */
/* n bf16 values ~ N(0, std^2): splitmix64(seed) -> two uniforms -> Box-Muller
 * in double -> f32 -> round to nearest even; element i is a function of
 * (seed, i) only, so any thread count gives the same bits. */
void hb_fill_normal_bf16(uint64_t seed, float std, uint16_t *out, uint64_t n, int threads);

/* ---- the selection layer: QwenEngine's kernel choice (qwen.rs) ---- */
typedef struct hb_engine hb_engine;

/* Tune::default + Tune::apply (qwen.rs:62-389) on `tune` ("key=value,..."),
 * over the context `gpu`.  HB_ERR_INVALID with the reference's message on a
 * bad key or value.  `gpu` may be null: a host-only engine (the --tune
 * table, the log, hb_engine_autotune_chunk over the host's callbacks) whose
 * kernel selections (gemm, gate_up, matvec, experts) return HB_ERR_INVALID. */
int hb_engine_open(hb_gpu *gpu, const char *tune, hb_engine **engine);
void hb_engine_close(hb_engine *engine);
/* Tune::summary (qwen.rs:391-398) of the settings this path reads. */
const char *hb_engine_tune_summary(hb_engine *engine);
/* The prefill buckets (qwen.rs:1051-1063): 64*2^i below prefill.block, then
 * prefill.block; *count of them written to out (capacity cap). */
int hb_engine_buckets(hb_engine *engine, uint32_t *out, uint32_t cap, uint32_t *count);

/* QwenEngine::gemm (qwen.rs:2200-2325): the kernel of Y[m][n] = X[m][k].W^T
 * written as `out`: the one gemm.mma/gemm.tn/gemm.mform name, or with
 * gemm.auto every candidate checked against the first (check_candidates,
 * qwen.rs:2497-2545: max|err| <= max|ref|/64 at m and m - m/3 - 3 rows) and
 * the fastest eligible kept (pick_flagged, qwen.rs:2547-2575), cached under
 * "{k}x{n} {Out}, {m} rows".  W, X, Y and the 16-byte state are the buffers
 * timed on (state[3] and Y restored afterwards).  Logs [autotune] lines. */
int hb_engine_gemm(hb_engine *engine, uint32_t k, uint32_t n, uint32_t out, hb_range state,
                   hb_range w, hb_range x, hb_range y, uint32_t m, int32_t *kernel);

/* The descriptors QwenEngine::gemm (qwen.rs:2200-2325) times for a k x n
 * GEMM written as `out`, in candidate order (the first is the production
 * kernel the others are checked against); *count = how many, the first
 * min(count, cap) written.  Lets a caller check or build every kernel the
 * timed choice can pick. */
int hb_engine_gemm_candidates(hb_engine *engine, uint32_t k, uint32_t n, uint32_t out,
                              hb_desc *descs, uint32_t cap, uint32_t *count);

/* QwenEngine::gate_up_pipes (qwen.rs:2148-2193): the prefill's [gate | up]
 * GEMM (K = h, N = 2*inter, Bf16 into `gu`) and its SwiGLU into `hout`
 * ([m][inter]).  pf.fswi 0: apart; 1: the first fused form
 * (gemm_nax_swiglu, prefill.rs:755-824); 2 (default, with gemm.auto): the
 * GEMM's pick + swiglu_rows timed against the fused forms after
 * check_candidates, the fastest kept under "{h}x{2 inter}, {m} rows".
 * *gemm_kernel: the GEMM (bindings state, W, X, gu) or the fused kernel
 * (state, W, X, hout); *swiglu_kernel: the SwiGLU (bindings gu, hout) or
 * -1 when fused. */
int hb_engine_gate_up(hb_engine *engine, uint32_t h, uint32_t inter, hb_range state, hb_range w,
                      hb_range x, hb_range gu, hb_range hout, uint32_t m, int32_t *gemm_kernel,
                      int32_t *swiglu_kernel);

/* QwenEngine::mv_full (qwen.rs:1311-1511) for M rows of x: with mv.auto the
 * forms timed over every matrix of the shape (`ws`, mv.cold) and the fastest
 * kept under "{k}x{n} {Out}"; else the form mv.split/mv.persist name. */
int hb_engine_matvec(hb_engine *engine, uint32_t k, uint32_t n, uint32_t out, uint32_t mv_m,
                     const hb_range *ws, uint32_t nws, hb_range x, hb_range y, int32_t *kernel);
/* mv_full with its decode fusions (qwen.rs:1311-1336: `out`, `xsrc`,
 * `norm_w`): out may be HB_OUT_SWIGLU (W the [gate | up] rows, n their
 * count), xsrc an enum hb_xsrc, with XSrc::Norm's epsilon bits, plus_one
 * and its weights `norm_w` (bound 4th); the VALU forms only.  The pick is
 * kept under "{k}x{n}{xsrc} {Out} m{mv_m}". */
int hb_engine_matvec_fused(hb_engine *engine, uint32_t k, uint32_t n, uint32_t out, uint32_t xsrc,
                           uint32_t eps_bits, uint32_t plus_one, uint32_t mv_m, const hb_range *ws,
                           uint32_t nws, hb_range x, hb_range y, hb_range norm_w, int32_t *kernel);
/* The descriptors mv_full (qwen.rs:1311-1511) times for a k x n matvec of
 * mv_m rows written as `out`, with XSrc `xsrc` (eps_bits, plus_one for
 * XSrc::Norm), in candidate order; *count = how many, the first
 * min(count, cap) written.  The timed choice checks no candidate, so a
 * caller can check every kernel it can pick. */
int hb_engine_matvec_candidates(hb_engine *engine, uint32_t k, uint32_t n, uint32_t out,
                                uint32_t xsrc, uint32_t eps_bits, uint32_t plus_one, uint32_t mv_m,
                                hb_desc *descs, uint32_t cap, uint32_t *count);

/* QwenEngine::expert_pipes (qwen.rs:2326-2391): the sort, the grouped
 * gate_up GEMM (Gather) and down GEMM (Scatter) of an MoE layer of `experts`
 * experts, top_k slots, hidden `hidden`, expert intermediate `inter`, for
 * blocks of m rows: with gemm.auto, tiles of 16, 32, 64 and 128 rows
 * (moe.tile only, if given) each timed, the tile whose kernels sum the least
 * kept.  The route buffer must hold a real route of m rows when this runs
 * (the reference times these only after a first prefill, real_route,
 * qwen.rs:2340): the tiles and the expert weights read follow from it.
 * Buffers: state, route [m][2*top_k], list, tiles, X [m][hidden], the
 * experts' gate_up W [experts*2*inter][hidden], EGU [m*top_k][2*inter],
 * EHB [m*top_k][inter], down W [experts*hidden][inter], EY
 * [m*top_k][hidden], XS [m*top_k][hidden] (the gather's output).
 * kernels[0..3] = sort, gate_up GEMM, down GEMM, gather (-1: gate_up reads
 * X through the list itself); *bm = rows per tile.  A gate_up kernel of kind
 * HB_KIND_GEMM_SWIGLU has swiglu_slots fused: it writes EHB (bind EHB as
 * its Y) and no SwiGLU pass runs; else it writes EGU and swiglu_slots
 * (HB_KIND_SWIGLU, EGU -> EHB over m*top_k rows) follows. */
typedef struct hb_moe_io {
    hb_range state, route, list, tiles, x, w_gate_up, egu, ehb, w_down, ey, xs;
} hb_moe_io;
int hb_engine_experts(hb_engine *engine, uint32_t experts, uint32_t top_k, uint32_t hidden,
                      uint32_t inter, uint32_t m, const hb_moe_io *io, int32_t kernels[4],
                      uint32_t *bm);

/* The routed experts of one MoE layer over m rows, as QwenEngine encodes
 * them per block (qwen.rs:2705-2735): moe_sort -> [moe_gather] -> grouped
 * gate|up -> [swiglu_slots] -> grouped down (scatter to slot rows) ->
 * moe_combine, on the stream, nothing allocated.  kernels: hb_engine_experts'
 * four (sort, gate_up, down, gather or -1); swiglu: the swiglu_slots kernel
 * (HB_KIND_SWIGLU, n = inter; ignored when the gate|up kernel is of kind
 * HB_KIND_GEMM_SWIGLU); combine: moe_combine (n = hidden).  io as for
 * hb_engine_experts (state[3] = m; route holds the m rows' route; xs is
 * read only with a gather, egu only without the fused SwiGLU); out
 * [m][hidden] bf16.  Every launch's bindings are checked first. */
int hb_moe_experts_run(hb_gpu *gpu, const int32_t kernels[4], int32_t swiglu, int32_t combine,
                       const hb_moe_io *io, hb_range out, uint32_t m);

/* hb_moe_experts_run with no caller workspace and nothing allocated: the
 * sort's list and tile table, the gathered rows, the gate|up sums, the
 * SwiGLU rows and the slot rows live in a fixed 64 MiB device array of
 * the library (one per GPU, held until the process ends).  No counterpart
 * in the reference; for callers that cannot allocate (code under HIP graph
 * capture, tight decode loops, harnesses that forbid hipMalloc).  Rejects
 * (HB_ERR_INVALID) a block whose intermediates exceed the array, e.g. more
 * than ~700 rows at BASELINE config 5's shape (decode blocks of 1-64 rows
 * need under 6 MiB).  Calls that overlap on one GPU share the array and
 * race: issue them in stream order on one context per GPU.  Nothing in the
 * array needs to start at zero (every intermediate a call reads, it wrote). */
int hb_moe_experts_run_static(hb_gpu *gpu, const int32_t kernels[4], int32_t swiglu,
                              int32_t combine, hb_range route, hb_range x, hb_range w_gate_up,
                              hb_range w_down, hb_range out, uint32_t m);

/* Seconds the engine spent timing candidates (autotune_seconds). */
double hb_engine_autotune_seconds(hb_engine *engine);
/* The value of a --tune key after defaults and hb_engine_open's string (the
 * fields QwenEngine reads from self.tune, e.g. prefill.block, auto.heat);
 * HB_ERR_INVALID for a key the table does not hold. */
int hb_engine_tune_get(hb_engine *engine, const char *key, uint32_t *value);
/* A line of the host's own timed choices (the reference's eprintln! of
 * QwenEngine, e.g. autotune_chunk's "[autotune] blocks over ..." at
 * qwen.rs:3003) into the engine's log and stderr; `seconds` of timing are
 * added to hb_engine_autotune_seconds. */
int hb_engine_log_line(hb_engine *engine, const char *line, double seconds);

/* Every line the engine logged ([autotune] ..., [hip] ...), also written to
 * stderr as the reference's eprintln! does. */
const char *hb_engine_log(hb_engine *engine);
/* The load's closing line, the reference's "[metal] N kernels compiled in
 * ..., GEMMs and blocks timed in ..." (qwen.rs:1069), as "[hip] ...". */
int hb_engine_log_summary(hb_engine *engine);
/* The engine's timed choices so far as text (no counterpart in the
 * reference, which re-times at every load): one line per choice, tab
 * separated -- "gemm" / "gate_up" / "mv" / "experts", the choice's key (as
 * the [autotune] lines print it), then each kernel of the choice as its
 * name and its descriptor's fields (decimal, hb_desc order; "-" for none;
 * experts: the tile rows first).  *len = the text's length; up to cap - 1
 * bytes and a terminating zero into buf (buf may be null). */
int hb_engine_picks(hb_engine *engine, char *buf, uint64_t cap, uint64_t *len);
/* Seeds the engine's choices with text hb_engine_picks wrote (on this or
 * another process or box): each kernel is built from its descriptor and
 * must come out under the recorded name; later selections of those keys
 * return them without timing.  HB_ERR_INVALID naming the line otherwise. */
int hb_engine_pin(hb_engine *engine, const char *text);
/* One more candidate for the engine's next GEMM choices, after the built-in
 * ones (the way check_candidates meets a kernel that builds but computes
 * something else, qwen.rs:2488-2496: it must be logged wrong, never picked). */
int hb_engine_add_gemm_candidate(hb_engine *engine, const char *name, const hb_desc *desc);
/* ---- the checkpoint (model/qwen.rs:155-375) ---------------------------
 * Checkpoint::load: `dir` holds model.safetensors.index.json (its shards)
 * or model.safetensors; the shards are mapped read-only and every tensor
 * name normalised to the engine's key (model/qwen.rs:102-153: "N.field" for
 * "model.language_model.layers.N.field" and the other Hugging Face
 * prefixes; "embed_tokens", "norm", "lm_head"), the fields of the matmul
 * path and its norms kept, the others counted in hb_ckpt_skipped (the
 * reference's "[loader] skipped" line).  BF16, F16 and F32 tensors; each
 * element rounded once to bf16 when read (bf16_at, :92-99). */
typedef struct hb_ckpt hb_ckpt;
int hb_ckpt_open(const char *dir, hb_ckpt **ckpt);
void hb_ckpt_close(hb_ckpt *ckpt);
const char *hb_ckpt_skipped(hb_ckpt *ckpt);
/* The key's element count, 0 when the checkpoint has no such tensor. */
uint64_t hb_ckpt_elements(hb_ckpt *ckpt, const char *key);
/* read_bf16_into (model/qwen.rs:338-361): the tensors `keys`, each checked
 * against `lens` elements, one after the other into dst (bf16). */
int hb_ckpt_read(hb_ckpt *ckpt, const char *const *keys, const uint64_t *lens, uint32_t n,
                 uint16_t *dst, uint64_t dst_elements);
/* QwenEngine's upload(&mut gpu, &ck, &[(key, len), ...]) (qwen.rs:776-835):
 * the same parts stacked into one new buffer, e.g. [q | k | v] or
 * [gate | up] rows, the fused layouts the GEMMs read. */
int hb_ckpt_upload(hb_gpu *gpu, hb_ckpt *ckpt, const char *const *keys, const uint64_t *lens,
                   uint32_t n, hb_buf *out);

/* blocks_of (qwen.rs:3017-3027): a prompt of n rows cut into ceil(n / chunk)
 * blocks of equal size rounded up to 64 rows (the last shorter); starts and
 * rows of up to `cap` blocks; returns the count. */
uint32_t hb_blocks_of(uint32_t n, uint32_t chunk, uint32_t *starts, uint32_t *rows, uint32_t cap);

/* The host's side of a prefill, for autotune_chunk: `block_in` runs the
 * block of `rows` prompt rows starting at row `start` through every layer
 * the host prefills (QwenEngine::block_in, qwen.rs:2637-2894) and returns
 * its GPU seconds in *seconds; `reset` empties the conversation
 * (QwenEngine::reset: here, whatever state a block updates in place, e.g.
 * the residual stream, restored; may be null).  Both return 0 on success. */
typedef struct hb_prefill_host {
    void *ctx;
    int (*block_in)(void *ctx, uint32_t start, uint32_t rows, double *seconds);
    int (*reset)(void *ctx);
} hb_prefill_host;

/* autotune_chunk (qwen.rs:2962-3010): the rows per block for long prompts.
 * Candidates 1024, 2048, 4096 and 8192 below prefill.block, and
 * prefill.block; the first block of cands[0] rows run (after a reset) until
 * auto.heat ms of GPU time have passed; then three rounds, the order
 * reversed every other one, each a reset and a prompt of prefill.block rows
 * cut by hb_blocks_of(prefill.block, candidate); the median of each
 * candidate; the fastest into *chunk (prefill.block alone: no timing) and
 * the line "[autotune] blocks over B rows, every layer, heated X s, median
 * of 3 rounds: c t ms, ... -> best" logged.  HB_ERR_INVALID when a host
 * callback fails. */
int hb_engine_autotune_chunk(hb_engine *engine, const hb_prefill_host *host, uint32_t *chunk);

/* Tune::default + Tune::apply + Tune::summary without a device: HB_OK and
 * the summary in `summary` (cap bytes), or HB_ERR_INVALID and the
 * reference's message in hb_last_error(). */
int hb_tune_check(const char *tune, char *summary, uint64_t cap);

#ifdef __cplusplus
}
#endif

#endif /* HERBERT_HIP_H */
