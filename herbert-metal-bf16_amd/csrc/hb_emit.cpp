// hb_emit.cpp -- descriptor -> kernel: the name, source and -D constants of
// each kind, its grid and the sizes of its bindings.  The role of the
// reference's emitter functions and their grid companions (prefill.rs
// gemm_mma_rows :418 / gemm_mma_groups :406, gemm_mma_expert_groups :826,
// moe_tiles :832; kernels.rs matvec :146 / matvec_groups :1456;
// qwen_kernels.rs route_qwen :1802, swiglu_slots :2087, moe_combine :2119),
// with the kernel names following theirs (prefill.rs:1295-1300,
// kernels.rs:960-975).
#include <cctype>
#include <cstdlib>
#include <cstdio>
#include <cstring>

#include "hb_internal.h"

namespace hb {

static const char* out_tag(uint32_t out) {
    switch (out) {
        case HB_OUT_F32: return "f32";
        case HB_OUT_RESIDUAL: return "res";
        default: return "bf16";
    }
}

static uint32_t out_bytes(uint32_t out) { return out == HB_OUT_F32 ? 4 : 2; }
static uint32_t cdiv(uint32_t a, uint32_t b) { return (a + b - 1) / b; }
static bool pow2(uint32_t v) { return v && !(v & (v - 1)); }

static std::string D(const char* k, uint64_t v) {
    return std::string("-D") + k + "=" + std::to_string(v);
}

static bool is_gemm(uint32_t kind) {
    return kind == HB_KIND_GEMM || kind == HB_KIND_GEMM_DIRECT || kind == HB_KIND_GEMM_SIMT ||
           kind == HB_KIND_GEMM_SWIGLU;
}

hb_desc with_defaults(const hb_desc& in) {
    hb_desc d = in;
    if (d.ksplit == 1) d.ksplit = 0;  // one part: no split
    if (d.kind == HB_KIND_GEMM || d.kind == HB_KIND_GEMM_SWIGLU) {
        bool experts = d.rows_of != HB_ROWS_DENSE;
        if (!d.bm) d.bm = experts ? 32 : 128;
        if (!d.bn) d.bn = 128;
        if (!d.bk) d.bk = 64;
        if (!d.wm) d.wm = experts ? 1 : 2;
        if (!d.wn) d.wn = experts ? 4 : 2;
        if (!d.mfma) d.mfma = 16;
    } else if (d.kind == HB_KIND_GEMM_DIRECT) {
        if (!d.bm) d.bm = 64;
        if (!d.bn) d.bn = 64;
        if (!d.mfma) d.mfma = 16;
    } else if (d.kind == HB_KIND_GEMM_SIMT) {
        if (!d.bm) d.bm = 64;
        if (!d.bn) d.bn = 64;
    } else if (d.kind == HB_KIND_MATVEC) {
        if (!d.mv_m) d.mv_m = 1;
        if (!d.split) d.split = 1;
        if (!d.rows) d.rows = 4;
        if (!d.unroll) d.unroll = 4;
        if (d.form == 1 || (d.form == 3 && d.rows != 32)) d.rows = 16;
        if (d.form == 4 && d.rows != 8 && d.rows != 16) d.rows = 4;
        if (!d.mv_waves) d.mv_waves = 4;
    }
    return d;
}

static int emit_kind(const hb_desc& d, Emitted* e) {
    char name[256];
    e->defines.clear();
    switch (d.kind) {
        case 0xffff:  // hb_zero's fill kernel
            e->name = "fill_zero";
            e->source = "fill.hip";
            e->threads = 256;
            e->nbind = 1;
            return HB_OK;
        case HB_KIND_GEMM:
        case HB_KIND_GEMM_SWIGLU: {
            const bool swi = d.kind == HB_KIND_GEMM_SWIGLU;
            if (d.rows_of > HB_ROWS_SORTED || d.out > HB_OUT_RESIDUAL)
                return fail(HB_ERR_INVALID, "gemm: rows_of/out out of range");
            if (swi && (d.rows_of == HB_ROWS_SCATTER || d.out != HB_OUT_BF16))
                return fail(HB_ERR_UNSUPPORTED, "gemm_swiglu: dense or gathered rows, bf16 out");
            if (d.band && d.rows_of != HB_ROWS_DENSE)
                return fail(HB_ERR_UNSUPPORTED, "gemm: band order over dense rows only");
            if (d.mfma != 16 && d.mfma != 32) return fail(HB_ERR_UNSUPPORTED, "gemm: mfma 16 or 32");
            if (!d.k || !d.n || d.k % d.bk || d.n % 4 || !pow2(d.bk) || d.bk < 32)
                return fail(HB_ERR_UNSUPPORTED, "gemm " + std::to_string(d.k) + "x" +
                                                    std::to_string(d.n) + ": K a multiple of bk=" +
                                                    std::to_string(d.bk) + ", N of 4");
            if (!d.wm || !d.wn || d.wm * d.wn > 16 || d.bm % (d.wm * d.mfma) ||
                d.bn % (d.wn * d.mfma))
                return fail(HB_ERR_UNSUPPORTED, "gemm: tile not a multiple of waves x mfma");
            if (swi && (d.bn / (d.wn * d.mfma)) % 2)
                return fail(HB_ERR_UNSUPPORTED,
                            "gemm_swiglu: an even count of W fragments per wave (bn / (wn * mfma))");
            bool experts = d.rows_of != HB_ROWS_DENSE;
            if (experts && (!d.top_k || !d.experts || !d.tiles))
                return fail(HB_ERR_INVALID, "gemm over experts: top_k, experts and tiles");
            e->threads = 64 * d.wm * d.wn;
            // LDS swizzle shift: 0 = the conflict-free one on gfx950; s+1 =
            // s.  The fragment reads (ds_read_b128, 16 rows at one chunk)
            // measured conflict-free (SQ_LDS_BANK_CONFLICT = 0) with the chunk
            // XORed by row >> 1 for rows of 4 and of 8 chunks (BK 32 and 64);
            // row >> 2 for rows of 4 chunks conflicted on half of the LDS
            // cycles.  Rows of 16 chunks: row >> 0.
            uint32_t ch = d.bk / 8, shift = ch >= 16 ? 0 : 1;
            if (d.swz) shift = d.swz - 1;
            std::string rows;
            if (d.rows_of == HB_ROWS_GATHER) {
                snprintf(name, sizeof name, "_gather_k%u_t%u_m%u", d.top_k, d.tiles, d.bm);
                rows = name;
            } else if (d.rows_of == HB_ROWS_SCATTER) {
                snprintf(name, sizeof name, "_scatter_t%u_m%u", d.tiles, d.bm);
                rows = name;
            } else if (d.rows_of == HB_ROWS_SORTED) {
                snprintf(name, sizeof name, "_sorted_k%u_t%u_m%u", d.top_k, d.tiles, d.bm);
                rows = name;
            }
            if (d.dbuf > 3 || (!d.lds_dma && d.dbuf > 1))
                return fail(HB_ERR_UNSUPPORTED, "gemm: stages 1..4 (1..2 through registers)");
            if (d.w_nt > 1 || (d.w_nt && !d.lds_dma))
                return fail(HB_ERR_UNSUPPORTED, "gemm: w_nt with direct-to-LDS staging");
            if (d.sched > 3) return fail(HB_ERR_INVALID, "gemm: sched 0..3");
            if (d.sched && (swi || experts || !d.lds_dma || d.dbuf < 2 || d.w_nt ||
                            d.wm * d.wn != (d.sched == 3 ? 4u : 8u) ||
                            ((d.bm * d.bk / 8) % 64) || ((d.bn * d.bk / 8) % 64) ||
                            (d.sched == 3 && (d.k / d.bk) % 2) ||
                            (d.bm * d.bk / 8 / 64 + d.bn * d.bk / 8 / 64) < d.wm * d.wn))
                return fail(HB_ERR_UNSUPPORTED,
                            "gemm (pipelined schedules): dense rows, direct-to-LDS, 3 or 4 stages, "
                            "8 waves (sched 1, 2) or 4 (sched 3, an even count of K tiles), whole "
                            "1 KiB loads per stage, no w_nt");
            if (d.sched &&
                (uint64_t)(d.dbuf + 1) * (d.bm + d.bn) * d.bk * 2 > 160 * 1024)
                return fail(HB_ERR_UNSUPPORTED, "gemm (pipelined schedules): stages beyond 160 KiB of LDS");
            if (d.ksplit > 16 || (d.ksplit > 1 && (swi || experts || d.k % (d.bk * d.ksplit) ||
                                                   (d.sched == 3 && (d.k / d.bk / d.ksplit) % 2))))
                return fail(HB_ERR_UNSUPPORTED,
                            "gemm split K: 2..16 parts, dense rows, K a multiple of bk x parts "
                            "(sched 3: an even count of K tiles per part)");
            std::string band = d.band ? "_b" + std::to_string(d.band) : "";
            if (d.w_nt) band += "_wnt";
            if (d.ksplit > 1) band += "_ks" + std::to_string(d.ksplit);
            if (d.sched) band += d.sched == 1 ? "_pp" : d.sched == 2 ? "_pp2" : "_il";
            snprintf(name, sizeof name, "gemm_mma%s_%ux%u_%s%s_t%ux%u_k%u_w%ux%u_x%u_d%u%s_s%u_o%u%s%s",
                     swi ? "_swiglu" : "", d.k, d.n, out_tag(d.out), d.m_first ? "_mf" : "", d.bn,
                     d.bm, d.bk, d.wn, d.wm, d.mfma, d.dbuf, d.lds_dma ? "_dma" : "", shift, d.order,
                     band.c_str(), rows.c_str());
            e->name = name;
            e->source = d.sched ? "gemm_pp.hip" : "gemm_mfma.hip";
            e->threads = 64 * d.wm * d.wn;
            e->nbind = 6;
            e->defines = {D("HB_K", d.k),        D("HB_N", d.n),       D("HB_OUT", d.out),
                          D("HB_ROWS", d.rows_of), D("HB_TOPK", experts ? d.top_k : 1),
                          D("HB_BM", d.bm),      D("HB_BN", d.bn),     D("HB_BK", d.bk),
                          D("HB_WM", d.wm),      D("HB_WN", d.wn),     D("HB_MFMA", d.mfma),
                          D("HB_STAGES", d.dbuf + 1), D("HB_SWZ", shift),
                          D("HB_ORDER", d.order), D("HB_MFIRST", d.m_first ? 1 : 0),
                          D("HB_DMA", d.lds_dma ? 1 : 0), D("HB_SWIGLU", swi ? 1 : 0),
                          D("HB_BAND", d.band), D("HB_W_NT", d.w_nt)};
            if (d.ksplit > 1) {
                // The parts' f32 sums into the workspace; Out is the second
                // kernel's.
                e->defines[2] = D("HB_OUT", HB_OUT_F32);
                e->defines.push_back(D("HB_KSPLIT", d.ksplit));
            }
            if (d.sched) {
                e->defines.push_back(D("HB_SCHED", d.sched == 3 ? 3 : 1));
                e->defines.push_back(D("HB_GRP", d.sched == 2 ? 1 : 0));
            }
            return HB_OK;
        }
        case KIND_SPLITK_REDUCE:
            if (!d.n || d.n % 4 || d.ksplit < 2 || d.ksplit > 16 || d.out > HB_OUT_RESIDUAL)
                return fail(HB_ERR_INVALID, "split-K reduce: N a multiple of 4, 2..16 parts");
            snprintf(name, sizeof name, "gemm_splitk_%u_%s_s%u", d.n, out_tag(d.out), d.ksplit);
            e->name = name;
            e->source = "gemm_splitk.hip";
            e->threads = 256;
            e->nbind = 3;
            e->defines = {D("HB_N", d.n), D("HB_OUT", d.out), D("HB_KSPLIT", d.ksplit)};
            return HB_OK;
        case HB_KIND_GEMM_SIMT:
            if (d.rows_of != HB_ROWS_DENSE || d.out > HB_OUT_RESIDUAL || !d.k || d.k % 16 || !d.n)
                return fail(HB_ERR_UNSUPPORTED, "gemm_simt: dense rows, K a multiple of 16");
            snprintf(name, sizeof name, "gemm_simt_%ux%u_%s%s", d.k, d.n, out_tag(d.out),
                     d.m_first ? "_mf" : "");
            e->name = name;
            e->source = "gemm_simt.hip";
            e->threads = 256;
            e->nbind = 6;
            e->defines = {D("HB_K", d.k), D("HB_N", d.n), D("HB_OUT", d.out),
                          D("HB_MFIRST", d.m_first ? 1 : 0)};
            return HB_OK;
        case HB_KIND_GEMM_DIRECT:
            if (d.rows_of != HB_ROWS_DENSE || d.out > HB_OUT_RESIDUAL || !d.k || d.k % 32 ||
                !d.n || d.n % 4 || d.bm % 16 || d.bn % 16 || !d.bm || !d.bn ||
                (d.bm / 16) * (d.bn / 16) > 16)
                return fail(HB_ERR_UNSUPPORTED, "gemm_mm2d: dense, K a multiple of 32, tiles of 16..64");
            snprintf(name, sizeof name, "gemm_mm2d_%ux%u_%s%s_%ux%u", d.k, d.n, out_tag(d.out),
                     d.m_first ? "_mf" : "", d.bm, d.bn);
            e->name = name;
            e->source = "gemm_direct.hip";
            e->threads = 64 * (d.bm / 16) * (d.bn / 16);
            e->nbind = 6;
            e->defines = {D("HB_K", d.k), D("HB_N", d.n), D("HB_OUT", d.out), D("HB_BM", d.bm),
                          D("HB_BN", d.bn), D("HB_MFIRST", d.m_first ? 1 : 0)};
            return HB_OK;
        case HB_KIND_MATVEC: {
            if (d.out > HB_OUT_SWIGLU || d.form > 4 || d.xsrc > HB_XSRC_NORM)
                return fail(HB_ERR_INVALID, "matvec: out / form / xsrc out of range");
            if (d.form == 4 && (d.mv_m > 8 || !d.split || d.k % (128 * d.split) || d.xsrc ||
                                d.out == HB_OUT_SWIGLU || d.x_lds))
                return fail(HB_ERR_UNSUPPORTED,
                            "matvec (MFMA 4x4x4): m <= 8, K/split a multiple of 128, no fusions, no x_lds");
            const bool mma = d.form == 1 || d.form == 3 || d.form == 4;
            if ((d.xsrc || d.out == HB_OUT_SWIGLU) && mma)
                return fail(HB_ERR_UNSUPPORTED, "matvec: XSrc and Out::Swiglu fusions in the VALU forms");
            if (d.out == HB_OUT_SWIGLU && (d.rows % 2 || d.n % 2))
                return fail(HB_ERR_UNSUPPORTED, "matvec Out::Swiglu: even rows (gate and up) and n");
            if (d.xsrc == HB_XSRC_NORM && ((uint64_t)d.mv_m * d.k * 2 > 65536 || d.k % 256))
                return fail(HB_ERR_UNSUPPORTED, "matvec XSrc::Norm: m*k*2 <= 64 KiB of LDS, k a multiple of 256");
            if (d.mv_waves != 4 && d.mv_waves != 8 && d.mv_waves != 16)
                return fail(HB_ERR_UNSUPPORTED, "matvec: mv_waves 4, 8 or 16");
            if (d.mv_waves != 4 && d.xsrc == HB_XSRC_NORM)
                return fail(HB_ERR_UNSUPPORTED, "matvec XSrc::Norm: 4 waves");
            if (d.x_lds > 1 ||
                (d.x_lds && (d.form == 1 || (uint64_t)d.mv_m * d.k * 2 > (d.mv_waves == 4 ? 65536u : 147456u))))
                return fail(HB_ERR_UNSUPPORTED,
                            "matvec x_lds: VALU forms and form 3, m*k*2 <= 64 KiB of LDS (144 KiB with 8 or 16 waves)");
            const bool xl = d.x_lds && d.xsrc != HB_XSRC_NORM;
            if (!d.k || !d.n || d.k % (8 * d.split) || !d.split || (d.split & (d.split - 1)) ||
                d.split > d.mv_waves)
                return fail(HB_ERR_UNSUPPORTED, "matvec: K a multiple of 8*split, split 1, 2, 4 (8, 16 with as many waves)");
            if (!mma && (d.rows > 8 || !d.rows || d.rows * d.mv_m > 64 || d.mv_m > 16))
                return fail(HB_ERR_UNSUPPORTED, "matvec: rows 1..8, rows*m <= 64");
            if (mma && (d.mv_m > 16 || (d.k / d.split) % 32))
                return fail(HB_ERR_UNSUPPORTED, "matvec (MFMA): m <= 16, K/split a multiple of 32");
            if (d.form == 3 && ((d.unroll != 4 && d.unroll != 8 && d.unroll != 16) ||
                                d.mv_waves * d.unroll * (d.rows / 16) > 64))
                return fail(HB_ERR_UNSUPPORTED,
                            "matvec (MFMA, W through LDS): unroll 4, 8 or 16, waves*unroll*rows/16 <= 64");
            if (!d.unroll || d.unroll > (mma ? 16u : 8u))
                return fail(HB_ERR_UNSUPPORTED, "matvec: unroll 1..8 (MFMA form 1..16)");
            char xtag[48] = "";
            if (d.xsrc == HB_XSRC_SWIGLU) snprintf(xtag, sizeof xtag, "_swi");
            if (d.xsrc == HB_XSRC_NORM)
                snprintf(xtag, sizeof xtag, "_nrm%08x%s", d.eps_bits, d.plus_one ? "p1" : "");
            if (xl) strncat(xtag, "_xl", sizeof xtag - strlen(xtag) - 1);
            if (d.mv_waves != 4) strncat(xtag, d.mv_waves == 8 ? "_w8" : "_w16", sizeof xtag - strlen(xtag) - 1);
            snprintf(name, sizeof name, "matvec_%ux%u%s%s_r%u_k%u%s_m%u_%s_u%u", d.k, d.n, xtag,
                     d.out == HB_OUT_F32 ? "_f32" : d.out == HB_OUT_RESIDUAL ? "_res"
                                                  : d.out == HB_OUT_SWIGLU ? "_sw" : "",
                     d.rows, d.split, d.persist ? ("_p" + std::to_string(d.persist)).c_str() : "",
                     d.mv_m,
                     d.form == 1 ? "mfma" : d.form == 2 ? "dot2" : d.form == 3 ? "mfl" : d.form == 4 ? "mf4" : "valu",
                     d.unroll);
            e->name = name;
            e->source = "matvec.hip";
            e->threads = 64 * d.mv_waves;
            e->nbind = d.xsrc == HB_XSRC_NORM ? 4 : 3;
            e->defines = {D("HB_K", d.k),         D("HB_N", d.n),          D("HB_OUT", d.out),
                          D("HB_MV_M", d.mv_m),   D("HB_FORM", d.form),    D("HB_ROWS", d.rows),
                          D("HB_SPLIT", d.split), D("HB_PERSIST", d.persist), D("HB_UNROLL", d.unroll),
                          D("HB_XSRC", d.xsrc),   D("HB_EPS", d.eps_bits), D("HB_PLUS1", d.plus_one),
                          D("HB_XLDS", xl ? 1 : 0), D("HB_WAVES", d.mv_waves)};
            return HB_OK;
        }
        case HB_KIND_ROUTE:
            if (!d.experts || d.experts % 64 || d.experts > 1024 || !d.top_k || d.top_k > 64 ||
                d.top_k > d.experts)
                return fail(HB_ERR_UNSUPPORTED, "route: experts a multiple of 64 up to 1024, top_k <= 64");
            snprintf(name, sizeof name, "route_qwen_%u_k%u", d.experts, d.top_k);
            e->name = name;
            e->source = "moe.hip";
            e->threads = 256;
            e->nbind = 2;
            e->defines = {D("HB_OP", 1), D("HB_E", d.experts), D("HB_TOPK", d.top_k), D("HB_D", 8)};
            return HB_OK;
        case HB_KIND_SORT:
        case HB_KIND_SORT_ATOMIC: {
            if (!d.experts || d.experts > 1024 || !d.top_k || !d.bm || !d.rows_max)
                return fail(HB_ERR_UNSUPPORTED, "sort: experts <= 1024, top_k, bm, rows_max");
            uint32_t tiles = cdiv(d.rows_max * d.top_k, d.bm) + d.experts;  // moe_tiles
            if (d.tiles && d.tiles < tiles)
                return fail(HB_ERR_INVALID, "sort: tile table smaller than moe_tiles");
            bool atomic = d.kind == HB_KIND_SORT_ATOMIC;
            snprintf(name, sizeof name, "moe_sort%s_%u_k%u_r%u_m%u", atomic ? "_atomic" : "",
                     d.experts, d.top_k, d.rows_max, d.bm);
            e->name = name;
            e->source = "moe.hip";
            e->threads = 1024;
            e->nbind = 4;
            e->defines = {D("HB_OP", atomic ? 3 : 2), D("HB_E", d.experts), D("HB_TOPK", d.top_k),
                          D("HB_BM", d.bm), D("HB_D", 8), D("HB_RMAX", d.rows_max)};
            return HB_OK;
        }
        case HB_KIND_GATHER:
            if (!d.n || d.n % 8 || !d.top_k) return fail(HB_ERR_UNSUPPORTED, "gather: hidden a multiple of 8");
            snprintf(name, sizeof name, "moe_gather_%u_k%u", d.n, d.top_k);
            e->name = name;
            e->source = "moe.hip";
            e->threads = 256;
            e->nbind = 4;
            e->defines = {D("HB_OP", 4), D("HB_E", 64), D("HB_TOPK", d.top_k), D("HB_D", d.n)};
            return HB_OK;
        case HB_KIND_SWIGLU:
            if (!d.n || d.n % 8) return fail(HB_ERR_UNSUPPORTED, "swiglu: n a multiple of 8");
            snprintf(name, sizeof name, "swiglu_%u", d.n);
            e->name = name;
            e->source = "moe.hip";
            e->threads = 256;
            e->nbind = 2;
            e->defines = {D("HB_OP", 5), D("HB_E", 64), D("HB_TOPK", 1), D("HB_D", d.n)};
            return HB_OK;
        case HB_KIND_COMBINE:
            if (!d.n || d.n % 8 || !d.top_k || d.top_k > 16)
                return fail(HB_ERR_UNSUPPORTED, "combine: d a multiple of 8, top_k 1..16");
            snprintf(name, sizeof name, "moe_combine_%u_k%u", d.n, d.top_k);
            e->name = name;
            e->source = "moe.hip";
            e->threads = 256;
            e->nbind = 3;
            e->defines = {D("HB_OP", 6), D("HB_E", 64), D("HB_TOPK", d.top_k), D("HB_D", d.n)};
            return HB_OK;
        case HB_KIND_MOE_OUT:
            if (!d.n || d.n % 256) return fail(HB_ERR_UNSUPPORTED, "moe_out: d a multiple of 256");
            snprintf(name, sizeof name, "moe_out_%u", d.n);
            e->name = name;
            e->source = "moe.hip";
            e->threads = 256;
            e->nbind = 5;
            e->defines = {D("HB_OP", 7), D("HB_E", 64), D("HB_TOPK", 1), D("HB_D", d.n)};
            return HB_OK;
        case HB_KIND_RMSNORM:
            if (!d.n || d.n % 256) return fail(HB_ERR_UNSUPPORTED, "rmsnorm: d a multiple of 256");
            snprintf(name, sizeof name, "rmsnorm_%u_e%08x%s", d.n, d.eps_bits, d.plus_one ? "_p1" : "");
            e->name = name;
            e->source = "moe.hip";
            e->threads = 256;
            e->nbind = 3;
            e->defines = {D("HB_OP", 8), D("HB_E", 64), D("HB_TOPK", 1), D("HB_D", d.n),
                          D("HB_EPS", d.eps_bits), D("HB_PLUS1", d.plus_one)};
            return HB_OK;
        case HB_KIND_ROUND_PROBE:
            e->name = "round_probe_bf16";
            e->source = "probe.hip";
            e->threads = 256;
            e->nbind = 3;
            return HB_OK;
        default:
            return fail(HB_ERR_UNSUPPORTED, "kernel kind " + std::to_string(d.kind) + " not built");
    }
}

// A development build of the library (build.py --dev, never the shipped
// one) adds HB_DEV_DEFINES="-DX=1 -DY=2" to every kernel built while it is
// set, for variants under study; the kernel's name (its cache key) then
// carries them.  The shipped library has no such hook: no environment
// variable changes what its kernels compute.
int emit(const hb_desc& d, Emitted* e) {
    int rc = emit_kind(d, e);
#ifdef HB_DEV_BUILD
    const char* dev = getenv("HB_DEV_DEFINES");
    if (rc || !dev || !*dev) return rc;
    std::string tag = "_dev";
    std::string cur;
    for (const char* c = dev;; c++) {
        if (*c == ' ' || *c == 0) {
            if (!cur.empty()) e->defines.push_back(cur);
            cur.clear();
            if (!*c) break;
            continue;
        }
        cur += *c;
        tag += isalnum((unsigned char)*c) ? *c : '_';
    }
    e->name += tag;
#endif
    return rc;
}

uint32_t groups_of(const hb_desc& d, uint32_t m) {
    switch (d.kind) {
        case HB_KIND_GEMM:
        case HB_KIND_GEMM_DIRECT:
        case HB_KIND_GEMM_SIMT:
        case HB_KIND_GEMM_SWIGLU: {
            uint32_t bm = d.kind == HB_KIND_GEMM_SIMT ? 64 : d.bm;
            uint32_t bn = d.kind == HB_KIND_GEMM_SIMT ? 64 : d.kind == HB_KIND_GEMM_SWIGLU ? d.bn / 2 : d.bn;
            uint32_t nt = cdiv(d.n, bn);
            if (d.rows_of != HB_ROWS_DENSE) return d.tiles * nt;  // gemm_mma_expert_groups
            return cdiv(m, bm) * nt * (d.ksplit > 1 ? d.ksplit : 1);  // gemm_mma_groups
        }
        case KIND_SPLITK_REDUCE: {  // 4 outputs a thread, at most 8 workgroups a CU
            const uint64_t g = ((uint64_t)m * (d.n / 4) + 255) / 256;
            return (uint32_t)(g < 2048 ? g : 2048);
        }
        case HB_KIND_MATVEC: {  // matvec_groups / matvec_split_groups / matvec_full_groups
            uint32_t rb = d.form == 1 ? 16 : d.rows, per = d.mv_waves / d.split;
            uint32_t n = d.n;
            if (d.out == HB_OUT_SWIGLU) n /= 2, rb /= 2;  // output rows: gate rows
            uint32_t wgs = cdiv(cdiv(n, rb), per);
            return d.persist ? (d.persist < wgs ? d.persist : wgs) : wgs;
        }
        case HB_KIND_ROUTE:
            return cdiv(m, 4);  // a wavefront per row
        case HB_KIND_SORT:
        case HB_KIND_SORT_ATOMIC:
            return 1;
        case HB_KIND_GATHER:
            return (uint32_t)(((uint64_t)m * d.top_k * (d.n / 8) + 255) / 256);
        case HB_KIND_SWIGLU:
        case HB_KIND_COMBINE:
            return (uint32_t)(((uint64_t)m * (d.n / 8) + 255) / 256);
        case HB_KIND_MOE_OUT:
        case HB_KIND_RMSNORM:
            return m;  // a workgroup per row
        case HB_KIND_ROUND_PROBE:
            return (1u << 24) / 256;  // one pattern per thread
        default:
            return 0;
    }
}

uint64_t workspace_of(const hb_desc& d, uint32_t m) {
    if (d.kind != HB_KIND_GEMM || d.ksplit < 2) return 0;
    return (uint64_t)d.ksplit * m * d.n * 4;
}

static int need(const uint64_t* sizes, uint32_t i, uint64_t bytes, const char* what) {
    if (sizes[i] < bytes)
        return fail(HB_ERR_INVALID, std::string("binding ") + std::to_string(i) + " (" + what +
                                        ") holds " + std::to_string(sizes[i]) + " bytes, needs " +
                                        std::to_string(bytes));
    return HB_OK;
}

int check_bindings(const hb_desc& d, const uint64_t* s, uint32_t nbind, uint32_t m) {
    int rc = HB_OK;
    (void)nbind;
    if (is_gemm(d.kind)) {
        uint64_t k = d.k, n = d.n, mm = m;
        uint64_t nw = d.kind == HB_KIND_GEMM_SWIGLU ? 2 * n : n;  // [gate | up] rows
        uint64_t yn = n;
        if (m == 0) return fail(HB_ERR_INVALID, "0 rows");
        if ((rc = need(s, 0, 16, "state"))) return rc;
        if (d.rows_of == HB_ROWS_DENSE) {
            if ((rc = need(s, 1, nw * k * 2, "W"))) return rc;
            if ((rc = need(s, 2, mm * k * 2, "X"))) return rc;
            if ((rc = need(s, 3, mm * yn * out_bytes(d.out), "Y"))) return rc;
        } else {
            uint64_t pairs = mm * d.top_k;
            if ((rc = need(s, 1, (uint64_t)d.experts * nw * k * 2, "W"))) return rc;
            uint64_t xrows = d.rows_of == HB_ROWS_GATHER ? mm : pairs;  // scatter, sorted: pairs
            if ((rc = need(s, 2, xrows * k * 2, "X"))) return rc;
            if ((rc = need(s, 3, pairs * yn * out_bytes(d.out), "Y"))) return rc;
            if ((rc = need(s, 4, pairs * 4, "list"))) return rc;
            if ((rc = need(s, 5, (1 + 3ull * d.tiles) * 4, "tiles"))) return rc;
            if (d.rows_max && m > d.rows_max)
                return fail(HB_ERR_INVALID, "m beyond the kernel's rows_max");
        }
        // Direct-to-LDS staging addresses each operand through a buffer
        // resource of 2^31 - 1 bytes (a load past it reads zeros).
        if ((d.kind == HB_KIND_GEMM || d.kind == HB_KIND_GEMM_SWIGLU) && d.lds_dma) {
            const uint64_t wb = (d.rows_of == HB_ROWS_DENSE ? 1ull : d.experts) * nw * k * 2;
            const uint64_t xb = (d.rows_of == HB_ROWS_DENSE || d.rows_of == HB_ROWS_GATHER ? mm : mm * d.top_k) * k * 2;
            if (wb > 0x7fffffffull || xb > 0x7fffffffull)
                return fail(HB_ERR_UNSUPPORTED, "gemm (direct-to-LDS staging): W and X at most 2 GiB - 1 bytes each");
        }
        return HB_OK;
    }
    if (m == 0) return fail(HB_ERR_INVALID, "0 rows");
    uint64_t mm = m, k2 = 2ull * d.top_k;
    switch (d.kind) {
        case HB_KIND_ROUTE:
            if ((rc = need(s, 0, mm * d.experts * 2, "scores"))) return rc;
            return need(s, 1, mm * k2 * 4, "route");
        case HB_KIND_SORT:
        case HB_KIND_SORT_ATOMIC: {
            if (m > d.rows_max) return fail(HB_ERR_INVALID, "sort: m beyond rows_max");
            uint64_t tiles = cdiv(d.rows_max * d.top_k, d.bm) + d.experts;
            if ((rc = need(s, 0, 16, "state"))) return rc;
            if ((rc = need(s, 1, mm * k2 * 4, "route"))) return rc;
            if ((rc = need(s, 2, mm * d.top_k * 4, "list"))) return rc;
            return need(s, 3, (1 + 3 * tiles) * 4, "tiles");
        }
        case HB_KIND_GATHER:
            if ((rc = need(s, 0, 16, "state"))) return rc;
            if ((rc = need(s, 1, mm * d.top_k * 4, "list"))) return rc;
            if ((rc = need(s, 2, mm * d.n * 2, "X"))) return rc;
            return need(s, 3, mm * d.top_k * d.n * 2, "XS");
        case HB_KIND_SWIGLU:
            if ((rc = need(s, 0, mm * 2 * d.n * 2, "gate_up"))) return rc;
            return need(s, 1, mm * d.n * 2, "h");
        case HB_KIND_ROUND_PROBE:
            if ((rc = need(s, 0, 16, "state"))) return rc;
            if ((rc = need(s, 1, 2ull << 24, "out_int"))) return rc;
            return need(s, 2, 2ull << 24, "out_hw");
        case HB_KIND_RMSNORM:
            if ((rc = need(s, 0, mm * d.n * 2, "x"))) return rc;
            if ((rc = need(s, 1, (uint64_t)d.n * 2, "w"))) return rc;
            return need(s, 2, mm * d.n * 2, "y");
        case HB_KIND_MOE_OUT:
            if ((rc = need(s, 0, mm * d.n * 2, "xn"))) return rc;
            if ((rc = need(s, 1, (uint64_t)d.n * 2, "shared_gate"))) return rc;
            if ((rc = need(s, 2, mm * d.n * 2, "experts"))) return rc;
            if ((rc = need(s, 3, mm * d.n * 2, "shared"))) return rc;
            return need(s, 4, mm * d.n * 2, "x");
        case KIND_SPLITK_REDUCE:
            if ((rc = need(s, 0, 16, "state"))) return rc;
            if ((rc = need(s, 1, (uint64_t)d.ksplit * mm * d.n * 4, "slabs"))) return rc;
            return need(s, 2, mm * d.n * out_bytes(d.out), "Y");
        case HB_KIND_COMBINE:
            if ((rc = need(s, 0, mm * d.top_k * d.n * 2, "y"))) return rc;
            if ((rc = need(s, 1, mm * k2 * 4, "route"))) return rc;
            return need(s, 2, mm * d.n * 2, "out");
        default:
            break;
    }
    if (d.kind == HB_KIND_MATVEC) {
        uint64_t k = d.k, n = d.n;
        if (m > d.mv_m)
            return fail(HB_ERR_INVALID, "matvec of " + std::to_string(m) + " rows: 1.." +
                                            std::to_string(d.mv_m));
        if ((rc = need(s, 0, n * k * 2, "W"))) return rc;
        if ((rc = need(s, 1, mm * k * 2 * (d.xsrc == HB_XSRC_SWIGLU ? 2 : 1), "x"))) return rc;
        uint64_t yn = d.out == HB_OUT_SWIGLU ? n / 2 : n;
        if ((rc = need(s, 2, mm * yn * out_bytes(d.out), "y"))) return rc;
        if (d.xsrc == HB_XSRC_NORM && (rc = need(s, 3, k * 2, "norm weights"))) return rc;
        return HB_OK;
    }
    return fail(HB_ERR_UNSUPPORTED, "kind " + std::to_string(d.kind));
}

}  // namespace hb
