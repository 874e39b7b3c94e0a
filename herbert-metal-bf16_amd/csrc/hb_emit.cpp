// hb_emit.cpp -- descriptor -> kernel: the name, source and -D constants of
// each kind, its grid and the sizes of its bindings.  The role of the
// reference's emitter functions and their grid companions (prefill.rs
// gemm_mma_rows :418 / gemm_mma_groups :406, gemm_mma_expert_groups :826,
// moe_tiles :832; kernels.rs matvec :146 / matvec_groups :1456;
// qwen_kernels.rs route_qwen :1802, swiglu_slots :2087, moe_combine :2119),
// with the kernel names following theirs (prefill.rs:1295-1300,
// kernels.rs:960-975).
#include <cstdio>

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
    }
    return d;
}

int emit(const hb_desc& d, Emitted* e) {
    char name[256];
    e->defines.clear();
    switch (d.kind) {
        case 0xffff:  // hb_zero's fill kernel
            e->name = "fill_zero";
            e->source = "fill.hip";
            e->threads = 256;
            e->nbind = 1;
            return HB_OK;
        case HB_KIND_GEMM: {
            if (d.rows_of > HB_ROWS_SCATTER || d.out > HB_OUT_RESIDUAL)
                return fail(HB_ERR_INVALID, "gemm: rows_of/out out of range");
            if (d.mfma != 16 && d.mfma != 32) return fail(HB_ERR_UNSUPPORTED, "gemm: mfma 16 or 32");
            if (!d.k || !d.n || d.k % d.bk || d.n % 4 || !pow2(d.bk) || d.bk < 32)
                return fail(HB_ERR_UNSUPPORTED, "gemm " + std::to_string(d.k) + "x" +
                                                    std::to_string(d.n) + ": K a multiple of bk=" +
                                                    std::to_string(d.bk) + ", N of 4");
            if (!d.wm || !d.wn || d.wm * d.wn > 16 || d.bm % (d.wm * d.mfma) ||
                d.bn % (d.wn * d.mfma))
                return fail(HB_ERR_UNSUPPORTED, "gemm: tile not a multiple of waves x mfma");
            bool experts = d.rows_of != HB_ROWS_DENSE;
            if (experts && (!d.top_k || !d.experts || !d.tiles))
                return fail(HB_ERR_INVALID, "gemm over experts: top_k, experts and tiles");
            std::string rows;
            if (d.rows_of == HB_ROWS_GATHER) {
                snprintf(name, sizeof name, "_gather_k%u_t%u_m%u", d.top_k, d.tiles, d.bm);
                rows = name;
            } else if (d.rows_of == HB_ROWS_SCATTER) {
                snprintf(name, sizeof name, "_scatter_t%u_m%u", d.tiles, d.bm);
                rows = name;
            }
            snprintf(name, sizeof name, "gemm_mma_%ux%u_%s%s_t%ux%u_k%u_w%ux%u_x%u%s_s%u_o%u%s", d.k,
                     d.n, out_tag(d.out), d.m_first ? "_mf" : "", d.bn, d.bm, d.bk, d.wn, d.wm,
                     d.mfma, d.dbuf ? "_d" : "", d.swz, d.order, rows.c_str());
            e->name = name;
            e->source = "gemm_mfma.hip";
            e->threads = 64 * d.wm * d.wn;
            e->nbind = 6;
            e->defines = {D("HB_K", d.k),        D("HB_N", d.n),       D("HB_OUT", d.out),
                          D("HB_ROWS", d.rows_of), D("HB_TOPK", experts ? d.top_k : 1),
                          D("HB_BM", d.bm),      D("HB_BN", d.bn),     D("HB_BK", d.bk),
                          D("HB_WM", d.wm),      D("HB_WN", d.wn),     D("HB_MFMA", d.mfma),
                          D("HB_DBUF", d.dbuf ? 1 : 0), D("HB_SWZ", d.swz),
                          D("HB_ORDER", d.order), D("HB_MFIRST", d.m_first ? 1 : 0)};
            return HB_OK;
        }
        default:
            return fail(HB_ERR_UNSUPPORTED, "kernel kind " + std::to_string(d.kind) + " not built");
    }
}

uint32_t groups_of(const hb_desc& d, uint32_t m) {
    switch (d.kind) {
        case HB_KIND_GEMM:
        case HB_KIND_GEMM_DIRECT:
        case HB_KIND_GEMM_SIMT:
        case HB_KIND_GEMM_SWIGLU: {
            uint32_t nt = cdiv(d.n, d.bn);
            if (d.rows_of != HB_ROWS_DENSE) return d.tiles * nt;  // gemm_mma_expert_groups
            return cdiv(m, d.bm) * nt;                               // gemm_mma_groups
        }
        default:
            return 0;
    }
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
            uint64_t xrows = d.rows_of == HB_ROWS_GATHER ? mm : pairs;
            if ((rc = need(s, 2, xrows * k * 2, "X"))) return rc;
            if ((rc = need(s, 3, pairs * yn * out_bytes(d.out), "Y"))) return rc;
            if ((rc = need(s, 4, pairs * 4, "list"))) return rc;
            if ((rc = need(s, 5, (1 + 3ull * d.tiles) * 4, "tiles"))) return rc;
            if (d.rows_max && m > d.rows_max)
                return fail(HB_ERR_INVALID, "m beyond the kernel's rows_max");
        }
        return HB_OK;
    }
    return fail(HB_ERR_UNSUPPORTED, "kind " + std::to_string(d.kind));
}

}  // namespace hb
