// hb_moe.cpp -- the routed experts of one MoE layer as one host call: the
// dispatch sequence QwenEngine encodes per prefill block or decode step
// (src/metal/qwen.rs:2705-2735), on the kernels the selection picked
// (hb_engine_experts, expert_pipes qwen.rs:2326-2391).
#include "hb_internal.h"

namespace hb {

// ptr/size: state, route, list, tiles, x, w_gate_up, egu, ehb, w_down, ey,
// xs, out (hb_moe_io's order, then out).
int moe_experts_run(hb_gpu* g, const int32_t kernels[4], int32_t swiglu, int32_t combine,
                    void* const ptr[12], const uint64_t size[12], uint32_t m) {
    enum { STATE, ROUTE, LIST, TILES, X, WGU, EGU, EHB, WDN, EY, XS, OUT };
    const int32_t sort = kernels[0], gu = kernels[1], dn = kernels[2], gather = kernels[3];
    const hb_desc* sd = kernel_desc(g, sort);
    const hb_desc* gd = kernel_desc(g, gu);
    if (!sd || !gd || !kernel_desc(g, dn) || !kernel_desc(g, combine))
        return fail(HB_ERR_INVALID, "moe experts: a kernel of the layer is not built");
    if (sd->kind != HB_KIND_SORT && sd->kind != HB_KIND_SORT_ATOMIC)
        return fail(HB_ERR_INVALID, "moe experts: kernels[0] is not a moe_sort");
    // Grouped expert GEMMs only (never a dense split-K pair, whose
    // workspace the static entry point could not allocate).
    if (gd->rows_of == HB_ROWS_DENSE || kernel_desc(g, dn)->rows_of == HB_ROWS_DENSE ||
        kernel_desc(g, dn)->kind != HB_KIND_GEMM)
        return fail(HB_ERR_INVALID, "moe experts: kernels[1] and kernels[2] are grouped expert GEMMs");
    const bool fused = gd->kind == HB_KIND_GEMM_SWIGLU;
    if (!fused && !kernel_desc(g, swiglu))
        return fail(HB_ERR_INVALID, "moe experts: the gate|up GEMM needs the swiglu_slots kernel");
    const uint32_t top_k = sd->top_k;
    int rc;
    auto run = [&](int32_t k, std::initializer_list<int> b, uint32_t rows) {
        void* p[8];
        uint64_t s[8];
        uint32_t n = 0;
        for (int i : b) {
            p[n] = ptr[i];
            s[n] = size[i];
            n++;
        }
        return launch_ptrs(g, k, p, s, n, rows);
    };
    if ((rc = run(sort, {STATE, ROUTE, LIST, TILES}, m))) return rc;
    int xin = X;
    if (gather >= 0) {
        if ((rc = run(gather, {STATE, LIST, X, XS}, m))) return rc;
        xin = XS;
    }
    if (fused) {
        // The grouped gate|up writes the SwiGLU of its sums itself.
        if ((rc = run(gu, {STATE, WGU, xin, EHB, LIST, TILES}, m))) return rc;
    } else {
        if ((rc = run(gu, {STATE, WGU, xin, EGU, LIST, TILES}, m))) return rc;
        if ((rc = run(swiglu, {EGU, EHB}, m * top_k))) return rc;
    }
    if ((rc = run(dn, {STATE, WDN, EHB, EY, LIST, TILES}, m))) return rc;
    return run(combine, {EY, ROUTE, OUT}, m);
}

}  // namespace hb

using namespace hb;

extern "C" int hb_moe_experts_run(hb_gpu* g, const int32_t kernels[4], int32_t swiglu,
                                  int32_t combine, const hb_moe_io* io, hb_range out, uint32_t m) {
    const hb_range r[12] = {io->state, io->route, io->list, io->tiles, io->x, io->w_gate_up,
                            io->egu,   io->ehb,   io->w_down, io->ey,  io->xs, out};
    // xs is bound only with a gather, egu only when the SwiGLU is not fused
    // into the gate|up GEMM: otherwise those ranges are not looked at.
    const hb_desc* gd = kernel_desc(g, kernels[1]);
    const bool need_xs = kernels[3] >= 0, need_egu = !gd || gd->kind != HB_KIND_GEMM_SWIGLU;
    void* ptr[12];
    uint64_t size[12];
    for (int i = 0; i < 12; i++) {
        ptr[i] = nullptr;
        size[i] = 0;
        if ((i == 10 && !need_xs) || (i == 6 && !need_egu)) continue;
        char* p = nullptr;
        int rc = resolve(g, r[i], &p, &size[i]);
        if (rc) return rc;
        ptr[i] = p;
    }
    return moe_experts_run(g, kernels, swiglu, combine, ptr, size, m);
}
