// hb_static.hip -- hb_moe_experts_run_static: the routed experts of an MoE
// layer (hb_moe_experts_run) with every intermediate in a fixed device array
// of this library instead of caller buffers, for callers that cannot
// allocate (code under HIP graph capture, tight decode loops).  Compiled as
// HIP for gfx950 so that the array is a device global of the library's own
// code object; the kernels (hiprtc modules) receive its address.
#include <mutex>
#include <unordered_map>

#include "hb_internal.h"

// The array every call on a device shares: the sort's list and tile table,
// the gathered rows, the grouped gate|up's sums, the SwiGLU rows, the slot
// rows of the down GEMM, and a state word.  Each GPU the library runs on
// holds its own copy until the process ends.
#define HB_SCRATCH_BYTES (64ull << 20)
static __device__ __align__(256) unsigned char scratch[HB_SCRATCH_BYTES];

namespace hb {

// The scratch's first 256 bytes: a state whose state[3] (the row count the
// kernels read, at most their launch's m) is 0xffffffff, so every launch
// runs its own m.  Written once per device at set-up; no kernel writes it.
static const uint32_t kStateInit[4] = {0, 0, 0, 0xffffffffu};
static const uint64_t kStateBytes = 256;

// Once per device, with that device current: the array's device address
// (hipGetSymbolAddress; the array's host-side name is not a device address)
// and the state word.  Later calls return the kept address.
int static_scratch(int device, void** out) {
    static std::mutex mu;
    static std::unordered_map<int, void*> addr;
    std::lock_guard<std::mutex> lock(mu);
    auto it = addr.find(device);
    if (it != addr.end()) {
        *out = it->second;
        return HB_OK;
    }
    void* p = nullptr;
    HB_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    HB_HIP(hipMemcpy(p, kStateInit, sizeof kStateInit, hipMemcpyHostToDevice));
    addr[device] = p;
    *out = p;
    return HB_OK;
}

}  // namespace hb

using namespace hb;

static uint64_t up256(uint64_t v) { return (v + 255) & ~255ull; }

extern "C" int hb_moe_experts_run_static(hb_gpu* g, const int32_t kernels[4], int32_t swiglu,
                                         int32_t combine, hb_range route, hb_range x,
                                         hb_range w_gate_up, hb_range w_down, hb_range out,
                                         uint32_t m) {
    if (!g->scratch) return fail(HB_ERR_INVALID, "moe experts (static): no scratch on this context");
    const hb_desc* sd = kernel_desc(g, kernels[0]);
    const hb_desc* gd = kernel_desc(g, kernels[1]);
    const hb_desc* dd = kernel_desc(g, kernels[2]);
    if (!sd || !gd || !dd || (sd->kind != HB_KIND_SORT && sd->kind != HB_KIND_SORT_ATOMIC) ||
        gd->rows_of == HB_ROWS_DENSE || dd->rows_of == HB_ROWS_DENSE)
        return fail(HB_ERR_INVALID, "moe experts (static): kernels[0..2] must be a built sort and grouped GEMMs");
    if (m == 0) return fail(HB_ERR_INVALID, "moe experts (static): 0 rows");
    const bool fused = gd->kind == HB_KIND_GEMM_SWIGLU, gather = kernels[3] >= 0;
    const uint64_t pairs = (uint64_t)m * sd->top_k, hidden = dd->n, inter = dd->k;
    // The table's capacity: what the sort and the GEMMs were built for.
    const uint64_t cap_sort = (sd->rows_max * (uint64_t)sd->top_k + sd->bm - 1) / sd->bm + sd->experts;
    const uint64_t cap = cap_sort > gd->tiles ? cap_sort : gd->tiles;
    // Layout: state, list, tiles, xs, egu, ehb, ey (each 256-byte aligned).
    const uint64_t sz[7] = {kStateBytes,
                            pairs * 4,
                            (1 + 3 * (cap > dd->tiles ? cap : dd->tiles)) * 4,
                            gather ? pairs * hidden * 2 : 0,
                            fused ? 0 : pairs * 2 * inter * 2,
                            pairs * inter * 2,
                            pairs * hidden * 2};
    uint64_t off[7], total = 0;
    for (int i = 0; i < 7; i++) {
        off[i] = total;
        total += up256(sz[i]);
    }
    if (total > HB_SCRATCH_BYTES)
        return fail(HB_ERR_INVALID, "moe experts (static): " + std::to_string(m) + " rows need " +
                                        std::to_string(total) + " bytes of scratch, it holds " +
                                        std::to_string(HB_SCRATCH_BYTES) +
                                        " (use hb_moe_experts_run with caller buffers)");
    char* base = (char*)g->scratch;
    enum { STATE, ROUTE, LIST, TILES, X, WGU, EGU, EHB, WDN, EY, XS, OUT };
    void* ptr[12] = {};
    uint64_t size[12] = {};
    const int seg[7] = {STATE, LIST, TILES, XS, EGU, EHB, EY};
    for (int i = 0; i < 7; i++) {
        ptr[seg[i]] = sz[i] ? base + off[i] : nullptr;
        size[seg[i]] = sz[i];
    }
    const hb_range* r[5] = {&route, &x, &w_gate_up, &w_down, &out};
    const int at[5] = {ROUTE, X, WGU, WDN, OUT};
    for (int i = 0; i < 5; i++) {
        char* p = nullptr;
        int rc = resolve(g, *r[i], &p, &size[at[i]]);
        if (rc) return rc;
        ptr[at[i]] = p;
    }
    return moe_experts_run(g, kernels, swiglu, combine, ptr, size, m);
}
