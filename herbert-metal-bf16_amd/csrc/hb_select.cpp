// hb_select.cpp -- placeholder until the selection layer lands.
#include "hb_internal.h"
using namespace hb;
struct hb_engine { hb_gpu* gpu; };
extern "C" {
int hb_engine_open(hb_gpu*, const char*, hb_engine** e) { *e = nullptr; return fail(HB_ERR_UNSUPPORTED, "engine"); }
void hb_engine_close(hb_engine*) {}
const char* hb_engine_tune_summary(hb_engine*) { return ""; }
int hb_engine_buckets(hb_engine*, uint32_t*, uint32_t, uint32_t*) { return HB_ERR_UNSUPPORTED; }
int hb_engine_gemm(hb_engine*, uint32_t, uint32_t, uint32_t, hb_range, hb_range, hb_range, hb_range, uint32_t, int32_t*) { return HB_ERR_UNSUPPORTED; }
int hb_engine_matvec(hb_engine*, uint32_t, uint32_t, uint32_t, uint32_t, const hb_range*, uint32_t, hb_range, hb_range, int32_t*) { return HB_ERR_UNSUPPORTED; }
int hb_engine_experts(hb_engine*, uint32_t, uint32_t, uint32_t, uint32_t, uint32_t, const hb_moe_io*, int32_t*, uint32_t*) { return HB_ERR_UNSUPPORTED; }
double hb_engine_autotune_seconds(hb_engine*) { return 0; }
}
