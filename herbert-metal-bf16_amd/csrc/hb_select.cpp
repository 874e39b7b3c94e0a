// hb_select.cpp -- the kernel-selection part of the reference's QwenEngine,
// over this library's kernels: the --tune settings (Tune::apply / summary),
// the shape-keyed GEMM choice with its candidates checked against the first
// one and timed (gemm, check_candidates, pick_flagged), the decode matvec's
// form (mv_full) and the MoE layer's sort / grouped GEMMs / tile rows
// (expert_pipes), with the reference's [autotune] log lines.
//
// Reference: src/metal/qwen.rs:62-398 (Tune), :1051-1063 (buckets),
// :1311-1511 (mv_full), :2200-2325 (gemm), :2326-2391 (expert_pipes),
// :2483-2628 (pick, check_candidates, pick_flagged, heat, time_ops).
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <sstream>

#include "hb_internal.h"

using namespace hb;

namespace {

// ---- Tune (qwen.rs:62-398) ----

// Every key of the reference's --tune, with its default, in the order of
// Tune::summary.  The keys of this path act (prefill.block, gemm.*, moe.*,
// mv.*, auto.heat, pf.fswi); the others are accepted and echoed, as the
// reference's subsystems they name (attention, DeltaNet, decode fusions, Q4)
// are not part of this library.
struct Key {
    const char* name;
    uint32_t def;
};
const Key kKeys[] = {
    {"prefill.block", 2048}, {"rec.chunk", 3},   {"rec.pcols", 16},  {"rec.pslices", 16},
    {"rec.vec", 0},          {"rec.pair", 0},    {"rec.stage", 0},   {"conv.cols", 32},
    {"sdpa.prefill", 1},     {"sdpa.bq", 16},    {"sdpa.bk", 16},    {"sdpa.mq", 0},
    {"sdpa.mk", 32},         {"sdpa.qreg", 0},   {"sdpa.kt", 0},     {"sdpa.msg", 8},
    {"sdpa.auto", 1},        {"auto.heat", 0},   {"gemm.simt", 1},   {"gemm.auto", 1},
    {"gemm.mma", 1},         {"gemm.tn", 64},    {"gemm.mform", 0},  {"gemm.half", 1},
    {"gemm.mfirst", 1},      {"moe.grouped", 1}, {"moe.tile", 16},   {"q4.fuse", 0},
    {"mv.auto", 1},          {"mv.masks", 0},    {"mv.split", 1},    {"mv.splitauto", 1},
    {"mv.persist", 0},       {"mv.persists", 0}, {"dec.sdpa", 32},   {"mv.cold", 1},
    {"dec.swiglu", 0},       {"dec.prep", 0},    {"dec.conc", 0},    {"dec.pf", 0},
    {"dec.pfk", 0},          {"dec.auto", 1},    {"dec.gnorm", 0},   {"dec.pfdn", 0},
    {"dec.fnorm", 0},        {"dec.fswi", 0},    {"pf.fswi", 2},     {"dec.fdn", 0},
    {"dec.frope", 0},        {"dec.rec", 1},     {"dec.cols", 16},   {"dec.slices", 16},
    {"dn.sscale", 0},        {"dn.oscale", 0},   {"dn.tscale", 0},
};

struct Tune {
    std::map<std::string, uint32_t> v;
    std::vector<uint32_t> mv_persists;
    std::vector<std::string> given;
    bool block_set = false, gemm_set = false, moe_tile_set = false, sdpa_set = false;

    Tune() {
        for (const auto& k : kKeys) v[k.name] = k.def;
    }
    uint32_t operator[](const char* k) const { return v.at(k); }

    // Rust's u32::from_str errors, as `--tune {kv}: {e}` prints them.
    static bool parse_u32(const std::string& s, uint32_t* out, std::string* err) {
        if (s.empty()) {
            *err = "cannot parse integer from empty string";
            return false;
        }
        uint64_t n = 0;
        size_t i = s[0] == '+' ? 1 : 0;
        if (i == s.size()) {
            *err = "invalid digit found in string";
            return false;
        }
        for (; i < s.size(); i++) {
            if (s[i] < '0' || s[i] > '9') {
                *err = "invalid digit found in string";
                return false;
            }
            n = n * 10 + (uint64_t)(s[i] - '0');
            if (n > 0xffffffffull) {
                *err = "number too large to fit in target type";
                return false;
            }
        }
        *out = (uint32_t)n;
        return true;
    }

    // Tune::apply (qwen.rs:296-389): "key=value" settings, comma separated.
    bool apply(const std::string& list, std::string* err) {
        std::stringstream ss(list);
        std::string kv;
        while (std::getline(ss, kv, ',')) {
            if (kv.empty()) continue;
            size_t eq = kv.find('=');
            if (eq == std::string::npos) {
                *err = "--tune " + kv + ": key=value";
                return false;
            }
            std::string key = kv.substr(0, eq), value = kv.substr(eq + 1);
            given.push_back(key);
            if (key == "mv.persists") {
                mv_persists.clear();
                std::stringstream vs(value);
                std::string item;
                while (std::getline(vs, item, '/')) {
                    if (item.empty()) continue;
                    uint32_t n;
                    std::string e;
                    if (!parse_u32(item, &n, &e)) {
                        *err = "--tune " + kv + ": " + e;
                        return false;
                    }
                    mv_persists.push_back(n);
                }
                continue;
            }
            uint32_t n;
            std::string e;
            if (!parse_u32(value, &n, &e)) {
                *err = "--tune " + kv + ": " + e;
                return false;
            }
            if (!v.count(key)) {
                *err = "--tune " + key + ": unknown";
                return false;
            }
            if (key == "prefill.block") {
                v[key] = std::max<uint32_t>(n, 1);
                block_set = true;
            } else if (key == "sdpa.prefill") {
                v[key] = n;
                sdpa_set = true;
            } else if (key == "gemm.mma" || key == "gemm.tn" || key == "gemm.mform" ||
                       key == "q4.fuse") {
                v[key] = n;
                gemm_set = true;
            } else if (key == "moe.tile") {
                v[key] = n;
                moe_tile_set = true;
            } else if (key == "mv.masks" || key == "mv.split" || key == "mv.persist") {
                v[key] = n;
                v["mv.auto"] = 0;
            } else if (key == "dec.sdpa") {
                v[key] = std::min<uint32_t>(n, 64);
            } else {
                v[key] = n;
            }
        }
        return validate(err);
    }

    uint32_t mq() const {
        if ((*this)["sdpa.mq"]) return (*this)["sdpa.mq"];
        return (*this)["sdpa.prefill"] >= 4 ? 64 : 16;
    }

    std::string brief() const {
        char b[160];
        snprintf(b, sizeof b, "rec.chunk=%u sdpa.prefill=%u gemm.simt=%u", (*this)["rec.chunk"],
                 (*this)["sdpa.prefill"], (*this)["gemm.simt"]);
        return b;
    }

    // The checks of Tune::apply (qwen.rs:367-388) that concern settings this
    // library reads or that the reference refuses outright.
    bool validate(std::string* err) const {
        char b[256];
        const Tune& t = *this;
        if (t["q4.fuse"] > 1 || (t["q4.fuse"] == 1 && t["gemm.mma"] != 1)) {
            snprintf(b, sizeof b, "--tune q4.fuse=%u: 0, or 1 with gemm.mma=1", t["q4.fuse"]);
            *err = b;
            return false;
        }
        uint32_t mma = t["gemm.mma"], tn = t["gemm.tn"];
        bool tn_ok = tn == 16 || tn == 32 || tn == 64 || (mma == 3 && tn == 128);
        if (mma > 3 || !tn_ok || t["gemm.mform"] > 9) {
            snprintf(b, sizeof b,
                     "--tune gemm.mma=%u gemm.tn=%u gemm.mform=%u: gemm.mma 0..2, gemm.tn 16, 32 "
                     "or 64, gemm.mform 0..9",
                     mma, tn, t["gemm.mform"]);
            *err = b;
            return false;
        }
        uint32_t mt = t["moe.tile"];
        if (mt != 16 && mt != 32 && mt != 64) {
            snprintf(b, sizeof b, "--tune moe.tile=%u: 16, 32 or 64", mt);
            *err = b;
            return false;
        }
        if (t["rec.chunk"] > 4 || t["sdpa.prefill"] > 7 || t["gemm.simt"] < 1 || t["gemm.simt"] > 2) {
            *err = "--tune: rec.chunk 0..4, sdpa.prefill 0..7, gemm.simt 1..2 (" + brief() + ")";
            return false;
        }
        uint32_t mk = t["sdpa.mk"];
        if (t["sdpa.prefill"] >= 2 && (t["sdpa.mq"] % 8 != 0 || !(mk == 8 || mk == 16 || mk == 32 || mk == 64) ||
                                       t["prefill.block"] % mq() != 0)) {
            *err = "--tune sdpa.prefill=2|3|4: sdpa.mq a multiple of 8 dividing prefill.block, "
                   "sdpa.mk 8, 16, 32 or 64 (" + brief() + ")";
            return false;
        }
        return true;
    }

    // Tune::summary (qwen.rs:391-398), same keys and order.
    std::string summary() const {
        std::string s;
        for (const auto& k : kKeys) {
            std::string name = k.name;
            uint32_t val = v.at(name);
            if (name == "sdpa.auto") val = (val && !sdpa_set) ? 1 : 0;
            if (name == "gemm.auto") val = (val && !gemm_set) ? 1 : 0;
            if (!s.empty()) s += " ";
            if (name == "mv.persists") {
                s += "mv.persists=[";
                for (size_t i = 0; i < mv_persists.size(); i++)
                    s += (i ? ", " : "") + std::to_string(mv_persists[i]);
                s += "]";
            } else {
                s += name + "=" + std::to_string(val);
            }
        }
        return s;
    }
};

// The dense GEMM candidates of this library, in candidate order: the first
// is the production kernel every other is checked against.  gemm.mform
// indexes this table (gemm.mma=1).
struct Form {
    const char* name;
    uint32_t bm, bn, bk, wm, wn, mfma, dbuf, dma, order, band, sched, ksplit;
};
const Form kForms[10] = {
    {"mma", 128, 128, 64, 2, 2, 16, 1, 1, 1},
    {"mma_x32", 128, 128, 64, 2, 2, 32, 1, 1, 1},
    {"mma_t256", 256, 256, 64, 2, 2, 32, 1, 1, 1},
    {"mma_t256_w8", 256, 256, 32, 4, 2, 32, 3, 1, 1},
    {"mma_t128x256", 128, 256, 32, 2, 2, 32, 3, 1, 1},
    {"mma_t256x128", 256, 128, 32, 2, 2, 32, 3, 1, 1},
    {"mma_s4", 128, 128, 64, 2, 2, 16, 3, 1, 1},
    {"mma_k32_s4", 128, 128, 32, 2, 2, 16, 3, 1, 1},
    {"mma_reg", 128, 128, 64, 2, 2, 16, 1, 0, 0},
    {"mma_t64", 64, 64, 32, 1, 4, 16, 0, 0, 0},
};
// Timed with the table but not named by gemm.mform: tiles whose counts
// fill whole rounds of the 256 CUs on this build's shapes (256 x 192:
// 768 tiles at 2048 x 18432; 128 x 160: 256 at 2048 x 2560; 128 x 192:
// 224 at 2048 x 2560, 8 wavefronts), three and four stages of 64 K for the
// long-K shapes, and the band tile order of gemm_nax (prefill.rs:615-631):
// with bands of 4 row tiles each XCD's 32 concurrent 256 x 192 tiles are 4
// row tiles by 8 column tiles, fewer compulsory L2 misses than 8 by 4.
const Form kMoreForms[] = {
    {"mma_t256x192_w8", 256, 192, 64, 4, 2, 32, 1, 1, 1},
    {"mma_t256x192_w8_x16", 256, 192, 64, 4, 2, 16, 1, 1, 1},
    {"mma_t256x192_w8_x16_b4", 256, 192, 64, 4, 2, 16, 1, 1, 1, 4},
    {"mma_t256_w8_x32_b4", 256, 256, 64, 4, 2, 32, 1, 1, 1, 4},
    {"mma_t128x160", 128, 160, 64, 2, 2, 16, 1, 1, 1},
    {"mma_t128x160_s4", 128, 160, 64, 2, 2, 16, 3, 1, 0},
    {"mma_t128x192_w8_s3", 128, 192, 64, 2, 4, 16, 2, 1, 0},
    {"mma_t128x192_w8_s4", 128, 192, 64, 2, 4, 16, 3, 1, 0},
    {"mma_t128x192_w8_s4_b2", 128, 192, 64, 2, 4, 16, 3, 1, 0, 2},
    {"mma_t128x192_w8_s4_o1_b4", 128, 192, 64, 2, 4, 16, 3, 1, 1, 4},
    {"mma_t128x160_s4_o1_b4", 128, 160, 64, 2, 2, 16, 3, 1, 1, 4},
    {"mma_t256x128_w8_s3", 256, 128, 64, 4, 2, 16, 2, 1, 1},
    {"mma_b2", 128, 128, 64, 2, 2, 16, 1, 1, 0, 2},
    // Small tiles for narrow outputs (the MoE router's 256 columns, the
    // shared expert): enough tiles to reach every CU.
    {"mma_t64x128", 64, 128, 64, 2, 2, 16, 2, 1, 1},
    // Four stages for the short-K, few-tile shapes (config 1: 448 tiles of
    // 64 x 128 over K = 1024; 8.4 -> 6.6-7.0 us against the 3-stage 64 x 64).
    {"mma_t64x128_s4", 64, 128, 64, 2, 2, 16, 3, 1, 1},
    {"mma_t64x128_s4_w8", 64, 128, 64, 2, 4, 16, 3, 1, 1},
    {"mma_t128x64_s4_w8", 128, 64, 64, 4, 2, 16, 3, 1, 1},
    {"mma_t64x64", 64, 64, 64, 2, 2, 16, 2, 1, 1},
    {"mma_t32x64", 32, 64, 64, 1, 4, 16, 2, 1, 1},
    // Eight waves in two groups taking turns between memory and MFMA phases
    // (hb_desc.sched 1), four stages of 32 K: 256 x 288 tiles fill exactly
    // two rounds of the CUs on 2048 x 18432 (and 4608: 128 tiles).
    {"pp_t256x288", 256, 288, 32, 4, 2, 16, 3, 1, 1, 0, 1},
    {"pp_t256x288_b4", 256, 288, 32, 4, 2, 16, 3, 1, 1, 4, 1},
    {"pp_t256x256_b4", 256, 256, 32, 4, 2, 16, 3, 1, 1, 4, 1},
    {"pp_t256x256", 256, 256, 32, 4, 2, 16, 3, 1, 1, 0, 1},
    {"pp_t256x192", 256, 192, 32, 4, 2, 16, 3, 1, 1, 0, 1},
    {"pp_t256x128", 256, 128, 32, 4, 2, 16, 3, 1, 1, 0, 1},
    {"pp_t128x256", 128, 256, 32, 2, 4, 16, 3, 1, 1, 0, 1},
    {"pp_t128x128", 128, 128, 32, 2, 4, 16, 3, 1, 1, 0, 1},
    // One round of tiles on the narrower layer shapes: 256 x 160 on 2048 x
    // 4608 (232 tiles), 128 x 160 on 2048 x 2560 (256), three or four
    // stages of 64 K (longer MFMA phases than 32 K at these wave tiles).
    {"pp_t256x160_k64", 256, 160, 64, 4, 2, 16, 2, 1, 1, 0, 1},
    {"pp_t256x160_k64_b2", 256, 160, 64, 4, 2, 16, 2, 1, 1, 2, 1},
    {"pp_t256x160_k64_b4", 256, 160, 64, 4, 2, 16, 2, 1, 1, 4, 1},
    {"pp_t128x160_k64", 128, 160, 64, 4, 2, 16, 3, 1, 1, 0, 1},
    {"pp_t128x160_k64_b4", 128, 160, 64, 4, 2, 16, 3, 1, 1, 4, 1},
    {"pp_t128x288_k64", 128, 288, 64, 4, 2, 16, 2, 1, 1, 0, 1},
};
// Split K (hb_desc.ksplit) for the shapes whose tiles fill less than a
// round of the 256 CUs (M = 512 and 1024, and the narrow N = 2560 outputs
// at 2048): s workgroups per tile, each over K/s, the f32 parts added by a
// second kernel.  Forms whose K/s is not a whole count of K tiles are not
// built for that shape.
const Form kSplitForms[] = {
    {"mma_t128x160_s4_ks2", 128, 160, 64, 2, 2, 16, 3, 1, 1, 0, 0, 2},
    {"mma_t128x160_s4_ks3", 128, 160, 64, 2, 2, 16, 3, 1, 1, 0, 0, 3},
    {"mma_t128x160_s4_ks4", 128, 160, 64, 2, 2, 16, 3, 1, 1, 0, 0, 4},
    {"mma_t128x192_w8_s4_ks2", 128, 192, 64, 2, 4, 16, 3, 1, 1, 0, 0, 2},
    {"mma_t128x192_w8_s4_ks4", 128, 192, 64, 2, 4, 16, 3, 1, 1, 0, 0, 4},
    {"mma_t128x192_w8_s4_ks8", 128, 192, 64, 2, 4, 16, 3, 1, 1, 0, 0, 8},
    {"pp_t256x160_k64_ks2", 256, 160, 64, 4, 2, 16, 2, 1, 1, 0, 1, 2},
    {"pp_t256x160_k64_ks4", 256, 160, 64, 4, 2, 16, 2, 1, 1, 0, 1, 4},
    {"pp_t128x160_k64_ks2", 128, 160, 64, 4, 2, 16, 3, 1, 1, 0, 1, 2},
    {"pp_t128x160_k64_ks4", 128, 160, 64, 4, 2, 16, 3, 1, 1, 0, 1, 4},
    {"pp_t128x256_ks2", 128, 256, 32, 2, 4, 16, 3, 1, 1, 0, 1, 2},
    {"pp_t128x256_ks4", 128, 256, 32, 2, 4, 16, 3, 1, 1, 0, 1, 4},
    {"pp_t256x256_ks2", 256, 256, 32, 4, 2, 16, 3, 1, 1, 0, 1, 2},
    {"pp_t256x256_ks4", 256, 256, 32, 4, 2, 16, 3, 1, 1, 0, 1, 4},
};
// The fused [gate | up] + SwiGLU forms (gate_up_pipes, qwen.rs:2148-2193):
// bn W rows per tile = bn/2 features.
const Form kFusedForms[] = {
    {"fused128x64", 128, 128, 64, 2, 2, 16, 1, 1, 1},
    {"fused128x64b2", 128, 128, 64, 2, 2, 16, 1, 1, 0, 2},
    {"fused256x96", 256, 192, 64, 4, 2, 16, 1, 1, 1},
    {"fused256x128", 256, 256, 64, 4, 2, 32, 1, 1, 1},
};

hb_desc form_desc(const Form& f, uint32_t k, uint32_t n, uint32_t out, bool mf) {
    hb_desc d{};
    d.kind = HB_KIND_GEMM;
    d.k = k;
    d.n = n;
    d.out = out;
    d.rows_of = HB_ROWS_DENSE;
    d.m_first = mf;
    d.bm = f.bm;
    d.bn = f.bn;
    d.bk = f.bk;
    d.wm = f.wm;
    d.wn = f.wn;
    d.mfma = f.mfma;
    d.dbuf = f.dbuf;
    d.lds_dma = f.dma;
    d.order = f.order;
    d.band = f.band;
    d.sched = f.sched;
    d.ksplit = f.ksplit;
    return d;
}

hb_desc mm2d_desc(uint32_t k, uint32_t n, uint32_t out, bool mf, uint32_t tm, uint32_t tn) {
    hb_desc d{};
    d.kind = HB_KIND_GEMM_DIRECT;
    d.k = k;
    d.n = n;
    d.out = out;
    d.m_first = mf;
    d.bm = tm;
    d.bn = tn;
    return d;
}

const char* out_name(uint32_t out) {
    return out == HB_OUT_F32 ? "F32" : out == HB_OUT_RESIDUAL ? "Residual" : out == HB_OUT_SWIGLU ? "Swiglu" : "Bf16";
}

struct Cand {
    std::string name;
    int32_t kernel;
    std::vector<hb_op> ops;
};

hb_op make_op(int32_t kernel, uint32_t m, std::initializer_list<hb_range> b) {
    hb_op op{};
    op.kernel = kernel;
    op.m = m;
    op.nbind = 0;
    for (const auto& r : b) op.bind[op.nbind++] = r;
    return op;
}

hb_op make_op(int32_t kernel, uint32_t m, const std::vector<hb_range>& b) {
    hb_op op{};
    op.kernel = kernel;
    op.m = m;
    op.nbind = 0;
    for (const auto& r : b) op.bind[op.nbind++] = r;
    return op;
}

}  // namespace

struct hb_engine {
    hb_gpu* g = nullptr;
    Tune t;
    std::string tune_summary, log;
    std::map<std::string, int32_t> gemm_pick;
    std::map<std::string, std::pair<int32_t, int32_t>> gate_up_pick;
    std::map<std::string, hb_desc> mv_pick;
    struct ExpertsPick {
        int32_t kernels[4];
        uint32_t bm;
    };
    std::map<std::string, ExpertsPick> experts_pick;
    std::vector<std::pair<std::string, hb_desc>> extra;  // hb_engine_add_gemm_candidate
    double autotune_seconds = 0.0;
    bool timed = false;
    std::chrono::steady_clock::time_point last_timed;

    void logf(const char* fmt, ...) {
        char buf[8192];
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(buf, sizeof buf, fmt, ap);
        va_end(ap);
        fprintf(stderr, "%s\n", buf);
        log += buf;
        log += "\n";
    }

    // time_ops (qwen.rs:2593).
    int time_ops(const std::vector<hb_op>& ops, uint32_t reps, double* s) {
        return hb_time(g, ops.data(), (uint32_t)ops.size(), reps, s);
    }

    // heat (qwen.rs:2577-2591): auto.heat ms of load after > 200 ms idle.
    int heat(const std::vector<hb_op>& ops) {
        double heat_s = t["auto.heat"] * 1e-3;
        if (heat_s <= 0 ||
            (timed && std::chrono::duration<double>(std::chrono::steady_clock::now() - last_timed).count() < 0.2))
            return HB_OK;
        double one;
        int rc = time_ops(ops, 1, &one);
        if (rc) return rc;
        uint32_t reps = (uint32_t)std::min(256.0, std::max(1.0, std::ceil(0.05 / std::max(one, 1e-6))));
        double total = 0;
        while (total < heat_s) {
            double s;
            if ((rc = time_ops(ops, reps, &s))) return rc;
            total += s;
        }
        timed = true;
        last_timed = std::chrono::steady_clock::now();
        return HB_OK;
    }

    // The op that evicts the last-level cache: a SwiGLU pass reading 256 MiB
    // and writing 128 MiB of the context's flush buffers.
    int flush_op(hb_op* op) {
        constexpr uint32_t F = 8192;
        int rc;
        if (g->flush_kernel < 0) {
            hb_desc d{};
            d.kind = HB_KIND_SWIGLU;
            d.n = F;
            int32_t k;
            if ((rc = build(d, &k))) return rc;
            if ((rc = hb_alloc(g, (uint64_t)F * 2 * F * 2, &g->flush_gu)) ||
                (rc = hb_alloc(g, (uint64_t)F * F * 2, &g->flush_h)) ||
                (rc = hb_zero(g, g->flush_gu, 0, (uint64_t)F * 2 * F * 2)))
                return rc;
            g->flush_kernel = k;
        }
        *op = make_op(g->flush_kernel, F, {hb_range{g->flush_gu, 0, 0, 0}, hb_range{g->flush_h, 0, 0, 0}});
        return HB_OK;
    }

    // GPU seconds of `reps` runs of `ops`; cold: each run after the cache
    // flush, only the ops' own launches counted (an event after each
    // launch), so the weights come from HBM as in a layer step.
    int run_ops(const std::vector<hb_op>& ops, uint32_t reps, bool cold, double* s) {
        if (!cold) return time_ops(ops, reps, s);
        std::vector<hb_op> seq(1);
        int rc = flush_op(&seq[0]);
        if (rc) return rc;
        seq.insert(seq.end(), ops.begin(), ops.end());
        std::vector<double> each(seq.size());
        double total;
        if ((rc = hb_time_each(g, seq.data(), (uint32_t)seq.size(), reps, &total, each.data()))) return rc;
        *s = 0;
        for (size_t i = 1; i < seq.size(); i++) *s += each[i] * reps;
        return HB_OK;
    }

    // pick_flagged (qwen.rs:2547-2575): reps so one run lasts ~2 ms, five
    // interleaved rounds, medians, the fastest eligible kept; logged with
    // `*` after the ineligible.  cold (the dense GEMMs): every run after the
    // cache flush -- MI355X's 256 MiB last-level cache would otherwise hold
    // a candidate's W and X between its own runs, which a layer step never
    // sees, and the ranking of warm runs is not the ranking in the step.
    int pick_flagged(const std::string& what, const std::vector<Cand>& c,
                     const std::vector<bool>& eligible, size_t* best, double* best_s,
                     bool cold = false) {
        auto t0 = std::chrono::steady_clock::now();
        if (c.empty() || std::none_of(eligible.begin(), eligible.end(), [](bool e) { return e; }))
            return fail(HB_ERR_INVALID, what + ": no eligible candidate");
        int rc = heat(c[0].ops);
        double one;
        if (rc || (rc = run_ops(c[0].ops, 1, cold, &one)) || (rc = run_ops(c[0].ops, 1, cold, &one)))
            return rc;
        uint32_t reps = (uint32_t)std::min(64.0, std::max(1.0, std::ceil(2e-3 / std::max(one, 1e-6))));
        std::vector<std::vector<double>> times(c.size());
        for (int round = 0; round < 5; round++)
            for (size_t i = 0; i < c.size(); i++) {
                double s;
                if ((rc = run_ops(c[i].ops, reps, cold, &s))) return rc;
                times[i].push_back(s / reps);
            }
        std::vector<double> med(c.size());
        for (size_t i = 0; i < c.size(); i++) {
            std::sort(times[i].begin(), times[i].end());
            med[i] = times[i][times[i].size() / 2];
        }
        size_t b = c.size();
        for (size_t i = 0; i < c.size(); i++)
            if (eligible[i] && (b == c.size() || med[i] < med[b])) b = i;
        std::string line;
        for (size_t i = 0; i < c.size(); i++) {
            char buf[256];
            snprintf(buf, sizeof buf, "%s%s%s %.3f ms", i ? ", " : "", c[i].name.c_str(),
                     eligible[i] ? "" : "*", med[i] * 1e3);
            line += buf;
        }
        logf("[autotune] %s: %s -> %s", what.c_str(), line.c_str(), c[b].name.c_str());
        autotune_seconds += std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
        timed = true;
        last_timed = std::chrono::steady_clock::now();
        *best = b;
        if (best_s) *best_s = med[b];
        return HB_OK;
    }

    // check_candidates (qwen.rs:2497-2545): each candidate on the full block
    // and on m - m/3 - 3 rows from a zeroed output, against candidate 0; an
    // error beyond max|ref|/64 marks it wrong, logged, never picked.  The
    // output and state[3] are restored.
    int check_candidates(const std::string& what, std::vector<Cand>& c,
                         std::vector<bool>& eligible, hb_range state, hb_range out,
                         bool f32_out, uint32_t m, uint32_t row_bytes) {
        char* optr;
        uint64_t osize;
        int rc = resolve(g, out, &optr, &osize);
        if (rc) return rc;
        std::vector<char> before(osize);
        if ((rc = hb_download(g, out.buf, out.offset, before.data(), osize))) return rc;
        std::vector<std::string> wrong;
        for (uint32_t rows : {m, std::max<uint32_t>(m - m / 3 - 3, 1)}) {
            if (rows > m) rows = 1;
            uint32_t st[4] = {0, 0, 0, rows};
            if ((rc = hb_upload(g, state.buf, state.offset, st, 16))) return rc;
            uint64_t used = std::min<uint64_t>((uint64_t)rows * row_bytes, osize);
            auto values = [&](std::vector<float>* v) -> int {
                std::vector<char> raw(used);
                int r2 = hb_download(g, out.buf, out.offset, raw.data(), used);
                if (r2) return r2;
                if (f32_out) {
                    v->resize(used / 4);
                    memcpy(v->data(), raw.data(), used / 4 * 4);
                } else {
                    v->resize(used / 2);
                    for (size_t i = 0; i < v->size(); i++) {
                        uint32_t b = (uint32_t)((uint16_t*)raw.data())[i] << 16;
                        memcpy(&(*v)[i], &b, 4);
                    }
                }
                return HB_OK;
            };
            auto run = [&](size_t i) -> int {
                int r2 = hb_zero(g, out.buf, out.offset, osize);
                if (r2) return r2;
                std::vector<hb_op> ops = c[i].ops;
                for (auto& op : ops) op.m = rows;
                double s;
                return time_ops(ops, 1, &s);
            };
            std::vector<float> ref, got;
            if ((rc = run(0)) || (rc = values(&ref))) return rc;
            float scale = 1e-6f;
            for (float x : ref) scale = std::max(scale, std::fabs(x));
            for (size_t i = 1; i < c.size(); i++) {
                if (!eligible[i]) continue;
                if ((rc = run(i)) || (rc = values(&got))) return rc;
                float err = 0;
                for (size_t j = 0; j < ref.size(); j++) {
                    float e = std::fabs(ref[j] - got[j]);
                    if (!(e <= err)) err = e;  // NaN propagates as "wrong"
                }
                if (!(err <= scale / 64)) {
                    eligible[i] = false;
                    char buf[256];
                    snprintf(buf, sizeof buf, "%s (%u rows: max err %.3e of %.3e)", c[i].name.c_str(),
                             rows, err, scale);
                    wrong.push_back(buf);
                }
            }
        }
        if ((rc = hb_upload(g, out.buf, out.offset, before.data(), osize))) return rc;
        uint32_t st[4] = {0, 0, 0, m};
        if ((rc = hb_upload(g, state.buf, state.offset, st, 16))) return rc;
        if (!wrong.empty()) {
            std::string l;
            for (size_t i = 0; i < wrong.size(); i++) l += (i ? ", " : "") + wrong[i];
            logf("[autotune] %s: wrong against %s, never picked: %s", what.c_str(), c[0].name.c_str(),
                 l.c_str());
        }
        return HB_OK;
    }

    int build(const hb_desc& d, int32_t* k) { return hb_kernel_build(g, &d, k); }
};

extern "C" {

int hb_engine_open(hb_gpu* g, const char* tune, hb_engine** out) {
    *out = nullptr;
    // No context: a host-only engine (the --tune table, the log and the
    // host-driven autotune_chunk); the kernel selections refuse.
    hb_engine* e = new hb_engine();
    e->g = g;
    std::string err;
    if (tune && !e->t.apply(tune, &err)) {
        delete e;
        return fail(HB_ERR_INVALID, err);
    }
    e->tune_summary = e->t.summary();
    *out = e;
    return HB_OK;
}

void hb_engine_close(hb_engine* e) { delete e; }

const char* hb_engine_tune_summary(hb_engine* e) { return e->tune_summary.c_str(); }

const char* hb_engine_log(hb_engine* e) { return e->log.c_str(); }

double hb_engine_autotune_seconds(hb_engine* e) { return e->autotune_seconds; }

int hb_engine_tune_get(hb_engine* e, const char* key, uint32_t* value) {
    auto it = e->t.v.find(key ? key : "");
    if (it == e->t.v.end()) return fail(HB_ERR_INVALID, std::string("--tune: unknown key ") + (key ? key : ""));
    *value = it->second;
    return HB_OK;
}

int hb_engine_log_line(hb_engine* e, const char* line, double seconds) {
    e->logf("%s", line ? line : "");
    e->autotune_seconds += seconds;
    return HB_OK;
}

int hb_tune_check(const char* tune, char* summary, uint64_t cap) {
    Tune t;
    std::string err;
    if (tune && !t.apply(tune, &err)) return fail(HB_ERR_INVALID, err);
    std::string s = t.summary();
    if (summary && cap) {
        size_t n = std::min<size_t>(s.size(), cap - 1);
        memcpy(summary, s.data(), n);
        summary[n] = 0;
    }
    return HB_OK;
}

int hb_engine_buckets(hb_engine* e, uint32_t* out, uint32_t cap, uint32_t* count) {
    // qwen.rs:1051-1063: m in {64, 128, 256, ...} below prefill.block, then it.
    std::vector<uint32_t> b;
    uint32_t block = e->t["prefill.block"];
    for (uint32_t m = 64; m < block; m *= 2) b.push_back(m);
    b.push_back(block);
    *count = (uint32_t)b.size();
    for (uint32_t i = 0; i < b.size() && i < cap; i++) out[i] = b[i];
    return HB_OK;
}

int hb_engine_add_gemm_candidate(hb_engine* e, const char* name, const hb_desc* desc) {
    e->extra.emplace_back(name ? name : "extra", *desc);
    return HB_OK;
}

int hb_engine_log_summary(hb_engine* e) {
    if (!e->g) return fail(HB_ERR_INVALID, "log_summary: an engine without a context");
    e->logf("[hip] %zu kernels compiled in %.1f s, GEMMs and blocks timed in %.1f s",
            e->g->kernels.size(), e->g->compile_seconds, e->autotune_seconds);
    return HB_OK;
}

// The dense GEMM candidates of QwenEngine::gemm's timed choice, in order
// (qwen.rs:2200-2325): the gemm.mform table (its first the production
// kernel every other is checked against), the further tile forms, the
// direct MFMA forms (gemm_mm2d), then candidates a caller added.
std::vector<std::pair<std::string, hb_desc>> gemm_candidates(hb_engine* e, uint32_t k, uint32_t n,
                                                             uint32_t out, bool mf) {
    std::vector<std::pair<std::string, hb_desc>> v;
    for (const auto& f : kForms) v.emplace_back(f.name, form_desc(f, k, n, out, mf));
    for (const auto& f : kMoreForms) v.emplace_back(f.name, form_desc(f, k, n, out, mf));
    for (const auto& f : kSplitForms)
        if (k % (f.bk * f.ksplit) == 0) v.emplace_back(f.name, form_desc(f, k, n, out, mf));
    for (auto tm_tn : {std::make_pair(64u, 64u), std::make_pair(64u, 32u), std::make_pair(32u, 64u),
                       std::make_pair(32u, 32u), std::make_pair(64u, 16u), std::make_pair(32u, 16u)}) {
        char nm[32];
        snprintf(nm, sizeof nm, "mm2d%ux%u", tm_tn.first, tm_tn.second);
        v.emplace_back(nm, mm2d_desc(k, n, out, mf, tm_tn.first, tm_tn.second));
    }
    for (const auto& ex : e->extra) v.push_back(ex);
    return v;
}

int hb_engine_gemm_candidates(hb_engine* e, uint32_t k, uint32_t n, uint32_t out, hb_desc* descs,
                              uint32_t cap, uint32_t* count) {
    const auto v = gemm_candidates(e, k, n, out, e->t["gemm.mfirst"] != 0);
    *count = (uint32_t)v.size();
    for (uint32_t i = 0; i < v.size() && i < cap; i++) descs[i] = v[i].second;
    return HB_OK;
}

int hb_engine_gemm(hb_engine* e, uint32_t k, uint32_t n, uint32_t out, hb_range state,
                   hb_range w, hb_range x, hb_range y, uint32_t m, int32_t* kernel) {
    if (!e->g) return fail(HB_ERR_INVALID, "gemm: an engine without a context");
    const Tune& t = e->t;
    bool mf = t["gemm.mfirst"] != 0;
    int rc;
    if (!t["gemm.auto"] || t.gemm_set) {
        // The kernel gemm.mma / gemm.tn / gemm.mform name, nothing timed.
        hb_desc d{};
        switch (t["gemm.mma"]) {
            case 0:
                d.kind = HB_KIND_GEMM_SIMT;
                d.k = k;
                d.n = n;
                d.out = out;
                d.m_first = mf;
                break;
            case 2: d = mm2d_desc(k, n, out, mf, 64, t["gemm.tn"]); break;
            case 3: d = form_desc(kForms[3], k, n, out, mf); break;
            default: d = form_desc(kForms[t["gemm.mform"]], k, n, out, mf); break;
        }
        return e->build(d, kernel);
    }
    char key[128];
    snprintf(key, sizeof key, "%ux%u %s, %u rows", k, n, out_name(out), m);
    auto it = e->gemm_pick.find(key);
    if (it != e->gemm_pick.end()) {
        *kernel = it->second;
        return HB_OK;
    }
    std::string what = std::string("gemm ") + key;
    std::vector<Cand> c;
    std::vector<bool> eligible;
    // Operands past 2 GiB: the direct-to-LDS forms cannot address them (their
    // buffer resources span 2^31 - 1 bytes); the others run, the first of
    // them the reference of the check.
    const bool big = (uint64_t)n * k * 2 > 0x7fffffffull || (uint64_t)m * k * 2 > 0x7fffffffull;
    auto add = [&](const std::string& name, const hb_desc& d) {
        if (big && d.kind == HB_KIND_GEMM && d.lds_dma) {
            e->logf("[autotune] gemm %s: %s skipped (operands past 2 GiB)", key, name.c_str());
            return;
        }
        int32_t kk;
        int r = e->build(d, &kk);
        if (r) {
            e->logf("[autotune] gemm %s: %s not built (%s)", key, name.c_str(), hb_last_error());
            return;
        }
        c.push_back({name, kk, {make_op(kk, m, {state, w, x, y, state, state})}});
        eligible.push_back(true);
    };
    const auto list = gemm_candidates(e, k, n, out, mf);
    for (size_t i = 0; i < list.size(); i++) {
        add(list[i].first, list[i].second);
        if (i + 1 == sizeof kForms / sizeof kForms[0] && (c.empty() || (!big && c[0].name != "mma")))
            return fail(HB_ERR_COMPILE, what + ": the production kernel mma is not built: " + hb_last_error());
    }
    uint32_t row_bytes = n * (out == HB_OUT_F32 ? 4 : 2);
    if ((rc = e->check_candidates(what, c, eligible, state, y, out == HB_OUT_F32, m, row_bytes))) return rc;
    size_t best;
    if ((rc = e->pick_flagged(what, c, eligible, &best, nullptr, true))) return rc;
    e->gemm_pick[key] = c[best].kernel;
    *kernel = c[best].kernel;
    return HB_OK;
}

int hb_engine_gate_up(hb_engine* e, uint32_t h, uint32_t inter, hb_range state, hb_range w,
                      hb_range x, hb_range gu, hb_range hout, uint32_t m, int32_t* gemm_kernel,
                      int32_t* swiglu_kernel) {
    if (!e->g) return fail(HB_ERR_INVALID, "gate_up: an engine without a context");
    const Tune& t = e->t;
    int rc;
    *gemm_kernel = *swiglu_kernel = -1;
    char key[128];
    snprintf(key, sizeof key, "%ux%u, %u rows", h, 2 * inter, m);
    auto it = e->gate_up_pick.find(key);
    if (it != e->gate_up_pick.end()) {
        *gemm_kernel = it->second.first;
        *swiglu_kernel = it->second.second;
        return HB_OK;
    }
    int32_t gk, sk;
    if ((rc = hb_engine_gemm(e, h, 2 * inter, HB_OUT_BF16, state, w, x, gu, m, &gk))) return rc;
    hb_desc sd{};
    sd.kind = HB_KIND_SWIGLU;
    sd.n = inter;
    if ((rc = e->build(sd, &sk))) return rc;
    const bool timed = t["gemm.auto"] && !t.gemm_set;
    const uint32_t fswi = t["pf.fswi"];
    auto keep = [&](int32_t a, int32_t b) {
        e->gate_up_pick[key] = {a, b};
        *gemm_kernel = a;
        *swiglu_kernel = b;
        return HB_OK;
    };
    // The fused forms stage through LDS directly: W and X within 2 GiB.
    if (fswi == 0 || (fswi == 2 && !timed) || h % 32 || 4ull * inter * h > 0x7fffffffull ||
        2ull * m * h > 0x7fffffffull)
        return keep(gk, sk);
    bool mf = t["gemm.mfirst"] != 0;
    std::string what = std::string("gate_up+swiglu ") + key;
    std::vector<Cand> c;
    std::vector<bool> eligible;
    if (fswi == 2) {
        c.push_back({"apart", gk, {make_op(gk, m, {state, w, x, gu, state, state}), make_op(sk, m, {gu, hout})}});
        eligible.push_back(true);
    }
    for (const auto& f : kFusedForms) {
        hb_desc d = form_desc(f, h, inter, HB_OUT_BF16, mf);
        d.kind = HB_KIND_GEMM_SWIGLU;
        int32_t kk;
        if (e->build(d, &kk)) {
            e->logf("[autotune] gate_up+swiglu: %s not built (%s)", f.name, hb_last_error());
            continue;
        }
        c.push_back({f.name, kk, {make_op(kk, m, {state, w, x, hout, state, state})}});
        eligible.push_back(true);
    }
    if (c.empty()) return keep(gk, sk);
    if (fswi == 1) return c[0].name == "apart" ? keep(gk, sk) : keep(c[0].kernel, -1);
    if ((rc = e->check_candidates(what, c, eligible, state, hout, false, m, inter * 2))) return rc;
    size_t best;
    if ((rc = e->pick_flagged(what, c, eligible, &best, nullptr, true))) return rc;
    return best == 0 ? keep(gk, sk) : keep(c[best].kernel, -1);
}

int hb_engine_matvec(hb_engine* e, uint32_t k, uint32_t n, uint32_t out, uint32_t mv_m,
                     const hb_range* ws, uint32_t nws, hb_range x, hb_range y, int32_t* kernel) {
    if (!e->g) return fail(HB_ERR_INVALID, "matvec: an engine without a context");
    return hb_engine_matvec_fused(e, k, n, out, HB_XSRC_PLAIN, 0, 0, mv_m, ws, nws, x, y,
                                  hb_range{}, kernel);
}

// The matvec candidates of mv_full's timed choice (qwen.rs:1311-1511), in
// order, for one shape, m, fusion and the tune's splits and persistent
// counts.
std::vector<std::pair<std::string, hb_desc>> mv_candidates(hb_engine* e, uint32_t k, uint32_t n,
                                                           uint32_t out, uint32_t xsrc,
                                                           uint32_t eps_bits, uint32_t plus_one,
                                                           uint32_t mv_m) {
    const Tune& t = e->t;
    const bool fused = xsrc != HB_XSRC_PLAIN || out == HB_OUT_SWIGLU;
    auto desc = [&](uint32_t form, uint32_t rows, uint32_t split, uint32_t persist) {
        hb_desc d{};
        d.kind = HB_KIND_MATVEC;
        d.k = k;
        d.n = n;
        d.out = out;
        d.mv_m = mv_m;
        d.form = form;
        d.rows = rows;
        d.split = split;
        d.persist = persist;
        d.unroll = 4;
        d.xsrc = xsrc;
        d.eps_bits = eps_bits;
        d.plus_one = plus_one;
        return d;
    };
    std::vector<std::pair<std::string, hb_desc>> v;
    std::vector<uint32_t> splits = t["mv.splitauto"] ? std::vector<uint32_t>{1, 2, 4} : std::vector<uint32_t>{1};
    std::vector<uint32_t> pers = {0};
    for (uint32_t p : t.mv_persists) pers.push_back(p);
    // XSrc::Norm computes the norm once per workgroup: persistent
    // workgroups (two and four per CU) amortise it unless mv.persists names
    // its own counts.
    if (xsrc == HB_XSRC_NORM && t.mv_persists.empty())
        for (uint32_t p : {512u, 1024u}) pers.push_back(p);
    for (uint32_t split : splits)
        for (uint32_t p : pers)
            for (uint32_t rows : {1u, 2u, 4u, 8u}) {
                if (rows * mv_m > 64 || (p > 0 && rows == 8)) continue;
                if (out == HB_OUT_SWIGLU && rows < 2) continue;
                std::string tag = (split > 1 ? "k" + std::to_string(split) : "") +
                                  (p ? "p" + std::to_string(p) : "");
                v.emplace_back("r" + std::to_string(rows) + tag, desc(0, rows, split, p));
                v.emplace_back("d" + std::to_string(rows) + tag, desc(2, rows, split, p));
                if (rows <= 2) {
                    // A whole row's chunks in one batch of loads when K /
                    // split <= 4096: one HBM latency per wave, not two.
                    hb_desc d8 = desc(mv_m > 1 ? 2 : 0, rows, split, p);
                    d8.unroll = 8;
                    v.emplace_back((mv_m > 1 ? "d" : "r") + std::to_string(rows) + tag + "u8", d8);
                }
            }
    // The x rows staged in LDS once per workgroup (plain or XSrc::Swiglu,
    // m*K*2 <= 64 KiB): for several rows, where reloading x per row block
    // through the vector memory path costs more than the W stream, and for
    // XSrc::Swiglu, whose SwiGLU is then computed once per workgroup.
    // Persistent workgroups (two and four per CU) stage it fewer times.
    if ((mv_m > 1 || xsrc == HB_XSRC_SWIGLU) && xsrc != HB_XSRC_NORM && (uint64_t)mv_m * k * 2 <= 65536)
        for (uint32_t p : {0u, 512u, 1024u})
            for (uint32_t rows : {1u, 2u, 4u}) {
                if (rows * mv_m > 64 || (out == HB_OUT_SWIGLU && rows < 2)) continue;
                hb_desc dx = desc(mv_m > 1 ? 2 : 0, rows, 1, p);
                dx.unroll = 8;
                dx.x_lds = 1;
                v.emplace_back((mv_m > 1 ? "d" : "r") + std::to_string(rows) + (p ? "p" + std::to_string(p) : "") + "u8xl", dx);
            }
    // For several rows, x staged once per CU by one 16-wave workgroup (or
    // two 8-wave ones) with up to 144 KiB of LDS: the long-K o and down
    // shapes, whose x the 4-wave workgroups cannot hold or would stage per
    // four waves (measured at m=8: down 2.6 -> 3.5 TB/s, o 2.1 -> 2.5).
    if (mv_m > 1 && xsrc != HB_XSRC_NORM && (uint64_t)mv_m * k * 2 <= 147456) {
        const bool small = (uint64_t)mv_m * k * 2 <= 65536;
        const uint32_t r1 = out == HB_OUT_SWIGLU ? 2 : 1;
        struct W { uint32_t waves, rows, persist, unroll; };
        for (W w : {W{16, r1, 0, 8}, W{16, r1, 256, 4}, W{16, r1, 256, 8}, W{8, 2, 256, 4}}) {
            if (!small && w.persist != 256) continue;  // one workgroup per CU
            if (w.rows * mv_m > 64) continue;
            hb_desc dw = desc(2, w.rows, 1, w.persist);
            dw.unroll = w.unroll;
            dw.x_lds = 1;
            dw.mv_waves = w.waves;
            v.emplace_back("d" + std::to_string(w.rows) + (w.persist ? "p" + std::to_string(w.persist) : "") + "u" +
                    std::to_string(w.unroll) + "xl_w" + std::to_string(w.waves), dw);
        }
    }
    // The MFMA arithmetic with W read in row order through a wave-private
    // LDS tile (form 3): for several rows, where the VALU forms run out of
    // issue (measured at m=8: gate_up 4.4 -> 5.0 TB/s, lm_head 5.3 -> 6.1).
    if (mv_m > 1 && !fused && k % 128 == 0) {
        // rows 32: two 16-row tiles per wave share each x fragment (half
        // the x loads per W byte; lm_head at m=8: 6.1 -> 6.7 TB/s).
        struct F { uint32_t unroll, split, persist, rows; };
        for (F f : {F{4, 4, 0, 16}, F{4, 2, 0, 16}, F{4, 1, 512, 16}, F{4, 4, 512, 16}, F{8, 2, 0, 16},
                    F{8, 4, 0, 16}, F{8, 4, 512, 16}, F{4, 4, 0, 32}, F{4, 4, 512, 32}}) {
            hb_desc d3 = desc(3, f.rows, f.split, f.persist);
            d3.unroll = f.unroll;
            const std::string nm = "mfl" + std::string(f.rows == 32 ? "_r32" : "") + "_u" + std::to_string(f.unroll) +
                                   "k" + std::to_string(f.split) + (f.persist ? "p" + std::to_string(f.persist) : "");
            v.emplace_back(nm, d3);
            // x (the B operand) staged in LDS once per workgroup: its loads
            // were a fifth of the form's time, one per row block.
            if ((uint64_t)mv_m * (k + 8) * 2 + 4ull * (f.rows / 16) * 16 * f.unroll * 16 * 4 <= 160 * 1024 &&
                (uint64_t)mv_m * k * 2 <= 65536) {
                d3.x_lds = 1;
                v.emplace_back(nm + "xl", d3);
            }
        }
    }
    // The MFMA 4x4x4 form (W straight from memory as 4 rows x 256 bytes per
    // load instruction, x in registers): waves sharing a row block's K so
    // that each wave's x fits in at most 72 registers; 4, 8 or 16 W rows per
    // wave and persistent workgroups (each wave's x serves more rows, which
    // measured decisive at 4 and 8 rows: the lm_head at m=4 0.168 ms with
    // one row block per wave, 0.126 with 1024 workgroups), within about 168
    // registers (three waves a SIMD; 120 with 16-wave workgroups, whose
    // limit is 128) (x, two row blocks of W in flight, the sums).
    if (!fused && mv_m <= 8) {
        const uint32_t mq = (mv_m + 3) / 4;
        for (uint32_t waves : {4u, 8u, 16u})
            for (uint32_t split : {1u, 2u, 4u, 8u}) {
                if (waves == 16 && split < 8) continue;
                if (split > waves || k % (128 * split)) continue;
                const uint32_t li = k / split / 128;
                if (li * mq > 18 || li < 2) continue;
                for (uint32_t rows : {4u, 8u, 16u})
                    for (uint32_t p : {0u, 256u, 1024u}) {
                        const uint32_t tg = rows / 4, vg = li * mq * 4 + (p ? 2 : 1) * tg * li * 4 + tg * mq * 8;
                        if (vg > (waves == 16 ? 120u : 168u) || (p == 0 && rows > 4) || (mv_m == 1 && p == 256)) continue;
                        hb_desc d4 = desc(4, rows, split, p);
                        d4.mv_waves = waves;
                        v.emplace_back("mf4_r" + std::to_string(rows) + "k" + std::to_string(split) + "_w" +
                                           std::to_string(waves) + (p ? "p" + std::to_string(p) : ""),
                                       d4);
                    }
            }
    }
    for (uint32_t split : splits)
        for (uint32_t p : pers) {
            if (fused) break;  // the fusions are VALU forms
            std::string tag = (split > 1 ? "k" + std::to_string(split) : "") + (p ? "p" + std::to_string(p) : "");
            v.emplace_back("mfma" + tag, desc(1, 16, split, p));
            for (uint32_t u : {8u, 16u}) {
                hb_desc du = desc(1, 16, split, p);
                du.unroll = u;
                v.emplace_back("mfma_u" + std::to_string(u) + tag, du);
            }
        }
    return v;
}

int hb_engine_matvec_candidates(hb_engine* e, uint32_t k, uint32_t n, uint32_t out, uint32_t xsrc,
                                uint32_t eps_bits, uint32_t plus_one, uint32_t mv_m, hb_desc* descs,
                                uint32_t cap, uint32_t* count) {
    const auto v = mv_candidates(e, k, n, out, xsrc, eps_bits, plus_one, mv_m);
    *count = (uint32_t)v.size();
    for (uint32_t i = 0; i < v.size() && i < cap; i++) descs[i] = v[i].second;
    return HB_OK;
}

int hb_engine_matvec_fused(hb_engine* e, uint32_t k, uint32_t n, uint32_t out, uint32_t xsrc,
                           uint32_t eps_bits, uint32_t plus_one, uint32_t mv_m, const hb_range* ws,
                           uint32_t nws, hb_range x, hb_range y, hb_range norm_w, int32_t* kernel) {
    if (!e->g) return fail(HB_ERR_INVALID, "matvec_fused: an engine without a context");
    const Tune& t = e->t;
    if (!nws) return fail(HB_ERR_INVALID, "matvec: no weights");
    // A fusion (kernels.rs:236-290): the VALU forms, rows in gate/up pairs
    // for Out::Swiglu (qwen.rs:1393-1397: rows.max(2)).
    const bool fused = xsrc != HB_XSRC_PLAIN || out == HB_OUT_SWIGLU;
    auto desc = [&](uint32_t form, uint32_t rows, uint32_t split, uint32_t persist) {
        hb_desc d{};
        d.kind = HB_KIND_MATVEC;
        d.k = k;
        d.n = n;
        d.out = out;
        d.mv_m = mv_m;
        d.form = form;
        d.rows = rows;
        d.split = split;
        d.persist = persist;
        d.unroll = 4;
        d.xsrc = xsrc;
        d.eps_bits = eps_bits;
        d.plus_one = plus_one;
        return d;
    };
    auto bind = [&](uint32_t i) {
        std::vector<hb_range> b = {ws[i], x, y};
        if (xsrc == HB_XSRC_NORM) b.push_back(norm_w);
        return b;
    };
    if (!t["mv.auto"]) {
        // mv.split / mv.persist, the engine's rows (Options::matvec_rows).
        uint32_t rows = std::max<uint32_t>(1, std::min<uint32_t>(4, 64 / std::max<uint32_t>(mv_m, 1)));
        if (out == HB_OUT_SWIGLU) rows = std::max<uint32_t>(rows, 2);
        return e->build(desc(0, rows, t["mv.split"], t["mv.persist"]), kernel);
    }
    std::string persists;
    if (!t.mv_persists.empty()) {
        persists = " p[";
        for (size_t i = 0; i < t.mv_persists.size(); i++)
            persists += (i ? ", " : "") + std::to_string(t.mv_persists[i]);
        persists += "]";
    }
    char key[160];
    char xs[32] = "";
    if (xsrc == HB_XSRC_SWIGLU) snprintf(xs, sizeof xs, " Swiglu");
    if (xsrc == HB_XSRC_NORM) snprintf(xs, sizeof xs, " Norm(%08x%s)", eps_bits, plus_one ? ",+1" : "");
    snprintf(key, sizeof key, "%ux%u%s %s m%u%s", k, n, xs, out_name(out), mv_m, persists.c_str());
    auto it = e->mv_pick.find(key);
    if (it != e->mv_pick.end()) return e->build(it->second, kernel);
    // Each form timed over every matrix of the shape (mv.cold) or the first.
    uint32_t nw = t["mv.cold"] ? nws : 1;
    std::vector<Cand> c;
    std::vector<hb_desc> descs;
    auto add = [&](const std::string& name, const hb_desc& d) {
        int32_t kk;
        if (e->build(d, &kk)) {
            e->logf("[autotune] matvec %s: %s not built (%s)", key, name.c_str(), hb_last_error());
            return;
        }
        std::vector<hb_op> ops;
        for (uint32_t i = 0; i < nw; i++) ops.push_back(make_op(kk, mv_m, bind(i)));
        c.push_back({name, kk, ops});
        descs.push_back(d);
    };
    for (const auto& cd : mv_candidates(e, k, n, out, xsrc, eps_bits, plus_one, mv_m))
        add(cd.first, cd.second);
    if (c.empty()) return fail(HB_ERR_COMPILE, std::string("matvec ") + key + ": no form built");
    std::vector<bool> all(c.size(), true);
    size_t best;
    // Cold as in a decode step (a model's weights are far larger than the
    // 256 MiB last-level cache, every matrix is read from HBM once per
    // token): the flush before each run, only the matvec launches counted.
    int rc = e->pick_flagged(std::string("matvec ") + key, c, all, &best, nullptr, true);
    if (rc) return rc;
    e->mv_pick[key] = descs[best];
    *kernel = c[best].kernel;
    return HB_OK;
}

int hb_engine_experts(hb_engine* e, uint32_t experts, uint32_t top_k, uint32_t hidden,
                      uint32_t inter, uint32_t m, const hb_moe_io* io, int32_t kernels[4],
                      uint32_t* bm_out) {
    if (!e->g) return fail(HB_ERR_INVALID, "experts: an engine without a context");
    const Tune& t = e->t;
    bool mf = t["gemm.mfirst"] != 0;
    int rc;
    auto sort_desc = [&](bool atomic, uint32_t bm) {
        hb_desc d{};
        d.kind = atomic ? HB_KIND_SORT_ATOMIC : HB_KIND_SORT;
        d.experts = experts;
        d.top_k = top_k;
        d.bm = bm;
        d.rows_max = m;
        return d;
    };
    // An expert GEMM over tiles of bm rows: W rows by bn, wm x wn waves
    // (default four along N), stages - 1 = dbuf.
    auto gemm_desc = [&](uint32_t k, uint32_t n, uint32_t rows_of, uint32_t bm, uint32_t bn,
                         uint32_t wm = 1, uint32_t wn = 4, uint32_t dbuf = 1) {
        hb_desc d{};
        d.kind = HB_KIND_GEMM;
        d.k = k;
        d.n = n;
        d.out = HB_OUT_BF16;
        d.rows_of = rows_of;
        d.m_first = mf;
        d.bm = bm;
        d.bn = bn;
        d.bk = 64;
        d.wm = wm;
        d.wn = wn;
        d.mfma = 16;
        d.lds_dma = 1;
        d.dbuf = dbuf;
        d.top_k = top_k;
        d.experts = experts;
        d.tiles = (m * top_k + bm - 1) / bm + experts;  // moe_tiles
        d.rows_max = m;
        return d;
    };
    hb_desc gd{};
    gd.kind = HB_KIND_GATHER;
    gd.n = hidden;
    gd.top_k = top_k;
    int32_t gather;
    if ((rc = e->build(gd, &gather))) return rc;
    auto kernels_for = [&](uint32_t bm, int32_t* sort, int32_t* gu, int32_t* dn) -> int {
        int r;
        if ((r = e->build(sort_desc(false, bm), sort))) return r;
        if ((r = e->build(gemm_desc(hidden, 2 * inter, HB_ROWS_GATHER, bm, 128), gu))) return r;
        return e->build(gemm_desc(inter, hidden, HB_ROWS_SCATTER, bm, 128), dn);
    };
    if (!t["gemm.auto"] || t.gemm_set) {
        uint32_t bm = t["moe.tile"];
        if ((rc = kernels_for(bm, &kernels[0], &kernels[1], &kernels[2]))) return rc;
        kernels[3] = -1;
        *bm_out = bm;
        return HB_OK;
    }
    char ekey[96];
    snprintf(ekey, sizeof ekey, "%u %u %u %u, %u rows", experts, top_k, hidden, inter, m);
    auto eit = e->experts_pick.find(ekey);
    if (eit != e->experts_pick.end()) {
        for (int i = 0; i < 4; i++) kernels[i] = eit->second.kernels[i];
        *bm_out = eit->second.bm;
        return HB_OK;
    }
    // swiglu_slots after an unfused gate|up (EGU -> EHB), timed with it.
    hb_desc swd{};
    swd.kind = HB_KIND_SWIGLU;
    swd.n = inter;
    int32_t swiglu;
    if ((rc = e->build(swd, &swiglu))) return rc;
    const hb_op sw_op = make_op(swiglu, m * top_k, {io->egu, io->ehb});
    auto gu_ops = [&](int32_t k, hb_range xin) {
        return make_op(k, m, {io->state, io->w_gate_up, xin, io->egu, io->list, io->tiles});
    };
    hb_op dn_op = make_op(0, m, {io->state, io->w_down, io->ehb, io->ey, io->list, io->tiles});
    hb_op g_op = make_op(gather, m, {io->state, io->list, io->x, io->xs});
    // moe.tile's 16, 32, 64, and (timed only) 128: at ~64 rows per expert a
    // tile of 128 holds every row of most experts, so each expert's W is
    // read once (HBM-bound) at the price of MFMA work on padding rows.
    std::vector<uint32_t> tiles_rows = t.moe_tile_set ? std::vector<uint32_t>{t["moe.tile"]}
                                                      : std::vector<uint32_t>{16, 32, 64, 128};
    double best_total = 1e30;
    for (uint32_t bm : tiles_rows) {
        int32_t scan, atomic, mma_gu, mma_dn;
        if ((rc = kernels_for(bm, &scan, &mma_gu, &mma_dn))) return rc;
        if ((rc = e->build(sort_desc(true, bm), &atomic))) return rc;
        auto sort_op = [&](int32_t k) {
            return std::vector<hb_op>{make_op(k, m, {io->state, io->route, io->list, io->tiles})};
        };
        char what[160];
        snprintf(what, sizeof what, "experts sort by %u rows, %u rows", bm, m);
        std::vector<Cand> cs = {{"scan", scan, sort_op(scan)}, {"atomic", atomic, sort_op(atomic)}};
        size_t bs;
        double s_sort;
        if ((rc = e->pick_flagged(what, cs, {true, true}, &bs, &s_sort))) return rc;
        // The list and table of these tiles, by the sort kept.
        double tmp;
        if ((rc = e->time_ops(cs[bs].ops, 1, &tmp))) return rc;
        std::vector<Cand> cgu, cdn;
        auto add_gu = [&](const std::string& name, const hb_desc& d, bool gathered) {
            int32_t k;
            if (e->build(d, &k)) {
                e->logf("[autotune] experts: %s by %u rows not built (%s)", name.c_str(), bm, hb_last_error());
                return;
            }
            std::vector<hb_op> ops;
            if (gathered) ops.push_back(g_op);
            if (d.kind == HB_KIND_GEMM_SWIGLU) {
                // The SwiGLU in the epilogue: EHB written directly.
                ops.push_back(make_op(k, m, {io->state, io->w_gate_up, gathered ? io->xs : io->x, io->ehb,
                                             io->list, io->tiles}));
            } else {
                ops.push_back(gu_ops(k, gathered ? io->xs : io->x));
                ops.push_back(sw_op);
            }
            cgu.push_back({name, k, ops});
        };
        // gemm_desc of the fused [gate | up] + SwiGLU form: inter features,
        // bn W rows (bn/2 features) per tile.
        auto swi_desc = [&](uint32_t bn, uint32_t wm = 1, uint32_t wn = 4) {
            hb_desc d = gemm_desc(hidden, inter, HB_ROWS_GATHER, bm, bn, wm, wn);
            d.kind = HB_KIND_GEMM_SWIGLU;
            return d;
        };
        auto add_dn = [&](const std::string& name, const hb_desc& d) {
            int32_t k;
            if (e->build(d, &k)) {
                e->logf("[autotune] experts: %s by %u rows not built (%s)", name.c_str(), bm, hb_last_error());
                return;
            }
            hb_op op = dn_op;
            op.kernel = k;
            cdn.push_back({name, k, {op}});
        };
        add_gu("mma", gemm_desc(hidden, 2 * inter, HB_ROWS_GATHER, bm, 128), false);
        add_gu("mma_n256", gemm_desc(hidden, 2 * inter, HB_ROWS_GATHER, bm, 256), false);
        add_gu("gather+mma", gemm_desc(hidden, 2 * inter, HB_ROWS_SORTED, bm, 128), true);
        if (bm >= 32) add_gu("mma_w2x2", gemm_desc(hidden, 2 * inter, HB_ROWS_GATHER, bm, 128, 2, 2), false);
        {
            hb_desc d = gemm_desc(hidden, 2 * inter, HB_ROWS_GATHER, bm, 128);
            d.m_first = !d.m_first;
            add_gu(d.m_first ? "mma_mf" : "mma_nf", d, false);
            hb_desc ds = swi_desc(128);
            ds.m_first = !ds.m_first;
            add_gu(ds.m_first ? "mma_swiglu_mf" : "mma_swiglu_nf", ds, false);
        }
        add_gu("mma_swiglu", swi_desc(128), false);
        {
            // Each expert's W streamed once: its loads non-temporal.
            hb_desc d = swi_desc(128);
            d.w_nt = 1;
            add_gu("mma_swiglu_wnt", d, false);
        }
        add_gu("mma_swiglu_n256", swi_desc(256), false);
        if (bm >= 32) add_gu("mma_swiglu_w2x2", swi_desc(128, 2, 2), false);
        add_dn("mma", gemm_desc(inter, hidden, HB_ROWS_SCATTER, bm, 128));
        add_dn("mma_n256", gemm_desc(inter, hidden, HB_ROWS_SCATTER, bm, 256));
        {
            // Column tiles first: the expert tile's 16 column tiles in turn.
            hb_desc d = gemm_desc(inter, hidden, HB_ROWS_SCATTER, bm, 128);
            d.m_first = !d.m_first;
            add_dn(d.m_first ? "mma_mf" : "mma_nf", d);
            d.w_nt = 1;
            add_dn(d.m_first ? "mma_mf_wnt" : "mma_nf_wnt", d);
            hb_desc d2 = gemm_desc(inter, hidden, HB_ROWS_SCATTER, bm, 128);
            d2.w_nt = 1;
            add_dn("mma_wnt", d2);
            if (bm >= 32) {
                // 256-wide W tiles, 8 waves, 3 stages, in the same order.
                hb_desc d3 = gemm_desc(inter, hidden, HB_ROWS_SCATTER, bm, 256, 2, 4, 2);
                d3.m_first = d.m_first;
                d3.w_nt = 1;
                d3.order = 1;  // each XCD a contiguous share of the table's tiles
                add_dn(d3.m_first ? "mma_n256_w8_s3_mf_wnt" : "mma_n256_w8_s3_nf_wnt", d3);
            }
        }
        if (bm >= 32) add_dn("mma_w2x4_s3", gemm_desc(inter, hidden, HB_ROWS_SCATTER, bm, 128, 2, 4, 2));
        size_t bgu, bdn;
        double s_gu, s_dn;
        snprintf(what, sizeof what, "experts gate_up %ux%u by %u rows, %u rows", hidden, 2 * inter, bm, m);
        if ((rc = e->pick_flagged(what, cgu, std::vector<bool>(cgu.size(), true), &bgu, &s_gu))) return rc;
        snprintf(what, sizeof what, "experts down %ux%u by %u rows, %u rows", inter, hidden, bm, m);
        if ((rc = e->pick_flagged(what, cdn, std::vector<bool>(cdn.size(), true), &bdn, &s_dn))) return rc;
        double total = s_gu + s_dn + s_sort;
        e->logf("[autotune] experts by %u rows, %u rows: sort %.3f ms, total %.3f ms", bm, m,
                s_sort * 1e3, total * 1e3);
        if (total < best_total) {
            best_total = total;
            kernels[0] = cs[bs].kernel;
            kernels[1] = cgu[bgu].kernel;
            kernels[2] = cdn[bdn].kernel;
            kernels[3] = cgu[bgu].ops[0].kernel == gather ? gather : -1;
            *bm_out = bm;
        }
    }
    e->logf("[autotune] experts, %u rows -> tiles of %u rows", m, *bm_out);
    hb_engine::ExpertsPick ep;
    for (int i = 0; i < 4; i++) ep.kernels[i] = kernels[i];
    ep.bm = *bm_out;
    e->experts_pick[ekey] = ep;
    return HB_OK;
}

// The picks as text, one line per choice, tab-separated: the choice's kind
// and key, then for each kernel of it its name and its descriptor's fields
// (decimal, in hb_desc order; "-" for none).  hb_engine_pin reads the same.
static std::string desc_text(hb_gpu* g, int32_t k) {
    if (k < 0) return "-\t-";
    const hb_desc* d = kernel_desc(g, k);
    std::string s = std::string(hb_kernel_name(g, k)) + "\t";
    const uint32_t* w = (const uint32_t*)d;
    for (size_t i = 0; i < sizeof(hb_desc) / 4; i++) s += (i ? " " : "") + std::to_string(w[i]);
    return s;
}

int hb_engine_picks(hb_engine* e, char* buf, uint64_t cap, uint64_t* len) {
    if (!e->g) return fail(HB_ERR_INVALID, "picks: an engine without a context");
    std::string s;
    for (const auto& kv : e->gemm_pick) s += "gemm\t" + kv.first + "\t" + desc_text(e->g, kv.second) + "\n";
    for (const auto& kv : e->gate_up_pick)
        s += "gate_up\t" + kv.first + "\t" + desc_text(e->g, kv.second.first) + "\t" +
             desc_text(e->g, kv.second.second) + "\n";
    for (const auto& kv : e->mv_pick) {
        int32_t k;
        int rc = e->build(kv.second, &k);
        if (rc) return rc;
        s += "mv\t" + kv.first + "\t" + desc_text(e->g, k) + "\n";
    }
    for (const auto& kv : e->experts_pick) {
        s += "experts\t" + kv.first + "\t" + std::to_string(kv.second.bm);
        for (int i = 0; i < 4; i++) s += "\t" + desc_text(e->g, kv.second.kernels[i]);
        s += "\n";
    }
    *len = s.size();
    if (buf && cap) {
        const uint64_t n = std::min<uint64_t>(cap - 1, s.size());
        memcpy(buf, s.data(), n);
        buf[n] = 0;
    }
    return HB_OK;
}

int hb_engine_pin(hb_engine* e, const char* text) {
    if (!e->g) return fail(HB_ERR_INVALID, "pin: an engine without a context");
    std::istringstream in(text ? text : "");
    std::string line;
    int no = 0;
    while (std::getline(in, line)) {
        no++;
        if (line.empty()) continue;
        std::vector<std::string> f;
        std::string cell;
        std::istringstream ls(line);
        while (std::getline(ls, cell, '\t')) f.push_back(cell);
        auto bad = [&](const std::string& why) {
            return fail(HB_ERR_INVALID, "pin, line " + std::to_string(no) + ": " + why);
        };
        // Builds the kernel of fields f[at] (name) and f[at + 1] (descriptor).
        auto kernel_at = [&](size_t at, int32_t* k) -> int {
            if (at + 1 >= f.size()) return bad("too few fields");
            if (f[at] == "-") {
                *k = -1;
                return HB_OK;
            }
            hb_desc d{};
            uint32_t* w = (uint32_t*)&d;
            std::istringstream ds(f[at + 1]);
            for (size_t i = 0; i < sizeof(hb_desc) / 4; i++)
                if (!(ds >> w[i])) return bad("descriptor of " + f[at]);
            int rc = e->build(d, k);
            if (rc) return rc;
            if (f[at] != hb_kernel_name(e->g, *k))
                return bad("the descriptor builds " + std::string(hb_kernel_name(e->g, *k)) + ", not " + f[at]);
            return HB_OK;
        };
        int rc;
        if (f.size() < 2) return bad("no key");
        if (f[0] == "gemm") {
            int32_t k;
            if ((rc = kernel_at(2, &k))) return rc;
            e->gemm_pick[f[1]] = k;
        } else if (f[0] == "gate_up") {
            int32_t a, b;
            if ((rc = kernel_at(2, &a)) || (rc = kernel_at(4, &b))) return rc;
            e->gate_up_pick[f[1]] = {a, b};
        } else if (f[0] == "mv") {
            int32_t k;
            if ((rc = kernel_at(2, &k))) return rc;
            if (k < 0) return bad("no matvec kernel");
            e->mv_pick[f[1]] = *kernel_desc(e->g, k);
        } else if (f[0] == "experts") {
            if (f.size() < 11) return bad("too few fields");
            hb_engine::ExpertsPick ep;
            ep.bm = (uint32_t)std::stoul(f[2]);
            for (int i = 0; i < 4; i++)
                if ((rc = kernel_at(3 + 2 * i, &ep.kernels[i]))) return rc;
            e->experts_pick[f[1]] = ep;
        } else {
            return bad("unknown kind " + f[0]);
        }
    }
    return HB_OK;
}

// autotune_chunk (qwen.rs:2962-3010): the candidates 1024, 2048, 4096, 8192
// below prefill.block and prefill.block itself; the host's first block of
// cands[0] rows run until auto.heat ms of GPU time have passed; then three
// rounds, the order reversed every other one, each candidate's prompt of
// prefill.block rows cut by blocks_of and its blocks' GPU times summed; the
// median of each; the fastest kept (the first on a tie, as min_by does).
int hb_engine_autotune_chunk(hb_engine* e, const hb_prefill_host* host, uint32_t* chunk) {
    if (!host || !host->block_in || !chunk) return fail(HB_ERR_INVALID, "autotune_chunk: host and chunk");
    const auto started = std::chrono::steady_clock::now();
    const uint32_t block = e->t["prefill.block"];
    std::vector<uint32_t> cands;
    for (uint32_t c : {1024u, 2048u, 4096u, 8192u})
        if (c < block) cands.push_back(c);
    cands.push_back(block);
    *chunk = block;
    if (cands.size() < 2) return HB_OK;
    auto reset = [&]() -> int {
        if (host->reset && host->reset(host->ctx))
            return fail(HB_ERR_INVALID, "autotune_chunk: the host's reset failed");
        return HB_OK;
    };
    auto run = [&](uint32_t start, uint32_t rows, double* s) -> int {
        *s = 0.0;
        if (host->block_in(host->ctx, start, rows, s))
            return fail(HB_ERR_INVALID, "autotune_chunk: the host's block_in failed over " +
                                            std::to_string(rows) + " rows at " + std::to_string(start));
        return HB_OK;
    };
    int rc;
    const double heat = e->t["auto.heat"] * 1e-3;
    double warmed = 0.0, s;
    do {
        if ((rc = reset()) || (rc = run(0, cands[0], &s))) return rc;
        warmed += s;
    } while (warmed < heat);
    std::vector<std::vector<double>> times(cands.size());
    std::vector<uint32_t> starts, rows;
    for (int round = 0; round < 3; round++)
        for (size_t j = 0; j < cands.size(); j++) {
            const size_t i = round % 2 == 0 ? j : cands.size() - 1 - j;
            if ((rc = reset())) return rc;
            const uint32_t nb = hb_blocks_of(block, cands[i], nullptr, nullptr, 0);
            starts.resize(nb);
            rows.resize(nb);
            hb_blocks_of(block, cands[i], starts.data(), rows.data(), nb);
            double t = 0.0;
            for (uint32_t b = 0; b < nb; b++) {
                if ((rc = run(starts[b], rows[b], &s))) return rc;
                t += s;
            }
            times[i].push_back(t);
        }
    std::vector<double> med(cands.size());
    size_t best = 0;
    std::string line;
    for (size_t i = 0; i < cands.size(); i++) {
        std::sort(times[i].begin(), times[i].end());
        med[i] = times[i][times[i].size() / 2];
        if (med[i] < med[best]) best = i;
        char one[64];
        snprintf(one, sizeof one, "%s%u %.3f ms", i ? ", " : "", cands[i], med[i] * 1e3);
        line += one;
    }
    if ((rc = reset())) return rc;
    *chunk = cands[best];
    e->logf("[autotune] blocks over %u rows, every layer, heated %.1f s, median of 3 rounds: %s -> %u", block,
            warmed, line.c_str(), cands[best]);
    e->autotune_seconds += std::chrono::duration<double>(std::chrono::steady_clock::now() - started).count();
    e->timed = true;
    e->last_timed = std::chrono::steady_clock::now();
    return HB_OK;
}

uint32_t hb_blocks_of(uint32_t n, uint32_t chunk, uint32_t* starts, uint32_t* rows, uint32_t cap) {
    if (!n) return 0;
    const uint32_t c = chunk ? chunk : 1;
    const uint32_t k = (n + c - 1) / c;
    uint32_t size = (n + k - 1) / k;
    size = (size + 63) / 64 * 64;
    if (size > c) size = c;
    uint32_t count = 0;
    for (uint32_t at = 0; at < n; at += size, count++)
        if (count < cap) {
            starts[count] = at;
            rows[count] = size < n - at ? size : n - at;
        }
    return count;
}

}  // extern "C"
