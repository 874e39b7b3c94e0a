// hb_gemm -- a native host of the C ABI (include/herbert_hip.h): for each
// shape on the command line the selection layer picks a kernel (the
// engine's --tune settings, the [autotune] log on stderr), then the pick is
// timed on this GPU and one line per shape printed.  The inputs come from
// the library's seeded generator (X ~ N(0,1), W ~ N(0,0.02), bf16).
//
//   hb_gemm [--tune key=value,...] [--reps N] SHAPE...
//   SHAPE  MxKxN      a dense GEMM, Y = X.W^T, Out::Bf16
//          MxKxNr     the same with Out::Residual (Y += ...)
//          MxKxNf     the same with Out::F32
//          mv:MxKxN   the decode matvec over M <= 16 rows
//
// Output per shape: shape, kernel, microseconds per launch, TFLOP/s (GEMM)
// or GB/s of algorithmic bytes (matvec).  The reference's counterpart is
// its prefill/decode benchmarks driving QwenEngine (src/metal/qwen.rs) with
// --tune; this links the library the same way a Rust host would.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "herbert_hip.h"

namespace {

int die(const char* what) {
    fprintf(stderr, "hb_gemm: %s: %s\n", what, hb_last_error());
    return 1;
}

struct Shape {
    bool matvec = false;
    uint32_t m = 0, k = 0, n = 0, out = HB_OUT_BF16;
};

bool parse(const char* s, Shape* sh) {
    if (!strncmp(s, "mv:", 3)) {
        sh->matvec = true;
        s += 3;
    }
    char tail[8] = "";
    if (sscanf(s, "%ux%ux%u%7s", &sh->m, &sh->k, &sh->n, tail) < 3) return false;
    if (!strcmp(tail, "r")) sh->out = HB_OUT_RESIDUAL;
    else if (!strcmp(tail, "f")) sh->out = HB_OUT_F32;
    else if (tail[0]) return false;
    return sh->m && sh->k && sh->n && (!sh->matvec || sh->m <= 16);
}

hb_range whole(hb_buf b) {
    hb_range r;
    memset(&r, 0, sizeof r);
    r.buf = b;
    return r;
}

// A buffer of `count` bf16 from the seeded generator.
int normal_buf(hb_gpu* g, uint64_t seed, float std, uint64_t count, hb_buf* out) {
    std::vector<uint16_t> h(count);
    hb_fill_normal_bf16(seed, std, h.data(), count, 8);
    int rc = hb_alloc(g, count * 2, out);
    if (rc) return rc;
    return hb_upload(g, *out, 0, h.data(), count * 2);
}

}  // namespace

int main(int argc, char** argv) {
    std::string tune;
    uint32_t reps = 20;
    std::vector<Shape> shapes;
    for (int i = 1; i < argc; i++) {
        if (!strcmp(argv[i], "--tune") && i + 1 < argc) {
            tune = argv[++i];
        } else if (!strcmp(argv[i], "--reps") && i + 1 < argc) {
            reps = (uint32_t)atoi(argv[++i]);
        } else {
            Shape sh;
            if (!parse(argv[i], &sh)) {
                fprintf(stderr, "hb_gemm: bad shape '%s' (MxKxN[r|f] or mv:MxKxN, M <= 16)\n", argv[i]);
                return 2;
            }
            shapes.push_back(sh);
        }
    }
    if (shapes.empty() || !reps) {
        fprintf(stderr, "usage: hb_gemm [--tune key=value,...] [--reps N] MxKxN[r|f] | mv:MxKxN ...\n");
        return 2;
    }
    hb_gpu* g = nullptr;
    if (hb_open(0, &g)) return die("hb_open");
    fprintf(stderr, "[gpu] %s\n", hb_device_summary(g));
    hb_engine* e = nullptr;
    if (hb_engine_open(g, tune.c_str(), &e)) return die("hb_engine_open");
    int status = 0;
    for (const Shape& s : shapes) {
        const uint64_t ysz = (uint64_t)s.m * s.n * (s.out == HB_OUT_F32 ? 4 : 2);
        hb_buf x, w, y, st;
        if (normal_buf(g, 0x5EED0000u + s.k, 1.0f, (uint64_t)s.m * s.k, &x) ||
            normal_buf(g, 0x5EED0001u + s.k, 0.02f, (uint64_t)s.n * s.k, &w) || hb_alloc(g, ysz, &y) ||
            hb_zero(g, y, 0, ysz) || hb_alloc(g, 16, &st))
            return die("buffers");
        const uint32_t state[4] = {0, 0, 0, s.m};
        if (hb_upload(g, st, 0, state, sizeof state)) return die("state");
        int32_t kern = -1;
        hb_op op;
        memset(&op, 0, sizeof op);
        op.m = s.m;
        if (s.matvec) {
            hb_range wr = whole(w);
            if (hb_engine_matvec(e, s.k, s.n, s.out, s.m, &wr, 1, whole(x), whole(y), &kern)) {
                status = die("hb_engine_matvec");
                continue;
            }
            op.nbind = 3;
            op.bind[0] = whole(w);
            op.bind[1] = whole(x);
            op.bind[2] = whole(y);
        } else {
            if (hb_engine_gemm(e, s.k, s.n, s.out, whole(st), whole(w), whole(x), whole(y), s.m, &kern)) {
                status = die("hb_engine_gemm");
                continue;
            }
            op.nbind = 6;
            op.bind[0] = whole(st);
            op.bind[1] = whole(w);
            op.bind[2] = whole(x);
            op.bind[3] = whole(y);
            op.bind[4] = whole(st);
            op.bind[5] = whole(st);
        }
        op.kernel = kern;
        double secs = 0;
        if (hb_time(g, &op, 1, 3, &secs) || hb_time(g, &op, 1, reps, &secs)) return die("hb_time");
        const double t = secs / reps;
        if (s.matvec) {
            const double bytes = 2.0 * s.n * s.k + 2.0 * s.m * s.k +
                                 2.0 * s.m * s.n * (s.out == HB_OUT_RESIDUAL ? 2 : 1);
            printf("mv:%ux%ux%u %s %.2f us %.1f GB/s\n", s.m, s.k, s.n, hb_kernel_name(g, kern), t * 1e6,
                   bytes / t / 1e9);
        } else {
            printf("%ux%ux%u%s %s %.2f us %.1f TFLOP/s\n", s.m, s.k, s.n,
                   s.out == HB_OUT_RESIDUAL ? "r" : s.out == HB_OUT_F32 ? "f" : "", hb_kernel_name(g, kern),
                   t * 1e6, 2.0 * s.m * s.n * s.k / t / 1e12);
        }
        fflush(stdout);
        for (hb_buf b : {x, w, y, st}) hb_free(g, b);
    }
    hb_engine_log_summary(e);
    hb_engine_close(e);
    hb_close(g);
    return status;
}
