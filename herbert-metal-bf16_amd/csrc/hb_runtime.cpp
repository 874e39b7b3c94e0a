// hb_runtime.cpp -- the HIP runtime under the C ABI: device context, buffer
// arena, hiprtc kernel builds with an in-memory cache keyed by kernel name
// and an on-disk code-object cache keyed by source hash, launches on the
// context's stream and event timing.
//
// Reference: src/metal/gpu.rs (Gpu::open :70, alloc :150-157, pipeline
// :127-148, dispatch :166-201, submit_wait :209-221) and the pipeline cache
// QwenEngine::get (src/metal/qwen.rs:1156-1166).
#include <hip/hiprtc.h>

#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <sstream>
#include <dlfcn.h>
#include <utime.h>
#include <sys/stat.h>
#include <unistd.h>

#include "hb_internal.h"

// The kernel sources, embedded by the build (name, text) pairs.
#include "hb_sources.inc"

namespace hb {

static thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(HB_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

int resolve(hb_gpu* g, const hb_range& r, char** ptr, uint64_t* size) {
    if (r.buf >= g->bufs.size() || !g->bufs[r.buf].live)
        return fail(HB_ERR_INVALID, "range on buffer " + std::to_string(r.buf) + ": no such buffer");
    const Buffer& b = g->bufs[r.buf];
    if (r.offset > b.size || (r.size && r.offset + r.size > b.size))
        return fail(HB_ERR_INVALID, "range [" + std::to_string(r.offset) + ", +" +
                                        std::to_string(r.size) + ") outside buffer " +
                                        std::to_string(r.buf) + " of " + std::to_string(b.size) +
                                        " bytes");
    *ptr = (char*)b.ptr + r.offset;
    *size = r.size ? r.size : b.size - r.offset;
    return HB_OK;
}

static const char* source_text(const std::string& name) {
    for (const auto& s : kSources)
        if (name == s.name) return s.text;
    return nullptr;
}

static uint64_t fnv1a(const std::string& s, uint64_t h = 1469598103934665603ull) {
    for (unsigned char c : s) {
        h ^= c;
        h *= 1099511628211ull;
    }
    return h;
}

// The disk cache of compiled kernels: $HB_CACHE_DIR ("" disables it), else
// _kcache beside this library (build.py fills it for the kernels its
// manifest lists, so a fresh box finds them compiled), else
// ~/.cache/herbert_hip when that directory cannot be written.
static std::string cache_dir() {
    const char* d = getenv("HB_CACHE_DIR");
    if (d) return d;
    Dl_info info;
    if (dladdr((void*)&cache_dir, &info) && info.dli_fname) {
        std::string lib = info.dli_fname;
        const size_t slash = lib.rfind('/');
        const std::string dir = (slash == std::string::npos ? std::string(".") : lib.substr(0, slash)) + "/_kcache";
        mkdir(dir.c_str(), 0755);
        if (access(dir.c_str(), W_OK) == 0) return dir;
    }
    const char* home = getenv("HOME");
    if (!home || !*home) return "";
    return std::string(home) + "/.cache/herbert_hip";
}

// HB_KERNEL_MANIFEST=path: every kernel a context builds appends its
// descriptor (the hb_desc fields in order, decimal) to that file, the list
// build.py precompiles.
static void manifest_add(const hb_desc& d) {
    const char* path = getenv("HB_KERNEL_MANIFEST");
    if (!path || !*path) return;
    std::ofstream f(path, std::ios::app);
    const uint32_t* w = (const uint32_t*)&d;
    for (size_t i = 0; i < sizeof(hb_desc) / 4; i++) f << (i ? " " : "") << w[i];
    f << "\n";
}

static void mkdirs(const std::string& p) {
    std::string cur;
    std::stringstream ss(p);
    std::string part;
    if (!p.empty() && p[0] == '/') cur = "/";
    while (std::getline(ss, part, '/')) {
        if (part.empty()) continue;
        cur += part + "/";
        mkdir(cur.c_str(), 0755);
    }
}

// Compiles `em` for `arch` with hiprtc; the code object into *code.
static int compile(const Emitted& em, const std::string& arch, std::string* code) {
    const char* text = source_text(em.source);
    if (!text) return fail(HB_ERR_COMPILE, "no embedded source " + em.source);
    std::vector<std::string> opts = {"--offload-arch=" + arch, "-O3", "-ffp-contract=off",
                                     "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
                                     "-packed-fp32-ops"};
    for (const auto& d : em.defines) opts.push_back(d);
    opts.push_back("-DHB_NAME=" + em.name);
    // The disk cache: the source, the headers (every embedded .h) and the
    // options hashed; an edit to another kernel source keeps this entry.
    std::string key = text;
    for (const auto& s : kSources) {
        const size_t len = strlen(s.name);
        if (len > 2 && strcmp(s.name + len - 2, ".h") == 0) key += s.text;
    }
    for (const auto& o : opts) key += "\n" + o;
    key += "\nhiprtc" + std::to_string(HIP_VERSION);
    char hex[32];
    snprintf(hex, sizeof hex, "%016llx", (unsigned long long)fnv1a(key));
    std::string dir = cache_dir();
    std::string path = dir.empty() ? "" : dir + "/" + em.name + "-" + hex + ".co";
    if (!path.empty()) {
        std::ifstream f(path, std::ios::binary);
        if (f) {
            std::stringstream b;
            b << f.rdbuf();
            *code = b.str();
            if (!code->empty()) {
                utime(path.c_str(), nullptr);  // in use: build.py keeps entries touched by its warm-up
                return HB_OK;
            }
        }
    }
    std::vector<const char*> hnames, htexts;
    for (const auto& s : kSources) {
        if (em.source == s.name) continue;
        hnames.push_back(s.name);
        htexts.push_back(s.text);
    }
    hiprtcProgram prog;
    hiprtcResult r = hiprtcCreateProgram(&prog, text, em.source.c_str(), (int)hnames.size(),
                                         htexts.data(), hnames.data());
    if (r != HIPRTC_SUCCESS)
        return fail(HB_ERR_COMPILE, std::string("hiprtcCreateProgram: ") + hiprtcGetErrorString(r));
    std::vector<const char*> copts;
    for (const auto& o : opts) copts.push_back(o.c_str());
    r = hiprtcCompileProgram(prog, (int)copts.size(), copts.data());
    if (r != HIPRTC_SUCCESS) {
        size_t n = 0;
        hiprtcGetProgramLogSize(prog, &n);
        std::string log(n, '\0');
        if (n) hiprtcGetProgramLog(prog, &log[0]);
        hiprtcDestroyProgram(&prog);
        // Keep the first error lines: the reason a candidate is "not built".
        std::string first;
        std::stringstream ls(log);
        std::string line;
        int kept = 0;
        while (std::getline(ls, line) && kept < 6) {
            if (line.find("error") != std::string::npos || kept) {
                first += line + "\n";
                kept++;
            }
        }
        return fail(HB_ERR_COMPILE, em.name + ": " + (first.empty() ? log : first));
    }
    size_t n = 0;
    hiprtcGetCodeSize(prog, &n);
    code->assign(n, '\0');
    hiprtcGetCode(prog, &(*code)[0]);
    hiprtcDestroyProgram(&prog);
    if (!path.empty()) {
        mkdirs(dir);
        std::string tmp = path + ".tmp" + std::to_string(getpid());
        {
            std::ofstream f(tmp, std::ios::binary);
            f.write(code->data(), (std::streamsize)code->size());
        }
        rename(tmp.c_str(), path.c_str());
    }
    return HB_OK;
}

static int load_kernel(hb_gpu* g, const hb_desc& d, Kernel* k) {
    k->desc = d;
    int rc = emit(d, &k->em);
    if (rc) return rc;
    manifest_add(d);
    auto t0 = std::chrono::steady_clock::now();
    std::string code;
    rc = compile(k->em, g->arch, &code);
    if (rc) return rc;
    HB_HIP(hipSetDevice(g->device));
    HB_HIP(hipModuleLoadData(&k->module, code.data()));
    HB_HIP(hipModuleGetFunction(&k->fn, k->module, k->em.name.c_str()));
    g->compile_seconds +=
        std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    return HB_OK;
}

// The context's workspace grown to `bytes` (the stream drained first: a
// launch in flight may still read the old one).
static int ensure_ws(hb_gpu* g, uint64_t bytes) {
    if (bytes <= g->ws_bytes) return HB_OK;
    if (g->graphs_live)
        return fail(HB_ERR_INVALID, "the split-K workspace cannot grow while a recorded graph holds its "
                                    "address (free the graphs first, or record after the largest launch)");
    HB_HIP(hipSetDevice(g->device));
    HB_HIP(hipStreamSynchronize(g->stream));
    if (g->ws) HB_HIP(hipFree(g->ws));
    g->ws = nullptr;
    g->ws_bytes = 0;
    const uint64_t sz = (bytes + (1ull << 20) - 1) & ~((1ull << 20) - 1);
    HB_HIP(hipMalloc(&g->ws, sz));
    g->ws_bytes = sz;
    return HB_OK;
}

static int launch_one(hb_gpu* g, const Kernel& k, void** ptrs, uint32_t nptr, uint32_t m,
                      uint32_t groups) {
    if (groups == 0) return HB_OK;
    // Kernel arguments: the binding pointers, then the launch's row count.
    void* args[12];
    for (uint32_t i = 0; i < nptr; i++) args[i] = &ptrs[i];
    args[nptr] = &m;
    HB_HIP(hipModuleLaunchKernel(k.fn, groups, 1, 1, k.em.threads, 1, 1, 0, g->stream, args,
                                 nullptr));
    return HB_OK;
}

// One launch of `k`; a split-K GEMM is two: the parts into the workspace
// (ensure_ws has sized it), then its reduce from there into Y.
static int launch_raw(hb_gpu* g, const Kernel& k, void** ptrs, uint32_t nptr, uint32_t m,
                      uint32_t groups) {
    if (k.reduce < 0) return launch_one(g, k, ptrs, nptr, m, groups);
    void* p[10];
    for (uint32_t i = 0; i < nptr; i++) p[i] = ptrs[i];
    p[3] = g->ws;
    int rc = launch_one(g, k, p, nptr, m, groups);
    if (rc) return rc;
    const Kernel& r = g->kernels[k.reduce];
    void* q[3] = {ptrs[0], g->ws, ptrs[3]};
    return launch_one(g, r, q, 3, m, groups_of(r.desc, m));
}

int launch_ptrs(hb_gpu* g, int32_t kernel, void* const* ptrs, const uint64_t* sizes, uint32_t nbind,
                uint32_t m) {
    if (kernel < 0 || (size_t)kernel >= g->kernels.size())
        return fail(HB_ERR_INVALID, "no kernel " + std::to_string(kernel));
    const Kernel& k = g->kernels[kernel];
    if (nbind != k.em.nbind)
        return fail(HB_ERR_INVALID, k.em.name + ": " + std::to_string(nbind) +
                                        " bindings given, it takes " + std::to_string(k.em.nbind));
    int rc = check_bindings(k.desc, sizes, nbind, m);
    if (rc) return fail(rc, k.em.name + ": " + hb_last_error());
    if ((rc = ensure_ws(g, workspace_of(k.desc, m)))) return rc;
    void* p[10];
    for (uint32_t i = 0; i < nbind; i++) p[i] = ptrs[i];
    return launch_raw(g, k, p, nbind, m, groups_of(k.desc, m));
}

const hb_desc* kernel_desc(hb_gpu* g, int32_t kernel) {
    if (kernel < 0 || (size_t)kernel >= g->kernels.size()) return nullptr;
    return &g->kernels[kernel].desc;
}

static int launch(hb_gpu* g, int32_t kernel, const hb_range* b, uint32_t nbind, uint32_t m) {
    if (nbind > 10) return fail(HB_ERR_INVALID, "more than 10 bindings");
    void* ptrs[10];
    uint64_t sizes[10];
    for (uint32_t i = 0; i < nbind; i++) {
        char* p;
        int rc = resolve(g, b[i], &p, &sizes[i]);
        if (rc) return rc;
        ptrs[i] = p;
    }
    return launch_ptrs(g, kernel, ptrs, sizes, nbind, m);
}

}  // namespace hb

using namespace hb;

extern "C" {

const char* hb_last_error(void) { return g_last_error.c_str(); }

int hb_open(int device, hb_gpu** out) {
    *out = nullptr;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0) return fail(HB_ERR_NO_DEVICE, "no HIP device");
    if (device < 0 || device >= n)
        return fail(HB_ERR_INVALID, "device " + std::to_string(device) + " of " + std::to_string(n));
    hb_gpu* g = new hb_gpu();
    g->device = device;
    hipDeviceProp_t p;
    if ((e = hipSetDevice(device)) != hipSuccess || (e = hipGetDeviceProperties(&p, device)) != hipSuccess) {
        delete g;
        return hip_fail(e, "hipGetDeviceProperties");
    }
    std::string arch = p.gcnArchName;
    g->arch = arch.substr(0, arch.find(':'));
    if (g->arch != "gfx950") {
        delete g;
        return fail(HB_ERR_UNSUPPORTED, "device " + std::to_string(device) + " is " + arch +
                                            ": the kernels are written for gfx950");
    }
    char buf[512];
    snprintf(buf, sizeof buf, "%s, %d CUs, %.1f GiB, %s, LDS %zu KiB/workgroup", p.name,
             p.multiProcessorCount, p.totalGlobalMem / 1073741824.0, p.gcnArchName,
             (size_t)p.sharedMemPerBlock / 1024);
    g->summary = buf;
    if ((e = hipStreamCreateWithFlags(&g->stream, hipStreamNonBlocking)) != hipSuccess ||
        (e = hipEventCreate(&g->ev0)) != hipSuccess || (e = hipEventCreate(&g->ev1)) != hipSuccess) {
        delete g;
        return hip_fail(e, "stream/event");
    }
    // The static scratch of hb_moe_experts_run_static on this device (the
    // device is current): its address, once per device.
    int rc = static_scratch(device, &g->scratch);
    if (rc) {
        hb_close(g);
        return rc;
    }
    *out = g;
    return HB_OK;
}

void hb_close(hb_gpu* g) {
    if (!g) return;
    hipSetDevice(g->device);
    hipStreamSynchronize(g->stream);
    for (auto& k : g->kernels)
        if (k.module) hipModuleUnload(k.module);
    if (g->zero_kernel.module) hipModuleUnload(g->zero_kernel.module);
    for (auto& b : g->bufs)
        if (b.live) hipFree(b.ptr);
    if (g->ws) hipFree(g->ws);
    hipEventDestroy(g->ev0);
    hipEventDestroy(g->ev1);
    hipStreamDestroy(g->stream);
    delete g;
}

const char* hb_device_summary(hb_gpu* g) { return g ? g->summary.c_str() : ""; }

int hb_alloc(hb_gpu* g, uint64_t bytes, hb_buf* out) {
    if (!bytes) return fail(HB_ERR_INVALID, "hb_alloc of 0 bytes");
    HB_HIP(hipSetDevice(g->device));
    Buffer b;
    // 256-byte aligned by hipMalloc; sizes rounded up to 256 so 128-bit
    // loads of a last partial chunk stay inside the allocation.
    HB_HIP(hipMalloc(&b.ptr, (bytes + 255) & ~255ull));
    b.size = bytes;
    b.live = true;
    g->bufs.push_back(b);
    *out = (hb_buf)(g->bufs.size() - 1);
    return HB_OK;
}

int hb_free(hb_gpu* g, hb_buf buf) {
    if (buf >= g->bufs.size() || !g->bufs[buf].live)
        return fail(HB_ERR_INVALID, "hb_free: no buffer " + std::to_string(buf));
    HB_HIP(hipStreamSynchronize(g->stream));
    HB_HIP(hipFree(g->bufs[buf].ptr));
    g->bufs[buf].live = false;
    g->bufs[buf].ptr = nullptr;
    return HB_OK;
}

int hb_buffer_ptr(hb_gpu* g, hb_buf buf, void** ptr) {
    if (buf >= g->bufs.size() || !g->bufs[buf].live)
        return fail(HB_ERR_INVALID, "no buffer " + std::to_string(buf));
    *ptr = g->bufs[buf].ptr;
    return HB_OK;
}

int hb_upload(hb_gpu* g, hb_buf buf, uint64_t offset, const void* src, uint64_t bytes) {
    hb_range r{buf, 0, offset, bytes};
    char* p;
    uint64_t n;
    int rc = resolve(g, r, &p, &n);
    if (rc) return rc;
    HB_HIP(hipMemcpyAsync(p, src, bytes, hipMemcpyHostToDevice, g->stream));
    HB_HIP(hipStreamSynchronize(g->stream));
    return HB_OK;
}

int hb_download(hb_gpu* g, hb_buf buf, uint64_t offset, void* dst, uint64_t bytes) {
    hb_range r{buf, 0, offset, bytes};
    char* p;
    uint64_t n;
    int rc = resolve(g, r, &p, &n);
    if (rc) return rc;
    HB_HIP(hipMemcpyAsync(dst, p, bytes, hipMemcpyDeviceToHost, g->stream));
    HB_HIP(hipStreamSynchronize(g->stream));
    return HB_OK;
}

int hb_copy(hb_gpu* g, hb_range dst, hb_range src) {
    char *pd, *ps;
    uint64_t nd, ns;
    int rc = resolve(g, dst, &pd, &nd);
    if (rc || (rc = resolve(g, src, &ps, &ns))) return rc;
    if (nd != ns) return fail(HB_ERR_INVALID, "hb_copy: ranges of different sizes");
    if ((pd < ps + ns) && (ps < pd + nd) && nd) return fail(HB_ERR_INVALID, "hb_copy: ranges overlap");
    HB_HIP(hipMemcpyAsync(pd, ps, nd, hipMemcpyDeviceToDevice, g->stream));
    return HB_OK;
}

int hb_zero(hb_gpu* g, hb_buf buf, uint64_t offset, uint64_t bytes) {
    hb_range r{buf, 0, offset, bytes};
    char* p;
    uint64_t n;
    int rc = resolve(g, r, &p, &n);
    if (rc) return rc;
    if (!g->zero_built) {
        hb_desc d{};
        d.kind = 0xffff;  // the fill kernel (emit's internal kind)
        rc = load_kernel(g, d, &g->zero_kernel);
        if (rc) return rc;
        g->zero_built = true;
    }
    // One thread per 16-byte-aligned word of the span; the kernel zeroes a
    // ragged first or last word byte by byte.
    if (n) {
        const uint64_t words = (((uint64_t)p + n + 15) >> 4) - ((uint64_t)p >> 4);
        const uint64_t groups = (words + 255) / 256;
        if (groups > 0x7fffffffull) return fail(HB_ERR_INVALID, "hb_zero: too large");
        void* ptr = p;
        void* args[2] = {&ptr, &n};
        HB_HIP(hipModuleLaunchKernel(g->zero_kernel.fn, (uint32_t)groups, 1, 1, 256, 1, 1, 0,
                                     g->stream, args, nullptr));
    }
    return HB_OK;
}

int hb_kernel_precompile(const hb_desc* desc) {
    hb_desc d = with_defaults(*desc);
    Emitted em;
    int rc = emit(d, &em);
    if (rc) return rc;
    std::string code;
    if ((rc = compile(em, "gfx950", &code))) return rc;
    if (d.kind == HB_KIND_GEMM && d.ksplit > 1) {
        hb_desc rd{};
        rd.kind = KIND_SPLITK_REDUCE;
        rd.n = d.n;
        rd.out = d.out;
        rd.ksplit = d.ksplit;
        return hb_kernel_precompile(&rd);
    }
    return HB_OK;
}

int hb_kernel_build(hb_gpu* g, const hb_desc* desc, int32_t* kernel) {
    hb_desc d = with_defaults(*desc);
    Emitted em;
    int rc = emit(d, &em);
    if (rc) return rc;
    auto it = g->by_name.find(em.name);
    if (it != g->by_name.end()) {
        *kernel = it->second;
        return HB_OK;
    }
    Kernel k;
    rc = load_kernel(g, d, &k);
    if (rc) return rc;
    if (d.kind == HB_KIND_GEMM && d.ksplit > 1) {
        // Its second kernel, built (or found) first.
        hb_desc rd{};
        rd.kind = KIND_SPLITK_REDUCE;
        rd.n = d.n;
        rd.out = d.out;
        rd.ksplit = d.ksplit;
        if ((rc = hb_kernel_build(g, &rd, &k.reduce))) {
            hipModuleUnload(k.module);
            return rc;
        }
    }
    g->kernels.push_back(k);
    *kernel = (int32_t)(g->kernels.size() - 1);
    g->by_name[em.name] = *kernel;
    return HB_OK;
}

const char* hb_kernel_name(hb_gpu* g, int32_t kernel) {
    if (kernel < 0 || (size_t)kernel >= g->kernels.size()) return "";
    return g->kernels[kernel].em.name.c_str();
}

uint32_t hb_kernel_groups(hb_gpu* g, int32_t kernel, uint32_t m) {
    if (kernel < 0 || (size_t)kernel >= g->kernels.size()) return 0;
    return groups_of(g->kernels[kernel].desc, m);
}

uint32_t hb_kernel_bindings(hb_gpu* g, int32_t kernel) {
    if (kernel < 0 || (size_t)kernel >= g->kernels.size()) return 0;
    return g->kernels[kernel].em.nbind;
}

uint32_t hb_kernel_kind(hb_gpu* g, int32_t kernel) {
    if (kernel < 0 || (size_t)kernel >= g->kernels.size()) return 0;
    return g->kernels[kernel].desc.kind;
}

double hb_compile_seconds(hb_gpu* g) { return g->compile_seconds; }

int hb_launch(hb_gpu* g, int32_t kernel, const hb_range* b, uint32_t nbind, uint32_t m) {
    return launch(g, kernel, b, nbind, m);
}

int hb_time(hb_gpu* g, const hb_op* ops, uint32_t nops, uint32_t reps, double* seconds) {
    return hb_time_each(g, ops, nops, reps, seconds, nullptr);
}

}  // extern "C"

namespace hb {
// Ops checked once and resolved to what a launch needs (the split-K
// workspace sized for them), so they can be launched without re-checking.
struct Ready {
    const Kernel* k;
    void* ptrs[10];
    uint32_t n, m, groups;
};

static int prepare(hb_gpu* g, const hb_op* ops, uint32_t nops, std::vector<Ready>* out) {
    std::vector<Ready>& ready = *out;
    ready.resize(nops);
    for (uint32_t i = 0; i < nops; i++) {
        const hb_op& op = ops[i];
        if (op.kernel < 0 || (size_t)op.kernel >= g->kernels.size())
            return fail(HB_ERR_INVALID, "no kernel " + std::to_string(op.kernel));
        const Kernel& k = g->kernels[op.kernel];
        if (op.nbind != k.em.nbind || op.nbind > 8)
            return fail(HB_ERR_INVALID, k.em.name + ": wrong number of bindings");
        uint64_t sizes[10];
        for (uint32_t j = 0; j < op.nbind; j++) {
            char* p;
            int rc = resolve(g, op.bind[j], &p, &sizes[j]);
            if (rc) return rc;
            ready[i].ptrs[j] = p;
        }
        int rc = check_bindings(k.desc, sizes, op.nbind, op.m);
        if (rc) return fail(rc, k.em.name + ": " + hb_last_error());
        if ((rc = ensure_ws(g, workspace_of(k.desc, op.m)))) return rc;
        ready[i].k = &k;
        ready[i].n = op.nbind;
        ready[i].m = op.m;
        ready[i].groups = groups_of(k.desc, op.m);
    }
    return HB_OK;
}
}  // namespace hb

extern "C" {

int hb_time_each(hb_gpu* g, const hb_op* ops, uint32_t nops, uint32_t reps, double* seconds,
                 double* op_seconds) {
    std::vector<Ready> ready;
    int prc = prepare(g, ops, nops, &ready);
    if (prc) return prc;
    if (!op_seconds) {
        HB_HIP(hipEventRecord(g->ev0, g->stream));
        for (uint32_t r = 0; r < reps; r++)
            for (auto& x : ready) {
                int rc = launch_raw(g, *x.k, x.ptrs, x.n, x.m, x.groups);
                if (rc) return rc;
            }
        HB_HIP(hipEventRecord(g->ev1, g->stream));
        HB_HIP(hipEventSynchronize(g->ev1));
        float ms = 0;
        HB_HIP(hipEventElapsedTime(&ms, g->ev0, g->ev1));
        *seconds = ms * 1e-3;
        return HB_OK;
    }
    // An event between consecutive launches (the same stream, so the
    // launches still run back to back): event i..i+1 brackets launch i.
    const size_t nev = (size_t)reps * nops + 1;
    std::vector<hipEvent_t> ev(nev, nullptr);
    int rc = HB_OK;
    hipError_t he = hipSuccess;
    for (auto& e : ev)
        if ((he = hipEventCreate(&e)) != hipSuccess) {
            rc = hip_fail(he, "hipEventCreate");
            break;
        }
    size_t at = 0;
    if (!rc && (he = hipEventRecord(ev[at++], g->stream)) != hipSuccess) rc = hip_fail(he, "hipEventRecord");
    for (uint32_t r = 0; r < reps && !rc; r++)
        for (auto& x : ready) {
            if ((rc = launch_raw(g, *x.k, x.ptrs, x.n, x.m, x.groups))) break;
            if ((he = hipEventRecord(ev[at++], g->stream)) != hipSuccess) {
                rc = hip_fail(he, "hipEventRecord");
                break;
            }
        }
    if (!rc && (he = hipEventSynchronize(ev[nev - 1])) != hipSuccess) rc = hip_fail(he, "hipEventSynchronize");
    if (!rc) {
        for (uint32_t i = 0; i < nops; i++) op_seconds[i] = 0;
        float ms = 0;
        for (size_t j = 0; j + 1 < nev && !rc; j++) {
            if ((he = hipEventElapsedTime(&ms, ev[j], ev[j + 1])) != hipSuccess) rc = hip_fail(he, "hipEventElapsedTime");
            op_seconds[j % nops] += ms * 1e-3 / reps;
        }
        if (!rc && (he = hipEventElapsedTime(&ms, ev[0], ev[nev - 1])) != hipSuccess) rc = hip_fail(he, "hipEventElapsedTime");
        *seconds = ms * 1e-3;
    }
    for (auto& e : ev)
        if (e) hipEventDestroy(e);
    return rc;
}

// A recorded op sequence: the ops captured from the context's stream into a
// HIP graph (kernel nodes only: nothing here records a memset) and
// instantiated once, then replayed with one launch per run.
struct hb_graph {
    hb_gpu* g = nullptr;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

int hb_graph_record(hb_gpu* g, const hb_op* ops, uint32_t nops, hb_graph** out) {
    *out = nullptr;
    if (!nops) return fail(HB_ERR_INVALID, "hb_graph_record: no ops");
    std::vector<Ready> ready;
    int rc = prepare(g, ops, nops, &ready);  // sizes the split-K workspace before the capture
    if (rc) return rc;
    HB_HIP(hipSetDevice(g->device));
    HB_HIP(hipStreamBeginCapture(g->stream, hipStreamCaptureModeThreadLocal));
    for (auto& x : ready)
        if ((rc = launch_raw(g, *x.k, x.ptrs, x.n, x.m, x.groups))) break;
    hipGraph_t graph = nullptr;
    hipError_t he = hipStreamEndCapture(g->stream, &graph);
    if (rc || he != hipSuccess) {
        if (graph) hipGraphDestroy(graph);
        return rc ? rc : hip_fail(he, "hipStreamEndCapture");
    }
    hipGraphExec_t exec = nullptr;
    if ((he = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0)) != hipSuccess) {
        hipGraphDestroy(graph);
        return hip_fail(he, "hipGraphInstantiate");
    }
    hb_graph* r = new hb_graph();
    r->g = g;
    r->graph = graph;
    r->exec = exec;
    g->graphs_live++;
    *out = r;
    return HB_OK;
}

int hb_graph_launch(hb_graph* gr, uint32_t reps) {
    for (uint32_t i = 0; i < reps; i++) HB_HIP(hipGraphLaunch(gr->exec, gr->g->stream));
    return HB_OK;
}

int hb_graph_time(hb_graph* gr, uint32_t reps, double* seconds) {
    hb_gpu* g = gr->g;
    HB_HIP(hipEventRecord(g->ev0, g->stream));
    for (uint32_t i = 0; i < reps; i++) HB_HIP(hipGraphLaunch(gr->exec, g->stream));
    HB_HIP(hipEventRecord(g->ev1, g->stream));
    HB_HIP(hipEventSynchronize(g->ev1));
    float ms = 0;
    HB_HIP(hipEventElapsedTime(&ms, g->ev0, g->ev1));
    *seconds = ms * 1e-3;
    return HB_OK;
}

void hb_graph_free(hb_graph* gr) {
    if (!gr) return;
    hipStreamSynchronize(gr->g->stream);
    if (gr->exec) hipGraphExecDestroy(gr->exec);
    if (gr->graph) hipGraphDestroy(gr->graph);
    gr->g->graphs_live--;
    delete gr;
}

int hb_sync(hb_gpu* g) {
    HB_HIP(hipStreamSynchronize(g->stream));
    return HB_OK;
}

}  // extern "C"
