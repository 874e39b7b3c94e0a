// hb_internal.h -- the host library's internal types: the context (the
// reference's Gpu, src/metal/gpu.rs:22-124), the kernel descriptor's emitted
// form (Emitted, src/msl/mod.rs:1461-1475) and the error channel.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

#include "herbert_hip.h"

namespace hb {

// Sets the thread's last error and returns `code`.
int fail(int code, const std::string& msg);
int hip_fail(hipError_t e, const char* what);

#define HB_HIP(call)                                     \
    do {                                                 \
        hipError_t e_ = (call);                          \
        if (e_ != hipSuccess) return hb::hip_fail(e_, #call); \
    } while (0)

// What a descriptor emits: the kernel's name (its cache key, as the
// reference's Emitted::name), the source file and the -D constants hiprtc
// compiles it with, its workgroup size and its bindings.
struct Emitted {
    std::string name;
    std::string source;               // file name among the embedded sources
    std::vector<std::string> defines; // "-DHB_K=2560", ...
    uint32_t threads = 256;
    uint32_t nbind = 0;
};

// Fills `e` for `d`, or returns an error (descriptor not implemented).
int emit(const hb_desc& d, Emitted* e);
// Workgroups of a launch of `d` over m rows (the reference's xxx_groups).
uint32_t groups_of(const hb_desc& d, uint32_t m);
// Checks the bindings' byte sizes against what `d` reads and writes over m
// rows; returns HB_OK or an error naming the binding.
int check_bindings(const hb_desc& d, const uint64_t* sizes, uint32_t nbind, uint32_t m);
// Fills defaults of the descriptor's zero fields (tile sizes, ...).
hb_desc with_defaults(const hb_desc& d);

struct Buffer {
    void* ptr = nullptr;
    uint64_t size = 0;
    bool live = false;
};

struct Kernel {
    hb_desc desc;
    Emitted em;
    hipModule_t module = nullptr;
    hipFunction_t fn = nullptr;
    // A split-K GEMM (desc.ksplit > 1): the kernel that adds its parts'
    // slabs and applies Out, launched after it by every launch of this one.
    int32_t reduce = -1;
};

// The descriptor kind of a split-K GEMM's second kernel (built by the
// library with its GEMM, never named by a caller).
constexpr uint32_t KIND_SPLITK_REDUCE = 0xfffe;
// Workspace bytes a launch of `d` over m rows needs (split-K slabs), 0 if none.
uint64_t workspace_of(const hb_desc& d, uint32_t m);

}  // namespace hb

struct hb_gpu {
    int device = 0;
    hipStream_t stream = nullptr;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    std::vector<hb::Buffer> bufs;
    std::vector<hb::Kernel> kernels;
    std::unordered_map<std::string, int32_t> by_name;
    std::string summary;
    std::string arch;
    double compile_seconds = 0.0;
    hb::Kernel zero_kernel;  // the fill kernel of hb_zero
    bool zero_built = false;
    // The selection layer's cache flush (a SwiGLU pass over 384 MiB, more
    // than the 256 MiB last-level cache), built on first use.
    hb_buf flush_gu = 0, flush_h = 0;
    int32_t flush_kernel = -1;
    // The device address of the library's static scratch on this device
    // (hb_static.hip), taken at hb_open.
    void* scratch = nullptr;
    // The split-K GEMMs' slabs: one workspace for every launch on the
    // context's stream (launches are in stream order, so one split GEMM's
    // second kernel has read the slabs before the next GEMM writes them),
    // grown before a launch that needs more, freed at hb_close.
    void* ws = nullptr;
    uint64_t ws_bytes = 0;
    // Recorded graphs alive on this context: they hold the workspace's
    // address, so it may not be reallocated meanwhile.
    int graphs_live = 0;
};

namespace hb {
// Resolves a range to a device pointer and byte size (size 0 = to the end).
int resolve(hb_gpu* g, const hb_range& r, char** ptr, uint64_t* size);
// hb_launch over device pointers and their byte sizes (checked against the
// kernel's descriptor and m first).
int launch_ptrs(hb_gpu* g, int32_t kernel, void* const* ptrs, const uint64_t* sizes, uint32_t nbind,
                uint32_t m);
// The descriptor a kernel was built from (defaults filled), or null.
const hb_desc* kernel_desc(hb_gpu* g, int32_t kernel);
// The device address of the static scratch (hb_static.hip) on `device`,
// which must be current: looked up, and its state word written, once per
// device.
int static_scratch(int device, void** out);
// The routed experts of an MoE layer over device pointers (hb_moe.cpp):
// bindings in hb_moe_io's order (state, route, list, tiles, x, w_gate_up,
// egu, ehb, w_down, ey, xs), then out.
int moe_experts_run(hb_gpu* g, const int32_t kernels[4], int32_t swiglu, int32_t combine,
                    void* const ptr[12], const uint64_t size[12], uint32_t m);
}  // namespace hb
