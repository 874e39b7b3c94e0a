"""Builds libherbert_hip.so in this directory: the C++ host runtime (HIP +
hiprtc) with the HIP kernel sources embedded as text for hiprtc to compile at
load, and checks every kernel source compiles for gfx950 with hipcc; then
hb_gemm, a native command-line host of the C ABI linked against it.

    python herbert-metal-bf16_amd/build.py [--no-check]

Kernel development only: `--dev --kdir DIR --lib PATH` builds a separate
library at PATH from the kernel sources in DIR, with the HB_DEV_DEFINES hook
compiled in (extra -D constants for every kernel built while it is set).
The shipped libherbert_hip.so never has that hook.
"""
import os
import subprocess
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
KDIR = os.path.join(CSRC, "kernels")
OUT_DIR = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libherbert_hip.so")
CLI = os.path.join(HERE, "hb_gemm")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
HOST_SOURCES = ["hb_runtime.cpp", "hb_emit.cpp", "hb_select.cpp", "hb_fill.cpp", "hb_checkpoint.cpp",
                "hb_moe.cpp", "hb_static.hip"]
# Compile-only checks of each kernel source with representative constants
# (hiprtc compiles the real shapes at load).
CHECKS = {
    "gemm_mfma.hip": [
        "-DHB_K=2560 -DHB_N=4608 -DHB_OUT=0 -DHB_ROWS=0 -DHB_TOPK=1 -DHB_BM=128 -DHB_BN=192 "
        "-DHB_BK=64 -DHB_WM=2 -DHB_WN=4 -DHB_MFMA=16 -DHB_STAGES=3 -DHB_SWZ=1 -DHB_ORDER=1 -DHB_MFIRST=1 -DHB_DMA=1",
        "-DHB_K=2048 -DHB_N=1024 -DHB_OUT=2 -DHB_ROWS=1 -DHB_TOPK=8 -DHB_BM=16 -DHB_BN=128 "
        "-DHB_BK=64 -DHB_WM=1 -DHB_WN=4 -DHB_MFMA=16 -DHB_STAGES=1 -DHB_SWZ=1 -DHB_ORDER=0 -DHB_MFIRST=1 -DHB_DMA=0",
        "-DHB_K=2560 -DHB_N=9216 -DHB_OUT=0 -DHB_ROWS=0 -DHB_TOPK=1 -DHB_BM=128 -DHB_BN=128 "
        "-DHB_BK=64 -DHB_WM=2 -DHB_WN=2 -DHB_MFMA=16 -DHB_STAGES=2 -DHB_SWZ=1 -DHB_ORDER=1 -DHB_MFIRST=1 -DHB_DMA=1 "
        "-DHB_SWIGLU=1 -DHB_BAND=2",
        "-DHB_K=9216 -DHB_N=2560 -DHB_OUT=1 -DHB_ROWS=0 -DHB_TOPK=1 -DHB_BM=128 -DHB_BN=160 "
        "-DHB_BK=64 -DHB_WM=2 -DHB_WN=2 -DHB_MFMA=16 -DHB_STAGES=4 -DHB_SWZ=1 -DHB_ORDER=1 -DHB_MFIRST=1 -DHB_DMA=1 "
        "-DHB_KSPLIT=3",
    ],
    "gemm_splitk.hip": ["-DHB_N=2560 -DHB_OUT=2 -DHB_KSPLIT=3", "-DHB_N=3584 -DHB_OUT=0 -DHB_KSPLIT=2"],
    "gemm_pp.hip": [
        "-DHB_K=2560 -DHB_N=18432 -DHB_OUT=0 -DHB_BM=256 -DHB_BN=256 -DHB_BK=32 -DHB_WM=4 -DHB_WN=2 "
        "-DHB_MFMA=16 -DHB_STAGES=4 -DHB_SWZ=2 -DHB_ORDER=1 -DHB_MFIRST=1 -DHB_BAND=4 -DHB_GRP=0",
        "-DHB_K=9216 -DHB_N=2560 -DHB_OUT=2 -DHB_BM=256 -DHB_BN=192 -DHB_BK=32 -DHB_WM=4 -DHB_WN=2 "
        "-DHB_MFMA=32 -DHB_STAGES=3 -DHB_SWZ=2 -DHB_ORDER=1 -DHB_MFIRST=1 -DHB_BAND=0 -DHB_GRP=1",
        "-DHB_K=2560 -DHB_N=18432 -DHB_OUT=0 -DHB_BM=256 -DHB_BN=288 -DHB_BK=32 -DHB_WM=2 -DHB_WN=2 "
        "-DHB_MFMA=16 -DHB_STAGES=4 -DHB_SWZ=2 -DHB_ORDER=1 -DHB_MFIRST=1 -DHB_BAND=4 -DHB_SCHED=3",
    ],
    "mv_chain.hip": ["-DHB_MV_M=4 -DHB_NPH=5 -DHB_PH_K=2560,4096,2560,9216,2560 "
                     "-DHB_PH_N=4608,2560,18432,2560,151936 -DHB_PH_OUT=0,2,0,2,0 -DHB_CPL=18",
                     "-DHB_MV_M=8 -DHB_NPH=3 -DHB_PH_K=512,1536,1024 -DHB_PH_N=1536,1024,700 "
                     "-DHB_PH_OUT=0,2,1 -DHB_CPL=3"],
    "fill.hip": [""],
    "probe.hip": [""],
    "gemm_simt.hip": ["-DHB_K=2560 -DHB_N=4608 -DHB_OUT=2 -DHB_MFIRST=1"],
    "gemm_direct.hip": ["-DHB_K=2560 -DHB_N=4608 -DHB_OUT=0 -DHB_BM=64 -DHB_BN=32 -DHB_MFIRST=1"],
    "moe.hip": ["-DHB_OP=%d -DHB_E=256 -DHB_TOPK=8 -DHB_BM=32 -DHB_D=2048 -DHB_RMAX=2048" % op for op in range(1, 9)]
    + ["-DHB_OP=%d -DHB_E=200 -DHB_TOPK=6 -DHB_BM=16 -DHB_D=2048 -DHB_RMAX=8192" % op for op in (2, 3)],
    "matvec.hip": [
        "-DHB_K=2560 -DHB_N=151936 -DHB_OUT=0 -DHB_MV_M=1 -DHB_FORM=0 -DHB_ROWS=4 -DHB_SPLIT=1 -DHB_PERSIST=0 -DHB_UNROLL=4",
        "-DHB_K=9216 -DHB_N=2560 -DHB_OUT=2 -DHB_MV_M=8 -DHB_FORM=1 -DHB_ROWS=16 -DHB_SPLIT=4 -DHB_PERSIST=512 -DHB_UNROLL=4",
        "-DHB_K=9216 -DHB_N=2560 -DHB_OUT=2 -DHB_MV_M=8 -DHB_FORM=2 -DHB_ROWS=1 -DHB_SPLIT=1 -DHB_PERSIST=256 "
        "-DHB_UNROLL=4 -DHB_XLDS=1 -DHB_WAVES=16",
        "-DHB_K=2560 -DHB_N=151936 -DHB_OUT=0 -DHB_MV_M=8 -DHB_FORM=3 -DHB_ROWS=16 -DHB_SPLIT=4 -DHB_PERSIST=0 -DHB_UNROLL=8",
        "-DHB_K=2560 -DHB_N=4608 -DHB_OUT=0 -DHB_MV_M=4 -DHB_FORM=4 -DHB_ROWS=4 -DHB_SPLIT=2 -DHB_PERSIST=1024 "
        "-DHB_UNROLL=4 -DHB_WAVES=8",
        "-DHB_K=9216 -DHB_N=2560 -DHB_OUT=2 -DHB_MV_M=8 -DHB_FORM=4 -DHB_ROWS=4 -DHB_SPLIT=8 -DHB_PERSIST=0 "
        "-DHB_UNROLL=4 -DHB_WAVES=16",
    ],
}
DEVICE_FLAGS = ["--offload-arch=gfx950", "-O3", "-ffp-contract=off", "-std=c++17",
                "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def embed_sources(kdir=KDIR, out_dir=OUT_DIR):
    """Writes hb_sources.inc: every kernel source as a raw string."""
    os.makedirs(out_dir, exist_ok=True)
    names = sorted(f for f in os.listdir(kdir) if f.endswith((".hip", ".h")))
    lines = ["// generated by build.py: the HIP kernel sources hiprtc compiles at load",
             "struct HbSource { const char* name; const char* text; };",
             "static const HbSource kSources[] = {"]
    for n in names:
        text = open(os.path.join(kdir, n)).read()
        assert ")HBSRC\"" not in text
        lines.append('    {"%s", R"HBSRC(%s)HBSRC"},' % (n, text))
    lines.append("};")
    path = os.path.join(out_dir, "hb_sources.inc")
    new = "\n".join(lines) + "\n"
    if not os.path.exists(path) or open(path).read() != new:
        open(path, "w").write(new)
    return names


def check_kernels(jobs=8):
    """hipcc --cuda-device-only of every kernel source, in parallel."""
    procs = []
    for src, variants in CHECKS.items():
        for i, defs in enumerate(variants):
            out = os.path.join(OUT_DIR, "%s.%d.o" % (src, i))
            cmd = [HIPCC, *DEVICE_FLAGS, "--cuda-device-only", "-c", "-include", "hip/hip_runtime.h",
                   "-I", KDIR, "-x", "hip", os.path.join(KDIR, src), "-o", out] + defs.split()
            procs.append((src, defs, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
            if len(procs) >= jobs:
                _wait(procs.pop(0))
    for p in procs:
        _wait(p)


def _wait(p):
    src, defs, proc = p
    out = proc.communicate()[0].decode(errors="replace")
    if proc.returncode != 0:
        raise RuntimeError("kernel %s (%s) does not compile for gfx950:\n%s" % (src, defs, out))


def build_host(out_dir=OUT_DIR, lib=LIB, dev=False):
    objs = []
    procs = []
    for s in HOST_SOURCES:
        o = os.path.join(out_dir, s + ".o")
        cmd = [HIPCC, "-O2", "-std=c++17", "-fPIC", "-Wall", "-c", os.path.join(CSRC, s),
               "-I", CSRC, "-I", INCLUDE, "-I", out_dir, "-o", o] + (["-DHB_DEV_BUILD"] if dev else [])
        if s.endswith(".hip"):
            # Device code of the library itself (the static scratch): gfx950.
            cmd[1:1] = ["-x", "hip", "--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang",
                        "-packed-fp32-ops"]
        procs.append((s, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
        objs.append(o)
    for s, p in procs:
        out = p.communicate()[0].decode(errors="replace")
        if p.returncode != 0:
            raise RuntimeError("host source %s does not compile:\n%s" % (s, out))
    tmp = lib + ".tmp"
    cmd = [HIPCC, "-shared", "-fPIC", "-o", tmp, *objs, "-lhiprtc", "-lpthread", "-ldl",
           "-Wl,-soname,libherbert_hip.so"]
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stdout.decode(errors="replace"))
    os.replace(tmp, lib)
    if dev:
        return
    # hb_gemm: a native host of the C ABI, linked against the library.
    cli_tmp = CLI + ".tmp"
    cmd = [HIPCC, "-O2", "-std=c++17", "-Wall", os.path.join(CSRC, "hb_cli.cpp"), "-I", INCLUDE,
           "-L", HERE, "-lherbert_hip", "-Wl,-rpath,$ORIGIN", "-o", cli_tmp]
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    if r.returncode != 0:
        raise RuntimeError("hb_gemm does not build:\n" + r.stdout.decode(errors="replace"))
    os.replace(cli_tmp, CLI)


MANIFEST = os.path.join(HERE, "kernel_manifest.txt")
KCACHE = os.path.join(HERE, "_kcache")


def _precompile_part(lines):
    """One worker: hb_kernel_precompile of each descriptor line (the
    library's own hiprtc path and cache key; no GPU is touched)."""
    import ctypes
    lib = ctypes.CDLL(LIB)
    lib.hb_last_error.restype = ctypes.c_char_p
    failed = []
    for ln in lines:
        words = [int(w) for w in ln.split()]
        desc = (ctypes.c_uint32 * len(words))(*words)
        if lib.hb_kernel_precompile(desc) != 0:
            failed.append((ln, lib.hb_last_error().decode(errors="replace")))
    return failed


def precompile(manifest=MANIFEST, procs=None):
    """Fills the kernel cache beside the library (_kcache) with every kernel
    the manifest lists -- the kernels the bench and the GPU tests build,
    recorded from a GPU run with HB_KERNEL_MANIFEST set -- compiled in
    parallel processes, so a fresh GPU box loads them instead of compiling
    them at load (minutes of hiprtc).  Descriptors the library refuses are
    reported and skipped; a kernel missing from the cache is compiled at
    load as before."""
    if not os.path.exists(manifest):
        return 0, 0
    if HERE not in sys.path:
        sys.path.insert(0, HERE)
    import herbert_hip as hb  # loads the library: fails here, not in the workers
    nfields = len(hb.Desc._fields_)
    lines = []
    seen = set()
    for ln in open(manifest):
        ln = ln.strip()
        if ln and not ln.startswith("#") and ln not in seen and len(ln.split()) == nfields:
            seen.add(ln)
            lines.append(ln)
    from concurrent.futures import ProcessPoolExecutor
    procs = procs or max(1, min(16, os.cpu_count() or 1))
    t0 = time.time() - 2
    parts = [lines[i::procs] for i in range(procs)]
    old = os.environ.get("HB_CACHE_DIR")
    os.environ["HB_CACHE_DIR"] = KCACHE
    try:
        with ProcessPoolExecutor(procs) as ex:
            failed = [f for part in ex.map(_precompile_part, parts) for f in part]
    finally:
        if old is None:
            del os.environ["HB_CACHE_DIR"]
        else:
            os.environ["HB_CACHE_DIR"] = old
    # Entries the manifest did not touch (kernels of older sources, or ones
    # compiled at load and not listed) are dropped: the cache travels with
    # the tree.
    if os.path.isdir(KCACHE):
        for f in os.listdir(KCACHE):
            fp = os.path.join(KCACHE, f)
            if f.endswith(".co") and os.path.getmtime(fp) < t0:
                os.remove(fp)
    for ln, err in failed[:5]:
        print("precompile: not built: %s (%s)" % (ln, err.splitlines()[0] if err else ""), file=sys.stderr)
    return len(lines), len(failed)


def build(check=True):
    t = time.time()
    embed_sources()
    if check:
        check_kernels()
    build_host()
    n, bad = precompile()
    if n:
        print("kernel cache: %d kernels from %s (%d not built)" % (n, os.path.basename(MANIFEST), bad))
    return time.time() - t


def build_dev(kdir, lib):
    out_dir = os.path.join(os.path.dirname(os.path.abspath(lib)), "_build_dev")
    embed_sources(kdir, out_dir)
    build_host(out_dir, os.path.abspath(lib), dev=True)


if __name__ == "__main__":
    if "--dev" in sys.argv:
        a = sys.argv
        build_dev(a[a.index("--kdir") + 1], a[a.index("--lib") + 1])
        print("built the development library", a[a.index("--lib") + 1])
    else:
        dt = build(check="--no-check" not in sys.argv)
        print("built %s in %.1f s" % (LIB, dt))
