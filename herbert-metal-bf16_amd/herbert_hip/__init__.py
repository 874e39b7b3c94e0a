"""herbert_hip -- the Python host side of the MI355X bf16 matrix-multiplication
path of herbert-metal-bf16, over the C ABI of libherbert_hip.so
(include/herbert_hip.h) through ctypes.

It mirrors the reference's Rust interface for this path, same names and
argument meaning:
  - Gpu            src/metal/gpu.rs:22-277 (open, alloc, alloc_with, pipeline,
                   dispatch, submit_wait -> here launch / time_ops / sync)
  - Range          src/metal/gpu.rs:40-57
  - Out, MmaRows   src/metal/kernels.rs:30-43, src/metal/prefill.rs:317-338
  - the emitters   gemm_mma_rows / gemm_mma_form (prefill.rs:418-431),
                   gemm_simt (:133), gemm_mm2d (:442), gemm_nax_swiglu (:755),
                   matvec / matvec_split (kernels.rs:146, 502), route_qwen,
                   swiglu_slots, moe_combine (qwen_kernels.rs:1802, 2087,
                   2119), moe_sort / moe_sort_atomic / moe_gather
                   (prefill.rs:1315, 1450, 579): here they return a Desc,
                   which Gpu.pipeline compiles (hiprtc, gfx950).
  - Engine         the kernel-selection part of QwenEngine (qwen.rs): gemm,
                   mv_full, expert_pipes, Tune.

Errors raise HerbertError with the library's message (the reference's
HerbertError::Backend(String), src/core/error.rs:9-27).  Nothing here falls
back to the CPU: without libherbert_hip.so, importing the package raises.
"""
import ctypes
import enum
import struct
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(os.path.dirname(_HERE), "libherbert_hip.so")


# Status codes (include/herbert_hip.h).
HB_ERR_INVALID, HB_ERR_HIP, HB_ERR_COMPILE, HB_ERR_UNSUPPORTED, HB_ERR_NO_DEVICE = -1, -2, -3, -4, -5


class HerbertError(RuntimeError):
    """A failing library call: the status code and the library's message."""

    def __init__(self, code, msg):
        super().__init__("herbert_hip error %d: %s" % (code, msg))
        self.code = code
        self.msg = msg


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            "libherbert_hip.so is not built (%s): run `python herbert-metal-bf16_amd/build.py` "
            "or __graft_entry__.build()" % LIB_PATH)
    return ctypes.CDLL(LIB_PATH)


lib = _load()

OK, ERR_INVALID, ERR_HIP, ERR_COMPILE, ERR_UNSUPPORTED, ERR_NO_DEVICE = 0, -1, -2, -3, -4, -5


class Out(enum.IntEnum):
    """Out (src/metal/kernels.rs:30-43)."""
    Bf16 = 0
    F32 = 1
    Residual = 2
    Swiglu = 3


class XSrc(enum.IntEnum):
    """XSrc (src/metal/kernels.rs:236-256): what a matvec's x holds."""
    Plain = 0
    Swiglu = 1
    Norm = 2


class Kind(enum.IntEnum):
    GEMM = 0
    GEMM_SIMT = 1
    GEMM_DIRECT = 2
    GEMM_SWIGLU = 3
    MATVEC = 4
    ROUTE = 5
    SORT = 6
    SORT_ATOMIC = 7
    GATHER = 8
    SWIGLU = 9
    COMBINE = 10
    ROUND_PROBE = 11
    MOE_OUT = 12
    RMSNORM = 13


class Rows(enum.IntEnum):
    """MmaRows (src/metal/prefill.rs:317-338)."""
    Dense = 0
    Gather = 1
    Scatter = 2
    Sorted = 3


class Range(ctypes.Structure):
    """Range {buf, offset, size} (src/metal/gpu.rs:40-57); size 0 = to the end."""
    _fields_ = [("buf", ctypes.c_uint32), ("reserved", ctypes.c_uint32),
                ("offset", ctypes.c_uint64), ("size", ctypes.c_uint64)]

    def __repr__(self):
        return "Range(buf=%d, offset=%d, size=%d)" % (self.buf, self.offset, self.size)


_DESC_FIELDS = ["kind", "k", "n", "out", "rows_of", "m_first", "bm", "bn", "bk", "wm", "wn",
                "mfma", "dbuf", "swz", "order", "mv_m", "split", "persist", "rows", "form",
                "top_k", "experts", "tiles", "rows_max", "lds_dma", "unroll", "band", "xsrc", "eps_bits", "plus_one",
                "x_lds", "w_nt", "mv_waves", "sched", "ksplit"]


class Desc(ctypes.Structure):
    """hb_desc: a kernel's shape-keyed descriptor (what an emitter fixes)."""
    _fields_ = [(f, ctypes.c_uint32) for f in _DESC_FIELDS]

    def __init__(self, **kw):
        super().__init__()
        for k, v in kw.items():
            setattr(self, k, int(v))

    def replace(self, **kw):
        d = Desc(**{f: getattr(self, f) for f in _DESC_FIELDS})
        for k, v in kw.items():
            setattr(d, k, int(v))
        return d

    def __repr__(self):
        return "Desc(%s)" % ", ".join("%s=%d" % (f, getattr(self, f)) for f in _DESC_FIELDS
                                      if getattr(self, f))


class Op(ctypes.Structure):
    """Op {pipe, ranges, groups} (qwen.rs:650-655); the groups follow from m."""
    _fields_ = [("kernel", ctypes.c_int32), ("m", ctypes.c_uint32), ("nbind", ctypes.c_uint32),
                ("reserved", ctypes.c_uint32), ("bind", Range * 8)]

    def __init__(self, kernel, ranges, m):
        super().__init__()
        self.kernel = int(kernel)
        self.m = int(m)
        self.nbind = len(ranges)
        for i, r in enumerate(ranges):
            self.bind[i] = r


class MoeIo(ctypes.Structure):
    _fields_ = [(f, Range) for f in ("state", "route", "list", "tiles", "x", "w_gate_up", "egu",
                                     "ehb", "w_down", "ey", "xs")]


_P = ctypes.c_void_p
_u32, _u64, _i32 = ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int32
lib.hb_last_error.restype = ctypes.c_char_p
lib.hb_open.argtypes = [ctypes.c_int, ctypes.POINTER(_P)]
lib.hb_close.argtypes = [_P]
lib.hb_close.restype = None
lib.hb_device_summary.argtypes = [_P]
lib.hb_device_summary.restype = ctypes.c_char_p
lib.hb_alloc.argtypes = [_P, _u64, ctypes.POINTER(_u32)]
lib.hb_free.argtypes = [_P, _u32]
lib.hb_upload.argtypes = [_P, _u32, _u64, _P, _u64]
lib.hb_download.argtypes = [_P, _u32, _u64, _P, _u64]
lib.hb_zero.argtypes = [_P, _u32, _u64, _u64]
lib.hb_copy.argtypes = [_P, Range, Range]
lib.hb_buffer_ptr.argtypes = [_P, _u32, ctypes.POINTER(_P)]
lib.hb_kernel_build.argtypes = [_P, ctypes.POINTER(Desc), ctypes.POINTER(_i32)]
lib.hb_kernel_name.argtypes = [_P, _i32]
lib.hb_kernel_name.restype = ctypes.c_char_p
lib.hb_kernel_groups.argtypes = [_P, _i32, _u32]
lib.hb_kernel_groups.restype = _u32
lib.hb_kernel_bindings.argtypes = [_P, _i32]
lib.hb_kernel_bindings.restype = _u32
lib.hb_kernel_kind.argtypes = [_P, _i32]
lib.hb_kernel_kind.restype = _u32
lib.hb_compile_seconds.argtypes = [_P]
lib.hb_compile_seconds.restype = ctypes.c_double
lib.hb_launch.argtypes = [_P, _i32, ctypes.POINTER(Range), _u32, _u32]
lib.hb_time.argtypes = [_P, ctypes.POINTER(Op), _u32, _u32, ctypes.POINTER(ctypes.c_double)]
lib.hb_time_each.argtypes = [_P, ctypes.POINTER(Op), _u32, _u32, ctypes.POINTER(ctypes.c_double),
                             ctypes.POINTER(ctypes.c_double)]
lib.hb_sync.argtypes = [_P]
lib.hb_fill_normal_bf16.argtypes = [_u64, ctypes.c_float, _P, _u64, ctypes.c_int]
lib.hb_fill_normal_bf16.restype = None
lib.hb_engine_open.argtypes = [_P, ctypes.c_char_p, ctypes.POINTER(_P)]
lib.hb_engine_close.argtypes = [_P]
lib.hb_engine_close.restype = None
lib.hb_engine_tune_summary.argtypes = [_P]
lib.hb_engine_tune_summary.restype = ctypes.c_char_p
lib.hb_engine_buckets.argtypes = [_P, ctypes.POINTER(_u32), _u32, ctypes.POINTER(_u32)]
lib.hb_engine_gemm.argtypes = [_P, _u32, _u32, _u32, Range, Range, Range, Range, _u32,
                               ctypes.POINTER(_i32)]
lib.hb_engine_gate_up.argtypes = [_P, _u32, _u32, Range, Range, Range, Range, Range, _u32,
                                  ctypes.POINTER(_i32), ctypes.POINTER(_i32)]
lib.hb_engine_matvec.argtypes = [_P, _u32, _u32, _u32, _u32, ctypes.POINTER(Range), _u32, Range,
                                 Range, ctypes.POINTER(_i32)]
lib.hb_engine_matvec_fused.argtypes = [_P, _u32, _u32, _u32, _u32, _u32, _u32, _u32,
                                       ctypes.POINTER(Range), _u32, Range, Range, Range,
                                       ctypes.POINTER(_i32)]
lib.hb_engine_experts.argtypes = [_P, _u32, _u32, _u32, _u32, _u32, ctypes.POINTER(MoeIo),
                                  ctypes.POINTER(_i32), ctypes.POINTER(_u32)]
lib.hb_engine_gemm_candidates.argtypes = [_P, _u32, _u32, _u32, ctypes.POINTER(Desc), _u32,
                                          ctypes.POINTER(_u32)]
lib.hb_engine_matvec_candidates.argtypes = [_P, _u32, _u32, _u32, _u32, _u32, _u32, _u32,
                                            ctypes.POINTER(Desc), _u32, ctypes.POINTER(_u32)]
lib.hb_moe_experts_run.argtypes = [_P, ctypes.POINTER(_i32), _i32, _i32, ctypes.POINTER(MoeIo), Range,
                                   _u32]
lib.hb_engine_tune_get.argtypes = [_P, ctypes.c_char_p, ctypes.POINTER(_u32)]
lib.hb_engine_log_line.argtypes = [_P, ctypes.c_char_p, ctypes.c_double]
lib.hb_engine_autotune_seconds.argtypes = [_P]
lib.hb_engine_autotune_seconds.restype = ctypes.c_double


def last_error():
    return lib.hb_last_error().decode(errors="replace")


def check(rc):
    if rc != OK:
        raise HerbertError(rc, last_error())
    return rc


# ---- bf16 helpers (src/core/bf16.rs:7-23), vectorised ----

def f32_to_bf16(a):
    """Round to nearest even in integers: (bits + 0x7fff + lsb) >> 16."""
    b = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    return ((b + np.uint32(0x7FFF) + ((b >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)


def bf16_to_f32(h):
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def normal_bf16(seed, std, shape, threads=None):
    """bf16 bits ~ N(0, std^2) from the library's seeded generator."""
    n = int(np.prod(shape))
    out = np.empty(n, dtype=np.uint16)
    lib.hb_fill_normal_bf16(int(seed), float(std), out.ctypes.data_as(_P), n,
                            int(threads or min(16, os.cpu_count() or 1)))
    return out.reshape(shape)


# ---- the emitters: descriptors named after the reference's functions ----

def moe_tiles(rows, top_k, experts, bm):
    """moe_tiles (prefill.rs:832-835): the most expert tiles a block can need."""
    return -(-rows * top_k // bm) + experts


def gemm_mma_rows(kdim, n, out, m_first=True, rows_of=Rows.Dense, top_k=0, tiles=0, bm=0,
                  experts=0, rows_max=0, **tile):
    """gemm_mma_rows (prefill.rs:418-431): the MFMA GEMM over `rows_of`."""
    return Desc(kind=Kind.GEMM, k=kdim, n=n, out=out, m_first=m_first, rows_of=rows_of,
                top_k=top_k, tiles=tiles, bm=bm, experts=experts, rows_max=rows_max, **tile)


def gemm_simt(kdim, n, out, m_first=True):
    """gemm_simt (prefill.rs:133): the VALU GEMM, the contract's summation order."""
    return Desc(kind=Kind.GEMM_SIMT, k=kdim, n=n, out=out, m_first=m_first)


def gemm_mm2d(kdim, n, out, tm=64, tn=64, m_first=True):
    """gemm_mm2d (prefill.rs:442): MFMA operands straight from memory, tm x tn tiles."""
    return Desc(kind=Kind.GEMM_DIRECT, k=kdim, n=n, out=out, bm=tm, bn=tn, m_first=m_first)


def gemm_mma(kdim, n, out, m_first=True, **tile):
    """gemm_mma (prefill.rs:418): the dense MFMA GEMM."""
    return gemm_mma_rows(kdim, n, out, m_first, Rows.Dense, **tile)


def gemm_mma_swiglu(kdim, nf, m_first=True, **tile):
    """gemm_nax_swiglu (prefill.rs:755-824): W [2*nf][K] (gate rows, then up rows),
    H [m][nf] = rne(g * sigmoid(g) * u) of the bf16-rounded sums, in one MFMA GEMM."""
    return Desc(kind=Kind.GEMM_SWIGLU, k=kdim, n=nf, out=Out.Bf16, m_first=m_first, **tile)


def swiglu_rows(nf):
    """swiglu_rows (prefill.rs:2790) / swiglu_slots: H[r] from the row's [gate | up]."""
    return Desc(kind=Kind.SWIGLU, n=nf)


def matvec(kdim, n, out, mv_m=1, rows=4, split=1, persist=0, form=0, unroll=4, xsrc=0, eps=0.0,
           plus_one=False, x_lds=False, waves=0):
    """matvec / matvec_split (kernels.rs:146, 502, 640): y[m][n] = x[m][k].W^T for m <= mv_m;
    form 0 the VALU layout (rows per wave), 1 the MFMA layout (16 rows per wave), 2 the VALU
    layout with v_dot2, 3 the MFMA form with W read in row order through LDS, 4 the 4x4x4 MFMA
    form (4 rows per wave, W loaded straight into the operand, x in registers); xsrc / out Swiglu the decode fusions (VALU forms); x_lds the x rows
    staged in LDS once per workgroup (VALU forms); waves: wavefronts per workgroup (0 = 4, 8, 16;
    with x_lds up to 144 KiB of x)."""
    import struct
    eps_bits = struct.unpack("<I", struct.pack("<f", eps))[0]
    return Desc(kind=Kind.MATVEC, k=kdim, n=n, out=out, mv_m=mv_m, rows=rows, split=split,
                persist=persist, form=form, unroll=unroll, xsrc=xsrc, eps_bits=eps_bits,
                plus_one=1 if plus_one else 0, x_lds=1 if x_lds else 0, mv_waves=waves)


class Gpu:
    """Gpu (src/metal/gpu.rs): one HIP device, its stream, buffers and kernels."""

    def __init__(self, device=0):
        h = _P()
        check(lib.hb_open(int(device), ctypes.byref(h)))
        self.h = h
        self._sizes = {}

    @classmethod
    def open(cls, device=0):
        return cls(device)

    def close(self):
        if self.h:
            lib.hb_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def summary(self):
        return lib.hb_device_summary(self.h).decode()

    # memory
    def alloc(self, nbytes):
        b = _u32()
        check(lib.hb_alloc(self.h, int(nbytes), ctypes.byref(b)))
        self._sizes[b.value] = int(nbytes)
        return b.value

    def alloc_with(self, array):
        a = np.ascontiguousarray(array)
        b = self.alloc(max(a.nbytes, 1))
        if a.nbytes:
            self.upload(b, a)
        return b

    def free(self, buf):
        check(lib.hb_free(self.h, int(buf)))
        self._sizes.pop(int(buf), None)

    def upload(self, buf, array, offset=0):
        a = np.ascontiguousarray(array)
        check(lib.hb_upload(self.h, int(buf), int(offset), a.ctypes.data_as(_P), a.nbytes))

    def download(self, buf, dtype, count, offset=0):
        out = np.empty(int(count), dtype=dtype)
        check(lib.hb_download(self.h, int(buf), int(offset), out.ctypes.data_as(_P), out.nbytes))
        return out

    def zero(self, buf, offset=0, nbytes=None):
        n = self._sizes[int(buf)] - offset if nbytes is None else nbytes
        check(lib.hb_zero(self.h, int(buf), int(offset), int(n)))

    def copy(self, dst, src):
        """Device-to-device copy of Range src into Range dst (same size)."""
        check(lib.hb_copy(self.h, dst, src))

    def size(self, buf):
        return self._sizes[int(buf)]

    # kernels
    def pipeline(self, desc):
        """Gpu::pipeline: compile (hiprtc) or find the kernel `desc` names."""
        k = _i32()
        check(lib.hb_kernel_build(self.h, ctypes.byref(desc), ctypes.byref(k)))
        return k.value

    def kernel_name(self, k):
        return lib.hb_kernel_name(self.h, int(k)).decode()

    def kernel_kind(self, k):
        return lib.hb_kernel_kind(self.h, int(k))

    def groups(self, k, m):
        return lib.hb_kernel_groups(self.h, int(k), int(m))

    def compile_seconds(self):
        return lib.hb_compile_seconds(self.h)

    def launch(self, k, ranges, m):
        """Gpu::dispatch over m rows (sizes checked by the library first)."""
        arr = (Range * len(ranges))(*ranges)
        check(lib.hb_launch(self.h, int(k), arr, len(ranges), int(m)))

    def time_ops(self, ops, reps=1):
        """time_ops (qwen.rs:2593): GPU seconds of `reps` runs of `ops`."""
        arr = (Op * len(ops))(*ops)
        s = ctypes.c_double()
        check(lib.hb_time(self.h, arr, len(ops), int(reps), ctypes.byref(s)))
        return s.value

    def graph(self, ops):
        """The ops recorded into a HIP graph (hb_graph_record): a Graph."""
        arr = (Op * len(ops))(*ops)
        h = _P()
        check(lib.hb_graph_record(self.h, arr, len(ops), ctypes.byref(h)))
        return Graph(h)

    def time_each(self, ops, reps=1):
        """(GPU seconds of `reps` runs of `ops`, mean seconds of each op), one
        event after every launch on the library's stream."""
        arr = (Op * len(ops))(*ops)
        s = ctypes.c_double()
        each = (ctypes.c_double * len(ops))()
        check(lib.hb_time_each(self.h, arr, len(ops), int(reps), ctypes.byref(s), each))
        return s.value, list(each)

    def sync(self):
        check(lib.hb_sync(self.h))


def r(buf, offset=0, size=0):
    """Range over a buffer (`Range::whole` when offset and size are 0)."""
    return Range(int(buf), 0, int(offset), int(size))


lib.hb_engine_log.argtypes = [_P]
lib.hb_engine_log.restype = ctypes.c_char_p
lib.hb_engine_log_summary.argtypes = [_P]
lib.hb_engine_add_gemm_candidate.argtypes = [_P, ctypes.c_char_p, ctypes.POINTER(Desc)]
lib.hb_tune_check.argtypes = [ctypes.c_char_p, ctypes.c_char_p, _u64]


def tune_check(tune):
    """Tune::apply + Tune::summary (qwen.rs:296-398) without a device: the
    summary, or HerbertError with the reference's message."""
    buf = ctypes.create_string_buffer(8192)
    check(lib.hb_tune_check(tune.encode(), buf, len(buf)))
    return buf.value.decode()


lib.hb_engine_picks.argtypes = [_P, ctypes.c_char_p, _u64, ctypes.POINTER(_u64)]
lib.hb_engine_pin.argtypes = [_P, ctypes.c_char_p]
lib.hb_graph_record.argtypes = [_P, ctypes.POINTER(Op), _u32, ctypes.POINTER(_P)]
lib.hb_graph_launch.argtypes = [_P, _u32]
lib.hb_graph_time.argtypes = [_P, _u32, ctypes.POINTER(ctypes.c_double)]
lib.hb_graph_free.argtypes = [_P]
lib.hb_graph_free.restype = None


class Graph:
    """A recorded op sequence (hb_graph): replays with one launch each."""

    def __init__(self, h):
        self.h = h

    def launch(self, reps=1):
        check(lib.hb_graph_launch(self.h, int(reps)))

    def time(self, reps=1):
        s = ctypes.c_double()
        check(lib.hb_graph_time(self.h, int(reps), ctypes.byref(s)))
        return s.value

    def free(self):
        if self.h:
            lib.hb_graph_free(self.h)
            self.h = None


class Engine:
    """The kernel-selection part of QwenEngine (qwen.rs): --tune settings,
    gemm (:2200), mv_full (:1311), expert_pipes (:2326), with the
    [autotune] log."""

    def __init__(self, gpu, tune=""):
        """gpu None: a host-only engine (tune, log, autotune_chunk)."""
        h = _P()
        check(lib.hb_engine_open(gpu.h if gpu is not None else None, tune.encode(), ctypes.byref(h)))
        self.h = h
        self.gpu = gpu

    def close(self):
        if self.h:
            lib.hb_engine_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def tune_summary(self):
        return lib.hb_engine_tune_summary(self.h).decode()

    def log(self):
        return lib.hb_engine_log(self.h).decode()

    def log_summary(self):
        check(lib.hb_engine_log_summary(self.h))

    def autotune_seconds(self):
        return lib.hb_engine_autotune_seconds(self.h)

    def buckets(self):
        out = (_u32 * 32)()
        n = _u32()
        check(lib.hb_engine_buckets(self.h, out, 32, ctypes.byref(n)))
        return list(out[:n.value])

    def picks(self):
        """The engine's timed choices as text (hb_engine_picks)."""
        n = _u64()
        check(lib.hb_engine_picks(self.h, None, 0, ctypes.byref(n)))
        buf = ctypes.create_string_buffer(n.value + 1)
        check(lib.hb_engine_picks(self.h, buf, n.value + 1, ctypes.byref(n)))
        return buf.value.decode()

    def pin(self, text):
        """Seeds the choices with text picks() wrote (hb_engine_pin)."""
        check(lib.hb_engine_pin(self.h, text.encode()))

    def add_gemm_candidate(self, name, desc):
        check(lib.hb_engine_add_gemm_candidate(self.h, name.encode(), ctypes.byref(desc)))

    def tune_get(self, key):
        """The --tune value of `key` (defaults + the engine's string)."""
        v = _u32()
        check(lib.hb_engine_tune_get(self.h, key.encode(), ctypes.byref(v)))
        return v.value

    def log_line(self, line, seconds=0.0):
        """A line of the host's own timed choice into the engine's log."""
        check(lib.hb_engine_log_line(self.h, line.encode(), float(seconds)))

    def gemm_candidates(self, k, n, out):
        """The descriptors gemm() times for a k x n GEMM, in candidate order."""
        cap = 256
        arr = (Desc * cap)()
        cnt = _u32()
        check(lib.hb_engine_gemm_candidates(self.h, k, n, int(out), arr, cap, ctypes.byref(cnt)))
        return [arr[i].replace() for i in range(min(cnt.value, cap))]

    def matvec_candidates(self, k, n, out, mv_m, xsrc=0, eps=0.0, plus_one=False):
        """The descriptors mv_full times for a k x n matvec of mv_m rows, in order."""
        cap = 256
        arr = (Desc * cap)()
        cnt = _u32()
        eps_bits = struct.unpack("<I", struct.pack("<f", eps))[0]
        check(lib.hb_engine_matvec_candidates(self.h, k, n, int(out), int(xsrc), eps_bits, int(plus_one),
                                              mv_m, arr, cap, ctypes.byref(cnt)))
        return [arr[i].replace() for i in range(min(cnt.value, cap))]

    def gemm(self, k, n, out, state, w, x, y, m):
        kern = _i32()
        check(lib.hb_engine_gemm(self.h, k, n, int(out), state, w, x, y, m, ctypes.byref(kern)))
        return kern.value

    def gate_up(self, h, inter, state, w, x, gu, hout, m):
        """gate_up_pipes (qwen.rs:2148): (GEMM or fused kernel, SwiGLU kernel or -1)."""
        a, b = _i32(), _i32()
        check(lib.hb_engine_gate_up(self.h, h, inter, state, w, x, gu, hout, m, ctypes.byref(a),
                                    ctypes.byref(b)))
        return a.value, b.value

    def mv(self, k, n, out, mv_m, ws, x, y):
        arr = (Range * len(ws))(*ws)
        kern = _i32()
        check(lib.hb_engine_matvec(self.h, k, n, int(out), mv_m, arr, len(ws), x, y,
                                   ctypes.byref(kern)))
        return kern.value

    def mv_fused(self, k, n, out, mv_m, ws, x, y, xsrc=0, eps=0.0, plus_one=False, norm_w=None):
        """mv_full with its fusions (qwen.rs:1311): xsrc XSrc.Swiglu / Norm
        (eps, plus_one, the norm weights' Range), out Out.Swiglu."""
        import struct
        arr = (Range * len(ws))(*ws)
        kern = _i32()
        eps_bits = struct.unpack("<I", struct.pack("<f", eps))[0]
        check(lib.hb_engine_matvec_fused(self.h, k, n, int(out), int(xsrc), eps_bits,
                                         1 if plus_one else 0, mv_m, arr, len(ws), x, y,
                                         norm_w if norm_w is not None else Range(), ctypes.byref(kern)))
        return kern.value

    def experts(self, experts, top_k, hidden, inter, m, io):
        """io: MoeIo; returns ([sort, gate_up, down, gather or -1], rows per tile)."""
        ks = (_i32 * 4)()
        bm = _u32()
        check(lib.hb_engine_experts(self.h, experts, top_k, hidden, inter, m, ctypes.byref(io), ks,
                                    ctypes.byref(bm)))
        return list(ks), bm.value


class MoeLayer:
    """The routed experts of one MoE layer over blocks of up to `rows` rows,
    in the reference's op order (qwen.rs:2705-2735): route_qwen -> moe_sort
    -> [moe_gather] -> grouped gate|up -> swiglu_slots (or fused into the
    gate|up, when the selection picked that form) -> grouped down
    (scatter to slot rows) -> moe_combine.  Owns its device buffers; the
    kernels come from Engine.experts (expert_pipes), timed on the route of
    `scores` ([rows][experts] bf16, routed here first: the reference's
    real_route, qwen.rs:2340) and `x` if given."""

    def __init__(self, gpu, engine, experts, top_k, hidden, inter, rows, w_gate_up, w_down,
                 scores=None, x=None):
        self.gpu, self.e, self.k, self.h, self.mi, self.rows = gpu, experts, top_k, hidden, inter, rows
        pairs = rows * top_k
        g = gpu
        self.buf = {
            "state": g.alloc_with(np.array([0, 0, 0, rows], np.uint32)),
            "scores": g.alloc(rows * experts * 2),
            "route": g.alloc(rows * 2 * top_k * 4),
            "list": g.alloc(pairs * 4),
            "tiles": g.alloc((1 + 3 * moe_tiles(rows, top_k, experts, 16)) * 4),
            "x": g.alloc(rows * hidden * 2),
            "w_gate_up": w_gate_up,
            "egu": g.alloc(pairs * 2 * inter * 2),
            "ehb": g.alloc(pairs * inter * 2),
            "w_down": w_down,
            "ey": g.alloc(pairs * hidden * 2),
            "xs": g.alloc(pairs * hidden * 2),
            "out": g.alloc(rows * hidden * 2),
        }
        b = self.buf
        self.io = MoeIo(*[r(b[f]) for f in ("state", "route", "list", "tiles", "x", "w_gate_up",
                                             "egu", "ehb", "w_down", "ey", "xs")])
        self.route_k = gpu.pipeline(Desc(kind=Kind.ROUTE, experts=experts, top_k=top_k))
        self.swiglu_k = gpu.pipeline(Desc(kind=Kind.SWIGLU, n=inter))
        self.combine_k = gpu.pipeline(Desc(kind=Kind.COMBINE, n=hidden, top_k=top_k))
        if x is not None:
            g.upload(b["x"], x)
        if scores is not None:
            g.upload(b["scores"], scores)
            g.launch(self.route_k, [r(b["scores"]), r(b["route"])], rows)
            g.sync()
        self.kernels, self.bm = engine.experts(experts, top_k, hidden, inter, rows, self.io)
        self.fused = gpu.kernel_kind(self.kernels[1]) == Kind.GEMM_SWIGLU

    def ops(self, m=None):
        """The layer's dispatches over m rows (m <= rows; state[3] must be m)."""
        m = self.rows if m is None else m
        b, k = self.buf, self.k
        sort, gu, dn, gather = self.kernels
        ops = [Op(self.route_k, [r(b["scores"]), r(b["route"])], m),
               Op(sort, [r(b["state"]), r(b["route"]), r(b["list"]), r(b["tiles"])], m)]
        xin = b["x"]
        if gather >= 0:
            ops.append(Op(gather, [r(b["state"]), r(b["list"]), r(b["x"]), r(b["xs"])], m))
            xin = b["xs"]
        if self.fused:
            # The grouped gate|up writes the SwiGLU itself.
            ops.append(Op(gu, [r(b["state"]), r(b["w_gate_up"]), r(xin), r(b["ehb"]), r(b["list"]),
                               r(b["tiles"])], m))
        else:
            ops.append(Op(gu, [r(b["state"]), r(b["w_gate_up"]), r(xin), r(b["egu"]), r(b["list"]),
                               r(b["tiles"])], m))
            ops.append(Op(self.swiglu_k, [r(b["egu"]), r(b["ehb"])], m * k))
        ops.append(Op(dn, [r(b["state"]), r(b["w_down"]), r(b["ehb"]), r(b["ey"]), r(b["list"]),
                           r(b["tiles"])], m))
        ops.append(Op(self.combine_k, [r(b["ey"]), r(b["route"]), r(b["out"])], m))
        return ops

    def run(self, m=None):
        """The layer in two host calls: route_qwen, then hb_moe_experts_run
        (the rest of ops() as one native dispatch sequence)."""
        m = self.rows if m is None else m
        b = self.buf
        self.gpu.launch(self.route_k, [r(b["scores"]), r(b["route"])], m)
        ks = (ctypes.c_int32 * 4)(*self.kernels)
        check(lib.hb_moe_experts_run(self.gpu.h, ks, self.swiglu_k, self.combine_k,
                                     ctypes.byref(self.io), r(b["out"]), m))

    def free(self):
        for name, buf in self.buf.items():
            if name not in ("w_gate_up", "w_down"):
                self.gpu.free(buf)


def rmsnorm(d, eps, plus_one=False):
    """rmsnorm (kernels.rs:48-103): y = bf16(x / sqrt(mean(x^2) + eps) * w) per row of d."""
    import struct
    eps_bits = struct.unpack("<I", struct.pack("<f", eps))[0]
    return Desc(kind=Kind.RMSNORM, n=d, eps_bits=eps_bits, plus_one=1 if plus_one else 0)


def moe_out(d):
    """moe_out (qwen_kernels.rs:2163-2214): x = bf16(x + bf16(experts + bf16(g * shared)))
    with g = bf16(sigmoid(bf16(shared_gate . xn))), in place, a row per workgroup."""
    return Desc(kind=Kind.MOE_OUT, n=d)


class MoeBlock:
    """The sparse MLP of a qwen3_5_moe layer over blocks of up to `rows` rows,
    in the reference's op order (qwen.rs:2691-2732): the post norm (x ->
    xn), the shared expert (gate|up GEMM [+ SwiGLU] and down, gate_up_pipes
    and gemm picks), the router GEMM (xn -> scores), the routed experts
    (MoeLayer: route, sort, [gather], grouped gate|up, SwiGLU, grouped down,
    combine -> esum), moe_out (x += experts + gated shared output).

    `w`: device buffers {"post_norm": [h], "router": [E][h], "w_gate_up":
    [E*2*inter][h], "w_down": [E*h][inter], "s_gate_up": [2*si][h], "s_down":
    [h][si], "shared_gate": [h]}.  `x` (host [rows][h]) is the residual
    stream the selection runs on; the block updates buf["x"] in place."""

    def __init__(self, gpu, engine, experts, top_k, hidden, inter, shared_inter, rows, w, x,
                 eps=1e-6, plus_one=True):
        g, h, si = gpu, hidden, shared_inter
        self.gpu, self.rows, self.h, self.si, self.w = gpu, rows, h, si, w
        self.buf = {"state": g.alloc_with(np.array([0, 0, 0, rows], np.uint32)),
                    "x": g.alloc_with(x),
                    "s_gu": g.alloc(rows * 2 * si * 2), "s_h": g.alloc(rows * si * 2),
                    "sout": g.alloc(rows * h * 2)}
        b = self.buf
        self.norm_k = g.pipeline(rmsnorm(h, eps, plus_one))
        self.out_k = g.pipeline(moe_out(h))
        # xn and the router's scores on the selection's input, for the
        # experts' timing on a real route (the reference's real_route).
        xn_t, sc_t = g.alloc(rows * h * 2), g.alloc(rows * experts * 2)
        g.launch(self.norm_k, [r(b["x"]), r(w["post_norm"]), r(xn_t)], rows)
        self.router_k = engine.gemm(h, experts, Out.Bf16, r(b["state"]), r(w["router"]), r(xn_t),
                                    r(sc_t), rows)
        g.launch(self.router_k, [r(b["state"]), r(w["router"]), r(xn_t), r(sc_t), r(b["state"]),
                                 r(b["state"])], rows)
        g.sync()
        xn = g.download(xn_t, np.uint16, rows * h).reshape(rows, h)
        scores = g.download(sc_t, np.uint16, rows * experts).reshape(rows, experts)
        g.free(xn_t)
        g.free(sc_t)
        self.layer = MoeLayer(g, engine, experts, top_k, h, inter, rows, w["w_gate_up"], w["w_down"],
                              scores=scores, x=xn)
        L = self.layer.buf
        self.s_gu_k, self.s_sw_k = engine.gate_up(h, si, r(b["state"]), r(w["s_gate_up"]), r(L["x"]),
                                                  r(b["s_gu"]), r(b["s_h"]), rows)
        self.s_dn_k = engine.gemm(si, h, Out.Bf16, r(b["state"]), r(w["s_down"]), r(b["s_h"]),
                                  r(b["sout"]), rows)

    def ops(self, m=None):
        m = self.rows if m is None else m
        b, L, w, st = self.buf, self.layer.buf, self.w, r(self.buf["state"])
        ops = [Op(self.norm_k, [r(b["x"]), r(w["post_norm"]), r(L["x"])], m)]
        if self.s_sw_k >= 0:
            ops.append(Op(self.s_gu_k, [st, r(w["s_gate_up"]), r(L["x"]), r(b["s_gu"]), st, st], m))
            ops.append(Op(self.s_sw_k, [r(b["s_gu"]), r(b["s_h"])], m))
        else:
            ops.append(Op(self.s_gu_k, [st, r(w["s_gate_up"]), r(L["x"]), r(b["s_h"]), st, st], m))
        ops.append(Op(self.s_dn_k, [st, r(w["s_down"]), r(b["s_h"]), r(b["sout"]), st, st], m))
        ops.append(Op(self.router_k, [st, r(w["router"]), r(L["x"]), r(L["scores"]), st, st], m))
        ops += self.layer.ops(m)
        ops.append(Op(self.out_k, [r(L["x"]), r(w["shared_gate"]), r(L["out"]), r(b["sout"]), r(b["x"])], m))
        return ops

    def free(self):
        self.layer.free()
        for buf in self.buf.values():
            self.gpu.free(buf)


# ---- the checkpoint (model/qwen.rs:155-375) and the prefill block loop ----

lib.hb_ckpt_open.argtypes = [ctypes.c_char_p, ctypes.POINTER(_P)]
lib.hb_ckpt_close.argtypes = [_P]
lib.hb_ckpt_close.restype = None
lib.hb_ckpt_skipped.argtypes = [_P]
lib.hb_ckpt_skipped.restype = ctypes.c_char_p
lib.hb_ckpt_elements.argtypes = [_P, ctypes.c_char_p]
lib.hb_ckpt_elements.restype = _u64
lib.hb_ckpt_read.argtypes = [_P, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(_u64), _u32, _P, _u64]
lib.hb_ckpt_upload.argtypes = [_P, _P, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(_u64), _u32,
                               ctypes.POINTER(_u32)]
lib.hb_blocks_of.argtypes = [_u32, _u32, ctypes.POINTER(_u32), ctypes.POINTER(_u32), _u32]
lib.hb_blocks_of.restype = _u32


class Checkpoint:
    """Checkpoint (model/qwen.rs:155-375): the shards of `model_dir` mapped,
    names normalised to the engine's keys ("N.field"), tensors read as bf16."""

    def __init__(self, model_dir):
        h = _P()
        check(lib.hb_ckpt_open(os.fsencode(model_dir), ctypes.byref(h)))
        self.h = h

    def close(self):
        if self.h:
            lib.hb_ckpt_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def skipped(self):
        return lib.hb_ckpt_skipped(self.h).decode()

    def elements(self, key):
        return lib.hb_ckpt_elements(self.h, key.encode())

    def has(self, key):
        return self.elements(key) > 0

    @staticmethod
    def _parts(parts):
        keys = (ctypes.c_char_p * len(parts))(*[k.encode() for k, _ in parts])
        lens = (_u64 * len(parts))(*[int(n) for _, n in parts])
        return keys, lens

    def read(self, parts):
        """read_bf16_into: the (key, elements) parts one after the other, bf16."""
        keys, lens = self._parts(parts)
        total = sum(int(n) for _, n in parts)
        out = np.empty(total, np.uint16)
        check(lib.hb_ckpt_read(self.h, keys, lens, len(parts), out.ctypes.data_as(_P), total))
        return out

    def upload(self, gpu, parts):
        """upload(&mut gpu, &ck, parts): the parts stacked in one new buffer."""
        keys, lens = self._parts(parts)
        b = _u32()
        check(lib.hb_ckpt_upload(gpu.h, self.h, keys, lens, len(parts), ctypes.byref(b)))
        gpu._sizes[b.value] = 2 * sum(int(n) for _, n in parts)
        return b.value


_BLOCK_IN = ctypes.CFUNCTYPE(ctypes.c_int, _P, _u32, _u32, ctypes.POINTER(ctypes.c_double))
_RESET = ctypes.CFUNCTYPE(ctypes.c_int, _P)


class PrefillHost(ctypes.Structure):
    """hb_prefill_host: the host's block_in and reset, for autotune_chunk."""
    _fields_ = [("ctx", _P), ("block_in", _BLOCK_IN), ("reset", _RESET)]


lib.hb_engine_autotune_chunk.argtypes = [_P, ctypes.POINTER(PrefillHost), ctypes.POINTER(_u32)]


def autotune_chunk(engine, block_in, reset=None):
    """autotune_chunk (qwen.rs:2962-3010) through the library's
    hb_engine_autotune_chunk: `block_in(start, rows)` runs one block of the
    prompt and returns its GPU seconds, `reset()` restores what a block
    updates in place.  Returns the chosen rows per block (the library logs
    the reference's "[autotune] blocks over ..." line)."""
    err = []

    def _blk(_ctx, start, rows, out):
        try:
            out[0] = float(block_in(int(start), int(rows)))
            return 0
        except Exception as ex:  # reported after the call: ctypes cannot raise through C
            err.append(ex)
            return 1

    def _rst(_ctx):
        try:
            if reset is not None:
                reset()
            return 0
        except Exception as ex:
            err.append(ex)
            return 1

    host = PrefillHost(None, _BLOCK_IN(_blk), _RESET(_rst))
    chunk = _u32()
    rc = lib.hb_engine_autotune_chunk(engine.h, ctypes.byref(host), ctypes.byref(chunk))
    if err:
        raise err[0]
    check(rc)
    return chunk.value


def blocks_of(n, chunk):
    """blocks_of (qwen.rs:3017-3027): [(start, rows)] of a prompt of n rows."""
    cap = n // 64 + 2
    st, rw = (_u32 * cap)(), (_u32 * cap)()
    c = lib.hb_blocks_of(int(n), int(chunk), st, rw, cap)
    return [(st[i], rw[i]) for i in range(min(c, cap))]


class PrefillMlp:
    """The dense MLP half of a qwen layer's prefill (block_in, qwen.rs:2691-
    2697 without the MoE): x -> post norm -> [gate | up] GEMM (+ SwiGLU, or
    the fused kernel, gate_up_pipes) -> down GEMM added to x (Out::Residual),
    over a prompt cut into blocks (blocks_of) with each block on the kernels
    picked for its bucket (the smallest of the prefill buckets, qwen.rs:
    1051-1063, holding its rows).  Weights from the checkpoint in the fused
    layout the GEMMs read (qwen.rs:790-794)."""

    def __init__(self, gpu, engine, ckpt, layer, hidden, inter, eps=1e-6, plus_one=True):
        self.gpu, self.h, self.inter = gpu, hidden, inter
        p = lambda f: "%d.%s" % (layer, f)  # noqa: E731
        mlp = "mlp.shared_expert" if ckpt.has(p("mlp.shared_expert.gate_proj.weight")) else "mlp"
        self.w = {"post_norm": ckpt.upload(gpu, [(p("post_attention_layernorm.weight"), hidden)]),
                  "gate_up": ckpt.upload(gpu, [(p(mlp + ".gate_proj.weight"), inter * hidden),
                                               (p(mlp + ".up_proj.weight"), inter * hidden)]),
                  "down": ckpt.upload(gpu, [(p(mlp + ".down_proj.weight"), hidden * inter)])}
        self.buckets = engine.buckets()
        self.chunk = self.buckets[-1]
        B = self.chunk
        g = gpu
        self.buf = {"xn": g.alloc(B * hidden * 2), "gu": g.alloc(B * 2 * inter * 2),
                    "hh": g.alloc(B * inter * 2), "x": g.alloc(B * hidden * 2)}
        self.norm_k = g.pipeline(rmsnorm(hidden, eps, plus_one))
        self.kern = {}
        for m in self.buckets:
            st = g.alloc_with(np.array([0, 0, 0, m], np.uint32))
            b, w = self.buf, self.w
            gu_k, sw_k = engine.gate_up(hidden, inter, r(st), r(w["gate_up"]), r(b["xn"]), r(b["gu"]),
                                        r(b["hh"]), m)
            dn_k = engine.gemm(inter, hidden, Out.Residual, r(st), r(w["down"]), r(b["hh"]), r(b["x"]), m)
            self.kern[m] = (gu_k, sw_k, dn_k)
            g.free(st)

    def ops(self, x, n, states, chunk=None):
        """The ops of a prompt of n rows of the residual stream `x` (a buffer
        of [n][hidden] bf16, updated in place); `states`: one state buffer per
        block (blocks_of(n, chunk)), state[3] its rows."""
        ops = []
        for (start, rows), st in zip(blocks_of(n, chunk or self.chunk), states):
            ops += self.block_ops(x, start, rows, st, min(bk for bk in self.buckets if bk >= rows))
        return ops

    def block_ops(self, x, start, rows, st, m):
        """The ops of one block (block_in): rows `start..start+rows` of x on
        the kernels picked for bucket m; `st` holds state[3] = rows."""
        h, b, w = self.h, self.buf, self.w
        gu_k, sw_k, dn_k = self.kern[m]
        xr = r(x, start * h * 2, rows * h * 2)
        s = r(st)
        ops = [Op(self.norm_k, [xr, r(w["post_norm"]), r(b["xn"])], rows)]
        if sw_k >= 0:
            ops.append(Op(gu_k, [s, r(w["gate_up"]), r(b["xn"]), r(b["gu"]), s, s], rows))
            ops.append(Op(sw_k, [r(b["gu"]), r(b["hh"])], rows))
        else:
            ops.append(Op(gu_k, [s, r(w["gate_up"]), r(b["xn"]), r(b["hh"]), s, s], rows))
        ops.append(Op(dn_k, [s, r(w["down"]), r(b["hh"]), xr, s, s], rows))
        return ops

    def states(self, n, chunk=None):
        """One state buffer per block of a prompt of n rows (free them after)."""
        return [self.gpu.alloc_with(np.array([0, 0, 0, rows], np.uint32))
                for _, rows in blocks_of(n, chunk or self.chunk)]

    def autotune_chunk(self, engine, seed=0x5EED00C0):
        """autotune_chunk (qwen.rs:2962-3027) over this MLP half, the policy
        in the library (hb_engine_autotune_chunk): this side runs one block
        of a prompt of prefill.block seeded N(0,1) residual rows (block_in)
        and restores the rows a block adds into (reset).  The choice is kept
        as self.chunk."""
        g, n = self.gpu, engine.tune_get("prefill.block")
        x0 = normal_bf16(seed, 1.0, (n, self.h))
        X = g.alloc_with(x0)
        states = {}

        def block_in(start, rows):
            if rows not in states:
                states[rows] = g.alloc_with(np.array([0, 0, 0, rows], np.uint32))
            m = min(bk for bk in self.buckets if bk >= rows)
            return g.time_ops(self.block_ops(X, start, rows, states[rows], m), 1)

        try:
            self.chunk = autotune_chunk(engine, block_in, lambda: g.upload(X, x0))
            return self.chunk
        finally:
            for b in states.values():
                g.free(b)
            g.free(X)

    def free(self):
        for buf in list(self.buf.values()) + list(self.w.values()):
            self.gpu.free(buf)


class PrefillAttnProj:
    """The projections of an attention layer's prefill (block_in, qwen.rs:
    2653-2668): x -> input norm -> the fused [q | k | v] GEMM (Bf16 into
    `qkv`, [n][q_width + 2 kv_width]); and o from the attention's output
    added to x (Out::Residual).  RoPE and the attention itself sit between
    them in the reference and are not part of this library: the caller
    brings the attention output.  Weights from the checkpoint, [q | k | v]
    stacked as QwenEngine::load does (qwen.rs:831-835); blocks and buckets
    as PrefillMlp."""

    def __init__(self, gpu, engine, ckpt, layer, hidden, q_width, kv_width, out_width, eps=1e-6,
                 plus_one=True):
        self.gpu, self.h, self.qkv_w, self.out_w = gpu, hidden, q_width + 2 * kv_width, out_width
        p = lambda f: "%d.%s" % (layer, f)  # noqa: E731
        self.w = {"input_norm": ckpt.upload(gpu, [(p("input_layernorm.weight"), hidden)]),
                  "qkv": ckpt.upload(gpu, [(p("self_attn.q_proj.weight"), q_width * hidden),
                                           (p("self_attn.k_proj.weight"), kv_width * hidden),
                                           (p("self_attn.v_proj.weight"), kv_width * hidden)]),
                  "o": ckpt.upload(gpu, [(p("self_attn.o_proj.weight"), hidden * out_width)])}
        self.buckets = engine.buckets()
        self.chunk = self.buckets[-1]
        B = self.chunk
        g = gpu
        self.buf = {"xn": g.alloc(B * hidden * 2)}
        self.norm_k = g.pipeline(rmsnorm(hidden, eps, plus_one))
        self.kern = {}
        for m in self.buckets:
            st = g.alloc_with(np.array([0, 0, 0, m], np.uint32))
            qkv_t, ao_t, x_t = g.alloc(m * self.qkv_w * 2), g.alloc(m * out_width * 2), g.alloc(m * hidden * 2)
            qk = engine.gemm(hidden, self.qkv_w, Out.Bf16, r(st), r(self.w["qkv"]), r(self.buf["xn"]), r(qkv_t), m)
            ok = engine.gemm(out_width, hidden, Out.Residual, r(st), r(self.w["o"]), r(ao_t), r(x_t), m)
            self.kern[m] = (qk, ok)
            for b in (st, qkv_t, ao_t, x_t):
                g.free(b)

    def ops_qkv(self, x, qkv, n, states):
        """norm + [q | k | v] of a prompt of n rows: x [n][hidden] -> qkv."""
        ops = []
        for (start, rows), st in zip(blocks_of(n, self.chunk), states):
            qk, _ = self.kern[min(bk for bk in self.buckets if bk >= rows)]
            s = r(st)
            ops.append(Op(self.norm_k, [r(x, start * self.h * 2, rows * self.h * 2), r(self.w["input_norm"]),
                                        r(self.buf["xn"])], rows))
            ops.append(Op(qk, [s, r(self.w["qkv"]), r(self.buf["xn"]),
                               r(qkv, start * self.qkv_w * 2, rows * self.qkv_w * 2), s, s], rows))
        return ops

    def ops_o(self, attn_out, x, n, states):
        """x += o(attn_out) over a prompt of n rows."""
        ops = []
        for (start, rows), st in zip(blocks_of(n, self.chunk), states):
            _, ok = self.kern[min(bk for bk in self.buckets if bk >= rows)]
            s = r(st)
            ops.append(Op(ok, [s, r(self.w["o"]), r(attn_out, start * self.out_w * 2, rows * self.out_w * 2),
                               r(x, start * self.h * 2, rows * self.h * 2), s, s], rows))
        return ops

    def states(self, n):
        return [self.gpu.alloc_with(np.array([0, 0, 0, rows], np.uint32)) for _, rows in blocks_of(n, self.chunk)]

    def free(self):
        for buf in list(self.buf.values()) + list(self.w.values()):
            self.gpu.free(buf)


def probe_ids(n):
    """probe_ids (qwen.rs:2952-2955): the pseudo-random token ids the load's
    timings run on."""
    return [1000 + (i * 7919) % 50000 for i in range(n)]


def route_probe_rows(ckpt, block, hidden):
    """route_probe (qwen.rs:2928-2946) as far as the matmul path reaches: the
    reference prefills `prefill.block` probe ids through the first period of
    layers, so that the experts are timed on the route its router gives
    them; here the residual stream those rows start from -- the checkpoint's
    embedding rows of the probe ids (ids past the vocabulary wrap around) --
    for MoeBlock, which routes them with the layer's own norm and router
    before the experts are timed.  The mixer layers before the MoE (attention,
    DeltaNet) are not part of this library, so their contribution to the
    rows is missing."""
    n = ckpt.elements("embed_tokens")
    if not n or n % hidden:
        raise HerbertError(HB_ERR_INVALID, "route_probe: no embed_tokens of width %d" % hidden)
    vocab = n // hidden
    emb = ckpt.read([("embed_tokens", n)]).reshape(vocab, hidden)
    return emb[np.array(probe_ids(block), dtype=np.int64) % vocab]


def moe_weights_from_checkpoint(gpu, ckpt, layer, experts, hidden, inter, shared_inter):
    """The device weights of a qwen3_5_moe layer's sparse MLP as
    QwenEngine::load uploads them (qwen.rs:788-801): the post norm, the
    router (mlp.gate), the experts' [gate | up] rows and down rows
    (mlp.experts.gate_up_proj [E][2 inter][h], down_proj [E][h][inter]),
    the shared expert stacked [gate | up], its down and its gate; the dict
    MoeBlock takes."""
    p = lambda f: "%d.%s" % (layer, f)  # noqa: E731
    h, e, mi, si = hidden, experts, inter, shared_inter
    return {"post_norm": ckpt.upload(gpu, [(p("post_attention_layernorm.weight"), h)]),
            "router": ckpt.upload(gpu, [(p("mlp.gate.weight"), e * h)]),
            "w_gate_up": ckpt.upload(gpu, [(p("mlp.experts.gate_up_proj"), e * 2 * mi * h)]),
            "w_down": ckpt.upload(gpu, [(p("mlp.experts.down_proj"), e * h * mi)]),
            "s_gate_up": ckpt.upload(gpu, [(p("mlp.shared_expert.gate_proj.weight"), si * h),
                                           (p("mlp.shared_expert.up_proj.weight"), si * h)]),
            "s_down": ckpt.upload(gpu, [(p("mlp.shared_expert.down_proj.weight"), h * si)]),
            "shared_gate": ckpt.upload(gpu, [(p("mlp.shared_expert_gate.weight"), h)])}
