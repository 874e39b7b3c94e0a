"""Parity of the HIP decode matvec (kernels.rs:146-220 matvec, 502-519 and
640-975 matvec_split) with the CPU oracle on BASELINE config 3: M in
{1, 4, 8} over the 4B-class layer's weights and the lm_head, every form the
autotuner can pick (VALU rows/split, MFMA split, persistent groups)."""
import numpy as np
import pytest

import herbert_hip as hb
import hb_oracle as orc
from parity import abs_products, check_close

pytestmark = pytest.mark.gpu

FORMS = {
    "valu_r1": dict(form=0, rows=1, split=1),
    "valu_r4": dict(form=0, rows=4, split=1),
    "valu_r2_k4": dict(form=0, rows=2, split=4),
    "valu_r8_k2_p": dict(form=0, rows=8, split=2, persist=512),
    "dot2_r2": dict(form=2, rows=2, split=1),
    "dot2_r1_k2": dict(form=2, rows=1, split=2),
    "mfma_k1": dict(form=1, split=1),
    "mfma_u8_k2": dict(form=1, split=2, unroll=8),
    "mfma_u16": dict(form=1, split=1, unroll=16),
    "mfma_k4": dict(form=1, split=4),
    "mfma_k2_p": dict(form=1, split=2, persist=1024, unroll=2),
    "mfl_u4_k4": dict(form=3, split=4, unroll=4),
    "mfl_u8_k2_p": dict(form=3, split=2, persist=512, unroll=8),
    "mfl_u16": dict(form=3, split=1, unroll=16),
    "mfl_r32_u4_k4": dict(form=3, rows=32, split=4, unroll=4),
}


def run_mv(gpu, x, w, out=0, y0=None, mv_m=8, **form):
    m, k = x.shape
    n = w.shape[0]
    W, X = gpu.alloc_with(w), gpu.alloc_with(x)
    esz = 4 if out == 1 else 2
    Y = gpu.alloc_with(y0) if y0 is not None else gpu.alloc(m * n * esz)
    try:
        kern = gpu.pipeline(hb.matvec(k, n, out, mv_m=mv_m, **form))
        gpu.launch(kern, [hb.r(W), hb.r(X), hb.r(Y)], m)
        gpu.sync()
        return gpu.download(Y, np.float32 if out == 1 else np.uint16, m * n).reshape(m, n)
    finally:
        for b in (W, X, Y):
            gpu.free(b)


SHAPES = [("qkv", 2560, 4608, 0), ("o", 4096, 2560, 2), ("gate_up", 2560, 18432, 0),
          ("down", 9216, 2560, 2)]


@pytest.mark.parametrize("m", [1, 4, 8])
@pytest.mark.parametrize("form", sorted(FORMS))
@pytest.mark.parametrize("name,k,n,out", SHAPES)
def test_matvec_config3_layer(gpu, name, k, n, out, form, m):
    x = hb.normal_bf16(0x5EED0003, 1.0, (m, k))
    w = hb.normal_bf16(0x5EED0004, 0.02, (n, k))
    y0 = hb.normal_bf16(9, 1.0, (m, n)) if out == 2 else None
    got = run_mv(gpu, x, w, out, y0, **FORMS[form])
    want = orc.gemm(x, w, out, y0)
    acc = orc.gemm(x, w, orc.OUT_F32) if out == 2 else None
    check_close(got, want, k, abs_products(x, w), "%s %s m=%d" % (name, form, m), acc=acc)


@pytest.mark.parametrize("m", [1, 4, 8])
@pytest.mark.parametrize("form", ["valu_r4", "dot2_r2", "mfma_k1", "mfl_u4_k4", "mfl_r32_u4_k4"])
def test_matvec_lm_head(gpu, form, m):
    """lm_head K=2560, N=151936 (778 MB of weights), all outputs checked."""
    k, n = 2560, 151936
    x = hb.normal_bf16(0x5EED0005, 1.0, (m, k))
    w = hb.normal_bf16(0x5EED0006, 0.02, (n, k))
    got = run_mv(gpu, x, w, 0, **FORMS[form])
    want = orc.gemm(x, w)
    check_close(got, want, k, abs_products(x, w), "lm_head %s m=%d" % (form, m))


@pytest.mark.parametrize("rows", [16, 32])
@pytest.mark.parametrize("u,split,persist", [(4, 1, 0), (8, 1, 0), (16, 2, 0), (8, 4, 7), (4, 2, 3)])
@pytest.mark.parametrize("k,n", [(1056, 100), (4096, 33), (2560, 4608)])
def test_matvec_w_through_lds_equals_mfma(gpu, k, n, u, split, persist, rows):
    """Form 3 (W read in row order, turned into the MFMA A operand through a
    per-wave LDS tile) runs form 1's MFMAs on the same operands: bit-equal
    to form 1, with N not a multiple of the 16-row block (rows past N read
    row N-1, never stored), K / split not a multiple of the 32*unroll block
    (the tail in form 1's loads), and a few persistent workgroups looping
    over the row blocks; rows 32: two 16-row tiles per wave, each the same
    MFMAs as form 1's tile; within the contract of the oracle."""
    if (k // split) % 32:
        pytest.skip("K/split a multiple of 32")
    if rows == 32 and 4 * u * 2 > 64:
        pytest.skip("4 waves x unroll x 2 tiles: more than 64 KiB of LDS")
    m = 5
    x = hb.normal_bf16(0x5EED0041, 1.0, (m, k))
    w = hb.normal_bf16(0x5EED0042, 0.02, (n, k))
    y0 = hb.normal_bf16(27, 1.0, (m, n))
    f = dict(split=split, persist=persist, unroll=u)
    got = run_mv(gpu, x, w, 2, y0, form=3, rows=rows, **f)
    ref = run_mv(gpu, x, w, 2, y0, form=1, **f)
    assert np.array_equal(got, ref), "form 3 differs from form 1 (k=%d n=%d rows=%d %s)" % (k, n, rows, f)
    check_close(got, orc.gemm(x, w, orc.OUT_RESIDUAL, y0), k, abs_products(x, w), "form 3 %d x %d" % (k, n),
                acc=orc.gemm(x, w, orc.OUT_F32))


def test_matvec_f32_out_and_fewer_rows_than_built(gpu):
    """A kernel built for 8 rows run on 3: rows 3.. of y untouched."""
    k, n = 1024, 512
    x = hb.normal_bf16(1, 1.0, (3, k))
    w = hb.normal_bf16(2, 0.02, (n, k))
    for form in ("valu_r4", "mfma_k4"):
        got = run_mv(gpu, x, w, 1, **FORMS[form])
        want = orc.gemm(x, w, orc.OUT_F32)
        check_close(got, want, k, abs_products(x, w), "f32 " + form)


def test_matvec_rows_beyond_built_refused(gpu):
    k, n = 256, 64
    kern = gpu.pipeline(hb.matvec(k, n, 0, mv_m=2))
    W, X, Y = gpu.alloc(n * k * 2), gpu.alloc(4 * k * 2), gpu.alloc(4 * n * 2)
    with pytest.raises(hb.HerbertError):
        gpu.launch(kern, [hb.r(W), hb.r(X), hb.r(Y)], 4)
    for b in (W, X, Y):
        gpu.free(b)


# ---- decode fusions (kernels.rs:236-290, 355-440, 640-975): XSrc::Swiglu,
# XSrc::Norm, Out::Swiglu.  Each is checked twice: within the contract of the
# oracle's GEMM on the oracle's fused input (or fused output), and bit for
# bit against the same matvec form run plain on that input (the fusion
# changes where x comes from or how y is written, never a sum's order).

FUSION_FORMS = {"valu_r2": dict(form=0, rows=2, split=1), "dot2_r4_k2": dict(form=2, rows=4, split=2),
                "valu_r2_k4": dict(form=0, rows=2, split=4)}


def run_mv_fused(gpu, x, w, out, y0, mv_m, extra=None, **form):
    """The matvec with its fusion fields in `form`; extra: the norm weights."""
    m = x.shape[0]
    n = w.shape[0]
    yn = n // 2 if out == hb.Out.Swiglu else n
    esz = 4 if out == hb.Out.F32 else 2
    bufs = [gpu.alloc_with(w), gpu.alloc_with(x),
            gpu.alloc_with(y0) if y0 is not None else gpu.alloc(m * yn * esz)]
    if extra is not None:
        bufs.append(gpu.alloc_with(extra))
    try:
        kern = gpu.pipeline(hb.matvec(x.shape[1] // (2 if form.get("xsrc") == hb.XSrc.Swiglu else 1),
                                      n, out, mv_m=mv_m, **form))
        gpu.launch(kern, [hb.r(b) for b in bufs], m)
        gpu.sync()
        return gpu.download(bufs[2], np.float32 if out == hb.Out.F32 else np.uint16,
                            m * yn).reshape(m, yn)
    finally:
        for b in bufs:
            gpu.free(b)


@pytest.mark.parametrize("m", [1, 4])
@pytest.mark.parametrize("form", sorted(FUSION_FORMS))
def test_matvec_xsrc_swiglu(gpu, form, m):
    """down with x = swiglu([gate | up]) on load: K=9216, N=2560, Residual."""
    k, n = 9216, 2560
    gu = hb.normal_bf16(0x5EED0011, 1.0, (m, 2 * k))
    w = hb.normal_bf16(0x5EED0012, 0.02, (n, k))
    y0 = hb.normal_bf16(13, 1.0, (m, n))
    f = FUSION_FORMS[form]
    got = run_mv_fused(gpu, gu, w, hb.Out.Residual, y0, 8, xsrc=hb.XSrc.Swiglu, **f)
    xs = orc.swiglu(gu, k)
    check_close(got, orc.gemm(xs, w, orc.OUT_RESIDUAL, y0), k, abs_products(xs, w),
                "swiglu x %s m=%d" % (form, m), acc=orc.gemm(xs, w, orc.OUT_F32))
    plain = run_mv_fused(gpu, xs, w, hb.Out.Residual, y0, 8, **f)
    assert np.array_equal(got, plain), "XSrc::Swiglu differs from the plain matvec on swiglu(x)"


@pytest.mark.parametrize("plus_one", [False, True])
@pytest.mark.parametrize("m", [1, 4])
@pytest.mark.parametrize("form", sorted(FUSION_FORMS))
def test_matvec_xsrc_norm(gpu, form, m, plus_one):
    """qkv with x = RMSNorm(residual) computed into LDS first (eps 1e-6):
    the normed input bit for bit the oracle's in the kernel's summation order
    (shown by the plain matvec on the oracle's normed rows giving the same
    bits), the output within the contract."""
    k, n, eps = 2560, 4608, 1e-6
    xr = hb.normal_bf16(0x5EED0013, 3.0, (m, k))
    wn = hb.normal_bf16(0x5EED0014, 0.1, (k,))
    w = hb.normal_bf16(0x5EED0015, 0.02, (n, k))
    f = FUSION_FORMS[form]
    got = run_mv_fused(gpu, xr, w, hb.Out.Bf16, None, 8, extra=wn, xsrc=hb.XSrc.Norm, eps=eps,
                       plus_one=plus_one, **f)
    xn = orc.rmsnorm_rows(xr, wn, eps, plus_one, 0)
    check_close(got, orc.gemm(xn, w), k, abs_products(xn, w), "norm x %s m=%d" % (form, m))
    plain = run_mv_fused(gpu, xn, w, hb.Out.Bf16, None, 8, **f)
    assert np.array_equal(got, plain), "XSrc::Norm differs from the plain matvec on the oracle's norm"


@pytest.mark.parametrize("m", [1, 4])
@pytest.mark.parametrize("form", sorted(FUSION_FORMS))
def test_matvec_out_swiglu(gpu, form, m):
    """gate|up with y = swiglu(rne(g), rne(u)): K=2560, W [gate 9216 | up
    9216] rows, 9216 outputs.  The f32 sums of the same form (Out::F32) within
    the contract of the oracle's, and the fused output == the oracle's
    SwiGLU of those sums rounded, bit for bit; and within the contract of
    the oracle's fused GEMM."""
    k, nf = 2560, 9216
    x = hb.normal_bf16(0x5EED0016, 1.0, (m, k))
    w = hb.normal_bf16(0x5EED0017, 0.02, (2 * nf, k))
    f = FUSION_FORMS[form]
    got = run_mv_fused(gpu, x, w, hb.Out.Swiglu, None, 8, **f)
    sums = run_mv_fused(gpu, x, w, hb.Out.F32, None, 8, **f)
    ap = abs_products(x, w)
    check_close(sums, orc.gemm(x, w, orc.OUT_F32), k, ap, "swiglu sums %s m=%d" % (form, m))
    rs = hb.f32_to_bf16(sums)
    want_bits = orc.swiglu(np.concatenate([rs[:, :nf], rs[:, nf:]], axis=1), nf)
    assert np.array_equal(got, want_bits), "Out::Swiglu != swiglu of the rounded sums"
    check_close(got, orc.gemm_swiglu(x, w, nf), k,
                np.maximum(ap[:, :nf], ap[:, nf:]) * 2, "out swiglu %s m=%d" % (form, m), ulps=4.0)


XL_FORMS = {"dot2_r2_u8_xl_p512": dict(form=2, rows=2, split=1, unroll=8, persist=512),
            "valu_r4_xl": dict(form=0, rows=4, split=1),
            "dot2_r1_u8_xl_p1024": dict(form=2, rows=1, split=1, unroll=8, persist=1024)}


@pytest.mark.parametrize("m", [1, 3, 8])
@pytest.mark.parametrize("form", sorted(XL_FORMS))
@pytest.mark.parametrize("name,k,n,out", SHAPES[:3])
def test_matvec_x_in_lds(gpu, name, k, n, out, form, m):
    """x staged in LDS once per workgroup: bit-equal to the same form reading
    x from memory (the same sums in the same order), and within the contract
    of the oracle; m=3 on a kernel built for 8 rows."""
    x = hb.normal_bf16(0x5EED0023, 1.0, (m, k))
    w = hb.normal_bf16(0x5EED0024, 0.02, (n, k))
    y0 = hb.normal_bf16(19, 1.0, (m, n)) if out == 2 else None
    got = run_mv(gpu, x, w, out, y0, x_lds=True, **XL_FORMS[form])
    ref = run_mv(gpu, x, w, out, y0, **XL_FORMS[form])
    assert np.array_equal(got, ref), "%s %s m=%d: x in LDS differs from x from memory" % (name, form, m)
    want = orc.gemm(x, w, out, y0)
    acc = orc.gemm(x, w, orc.OUT_F32) if out == 2 else None
    check_close(got, want, k, abs_products(x, w), "%s %s xl m=%d" % (name, form, m), acc=acc)


MFL_XL_FORMS = {"mfl_u4_k4": dict(form=3, split=4, unroll=4),
                "mfl_r32_u4_k4_p512": dict(form=3, rows=32, split=4, unroll=4, persist=512),
                "mfl_u8_k2": dict(form=3, split=2, unroll=8)}


@pytest.mark.parametrize("m", [1, 3, 8])
@pytest.mark.parametrize("form", sorted(MFL_XL_FORMS))
@pytest.mark.parametrize("name,k,n,out", SHAPES[:3])
def test_matvec_mfl_x_in_lds(gpu, name, k, n, out, form, m):
    """Form 3 with its B operand (x) staged in LDS once per workgroup, rows
    one chunk apart: bit-equal to the same form reading x from memory, and
    within the contract of the oracle; m=3 on a kernel built for 8 rows."""
    x = hb.normal_bf16(0x5EED0025, 1.0, (m, k))
    w = hb.normal_bf16(0x5EED0026, 0.02, (n, k))
    y0 = hb.normal_bf16(21, 1.0, (m, n)) if out == 2 else None
    got = run_mv(gpu, x, w, out, y0, x_lds=True, **MFL_XL_FORMS[form])
    ref = run_mv(gpu, x, w, out, y0, **MFL_XL_FORMS[form])
    assert np.array_equal(got, ref), "%s %s m=%d: form 3 with x in LDS differs" % (name, form, m)
    acc = orc.gemm(x, w, orc.OUT_F32) if out == 2 else None
    check_close(got, orc.gemm(x, w, out, y0), k, abs_products(x, w), "%s %s m=%d" % (name, form, m), acc=acc)


WAVE_FORMS = {"w16_r1_p256_u4": dict(waves=16, rows=1, persist=256, unroll=4),
              "w16_r1_u8": dict(waves=16, rows=1, unroll=8),
              "w8_r2_p256_u4": dict(waves=8, rows=2, persist=256, unroll=4)}


@pytest.mark.parametrize("m", [3, 8])
@pytest.mark.parametrize("form", sorted(WAVE_FORMS))
@pytest.mark.parametrize("name,k,n,out", [SHAPES[0], SHAPES[1], SHAPES[3]])
def test_matvec_x_in_lds_waves(gpu, name, k, n, out, form, m):
    """x staged in LDS by 8- and 16-wave workgroups (down at 8 rows: 144 KiB):
    bit-equal to the 4-wave form reading x from memory (each row's sum is one
    wave's in the same order), within the contract of the oracle; m=3 on a
    kernel built for 8 rows."""
    f = dict(WAVE_FORMS[form], form=2, split=1)
    if 8 * k * 2 > 65536 and not f.get("persist"):
        pytest.skip("past 64 KiB of x: one workgroup per CU (persistent)")
    x = hb.normal_bf16(0x5EED0031, 1.0, (m, k))
    w = hb.normal_bf16(0x5EED0032, 0.02, (n, k))
    y0 = hb.normal_bf16(23, 1.0, (m, n)) if out == 2 else None
    got = run_mv(gpu, x, w, out, y0, x_lds=True, **f)
    ref = run_mv(gpu, x, w, out, y0, form=2, split=1, rows=f["rows"], unroll=f["unroll"])
    assert np.array_equal(got, ref), "%s %s m=%d: 8/16-wave x in LDS differs" % (name, form, m)
    acc = orc.gemm(x, w, orc.OUT_F32) if out == 2 else None
    check_close(got, orc.gemm(x, w, out, y0), k, abs_products(x, w), "%s %s m=%d" % (name, form, m), acc=acc)


def test_matvec_waves_fusions(gpu):
    """XSrc::Swiglu (down, 8 rows: the swiglu'd x, 144 KiB, in LDS) and
    Out::Swiglu with 16-wave workgroups: bit-equal to the 4-wave forms
    reading x from memory."""
    m, k, n = 8, 9216, 2560
    gu = hb.normal_bf16(0x5EED0033, 1.0, (m, 2 * k))
    w = hb.normal_bf16(0x5EED0034, 0.02, (n, k))
    y0 = hb.normal_bf16(25, 1.0, (m, n))
    f = dict(form=2, rows=2, split=1, unroll=4)
    got = run_mv_fused(gpu, gu, w, hb.Out.Residual, y0, m, xsrc=hb.XSrc.Swiglu, x_lds=True, waves=16,
                       persist=256, **f)
    ref = run_mv_fused(gpu, gu, w, hb.Out.Residual, y0, m, xsrc=hb.XSrc.Swiglu, **f)
    assert np.array_equal(got, ref), "XSrc::Swiglu: 16-wave x in LDS differs from x from memory"
    k2, nf = 2560, 9216
    x = hb.normal_bf16(0x5EED0035, 1.0, (m, k2))
    w2 = hb.normal_bf16(0x5EED0036, 0.02, (2 * nf, k2))
    got = run_mv_fused(gpu, x, w2, hb.Out.Swiglu, None, m, x_lds=True, waves=16, **f)
    ref = run_mv_fused(gpu, x, w2, hb.Out.Swiglu, None, m, **f)
    assert np.array_equal(got, ref), "Out::Swiglu: 16-wave x in LDS differs from x from memory"


@pytest.mark.parametrize("m", [1, 2])
def test_matvec_x_in_lds_fusions(gpu, m):
    """XSrc::Swiglu with the swiglu'd x staged in LDS (down, K=9216, built for
    2 rows: 36 KiB), and Out::Swiglu with x in LDS: bit-equal to the forms
    reading x from memory."""
    k, n = 9216, 2560
    gu = hb.normal_bf16(0x5EED0025, 1.0, (m, 2 * k))
    w = hb.normal_bf16(0x5EED0026, 0.02, (n, k))
    y0 = hb.normal_bf16(21, 1.0, (m, n))
    f = dict(form=2 if m > 1 else 0, rows=2, split=1, unroll=8, persist=512)
    got = run_mv_fused(gpu, gu, w, hb.Out.Residual, y0, 2, xsrc=hb.XSrc.Swiglu, x_lds=True, **f)
    ref = run_mv_fused(gpu, gu, w, hb.Out.Residual, y0, 2, xsrc=hb.XSrc.Swiglu, **f)
    assert np.array_equal(got, ref), "XSrc::Swiglu: x in LDS differs from x from memory"
    xs = orc.swiglu(gu, k)
    check_close(got, orc.gemm(xs, w, orc.OUT_RESIDUAL, y0), k, abs_products(xs, w),
                "swiglu x xl m=%d" % m, acc=orc.gemm(xs, w, orc.OUT_F32))
    k2, nf = 2560, 9216
    x = hb.normal_bf16(0x5EED0027, 1.0, (m, k2))
    w2 = hb.normal_bf16(0x5EED0028, 0.02, (2 * nf, k2))
    got = run_mv_fused(gpu, x, w2, hb.Out.Swiglu, None, 2, x_lds=True, **f)
    ref = run_mv_fused(gpu, x, w2, hb.Out.Swiglu, None, 2, **f)
    assert np.array_equal(got, ref), "Out::Swiglu: x in LDS differs from x from memory"


# ---- form 4: v_mfma_f32_4x4x4_16b_bf16, W loaded straight into the B
# operand (4 rows x 256 bytes per load instruction), x in registers; the 16
# blocks' sums added by DPP and lane swaps, the split waves' partials in wave
# order through LDS.

MF4_FORMS = {"mf4_k1": dict(form=4, split=1), "mf4_k2": dict(form=4, split=2),
             "mf4_k4_w8_p": dict(form=4, split=4, waves=8, persist=1024),
             "mf4_k8_w16": dict(form=4, split=8, waves=16),
             "mf4_k2_p3": dict(form=4, split=2, persist=3),
             "mf4_r8_k4_p256": dict(form=4, rows=8, split=4, persist=256),
             "mf4_r8_k8_w8_p7": dict(form=4, rows=8, split=8, waves=8, persist=7),
             "mf4_r16_k4_w8_p256": dict(form=4, rows=16, split=4, waves=8, persist=256)}


def mf4_ok(k, split, mv_m):
    """The form's own limits and the candidate list's: K/split a multiple of
    128, x of a wave in at most 72 registers."""
    if k % (128 * split):
        return False
    return (k // split // 128) * ((mv_m + 3) // 4) <= 18


@pytest.mark.parametrize("mv_m,m", [(8, 8), (8, 5), (4, 4), (4, 3), (1, 1)])
@pytest.mark.parametrize("form", sorted(MF4_FORMS))
@pytest.mark.parametrize("name,k,n,out", SHAPES)
def test_matvec_mf4_config3_layer(gpu, name, k, n, out, form, mv_m, m):
    f = MF4_FORMS[form]
    if not mf4_ok(k, f["split"], mv_m):
        pytest.skip("K/split not a whole number of 128-element loads, or x over 64 registers")
    x = hb.normal_bf16(0x5EED0013, 1.0, (m, k))
    w = hb.normal_bf16(0x5EED0014, 0.02, (n, k))
    y0 = hb.normal_bf16(19, 1.0, (m, n)) if out == 2 else None
    got = run_mv(gpu, x, w, out, y0, mv_m=mv_m, **f)
    want = orc.gemm(x, w, out, y0)
    acc = orc.gemm(x, w, orc.OUT_F32) if out == 2 else None
    check_close(got, want, k, abs_products(x, w), "%s %s m=%d/%d" % (name, form, m, mv_m), acc=acc)


@pytest.mark.parametrize("rows", [4, 16])
@pytest.mark.parametrize("persist", [0, 5])
@pytest.mark.parametrize("k,n,split", [(1024, 100, 1), (512, 33, 2), (2048, 6, 4), (256, 4097, 1)])
def test_matvec_mf4_ragged(gpu, k, n, split, persist, rows):
    """N not a multiple of the 4-row block (rows past N clamped, never
    stored), fewer row blocks than waves, f32 out; x rows 0..m-1 of 8."""
    for m in (1, 2, 7):
        x = hb.normal_bf16(0x5EED0015 + m, 1.0, (m, k))
        w = hb.normal_bf16(0x5EED0016, 0.02, (n, k))
        got = run_mv(gpu, x, w, 1, form=4, rows=rows, split=split, persist=persist, waves=8 if split > 4 else 4)
        check_close(got, orc.gemm(x, w, orc.OUT_F32), k, abs_products(x, w),
                    "mf4 %dx%d r%d k%d p%d m=%d" % (k, n, rows, split, persist, m))


@pytest.mark.parametrize("m", [1, 4, 8])
def test_matvec_mf4_lm_head(gpu, m):
    k, n = 2560, 151936
    x = hb.normal_bf16(0x5EED0005, 1.0, (m, k))
    w = hb.normal_bf16(0x5EED0006, 0.02, (n, k))
    got = run_mv(gpu, x, w, 0, mv_m=m, form=4, split=4, waves=8, persist=1024)
    check_close(got, orc.gemm(x, w), k, abs_products(x, w), "lm_head mf4 m=%d" % m)
