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


@pytest.mark.parametrize("m", [1, 8])
@pytest.mark.parametrize("form", ["valu_r4", "dot2_r2", "mfma_k1"])
def test_matvec_lm_head(gpu, form, m):
    """lm_head K=2560, N=151936 (778 MB of weights), all outputs checked."""
    k, n = 2560, 151936
    x = hb.normal_bf16(0x5EED0005, 1.0, (m, k))
    w = hb.normal_bf16(0x5EED0006, 0.02, (n, k))
    got = run_mv(gpu, x, w, 0, **FORMS[form])
    want = orc.gemm(x, w)
    check_close(got, want, k, abs_products(x, w), "lm_head %s m=%d" % (form, m))


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
