"""The fused [gate | up] GEMM + SwiGLU (gemm_nax_swiglu, prefill.rs:755-824)
and its selection (gate_up_pipes, qwen.rs:2148-2193).  The reference's
invariant: the fused kernel's h equals the GEMM (Out::Bf16) followed by
swiglu_rows bit for bit (prefill.rs:746-750); here the unfused GEMM runs the
same MFMA block (the sums of an output follow the same K steps), and the
SwiGLU of its bf16 output is checked against the CPU oracle's SwiGLU."""
import numpy as np
import pytest

import herbert_hip as hb
import hb_oracle as orc
from parity import abs_products, check_close

pytestmark = pytest.mark.gpu

FUSED = {
    "fused128x64": dict(bm=128, bn=128, bk=64, wm=2, wn=2, mfma=16, dbuf=1, lds_dma=1, order=1),
    "fused128x64b2": dict(bm=128, bn=128, bk=64, wm=2, wn=2, mfma=16, dbuf=1, lds_dma=1, band=2),
    "fused256x96": dict(bm=256, bn=192, bk=64, wm=4, wn=2, mfma=16, dbuf=1, lds_dma=1, order=1),
    "fused256x128": dict(bm=256, bn=256, bk=64, wm=4, wn=2, mfma=32, dbuf=1, lds_dma=1, order=1),
    "fused64x32_reg": dict(bm=64, bn=64, bk=32, wm=1, wn=2, mfma=16, dbuf=0, lds_dma=0, order=0),
}
APART = dict(bm=128, bn=128, bk=64, wm=2, wn=2, mfma=16, dbuf=1, lds_dma=1, order=1)


class Bufs:
    def __init__(self, gpu, x, w, m):
        self.gpu = gpu
        mr, k = x.shape
        nf = w.shape[0] // 2
        self.st = gpu.alloc_with(np.array([0, 0, 0, m], np.uint32))
        self.W, self.X = gpu.alloc_with(w), gpu.alloc_with(x)
        self.GU = gpu.alloc_with(np.full((mr, 2 * nf), 0x7FC1, np.uint16))
        self.H = gpu.alloc_with(np.full((mr, nf), 0x7FC1, np.uint16))
        self.shape = (mr, k, nf)

    def gemm(self, kern, m):
        g = self.gpu
        g.launch(kern, [hb.r(self.st), hb.r(self.W), hb.r(self.X), hb.r(self.GU), hb.r(self.st),
                        hb.r(self.st)], m)

    def fused(self, kern, m):
        g = self.gpu
        g.launch(kern, [hb.r(self.st), hb.r(self.W), hb.r(self.X), hb.r(self.H), hb.r(self.st),
                        hb.r(self.st)], m)

    def swiglu(self, kern, m):
        self.gpu.launch(kern, [hb.r(self.GU), hb.r(self.H)], m)

    def get(self, which):
        mr, _, nf = self.shape
        self.gpu.sync()
        if which == "gu":
            return self.gpu.download(self.GU, np.uint16, mr * 2 * nf).reshape(mr, 2 * nf)
        return self.gpu.download(self.H, np.uint16, mr * nf).reshape(mr, nf)

    def free(self):
        for b in (self.st, self.W, self.X, self.GU, self.H):
            self.gpu.free(b)


def inputs(m, k, nf, seed):
    return hb.normal_bf16(seed, 1.0, (m, k)), hb.normal_bf16(seed + 1, 0.02, (2 * nf, k))


@pytest.mark.parametrize("form", sorted(FUSED))
@pytest.mark.parametrize("m,k,nf", [(512, 1024, 1792), (131, 256, 200)])
def test_fused_swiglu_equals_gemm_then_swiglu(gpu, form, m, k, nf):
    """h of the fused kernel == swiglu_rows(GEMM Bf16) with the same MFMA
    block, bit for bit; that GEMM within the contract of the oracle's; the
    SwiGLU of its output == the oracle's SwiGLU, bit for bit; rows past m and
    features past nf untouched (131 rows, 200 features: partial tiles)."""
    t = FUSED[form]
    x, w = inputs(m, k, nf, 0x5EED0003)
    b = Bufs(gpu, x, w, m)
    try:
        fused = gpu.pipeline(hb.gemm_mma_swiglu(k, nf, **t))
        b.fused(fused, m)
        h_fused = b.get("h")
        apart = dict(APART, mfma=t["mfma"])
        b.gemm(gpu.pipeline(hb.gemm_mma(k, 2 * nf, 0, **apart)), m)
        b.swiglu(gpu.pipeline(hb.swiglu_rows(nf)), m)
        gu, h_apart = b.get("gu"), b.get("h")
    finally:
        b.free()
    assert np.array_equal(h_fused, h_apart), "%s: fused != GEMM then SwiGLU" % form
    check_close(gu, orc.gemm(x, w), k, abs_products(x, w), "gate|up %s" % form)
    assert np.array_equal(h_apart, orc.swiglu(gu, nf))


def test_fused_swiglu_state_rows(gpu):
    """state[3] below the launch's rows: only state[3] rows of h written."""
    m, k, nf = 256, 256, 512
    x, w = inputs(m, k, nf, 21)
    b = Bufs(gpu, x, w, 100)
    try:
        b.fused(gpu.pipeline(hb.gemm_mma_swiglu(k, nf, **FUSED["fused128x64"])), m)
        h = b.get("h")
    finally:
        b.free()
    assert np.all(h[100:] == 0x7FC1)
    want = orc.gemm_swiglu(x[:100], w, nf)
    hf, wf = hb.bf16_to_f32(h[:100]), hb.bf16_to_f32(want)
    assert np.max(np.abs(hf - wf)) <= np.max(np.abs(wf)) / 64
    assert np.mean(h[:100] == want) > 0.95


def test_fused_swiglu_config2_gate_up(gpu):
    """The 4B-class [gate | up] (K=2560, 2 x 9216) at M=2048 in the largest
    fused form, rows sampled: equal to GEMM + SwiGLU of the same MFMA block."""
    m, k, nf = 2048, 2560, 9216
    x, w = inputs(m, k, nf, 0x5EED0002)
    b = Bufs(gpu, x, w, m)
    try:
        b.fused(gpu.pipeline(hb.gemm_mma_swiglu(k, nf, **FUSED["fused256x128"])), m)
        h_fused = b.get("h")
        b.gemm(gpu.pipeline(hb.gemm_mma(k, 2 * nf, 0, **dict(APART, mfma=32))), m)
        b.swiglu(gpu.pipeline(hb.swiglu_rows(nf)), m)
        gu, h_apart = b.get("gu"), b.get("h")
    finally:
        b.free()
    assert np.array_equal(h_fused, h_apart)
    rows = np.array([0, 1, 700, 1337, 2046, 2047])
    check_close(gu[rows], orc.gemm(x[rows], w), k, abs_products(x, w, rows), "gate|up 4B")


def test_fused_swiglu_refusals(gpu):
    """Odd W fragments per wave, scattered expert rows and non-bf16 out are
    refused (gathered expert rows are the grouped gate|up's fused form)."""
    with pytest.raises(hb.HerbertError, match="even count"):
        gpu.pipeline(hb.gemm_mma_swiglu(256, 512, bm=128, bn=96, wm=2, wn=2, mfma=16))
    with pytest.raises(hb.HerbertError, match="bf16 out"):
        gpu.pipeline(hb.Desc(kind=hb.Kind.GEMM_SWIGLU, k=256, n=512, out=hb.Out.F32))
    with pytest.raises(hb.HerbertError, match="dense or gathered rows"):
        gpu.pipeline(hb.Desc(kind=hb.Kind.GEMM_SWIGLU, k=256, n=512, out=hb.Out.Bf16,
                             rows_of=hb.Rows.Scatter, top_k=8, experts=64, tiles=100, rows_max=64))


@pytest.mark.parametrize("fswi", [0, 1, 2])
def test_engine_gate_up(gpu, fswi):
    """pf.fswi 0: GEMM + SwiGLU apart; 1: the first fused form; 2: timed, the
    log names the candidates; every pick gives the apart path's h (equal
    bits for the 16x16 MFMA forms, within the 1/64 gate for the 32x32 one)."""
    m, k, nf = 512, 1024, 1792
    x, w = inputs(m, k, nf, 0x5EED0003)
    b = Bufs(gpu, x, w, m)
    try:
        with hb.Engine(gpu, "pf.fswi=%d" % fswi) as e:
            gk, sk = e.gate_up(k, nf, hb.r(b.st), hb.r(b.W), hb.r(b.X), hb.r(b.GU), hb.r(b.H), m)
            log = e.log()
            assert e.gate_up(k, nf, hb.r(b.st), hb.r(b.W), hb.r(b.X), hb.r(b.GU), hb.r(b.H), m) == (gk, sk)
        if sk >= 0:
            b.gemm(gk, m)
            b.swiglu(sk, m)
        else:
            b.fused(gk, m)
        h = b.get("h")
        name = gpu.kernel_name(gk)
    finally:
        b.free()
    want = orc.gemm_swiglu(x, w, nf)
    if fswi == 0:
        assert sk >= 0 and "swiglu" not in name
    if fswi == 1:
        assert sk == -1 and name.startswith("gemm_mma_swiglu_1024x1792")
    if fswi == 2:
        assert "[autotune] gate_up+swiglu 1024x3584, 512 rows: apart" in log
        assert "fused128x64" in log and "fused256x128" in log
    hf, wf = hb.bf16_to_f32(h), hb.bf16_to_f32(want)
    assert np.max(np.abs(hf - wf)) <= np.max(np.abs(wf)) / 64
    assert np.mean(h == want) > 0.95
