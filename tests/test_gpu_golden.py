"""The HIP kernels on the committed fixtures (tests/golden/golden.npz):
bit for bit where the contract fixes every bit (exact-sum GEMMs in every
form and Out mode, gemm_simt, route, sort, SwiGLU, the fused SwiGLU on exact
sums, combine), within the GEMM contract elsewhere."""
import os

import numpy as np
import pytest

import herbert_hip as hb
from parity import abs_products, check_close
from test_gpu_gemm import TILES, run_gemm
from test_gpu_moe import launch, route_gpu, sort_gpu

pytestmark = pytest.mark.gpu

G = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden.npz"))
FORMS = ["t128x128_x16_d2", "t256x256_w8_d4", "t128x192_w8_s3", "t128x128_reg_d1", "t64x64_reg_s1"]


@pytest.mark.parametrize("form", FORMS)
def test_golden_exact_gemm_every_out(gpu, form):
    x, w = G["gx"], G["gw"]
    assert np.array_equal(run_gemm(gpu, x, w, 0, **TILES[form]), G["gy_bf16"])
    assert np.array_equal(run_gemm(gpu, x, w, 1, **TILES[form]), G["gy_f32"])
    assert np.array_equal(run_gemm(gpu, x, w, 2, G["gy0"].copy(), **TILES[form]), G["gy_res"])


def _run(gpu, desc, x, w, out_dtype=np.uint16):
    m, k = x.shape
    n = w.shape[0]
    st = gpu.alloc_with(np.array([0, 0, 0, m], np.uint32))
    W, X, Y = gpu.alloc_with(w), gpu.alloc_with(x), gpu.alloc(m * n * 4)
    try:
        kern = gpu.pipeline(desc)
        gpu.launch(kern, [hb.r(st), hb.r(W), hb.r(X), hb.r(Y), hb.r(st), hb.r(st)], m)
        gpu.sync()
        return gpu.download(Y, out_dtype, m * n).reshape(m, n)
    finally:
        for b in (st, W, X, Y):
            gpu.free(b)


def test_golden_gemm_simt_mm2d(gpu):
    x, w = G["rx"], G["rw"]
    assert np.array_equal(_run(gpu, hb.gemm_simt(128, 24, 0), x, w), G["ry_bf16"])
    got = _run(gpu, hb.gemm_mm2d(128, 24, 0, 32, 16), x, w)
    check_close(got, G["ry_bf16"], 128, abs_products(x, w), "mm2d golden")
    got = _run(gpu, hb.gemm_mma(128, 24, 0), x, w)
    check_close(got, G["ry_bf16"], 128, abs_products(x, w), "mma golden")
    assert np.array_equal(_run(gpu, hb.gemm_mma(64, 40, 0), G["gx"], G["gw"]), G["gy_bf16"])


@pytest.mark.parametrize("m", [1, 4])
@pytest.mark.parametrize("form", [0, 1, 2])
def test_golden_matvec(gpu, m, form):
    x, w = G["mx%d" % m], G["mw%d" % m]
    d = hb.matvec(128, 16, 0, mv_m=m, form=form, rows=16 if form == 1 else 2, split=2)
    res = launch(gpu, d, [w, x, m * 16 * 2], m, {2: (np.uint16, m * 16)})
    check_close(res[2].reshape(m, 16), G["my%d" % m], 128, abs_products(x, w), "matvec golden")


def test_golden_moe_kernels(gpu):
    assert np.array_equal(route_gpu(gpu, G["scores"], 8), G["route"])
    lst, tiles = sort_gpu(gpu, G["route"], 8, 64, 16, 9)
    assert np.array_equal(lst, G["list"])
    assert np.array_equal(tiles[:len(G["tiles"])], G["tiles"])
    res = launch(gpu, hb.swiglu_rows(32), [G["gu"], 3 * 32 * 2], 3, {1: (np.uint16, 3 * 32)})
    assert np.array_equal(res[1].reshape(3, 32), G["h"])
    res = launch(gpu, hb.Desc(kind=hb.Kind.COMBINE, n=32, top_k=8), [G["cy"], G["route"], 9 * 32 * 2],
                 9, {2: (np.uint16, 9 * 32)})
    assert np.array_equal(res[2].reshape(9, 32), G["cout"])


def test_golden_fused_swiglu(gpu):
    x, w = G["sx"], G["sw"]
    d = hb.gemm_mma_swiglu(64, 24, bm=128, bn=128, bk=64, wm=2, wn=2, mfma=16, dbuf=1, lds_dma=1)
    assert np.array_equal(_run_h(gpu, d, x, w), G["sh"])


def _run_h(gpu, desc, x, w):
    m, k = x.shape
    nf = w.shape[0] // 2
    st = gpu.alloc_with(np.array([0, 0, 0, m], np.uint32))
    W, X, H = gpu.alloc_with(w), gpu.alloc_with(x), gpu.alloc(m * nf * 2)
    try:
        kern = gpu.pipeline(desc)
        gpu.launch(kern, [hb.r(st), hb.r(W), hb.r(X), hb.r(H), hb.r(st), hb.r(st)], m)
        gpu.sync()
        return gpu.download(H, np.uint16, m * nf).reshape(m, nf)
    finally:
        for b in (st, W, X, H):
            gpu.free(b)


def test_golden_rmsnorm_and_moe_out_kernels(gpu):
    """The block's norm and moe_out kernels on the fixtures, bit for bit
    (the oracle restates their reduction order)."""
    res = launch(gpu, hb.rmsnorm(512, 1e-6, True), [G["nx"], G["nw"], 3 * 512 * 2], 3,
                 {2: (np.uint16, 3 * 512)})
    assert np.array_equal(res[2].reshape(3, 512), G["ny"])
    res = launch(gpu, hb.moe_out(512), [G["ox"], G["og"], G["oe"], G["os"], G["ox0"]], 3,
                 {4: (np.uint16, 3 * 512)})
    assert np.array_equal(res[4].reshape(3, 512), G["oy"])
