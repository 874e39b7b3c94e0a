"""Every kernel the decode matvec selection can pick, on the bench's decode
shapes, against the CPU oracle.

mv_full (qwen.rs:1311-1511) times its candidate forms and keeps the fastest,
with no correctness check of its own, so every candidate
(hb_engine_matvec_candidates) is run here on BASELINE config 3 -- the
4B-class layer's four projections and the lm_head at M = 1, 4 and 8 -- and
on the decode fusions the bench's fused step selects (XSrc::Norm into qkv,
XSrc::Norm with Out::Swiglu into gate|up), and a sample of its outputs
(W rows spread over N, both ends included) is checked to the contract:
whatever form, rows, split, persistence or dot2 variant the selection picks
on the bench's box has passed this check."""
import numpy as np
import pytest

import herbert_hip as hb
import hb_oracle as orc
from parity import abs_products, check_close

pytestmark = pytest.mark.gpu

SHAPES = [("qkv", 2560, 4608, 0), ("o", 4096, 2560, 2), ("gate_up", 2560, 18432, 0),
          ("down", 9216, 2560, 2), ("lm_head", 2560, 151936, 0)]


def sample_rows(n, count=384):
    return np.unique(np.concatenate([np.arange(min(n, 40)), np.arange(max(0, n - 40), n),
                                     np.linspace(0, n - 1, count).astype(int)]))


@pytest.mark.parametrize("m", [1, 4, 8])
@pytest.mark.parametrize("name,k,n,out", SHAPES, ids=[s[0] for s in SHAPES])
def test_every_matvec_candidate_within_contract(gpu, name, k, n, out, m):
    x = hb.normal_bf16(0x5EED0200 + k, 1.0, (m, k))
    w = hb.normal_bf16(0x5EED0201 + n, 0.02, (n, k))
    y0 = hb.normal_bf16(0x5EED0202, 1.0, (m, n)) if out == 2 else None
    sel = sample_rows(n)
    ws = w[sel]
    want = orc.gemm(x, ws, out, None if y0 is None else y0[:, sel])
    acc = orc.gemm(x, ws, orc.OUT_F32) if out == 2 else None
    ap = abs_products(x, ws)
    W, X = gpu.alloc_with(w), gpu.alloc_with(x)
    Y = gpu.alloc(m * n * 2)
    e = hb.Engine(gpu, "")
    checked = []
    try:
        cands = e.matvec_candidates(k, n, out, m)
        assert len(cands) >= 10
        for i, d in enumerate(cands):
            try:
                kern = gpu.pipeline(d)
            except hb.HerbertError as ex:
                # only the emitter's refusals for this shape are skipped
                assert i > 0 and ex.code in (hb.HB_ERR_UNSUPPORTED, hb.HB_ERR_INVALID), \
                    "%s: candidate %d not built: %s" % (name, i, ex)
                continue
            if y0 is not None:
                gpu.upload(Y, y0)
            gpu.launch(kern, [hb.r(W), hb.r(X), hb.r(Y)], m)
            gpu.sync()
            got = gpu.download(Y, np.uint16, m * n).reshape(m, n)[:, sel]
            kn = gpu.kernel_name(kern)
            print("[mv picks] %s m=%d %s" % (name, m, kn), flush=True)
            check_close(got, want, k, ap, "%s m=%d %s" % (name, m, kn), acc=acc, min_exact=0.98)
            checked.append(kn)
    finally:
        e.close()
        for b in (W, X, Y):
            gpu.free(b)
    assert len(checked) >= 10, checked
    if m > 1:
        assert any("dot2" in c for c in checked) and any("mfl" in c for c in checked), checked


FUSED = [("qkv_norm", 2560, 4608, hb.Out.Bf16), ("gate_up_norm_swiglu", 2560, 18432, hb.Out.Swiglu)]


@pytest.mark.parametrize("m", [1, 4])
@pytest.mark.parametrize("name,k,n,out", FUSED, ids=[s[0] for s in FUSED])
def test_every_fused_matvec_candidate_within_contract(gpu, name, k, n, out, m):
    """XSrc::Norm (eps 1e-6, plus_one) into qkv and into gate|up with
    Out::Swiglu: the oracle's RMSNorm of the residual rows (the kernels'
    summation order), then its GEMM (and SwiGLU of the rounded sums)."""
    eps = 1e-6
    xr = hb.normal_bf16(0x5EED0210, 2.0, (m, k))
    wn = hb.normal_bf16(0x5EED0211, 0.1, (k,))
    w = hb.normal_bf16(0x5EED0212 + n, 0.02, (n, k))
    xn = orc.rmsnorm_rows(xr, wn, eps, True, 0)
    if out == hb.Out.Swiglu:
        nf = n // 2
        fs = sample_rows(nf, 256)
        wsel = np.concatenate([w[fs], w[nf + fs]])
        want = orc.gemm_swiglu(xn, wsel, len(fs))
        ap = abs_products(xn, wsel)
        ap = np.maximum(ap[:, :len(fs)], ap[:, len(fs):]) * 2
        sel, yn, ulps = fs, nf, 4.0
    else:
        sel = sample_rows(n)
        want = orc.gemm(xn, w[sel])
        ap = abs_products(xn, w[sel])
        yn, ulps = n, 2.0
    W, X, NW = gpu.alloc_with(w), gpu.alloc_with(xr), gpu.alloc_with(wn)
    Y = gpu.alloc(m * yn * 2)
    e = hb.Engine(gpu, "")
    checked = []
    try:
        cands = e.matvec_candidates(k, n, out, m, xsrc=hb.XSrc.Norm, eps=eps, plus_one=True)
        assert len(cands) >= 5
        for i, d in enumerate(cands):
            try:
                kern = gpu.pipeline(d)
            except hb.HerbertError as ex:
                assert i > 0 and ex.code in (hb.HB_ERR_UNSUPPORTED, hb.HB_ERR_INVALID), \
                    "%s: candidate %d not built: %s" % (name, i, ex)
                continue
            gpu.launch(kern, [hb.r(W), hb.r(X), hb.r(Y), hb.r(NW)], m)
            gpu.sync()
            got = gpu.download(Y, np.uint16, m * yn).reshape(m, yn)[:, sel]
            kn = gpu.kernel_name(kern)
            print("[mv picks] %s m=%d %s" % (name, m, kn), flush=True)
            check_close(got, want, k, ap, "%s m=%d %s" % (name, m, kn), ulps=ulps, min_exact=0.95)
            checked.append(kn)
    finally:
        e.close()
        for b in (W, X, NW, Y):
            gpu.free(b)
    assert len(checked) >= 5, checked
