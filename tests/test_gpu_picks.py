"""Every kernel the GEMM selection can pick, on the bench's own shapes,
against the CPU oracle.

QwenEngine::gemm (qwen.rs:2200-2325) times a list of candidates and keeps
the fastest that passes check_candidates (the 1/64-of-max gate at m and
m - m/3 - 3 rows, qwen.rs:2497-2545).  That gate is looser than the 2-ulp
contract, and the pick depends on timing, so here every candidate of the
list (hb_engine_gemm_candidates) is run on each BASELINE shape the bench
reports -- config 1, config 2 at M = 512, 1024 and 2048, config 4 -- and
sampled rows of its output are checked against the oracle to the contract.
Whatever the selection picks on the bench's box has passed this check."""
import numpy as np
import pytest

import herbert_hip as hb
import hb_oracle as orc
from parity import abs_products, check_close

pytestmark = pytest.mark.gpu

SHAPES = ([("config1", 512, 1024, 3584, 0)]
          + [("%s_m%d" % (nm, m), m, k, n, out) for m in (512, 1024, 2048)
             for nm, k, n, out in (("qkv", 2560, 4608, 0), ("o", 4096, 2560, 2),
                                   ("gate_up", 2560, 18432, 0), ("down", 9216, 2560, 2),
                                   # the real Qwen3.5-4B fused [q+gate | k | v] width
                                   # (qwen_kernels.rs:41-51, probe.rs:738-741)
                                   ("qkv10240", 2560, 10240, 0))]
          + [("27b_%s" % nm, 2048, k, n, 0) for nm, k, n in (("qkv", 5120, 7168),
                                                              ("gate_up", 5120, 34816),
                                                              ("down", 17408, 5120),
                                                              ("lm_head", 5120, 151936))])


@pytest.mark.parametrize("name,m,k,n,out", SHAPES, ids=[s[0] for s in SHAPES])
def test_every_selection_candidate_within_contract(gpu, name, m, k, n, out):
    x = hb.normal_bf16(0x5EED0100 + k, 1.0, (m, k))
    w = hb.normal_bf16(0x5EED0101 + n, 0.02, (n, k))
    y0 = hb.normal_bf16(0x5EED0102, 1.0, (m, n)) if out == 2 else None
    rows = np.unique(np.concatenate([[0, 1, m // 2, m - 2, m - 1],
                                     np.linspace(0, m - 1, 11).astype(int)]))
    want = orc.gemm(x[rows], w, out, None if y0 is None else y0[rows])
    acc = orc.gemm(x[rows], w, orc.OUT_F32) if out == 2 else None
    absprod = abs_products(x, w, rows)
    st = gpu.alloc_with(np.array([0, 0, 0, m], np.uint32))
    W, X = gpu.alloc_with(w), gpu.alloc_with(x)
    Y = gpu.alloc(m * n * 2)
    e = hb.Engine(gpu, "")
    checked = []
    try:
        cands = e.gemm_candidates(k, n, out)
        assert len(cands) >= 30
        for i, d in enumerate(cands):
            try:
                kern = gpu.pipeline(d)
            except hb.HerbertError as ex:
                # Only the emitter's refusals of a form for this shape (a K
                # that does not split into whole tiles, an odd tile count) are
                # skipped, as the selection skips them; a compile failure of a
                # form the shape admits, or of the production kernel, fails.
                assert i > 0 and ex.code in (hb.HB_ERR_UNSUPPORTED, hb.HB_ERR_INVALID), \
                    "%s: candidate %d not built: %s" % (name, i, ex)
                continue
            if y0 is not None:
                gpu.upload(Y, y0)
            gpu.launch(kern, [hb.r(st), hb.r(W), hb.r(X), hb.r(Y), hb.r(st), hb.r(st)], m)
            gpu.sync()
            got = gpu.download(Y, np.uint16, m * n).reshape(m, n)[rows]
            kn = gpu.kernel_name(kern)
            print("[picks] %s %s" % (name, kn), flush=True)
            check_close(got, want, k, absprod, "%s %s" % (name, kn), acc=acc, min_exact=0.98)
            checked.append(kn)
    finally:
        e.close()
        for b in (st, W, X, Y):
            gpu.free(b)
    # the production kernel and the ping-pong forms are among those checked
    assert any("_pp" in c for c in checked), checked
    assert len(checked) >= 20, checked
