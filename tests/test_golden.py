"""The committed fixtures (tests/golden/golden.npz, written and cross-checked
by tests/golden/make_golden.py) against the CPU oracle, bit for bit: a
change to the oracle that moves any of them fails here."""
import os

import numpy as np

import hb_oracle as orc

G = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden.npz"))


def test_golden_rne():
    got = np.array([orc.rne_range(int(p), 1)[0] for p in G["rne_in"]], np.uint16)
    assert np.array_equal(got, G["rne_out"])


def test_golden_gemm():
    assert np.array_equal(orc.gemm(G["gx"], G["gw"], orc.OUT_BF16), G["gy_bf16"])
    assert np.array_equal(orc.gemm(G["gx"], G["gw"], orc.OUT_F32), G["gy_f32"])
    assert np.array_equal(orc.gemm(G["gx"], G["gw"], orc.OUT_RESIDUAL, G["gy0"]), G["gy_res"])
    assert np.array_equal(orc.gemm(G["rx"], G["rw"], orc.OUT_BF16), G["ry_bf16"])
    for m in (1, 4):
        assert np.array_equal(orc.gemm(G["mx%d" % m], G["mw%d" % m], orc.OUT_BF16), G["my%d" % m])


def test_golden_moe():
    assert np.array_equal(orc.route(G["scores"], 8), G["route"])
    lst, tiles = orc.moe_sort(G["route"], 8, 64, 16)
    assert np.array_equal(lst, G["list"])
    assert np.array_equal(tiles[:len(G["tiles"])], G["tiles"])
    assert np.array_equal(orc.swiglu(G["gu"], 32), G["h"])
    assert np.array_equal(orc.gemm_swiglu(G["sx"], G["sw"], 24), G["sh"])
    assert np.array_equal(orc.combine(G["cy"], G["route"], 8, 32), G["cout"])


def test_golden_expf():
    got = np.array([orc.expf(float(v)) for v in G["exp_in"]], np.float32)
    assert np.array_equal(got.view(np.uint32), G["exp_out"].view(np.uint32))


def test_golden_rmsnorm_and_moe_out():
    assert np.array_equal(orc.rmsnorm_rows(G["nx"], G["nw"], 1e-6, True, 0), G["ny"])
    assert np.array_equal(orc.moe_out(G["ox"], G["og"], G["oe"], G["os"], G["ox0"]), G["oy"])
