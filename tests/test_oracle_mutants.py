"""The SwiGLU and combine pins of tests/test_oracle.py must catch plausible
mistakes: each case here builds the oracle's C source with one deliberate
error (a copy in a temporary directory, never the shipped checker) and
asserts that the pins fail on it while passing on the unchanged source.
Mistakes covered: g*sigmoid(g) rounded before the multiply by u, the
sigmoid's sign flipped, the slots summed in reverse, the sum rounded only
at the end, the product not rounded before the add."""
import ctypes
import os
import subprocess

import numpy as np
import pytest

from test_oracle import combine_pins, swiglu_pins

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "oracle", "hb_oracle.c")

MUTANTS = {
    "none": [],
    "swiglu_double_rounding": [("float gs = g * sigmoid(g);", "float gs = hbo_round_bf16(g * sigmoid(g));")],
    "swiglu_sigmoid_sign": [("static float sigmoid(float x) { return 1.0f / (1.0f + hbo_expf(-x)); }",
                             "static float sigmoid(float x) { return 1.0f / (1.0f + hbo_expf(x)); }")],
    "combine_reversed": [("for (int s = 0; s < top_k; s++) {\n                float yf",
                          "for (int s = top_k - 1; s >= 0; s--) {\n                float yf")],
    "combine_one_rounding": [("acc = hbo_round_bf16(acc + hbo_round_bf16(yf * wf));",
                              "acc = acc + hbo_round_bf16(yf * wf);")],
    "combine_product_unrounded": [("acc = hbo_round_bf16(acc + hbo_round_bf16(yf * wf));",
                                   "acc = hbo_round_bf16(acc + yf * wf);")],
}


def build(tmp_path, name):
    text = open(SRC).read()
    for old, new in MUTANTS[name]:
        assert old in text, (name, old)
        text = text.replace(old, new)
    c = tmp_path / ("%s.c" % name)
    so = tmp_path / ("%s.so" % name)
    c.write_text(text)
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-fno-fast-math", "-fPIC", "-pthread", "-shared",
                    "-o", str(so), str(c), "-lm"], check=True)
    lib = ctypes.CDLL(str(so))
    P = ctypes.c_void_p
    lib.hbo_swiglu.argtypes = [P, ctypes.c_int, ctypes.c_int, P]
    lib.hbo_combine.argtypes = [P, P, ctypes.c_int, ctypes.c_int, ctypes.c_int, P]

    def swiglu(gu, n):
        gu = np.ascontiguousarray(gu, np.uint16)
        h = np.zeros((gu.shape[0], n), np.uint16)
        lib.hbo_swiglu(gu.ctypes.data, gu.shape[0], n, h.ctypes.data)
        return h

    def combine(y, route, k, d):
        y = np.ascontiguousarray(y, np.uint16)
        route = np.ascontiguousarray(route, np.uint32)
        out = np.zeros((route.shape[0], d), np.uint16)
        lib.hbo_combine(y.ctypes.data, route.ctypes.data, route.shape[0], k, d, out.ctypes.data)
        return out

    return swiglu, combine


@pytest.mark.parametrize("name", sorted(MUTANTS))
def test_pins_catch_the_mutant(tmp_path, name):
    swiglu, combine = build(tmp_path, name)
    if name == "none":
        swiglu_pins(swiglu)
        combine_pins(combine)
        return
    pins = swiglu_pins if name.startswith("swiglu") else combine_pins
    fn = swiglu if name.startswith("swiglu") else combine
    with pytest.raises(AssertionError):
        pins(fn)
