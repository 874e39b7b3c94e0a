"""The SwiGLU and combine pins of tests/test_oracle.py must catch plausible
mistakes: each case here builds the oracle's C source with one deliberate
error (a copy in a temporary directory, never the shipped checker) and
asserts that the pins fail on it while passing on the unchanged source.
Mistakes covered: g*sigmoid(g) rounded before the multiply by u, the
sigmoid's sign flipped, the slots summed in reverse, the sum rounded only
at the end, the product not rounded before the add; and the gather's row
taken as list[p] % top_k or as list[p] itself in place of list[p] / top_k."""
import ctypes
import os
import subprocess

import numpy as np
import pytest

from test_oracle import combine_pins, gather_pins, swiglu_pins

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
    "gather_row_mod": [("x + (size_t)(list[p] / top_k) * hidden", "x + (size_t)(list[p] % top_k) * hidden")],
    "gather_row_is_pair": [("x + (size_t)(list[p] / top_k) * hidden", "x + (size_t)(list[p]) * hidden")],
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

    lib.hbo_gather_rows.argtypes = [P, P, ctypes.c_int, ctypes.c_int, ctypes.c_int, P]

    def gather(x, list_, k):
        # X padded with rows of a sentinel, so a mutant that reads past the
        # token rows reads defined memory (and fails the pins on its values).
        x = np.ascontiguousarray(x, np.uint16)
        pad = np.vstack([x, np.full((len(list_) + 1, x.shape[1]), 0xDEAD, np.uint16)])
        list_ = np.ascontiguousarray(list_, np.uint32)
        xs = np.zeros((len(list_), x.shape[1]), np.uint16)
        lib.hbo_gather_rows(pad.ctypes.data, list_.ctypes.data, len(list_), k, x.shape[1], xs.ctypes.data)
        return xs

    return swiglu, combine, gather


@pytest.mark.parametrize("name", sorted(MUTANTS))
def test_pins_catch_the_mutant(tmp_path, name):
    swiglu, combine, gather = build(tmp_path, name)
    if name == "none":
        swiglu_pins(swiglu)
        combine_pins(combine)
        gather_pins(gather)
        return
    family = name.split("_")[0]
    pins = {"swiglu": swiglu_pins, "combine": combine_pins, "gather": gather_pins}[family]
    fn = {"swiglu": swiglu, "combine": combine, "gather": gather}[family]
    with pytest.raises(AssertionError):
        pins(fn)
