"""The rounding probe of herbert-metal-probe `round`
(src/bin/herbert-metal-probe.rs:7-11): every f32 bit pattern, in 256 chunks
of 2^24, rounded to bf16 on the GPU by the integer form every epilogue uses,
compared with the CPU oracle's f32_to_bf16 (src/core/bf16.rs:13-23) and the
differences counted by class of the input.  The compiler's own conversion
(gfx950 v_cvt_pk_bf16_f32) is probed the same way: it must agree on every
non-NaN pattern (NaN payloads may differ; they are counted, not required)."""
import numpy as np
import pytest

import herbert_hip as hb
import hb_oracle as orc

pytestmark = pytest.mark.gpu

CLASSES = ("zero", "subnormal", "normal", "inf", "nan")


def classify(bits):
    e = (bits >> np.uint32(23)) & np.uint32(0xFF)
    m = bits & np.uint32(0x7FFFFF)
    return {"zero": (e == 0) & (m == 0), "subnormal": (e == 0) & (m != 0),
            "normal": (e != 0) & (e != 255), "inf": (e == 255) & (m == 0),
            "nan": (e == 255) & (m != 0)}


def test_round_every_f32_pattern(gpu):
    n = 1 << 24
    st = gpu.alloc(16)
    A, B = gpu.alloc(2 * n), gpu.alloc(2 * n)
    kern = gpu.pipeline(hb.Desc(kind=hb.Kind.ROUND_PROBE))
    bad_int = dict.fromkeys(CLASSES, 0)
    bad_hw = dict.fromkeys(CLASSES, 0)
    first = {}
    try:
        for c in range(256):
            gpu.upload(st, np.array([c, 0, 0, 0], np.uint32))
            gpu.launch(kern, [hb.r(st), hb.r(A), hb.r(B)], 1)
            got = gpu.download(A, np.uint16, n)
            hw = gpu.download(B, np.uint16, n)
            want = orc.rne_range(c << 24, n)
            if np.array_equal(got, want) and np.array_equal(hw, want):
                continue
            bits = (np.uint32(c) << np.uint32(24)) | np.arange(n, dtype=np.uint32)
            cls = classify(bits)
            for name, sel in cls.items():
                di = int(np.count_nonzero(sel & (got != want)))
                dh = int(np.count_nonzero(sel & (hw != want)))
                bad_int[name] += di
                bad_hw[name] += dh
                if (di or dh) and name not in first:
                    j = int(np.flatnonzero(sel & ((got != want) | (hw != want)))[0])
                    first[name] = (hex(int(bits[j])), hex(int(got[j])), hex(int(hw[j])), hex(int(want[j])))
    finally:
        for b in (st, A, B):
            gpu.free(b)
    print("integer form differences by class:", bad_int)
    print("hardware conversion differences by class:", bad_hw, "first:", first)
    assert sum(bad_int.values()) == 0, (bad_int, first)
    assert all(bad_hw[c] == 0 for c in CLASSES if c != "nan"), (bad_hw, first)
