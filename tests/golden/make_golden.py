"""Writes tests/golden/golden.npz: small input/output vectors of every
function on the path, from the CPU oracle, each cross-checked here before it
is written against what fixes it independently of the oracle's code:
exact-sum GEMMs against f64 (every summation order agrees), the RNE table
against the reference's branchy form (src/core/bf16.rs:13-23), expf against
libm within 2 ulp, the route's top-k against a brute-force ranking.

    python tests/golden/make_golden.py

The reference has no golden vectors for this path (its unit tests cover
f16 / Q4 conversions only), so these fixtures pin this build's oracle and
kernels against regressions; the oracle itself is pinned by
tests/test_oracle.py."""
import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
sys.path.insert(0, os.path.join(HERE, ".."))
import hb_oracle as orc  # noqa: E402
from test_oracle import combine_pins, swiglu_pins  # noqa: E402


def f32(b):
    return (np.asarray(b, np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def exact_bf16(rng, shape, emin=-3, emax=3, mbits=3):
    """bf16 values with `mbits` mantissa bits: their products and short sums are exact in f32."""
    m = rng.integers(0, 1 << mbits, size=shape)
    e = rng.integers(emin, emax + 1, size=shape)
    s = rng.choice([-1.0, 1.0], size=shape)
    v = (s * (1 + m / (1 << mbits)) * np.exp2(e)).astype(np.float32)
    return (v.view(np.uint32) >> np.uint32(16)).astype(np.uint16)


def rne_branchy(bits):
    bits = np.asarray(bits, np.uint32)
    lsb = (bits >> 16) & 1
    rnd = (bits >> 15) & 1
    sticky = bits & 0x7FFF
    return ((bits >> 16) + (rnd & ((sticky != 0) | lsb))).astype(np.uint16)


def main():
    rng = np.random.default_rng(0x601DE)
    g = {}
    # a1: RNE of special and tie patterns
    pats = [0, 0x80000000, 0x7F800000, 0xFF800000, 0x7FC00000, 0x7F800001, 0xFFFFFFFF, 0x00000001,
            0x007FFFFF, 0x00800000, 0x3F808000, 0x3F818000, 0x3F80FFFF, 0x3F817FFF, 0x7F7FFFFF,
            0x7F7F8000, 0xBF808000, 0x47FFF000]
    pats += list(rng.integers(0, 1 << 32, size=238, dtype=np.uint64).astype(np.uint32))
    pats = np.array(pats, np.uint32)
    rne = np.array([orc.rne_range(int(p), 1)[0] for p in pats], np.uint16)
    assert np.array_equal(rne, rne_branchy(pats))
    g["rne_in"], g["rne_out"] = pats, rne

    # a2/a3: exact-sum GEMM, every Out mode; f64 fixes every output
    x = exact_bf16(rng, (6, 64))
    w = exact_bf16(rng, (40, 64))
    y0 = exact_bf16(rng, (6, 40), -1, 1)
    acc = f32(x).astype(np.float64) @ f32(w).astype(np.float64).T
    assert np.all(acc == acc.astype(np.float32))
    g["gx"], g["gw"], g["gy0"] = x, w, y0
    g["gy_bf16"] = orc.gemm(x, w, orc.OUT_BF16)
    g["gy_f32"] = orc.gemm(x, w, orc.OUT_F32)
    g["gy_res"] = orc.gemm(x, w, orc.OUT_RESIDUAL, y0)
    assert np.array_equal(g["gy_f32"], acc.astype(np.float32))
    assert np.array_equal(g["gy_bf16"], rne_branchy(acc.astype(np.float32).view(np.uint32)))
    r = rne_branchy((f32(y0) + f32(g["gy_bf16"])).astype(np.float32).view(np.uint32))
    assert np.array_equal(g["gy_res"], r)

    # a3 with rounding inside the sums (the contract's k order matters)
    x = rne_branchy(rng.standard_normal((5, 128)).astype(np.float32).view(np.uint32))
    w = rne_branchy((0.02 * rng.standard_normal((24, 128))).astype(np.float32).view(np.uint32))
    g["rx"], g["rw"], g["ry_bf16"] = x, w, orc.gemm(x, w, orc.OUT_BF16)
    ref = f32(x).astype(np.float64) @ f32(w).astype(np.float64).T
    assert np.max(np.abs(f32(g["ry_bf16"]) - ref)) <= 2 ** -6 * np.max(np.abs(ref))

    # a7: decode matvec rows (M = 1 and 4)
    for m in (1, 4):
        xv = rne_branchy(rng.standard_normal((m, 128)).astype(np.float32).view(np.uint32))
        wv = rne_branchy((0.02 * rng.standard_normal((16, 128))).astype(np.float32).view(np.uint32))
        g["mx%d" % m], g["mw%d" % m], g["my%d" % m] = xv, wv, orc.gemm(xv, wv, orc.OUT_BF16)

    # a8: route with planted ties (lowest index wins)
    scores = rne_branchy(rng.standard_normal((9, 64)).astype(np.float32).view(np.uint32))
    scores[0, :] = scores[0, 0]
    scores[1, 10] = scores[1, 20] = scores[1, 30] = 0x4100
    route = orc.route(scores, 8)
    for rr in range(9):
        s = f32(scores[rr]).astype(np.float64)
        order = sorted(range(64), key=lambda i: (-s[i], i))[:8]
        assert sorted(order) == list(route[rr, :8]), rr
    g["scores"], g["route"] = scores, route

    # a9: sort of that route into tiles of 16 rows
    lst, tiles = orc.moe_sort(route, 8, 64, 16)
    assert sorted(lst) == list(range(72))
    g["list"], g["tiles"] = lst, tiles[:1 + 3 * int(tiles[0])]

    # a12: SwiGLU (the oracle first passes the pins the mathematics fixes);
    # the fixture within 1 ulp of f64, and one rounding of the f64 value
    # wherever that value is clear of a rounding boundary.
    swiglu_pins(orc.swiglu)
    combine_pins(orc.combine)
    gu = rne_branchy((2 * rng.standard_normal((3, 64))).astype(np.float32).view(np.uint32))
    g["gu"], g["h"] = gu, orc.swiglu(gu, 32)
    gf, uf = f32(gu[:, :32]).astype(np.float64), f32(gu[:, 32:]).astype(np.float64)
    t = gf / (1 + np.exp(-gf)) * uf
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(t), 2.0 ** -126))) - 7)
    assert np.all(np.abs(f32(g["h"]) - t) <= ulp)
    frac = np.abs(t) / ulp - np.floor(np.abs(t) / ulp)
    clear = np.abs(frac - 0.5) > 2.0 ** -12
    assert np.array_equal(g["h"][clear], rne_branchy(t.astype(np.float32).view(np.uint32))[clear])
    # a5: fused [gate | up] GEMM + SwiGLU on exact sums
    xs = exact_bf16(rng, (4, 64))
    ws = exact_bf16(rng, (48, 64), -4, 0)
    g["sx"], g["sw"], g["sh"] = xs, ws, orc.gemm_swiglu(xs, ws, 24)
    assert np.array_equal(g["sh"], orc.swiglu(orc.gemm(xs, ws, orc.OUT_BF16), 24))

    # a13: combine of the routed slots, each step from exact f64 values (a
    # bf16 product and a sum of two bf16 are exact in f64) rounded by the
    # branchy RNE, in the route's slot order.
    y = rne_branchy(rng.standard_normal((9 * 8, 32)).astype(np.float32).view(np.uint32))
    g["cy"], g["cout"] = y, orc.combine(y, route, 8, 32)
    rb64 = lambda v: f32(rne_branchy(np.asarray(v, np.float64).astype(np.float32).view(np.uint32)))  # noqa: E731
    wts = route[:, 8:].view(np.float32).astype(np.float64)
    acc = np.zeros((9, 32))
    for s_ in range(8):
        acc = rb64(acc + rb64(f32(y).reshape(9, 8, 32)[:, s_].astype(np.float64) * wts[:, s_:s_ + 1]))
    assert np.array_equal(f32(g["cout"]), acc)

    # expf samples (the route's softmax and SwiGLU's sigmoid)
    xe = np.concatenate([np.linspace(-100, 88, 97), [-104.0, 89.0, 0.0, -0.0, 1e-30, -1e-30]]).astype(np.float32)
    ye = np.array([orc.expf(float(v)) for v in xe], np.float32)
    for v, e in zip(xe, ye):
        if -87 < v < 88:
            ulp = float(np.spacing(np.float32(math.exp(float(v)))))
            assert abs(float(e) - math.exp(float(v))) <= 2 * ulp, v
    g["exp_in"], g["exp_out"] = xe, ye

    # XSrc::Norm / rmsnorm: rows of 512 (the kernel's summation order, eps
    # 1e-6, plus_one); row 0 constant 2 with eps 0 would give w + 1 exactly --
    # here with eps each row is within one bf16 ulp of an f64 restatement.
    nx = rne_branchy((rng.standard_normal((3, 512)) * 3).astype(np.float32).view(np.uint32))
    nx[0] = 0x4000  # 2.0 everywhere
    nw = rne_branchy((rng.standard_normal(512) * 0.1).astype(np.float32).view(np.uint32))
    ny = orc.rmsnorm_rows(nx, nw, 1e-6, True, 0)
    xf = f32(nx).astype(np.float64)
    ref = xf / np.sqrt((xf * xf).mean(axis=1, keepdims=True) + 1e-6) * (f32(nw).astype(np.float64) + 1)
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(ref), 2.0 ** -126))) - 7)
    assert np.all(np.abs(f32(ny) - ref) <= ulp)
    assert np.array_equal(orc.rmsnorm_rows(nx[:1], nw, 0.0, True, 0)[0],
                          rne_branchy((f32(nw) + np.float32(1)).view(np.uint32)))
    g["nx"], g["nw"], g["ny"] = nx, nw, ny

    # moe_out: rows of 512; with zero gate weights g = 0.5 exactly (closed
    # form checked), and random gate weights checked against f64 within 3 ulp.
    ox = rne_branchy(rng.standard_normal((3, 512)).astype(np.float32).view(np.uint32))
    oe = rne_branchy(rng.standard_normal((3, 512)).astype(np.float32).view(np.uint32))
    osh = rne_branchy(rng.standard_normal((3, 512)).astype(np.float32).view(np.uint32))
    ox0 = rne_branchy(rng.standard_normal((3, 512)).astype(np.float32).view(np.uint32))
    og = rne_branchy((rng.standard_normal(512) * 0.05).astype(np.float32).view(np.uint32))
    rb = lambda v: f32(rne_branchy(np.asarray(v, np.float32).view(np.uint32)))  # noqa: E731
    zero = orc.moe_out(ox, np.zeros(512, np.uint16), oe, osh, ox0)
    assert np.array_equal(f32(zero), rb(f32(ox0) + rb(f32(oe) + rb(np.float32(0.5) * f32(osh)))))
    oy = orc.moe_out(ox, og, oe, osh, ox0)
    gate = 1 / (1 + np.exp(-(f32(ox).astype(np.float64) @ f32(og).astype(np.float64))))
    ref = f32(ox0) + f32(oe) + gate[:, None] * f32(osh)
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(ref), 2.0 ** -126))) - 7)
    assert np.all(np.abs(f32(oy) - ref) <= 3 * ulp + 2 ** -8 * (np.abs(f32(oe)) + np.abs(f32(osh))))
    g["ox"], g["og"], g["oe"], g["os"], g["ox0"], g["oy"] = ox, og, oe, osh, ox0, oy

    path = os.path.join(HERE, "golden.npz")
    np.savez_compressed(path, **g)
    print("wrote %s (%d bytes, %d arrays)" % (path, os.path.getsize(path), len(g)))


if __name__ == "__main__":
    main()
