"""CPU checks that pin the oracle (oracle/hb_oracle.c) to the reference's
contract independently of its own code: the reference's branchy RNE over
every f32 pattern, exact-sum GEMM cases, identity / permutation / scaling
invariants, float32 scalar restatements of the summation order, and numpy
restatements of the route, sort, SwiGLU and combine."""
import math
import struct

import numpy as np
import pytest

import hb_oracle as orc
from parity import bf16_to_f32


def rne_branchy(bits):
    """src/core/bf16.rs:13-23 as written there: round bit and sticky bits."""
    bits = bits.astype(np.uint32)
    lsb = (bits >> np.uint32(16)) & np.uint32(1)
    rnd = (bits >> np.uint32(15)) & np.uint32(1)
    sticky = bits & np.uint32(0x7FFF)
    res = bits >> np.uint32(16)
    up = (rnd == 1) & ((sticky != 0) | (lsb == 1))
    return (res + up.astype(np.uint32)).astype(np.uint16)


def test_rne_exhaustive_all_f32_patterns():
    """Every one of the 2^32 f32 bit patterns (bf16.rs:13-23), as the
    reference's own `herbert-metal-probe round` checks its GPU text."""
    chunk = 1 << 24
    out = np.empty(chunk, np.uint16)
    base = np.arange(chunk, dtype=np.uint32)
    bits = np.empty(chunk, np.uint32)
    t = np.empty(chunk, np.uint32)
    up = np.empty(chunk, np.uint32)
    for c in range(1 << 32 >> 24):
        first = c * chunk
        orc.lib.hbo_f32_to_bf16_range(first, chunk, out.ctypes.data_as(orc._P))
        np.add(base, np.uint32(first), out=bits)
        # branchy form: up = round_bit & (sticky != 0 | lsb)
        np.bitwise_and(bits, np.uint32(0x7FFF), out=t)
        np.not_equal(t, 0, out=up, casting="unsafe")
        np.right_shift(bits, np.uint32(16), out=t)
        np.bitwise_and(t, np.uint32(1), out=t)
        np.bitwise_or(up, t, out=up)
        np.right_shift(bits, np.uint32(15), out=t)
        np.bitwise_and(up, t, out=up)
        np.bitwise_and(up, np.uint32(1), out=up)
        np.right_shift(bits, np.uint32(16), out=t)
        np.add(t, up, out=t)
        if not np.array_equal(out, t.astype(np.uint16)):
            want = t.astype(np.uint16)
            i = int(np.argmax(out != want))
            raise AssertionError("pattern %#010x: %#06x vs %#06x" % (first + i, out[i], want[i]))


def test_rne_special_values():
    f = orc.lib.hbo_f32_to_bf16
    assert f(0.0) == 0x0000 and f(-0.0) == 0x8000
    assert f(float("inf")) == 0x7F80 and f(float("-inf")) == 0xFF80
    assert f(1.0) == 0x3F80
    # ties to even: 1 + 2^-8 is halfway between 1 and 1 + 2^-7 -> 1
    assert f(1.0 + 2.0 ** -8) == 0x3F80
    assert f(1.0 + 3 * 2.0 ** -8) == 0x3F82  # halfway, odd below -> up
    # the largest finite f32 rounds to infinity
    assert f(struct.unpack("<f", struct.pack("<I", 0x7F7FFFFF))[0]) == 0x7F80
    for h in (0x0001, 0x3F80, 0x7F7F, 0x8001, 0xC2F7):
        assert orc.lib.hbo_f32_to_bf16(orc.lib.hbo_bf16_to_f32(h)) == h


def _exact_inputs(rng, shape, emin, emax, mbits):
    """bf16 values with few mantissa bits and a narrow exponent range, so that
    every product and partial sum below is exact in f32 and f64 alike."""
    sign = rng.integers(0, 2, shape) * 2 - 1
    e = rng.integers(emin, emax + 1, shape).astype(np.float64)
    m = rng.integers(0, 1 << mbits, shape).astype(np.float64)
    v = sign * (1 + m / (1 << mbits)) * 2.0 ** e
    return orc_f32_to_bf16(v)


def orc_f32_to_bf16(a):
    b = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    return rne_branchy(b)


@pytest.mark.parametrize("k", [1, 2, 8, 64])
def test_gemm_exact_sums_match_f64(k):
    """Small K with short mantissas: every summation order is exact, so the
    oracle must equal rne of the f64 dot product."""
    rng = np.random.default_rng(k)
    m, n = 7, 13
    x = _exact_inputs(rng, (m, k), -2, 2, 3)
    w = _exact_inputs(rng, (n, k), -2, 2, 3)
    want64 = bf16_to_f32(x).astype(np.float64) @ bf16_to_f32(w).astype(np.float64).T
    got = orc.gemm(x, w, orc.OUT_F32)
    assert np.array_equal(got.astype(np.float64), want64)
    got16 = orc.gemm(x, w, orc.OUT_BF16)
    assert np.array_equal(got16, orc_f32_to_bf16(want64))


def test_gemm_identity_and_permutation():
    rng = np.random.default_rng(1)
    m, k = 9, 48
    x = orc_f32_to_bf16(rng.standard_normal((m, k)))
    eye = orc_f32_to_bf16(np.eye(k))
    assert np.array_equal(orc.gemm(x, eye), x)
    perm = rng.permutation(k)
    assert np.array_equal(orc.gemm(x, eye[perm]), x[:, perm])
    # Residual: y = rne(y + rne(acc)); with acc = x exactly.
    y0 = orc_f32_to_bf16(rng.standard_normal((m, k)))
    want = orc_f32_to_bf16(bf16_to_f32(y0) + bf16_to_f32(x))
    assert np.array_equal(orc.gemm(x, eye, orc.OUT_RESIDUAL, y=y0), want)


def test_gemm_power_of_two_scaling_is_exact():
    rng = np.random.default_rng(2)
    x = orc_f32_to_bf16(rng.standard_normal((5, 256)))
    w = orc_f32_to_bf16(rng.standard_normal((11, 256)) * 0.02)
    y = orc.gemm(x, w, orc.OUT_F32)
    y4 = orc.gemm(x, orc_f32_to_bf16(bf16_to_f32(w) * 4), orc.OUT_F32)
    assert np.array_equal(y4, y * 4)


def test_gemm_sums_in_increasing_k_order():
    """The contract's order: f32 adds in increasing k (a float32 scalar loop
    in numpy, not the oracle's C), visible under cancellation."""
    rng = np.random.default_rng(3)
    k = 97
    x = orc_f32_to_bf16(rng.standard_normal((3, k)) * np.float32(1e3) ** rng.integers(0, 2, (3, k)))
    w = orc_f32_to_bf16(rng.standard_normal((4, k)))
    got = orc.gemm(x, w, orc.OUT_F32)
    xf, wf = bf16_to_f32(x), bf16_to_f32(w)
    for i in range(3):
        for j in range(4):
            acc = np.float32(0)
            for t in range(k):
                acc = np.float32(acc + np.float32(xf[i, t] * wf[j, t]))
            assert got[i, j] == acc
    # and the order matters here: the reversed order differs somewhere
    rev = [[np.float32(0)] * 4 for _ in range(3)]
    for i in range(3):
        for j in range(4):
            acc = np.float32(0)
            for t in reversed(range(k)):
                acc = np.float32(acc + np.float32(xf[i, t] * wf[j, t]))
            rev[i][j] = acc
    assert not np.array_equal(np.array(rev, np.float32), got)


def test_threads_do_not_change_bits():
    rng = np.random.default_rng(4)
    x = orc_f32_to_bf16(rng.standard_normal((33, 200)))
    w = orc_f32_to_bf16(rng.standard_normal((70, 200)) * 0.02)
    assert np.array_equal(orc.gemm(x, w, threads=1), orc.gemm(x, w, threads=7))


def test_expf_within_two_ulp_of_libm():
    xs = np.concatenate([np.linspace(-100, 88, 200001), np.linspace(-1, 1, 20001),
                         [0.0, -0.0, 1e-30, -1e-30, 88.5, -87.0]]).astype(np.float32)
    for x in xs[::7]:
        got = orc.expf(float(x))
        want = math.exp(float(x))
        if want < 1.2e-38:  # subnormal results: absolute bound
            assert abs(got - want) <= 2 * 2.0 ** -149
            continue
        ulp = 2.0 ** (math.floor(math.log2(want)) - 23)
        assert abs(got - want) <= 2 * ulp, (x, got, want)
    assert orc.expf(float("inf")) == float("inf") and orc.expf(-1000.0) == 0.0


def np_expf(x):
    return np.array([orc.expf(float(v)) for v in np.asarray(x, np.float32).ravel()],
                    np.float32).reshape(np.shape(x))


def route_numpy(scores, top_k):
    """qwen_kernels.rs:1802-1884 restated with numpy: the tie rule by a stable
    sort on (-p, index), the sums in the documented tree / selection order."""
    rows, experts = scores.shape
    s = bf16_to_f32(scores)
    out = np.zeros((rows, 2 * top_k), np.uint32)
    for r in range(rows):
        mx = s[r].max()
        e = np_expf(s[r] - mx)
        t = e.copy()
        h = experts // 2
        while h >= 1:
            t[:h] = t[:h] + t[h:2 * h]
            h //= 2
        p = (e / t[0]).astype(np.float32)
        order = np.lexsort((np.arange(experts), -p.astype(np.float64)))
        chosen = order[:top_k]
        vals = p[chosen]
        total = np.float32(0)
        for v in vals:
            total = np.float32(total + v)
        wts = orc_f32_to_bf16((vals / total).astype(np.float32))
        idx = np.argsort(chosen, kind="stable")
        out[r, :top_k] = chosen[idx]
        out[r, top_k:] = (wts[idx].astype(np.uint32) << np.uint32(16))
    return out


def test_route_matches_numpy_restatement_with_ties():
    rng = np.random.default_rng(5)
    scores = orc_f32_to_bf16(rng.standard_normal((40, 256)))
    # force exact ties in a few rows (lowest index must win)
    scores[3, 10] = scores[3, 200] = orc_f32_to_bf16(np.float32([9.0]))[0]
    scores[4, :] = orc_f32_to_bf16(np.float32([0.5]))[0]
    got = orc.route(scores, 8)
    assert np.array_equal(got, route_numpy(scores, 8))
    assert 10 in got[3, :8] and 200 in got[3, :8]
    assert list(got[4, :8]) == list(range(8))
    w = bf16_to_f32((got[:, 8:] >> 16).astype(np.uint16))
    assert np.all(np.abs(w.sum(1) - 1) < 0.05)


def test_moe_sort_invariants():
    rng = np.random.default_rng(6)
    rows, top_k, experts = 300, 8, 64
    route = np.zeros((rows, 2 * top_k), np.uint32)
    for r in range(rows):
        route[r, :top_k] = np.sort(rng.choice(experts, top_k, replace=False))
    for bm in (16, 32, 64):
        lst, tiles = orc.moe_sort(route, top_k, experts, bm)
        pairs = rows * top_k
        assert sorted(lst.tolist()) == list(range(pairs))
        ex = route[lst // top_k, lst % top_k]
        assert np.all(np.diff(ex.astype(np.int64)) >= 0)
        for e in range(experts):
            sel = lst[ex == e]
            assert np.all(np.diff(sel.astype(np.int64)) > 0)
        counts = np.bincount(ex, minlength=experts)
        nt = int(tiles[0])
        assert nt == int(sum(-(-c // bm) for c in counts))
        covered = np.zeros(pairs, np.int64)
        for t in range(nt):
            e, start, cnt = tiles[1 + 3 * t: 4 + 3 * t]
            assert 1 <= cnt <= bm
            assert np.all(ex[start:start + cnt] == e)
            covered[start:start + cnt] += 1
        assert np.all(covered == 1)


def test_experts_gemm_equals_dense_gemm_per_expert():
    rng = np.random.default_rng(7)
    rows, top_k, experts, hidden, n = 24, 4, 8, 64, 32
    route = np.zeros((rows, 2 * top_k), np.uint32)
    for r in range(rows):
        route[r, :top_k] = np.sort(rng.choice(experts, top_k, replace=False))
    x = orc_f32_to_bf16(rng.standard_normal((rows, hidden)))
    w = orc_f32_to_bf16(rng.standard_normal((experts * n, hidden)) * 0.02)
    lst, tiles = orc.moe_sort(route, top_k, experts, 16)
    pairs = rows * top_k
    gu = orc.experts_gemm(x, w, lst, tiles, hidden, n, 1, top_k, pairs)
    for p in range(pairs):
        pair = lst[p]
        e = route[pair // top_k, pair % top_k]
        want = orc.gemm(x[pair // top_k][None], w[e * n:(e + 1) * n])
        assert np.array_equal(gu[p], want[0])
    # Scatter: sorted row p lands at its slot row list[p].
    xs = orc_f32_to_bf16(rng.standard_normal((pairs, n)))
    w2 = orc_f32_to_bf16(rng.standard_normal((experts * hidden, n)) * 0.02)
    y = orc.experts_gemm(xs, w2, lst, tiles, n, hidden, 2, top_k, pairs)
    for p in range(0, pairs, 5):
        pair = lst[p]
        e = route[pair // top_k, pair % top_k]
        want = orc.gemm(xs[p][None], w2[e * hidden:(e + 1) * hidden])
        assert np.array_equal(y[pair], want[0])


# ---- swiglu_slots / moe_combine: checks the mathematics fixes ------------
# (qwen_kernels.rs:2087-2117: h = bf16(g * sigmoid(g) * u) in f32, one
# rounding; qwen_kernels.rs:2119-2165: acc = bf16(acc + bf16(y_s * w_s)) over
# the slots in route order.)  Written as functions of the implementation so
# that tests/test_oracle_mutants.py can run them against deliberately wrong
# builds of the oracle and see them fail.


def _bf16_of(v):
    """RNE of f32 values to bf16 bits (the reference's branchy form)."""
    return rne_branchy(np.asarray(v, np.float32).view(np.uint32))


def _ulp(v):
    a = np.abs(np.asarray(v, np.float64))
    return np.exp2(np.floor(np.log2(np.maximum(a, 2.0 ** -126))) - 7)


def swiglu_pins(swiglu):
    """swiglu(gu [slots][2n] bf16 bits, n) -> h [slots][n] bf16 bits."""
    rng = np.random.default_rng(0x5A1)
    n = 512
    u = _bf16_of(rng.standard_normal(n) * 2)
    g = _bf16_of(rng.standard_normal(n) * 2)
    # g = 0 or u = 0: h is zero (of either sign).
    zero = np.zeros(n, np.uint16)
    for gg, uu in ((zero, u), (g, zero)):
        h = swiglu(np.concatenate([gg, uu])[None], n)[0]
        assert np.all(bf16_to_f32(h) == 0), "swiglu with a zero factor"
    # g >= 20: sigmoid(g) is 1 in f32 (1 - 2e-9), so h = bf16(g * u), the
    # product of two bf16 exact in f32.
    big = _bf16_of(20 + np.abs(rng.standard_normal(n)) * 30)
    h = swiglu(np.concatenate([big, u])[None], n)[0]
    assert np.array_equal(h, _bf16_of(bf16_to_f32(big) * bf16_to_f32(u))), "swiglu at g >= 20"
    # g <= -104: exp(-g) overflows f32, sigmoid is 0, h = 0.
    neg = _bf16_of(-104 - np.abs(rng.standard_normal(n)) * 50)
    h = swiglu(np.concatenate([neg, u])[None], n)[0]
    assert np.all(bf16_to_f32(h) == 0), "swiglu at g <= -104"
    # Random g in [-12, 12]: h is the f64 value g * sigmoid(g) * u rounded
    # once to bf16, wherever that value sits further than 2^-12 of an ulp
    # from a rounding boundary (the f32 evaluation's error is ~2^-22
    # relative): a rounding of g * sigmoid(g) before the multiply by u, or a
    # wrong sigmoid, moves many outputs by an ulp.  Everywhere within 1 ulp.
    slots = 64
    gg = _bf16_of(rng.uniform(-12, 12, (slots, n)))
    uu = _bf16_of(rng.standard_normal((slots, n)) * 3)
    h = swiglu(np.concatenate([gg, uu], axis=1), n)
    gf, uf = bf16_to_f32(gg).astype(np.float64), bf16_to_f32(uu).astype(np.float64)
    t = gf / (1.0 + np.exp(-gf)) * uf
    hf = bf16_to_f32(h).astype(np.float64)
    assert np.all(np.abs(hf - t) <= _ulp(t)), "swiglu beyond 1 ulp of f64"
    frac = np.abs(t) / _ulp(t)
    frac -= np.floor(frac)
    clear = (np.abs(frac - 0.5) > 2.0 ** -12) & (np.abs(t) > 2.0 ** -100)
    assert clear.mean() > 0.95
    want = _bf16_of(t.astype(np.float32))
    bad = (h != want) & clear
    assert not bad.any(), "swiglu != one rounding of g*sigmoid(g)*u at %d outputs" % bad.sum()


def _route(experts_rows, weights):
    weights = np.asarray(weights, np.float32)
    rows, k = weights.shape
    r = np.zeros((rows, 2 * k), np.uint32)
    r[:, :k] = experts_rows
    r[:, k:] = weights.view(np.uint32)
    return r


def combine_pins(combine):
    """combine(y [rows*k][d] bf16 bits, route [rows][2k], k, d) -> [rows][d]."""
    rng = np.random.default_rng(0xC0B)
    rows, k, d = 16, 8, 64
    ex = np.sort(rng.choice(256, (rows, k)), axis=1)
    # Every rounding exact: small integers times 1/2 or 1/4, partial sums
    # below 2^5 in steps of 1/4 (8 significant bits suffice): the f64 sum.
    y = rng.integers(-3, 4, (rows * k, d)).astype(np.float32)
    w = rng.choice([0.25, 0.5], (rows, k)).astype(np.float32)
    out = combine(_bf16_of(y), _route(ex, w), k, d)
    want = (y.reshape(rows, k, d).astype(np.float64) * w[:, :, None]).sum(axis=1)
    assert np.array_equal(bf16_to_f32(out).astype(np.float64), want), "combine of exact terms"
    # One slot of weight 1: the identity.
    y1 = _bf16_of(rng.standard_normal((rows, d)))
    out = combine(y1, _route(ex[:, :1], np.ones((rows, 1), np.float32)), 1, d)
    assert np.array_equal(out, y1), "combine with top_k 1, weight 1"
    # Planted: slots (256, 1, -256), weights 1, in slot order with each sum
    # rounded: 256 + 1 = 257 ties to 256 (bf16 spacing 2 there), 256 - 256 =
    # 0.  Reversed order gives -256 + 1 = -255 (exact), then + 256 = 1; one
    # rounding at the end gives 1.
    yp = np.zeros((1, 3, d), np.float32)
    yp[0, :, 0] = [256.0, 1.0, -256.0]
    out = combine(_bf16_of(yp.reshape(3, d)), _route([[3, 7, 9]], [[1.0, 1.0, 1.0]]), 3, d)
    assert bf16_to_f32(out)[0, 0] == 0.0, "combine order / per-step rounding"
    # Planted: the product rounded before the add.  Slot 0: 1 * 1 = 1.
    # Slot 1: y = (1 + 66/128)/16, w = (1 + 125/128)/16, y*w =
    # 0.011702060699462890625 rounds to 3 * 2^-8 = 0.01171875; 1 + that =
    # 1 + 1.5 * 2^-7 is a tie that goes to the even 1 + 2^-6 = 1.015625.
    # Unrounded, 1 + 0.0117020607 is below the tie: 1 + 2^-7.
    yq = np.zeros((2, d), np.float32)
    yq[:, 0] = [1.0, (1 + 66 / 128) / 16]
    out = combine(_bf16_of(yq), _route([[1, 2]], [[1.0, (1 + 125 / 128) / 16]]), 2, d)
    assert bf16_to_f32(out)[0, 0] == 1.015625, "combine product rounding"


def gather_pins(gather):
    """Pins moe_gather (prefill.rs:579-610): XS[p] = X[list[p] / top_k],
    with every X row carrying its own index so a misread row shows.
    Checked against what the mapping fixes without restating it: the
    identity list repeats each X row top_k times (np.repeat); top_k = 1 is a
    plain row permutation (np.take); for any permutation of the pairs, each
    token's row appears exactly top_k times and the pairs of one token
    (consecutive pair ids, row*top_k + slot) all read that token's row."""
    rng = np.random.default_rng(21)
    rows, hidden = 37, 24
    x = np.empty((rows, hidden), np.uint16)
    x[:, 0::2] = np.arange(rows, dtype=np.uint16)[:, None]          # the row's id
    x[:, 1::2] = (0x4000 + np.arange(hidden // 2, dtype=np.uint16))[None, :]  # the column's id
    for top_k in (1, 2, 8):
        pairs = rows * top_k
        ident = np.arange(pairs, dtype=np.uint32)
        assert np.array_equal(gather(x, ident, top_k), np.repeat(x, top_k, axis=0)), \
            "identity list: each row top_k times (top_k=%d)" % top_k
        perm = rng.permutation(pairs).astype(np.uint32)
        xs = gather(x, perm, top_k)
        assert xs.shape == (pairs, hidden)
        assert np.all(xs[:, 1::2] == x[0, 1::2]), "columns kept in place"
        ids = xs[:, 0].astype(np.int64)
        assert np.array_equal(np.bincount(ids, minlength=rows), np.full(rows, top_k)), \
            "each token's row exactly top_k times (top_k=%d)" % top_k
        inv = np.argsort(perm)   # where pair q landed
        for r in range(rows):
            got = ids[inv[r * top_k:(r + 1) * top_k]]
            assert np.all(got == r), "pairs of token %d read rows %s" % (r, got)
        if top_k == 1:
            assert np.array_equal(xs, np.take(x, perm, axis=0)), "top_k=1 is a row permutation"
        assert np.array_equal(xs[:, 0::2], np.repeat(ids[:, None], hidden // 2, axis=1).astype(np.uint16))


def test_gather_rows_pinned():
    gather_pins(lambda x, list_, k: orc.gather_rows(x, list_, k))


def test_swiglu_pinned():
    swiglu_pins(lambda gu, n: orc.swiglu(gu, n))


def test_combine_pinned():
    combine_pins(lambda y, route, k, d: orc.combine(y, route, k, d))


def test_fused_swiglu_is_gemm_then_swiglu():
    """prefill.rs:746-750: the fused [gate | up] GEMM + SwiGLU is bit-equal to
    the GEMM (Out::Bf16) followed by swiglu_rows."""
    rng = np.random.default_rng(8)
    n = 48
    x = orc_f32_to_bf16(rng.standard_normal((6, 64)))
    w = orc_f32_to_bf16(rng.standard_normal((2 * n, 64)) * 0.1)
    assert np.array_equal(orc.gemm_swiglu(x, w, n), orc.swiglu(orc.gemm(x, w), n))


# ---- decode fusion XSrc::Norm (kernels.rs:48-103, 355-440) ---------------

def _bf16(v):
    return orc.lib.hbo_f32_to_bf16(float(v))


def hb_normal(seed, std, shape):
    """bf16 bits ~ N(0, std^2) from numpy's generator, rounded RNE."""
    b = (np.random.default_rng(seed).normal(0.0, std, shape).astype(np.float32)).view(np.uint32)
    return ((b + np.uint32(0x7FFF) + ((b >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)


@pytest.mark.parametrize("plus_one", [False, True])
def test_rmsnorm_constant_rows_are_the_weights(plus_one):
    """x = 2 everywhere, k a power of two, eps = 0: ss = 4k exactly, m = 4,
    inv = 1/2, so x' = bf16(1 * w') = w' (w + 1 rounded for plus_one), in
    both summation orders."""
    k = 2048
    x = np.full((2, k), _bf16(2.0), np.uint16)
    w = hb_normal(7, 0.5, k)
    want = w if not plus_one else np.array([_bf16(float(v) + 1.0) for v in bf16_to_f32(w)],
                                            np.uint16)
    for order in (0, 1):
        got = orc.rmsnorm_rows(x, w, 0.0, plus_one, order)
        assert np.array_equal(got[0], want) and np.array_equal(got[1], want)


def test_rmsnorm_one_nonzero_element():
    """x = (c, 0, ..., 0) with c and k powers of two, eps = 0: ss = c^2, m =
    c^2/k, sqrt(m) = |c|/sqrt(k) exact for k a power of 4, so x'_0 =
    bf16(sign(c) sqrt(k) w_0) and x'_i = 0 elsewhere."""
    k = 4096
    for c in (0.5, -8.0, 2.0 ** -20):
        x = np.zeros((1, k), np.uint16)
        x[0, 0] = _bf16(c)
        w = hb_normal(9, 1.0, k)
        got = orc.rmsnorm_rows(x, w, 0.0, False, 0)
        want0 = _bf16(math.copysign(64.0, c) * float(bf16_to_f32(w[:1])[0]))
        assert got[0, 0] == want0 and not np.any(bf16_to_f32(got[0, 1:]))


def test_rmsnorm_orders_and_f64_within_one_ulp():
    """The kernel's summation order and the increasing-index order differ in
    the last bits of ss only: x' within one bf16 ulp of each other and of an
    f64 restatement; and the order matters (some elements differ)."""
    m, k, eps = 6, 2560, 1e-6
    x = hb_normal(11, 1.0, (m, k))
    w = hb_normal(12, 0.1, k)
    a = orc.rmsnorm_rows(x, w, eps, True, 0)
    b = orc.rmsnorm_rows(x, w, eps, True, 1)
    xf = bf16_to_f32(x).astype(np.float64)
    wf = bf16_to_f32(w).astype(np.float64) + 1.0
    ref = xf / np.sqrt((xf * xf).sum(axis=1, keepdims=True) / k + eps) * wf
    for got in (a, b):
        g = bf16_to_f32(got).astype(np.float64)
        ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(ref), 2.0 ** -126))) - 7)
        assert np.all(np.abs(g - ref) <= ulp * 1.0001)
    d = np.abs(bf16_to_f32(a).astype(np.float64) - bf16_to_f32(b))
    assert np.all(d <= 2.0 ** (np.floor(np.log2(np.maximum(np.abs(bf16_to_f32(a)), 2.0 ** -126))) - 7))


# ---- moe_out (qwen_kernels.rs:2163-2214) ----------------------------------

def test_moe_out_closed_forms():
    """Zero gate weights: dot = 0, g = bf16(sigmoid(0)) = 0.5 exactly, so x'
    = bf16(x + bf16(ex + bf16(sh / 2))); shared = 0: x' = bf16(x + ex) --
    and an f64 restatement of the gate within one bf16 ulp."""
    rows, d = 3, 512
    xn = hb_normal(41, 1.0, (rows, d))
    ex = hb_normal(42, 1.0, (rows, d))
    sh = hb_normal(43, 1.0, (rows, d))
    x = hb_normal(44, 1.0, (rows, d))
    f = lambda a: bf16_to_f32(a).astype(np.float32)  # noqa: E731
    r = lambda v: bf16_to_f32(np.array([_bf16(t) for t in np.ravel(v)], np.uint16)).reshape(np.shape(v))  # noqa: E731
    got = orc.moe_out(xn, np.zeros(d, np.uint16), ex, sh, x)
    want = r(f(x) + r(f(ex) + r(np.float32(0.5) * f(sh))))
    assert np.array_equal(bf16_to_f32(got), want.astype(np.float32))
    got = orc.moe_out(xn, hb_normal(45, 0.05, d), ex, np.zeros((rows, d), np.uint16), x)
    assert np.array_equal(bf16_to_f32(got), r(f(x) + f(ex)).astype(np.float32))
    gate = hb_normal(46, 0.05, d)
    for order in (0, 1):
        got = orc.moe_out(xn, gate, np.zeros((rows, d), np.uint16), sh, np.zeros((rows, d), np.uint16), order)
        dot = bf16_to_f32(xn).astype(np.float64) @ bf16_to_f32(gate).astype(np.float64)
        g64 = 1.0 / (1.0 + np.exp(-dot))
        ref = g64[:, None] * bf16_to_f32(sh).astype(np.float64)
        ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(ref), 2.0 ** -126))) - 7)
        assert np.all(np.abs(bf16_to_f32(got) - ref) <= 3 * ulp)


def test_residual_input_layout_does_not_matter():
    """Out::Residual's y may be any numpy view (a column selection is not C
    ordered): the oracle reads it in row order either way."""
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((4, 64)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    w = (rng.standard_normal((40, 64)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    y0 = (rng.standard_normal((4, 100)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    sel = np.array([3, 0, 7, 9, 11, 20, 31, 39, 50, 60, 77, 80, 90, 95, 97, 99, 1, 2, 4, 5, 6, 8, 10, 12,
                    13, 14, 15, 16, 17, 18, 19, 21, 22, 23, 24, 25, 26, 27, 28, 29])
    view = y0[:, sel]
    assert not view.flags["C_CONTIGUOUS"] or view.flags["F_CONTIGUOUS"]
    assert np.array_equal(orc.gemm(x, w, orc.OUT_RESIDUAL, view),
                          orc.gemm(x, w, orc.OUT_RESIDUAL, np.ascontiguousarray(view)))
    assert np.array_equal(orc.moe_out(x, x[0], x, x, view[:, :64].T.copy().T),
                          orc.moe_out(x, x[0], x, x, np.ascontiguousarray(view[:, :64])))
