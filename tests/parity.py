"""Tolerance checks of the numerical contract, shared by the parity tests.

The contract: each output within 2 bf16 ulp of
the CPU oracle's (scalar f32 accumulation in increasing k, one RNE), and
within the reference's own gate max|err| <= max|ref|/64
(src/metal/qwen.rs:2497-2545).  Near zero, where cancellation makes 2 ulp of
a tiny result meaningless, the per-element bound also admits the f32
rounding bound of two summation orders, 2*gamma_K*sum|x_k w_k| with
gamma_K = K*u/(1-K*u), u = 2^-24 (Higham, Accuracy and Stability of
Numerical Algorithms, 2nd ed., eq. 3.5).
"""
import numpy as np


def bf16_to_f32(h):
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def bf16_ulp(v):
    """The spacing of bf16 numbers at |v| (8 significant bits)."""
    a = np.abs(np.asarray(v, dtype=np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -126)))
    return 2.0 ** (e - 7)


def gamma(k):
    u = 2.0 ** -24
    return k * u / (1 - k * u)


def abs_products(x, w, rows=None):
    """sum_k |x_k w_k| per output, in float64 (rows: the X rows to use)."""
    if rows is not None:
        x = x[rows]
    xf = np.abs(bf16_to_f32(x).astype(np.float64))
    out = np.empty((x.shape[0], w.shape[0]), np.float64)
    step = 8192  # W by row chunks: a full lm_head in f64 would not fit
    for c in range(0, w.shape[0], step):
        out[:, c:c + step] = xf @ np.abs(bf16_to_f32(w[c:c + step]).astype(np.float64)).T
    return out


def check_close(got, want, k, absprod, what="", ulps=2.0, acc=None, min_exact=None):
    """Asserts the contract; returns a dict of statistics for the report.
    acc: Out::Residual's f32 sums (y = rne(y + rne(acc)) rounds twice: one
    bf16 ulp of rne(acc) joins the bound).
    min_exact: the least fraction of outputs that must equal the oracle's
    bit for bit, and then, outside the cancellation band
    |want| > 16*gamma_K*sum|x_k w_k|, every output within `ulps` bf16 ulp
    (plus Residual's one ulp of rne(acc)) with no f32 term.  A correct
    f32-accumulating kernel moves each sum by ~sqrt(K)*2^-24*|partial sums|
    against the oracle's order, far below a bf16 ulp, so >98% of its outputs
    are bit-identical even at K = 17408; a kernel that drops a 32-wide slice
    of K moves them by sigma*sqrt(32/K) of the sum, many ulp."""
    g = bf16_to_f32(got).astype(np.float64) if got.dtype == np.uint16 else got.astype(np.float64)
    t = bf16_to_f32(want).astype(np.float64) if want.dtype == np.uint16 else want.astype(np.float64)
    assert g.shape == t.shape, (g.shape, t.shape)
    assert np.all(np.isfinite(g)), what + ": non-finite outputs"
    err = np.abs(g - t)
    bound = ulps * bf16_ulp(np.maximum(np.abs(g), np.abs(t))) + 2 * gamma(k) * absprod
    if acc is not None:
        bound = bound + bf16_ulp(np.abs(np.asarray(acc, np.float64)))
    bad = err > bound
    scale = max(np.abs(t).max(), 1e-6)
    stats = {
        "n": int(err.size),
        "exact": float(np.mean(err == 0)),
        "max_err": float(err.max()),
        "max_ulp": float((err / bf16_ulp(np.maximum(np.abs(t), 2.0 ** -126))).max()),
        "gate": float(err.max() / scale),
    }
    if bad.any():
        i = np.argwhere(bad)[0]
        raise AssertionError("%s: %d of %d outputs beyond 2 ulp + f32 bound, first at %s: got %r "
                             "want %r bound %r" % (what, int(bad.sum()), bad.size, tuple(i),
                                                   g[tuple(i)], t[tuple(i)], bound[tuple(i)]))
    assert err.max() <= scale / 64, what + ": beyond the 1/64-of-max gate"
    if min_exact is not None:
        assert stats["exact"] >= min_exact, "%s: %.4f of outputs bit-exact, below %.2f" % (
            what, stats["exact"], min_exact)
        clear = np.abs(t) > 16 * gamma(k) * absprod
        tight = ulps * bf16_ulp(np.abs(t))
        if acc is not None:
            tight = tight + bf16_ulp(np.abs(np.asarray(acc, np.float64)))
        far = clear & (err > tight)
        if far.any():
            i = np.argwhere(far)[0]
            raise AssertionError("%s: %d outputs outside the cancellation band beyond %g ulp, first at "
                                 "%s: got %r want %r" % (what, int(far.sum()), ulps, tuple(i),
                                                         g[tuple(i)], t[tuple(i)]))
        stats["clear"] = float(np.mean(clear))
    return stats
