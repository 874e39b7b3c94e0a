"""The parity check itself (tests/parity.py check_close) must see the
mistakes a GEMM kernel plausibly makes at large K, and must pass correct
kernels that only sum in another order.  CPU only: the "kernels" here are
the oracle with one 32-wide slice of K removed, and float32 sums in other
orders (BLAS, split K in parts added in part order), rounded once."""
import numpy as np
import pytest

import hb_oracle as orc
from parity import abs_products, check_close
from test_oracle import orc_f32_to_bf16


def _inputs(m, k, n, seed):
    rng = np.random.default_rng(seed)
    x = orc_f32_to_bf16(rng.standard_normal((m, k)))
    w = orc_f32_to_bf16(rng.standard_normal((n, k)) * 0.02)
    return x, w


def _f32(b):
    return (b.astype(np.uint32) << np.uint32(16)).view(np.float32)


K_LARGE = 17408  # the 27B-class down projection


def test_dropped_k_slice_is_caught_at_large_k():
    m, n = 8, 256
    x, w = _inputs(m, K_LARGE, n, 1)
    want = orc.gemm(x, w)
    ap = abs_products(x, w)
    for lo in (0, 4096, K_LARGE - 32):
        xd = x.copy()
        xd[:, lo:lo + 32] = 0            # the kernel skipped K slice [lo, lo+32)
        bad = orc.gemm(xd, w)
        # the plain per-element bound (2 ulp + the f32 term) alone can miss it ...
        # ... but the bit-exact fraction and the tight bound cannot
        with pytest.raises(AssertionError):
            check_close(bad, want, K_LARGE, ap, "dropped slice %d" % lo, min_exact=0.98)


def test_dropped_k_slice_is_caught_with_residual():
    m, n = 8, 256
    x, w = _inputs(m, K_LARGE, n, 2)
    rng = np.random.default_rng(3)
    y0 = orc_f32_to_bf16(rng.standard_normal((m, n)))
    want = orc.gemm(x, w, orc.OUT_RESIDUAL, y0)
    acc = orc.gemm(x, w, orc.OUT_F32)
    xd = x.copy()
    xd[:, 9000:9032] = 0
    bad = orc.gemm(xd, w, orc.OUT_RESIDUAL, y0)
    with pytest.raises(AssertionError):
        check_close(bad, want, K_LARGE, abs_products(x, w), "residual dropped slice", acc=acc,
                    min_exact=0.98)


@pytest.mark.parametrize("k", [1024, 9216, K_LARGE])
def test_reordered_f32_sums_pass(k):
    """Correct kernels summing in another order: numpy's float32 matmul
    (BLAS blocking) and a 4-part split K added in part order."""
    m, n = 8, 512
    x, w = _inputs(m, k, n, k)
    want = orc.gemm(x, w)
    ap = abs_products(x, w)
    xf, wf = _f32(x), _f32(w)
    blas = orc_f32_to_bf16(xf @ wf.T)
    st = check_close(blas, want, k, ap, "blas order k=%d" % k, min_exact=0.98)
    assert st["exact"] > 0.99
    parts = np.zeros((m, n), np.float32)
    q = k // 4
    for p in range(4):
        parts = parts + (xf[:, p * q:(p + 1) * q] @ wf[:, p * q:(p + 1) * q].T).astype(np.float32)
    check_close(orc_f32_to_bf16(parts), want, k, ap, "split-4 order k=%d" % k, min_exact=0.98)
