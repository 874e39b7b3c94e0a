"""The device-memory plumbing around the kernels: hb_copy and hb_zero."""
import numpy as np
import pytest

import herbert_hip as hb

pytestmark = pytest.mark.gpu


def test_copy_and_refusals(gpu):
    a = np.arange(100003, dtype=np.uint8) * 7
    A = gpu.alloc_with(a)
    B = gpu.alloc(len(a))
    try:
        gpu.copy(hb.r(B, 0, len(a)), hb.r(A, 0, len(a)))
        gpu.sync()
        assert np.array_equal(gpu.download(B, np.uint8, len(a)), a)
        gpu.copy(hb.r(B, 5, 1000), hb.r(A, 77, 1000))
        gpu.sync()
        assert np.array_equal(gpu.download(B, np.uint8, 1000, 5), a[77:1077])
        with pytest.raises(hb.HerbertError, match="different sizes"):
            gpu.copy(hb.r(B, 0, 10), hb.r(A, 0, 11))
        with pytest.raises(hb.HerbertError, match="overlap"):
            gpu.copy(hb.r(A, 0, 100), hb.r(A, 50, 100))
    finally:
        gpu.free(A)
        gpu.free(B)


def test_zero_ragged(gpu):
    a = np.full(1000, 0xAB, np.uint8)
    A = gpu.alloc_with(a)
    try:
        gpu.zero(A, 3, 517)
        got = gpu.download(A, np.uint8, 1000)
    finally:
        gpu.free(A)
    want = a.copy()
    want[3:520] = 0
    assert np.array_equal(got, want)
