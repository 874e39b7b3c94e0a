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
    """hb_zero of byte ranges with a ragged head, a ragged tail, both inside
    one 16-byte word, and whole words: exactly [offset, offset + bytes)
    becomes zero."""
    a = np.full(1000, 0xAB, np.uint8)
    A = gpu.alloc_with(a)
    try:
        for off, n in [(3, 517), (0, 1000), (5, 3), (16, 32), (15, 2), (1, 15), (0, 1),
                       (999, 1), (8, 992)]:
            gpu.upload(A, a)
            gpu.zero(A, off, n)
            got = gpu.download(A, np.uint8, 1000)
            want = a.copy()
            want[off:off + n] = 0
            assert np.array_equal(got, want), (off, n)
    finally:
        gpu.free(A)


def test_native_cli_runs_gemm_and_matvec():
    """hb_gemm picks, checks and times a GEMM of each Out mode and a matvec
    through the C ABI from a native process: one line per shape, the
    [autotune] log on stderr."""
    import os
    import subprocess
    cli = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                       "herbert-metal-bf16_amd", "hb_gemm")
    r = subprocess.run([cli, "--reps", "5", "512x1024x3584", "256x512x768r", "128x256x512f", "mv:4x2560x4608"],
                       capture_output=True, text=True, timeout=110)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = r.stdout.strip().splitlines()
    assert len(lines) == 4, r.stdout
    assert lines[0].startswith("512x1024x3584 gemm_") and lines[0].endswith("TFLOP/s")
    assert lines[1].startswith("256x512x768r gemm_") and "_res" in lines[1]
    assert lines[2].startswith("128x256x512f gemm_") and "_f32" in lines[2]
    assert lines[3].startswith("mv:4x2560x4608 matvec_") and lines[3].endswith("GB/s")
    assert "[autotune] gemm 1024x3584" in r.stderr
