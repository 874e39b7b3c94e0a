"""The C ABI (include/herbert_hip.h) without a GPU: the library loads, every
declared function is exported, the ctypes structs match the C layout, and
the calls that need no device behave (hb_open reports the missing device,
the seeded generator is deterministic and thread-count independent)."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

import herbert_hip as hb

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "herbert_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(hb_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported():
    names = declared_functions()
    assert len(names) >= 25, names
    missing = [n for n in names if not hasattr(hb.lib, n)]
    assert not missing, missing
    out = subprocess.run(["nm", "-D", "--defined-only", hb.LIB_PATH], capture_output=True,
                         text=True).stdout
    exported = set(re.findall(r" T (hb_\w+)", out))
    assert set(names) <= exported, set(names) - exported


def test_struct_layouts_match_c():
    src = """
#include <stdio.h>
#include <stddef.h>
#include "herbert_hip.h"
int main(void) {
  printf("%zu %zu %zu %zu %zu\\n", sizeof(hb_desc), sizeof(hb_range), sizeof(hb_op),
         sizeof(hb_moe_io), offsetof(hb_desc, unroll));
  return 0;
}
"""
    exe = os.path.join(ROOT, "herbert-metal-bf16_amd", "_build", "layout_check")
    os.makedirs(os.path.dirname(exe), exist_ok=True)
    r = subprocess.run(["gcc", "-x", "c", "-", "-I", os.path.dirname(HEADER), "-o", exe],
                       input=src, text=True, capture_output=True)
    assert r.returncode == 0, r.stderr
    sizes = [int(v) for v in subprocess.run([exe], capture_output=True, text=True).stdout.split()]
    assert sizes == [ctypes.sizeof(hb.Desc), ctypes.sizeof(hb.Range), ctypes.sizeof(hb.Op),
                     ctypes.sizeof(hb.MoeIo), hb.Desc.unroll.offset]


def test_open_without_device_reports_it():
    if os.environ.get("HIP_VISIBLE_DEVICES") is None and os.path.exists("/dev/kfd"):
        pytest.skip("a GPU is visible")
    h = ctypes.c_void_p()
    rc = hb.lib.hb_open(0, ctypes.byref(h))
    assert rc == hb.ERR_NO_DEVICE
    assert "no HIP device" in hb.last_error()


def test_seeded_generator_is_deterministic_and_normal():
    a = hb.normal_bf16(0x5EED0001, 1.0, (1000, 257), threads=1)
    b = hb.normal_bf16(0x5EED0001, 1.0, (1000, 257), threads=7)
    assert np.array_equal(a, b)
    c = hb.normal_bf16(0x5EED0002, 1.0, (1000, 257))
    assert not np.array_equal(a, c)
    f = hb.bf16_to_f32(a).astype(np.float64)
    assert abs(f.mean()) < 0.01 and abs(f.std() - 1) < 0.01
    g = hb.bf16_to_f32(hb.normal_bf16(3, 0.02, (100000,))).astype(np.float64)
    assert abs(g.std() - 0.02) < 0.001
    # every value is already a bf16 (round trip is the identity)
    assert np.array_equal(hb.f32_to_bf16(hb.bf16_to_f32(a)), a)


def test_library_fails_loudly_without_build(tmp_path):
    """Importing the package with no built library raises: no fallback."""
    code = ("import sys; sys.path.insert(0, %r); import herbert_hip" %
            os.path.join(ROOT, "herbert-metal-bf16_amd"))
    env = dict(os.environ)
    r = subprocess.run(["python3", "-c", code.replace("import herbert_hip",
                        "import builtins, os; os.path.exists = lambda p: False if p.endswith('libherbert_hip.so') else True; import herbert_hip")],
                       capture_output=True, text=True, env=env)
    assert r.returncode != 0 and "not built" in r.stderr


CLI = os.path.join(ROOT, "herbert-metal-bf16_amd", "hb_gemm")


def test_native_cli_usage_and_no_device():
    """hb_gemm (a C++ host linked against the library): usage on no shapes or
    a bad one (status 2); without a GPU the library's error, status 1."""
    r = subprocess.run([CLI], capture_output=True, text=True)
    assert r.returncode == 2 and "usage" in r.stderr
    r = subprocess.run([CLI, "12x34"], capture_output=True, text=True)
    assert r.returncode == 2 and "bad shape" in r.stderr
    if os.environ.get("HIP_VISIBLE_DEVICES") is None and os.path.exists("/dev/kfd"):
        pytest.skip("a GPU is visible")
    r = subprocess.run([CLI, "64x128x256"], capture_output=True, text=True)
    assert r.returncode == 1 and "no HIP device" in r.stderr


def test_shipped_library_has_no_development_hook():
    """The shipped library reads no HB_DEV_DEFINES (only a development build
    made by build.py --dev does): no environment variable can change what
    its kernels compute."""
    import herbert_hip as hb
    assert b"HB_DEV_DEFINES" not in open(hb.LIB_PATH, "rb").read()
