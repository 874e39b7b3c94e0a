"""hb_moe_experts_run_static (no caller workspace, nothing allocated)
against hb_moe_experts_run (caller buffers) through the C ABI: bit-equal
outputs on two calls in a row, the second over fewer rows (the array keeps
the first call's contents), and a block too large for the array refused."""
import ctypes

import numpy as np
import pytest

import herbert_hip as hb

pytestmark = pytest.mark.gpu

hb.lib.hb_moe_experts_run_static.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_int32),
                                             ctypes.c_int32, ctypes.c_int32, hb.Range, hb.Range,
                                             hb.Range, hb.Range, hb.Range, ctypes.c_uint32]


def run_static(gpu, layer, out, m):
    b = layer.buf
    ks = (ctypes.c_int32 * 4)(*layer.kernels)
    return hb.lib.hb_moe_experts_run_static(gpu.h, ks, layer.swiglu_k, layer.combine_k,
                                            hb.r(b["route"]), hb.r(b["x"]), hb.r(b["w_gate_up"]),
                                            hb.r(b["w_down"]), hb.r(out), m)


@pytest.mark.parametrize("E,K,H,MI,rows", [(256, 8, 2048, 512, 64), (64, 4, 1024, 256, 512)])
def test_static_matches_caller_buffers(gpu, E, K, H, MI, rows):
    wgu = hb.normal_bf16(0x5EED0061, 0.02, (E * 2 * MI, H))
    wdn = hb.normal_bf16(0x5EED0062, 0.02, (E * H, MI))
    Wgu, Wdn = gpu.alloc_with(wgu), gpu.alloc_with(wdn)
    out = gpu.alloc(rows * H * 2)
    with hb.Engine(gpu, "") as e:
        layer = hb.MoeLayer(gpu, e, E, K, H, MI, rows, Wgu, Wdn,
                            scores=hb.normal_bf16(0x5EED0063, 1.0, (rows, E)),
                            x=hb.normal_bf16(0x5EED0064, 1.0, (rows, H)))
    try:
        b = layer.buf
        for i, m in enumerate((rows, rows // 2 - 3)):
            scores = hb.normal_bf16(0x5EED0070 + i, 1.0, (rows, E))
            x = hb.normal_bf16(0x5EED0080 + i, 1.0, (rows, H))
            gpu.upload(b["scores"], scores)
            gpu.upload(b["x"], x)
            gpu.upload(b["state"], np.array([0, 0, 0, m], np.uint32))
            print("[no-alloc] E=%d rows=%d call %d m=%d" % (E, rows, i, m), flush=True)
            layer.run(m)  # route, then the caller-buffer path into b["out"]
            gpu.sync()
            want = gpu.download(b["out"], np.uint16, m * H)
            gpu.zero(out)
            hb.check(run_static(gpu, layer, out, m))
            gpu.sync()
            got = gpu.download(out, np.uint16, m * H)
            assert np.array_equal(got, want), "call %d (m=%d): static scratch differs" % (i, m)
            assert not np.all(got == 0)
    finally:
        layer.free()
        for buf in (Wgu, Wdn, out):
            gpu.free(buf)


def test_static_refuses_blocks_beyond_the_array(gpu):
    """BASELINE config 5 at 2048 rows needs ~176 MiB of intermediates: refused
    with a message, nothing launched."""
    E, K, H, MI, rows = 256, 8, 2048, 512, 2048
    Wgu, Wdn = gpu.alloc(E * 2 * MI * H * 2), gpu.alloc(E * H * MI * 2)
    gpu.zero(Wgu)
    gpu.zero(Wdn)
    out = gpu.alloc(rows * H * 2)
    with hb.Engine(gpu, "moe.tile=64") as e:
        layer = hb.MoeLayer(gpu, e, E, K, H, MI, rows, Wgu, Wdn,
                            scores=hb.normal_bf16(5, 1.0, (rows, E)), x=hb.normal_bf16(6, 1.0, (rows, H)))
    try:
        rc = run_static(gpu, layer, out, rows)
        assert rc == hb.ERR_INVALID
        assert "bytes of scratch" in hb.last_error()
    finally:
        layer.free()
        for buf in (Wgu, Wdn, out):
            gpu.free(buf)


def test_static_refuses_a_dense_kernel_for_the_experts(gpu):
    """A dense GEMM (here a split-K pair, whose workspace the context would
    have to allocate) passed where a grouped expert GEMM belongs: refused
    before anything is launched or allocated."""
    E, K, H, MI, rows = 64, 4, 1024, 256, 64
    Wgu, Wdn = gpu.alloc(E * 2 * MI * H * 2), gpu.alloc(E * H * MI * 2)
    gpu.zero(Wgu)
    gpu.zero(Wdn)
    out = gpu.alloc(rows * H * 2)
    with hb.Engine(gpu, "") as e:
        layer = hb.MoeLayer(gpu, e, E, K, H, MI, rows, Wgu, Wdn,
                            scores=hb.normal_bf16(7, 1.0, (rows, E)), x=hb.normal_bf16(8, 1.0, (rows, H)))
    try:
        dense = gpu.pipeline(hb.gemm_mma(H, 2 * MI, 0, bm=128, bn=128, bk=64, wm=2, wn=2, mfma=16, dbuf=1,
                                         lds_dma=1, order=1, ksplit=2))
        good = list(layer.kernels)
        for slot in (1, 2):
            layer.kernels = list(good)
            layer.kernels[slot] = dense
            rc = run_static(gpu, layer, out, rows)
            assert rc == hb.ERR_INVALID, slot
            assert "grouped" in hb.last_error()
        layer.kernels = good
    finally:
        layer.free()
        for buf in (Wgu, Wdn, out):
            gpu.free(buf)
