"""BASELINE config 5 at full size through the selection's own picks: an MoE
layer of 2048 tokens, 256 experts, top 8, hidden 2048, expert intermediate
512 (qwen.rs:2326-2391 expert_pipes picks the sort and the grouped GEMMs,
qwen.rs:2705-2735 the op order), with the tile rows chosen by the timed
selection and forced to 16, 32 and 64 (moe.tile).  Checked against the
oracle: the route and the sort bit for bit (the atomic sort by its
invariants), the grouped gate|up's SwiGLU output and the grouped down within
the contract, the combine bit for bit on the GPU's slot rows; and the native
dispatch sequence (hb_moe_experts_run) bit-equal to the op list."""
import numpy as np
import pytest

import herbert_hip as hb
import hb_oracle as orc
from parity import abs_products, bf16_to_f32, bf16_ulp, check_close, gamma

pytestmark = pytest.mark.gpu

T, E, TOPK, H, MI = 2048, 256, 8, 2048, 512
P = T * TOPK


def sorted_experts(lst, route):
    return route[lst // TOPK, lst % TOPK]


def check_sort(lst, tiles, route, bm):
    """The scan form's exact list and table, or the atomic form's invariants
    (any order within an expert): a permutation of the pairs grouped by
    ascending expert, the table covering each expert's run in chunks of at
    most bm (prefill.rs:1315-1531)."""
    want_l, want_t = orc.moe_sort(route, TOPK, E, bm)
    if np.array_equal(lst, want_l):
        assert np.array_equal(tiles[:1 + 3 * int(want_t[0])], want_t[:1 + 3 * int(want_t[0])])
        return
    assert np.array_equal(np.sort(lst), np.arange(P))
    ex = sorted_experts(lst, route)
    assert np.all(np.diff(ex.astype(np.int64)) >= 0)
    assert np.array_equal(tiles[:1 + 3 * int(want_t[0])], want_t[:1 + 3 * int(want_t[0])])


def swiglu_bound(g, u, dg, du, h):
    """|dh| for h = g sigmoid(g) u with g, u known to within dg, du, plus the
    final rounding of h: the contract's bound carried through the SwiGLU."""
    s = 1.0 / (1.0 + np.exp(-g))
    dhdg = np.abs(u * s * (1.0 + g * (1.0 - s)))
    dhdu = np.abs(g * s)
    return dhdg * dg + dhdu * du + 2 * bf16_ulp(h)


@pytest.mark.parametrize("tune", ["", "moe.tile=16", "moe.tile=32", "moe.tile=64"])
def test_config5_layer_through_picks(gpu, tune):
    wgu = hb.normal_bf16(0x5EED0051, 0.02, (E * 2 * MI, H))
    wdn = hb.normal_bf16(0x5EED0052, 0.02, (E * H, MI))
    scores = hb.normal_bf16(0x5EED0005, 1.0, (T, E))
    x = hb.normal_bf16(0x5EED0053, 1.0, (T, H))
    Wgu, Wdn = gpu.alloc_with(wgu), gpu.alloc_with(wdn)
    with hb.Engine(gpu, tune) as e:
        layer = hb.MoeLayer(gpu, e, E, TOPK, H, MI, T, Wgu, Wdn, scores=scores, x=x)
    try:
        names = [gpu.kernel_name(k) for k in layer.kernels if k >= 0]
        print("[moe full] tune=%r bm=%d %s" % (tune, layer.bm, names), flush=True)
        if tune:
            assert layer.bm == int(tune.split("=")[1])
        b = layer.buf
        gpu.time_ops(layer.ops(), 1)
        out_ops = gpu.download(b["out"], np.uint16, T * H).reshape(T, H)
        gpu.zero(b["out"])
        layer.run()
        gpu.sync()
        out = gpu.download(b["out"], np.uint16, T * H).reshape(T, H)
        assert np.array_equal(out, out_ops), "hb_moe_experts_run differs from the op list"

        route = gpu.download(b["route"], np.uint32, T * 2 * TOPK).reshape(T, -1)
        assert np.array_equal(route, orc.route(scores, TOPK))
        lst = gpu.download(b["list"], np.uint32, P)
        nt = hb.moe_tiles(T, TOPK, E, layer.bm)
        tiles = gpu.download(b["tiles"], np.uint32, 1 + 3 * nt)
        check_sort(lst, tiles, route, layer.bm)
        ex = sorted_experts(lst, route)

        # The grouped gate|up + SwiGLU (fused or not) against the oracle's
        # sums carried through the SwiGLU, every sorted pair.
        ehb = gpu.download(b["ehb"], np.uint16, P * MI).reshape(P, MI)
        xr = x[lst // TOPK]
        gu = np.empty((P, 2 * MI), np.uint16)
        ap = np.empty((P, 2 * MI))
        for e_ in np.unique(ex):
            sel = np.nonzero(ex == e_)[0]
            wr = wgu[e_ * 2 * MI:(e_ + 1) * 2 * MI]
            gu[sel] = orc.gemm(xr[sel], wr)
            ap[sel] = abs_products(xr[sel], wr)
        if not layer.fused:
            egu = gpu.download(b["egu"], np.uint16, P * 2 * MI).reshape(P, 2 * MI)
            check_close(egu, gu, H, ap, "grouped gate|up " + tune, min_exact=0.98)
        g, u = (bf16_to_f32(gu[:, :MI]).astype(np.float64), bf16_to_f32(gu[:, MI:]).astype(np.float64))
        dg = 2 * bf16_ulp(g) + 2 * gamma(H) * ap[:, :MI]
        du = 2 * bf16_ulp(u) + 2 * gamma(H) * ap[:, MI:]
        want_h = orc.swiglu(gu, MI).reshape(P, MI)
        hf, wf = bf16_to_f32(ehb).astype(np.float64), bf16_to_f32(want_h).astype(np.float64)
        bound = swiglu_bound(g, u, dg, du, np.maximum(np.abs(hf), np.abs(wf)))
        bad = np.abs(hf - wf) > bound
        assert not bad.any(), ("swiglu'd gate|up beyond the bound", int(bad.sum()))
        assert np.mean(ehb == want_h) > 0.95

        # The grouped down (Scatter to slot rows) on the GPU's h.
        ey = gpu.download(b["ey"], np.uint16, P * H).reshape(P, H)
        want_ey = orc.experts_gemm(ehb, wdn, lst, tiles, MI, H, 2, TOPK, P)
        apd = np.empty((P, H))
        for e_ in np.unique(ex):
            sel = np.nonzero(ex == e_)[0]
            apd[lst[sel]] = abs_products(ehb[sel], wdn[e_ * H:(e_ + 1) * H])
        check_close(ey, want_ey, MI, apd, "grouped down " + tune, min_exact=0.98)

        # moe_combine on the GPU's slot rows: bit for bit.
        assert np.array_equal(out, orc.combine(ey, route, TOPK, H))
    finally:
        layer.free()
        gpu.free(Wgu)
        gpu.free(Wdn)
