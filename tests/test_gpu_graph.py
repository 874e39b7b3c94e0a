"""Recorded op sequences (hb_graph_record: the step's ops captured into a HIP
graph, the reference's one command buffer per step, qwen.rs:3177): every
replay gives the stream launches' bits, with eager work and synchronisation
between the replays, and the split-K workspace cannot move under a graph."""
import numpy as np
import pytest

import herbert_hip as hb

pytestmark = pytest.mark.gpu

SPLIT = dict(bm=128, bn=128, bk=64, wm=2, wn=2, mfma=16, dbuf=1, lds_dma=1, order=1, ksplit=2)


def test_graph_replays_equal_stream_launches():
    g = hb.Gpu(0)  # a context of its own: a fresh split-K workspace
    m, k, n, nv = 256, 768, 640, 1536
    x = hb.normal_bf16(0x5EED0300, 1.0, (m, k))
    w = hb.normal_bf16(0x5EED0301, 0.02, (n, k))
    y0 = hb.normal_bf16(0x5EED0302, 1.0, (m, n))
    wv = hb.normal_bf16(0x5EED0303, 0.02, (nv, n))
    try:
        st = g.alloc_with(np.array([0, 0, 0, m], np.uint32))
        W, X, Y, WV = g.alloc_with(w), g.alloc_with(x), g.alloc_with(y0), g.alloc_with(wv)
        Z = g.alloc(4 * nv * 2)
        kg = g.pipeline(hb.gemm_mma(k, n, hb.Out.Residual, **SPLIT))
        kv = g.pipeline(hb.matvec(n, nv, 0, mv_m=4, rows=1, split=1, form=2))
        # the matvec reads the GEMM's first 4 output rows: a dependent chain
        ops = [hb.Op(kg, [hb.r(st), hb.r(W), hb.r(X), hb.r(Y), hb.r(st), hb.r(st)], m),
               hb.Op(kv, [hb.r(WV), hb.r(Y, 0, 4 * n * 2), hb.r(Z)], 4)]
        g.time_ops(ops, 1)
        want_y = g.download(Y, np.uint16, m * n).reshape(m, n)
        want_z = g.download(Z, np.uint16, 4 * nv).reshape(4, nv)
        assert not np.array_equal(want_y, y0)
        gr = g.graph(ops)
        try:
            for rep in range(4):
                g.upload(Y, y0)          # eager work between replays
                g.zero(Z)
                if rep == 2:
                    g.time_ops(ops, 2)   # stream launches in between (they reuse the workspace)
                    g.upload(Y, y0)
                g.sync()
                gr.launch(1)
                g.sync()
                got_y = g.download(Y, np.uint16, m * n).reshape(m, n)
                got_z = g.download(Z, np.uint16, 4 * nv).reshape(4, nv)
                assert np.array_equal(got_y, want_y), "replay %d: the GEMM's rows" % rep
                assert np.array_equal(got_z, want_z), "replay %d: the matvec's rows" % rep
            # timing replays run (the output then holds several residual adds)
            assert gr.time(3) > 0
            # a split launch over more rows would grow the workspace: refused
            m2 = 512
            st2 = g.alloc_with(np.array([0, 0, 0, m2], np.uint32))
            X2, Y2 = g.alloc_with(hb.normal_bf16(1, 1.0, (m2, k))), g.alloc(m2 * n * 2)
            big = [hb.r(st2), hb.r(W), hb.r(X2), hb.r(Y2), hb.r(st2), hb.r(st2)]
            with pytest.raises(hb.HerbertError, match="cannot grow"):
                g.launch(kg, big, m2)
        finally:
            gr.free()
        g.launch(kg, big, m2)  # no graph alive: it grows
        g.sync()
    finally:
        g.close()
