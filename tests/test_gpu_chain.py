"""The decode chain (hb_mv_chain_build: a step's matvecs in one cooperative
launch, each phase waiting for the one before it) against the oracle: a
chain whose phases read the previous phase's output, so a phase that ran
before its input was complete reads stale rows and fails the contract; the
sync words back at zero after every launch; replays; and the decode step's
own shapes (qkv, o, gate|up, down, lm_head) at 1, 4 and 8 rows."""
import numpy as np
import pytest

import herbert_hip as hb
import hb_oracle as orc
from parity import abs_products, check_close

pytestmark = pytest.mark.gpu


def _run_chain(gpu, shapes, xs0, ws, y0s, m, groups=0, launches=1, dependent=True):
    """Builds the chain, its table (phase p's x = phase p-1's y when
    dependent), launches it `launches` times (the Residual outputs reset to
    y0 before each), returns the outputs of the last launch and the sync
    words after each."""
    k = gpu.mv_chain(shapes, m, groups)
    W = [gpu.alloc_with(w) for w in ws]
    X0 = gpu.alloc_with(xs0)
    Y = [gpu.alloc_with(y0) for y0 in y0s]
    T = gpu.alloc(24 * len(shapes))
    S = gpu.alloc(4 * (len(shapes) + 1))
    gpu.zero(S)
    io = []
    for p, (kk, n, out) in enumerate(shapes):
        x = hb.r(X0) if p == 0 or not dependent else hb.r(Y[p - 1], 0, m * kk * 2)
        io.append((hb.r(W[p]), x, hb.r(Y[p])))
    gpu.mv_chain_table(k, io, m, hb.r(T))
    syncs = []
    try:
        for _ in range(launches):
            for p, y0 in enumerate(y0s):
                gpu.upload(Y[p], y0)
            gpu.launch(k, [hb.r(T), hb.r(S)], m)
            gpu.sync()
            syncs.append(gpu.download(S, np.uint32, len(shapes) + 1))
        outs = []
        for p, (kk, n, out) in enumerate(shapes):
            dt = np.float32 if out == 1 else np.uint16
            outs.append(gpu.download(Y[p], dt, m * n).reshape(m, n))
        return gpu.kernel_name(k), outs, syncs
    finally:
        for b in W + Y + [X0, T, S]:
            gpu.free(b)


@pytest.mark.parametrize("m", [1, 4, 8])
@pytest.mark.parametrize("groups", [0, 512])
def test_dependent_chain_within_contract(gpu, m, groups):
    shapes = [(512, 1536, 0), (1536, 1024, 2), (1024, 700, 1)]
    rng = np.random.default_rng(m)
    x0 = hb.normal_bf16(0x5EED0400 + m, 1.0, (m, 512))
    ws = [hb.normal_bf16(0x5EED0410 + p, 0.02 if p != 1 else 0.05, (n, kk)) for p, (kk, n, _) in enumerate(shapes)]
    # every output starts from rows the chain must overwrite (stale values)
    y0s = [hb.normal_bf16(0x5EED0420 + p, 3.0, (m, n)) if out != 1 else
           rng.standard_normal((m, n)).astype(np.float32) for p, (kk, n, out) in enumerate(shapes)]
    name, outs, syncs = _run_chain(gpu, shapes, x0, ws, y0s, m, groups, launches=3)
    print("[chain]", name, flush=True)
    for s in syncs:
        assert np.all(s == 0), ("sync words after a launch", s)
    ya, yb, yc = outs
    check_close(ya, orc.gemm(x0, ws[0]), 512, abs_products(x0, ws[0]), "phase 0 m=%d" % m, min_exact=0.98)
    check_close(yb, orc.gemm(ya, ws[1], orc.OUT_RESIDUAL, y0s[1]), 1536, abs_products(ya, ws[1]),
                "phase 1 (Residual on phase 0's rows) m=%d" % m, acc=orc.gemm(ya, ws[1], orc.OUT_F32))
    check_close(yc, orc.gemm(yb, ws[2], orc.OUT_F32), 1024, abs_products(yb, ws[2]),
                "phase 2 (F32 on phase 1's rows) m=%d" % m)


DECODE = [("qkv", 2560, 4608, 0), ("o", 4096, 2560, 2), ("gate_up", 2560, 18432, 0),
          ("down", 9216, 2560, 2), ("lm_head", 2560, 151936, 0)]


@pytest.mark.parametrize("m", [1, 4, 8])
def test_decode_shapes_within_contract(gpu, m):
    """The decode step's five shapes as independent phases (each reads its
    own x), sampled output columns against the oracle."""
    shapes = [(k, n, o) for _, k, n, o in DECODE]
    xs = {k: hb.normal_bf16(0x5EED0003, 1.0, (m, k)) for _, k, _, _ in DECODE}
    ws = [hb.normal_bf16(0x5EED0430 + i, 0.02, (n, k)) for i, (_, k, n, _) in enumerate(DECODE)]
    y0s = [hb.normal_bf16(0x5EED0440 + i, 1.0, (m, n)) for i, (_, k, n, _) in enumerate(DECODE)]
    k_ = gpu.mv_chain(shapes, m)
    W = [gpu.alloc_with(w) for w in ws]
    X = {k: gpu.alloc_with(x) for k, x in xs.items()}
    Y = [gpu.alloc_with(y0) for y0 in y0s]
    T, S = gpu.alloc(24 * len(shapes)), gpu.alloc(4 * (len(shapes) + 1))
    gpu.zero(S)
    try:
        gpu.mv_chain_table(k_, [(hb.r(W[i]), hb.r(X[k]), hb.r(Y[i])) for i, (_, k, n, o) in enumerate(DECODE)],
                           m, hb.r(T))
        gpu.launch(k_, [hb.r(T), hb.r(S)], m)
        gpu.sync()
        assert np.all(gpu.download(S, np.uint32, len(shapes) + 1) == 0)
        for i, (nm, k, n, o) in enumerate(DECODE):
            got = gpu.download(Y[i], np.uint16, m * n).reshape(m, n)
            sel = np.unique(np.concatenate([np.arange(0, n, max(1, n // 509)), [n - 1]]))
            want = orc.gemm(xs[k], ws[i][sel], o, None if o != 2 else y0s[i][:, sel])
            acc = orc.gemm(xs[k], ws[i][sel], orc.OUT_F32) if o == 2 else None
            check_close(got[:, sel], want, k, abs_products(xs[k], ws[i][sel]), "%s m=%d" % (nm, m), acc=acc,
                        min_exact=0.98)
    finally:
        for b in W + Y + list(X.values()) + [T, S]:
            gpu.free(b)


def test_chain_refusals(gpu):
    with pytest.raises(hb.HerbertError, match="multiple of 512"):
        gpu.mv_chain([(2000, 64, 0)], 1)
    with pytest.raises(hb.HerbertError, match="LDS"):
        gpu.mv_chain([(17408, 64, 0)], 8)
    k = gpu.mv_chain([(512, 64, 0)], 2)
    T, S = gpu.alloc(24), gpu.alloc(8)
    W, X, Y = gpu.alloc(64 * 512 * 2), gpu.alloc(2 * 512 * 2), gpu.alloc(2 * 64 * 2 - 2)
    try:
        with pytest.raises(hb.HerbertError, match="y holds"):
            gpu.mv_chain_table(k, [(hb.r(W), hb.r(X), hb.r(Y))], 2, hb.r(T))
        with pytest.raises(hb.HerbertError, match="rows"):
            gpu.launch(k, [hb.r(T), hb.r(S)], 3)
    finally:
        for b in (T, S, W, X, Y):
            gpu.free(b)
