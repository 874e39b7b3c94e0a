"""Parity of the HIP MoE path with the CPU oracle: route (route_qwen,
qwen_kernels.rs:1802-1884) and sort (moe_sort, prefill.rs:1315-1448) bit for
bit, the atomic sort by its invariants, gather, SwiGLU and combine bit for
bit, and the grouped gate|up (Gather) / down (Scatter) GEMM within the
contract, at BASELINE config 5's shape (2048 tokens, 256 experts, top 8)."""
import numpy as np
import pytest

import herbert_hip as hb
import hb_oracle as orc
from parity import abs_products, bf16_to_f32, check_close

pytestmark = pytest.mark.gpu

T, E, TOPK, H, MI = 2048, 256, 8, 2048, 512


def launch(gpu, desc, arrays, m, outs):
    """Runs one kernel on uploaded arrays; returns the downloaded `outs`
    ({index: (dtype, count)})."""
    bufs = [gpu.alloc_with(a) if isinstance(a, np.ndarray) else gpu.alloc(a) for a in arrays]
    try:
        kern = gpu.pipeline(desc)
        gpu.launch(kern, [hb.r(b) for b in bufs], m)
        gpu.sync()
        return {i: gpu.download(bufs[i], dt, cnt) for i, (dt, cnt) in outs.items()}
    finally:
        for b in bufs:
            gpu.free(b)


def route_gpu(gpu, scores, top_k):
    rows, experts = scores.shape
    d = hb.Desc(kind=hb.Kind.ROUTE, experts=experts, top_k=top_k)
    res = launch(gpu, d, [scores, rows * 2 * top_k * 4], rows, {1: (np.uint32, rows * 2 * top_k)})
    return res[1].reshape(rows, 2 * top_k)


def test_route_bit_exact(gpu):
    scores = hb.normal_bf16(0x5EED0005, 1.0, (T, E))
    scores[5, 17] = scores[5, 100] = scores[5].max()  # an exact tie at the top
    scores[6, :] = scores[6, 0]  # a row of equal scores
    got = route_gpu(gpu, scores, TOPK)
    want = orc.route(scores, TOPK)
    assert np.array_equal(got, want)
    small = hb.normal_bf16(3, 1.0, (37, 64))
    assert np.array_equal(route_gpu(gpu, small, 4), orc.route(small, 4))


def sort_gpu(gpu, route, top_k, experts, bm, rows_max, atomic=False, m=None):
    rows = route.shape[0]
    m = rows if m is None else m
    tiles = hb.moe_tiles(rows_max, top_k, experts, bm)
    d = hb.Desc(kind=hb.Kind.SORT_ATOMIC if atomic else hb.Kind.SORT, experts=experts,
                top_k=top_k, bm=bm, rows_max=rows_max)
    st = np.array([0, 0, 0, m], np.uint32)
    res = launch(gpu, d, [st, route, rows * top_k * 4, (1 + 3 * tiles) * 4], m,
                 {2: (np.uint32, m * top_k), 3: (np.uint32, 1 + 3 * tiles)})
    return res[2], res[3]


@pytest.mark.parametrize("bm", [16, 32, 64, 128])
def test_sort_bit_exact_and_atomic_invariants(gpu, bm):
    scores = hb.normal_bf16(0x5EED0005, 1.0, (T, E))
    route = orc.route(scores, TOPK)
    lst, tiles = sort_gpu(gpu, route, TOPK, E, bm, T)
    wl, wt = orc.moe_sort(route, TOPK, E, bm)
    assert np.array_equal(lst, wl)
    assert np.array_equal(tiles[:1 + 3 * int(wt[0])], wt[:1 + 3 * int(wt[0])])
    al, at = sort_gpu(gpu, route, TOPK, E, bm, T, atomic=True)
    assert np.array_equal(at[:1 + 3 * int(wt[0])], wt[:1 + 3 * int(wt[0])])
    ex = route[al // TOPK, al % TOPK]
    wex = route[wl // TOPK, wl % TOPK]
    assert np.array_equal(ex, wex)  # same expert runs
    assert np.array_equal(np.sort(al), np.arange(T * TOPK))  # a permutation


def test_sort_partial_block(gpu):
    """state[3] rows below the kernel's rows_max (a prompt's last block)."""
    scores = hb.normal_bf16(4, 1.0, (300, E))
    route = orc.route(scores, TOPK)
    lst, tiles = sort_gpu(gpu, route, TOPK, E, 32, 512, m=300)
    wl, wt = orc.moe_sort(route, TOPK, E, 32)
    assert np.array_equal(lst, wl)
    used = 1 + 3 * int(wt[0])
    assert np.array_equal(tiles[:used], wt[:used])


@pytest.mark.parametrize("experts,top_k,rows,rows_max,bm", [(200, 6, 5000, 8192, 16),
                                                         (1000, 2, 333, 512, 64),
                                                         (64, 1, 1, 64, 32)])
def test_sort_other_shapes(gpu, experts, top_k, rows, rows_max, bm):
    """Expert counts that are not a multiple of 64 and up to 1024, blocks
    whose pairs exceed what a thread keeps in registers (8192 rows x 6 slots)
    and a single row: the scan sort bit for bit, the atomic sort by its
    invariants."""
    rng = np.random.default_rng(experts * 7 + top_k)
    route = np.zeros((rows, 2 * top_k), np.uint32)
    for r in range(rows):
        route[r, :top_k] = np.sort(rng.choice(experts, top_k, replace=False))
        route[r, top_k:] = np.float32(1.0 / top_k).view(np.uint32)
    lst, tiles = sort_gpu(gpu, route, top_k, experts, bm, rows_max)
    wl, wt = orc.moe_sort(route, top_k, experts, bm)
    used = 1 + 3 * int(wt[0])
    assert np.array_equal(lst, wl)
    assert np.array_equal(tiles[:used], wt[:used])
    al, at = sort_gpu(gpu, route, top_k, experts, bm, rows_max, atomic=True)
    assert np.array_equal(at[:used], wt[:used])
    assert np.array_equal(route[al // top_k, al % top_k], route[wl // top_k, wl % top_k])
    assert np.array_equal(np.sort(al), np.arange(rows * top_k))


def test_gather_swiglu_combine_bit_exact(gpu):
    rows = 300
    x = hb.normal_bf16(5, 1.0, (rows, H))
    route = orc.route(hb.normal_bf16(6, 1.0, (rows, E)), TOPK)
    lst, _ = orc.moe_sort(route, TOPK, E, 32)
    st = np.array([0, 0, 0, rows], np.uint32)
    d = hb.Desc(kind=hb.Kind.GATHER, n=H, top_k=TOPK)
    xs = launch(gpu, d, [st, lst, x, rows * TOPK * H * 2], rows, {3: (np.uint16, rows * TOPK * H)})[3]
    assert np.array_equal(xs.reshape(-1, H), orc.gather_rows(x, lst, TOPK))

    gu = hb.normal_bf16(7, 2.0, (rows * TOPK, 2 * MI))
    d = hb.Desc(kind=hb.Kind.SWIGLU, n=MI)
    h = launch(gpu, d, [gu, rows * TOPK * MI * 2], rows * TOPK, {1: (np.uint16, rows * TOPK * MI)})[1]
    assert np.array_equal(h.reshape(-1, MI), orc.swiglu(gu, MI))

    y = hb.normal_bf16(8, 1.0, (rows * TOPK, H))
    d = hb.Desc(kind=hb.Kind.COMBINE, n=H, top_k=TOPK)
    out = launch(gpu, d, [y, route, rows * H * 2], rows, {2: (np.uint16, rows * H)})[2]
    assert np.array_equal(out.reshape(rows, H), orc.combine(y, route, TOPK, H))


def experts_run(gpu, x, w, lst, tiles, k, n, rows_of, rows, bm, m_first=True, **tile):
    pairs = rows * TOPK
    ntiles = hb.moe_tiles(rows, TOPK, E, bm)
    d = hb.gemm_mma_rows(k, n, 0, m_first, rows_of, top_k=TOPK, tiles=ntiles, bm=bm, experts=E,
                         rows_max=rows, **tile)
    st = np.array([0, 0, 0, rows], np.uint32)
    tl = np.zeros(1 + 3 * ntiles, np.uint32)
    tl[:len(tiles)] = tiles
    y = np.zeros((pairs, n), np.uint16)
    return launch(gpu, d, [st, w, x, y, lst, tl], rows, {3: (np.uint16, pairs * n)})[3].reshape(pairs, n)


EXPERT_TILES = {
    "m16_reg": dict(wm=1, wn=4, mfma=16, bn=128, bk=64, dbuf=0, lds_dma=0),
    "m32_reg_d": dict(wm=1, wn=4, mfma=16, bn=128, bk=64, dbuf=1, lds_dma=0),
    "m64_dma": dict(wm=1, wn=4, mfma=16, bn=256, bk=64, dbuf=1, lds_dma=1),
    "m16_dma": dict(wm=1, wn=4, mfma=16, bn=128, bk=64, dbuf=1, lds_dma=1),
    "m128_w2x2": dict(wm=2, wn=2, mfma=16, bn=128, bk=64, dbuf=1, lds_dma=1),
    "m64_w2x4_s3": dict(wm=2, wn=4, mfma=16, bn=128, bk=64, dbuf=2, lds_dma=1),
    "m16_dma_nf": dict(wm=1, wn=4, mfma=16, bn=128, bk=64, dbuf=1, lds_dma=1, m_first=False),
    "m128_wnt_nf": dict(wm=1, wn=4, mfma=16, bn=128, bk=64, dbuf=1, lds_dma=1, m_first=False, w_nt=1),
    "m128_n256_w8_s3_nf_wnt": dict(wm=2, wn=4, mfma=16, bn=256, bk=64, dbuf=2, lds_dma=1, m_first=False,
                                   w_nt=1, order=1),
    "m32_mf_o1": dict(wm=1, wn=4, mfma=16, bn=128, bk=64, dbuf=1, lds_dma=1, order=1),
}


@pytest.mark.parametrize("tname,bm", [("m16_reg", 16), ("m32_reg_d", 32), ("m64_dma", 64),
                                      ("m16_dma", 16), ("m128_w2x2", 128), ("m64_w2x4_s3", 64),
                                      ("m16_dma_nf", 16), ("m128_wnt_nf", 128),
                                      ("m128_n256_w8_s3_nf_wnt", 128), ("m32_mf_o1", 32)])
def test_grouped_gemm_gather_and_scatter(gpu, tname, bm):
    """Config 5's grouped gate|up (Gather: sorted row p reads X row
    list[p]/top_k) and down (Scatter: writes row list[p]), on 512 tokens
    (4096 pairs) with every output checked against the oracle."""
    rows = 512
    x = hb.normal_bf16(0x5EED0007, 1.0, (rows, H))
    route = orc.route(hb.normal_bf16(0x5EED0005, 1.0, (rows, E)), TOPK)
    lst, tiles = orc.moe_sort(route, TOPK, E, bm)
    wgu = hb.normal_bf16(0x5EED0008, 0.02, (E * 2 * MI, H))
    got = experts_run(gpu, x, wgu, lst, tiles, H, 2 * MI, hb.Rows.Gather, rows, bm, **EXPERT_TILES[tname])
    want = orc.experts_gemm(x, wgu, lst, tiles, H, 2 * MI, 1, TOPK, rows * TOPK)
    # abs products per sorted row: its token row against its expert's rows
    ap = np.empty(want.shape)
    ex = route[lst // TOPK, lst % TOPK]
    for e in np.unique(ex):
        sel = np.nonzero(ex == e)[0]
        ap[sel] = abs_products(x[lst[sel] // TOPK], wgu[e * 2 * MI:(e + 1) * 2 * MI])
    check_close(got, want, H, ap, "gate_up " + tname, min_exact=0.98)

    xs = hb.normal_bf16(0x5EED0009, 1.0, (rows * TOPK, MI))
    wd = hb.normal_bf16(0x5EED000A, 0.02, (E * H, MI))
    got = experts_run(gpu, xs, wd, lst, tiles, MI, H, hb.Rows.Scatter, rows, bm, **EXPERT_TILES[tname])
    want = orc.experts_gemm(xs, wd, lst, tiles, MI, H, 2, TOPK, rows * TOPK)
    ap = np.empty(want.shape)
    for e in np.unique(ex):
        sel = np.nonzero(ex == e)[0]
        ap[lst[sel]] = abs_products(xs[sel], wd[e * H:(e + 1) * H])
    check_close(got, want, MI, ap, "down " + tname, min_exact=0.98)


@pytest.mark.parametrize("bm,bn,wm,wn", [(32, 128, 1, 4), (128, 128, 2, 2), (64, 256, 1, 4)])
def test_grouped_gate_up_swiglu_fused(gpu, bm, bn, wm, wn):
    """The grouped gate|up with swiglu_slots in its epilogue: bit-equal to the
    same tile form's GEMM (EGU) followed by swiglu_slots (the sums run the
    same MFMA sequence), over the bench's route; rows of each expert's
    [gate | up] W."""
    rows, experts, top_k, hidden, inter = 512, 64, 4, 512, 256
    scores = hb.normal_bf16(0x5EED0041, 1.0, (rows, experts))
    route = orc.route(scores, top_k)
    lst, tiles = sort_gpu(gpu, route, top_k, experts, bm, rows)
    x = hb.normal_bf16(0x5EED0042, 1.0, (rows, hidden))
    w = hb.normal_bf16(0x5EED0043, 0.05, (experts * 2 * inter, hidden))
    P = rows * top_k
    nt = hb.moe_tiles(rows, top_k, experts, bm)
    st = np.array([0, 0, 0, rows], np.uint32)
    tile = dict(bm=bm, bn=bn, bk=64, wm=wm, wn=wn, mfma=16, dbuf=1, lds_dma=1, order=0)
    common = dict(top_k=top_k, tiles=nt, experts=experts, rows_max=rows)
    d = hb.gemm_mma_rows(hidden, 2 * inter, 0, True, hb.Rows.Gather, **common, **tile)
    egu = launch(gpu, d, [st, w, x, P * 2 * inter * 2, lst, tiles], rows,
                 {3: (np.uint16, P * 2 * inter)})[3].reshape(P, 2 * inter)
    want = launch(gpu, hb.swiglu_rows(inter), [egu, P * inter * 2], P, {1: (np.uint16, P * inter)})[1]
    ds = hb.Desc(kind=hb.Kind.GEMM_SWIGLU, k=hidden, n=inter, out=0, m_first=True, rows_of=hb.Rows.Gather,
                 **common, **tile)
    got = launch(gpu, ds, [st, w, x, P * inter * 2, lst, tiles], rows, {3: (np.uint16, P * inter)})[3]
    assert np.array_equal(got, want), "fused grouped gate|up+SwiGLU != GEMM then swiglu_slots"
    # And the unfused GEMM within the contract of the oracle on sampled pairs.
    sel = np.arange(0, P, 37)
    xr = x[lst[sel] // top_k]
    ex = route[lst[sel] // top_k, lst[sel] % top_k]
    for i, p in enumerate(sel):
        wr = w[ex[i] * 2 * inter:(ex[i] + 1) * 2 * inter]
        check_close(egu[p:p + 1], orc.gemm(xr[i:i + 1], wr), hidden, abs_products(xr[i:i + 1], wr),
                    "pair %d" % p)


@pytest.mark.parametrize("tname,bm", [("m128_w2x2", 128), ("m16_dma", 16),
                                      ("m128_n256_w8_s3_nf_wnt", 128)])
def test_skewed_route(gpu, tname, bm):
    """A route a trained router could give: three experts chosen by every
    token (512 rows each: several tiles of one expert), one by half the
    tokens, most experts by none.  The sort (both forms) against the oracle,
    the grouped gate|up / down within the contract on every output, and the
    combine of the GPU's slot rows bit for bit."""
    rows = 512
    scores = hb.normal_bf16(0x5EED0600, 1.0, (rows, E)).astype(np.uint32)
    f = (scores << 16).view(np.float32)
    f[:, [3, 7, 200]] += 8.0
    f[: rows // 2, 11] += 8.0
    cold = np.setdiff1d(np.arange(128, E), [200])
    f[:, cold] -= 8.0  # never chosen
    scores = orc_round(f)
    route = orc.route(scores, TOPK)
    counts = np.bincount(route[:, :TOPK].ravel(), minlength=E)
    assert counts[3] == counts[7] == counts[200] == rows and counts[11] >= rows // 2
    assert (counts == 0).sum() > E // 4
    lst, tiles = sort_gpu(gpu, route, TOPK, E, bm, rows)
    wl, wt = orc.moe_sort(route, TOPK, E, bm)
    used = 1 + 3 * int(wt[0])
    assert np.array_equal(lst, wl) and np.array_equal(tiles[:used], wt[:used])
    al, at = sort_gpu(gpu, route, TOPK, E, bm, rows, atomic=True)
    assert np.array_equal(at[:used], wt[:used])
    assert np.array_equal(route[al // TOPK, al % TOPK], route[wl // TOPK, wl % TOPK])

    x = hb.normal_bf16(0x5EED0601, 1.0, (rows, H))
    wgu = hb.normal_bf16(0x5EED0602, 0.02, (E * 2 * MI, H))
    got = experts_run(gpu, x, wgu, wl, wt, H, 2 * MI, hb.Rows.Gather, rows, bm, **EXPERT_TILES[tname])
    want = orc.experts_gemm(x, wgu, wl, wt, H, 2 * MI, 1, TOPK, rows * TOPK)
    ex = route[wl // TOPK, wl % TOPK]
    ap = np.empty(want.shape)
    for e in np.unique(ex):
        sel = np.nonzero(ex == e)[0]
        ap[sel] = abs_products(x[wl[sel] // TOPK], wgu[e * 2 * MI:(e + 1) * 2 * MI])
    check_close(got, want, H, ap, "skewed gate_up " + tname, min_exact=0.98)

    h = orc.swiglu(want, MI)
    wd = hb.normal_bf16(0x5EED0603, 0.02, (E * H, MI))
    ey = experts_run(gpu, h, wd, wl, wt, MI, H, hb.Rows.Scatter, rows, bm, **EXPERT_TILES[tname])
    want_ey = orc.experts_gemm(h, wd, wl, wt, MI, H, 2, TOPK, rows * TOPK)
    apd = np.empty(want_ey.shape)
    for e in np.unique(ex):
        sel = np.nonzero(ex == e)[0]
        apd[wl[sel]] = abs_products(h[sel], wd[e * H:(e + 1) * H])
    check_close(ey, want_ey, MI, apd, "skewed down " + tname, min_exact=0.98)
    d = hb.Desc(kind=hb.Kind.COMBINE, n=H, top_k=TOPK)
    out = launch(gpu, d, [ey, route, rows * H * 2], rows, {2: (np.uint16, rows * H)})[2]
    assert np.array_equal(out.reshape(rows, H), orc.combine(ey, route, TOPK, H))


def orc_round(f):
    """bf16 bits of float32 values, round to nearest even (core/bf16.rs:13-23)."""
    b = np.ascontiguousarray(f, np.float32).view(np.uint32)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
