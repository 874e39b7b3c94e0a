"""Parity of the HIP prefill GEMM (gemm_mma_rows, prefill.rs:838-1307) with
the CPU oracle: every Out mode, partial row tiles, every tile family the
autotuner can pick, the BASELINE configs (rows sampled for the oracle), and
size-independent properties at full size."""
import numpy as np
import pytest

import herbert_hip as hb
import hb_oracle as orc
from parity import abs_products, bf16_to_f32, check_close

pytestmark = pytest.mark.gpu

# The tile families of the candidate list (bm, bn, bk, wm, wn, mfma, stages, dma).
TILES = {
    "t128x128_x16_d2": dict(bm=128, bn=128, bk=64, wm=2, wn=2, mfma=16, dbuf=1, lds_dma=1, order=1),
    "t128x128_x32_d2": dict(bm=128, bn=128, bk=64, wm=2, wn=2, mfma=32, dbuf=1, lds_dma=1, order=1),
    "t256x256_x32_d2": dict(bm=256, bn=256, bk=64, wm=2, wn=2, mfma=32, dbuf=1, lds_dma=1, order=1),
    "t256x256_w8_d4": dict(bm=256, bn=256, bk=32, wm=4, wn=2, mfma=32, dbuf=3, lds_dma=1, order=1),
    "t256x128_d4": dict(bm=128, bn=256, bk=32, wm=2, wn=2, mfma=32, dbuf=3, lds_dma=1, order=1),
    "t128x128_reg_d1": dict(bm=128, bn=128, bk=64, wm=2, wn=2, mfma=16, dbuf=1, lds_dma=0, order=0),
    "t64x64_reg_s1": dict(bm=64, bn=64, bk=32, wm=1, wn=4, mfma=16, dbuf=0, lds_dma=0, order=0),
    "t256x192_w8_x32": dict(bm=256, bn=192, bk=64, wm=4, wn=2, mfma=32, dbuf=1, lds_dma=1, order=1),
    "t128x192_w8_s3": dict(bm=128, bn=192, bk=64, wm=2, wn=4, mfma=16, dbuf=2, lds_dma=1, order=0),
    "t128x192_w8_s4": dict(bm=128, bn=192, bk=64, wm=2, wn=4, mfma=16, dbuf=3, lds_dma=1, order=0),
    "t128x160_s3_k32": dict(bm=128, bn=160, bk=32, wm=2, wn=2, mfma=16, dbuf=2, lds_dma=1, order=1),
    "t128x160_x16": dict(bm=128, bn=160, bk=64, wm=2, wn=2, mfma=16, dbuf=1, lds_dma=1, order=1),
    "t128x128_band2": dict(bm=128, bn=128, bk=64, wm=2, wn=2, mfma=16, dbuf=1, lds_dma=1, order=0,
                           band=2),
    "t256x192_w8_x16_b4": dict(bm=256, bn=192, bk=64, wm=4, wn=2, mfma=16, dbuf=1, lds_dma=1, order=1,
                               band=4),
    "t256x256_w8_x32_b4": dict(bm=256, bn=256, bk=64, wm=4, wn=2, mfma=32, dbuf=1, lds_dma=1, order=1,
                               band=4),
    "t128x160_s4_b4": dict(bm=128, bn=160, bk=64, wm=2, wn=2, mfma=16, dbuf=3, lds_dma=1, order=1, band=4),
    "t64x128_s4_w8": dict(bm=64, bn=128, bk=64, wm=2, wn=4, mfma=16, dbuf=3, lds_dma=1, order=1),
    "t32x64_s3": dict(bm=32, bn=64, bk=64, wm=1, wn=4, mfma=16, dbuf=2, lds_dma=1, order=1),
    # the ping-pong schedule (hb_desc.sched 1, 2: two wave groups taking turns)
    "pp_t256x288": dict(bm=256, bn=288, bk=32, wm=4, wn=2, mfma=16, dbuf=3, lds_dma=1, order=1, sched=1),
    "pp_t256x256_b4": dict(bm=256, bn=256, bk=32, wm=4, wn=2, mfma=16, dbuf=3, lds_dma=1, order=1,
                           band=4, sched=1),
    "pp_t256x288_b4": dict(bm=256, bn=288, bk=32, wm=4, wn=2, mfma=16, dbuf=3, lds_dma=1, order=1,
                           band=4, sched=1),
    "pp_t128x128": dict(bm=128, bn=128, bk=32, wm=2, wn=4, mfma=16, dbuf=3, lds_dma=1, order=1, sched=1),
    "pp_t128x256_s3": dict(bm=128, bn=256, bk=32, wm=2, wn=4, mfma=16, dbuf=2, lds_dma=1, order=0,
                           sched=1),
    "pp_t256x192_x32_g2": dict(bm=256, bn=192, bk=32, wm=4, wn=2, mfma=32, dbuf=3, lds_dma=1, order=1,
                               sched=2),
    "pp_t256x160_k64": dict(bm=256, bn=160, bk=64, wm=4, wn=2, mfma=16, dbuf=2, lds_dma=1, order=1,
                            sched=1),
    "pp_t128x160_k64_b4": dict(bm=128, bn=160, bk=64, wm=4, wn=2, mfma=16, dbuf=3, lds_dma=1, order=1,
                               band=4, sched=1),
    # four waves, each reading its next K tile between its MFMAs (sched 3)
    "il_t256x256": dict(bm=256, bn=256, bk=32, wm=2, wn=2, mfma=16, dbuf=3, lds_dma=1, order=1, sched=3),
    "il_t256x192_s3": dict(bm=256, bn=192, bk=32, wm=2, wn=2, mfma=16, dbuf=2, lds_dma=1, order=1,
                           sched=3),
    # split K (hb_desc.ksplit): the parts' f32 sums added by a second kernel
    "ks2_t128x128": dict(bm=128, bn=128, bk=64, wm=2, wn=2, mfma=16, dbuf=1, lds_dma=1, order=1, ksplit=2),
    "ks4_t128x160_s4": dict(bm=128, bn=160, bk=64, wm=2, wn=2, mfma=16, dbuf=3, lds_dma=1, order=1,
                            ksplit=4),
    "ks2_t256x192_w8_b4": dict(bm=256, bn=192, bk=64, wm=4, wn=2, mfma=16, dbuf=1, lds_dma=1, order=1,
                               band=4, ksplit=2),
    "ks2_pp_t128x256": dict(bm=128, bn=256, bk=32, wm=2, wn=4, mfma=16, dbuf=3, lds_dma=1, order=1,
                            sched=1, ksplit=2),
    "ks4_pp_t256x160_k64": dict(bm=256, bn=160, bk=64, wm=4, wn=2, mfma=16, dbuf=2, lds_dma=1, order=1,
                                sched=1, ksplit=4),
    "ks2_il_t256x192": dict(bm=256, bn=192, bk=32, wm=2, wn=2, mfma=16, dbuf=2, lds_dma=1, order=1,
                            sched=3, ksplit=2),
    "ks4_t64x128_reg": dict(bm=64, bn=128, bk=64, wm=2, wn=2, mfma=16, dbuf=1, lds_dma=0, order=0,
                            ksplit=4),
}


def run_gemm(gpu, x, w, out=0, y0=None, m=None, **tile):
    m_rows, k = x.shape
    n = w.shape[0]
    m = m_rows if m is None else m
    st = gpu.alloc_with(np.array([0, 0, 0, m], np.uint32))
    W = gpu.alloc_with(w)
    X = gpu.alloc_with(x)
    esz = 4 if out == 1 else 2
    Y = gpu.alloc_with(y0) if y0 is not None else gpu.alloc(m_rows * n * esz)
    try:
        kern = gpu.pipeline(hb.gemm_mma(k, n, out, **tile))
        gpu.launch(kern, [hb.r(st), hb.r(W), hb.r(X), hb.r(Y), hb.r(st), hb.r(st)], m)
        gpu.sync()
        return gpu.download(Y, np.float32 if out == 1 else np.uint16, m_rows * n).reshape(m_rows, n)
    finally:
        for b in (st, W, X, Y):
            gpu.free(b)


def inputs(m, k, n, seed):
    return hb.normal_bf16(seed, 1.0, (m, k)), hb.normal_bf16(seed + 1, 0.02, (n, k))


@pytest.mark.parametrize("out", [0, 1, 2])
@pytest.mark.parametrize("tile", sorted(TILES))
def test_gemm_config1_all_out_modes(gpu, tile, out):
    """M=512, K=1024, N=3584, full check of every output."""
    m, k, n = 512, 1024, 3584
    x, w = inputs(m, k, n, 0x5EED0001)
    y0 = hb.normal_bf16(77, 1.0, (m, n)) if out == 2 else None
    got = run_gemm(gpu, x, w, out, y0, **TILES[tile])
    want = orc.gemm(x, w, out, y0)
    acc = orc.gemm(x, w, orc.OUT_F32) if out == 2 else None
    st = check_close(got, want, k, abs_products(x, w), "config1 %s out=%d" % (tile, out), acc=acc)
    if out != 1:
        assert st["exact"] > 0.99, st


@pytest.mark.parametrize("tile", sorted(TILES))
def test_gemm_partial_tiles(gpu, tile):
    """A row count that is a multiple of no tile (m - m/3 - 3, the reference's
    partial check, qwen.rs:2518): rows past m are neither wrong nor written."""
    m_alloc, k, n = 200, 512, 1024
    m = m_alloc - m_alloc // 3 - 3
    x, w = inputs(m_alloc, k, n, 11)
    sentinel = np.full((m_alloc, n), 0x7FC1, np.uint16)
    got = run_gemm(gpu, x, w, 0, sentinel, m=m, **TILES[tile])
    want = orc.gemm(x[:m], w)
    check_close(got[:m], want, k, abs_products(x[:m], w), "partial " + tile)
    assert np.all(got[m:] == 0x7FC1), "rows past m were written"


def test_gemm_state_rows_below_launch_rows(gpu):
    """state[3] < the launch's m: the kernel does only state[3] rows."""
    m, k, n = 256, 256, 512
    x, w = inputs(m, k, n, 12)
    st = gpu.alloc_with(np.array([0, 0, 0, 100], np.uint32))
    W, X = gpu.alloc_with(w), gpu.alloc_with(x)
    Y = gpu.alloc_with(np.zeros((m, n), np.uint16))
    kern = gpu.pipeline(hb.gemm_mma(k, n, 0, **TILES["t128x128_x16_d2"]))
    gpu.launch(kern, [hb.r(st), hb.r(W), hb.r(X), hb.r(Y), hb.r(st), hb.r(st)], m)
    got = gpu.download(Y, np.uint16, m * n).reshape(m, n)
    for b in (st, W, X, Y):
        gpu.free(b)
    assert np.all(got[100:] == 0)
    check_close(got[:100], orc.gemm(x[:100], w), k, abs_products(x[:100], w), "state rows")


@pytest.mark.parametrize("ksplit", [2, 3])
def test_gemm_split_k_state_rows_below_launch_rows(gpu, ksplit):
    """Split K with state[3] < the launch's m: the parts' slabs are the
    launch's rows apart, only state[3] rows are added and written; Out
    Residual adds to Y once."""
    m, k, n = 300, 768, 640
    x, w = inputs(m, k, n, 14)
    y0 = hb.normal_bf16(15, 1.0, (m, n))
    got = run_gemm(gpu, x, w, 2, y0, m=m, **dict(TILES["ks2_t128x128"], ksplit=ksplit))
    check_close(got, orc.gemm(x, w, 2, y0), k, abs_products(x, w), "split rows m",
                acc=orc.gemm(x, w, orc.OUT_F32))
    st = gpu.alloc_with(np.array([0, 0, 0, 100], np.uint32))
    W, X = gpu.alloc_with(w), gpu.alloc_with(x)
    Y = gpu.alloc_with(y0)
    kern = gpu.pipeline(hb.gemm_mma(k, n, 2, **dict(TILES["ks2_t128x128"], ksplit=ksplit)))
    assert gpu.kernel_name(kern).endswith("_ks%d" % ksplit)
    gpu.launch(kern, [hb.r(st), hb.r(W), hb.r(X), hb.r(Y), hb.r(st), hb.r(st)], m)
    got = gpu.download(Y, np.uint16, m * n).reshape(m, n)
    for b in (st, W, X, Y):
        gpu.free(b)
    assert np.array_equal(got[100:], y0[100:])
    check_close(got[:100], orc.gemm(x[:100], w, 2, y0[:100]), k, abs_products(x[:100], w),
                "split state rows", acc=orc.gemm(x[:100], w, orc.OUT_F32))


def test_gemm_split_k_is_deterministic_and_refused_where_unsplittable(gpu):
    """The parts are added in a fixed order: two launches give the same bits.
    K not a multiple of bk x parts, expert rows and the pipelined schedules
    are refused."""
    m, k, n = 512, 1024, 3584
    x, w = inputs(m, k, n, 16)
    a = run_gemm(gpu, x, w, 0, **TILES["ks4_t128x160_s4"])
    b = run_gemm(gpu, x, w, 0, **TILES["ks4_t128x160_s4"])
    assert np.array_equal(a, b)
    for bad in (dict(TILES["ks2_t128x128"], ksplit=3),
                dict(TILES["ks2_t128x128"], ksplit=17),
                dict(TILES["il_t256x192_s3"], ksplit=32)):
        with pytest.raises(hb.HerbertError):
            gpu.pipeline(hb.gemm_mma(k, n, 0, **bad))


@pytest.mark.parametrize("band", [1, 2, 3])
def test_gemm_band_order_covers_every_tile(gpu, band):
    """nax_tile_order's bands (prefill.rs:615-631) with a last band shorter
    than the others (5 row tiles): same output as the m_first walk, bit for
    bit, every row written."""
    m, k, n = 600, 256, 1000
    x, w = inputs(m, k, n, 13)
    base = dict(TILES["t128x128_x16_d2"], order=0)
    want = run_gemm(gpu, x, w, 0, **base)
    got = run_gemm(gpu, x, w, 0, np.full((m, n), 0x7FC1, np.uint16), band=band, **base)
    assert np.array_equal(got, want)


LAYER4B = [("qkv", 2560, 4608, 0), ("o", 4096, 2560, 2), ("gate_up", 2560, 18432, 0),
           ("down", 9216, 2560, 2)]


@pytest.mark.parametrize("m", [512, 2048])
@pytest.mark.parametrize("name,k,n,out", LAYER4B)
def test_gemm_config2_layer_shapes(gpu, name, k, n, out, m):
    """BASELINE config 2 (4B-class layer) at M=512 and 2048: 48 rows sampled
    across the block (first, last, spread) against the oracle."""
    tile = TILES["t128x128_x16_d2"] if m == 512 else TILES["t256x256_w8_d4"]
    x, w = inputs(m, k, n, 0x5EED0002)
    y0 = hb.normal_bf16(5, 1.0, (m, n)) if out == 2 else None
    got = run_gemm(gpu, x, w, out, y0, **tile)
    rows = np.unique(np.concatenate([[0, 1, m - 1], np.linspace(0, m - 1, 45).astype(int)]))
    want = orc.gemm(x[rows], w, out, None if y0 is None else y0[rows])
    acc = orc.gemm(x[rows], w, orc.OUT_F32) if out == 2 else None
    check_close(got[rows], want, k, abs_products(x, w, rows), "%s m=%d" % (name, m), acc=acc,
                min_exact=0.98)


@pytest.mark.parametrize("name,k,n", [("qkv", 5120, 7168), ("gate_up", 5120, 34816),
                                      ("down", 17408, 5120), ("lm_head", 5120, 151936)])
def test_gemm_config4_27b_shapes(gpu, name, k, n):
    """BASELINE config 4 (27B-class) at M=2048, 8 rows sampled."""
    m = 2048
    x, w = inputs(m, k, n, 0x5EED0004)
    got = run_gemm(gpu, x, w, 0, **TILES["t256x256_w8_d4"])
    rows = np.array([0, 1, 517, 1024, 1500, 2000, 2046, 2047])
    want = orc.gemm(x[rows], w)
    check_close(got[rows], want, k, abs_products(x, w, rows), name, min_exact=0.98)


def test_gemm_full_size_properties(gpu):
    """Size-independent invariants at M=2048 on the gate|up shape: scaling W
    by 2 scales Y exactly; permuting X's rows permutes Y's rows exactly;
    every tile family gives outputs within the contract of each other."""
    m, k, n = 2048, 2560, 18432
    x, w = inputs(m, k, n, 21)
    tile = TILES["t256x256_w8_d4"]
    y = run_gemm(gpu, x, w, 0, **tile)
    w2 = hb.f32_to_bf16(bf16_to_f32(w) * 2)
    y2 = run_gemm(gpu, x, w2, 0, **tile)
    assert np.array_equal(bf16_to_f32(y2), bf16_to_f32(y) * 2)
    perm = np.random.default_rng(0).permutation(m)
    yp = run_gemm(gpu, x[perm], w, 0, **tile)
    assert np.array_equal(yp, y[perm])
    other = run_gemm(gpu, x, w, 0, **TILES["t128x128_x16_d2"])
    scale = np.abs(bf16_to_f32(y)).max()
    assert np.abs(bf16_to_f32(other) - bf16_to_f32(y)).max() <= scale / 64


def test_gemm_identity_is_exact(gpu):
    m, k = 384, 512
    x = hb.normal_bf16(3, 1.0, (m, k))
    eye = hb.f32_to_bf16(np.eye(k, dtype=np.float32))
    for tile in ("t128x128_x16_d2", "t256x256_x32_d2"):
        assert np.array_equal(run_gemm(gpu, x, eye, 0, **TILES[tile]), x)


def test_gemm_bindings_checked(gpu):
    """A binding smaller than the descriptor and m need is refused before
    anything runs (HerbertError, no launch)."""
    k, n, m = 256, 512, 64
    kern = gpu.pipeline(hb.gemm_mma(k, n, 0, **TILES["t128x128_x16_d2"]))
    st = gpu.alloc_with(np.array([0, 0, 0, m], np.uint32))
    W = gpu.alloc(n * k * 2)
    X = gpu.alloc(m * k * 2 - 2)
    Y = gpu.alloc(m * n * 2)
    with pytest.raises(hb.HerbertError) as e:
        gpu.launch(kern, [hb.r(st), hb.r(W), hb.r(X), hb.r(Y), hb.r(st), hb.r(st)], m)
    assert "X" in str(e.value)
    for b in (st, W, X, Y):
        gpu.free(b)


def test_gemm_operands_past_2gib(gpu):
    """W of 2 GiB (K = N = 32768): the direct-to-LDS forms, whose buffer
    resources span 2^31 - 1 bytes, refuse it before anything runs; the
    register-staged form reads every row (rows near the end of W included)
    and matches the oracle on them (the other rows are zero)."""
    k = n = 32768
    m = 16
    rows = [5, n // 2, n - 3, n - 1]
    wr = hb.normal_bf16(0x5EED0031, 0.02, (len(rows), k))
    x = hb.normal_bf16(0x5EED0032, 1.0, (m, k))
    st = gpu.alloc_with(np.array([0, 0, 0, m], np.uint32))
    W = gpu.alloc(n * k * 2)
    X = gpu.alloc_with(x)
    Y = gpu.alloc(m * n * 2)
    try:
        gpu.zero(W)
        for i, r in enumerate(rows):
            gpu.upload(W, wr[i], offset=r * k * 2)
        bind = [hb.r(st), hb.r(W), hb.r(X), hb.r(Y), hb.r(st), hb.r(st)]
        dma = gpu.pipeline(hb.gemm_mma(k, n, 0, **TILES["t128x128_x16_d2"]))
        with pytest.raises(hb.HerbertError) as e:
            gpu.launch(dma, bind, m)
        assert "2 GiB" in str(e.value)
        reg = gpu.pipeline(hb.gemm_mma(k, n, 0, **TILES["t64x64_reg_s1"]))
        gpu.launch(reg, bind, m)
        gpu.sync()
        y = gpu.download(Y, np.uint16, m * n).reshape(m, n)
        check_close(y[:, rows], orc.gemm(x, wr), k, abs_products(x, wr), "2 GiB W rows")
        others = np.delete(np.arange(n), rows)[::97]
        assert not np.any(y[:, others] & 0x7fff), "zero rows of W gave nonzero outputs"
        # The selection skips the direct-to-LDS forms for this shape and
        # picks, checks and times the others.
        e = hb.Engine(gpu, "")
        try:
            kern = e.gemm(k, n, 0, hb.r(st), hb.r(W), hb.r(X), hb.r(Y), m)
            assert "_dma" not in gpu.kernel_name(kern)
            assert "skipped (operands past 2 GiB)" in e.log()
            gpu.zero(Y)
            gpu.launch(kern, bind, m)
            gpu.sync()
            y2 = gpu.download(Y, np.uint16, m * n).reshape(m, n)
            check_close(y2[:, rows], orc.gemm(x, wr), k, abs_products(x, wr), "2 GiB W rows, picked")
        finally:
            e.close()
    finally:
        for b in (st, W, X, Y):
            gpu.free(b)


def test_time_each_brackets_every_launch(gpu):
    """hb_time_each: the per-op means telescope to the whole run's time, and
    the larger GEMM takes longer than the smaller one."""
    k, m = 2048, 2048
    x = hb.normal_bf16(1, 1.0, (m, k))
    ws = [hb.normal_bf16(2, 0.02, (n, k)) for n in (512, 16384)]
    st = gpu.alloc_with(np.array([0, 0, 0, m], np.uint32))
    X = gpu.alloc_with(x)
    bufs, ops = [st, X], []
    for w in ws:
        W, Y = gpu.alloc_with(w), gpu.alloc(m * w.shape[0] * 2)
        bufs += [W, Y]
        kern = gpu.pipeline(hb.gemm_mma(k, w.shape[0], 0))
        ops.append(hb.Op(kern, [hb.r(st), hb.r(W), hb.r(X), hb.r(Y), hb.r(st), hb.r(st)], m))
    total, each = gpu.time_each(ops, 7)
    for b in bufs:
        gpu.free(b)
    assert abs(sum(each) * 7 - total) <= 1e-3 * total + 1e-6
    assert each[1] > 4 * each[0] > 0


def test_descriptor_refusals(gpu):
    """Fields a kernel cannot honour are refused at build, naming the rule:
    w_nt without direct-to-LDS staging, x_lds past 64 KiB of x (144 KiB with
    8 or 16 waves; or on the MFMA matvec), matvec waves other than 4, 8, 16
    (4 for XSrc::Norm), form 3 with an unroll other than 4, 8, 16, a combine of more than 16 slots."""
    with pytest.raises(hb.HerbertError, match="w_nt"):
        gpu.pipeline(hb.gemm_mma(256, 512, 0, bm=128, bn=128, bk=64, wm=2, wn=2, mfma=16, dbuf=1,
                                 lds_dma=0, w_nt=1))
    with pytest.raises(hb.HerbertError, match="x_lds"):
        gpu.pipeline(hb.matvec(9216, 2560, 0, mv_m=8, rows=2, form=2, x_lds=True))
    with pytest.raises(hb.HerbertError, match="x_lds"):
        gpu.pipeline(hb.matvec(2560, 4608, 0, mv_m=4, form=1, x_lds=True))
    with pytest.raises(hb.HerbertError, match="x_lds"):  # 144 KiB + 16 bytes
        gpu.pipeline(hb.matvec(9216 + 8, 2560, 0, mv_m=8, rows=1, form=2, x_lds=True, waves=16))
    with pytest.raises(hb.HerbertError, match="W through LDS"):
        gpu.pipeline(hb.matvec(2560, 4608, 0, mv_m=4, form=3, unroll=6))
    with pytest.raises(hb.HerbertError, match="W through LDS"):  # 4 waves x 16 x 2 tiles: 128 KiB
        gpu.pipeline(hb.matvec(2560, 4608, 0, mv_m=4, form=3, unroll=16, rows=32))
    with pytest.raises(hb.HerbertError, match="mv_waves"):
        gpu.pipeline(hb.matvec(2560, 4608, 0, mv_m=4, form=2, waves=12))
    with pytest.raises(hb.HerbertError, match="Norm"):
        gpu.pipeline(hb.matvec(2560, 4608, 0, mv_m=4, form=2, waves=8, xsrc=hb.XSrc.Norm))
    with pytest.raises(hb.HerbertError, match="top_k"):
        gpu.pipeline(hb.Desc(kind=hb.Kind.COMBINE, n=2048, top_k=17))
    assert gpu.kernel_kind(-1) == 0
    k = gpu.pipeline(hb.gemm_mma(256, 512, 0, bm=128, bn=128, bk=64, wm=2, wn=2, mfma=16, dbuf=1,
                                 lds_dma=1, w_nt=1))
    assert gpu.kernel_kind(k) == hb.Kind.GEMM and gpu.kernel_name(k).find("_wnt") > 0
