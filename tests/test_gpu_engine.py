"""The selection layer on the GPU (qwen.rs gemm :2200, check_candidates
:2497, pick_flagged :2547, mv_full :1311, expert_pipes :2326): candidates
checked against the first, a wrong one logged and never picked, an
unbuildable one skipped, the [autotune] lines in the reference's format,
and the kernels picked computing the contract (the whole MoE layer through
the picked kernels against the oracle)."""
import re

import numpy as np
import pytest

import herbert_hip as hb
import hb_oracle as orc
from parity import abs_products, check_close

pytestmark = pytest.mark.gpu


def test_gemm_autotune_checks_and_picks(gpu, capfd):
    m, k, n = 512, 1024, 3584
    x = hb.normal_bf16(0x5EED0001, 1.0, (m, k))
    w = hb.normal_bf16(0x5EED0002, 0.02, (n, k))
    st, W, X = gpu.alloc_with(np.array([0, 0, 0, m], np.uint32)), gpu.alloc_with(w), gpu.alloc_with(x)
    Y = gpu.alloc(m * n * 2)
    with hb.Engine(gpu, "") as e:
        # a kernel that builds and runs but computes another function: the
        # same GEMM with half the K (rows read at the wrong stride)
        wrong = hb.gemm_mma(k // 2, n, 0, bm=128, bn=128, bk=64, wm=2, wn=2, mfma=16, dbuf=1,
                            lds_dma=1, order=1)
        e.add_gemm_candidate("halfk", wrong)
        e.add_gemm_candidate("bk48", hb.gemm_mma(k, n, 0, bk=48))  # does not build
        kern = e.gemm(k, n, 0, hb.r(st), hb.r(W), hb.r(X), hb.r(Y), m)
        log = e.log()
        again = e.gemm(k, n, 0, hb.r(st), hb.r(W), hb.r(X), hb.r(Y), m)
        assert again == kern  # cached under the shape key
        e.log_summary()
        assert "[hip] " in e.log()
    print(log)
    assert re.search(r"\[autotune\] gemm 1024x3584 Bf16, 512 rows: bk48 not built", log)
    assert re.search(r"\[autotune\] gemm 1024x3584 Bf16, 512 rows: wrong against mma, never "
                     r"picked: halfk \(512 rows: max err [0-9.e+-]+ of [0-9.e+-]+\)$", log, re.M)
    line = [l for l in log.splitlines() if "-> " in l][0]
    assert line.startswith("[autotune] gemm 1024x3584 Bf16, 512 rows: mma ")
    assert "halfk* " in line
    picked = line.split("-> ")[1]
    assert picked != "halfk" and gpu.kernel_name(kern)
    # the pick computes the contract (Y is scratch while candidates are timed,
    # as in the reference, qwen.rs:1414)
    gpu.launch(kern, [hb.r(st), hb.r(W), hb.r(X), hb.r(Y), hb.r(st), hb.r(st)], m)
    got = gpu.download(Y, np.uint16, m * n).reshape(m, n)
    check_close(got, orc.gemm(x, w), k, abs_products(x, w), "picked " + picked)
    for b in (st, W, X, Y):
        gpu.free(b)


def test_gemm_explicit_forms(gpu):
    """gemm.mma / gemm.mform / gemm.tn name the kernel; nothing is timed."""
    m, k, n = 256, 512, 1024
    x = hb.normal_bf16(1, 1.0, (m, k))
    w = hb.normal_bf16(2, 0.02, (n, k))
    st, W, X = gpu.alloc_with(np.array([0, 0, 0, m], np.uint32)), gpu.alloc_with(w), gpu.alloc_with(x)
    Y = gpu.alloc(m * n * 2)
    want = orc.gemm(x, w)
    for tune in ["gemm.mma=0", "gemm.mma=2,gemm.tn=32", "gemm.mma=3"] + \
            ["gemm.mform=%d" % f for f in range(10)]:
        with hb.Engine(gpu, tune) as e:
            kern = e.gemm(k, n, 0, hb.r(st), hb.r(W), hb.r(X), hb.r(Y), m)
            assert e.log() == ""
        gpu.launch(kern, [hb.r(st), hb.r(W), hb.r(X), hb.r(Y), hb.r(st), hb.r(st)], m)
        got = gpu.download(Y, np.uint16, m * n).reshape(m, n)
        st_ = check_close(got, want, k, abs_products(x, w), tune)
        if tune == "gemm.mma=0":
            assert st_["exact"] == 1.0  # the VALU GEMM sums in the contract's order
    for b in (st, W, X, Y):
        gpu.free(b)


def test_matvec_autotune_cold(gpu):
    k, n, m = 2560, 4608, 4
    ws = [hb.normal_bf16(10 + i, 0.02, (n, k)) for i in range(3)]
    x = hb.normal_bf16(9, 1.0, (m, k))
    Wb = [gpu.alloc_with(w) for w in ws]
    X, Y = gpu.alloc_with(x), gpu.alloc(m * n * 2)
    with hb.Engine(gpu, "") as e:
        kern = e.mv(k, n, 0, m, [hb.r(b) for b in Wb], hb.r(X), hb.r(Y))
        log = e.log()
    assert re.search(r"\[autotune\] matvec 2560x4608 Bf16 m4: r1 .* -> ", log), log
    gpu.launch(kern, [hb.r(Wb[1]), hb.r(X), hb.r(Y)], m)
    got = gpu.download(Y, np.uint16, m * n).reshape(m, n)
    check_close(got, orc.gemm(x, ws[1]), k, abs_products(x, ws[1]), "mv pick")
    for b in Wb + [X, Y]:
        gpu.free(b)


@pytest.mark.parametrize("k,n,out", [(2560, 4608, 0), (9216, 2560, 2)])
def test_matvec_autotune_eight_rows(gpu, k, n, out):
    """At 8 rows the candidates include form 3 (MFMA, W through LDS; 16 and
    32 rows per wave) and the 16-wave workgroups staging x once per CU (down:
    144 KiB of x): they build, are timed under their names, and the pick
    computes the contract."""
    m = 8
    w = hb.normal_bf16(41, 0.02, (n, k))
    x = hb.normal_bf16(42, 1.0, (m, k))
    y0 = hb.normal_bf16(43, 1.0, (m, n)) if out == 2 else None
    Wb, X = gpu.alloc_with(w), gpu.alloc_with(x)
    Y = gpu.alloc_with(y0) if y0 is not None else gpu.alloc(m * n * 2)
    try:
        with hb.Engine(gpu, "") as e:
            kern = e.mv(k, n, out, m, [hb.r(Wb)], hb.r(X), hb.r(Y))
            log = e.log()
        assert "not built" not in log, log
        assert re.search(r"mfl_u4k4", log) and re.search(r"mfl_r32_u4k4", log), log
        assert re.search(r"xl_w16", log), log
        if y0 is not None:
            gpu.upload(Y, y0)
        gpu.launch(kern, [hb.r(Wb), hb.r(X), hb.r(Y)], m)
        got = gpu.download(Y, np.uint16, m * n).reshape(m, n)
        acc = orc.gemm(x, w, orc.OUT_F32) if out == 2 else None
        check_close(got, orc.gemm(x, w, out, y0), k, abs_products(x, w), "mv pick m=8 %dx%d" % (k, n), acc=acc)
    finally:
        for b in (Wb, X, Y):
            gpu.free(b)


def test_matvec_fused_autotune(gpu):
    """mv_full with its fusions (qwen.rs:1311-1336): the pick of a decode
    layer's gate|up with XSrc::Norm and Out::Swiglu, then the down with
    XSrc::Swiglu, each logged under its key and computing the contract."""
    k, nf, m, eps = 2560, 9216, 1, 1e-6
    xr = hb.normal_bf16(31, 2.0, (m, k))
    wn = hb.normal_bf16(32, 0.1, (k,))
    wgu = hb.normal_bf16(33, 0.02, (2 * nf, k))
    wd = hb.normal_bf16(34, 0.02, (k, nf))
    gu = hb.normal_bf16(35, 1.0, (m, 2 * nf))
    bufs = {nm: gpu.alloc_with(a) for nm, a in
            (("xr", xr), ("wn", wn), ("wgu", wgu), ("wd", wd), ("gu", gu))}
    H, Y = gpu.alloc(m * nf * 2), gpu.alloc(m * k * 2)
    try:
        with hb.Engine(gpu, "") as e:
            k1 = e.mv_fused(k, 2 * nf, hb.Out.Swiglu, m, [hb.r(bufs["wgu"])], hb.r(bufs["xr"]), hb.r(H),
                            xsrc=hb.XSrc.Norm, eps=eps, plus_one=True, norm_w=hb.r(bufs["wn"]))
            k2 = e.mv_fused(nf, k, hb.Out.Bf16, m, [hb.r(bufs["wd"])], hb.r(bufs["gu"]), hb.r(Y),
                            xsrc=hb.XSrc.Swiglu)
            log = e.log()
        assert re.search(r"\[autotune\] matvec 2560x18432 Norm\(358637bd,\+1\) Swiglu m1: r2 .* -> ", log), log
        assert re.search(r"\[autotune\] matvec 9216x2560 Swiglu Bf16 m1: r1 .* -> ", log), log
        assert "mfma" not in log.split("Norm(")[1].split("\n")[0]
        gpu.launch(k1, [hb.r(bufs["wgu"]), hb.r(bufs["xr"]), hb.r(H), hb.r(bufs["wn"])], m)
        h = gpu.download(H, np.uint16, m * nf).reshape(m, nf)
        xn = orc.rmsnorm_rows(xr, wn, eps, True, 0)
        ap = abs_products(xn, wgu)
        check_close(h, orc.gemm_swiglu(xn, wgu, nf), k, np.maximum(ap[:, :nf], ap[:, nf:]) * 2,
                    "fused gate_up pick", ulps=4.0)
        gpu.launch(k2, [hb.r(bufs["wd"]), hb.r(bufs["gu"]), hb.r(Y)], m)
        y = gpu.download(Y, np.uint16, m * k).reshape(m, k)
        xs = orc.swiglu(gu, nf)
        check_close(y, orc.gemm(xs, wd), nf, abs_products(xs, wd), "fused down pick")
    finally:
        for b in list(bufs.values()) + [H, Y]:
            gpu.free(b)


def test_moe_layer_through_picked_kernels(gpu):
    """expert_pipes picks sort, grouped GEMMs and tile rows; the whole routed
    layer through them equals the oracle's (route, sort, gather, GEMMs,
    SwiGLU, combine), the GEMM rounding within the contract."""
    E, K_, H, MI, rows = 64, 8, 512, 256, 256
    wgu = hb.normal_bf16(21, 0.02, (E * 2 * MI, H))
    wdn = hb.normal_bf16(22, 0.02, (E * H, MI))
    Wgu, Wdn = gpu.alloc_with(wgu), gpu.alloc_with(wdn)
    scores = hb.normal_bf16(23, 1.0, (rows, E))
    x = hb.normal_bf16(24, 1.0, (rows, H))
    with hb.Engine(gpu, "") as e:
        layer = hb.MoeLayer(gpu, e, E, K_, H, MI, rows, Wgu, Wdn, scores=scores, x=x)
        log = e.log()
    assert "[autotune] experts, 256 rows -> tiles of" in log
    assert re.search(r"\[autotune\] experts sort by 16 rows, 256 rows: scan .*atomic", log)
    gpu.upload(layer.buf["scores"], scores)
    gpu.upload(layer.buf["x"], x)
    gpu.time_ops(layer.ops(), 1)
    out = gpu.download(layer.buf["out"], np.uint16, rows * H).reshape(rows, H)
    route = orc.route(scores, K_)
    assert np.array_equal(gpu.download(layer.buf["route"], np.uint32, rows * 2 * K_).reshape(rows, -1), route)
    lst, tiles = orc.moe_sort(route, K_, E, layer.bm)
    gu = orc.experts_gemm(x, wgu, lst, tiles, H, 2 * MI, 1, K_, rows * K_)
    h = orc.swiglu(gu, MI)
    ey = orc.experts_gemm(h, wdn, lst, tiles, MI, H, 2, K_, rows * K_)
    want = orc.combine(ey, route, K_, H)
    from parity import bf16_to_f32
    err = np.abs(bf16_to_f32(out).astype(np.float64) - bf16_to_f32(want))
    scale = np.abs(bf16_to_f32(want)).max()
    assert err.max() <= scale / 64, (err.max(), scale)
    assert np.mean(out == want) > 0.9
    layer.free()
    gpu.free(Wgu)
    gpu.free(Wdn)


def test_rmsnorm_kernel_bit_exact(gpu):
    """The block's input norm: the oracle restates the kernel's summation
    order, so every output bit matches (rows of 2048 and of 2560)."""
    for d, p1 in ((2048, True), (2560, False)):
        x = hb.normal_bf16(51, 2.0, (37, d))
        w = hb.normal_bf16(52, 0.1, (d,))
        X, Wb, Y = gpu.alloc_with(x), gpu.alloc_with(w), gpu.alloc(37 * d * 2)
        k = gpu.pipeline(hb.rmsnorm(d, 1e-6, p1))
        gpu.launch(k, [hb.r(X), hb.r(Wb), hb.r(Y)], 37)
        got = gpu.download(Y, np.uint16, 37 * d).reshape(37, d)
        assert np.array_equal(got, orc.rmsnorm_rows(x, w, 1e-6, p1, 0)), d
        for b in (X, Wb, Y):
            gpu.free(b)


def test_moe_block_through_picked_kernels(gpu):
    """The whole sparse MLP of a qwen3_5_moe layer (qwen.rs:2691-2732) on the
    picked kernels, each stage against the oracle from the GPU's own input to
    it: the norm and the route bit for bit, the router GEMM and the shared
    expert within the contract, the routed experts within the reference's
    gate, and moe_out bit for bit."""
    E, K_, H, MI, SI, rows = 64, 8, 512, 256, 256, 192
    host = {"post_norm": hb.normal_bf16(61, 0.1, (H,)), "router": hb.normal_bf16(62, 0.05, (E, H)),
            "w_gate_up": hb.normal_bf16(63, 0.02, (E * 2 * MI, H)),
            "w_down": hb.normal_bf16(64, 0.02, (E * H, MI)),
            "s_gate_up": hb.normal_bf16(65, 0.02, (2 * SI, H)), "s_down": hb.normal_bf16(66, 0.02, (H, SI)),
            "shared_gate": hb.normal_bf16(67, 0.05, (H,))}
    w = {nm: gpu.alloc_with(a) for nm, a in host.items()}
    x0 = hb.normal_bf16(68, 1.0, (rows, H))
    with hb.Engine(gpu, "") as e:
        blk = hb.MoeBlock(gpu, e, E, K_, H, MI, SI, rows, w, x0)
    try:
        gpu.upload(blk.buf["x"], x0)
        gpu.time_ops(blk.ops(), 1)
        L = blk.layer.buf
        dl = lambda b, n, t=np.uint16: gpu.download(b, t, n)  # noqa: E731
        xn = dl(L["x"], rows * H).reshape(rows, H)
        assert np.array_equal(xn, orc.rmsnorm_rows(x0, host["post_norm"], 1e-6, True, 0))
        scores = dl(L["scores"], rows * E).reshape(rows, E)
        check_close(scores, orc.gemm(xn, host["router"]), H, abs_products(xn, host["router"]), "router")
        route = dl(L["route"], rows * 2 * K_, np.uint32).reshape(rows, -1)
        assert np.array_equal(route, orc.route(scores, K_))
        sh = dl(blk.buf["s_h"], rows * SI).reshape(rows, SI)
        ap = abs_products(xn, host["s_gate_up"])
        check_close(sh, orc.gemm_swiglu(xn, host["s_gate_up"], SI), H,
                    np.maximum(ap[:, :SI], ap[:, SI:]) * 2, "shared gate_up", ulps=4.0)
        sout = dl(blk.buf["sout"], rows * H).reshape(rows, H)
        check_close(sout, orc.gemm(sh, host["s_down"]), SI, abs_products(sh, host["s_down"]), "shared down")
        esum = dl(L["out"], rows * H).reshape(rows, H)
        lst, tiles = orc.moe_sort(route, K_, E, blk.layer.bm)
        gu = orc.experts_gemm(xn, host["w_gate_up"], lst, tiles, H, 2 * MI, 1, K_, rows * K_)
        ey = orc.experts_gemm(orc.swiglu(gu, MI), host["w_down"], lst, tiles, MI, H, 2, K_, rows * K_)
        want = orc.combine(ey, route, K_, H)
        from parity import bf16_to_f32
        err = np.abs(bf16_to_f32(esum).astype(np.float64) - bf16_to_f32(want))
        assert err.max() <= np.abs(bf16_to_f32(want)).max() / 64
        x1 = dl(blk.buf["x"], rows * H).reshape(rows, H)
        assert np.array_equal(x1, orc.moe_out(xn, host["shared_gate"], esum, sout, x0))
    finally:
        blk.free()
        for b in w.values():
            gpu.free(b)


def test_prefill_mlp_from_checkpoint_in_blocks(gpu, tmp_path):
    """The dense MLP half of a layer's prefill over a 300-row prompt cut into
    blocks of prefill.block=128 (blocks_of: 128, 128, 44 rows, on the picks of
    buckets 128 and 64), weights read from a two-shard checkpoint in the
    Hugging Face layout and stacked [gate | up]: every row within the contract
    of the oracle's norm -> GEMM -> SwiGLU -> GEMM (Residual) chain."""
    from st_writer import write_model
    h, inter, n = 512, 768, 300
    gate = hb.normal_bf16(71, 0.02, (inter, h))
    up = hb.normal_bf16(72, 0.02, (inter, h))
    down = hb.normal_bf16(73, 0.02, (h, inter))
    pn = hb.normal_bf16(74, 0.1, (h,))
    write_model(str(tmp_path / "m"), [
        {"model.language_model.layers.3.mlp.gate_proj.weight": ("BF16", gate),
         "model.language_model.layers.3.post_attention_layernorm.weight": ("BF16", pn)},
        {"model.language_model.layers.3.mlp.up_proj.weight": ("BF16", up),
         "model.language_model.layers.3.mlp.down_proj.weight": ("BF16", down)}])
    x0 = hb.normal_bf16(75, 1.0, (n, h))
    with hb.Checkpoint(str(tmp_path / "m")) as ck, hb.Engine(gpu, "prefill.block=128") as e:
        mlp = hb.PrefillMlp(gpu, e, ck, 3, h, inter)
        log = e.log()
    assert mlp.buckets == [64, 128], mlp.buckets
    assert "512x1536, 64 rows" in log and "512x1536, 128 rows" in log, log
    X = gpu.alloc_with(x0)
    states = mlp.states(n)
    try:
        gpu.time_ops(mlp.ops(X, n, states), 1)
        got = gpu.download(X, np.uint16, n * h).reshape(n, h)
        xn = orc.rmsnorm_rows(x0, pn, 1e-6, True, 0)
        w_gu = np.concatenate([gate, up])
        hh = orc.gemm_swiglu(xn, w_gu, inter)
        want = orc.gemm(hh, down, orc.OUT_RESIDUAL, x0)
        # Each stage's rounding (the SwiGLU's inputs within 2 ulp) joins the
        # down GEMM's: the bound of the h values' ulps through |W_down|.
        from parity import bf16_to_f32, bf16_ulp
        hf = np.abs(bf16_to_f32(hh).astype(np.float64))
        extra = 4 * bf16_ulp(hf) @ np.abs(bf16_to_f32(down).astype(np.float64)).T
        check_close(got, want, inter, abs_products(hh, down) + extra, "prefill mlp", ulps=3.0,
                    acc=orc.gemm(hh, down, orc.OUT_F32))
    finally:
        for b in states + [X]:
            gpu.free(b)
        mlp.free()


def test_picks_pinned_in_another_engine(gpu):
    """hb_engine_picks / hb_engine_pin: a second engine seeded with the
    first one's choices returns the same kernels without timing them, and a
    descriptor that does not build the recorded name is refused."""
    m, k, n = 256, 512, 1024
    x = hb.normal_bf16(31, 1.0, (m, k))
    w = hb.normal_bf16(32, 0.02, (n, k))
    st = gpu.alloc_with(np.array([0, 0, 0, m], np.uint32))
    W, X, Y = gpu.alloc_with(w), gpu.alloc_with(x), gpu.alloc(m * n * 2)
    xv, yv = gpu.alloc_with(hb.normal_bf16(33, 1.0, (4, k))), gpu.alloc(4 * n * 2)
    try:
        with hb.Engine(gpu, "") as a:
            ka = a.gemm(k, n, 0, hb.r(st), hb.r(W), hb.r(X), hb.r(Y), m)
            va = a.mv(k, n, 0, 4, [hb.r(W)], hb.r(xv), hb.r(yv))
            text = a.picks()
        lines = text.splitlines()
        assert any(ln.startswith("gemm\t%dx%d Bf16, %d rows\t" % (k, n, m)) for ln in lines), text
        assert any(ln.startswith("mv\t") for ln in lines), text
        with hb.Engine(gpu, "") as b:
            b.pin(text)
            kb = b.gemm(k, n, 0, hb.r(st), hb.r(W), hb.r(X), hb.r(Y), m)
            vb = b.mv(k, n, 0, 4, [hb.r(W)], hb.r(xv), hb.r(yv))
            assert "[autotune]" not in b.log()  # nothing timed
            assert gpu.kernel_name(kb) == gpu.kernel_name(ka)
            assert gpu.kernel_name(vb) == gpu.kernel_name(va)
            gl = [ln for ln in lines if ln.startswith("gemm\t")][0].split("\t")
            gl[2] = "gemm_mma_not_this_name"
            with pytest.raises(hb.HerbertError, match="not gemm_mma_not_this_name"):
                b.pin("\t".join(gl))
            with pytest.raises(hb.HerbertError, match="unknown kind"):
                b.pin("conv\tkey\tname\t1 2 3")
    finally:
        for buf in (st, W, X, Y, xv, yv):
            gpu.free(buf)
