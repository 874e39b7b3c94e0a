"""The matmul path of a layer read from a checkpoint in the Hugging Face
layout (model/qwen.rs:155-375; QwenEngine::load's fused layouts, qwen.rs:
776-835), run through the engine's picks against the oracle:
  - an attention layer's projections: input norm -> the stacked
    [q | k | v] GEMM, and o added to the residual stream (qwen.rs:2653-2668);
  - a qwen3_5_moe layer's sparse MLP from mlp.gate, mlp.experts.gate_up_proj
    / down_proj and the shared expert (qwen.rs:788-801, 2691-2732);
  - autotune_chunk's timed block size over the dense MLP half
    (qwen.rs:2962-3027), then a prompt cut by the chosen size."""
import re

import numpy as np
import pytest

import herbert_hip as hb
import hb_oracle as orc
from parity import abs_products, bf16_to_f32, check_close

pytestmark = pytest.mark.gpu

PFX = "model.language_model.layers.%d."


def test_attention_projections_from_checkpoint(gpu, tmp_path):
    from st_writer import write_model
    L, h, qw, kvw, ow, n = 2, 512, 1024, 256, 1024, 300
    wq, wk, wv = (hb.normal_bf16(81 + i, 0.02, (c, h)) for i, c in enumerate((qw, kvw, kvw)))
    wo = hb.normal_bf16(84, 0.02, (h, ow))
    nw = hb.normal_bf16(85, 0.1, (h,))
    p = PFX % L
    write_model(str(tmp_path / "m"), [
        {p + "self_attn.q_proj.weight": ("BF16", wq), p + "input_layernorm.weight": ("BF16", nw)},
        # k as F32 (bf16 values: read back exactly), v and o as BF16
        {p + "self_attn.k_proj.weight": ("F32", bf16_to_f32(wk).reshape(kvw, h)),
         p + "self_attn.v_proj.weight": ("BF16", wv), p + "self_attn.o_proj.weight": ("BF16", wo)}])
    x0 = hb.normal_bf16(86, 1.0, (n, h))
    ao = hb.normal_bf16(87, 1.0, (n, ow))
    with hb.Checkpoint(str(tmp_path / "m")) as ck, hb.Engine(gpu, "prefill.block=128") as e:
        proj = hb.PrefillAttnProj(gpu, e, ck, L, h, qw, kvw, ow)
        log = e.log()
    assert "512x1536 Bf16, 128 rows" in log and "1024x512 Residual, 64 rows" in log, log
    X, AO, QKV = gpu.alloc_with(x0), gpu.alloc_with(ao), gpu.alloc(n * (qw + 2 * kvw) * 2)
    states = proj.states(n)
    try:
        gpu.time_ops(proj.ops_qkv(X, QKV, n, states), 1)
        got = gpu.download(QKV, np.uint16, n * (qw + 2 * kvw)).reshape(n, -1)
        xn = orc.rmsnorm_rows(x0, nw, 1e-6, True, 0)
        w_qkv = np.concatenate([wq, wk, wv])
        check_close(got, orc.gemm(xn, w_qkv), h, abs_products(xn, w_qkv), "qkv from checkpoint")
        gpu.time_ops(proj.ops_o(AO, X, n, states), 1)
        x1 = gpu.download(X, np.uint16, n * h).reshape(n, h)
        check_close(x1, orc.gemm(ao, wo, orc.OUT_RESIDUAL, x0), ow, abs_products(ao, wo), "o from checkpoint",
                    acc=orc.gemm(ao, wo, orc.OUT_F32))
    finally:
        for b in states + [X, AO, QKV]:
            gpu.free(b)
        proj.free()


def test_moe_block_from_checkpoint(gpu, tmp_path):
    from st_writer import write_model
    L, E, K_, H, MI, SI, rows = 1, 64, 4, 512, 256, 256, 192
    host = {"post_norm": hb.normal_bf16(91, 0.1, (H,)), "router": hb.normal_bf16(92, 0.05, (E, H)),
            "w_gate_up": hb.normal_bf16(93, 0.02, (E * 2 * MI, H)),
            "w_down": hb.normal_bf16(94, 0.02, (E * H, MI)),
            "s_gate": hb.normal_bf16(95, 0.02, (SI, H)), "s_up": hb.normal_bf16(96, 0.02, (SI, H)),
            "s_down": hb.normal_bf16(97, 0.02, (H, SI)), "shared_gate": hb.normal_bf16(98, 0.05, (H,))}
    p = PFX % L
    vocab = 3001  # the probe ids (1000 + 7919 i mod 50000) wrap around it
    emb = hb.normal_bf16(90, 1.0, (vocab, H))
    write_model(str(tmp_path / "m"), [
        {"model.language_model.embed_tokens.weight": ("BF16", emb),
         p + "post_attention_layernorm.weight": ("BF16", host["post_norm"]),
         p + "mlp.gate.weight": ("BF16", host["router"]),
         p + "mlp.experts.gate_up_proj": ("BF16", host["w_gate_up"].reshape(E, 2 * MI, H))},
        {p + "mlp.experts.down_proj": ("BF16", host["w_down"].reshape(E, H, MI)),
         p + "mlp.shared_expert.gate_proj.weight": ("BF16", host["s_gate"]),
         p + "mlp.shared_expert.up_proj.weight": ("BF16", host["s_up"]),
         p + "mlp.shared_expert.down_proj.weight": ("BF16", host["s_down"]),
         p + "mlp.shared_expert_gate.weight": ("BF16", host["shared_gate"].reshape(1, H))}])
    with hb.Checkpoint(str(tmp_path / "m")) as ck:
        w = hb.moe_weights_from_checkpoint(gpu, ck, L, E, H, MI, SI)
        # route_probe: the experts timed on the route of the probe ids' rows
        x0 = hb.route_probe_rows(ck, rows, H)
    assert np.array_equal(x0, emb[(1000 + (7919 * np.arange(rows)) % 50000) % vocab])
    with hb.Engine(gpu, "") as e:
        blk = hb.MoeBlock(gpu, e, E, K_, H, MI, SI, rows, w, x0)
    try:
        gpu.upload(blk.buf["x"], x0)
        gpu.time_ops(blk.ops(), 1)
        Lb = blk.layer.buf
        dl = lambda b, n, t=np.uint16: gpu.download(b, t, n)  # noqa: E731
        xn = dl(Lb["x"], rows * H).reshape(rows, H)
        assert np.array_equal(xn, orc.rmsnorm_rows(x0, host["post_norm"], 1e-6, True, 0))
        scores = dl(Lb["scores"], rows * E).reshape(rows, E)
        check_close(scores, orc.gemm(xn, host["router"]), H, abs_products(xn, host["router"]), "router")
        route = dl(Lb["route"], rows * 2 * K_, np.uint32).reshape(rows, -1)
        assert np.array_equal(route, orc.route(scores, K_))
        # The experts from the GPU's own route: grouped GEMMs within the
        # reference's gate, the sum exactly the combine of the GPU's rows.
        esum = dl(Lb["out"], rows * H).reshape(rows, H)
        lst, tiles = orc.moe_sort(route, K_, E, blk.layer.bm)
        gu = orc.experts_gemm(xn, host["w_gate_up"], lst, tiles, H, 2 * MI, 1, K_, rows * K_)
        ey = orc.experts_gemm(orc.swiglu(gu, MI), host["w_down"], lst, tiles, MI, H, 2, K_, rows * K_)
        want = orc.combine(ey, route, K_, H)
        err = np.abs(bf16_to_f32(esum).astype(np.float64) - bf16_to_f32(want))
        assert err.max() <= np.abs(bf16_to_f32(want)).max() / 64
        assert np.mean(esum == want) > 0.8
        sout = dl(blk.buf["sout"], rows * H).reshape(rows, H)
        sh = dl(blk.buf["s_h"], rows * SI).reshape(rows, SI)
        check_close(sout, orc.gemm(sh, host["s_down"]), SI, abs_products(sh, host["s_down"]), "shared down")
        x1 = dl(blk.buf["x"], rows * H).reshape(rows, H)
        assert np.array_equal(x1, orc.moe_out(xn, host["shared_gate"], esum, sout, x0))
    finally:
        blk.free()
        for b in w.values():
            gpu.free(b)


def test_autotune_chunk_then_prompt(gpu, tmp_path):
    from st_writer import write_model
    L, h, inter = 0, 512, 768
    gate, up = hb.normal_bf16(101, 0.02, (inter, h)), hb.normal_bf16(102, 0.02, (inter, h))
    down, pn = hb.normal_bf16(103, 0.02, (h, inter)), hb.normal_bf16(104, 0.1, (h,))
    p = PFX % L
    write_model(str(tmp_path / "m"), [{p + "mlp.gate_proj.weight": ("BF16", gate),
                                       p + "mlp.up_proj.weight": ("BF16", up),
                                       p + "mlp.down_proj.weight": ("BF16", down),
                                       p + "post_attention_layernorm.weight": ("BF16", pn)}])
    with hb.Checkpoint(str(tmp_path / "m")) as ck, hb.Engine(gpu, "prefill.block=2048") as e:
        mlp = hb.PrefillMlp(gpu, e, ck, L, h, inter)
        chunk = mlp.autotune_chunk(e)
        log = e.log()
    m_ = re.search(r"\[autotune\] blocks over 2048 rows, every layer, heated [0-9.]+ s, median of 3 rounds: "
                   r"1024 [0-9.]+ ms, 2048 [0-9.]+ ms -> (\d+)", log)
    assert m_ and int(m_.group(1)) == chunk and chunk in (1024, 2048), log[-600:]
    n = 2500
    x0 = hb.normal_bf16(105, 1.0, (n, h))
    X = gpu.alloc_with(x0)
    states = mlp.states(n)
    try:
        gpu.time_ops(mlp.ops(X, n, states), 1)
        got = gpu.download(X, np.uint16, n * h).reshape(n, h)
        xn = orc.rmsnorm_rows(x0, pn, 1e-6, True, 0)
        hh = orc.gemm_swiglu(xn, np.concatenate([gate, up]), inter)
        want = orc.gemm(hh, down, orc.OUT_RESIDUAL, x0)
        from parity import bf16_ulp
        hf = np.abs(bf16_to_f32(hh).astype(np.float64))
        extra = 4 * bf16_ulp(hf) @ np.abs(bf16_to_f32(down).astype(np.float64)).T
        check_close(got, want, inter, abs_products(hh, down) + extra, "prefill mlp after autotune_chunk",
                    ulps=3.0, acc=orc.gemm(hh, down, orc.OUT_F32))
    finally:
        for b in states + [X]:
            gpu.free(b)
        mlp.free()
