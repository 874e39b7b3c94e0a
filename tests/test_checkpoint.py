"""The checkpoint reader (model/qwen.rs:155-375: Checkpoint::load, normalize
:102-153, bf16_at :92-99, read_bf16_into :338-361) and blocks_of
(qwen.rs:3017-3027), on the CPU: synthetic shards in the Hugging Face
layout written by tests/st_writer.py."""
import math

import numpy as np
import pytest

import herbert_hip as hb
from st_writer import write_model, write_safetensors


def bf16_bits(a):
    b = np.ascontiguousarray(a, np.float32).view(np.uint32)
    return ((b + np.uint32(0x7FFF) + ((b >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)


@pytest.fixture
def model(tmp_path):
    rng = np.random.default_rng(5)
    h, inter = 64, 96
    t = {
        "gate": rng.normal(0, 1, (inter, h)).astype(np.float32),
        "up": rng.normal(0, 1, (inter, h)).astype(np.float32),
        "down": rng.normal(0, 1, (h, inter)).astype(np.float32),
        "norm": rng.normal(0, 1, (h,)).astype(np.float32),
        "q": rng.normal(0, 1, (32, h)).astype(np.float32),
    }
    shards = [
        {"model.language_model.layers.0.mlp.gate_proj.weight": ("BF16", bf16_bits(t["gate"])),
         "model.language_model.layers.0.mlp.up_proj.weight": ("F32", t["up"]),
         "model.language_model.layers.0.post_attention_layernorm.weight": ("F16", t["norm"].astype(np.float16)),
         "model.visual.blocks.0.attn.qkv.weight": ("BF16", np.zeros((4, 4), np.uint16))},
        {"model.language_model.layers.0.mlp.down_proj.weight": ("BF16", bf16_bits(t["down"])),
         "model.layers.1.self_attn.q_proj.weight": ("BF16", bf16_bits(t["q"])),
         "model.language_model.layers.0.mlp.gate_proj.weight": ("BF16", np.zeros((inter, h), np.uint16)),
         "lm_head.weight": ("BF16", np.ones((8, h), np.uint16)),
         "model.language_model.layers.0.linear_attn.A_log": ("F32", np.zeros(4, np.float32))},
    ]
    write_model(str(tmp_path / "m"), shards)
    return str(tmp_path / "m"), t, h, inter


def test_names_normalised_and_skipped(model):
    d, t, h, inter = model
    with hb.Checkpoint(d) as ck:
        assert ck.elements("0.mlp.gate_proj.weight") == inter * h
        assert ck.elements("1.self_attn.q_proj.weight") == 32 * h  # "model.layers." prefix
        assert ck.elements("lm_head") == 8 * h
        assert not ck.has("0.linear_attn.A_log")  # not a field of the matmul path
        assert "model.visual.* x1" in ck.skipped()


def test_read_rounds_once_and_stacks_parts(model):
    """[gate | up] read as one: gate's bf16 bits as stored (the first shard
    wins a name present in two), up's f32 rounded once (RNE), the f16 norm
    widened exactly then rounded."""
    d, t, h, inter = model
    with hb.Checkpoint(d) as ck:
        gu = ck.read([("0.mlp.gate_proj.weight", inter * h), ("0.mlp.up_proj.weight", inter * h)])
        assert np.array_equal(gu[:inter * h], bf16_bits(t["gate"]).ravel())
        assert np.array_equal(gu[inter * h:], bf16_bits(t["up"]).ravel())
        n = ck.read([("0.post_attention_layernorm.weight", h)])
        assert np.array_equal(n, bf16_bits(t["norm"].astype(np.float16).astype(np.float32)))


def test_errors_name_the_tensor(model, tmp_path):
    d, t, h, inter = model
    with hb.Checkpoint(d) as ck:
        with pytest.raises(hb.HerbertError, match="missing tensor 0.mlp.nope"):
            ck.read([("0.mlp.nope", 4)])
        with pytest.raises(hb.HerbertError, match="elements"):
            ck.read([("0.mlp.down_proj.weight", 5)])
    bad = tmp_path / "bad"
    bad.mkdir()
    write_safetensors(str(bad / "model.safetensors"),
                      {"model.layers.0.mlp.down_proj.weight": ("I8", np.zeros(4, np.int8))})
    with pytest.raises(hb.HerbertError, match="unsupported dtype I8"):
        hb.Checkpoint(str(bad))
    trunc = tmp_path / "trunc"
    trunc.mkdir()
    with open(trunc / "model.safetensors", "wb") as f:
        f.write((1000).to_bytes(8, "little") + b"{}")
    with pytest.raises(hb.HerbertError, match="header runs past"):
        hb.Checkpoint(str(trunc))


def blocks_of_restated(n, chunk):
    """qwen.rs:3017-3027 as written there."""
    chunk = max(chunk, 1)
    k = -(-n // chunk)
    size = min(-(-(-(-n // k)) // 64) * 64, chunk)
    return [(at, min(size, n - at)) for at in range(0, n, size)]


@pytest.mark.parametrize("chunk", [64, 1000, 1024, 2048, 4096])
def test_blocks_of(chunk):
    for n in list(range(1, 300)) + [1023, 1024, 1025, 2047, 2048, 2049, 5000, 8192, 9000]:
        got = hb.blocks_of(n, chunk)
        assert got == blocks_of_restated(n, chunk), (n, chunk)
        assert sum(r for _, r in got) == n and all(r <= chunk for _, r in got)
        assert len(got) == math.ceil(n / chunk)


def test_probe_ids_are_the_reference_formula():
    """probe_ids (qwen.rs:2952-2955): 1000 + (i * 7919) % 50000."""
    ids = hb.probe_ids(10)
    assert ids == [1000, 8919, 16838, 24757, 32676, 40595, 48514, 6433, 14352, 22271]
    assert all(1000 <= v < 51000 for v in hb.probe_ids(4096))


def test_route_probe_rows_are_the_probe_ids_embeddings(tmp_path):
    """route_probe's rows: the embedding rows of the probe ids, wrapped
    around the vocabulary; refused without an embedding of that width."""
    vocab, h = 97, 16
    emb = (np.arange(vocab * h, dtype=np.uint32) % 60000).astype(np.uint16).reshape(vocab, h)
    write_model(str(tmp_path / "m"), [{"model.embed_tokens.weight": ("BF16", emb)}])
    with hb.Checkpoint(str(tmp_path / "m")) as ck:
        rows = hb.route_probe_rows(ck, 40, h)
        assert np.array_equal(rows, emb[np.array(hb.probe_ids(40)) % vocab])
        with pytest.raises(hb.HerbertError, match="embed_tokens"):
            hb.route_probe_rows(ck, 4, 24)
