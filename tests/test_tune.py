"""--tune parsing and validation of the selection layer against
src/metal/qwen.rs:296-398 (Tune::apply, Tune::summary): the reference's
key names, side effects and error messages, without a device."""
import pytest

import herbert_hip as hb


def summary_dict(s):
    out = {}
    for part in s.replace(", ", ",").split(" "):
        k, v = part.split("=", 1)
        out[k] = v
    return out


def test_defaults():
    d = summary_dict(hb.tune_check(""))
    assert d["prefill.block"] == "2048" and d["gemm.auto"] == "1" and d["gemm.mma"] == "1"
    assert d["moe.tile"] == "16" and d["mv.auto"] == "1" and d["mv.cold"] == "1"
    assert d["pf.fswi"] == "2" and d["mv.persists"] == "[]" and d["gemm.mfirst"] == "1"
    assert list(d)[0] == "prefill.block" and list(d)[-1] == "dn.tscale"


def test_side_effects():
    d = summary_dict(hb.tune_check("gemm.mma=2,gemm.tn=32"))
    assert d["gemm.auto"] == "0"  # gemm.mma given: nothing timed
    d = summary_dict(hb.tune_check("mv.split=4"))
    assert d["mv.auto"] == "0" and d["mv.split"] == "4"
    d = summary_dict(hb.tune_check("prefill.block=0"))
    assert d["prefill.block"] == "1"
    d = summary_dict(hb.tune_check("dec.sdpa=100"))
    assert d["dec.sdpa"] == "64"
    d = summary_dict(hb.tune_check("mv.persists=256/512"))
    assert d["mv.persists"] == "[256,512]" or d["mv.persists"] == "[256, 512]"
    d = summary_dict(hb.tune_check("sdpa.prefill=1"))
    assert d["sdpa.auto"] == "0"


@pytest.mark.parametrize("tune,msg", [
    ("gemm.mma", "--tune gemm.mma: key=value"),
    ("gemm.mma=x", "--tune gemm.mma=x: invalid digit found in string"),
    ("gemm.mma=", "--tune gemm.mma=: cannot parse integer from empty string"),
    ("gemm.mma=4294967296", "--tune gemm.mma=4294967296: number too large to fit in target type"),
    ("no.such=1", "--tune no.such: unknown"),
    ("gemm.tn=48", "--tune gemm.mma=1 gemm.tn=48 gemm.mform=0: gemm.mma 0..2, gemm.tn 16, 32 or 64, gemm.mform 0..9"),
    ("gemm.mma=3,gemm.tn=128", None),
    ("gemm.mma=2,gemm.tn=128", "--tune gemm.mma=2 gemm.tn=128 gemm.mform=0: gemm.mma 0..2, gemm.tn 16, 32 or 64, gemm.mform 0..9"),
    ("gemm.mform=10", "--tune gemm.mma=1 gemm.tn=64 gemm.mform=10: gemm.mma 0..2, gemm.tn 16, 32 or 64, gemm.mform 0..9"),
    ("moe.tile=48", "--tune moe.tile=48: 16, 32 or 64"),
    ("q4.fuse=1,gemm.mma=2", "--tune q4.fuse=1: 0, or 1 with gemm.mma=1"),
    ("q4.fuse=2", "--tune q4.fuse=2: 0, or 1 with gemm.mma=1"),
    ("gemm.simt=3", "--tune: rec.chunk 0..4, sdpa.prefill 0..7, gemm.simt 1..2"),
])
def test_errors(tune, msg):
    if msg is None:
        hb.tune_check(tune)
        return
    with pytest.raises(hb.HerbertError) as e:
        hb.tune_check(tune)
    assert e.value.msg.startswith(msg), e.value.msg
