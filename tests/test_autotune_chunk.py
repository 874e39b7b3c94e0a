"""autotune_chunk's policy (src/metal/qwen.rs:2962-3010) in the library
(hb_engine_autotune_chunk), driven on the CPU through a host-only engine
with a host whose block_in reports modelled GPU times: the candidates, the
heat over the first candidate's one block, the reset before every run, the
three rounds in alternating order, the median, the first of equal times,
and the reference's log line."""
import re

import pytest

import herbert_hip as hb


def cost(rows):
    """Modelled GPU seconds of one block: a fixed part and a part growing
    faster than the rows, so 2048-row blocks win a 4096-row prompt."""
    return 1e-4 + (rows / 1024.0) ** 2 * 2e-5


def run(tune, block_in_cost=cost, fail_at=None):
    calls = []

    def block_in(start, rows):
        calls.append(("block", start, rows))
        if fail_at is not None and len(calls) == fail_at:
            raise RuntimeError("block_in failed")
        return block_in_cost(rows)

    def reset():
        calls.append(("reset",))

    with hb.Engine(None, tune) as e:
        chunk = hb.autotune_chunk(e, block_in, reset)
        return chunk, calls, e.log(), e.autotune_seconds()


def expected_calls(block, cands, heat_s, block_cost=cost):
    out, warmed = [], 0.0
    while True:
        out += [("reset",), ("block", 0, cands[0])]
        warmed += block_cost(cands[0])
        if warmed >= heat_s:
            break
    for rnd in range(3):
        for c in (cands if rnd % 2 == 0 else cands[::-1]):
            out.append(("reset",))
            out += [("block", s, r) for s, r in hb.blocks_of(block, c)]
    out.append(("reset",))
    return out


def test_policy_protocol_and_choice():
    chunk, calls, log, secs = run("prefill.block=4096,auto.heat=1")
    assert chunk == 2048
    assert calls == expected_calls(4096, [1024, 2048, 4096], 1e-3)
    line = [ln for ln in log.splitlines() if ln.startswith("[autotune] blocks")]
    assert len(line) == 1
    assert re.fullmatch(r"\[autotune\] blocks over 4096 rows, every layer, heated 0\.0 s, median of 3 rounds: "
                        r"1024 0\.480 ms, 2048 0\.360 ms, 4096 0\.420 ms -> 2048", line[0]), line[0]
    assert secs >= 0.0


def test_candidates_below_block_and_odd_block():
    # prefill.block 3000: 1024 and 2048 below it, then 3000 itself; blocks_of
    # cuts 3000 by 2048 into two blocks of 1536 rows.
    chunk, calls, _, _ = run("prefill.block=3000,auto.heat=0")
    blocks = [c[2] for c in calls if c[0] == "block"]
    assert blocks[:1] == [1024]  # the heat: one block of cands[0]
    assert calls == expected_calls(3000, [1024, 2048, 3000], 0.0)
    assert [r for _, r in hb.blocks_of(3000, 2048)] == [1536, 1464]
    assert chunk in (1024, 2048, 3000)


def test_median_not_mean_and_first_on_ties():
    # every block the same time: the candidate with the fewest blocks wins ...
    chunk, _, _, _ = run("prefill.block=4096,auto.heat=0", lambda rows: 1e-4)
    assert chunk == 4096
    # ... and equal totals keep the first candidate (min_by's first minimum)
    chunk, _, _, _ = run("prefill.block=2048,auto.heat=0", lambda rows: rows * 1e-7)
    assert chunk == 1024


def test_block_at_most_1024_is_not_timed():
    chunk, calls, log, _ = run("prefill.block=1024")
    assert chunk == 1024 and calls == [] and "[autotune] blocks" not in log


def test_host_failure_is_reported():
    with pytest.raises(RuntimeError, match="block_in failed"):
        run("prefill.block=4096,auto.heat=0", fail_at=5)


def test_host_only_engine_refuses_selection():
    with hb.Engine(None, "") as e:
        with pytest.raises(hb.HerbertError, match="without a context"):
            e.log_summary()
