"""moeinfra_amd.profiling: the decode-step and per-kernel tables read from a rocprofv3
kernel-trace database (a hand-built SQLite file with the `kernels` columns it reads)."""
from __future__ import annotations

import sqlite3

import pytest

from moeinfra_amd import profiling


def _db(tmp_path, rows):
    p = tmp_path / "run_results.db"
    con = sqlite3.connect(p)
    con.execute("create table kernels (name text, grid_x int, start int, end int)")
    con.executemany("insert into kernels values (?, ?, ?, ?)", rows)
    con.commit()
    con.close()
    return str(p)


def test_step_table_by_hand(tmp_path):
    gu = "void moe::(anonymous namespace)::decode_gateup_kernel<8, true>(moe::ExpertTable)"
    fin = "moe::(anonymous namespace)::argmax_finish_kernel(int)"
    rows = [("prefill_thing()", 64, 0, 50), (fin, 256, 60, 70)]
    t = 1000
    for s in range(3):  # three steps: gate/up 10 us, 1 us gap, gate/up 12 us, 2 us gap, finish 3 us
        rows += [(gu, 131072, t, t + 10_000), (gu, 131072, t + 11_000, t + 23_000),
                 (fin, 256, t + 25_000, t + 28_000)]
        t += 100_000
    launches = profiling.read_launches(_db(tmp_path, rows))
    steps = profiling.split_steps(launches)
    assert len(steps) == 3 and [r[0] for r in steps[0]] == [gu, gu, fin]
    summary, table = profiling.step_table(profiling.split_steps(launches, last=2))
    assert summary["steps"] == 2 and summary["launches"] == 3
    assert summary["wall_us"] == pytest.approx(28.0) and summary["busy_us"] == pytest.approx(25.0)
    assert summary["idle_us"] == pytest.approx(3.0)
    top = table[0]
    assert top[:2] == ("decode_gateup_kernel<8, true>", 131072)
    assert top[2] == 2 and top[3] == pytest.approx(11.0) and top[4] == pytest.approx(22.0)
    assert top[5] == pytest.approx(88.0)
    kt = profiling.kernel_table(launches, "gateup")
    assert kt == [("decode_gateup_kernel<8, true>", 131072, 6, pytest.approx(11.0), pytest.approx(11.0),
                   pytest.approx(10.0))]


def test_no_complete_step_is_an_error(tmp_path):
    launches = profiling.read_launches(_db(tmp_path, [("k()", 1, 0, 5)]))
    with pytest.raises(ValueError, match="argmax_finish_kernel"):
        profiling.step_table(profiling.split_steps(launches))
