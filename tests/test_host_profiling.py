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


def test_copy_table_by_hand(tmp_path):
    """Two decode steps of 100 us; per step two 2 MB host-to-device copies, one entirely
    under a kernel and one half under it, plus a small copy that is ignored."""
    fin = "moe::(anonymous namespace)::argmax_finish_kernel(int)"
    k = "void moe::(anonymous namespace)::decode_gateup_kernel<8, false>(moe::ExpertTable)"
    p = tmp_path / "run_results.db"
    con = sqlite3.connect(p)
    con.execute("create table kernels (name text, grid_x int, start int, end int)")
    con.execute("create table memory_copies (start int, end int, size int, src_agent_type text, "
                "dst_agent_type text)")
    kern = [(fin, 1, 0, 1_000)]
    cps = []
    for s in range(2):
        t = 1_000 + 100_000 * s
        kern += [(k, 256, t + 10_000, t + 50_000), (fin, 1, t + 95_000, t + 100_000)]
        cps += [(t + 20_000, t + 40_000, 2_000_000, "CPU", "GPU"),   # under the kernel
                (t + 40_000, t + 60_000, 2_000_000, "CPU", "GPU"),   # half under it
                (t + 70_000, t + 71_000, 4096, "CPU", "GPU")]        # below the size floor
    con.executemany("insert into kernels values (?, ?, ?, ?)", kern)
    con.executemany("insert into memory_copies values (?, ?, ?, ?, ?)", cps)
    con.commit()
    con.close()
    launches = profiling.read_launches(str(p))
    copies = profiling.read_h2d_copies(str(p))
    assert len(copies) == 4
    t = profiling.copy_table(launches, copies)
    assert t["steps"] == 2 and t["copies_per_step"] == 2
    # window: first kernel of step 1 (t=11 us) to the end of step 2's finish (201 us)
    wall = 201_000 - 11_000
    assert t["link_busy_frac"] == pytest.approx(80_000 / wall)
    assert t["gbps_while_busy"] == pytest.approx(8e6 / 80_000)
    assert t["copy_time_with_kernel_frac"] == pytest.approx(60_000 / 80_000)
    assert t["kernel_time_with_copy_frac"] == pytest.approx(60_000 / 90_000)


def test_counter_table_by_hand(tmp_path):
    p = tmp_path / "pmc_results.db"
    con = sqlite3.connect(p)
    con.execute("create table counters_collection (kernel_name text, counter_name text, value real)")
    k = "void moe::(anonymous namespace)::mid_down_kernel(moe::ExpertTable)"
    con.executemany("insert into counters_collection values (?, ?, ?)",
                    [(k, "FETCH_SIZE", v) for v in (10.0, 30.0, 20.0)] + [("other()", "FETCH_SIZE", 5.0)])
    con.commit()
    con.close()
    assert profiling.counter_table(str(p), "mid_down") == [("mid_down_kernel", "FETCH_SIZE", 3, 20.0, 20.0)]
