"""Kernel tables from a rocprofv3 kernel-trace database (the SQLite file that
``rocprofv3 --kernel-trace -d DIR -o NAME -- python3 bench.py ...`` writes as
``DIR/.../NAME_results.db``).

``python -m moeinfra_amd.profiling steps DB [N]`` prints the per-step kernel table of the
last N decode steps of an end-to-end run (a step ends with ``argmax_finish_kernel``, the
last launch of the captured decode step): wall time from the step's first kernel start to
its last kernel end, busy time (sum of kernel durations), and per kernel and grid the
launches, average duration and share of the busy time.

``python -m moeinfra_amd.profiling kernels DB [SUBSTR]`` prints count / average / median /
min duration per kernel and grid over the whole trace (optionally only names containing
SUBSTR).

``python -m moeinfra_amd.profiling copies DB [N] [MIN_MIB]`` (a run traced with
``--kernel-trace --memory-copy-trace``, e.g. ``bench.py --offload``) prints, over the last N
decode steps, the host-to-device copies of at least MIN_MIB MiB (default 1): count, bytes,
the time the host link is busy with at least one of them (union of their intervals) as a
share of the steps' wall time, the rate while busy, and how much of that copy time a
kernel runs alongside (copy/compute overlap).

``python -m moeinfra_amd.profiling counters DB [SUBSTR]`` (a ``rocprofv3 --pmc ...`` run)
prints the median of each counter per kernel (dispatches counted), e.g. FETCH_SIZE and
WRITE_SIZE in KiB per dispatch.

Only the ``kernels`` view (columns name, grid_x, start, end in nanoseconds) and, for
``copies``, the ``memory_copies`` view (start, end, size, src_agent_type, dst_agent_type)
and, for ``counters``, the ``counters_collection`` view (kernel_name, counter_name, value)
of the database are read.
"""
from __future__ import annotations

import sqlite3
import statistics as st
import sys
from typing import Dict, List, Sequence, Tuple

Launch = Tuple[str, int, int, int]  # (name, grid_x, start ns, end ns)

STEP_END_KERNEL = "argmax_finish_kernel"


def short_name(name: str) -> str:
    """Kernel name without the namespace, `void ` and the argument list."""
    return name.replace("moe::(anonymous namespace)::", "").replace("void ", "").split("(")[0]


def read_launches(db_path: str) -> List[Launch]:
    con = sqlite3.connect(db_path)
    try:
        rows = con.execute("select name, grid_x, start, end from kernels order by start").fetchall()
    finally:
        con.close()
    return [(str(n), int(g), int(a), int(b)) for n, g, a, b in rows]


def split_steps(launches: Sequence[Launch], last: int | None = None) -> List[List[Launch]]:
    """Launches grouped into decode steps: each step runs from the launch after one
    argmax_finish_kernel to the next one, inclusive; the last `last` steps."""
    ends = [i for i, r in enumerate(launches) if STEP_END_KERNEL in r[0]]
    steps = [list(launches[a + 1:b + 1]) for a, b in zip(ends[:-1], ends[1:])]
    return steps[-last:] if last else steps


def step_table(steps: Sequence[Sequence[Launch]]) -> Tuple[Dict[str, float], List[Tuple[str, int, float, float, float, float]]]:
    """(summary, rows): summary has wall/busy/idle microseconds per step and launches per
    step; rows are (kernel, grid, launches per step, avg us, us per step, % of busy),
    the heaviest first."""
    if not steps:
        raise ValueError(f"no complete decode step (no two {STEP_END_KERNEL} launches) in the trace")
    walls = [s[-1][3] - s[0][2] for s in steps]
    busy = [sum(b - a for _, _, a, b in s) for s in steps]
    summary = {
        "steps": float(len(steps)),
        "wall_us": st.mean(walls) / 1e3,
        "busy_us": st.mean(busy) / 1e3,
        "idle_us": (st.mean(walls) - st.mean(busy)) / 1e3,
        "launches": st.mean(len(s) for s in steps),
    }
    agg: Dict[Tuple[str, int], List[float]] = {}
    for s in steps:
        for n, g, a, b in s:
            agg.setdefault((short_name(n), g), []).append((b - a) / 1e3)
    rows = []
    for (n, g), v in agg.items():
        per_step = sum(v) / len(steps)
        rows.append((n, g, len(v) / len(steps), st.mean(v), per_step, 100.0 * per_step / summary["busy_us"]))
    rows.sort(key=lambda r: -r[4])
    return summary, rows


def kernel_table(launches: Sequence[Launch], substr: str = "") -> List[Tuple[str, int, int, float, float, float]]:
    """(kernel, grid, count, avg us, median us, min us) per kernel and grid, the largest
    total first."""
    by: Dict[Tuple[str, int], List[float]] = {}
    for n, g, a, b in launches:
        if substr and substr not in n:
            continue
        by.setdefault((short_name(n), g), []).append((b - a) / 1e3)
    rows = [(n, g, len(v), st.mean(v), st.median(v), min(v)) for (n, g), v in by.items()]
    rows.sort(key=lambda r: -r[2] * r[3])
    return rows


Copy = Tuple[int, int, int]  # (start ns, end ns, bytes)


def read_h2d_copies(db_path: str, min_bytes: int = 1 << 20) -> List[Copy]:
    """Host-to-device copies of at least min_bytes, by start time."""
    con = sqlite3.connect(db_path)
    try:
        rows = con.execute("select start, end, size, src_agent_type, dst_agent_type from memory_copies "
                           "order by start").fetchall()
    finally:
        con.close()
    return [(int(a), int(b), int(n)) for a, b, n, src, dst in rows
            if str(src).upper() == "CPU" and str(dst).upper() == "GPU" and int(n) >= min_bytes]


def _union(iv: Sequence[Tuple[int, int]]) -> List[Tuple[int, int]]:
    out: List[Tuple[int, int]] = []
    for a, b in sorted(iv):
        if out and a <= out[-1][1]:
            out[-1] = (out[-1][0], max(out[-1][1], b))
        else:
            out.append((a, b))
    return out


def _overlap(u: Sequence[Tuple[int, int]], v: Sequence[Tuple[int, int]]) -> int:
    """Total length of the intersection of two sorted disjoint interval lists."""
    i = j = tot = 0
    while i < len(u) and j < len(v):
        a, b = max(u[i][0], v[j][0]), min(u[i][1], v[j][1])
        if a < b:
            tot += b - a
        if u[i][1] < v[j][1]:
            i += 1
        else:
            j += 1
    return tot


def interval_stats(copies: Sequence[Copy], compute: Sequence[Tuple[int, int]], lo: int, hi: int,
                   steps: int) -> Dict[str, float]:
    """Host-link use inside the window [lo, hi) (nanoseconds) that holds `steps` decode
    steps: copies (start, end, bytes) and compute intervals are clipped to the window (a
    clipped copy keeps its share of the bytes); the link is busy while at least one copy
    runs.  Returns per-step figures, the busy share of the wall time, the rate while busy,
    and the share of copy time during which compute runs (and vice versa)."""
    clip = lambda a, b: (max(a, lo), min(b, hi))
    cp = [(clip(a, b), n * (min(b, hi) - max(a, lo)) / max(1, b - a)) for a, b, n in copies
          if b > lo and a < hi]
    cu = _union([iv for iv, _ in cp])
    ku = _union([clip(a, b) for a, b in compute if b > lo and a < hi])
    busy = sum(b - a for a, b in cu)
    kbusy = sum(b - a for a, b in ku)
    moved = sum(n for _, n in cp)
    both = _overlap(cu, ku)
    wall = hi - lo
    return {
        "steps": float(steps),
        "wall_ms_per_step": wall / 1e6 / steps,
        "copies_per_step": len(cp) / steps,
        "mb_per_step": moved / 1e6 / steps,
        "link_busy_frac": busy / wall if wall else 0.0,
        "gbps_while_busy": moved / busy if busy else 0.0,
        "gbps_over_wall": moved / wall if wall else 0.0,
        "kernel_busy_frac": kbusy / wall if wall else 0.0,
        "copy_time_with_kernel_frac": both / busy if busy else 0.0,
        "kernel_time_with_copy_frac": both / kbusy if kbusy else 0.0,
    }


def copy_table(launches: Sequence[Launch], copies: Sequence[Copy], last: int | None = None) -> Dict[str, float]:
    """Host-link use over the last `last` decode steps (all complete steps if None): the
    window runs from the first kernel of the first of those steps to the end of the last;
    the compute intervals are every kernel's."""
    steps = split_steps(launches, last)
    if not steps:
        raise ValueError(f"no complete decode step (no two {STEP_END_KERNEL} launches) in the trace")
    return interval_stats(copies, [(a, b) for _, _, a, b in launches], steps[0][0][2],
                          steps[-1][-1][3], len(steps))


def counter_table(db_path: str, substr: str = "") -> List[Tuple[str, str, int, float, float]]:
    """(kernel, counter, dispatches, median value, mean value) per kernel and counter."""
    con = sqlite3.connect(db_path)
    try:
        rows = con.execute("select kernel_name, counter_name, value from counters_collection").fetchall()
    finally:
        con.close()
    by: Dict[Tuple[str, str], List[float]] = {}
    for n, c, v in rows:
        if substr and substr not in str(n):
            continue
        by.setdefault((short_name(str(n)), str(c)), []).append(float(v))
    return sorted((n, c, len(v), st.median(v), st.mean(v)) for (n, c), v in by.items())


def _main(argv: Sequence[str]) -> int:
    if len(argv) >= 2 and argv[0] == "counters":
        print("| kernel | counter | dispatches | median | mean |")
        print("|---|---|---:|---:|---:|")
        for n, c, cnt, med, mean in counter_table(argv[1], argv[2] if len(argv) > 2 else ""):
            print(f"| {n} | {c} | {cnt} | {med:.1f} | {mean:.1f} |")
        return 0
    if len(argv) >= 2 and argv[0] == "copies":
        last = int(argv[2]) if len(argv) > 2 else None
        min_mib = float(argv[3]) if len(argv) > 3 else 1.0
        t = copy_table(read_launches(argv[1]), read_h2d_copies(argv[1], int(min_mib * (1 << 20))), last)
        print("| quantity | value |")
        print("|---|---:|")
        for k, v in t.items():
            print(f"| {k} | {v:.4g} |")
        return 0
    if len(argv) < 2 or argv[0] not in ("steps", "kernels"):
        print(__doc__)
        return 2
    launches = read_launches(argv[1])
    if argv[0] == "steps":
        last = int(argv[2]) if len(argv) > 2 else None
        summary, rows = step_table(split_steps(launches, last))
        print(f"steps {summary['steps']:.0f}: wall/step {summary['wall_us']:.1f} us, busy/step "
              f"{summary['busy_us']:.1f} us, idle/step {summary['idle_us']:.1f} us, launches/step "
              f"{summary['launches']:.1f}")
        print("| kernel | grid | launches/step | avg us | us/step | % of busy |")
        print("|---|---|---:|---:|---:|---:|")
        for n, g, per, avg, us, pct in rows:
            print(f"| {n} | {g}x1 | {per:.0f} | {avg:.2f} | {us:.1f} | {pct:.1f} |")
    else:
        substr = argv[2] if len(argv) > 2 else ""
        print("| kernel | grid | launches | avg us | median us | min us |")
        print("|---|---|---:|---:|---:|---:|")
        for n, g, cnt, avg, med, mn in kernel_table(launches, substr):
            print(f"| {n} | {g}x1 | {cnt} | {avg:.2f} | {med:.2f} | {mn:.2f} |")
    return 0


if __name__ == "__main__":
    sys.exit(_main(sys.argv[1:]))
