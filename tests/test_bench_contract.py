"""bench.py on the CPU: its byte accounting and its single-GPU guard."""
from __future__ import annotations

import os
import subprocess
import sys

import bench
from moeinfra_amd.engine.decoder import MixtralShape

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_nf4_expert_bytes_mixtral():
    # w1, w3, w2 of 14336 x 4096 each: packed nibbles + one fp32 absmax per 64 values
    n = 14336 * 4096
    assert bench.nf4_expert_bytes(4096, 14336) == 3 * (n // 2 + (n // 64) * 4) == 99_090_432


def test_gateup_bytes_decode_form():
    n = 14336 * 4096
    want = 2 * 2 * (n // 2 + n // 64 * 4) + 4096 * 2 + 2 * 14336 * 2 + 8 * 4096 * 2
    assert bench.decode_form(1, 2, 8, 4096, 14336)
    assert bench.gateup_bytes(2, 4096, 14336, 1, 2, 8) == want
    assert not bench.decode_form(16, 2, 8, 4096, 14336)


def test_decode_step_bytes_mixtral():
    s = MixtralShape()
    pos = 55
    per_layer = ((6144 * 4096 + 4096 * 4096) * 2 + 2 * 8 * (pos + 1) * 128 * 2
                 + 2 * 99_090_432 + 8 * 4096 * 2)
    want = 32 * per_layer + 32000 * 4096 * 2 + 4096 * 2
    assert bench.decode_step_bytes(s, [2] * 32, pos) == want
    # about 9.3 GB per token: ~1.9 ms at 5 TB/s
    assert 9.2e9 < want < 9.4e9


def test_more_than_one_gpu_is_refused():
    p = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, cwd=ROOT, timeout=300)
    assert p.returncode == 2
    assert "one GPU" in p.stderr
