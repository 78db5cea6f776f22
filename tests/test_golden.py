"""Golden fixtures (tests/golden/, written by tests/golden/make_fixtures.py).

CPU: the fixtures' hashes, the regenerated inputs' hashes and the oracle's outputs all
match what was committed.  GPU: the HIP kernels reproduce the committed outputs (bit-exact
for the NF4 byte work, rel-L2 <= 1e-2 and equal top-k away from near-ties for layers)."""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np
import pytest

from helpers import bits, near_tie_rows
from oracle import moe_oracle as orc

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, GOLDEN)
import make_fixtures as mk  # noqa: E402

MANIFEST = json.load(open(os.path.join(GOLDEN, "manifest.json")))


def _load(name):
    with np.load(os.path.join(GOLDEN, MANIFEST[name]["file"])) as z:
        return {k: z[k] for k in z.files}


def test_manifest_covers_every_case():
    assert sorted(MANIFEST) == sorted(mk.all_cases())


@pytest.mark.parametrize("name", mk.all_cases())
def test_fixture_files_match_manifest(name):
    data = _load(name)
    assert {k: mk.sha(v) for k, v in data.items()} == MANIFEST[name]["outputs_sha256"]


@pytest.mark.parametrize("name", mk.all_cases())
def test_oracle_and_generators_reproduce_fixture(name):
    out, hashes = mk.compute_case(name)
    assert hashes == MANIFEST[name]["inputs_sha256"], "seeded generators or RNG changed"
    want = _load(name)
    for k, v in out.items():
        np.testing.assert_array_equal(v, want[k], err_msg=f"{name}:{k}")


@pytest.mark.gpu
def test_gpu_nf4_matches_golden(cuda_device):
    import torch

    from moeinfra_amd import ops

    packed, absmax, w = mk.nf4_inputs(7)
    want = _load("nf4")
    t = lambda a: torch.from_numpy(a.copy()).to(cuda_device)
    code = t(orc.NF4_CODE)
    got = ops.nf4_dequant(t(packed), t(absmax), code, (packed.size * 2,), 64)
    np.testing.assert_array_equal(bits(got), want["dequant"])
    wt = torch.from_numpy(w.view(np.int16).copy()).view(torch.bfloat16).to(cuda_device)
    qp, qa, _ = ops.nf4_quantize(wt, 64)
    np.testing.assert_array_equal(qp.cpu().numpy().reshape(-1), want["quant_packed"])
    np.testing.assert_array_equal(qa.cpu().numpy(), want["quant_absmax"])


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(mk.LAYER_CASES))
def test_gpu_layer_matches_golden(cuda_device, name):
    from moeinfra_amd import ops

    p = mk.LAYER_CASES[name]
    gate, experts, x, bias = mk.layer_inputs(p)
    for ex in experts:
        ex.to(cuda_device)
    table = ops.expert_table([ex.c_struct() for ex in experts])
    out, lg, w, idx = ops.layer_forward(table, p["E"], gate.to(cuda_device), x.to(cuda_device),
                                        2, p["F"], bias=None if bias is None else bias.to(cuda_device),
                                        want_logits=True)
    want = _load(name)
    ok = ~near_tie_rows(want["logits"], None if bias is None else bias.numpy())
    assert ok.sum() >= max(1, ok.size // 2)
    np.testing.assert_array_equal(idx.cpu().numpy()[ok], want["idx"][ok])
    np.testing.assert_allclose(w.cpu().numpy()[ok], want["weights"][ok], rtol=1e-5, atol=1e-6)
    assert np.abs(bits(lg).astype(np.int32) - want["logits"].astype(np.int32)).max() <= 1
    err = orc.rel_l2(orc.bf16_to_f32(bits(out)[ok]), orc.bf16_to_f32(want["out"][ok]))
    assert err <= 1e-2, err
