"""Writes the golden fixtures of tests/golden/ from the oracle (run from the repo root:
``python tests/golden/make_fixtures.py``).

The reference ships no numeric golden values for this path (its numeric tests compare
bitsandbytes with itself), so these fixtures pin the oracle's own outputs on small
seeded cases.  Inputs are not stored: they are regenerated from the recorded seeds by
the seeded generators (CPU torch.Generator, fixed draw order), and the manifest keeps a
SHA-256 of every regenerated input so that a change in the generators or in torch's RNG
is detected instead of silently moving the expected values.
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from helpers import bits, build_layer, oracle_layer  # noqa: E402
from oracle import moe_oracle as orc  # noqa: E402

# name -> parameters; layer cases: hidden, ffn, experts, tokens, seed, zipf routing bias
LAYER_CASES = {
    "layer_decode_t1": dict(H=512, F=1024, E=8, T=1, seed=101, zipf=False),
    "layer_decode_t4_zipf": dict(H=512, F=1024, E=8, T=4, seed=102, zipf=True),
    "layer_grouped_t16": dict(H=256, F=512, E=8, T=16, seed=103, zipf=False),
    "layer_grouped_t40_zipf": dict(H=256, F=768, E=8, T=40, seed=104, zipf=True),
}


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def nf4_inputs(seed: int):
    rng = np.random.default_rng(seed)
    n = 64 * 64 + 32
    packed = rng.integers(0, 256, n // 2, dtype=np.uint8)
    absmax = (rng.random((n + 63) // 64, dtype=np.float32) * 0.5).astype(np.float32)
    w = orc.bf16_round((rng.standard_normal(64 * 40) * 0.02).astype(np.float32))
    return packed, absmax, w


def layer_inputs(p):
    from moeinfra_amd import synth

    gate, experts, x = build_layer(p["H"], p["F"], p["E"], p["T"], p["seed"])
    bias = synth.zipf_bias(p["E"], p["seed"]) if p["zipf"] else None
    return gate, experts, x, bias


def compute_case(name):
    """(expected outputs, input hashes) of one case, from the oracle."""
    if name == "nf4":
        packed, absmax, w = nf4_inputs(7)
        deq = orc.nf4_dequant(packed, absmax, numel=packed.size * 2)
        qp, qa = orc.nf4_quantize(w)
        out = {"dequant": deq, "quant_packed": qp, "quant_absmax": qa}
        hashes = {"packed": sha(packed), "absmax": sha(absmax), "w": sha(w)}
        return out, hashes
    p = LAYER_CASES[name]
    gate, experts, x, bias = layer_inputs(p)
    o, (lg, w, idx) = oracle_layer(gate, experts, x, bias=bias)
    out = {"out": o, "logits": lg, "weights": w, "idx": idx}
    hashes = {"x": sha(bits(x)), "gate": sha(bits(gate))}
    for e, ex in enumerate(experts):
        for proj, (pk, am) in ex.np.items():
            hashes[f"e{e}_{proj}_packed"] = sha(pk)
            hashes[f"e{e}_{proj}_absmax"] = sha(am)
    if bias is not None:
        hashes["bias"] = sha(bias.numpy())
    return out, hashes


def all_cases():
    return ["nf4", *LAYER_CASES]


def main():
    manifest = {}
    for name in all_cases():
        out, hashes = compute_case(name)
        path = os.path.join(HERE, f"{name}.npz")
        np.savez(path, **out)
        manifest[name] = {"file": f"{name}.npz", "inputs_sha256": hashes,
                          "params": LAYER_CASES.get(name, {"seed": 7}),
                          "outputs_sha256": {k: sha(v) for k, v in out.items()}}
    with open(os.path.join(HERE, "manifest.json"), "w") as fh:
        json.dump(manifest, fh, indent=1, sort_keys=True)
    print("wrote", len(manifest), "fixtures")


if __name__ == "__main__":
    main()
