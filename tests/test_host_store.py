"""The on-disk NF4 expert store (model/loader.py:303-381 file and key scheme) and the
nested-absmax restatement of the oracle, on the CPU."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import moe_oracle as orc


def _expert(H=128, F=256, seed=0, nested=False):
    from moeinfra_amd.model.expert import NF4QuantState, PrequantizedNF4Expert, _BLOB_KEY

    g = torch.Generator().manual_seed(seed)
    shapes = {"w1": (F, H), "w3": (F, H), "w2": (H, F)}
    ser = {}
    for name, (o, i) in shapes.items():
        n = o * i
        packed = torch.randint(0, 256, (n // 2, 1), generator=g, dtype=torch.int64).to(torch.uint8)
        absmax = torch.rand(n // 64, generator=g) + 0.01
        code = torch.linspace(-1, 1, 16)
        st = {"weight": packed, "weight.quant_map": code}
        if nested:
            q, a2, c2, off = orc.double_quantize_absmax(absmax.numpy(), 256)
            qs = NF4QuantState(absmax=torch.from_numpy(q), code=code, shape=torch.Size((o, i)),
                               offset=torch.tensor(off),
                               state2=NF4QuantState(absmax=torch.from_numpy(a2),
                                                    code=torch.from_numpy(c2),
                                                    shape=torch.Size((n // 64,)), blocksize=256,
                                                    quant_type=None, dtype=torch.float32))
            st.update({"weight.absmax": torch.from_numpy(q),
                       "weight.nested_absmax": torch.from_numpy(a2),
                       "weight.nested_quant_map": torch.from_numpy(c2)})
        else:
            qs = NF4QuantState(absmax=absmax, code=code, shape=torch.Size((o, i)))
            st["weight.absmax"] = absmax
        st["weight." + _BLOB_KEY] = qs.blob()
        ser[name] = st
    return PrequantizedNF4Expert.from_serialized(ser["w1"], ser["w2"], ser["w3"], H, F)


def test_expert_filename():
    from moeinfra_amd.model.store import expert_filename

    assert expert_filename(3, 7) == "layer_03_expert_07.safetensors"
    assert expert_filename(31, 0) == "layer_31_expert_00.safetensors"


@pytest.mark.parametrize("nested", [False, True])
def test_store_round_trip(tmp_path, nested):
    """Written and read back: the same tensors under the reference's key names, found in
    the second of two store directories."""
    from moeinfra_amd.model.store import NF4ExpertStore, expert_state_dict, save_expert

    ex = _expert(nested=nested)
    path = save_expert(tmp_path / "b", 2, 5, ex)
    assert path.name == "layer_02_expert_05.safetensors"
    keys = set(expert_state_dict(ex))
    want = {f"{p}.{k}" for p in ("w1", "w2", "w3")
            for k in ("weight", "weight.absmax", "weight.quant_map",
                      "weight.quant_state.bitsandbytes__nf4")}
    if nested:
        want |= {f"{p}.weight.nested_{k}" for p in ("w1", "w2", "w3") for k in ("absmax", "quant_map")}
    assert keys == want
    store = NF4ExpertStore([tmp_path / "a", tmp_path / "b"], 128, 256, num_layers=4, num_experts=8)
    back = store.load_expert(2, 5)
    for name in ("w1", "w2", "w3"):
        a, b = getattr(ex, name), getattr(back, name)
        assert a.keys() == b.keys()
        for k in a:
            assert a[k].dtype == b[k].dtype and torch.equal(a[k], b[k]), (name, k)
    assert back.size_bytes == ex.size_bytes


def test_store_nested_state_is_parsed(tmp_path):
    from moeinfra_amd.model.expert import _linear_from_serialized
    from moeinfra_amd.model.store import NF4ExpertStore, save_expert

    ex = _expert(nested=True)
    save_expert(tmp_path, 0, 0, ex)
    back = NF4ExpertStore([tmp_path], 128, 256).load_expert(0, 0)
    lin = _linear_from_serialized(back.w1, 128, 256)
    qs = lin.quant_state
    assert qs.nested and qs.state2.blocksize == 256 and qs.absmax.dtype == torch.uint8
    want_off = float(orc.double_quantize_absmax(
        _expert(nested=False).w1["weight.absmax"].numpy(), 256)[3])
    assert float(qs.offset) == pytest.approx(want_off, rel=0, abs=0)


def test_store_errors(tmp_path):
    from moeinfra_amd.model.store import NF4ExpertStore

    store = NF4ExpertStore([tmp_path / "x", tmp_path / "y"], 128, 256, num_layers=2, num_experts=8)
    with pytest.raises(FileNotFoundError, match="layer_01_expert_03.safetensors.*Searched stores"):
        store.load_expert(1, 3)
    with pytest.raises(IndexError):
        store.load_expert(2, 0)
    with pytest.raises(IndexError):
        store.load_expert(0, 8)


def test_expand_absmax_hand_case():
    """Two groups of two: the group index is i // blocksize2 (not i % ...), the product is
    rounded before the offset is added."""
    code2 = np.linspace(-1, 1, 256, dtype=np.float32)
    q = np.array([0, 255, 128, 1], dtype=np.uint8)
    a2 = np.array([2.0, 4.0], dtype=np.float32)
    got = orc.expand_absmax(q, a2, code2, 0.5, 2)
    want = np.array([-1 * 2 + 0.5, 1 * 2 + 0.5,
                     np.float32(np.float32(code2[128]) * np.float32(4)) + np.float32(0.5),
                     np.float32(np.float32(code2[1]) * np.float32(4)) + np.float32(0.5)],
                    dtype=np.float32)
    np.testing.assert_array_equal(got, want)
    # a product that is inexact in fp32: rounded once, then the offset added
    v = np.float32(1.0) / np.float32(3.0)
    c = code2.copy()
    c[7] = v
    out = orc.expand_absmax(np.array([7], np.uint8), np.array([3.0], np.float32), c, 1e-8, 256)
    assert out[0] == np.float32(np.float32(v * np.float32(3.0)) + np.float32(1e-8))


def test_double_quantize_round_trip_error_bound():
    """expand(double_quantize(a)) is within half a code step of a, per group."""
    rng = np.random.default_rng(0)
    a = (rng.random(5000, dtype=np.float32) * 0.1 + 1e-3).astype(np.float32)
    q, a2, c2, off = orc.double_quantize_absmax(a, 256)
    back = orc.expand_absmax(q, a2, c2, off, 256)
    step = float(c2[1] - c2[0])
    grp = np.arange(a.size) // 256
    assert np.all(np.abs(back - a) <= a2[grp] * step * 0.5 * (1 + 1e-5) + 1e-7)
