"""The canonical NF4 state of an expert and its contiguous image (transfer/expert_image.py),
on the CPU: every form a CPU-tier expert may take gives the same canonical tensors (the
reference's staging keys, transfer/reusable_staging.py:126-222), the image layout is
aligned and non-overlapping, and packing then viewing an image reproduces the state bit for
bit."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from moeinfra_amd.model.expert import NF4Linear, NF4QuantState, PrequantizedNF4Expert
from moeinfra_amd.transfer.expert_image import (IMAGE_ALIGN, ImageLayout, canonical_expert,
                                                canonical_projection, pack_image)
from oracle import moe_oracle as orc

H, F = 128, 192


def _state(seed):
    g = torch.Generator().manual_seed(seed)
    out = {}
    for name, (o, i) in (("w1", (F, H)), ("w3", (F, H)), ("w2", (H, F))):
        w = (torch.randn((o, i), generator=g) * 0.02).to(torch.bfloat16)
        p, a = orc.nf4_quantize(w.view(torch.int16).numpy().view(np.uint16).reshape(-1))
        out[name] = (torch.from_numpy(p), torch.from_numpy(a), torch.from_numpy(orc.NF4_CODE.copy()))
    return out


def _same(a, b):
    assert a.dtype == b.dtype and torch.equal(a.reshape(-1), b.reshape(-1))


def test_every_expert_form_gives_the_same_canonical_state():
    st = _state(1)
    serialized = PrequantizedNF4Expert.from_nf4_tensors(st, H, F)
    canonical = type("E", (), {n: {"weight": st[n][0], "absmax": st[n][1], "quant_map": st[n][2]}
                               for n in st})()
    shapes = {"w1": (F, H), "w3": (F, H), "w2": (H, F)}
    linear = type("E", (), {n: NF4Linear(st[n][0].reshape(-1, 1), shapes[n][1], shapes[n][0],
                                         NF4QuantState(st[n][1], st[n][2], torch.Size(shapes[n])))
                            for n in st})()
    for expert in (serialized, canonical, linear):
        got = canonical_expert(expert)
        for n in ("w1", "w2", "w3"):
            assert list(got[n]) == ["weight", "absmax", "code", "offset"]
            _same(got[n]["weight"], st[n][0])
            _same(got[n]["absmax"], st[n][1])
            _same(got[n]["code"], st[n][2])
            assert got[n]["offset"] is None


def test_serialized_nested_state_keeps_the_second_level():
    st = _state(2)
    q, a2, c2, off = orc.double_quantize_absmax(st["w1"][1].numpy())
    ser = PrequantizedNF4Expert.from_nf4_tensors(st, H, F).w1
    ser["weight.absmax"] = torch.from_numpy(q)
    ser["weight.nested_absmax"] = torch.from_numpy(a2)
    ser["weight.nested_quant_map"] = torch.from_numpy(c2)
    meta = NF4QuantState(torch.from_numpy(q), st["w1"][2], torch.Size((F, H)),
                         offset=torch.tensor(off),
                         state2=NF4QuantState(torch.from_numpy(a2), torch.from_numpy(c2),
                                              torch.Size(q.shape), blocksize=256))
    ser["weight.quant_state.bitsandbytes__nf4"] = meta.blob()
    got = canonical_projection(type("E", (), {"w1": ser})(), "w1")
    assert list(got) == ["weight", "absmax", "code", "offset", "state2_absmax", "state2_code",
                         "state2_offset"]
    _same(got["absmax"], torch.from_numpy(q))
    _same(got["state2_absmax"], torch.from_numpy(a2))
    assert float(got["offset"]) == pytest.approx(off)


def test_incomplete_states_are_refused():
    st = _state(3)
    ser = PrequantizedNF4Expert.from_nf4_tensors(st, H, F).w2
    with pytest.raises(ValueError, match="missing 'weight'"):
        canonical_projection(type("E", (), {"w2": {"absmax": st["w2"][1]}})(), "w2")
    bad = {k: v for k, v in ser.items() if k != "weight.quant_map"}
    with pytest.raises(ValueError, match="weight.quant_map"):
        canonical_projection(type("E", (), {"w2": bad})(), "w2")
    with pytest.raises(TypeError):
        canonical_projection(type("E", (), {"w2": 3})(), "w2")


def test_image_layout_round_trip():
    st = canonical_expert(PrequantizedNF4Expert.from_nf4_tensors(_state(4), H, F))
    lay = ImageLayout.of(st)
    prev_end = 0
    for f in lay.fields:
        assert f.offset % IMAGE_ALIGN == 0 and f.offset >= prev_end
        prev_end = f.offset + f.nbytes
    assert lay.nbytes % IMAGE_ALIGN == 0 and lay.nbytes >= prev_end
    assert {(f.projection, f.key) for f in lay.fields} == {(n, k) for n in st for k in st[n]
                                                         if st[n][k] is not None}
    buf = torch.full((lay.nbytes,), 0xAB, dtype=torch.uint8)
    views = pack_image(st, buf, lay)
    for n in st:
        for k, t in st[n].items():
            if t is not None:
                _same(views[n][k], t)
                assert views[n][k].data_ptr() - buf.data_ptr() == \
                    next(f.offset for f in lay.fields if (f.projection, f.key) == (n, k))
    again = lay.views(buf)
    for f in lay.fields:
        _same(again[f.projection][f.key], st[f.projection][f.key])
