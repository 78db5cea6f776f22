"""Pins of the router / dispatch / combine / SwiGLU oracle -- CPU only.

The router is checked against torch's own F.linear / F.softmax / topk -- the calls
engine/router.py:66-92 makes -- and the closed form of the top-2 weights; the combine
against the reference's statements of model/moe_layer.py:147,187-191 executed by torch;
dispatch against the fake-expert closed form of the reference's
tests/test_moe_layer.py:180-266 setup; SwiGLU against a permutation-matrix closed form
and a torch float32 chain.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from helpers import bits, near_tie_rows
from oracle import moe_oracle as orc


def _bf16(shape, seed, std=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * std).to(torch.bfloat16)


@pytest.mark.parametrize("T,H,E,k", [(16, 1024, 8, 2), (33, 256, 8, 2), (9, 128, 16, 4)])
def test_router_matches_torch_reference_ops(T, H, E, k):
    x, gate = _bf16((T, H), T), _bf16((E, H), H, 0.02)
    lg, w, idx = orc.router(bits(x), bits(gate), k=k)
    t_logits = F.linear(x, gate)
    p = F.softmax(t_logits.float(), dim=-1)
    tw, ti = torch.topk(p, k, dim=-1)
    tw = tw / tw.sum(dim=-1, keepdim=True)
    assert np.abs(bits(t_logits).astype(np.int32) - lg.astype(np.int32)).max() <= 1
    keep = ~near_tie_rows(lg, k=k)
    np.testing.assert_array_equal(idx[keep], ti.numpy()[keep])
    np.testing.assert_allclose(w[keep], tw.numpy()[keep], rtol=1e-6, atol=1e-7)


def test_router_top2_closed_form_and_invariants():
    x, gate = _bf16((64, 512), 1), _bf16((8, 512), 2, 0.02)
    lg, w, idx = orc.router(bits(x), bits(gate), k=2)
    lf = orc.bf16_to_f32(lg).astype(np.float64)
    l0 = np.take_along_axis(lf, idx[:, :1], 1)[:, 0]
    l1 = np.take_along_axis(lf, idx[:, 1:], 1)[:, 0]
    np.testing.assert_allclose(w[:, 0], 1.0 / (1.0 + np.exp(l1 - l0)), rtol=2e-6)
    np.testing.assert_allclose(w.sum(-1), 1.0, atol=1e-6)
    assert np.all(w[:, 0] >= w[:, 1]) and np.all((idx >= 0) & (idx < 8))
    assert np.all(np.sort(-lf, 1)[:, :2] == -np.take_along_axis(lf, idx, 1))


def test_router_bias_shifts_logits_before_softmax():
    x, gate = _bf16((20, 256), 3), _bf16((8, 256), 4, 0.02)
    bias = np.log(np.arange(1, 9, dtype=np.float32)[::-1] / 36.0).astype(np.float32) * 4
    lg, w, idx = orc.router(bits(x), bits(gate), k=2, bias=bias)
    p = F.softmax(torch.from_numpy(orc.bf16_to_f32(lg)) + torch.from_numpy(bias), dim=-1)
    tw, ti = torch.topk(p, 2, dim=-1)
    keep = ~near_tie_rows(lg, bias)
    np.testing.assert_array_equal(idx[keep], ti.numpy()[keep])
    np.testing.assert_allclose(w[keep], (tw / tw.sum(-1, keepdim=True)).numpy()[keep], rtol=1e-6)


def test_predict_next_layer_experts_known_answer():
    """tests/test_engine.py:93-108 of the reference."""
    from moeinfra_amd.engine.router import ExpertRouter

    idx = torch.tensor([[3, 1], [5, 2], [1, 4]])
    assert orc.predict_next_layer_experts(idx.numpy()) == [1, 2, 3, 4, 5]
    r = ExpertRouter(torch.zeros(8, 16, dtype=torch.bfloat16), 2)
    assert r.predict_next_layer_experts(idx) == [1, 2, 3, 4, 5]


def test_combine_matches_reference_statements_in_torch():
    """out = zeros_like(x); out[mask] += y_e * w_e, ascending e (bf16 out, fp32 weights)."""
    T, H, E = 24, 64, 8
    x = _bf16((T, H), 7)
    gate = _bf16((E, H), 8, 0.05)
    ys = {e: _bf16((T, H), 100 + e) for e in range(E)}     # expert e's output for every row
    lg, w, idx = orc.router(bits(x), bits(gate), k=2)

    out_o, _ = orc.moe_layer(bits(x), bits(gate), lambda e, rows: bits(ys[e])[_rows(idx, e)])

    ti, tw = torch.from_numpy(idx), torch.from_numpy(w)
    out_t = torch.zeros_like(x)
    for e in sorted(torch.unique(ti).tolist()):
        m = ti == e
        mask = m.any(-1)
        token_w = (tw * m.to(tw.dtype)).sum(-1)
        out_t[mask] += ys[e][mask] * token_w[mask].unsqueeze(-1)
    np.testing.assert_array_equal(out_o, bits(out_t))


def _rows(idx, e):
    return np.nonzero((idx == e).any(-1))[0]


def test_fake_expert_closed_form():
    """Fake experts f_e(x) = x*(e+1): out[t] = x[t] * sum_k w[t,k]*(idx[t,k]+1)."""
    T, H = 32, 128
    x, gate = _bf16((T, H), 11), _bf16((8, H), 12, 0.02)
    out, (lg, w, idx) = orc.moe_layer(
        bits(x), bits(gate),
        lambda e, rows: orc.bf16_round(orc.bf16_to_f32(rows) * np.float32(e + 1)))
    want = orc.bf16_to_f32(bits(x)).astype(np.float64) * (w * (idx + 1)).sum(-1, keepdims=True)
    np.testing.assert_allclose(orc.bf16_to_f32(out), want, rtol=2e-2, atol=1e-2)
    assert orc.rel_l2(orc.bf16_to_f32(out), want) < 5e-3


def test_swiglu_permutation_closed_form():
    """NF4 can hold a*P exactly (code 15 = 1.0, code 7 = 0): with W1 = a P1, W3 = b P3,
    W2 = c P2 the expert is y[i] = c * h[p2(i)], h[j] = silu(a x[p1(j)]) * (b x[p3(j)])
    with bf16 rounding between the ops.  Catches transposed operands and swapped w1/w3."""
    H, Fd = 128, 256
    rng = np.random.default_rng(0)
    p1, p3 = rng.permutation(H * 2)[:Fd] % H, rng.permutation(H * 2)[:Fd] % H
    p2 = rng.permutation(Fd)[:H]
    a, b, c = np.float32(0.5), np.float32(2.0), np.float32(0.25)

    def nf4_of(rows, cols, src, scale):
        m = np.zeros((rows, cols), dtype=np.float32)
        m[np.arange(rows), src] = scale
        packed, absmax = orc.nf4_quantize(orc.bf16_round(m).reshape(-1))
        return orc.nf4_dequant(packed, absmax).reshape(rows, cols), m

    w1, m1 = nf4_of(Fd, H, p1, a)
    w3, m3 = nf4_of(Fd, H, p3, b)
    w2, m2 = nf4_of(H, Fd, p2, c)
    np.testing.assert_array_equal(orc.bf16_to_f32(w1), m1)   # exactly representable
    x = bits(_bf16((5, H), 21))
    y = orc.swiglu(x, w1, w3, w2)
    xf = orc.bf16_to_f32(x)
    g = orc.bf16_round(a * xf[:, p1])
    u = orc.bf16_round(b * xf[:, p3])
    s = orc.bf16_round(orc.silu_f32(orc.bf16_to_f32(g)))
    h = orc.bf16_to_f32(orc.bf16_round(orc.bf16_to_f32(s) * orc.bf16_to_f32(u)))
    np.testing.assert_array_equal(y, orc.bf16_round(c * h[:, p2]))


def test_swiglu_matches_torch_chain():
    H, Fd = 96, 160
    w1, w3 = bits(_bf16((Fd, H), 31, 0.05)), bits(_bf16((Fd, H), 32, 0.05))
    w2, x = bits(_bf16((H, Fd), 33, 0.05)), bits(_bf16((7, H), 34))
    t = lambda a: torch.from_numpy(orc.bf16_to_f32(a))
    g = (t(x) @ t(w1).T).to(torch.bfloat16)
    u = (t(x) @ t(w3).T).to(torch.bfloat16)
    hh = (F.silu(g.float()).to(torch.bfloat16).float() * u.float()).to(torch.bfloat16)
    y = (hh.float() @ t(w2).T).to(torch.bfloat16)
    got = orc.swiglu(x, w1, w3, w2)
    assert orc.rel_l2(orc.bf16_to_f32(got), y.float().numpy()) < 3e-3
