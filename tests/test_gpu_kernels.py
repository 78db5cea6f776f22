"""GPU parity of the individual kernels (K0-K5) against the CPU oracle."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import (NF4Expert, assert_weights_close, bits, build_layer, from_bits, logit_slack,
                     near_tie_rows, oracle_layer)
from oracle import moe_oracle as orc

pytestmark = pytest.mark.gpu


def _code(dev):
    return torch.from_numpy(orc.NF4_CODE.copy()).to(dev)


# ------------------------------------------------------------------------------ K1
@pytest.mark.parametrize("numel", [64, 96, 4096 + 32 + 2, 3584 * 1024])
def test_dequant_bitexact(cuda_device, numel):
    from moeinfra_amd import ops

    rng = np.random.default_rng(numel)
    packed = rng.integers(0, 256, size=(numel + 1) // 2, dtype=np.uint8)
    absmax = (rng.random((numel + 63) // 64, dtype=np.float32) * 0.1).astype(np.float32)
    absmax[0] = 0.0
    want = orc.nf4_dequant(packed, absmax, numel=numel)
    got = ops.nf4_dequant(torch.from_numpy(packed).to(cuda_device),
                          torch.from_numpy(absmax).to(cuda_device), _code(cuda_device), (numel,))
    np.testing.assert_array_equal(bits(got), want)


def test_dequant_full_expert_projection(cuda_device):
    """One Mixtral-8x7B w1 [14336, 4096] from real quantised bf16 N(0, 0.02) weights."""
    from moeinfra_amd import ops, synth

    gen = synth.make_generator(2)
    w = synth._normal((14336, 4096), gen, "cpu", 0.02)
    packed, absmax = orc.nf4_quantize(bits(w).reshape(-1))
    want = orc.nf4_dequant(packed, absmax)
    got = ops.nf4_dequant(torch.from_numpy(packed).to(cuda_device),
                          torch.from_numpy(absmax).to(cuda_device), _code(cuda_device),
                          (14336, 4096))
    np.testing.assert_array_equal(bits(got).reshape(-1), want)


# ------------------------------------------------------------------------------ K0
@pytest.mark.parametrize("shape", [(64, 64), (256, 1024), (3, 130), (14336, 4096)])
def test_quantize_bitexact(cuda_device, shape):
    """Blocksize 64 over whole 512-value chunks takes the eight-lanes-per-block kernel, other
    sizes the per-block one; both bit-exact, including an all-zero block, signed zeros and
    a block whose maximum is negative."""
    from moeinfra_amd import ops, synth

    gen = synth.make_generator(11)
    w = synth._normal(shape, gen, "cpu", 0.02)
    flat = w.view(-1)
    flat[5] = 0.0
    if flat.numel() >= 256:
        flat[64:128] = 0.0                       # absmax 0: every value maps to code 7
        flat[130] = -0.0
        flat[192:256] = -flat[192:256].abs()
        flat[200] = -0.5                         # a negative maximum magnitude
    p_want, a_want = orc.nf4_quantize(bits(w).reshape(-1))
    p_got, a_got, _ = ops.nf4_quantize(w.to(cuda_device))
    np.testing.assert_array_equal(p_got.cpu().numpy().reshape(-1), p_want)
    np.testing.assert_array_equal(a_got.cpu().numpy(), a_want)


# ------------------------------------------------------------------------------ K2
@pytest.mark.parametrize("T,H,E,skew,k", [(1, 4096, 8, False, 2), (16, 1024, 8, False, 2),
                                          (40, 4096, 8, True, 2), (513, 4096, 8, False, 2),
                                          (7, 256, 16, False, 2), (4096, 4096, 8, False, 2),
                                          (4096, 4096, 8, True, 2), (9, 1000, 32, True, 4),
                                          (33, 4104, 16, False, 8), (3, 8, 8, False, 1)])
def test_router_matches_oracle(cuda_device, T, H, E, skew, k):
    """One wavefront per token: T not a multiple of the eight tokens of a workgroup, H not
    a multiple of the gate chunk (512 / 256 / 128 values for E <= 8 / 16 / 32), E = 32."""
    from moeinfra_amd import ops, synth

    gen = synth.make_generator(T * 31 + H)
    gate = synth._normal((E, H), gen, "cpu", 0.02)
    x = synth.make_activations(T, H, gen)
    bias = synth.zipf_bias(E, seed=T) if skew else None
    lg_want, w_want, i_want = orc.router(bits(x), bits(gate), k=k,
                                         bias=None if bias is None else bias.numpy())
    lg, w, idx = ops.router_topk(x.to(cuda_device), gate.to(cuda_device), k,
                                 bias=None if bias is None else bias.to(cuda_device))
    # fp32 accumulation order differs from the oracle's: the bf16 logits agree within one
    # bf16 ulp plus the reordering error of an fp32 dot product, bounded by
    # 2^-18 * sum_i |x_i g_ei| (H <= 8192 terms); for logits far from zero that is 1 ulp.
    lf_g = orc.bf16_to_f32(bits(lg)).astype(np.float64)
    lf_w = orc.bf16_to_f32(lg_want).astype(np.float64)
    mag = np.abs(orc.bf16_to_f32(bits(x)).astype(np.float64)) @ \
        np.abs(orc.bf16_to_f32(bits(gate)).astype(np.float64)).T
    ulp = np.maximum(np.abs(lf_w), 1e-30) * 2.0 ** -7
    assert (np.abs(lf_g - lf_w) <= ulp + 2.0 ** -18 * mag).all()
    # Rows where any two of the k + 1 largest logits are within 1 bf16 ulp may order (or
    # choose) differently.
    tie = np.zeros(T, dtype=bool)
    slack = logit_slack(bits(x), bits(gate))
    for kk in range(1, min(k, E - 1) + 1):
        tie |= near_tie_rows(lg_want, None if bias is None else bias.numpy(), k=kk, slack=slack)
    keep = ~tie
    assert keep.sum() >= max(1, T // 2)
    np.testing.assert_array_equal(idx.cpu().numpy()[keep], i_want[keep])
    assert_weights_close(w.cpu().numpy()[keep], w_want[keep], bits(lg)[keep], lg_want[keep],
                         rtol=2e-5)
    assert (lf_g == lf_w).all(axis=-1).mean() > 0.9
    np.testing.assert_allclose(w.sum(-1).cpu().numpy(), 1.0, atol=1e-5)


# ------------------------------------------------------------------------------ K3
@pytest.mark.parametrize("T,E", [(1, 8), (16, 8), (600, 8), (4096, 8), (33, 32)])
def test_permute_stable_grouping(cuda_device, T, E):
    from moeinfra_amd import ops

    rng = np.random.default_rng(T)
    idx = np.stack([rng.choice(E, size=2, replace=False) for _ in range(T)]).astype(np.int32)
    r = ops.permute(torch.from_numpy(idx).to(cuda_device), E)
    flat = idx.reshape(-1)
    order = np.argsort(flat, kind="stable")
    counts = np.bincount(flat, minlength=E)
    np.testing.assert_array_equal(r["counts"].cpu().numpy(), counts)
    np.testing.assert_array_equal(r["offsets"].cpu().numpy(), np.concatenate([[0], np.cumsum(counts)]))
    np.testing.assert_array_equal(r["perm_tok"].cpu().numpy(), order // 2)
    pos = np.empty_like(order)
    pos[order] = np.arange(order.size)
    np.testing.assert_array_equal(r["slot_pos"].cpu().numpy(), pos)
    act = r["active"].cpu().numpy()
    present = np.nonzero(counts)[0]
    assert act[0] == present.size
    np.testing.assert_array_equal(act[1:1 + present.size], present)


# ------------------------------------------------------------------------------ K4 + K5
def _layer_case(dev, H, F, E, T, seed, skew=False, codes=None):
    from moeinfra_amd import ops, synth

    gate, experts, x = build_layer(H, F, E, T, seed, codes=codes)
    bias = synth.zipf_bias(E, seed) if skew else None
    want, (lg_w, w_w, i_w) = oracle_layer(gate, experts, x, bias=bias)
    for ex in experts:
        ex.to(dev)
    table = ops.expert_table([ex.c_struct() for ex in experts])
    out, lg, w, idx = ops.layer_forward(table, E, gate.to(dev), x.to(dev), 2, F,
                                        bias=None if bias is None else bias.to(dev),
                                        want_logits=True)
    torch.cuda.synchronize()
    # The router's logits output against the oracle's: both round an fp32 sum of the same
    # products to bf16, summed in different orders, so they may differ by the two sums'
    # distance (2 x the reordering bound of logit_slack) and one bf16 step.
    lg_g = orc.bf16_to_f32(bits(lg)).astype(np.float64)
    lg_o = orc.bf16_to_f32(lg_w).astype(np.float64)
    slack = logit_slack(bits(x), bits(gate))[:, None]
    assert (np.abs(lg_g - lg_o) <= 2.0 ** -7 * np.maximum(np.abs(lg_g), np.abs(lg_o)) + 2.0 * slack).all()
    return want, i_w, bits(out), idx.cpu().numpy(), lg_w


@pytest.mark.parametrize("H,F,E,T,seed,skew", [
    (256, 512, 8, 16, 3, False),
    (256, 512, 8, 1, 4, False),
    (1024, 3584, 8, 16, 0, False),      # the reduced Mixtral layer
    (512, 1024, 8, 37, 5, True),
    (256, 768, 4, 5, 6, False),
    (512, 1024, 8, 2, 7, False),        # <= 4 tokens per expert: 4x4x4 MFMA GEMV
    (1024, 3584, 8, 4, 8, True),
    (512, 1536, 8, 3, 9, False),
])
def test_layer_matches_oracle(cuda_device, H, F, E, T, seed, skew):
    want, i_want, got, i_got, lg = _layer_case(cuda_device, H, F, E, T, seed, skew)
    tie = near_tie_rows(lg)
    np.testing.assert_array_equal(i_got[~tie], i_want[~tie])
    ok = ~tie
    err = orc.rel_l2(orc.bf16_to_f32(got[ok]), orc.bf16_to_f32(want[ok]))
    assert err <= 1e-2, err


@pytest.mark.parametrize("H,F,T", [(512, 1024, 3), (256, 512, 12), (4096, 1024, 1), (512, 1024, 1)])
def test_layer_mixed_codebooks(cuda_device, H, F, T):
    """Experts whose codebooks differ from the first active one (per-expert fallback).  One
    token: the gate products read the workgroup's LDS copy of the token while the per-nibble
    stream reads it from global memory."""
    codes = {e: (orc.NF4_CODE * np.float32(0.75 + 0.05 * e)).astype(np.float32)
             for e in (1, 4, 6)}
    want, i_want, got, i_got, lg = _layer_case(cuda_device, H, F, 8, T, 10 + T, codes=codes)
    tie = near_tie_rows(lg)
    np.testing.assert_array_equal(i_got[~tie], i_want[~tie])
    ok = ~tie
    err = orc.rel_l2(orc.bf16_to_f32(got[ok]), orc.bf16_to_f32(want[ok]))
    assert err <= 1e-2, err


@pytest.mark.parametrize("T,H,F", [(1, 256, 512), (3, 1024, 3584), (20, 512, 768)])
def test_single_expert_matches_oracle(cuda_device, T, H, F):
    from moeinfra_amd import ops, synth

    gen = synth.make_generator(T + H)
    w1 = synth._normal((F, H), gen, "cpu", 0.02)
    w3 = synth._normal((F, H), gen, "cpu", 0.02)
    w2 = synth._normal((H, F), gen, "cpu", 0.02)
    x = synth.make_activations(T, H, gen)
    ex = NF4Expert(w1, w3, w2)
    d1, d3, d2 = ex.dequant_np()
    want = orc.swiglu(bits(x), d1, d3, d2)
    ex.to(cuda_device)
    got = ops.expert_swiglu(ex.c_struct(), x.to(cuda_device), H, F)
    err = orc.rel_l2(orc.bf16_to_f32(bits(got)), orc.bf16_to_f32(want))
    assert err <= 1e-2, err


# ------------------------------------------------------------------------------ decode layer
# Shapes that reach the branches of the two-launch decode form (T <= 4, T*k <= 8, E <= 16,
# H and F multiples of 512): 16 experts (the 16-expert kernel instantiation), an odd number
# of 4-row output tiles per workgroup in the single-token down GEMV's two-tile units
# (H = 2560: 640 tiles over 256 CUs -> 3 per workgroup), and two-token batches with 16
# experts and a skewed router.
@pytest.mark.parametrize("H,F,E,T,seed,skew", [
    (512, 1024, 16, 1, 21, False),
    (512, 1024, 16, 4, 22, False),
    (1024, 2048, 16, 2, 23, True),
    (2560, 2048, 8, 1, 24, False),
])
def test_decode_layer_branches(cuda_device, H, F, E, T, seed, skew):
    want, i_want, got, i_got, lg = _layer_case(cuda_device, H, F, E, T, seed, skew)
    tie = near_tie_rows(lg)
    np.testing.assert_array_equal(i_got[~tie], i_want[~tie])
    ok = ~tie
    err = orc.rel_l2(orc.bf16_to_f32(got[ok]), orc.bf16_to_f32(want[ok]))
    assert err <= 1e-2, err


def test_decode_single_token_long_ffn(cuda_device):
    """Single token, hidden 4096 (the single-token gate/up stream) with F = 16896: 33 items
    per workgroup on 256 CUs, more than the workgroup keeps in LDS, so the per-item
    reduction path runs.  Weights are drawn and quantised on the GPU; the oracle
    dequantises the routed experts."""
    from moeinfra_amd import ops
    from moeinfra_amd._lib import MoeNf4Expert

    H, F, E = 4096, 16896, 4
    g = torch.Generator(device=cuda_device).manual_seed(77)
    keep = []
    for e in range(E):
        st = {}
        for name, shape in (("w1", (F, H)), ("w3", (F, H)), ("w2", (H, F))):
            w = (torch.randn(shape, generator=g, device=cuda_device) * 0.02).to(torch.bfloat16)
            st[name] = ops.nf4_quantize(w)
            del w
        keep.append(st)
    gate = (torch.randn((E, H), generator=g, device=cuda_device) * 0.02).to(torch.bfloat16)
    table = ops.expert_table([MoeNf4Expert(*(t.data_ptr() for n in ("w1", "w3", "w2")
                                             for t in st[n])) for st in keep])
    x = torch.randn((1, H), generator=g, device=cuda_device).to(torch.bfloat16)
    out, _, w, idx = ops.layer_forward(table, E, gate, x, 2, F)
    torch.cuda.synchronize()

    def expert_fn(e, rows):
        st = {n: (keep[e][n][0].cpu().numpy().reshape(-1), keep[e][n][1].cpu().numpy())
              for n in ("w1", "w3", "w2")}
        return orc.swiglu(rows, *orc.dequant_expert(st, H, F, threads=8))

    want, (lg_o, w_o, idx_o) = orc.moe_layer(bits(x), bits(gate), expert_fn)
    ok = ~near_tie_rows(lg_o)
    np.testing.assert_array_equal(idx.cpu().numpy()[ok], idx_o[ok])
    err = orc.rel_l2(orc.bf16_to_f32(bits(out)[ok]), orc.bf16_to_f32(want[ok]))
    assert err <= 1e-2, err


# ------------------------------------------------------------------------------ batched GEMM
# From 32 routed rows per expert on average the layer runs the LDS-staged expert GEMM
# (expert_gemm.hip): partial 128-token tiles, uniform and skewed routing, several tiles
# per expert.
@pytest.mark.parametrize("H,F,E,T,seed,skew", [
    (512, 1024, 8, 160, 31, False),
    (256, 512, 8, 300, 32, True),     # H % 512 != 0: the per-tile kernels
    (512, 768, 8, 300, 35, True),
    (512, 1024, 4, 1100, 36, False),  # >= 512 rows per expert: 256-token items, K splits
    (512, 768, 8, 2500, 37, True),    # skewed: 128- and 256-token tiles, partial tiles
    (1024, 3584, 8, 512, 33, False),
    (1024, 3584, 8, 700, 34, True),
])
def test_layer_batched_gemm(cuda_device, H, F, E, T, seed, skew):
    want, i_want, got, i_got, lg = _layer_case(cuda_device, H, F, E, T, seed, skew)
    tie = near_tie_rows(lg)
    np.testing.assert_array_equal(i_got[~tie], i_want[~tie])
    ok = ~tie
    err = orc.rel_l2(orc.bf16_to_f32(got[ok]), orc.bf16_to_f32(want[ok]))
    assert err <= 1e-2, err


# Batched layers whose experts do not share one codebook: the GEMM rebuilds its lookup
# table per work item.  Expert 0 keeps the NF4 codebook, so the first active expert's
# table is not the one of every item.
@pytest.mark.parametrize("H,F,T", [(512, 1024, 300), (256, 512, 160), (512, 768, 160),
                                   (512, 768, 2100)])  # >= 512 rows per expert: 256-token items
def test_layer_batched_gemm_mixed_codebooks(cuda_device, H, F, T):
    codes = {e: (orc.NF4_CODE * np.float32(0.75 + 0.05 * e)).astype(np.float32)
             for e in (1, 4, 6)}
    want, i_want, got, i_got, lg = _layer_case(cuda_device, H, F, 8, T, 40 + T, codes=codes)
    tie = near_tie_rows(lg)
    np.testing.assert_array_equal(i_got[~tie], i_want[~tie])
    ok = ~tie
    err = orc.rel_l2(orc.bf16_to_f32(got[ok]), orc.bf16_to_f32(want[ok]))
    assert err <= 1e-2, err


# A layer whose table has an absent expert (all nine pointers null) that the router never
# selects (a -1e4 logit bias): every kernel family skips it.  T = 24 runs the mid-batch
# kernels, T = 300 the batched GEMM.
@pytest.mark.parametrize("T", [24, 300])
def test_layer_absent_expert(cuda_device, T):
    from moeinfra_amd import ops
    from moeinfra_amd._lib import MoeNf4Expert

    H, F, E, absent = 512, 1024, 8, 3
    gate, experts, x = build_layer(H, F, E, T, 70 + T)
    bias = torch.zeros(E, dtype=torch.float32)
    bias[absent] = -1.0e4
    want, (lg_w, w_w, i_w) = oracle_layer(gate, experts, x, bias=bias)
    assert not (i_w == absent).any()
    structs = []
    for e, ex in enumerate(experts):
        if e == absent:
            structs.append(MoeNf4Expert())
        else:
            ex.to(cuda_device)
            structs.append(ex.c_struct())
    table = ops.expert_table(structs)
    out, _, w, idx = ops.layer_forward(table, E, gate.to(cuda_device), x.to(cuda_device), 2, F,
                                       bias=bias.to(cuda_device))
    torch.cuda.synchronize()
    ok = ~near_tie_rows(lg_w, bias=bias.numpy())
    np.testing.assert_array_equal(idx.cpu().numpy()[ok], i_w[ok])
    err = orc.rel_l2(orc.bf16_to_f32(bits(out)[ok]), orc.bf16_to_f32(want[ok]))
    assert err <= 1e-2, err


# ------------------------------------------------------------------------------ mid-size batches
# Between the decode form (T <= 4) and the batched GEMM (>= 32 routed rows per expert on
# average), outside the mid-size kernels' shapes (H 2048 / 4096, up to 64 tokens; those are
# below), the layer runs the mid-batch kernels: the streamed form (expert_midbatch.hip;
# H and F multiples of 512, K splits of the down projection when few experts are active)
# or, for other shapes, the K-split form (expert_skinny.hip; F = 768 here).  32-token
# chunks per expert (a hot expert under skewed routing takes several), uniform and skewed
# routing.
@pytest.mark.parametrize("H,F,E,T,seed,skew", [
    (512, 1024, 8, 6, 51, False),
    (512, 768, 8, 9, 52, True),
    (1024, 2048, 8, 64, 53, False),
    (512, 1024, 8, 100, 54, True),
    (1024, 3584, 8, 40, 55, True),
])
def test_layer_mid_batch(cuda_device, H, F, E, T, seed, skew):
    want, i_want, got, i_got, lg = _layer_case(cuda_device, H, F, E, T, seed, skew)
    tie = near_tie_rows(lg)
    np.testing.assert_array_equal(i_got[~tie], i_want[~tie])
    ok = ~tie
    err = orc.rel_l2(orc.bf16_to_f32(got[ok]), orc.bf16_to_f32(want[ok]))
    assert err <= 1e-2, err


# One expert takes every token (a +1e4 selection bias): 120 rows, four 32-token chunks of
# the streamed kernels, with the down projection split over K (H = 1024, F = 2048).
def test_layer_mid_batch_hot_expert(cuda_device):
    from moeinfra_amd import ops

    H, F, E, T, hot = 1024, 2048, 8, 120, 5
    gate, experts, x = build_layer(H, F, E, T, 56)
    bias = torch.zeros(E, dtype=torch.float32)
    bias[hot] = 1.0e4
    want, (lg_w, w_w, i_w) = oracle_layer(gate, experts, x, bias=bias)
    assert (i_w == hot).any(axis=1).all()
    for ex in experts:
        ex.to(cuda_device)
    table = ops.expert_table([ex.c_struct() for ex in experts])
    out, _, w, idx = ops.layer_forward(table, E, gate.to(cuda_device), x.to(cuda_device), 2, F,
                                       bias=bias.to(cuda_device))
    torch.cuda.synchronize()
    ok = ~near_tie_rows(lg_w, bias=bias.numpy())
    np.testing.assert_array_equal(idx.cpu().numpy()[ok], i_w[ok])
    err = orc.rel_l2(orc.bf16_to_f32(bits(out)[ok]), orc.bf16_to_f32(want[ok]))
    assert err <= 1e-2, err


def test_layer_mid_batch_mixed_codebooks(cuda_device):
    """Mid-batch layer whose experts do not share one codebook: the kernels rebuild the
    lookup table at the work items whose codebooks differ."""
    codes = {e: (orc.NF4_CODE * np.float32(0.75 + 0.05 * e)).astype(np.float32)
             for e in (1, 4, 6)}
    want, i_want, got, i_got, lg = _layer_case(cuda_device, 512, 1024, 8, 24, 56, codes=codes)
    tie = near_tie_rows(lg)
    np.testing.assert_array_equal(i_got[~tie], i_want[~tie])
    ok = ~tie
    err = orc.rel_l2(orc.bf16_to_f32(got[ok]), orc.bf16_to_f32(want[ok]))
    assert err <= 1e-2, err


@pytest.mark.parametrize("T,skew", [(16, False), (32, True)])
def test_layer_mid_batch_mixtral(cuda_device, T, skew):
    """Full Mixtral-8x7B expert shapes (hidden 4096, FFN 14336) at decode batches 16 and 32:
    weights drawn and quantised on the GPU, the oracle dequantises the routed experts."""
    from moeinfra_amd import ops, synth
    from moeinfra_amd._lib import MoeNf4Expert

    H, F, E = 4096, 14336, 8
    g = torch.Generator(device=cuda_device).manual_seed(600 + T)
    keep = []
    for e in range(E):
        st = {}
        for name, shape in (("w1", (F, H)), ("w3", (F, H)), ("w2", (H, F))):
            w = (torch.randn(shape, generator=g, device=cuda_device) * 0.02).to(torch.bfloat16)
            st[name] = ops.nf4_quantize(w)
            del w
        keep.append(st)
    gate = (torch.randn((E, H), generator=g, device=cuda_device) * 0.02).to(torch.bfloat16)
    table = ops.expert_table([MoeNf4Expert(*(t.data_ptr() for n in ("w1", "w3", "w2")
                                             for t in st[n])) for st in keep])
    x = torch.randn((T, H), generator=g, device=cuda_device).to(torch.bfloat16)
    bias = synth.zipf_bias(E, T).to(cuda_device) if skew else None
    out, _, w, idx = ops.layer_forward(table, E, gate, x, 2, F, bias=bias)
    torch.cuda.synchronize()
    cache = {}

    def expert_fn(e, rows):
        if e not in cache:
            st = {n: (keep[e][n][0].cpu().numpy().reshape(-1), keep[e][n][1].cpu().numpy())
                  for n in ("w1", "w3", "w2")}
            cache[e] = orc.dequant_expert(st, H, F, threads=8)
        return orc.swiglu(rows, *cache[e])

    b = None if bias is None else bias.cpu().numpy()
    want, (lg_o, w_o, idx_o) = orc.moe_layer(bits(x), bits(gate), expert_fn, bias=b)
    ok = ~near_tie_rows(lg_o, bias=b)
    np.testing.assert_array_equal(idx.cpu().numpy()[ok], idx_o[ok])
    err = orc.rel_l2(orc.bf16_to_f32(bits(out)[ok]), orc.bf16_to_f32(want[ok]))
    assert err <= 1e-2, err


# ------------------------------------------------------------------------------ mid-size gate/up
# 5 to 64 tokens at hidden size 2048 or 4096: 16-row weight tiles on the 16x16x32 MFMA, one
# virtual expert (<= 16 rows of one expert, each wave's K slice of them in registers) per
# workgroup; an expert with more rows is several virtual experts, which read its tiles side
# by side.  Up to 16 tokens every workgroup routes the tokens itself.  Hidden 2048 here
# (the Mixtral shape is in the full-shape tests).
def _check_layer(want, i_want, got, i_got, lg, bias=None):
    tie = near_tie_rows(lg, bias=bias)
    np.testing.assert_array_equal(i_got[~tie], i_want[~tie])
    err = orc.rel_l2(orc.bf16_to_f32(got[~tie]), orc.bf16_to_f32(want[~tie]))
    assert err <= 1e-2, err


# F a multiple of 2048 also takes the mid-size down projection (virtual experts over parts
# of 2048 values of F, one fp32 plane per part; 1 and 2 parts here).  Above 16 tokens the
# gate/up launch groups the slots of a separate router launch (up to 128 slots: T = 64,
# k = 2), and experts with more than 16 rows split into several virtual experts.
@pytest.mark.parametrize("H,F,E,T,seed,skew", [
    (2048, 1024, 8, 24, 95, False),
    (2048, 2048, 16, 40, 96, True),
    (2048, 1024, 8, 64, 97, True),
    (4096, 2048, 8, 33, 98, True),
    (2048, 1024, 8, 5, 81, False),
    (2048, 1536, 8, 12, 82, True),
    (2048, 1024, 8, 16, 83, False),
    (2048, 512, 4, 11, 84, False),     # four experts: most hold more than 4 rows, some > 8
    (2048, 768, 16, 16, 85, True),
    (2048, 2048, 8, 7, 91, False),
    (2048, 4096, 8, 16, 92, True),
    (4096, 4096, 4, 13, 93, False),
])
def test_layer_mid_gateup(cuda_device, H, F, E, T, seed, skew):
    _check_layer(*_layer_case(cuda_device, H, F, E, T, seed, skew))


def test_expert_ffn_mid_size_external_route(cuda_device):
    """The mid-size kernels behind the generic entry points (router and grouping launched
    apart, as MoELayer's offload path does): gate/up from the given grouping, the down
    projection into the library's default number of planes, then the combine."""
    from moeinfra_amd import ops

    H, F, E, T = 2048, 4096, 8, 14
    gate, experts, x = build_layer(H, F, E, T, 94)
    want, (lg_w, w_w, i_w) = oracle_layer(gate, experts, x)
    for ex in experts:
        ex.to(cuda_device)
    table = ops.expert_table([ex.c_struct() for ex in experts])
    xd = x.to(cuda_device)
    idx32 = torch.empty((T, 2), dtype=torch.int32, device=cuda_device)
    _, w, idx = ops.router_topk(xd, gate.to(cuda_device), 2, want_logits=False, idx32_out=idx32)
    route = ops.permute(idx32, E)
    assert ops.choose_nsplit(T, 2, E, H, F) == 2
    _, ypart = ops.expert_ffn(table, E, xd, 2, H, F, route)
    out = ops.combine(ypart, w, idx32, route["slot_pos"])
    torch.cuda.synchronize()
    _check_layer(want, i_w, bits(out), idx.cpu().numpy(), lg_w)


def test_layer_mid_gateup_mixed_codebooks(cuda_device):
    """Each workgroup builds its table from its own expert's w1 / w3 codebooks."""
    codes = {e: (orc.NF4_CODE * np.float32(0.75 + 0.05 * e)).astype(np.float32)
             for e in (1, 4, 6)}
    _check_layer(*_layer_case(cuda_device, 2048, 1024, 8, 14, 86, codes=codes))


@pytest.mark.parametrize("T", [9, 16])
def test_layer_mid_gateup_hot_and_absent(cuda_device, T):
    """One expert takes every token (+1e4 bias: 9 or 16 rows, two virtual experts, the
    second of 1 or 8 rows) and one is absent from the table (-1e4: never routed)."""
    from moeinfra_amd import ops
    from moeinfra_amd._lib import MoeNf4Expert

    H, F, E, hot, absent = 2048, 2048, 8, 2, 6
    gate, experts, x = build_layer(H, F, E, T, 87 + T)
    bias = torch.zeros(E, dtype=torch.float32)
    bias[hot], bias[absent] = 1.0e4, -1.0e4
    want, (lg_w, w_w, i_w) = oracle_layer(gate, experts, x, bias=bias)
    assert (i_w == hot).any(axis=1).all() and not (i_w == absent).any()
    structs = []
    for e, ex in enumerate(experts):
        if e == absent:
            structs.append(MoeNf4Expert())
        else:
            ex.to(cuda_device)
            structs.append(ex.c_struct())
    table = ops.expert_table(structs)
    out, _, w, idx = ops.layer_forward(table, E, gate.to(cuda_device), x.to(cuda_device), 2, F,
                                       bias=bias.to(cuda_device))
    torch.cuda.synchronize()
    _check_layer(want, i_w, bits(out), idx.cpu().numpy(), lg_w, bias=bias.numpy())


def test_layer_mid_many_experts_hot(cuda_device):
    """32 experts at 64 tokens: one expert takes every token (+1e4 bias: 64 rows, four
    virtual experts that read its tiles side by side), the other 31 share the second slots
    (one virtual expert each); gate/up and down both on the mid-size kernels (F = 2048: one
    part), so the workgroups are dealt to 35 virtual experts of very different experts."""
    from moeinfra_amd import ops

    H, F, E, T, hot = 2048, 2048, 32, 64, 3
    gate, experts, x = build_layer(H, F, E, T, 131)
    bias = torch.zeros(E, dtype=torch.float32)
    bias[hot] = 1.0e4
    want, (lg_w, w_w, i_w) = oracle_layer(gate, experts, x, bias=bias)
    assert (i_w == hot).any(axis=1).all()
    assert ops.choose_nsplit(T, 2, E, H, F) == 1  # the mid-size down projection's one part
    for ex in experts:
        ex.to(cuda_device)
    table = ops.expert_table([ex.c_struct() for ex in experts])
    out, _, w, idx = ops.layer_forward(table, E, gate.to(cuda_device), x.to(cuda_device), 2, F,
                                       bias=bias.to(cuda_device))
    torch.cuda.synchronize()
    _check_layer(want, i_w, bits(out), idx.cpu().numpy(), lg_w, bias=bias.numpy())


def test_mid_down_needs_a_workgroup_per_pair(cuda_device):
    """The mid-size down projection gives every (virtual expert, part of 2048 values of F)
    pair a workgroup of its own: at 64 tokens, top-2 and F = 14336 (7 parts), 8 experts
    (at most 16 virtual experts, 112 pairs) take it, 32 experts (up to 40 virtual experts,
    280 pairs) take another path."""
    from moeinfra_amd import ops

    cus = torch.cuda.get_device_properties(cuda_device).multi_processor_count
    assert ops.choose_nsplit(64, 2, 8, 2048, 14336) == 7
    if (32 + 64 * 2 // 16) * 7 > cus:
        assert ops.choose_nsplit(64, 2, 32, 2048, 14336) != 7
