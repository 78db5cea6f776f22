"""Pins of the NF4 oracle (oracle/nf4_oracle.c, oracle/moe_oracle.py) -- CPU only.

Each check compares the oracle against something it does not share code with: the NF4
codebook's published construction, closed forms, torch's float32 multiply and bfloat16
conversion, or brute force.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import moe_oracle as orc


def test_codebook_matches_normal_quantile_construction():
    """NF4 (QLoRA, Dettmers et al. 2023): 8 positive and 7 negative normal quantiles
    between offset 0.9677083 and 0.5, plus an exact zero, normalised to [-1, 1]."""
    from scipy.stats import norm

    offset = 0.9677083
    pos = norm.ppf(np.linspace(offset, 0.5, 9)[:-1])
    neg = -norm.ppf(np.linspace(offset, 0.5, 8)[:-1])
    v = np.sort(np.concatenate([pos, [0.0], neg]))
    v = v / np.abs(v).max()
    np.testing.assert_allclose(orc.NF4_CODE.astype(np.float64), v, rtol=0, atol=2e-7)
    assert orc.NF4_CODE[7] == 0.0 and orc.NF4_CODE[0] == -1.0 and orc.NF4_CODE[15] == 1.0
    assert np.all(np.diff(orc.NF4_CODE) > 0)


def test_product_codebook_equals_oracle_codebook():
    from moeinfra_amd.nf4 import NF4_CODE_VALUES

    np.testing.assert_array_equal(np.array(NF4_CODE_VALUES, dtype=np.float32), orc.NF4_CODE)


@pytest.mark.parametrize("seed", [0, 1])
def test_bf16_rounding_matches_torch(seed):
    rng = np.random.default_rng(seed)
    f = np.concatenate([
        rng.standard_normal(4096).astype(np.float32) * 10.0 ** rng.integers(-6, 6, 4096),
        np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-40, -3e-39, 3.4e38, 65504.0],
                 dtype=np.float32),
        # exact ties at the rounding boundary (low 16 bits 0x8000)
        (np.arange(64, dtype=np.uint32) << 16 | 0x8000).view(np.float32) * np.float32(1.0),
    ]).astype(np.float32)
    want = torch.from_numpy(f).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = orc.bf16_round(f)
    finite = ~np.isnan(f)
    np.testing.assert_array_equal(got[finite], want[finite])
    assert np.all(got[~finite] == 0x7FC0)
    lib = orc.lib()
    for v, w in zip(f[finite][:200], want[finite][:200]):
        assert lib.oracle_bf16_rne(float(v)) == w


def test_dequant_closed_forms_and_nibble_order():
    """Byte 0xF0 is (code[15], code[0]); absmax 1 gives bf16(code) for every byte value."""
    packed = np.arange(256, dtype=np.uint8)
    absmax = np.ones(8, dtype=np.float32)
    out = orc.nf4_dequant(packed, absmax)
    hi, lo = packed >> 4, packed & 15
    np.testing.assert_array_equal(out[0::2], orc.bf16_round(orc.NF4_CODE[hi]))
    np.testing.assert_array_equal(out[1::2], orc.bf16_round(orc.NF4_CODE[lo]))
    a = np.float32(0.0371)
    one = orc.nf4_dequant(np.array([0xF0, 0x7F], np.uint8), np.array([a], np.float32), numel=4)
    np.testing.assert_array_equal(one, orc.bf16_round(np.array([a, -a, 0.0, a], np.float32)))


def test_dequant_matches_torch_float32_multiply():
    rng = np.random.default_rng(3)
    n = 64 * 257 + 32
    packed = rng.integers(0, 256, n // 2, dtype=np.uint8)
    absmax = (rng.random((n + 63) // 64, dtype=np.float32) * 0.2).astype(np.float32)
    q = np.empty(n, dtype=np.int64)
    q[0::2], q[1::2] = packed >> 4, packed & 15
    code = torch.from_numpy(orc.NF4_CODE.copy())
    blocks = torch.from_numpy(absmax)[torch.arange(n) // 64]
    want = (code[torch.from_numpy(q)] * blocks).to(torch.bfloat16)
    got = orc.nf4_dequant(packed, absmax, numel=n)
    np.testing.assert_array_equal(got, want.view(torch.int16).numpy().view(np.uint16))


def _bf16_normal(n, seed, std=0.02):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(n, generator=g) * std).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def test_quantize_is_nearest_code_by_brute_force():
    w = _bf16_normal(64 * 64, 5)
    packed, absmax = orc.nf4_quantize(w)
    q = np.empty(w.size, dtype=np.int64)
    q[0::2], q[1::2] = packed >> 4, packed & 15
    x = orc.bf16_to_f32(w) * (np.float32(1.0) / np.repeat(absmax, 64))
    dist = np.abs(x[:, None].astype(np.float64) - orc.NF4_CODE[None, :].astype(np.float64))
    best = dist.argmin(axis=1)
    second = np.sort(dist, axis=1)[:, 1]
    clear = (second - dist.min(axis=1)) > 1e-6
    np.testing.assert_array_equal(q[clear], best[clear])
    np.testing.assert_array_equal(absmax, np.abs(orc.bf16_to_f32(w)).reshape(-1, 64).max(axis=1))


def test_quantize_dequantize_idempotent_and_bounded():
    w = _bf16_normal(64 * 100 + 6, 9)
    w[:64] = 0  # an all-zero block
    p1, a1 = orc.nf4_quantize(w)
    d1 = orc.nf4_dequant(p1, a1, numel=w.size)
    p2, a2 = orc.nf4_quantize(d1)
    np.testing.assert_array_equal(p2, p1)
    np.testing.assert_array_equal(a2, a1)
    assert np.all(np.abs(orc.bf16_to_f32(d1)) <= np.repeat(a1, 64)[: w.size] * (1 + 2 ** -8))
    assert np.all(p1[:32] == 0x77) and a1[0] == 0.0  # zero block -> code 7 (0.0)


def test_threaded_dequant_equals_single_thread():
    rng = np.random.default_rng(4)
    n = 64 * 1000
    packed = rng.integers(0, 256, n // 2, dtype=np.uint8)
    absmax = rng.random(n // 64, dtype=np.float32)
    np.testing.assert_array_equal(orc.nf4_dequant(packed, absmax, threads=7),
                                  orc.nf4_dequant(packed, absmax))
