"""Shared test helpers: oracle-quantised NF4 experts, device staging, bf16 bit views."""
from __future__ import annotations

import numpy as np
import torch

from oracle import moe_oracle as orc


def bits(t: torch.Tensor) -> np.ndarray:
    """bf16 tensor (any device) -> numpy uint16 bit patterns."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def from_bits(a: np.ndarray, device="cpu") -> torch.Tensor:
    a = np.ascontiguousarray(a, dtype=np.uint16)
    return torch.from_numpy(a.view(np.int16)).view(torch.bfloat16).to(device)


def quantize_np(w: torch.Tensor):
    """bf16 CPU tensor -> (packed uint8 [n/2], absmax fp32) with the oracle quantiser."""
    return orc.nf4_quantize(bits(w).reshape(-1))


class NF4Expert:
    """One expert quantised on the CPU by the oracle: numpy state + device copies."""

    def __init__(self, w1: torch.Tensor, w3: torch.Tensor, w2: torch.Tensor, code=None):
        self.inter, self.hidden = w1.shape
        self.code = orc.NF4_CODE if code is None else np.asarray(code, dtype=np.float32)
        q = lambda w: orc.nf4_quantize(bits(w).reshape(-1), code=self.code)
        self.np = {"w1": q(w1), "w3": q(w3), "w2": q(w2)}
        self.dev = None

    def to(self, device):
        code = torch.from_numpy(self.code.copy()).to(device)
        self.dev = {}
        for name, (p, a) in self.np.items():
            self.dev[name] = (torch.from_numpy(p.copy()).to(device),
                              torch.from_numpy(a.copy()).to(device), code.clone())
        return self

    def c_struct(self):
        from moeinfra_amd._lib import MoeNf4Expert

        d = self.dev
        return MoeNf4Expert(
            d["w1"][0].data_ptr(), d["w1"][1].data_ptr(), d["w1"][2].data_ptr(),
            d["w3"][0].data_ptr(), d["w3"][1].data_ptr(), d["w3"][2].data_ptr(),
            d["w2"][0].data_ptr(), d["w2"][1].data_ptr(), d["w2"][2].data_ptr(),
        )

    def dequant_np(self):
        return orc.dequant_expert(self.np, self.hidden, self.inter, code=self.code)


def build_layer(hidden: int, inter: int, num_experts: int, tokens: int, seed: int,
                codes=None):
    """Seeded layer (gate, NF4 experts quantised by the oracle, activations), CPU-side.
    ``codes`` optionally maps expert id -> a codebook to use instead of NF4."""
    from moeinfra_amd import synth

    codes = codes or {}
    gen = synth.make_generator(seed)
    lw = synth.make_layer(hidden, inter, num_experts, gen,
                          expert_sink=lambda e, w1, w3, w2: NF4Expert(w1, w3, w2, codes.get(e)))
    x = synth.make_activations(tokens, hidden, gen)
    return lw.gate, lw.experts, x


def oracle_layer(gate: torch.Tensor, experts, x: torch.Tensor, k: int = 2, bias=None):
    """Oracle MoE layer output (bf16 bits) and routing for oracle-quantised experts."""
    cache = {}

    def expert_fn(e, rows):
        if e not in cache:
            cache[e] = experts[e].dequant_np()
        w1, w3, w2 = cache[e]
        return orc.swiglu(rows, w1, w3, w2)

    b = None if bias is None else bias.detach().cpu().numpy()
    return orc.moe_layer(bits(x), bits(gate), expert_fn, k=k, bias=b)


def near_tie_rows(logits_bits: np.ndarray, bias=None, k: int = 2, slack=None) -> np.ndarray:
    """Rows whose k-th and (k+1)-th largest fp32 logits are within 1 bf16 ulp, plus
    ``slack`` (scalar or per row: the reordering error of the fp32 dot products behind the
    logits, which two implementations may sum in different orders)."""
    lf = orc.bf16_to_f32(logits_bits).astype(np.float64)
    if bias is not None:
        lf = lf + np.asarray(bias, dtype=np.float64)[None, :]
    s = -np.sort(-lf, axis=-1)
    if s.shape[1] <= k:
        return np.zeros(s.shape[0], dtype=bool)
    gap = s[:, k - 1] - s[:, k]
    ulp = np.maximum(np.abs(s[:, k - 1]), 1e-30) * 2.0 ** -7
    if slack is not None:
        ulp = ulp + 2.0 * np.asarray(slack, dtype=np.float64)
    return gap <= ulp


def logit_slack(x_bits: np.ndarray, gate_bits: np.ndarray) -> np.ndarray:
    """Per token: 2^-18 * max_e sum_h |x_h g_eh|, a bound on how far two fp32 summation
    orders of the router's dot products (H <= 8192 terms) can land apart."""
    xa = np.abs(orc.bf16_to_f32(x_bits).astype(np.float64))
    ga = np.abs(orc.bf16_to_f32(gate_bits).astype(np.float64))
    return 2.0 ** -18 * (xa @ ga.T).max(axis=-1)


def assert_weights_close(w_got, w_want, lg_got_bits, lg_want_bits, rtol=1e-5, atol=1e-6):
    """Routing weights: fp32 softmax rounding where a row's bf16 logits equal the oracle's;
    elsewhere the logit difference propagates (a renormalised softmax moves by at most
    half of it)."""
    dl = np.abs(orc.bf16_to_f32(lg_got_bits).astype(np.float64) -
                orc.bf16_to_f32(lg_want_bits).astype(np.float64)).max(axis=-1, keepdims=True)
    w_got, w_want = np.asarray(w_got, np.float64), np.asarray(w_want, np.float64)
    assert (np.abs(w_got - w_want) <= rtol * np.abs(w_want) + atol + 0.5 * dl).all()


def record_parity(**fields) -> None:
    """Appends one JSON line of measured parity figures (test, config, rel-L2, ...) to the
    file named by $MOE_PARITY_LOG, when set; a no-op otherwise."""
    import json
    import os

    path = os.environ.get("MOE_PARITY_LOG")
    if not path:
        return
    with open(path, "a") as f:
        f.write(json.dumps(fields, sort_keys=True) + "\n")


def dequant_code_scaled(packed: np.ndarray, absmax: np.ndarray, numel: int, code=None) -> np.ndarray:
    """float32 weights bf16(code[q]) * absmax[block] (an fp32 product, not rounded): the
    effective weights of the decode, GEMV and mid-batch kernels, which round the codebook
    value to bf16 and apply the block's absmax to fp32 partial sums.  A measuring device
    for how much of a kernel's distance to the oracle (whose weights are
    bf16(code * absmax), as the reference materialises them) comes from that weight form
    rather than from summation order."""
    code = orc.NF4_CODE if code is None else np.asarray(code, dtype=np.float32)
    cb = orc.bf16_to_f32(orc.bf16_round(code))
    p = np.asarray(packed, dtype=np.uint8).reshape(-1)
    q = np.empty(2 * p.size, dtype=np.uint8)
    q[0::2] = p >> 4
    q[1::2] = p & 15
    blk = np.repeat(np.asarray(absmax, dtype=np.float32).reshape(-1), orc.NF4_BLOCKSIZE)
    return (cb[q[:numel]] * blk[:numel]).astype(np.float32)
