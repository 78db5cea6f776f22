"""CPU oracle for the MoE expert-execution path (numpy + the C NF4 restatement).

TEST INFRASTRUCTURE ONLY.  The product package ``moeinfra_amd`` never imports this
module; only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, and only as the checker.

Each function restates one piece of the reference (ParshwaPatel-07/MoEInfra) and cites
the file:line it follows:

* ``nf4_dequant`` / ``nf4_quantize``: ``oracle/nf4_oracle.c`` (bitsandbytes NF4 arithmetic
  behind ``transfer/nf4_reconstruct.py:17-114`` and ``model/expert.py:32-63``).
* ``router``: ``engine/router.py:50-94`` (gate linear -> fp32 softmax -> top-k -> renorm).
* ``moe_layer`` / ``dispatch``: ``model/moe_layer.py:142-191`` (ascending-expert dispatch,
  fp32 product, bf16 destination rounded after every add).
* ``swiglu``: ``transfer/nf4_reconstruct.py:152-155`` / ``model/expert.py:65-75``
  (``w2(silu(w1 x) * w3 x)`` with bf16 tensors between the ops).

Numbers are carried as raw bf16 bit patterns (``np.uint16``) so that every rounding
step is explicit.

Pinning (see tests/test_oracle_*.py): the codebook is rebuilt from its normal-quantile
construction; dequant is checked against closed forms and an independent torch
float32-multiply + bf16 conversion; the router against torch's own ``F.linear`` /
``F.softmax`` / ``topk`` (the calls the reference makes) and the closed form
``w0 = 1 / (1 + exp(l1 - l0))``; dispatch/combine against the fake-expert closed form
``out[t] = x[t] * sum_k w[t,k] * (idx[t,k] + 1)`` of the reference's
tests/test_moe_layer.py:180-266 setup; SwiGLU against a permutation-matrix closed form
and a torch float32 matmul.  Parity unpinned: the bitsandbytes storage format details
listed in nf4_oracle.c.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from typing import Callable, Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_nf4.so")

#: The 16-level NF4 codebook (QLoRA, Dettmers et al. 2023; bitsandbytes' NF4 table).
NF4_CODE = np.array(
    [
        -1.0,
        -0.6961928009986877,
        -0.5250730514526367,
        -0.39491748809814453,
        -0.28444138169288635,
        -0.18477343022823334,
        -0.09105003625154495,
        0.0,
        0.07958029955625534,
        0.16093020141124725,
        0.24611230194568634,
        0.33791524242401123,
        0.44070982933044434,
        0.5626170039176941,
        0.7229568362236023,
        1.0,
    ],
    dtype=np.float32,
)

NF4_BLOCKSIZE = 64

_lib: Optional[ctypes.CDLL] = None


def build() -> str:
    """Compile ``liboracle_nf4.so`` with the Makefile next to this file."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        l = ctypes.CDLL(_LIB_PATH)
        l.oracle_bf16_rne.argtypes = [ctypes.c_float]
        l.oracle_bf16_rne.restype = ctypes.c_uint16
        l.oracle_nf4_dequant.argtypes = [
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
            ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p,
        ]
        l.oracle_nf4_dequant.restype = ctypes.c_int
        l.oracle_nf4_quantize.argtypes = [
            ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p,
            ctypes.c_void_p, ctypes.c_void_p,
        ]
        l.oracle_nf4_quantize.restype = ctypes.c_int
        _lib = l
    return _lib


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


# --------------------------------------------------------------------------- bf16
def bf16_round(a) -> np.ndarray:
    """float32 -> bf16 bit patterns, round to nearest even, NaN -> 0x7FC0."""
    f = np.ascontiguousarray(np.asarray(a, dtype=np.float32))
    u = f.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(f)
    if nan.any():
        r = np.where(nan, np.uint16(0x7FC0), r)
    return r


def bf16_to_f32(u) -> np.ndarray:
    u = np.ascontiguousarray(np.asarray(u, dtype=np.uint16))
    return (u.astype(np.uint32) << 16).view(np.float32)


# --------------------------------------------------------------------------- NF4
def nf4_dequant(packed: np.ndarray, absmax: np.ndarray, code: np.ndarray = NF4_CODE,
                numel: Optional[int] = None, blocksize: int = NF4_BLOCKSIZE,
                threads: int = 1) -> np.ndarray:
    """Packed NF4 -> bf16 bit patterns (flat) via nf4_oracle.c:oracle_nf4_dequant, optionally
    split over ``threads`` host threads (the C call releases the GIL)."""
    packed = np.ascontiguousarray(packed, dtype=np.uint8).reshape(-1)
    absmax = np.ascontiguousarray(absmax, dtype=np.float32).reshape(-1)
    code = np.ascontiguousarray(code, dtype=np.float32).reshape(-1)
    if numel is None:
        numel = packed.size * 2
    assert packed.size * 2 >= numel and absmax.size * blocksize >= numel and code.size == 16
    out = np.empty(numel, dtype=np.uint16)
    threads = max(1, int(threads))
    # Chunks start on quantisation-block boundaries so each call sees whole blocks.
    step = -(-numel // threads)
    step = -(-step // (2 * blocksize)) * (2 * blocksize)
    chunks = [(s, min(numel, s + step)) for s in range(0, numel, step)] or [(0, 0)]

    def run(lo_hi):
        lo, hi = lo_hi
        return lib().oracle_nf4_dequant(
            packed.ctypes.data + lo // 2, absmax.ctypes.data + (lo // blocksize) * 4,
            _ptr(code), hi - lo, blocksize, out.ctypes.data + lo * 2)

    if len(chunks) == 1:
        rcs = [run(chunks[0])]
    else:
        from concurrent.futures import ThreadPoolExecutor

        with ThreadPoolExecutor(max_workers=len(chunks)) as pool:
            rcs = list(pool.map(run, chunks))
    if any(rc != 0 for rc in rcs):
        raise ValueError("oracle_nf4_dequant rejected its arguments")
    return out


def nf4_quantize(w_bf16: np.ndarray, code: np.ndarray = NF4_CODE,
                 blocksize: int = NF4_BLOCKSIZE) -> tuple[np.ndarray, np.ndarray]:
    """bf16 bit patterns -> (packed uint8 [n/2], absmax fp32 [ceil(n/bs)])."""
    w = np.ascontiguousarray(w_bf16, dtype=np.uint16).reshape(-1)
    code = np.ascontiguousarray(code, dtype=np.float32)
    n = w.size
    packed = np.empty(n // 2, dtype=np.uint8)
    absmax = np.empty((n + blocksize - 1) // blocksize, dtype=np.float32)
    rc = lib().oracle_nf4_quantize(_ptr(w), n, blocksize, _ptr(code), _ptr(packed), _ptr(absmax))
    if rc != 0:
        raise ValueError("oracle_nf4_quantize rejected its arguments")
    return packed, absmax


# --------------------------------------------------------------------------- router
def router(x: np.ndarray, gate: np.ndarray, k: int = 2, bias: Optional[np.ndarray] = None):
    """Restates ExpertRouter.route_with_logits (engine/router.py:50-94).

    x: bf16 bits [T,H]; gate: bf16 bits [E,H]; bias: optional fp32 [E] added to the
    fp32 logits before the softmax (the Zipf-skew variant; the reference has no bias).
    Returns (logits bf16 bits [T,E], weights fp32 [T,k], indices int64 [T,k]).
    Ties in probability are ordered by ascending expert index.
    """
    xf = bf16_to_f32(x).astype(np.float64)
    gf = bf16_to_f32(gate).astype(np.float64)
    logits = bf16_round((xf @ gf.T).astype(np.float32))          # F.linear -> bf16 (:66-69)
    lf = bf16_to_f32(logits)                                     # .float() (:81-84)
    if bias is not None:
        lf = (lf + np.asarray(bias, dtype=np.float32)[None, :]).astype(np.float32)
    m = lf.max(axis=-1, keepdims=True)
    e = np.exp((lf - m).astype(np.float32)).astype(np.float32)
    p = (e / e.sum(axis=-1, keepdims=True, dtype=np.float32)).astype(np.float32)
    order = np.argsort(-p, axis=-1, kind="stable")[:, :k]        # topk (:86-90)
    w = np.take_along_axis(p, order, axis=-1).astype(np.float32)
    w = (w / w.sum(axis=-1, keepdims=True, dtype=np.float32)).astype(np.float32)  # (:92)
    return logits, w, order.astype(np.int64)


def predict_next_layer_experts(indices: np.ndarray) -> list[int]:
    """engine/router.py:96-105: the sorted set of expert ids seen in ``indices``."""
    return sorted(int(v) for v in np.unique(np.asarray(indices).reshape(-1)))


# --------------------------------------------------------------------------- dispatch
def dispatch(idx: np.ndarray, w: np.ndarray, num_experts: int):
    """model/moe_layer.py:150-183.  Per routed expert (ascending): its tokens in ascending
    order and their combined weight sum_k w[t,k]*[idx[t,k]==e] (fp32)."""
    out = []
    for e in sorted(int(v) for v in np.unique(idx)):
        match = idx == e
        mask = match.any(axis=-1)
        tw = (w * match.astype(np.float32)).sum(axis=-1, dtype=np.float32).astype(np.float32)
        out.append((e, np.nonzero(mask)[0], tw[mask]))
    return out


def combine_add(out_bits: np.ndarray, y_bits: np.ndarray, tw: np.ndarray) -> np.ndarray:
    """``out[mask] += y * w`` (model/moe_layer.py:187-191): the fp32 product is added in
    fp32 to the bf16 destination and the sum is rounded back to bf16."""
    prod = (bf16_to_f32(y_bits) * tw[:, None].astype(np.float32)).astype(np.float32)
    return bf16_round((bf16_to_f32(out_bits) + prod).astype(np.float32))


def moe_layer(x: np.ndarray, gate: np.ndarray, expert_fn: Callable[[int, np.ndarray], np.ndarray],
              k: int = 2, bias: Optional[np.ndarray] = None):
    """MoELayer._forward_tokens (model/moe_layer.py:117-211) on bf16 bits.

    ``expert_fn(e, x_rows_bits) -> y_rows_bits`` runs expert ``e`` on its gathered rows.
    Returns (out bf16 bits [T,H], (logits, w, idx)).
    """
    logits, w, idx = router(x, gate, k=k, bias=bias)
    out = np.zeros_like(x, dtype=np.uint16)                          # zeros_like (:147)
    for e, tokens, tw in dispatch(idx, w, gate.shape[0]):
        y = expert_fn(e, x[tokens])                                   # (:185-186)
        out[tokens] = combine_add(out[tokens], y, tw)                 # (:187-191)
    return out, (logits, w, idx)


# --------------------------------------------------------------------------- expert
def silu_f32(g: np.ndarray) -> np.ndarray:
    g = g.astype(np.float32)
    return (g / (np.float32(1.0) + np.exp(-g))).astype(np.float32)


def swiglu(x: np.ndarray, w1: np.ndarray, w3: np.ndarray, w2: np.ndarray) -> np.ndarray:
    """y = w2( silu(w1 x) * (w3 x) ) on bf16 bits, fp32 accumulation, bf16 between ops.

    x [n,H]; w1, w3 [F,H]; w2 [H,F] (dequantised bf16 bits).  Follows
    transfer/nf4_reconstruct.py:152-155: each linear returns the activation dtype (bf16),
    ``F.silu`` and ``*`` are bf16 ops computed in fp32 and rounded.
    """
    return swiglu_f32(x, bf16_to_f32(w1), bf16_to_f32(w3), bf16_to_f32(w2))


def swiglu_f32(x: np.ndarray, w1f: np.ndarray, w3f: np.ndarray, w2f: np.ndarray) -> np.ndarray:
    """``swiglu`` with the dequantised weights already widened to float32 (each bf16 value
    exactly), so that a caller running one expert many times converts them once."""
    xf = bf16_to_f32(x)
    g = bf16_round(xf @ w1f.T)
    u = bf16_round(xf @ w3f.T)
    s = bf16_round(silu_f32(bf16_to_f32(g)))
    h = bf16_round(bf16_to_f32(s) * bf16_to_f32(u))
    return bf16_round(bf16_to_f32(h) @ w2f.T)


def dequant_expert(state: dict, hidden: int, inter: int, code: np.ndarray = NF4_CODE,
                   threads: int = 1):
    """{'w1'|'w2'|'w3': (packed, absmax)} -> bf16 bits (w1 [F,H], w3 [F,H], w2 [H,F])."""
    n = inter * hidden
    w1 = nf4_dequant(*state["w1"], code=code, numel=n, threads=threads).reshape(inter, hidden)
    w3 = nf4_dequant(*state["w3"], code=code, numel=n, threads=threads).reshape(inter, hidden)
    w2 = nf4_dequant(*state["w2"], code=code, numel=n, threads=threads).reshape(hidden, inter)
    return w1, w3, w2


def expand_absmax(q: np.ndarray, absmax2: np.ndarray, code2: np.ndarray, offset: float,
                  blocksize2: int) -> np.ndarray:
    """fp32 block scales of a nested (double-quantised) NF4 state: ``code2[q[i]] *
    absmax2[i // blocksize2]`` rounded to fp32, then ``+ offset`` rounded to fp32 -- the
    nested branch of the state that transfer/nf4_reconstruct.py:22-43 assembles, which
    bitsandbytes resolves as ``dequantize_blockwise(absmax, state2) + offset``.
    Parity unpinned against bitsandbytes itself (absent here): pinned only by a hand case
    and by the double-quantisation round trip in tests/test_host_store.py."""
    q = np.asarray(q, dtype=np.uint8).reshape(-1)
    grp = np.arange(q.size, dtype=np.int64) // int(blocksize2)
    v = np.asarray(code2, dtype=np.float32)[q] * np.asarray(absmax2, dtype=np.float32)[grp]
    return (v.astype(np.float32) + np.float32(offset)).astype(np.float32)


def double_quantize_absmax(absmax: np.ndarray, blocksize2: int = 256):
    """A nested state for fp32 block scales (test fixtures): offset = mean, then per group
    of blocksize2 the largest |absmax - offset| as absmax2 and the nearest entry of a
    256-entry signed code (uniform on [-1, 1]) as the 8-bit index.  Returns
    (q uint8, absmax2 fp32, code2 fp32[256], offset float)."""
    a = np.asarray(absmax, dtype=np.float32).reshape(-1)
    offset = float(np.float32(a.mean(dtype=np.float64)))
    c = (a - np.float32(offset)).astype(np.float32)
    ngrp = -(-a.size // int(blocksize2))
    pad = np.zeros(ngrp * int(blocksize2), dtype=np.float32)
    pad[:a.size] = np.abs(c)
    absmax2 = pad.reshape(ngrp, int(blocksize2)).max(axis=1).astype(np.float32)
    absmax2 = np.where(absmax2 > 0, absmax2, np.float32(1.0)).astype(np.float32)
    code2 = np.linspace(-1.0, 1.0, 256, dtype=np.float32)
    grp = np.arange(a.size) // int(blocksize2)
    x = c / absmax2[grp]
    q = np.abs(x[:, None] - code2[None, :]).argmin(axis=1).astype(np.uint8)
    return q, absmax2, code2, offset


def rel_l2(a, b) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    den = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (den if den > 0 else 1.0))
