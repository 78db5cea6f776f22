"""Torch-tensor wrappers over the C ABI of ``libmoeinfra_hip.so``.

Every function validates dtype, shape and device first and raises ``ValueError`` the way
the reference does; kernels are enqueued on the current HIP stream of the tensors'
device (``torch.cuda.current_stream``).  Nothing here synchronises with the host, and
there is no non-HIP implementation: CPU tensors are rejected.
"""
from __future__ import annotations

import ctypes
from typing import Optional, Sequence

import torch

from . import _lib
from ._lib import MoeNf4Expert, check, lib
from .nf4 import NF4_BLOCKSIZE, nf4_code_tensor


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _require_cuda(t: torch.Tensor, name: str) -> None:
    if not isinstance(t, torch.Tensor):
        raise ValueError(f"{name} must be a torch.Tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be a GPU tensor (got device {t.device}); "
                         "the MoE path runs only on the HIP device")


def _require(t: torch.Tensor, name: str, dtype: torch.dtype, device: torch.device) -> None:
    _require_cuda(t, name)
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype} (got {t.dtype})")
    if t.device != device:
        raise ValueError(f"{name} device {t.device} != {device}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


# ----------------------------------------------------------------------------- K1
def nf4_expand_absmax(absmax_q: torch.Tensor, absmax2: torch.Tensor, code2: torch.Tensor,
                      offset, blocksize2: int) -> torch.Tensor:
    """fp32 block scales of a nested (double-quantised) NF4 state:
    ``code2[absmax_q[i]] * absmax2[i // blocksize2] + offset`` (bitsandbytes'
    dequantize_blockwise of the absmax, then ``+= offset``)."""
    dev = absmax_q.device
    _require(absmax_q, "absmax_q", torch.uint8, dev)
    _require(absmax2, "absmax2", torch.float32, dev)
    _require(code2, "code2", torch.float32, dev)
    if code2.numel() != 256:
        raise ValueError("the nested code must have 256 entries")
    n = absmax_q.numel()
    if absmax2.numel() * int(blocksize2) < n:
        raise ValueError(f"absmax2 has {absmax2.numel()} groups, {n} values need "
                         f"{(n + blocksize2 - 1) // blocksize2}")
    off = 0.0 if offset is None else float(offset)
    out = torch.empty(absmax_q.shape, dtype=torch.float32, device=dev)
    check(lib().moe_nf4_expand_absmax(absmax_q.data_ptr(), absmax2.data_ptr(), code2.data_ptr(), off,
                                      n, int(blocksize2), out.data_ptr(),
                                      torch.cuda.current_stream(dev).cuda_stream),
          "moe_nf4_expand_absmax")
    return out


def nf4_dequant(packed: torch.Tensor, absmax: torch.Tensor, code: torch.Tensor,
                shape: Sequence[int], blocksize: int = NF4_BLOCKSIZE,
                out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Packed NF4 -> bf16 tensor of ``shape`` (bitsandbytes ``dequantize_4bit`` semantics:
    ``bf16(code[q] * absmax[i // blocksize])``, high nibble first)."""
    dev = packed.device
    _require(packed, "packed", torch.uint8, dev)
    _require(absmax, "absmax", torch.float32, dev)
    _require(code, "code", torch.float32, dev)
    numel = 1
    for s in shape:
        numel *= int(s)
    if code.numel() != 16:
        raise ValueError("NF4 code must have 16 entries")
    if packed.numel() * 2 < numel:
        raise ValueError(f"packed has {packed.numel()} bytes, shape needs {(numel + 1) // 2}")
    if absmax.numel() * blocksize < numel:
        raise ValueError(f"absmax has {absmax.numel()} blocks, shape needs "
                         f"{(numel + blocksize - 1) // blocksize}")
    if out is None:
        out = torch.empty(tuple(int(s) for s in shape), dtype=torch.bfloat16, device=dev)
    else:
        _require(out, "out", torch.bfloat16, dev)
        if out.numel() != numel:
            raise ValueError("out has the wrong number of elements")
    check(lib().moe_nf4_dequant_bf16(packed.data_ptr(), absmax.data_ptr(), code.data_ptr(),
                                     out.data_ptr(), numel, blocksize, _stream(dev)),
          "nf4_dequant")
    return out


# ----------------------------------------------------------------------------- K0
def nf4_quantize(w: torch.Tensor, blocksize: int = NF4_BLOCKSIZE,
                 code: Optional[torch.Tensor] = None):
    """bf16 weight -> (packed uint8 [numel//2, 1], absmax fp32 [nblocks], code fp32 [16])."""
    dev = w.device
    _require_cuda(w, "weight")
    if w.dtype != torch.bfloat16:
        raise ValueError(f"Expected BF16 weights, got {w.dtype}")
    w = w.contiguous()
    if code is None:
        code = nf4_code_tensor(dev)
    _require(code, "code", torch.float32, dev)
    numel = w.numel()
    if numel % 2:
        raise ValueError("NF4 packing needs an even number of values")
    packed = torch.empty((numel // 2, 1), dtype=torch.uint8, device=dev)
    absmax = torch.empty(((numel + blocksize - 1) // blocksize,), dtype=torch.float32, device=dev)
    check(lib().moe_nf4_quantize_bf16(w.data_ptr(), numel, blocksize, code.data_ptr(),
                                      packed.data_ptr(), absmax.data_ptr(), _stream(dev)),
          "nf4_quantize")
    return packed, absmax, code


# ----------------------------------------------------------------------------- K2
def router_topk(x: torch.Tensor, gate: torch.Tensor, k: int,
                bias: Optional[torch.Tensor] = None, want_logits: bool = True,
                idx32_out: Optional[torch.Tensor] = None):
    """(logits bf16 [T,E] | None, weights fp32 [T,k], indices int64 [T,k])."""
    dev = x.device
    _require(x, "hidden_states", torch.bfloat16, dev)
    _require(gate, "gate_weight", torch.bfloat16, dev)
    if x.ndim != 2 or gate.ndim != 2 or x.shape[1] != gate.shape[1]:
        raise ValueError(f"shape mismatch: hidden {tuple(x.shape)} vs gate {tuple(gate.shape)}")
    T, H = x.shape
    E = gate.shape[0]
    if bias is not None:
        _require(bias, "bias", torch.float32, dev)
        if bias.numel() != E:
            raise ValueError("bias must have one value per expert")
    logits = torch.empty((T, E), dtype=torch.bfloat16, device=dev) if want_logits else None
    w = torch.empty((T, k), dtype=torch.float32, device=dev)
    idx = torch.empty((T, k), dtype=torch.int64, device=dev)
    if idx32_out is not None:
        _require(idx32_out, "idx32_out", torch.int32, dev)
    check(lib().moe_router_topk(x.data_ptr(), gate.data_ptr(), _ptr(bias), T, H, E, k,
                                _ptr(logits), w.data_ptr(), idx.data_ptr(), _ptr(idx32_out),
                                _stream(dev)), "router_topk")
    return logits, w, idx


# ----------------------------------------------------------------------------- K3
def permute(idx32: torch.Tensor, num_experts: int):
    """Expert-sorted grouping of routing slots.  Returns a dict of int32 device tensors:
    counts [E], offsets [E+1], perm_tok [T*k], slot_pos [T*k], active [E+1]."""
    dev = idx32.device
    _require(idx32, "idx32", torch.int32, dev)
    if idx32.ndim != 2:
        raise ValueError("idx32 must be [T, k]")
    T, k = idx32.shape
    E = int(num_experts)
    i32 = dict(dtype=torch.int32, device=dev)
    r = {
        "counts": torch.empty((E,), **i32),
        "offsets": torch.empty((E + 1,), **i32),
        "perm_tok": torch.empty((T * k,), **i32),
        "slot_pos": torch.empty((T * k,), **i32),
        "active": torch.empty((E + 1,), **i32),
    }
    check(lib().moe_permute(idx32.data_ptr(), T, k, E, r["counts"].data_ptr(),
                            r["offsets"].data_ptr(), r["perm_tok"].data_ptr(),
                            r["slot_pos"].data_ptr(), r["active"].data_ptr(), _stream(dev)),
          "permute")
    return r


# ----------------------------------------------------------------------------- K4/K5
def expert_table(experts: Sequence[Optional[MoeNf4Expert]]):
    """ctypes array of ``moe_nf4_expert_t`` (None -> an all-null, absent expert)."""
    if len(experts) > _lib.MOE_MAX_EXPERTS:
        raise ValueError(f"at most {_lib.MOE_MAX_EXPERTS} experts per call")
    arr = (MoeNf4Expert * max(1, len(experts)))()
    for i, e in enumerate(experts):
        if e is not None:
            arr[i] = e
    return arr


def choose_nsplit(T: int, k: int, E: int, H: int, F: int) -> int:
    """The library's default number of down-projection K splits (ypart planes) for a layer
    of T tokens, top-k k, E experts and hidden/FFN sizes H/F."""
    n = lib().moe_layer_down_splits(T, k, E, H, F)
    if n < 1:
        raise ValueError(f"invalid layer sizes T={T} k={k} E={E} H={H} F={F}")
    return n


def expert_ffn(table, num_experts: int, x: torch.Tensor, k: int, hidden: int, inter: int,
               route: dict, nsplit: Optional[int] = None):
    """K4 on routed rows: returns (h bf16 [T*k, F], ypart fp32 [nsplit, T*k, H])."""
    dev = x.device
    _require(x, "hidden_states", torch.bfloat16, dev)
    T = x.shape[0]
    if nsplit is None:
        nsplit = choose_nsplit(T, k, num_experts, hidden, inter)
    h = torch.empty((T * k, inter), dtype=torch.bfloat16, device=dev)
    ypart = torch.empty((nsplit, T * k, hidden), dtype=torch.float32, device=dev)
    check(lib().moe_expert_ffn_nf4(table, num_experts, x.data_ptr(), T, k, hidden, inter,
                                   route["counts"].data_ptr(), route["offsets"].data_ptr(),
                                   route["perm_tok"].data_ptr(), route["active"].data_ptr(),
                                   h.data_ptr(), ypart.data_ptr(), nsplit, _stream(dev)),
          "expert_ffn")
    return h, ypart


def combine(ypart: torch.Tensor, weights: torch.Tensor, idx32: torch.Tensor,
            slot_pos: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """K5: ascending-expert weighted combine into a bf16 [T, H] output."""
    dev = ypart.device
    _require(ypart, "ypart", torch.float32, dev)
    _require(weights, "weights", torch.float32, dev)
    _require(idx32, "idx32", torch.int32, dev)
    _require(slot_pos, "slot_pos", torch.int32, dev)
    nsplit, rows, H = ypart.shape
    T, k = weights.shape
    if out is None:
        out = torch.empty((T, H), dtype=torch.bfloat16, device=dev)
    check(lib().moe_combine(ypart.data_ptr(), nsplit, weights.data_ptr(), idx32.data_ptr(),
                            slot_pos.data_ptr(), T, k, H, out.data_ptr(), _stream(dev)),
          "combine")
    return out


def expert_swiglu(expert: MoeNf4Expert, x: torch.Tensor, hidden: int, inter: int) -> torch.Tensor:
    """One expert on all rows of x (bf16 [T, H]) -> bf16 [T, H]."""
    dev = x.device
    _require(x, "x", torch.bfloat16, dev)
    if x.ndim != 2 or x.shape[1] != hidden:
        raise ValueError(f"x must be [T, {hidden}] (got {tuple(x.shape)})")
    T = x.shape[0]
    y = torch.empty((T, hidden), dtype=torch.bfloat16, device=dev)
    if T == 0:
        return y
    ws_bytes = lib().moe_expert_workspace_bytes(T, hidden, inter)
    ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=dev)
    one = (MoeNf4Expert * 1)(expert)
    check(lib().moe_expert_swiglu_nf4(one, x.data_ptr(), T, hidden, inter, y.data_ptr(),
                                      ws.data_ptr(), ws_bytes, _stream(dev)), "expert_swiglu")
    return y


def layer_forward(table, num_experts: int, gate: torch.Tensor, x: torch.Tensor, k: int,
                  inter: int, bias: Optional[torch.Tensor] = None, want_logits: bool = False,
                  out: Optional[torch.Tensor] = None, workspace: Optional[torch.Tensor] = None):
    """Whole MoE layer (K2->K3->K4->K5) on resident experts.

    Returns (out bf16 [T,H], logits bf16 [T,E] | None, weights fp32 [T,k], idx int64 [T,k]).
    """
    dev = x.device
    _require(x, "hidden_states", torch.bfloat16, dev)
    _require(gate, "gate_weight", torch.bfloat16, dev)
    T, H = x.shape
    E = int(num_experts)
    if gate.shape != (E, H):
        raise ValueError(f"gate must be [{E}, {H}] (got {tuple(gate.shape)})")
    if bias is not None:
        _require(bias, "bias", torch.float32, dev)
    ws_bytes = lib().moe_layer_workspace_bytes(T, k, E, H, inter)
    if workspace is None or workspace.numel() < ws_bytes:
        workspace = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=dev)
    if out is None:
        out = torch.empty((T, H), dtype=torch.bfloat16, device=dev)
    logits = torch.empty((T, E), dtype=torch.bfloat16, device=dev) if want_logits else None
    w = torch.empty((T, k), dtype=torch.float32, device=dev)
    idx = torch.empty((T, k), dtype=torch.int64, device=dev)
    check(lib().moe_layer_forward_nf4(table, E, gate.data_ptr(), _ptr(bias), x.data_ptr(), T, H,
                                      inter, k, out.data_ptr(), _ptr(logits), w.data_ptr(),
                                      idx.data_ptr(), workspace.data_ptr(), workspace.numel(),
                                      _stream(dev)), "layer_forward")
    return out, logits, w, idx
