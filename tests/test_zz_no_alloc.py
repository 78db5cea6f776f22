"""The allocation-free layer entry point (moe_layer_forward_nf4_noalloc), called through the
C ABI, against moe_layer_forward_nf4 with a caller workspace: bit-identical outputs on
consecutive calls that shrink (mid-batch T = 40, fused small-batch routing T = 16, decode
form T = 3), so the static scratch's leftovers from a larger call change nothing; a batched
layer whose K-split workspace exceeds the scratch runs with one down-projection plane (same
routing, outputs within fp32 summation order); layers that exceed it even so are refused
before any launch."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import bits

pytestmark = pytest.mark.gpu


def _experts(dev, H, F, E, seed):
    from moeinfra_amd import ops
    from moeinfra_amd._lib import MoeNf4Expert

    g = torch.Generator(device=dev).manual_seed(seed)
    keep = []
    for _ in range(E):
        st = {}
        for name, shape in (("w1", (F, H)), ("w3", (F, H)), ("w2", (H, F))):
            w = (torch.randn(shape, generator=g, device=dev) * 0.02).to(torch.bfloat16)
            st[name] = ops.nf4_quantize(w)
        keep.append(st)
    table = ops.expert_table([MoeNf4Expert(*(t.data_ptr() for n in ("w1", "w3", "w2")
                                             for t in st[n])) for st in keep])
    gate = (torch.randn((E, H), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    return keep, table, gate


def _run(lib, table, E, gate, bias, x, F, k, noalloc):
    from moeinfra_amd import _lib

    dev = x.device
    T, H = x.shape
    out = torch.full((T, H), -1.0, dtype=torch.bfloat16, device=dev)
    logits = torch.full((T, E), -1.0, dtype=torch.bfloat16, device=dev)
    w = torch.full((T, k), -1.0, dtype=torch.float32, device=dev)
    idx = torch.full((T, k), -1, dtype=torch.int64, device=dev)
    bptr = None if bias is None else bias.data_ptr()
    stream = torch.cuda.current_stream(dev).cuda_stream
    if noalloc:
        rc = lib.moe_layer_forward_nf4_noalloc(table, E, gate.data_ptr(), bptr, x.data_ptr(), T, H,
                                               F, k, out.data_ptr(), logits.data_ptr(),
                                               w.data_ptr(), idx.data_ptr(), stream)
    else:
        ws_bytes = lib.moe_layer_workspace_bytes(T, k, E, H, F)
        ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=dev)
        rc = lib.moe_layer_forward_nf4(table, E, gate.data_ptr(), bptr, x.data_ptr(), T, H, F, k,
                                       out.data_ptr(), logits.data_ptr(), w.data_ptr(),
                                       idx.data_ptr(), ws.data_ptr(), ws_bytes, stream)
    _lib.check(rc, "noalloc" if noalloc else "layer")
    torch.cuda.synchronize(dev)
    return bits(out), bits(logits), w.cpu().numpy(), idx.cpu().numpy()


def test_noalloc_layer_matches_workspace_layer(cuda_device):
    from moeinfra_amd import _lib, synth

    lib = _lib.lib()
    H, F, E, k = 1024, 3584, 8, 2
    _keep, table, gate = _experts(cuda_device, H, F, E, seed=910)
    g = torch.Generator(device=cuda_device).manual_seed(911)
    for T, skew in ((40, True), (16, False), (3, False)):
        print(f"noalloc layer T={T} skew={skew}", flush=True)
        x = torch.randn((T, H), generator=g, device=cuda_device).to(torch.bfloat16)
        bias = synth.zipf_bias(E, T).to(cuda_device) if skew else None
        got = _run(lib, table, E, gate, bias, x, F, k, noalloc=True)
        want = _run(lib, table, E, gate, bias, x, F, k, noalloc=False)
        for a, b in zip(got, want):
            np.testing.assert_array_equal(a, b)


def test_noalloc_batched_layer_falls_back_to_one_plane(cuda_device):
    from moeinfra_amd import _lib

    lib = _lib.lib()
    H, F, E, k, T = 1024, 3584, 8, 2, 2200
    # The default layout (down-projection K splits) does not fit the scratch here.
    assert lib.moe_layer_workspace_bytes(T, k, E, H, F) > _lib.MOE_NOALLOC_SCRATCH_BYTES
    _keep, table, gate = _experts(cuda_device, H, F, E, seed=920)
    g = torch.Generator(device=cuda_device).manual_seed(921)
    x = torch.randn((T, H), generator=g, device=cuda_device).to(torch.bfloat16)
    print(f"noalloc batched layer T={T}", flush=True)
    got = _run(lib, table, E, gate, None, x, F, k, noalloc=True)
    want = _run(lib, table, E, gate, None, x, F, k, noalloc=False)
    for a, b in zip(got[1:], want[1:]):  # logits, weights, ids: the same kernels
        np.testing.assert_array_equal(a, b)
    # The outputs add the down projection's K splits in another order (fp32): rel-L2 bound.
    from oracle import moe_oracle as orc
    assert orc.rel_l2(orc.bf16_to_f32(got[0]), orc.bf16_to_f32(want[0])) <= 1e-3


def test_noalloc_refuses_a_layer_above_the_scratch():
    from moeinfra_amd import _lib

    lib = _lib.lib()
    H, F, E, k = 4096, 14336, 8, 2
    # Mixtral shape: the layer fits up to T = 744 (one down-projection plane above T = 210).
    # With null outputs, T = 744 passes the size check and stops at the pointer check, T = 745
    # is refused for its size; both before any launch.
    rc = lib.moe_layer_forward_nf4_noalloc(None, E, None, None, None, 744, H, F, k, None, None,
                                           None, None, None)
    assert rc == _lib.MOE_STATUS_INVALID_ARGUMENT
    assert "static scratch" not in lib.moe_last_error().decode()
    rc = lib.moe_layer_forward_nf4_noalloc(None, E, None, None, None, 745, H, F, k, None, None,
                                           None, None, None)
    assert rc == _lib.MOE_STATUS_INVALID_ARGUMENT
    assert "static scratch" in lib.moe_last_error().decode()


def _capture_and_compare(lib, table, E, gate, x, F, k, replays=3):
    """Captures the allocation-free layer into a graph, replays it `replays` times with
    eager work and host synchronisations between the replays, and checks every replay's
    outputs bit for bit against an eager call with a caller workspace."""
    from moeinfra_amd import _lib

    dev = x.device
    T, H = x.shape
    out = torch.empty((T, H), dtype=torch.bfloat16, device=dev)
    logits = torch.empty((T, E), dtype=torch.bfloat16, device=dev)
    w = torch.empty((T, k), dtype=torch.float32, device=dev)
    idx = torch.empty((T, k), dtype=torch.int64, device=dev)
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    rcs = []
    with torch.cuda.stream(side), torch.cuda.graph(graph, stream=side):
        rcs.append(lib.moe_layer_forward_nf4_noalloc(
            table, E, gate.data_ptr(), None, x.data_ptr(), T, H, F, k, out.data_ptr(),
            logits.data_ptr(), w.data_ptr(), idx.data_ptr(), side.cuda_stream))
    _lib.check(rcs[0], "captured noalloc layer")
    want = _run(lib, table, E, gate, None, x, F, k, noalloc=False)
    for r in range(replays):
        for t in (out, logits, w, idx):
            t.fill_(-1)                      # eager work between the replays
        torch.cuda.synchronize(dev)
        graph.replay()
        torch.cuda.synchronize(dev)
        got = (bits(out), bits(logits), w.cpu().numpy(), idx.cpu().numpy())
        for a, b in zip(got, want):
            np.testing.assert_array_equal(a, b, err_msg=f"replay {r}, T={T}")


def test_noalloc_layer_under_graph_capture(cuda_device):
    """After eager calls (the scratch address is known), the allocation-free layer captured
    into a HIP graph replays bit-identically to the workspace entry point: decode form
    (T = 1), fused small-batch routing (T = 16) and the mid-batch path (T = 40)."""
    from moeinfra_amd import _lib

    lib = _lib.lib()
    H, F, E, k = 1024, 3584, 8, 2
    _keep, table, gate = _experts(cuda_device, H, F, E, seed=930)
    g = torch.Generator(device=cuda_device).manual_seed(931)
    for T in (1, 16, 40):
        print(f"noalloc layer under graph capture T={T}", flush=True)
        x = torch.randn((T, H), generator=g, device=cuda_device).to(torch.bfloat16)
        _run(lib, table, E, gate, None, x, F, k, noalloc=True)   # warm-up call
        _capture_and_compare(lib, table, E, gate, x, F, k)


_FIRST_CALL_SCRIPT = r"""
import sys
sys.path[:0] = [{repo!r}, {tests!r}]
import torch
import test_zz_no_alloc as m
from moeinfra_amd import _lib
dev = torch.device("cuda:0")
lib = _lib.lib()
H, F, E, k, T = 1024, 3584, 8, 2, 16
_keep, table, gate = m._experts(dev, H, F, E, seed=940)
x = torch.randn((T, H), generator=torch.Generator(device=dev).manual_seed(941),
                device=dev).to(torch.bfloat16)
torch.cuda.synchronize()
m._capture_and_compare(lib, table, E, gate, x, F, k)   # the process's first noalloc call
print("first-call capture ok", flush=True)
"""


def test_noalloc_first_call_under_graph_capture(cuda_device):
    """In a fresh process whose first allocation-free call is made under graph capture (the
    scratch address is looked up inside the capture), the captured layer still replays
    bit-identically to the workspace entry point."""
    import os
    import subprocess
    import sys

    here = os.path.dirname(os.path.abspath(__file__))
    script = _FIRST_CALL_SCRIPT.format(repo=os.path.dirname(here), tests=here)
    print("noalloc first call under graph capture (child process)", flush=True)
    proc = subprocess.run([sys.executable, "-c", script], capture_output=True, text=True,
                          timeout=300)
    print(proc.stdout[-2000:], proc.stderr[-4000:], flush=True)
    assert proc.returncode == 0 and "first-call capture ok" in proc.stdout
