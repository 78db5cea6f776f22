"""The C-ABI library: it loads, exports every entry point include/moeinfra_hip.h declares
(and only those), and its host-side argument checks work without a GPU."""
from __future__ import annotations

import ctypes
import os
import re
import subprocess

import pytest

from moeinfra_amd import _lib

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "moeinfra_hip.h")


def _declared():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return set(re.findall(r"\b(moe_[a-z0-9_]+)\s*\(", src))


def _exported():
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if " T moe_" in line}


def test_library_built_and_loads():
    assert os.path.exists(_lib.LIB_PATH), "run __graft_entry__.build() first"
    lib = _lib.lib()
    assert lib.moe_version() >= 100


def test_header_declares_exactly_the_exports():
    assert _declared() == _exported()


def test_ctypes_table_covers_the_header():
    assert set(_lib.SIGNATURES) == _declared()


def test_workspace_sizes_are_host_functions():
    lib = _lib.lib()
    assert lib.moe_layer_workspace_bytes(1, 2, 8, 4096, 14336) > 2 * 14336 * 2
    assert lib.moe_layer_workspace_bytes(-1, 2, 8, 4096, 14336) == -1
    assert lib.moe_expert_workspace_bytes(3, 1024, 3584) >= 3 * 3584 * 2 + 3 * 1024 * 4
    a = lib.moe_layer_workspace_bytes(16, 2, 8, 1024, 3584)
    assert a % 256 == 0 and a < lib.moe_layer_workspace_bytes(32, 2, 8, 1024, 3584)


def test_down_splits_size_the_ypart_planes():
    # The default K splits of the down projection: one plane for the decode forms; for the
    # mid-size kernels (5-64 tokens) one plane per 2048 values of F; for the streamed
    # mid-batch kernels and the batched GEMM a power of two that divides the NF4 blocks of F
    # into whole 4-block absmax groups; the workspace holds that many fp32 ypart planes.
    lib = _lib.lib()
    H, F, E, k = 4096, 14336, 8, 2
    assert lib.moe_layer_down_splits(1, k, E, H, F) == 1
    assert lib.moe_layer_down_splits(-1, k, E, H, F) == -1
    for T in (1, 4, 16, 40, 300, 512, 4096):
        n = lib.moe_layer_down_splits(T, k, E, H, F)
        if 5 <= T <= 64:
            assert n == F // 2048
        else:
            assert 1 <= n <= 16 and n & (n - 1) == 0
        if T >= 300:  # the batched GEMM
            assert (F // 64) % n == 0 and (F // 64 // n) % 4 == 0
        ws = lib.moe_layer_workspace_bytes(T, k, E, H, F)
        assert ws >= n * T * k * H * 4 + T * k * F * 2


@pytest.mark.parametrize("call,needle", [
    (lambda l: l.moe_nf4_dequant_bf16(8, 8, 8, 8, 7, 64, None), "even"),
    (lambda l: l.moe_nf4_dequant_bf16(8, 8, 8, 8, 64, 48, None), "multiple of 32"),
    (lambda l: l.moe_nf4_quantize_bf16(8, 64, 4097, 8, 8, 8, None), "blocksize"),
    (lambda l: l.moe_router_topk(8, 8, None, 4, 4096, 40, 2, None, 8, 8, None, None), "num_experts"),
    (lambda l: l.moe_router_topk(8, 8, None, 4, 4096, 8, 9, None, 8, 8, None, None), "top-k"),
    (lambda l: l.moe_router_topk(8, 8, None, 4, 4095, 8, 2, None, 8, 8, None, None), "multiple of 8"),
    (lambda l: l.moe_permute(8, 4, 2, 0, 8, 8, 8, 8, 8, None), "num_experts"),
    (lambda l: l.moe_combine(16, 0, 8, 8, 8, 4, 2, 4096, 8, None), "nsplit"),
])
def test_invalid_arguments_are_rejected_before_any_launch(call, needle):
    lib = _lib.lib()
    assert call(lib) == _lib.MOE_STATUS_INVALID_ARGUMENT
    assert needle in lib.moe_last_error().decode()


def test_status_maps_to_reference_exceptions():
    lib = _lib.lib()
    lib.moe_nf4_dequant_bf16(8, 8, 8, 8, 7, 64, None)
    with pytest.raises(ValueError, match="even"):
        _lib.check(_lib.MOE_STATUS_INVALID_ARGUMENT, "nf4_dequant")
    with pytest.raises(_lib.MoeHipError):
        _lib.check(_lib.MOE_STATUS_HIP_ERROR, "x")


def test_expert_struct_layout_matches_header():
    assert ctypes.sizeof(_lib.MoeNf4Expert) == 9 * ctypes.sizeof(ctypes.c_void_p)
    src = open(HEADER).read()
    body = re.search(r"typedef struct moe_nf4_expert \{(.*?)\}", src, re.S).group(1)
    fields = re.findall(r"const void \*(\w+);", body)
    assert fields == [f for f, _ in _lib.MoeNf4Expert._fields_]


def test_product_package_never_imports_the_oracle():
    pkg = os.path.join(REPO, "moeinfra_amd")
    for root, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".h", ".cpp")):
                text = open(os.path.join(root, f)).read()
                assert "oracle" not in re.sub(r"#.*|//.*", "", text).lower() or f == "__init__.py" \
                    and "oracle" not in text.lower(), f
