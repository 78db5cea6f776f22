"""Drives the host-side argument checking of a libmoeinfra_hip build through its C ABI with
pointer values that are never dereferenced (every call must be refused before any launch,
so no GPU is needed).  Run by tests/test_capi_sanitized.py against the ASan/UBSan build,
in a process with the ASan runtime preloaded; prints "OK <calls>" when every call returned
the expected status.

Usage: python drive_capi.py LIB_PATH
"""
import ctypes
import importlib.util
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
spec = importlib.util.spec_from_file_location(
    "moe_lib", os.path.join(HERE, "..", "..", "moeinfra_amd", "_lib.py"))
L = importlib.util.module_from_spec(spec)
spec.loader.exec_module(L)

lib = ctypes.CDLL(sys.argv[1])
for name, (argtypes, restype) in L.SIGNATURES.items():
    fn = getattr(lib, name)
    fn.argtypes, fn.restype = argtypes, restype

BAD = L.MOE_STATUS_INVALID_ARGUMENT
A, B, C, D = 0x10000, 0x20000, 0x30000, 0x40000   # distinct fake device addresses
H, F, E, k = 4096, 14336, 8, 2
calls = 0


def expect(rc, needle, what):
    global calls
    calls += 1
    msg = lib.moe_last_error().decode()
    if rc != BAD or needle not in msg:
        sys.exit(f"{what}: status {rc}, message {msg!r} (wanted {needle!r})")


table = (L.MoeNf4Expert * E)()
expect(lib.moe_nf4_dequant_bf16(A, B, C, D, 7, 64, None), "even", "dequant odd")
expect(lib.moe_nf4_dequant_bf16(A, B, C, D, 64, 48, None), "multiple of 32", "dequant bs")
expect(lib.moe_nf4_dequant_bf16(A + 1, B, C, D, 64, 64, None), "aligned", "dequant align")
expect(lib.moe_nf4_quantize_bf16(A, 64, 4097, C, D, B, None), "blocksize", "quantize bs")
expect(lib.moe_nf4_quantize_bf16(A, -2, 64, C, D, B, None), "numel", "quantize numel")
expect(lib.moe_nf4_expand_absmax(A, B, C, 0.0, -1, 256, D, None), "non-negative", "expand n")
expect(lib.moe_router_topk(A, B, None, 4, H, 40, 2, None, C, D, None, None), "num_experts", "router E")
expect(lib.moe_router_topk(A, B, None, 4, H, 8, 9, None, C, D, None, None), "top-k", "router k")
expect(lib.moe_router_topk(A, B, None, 4, 4095, 8, 2, None, C, D, None, None), "multiple of 8",
       "router H")
expect(lib.moe_permute(A, 4, 2, 0, B, C, D, A, B, None), "num_experts", "permute E")
expect(lib.moe_combine(A, 0, B, C, D, 4, 2, H, A, None), "nsplit", "combine nsplit")
ws = lib.moe_layer_workspace_bytes(16, k, E, H, F)
assert ws > 0 and lib.moe_layer_workspace_bytes(-1, k, E, H, F) == -1
assert lib.moe_expert_workspace_bytes(3, 1024, 3584) > 0
expect(lib.moe_layer_forward_nf4(table, E, A, None, B, 16, H, F, k, C, None, D, A, B, ws - 1, None),
       "workspace too small", "layer workspace")
expect(lib.moe_layer_forward_nf4(table, E, A, None, B, 16, H, F, k, C, None, D, A, B + 8, ws, None),
       "aligned", "layer workspace alignment")
expect(lib.moe_layer_forward_nf4(table, E, A, None, B, 16, H, F, k, None, None, D, A, B, ws, None),
       "null output", "layer outputs")
expect(lib.moe_layer_forward_nf4(None, E, A, None, B, 1, H, F, k, C, None, D, A, B, ws, None),
       "null expert table", "decode layer table")
expect(lib.moe_layer_forward_nf4_noalloc(None, E, None, None, None, 745, H, F, k, None, None, None,
                                         None, None), "static scratch", "noalloc size")
nws = lib.moe_layer_norm_workspace_bytes(k, E, H, F)
assert nws > 0
xa, res, nw, out, good = 0x100000, 0x200000, 0x300000, 0x400000, 0x500000
gate = 0x600000
for bad in (xa, res, nw, gate + 100):
    expect(lib.moe_layer_forward_nf4_norm(table, E, gate, xa, res, nw, 1e-5, H, F, k, bad, out, A, B,
                                          0x1000000, nws, None), "must not overlap", "norm overlap")
expect(lib.moe_layer_forward_nf4_norm(table, E, gate, xa, res, nw, 1e-5, H, F, k, good, good, A, B,
                                      0x1000000, nws, None), "out must not overlap", "norm out")
expect(lib.moe_layer_forward_nf4_norm(table, E, gate, xa, res, nw, 1e-5, H, F, k, good, out, A, B,
                                      0x1000000, nws - 1, None), "workspace too small", "norm ws")
wq = 0x10000000
for bad, r in ((xa, res), (res, res), (nw, res), (wq + 64, res)):
    expect(lib.moe_qkv_rope_bf16(wq, xa, None, 1, r, nw, 1e-5, H, 32, 8, 128, A, B, 16, bad, C, D,
                                 A, None), "must not overlap", "qkv overlap")
expect(lib.moe_qkv_rope_bf16(wq, xa, None, 1, res, nw, 1e-5, 4000, 32, 8, 128, A, B, 16, good, C,
                             D, A, None), "multiple of 512", "qkv H")
expect(lib.moe_head_argmax_bf16(wq, xa, res, nw, 1e-5, 32000, 4000, A, B, 8, C, None, 0, None, None,
                                None), "multiple of 512", "head K")
expect(lib.moe_gemv_bf16(wq, xa, 0, 64, 512, A, None), "tokens", "gemv T")
expect(lib.moe_attention_bf16(A, B, C, 1, 32, 7, 128, D, 16, 0.1, A, None), "head", "attention heads")
print(f"OK {calls}")
