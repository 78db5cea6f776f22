"""MI355X (gfx950) MoE expert-execution path with the MoEInfra Python API.

The compute runs in ``libmoeinfra_hip.so`` (hand-written HIP kernels behind a C ABI,
include/moeinfra_hip.h): NF4 dequant/quantise, the top-k router, expert grouping, the
fused-dequant SwiGLU expert FFN and the weighted combine.  The Python modules mirror the
reference's module layout (engine/router.py, model/moe_layer.py, model/expert.py,
transfer/nf4_reconstruct.py, transfer/*, cache/*) so callers can switch imports.
"""
__version__ = "0.1.0"
