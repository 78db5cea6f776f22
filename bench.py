#!/usr/bin/env python3
"""Benchmark of the MI355X MoE expert path: Mixtral-8x7B-shaped NF4 experts, batch-1 decode.

One step = one decode token (T=1 by default) through 32 MoE layers (hidden 4096, FFN 14336,
8 NF4 experts per layer, top-2): router -> permute -> fused-dequant gate/up -> down ->
combine on the HIP kernels, with every expert resident in HBM (32 x 8 x 99,090,432 B NF4).
Weights are synthetic bf16 N(0, 0.02) drawn on the GPU from a seed and NF4-quantised by the
library's quantiser; activations are bf16 N(0, 1), a fixed input per layer.

Prints ONE JSON line.  ``value`` is decode tokens/s of the 32-layer MoE path; ``roofline``
is for the dominant kernel (the fused NF4 gate/up GEMV), timed with HIP events around each
of its launches inside the timed region; ``cpu_baseline`` times the CPU oracle (C NF4
dequant + numpy fp32 SwiGLU) on a bounded sample of the same layers.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

HBM_PEAK_GBPS = 8000.0
METRIC = "decode tok/s Mixtral-8x7B-shape NF4 (bs=1); MoE-layer HBM GB/s vs peak"
HERE = os.path.dirname(os.path.abspath(__file__))


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--layers", type=int, default=32)
    p.add_argument("--tokens", type=int, default=1, help="tokens per decode step (batch)")
    p.add_argument("--routing", choices=["uniform", "zipf"], default="uniform")
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--cpu-seconds", type=float, default=15.0,
                   help="approximate CPU time budget of the oracle baseline sample")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-kernel-events", action="store_true",
                   help="do not bracket kernels with HIP events (headline timing only)")
    return p.parse_args()


def nf4_expert_bytes(h: int, f: int) -> int:
    n = h * f
    return 3 * (n // 2 + n // 64 * 4)


def gateup_bytes(u: int, h: int, f: int, t: int, k: int) -> int:
    """Algorithmic HBM bytes of one gate/up launch: w1+w3 NF4 of the u routed experts,
    the T activations read, the T*k h rows written."""
    n = h * f
    return u * 2 * (n // 2 + n // 64 * 4) + t * h * 2 + t * k * f * 2


def down_bytes(u: int, h: int, f: int, t: int, k: int, nsplit: int) -> int:
    n = h * f
    return u * (n // 2 + n // 64 * 4) + t * k * f * 2 + nsplit * t * k * h * 4


def layer_bytes(u: int, h: int, f: int, t: int, e: int) -> int:
    """MoE-layer algorithmic bytes: routed experts' NF4 + x read + out written + gate."""
    return u * nf4_expert_bytes(h, f) + 2 * t * h * 2 + e * h * 2


def main() -> int:
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}, WORLD_SIZE {world}): "
              "this build has no multi-GPU path; run with --gpus 1.", file=sys.stderr)
        return 2

    import torch

    from moeinfra_amd import _lib, ops, synth

    H, F, E, K = synth.MIXTRAL_HIDDEN, synth.MIXTRAL_FFN, synth.MIXTRAL_EXPERTS, synth.MIXTRAL_TOPK
    L, T = args.layers, args.tokens
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    lib = _lib.lib()
    t_setup = time.time()

    # ------------------------------------------------------------------ model (all-resident)
    gen = synth.make_generator(args.seed, device=dev)
    layers = []

    def quantize(e, w1, w3, w2):
        out = {}
        for name, w in (("w1", w1), ("w3", w3), ("w2", w2)):
            packed, absmax, code = ops.nf4_quantize(w)
            out[name] = (packed, absmax, code)
        return out

    for _ in range(L):
        lw = synth.make_layer(H, F, E, gen, device=dev, expert_sink=quantize)
        structs = []
        for ex in lw.experts:
            structs.append(_lib.MoeNf4Expert(
                ex["w1"][0].data_ptr(), ex["w1"][1].data_ptr(), ex["w1"][2].data_ptr(),
                ex["w3"][0].data_ptr(), ex["w3"][1].data_ptr(), ex["w3"][2].data_ptr(),
                ex["w2"][0].data_ptr(), ex["w2"][1].data_ptr(), ex["w2"][2].data_ptr()))
        layers.append({"gate": lw.gate, "experts": lw.experts, "table": ops.expert_table(structs)})
    xs = [synth.make_activations(T, H, gen, device=dev) for _ in range(L)]
    bias = synth.zipf_bias(E, args.seed).to(dev) if args.routing == "zipf" else None
    torch.cuda.synchronize()
    setup_s = time.time() - t_setup

    # ------------------------------------------------------------------ per-layer buffers
    nsplit = ops.choose_nsplit(T, K, E, H)
    i32 = dict(dtype=torch.int32, device=dev)
    bufs = []
    for l in range(L):
        bufs.append({
            "w": torch.empty((T, K), dtype=torch.float32, device=dev),
            "idx": torch.empty((T, K), dtype=torch.int64, device=dev),
            "idx32": torch.empty((T, K), **i32),
            "counts": torch.empty((E,), **i32), "offsets": torch.empty((E + 1,), **i32),
            "perm": torch.empty((T * K,), **i32), "slot": torch.empty((T * K,), **i32),
            "active": torch.empty((E + 1,), **i32),
            "h": torch.empty((T * K, F), dtype=torch.bfloat16, device=dev),
            "ypart": torch.empty((nsplit, T * K, H), dtype=torch.float32, device=dev),
            "out": torch.empty((T, H), dtype=torch.bfloat16, device=dev),
        })
    stream = torch.cuda.current_stream(dev).cuda_stream
    bias_ptr = None if bias is None else bias.data_ptr()

    # Pre-bound argument tuples keep the host-side cost of a step to the ctypes calls.
    calls = []
    for l in range(L):
        b, lay = bufs[l], layers[l]
        calls.append((
            (xs[l].data_ptr(), lay["gate"].data_ptr(), bias_ptr, T, H, E, K, None,
             b["w"].data_ptr(), b["idx"].data_ptr(), b["idx32"].data_ptr(), stream),
            (b["idx32"].data_ptr(), T, K, E, b["counts"].data_ptr(), b["offsets"].data_ptr(),
             b["perm"].data_ptr(), b["slot"].data_ptr(), b["active"].data_ptr(), stream),
            (lay["table"], E, xs[l].data_ptr(), T, K, H, F, b["counts"].data_ptr(),
             b["offsets"].data_ptr(), b["perm"].data_ptr(), b["active"].data_ptr(),
             b["h"].data_ptr(), stream),
            (lay["table"], E, T, K, H, F, b["counts"].data_ptr(), b["offsets"].data_ptr(),
             b["perm"].data_ptr(), b["active"].data_ptr(), b["h"].data_ptr(),
             b["ypart"].data_ptr(), nsplit, stream),
            (b["ypart"].data_ptr(), nsplit, b["w"].data_ptr(), b["idx32"].data_ptr(),
             b["slot"].data_ptr(), T, K, H, b["out"].data_ptr(), stream),
        ))
    f_router, f_perm = lib.moe_router_topk, lib.moe_permute
    f_gu, f_down, f_comb = lib.moe_expert_gateup_nf4, lib.moe_expert_down_nf4, lib.moe_combine

    def step(ev=None):
        for l in range(L):
            a_r, a_p, a_g, a_d, a_c = calls[l]
            rc = f_router(*a_r) | f_perm(*a_p)
            if ev is not None:
                ev[l][0].record()
            rc |= f_gu(*a_g)
            if ev is not None:
                ev[l][1].record()
            rc |= f_down(*a_d)
            if ev is not None:
                ev[l][2].record()
            rc |= f_comb(*a_c)
            if rc:
                _lib.check(-2 if rc < -1 else rc, "bench step")

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # Routed experts per layer (inputs are fixed, so routing is the same every step).
    u_per_layer = [int(torch.unique(bufs[l]["idx"]).numel()) for l in range(L)]

    use_ev = not args.no_kernel_events
    evs = ([[[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(L)]
            for _ in range(args.steps)] if use_ev else None)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(args.steps):
        step(evs[s] if use_ev else None)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_per_step = elapsed * 1e3 / args.steps

    # ------------------------------------------------------------------ kernel times
    gu_us = down_us = None
    if use_ev:
        gu = [evs[s][l][0].elapsed_time(evs[s][l][1]) for s in range(args.steps) for l in range(L)]
        dn = [evs[s][l][1].elapsed_time(evs[s][l][2]) for s in range(args.steps) for l in range(L)]
        gu_us = 1e3 * sum(gu) / len(gu)
        down_us = 1e3 * sum(dn) / len(dn)
    u_mean = sum(u_per_layer) / L
    gu_bytes = sum(gateup_bytes(u, H, F, T, K) for u in u_per_layer) / L
    dn_bytes = sum(down_bytes(u, H, F, T, K, nsplit) for u in u_per_layer) / L
    ly_bytes = sum(layer_bytes(u, H, F, T, E) for u in u_per_layer) / L
    layer_us = ms_per_step * 1e3 / L
    layer_gbps = ly_bytes / (layer_us * 1e-6) / 1e9

    roofline = None
    if gu_us:
        ach = gu_bytes / (gu_us * 1e-6) / 1e9
        roofline = {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBPS,
                    "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBPS, 4),
                    "traffic": _traffic("gateup_nf4_decode_t%d" % T), "kernel": "gateup_kernel",
                    "bytes_per_launch": int(gu_bytes), "avg_launch_us": round(gu_us, 2)}

    # ------------------------------------------------------------------ CPU baseline
    cpu = None
    if not args.no_cpu_baseline:
        cpu = _cpu_baseline(layers, xs, bias, T, H, F, E, K, L, args.cpu_seconds)

    result = {
        "metric": METRIC,
        "value": round(T / (ms_per_step * 1e-3), 3),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded bf16 N(0,0.02) weights NF4-quantised on the GPU; bf16 N(0,1) activations)",
        "config": {
            "workload": f"Mixtral-8x7B-shaped NF4 MoE expert path, {L} layers, decode batch {T}, "
                        "all experts resident in HBM (router, permute, fused-dequant SwiGLU, combine)",
            "hidden": H, "ffn": F, "experts": E, "top_k": K, "layers": L, "tokens_per_step": T,
            "routing": args.routing, "weights": "NF4 blocksize 64, fp32 absmax",
            "nsplit_down": nsplit, "parallelism": "single GPU",
        },
        "roofline": roofline,
        "cpu_baseline": cpu,
        "per_layer_us": round(layer_us, 2),
        "layer_hbm_gbps": round(layer_gbps, 1),
        "layer_hbm_frac": round(layer_gbps / HBM_PEAK_GBPS, 4),
        "routed_experts_per_layer": round(u_mean, 3),
        "kernels_us": {"gateup": None if gu_us is None else round(gu_us, 2),
                       "down": None if down_us is None else round(down_us, 2)},
        "kernel_events_in_timed_region": use_ev,
        "setup_s": round(setup_s, 1),
    }
    print(json.dumps(result), flush=True)
    return 0


def _traffic(name: str):
    """HBM bytes per launch measured by rocprofv3 counters (committed under profiles/)."""
    path = os.path.join(HERE, "profiles", name + ".traffic.json")
    try:
        with open(path) as fh:
            return json.load(fh).get("hbm_bytes_per_launch")
    except (OSError, ValueError):
        return None


def _cpu_baseline(layers, xs, bias, T, H, F, E, K, L, budget_s):
    """The CPU oracle on a bounded sample: whole MoE layers at the same T, scaled to L layers."""
    import numpy as np
    import torch

    from oracle import moe_oracle as orc

    cores = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS")
    threads = min(cores, int(omp)) if omp and omp.isdigit() and int(omp) > 0 else cores

    def to_np(t, dt):
        return t.detach().cpu().contiguous().view(dt).numpy()

    times, n = [], 0
    t_start = time.perf_counter()
    for l in range(L):
        lay = layers[l]
        x = to_np(xs[l], torch.int16).view(np.uint16)
        gate = to_np(lay["gate"], torch.int16).view(np.uint16)
        b = None if bias is None else bias.cpu().numpy()
        # Only the experts this layer routes to are needed; copy them to host first.
        _, _, idx = orc.router(x, gate, k=K, bias=b)
        state = {}
        for e in sorted(set(int(v) for v in idx.reshape(-1))):
            ex = lay["experts"][e]
            state[e] = {nm: (ex[nm][0].cpu().numpy().reshape(-1), ex[nm][1].cpu().numpy())
                        for nm in ("w1", "w3", "w2")}

        def expert_fn(e, rows):
            w1, w3, w2 = orc.dequant_expert(state[e], H, F, threads=threads)
            return orc.swiglu(rows, w1, w3, w2)

        t0 = time.perf_counter()
        orc.moe_layer(x, gate, expert_fn, k=K, bias=b)
        times.append(time.perf_counter() - t0)
        n += 1
        if time.perf_counter() - t_start > budget_s:
            break
    per_layer = sorted(times)[len(times) // 2]
    return {"value": round(T / (per_layer * L), 5), "unit": "tok/s", "cores": threads,
            "kind": "port",
            "sample": f"CPU oracle (C NF4 dequant on {threads} threads + numpy fp32 SwiGLU, "
                      f"ascending-expert bf16 combine) on {n} of {L} layers at T={T}; "
                      f"median {per_layer * 1e3:.1f} ms/layer, scaled to {L} layers"}


if __name__ == "__main__":
    sys.exit(main())
