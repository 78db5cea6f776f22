#!/usr/bin/env python3
"""Benchmark of the MI355X MoE expert path: Mixtral-8x7B-shaped NF4 model, batch-1 decode.

Default (``--mode e2e``): the end-to-end random-init Mixtral-8x7B-shaped model (32 decoder
layers, hidden 4096, GQA 32/8 heads of 128, RoPE theta 1e6, vocab 32000, 8 NF4 experts of
FFN 14336 per layer, top-2), every expert resident in HBM.  A 40-token random-id prompt is
prefilled, then greedy decode; one step = one decode token through the whole model (one
replay of the captured decode-step HIP graph).  ``value`` is decode tokens/s over exactly
``--steps`` steps (the reference's generate() figure: generated-after-first / decode
seconds); ``ttft_ms`` is the prompt's prefill.  ``--offload`` runs the same workload with
the NF4 store in pinned host memory and a bounded GPU expert cache (eager steps).

In the same run, the MoE-layer pass times the 32 MoE layers alone (the library's
whole-layer entry point, T=1, fixed N(0,1) inputs per layer) for the second half of the
metric, MoE-layer HBM GB/s vs peak, and for ``roofline``: the dominant kernel (the fused
routing + NF4 gate/up GEMV) is bracketed by HIP events inside that pass's timed region, one
layer per step (layer s mod 32 at step s), so its average covers every layer.
``cpu_baseline`` times the CPU oracle decoder (C NF4 dequant + torch CPU bf16 attention and
numpy fp32 SwiGLU) on a bounded sample of layers of one decode token, scaled to the model.

``--mode decode`` keeps the MoE-layer pass alone at any batch (``--tokens``, ``--routing``)
as the headline; ``--mode reconstruct`` times one expert's NF4 -> bf16 reconstruction;
``--mode prefill`` times the prompt prefill alone (time to first token).
Weights are synthetic bf16 N(0, 0.02) drawn on the GPU from a seed, experts NF4-quantised
by the library's quantiser.  Prints ONE JSON line (two for reconstruct).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

HBM_PEAK_GBPS = 8000.0
MFMA_BF16_TFLOPS = 2500.0  # dense bf16 MFMA peak of MI355X
METRIC = "decode tok/s Mixtral-8x7B-shape NF4 (bs=1); MoE-layer HBM GB/s vs peak"
HERE = os.path.dirname(os.path.abspath(__file__))


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=32)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--layers", type=int, default=32)
    p.add_argument("--prompt", type=int, default=40, help="prompt tokens (e2e mode)")
    p.add_argument("--offload", action="store_true",
                   help="e2e mode with the NF4 store in pinned host memory and a bounded GPU cache")
    p.add_argument("--gpu-expert-slots", type=int, default=8,
                   help="GPU expert cache slots in offload mode (the reference's default: 8)")
    p.add_argument("--prefetch", choices=["none", "next_layer", "lookahead", "next_router"],
                   default="none",
                   help="offload mode's prefetch policy (the reference engine's default: none)")
    p.add_argument("--gpu-slots-per-layer", type=int, default=None,
                   help="offload mode: partition the GPU expert tier by layer and keep the "
                        "experts each layer transferred (default: the reference's contract, "
                        "transferred experts are demoted after their layer)")
    p.add_argument("--cache-policy", choices=["lru", "lfu", "arc"], default="lru",
                   help="offload mode's GPU-tier eviction policy (the reference's default: lru)")
    p.add_argument("--prefetch-depth", type=int, default=2)
    p.add_argument("--copy-timeline", action="store_true",
                   help="offload mode: time every host-to-device copy and every MoE layer's "
                        "expert kernels with HIP events in the timed run, and report the host "
                        "link's busy share and the copy/compute overlap over the decode steps")
    p.add_argument("--prefetch-prefix-mib", type=float, default=8.0,
                   help="offload mode with --prefetch next_router: copy only this many MiB of "
                        "each guessed expert ahead (a bounded prefix); 0: the whole image")
    p.add_argument("--tokens", type=int, default=1, help="tokens per decode step (decode mode)")
    p.add_argument("--routing", choices=["uniform", "zipf"], default="uniform")
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--cpu-seconds", type=float, default=15.0,
                   help="approximate CPU time budget of the oracle baseline sample")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                   help="only run 10 plain device copies of MIB MiB (the known-size kernel that "
                        "scales the FETCH_SIZE / WRITE_SIZE counters) and exit")
    p.add_argument("--no-kernel-events", action="store_true",
                   help="do not bracket kernels with HIP events (headline timing only)")
    p.add_argument("--mode", choices=["e2e", "decode", "reconstruct", "prefill"], default="e2e",
                   help="e2e (default): the end-to-end model's decode plus the MoE-layer pass; "
                        "decode: the MoE-layer pass alone at --tokens per step; reconstruct: one "
                        "Mixtral expert's NF4 -> bf16 reconstruction from HBM (K1) and from a "
                        "pinned host staging slot (H2D + K1), one JSON line each; prefill: the "
                        "end-to-end model's prompt prefill alone (time to first token), --steps "
                        "timed prompts of --prompt tokens")
    return p.parse_args()


def nf4_expert_bytes(h: int, f: int) -> int:
    n = h * f
    return 3 * (n // 2 + n // 64 * 4)


def decode_form(t: int, k: int, e: int, h: int, f: int) -> bool:
    """Whether the layer call runs as the two-launch decode form (routing fused into the
    gate/up kernel, combine into the down kernel)."""
    return t <= 4 and t * k <= 8 and e <= 16 and h % 512 == 0 and f % 512 == 0


def gemm_form(t: int, k: int, e: int, h: int, f: int) -> bool:
    """Whether the layer call runs the LDS-staged batched GEMM (32 or more rows per routed
    expert on average)."""
    return not decode_form(t, k, e, h, f) and t * k >= 32 * min(t * k, e)


def mid_form(t: int, k: int, e: int, h: int, f: int, cus: int = 256) -> bool:
    """Whether the layer call runs the mid-size kernels (5-64 tokens, virtual experts of
    16 rows on 16-row weight tiles; hidden size 2048 or 4096)."""
    return (not decode_form(t, k, e, h, f) and 5 <= t <= 64 and h in (2048, 4096)
            and f % 16 == 0 and e <= 32 and t * h * 2 >= 2048 and e + t * k // 16 + 1 <= cus)


def midbatch_form(t: int, k: int, e: int, h: int, f: int) -> bool:
    """Whether the layer call runs the streamed mid-batch kernels (more than 4 and fewer
    than 32 rows per routed expert, shapes with whole 512-wide tiles, outside the mid-size
    kernels' range)."""
    return (not decode_form(t, k, e, h, f) and not gemm_form(t, k, e, h, f) and t > 4
            and not mid_form(t, k, e, h, f)
            and h % 512 == 0 and f % 512 == 0 and (f // 64) % 8 == 0 and t * k <= 2048)


def gateup_bytes(u: int, h: int, f: int, t: int, k: int, e: int) -> int:
    """Algorithmic HBM bytes of one gate/up launch: w1+w3 NF4 of the u routed experts,
    the T activations read, the T*k h rows written, and in the decode form the [E, H]
    router gate it reads for the fused routing."""
    n = h * f
    gate = e * h * 2 if decode_form(t, k, e, h, f) else 0
    return u * 2 * (n // 2 + n // 64 * 4) + t * h * 2 + t * k * f * 2 + gate


def down_bytes(u: int, h: int, f: int, t: int, k: int, nsplit: int) -> int:
    n = h * f
    return u * (n // 2 + n // 64 * 4) + t * k * f * 2 + nsplit * t * k * h * 4


def layer_bytes(u: int, h: int, f: int, t: int, e: int) -> int:
    """MoE-layer algorithmic bytes: routed experts' NF4 + x read + out written + gate."""
    return u * nf4_expert_bytes(h, f) + 2 * t * h * 2 + e * h * 2


def decode_step_bytes(s, u_per_layer, pos: int) -> int:
    """Algorithmic HBM bytes of one batch-1 decode step of the whole model: per layer the
    q/k/v and o projections (bf16), the routed experts' NF4 and the router gate, the KV
    cache read by attention over ``pos`` + 1 positions; then the final norm's lm_head and
    one embedding row.  Activations and norm weights (a few KB per layer) are left out."""
    H, hd = s.hidden, s.head_dim
    attn = (s.qkv_rows * H + H * s.n_heads * hd) * 2
    kv = 2 * s.n_kv_heads * (pos + 1) * hd * 2
    per_layer = [attn + kv + u * nf4_expert_bytes(H, s.ffn) + s.experts * H * 2 for u in u_per_layer]
    return sum(per_layer) + s.vocab * H * 2 + H * 2


def main() -> int:
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}, WORLD_SIZE {world}): "
              "this build has no multi-GPU path; run with --gpus 1.", file=sys.stderr)
        return 2

    import torch  # noqa: F401

    if args.copy_calibration > 0:
        return _copy_calibration(args.copy_calibration)
    if args.mode == "reconstruct":
        return _reconstruct(args)
    if args.mode == "e2e":
        return _e2e(args)
    if args.mode == "prefill":
        return _prefill(args)
    return _decode_layers(args)


def _prefill(args) -> int:
    """``--mode prefill``: the prompt prefill of the all-resident 32-layer model alone (the
    reference's ttft, engine/engine.py:478-484): W untimed prompts, then ``--steps`` timed
    ones, each the whole prefill through the last token's logits."""
    import torch

    from moeinfra_amd.engine.decoder import MixtralShape, synthesize
    from moeinfra_amd.engine.engine import InferenceEngine
    from moeinfra_amd.engine.types import ForwardRequest

    s = MixtralShape(layers=args.layers)
    P, K, W = args.prompt, max(args.steps, 1), args.warmup
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    w = synthesize(s, seed=args.seed, device=dev)
    eng = InferenceEngine(w, max_seq=P + 8, device=dev)
    prompt = torch.randint(0, s.vocab, (1, P), generator=torch.Generator().manual_seed(args.seed))
    for _ in range(W):
        eng.generate(ForwardRequest(prompt, max_new_tokens=1))
    torch.cuda.synchronize()
    ttft = [eng.generate(ForwardRequest(prompt, max_new_tokens=1)).ttft_ms for _ in range(K)]
    ms = sorted(ttft)[len(ttft) // 2]
    print(json.dumps({
        "metric": "time to first token, Mixtral-8x7B-shape NF4, all-resident", "value": round(ms, 3),
        "unit": "ms", "n_gpus": 1, "steps": K, "warmup": W, "higher_is_better": False,
        "dtype": "bf16", "data": "synthetic (seeded weights, random prompt ids)",
        "config": {"workload": f"{P}-token random-id prompt through the {s.layers}-layer "
                               "Mixtral-8x7B-shaped model (prefill to the last token's logits)",
                   "prompt_tokens": P, "layers": s.layers},
        "ttft_ms_all": [round(t, 3) for t in ttft]}), flush=True)
    return 0


# ---------------------------------------------------------------------------- MoE-layer pass
def _moe_pass(lib, layers, xs, bias, T, H, F, E, K, steps, warmup, events=True, routing="uniform"):
    """Times ``steps`` passes over the MoE layers (one call of the whole-layer entry point
    each), with one layer per step through the profiled entry when ``events`` is set.
    ``layers``: [{"gate": [E, H] bf16, "table": expert table}]; ``xs``: per-layer [T, H]."""
    import torch

    from moeinfra_amd import _lib, ops

    L = len(layers)
    dev = xs[0].device
    nsplit = ops.choose_nsplit(T, K, E, H, F)
    ws_bytes = lib.moe_layer_workspace_bytes(T, K, E, H, F)
    ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=dev)
    outs = [torch.empty((T, H), dtype=torch.bfloat16, device=dev) for _ in range(L)]
    wts = [torch.empty((T, K), dtype=torch.float32, device=dev) for _ in range(L)]
    idxs = [torch.empty((T, K), dtype=torch.int64, device=dev) for _ in range(L)]
    stream = torch.cuda.current_stream(dev).cuda_stream
    bias_ptr = None if bias is None else bias.data_ptr()
    call_args = [(layers[l]["table"], E, layers[l]["gate"].data_ptr(), bias_ptr, xs[l].data_ptr(), T,
                  H, F, K, outs[l].data_ptr(), None, wts[l].data_ptr(), idxs[l].data_ptr(),
                  ws.data_ptr(), ws_bytes) for l in range(L)]
    f_layer, f_prof = lib.moe_layer_forward_nf4, lib.moe_layer_forward_nf4_profiled
    hip = _HipEvents() if events else None

    def step(ev=None, prof_layer=-1):
        for l in range(L):
            if l != prof_layer:
                rc = f_layer(*call_args[l], stream)
            else:
                rc = f_prof(*call_args[l], ev, stream)
            if rc:
                _lib.check(rc, "moe_layer_forward_nf4")

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()

    # Routed experts per layer (inputs are fixed, so routing is the same every step).
    u_per_layer = [int(torch.unique(idxs[l]).numel()) for l in range(L)]

    evs = [hip.array4() for _ in range(steps)] if hip else None
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s_ in range(steps):
        if hip:
            step(evs[s_], s_ % L)
        else:
            step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_per_step = elapsed * 1e3 / steps

    gu_us = down_us = route_us = None
    if hip:
        # In the decode form the routing runs inside the gate/up kernel and events 0 and 1
        # are recorded back to back: no routing time of its own.
        route_us = None if decode_form(T, K, E, H, F) else hip.mean_us([(e[0], e[1]) for e in evs])
        gu_us = hip.mean_us([(e[1], e[2]) for e in evs])
        down_us = hip.mean_us([(e[2], e[3]) for e in evs])
    u_mean = sum(u_per_layer) / L
    prof_layers = [s_ % L for s_ in range(steps)]
    gu_bytes = sum(gateup_bytes(u_per_layer[l], H, F, T, K, E) for l in prof_layers) / len(prof_layers)
    ly_bytes = sum(layer_bytes(u, H, F, T, E) for u in u_per_layer) / L
    layer_us = ms_per_step * 1e3 / L
    layer_gbps = ly_bytes / (layer_us * 1e-6) / 1e9

    streamed = midbatch_form(T, K, E, H, F)
    mid = mid_form(T, K, E, H, F)
    if decode_form(T, K, E, H, F):
        gu_kernel = "decode_gateup_kernel (routing + NF4 w1/w3 GEMV + SwiGLU)"
    elif mid:
        gu_kernel = ("mid16_gateup_kernel (routing or grouping in the launch + NF4 w1/w3 "
                     "16x16x32 MFMA + SwiGLU)")
    elif gemm_form(T, K, E, H, F):
        gu_kernel = "expert_gemm_kernel<gate/up> (LDS-staged NF4 GEMM + SwiGLU)"
    elif streamed:
        gu_kernel = "midbatch_kernel<2> (streamed NF4 w1/w3 + SwiGLU, 32x32x16 MFMA)"
    else:
        gu_kernel = "skinny_kernel / gemv4_kernel (NF4 w1/w3 + SwiGLU)"
    roofline = None
    if gu_us and (decode_form(T, K, E, H, F) or streamed or mid):
        # Weight streaming: the routed experts' w1/w3 NF4 bytes per launch on the HBM roofline.
        ach = gu_bytes / (gu_us * 1e-6) / 1e9
        roofline = {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBPS,
                    "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBPS, 4),
                    "traffic": _traffic("gateup_nf4_decode_t%d" % T) if decode_form(T, K, E, H, F)
                    else None, "kernel": gu_kernel,
                    "bytes_per_launch": int(gu_bytes), "avg_launch_us": round(gu_us, 2)}
    elif gu_us:
        # Batches (prefill): the w1/w3 GEMMs, 2 x 2 * (T*k) * H * F flops per launch, on the
        # bf16 MFMA roofline.
        flops = 4.0 * T * K * H * F
        ach = flops / (gu_us * 1e-6) / 1e12
        roofline = {"bound": "mfma", "achieved": round(ach, 1), "peak": MFMA_BF16_TFLOPS,
                    "unit": "TFLOP/s", "frac": round(ach / MFMA_BF16_TFLOPS, 4), "traffic": None,
                    "kernel": gu_kernel, "flops_per_launch": flops, "avg_launch_us": round(gu_us, 2),
                    "gbps_algorithmic": round(gu_bytes / (gu_us * 1e-6) / 1e9, 1)}
    return {
        "ms_per_step": ms_per_step, "roofline": roofline, "nsplit": nsplit,
        "per_layer_us": round(layer_us, 2), "layer_hbm_gbps": round(layer_gbps, 1),
        "layer_hbm_frac": round(layer_gbps / HBM_PEAK_GBPS, 4),
        "routed_experts_per_layer": round(u_mean, 3),
        "kernels_us": {"route": None if route_us is None else round(route_us, 2),
                       "gateup": None if gu_us is None else round(gu_us, 2),
                       "down_combine": None if down_us is None else round(down_us, 2)},
        "kernel_events_in_timed_region": hip is not None,
    }


def _decode_layers(args) -> int:
    """``--mode decode``: the MoE-layer pass alone, L layers at ``--tokens`` per step."""
    import torch

    from moeinfra_amd import _lib, ops, synth

    H, F, E, K = synth.MIXTRAL_HIDDEN, synth.MIXTRAL_FFN, synth.MIXTRAL_EXPERTS, synth.MIXTRAL_TOPK
    L, T = args.layers, args.tokens
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    lib = _lib.lib()
    t_setup = time.time()
    gen = synth.make_generator(args.seed, device=dev)
    layers = []

    def quantize(e, w1, w3, w2):
        return {name: ops.nf4_quantize(w) for name, w in (("w1", w1), ("w3", w3), ("w2", w2))}

    for _ in range(L):
        lw = synth.make_layer(H, F, E, gen, device=dev, expert_sink=quantize)
        structs = [_lib.MoeNf4Expert(*(ex[n][i].data_ptr() for n in ("w1", "w3", "w2") for i in range(3)))
                   for ex in lw.experts]
        layers.append({"gate": lw.gate, "experts": lw.experts, "table": ops.expert_table(structs)})
    xs = [synth.make_activations(T, H, gen, device=dev) for _ in range(L)]
    bias = synth.zipf_bias(E, args.seed).to(dev) if args.routing == "zipf" else None
    torch.cuda.synchronize()
    setup_s = time.time() - t_setup

    r = _moe_pass(lib, layers, xs, bias, T, H, F, E, K, args.steps, args.warmup,
                  events=not args.no_kernel_events, routing=args.routing)
    cpu = None
    if not args.no_cpu_baseline:
        cpu = _cpu_baseline(layers, xs, bias, T, H, F, E, K, L, args.cpu_seconds)
    ms = r.pop("ms_per_step")
    nsplit = r.pop("nsplit")
    roofline = r.pop("roofline")
    result = {
        "metric": METRIC,
        "value": round(T / (ms * 1e-3), 3),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded bf16 N(0,0.02) weights NF4-quantised on the GPU; bf16 N(0,1) activations)",
        "config": {
            "workload": f"Mixtral-8x7B-shaped NF4 MoE expert path alone, {L} MoE layers, batch {T} "
                        "per step, all experts resident in HBM (router, permute, fused-dequant "
                        "SwiGLU, combine)",
            "hidden": H, "ffn": F, "experts": E, "top_k": K, "layers": L, "tokens_per_step": T,
            "routing": args.routing, "weights": "NF4 blocksize 64, fp32 absmax",
            "nsplit_down": nsplit, "parallelism": "single GPU",
        },
        "roofline": roofline,
        "cpu_baseline": cpu,
        **r,
        "setup_s": round(setup_s, 1),
    }
    print(json.dumps(result), flush=True)
    return 0


# ---------------------------------------------------------------------------- end to end
def _log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _e2e(args) -> int:
    import torch

    from moeinfra_amd import _lib, synth
    from moeinfra_amd.engine.decoder import MixtralShape, synthesize
    from moeinfra_amd.engine.engine import InferenceEngine
    from moeinfra_amd.engine.types import ForwardRequest, PrefetchPolicy

    s = MixtralShape(layers=args.layers)
    P, Ksteps, W = args.prompt, args.steps, args.warmup
    if P < 1 or Ksteps < 1 or W < 0:
        raise SystemExit("--prompt and --steps must be positive, --warmup non-negative")
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    lib = _lib.lib()
    t_setup = time.time()
    w = synthesize(s, seed=args.seed, device=dev, experts_on="cpu" if args.offload else None)
    prompt = torch.randint(0, s.vocab, (1, P), generator=torch.Generator().manual_seed(args.seed))
    policy = PrefetchPolicy(args.prefetch)
    eng = InferenceEngine(w, max_seq=P + max(Ksteps, W) + 8, device=dev, offload=args.offload,
                          gpu_expert_slots=args.gpu_expert_slots if args.offload else None,
                          prefetch=policy if args.offload else PrefetchPolicy.NONE,
                          prefetch_depth=args.prefetch_depth,
                          gpu_slots_per_layer=args.gpu_slots_per_layer if args.offload else None,
                          cache_policy=args.cache_policy,
                          prefetch_prefix_bytes=int(args.prefetch_prefix_mib * 2**20))
    _log(f"weights synthesized, engine built ({time.time() - t_setup:.1f} s)")
    eng.prepare(Ksteps + 1)
    torch.cuda.synchronize()
    setup_s = time.time() - t_setup
    _log(f"decode graph ready ({setup_s:.1f} s)")

    # Warm-up: one prompt and W decode steps.
    t_w = time.time()
    eng.generate(ForwardRequest(prompt, max_new_tokens=W + 1))
    torch.cuda.synchronize()
    warm_s = time.time() - t_w
    # Timed: prefill (ttft), then exactly Ksteps decode steps between two synchronizations.
    copies0 = dict(eng.transfer_scheduler.copies) if args.offload else None
    timeline = None
    if args.offload and args.copy_timeline:
        timeline = eng.transfer_scheduler.timeline = []
        t_base = torch.cuda.Event(enable_timing=True)
        t_base.record()
    res = eng.generate(ForwardRequest(prompt, max_new_tokens=Ksteps + 1))
    decode_ms = res.stage_timings["decode"]
    ms_per_step = decode_ms / Ksteps
    _log(f"timed: ttft {res.ttft_ms:.2f} ms, {Ksteps} decode steps {decode_ms:.2f} ms")
    u = [s.top_k] * s.layers  # batch 1: top-2 picks two distinct experts in every layer
    mid_pos = P + Ksteps // 2
    step_bytes = decode_step_bytes(s, u, mid_pos)
    step_gbps = step_bytes / (ms_per_step * 1e-3) / 1e9

    moe = None
    if not args.offload:
        gen = synth.make_generator(args.seed + 1, device=dev)
        xs = [synth.make_activations(1, s.hidden, gen, device=dev) for _ in range(s.layers)]
        layers = [{"gate": lw.gate, "table": lw.table} for lw in w.layers]
        moe = _moe_pass(lib, layers, xs, None, 1, s.hidden, s.ffn, s.experts, s.top_k, Ksteps,
                        W, events=not args.no_kernel_events)
        _log(f"MoE-layer pass: {moe['per_layer_us']} us/layer")

    cpu = None
    if not args.no_cpu_baseline:
        cpu = _cpu_baseline_e2e(eng, w, res.token_ids[-1], args.cpu_seconds)

    mode = "offload" if args.offload else "all-resident"
    config = {
        "workload": f"random-init Mixtral-8x7B-shaped model, {s.layers} decoder layers, NF4 experts "
                    + ("in pinned host memory with a bounded GPU expert cache"
                       if args.offload else "all resident in HBM")
                    + f"; {P}-token random-id prompt, then greedy decode at batch 1 (one step = "
                      "one decode token through the whole model"
                    + (")" if args.offload else ", one replay of the captured decode-step HIP graph)"),
        "mode": mode, "hidden": s.hidden, "ffn": s.ffn, "layers": s.layers, "experts": s.experts,
        "top_k": s.top_k, "heads": s.n_heads, "kv_heads": s.n_kv_heads, "head_dim": s.head_dim,
        "vocab": s.vocab, "rope_theta": s.rope_theta, "prompt_tokens": P, "decode_tokens": Ksteps,
        "weights": "attention/embeddings bf16, experts NF4 blocksize 64 fp32 absmax",
        "parallelism": "single GPU",
    }
    if args.offload:
        st = eng.cache_manager.stats()
        config.update({"gpu_expert_slots": args.gpu_expert_slots, "prefetch": args.prefetch,
                       "prefetch_depth": args.prefetch_depth,
                       "prefetch_prefix_mib": args.prefetch_prefix_mib,
                       "gpu_slots_per_layer": args.gpu_slots_per_layer,
                       "cache_policy": args.cache_policy})
    result = {
        "metric": METRIC,
        "value": round(res.tps, 3),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": Ksteps,
        "warmup": W,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded bf16 N(0,0.02) weights, experts NF4-quantised on the GPU; "
                "random prompt ids)",
        "config": config,
        "roofline": None if moe is None else moe.pop("roofline"),
        "cpu_baseline": cpu,
        "ttft_ms": round(res.ttft_ms, 2),
        "decode_step_bytes": step_bytes,
        "decode_step_hbm_gbps": round(step_gbps, 1),
        "decode_step_hbm_frac": round(step_gbps / HBM_PEAK_GBPS, 4),
        "setup_s": round(setup_s, 1),
        "warmup_s": round(warm_s, 2),
    }
    if moe is not None:
        moe_ms = moe.pop("ms_per_step")
        moe.pop("nsplit")
        result["moe_layer_pass"] = {"tok_s_moe_layers_only": round(1.0 / (moe_ms * 1e-3), 2),
                                    "ms_per_step": round(moe_ms, 4), **moe,
                                    "note": "the 32 MoE layers alone on fixed N(0,1) inputs, T=1; "
                                            "roofline events are in this pass's timed region"}
    if args.offload:
        c1 = eng.transfer_scheduler.copies
        moved = c1["bytes"] - copies0["bytes"]
        from moeinfra_amd.transfer import scheduler as sched_mod
        staging = [p.get("staging_ms", 0.0) for p in sched_mod.EXECUTE_NEXT_PROFILE]
        pe = eng.prefetch_engine
        result["offload_stats"] = {
            "cache_evictions": st.evictions,
            "expert_bytes": int(nf4_expert_bytes(s.hidden, s.ffn)),
            "pinned_store_bytes": eng.pinned_store.pinned_bytes,
            "copies_in_timed_run": {k: c1[k] - copies0[k] for k in ("image", "staged", "prefix")},
            "copies_per_decode_step": round((c1["image"] + c1["staged"] - copies0["image"]
                                             - copies0["staged"]) / (Ksteps + 1), 2),
            "host_link_gbps_timed_run": round(moved / ((res.ttft_ms + decode_ms) * 1e-3) / 1e9, 2),
            "execute_next_staging_ms_max": round(max(staging), 4) if staging else None,
            "prefetch": None if pe is None else dict(pe.counts),
        }
        if timeline is not None:
            eng.transfer_scheduler.timeline = None
            result["offload_stats"]["timeline"] = _copy_timeline(timeline, t_base, s.layers, Ksteps)
    print(json.dumps(result), flush=True)
    return 0


def _copy_timeline(timeline, t_base, layers: int, steps: int) -> dict:
    """Host-link and MoE-kernel intervals of the timed offload run (HIP events on the
    transfer and compute streams, in ns from t_base), summarised over its decode steps: the
    window runs from the end of the prompt pass's last MoE layer to the end of the last
    step's.  See moeinfra_amd.profiling.interval_stats."""
    import torch

    from moeinfra_amd import profiling

    torch.cuda.synchronize()
    ns = lambda ev: int(round(t_base.elapsed_time(ev) * 1e6))
    copies = [(ns(a), ns(b), int(n)) for kind, a, b, n in timeline if kind != "moe"]
    moe = [(ns(a), ns(b)) for kind, a, b, _ in timeline if kind == "moe"]
    if len(moe) != layers * (steps + 1):
        raise RuntimeError(f"timeline holds {len(moe)} MoE layers, expected {layers * (steps + 1)}")
    lo, hi = moe[layers - 1][1], moe[-1][1]
    stats = profiling.interval_stats(copies, moe, lo, hi, steps)
    stats = {k.replace("kernel", "moe_kernel"): round(v, 4) for k, v in stats.items()}
    stats["note"] = ("HIP events: each host-to-device copy on the transfer stream, each MoE layer's "
                     "expert kernels (permute, gate/up, down, combine) on the compute stream; "
                     "moe_kernel_* counts only those kernels")
    return stats


class _HipEvents:
    """Raw hipEvent_t handles (libamdhip64) for the profiled layer entry point, created with
    hipEventDisableSystemFence: timing-only events whose record skips the system-scope
    cache write-back, so they perturb the launches they bracket as little as possible."""

    DISABLE_SYSTEM_FENCE = 0x20000000

    def __init__(self):
        import ctypes

        self.ct = ctypes
        self.hip = ctypes.CDLL("libamdhip64.so")
        self.hip.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
        self.hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p,
                                                 ctypes.c_void_p]
        self.hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self.all = []

    def array4(self):
        arr = (self.ct.c_void_p * 4)()
        for i in range(4):
            h = self.ct.c_void_p()
            if self.hip.hipEventCreateWithFlags(self.ct.byref(h), self.DISABLE_SYSTEM_FENCE) != 0:
                raise RuntimeError("hipEventCreateWithFlags failed")
            arr[i] = h
            self.all.append(h)
        return arr

    def mean_us(self, pairs):
        ms = self.ct.c_float()
        tot = 0.0
        for a, b in pairs:
            if self.hip.hipEventElapsedTime(self.ct.byref(ms), a, b) != 0:
                raise RuntimeError("hipEventElapsedTime failed")
            tot += ms.value
        return 1e3 * tot / len(pairs)


def _copy_calibration(mib: int) -> int:
    """Ten device-to-device copies of `mib` MiB (reads and writes exactly that many bytes
    each): the reference kernel for converting FETCH_SIZE / WRITE_SIZE counter readings to
    bytes."""
    import torch

    n = mib << 20
    src = torch.empty(n, dtype=torch.uint8, device="cuda:0").fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": n, "copies": 10}), flush=True)
    return 0


def _reconstruct(args) -> int:
    """Standalone reconstruction of one Mixtral-8x7B expert (w1, w3 [14336, 4096], w2
    [4096, 14336]): (a) NF4 resident in HBM -> bf16 with the dequant kernel (451,411,968
    algorithmic bytes per expert: 99,090,432 read + 352,321,536 written); (b) from a pinned
    host staging slot (the reference's ReusablePinnedStagingPool hand-off): H2D of the
    99,090,432 NF4 bytes on a side stream, then the dequant.  Synthetic bf16 N(0, 0.02)
    weights quantised on the GPU."""
    import torch

    from moeinfra_amd import _lib, ops, synth

    H, F = synth.MIXTRAL_HIDDEN, synth.MIXTRAL_FFN
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    lib = _lib.lib()
    gen = torch.Generator(device=dev).manual_seed(args.seed)
    mats = {}
    for name, shape in (("w1", (F, H)), ("w3", (F, H)), ("w2", (H, F))):
        w = (torch.randn(shape, generator=gen, device=dev) * 0.02).to(torch.bfloat16)
        packed, absmax, code = ops.nf4_quantize(w)
        mats[name] = (packed, absmax, code, shape, torch.empty(shape, dtype=torch.bfloat16, device=dev))
        del w
    # Measured ceilings for the same traffic shapes: a device copy (read + write of n bytes)
    # and a fill (write only).
    n = 256 << 20
    src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
    dstc = torch.empty_like(src)
    c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for _ in range(3):
        dstc.copy_(src)
    c0.record()
    for _ in range(10):
        dstc.copy_(src)
    c1.record()
    torch.cuda.synchronize()
    copy_gbps = 2 * n / (c0.elapsed_time(c1) * 1e-3 / 10) / 1e9
    c0.record()
    for _ in range(10):
        dstc.fill_(3)
    c1.record()
    torch.cuda.synchronize()
    fill_gbps = n / (c0.elapsed_time(c1) * 1e-3 / 10) / 1e9
    del src, dstc
    nf4_bytes = sum(m[0].numel() + m[1].numel() * 4 for m in mats.values())
    alg = nf4_bytes + sum(m[4].numel() * 2 for m in mats.values())
    stream = torch.cuda.current_stream(dev)

    def dequant_all(src):
        for name, (packed, absmax, code, shape, out) in mats.items():
            p, a = src[name] if src else (packed, absmax)
            rc = lib.moe_nf4_dequant_bf16(p.data_ptr(), a.data_ptr(), code.data_ptr(),
                                          out.data_ptr(), out.numel(), 64, stream.cuda_stream)
            _lib.check(rc, "moe_nf4_dequant_bf16")

    reps = max(args.steps, 10)
    for _ in range(3):
        dequant_all(None)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        dequant_all(None)
    e1.record(stream)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / reps
    gbps = alg / (us * 1e-6) / 1e9
    print(json.dumps({
        "metric": "NF4 expert reconstruction from HBM (K1 dequant, w1+w3+w2)", "value": round(gbps, 1),
        "unit": "GB/s", "n_gpus": 1, "steps": reps, "higher_is_better": True, "dtype": "u8->bf16",
        "data": "synthetic (bf16 N(0,0.02) weights NF4-quantised on the GPU)",
        "config": {"workload": "one Mixtral-8x7B expert, w1/w3 [14336,4096] + w2 [4096,14336], NF4 blocksize 64"},
        "us_per_expert": round(us, 2), "bytes_per_expert": alg,
        "measured_ceilings_gbps": {"device_copy_read_plus_write": round(copy_gbps, 1),
                                   "fill_write_only": round(fill_gbps, 1)},
        "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gbps / HBM_PEAK_GBPS, 4), "kernel": "nf4_dequant_kernel"}}), flush=True)

    # (b) pinned host slot -> device (side stream) -> dequant
    host = {n: (m[0].cpu().pin_memory(), m[1].cpu().pin_memory()) for n, m in mats.items()}
    dst = {n: (torch.empty_like(m[0]), torch.empty_like(m[1])) for n, m in mats.items()}
    side = torch.cuda.Stream(dev)
    torch.cuda.synchronize()
    t_h2d, t_all = [], []
    for it in range(reps + 2):
        a0 = torch.cuda.Event(enable_timing=True)
        a1 = torch.cuda.Event(enable_timing=True)
        a2 = torch.cuda.Event(enable_timing=True)
        a0.record(side)
        with torch.cuda.stream(side):
            for n in mats:
                dst[n][0].copy_(host[n][0], non_blocking=True)
                dst[n][1].copy_(host[n][1], non_blocking=True)
        a1.record(side)
        stream.wait_stream(side)
        dequant_all(dst)
        a2.record(stream)
        torch.cuda.synchronize()
        if it >= 2:
            t_h2d.append(a0.elapsed_time(a1) * 1e3)
            t_all.append(a0.elapsed_time(a2) * 1e3)
    t_h2d.sort()
    t_all.sort()
    h2d_us, all_us = t_h2d[len(t_h2d) // 2], t_all[len(t_all) // 2]
    print(json.dumps({
        "metric": "NF4 expert H2D staging (pinned slot -> HBM) + reconstruction", "value": round(nf4_bytes / (h2d_us * 1e-6) / 1e9, 2),
        "unit": "GB/s (H2D)", "n_gpus": 1, "steps": reps, "higher_is_better": True, "dtype": "u8",
        "data": "synthetic (bf16 N(0,0.02) weights NF4-quantised on the GPU, copied to pinned host memory)",
        "config": {"workload": "one Mixtral-8x7B expert: 99,090,432 NF4 bytes host -> device on a side stream, then K1"},
        "h2d_us_median": round(h2d_us, 1), "h2d_plus_dequant_us_median": round(all_us, 1),
        "bytes_h2d": nf4_bytes}), flush=True)
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


def _cpu_baseline_e2e(eng, weights, last_token: int, budget_s: float):
    """The CPU oracle decoder on a bounded sample of one decode token: layers one at a time
    (each with the engine's KV cache of that layer as its history, so attention spans the
    same positions), each timed from its input norm to its output (attention, router, the
    NF4 dequantisation of its two routed experts, SwiGLU, combine), then the final norm and
    lm_head; the mean layer time is scaled to the model's layers."""
    import torch

    from oracle.decoder_oracle import RefDecoder, rmsnorm

    cores = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS")
    threads = min(cores, int(omp)) if omp and omp.isdigit() and int(omp) > 0 else cores
    torch.set_num_threads(threads)
    s = weights.shape
    dec = eng.decoder
    pos = int(dec.pos.item())
    h0 = weights.embed[last_token:last_token + 1].detach().cpu()
    times = []
    t_start = time.perf_counter()
    for li in range(s.layers):
        ref = RefDecoder(weights, layers=[li], threads=threads)
        ref.k[0] = dec.k_cache[li, :, :pos].cpu()
        ref.v[0] = dec.v_cache[li, :, :pos].cpu()
        ref.pos = pos
        t0 = time.perf_counter()
        ref.layer(0, h0)
        times.append(time.perf_counter() - t0)
        del ref
        if time.perf_counter() - t_start > budget_s:
            break
    ref = RefDecoder(weights, layers=0, threads=threads)
    t0 = time.perf_counter()
    with torch.no_grad():
        (rmsnorm(h0, ref.final_norm, s.rms_eps) @ ref.lm_head.t()).float()
    head_s = time.perf_counter() - t0
    per_layer = sum(times) / len(times)
    per_token = per_layer * s.layers + head_s
    return {"value": round(1.0 / per_token, 5), "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"CPU oracle decoder (torch CPU bf16 attention on {threads} threads, C NF4 "
                      f"dequant of the 2 routed experts on {threads} threads, numpy fp32 SwiGLU) "
                      f"for one decode token at position {pos} through {len(times)} of {s.layers} "
                      f"layers (mean {per_layer * 1e3:.1f} ms/layer) + lm_head "
                      f"({head_s * 1e3:.1f} ms), scaled to {s.layers} layers"}


if __name__ == "__main__":
    sys.exit(main())
