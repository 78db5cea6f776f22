"""The reference-compatible Python API on the GPU: expert containers, the staged H2D
transfer path, and MoELayer in all-resident and offload modes, each checked against the
oracle; plus a full Mixtral-8x7B-shape layer (hidden 4096, FFN 14336, 8 experts, top-2)."""
from __future__ import annotations

import time
import types

import numpy as np
import pytest
import torch

from helpers import bits, build_layer, near_tie_rows, oracle_layer
from oracle import moe_oracle as orc

pytestmark = pytest.mark.gpu

TOL = 1e-2   # rel-L2 bound on expert / layer outputs


def _layer_err(got_bits, want_bits, logits_bits):
    """rel-L2 over the tokens whose top-k is not decided by a 1-ulp logit tie (the device
    and the oracle round the gate logits independently)."""
    ok = ~near_tie_rows(logits_bits)
    assert ok.sum() >= max(1, ok.size // 2)
    return orc.rel_l2(orc.bf16_to_f32(got_bits[ok]), orc.bf16_to_f32(want_bits[ok]))


def _bf16(shape, seed, std=0.02):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * std).to(torch.bfloat16)


def _serialized(packed, absmax, shape):
    from moeinfra_amd.model.expert import NF4QuantState

    code = torch.from_numpy(orc.NF4_CODE.copy())
    qs = NF4QuantState(absmax=torch.from_numpy(absmax.copy()), code=code, shape=torch.Size(shape))
    return {"weight": torch.from_numpy(packed.copy()).reshape(-1, 1),
            "weight.absmax": qs.absmax, "weight.quant_map": code,
            "weight.quant_state.bitsandbytes__nf4": qs.blob()}


def _prequantized(ex):
    """helpers.NF4Expert (oracle-quantised) -> the CPU-authoritative serialized expert."""
    from moeinfra_amd.model.expert import PrequantizedNF4Expert

    shapes = {"w1": (ex.inter, ex.hidden), "w3": (ex.inter, ex.hidden),
              "w2": (ex.hidden, ex.inter)}
    s = {n: _serialized(*ex.np[n], shapes[n]) for n in ("w1", "w2", "w3")}
    return PrequantizedNF4Expert.from_serialized(s["w1"], s["w2"], s["w3"], ex.hidden, ex.inter)


def _resident(ex, device):
    """helpers.NF4Expert -> ReconstructedNF4Expert over device copies of its tensors."""
    from moeinfra_amd.transfer.nf4_reconstruct import ReconstructedNF4Expert

    code = torch.from_numpy(orc.NF4_CODE.copy()).to(device)
    state = {n: {"weight": torch.from_numpy(p.copy()).reshape(-1, 1).to(device),
                 "absmax": torch.from_numpy(a.copy()).to(device), "code": code, "offset": None}
             for n, (p, a) in ex.np.items()}
    meta = types.SimpleNamespace(hidden_size=ex.hidden, intermediate_size=ex.inter)
    return ReconstructedNF4Expert(meta, state)


def test_quantized_expert_cuda_matches_oracle(cuda_device):
    from moeinfra_amd.model.expert import QuantizedMixtralExpert

    H, F = 256, 512
    w1, w2, w3 = _bf16((F, H), 1), _bf16((H, F), 2), _bf16((F, H), 3)
    ex = QuantizedMixtralExpert(w1, w2, w3)
    assert ex.device.type == "cpu" and ex.size_bytes == 3 * H * F * 2
    ex.cuda()
    assert ex.device.type == "cuda" and ex.size_bytes == 3 * H * F // 2
    state = {}
    for name, w in (("w1", w1), ("w2", w2), ("w3", w3)):
        lin = getattr(ex, name)
        p, a = orc.nf4_quantize(bits(w).reshape(-1))
        np.testing.assert_array_equal(lin.weight.cpu().numpy().reshape(-1), p)
        np.testing.assert_array_equal(lin.quant_state.absmax.cpu().numpy(), a)
        np.testing.assert_array_equal(bits(lin.dequantize()).reshape(-1), orc.nf4_dequant(p, a))
        state[name] = (p, a)
    sd = ex.state_dict()
    assert {"w1.weight", "w1.weight.absmax", "w1.weight.quant_map",
            "w1.weight.quant_state.bitsandbytes__nf4"} <= set(sd)
    x = _bf16((3, H), 4, 1.0)
    want = orc.swiglu(bits(x), *orc.dequant_expert(state, H, F))
    got = ex(x.to(cuda_device))
    assert got.dtype == torch.bfloat16
    assert orc.rel_l2(orc.bf16_to_f32(bits(got)), orc.bf16_to_f32(want)) < TOL
    got32 = ex(x.float().to(cuda_device))
    assert got32.dtype == torch.float32
    np.testing.assert_array_equal(bits(got32.to(torch.bfloat16)), bits(got))


def _transfer_rig(cm, budget_slots, slot_bytes):
    from moeinfra_amd.transfer.pinned_memory import PinnedMemoryBudget
    from moeinfra_amd.transfer.reusable_staging import ReusablePinnedStagingPool
    from moeinfra_amd.transfer.scheduler import TransferScheduler

    pool = ReusablePinnedStagingPool(PinnedMemoryBudget(budget_slots * slot_bytes), slot_bytes)
    stream = torch.cuda.Stream()
    return TransferScheduler(cm, 24.0, 4, staging_pool=pool, transfer_stream=stream), pool


def _req(layer, e):
    from moeinfra_amd.transfer.types import TransferDirection, TransferPriority, TransferRequest

    return TransferRequest(f"t-{layer}-{e}-{time.monotonic_ns()}", layer, e,
                           TransferDirection.CPU_TO_GPU, TransferPriority.HIGH, time.monotonic())


def test_staged_transfer_reconstructs_the_expert(cuda_device):
    from moeinfra_amd.cache.manager import CacheManager
    from moeinfra_amd.cache.types import EvictionPolicy
    from moeinfra_amd.transfer.nf4_reconstruct import ReconstructedNF4Expert

    H, F = 512, 1024
    gate, experts, x = build_layer(H, F, 2, 4, seed=5)
    cm = CacheManager(gpu_slots=1, cpu_slots=4, policy=EvictionPolicy.LRU)
    cpu = [_prequantized(e) for e in experts]
    for e, ex in enumerate(cpu):
        cm.put(0, e, ex, "cpu")
    sch, pool = _transfer_rig(cm, 1, cpu[0].size_bytes)
    for e in range(2):
        assert sch.submit(_req(0, e))
        r = sch.execute_next()
        assert r.success, r.error
        assert r.bytes_transferred == cpu[e].size_bytes
        g = cm.peek_gpu(0, e)
        assert isinstance(g, ReconstructedNF4Expert) and g.device.type == "cuda"
        assert torch.equal(g.w2.weight.cpu(), cpu[e].w2["weight"])
        assert cm.peek_cpu(0, e) is cpu[e]                     # CPU copy stays authoritative
        want = orc.swiglu(bits(x), *experts[e].dequant_np())
        assert orc.rel_l2(orc.bf16_to_f32(bits(g(x.to(cuda_device)))),
                          orc.bf16_to_f32(want)) < TOL
    assert pool.slot_count == 1 and pool.active_slots == 0     # one slot, reused
    slot = next(iter(pool._slots.values()))
    assert all(t.is_pinned() for proj in slot.tensors.values() for t in proj.values()
               if t is not None)
    assert not cpu[0].w1["weight"].is_pinned()                 # the source stays pageable
    assert cm.stats().gpu_slots_used == 1                      # gpu_slots=1: expert 0 evicted
    assert not cm.is_gpu_resident(0, 0) and cm.is_gpu_resident(0, 1)


def _pinned(experts, device):
    """helpers.NF4Expert list -> PinnedNF4Expert list (one pinned arena)."""
    from moeinfra_amd.transfer.host_store import PinnedExpertStore

    store = PinnedExpertStore()
    return store, store.add_layer([_prequantized(e) for e in experts])


def test_async_transfers_publish_at_once_and_order_the_compute(cuda_device):
    """submit_async makes each expert GPU-resident immediately, behind its copy's event; a
    layer launched right away (no host synchronisation) must see the copied weights, which
    only the stream waits guarantee.  Experts come from the pinned store (one copy each, no
    staging); cancellation drops an in-flight expert."""
    from moeinfra_amd.cache.manager import CacheManager
    from moeinfra_amd.cache.types import EvictionPolicy
    from moeinfra_amd.transfer.scheduler import TransferScheduler
    from moeinfra_amd.transfer.types import TransferStatus

    H, F, E, T = 1024, 3584, 8, 12
    gate, experts, x = build_layer(H, F, E, T, seed=61)
    store, pinned = _pinned(experts, cuda_device)
    assert all(t.is_pinned() for a in store.arenas for t in (a,))
    cm = CacheManager(gpu_slots=E, cpu_slots=2 * E, policy=EvictionPolicy.LRU)
    for e, ex in enumerate(pinned):
        cm.put(0, e, ex, "cpu")
    cm.put(1, 0, pinned[0], "cpu")
    sch = TransferScheduler(cm, 24.0, 2 * E, transfer_stream=torch.cuda.Stream())
    handles = [sch.submit_async(_req(0, e)) for e in range(E)]
    # Every copy started (a handle turns READY once its copy has finished).
    assert all(h.event is not None and h.status in (TransferStatus.IN_FLIGHT, TransferStatus.READY)
               for h in handles)
    assert all(cm.is_gpu_resident(0, e) for e in range(E))
    again = sch.submit_async(_req(0, 0))
    assert again is handles[0] or again.status == TransferStatus.READY
    layer = _layer(cm, gate, cuda_device, scheduler=sch)
    out = layer.forward(x.to(cuda_device))                     # all-resident path, no sync
    want, (lg, _, _) = oracle_layer(gate, experts, x)
    assert _layer_err(bits(out), want, lg) < TOL
    h = sch.submit_async(_req(1, 0))
    assert h.status == TransferStatus.IN_FLIGHT and sch.cancel(h.request_id)
    assert not cm.is_gpu_resident(1, 0)
    torch.cuda.synchronize()
    assert sch.poll_async(1, 0) == TransferStatus.CANCELLED
    assert sch.poll_async(0, 3) == TransferStatus.READY
    assert sch.poll_async(0, 3) == TransferStatus.REJECTED      # retired
    # Once observed complete, every copy reached the bandwidth monitor once (the cancelled
    # one did not).
    for e in range(E):
        sch.poll_async(0, e)
    assert sch.bandwidth_monitor.bytes_in_window() == sum(h.nbytes for h in handles) > 0


def test_device_slots_are_leased_to_live_experts(cuda_device):
    """With two device slots, a third transferred expert that is still referenced elsewhere
    gets a buffer of its own; dropped experts give their slots back (fenced), and every
    expert dequantises bit-exactly whichever memory it landed in."""
    from moeinfra_amd.cache.manager import CacheManager
    from moeinfra_amd.cache.types import EvictionPolicy
    from moeinfra_amd.transfer.device_slots import DeviceExpertSlots
    from moeinfra_amd.transfer.scheduler import TransferScheduler

    H, F = 256, 512
    _, experts, _ = build_layer(H, F, 3, 1, seed=62)
    _store, pinned = _pinned(experts, cuda_device)
    cm = CacheManager(gpu_slots=2, cpu_slots=3, policy=EvictionPolicy.LRU)
    for e, ex in enumerate(pinned):
        cm.put(0, e, ex, "cpu")
    slots = DeviceExpertSlots(2, pinned[0].image_layout.nbytes, cuda_device)
    sch = TransferScheduler(cm, 24.0, 4, transfer_stream=torch.cuda.Stream(), device_slots=slots)
    held = []
    for e in range(3):
        assert sch.submit(_req(0, e)) and sch.execute_next().success
        held.append(cm.peek_gpu(0, e))
    assert slots.free_count == 0 and not cm.is_gpu_resident(0, 0)   # (0, 0) evicted, still held
    inside = [slots._mem.data_ptr() <= g.w1.weight.data_ptr() < slots._mem.data_ptr() + slots._mem.numel()
              for g in held]
    assert inside == [True, True, False]
    for e, g in enumerate(held):
        for n in ("w1", "w2", "w3"):
            want = orc.nf4_dequant(*experts[e].np[n])
            np.testing.assert_array_equal(bits(getattr(g, n).dequantize()).reshape(-1), want)
    sch._async.clear()
    held.clear()
    cm.demote_to_cpu(0, 1)
    cm.demote_to_cpu(0, 2)
    assert slots.free_count == 2 and all(slots.fence(i) is not None for i in range(2))


def _layer(cm, gate, device, layer_id=0, scheduler=None):
    from moeinfra_amd.engine.router import ExpertRouter
    from moeinfra_amd.model.moe_layer import MoELayer

    return MoELayer(layer_id, ExpertRouter(gate.to(device), 2), cm, model_loader=None,
                    transfer_scheduler=scheduler)


@pytest.mark.parametrize("T", [1, 5, 40])
def test_moe_layer_all_resident(cuda_device, T):
    from moeinfra_amd.cache.manager import CacheManager
    from moeinfra_amd.cache.types import EvictionPolicy

    H, F, E = 512, 1024, 8
    gate, experts, x = build_layer(H, F, E, T, seed=10 + T)
    cm = CacheManager(gpu_slots=E, cpu_slots=E, policy=EvictionPolicy.LRU)
    for e, ex in enumerate(experts):
        cm.put(0, e, _resident(ex.to(cuda_device), cuda_device), "cuda:0")
    layer = _layer(cm, gate, cuda_device)
    want, (lg, _, _) = oracle_layer(gate, experts, x)
    out1 = layer.forward(x.to(cuda_device))
    out2 = layer.forward(x.to(cuda_device).reshape(1, T, H))   # cached table + workspace
    assert _layer_err(bits(out1), want, lg) < TOL
    np.testing.assert_array_equal(bits(out2).reshape(T, H), bits(out1))


def test_moe_layer_offload(cuda_device):
    from moeinfra_amd.cache.manager import CacheManager
    from moeinfra_amd.cache.types import EvictionPolicy

    H, F, E, T = 512, 1024, 8, 12
    gate, experts, x = build_layer(H, F, E, T, seed=21)
    cm = CacheManager(gpu_slots=E, cpu_slots=E, policy=EvictionPolicy.LRU)
    for e, ex in enumerate(experts):
        cm.put(0, e, _prequantized(ex), "cpu")
    for e in (0, 3):                                           # two experts already resident
        cm.put(0, e, _resident(experts[e].to(cuda_device), cuda_device), "cuda:0")
    sch, pool = _transfer_rig(cm, 1, cm.get_size_bytes(0, 1))
    layer = _layer(cm, gate, cuda_device, scheduler=sch)
    want, (lg, _, idx) = oracle_layer(gate, experts, x)
    out = layer.forward(x.to(cuda_device))
    assert _layer_err(bits(out), want, lg) < TOL
    routed = set(np.unique(idx).tolist())
    assert routed - {0, 3}, "routing should need at least one transfer"
    assert cm.is_gpu_resident(0, 0) and cm.is_gpu_resident(0, 3)
    assert not any(cm.is_gpu_resident(0, e) for e in routed - {0, 3})
    assert pool.active_slots == 0 and sch.pending_count() == 0


# --------------------------------------------------------------------------- full size
_FULL = {}


def _full_layer(device):
    """Mixtral-8x7B MoE layer shape, weights drawn and NF4-quantised on the GPU."""
    if "layer" not in _FULL:
        from moeinfra_amd import ops

        H, F, E = 4096, 14336, 8
        g = torch.Generator(device=device).manual_seed(1234)
        experts, keep = [], []
        for e in range(E):
            st = {}
            for name, shape in (("w1", (F, H)), ("w3", (F, H)), ("w2", (H, F))):
                w = (torch.randn(shape, generator=g, device=device) * 0.02).to(torch.bfloat16)
                p, a, code = ops.nf4_quantize(w)
                st[name] = (p, a, code)
                del w
            keep.append(st)
        gate = (torch.randn((E, H), generator=g, device=device) * 0.02).to(torch.bfloat16)
        from moeinfra_amd._lib import MoeNf4Expert

        structs = [MoeNf4Expert(*(t.data_ptr() for n in ("w1", "w3", "w2") for t in st[n]))
                   for st in keep]
        _FULL["layer"] = (H, F, E, gate, keep, ops.expert_table(structs))
    return _FULL["layer"]


@pytest.mark.parametrize("T", [1, 4, 32])
def test_full_size_layer_matches_oracle(cuda_device, T):
    from moeinfra_amd import ops

    H, F, E, gate, keep, table = _full_layer(cuda_device)
    gen = torch.Generator(device=cuda_device).manual_seed(T)
    x = torch.randn((T, H), generator=gen, device=cuda_device).to(torch.bfloat16)
    out, _, w, idx = ops.layer_forward(table, E, gate, x, 2, F)
    torch.cuda.synchronize()
    xb, gb = bits(x), bits(gate)
    cache = {}

    def expert_fn(e, rows):
        if e not in cache:
            st = {n: (keep[e][n][0].cpu().numpy().reshape(-1), keep[e][n][1].cpu().numpy())
                  for n in ("w1", "w3", "w2")}
            cache[e] = orc.dequant_expert(st, H, F, threads=8)
        return orc.swiglu(rows, *cache[e])

    want, (lg_o, w_o, idx_o) = orc.moe_layer(xb, gb, expert_fn)
    ok = ~near_tie_rows(lg_o)
    np.testing.assert_array_equal(idx.cpu().numpy()[ok], idx_o[ok])
    np.testing.assert_allclose(w.cpu().numpy()[ok], w_o[ok], rtol=1e-5, atol=1e-6)
    err = _layer_err(bits(out), want, lg_o)
    print(f"full-size layer T={T}: rel-L2 {err:.2e}", flush=True)
    assert err < TOL


# --------------------------------------------------------------------------- nested absmax
def test_expand_absmax_kernel(cuda_device):
    """moe_nf4_expand_absmax against the oracle, bit for bit (a Mixtral w1 absmax count plus
    an odd tail; offsets zero and non-zero)."""
    from moeinfra_amd import ops

    rng = np.random.default_rng(11)
    for n, off in ((14336 * 4096 // 64, 0.0), (1037, 0.0123)):
        q = rng.integers(0, 256, n, dtype=np.uint8)
        a2 = (rng.random(-(-n // 256), dtype=np.float32) * 0.05 + 1e-4).astype(np.float32)
        c2 = np.sort(rng.standard_normal(256).astype(np.float32))
        got = ops.nf4_expand_absmax(torch.from_numpy(q).to(cuda_device),
                                    torch.from_numpy(a2).to(cuda_device),
                                    torch.from_numpy(c2).to(cuda_device), off, 256)
        want = orc.expand_absmax(q, a2, c2, off, 256)
        np.testing.assert_array_equal(got.cpu().numpy().view(np.uint32), want.view(np.uint32))


def test_nested_expert_from_store_to_gpu(cuda_device, tmp_path):
    """A nested (double-quantised) expert written to the on-disk store, read back, staged and
    transferred through the scheduler: each projection dequantises bit-exactly to the
    oracle's dequant with the expanded absmax, and the expert's forward equals, bit for
    bit, that of the same expert holding the expanded absmax as fp32."""
    from moeinfra_amd.cache.manager import CacheManager
    from moeinfra_amd.cache.types import EvictionPolicy
    from moeinfra_amd.model.expert import NF4QuantState, PrequantizedNF4Expert
    from moeinfra_amd.model.store import NF4ExpertStore, save_expert

    H, F = 512, 1024
    _gate, experts, x = build_layer(H, F, 1, 3, seed=9)
    ex = experts[0]
    shapes = {"w1": (F, H), "w3": (F, H), "w2": (H, F)}
    nested, flat, expanded = {}, {}, {}
    for n in ("w1", "w2", "w3"):
        packed, absmax = ex.np[n]
        q, a2, c2, off = orc.double_quantize_absmax(absmax, 256)
        expanded[n] = orc.expand_absmax(q, a2, c2, off, 256)
        code = torch.from_numpy(orc.NF4_CODE.copy())
        qs = NF4QuantState(absmax=torch.from_numpy(q), code=code, shape=torch.Size(shapes[n]),
                           offset=torch.tensor(off),
                           state2=NF4QuantState(absmax=torch.from_numpy(a2), code=torch.from_numpy(c2),
                                                shape=torch.Size((q.size,)), blocksize=256,
                                                quant_type=None, dtype=torch.float32))
        nested[n] = {"weight": torch.from_numpy(packed.copy()).reshape(-1, 1),
                     "weight.absmax": qs.absmax, "weight.quant_map": code,
                     "weight.nested_absmax": qs.state2.absmax,
                     "weight.nested_quant_map": qs.state2.code,
                     "weight.quant_state.bitsandbytes__nf4": qs.blob()}
        flat[n] = _serialized(packed, expanded[n], shapes[n])
    save_expert(tmp_path, 0, 0, PrequantizedNF4Expert.from_serialized(
        nested["w1"], nested["w2"], nested["w3"], H, F))
    back = NF4ExpertStore([tmp_path], H, F).load_expert(0, 0)
    flat_ex = PrequantizedNF4Expert.from_serialized(flat["w1"], flat["w2"], flat["w3"], H, F)
    gpu = []
    # One staging rig each: a slot's pinned buffers are reused only for tensors of the same
    # layout (the nested absmax is uint8, the flat one fp32).
    for ex_cpu in (back, flat_ex):
        cm = CacheManager(gpu_slots=1, cpu_slots=1, policy=EvictionPolicy.LRU)
        cm.put(0, 0, ex_cpu, "cpu")
        sch, _pool = _transfer_rig(cm, 1, ex_cpu.size_bytes)
        assert sch.submit(_req(0, 0))
        r = sch.execute_next()
        assert r.success, r.error
        gpu.append(cm.peek_gpu(0, 0))
    gn, gf = gpu
    for n in ("w1", "w2", "w3"):
        lin = getattr(gn, n)
        assert lin.quant_state.nested
        got = bits(lin.dequantize())
        want = orc.nf4_dequant(ex.np[n][0], expanded[n]).reshape(got.shape)
        np.testing.assert_array_equal(got, want)
    xd = x.to(cuda_device)
    np.testing.assert_array_equal(bits(gn(xd)), bits(gf(xd)))


def test_fused_entries_reject_overlapping_residual_out(cuda_device):
    """The fused single-token entry points write residual_out from one workgroup while the
    others still read x, residual, the norm weight and the gate (or projection weight), and
    the MoE layer's down kernel writes out afterwards: a residual_out overlapping any of
    them, an out overlapping residual_out, or a null expert table, is refused before any
    launch."""
    from moeinfra_amd import _lib
    lib = _lib.lib()
    H, F, E, k = 4096, 14336, 8, 2
    nq, nkv, hd = 32, 8, 128
    buf = torch.zeros((6, H), dtype=torch.bfloat16, device=cuda_device)
    x, res, nw, out, good, misc = (buf[i].data_ptr() for i in range(6))
    gate = torch.zeros((E, H), dtype=torch.bfloat16, device=cuda_device)
    wqkv = torch.zeros(((nq + 2 * nkv) * hd, H), dtype=torch.bfloat16, device=cuda_device)
    table = (_lib.MoeNf4Expert * E)()
    ws = torch.zeros((1 << 20,), dtype=torch.uint8, device=cuda_device)

    def layer(experts, res_out, out_ptr=out):
        return lib.moe_layer_forward_nf4_norm(experts, E, gate.data_ptr(), x, res, nw, 1e-5, H, F,
                                              k, res_out, out_ptr, misc, misc, ws.data_ptr(),
                                              ws.numel(), None)

    for bad in (x, res, x + 2 * H - 2, nw, gate.data_ptr() + 6 * H):
        with pytest.raises(ValueError, match="must not overlap"):
            _lib.check(layer(table, bad), "layer_norm")
    with pytest.raises(ValueError, match="out must not overlap residual_out"):
        _lib.check(layer(table, good, out_ptr=good + 2), "layer_norm")
    with pytest.raises(ValueError, match="null"):
        _lib.check(layer(None, good), "layer_norm")

    def qkv(res_out, residual):
        return lib.moe_qkv_rope_bf16(wqkv.data_ptr(), x, None, 1, residual, nw, 1e-5, H, nq, nkv,
                                     hd, misc, misc, 16, res_out, misc, misc, misc, None)

    for bad, residual in ((x, res), (res, res), (x, None), (nw, res),
                          (wqkv.data_ptr() + 2 * H * 100, res)):
        with pytest.raises(ValueError, match="must not overlap"):
            _lib.check(qkv(bad, residual), "qkv_rope")
