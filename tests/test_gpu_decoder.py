"""End-to-end decoder on the GPU: the dense kernels (RMSNorm, rotary + KV cache,
attention, GEMV) against CPU restatements of the Hugging Face modules the reference runs,
and the whole engine (prefill + greedy decode, graph-replayed and eager, all-resident and
offload) against the CPU reference decoder, teacher-forced on the engine's tokens."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from decoder_ref import RefDecoder, rel_l2, rmsnorm, rope, top2_gap
from helpers import bits

pytestmark = pytest.mark.gpu


def _bf16(shape, seed, std=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * std).to(torch.bfloat16)


def _ulps(a: torch.Tensor, b: torch.Tensor) -> np.ndarray:
    x = bits(a).astype(np.int32)
    y = bits(b).astype(np.int32)
    # bf16 bit patterns -> ordered integers (sign-magnitude to two's complement)
    x = np.where(x & 0x8000, -(x & 0x7FFF), x)
    y = np.where(y & 0x8000, -(y & 0x7FFF), y)
    return np.abs(x - y)


@pytest.mark.parametrize("T,H,with_res", [(1, 4096, True), (40, 4096, True), (3, 512, False)])
def test_add_rmsnorm(cuda_device, T, H, with_res):
    from moeinfra_amd import _lib

    x, r, w = _bf16((T, H), 1), _bf16((T, H), 2), _bf16((H,), 3, 0.5)
    dev = lambda t: t.to(cuda_device)
    out = torch.empty((T, H), dtype=torch.bfloat16, device=cuda_device)
    r_out = torch.empty_like(out)
    xd, rd, wd = dev(x), dev(r), dev(w)
    _lib.check(_lib.lib().moe_add_rmsnorm_bf16(xd.data_ptr(), rd.data_ptr() if with_res else 0,
                                               wd.data_ptr(), 1e-5, T, H,
                                               r_out.data_ptr() if with_res else 0, out.data_ptr(),
                                               torch.cuda.current_stream().cuda_stream), "norm")
    torch.cuda.synchronize()
    resid = x + r if with_res else x
    if with_res:
        np.testing.assert_array_equal(bits(r_out), bits(resid))        # one bf16 add: exact
    want = rmsnorm(resid, w, 1e-5)
    u = _ulps(out.cpu(), want)
    assert u.max() <= 1 and (u > 0).mean() < 0.02                     # fp32 sum order only


def test_rope_and_cache_write(cuda_device):
    from moeinfra_amd import _lib
    from moeinfra_amd.engine.decoder import MixtralShape, rope_inv_freq

    s = MixtralShape()
    T, p0, max_seq = 5, 37, 128
    qkv = _bf16((T, s.qkv_rows), 4)
    inv = rope_inv_freq(s)
    kc = torch.zeros((s.n_kv_heads, max_seq, s.head_dim), dtype=torch.bfloat16, device=cuda_device)
    vc = torch.zeros_like(kc)
    q = torch.empty((T, s.n_heads * s.head_dim), dtype=torch.bfloat16, device=cuda_device)
    pos = torch.tensor([p0], dtype=torch.int32, device=cuda_device)
    qd, invd = qkv.to(cuda_device), inv.to(cuda_device)
    _lib.check(_lib.lib().moe_rope_kv_bf16(qd.data_ptr(), T, s.n_heads, s.n_kv_heads, s.head_dim,
                                           invd.data_ptr(), pos.data_ptr(), max_seq, q.data_ptr(),
                                           kc.data_ptr(), vc.data_ptr(),
                                           torch.cuda.current_stream().cuda_stream), "rope")
    torch.cuda.synchronize()
    nq, nkv, hd = s.n_heads, s.n_kv_heads, s.head_dim
    positions = torch.arange(p0, p0 + T)
    want_q = rope(qkv[:, :nq * hd].reshape(T, nq, hd), positions, inv).reshape(T, -1)
    want_k = rope(qkv[:, nq * hd:(nq + nkv) * hd].reshape(T, nkv, hd), positions, inv)
    want_v = qkv[:, (nq + nkv) * hd:].reshape(T, nkv, hd)
    kc, vc = kc.cpu(), vc.cpu()
    assert _ulps(q.cpu(), want_q).max() <= 1                              # cos/sin libm last bit
    assert _ulps(kc[:, p0:p0 + T].transpose(0, 1).contiguous(), want_k).max() <= 1
    np.testing.assert_array_equal(bits(vc[:, p0:p0 + T].transpose(0, 1).contiguous()), bits(want_v))
    assert not kc[:, :p0].any() and not kc[:, p0 + T:].any()              # other rows untouched


@pytest.mark.parametrize("T,p0,max_seq,hd", [(1, 0, 256, 128), (1, 71, 256, 128), (40, 0, 256, 128),
                                             (7, 20, 256, 128), (1, 3000, 4096, 128),
                                             (16, 2040, 4096, 128),
                                             # a score sums over hd / 8 lanes: 4, 8 and 32 lanes
                                             (1, 71, 256, 32), (3, 200, 512, 64), (2, 129, 256, 256)])
def test_attention(cuda_device, T, p0, max_seq, hd):
    from moeinfra_amd import _lib

    nq, nkv = 32, 8
    S = p0 + T
    q = _bf16((T, nq, hd), 5)
    k = _bf16((nkv, S, hd), 6)
    v = _bf16((nkv, S, hd), 7)
    kc = torch.zeros((nkv, max_seq, hd), dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    kc[:, :S], vc[:, :S] = k, v
    out = torch.empty((T, nq * hd), dtype=torch.bfloat16, device=cuda_device)
    pos = torch.tensor([p0], dtype=torch.int32, device=cuda_device)
    qd, kd, vd = q.to(cuda_device), kc.to(cuda_device), vc.to(cuda_device)
    _lib.check(_lib.lib().moe_attention_bf16(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), T, nq, nkv,
                                             hd, pos.data_ptr(), max_seq, hd ** -0.5, out.data_ptr(),
                                             torch.cuda.current_stream().cuda_stream), "attention")
    torch.cuda.synchronize()
    # Reference: eager attention in fp32 with the bf16 roundings of the bf16 module.
    K = k.float().repeat_interleave(nq // nkv, dim=0)
    V = v.float().repeat_interleave(nq // nkv, dim=0)
    sc = torch.matmul(q.float().transpose(0, 1), K.transpose(1, 2)).to(torch.bfloat16)
    sc = (sc.float() * (hd ** -0.5)).to(torch.bfloat16).float()
    mask = torch.full((T, S), float("-inf"))
    for t in range(T):
        mask[t, :p0 + t + 1] = 0.0
    p = torch.softmax(sc + mask, dim=-1).to(torch.bfloat16).float()
    want = torch.matmul(p, V).transpose(0, 1).reshape(T, nq * hd)
    assert rel_l2(out.cpu(), want) < 4e-3


@pytest.mark.parametrize("T,N,K", [(1, 6144, 4096), (1, 4096, 4096), (1, 1000, 512), (4, 515, 1024)])
def test_gemv(cuda_device, T, N, K):
    from moeinfra_amd import _lib

    W = _bf16((N, K), 8, 0.02)
    x = _bf16((T, K), 9)
    y = torch.empty((T, N), dtype=torch.bfloat16, device=cuda_device)
    Wd, xd = W.to(cuda_device), x.to(cuda_device)
    _lib.check(_lib.lib().moe_gemv_bf16(Wd.data_ptr(), xd.data_ptr(), T, N, K, y.data_ptr(),
                                        torch.cuda.current_stream().cuda_stream), "gemv")
    torch.cuda.synchronize()
    want = (x.float() @ W.float().t()).to(torch.bfloat16)
    u = _ulps(y.cpu(), want)
    assert u.max() <= 1 and (u > 0).mean() < 0.05


# --------------------------------------------------------------------------- fused step
def _stream():
    return torch.cuda.current_stream().cuda_stream


def _unfused_norm(lib, x, res, w, eps=1e-5):
    out = torch.empty_like(x)
    r_out = torch.empty_like(x)
    _lib_check(lib.moe_add_rmsnorm_bf16(x.data_ptr(), 0 if res is None else res.data_ptr(),
                                        w.data_ptr(), eps, x.shape[0], x.shape[1], r_out.data_ptr(),
                                        out.data_ptr(), _stream()), "norm")
    return r_out, out


def _unfused_gemv(lib, W, x):
    y = torch.empty((x.shape[0], W.shape[0]), dtype=torch.bfloat16, device=x.device)
    _lib_check(lib.moe_gemv_bf16(W.data_ptr(), x.data_ptr(), x.shape[0], W.shape[0], W.shape[1],
                                 y.data_ptr(), _stream()), "gemv")
    return y


def _lib_check(rc, what):
    from moeinfra_amd import _lib

    _lib.check(rc, what)


@pytest.mark.parametrize("H,nq,nkv,hd,pos,row,with_res", [
    (4096, 32, 8, 128, 41, 7, True),     # Mixtral layer > 0
    (4096, 32, 8, 128, 0, 3, False),     # Mixtral layer 0: embedding row, no residual
    (512, 8, 2, 64, 13, -5, False),      # row ids outside the table clamp (to 0)
    (1024, 4, 4, 128, 63, 99, True),     # ... and to the last row
])
def test_qkv_rope_fused_matches_unfused(cuda_device, H, nq, nkv, hd, pos, row, with_res):
    """norm + q/k/v projection + rotary + cache write in one launch == the three kernels."""
    from moeinfra_amd import _lib
    from moeinfra_amd.engine.decoder import MixtralShape, rope_inv_freq

    lib = _lib.lib()
    rows, max_seq = 20, 64
    dev = cuda_device
    table = _bf16((rows, H), 11).to(dev)
    res = _bf16((1, H), 12).to(dev) if with_res else None
    nw = _bf16((H,), 13, 0.5).to(dev)
    W = _bf16(((nq + 2 * nkv) * hd, H), 14, 0.02).to(dev)
    inv = rope_inv_freq(MixtralShape(head_dim=hd)).to(dev)
    p0 = torch.tensor([pos], dtype=torch.int32, device=dev)
    rid = torch.tensor([row], dtype=torch.int64, device=dev)
    caches = [torch.zeros((nkv, max_seq, hd), dtype=torch.bfloat16, device=dev) for _ in range(4)]
    q_f = torch.empty((1, nq * hd), dtype=torch.bfloat16, device=dev)
    h_f = torch.empty((1, H), dtype=torch.bfloat16, device=dev)
    _lib.check(lib.moe_qkv_rope_bf16(W.data_ptr(), table.data_ptr(), rid.data_ptr(), rows,
                                     None if res is None else res.data_ptr(), nw.data_ptr(), 1e-5, H,
                                     nq, nkv, hd, inv.data_ptr(), p0.data_ptr(), max_seq,
                                     h_f.data_ptr(), q_f.data_ptr(), caches[0].data_ptr(),
                                     caches[1].data_ptr(), _stream()), "qkv_rope")
    x = table[min(max(row, 0), rows - 1)][None].contiguous()
    h_u, xn = _unfused_norm(lib, x, res, nw)
    qkv = _unfused_gemv(lib, W, xn)
    q_u = torch.empty_like(q_f)
    _lib.check(lib.moe_rope_kv_bf16(qkv.data_ptr(), 1, nq, nkv, hd, inv.data_ptr(), p0.data_ptr(),
                                    max_seq, q_u.data_ptr(), caches[2].data_ptr(),
                                    caches[3].data_ptr(), _stream()), "rope")
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(h_f), bits(h_u))
    np.testing.assert_array_equal(bits(q_f), bits(q_u))
    np.testing.assert_array_equal(bits(caches[0]), bits(caches[2]))   # k rows, others zero
    np.testing.assert_array_equal(bits(caches[1]), bits(caches[3]))   # v rows
    assert caches[0][:, pos].abs().sum() > 0 and not caches[0][:, :pos].any()


def test_head_argmax(cuda_device):
    """final norm + lm_head + argmax + step bookkeeping: logits equal the unfused kernels,
    the token is torch.argmax of them, ties go to the lower index, and gen[ctr] is written
    only inside gen_cap while ctr and pos always advance."""
    from moeinfra_amd import _lib

    lib = _lib.lib()
    dev = cuda_device
    V, H = 32000, 4096
    x = _bf16((1, H), 32).to(dev)
    res = _bf16((1, H), 33).to(dev)
    nw = torch.ones((H,), dtype=torch.bfloat16, device=dev)
    _, xn0 = _unfused_norm(lib, x, res, nw)
    W = _bf16((V, H), 31, 0.02).to(dev)
    # rows 777 and 20000 equal and aligned with the normalised input: a tie at the maximum
    W[777] = (xn0[0].float().sign() * 0.05).to(torch.bfloat16)
    W[20000] = W[777]
    logits = torch.empty((1, V), dtype=torch.bfloat16, device=dev)
    cu = torch.cuda.get_device_properties(dev).multi_processor_count
    cand = torch.empty((8 * 4 * cu,), dtype=torch.uint8, device=dev)
    tok = torch.full((1,), -1, dtype=torch.int64, device=dev)
    gen = torch.full((3,), -1, dtype=torch.int64, device=dev)
    gctr = torch.tensor([1], dtype=torch.int64, device=dev)
    pos = torch.tensor([9], dtype=torch.int32, device=dev)
    for cand_bytes in (cand.numel(), 8 * 3):  # full grid, then only three workgroups
        _lib.check(lib.moe_head_argmax_bf16(W.data_ptr(), x.data_ptr(), res.data_ptr(), nw.data_ptr(),
                                            1e-5, V, H, logits.data_ptr(), cand.data_ptr(),
                                            cand_bytes, tok.data_ptr(),
                                            gen.data_ptr(), gen.numel(), gctr.data_ptr(),
                                            pos.data_ptr(), _stream()), "head")
        torch.cuda.synchronize()
        _, xn = _unfused_norm(lib, x, res, nw)
        want = _unfused_gemv(lib, W, xn)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(bits(logits), bits(want))
        lg = want.float().cpu()[0]
        assert float(lg[777]) == float(lg[20000]) == float(lg.max())
        assert int(tok.item()) == int(torch.argmax(lg)) == 777
    assert gen.tolist() == [-1, 777, 777] and int(gctr.item()) == 3 and int(pos.item()) == 11
    # gen_ctr at the capacity: nothing written, the counter still advances
    _lib.check(lib.moe_head_argmax_bf16(W.data_ptr(), x.data_ptr(), res.data_ptr(), nw.data_ptr(),
                                        1e-5, V, H, logits.data_ptr(), cand.data_ptr(), cand.numel(),
                                        tok.data_ptr(), gen.data_ptr(), gen.numel(),
                                        gctr.data_ptr(), None, _stream()), "head")
    torch.cuda.synchronize()
    assert gen.tolist() == [-1, 777, 777] and int(gctr.item()) == 4 and int(pos.item()) == 11


@pytest.mark.parametrize("form", ["full", "small", "wide"])
def test_layer_norm_fused_matches_unfused(cuda_device, form):
    """The single-token MoE layer with the post-attention residual add + norm in its gate/up
    kernel == moe_add_rmsnorm_bf16 then moe_layer_forward_nf4, bit for bit (output,
    residual, routing weights and ids), on two calls in a row.  Hidden 4096 and 512 take the
    one-chunk-per-thread norm, 6144 the form with up to four chunks per thread."""
    from moeinfra_amd import _lib
    from moeinfra_amd.engine.decoder import MixtralShape, synthesize

    lib = _lib.lib()
    dev = cuda_device
    shape = {"full": MixtralShape(layers=1),
             "small": MixtralShape(hidden=512, ffn=1024, layers=1, n_heads=8, n_kv_heads=2,
                                   head_dim=64, vocab=64),
             "wide": MixtralShape(hidden=6144, ffn=1536, layers=1, n_heads=48, n_kv_heads=8,
                                  head_dim=128, vocab=64)}[form]
    w = synthesize(shape, seed=41, device=dev)
    lw = w.layers[0]
    H, F, E, k = shape.hidden, shape.ffn, shape.experts, shape.top_k
    nw = _bf16((H,), 42, 0.5).to(dev)
    ws_n = torch.empty((lib.moe_layer_norm_workspace_bytes(k, E, H, F),), dtype=torch.uint8, device=dev)
    ws_u = torch.empty((lib.moe_layer_workspace_bytes(1, k, E, H, F),), dtype=torch.uint8, device=dev)
    for seed in (43, 44):
        y = _bf16((1, H), seed).to(dev)
        h = _bf16((1, H), seed + 10).to(dev)
        outs = {}
        for fused in (True, False):
            r = torch.empty((1, H), dtype=torch.bfloat16, device=dev)
            out = torch.empty((1, H), dtype=torch.bfloat16, device=dev)
            wt = torch.empty((1, k), dtype=torch.float32, device=dev)
            idx = torch.empty((1, k), dtype=torch.int64, device=dev)
            if fused:
                _lib.check(lib.moe_layer_forward_nf4_norm(
                    lw.table, E, lw.gate.data_ptr(), y.data_ptr(), h.data_ptr(), nw.data_ptr(), 1e-5,
                    H, F, k, r.data_ptr(), out.data_ptr(), wt.data_ptr(), idx.data_ptr(),
                    ws_n.data_ptr(), ws_n.numel(), _stream()), "fused")
            else:
                x2 = torch.empty_like(y)
                _lib.check(lib.moe_add_rmsnorm_bf16(y.data_ptr(), h.data_ptr(), nw.data_ptr(), 1e-5, 1,
                                                    H, r.data_ptr(), x2.data_ptr(), _stream()), "norm")
                _lib.check(lib.moe_layer_forward_nf4(
                    lw.table, E, lw.gate.data_ptr(), None, x2.data_ptr(), 1, H, F, k, out.data_ptr(),
                    None, wt.data_ptr(), idx.data_ptr(), ws_u.data_ptr(), ws_u.numel(), _stream()),
                    "layer")
            torch.cuda.synchronize()
            outs[fused] = (bits(r), bits(out), wt.cpu().numpy(), idx.cpu().numpy())
        for a, b in zip(outs[True], outs[False]):
            np.testing.assert_array_equal(a, b)
        assert np.abs(outs[True][1].astype(np.int32)).sum() > 0


def test_decode_step_matches_forward(cuda_device):
    """The fused decode step == forward() + argmax, bit for bit, over several positions."""
    from moeinfra_amd.engine.decoder import NativeDecoder

    w = _small_engine_weights(cuda_device)
    prompt = torch.randint(0, w.shape.vocab, (7,), generator=torch.Generator().manual_seed(8))
    a = NativeDecoder(w, 32, cuda_device)
    b = NativeDecoder(w, 32, cuda_device)
    assert a.fused_step_supported()
    la = a.forward(prompt.to(cuda_device))
    lb = b.forward(prompt.to(cuda_device))
    tok = la.argmax(dim=-1)
    tok_b = tok.clone()
    for _ in range(5):
        lf = a.decode_step(tok)                       # writes the next token into tok
        lu = b.forward(tok_b)
        np.testing.assert_array_equal(bits(lf), bits(lu))
        tok_b = lu.argmax(dim=-1)
        assert int(tok.item()) == int(tok_b.item())
    assert int(a.pos.item()) == int(b.pos.item()) == 12
    np.testing.assert_array_equal(bits(a.k_cache), bits(b.k_cache))
    np.testing.assert_array_equal(bits(a.v_cache), bits(b.v_cache))


# --------------------------------------------------------------------------- engine
def _small_shape():
    from moeinfra_amd.engine.decoder import MixtralShape

    return MixtralShape(hidden=512, ffn=1024, layers=2, n_heads=8, n_kv_heads=2, head_dim=64,
                        vocab=640, experts=8, top_k=2)


_E2E = {}


def _small_engine_weights(device):
    if "w" not in _E2E:
        from moeinfra_amd.engine.decoder import synthesize

        _E2E["w"] = synthesize(_small_shape(), seed=5, device=device)
    return _E2E["w"]


def _check_against_reference(res, weights, prompt, tol=2e-2):
    ref = RefDecoder(weights)
    want = ref.forward(prompt[0].tolist())
    toks = res.token_ids
    logits_seen = [want]
    for t in toks[:-1]:
        logits_seen.append(ref.forward([t]))
    for step, (tok, lg) in enumerate(zip(toks, logits_seen)):
        if int(lg.argmax()) != tok:
            assert top2_gap(lg) < 0.05 * float(lg.abs().max()), (step, tok, int(lg.argmax()))
    assert rel_l2(res.logits.float().cpu().reshape(-1), logits_seen[-1].reshape(-1)) < tol


@pytest.mark.parametrize("use_graph", [True, False])
def test_engine_matches_reference(cuda_device, use_graph):
    from moeinfra_amd.engine.engine import InferenceEngine
    from moeinfra_amd.engine.types import ForwardRequest

    w = _small_engine_weights(cuda_device)
    prompt = torch.randint(0, w.shape.vocab, (1, 12), generator=torch.Generator().manual_seed(3))
    eng = InferenceEngine(w, max_seq=64, device=cuda_device, use_graph=use_graph)
    res = eng.generate(ForwardRequest(prompt, max_new_tokens=8))
    assert len(res.token_ids) == 8 and res.tps > 0 and res.ttft_ms > 0
    _check_against_reference(res, w, prompt)
    _E2E.setdefault("tokens", {})[use_graph] = (res.token_ids, bits(res.logits))


def test_engine_graph_replays_match_eager(cuda_device):
    """Graph replays give bit-identical tokens and logits to eager steps, also when the
    engine generates twice (a second prefill resets the position and cache)."""
    from moeinfra_amd.engine.engine import InferenceEngine
    from moeinfra_amd.engine.types import ForwardRequest

    w = _small_engine_weights(cuda_device)
    prompt = torch.randint(0, w.shape.vocab, (1, 9), generator=torch.Generator().manual_seed(4))
    outs = []
    for use_graph in (False, True):
        eng = InferenceEngine(w, max_seq=64, device=cuda_device, use_graph=use_graph)
        for _ in range(2):
            res = eng.generate(ForwardRequest(prompt, max_new_tokens=10))
            outs.append((res.token_ids, bits(res.logits)))
    for toks, lg in outs[1:]:
        assert toks == outs[0][0]
        np.testing.assert_array_equal(lg, outs[0][1])


@pytest.mark.parametrize("policy,slots,per_layer,evict", [
    ("NONE", 4, None, "lru"), ("NEXT_LAYER", 4, None, "lru"), ("NEXT_ROUTER", 4, None, "lru"),
    ("NONE", 3, 1, "lru"), ("NEXT_ROUTER", 6, 3, "lru"),
    ("NEXT_ROUTER", 4, None, "lfu"), ("NONE", 4, 2, "lfu"),
    ("NEXT_ROUTER", 4, None, "arc"), ("NONE", 4, 2, "arc")])
def test_engine_offload_matches_reference(cuda_device, policy, slots, per_layer, evict):
    """Offload mode: the NF4 store pinned on the host, a few GPU expert slots (fewer than a
    40-token prefill routes to per layer), the prefetch policies, the per-layer GPU tier
    that keeps transferred experts across tokens, and the LRU / LFU / ARC GPU tiers."""
    from moeinfra_amd.engine.engine import InferenceEngine
    from moeinfra_amd.engine.types import ForwardRequest, PrefetchPolicy
    from moeinfra_amd.transfer import scheduler as sched_mod

    w = _small_engine_weights(cuda_device)
    prompt = torch.randint(0, w.shape.vocab, (1, 6), generator=torch.Generator().manual_seed(6))
    eng = InferenceEngine(w, max_seq=64, device=cuda_device, offload=True, gpu_expert_slots=slots,
                          prefetch=PrefetchPolicy[policy], gpu_slots_per_layer=per_layer,
                          cache_policy=evict, prefetch_prefix_bytes=None)  # whole copies
    assert eng.cache_manager.policy.value == evict
    n_prof = len(sched_mod.EXECUTE_NEXT_PROFILE)
    res = eng.generate(ForwardRequest(prompt, max_new_tokens=5))
    _check_against_reference(res, w, prompt)
    assert eng.pinned_store.pinned_bytes > 0
    assert all(p.get("source", "image") == "image"                 # never staged
               for p in sched_mod.EXECUTE_NEXT_PROFILE[n_prof:])
    used = eng.cache_manager.stats().gpu_slots_used
    if per_layer is not None:                # transferred experts are kept, per layer
        assert 0 < used <= per_layer * w.shape.layers
        assert all(sum(1 for k in eng.cache_manager._gpu_cache if k[0] == l) <= per_layer
                   for l in range(w.shape.layers))
    elif policy == "NONE":                   # the reference's contract: demoted after use
        assert used == 0


@pytest.mark.parametrize("prefix,slots,per_layer", [
    (4096, 4, None), ("half", 4, None), ("whole", 4, None), ("half", 6, 3)])
def test_engine_offload_prefix_prefetch_matches_reference(cuda_device, prefix, slots, per_layer):
    """NEXT_ROUTER with bounded prefixes: the first bytes of each guessed expert's image go
    ahead into a spare slot; the layer's transfer copies the rest into the same slot (a
    prefix of a few KB, half the image, the whole image), or the unused prefix is dropped."""
    from moeinfra_amd.engine.engine import InferenceEngine
    from moeinfra_amd.engine.types import ForwardRequest, PrefetchPolicy

    w = _small_engine_weights(cuda_device)
    prompt = torch.randint(0, w.shape.vocab, (1, 6), generator=torch.Generator().manual_seed(7))
    probe = InferenceEngine(w, max_seq=64, device=cuda_device, offload=True, gpu_expert_slots=slots)
    image = probe.cache_manager.peek_cpu(0, 0).image_layout.nbytes
    del probe
    nbytes = {"half": image // 2 + 3, "whole": image}.get(prefix, prefix)
    eng = InferenceEngine(w, max_seq=64, device=cuda_device, offload=True, gpu_expert_slots=slots,
                          prefetch=PrefetchPolicy.NEXT_ROUTER, gpu_slots_per_layer=per_layer,
                          prefetch_prefix_bytes=nbytes)
    res = eng.generate(ForwardRequest(prompt, max_new_tokens=6))
    _check_against_reference(res, w, prompt)
    c = eng.prefetch_engine.counts
    assert c["prefixes"] > 0 and c["started"] == 0       # prefixes only, no whole copies
    assert c["prefixes_used"] > 0
    assert c["prefixes_used"] + c["prefixes_dropped"] <= c["prefixes"]
    assert eng.transfer_scheduler.copies["prefix"] == c["prefixes"]


def test_engine_full_mixtral_layer_matches_reference(cuda_device):
    """One decoder layer at the full Mixtral-8x7B shape (hidden 4096, 32/8 heads of 128,
    8 NF4 experts of 14336, vocab 32000): prefill of 6 tokens and 4 graph-replayed decode
    tokens against the CPU oracle decoder, teacher-forced on the engine's tokens."""
    from moeinfra_amd.engine.decoder import MixtralShape, synthesize
    from moeinfra_amd.engine.engine import InferenceEngine
    from moeinfra_amd.engine.types import ForwardRequest

    w = synthesize(MixtralShape(layers=1), seed=12, device=cuda_device)
    prompt = torch.randint(0, w.shape.vocab, (1, 6), generator=torch.Generator().manual_seed(13))
    eng = InferenceEngine(w, max_seq=32, device=cuda_device)
    res = eng.generate(ForwardRequest(prompt, max_new_tokens=5))
    assert len(res.token_ids) == 5
    _check_against_reference(res, w, prompt)


def test_engine_fills_max_seq_and_lookahead_offload(cuda_device):
    """A prompt plus generated tokens that fill the KV cache exactly, graph-replayed; and the
    offload engine with look-ahead prefetch, both against the oracle decoder."""
    from moeinfra_amd.engine.engine import InferenceEngine
    from moeinfra_amd.engine.types import ForwardRequest, PrefetchPolicy

    w = _small_engine_weights(cuda_device)
    prompt = torch.randint(0, w.shape.vocab, (1, 10), generator=torch.Generator().manual_seed(21))
    eng = InferenceEngine(w, max_seq=16, device=cuda_device)
    res = eng.generate(ForwardRequest(prompt, max_new_tokens=7))      # positions 0 .. 15
    assert len(res.token_ids) == 7
    _check_against_reference(res, w, prompt)
    eng = InferenceEngine(w, max_seq=32, device=cuda_device, offload=True, gpu_expert_slots=3,
                          prefetch=PrefetchPolicy.LOOKAHEAD, prefetch_depth=2)
    res = eng.generate(ForwardRequest(prompt[:, :5], max_new_tokens=4))
    _check_against_reference(res, w, prompt[:, :5])


def test_engine_rejects_bad_requests(cuda_device):
    from moeinfra_amd.engine.engine import InferenceEngine
    from moeinfra_amd.engine.types import ForwardRequest

    w = _small_engine_weights(cuda_device)
    eng = InferenceEngine(w, max_seq=16, device=cuda_device)
    with pytest.raises(ValueError):
        eng.generate(ForwardRequest(torch.zeros((12,), dtype=torch.long)))
    with pytest.raises(ValueError):
        eng.generate(ForwardRequest(torch.zeros((1, 20), dtype=torch.long)))
    with pytest.raises(ValueError):
        eng.generate(ForwardRequest(torch.zeros((1, 4), dtype=torch.long), max_new_tokens=-1))
