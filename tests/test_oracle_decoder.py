"""Pins the dense decoder oracle (oracle/decoder_oracle.py) to the Hugging Face modules the
reference runs (engine/engine.py:211-314: MixtralRMSNorm, MixtralRotaryEmbedding,
apply_rotary_pos_emb, the eager attention of MixtralAttention with a DynamicCache), on CPU
in bf16.  transformers is a dependency of the reference; where it is not importable these
tests are skipped."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import decoder_oracle as dor

mixtral = pytest.importorskip("transformers.models.mixtral.modeling_mixtral")
from transformers import MixtralConfig  # noqa: E402


def _cfg(**kw):
    base = dict(hidden_size=256, intermediate_size=512, num_hidden_layers=1, num_attention_heads=8,
                num_key_value_heads=2, head_dim=32, vocab_size=64, num_local_experts=4,
                num_experts_per_tok=2, rope_theta=1e6, rms_norm_eps=1e-5, max_position_embeddings=256)
    base.update(kw)
    cfg = MixtralConfig(**base)
    cfg._attn_implementation = "eager"
    return cfg


def _bf16(shape, seed, std=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * std).to(torch.bfloat16)


def _same(a, b):
    np.testing.assert_array_equal(a.contiguous().view(torch.int16).numpy(),
                                  b.contiguous().view(torch.int16).numpy())


def test_rmsnorm_is_mixtral_rmsnorm():
    norm = mixtral.MixtralRMSNorm(256, eps=1e-5).to(torch.bfloat16)
    with torch.no_grad():
        norm.weight.copy_(_bf16((256,), 1, 0.5))
    x = _bf16((7, 256), 2, 3.0)
    _same(dor.rmsnorm(x, norm.weight.detach(), 1e-5), norm(x).detach())


def test_rope_is_mixtral_rotary_embedding():
    cfg = _cfg()
    rot = mixtral.MixtralRotaryEmbedding(config=cfg)
    np.testing.assert_array_equal(rot.inv_freq.numpy(), dor.inv_freq(32, 1e6).numpy())
    T, p0 = 6, 41
    q = _bf16((1, 8, T, 32), 3)
    k = _bf16((1, 2, T, 32), 4)
    pos = torch.arange(p0, p0 + T)[None]
    cos, sin = rot(q, pos)
    qe, ke = mixtral.apply_rotary_pos_emb(q, k, cos, sin)
    _same(dor.rope(q[0].transpose(0, 1), pos[0], dor.inv_freq(32, 1e6)), qe[0].transpose(0, 1))
    _same(dor.rope(k[0].transpose(0, 1), pos[0], dor.inv_freq(32, 1e6)), ke[0].transpose(0, 1))


@pytest.mark.parametrize("T,p0", [(1, 0), (1, 13), (9, 0), (4, 6)])
def test_attention_is_eager_attention(T, p0):
    import types

    nq, nkv, hd = 8, 2, 32
    S = p0 + T
    q = _bf16((1, nq, T, hd), 5)
    k = _bf16((1, nkv, S, hd), 6)
    v = _bf16((1, nkv, S, hd), 7)
    mask = torch.full((T, S), torch.finfo(torch.bfloat16).min, dtype=torch.bfloat16)
    for t in range(T):
        mask[t, :p0 + t + 1] = 0
    module = types.SimpleNamespace(num_key_value_groups=nq // nkv, training=False)
    out, _ = mixtral.eager_attention_forward(module, q, k, v, mask[None, None], scaling=hd ** -0.5)
    want = out.reshape(T, nq * hd)
    got = dor.attention(q[0].transpose(0, 1), k[0], v[0], p0, hd ** -0.5)
    _same(got, want)


def test_attention_block_is_mixtral_attention_with_cache():
    """q/k/v/o projections + rotary + eager attention over a growing DynamicCache (prefill
    of 5 tokens, then 3 single-token steps) against MixtralAttention.forward."""
    from transformers.cache_utils import DynamicCache

    cfg = _cfg()
    att = mixtral.MixtralAttention(cfg, layer_idx=0).to(torch.bfloat16)
    rot = mixtral.MixtralRotaryEmbedding(config=cfg)
    with torch.no_grad():
        for i, lin in enumerate((att.q_proj, att.k_proj, att.v_proj, att.o_proj)):
            lin.weight.copy_(_bf16(lin.weight.shape, 10 + i, 0.05))
    cache = DynamicCache(config=cfg)
    qkv = torch.cat([att.q_proj.weight, att.k_proj.weight, att.v_proj.weight]).detach()
    kc = torch.zeros((2, 0, 32), dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    freqs = dor.inv_freq(32, 1e6)
    pos = 0
    for T in (5, 1, 1, 1):
        x = _bf16((1, T, 256), 20 + pos)
        S = pos + T
        mask = torch.full((T, S), torch.finfo(torch.bfloat16).min, dtype=torch.bfloat16)
        for t in range(T):
            mask[t, :pos + t + 1] = 0
        position_ids = torch.arange(pos, S)[None]
        with torch.no_grad():
            want, _ = att(x, rot(x, position_ids), mask[None, None], past_key_values=cache)
        y = x[0] @ qkv.t()
        q = y[:, :256].reshape(T, 8, 32)
        k = y[:, 256:320].reshape(T, 2, 32)
        v = y[:, 320:].reshape(T, 2, 32)
        positions = torch.arange(pos, S)
        q, k = dor.rope(q, positions, freqs), dor.rope(k, positions, freqs)
        kc = torch.cat([kc, k.transpose(0, 1)], dim=1)
        vc = torch.cat([vc, v.transpose(0, 1)], dim=1)
        got = dor.attention(q, kc, vc, pos, 32 ** -0.5) @ att.o_proj.weight.detach().t()
        _same(got, want[0])
        pos = S


def _tiny_weights(seed=0):
    """A 2-layer decoder weights object (the DecoderWeights fields the oracle reads) with
    experts quantised by the oracle."""
    import types

    from oracle import moe_oracle as orc

    s = types.SimpleNamespace(hidden=128, ffn=256, n_heads=4, n_kv_heads=2, head_dim=32, vocab=50,
                              experts=4, top_k=2, rope_theta=1e6, rms_eps=1e-5)
    g = lambda shape, i, std=0.02: _bf16(shape, seed * 100 + i, std)
    u16 = lambda t: t.contiguous().view(torch.int16).numpy().view(np.uint16).reshape(-1)
    layers = []
    for li in range(2):
        experts = []
        for e in range(s.experts):
            st = {}
            for j, (name, shape) in enumerate((("w1", (s.ffn, s.hidden)), ("w3", (s.ffn, s.hidden)),
                                              ("w2", (s.hidden, s.ffn)))):
                p, a = orc.nf4_quantize(u16(g(shape, 10 + 10 * li + 3 * e + j)))
                st[name] = (torch.from_numpy(p), torch.from_numpy(a), torch.from_numpy(orc.NF4_CODE.copy()))
            experts.append(st)
        qkv_rows = (s.n_heads + 2 * s.n_kv_heads) * s.head_dim
        layers.append(types.SimpleNamespace(
            input_norm=g((s.hidden,), 1 + li, 1.0), qkv=g((qkv_rows, s.hidden), 3 + li),
            o_proj=g((s.hidden, s.n_heads * s.head_dim), 5 + li), post_norm=g((s.hidden,), 7 + li, 1.0),
            gate=g((s.experts, s.hidden), 9 + li), experts=experts))
    return types.SimpleNamespace(shape=s, embed=g((s.vocab, s.hidden), 90, 1.0), layers=layers,
                                 final_norm=g((s.hidden,), 91, 1.0), lm_head=g((s.vocab, s.hidden), 92))


def test_layer_parts_compose_to_the_layer_and_forward():
    """layer_parts (attention, MoE at a given residual) and head() recompose forward(): the
    two residual adds of each layer in bf16 give forward()'s logits bit for bit, over a
    prompt and a decode token; an explicit residual equal to the default gives the same MoE
    output, and a different one changes it (the residual is really used)."""
    w = _tiny_weights()
    whole, parts, forced = (dor.RefDecoder(w, threads=1) for _ in range(3))
    for step in ([3, 17, 42, 8, 0], [11]):
        want = whole.forward(step)
        h = parts.embed[torch.as_tensor(step)]
        for li in range(2):
            attn, moe, (_lg, wts, idx) = parts.layer_parts(li, h)
            assert idx.shape == (len(step), 2) and np.allclose(wts.sum(-1), 1.0, atol=1e-6)
            attn_f, moe_f, _ = forced.layer_parts(li, h, resid=h + attn)
            _same(attn_f, attn)
            _same(moe_f, moe)
            h = (h + attn) + moe
        parts.advance(len(step))
        forced.advance(len(step))
        _same(parts.head(h).to(torch.bfloat16), want.to(torch.bfloat16))
    other = dor.RefDecoder(w, threads=1)
    h = other.embed[torch.as_tensor([5, 6])]
    _a, moe0, _ = other.layer_parts(0, h, resid=h)
    assert not torch.equal(moe0, dor.RefDecoder(w, threads=1).layer_parts(0, h)[1])
