"""CPU oracle of the dense decoder stack around the MoE block -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``
import this module, and only as the checker.

The reference runs the decoder as Hugging Face modules (engine/engine.py:211-314 builds
embed_tokens, MixtralRotaryEmbedding, MixtralDecoderLayer with the MoE block swapped for
MoELayer (engine/decoder_layer.py:37-41), the final MixtralRMSNorm and lm_head;
engine/engine.py:329-385 runs the layers, :500-627 prefill and greedy decode).  The
functions below restate those modules' arithmetic on CPU bf16 tensors (bf16 rounding
after every op, fp32 norm statistics and softmax); the MoE block is ``moe_oracle``'s
layer on the dequantised NF4 experts.

Pinned (tests/test_oracle_decoder.py) against transformers' own MixtralRMSNorm,
MixtralRotaryEmbedding + apply_rotary_pos_emb, eager_attention_forward and
MixtralAttention.forward with a DynamicCache, on CPU, bit for bit.
"""
from __future__ import annotations

import numpy as np
import torch

from . import moe_oracle as orc


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _from_bits(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint16).view(np.int16)).view(torch.bfloat16)


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """MixtralRMSNorm on bf16: fp32 mean of squares, rsqrt, bf16 cast, times the weight."""
    hs = x.float()
    var = hs.pow(2).mean(-1, keepdim=True)
    hs = hs * torch.rsqrt(var + eps)
    return w * hs.to(torch.bfloat16)


def inv_freq(head_dim: int, theta: float) -> torch.Tensor:
    """Default rotary frequencies 1 / theta^(2i / head_dim), fp32."""
    return 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim))


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def rope(x: torch.Tensor, positions: torch.Tensor, freqs_inv: torch.Tensor) -> torch.Tensor:
    """x [T, heads, hd] bf16 rotated at positions [T]: fp32 angles, cos/sin cast to bf16,
    x*cos + rotate_half(x)*sin in bf16."""
    freqs = positions.float()[:, None] * freqs_inv[None, :]
    emb = torch.cat((freqs, freqs), dim=-1)
    cos = emb.cos().to(torch.bfloat16)[:, None, :]
    sin = emb.sin().to(torch.bfloat16)[:, None, :]
    return (x * cos) + (rotate_half(x) * sin)


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, p0: int, scaling: float) -> torch.Tensor:
    """Eager grouped-query causal attention: q [T, nq, hd] at positions p0 .. p0+T-1, k/v
    [nkv, S, hd] (all positions so far) -> [T, nq * hd] bf16."""
    T, nq, hd = q.shape
    nkv, S, _ = k.shape
    rep = nq // nkv
    K = k.repeat_interleave(rep, dim=0)
    V = v.repeat_interleave(rep, dim=0)
    scores = torch.matmul(q.transpose(0, 1), K.transpose(1, 2).contiguous()) * scaling
    mask = torch.full((T, S), float("-inf"))
    for t in range(T):
        mask[t, :p0 + t + 1] = 0.0
    p = torch.softmax(scores.float() + mask, dim=-1, dtype=torch.float32).to(torch.bfloat16)
    out = torch.matmul(p, V)
    return out.transpose(0, 1).reshape(T, nq * hd)


class RefDecoder:
    """Teacher-forced reference decoder over a weights object with the fields of
    moeinfra_amd.engine.decoder.DecoderWeights (embed, layers[input_norm, qkv, o_proj,
    post_norm, gate, experts], final_norm, lm_head, shape); forward(ids) appends to its
    own KV cache and returns the last token's fp32 logits [1, V].  ``layers``: all (None),
    the first n (an int) or the listed layer indices; ``threads``: host threads of the NF4
    dequantisation."""

    def __init__(self, weights, layers=None, threads: int = 8):
        w = weights
        s = w.shape
        self.s = s
        self.threads = int(threads)
        cpu = lambda t: t.detach().cpu()
        self.embed, self.final_norm, self.lm_head = cpu(w.embed), cpu(w.final_norm), cpu(w.lm_head)
        self.layers = []
        if layers is None:
            chosen = w.layers
        elif isinstance(layers, int):
            chosen = w.layers[:layers]
        else:
            chosen = [w.layers[i] for i in layers]
        for lw in chosen:
            states = [{n: (cpu(p).numpy().reshape(-1), cpu(a).numpy()) for n, (p, a, _c) in st.items()}
                      for st in lw.experts]
            self.layers.append(dict(inn=cpu(lw.input_norm), qkv=cpu(lw.qkv), o=cpu(lw.o_proj),
                                    post=cpu(lw.post_norm), gate=cpu(lw.gate), states=states,
                                    cache={}))
        self.k = [torch.zeros((s.n_kv_heads, 0, s.head_dim), dtype=torch.bfloat16) for _ in self.layers]
        self.v = [torch.zeros_like(k) for k in self.k]
        self.inv_freq = inv_freq(s.head_dim, s.rope_theta)
        self.pos = 0

    def _moe(self, L, x: torch.Tensor) -> torch.Tensor:
        s = self.s

        def expert_fn(e, rows):
            if e not in L["cache"]:
                L["cache"][e] = orc.dequant_expert(L["states"][e], s.hidden, s.ffn, threads=self.threads)
            return orc.swiglu(rows, *L["cache"][e])

        out, _ = orc.moe_layer(_bits(x), _bits(L["gate"]), expert_fn, k=s.top_k)
        return _from_bits(out)

    def _attention(self, li, L, x1):
        s = self.s
        T = x1.shape[0]
        qkv = x1 @ L["qkv"].t()
        nq, nkv, hd = s.n_heads, s.n_kv_heads, s.head_dim
        q = qkv[:, :nq * hd].reshape(T, nq, hd)
        k = qkv[:, nq * hd:(nq + nkv) * hd].reshape(T, nkv, hd)
        v = qkv[:, (nq + nkv) * hd:].reshape(T, nkv, hd)
        positions = torch.arange(self.pos, self.pos + T)
        q, k = rope(q, positions, self.inv_freq), rope(k, positions, self.inv_freq)
        self.k[li] = torch.cat([self.k[li], k.transpose(0, 1)], dim=1)
        self.v[li] = torch.cat([self.v[li], v.transpose(0, 1)], dim=1)
        out = attention(q, self.k[li], self.v[li], self.pos, float(hd ** -0.5))
        return out @ L["o"].t()

    @torch.no_grad()
    def layer(self, li: int, h: torch.Tensor) -> torch.Tensor:
        """One decoder layer on h [T, H] at the current position (does not advance it)."""
        s, L = self.s, self.layers[li]
        h = h + self._attention(li, L, rmsnorm(h, L["inn"], s.rms_eps))
        return h + self._moe(L, rmsnorm(h, L["post"], s.rms_eps))

    @torch.no_grad()
    def layer_parts(self, li: int, h: torch.Tensor, resid: torch.Tensor = None, moe: bool = True):
        """Layer li split at its residual add, teacher-forced: the attention block's output
        for input h [T, H] at the current position (keys/values appended), and the MoE
        block's output (with its routing) on post_norm(resid), where resid is the caller's
        post-attention residual stream (default bf16(h + attention)).  Does not advance the
        position.  Returns (attention [T, H], moe [T, H] bf16, (logits, w, idx)); with
        moe=False only the attention block runs (the key/value rows of a pass that is not
        checked) and the last two are None."""
        s, L = self.s, self.layers[li]
        attn = self._attention(li, L, rmsnorm(h, L["inn"], s.rms_eps))
        if not moe:
            return attn, None, None
        if resid is None:
            resid = h + attn
        x2 = rmsnorm(resid, L["post"], s.rms_eps)

        wide = L.setdefault("cache_f32", {})

        def expert_fn(e, rows):
            if e not in wide:
                wide[e] = tuple(orc.bf16_to_f32(w) for w in
                                orc.dequant_expert(L["states"][e], s.hidden, s.ffn, threads=self.threads))
            return orc.swiglu_f32(rows, *wide[e])

        out, routing = orc.moe_layer(_bits(x2), _bits(L["gate"]), expert_fn, k=s.top_k)
        return attn, _from_bits(out), routing

    def advance(self, n: int) -> None:
        """Moves the position on by n tokens (after layer_parts calls for them)."""
        self.pos += int(n)

    @torch.no_grad()
    def head(self, h: torch.Tensor) -> torch.Tensor:
        """Final norm + lm_head of the last row of the residual stream h: fp32 logits [1, V]."""
        return (rmsnorm(h, self.final_norm, self.s.rms_eps)[-1:] @ self.lm_head.t()).float()

    @torch.no_grad()
    def forward(self, ids) -> torch.Tensor:
        s = self.s
        h = self.embed[torch.as_tensor(ids, dtype=torch.long)]
        for li in range(len(self.layers)):
            h = self.layer(li, h)
        self.pos += len(ids)
        return (rmsnorm(h, self.final_norm, s.rms_eps)[-1:] @ self.lm_head.t()).float()
