"""Native Mixtral decoder for the end-to-end run: the dense parts of each decoder layer
(RMSNorm, rotary embedding, grouped-query attention with a KV cache, the attention
projections, lm_head) on this package's HIP kernels, around the NF4 MoE layer.

The reference builds the same stack from Hugging Face modules (engine/engine.py:192-327:
embed_tokens, MixtralRotaryEmbedding, MixtralDecoderLayer with its MoE block swapped for
MoELayer, final MixtralRMSNorm, lm_head) and runs it eagerly with a DynamicCache
(engine/engine.py:329-385, 500-627).  Here the decoder layer is

    x1 = rmsnorm(h; input_layernorm)               h_mid = bf16(h + o_proj(attn(x1)))
    x2 = rmsnorm(h_mid; post_attention_layernorm)  h_out = bf16(h_mid + moe(x2))

with the residual adds fused into the next RMSNorm, q/k/v in one projection, the KV cache
preallocated [layer][kv head][max_seq][head_dim] and the position a device int32, so that
one decode step is a fixed sequence of kernel launches (capturable as a HIP graph).
Decode-size batches (up to 4 tokens) use the bandwidth-bound GEMV kernel for the
projections; longer prompts use the library GEMM.
"""
from __future__ import annotations

import dataclasses
from typing import List, Optional

import torch

from .. import _lib, ops


@dataclasses.dataclass(frozen=True)
class MixtralShape:
    """Architecture of the decoder (defaults: Mixtral-8x7B)."""

    hidden: int = 4096
    ffn: int = 14336
    layers: int = 32
    n_heads: int = 32
    n_kv_heads: int = 8
    head_dim: int = 128
    vocab: int = 32000
    experts: int = 8
    top_k: int = 2
    rope_theta: float = 1e6
    rms_eps: float = 1e-5

    @property
    def qkv_rows(self) -> int:
        return (self.n_heads + 2 * self.n_kv_heads) * self.head_dim


@dataclasses.dataclass
class LayerWeights:
    input_norm: torch.Tensor       # [H] bf16
    qkv: torch.Tensor              # [(nq + 2 nkv) hd, H] bf16: q_proj; k_proj; v_proj
    o_proj: torch.Tensor           # [H, nq hd] bf16
    post_norm: torch.Tensor        # [H] bf16
    gate: torch.Tensor             # [E, H] bf16 (router)
    experts: list                  # per expert {"w1"|"w3"|"w2": (packed, absmax, code)}
    table: Optional[object] = None  # ctypes expert table (device pointers), all-resident


@dataclasses.dataclass
class DecoderWeights:
    shape: MixtralShape
    embed: torch.Tensor            # [V, H] bf16
    layers: List[LayerWeights]
    final_norm: torch.Tensor       # [H] bf16
    lm_head: torch.Tensor          # [V, H] bf16


def _normal(shape, gen, device, std=0.02):
    return (torch.randn(shape, generator=gen, device=device) * std).to(torch.bfloat16)


def synthesize(shape: MixtralShape, seed: int, device, experts_on=None) -> DecoderWeights:
    """Random-init weights of the architecture (bf16 N(0, 0.02) linear and embedding weights,
    unit norm weights, as a freshly initialised model), experts NF4-quantised by the library.
    Drawn on ``device`` in a fixed order from one seeded generator; ``experts_on`` is where
    the NF4 expert tensors are kept (default: ``device``)."""
    from .._lib import MoeNf4Expert

    dev = torch.device(device)
    keep = torch.device(experts_on) if experts_on is not None else dev
    gen = torch.Generator(device=dev).manual_seed(seed)
    H, F, E = shape.hidden, shape.ffn, shape.experts
    embed = _normal((shape.vocab, H), gen, dev)
    layers = []
    for _ in range(shape.layers):
        qkv = _normal((shape.qkv_rows, H), gen, dev)
        o = _normal((H, shape.n_heads * shape.head_dim), gen, dev)
        gate = _normal((E, H), gen, dev)
        experts = []
        for _e in range(E):
            st = {}
            for name, s in (("w1", (F, H)), ("w3", (F, H)), ("w2", (H, F))):
                w = _normal(s, gen, dev)
                p, a, c = ops.nf4_quantize(w)
                del w
                st[name] = (p.to(keep), a.to(keep), c.to(keep)) if keep != dev else (p, a, c)
            experts.append(st)
        table = None
        if keep.type == "cuda":
            table = ops.expert_table([MoeNf4Expert(*(t.data_ptr() for n in ("w1", "w3", "w2")
                                                     for t in st[n])) for st in experts])
        ones = torch.ones(H, dtype=torch.bfloat16, device=dev)
        layers.append(LayerWeights(ones, qkv, o, ones.clone(), gate, experts, table))
    final = torch.ones(H, dtype=torch.bfloat16, device=dev)
    lm_head = _normal((shape.vocab, H), gen, dev)
    return DecoderWeights(shape, embed, layers, final, lm_head)


def rope_inv_freq(shape: MixtralShape) -> torch.Tensor:
    """inv_freq[i] = 1 / theta^(2i / head_dim) in fp32, as MixtralRotaryEmbedding computes it."""
    i = torch.arange(0, shape.head_dim, 2, dtype=torch.int64).float()
    return 1.0 / (shape.rope_theta ** (i / shape.head_dim))


class NativeDecoder:
    """Device state (KV cache, position, buffers) and the prefill / decode forward passes.

    ``moe`` is a callable (layer_id, x [T, H] bf16) -> [T, H] bf16 for the MoE block; by
    default the all-resident layer entry point on the weights' expert tables.
    """

    GEMV_MAX_TOKENS = 4

    def __init__(self, weights: DecoderWeights, max_seq: int, device, moe=None) -> None:
        s = weights.shape
        self.w = weights
        self.s = s
        self.dev = torch.device(device)
        self.max_seq = int(max_seq)
        self.lib = _lib.lib()
        L = s.layers
        self.k_cache = torch.zeros((L, s.n_kv_heads, self.max_seq, s.head_dim), dtype=torch.bfloat16,
                                   device=self.dev)
        self.v_cache = torch.zeros_like(self.k_cache)
        self.pos = torch.zeros((1,), dtype=torch.int32, device=self.dev)
        self.inv_freq = rope_inv_freq(s).to(self.dev)
        self.scaling = float(s.head_dim ** -0.5)
        self.moe = moe if moe is not None else self._moe_resident
        self._resident = moe is None
        self._moe_bufs = {}
        self._sb = None  # single-token step buffers

    # ------------------------------------------------------------------ pieces
    def _stream(self) -> int:
        return torch.cuda.current_stream(self.dev).cuda_stream

    def _linear(self, W: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
        T = x.shape[0]
        if T <= self.GEMV_MAX_TOKENS and W.shape[1] % 512 == 0:
            y = torch.empty((T, W.shape[0]), dtype=torch.bfloat16, device=self.dev)
            _lib.check(self.lib.moe_gemv_bf16(W.data_ptr(), x.data_ptr(), T, W.shape[0], W.shape[1],
                                              y.data_ptr(), self._stream()), "gemv")
            return y
        return x @ W.t()  # nn.Linear without bias on bf16 tensors

    def _norm(self, x, residual, weight, residual_out=None):
        out = torch.empty_like(x)
        _lib.check(self.lib.moe_add_rmsnorm_bf16(
            x.data_ptr(), 0 if residual is None else residual.data_ptr(), weight.data_ptr(),
            self.s.rms_eps, x.shape[0], x.shape[1],
            0 if residual_out is None else residual_out.data_ptr(), out.data_ptr(),
            self._stream()), "add_rmsnorm")
        return out

    def _attention(self, l: int, x1: torch.Tensor) -> torch.Tensor:
        s, T = self.s, x1.shape[0]
        qkv = self._linear(self.w.layers[l].qkv, x1)
        q = torch.empty((T, s.n_heads * s.head_dim), dtype=torch.bfloat16, device=self.dev)
        kc, vc = self.k_cache[l], self.v_cache[l]
        _lib.check(self.lib.moe_rope_kv_bf16(qkv.data_ptr(), T, s.n_heads, s.n_kv_heads, s.head_dim,
                                             self.inv_freq.data_ptr(), self.pos.data_ptr(),
                                             self.max_seq, q.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                                             self._stream()), "rope_kv")
        a = torch.empty_like(q)
        _lib.check(self.lib.moe_attention_bf16(q.data_ptr(), kc.data_ptr(), vc.data_ptr(), T,
                                               s.n_heads, s.n_kv_heads, s.head_dim,
                                               self.pos.data_ptr(), self.max_seq, self.scaling,
                                               a.data_ptr(), self._stream()), "attention")
        return self._linear(self.w.layers[l].o_proj, a)

    def _moe_resident(self, l: int, x: torch.Tensor) -> torch.Tensor:
        s, T = self.s, x.shape[0]
        lw = self.w.layers[l]
        if T not in self._moe_bufs:
            ws_bytes = self.lib.moe_layer_workspace_bytes(T, s.top_k, s.experts, s.hidden, s.ffn)
            self._moe_bufs[T] = (torch.empty((ws_bytes,), dtype=torch.uint8, device=self.dev),
                                 torch.empty((T, s.top_k), dtype=torch.float32, device=self.dev),
                                 torch.empty((T, s.top_k), dtype=torch.int64, device=self.dev))
        ws, w, idx = self._moe_bufs[T]
        out = torch.empty_like(x)
        _lib.check(self.lib.moe_layer_forward_nf4(lw.table, s.experts, lw.gate.data_ptr(), None,
                                                  x.data_ptr(), T, s.hidden, s.ffn, s.top_k,
                                                  out.data_ptr(), None, w.data_ptr(), idx.data_ptr(),
                                                  ws.data_ptr(), ws.numel(), self._stream()),
                   "moe_layer_forward_nf4")
        return out

    # ------------------------------------------------------------------ forward
    def forward(self, ids: torch.Tensor) -> torch.Tensor:
        """Run tokens ``ids`` [T] (device int64) at positions pos .. pos + T - 1 through the
        stack, append their keys/values to the cache, advance the position, and return the
        logits [1, V] (bf16) of the last token."""
        s = self.s
        T = ids.shape[0]
        h = self.w.embed.index_select(0, ids)          # [T, H]
        resid = torch.empty_like(h)
        x1 = self._norm(h, None, self.w.layers[0].input_norm)
        for l, lw in enumerate(self.w.layers):
            a = self._attention(l, x1)
            x2 = self._norm(a, h, lw.post_norm, residual_out=resid)    # resid = h + attn
            m = self.moe(l, x2)
            nxt = self.w.layers[l + 1].input_norm if l + 1 < s.layers else self.w.final_norm
            h_new = torch.empty_like(h)
            x1 = self._norm(m, resid, nxt, residual_out=h_new)          # h_new = resid + moe
            h = h_new
        self.pos += T
        return self._linear(self.w.lm_head, x1[T - 1:T].contiguous())

    # ------------------------------------------------------------------ decode step
    def fused_step_supported(self) -> bool:
        """Whether the shape fits the fused single-token kernels (hidden and the attention
        width multiples of 512, hidden up to 8192)."""
        s = self.s
        return (s.hidden % 512 == 0 and s.hidden <= 8192 and (s.n_heads * s.head_dim) % 512 == 0
                and s.head_dim % 2 == 0)

    def _decode_layer_shape(self) -> bool:
        """Whether the MoE layer runs as the single-token decode form (T = 1): top-k <= 8,
        at most 16 experts, H and F multiples of 512, at most 8 four-row output tiles of
        the down GEMV per CU."""
        s = self.s
        cu = torch.cuda.get_device_properties(self.dev).multi_processor_count
        return (s.top_k <= 8 and s.experts <= 16 and s.top_k <= s.experts and s.hidden % 512 == 0
                and s.ffn % 512 == 0 and (s.hidden // 4 + cu - 1) // cu <= 8)

    def _step_buffers(self) -> dict:
        if self._sb is None:
            s, d = self.s, self.dev
            bf = dict(dtype=torch.bfloat16, device=d)
            cu = torch.cuda.get_device_properties(d).multi_processor_count
            self._sb = {
                "h": torch.empty((1, s.hidden), **bf),        # layer input (residual stream)
                "resid": torch.empty((1, s.hidden), **bf),    # after attention
                "x2": torch.empty((1, s.hidden), **bf),       # post-attention norm (MoE input)
                "y": torch.empty((1, s.hidden), **bf),        # o_proj output
                "q": torch.empty((1, s.n_heads * s.head_dim), **bf),
                "a": torch.empty((1, s.n_heads * s.head_dim), **bf),
                "logits": torch.empty((1, s.vocab), **bf),
                "cand": torch.empty((8 * 4 * cu,), dtype=torch.uint8, device=d),
                "moe_w": torch.empty((1, s.top_k), dtype=torch.float32, device=d),
                "moe_idx": torch.empty((1, s.top_k), dtype=torch.int64, device=d),
                "moe_ws": None,
            }
            nbytes = self.lib.moe_layer_norm_workspace_bytes(s.top_k, s.experts, s.hidden, s.ffn)
            if self._resident and nbytes > 0 and s.hidden <= 8192 and self._decode_layer_shape():
                self._sb["moe_ws"] = torch.empty((nbytes,), dtype=torch.uint8, device=d)
        return self._sb

    def decode_step(self, tok: torch.Tensor, gen: Optional[torch.Tensor] = None,
                    gen_ctr: Optional[torch.Tensor] = None) -> torch.Tensor:
        """One generated token through the stack: ``tok`` (device int64 [1]) at the current
        position; the greedy next token is written back into ``tok``, and with ``gen`` /
        ``gen_ctr`` (device int64) stored at gen[gen_ctr] before gen_ctr += 1; the position
        advances by one.  Returns the logits [1, V] (a buffer that the next step reuses).

        Per layer three dense launches and the MoE layer's two: norm + q/k/v + rotary + cache
        write (moe_qkv_rope_bf16), attention, o_proj, then the MoE layer with the residual
        add and post-attention norm in its gate/up kernel (moe_layer_forward_nf4_norm; with
        a caller-supplied MoE block, e.g. offload, a separate norm launch and that block);
        then the final norm, lm_head and argmax with the step's bookkeeping
        (moe_head_argmax_bf16, two launches).  The results are bit-identical to forward()
        followed by argmax."""
        if not self.fused_step_supported():
            logits = self.forward(tok)
            nxt = logits.argmax(dim=-1)
            tok.copy_(nxt)
            if gen is not None and gen_ctr is not None:
                gen.index_copy_(0, gen_ctr.clamp(0, gen.numel() - 1), nxt)
                gen_ctr.add_(1)
            return logits
        s, b, st, lib = self.s, self._step_buffers(), self._stream(), self.lib
        nq, nkv, hd, H = s.n_heads, s.n_kv_heads, s.head_dim, s.hidden
        fused_moe = self._resident and b["moe_ws"] is not None
        x, x_row, x_rows, res = self.w.embed, tok.data_ptr(), s.vocab, None
        m = None
        for l, lw in enumerate(self.w.layers):
            kc, vc = self.k_cache[l], self.v_cache[l]
            _lib.check(lib.moe_qkv_rope_bf16(
                lw.qkv.data_ptr(), x.data_ptr(), x_row, x_rows, res, lw.input_norm.data_ptr(),
                s.rms_eps, H, nq, nkv, hd, self.inv_freq.data_ptr(), self.pos.data_ptr(),
                self.max_seq, b["h"].data_ptr(), b["q"].data_ptr(), kc.data_ptr(), vc.data_ptr(),
                st), "qkv_rope")
            _lib.check(lib.moe_attention_bf16(b["q"].data_ptr(), kc.data_ptr(), vc.data_ptr(), 1,
                                              nq, nkv, hd, self.pos.data_ptr(), self.max_seq,
                                              self.scaling, b["a"].data_ptr(), st), "attention")
            _lib.check(lib.moe_gemv_bf16(lw.o_proj.data_ptr(), b["a"].data_ptr(), 1, H, nq * hd,
                                         b["y"].data_ptr(), st), "o_proj")
            if fused_moe:
                # residual add + post-attention norm inside the MoE layer's gate/up kernel
                m = torch.empty_like(b["y"])
                _lib.check(lib.moe_layer_forward_nf4_norm(
                    lw.table, s.experts, lw.gate.data_ptr(), b["y"].data_ptr(), b["h"].data_ptr(),
                    lw.post_norm.data_ptr(), s.rms_eps, H, s.ffn, s.top_k, b["resid"].data_ptr(),
                    m.data_ptr(), b["moe_w"].data_ptr(), b["moe_idx"].data_ptr(),
                    b["moe_ws"].data_ptr(), b["moe_ws"].numel(), st), "moe layer + norm")
            else:
                _lib.check(lib.moe_add_rmsnorm_bf16(b["y"].data_ptr(), b["h"].data_ptr(),
                                                    lw.post_norm.data_ptr(), s.rms_eps, 1, H,
                                                    b["resid"].data_ptr(), b["x2"].data_ptr(), st),
                           "post-attention norm")
                m = self.moe(l, b["x2"])
            x, x_row, x_rows, res = m, None, 1, b["resid"].data_ptr()
        gen_p = gen.data_ptr() if gen is not None else None
        ctr_p = gen_ctr.data_ptr() if gen_ctr is not None else None
        _lib.check(lib.moe_head_argmax_bf16(
            self.w.lm_head.data_ptr(), m.data_ptr(), b["resid"].data_ptr(),
            self.w.final_norm.data_ptr(), s.rms_eps, s.vocab, H, b["logits"].data_ptr(),
            b["cand"].data_ptr(), b["cand"].numel(), tok.data_ptr(), gen_p,
            0 if gen is None else gen.numel(), ctr_p, self.pos.data_ptr(), st), "lm_head + argmax")
        return b["logits"]

    def reset(self) -> None:
        self.pos.zero_()
