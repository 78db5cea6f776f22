/*
 * moeinfra_hip.h -- C ABI of libmoeinfra_hip.so, the gfx950 (MI355X) MoE
 * expert-execution path.
 *
 * Every entry point takes raw device pointers, 64-bit sizes and a hipStream_t
 * (passed as void*), enqueues its kernels on that stream, performs no host<->device
 * synchronisation and allocates no memory: the caller owns every buffer, including the
 * workspace (moe_layer_forward_nf4_noalloc uses the library's static scratch instead).
 * Calls return MOE_STATUS_OK (0) or a negative status; the message of the last failure on
 * the calling thread is returned by moe_last_error().  Calls on one stream are ordered;
 * the library keeps no mutable global state besides per-device caches of the
 * compute-unit count and of the static scratch's address.
 *
 * Data formats (bitsandbytes NF4, as the reference stores it):
 *   - a weight W[O][I] is the row-major flatten of O*I values quantised in blocks of
 *     `blocksize` consecutive values (64 on the expert path);
 *   - packed byte j holds value 2j in its HIGH nibble and value 2j+1 in its low nibble;
 *   - absmax is fp32, one per block; code is the fp32[16] codebook (quant_map);
 *   - dequantised value = bf16_round_nearest_even(code[q] * absmax[block]).
 * Activations are bf16 (raw uint16 bit patterns in memory), routing weights fp32,
 * expert indices int64 (int32 copies are kept for the kernels).
 *
 * Reference citations are into ParshwaPatel-07/MoEInfra.
 */
#ifndef MOEINFRA_HIP_H
#define MOEINFRA_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MOE_STATUS_OK 0
#define MOE_STATUS_INVALID_ARGUMENT (-1)
#define MOE_STATUS_HIP_ERROR (-2)
#define MOE_STATUS_UNSUPPORTED (-3)

/* Largest number of experts one call can address (the pointer table travels as a
 * kernel argument). */
#define MOE_MAX_EXPERTS 32
/* Largest top-k. */
#define MOE_MAX_TOPK 8
/* Block size the fused expert kernels require (transfer/nf4_reconstruct.py:9). */
#define MOE_NF4_BLOCKSIZE 64

/* Device pointers of one NF4 expert: the packed weight, fp32 absmax and fp32[16]
 * codebook of each projection, w1 [F,H] (gate), w3 [F,H] (up), w2 [H,F] (down).
 * Mirrors the per-projection state dict {weight, absmax, code} that
 * transfer/nf4_transfer.py:8-40 produces on the device and
 * transfer/nf4_reconstruct.py:57-114 wraps. */
typedef struct moe_nf4_expert {
    const void *w1_packed;
    const void *w1_absmax;
    const void *w1_code;
    const void *w3_packed;
    const void *w3_absmax;
    const void *w3_code;
    const void *w2_packed;
    const void *w2_absmax;
    const void *w2_code;
} moe_nf4_expert_t;

/* Message of the last failed call on this thread ("" if none). */
const char *moe_last_error(void);

/* Library version (major*10000 + minor*100 + patch). */
int moe_version(void);

/* Count of bounded in-kernel waits that gave up on the current device (lanes), for tests:
 * the batched expert GEMM's waves meet through an LDS counter whose wait ends after ~1 ms
 * whatever happens, so that every kernel exits; a non-zero count means a counting error
 * (wrong results). reset != 0 clears it. Synchronous. No counterpart in the reference (its
 * kernels are bitsandbytes' and torch's). */
int moe_wait_timeouts(int64_t *count, int32_t reset);

/* ---------------------------------------------------------------- K1: NF4 dequant
 * out_bf16[i] = bf16(code[q_i] * absmax[i / blocksize]) for i < numel.
 * Replaces the bitsandbytes dequantize_4bit that Linear4bit runs on the state built
 * by _build_quant_state / _reconstruct_linear (transfer/nf4_reconstruct.py:17-114).
 * numel must be even, blocksize a positive multiple of 32. */
int moe_nf4_dequant_bf16(const void *packed, const void *absmax, const void *code16,
                         void *out_bf16, int64_t numel, int32_t blocksize, void *stream);

/* Nested (double-quantised) absmax of a bitsandbytes NF4 state (compress_statistics):
 * out_f32[i] = code2[absmax_u8[i]] * absmax2[i / blocksize2] + offset, in fp32 (product and
 * sum rounded separately), for i < n.  code2 has 256 entries.  The expanded absmax feeds
 * K1 and the fused expert kernels, which take fp32 block scales.  Replaces the nested
 * branch of the state that _build_quant_state assembles (transfer/nf4_reconstruct.py:22-43),
 * which bitsandbytes resolves inside dequantize_4bit. */
int moe_nf4_expand_absmax(const void *absmax_u8, const void *absmax2_f32, const void *code2_f32,
                          float offset, int64_t n, int32_t blocksize2, void *out_f32,
                          void *stream);

/* ---------------------------------------------------------------- K0: NF4 quantise
 * Blockwise NF4 quantisation of bf16 values: absmax = max|w| per block, q = nearest
 * code value of w*(1/absmax) (midpoint thresholds, ties to the lower code).
 * Replaces the bitsandbytes quantisation that QuantizedMixtralExpert triggers when
 * moved to the GPU (model/expert.py:32-63, model/loader.py:404-415).
 * numel even; blocksize even, 2..4096. absmax_out has ceil(numel/blocksize) floats. */
int moe_nf4_quantize_bf16(const void *w_bf16, int64_t numel, int32_t blocksize,
                          const void *code16, void *packed_out, void *absmax_out, void *stream);

/* ---------------------------------------------------------------- K2: router
 * logits = bf16(x . gate^T); p = softmax(float(logits) [+ bias]); (w, idx) = top-k(p)
 * in descending order (ties: lower expert index first); w /= sum(w).
 * Replaces ExpertRouter.logits / route / route_with_logits (engine/router.py:50-94).
 * x [T,H] bf16, gate [E,H] bf16, bias fp32 [E] or NULL; outputs logits bf16 [T,E]
 * (may be NULL), weights fp32 [T,k], idx int64 [T,k], idx32 int32 [T,k] (may be NULL).
 * Requires H % 8 == 0, 1 <= E <= MOE_MAX_EXPERTS, 1 <= k <= min(E, MOE_MAX_TOPK). */
int moe_router_topk(const void *x_bf16, const void *gate_bf16, const void *bias_f32,
                    int64_t T, int32_t H, int32_t E, int32_t k, void *logits_bf16,
                    void *weights_f32, void *idx_i64, void *idx_i32, void *stream);

/* ---------------------------------------------------------------- K3: permute
 * Groups the T*k (token, slot) pairs by expert, ascending expert id and ascending
 * token within an expert -- the order model/moe_layer.py:150-185 visits them in
 * (unique().tolist(), boolean-mask gather).  Outputs (int32):
 *   counts[E]        tokens per expert
 *   offsets[E+1]     exclusive prefix sum of counts
 *   perm_tok[T*k]    token id of each row of the expert-sorted order
 *   slot_pos[T*k]    row of flat slot t*k+j in that order
 *   active[E+1]      active[0] = number of experts with tokens, then their ids ascending
 * idx32 entries must lie in [0,E). */
int moe_permute(const void *idx_i32, int64_t T, int32_t k, int32_t E, void *counts,
                void *offsets, void *perm_tok, void *slot_pos, void *active, void *stream);

/* ---------------------------------------------------------------- K4: expert FFN
 * For every active expert e and its rows r in [offsets[e], offsets[e+1]):
 *   h[r]  = bf16( bf16(silu(bf16(w1_e x_t))) * bf16(w3_e x_t) )       t = perm_tok[r]
 *   y[r]  = w2_e h[r]   (fp32; written as `nsplit` partial sums ypart[s][r][H])
 * with NF4 weights dequantised in registers (blocksize 64) and bf16 MFMA, fp32
 * accumulation.  Replaces ReconstructedNF4Expert.forward (transfer/nf4_reconstruct.py:
 * 152-155) / QuantizedMixtralExpert.forward (model/expert.py:65-75) for all routed
 * experts of a layer at once.  h_ws has T*k*F bf16; ypart has nsplit*T*k*H floats.
 * Requires H % 256 == 0, F % 256 == 0, 1 <= nsplit <= 16. */
int moe_expert_ffn_nf4(const moe_nf4_expert_t *experts, int32_t E, const void *x_bf16,
                       int64_t T, int32_t k, int32_t H, int32_t F, const void *counts,
                       const void *offsets, const void *perm_tok, const void *active,
                       void *h_ws_bf16, void *ypart_f32, int32_t nsplit, void *stream);

/* The two halves of moe_expert_ffn_nf4, for callers that interleave other work:
 * gate/up (`gate = self.w1(x); up = self.w3(x); F.silu(gate) * up`,
 * transfer/nf4_reconstruct.py:153-155) writes h; down (`self.w2(...)`, :155) reads h and
 * writes the nsplit partial sums. */
int moe_expert_gateup_nf4(const moe_nf4_expert_t *experts, int32_t E, const void *x_bf16,
                          int64_t T, int32_t k, int32_t H, int32_t F, const void *counts,
                          const void *offsets, const void *perm_tok, const void *active,
                          void *h_ws_bf16, void *stream);
int moe_expert_down_nf4(const moe_nf4_expert_t *experts, int32_t E, int64_t T, int32_t k,
                        int32_t H, int32_t F, const void *counts, const void *offsets,
                        const void *perm_tok, const void *active, const void *h_ws_bf16,
                        void *ypart_f32, int32_t nsplit, void *stream);

/* ---------------------------------------------------------------- K5: combine
 * out[t] = 0; for the k slots of token t in ascending expert order:
 *   y = bf16(sum_s ypart[s][slot_pos[t*k+j]]);  out[t] = bf16(out[t] + y * w[t,j])
 * (fp32 product and sum, bf16 destination) -- model/moe_layer.py:147,187-191. */
int moe_combine(const void *ypart_f32, int32_t nsplit, const void *weights_f32,
                const void *idx_i32, const void *slot_pos, int64_t T, int32_t k, int32_t H,
                void *out_bf16, void *stream);

/* ---------------------------------------------------------------- single expert
 * y[T,H] = bf16(w2 (silu(w1 x) * w3 x)) for one expert on all T rows of x -- the
 * ReconstructedNF4Expert.__call__ of transfer/nf4_reconstruct.py:152-155.
 * workspace >= moe_expert_workspace_bytes(T, H, F). */
int64_t moe_expert_workspace_bytes(int64_t T, int32_t H, int32_t F);
int moe_expert_swiglu_nf4(const moe_nf4_expert_t *expert, const void *x_bf16, int64_t T,
                          int32_t H, int32_t F, void *y_bf16, void *workspace,
                          int64_t workspace_bytes, void *stream);

/* ---------------------------------------------------------------- whole layer
 * Router (K2) -> permute (K3) -> expert FFN (K4) -> combine (K5) in one call: the
 * device-resident form of MoELayer._forward_tokens (model/moe_layer.py:117-211) with
 * every routed expert resident.  Decode batches (T <= 4, T*k <= 8, E <= 16, H and F
 * multiples of 512) run as two launches: routing and grouping inside the gate/up kernel,
 * the weighted combine inside the down kernel; all E table entries must then be non-null.
 * Larger batches: one routing + grouping kernel (T <= 16) or router + permute, then
 * gate/up, down and combine.  Otherwise experts[e] must be valid for every e < E that
 * the router can select.  logits_bf16 may be NULL; weights_f32 [T,k] and idx_i64 [T,k]
 * receive the routing.  workspace >= moe_layer_workspace_bytes(T, k, E, H, F), 256-byte
 * aligned. */
int64_t moe_layer_workspace_bytes(int64_t T, int32_t k, int32_t E, int32_t H, int32_t F);
/* Number of fp32 ypart planes (K splits of the down projection) the layer and the expert
 * FFN use by default for this shape: what moe_expert_ffn_nf4 / moe_expert_down_nf4 callers
 * pass as nsplit to run the layer's kernels (sizing helper, like the workspace query; the
 * reference has no K splits).  -1 for invalid sizes. */
int32_t moe_layer_down_splits(int64_t T, int32_t k, int32_t E, int32_t H, int32_t F);
int moe_layer_forward_nf4(const moe_nf4_expert_t *experts, int32_t E, const void *gate_bf16,
                          const void *bias_f32, const void *x_bf16, int64_t T, int32_t H,
                          int32_t F, int32_t k, void *out_bf16, void *logits_bf16,
                          void *weights_f32, void *idx_i64, void *workspace,
                          int64_t workspace_bytes, void *stream);

/* moe_layer_forward_nf4 with hipEventRecord marks on the stream: events[0] before the
 * routing, events[1] after routing + grouping, events[2] after gate/up, events[3] after
 * down + combine.  In the two-launch decode form events[0] and events[1] are recorded
 * back to back (the routing runs inside the gate/up kernel).  The kernels are those of
 * moe_layer_forward_nf4; for profiling. */
int moe_layer_forward_nf4_profiled(const moe_nf4_expert_t *experts, int32_t E,
                                   const void *gate_bf16, const void *bias_f32,
                                   const void *x_bf16, int64_t T, int32_t H, int32_t F,
                                   int32_t k, void *out_bf16, void *logits_bf16,
                                   void *weights_f32, void *idx_i64, void *workspace,
                                   int64_t workspace_bytes, void *const *events, void *stream);

/* Allocation-free form of moe_layer_forward_nf4.  No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  Same kernels and results as
 * moe_layer_forward_nf4; the workspace is the library's static per-device scratch of
 * MOE_NOALLOC_SCRATCH_BYTES (each device holds it until the process ends), and the call
 * allocates nothing.  A layer whose workspace (moe_layer_workspace_bytes) exceeds the
 * scratch runs with one down-projection ypart plane instead of K splits when that fits
 * (same routing; outputs within fp32 summation order); larger layers are refused with
 * MOE_STATUS_INVALID_ARGUMENT (Mixtral-8x7B shape: T <= 744 at k = 2).  Every call on a
 * device shares that device's scratch: calls that overlap on one device (two streams, two
 * threads) race. */
#define MOE_NOALLOC_SCRATCH_BYTES (64ll << 20)
int moe_layer_forward_nf4_noalloc(const moe_nf4_expert_t *experts, int32_t E,
                                  const void *gate_bf16, const void *bias_f32,
                                  const void *x_bf16, int64_t T, int32_t H, int32_t F,
                                  int32_t k, void *out_bf16, void *logits_bf16,
                                  void *weights_f32, void *idx_i64, void *stream);

/* Single-token layer with the decoder's post-attention residual add and RMSNorm in front
 * (engine/decoder_layer.py:37-41 feeds the MoE block post_attention_layernorm(h + attn)):
 * r = x + residual -> residual_out, xn = moe_add_rmsnorm_bf16(r) with norm_weight, then
 * moe_layer_forward_nf4 of xn at T = 1 -- bit-identical to that sequence, in the layer's
 * two launches (every gate/up workgroup normalises the token itself).  No bias, no logits
 * output.  workspace: moe_layer_norm_workspace_bytes(k, E, H, F) bytes, 256-byte aligned;
 * H up to 8192.  residual_out must not overlap x or residual (refused: one workgroup
 * writes it while the others read them). */
int64_t moe_layer_norm_workspace_bytes(int32_t k, int32_t E, int32_t H, int32_t F);
int moe_layer_forward_nf4_norm(const moe_nf4_expert_t *experts, int32_t E, const void *gate_bf16,
                               const void *x_bf16, const void *residual_bf16,
                               const void *norm_weight_bf16, float eps, int32_t H, int32_t F,
                               int32_t k, void *residual_out_bf16, void *out_bf16,
                               void *weights_f32, void *idx_i64, void *workspace,
                               int64_t workspace_bytes, void *stream);

/* ---------------------------------------------------------------- decoder (end-to-end)
 * The dense parts of a Mixtral decoder layer around the MoE block, which the reference
 * runs as Hugging Face modules (engine/engine.py:211-314 builds MixtralRMSNorm,
 * MixtralRotaryEmbedding and the eager attention of MixtralDecoderLayer;
 * engine/decoder_layer.py:37-41 swaps in the MoE block).  bf16 tensors, fp32
 * accumulation, bf16 rounding after each elementwise op as on bf16 torch tensors.
 *
 * r = residual_in ? bf16(x + residual_in) : x (written to residual_out when given);
 * out = bf16(weight * bf16(r * rsqrt(mean(r^2) + eps))), per row of [T, H]. */
int moe_add_rmsnorm_bf16(const void *x, const void *residual_in, const void *weight, float eps,
                         int64_t T, int32_t H, void *residual_out, void *out, void *stream);

/* Rotary embedding (rotate-half convention, cos/sin of pos * inv_freq rounded to bf16) of
 * the q and k heads of qkv [T, (n_q + 2 n_kv) * head_dim] at positions *pos0 + t (pos0 a
 * device int32); q to q_out [T, n_q, head_dim], k and v to the caches
 * [n_kv, max_seq, head_dim] at those positions. */
int moe_rope_kv_bf16(const void *qkv, int64_t T, int32_t n_q_heads, int32_t n_kv_heads,
                     int32_t head_dim, const void *inv_freq_f32, const void *pos0_i32,
                     int64_t max_seq, void *q_out, void *k_cache, void *v_cache, void *stream);

/* Grouped-query causal attention of q [T, n_q, head_dim] (query t at position *pos0 + t)
 * against the caches: bf16(bf16(q.k) * scaling) scores, fp32 softmax rounded to bf16,
 * fp32-accumulated sum of the probabilities times v; out [T, n_q * head_dim]. */
int moe_attention_bf16(const void *q, const void *k_cache, const void *v_cache, int64_t T,
                       int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                       const void *pos0_i32, int64_t max_seq, float scaling, void *out,
                       void *stream);

/* y[T, N] = bf16(x[T, K] W[N, K]^T) with fp32 accumulation, 1 <= T <= 4: the decode-time
 * q/k/v/o projections and lm_head (nn.Linear without bias on bf16 tensors). */
int moe_gemv_bf16(const void *weight, const void *x, int64_t T, int32_t N, int32_t K, void *y,
                  void *stream);

/* Fused single-token (decode-step) forms of the above, bit-identical to the unfused
 * sequence; each saves a launch and its dependent-latency chain (engine/engine.py:568-627
 * runs these modules once per generated token).
 *
 * moe_qkv_rope_bf16: r = x[*x_row] (+ residual) -> residual_out (x_row: device int64, null
 * for row 0; rows outside [0, x_rows) clamp), then moe_add_rmsnorm_bf16 of r, the q/k/v
 * projection (weight [(n_q + 2 n_kv) * head_dim, H]) and moe_rope_kv_bf16 at *pos0: q to
 * q_out, k and v to the cache row *pos0.  H a multiple of 512 up to 8192.  residual_out
 * must not overlap x (all x_rows rows) or residual (refused). */
int moe_qkv_rope_bf16(const void *weight, const void *x, const void *x_row_i64, int64_t x_rows,
                      const void *residual, const void *norm_weight, float eps, int32_t H,
                      int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                      const void *inv_freq_f32, const void *pos0_i32, int64_t max_seq,
                      void *residual_out, void *q_out, void *k_cache, void *v_cache, void *stream);

/* moe_head_argmax_bf16: the final norm of r = x + residual, logits[N] = W[N, K] xn (bf16),
 * token = argmax (torch.argmax order: NaN first, then the larger value, then the lower
 * index) as a device int64; when gen_ctr is given, gen[*gen_ctr] = token (if the index is
 * in [0, gen_cap)) and *gen_ctr += 1; when pos is given, *pos += 1.  Two launches (the
 * head with per-workgroup candidates in cand_ws, then a one-workgroup reduction).
 * cand_ws: at least 8 bytes (8 per workgroup used, up to 4 per CU).  K a multiple of 512
 * up to 8192. */
int moe_head_argmax_bf16(const void *weight, const void *x, const void *residual,
                         const void *norm_weight, float eps, int32_t N, int32_t K, void *logits,
                         void *cand_ws, int64_t cand_ws_bytes, void *token_i64, void *gen_i64,
                         int64_t gen_cap, void *gen_ctr_i64, void *pos_i32, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* MOEINFRA_HIP_H */
