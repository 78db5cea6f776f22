// K2: gate linear + fp32 softmax + top-k + renormalise, one wavefront per token.
//
// Follows ExpertRouter.route_with_logits (engine/router.py:50-94):
//   logits = bf16(x . gate^T)          F.linear in the activation dtype  (:66-69)
//   p      = softmax(float(logits))    fp32                               (:81-84)
//   w, idx = topk(p, k)                descending                         (:86-90)
//   w     /= w.sum(-1)                                                    (:92)
// A workgroup holds eight tokens, one per wavefront.  The gate goes through LDS: whole when
// its E x H values fit 64 KB (the Mixtral router: 8 x 4096), staged with every load in
// flight at once, else in double-buffered 8 KB chunks; each workgroup reads it once for its
// eight tokens.  A wave's gate products run on the 4x4x4 MFMA (16 K slices and four experts
// per instruction, fp32 accumulation), a DPP/shuffle butterfly completes each expert's sum,
// and the E logits land in lanes 0..E-1.  Softmax and top-k run across those lanes with
// shuffle reductions and ballots.  An optional fp32 per-expert bias is added to
// float(logits) before the softmax (skewed-routing workloads).  Ties in p keep the lower
// index.
#include "common.h"

namespace moe {
namespace {

// One 8-value step of the gate products for every expert row.  All EMAX row loads are
// issued before any product (rows e >= E re-read row E-1; their sums are discarded), so a
// step costs one memory round trip.
template <int EMAX>
__device__ __forceinline__ void gate_step(const uint16_t *__restrict__ gate, int H, int E, int c,
                                          const float (&xf)[8], float (&acc)[EMAX]) {
  uint4 gv[EMAX];
#pragma unroll
  for (int e = 0; e < EMAX; ++e) {
    const int ee = e < E ? e : E - 1;
    gv[e] = *reinterpret_cast<const uint4 *>(gate + (int64_t)ee * H + c);
  }
  __builtin_amdgcn_sched_barrier(0);  // keep every load ahead of the products
#pragma unroll
  for (int e = 0; e < EMAX; ++e) {
    const uint32_t gw[4] = {gv[e].x, gv[e].y, gv[e].z, gv[e].w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      acc[e] = fmaf(xf[2 * j], bf16lo_to_f32(gw[j]), acc[e]);
      acc[e] = fmaf(xf[2 * j + 1], bf16hi_to_f32(gw[j]), acc[e]);
    }
  }
}

constexpr int kRtWaves = 8;  // tokens per workgroup, one wavefront each
constexpr int kRtThreads = kRtWaves * kWave;
constexpr int kRtChunkBytes = 8192;  // gate bytes per LDS chunk (all expert rows)
// WHOLE: the E x H gate fits kRtWholeBytes of LDS and is staged at once (every load in
// flight together: one memory round trip before the products); otherwise it streams in
// double-buffered 8 KB chunks.
constexpr int kRtWholeBytes = 65536;
constexpr int kRtPad = 8;  // values of padding per LDS gate row (rows 16 bytes apart in banks)

// Over lanes 0..N-1 (N = 16: DPP within the row; N = 32, 64: then permlane swaps): every lane
// of those rows gets the result, the same bits in all of them (each step combines two
// partials that the partner combines in the other order).
template <int N>
__device__ __forceinline__ float rt_max(float v) {
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xf, 0xf, false)));
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xf, 0xf, false)));
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x124, 0xf, 0xf, false)));
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x128, 0xf, 0xf, false)));
  if constexpr (N > 16) v = op_xor16<true>(v);
  if constexpr (N > 32) v = op_xor32<true>(v);
  return v;
}
// Sum over lanes 0..N-1 by the butterfly l ^ 1, 2, 4, ... (DPP for 1, 2 and 8, permlane
// swaps for 16 and 32, an LDS shuffle for 4).
template <int N>
__device__ __forceinline__ float rt_sum(float v) {
  if constexpr (N > 1) v += dpp_mov<0xB1>(v);
  if constexpr (N > 2) v += dpp_mov<0x4E>(v);
  if constexpr (N > 4) v += __shfl_xor(v, 4, kWave);
  if constexpr (N > 8) v += dpp_mov<0x128>(v);
  if constexpr (N > 16) v = op_xor16<false>(v);
  if constexpr (N > 32) v = op_xor32<false>(v);
  return v;
}

typedef __attribute__((__vector_size__(4 * sizeof(short)))) short rt_s16x4;
__device__ __forceinline__ rt_s16x4 rt_pair(uint32_t lo, uint32_t hi) {
  return __builtin_bit_cast(rt_s16x4, make_uint2(lo, hi));
}
// Sum over the 16 lanes that share lane % 4 (DPP rotations within rows, then across rows).
__device__ __forceinline__ float rt_sum16(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x124, 0xf, 0xf, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x128, 0xf, 0xf, false));
  v = op_xor16<false>(v);
  v = op_xor32<false>(v);
  return v;
}

// Gate products of one token per wavefront on v_mfma_f32_4x4x4_16b_bf16: per 128-value
// step of H, lane (b = lane / 4, j = lane % 4) holds values 8b .. 8b+7 of the token (A
// rows, the same token in all four) and of gate row 4g + j (B columns) for each group g of
// four experts; the 16 MFMA blocks are 16 K slices, summed by a butterfly at the end.
template <int EMAX, bool WHOLE>
__global__ void __launch_bounds__(kRtThreads)
router_topk_kernel(const uint16_t *__restrict__ x, const uint16_t *__restrict__ gate,
                   const float *__restrict__ bias, int64_t T, int H, int E, int k,
                   uint16_t *__restrict__ logits_out, float *__restrict__ w_out,
                   int64_t *__restrict__ idx_out, int32_t *__restrict__ idx32_out, int tpw) {
  static_assert(EMAX == 8 || EMAX == 16 || EMAX == 32, "EMAX must be 8, 16 or 32");
  constexpr int G = EMAX / 4;
  constexpr int CH = kRtChunkBytes / 2 / EMAX;  // streamed: values per LDS chunk (512, 256, 128)
  constexpr int SUB = CH / 128;                 // 128-value MFMA steps per streamed chunk
  constexpr int PPR = CH / 8;                   // 16-byte pieces per row and chunk
  static_assert(EMAX * PPR == kRtThreads, "one 16-byte gate piece per thread and chunk");
  constexpr int CROW = CH + kRtPad;             // streamed LDS row stride (values)
  __shared__ __attribute__((aligned(16))) uint16_t s_g[WHOLE ? 1 : 2][WHOLE ? 8 : EMAX * CROW];
  extern __shared__ __attribute__((aligned(16))) uint16_t s_whole[];  // WHOLE: [E][H + pad]

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid >> 6;
  const int lj = lane & 3, lb = lane >> 2;
  // Waves 0..tpw-1 hold tokens; every wave stages the gate (and, streamed, passes every
  // chunk's barrier).
  const int64_t t = (int64_t)blockIdx.x * tpw + wave;
  const bool live = wave < tpw && t < T;
  const uint16_t *xr = x + (live ? t : T - 1) * (int64_t)H;
  const int n_steps = (H + 127) / 128;
  // The lane's 8 values of 128-value step st (zeros past H, from a clamped in-bounds load).
  auto load_x16 = [&](int st) -> uint4 {
    const int v = st * 128 + 8 * lb;
    const uint4 q = *reinterpret_cast<const uint4 *>(xr + (v < H ? v : H - 8));
    const bool in = v < H;
    return make_uint4(in ? q.x : 0u, in ? q.y : 0u, in ? q.z : 0u, in ? q.w : 0u);
  };

  f32x4 gacc[G];
#pragma unroll
  for (int g = 0; g < G; ++g) gacc[g] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  if constexpr (WHOLE) {
    // Rows e < E of the gate in LDS, each padded with zeros to a multiple of 128 values
    // (+ kRtPad), so every step reads inside its row; every thread's pieces in flight at
    // once, with the token's first eight slices.
    const int hp = n_steps * 128;
    const int stride = hp + kRtPad;
    constexpr int XB = 8;
    uint4 xq[XB];
#pragma unroll
    for (int u = 0; u < XB; ++u) xq[u] = load_x16(u);
    const int ppr = hp / 8;
#pragma unroll 8
    for (int p = tid; p < E * ppr; p += kRtThreads) {
      const int e = p / ppr, o = (p - e * ppr) * 8;
      *reinterpret_cast<uint4 *>(s_whole + e * stride + o) =
          o < H ? *reinterpret_cast<const uint4 *>(gate + (int64_t)e * H + o)
                : make_uint4(0u, 0u, 0u, 0u);
    }
    __syncthreads();
    if (wave >= tpw) return;  // wave-uniform; no barrier follows
    // Groups' lanes past E read row E - 1 (their sums are discarded).
    const uint16_t *grow[G];
#pragma unroll
    for (int g = 0; g < G; ++g)
      grow[g] = s_whole + (4 * g + lj < E ? 4 * g + lj : E - 1) * stride + 8 * lb;
    for (int s0 = 0; s0 < n_steps; s0 += XB) {
      if (s0 > 0) {
#pragma unroll
        for (int u = 0; u < XB; ++u) xq[u] = load_x16(s0 + u);
      }
      // Steps past the last re-read the last one with a zero token slice (load_x16).
      uint4 gq[XB][G];
#pragma unroll
      for (int u = 0; u < XB; ++u) {
        const int st = s0 + u < n_steps ? s0 + u : n_steps - 1;
#pragma unroll
        for (int g = 0; g < G; ++g) gq[u][g] = *reinterpret_cast<const uint4 *>(grow[g] + st * 128);
      }
#pragma unroll
      for (int u = 0; u < XB; ++u)
#pragma unroll
        for (int g = 0; g < G; ++g) {
          gacc[g] = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(rt_pair(xq[u].x, xq[u].y),
                                                          rt_pair(gq[u][g].x, gq[u][g].y), gacc[g], 0, 0, 0);
          gacc[g] = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(rt_pair(xq[u].z, xq[u].w),
                                                          rt_pair(gq[u][g].z, gq[u][g].w), gacc[g], 0, 0, 0);
        }
    }
  } else {
    // This thread's gate piece of a chunk: row ge (clamped to E - 1), values go .. go + 7.
    const int ge = tid / PPR, go = (tid % PPR) * 8;
    const uint16_t *grow = gate + (int64_t)(ge < E ? ge : E - 1) * H;
    const int n_chunks = (H + CH - 1) / CH;
    auto load_piece = [&](int c) -> uint4 {
      const int v = c * CH + go;
      return v < H ? *reinterpret_cast<const uint4 *>(grow + v) : make_uint4(0u, 0u, 0u, 0u);
    };
    uint4 piece = load_piece(0);
    uint4 xq[SUB], xn[SUB];
#pragma unroll
    for (int u = 0; u < SUB; ++u) xq[u] = load_x16(u);
    for (int c = 0; c < n_chunks; ++c) {
      uint16_t *buf = s_g[c & 1];
      *reinterpret_cast<uint4 *>(buf + ge * CROW + go) = piece;
      __syncthreads();  // chunk c visible; the other buffer is free (its readers passed here)
      if (c + 1 < n_chunks) {
        piece = load_piece(c + 1);
#pragma unroll
        for (int u = 0; u < SUB; ++u) xn[u] = load_x16((c + 1) * SUB + u);
      }
      uint4 gq[SUB][G];
#pragma unroll
      for (int u = 0; u < SUB; ++u)
#pragma unroll
        for (int g = 0; g < G; ++g)
          gq[u][g] = *reinterpret_cast<const uint4 *>(buf + (4 * g + lj) * CROW + u * 128 + 8 * lb);
#pragma unroll
      for (int u = 0; u < SUB; ++u)
#pragma unroll
        for (int g = 0; g < G; ++g) {
          gacc[g] = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(rt_pair(xq[u].x, xq[u].y),
                                                          rt_pair(gq[u][g].x, gq[u][g].y), gacc[g], 0, 0, 0);
          gacc[g] = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(rt_pair(xq[u].z, xq[u].w),
                                                          rt_pair(gq[u][g].z, gq[u][g].w), gacc[g], 0, 0, 0);
        }
#pragma unroll
      for (int u = 0; u < SUB; ++u) xq[u] = xn[u];
    }
  }

  // Expert 4g + j's total: the butterfly over the 16 blocks leaves it in every lane with
  // lane % 4 == j; lane e (< E) takes expert e from lane e % 4.
  float sum = 0.0f;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float v = __shfl(rt_sum16(gacc[g][0]), lane & 3, kWave);
    if ((lane >> 2) == g) sum = v;
  }

  // ---- softmax and top-k across lanes 0..E-1 (lane e = expert e)
  const bool valid = lane < E;
  float l = -INFINITY;
  if (valid) {
    const uint16_t lb = f32_to_bf16(sum);
    if (live && logits_out != nullptr) logits_out[t * E + lane] = lb;
    l = bf16_to_f32(lb);
    if (bias != nullptr) l = l + bias[lane];
  }
  constexpr int NR = EMAX <= 16 ? 16 : 32;  // lanes holding experts
  const float mx = rt_max<NR>(l);
  const float pe = valid ? expf(l - mx) : 0.0f;
  const float p = pe / rt_sum<NR>(pe);
  bool taken = false;
  float wsum = 0.0f, my_w = 0.0f;
  int my_i = 0;
  for (int j = 0; j < k; ++j) {
    const bool cand = valid && !taken;
    const float best = rt_max<NR>(cand ? p : -1.0f);
    const uint64_t hit = __ballot(cand && p == best);
    // No candidate equal to the maximum (NaN probabilities): the lowest untaken expert.
    const uint64_t any = __ballot(cand);
    const int win = hit != 0 ? (int)__builtin_ctzll(hit) : (int)__builtin_ctzll(any);
    taken |= lane == win;
    wsum += best;
    if (lane == j) {
      my_i = win;
      my_w = best;
    }
  }
  if (live && lane < k) {
    w_out[t * k + lane] = my_w / wsum;
    idx_out[t * k + lane] = my_i;
    if (idx32_out != nullptr) idx32_out[t * k + lane] = my_i;
  }
}

}  // namespace
}  // namespace moe

extern "C" int moe_router_topk(const void *x_bf16, const void *gate_bf16, const void *bias_f32,
                               int64_t T, int32_t H, int32_t E, int32_t k, void *logits_bf16,
                               void *weights_f32, void *idx_i64, void *idx_i32, void *stream) {
  MOE_REQUIRE(T >= 0, "T must be non-negative");
  MOE_REQUIRE(H > 0 && H % 8 == 0, "hidden size must be a positive multiple of 8 (got %d)", H);
  MOE_REQUIRE(E >= 1 && E <= MOE_MAX_EXPERTS, "num_experts must be in [1, %d] (got %d)",
              MOE_MAX_EXPERTS, E);
  MOE_REQUIRE(k >= 1 && k <= E && k <= MOE_MAX_TOPK, "top-k must be in [1, min(E, %d)] (got %d)",
              MOE_MAX_TOPK, k);
  if (T == 0) return MOE_STATUS_OK;
  MOE_REQUIRE(x_bf16 && gate_bf16 && weights_f32 && idx_i64, "null device pointer");
  MOE_REQUIRE(((uintptr_t)x_bf16 % 16) == 0 && ((uintptr_t)gate_bf16 % 16) == 0,
              "x and gate must be 16-byte aligned");
  MOE_REQUIRE(T <= 0x7fffffff, "too many tokens");
  // Tokens per workgroup: eight once that still gives every CU a workgroup, fewer (down to
  // one wavefront with a token, the other seven only staging the gate) for smaller batches,
  // so that they spread over the CUs.
  const int64_t cus = moe::device_cu_count();
  int tpw = moe::kRtWaves;
  while (tpw > 1 && (T + tpw - 1) / tpw < cus) tpw >>= 1;
  const dim3 g((unsigned)((T + tpw - 1) / tpw)), b(moe::kRtThreads);
  hipStream_t s = (hipStream_t)stream;
  const int64_t gate_bytes = (int64_t)E * ((H + 127) / 128 * 128 + moe::kRtPad) * 2;
  const bool whole = gate_bytes <= moe::kRtWholeBytes + 16 * 32;
  auto args = [&](auto kern) {
    hipLaunchKernelGGL(kern, g, b, whole ? (size_t)gate_bytes : 0, s, (const uint16_t *)x_bf16,
                       (const uint16_t *)gate_bf16, (const float *)bias_f32, T, H, E, k,
                       (uint16_t *)logits_bf16, (float *)weights_f32, (int64_t *)idx_i64,
                       (int32_t *)idx_i32, tpw);
  };
  if (E <= 8)
    whole ? args(moe::router_topk_kernel<8, true>) : args(moe::router_topk_kernel<8, false>);
  else if (E <= 16)
    whole ? args(moe::router_topk_kernel<16, true>) : args(moe::router_topk_kernel<16, false>);
  else
    whole ? args(moe::router_topk_kernel<32, true>) : args(moe::router_topk_kernel<32, false>);
  MOE_LAUNCH_CHECK();
  return MOE_STATUS_OK;
}

// ----------------------------------------------------------------------------- K2+K3 fused
// Decode-sized batches (T <= 16): routing and the expert grouping in one 1024-thread
// workgroup.  Token t is handled by a group of 16/T waves that split H; the group's
// partial logits are summed in a fixed order, then one thread per token finishes the
// softmax / top-k exactly as router_topk_kernel does.  The grouping (stable counting
// sort over the T*k slots) follows in the same workgroup, and `zero_word` (if given) is
// cleared for a later kernel's completion counter.
namespace moe {
namespace {

constexpr int kRouteThreads = 1024;
constexpr int kRouteWaves = kRouteThreads / kWave;
constexpr int kRouteMaxTokens = 16;

constexpr int kRouteChunk = 256;  // values of H per wave and step in the chunked form

// Orders one wave's LDS writes before its own lanes' reads of other lanes' data
// (wavefront-scope fences around a wave barrier).
__device__ __forceinline__ void route_wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// CHUNKED: E <= 8 and H a multiple of 256 (the gate products by H chunk, below); else one
// group of 16/T waves per token streams its row and the gate.
template <int EMAX, bool CHUNKED>
__global__ void __launch_bounds__(kRouteThreads)
route_small_kernel(const uint16_t *__restrict__ x, const uint16_t *__restrict__ gate,
                   const float *__restrict__ bias, int T, int H, int E, int k,
                   uint16_t *__restrict__ logits_out, float *__restrict__ w_out,
                   int64_t *__restrict__ idx_out, int32_t *__restrict__ idx32_out,
                   int32_t *__restrict__ counts, int32_t *__restrict__ offsets,
                   int32_t *__restrict__ perm_tok, int32_t *__restrict__ slot_pos,
                   int32_t *__restrict__ active, uint32_t *__restrict__ zero_word) {
  __shared__ float s_part[kRouteWaves][EMAX];
  __shared__ float s_tpart[CHUNKED ? kRouteWaves : 1][kRouteMaxTokens][EMAX];
  __shared__ __attribute__((aligned(16))) uint16_t s_g[CHUNKED ? kRouteWaves : 1][EMAX * kRouteChunk];
  __shared__ int32_t s_idx[kRouteMaxTokens * MOE_MAX_TOPK];
  __shared__ int32_t s_off[MOE_MAX_EXPERTS + 1];
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid >> 6;
  const int wpt = kRouteWaves / T;           // waves per token
  const int t = wave / wpt;                  // this wave's token (t >= T: idle)
  const int gtid = (wave - t * wpt) * kWave + lane;
  const int gsize = wpt * kWave;

  if (tid == 0 && zero_word != nullptr) *zero_word = 0u;

  float acc[EMAX];
#pragma unroll
  for (int e = 0; e < EMAX; ++e) acc[e] = 0.0f;
  if (CHUNKED) {
    // Wave w takes the 256-value chunks w, w + 16, ... of H for every token, so each gate
    // value is read once per workgroup: the chunk's gate rows go to the wave's LDS slot,
    // lane (token tl = lane % 16, part p = lane / 16) multiplies its 64 values of the chunk
    // by them; parts are summed with two butterflies, waves in order below.
    const int tl = lane & 15, p = lane >> 4;
    uint16_t *sg = s_g[CHUNKED ? wave : 0];
    for (int ch = wave; ch < H / kRouteChunk; ch += kRouteWaves) {
      const int c0 = ch * kRouteChunk;
#pragma unroll
      for (int i = 0; i < EMAX * kRouteChunk / (8 * kWave); ++i) {
        const int v = (i * kWave + lane) * 8;  // value index within the EMAX x 256 block
        const int e = v / kRouteChunk, o = v - e * kRouteChunk;
        *reinterpret_cast<uint4 *>(sg + v) = *reinterpret_cast<const uint4 *>(
            gate + (int64_t)(e < E ? e : E - 1) * H + c0 + o);
      }
      const uint16_t *xr = x + (int64_t)(tl < T ? tl : T - 1) * H + c0 + p * 64;
      uint4 xv[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) xv[j] = *reinterpret_cast<const uint4 *>(xr + 8 * j);
      route_wave_sync();
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint32_t xw[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
#pragma unroll
        for (int e = 0; e < EMAX; ++e) {
          const uint4 gv = *reinterpret_cast<const uint4 *>(sg + e * kRouteChunk + p * 64 + 8 * j);
          const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w};
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            acc[e] = fmaf(bf16lo_to_f32(xw[q]), bf16lo_to_f32(gw[q]), acc[e]);
            acc[e] = fmaf(bf16hi_to_f32(xw[q]), bf16hi_to_f32(gw[q]), acc[e]);
          }
        }
      }
      route_wave_sync();  // the slot is rewritten by the next chunk
    }
#pragma unroll
    for (int e = 0; e < EMAX; ++e) {
      float v = acc[e];
      v = op_xor16<false>(v);
      v = op_xor32<false>(v);
      if (lane < kRouteMaxTokens) s_tpart[CHUNKED ? wave : 0][lane][e] = v;
    }
  } else if (t < T) {
    const uint16_t *xr = x + (int64_t)t * H;
    for (int c = gtid * 8; c < H; c += gsize * 8) {
      const uint4 xv = *reinterpret_cast<const uint4 *>(xr + c);
      const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
      float xf[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        xf[2 * j] = bf16lo_to_f32(xw[j]);
        xf[2 * j + 1] = bf16hi_to_f32(xw[j]);
      }
      gate_step<EMAX>(gate, H, E, c, xf, acc);
    }
  }
  if (!CHUNKED) {
#pragma unroll
    for (int e = 0; e < EMAX; ++e) {
      const float v = wave_sum(acc[e]);
      if (lane == 0) s_part[wave][e] = v;
    }
  }
  __syncthreads();

  if (tid < T) {
    const int tt = tid;
    float p[EMAX];
    float m = -INFINITY;
#pragma unroll
    for (int e = 0; e < EMAX; ++e) {
      if (e < E) {
        float v;
        if (CHUNKED) {
          v = s_tpart[0][tt][e];
          for (int w = 1; w < kRouteWaves; ++w) v += s_tpart[CHUNKED ? w : 0][tt][e];
        } else {
          v = s_part[tt * wpt][e];
          for (int w = 1; w < wpt; ++w) v += s_part[tt * wpt + w][e];
        }
        const uint16_t lb = f32_to_bf16(v);
        if (logits_out != nullptr) logits_out[(int64_t)tt * E + e] = lb;
        float l = bf16_to_f32(lb);
        if (bias != nullptr) l = l + bias[e];
        p[e] = l;
        m = fmaxf(m, l);
      }
    }
    float s = 0.0f;
#pragma unroll
    for (int e = 0; e < EMAX; ++e) {
      if (e < E) {
        p[e] = expf(p[e] - m);
        s += p[e];
      }
    }
#pragma unroll
    for (int e = 0; e < EMAX; ++e)
      if (e < E) p[e] = p[e] / s;
    float topw[MOE_MAX_TOPK];
    int topi[MOE_MAX_TOPK];
    uint64_t taken = 0;
    float wsum = 0.0f;
    for (int j = 0; j < k; ++j) {
      float best = -INFINITY;
      int bi = -1;
#pragma unroll
      for (int e = 0; e < EMAX; ++e) {
        if (e < E && !((taken >> e) & 1ull) && (bi < 0 || p[e] > best)) {
          best = p[e];
          bi = e;
        }
      }
      taken |= 1ull << bi;
      topw[j] = best;
      topi[j] = bi;
      wsum += best;
    }
    for (int j = 0; j < k; ++j) {
      w_out[tt * k + j] = topw[j] / wsum;
      idx_out[tt * k + j] = topi[j];
      if (idx32_out != nullptr) idx32_out[tt * k + j] = topi[j];
      s_idx[tt * k + j] = topi[j];
    }
  }
  __syncthreads();

  // Grouping: same outputs as permute_kernel (ascending expert, then ascending slot).
  const int n_slots = T * k;
  // Counts by one thread per expert (the slots read as a broadcast), then the running
  // offsets and the active list by thread 0 over the E counts.
  __shared__ int32_t s_cnt[MOE_MAX_EXPERTS];
  if (tid < E) {
    int c = 0;
    for (int s = 0; s < n_slots; ++s) c += s_idx[s] == tid;
    s_cnt[tid] = c;
    counts[tid] = c;
  }
  __syncthreads();
  if (tid == 0) {
    int run = 0, na = 0;
    for (int e = 0; e < E; ++e) {
      const int c = s_cnt[e];
      offsets[e] = run;
      s_off[e] = run;
      if (c > 0) active[1 + na++] = e;
      run += c;
    }
    offsets[E] = run;
    active[0] = na;
    for (int e = na; e < E; ++e) active[1 + e] = -1;
  }
  __syncthreads();
  if (tid < n_slots) {
    const int e = s_idx[tid];
    int rank = 0;
    for (int s = 0; s < tid; ++s) rank += s_idx[s] == e;
    const int pos = s_off[e] + rank;
    perm_tok[pos] = tid / k;
    slot_pos[tid] = pos;
  }
}

}  // namespace

bool route_small_supported(int64_t T, int32_t k) {
  return T >= 1 && T <= kRouteMaxTokens && k <= MOE_MAX_TOPK;
}

int launch_route_small(const void *x, const void *gate, const void *bias, int64_t T, int32_t H,
                       int32_t E, int32_t k, void *logits, void *w, void *idx64, void *idx32,
                       void *counts, void *offsets, void *perm_tok, void *slot_pos, void *active,
                       void *zero_word, hipStream_t stream) {
  MOE_REQUIRE(route_small_supported(T, k), "fused routing needs 1 <= T <= %d", kRouteMaxTokens);
  MOE_REQUIRE(H > 0 && H % 8 == 0, "hidden size must be a positive multiple of 8 (got %d)", H);
  MOE_REQUIRE(E >= 1 && E <= MOE_MAX_EXPERTS && k >= 1 && k <= E, "bad E or k");
  MOE_REQUIRE(((uintptr_t)x % 16) == 0 && ((uintptr_t)gate % 16) == 0,
              "x and gate must be 16-byte aligned");
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3(1), dim3(kRouteThreads), 0, stream, (const uint16_t *)x,
                       (const uint16_t *)gate, (const float *)bias, (int)T, H, E, k,
                       (uint16_t *)logits, (float *)w, (int64_t *)idx64, (int32_t *)idx32,
                       (int32_t *)counts, (int32_t *)offsets, (int32_t *)perm_tok,
                       (int32_t *)slot_pos, (int32_t *)active, (uint32_t *)zero_word);
  };
  if (E <= 8 && H % kRouteChunk == 0)
    go(route_small_kernel<8, true>);
  else if (E <= 8)
    go(route_small_kernel<8, false>);
  else if (E <= 16)
    go(route_small_kernel<16, false>);
  else
    go(route_small_kernel<32, false>);
  MOE_LAUNCH_CHECK();
  return MOE_STATUS_OK;
}

}  // namespace moe
