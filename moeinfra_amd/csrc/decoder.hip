// Dense parts of a Mixtral decoder layer around the MoE block, for the end-to-end decode
// (the reference runs them as Hugging Face modules: engine/engine.py:211-314 builds
// MixtralRMSNorm, MixtralRotaryEmbedding and the eager attention of MixtralDecoderLayer,
// engine/decoder_layer.py:37-41 swaps in the MoE block).  Numerics follow those modules on
// bf16 tensors: bf16 rounding after every elementwise op, fp32 accumulation in products,
// fp32 softmax.
//
//   add_rmsnorm   r = x (+ residual), out = bf16(w * bf16(r * rsqrt(mean(r^2) + eps)))
//   rope_kv       q, k rotated (rotate-half convention, cos/sin rounded to bf16) at
//                 positions pos0 + t; k and v written to the KV cache
//   attention     grouped-query causal attention of T query rows against the cache
//   gemv          y = bf16(W x) for up to 4 tokens (the decode projections and lm_head)
// and the fused single-token forms of a decode step:
//   qkv_rope      input norm + q/k/v projection + rotary + KV-cache write
//   head_logits   final norm + lm_head + per-workgroup argmax candidates, and
//   argmax_finish the token, the generated-id buffer, its counter and the position
// (the post-attention norm runs inside the MoE layer's gate/up kernel, decode_layer.hip).
#include "norm_row.h"

namespace moe {
namespace {

template <int CH, bool RES>
__global__ void __launch_bounds__(kNormThreads)
add_rmsnorm_kernel(const uint16_t *__restrict__ x, const uint16_t *__restrict__ res_in,
                   const uint16_t *__restrict__ w, float eps, int H,
                   uint16_t *__restrict__ res_out, uint16_t *__restrict__ out) {
  __shared__ float s_part[kNormThreads / kWave];
  const size_t base = (size_t)blockIdx.x * H;
  rmsnorm_row<CH, RES>(x + base, RES ? res_in + base : nullptr, w, eps, H,
                       res_out ? res_out + base : nullptr, out + base, s_part);
}

constexpr int kRopeThreads = 256;
constexpr int kRopeMaxHalf = 256;  // head_dim <= 512

__device__ __forceinline__ void unpack8(const uint4 v, float *f) {
  const uint32_t a[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    f[2 * e] = bf16lo_to_f32(a[e]);
    f[2 * e + 1] = bf16hi_to_f32(a[e]);
  }
}

// Token t (blockIdx.x) at position pos0 + t.  The hd/2 rotary angles of the position are
// evaluated once (cos/sin rounded to bf16, as the bf16 module's cos/sin tensors) into LDS;
// then each thread rotates 8 consecutive values of the first half of a q or k head with the
// matching 8 of the second half (value i pairs with i + hd/2), 16-byte loads and stores.
// q goes to q_out [T, nq, hd]; k and v go to the cache rows [kv head][pos][hd].
__global__ void __launch_bounds__(kRopeThreads)
rope_kv_kernel(const uint16_t *__restrict__ qkv, int nq, int nkv, int hd,
               const float *__restrict__ inv_freq, const int32_t *__restrict__ pos0,
               int64_t max_seq, uint16_t *__restrict__ q_out, uint16_t *__restrict__ kc,
               uint16_t *__restrict__ vc) {
  __shared__ float s_cos[kRopeMaxHalf], s_sin[kRopeMaxHalf];
  const int t = blockIdx.x;
  const int pos = *pos0 + t;
  if (pos < 0 || pos >= max_seq) return;  // the cache has no row for it (caller error)
  const int half = hd >> 1;
  for (int i = threadIdx.x; i < half; i += kRopeThreads) {
    const float ang = (float)pos * inv_freq[i];
    s_cos[i] = bf16r(cosf(ang));
    s_sin[i] = bf16r(sinf(ang));
  }
  __syncthreads();
  const int row = (nq + 2 * nkv) * hd;
  const uint16_t *src = qkv + (size_t)t * row;
  const int cph = half >> 3;  // 8-value chunks per half head
  for (int idx = threadIdx.x; idx < (nq + nkv) * cph; idx += kRopeThreads) {
    const int head = idx / cph, c = idx - head * cph;
    const uint16_t *hx = src + (size_t)head * hd + c * 8;  // k heads follow the q heads
    float x1[8], x2[8];
    unpack8(*reinterpret_cast<const uint4 *>(hx), x1);
    unpack8(*reinterpret_cast<const uint4 *>(hx + half), x2);
    uint32_t o1[4], o2[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float r1[2], r2[2];
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const int i = c * 8 + 2 * e + k;
        const float co = s_cos[i], si = s_sin[i];
        const float a = x1[2 * e + k], b = x2[2 * e + k];
        r1[k] = bf16r(a * co) + bf16r(-b * si);
        r2[k] = bf16r(b * co) + bf16r(a * si);
      }
      o1[e] = pack_bf16x2(r1[0], r1[1]);
      o2[e] = pack_bf16x2(r2[0], r2[1]);
    }
    uint16_t *dst = head < nq ? q_out + ((size_t)t * nq + head) * hd
                              : kc + ((size_t)(head - nq) * max_seq + pos) * hd;
    *reinterpret_cast<uint4 *>(dst + c * 8) = make_uint4(o1[0], o1[1], o1[2], o1[3]);
    *reinterpret_cast<uint4 *>(dst + half + c * 8) = make_uint4(o2[0], o2[1], o2[2], o2[3]);
  }
  const uint16_t *vsrc = src + (size_t)(nq + nkv) * hd;
  const int cpr = hd >> 3;
  for (int idx = threadIdx.x; idx < nkv * cpr; idx += kRopeThreads) {
    const int head = idx / cpr, c = idx - head * cpr;
    *reinterpret_cast<uint4 *>(vc + ((size_t)head * max_seq + pos) * hd + c * 8) =
        *reinterpret_cast<const uint4 *>(vsrc + (size_t)head * hd + c * 8);
  }
}

constexpr int kAttnThreads = 256;
constexpr int kAttnMaxKeys = 8192;
constexpr int kAttnMaxHeadDim = 256;
constexpr int kAttnRowsInFlight = 8;  // cache rows per thread per pass

// Scores of the pass starting at key j0 from its loaded K rows: s_p[j] = bf16(bf16(q.k_j) *
// scaling) for the keys j < nkeys, and the running maximum.  The eight rows' lane partials
// are formed first and summed over each row's lpr lanes together (DPP within a 16-lane row).
__device__ __forceinline__ void attn_scores(const uint4 (&kv)[kAttnRowsInFlight], const float (&qf)[8],
                                            int j0, int nkeys, int rpp, int rr, int lpr, int sub,
                                            float scaling, float *s_p, float &mx) {
  float dot[kAttnRowsInFlight];
#pragma unroll
  for (int u = 0; u < kAttnRowsInFlight; ++u) {
    float kf[8];
    unpack8(kv[u], kf);
    float d = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) d = fmaf(qf[e], kf[e], d);
    dot[u] = d;
  }
  lane_groups_reduce<false>(dot, lpr);
#pragma unroll
  for (int u = 0; u < kAttnRowsInFlight; ++u) {
    const int j = j0 + u * rpp + rr;
    const float sc = bf16r(bf16r(dot[u]) * scaling);
    const bool ok = j < nkeys;
    mx = ok ? fmaxf(mx, sc) : mx;
    if (ok && sub == 0) s_p[j] = sc;
  }
}

// acc += p_j v_j over the pass's rows j < nkeys, in row order.
__device__ __forceinline__ void attn_pv(const uint4 (&vv)[kAttnRowsInFlight], int j0, int nkeys,
                                        int rpp, int rr, const float *s_p, float (&acc)[8]) {
#pragma unroll
  for (int u = 0; u < kAttnRowsInFlight; ++u) {
    const int j = j0 + u * rpp + rr;
    if (j < nkeys) {
      const float p = s_p[j];
      float vf[8];
      unpack8(vv[u], vf);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = fmaf(p, vf[e], acc[e]);
    }
  }
}

// One workgroup per (query head, token): scores of keys 0 .. pos0 + t (causal), bf16 scores
// scaled in bf16, fp32 softmax rounded to bf16, then the bf16 probabilities times V with
// fp32 accumulation.  A cache row of hd bf16 is read by hd/8 consecutive lanes, 16 bytes
// each, so the workgroup covers rpp = 256/(hd/8) rows per load instruction and a pass takes
// 8 such loads per thread (128 rows at hd = 128); a score is the xor-shuffle sum over its
// row's lanes.  The first pass's K and V rows are loaded together with q and the position,
// before the key count is known (row indexes clamped to the cache, results of rows past the
// last key discarded), so a context of up to one pass of keys costs one memory round trip;
// later passes load rows clamped to the last key.
__global__ void __launch_bounds__(kAttnThreads)
attention_kernel(const uint16_t *__restrict__ q, const uint16_t *__restrict__ kc,
                 const uint16_t *__restrict__ vc, int nq, int nkv, int hd,
                 const int32_t *__restrict__ pos0, int64_t max_seq, float scaling,
                 uint16_t *__restrict__ out) {
  __shared__ float s_p[kAttnMaxKeys];
  __shared__ float s_red[kAttnThreads / kWave];
  __shared__ __attribute__((aligned(16))) float s_acc[kAttnThreads * 8];
  MOE_ARGS_FIRST(MOE_LIST("+s"(nq), "+s"(nkv), "+s"(hd), "+s"(max_seq), "+s"(scaling)),
                 MOE_LIST("s"(q), "s"(kc), "s"(vc), "s"(pos0), "s"(out)));
  const int h = blockIdx.x, t = blockIdx.y;
  const int kvh = h / (nq / nkv);
  const int lpr = hd >> 3;               // lanes per row: a power of two <= 32
  const int rpp = kAttnThreads / lpr;    // rows per load instruction of the workgroup
  const int npass = kAttnRowsInFlight * rpp;
  const int sub = threadIdx.x & (lpr - 1), rr = threadIdx.x / lpr;
  float qf[8];
  unpack8(*reinterpret_cast<const uint4 *>(q + ((size_t)t * nq + h) * hd + sub * 8), qf);
  const uint16_t *kbase = kc + (size_t)kvh * max_seq * hd + sub * 8;
  const uint16_t *vbase = vc + (size_t)kvh * max_seq * hd + sub * 8;
  uint4 kv[kAttnRowsInFlight], vv[kAttnRowsInFlight];
#pragma unroll
  for (int u = 0; u < kAttnRowsInFlight; ++u) {
    const int j = min(u * rpp + rr, (int)max_seq - 1);
    kv[u] = *reinterpret_cast<const uint4 *>(kbase + (size_t)j * hd);
    vv[u] = *reinterpret_cast<const uint4 *>(vbase + (size_t)j * hd);
  }
  // Keys 0 .. pos0 + t, bounded by the cache (a position past it is a caller error).
  const int nkeys = min(*pos0 + t + 1, (int)max_seq);
  float mx = -INFINITY;
  attn_scores(kv, qf, 0, nkeys, rpp, rr, lpr, sub, scaling, s_p, mx);
  for (int j0 = npass; j0 < nkeys; j0 += npass) {
#pragma unroll
    for (int u = 0; u < kAttnRowsInFlight; ++u) {
      const int j = min(j0 + u * rpp + rr, nkeys - 1);
      kv[u] = *reinterpret_cast<const uint4 *>(kbase + (size_t)j * hd);
    }
    attn_scores(kv, qf, j0, nkeys, rpp, rr, lpr, sub, scaling, s_p, mx);
  }
  // block max, then the block sum of the exponentials (each a wave reduction, then the
  // four waves' values through LDS in wave order)
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x >> 6;
  {
    float m[1] = {mx};
    lane_groups_reduce<true>(m, kWave);
    if (lane == 0) s_red[wave] = m[0];
    __syncthreads();
    mx = s_red[0];
    for (int w = 1; w < kAttnThreads / kWave; ++w) mx = fmaxf(mx, s_red[w]);
    __syncthreads();
  }
  float sum = 0.0f;
  for (int j = threadIdx.x; j < nkeys; j += kAttnThreads) {
    const float e = expf(s_p[j] - mx);
    s_p[j] = e;
    sum += e;
  }
  {
    float v[1] = {sum};
    lane_groups_reduce<false>(v, kWave);
    if (lane == 0) s_red[wave] = v[0];
    __syncthreads();
    sum = 0.0f;
    for (int w = 0; w < kAttnThreads / kWave; ++w) sum += s_red[w];
    __syncthreads();
  }
  for (int j = threadIdx.x; j < nkeys; j += kAttnThreads) s_p[j] = bf16r(s_p[j] / sum);
  __syncthreads();
  // out[d] = sum_j p_j v_j[d]: thread (rr, sub) accumulates dims sub*8 .. sub*8+7 over rows
  // rr, rr + rpp, ... in order; then the rpp partial rows are summed through LDS.
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
  attn_pv(vv, 0, nkeys, rpp, rr, s_p, acc);
  for (int j0 = npass; j0 < nkeys; j0 += npass) {
#pragma unroll
    for (int u = 0; u < kAttnRowsInFlight; ++u) {
      const int j = min(j0 + u * rpp + rr, nkeys - 1);
      vv[u] = *reinterpret_cast<const uint4 *>(vbase + (size_t)j * hd);
    }
    attn_pv(vv, j0, nkeys, rpp, rr, s_p, acc);
  }
  float4 *sa = reinterpret_cast<float4 *>(s_acc + rr * hd + sub * 8);
  sa[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
  sa[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
  __syncthreads();
  for (int d = threadIdx.x; d < hd; d += kAttnThreads) {
    float o = 0.0f;
    for (int r = 0; r < rpp; ++r) o += s_acc[r * hd + d];
    out[((size_t)t * nq + h) * hd + d] = f32_to_bf16(o);
  }
}

constexpr int kGemvThreads = 256;
constexpr int kGemvWaves = kGemvThreads / kWave;
constexpr int kGemvMaxTokens = 4;
constexpr int kGemvMaxK = 8192;

// y[t][n] = bf16(sum_k W[n][k] x[t][k]), fp32 accumulation.  Each wave streams whole rows,
// 1 KB of a row per load instruction (lane l: 16 bytes at 16*l), two rows at a time; the
// activations are staged in LDS once per workgroup.
template <int T>
__global__ void __launch_bounds__(kGemvThreads)
gemv_kernel(const uint16_t *__restrict__ W, const uint16_t *__restrict__ x, int N, int K,
            uint16_t *__restrict__ y) {
  __shared__ __attribute__((aligned(16))) uint16_t s_x[T * kGemvMaxK];
  for (int i = threadIdx.x * 8; i < T * K; i += kGemvThreads * 8)
    *reinterpret_cast<uint4 *>(s_x + i) = *reinterpret_cast<const uint4 *>(x + i);
  __syncthreads();
  const int lane = threadIdx.x & (kWave - 1);
  const int gw = blockIdx.x * kGemvWaves + (threadIdx.x >> 6);
  const int nw = gridDim.x * kGemvWaves;
  const int nchunk = K / 512;  // 1 KB chunks per row
  for (int n0 = gw * 2; n0 < N; n0 += nw * 2) {
    const int n1 = n0 + 1 < N ? n0 + 1 : n0;
    float acc[2][T];
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int t = 0; t < T; ++t) acc[r][t] = 0.0f;
    const uint16_t *w0 = W + (size_t)n0 * K + lane * 8;
    const uint16_t *w1 = W + (size_t)n1 * K + lane * 8;
    for (int c = 0; c < nchunk; c += 4) {
      uint4 wv[2][4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int cc = c + u < nchunk ? c + u : nchunk - 1;
        wv[0][u] = ld_stream16(w0 + cc * 512);
        wv[1][u] = ld_stream16(w1 + cc * 512);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (c + u >= nchunk) break;
#pragma unroll
        for (int t = 0; t < T; ++t) {
          const uint4 xv = *reinterpret_cast<const uint4 *>(s_x + t * K + (c + u) * 512 + lane * 8);
          const uint32_t xa[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
          for (int r = 0; r < 2; ++r) {
            const uint32_t wa[4] = {wv[r][u].x, wv[r][u].y, wv[r][u].z, wv[r][u].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              acc[r][t] = fmaf(bf16lo_to_f32(wa[e]), bf16lo_to_f32(xa[e]), acc[r][t]);
              acc[r][t] = fmaf(bf16hi_to_f32(wa[e]), bf16hi_to_f32(xa[e]), acc[r][t]);
            }
          }
        }
      }
    }
    float sums[2 * T];
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int t = 0; t < T; ++t) sums[r * T + t] = acc[r][t];
    lane_groups_reduce<false>(sums, kWave);
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int t = 0; t < T; ++t)
        if (lane == 0 && (r == 0 || n1 != n0)) y[(size_t)t * N + (r ? n1 : n0)] = f32_to_bf16(sums[r * T + t]);
  }
}

constexpr int kGemv1Chunks = 8;  // 1 KB chunks of a row in flight per step (8 KB)

__device__ __forceinline__ void gemv1_acc(const uint4 a, const uint4 b, const uint4 xv, float &acc0,
                                          float &acc1) {
  const uint32_t xa[4] = {xv.x, xv.y, xv.z, xv.w};
  const uint32_t wa[4] = {a.x, a.y, a.z, a.w};
  const uint32_t wb[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    acc0 = fmaf(bf16lo_to_f32(wa[e]), bf16lo_to_f32(xa[e]), acc0);
    acc0 = fmaf(bf16hi_to_f32(wa[e]), bf16hi_to_f32(xa[e]), acc0);
    acc1 = fmaf(bf16lo_to_f32(wb[e]), bf16lo_to_f32(xa[e]), acc1);
    acc1 = fmaf(bf16hi_to_f32(wb[e]), bf16hi_to_f32(xa[e]), acc1);
  }
}

// Chunks c .. c + 7 of a row (lane slice w = row + lane * 8); chunks past the row's end
// repeat its last chunk (in bounds) and are masked out by gemv1_dot8.
__device__ __forceinline__ void gemv1_load8(uint4 (&a)[kGemv1Chunks], const uint16_t *w, int c,
                                            int nchunk) {
#pragma unroll
  for (int u = 0; u < kGemv1Chunks; ++u) {
    const int cc = c + u < nchunk ? c + u : nchunk - 1;
    a[u] = ld_stream16(w + cc * 512);
  }
}

// acc += chunks c .. c + 7 (those < nchunk) of two rows against the x slices xl + chunk*512.
// The mask is a select, not a branch, so the loads before it stay where they are issued.
__device__ __forceinline__ void gemv1_dot8(const uint4 (&a)[kGemv1Chunks], const uint4 (&b)[kGemv1Chunks],
                                           const uint16_t *xl, int c, int nchunk, float &acc0,
                                           float &acc1) {
#pragma unroll
  for (int u = 0; u < kGemv1Chunks; ++u) {
    const int cc = c + u < nchunk ? c + u : nchunk - 1;
    const uint4 xv = *reinterpret_cast<const uint4 *>(xl + cc * 512);
    float t0 = acc0, t1 = acc1;
    gemv1_acc(a[u], b[u], xv, t0, t1);
    const bool ok = c + u < nchunk;
    acc0 = ok ? t0 : acc0;
    acc1 = ok ? t1 : acc1;
  }
}

// One token's rows n0 and n1 of W x: the whole row pair in steps of 8 KB per row, the
// first step optionally already loaded into a / b.
__device__ __forceinline__ void gemv1_pair(const uint16_t *w0, const uint16_t *w1, const uint16_t *xl,
                                           int nchunk, uint4 (&a)[kGemv1Chunks],
                                           uint4 (&b)[kGemv1Chunks], bool loaded, float &acc0,
                                           float &acc1) {
  acc0 = 0.0f;
  acc1 = 0.0f;
  for (int c = 0; c < nchunk; c += kGemv1Chunks) {
    if (c > 0 || !loaded) {
      gemv1_load8(a, w0, c, nchunk);
      gemv1_load8(b, w1, c, nchunk);
    }
    gemv1_dot8(a, b, xl, c, nchunk, acc0, acc1);
  }
}

// y = W x for one token, rows in pairs (n, n + 1) per wave, x read from xl's slices.
__device__ __forceinline__ void gemv1_rows(const uint16_t *W, const uint16_t *xl, int N, int K,
                                           int nblocks, uint16_t *y) {
  const int lane = threadIdx.x & (kWave - 1);
  const int gw = blockIdx.x * kGemvWaves + (threadIdx.x >> 6);
  const int nw = nblocks * kGemvWaves;
  const int nchunk = K / 512;
  uint4 a[kGemv1Chunks], b[kGemv1Chunks];
  for (int n0 = gw * 2; n0 < N; n0 += nw * 2) {
    const int n1 = n0 + 1 < N ? n0 + 1 : n0;
    float acc0, acc1;
    gemv1_pair(W + (size_t)n0 * K + lane * 8, W + (size_t)n1 * K + lane * 8, xl, nchunk, a, b, false,
               acc0, acc1);
    wave_sum_pair(acc0, acc1);
    if (lane == 0) {
      y[n0] = f32_to_bf16(acc0);
      if (n1 != n0) y[n1] = f32_to_bf16(acc1);
    }
  }
}

// T = 1: no LDS staging.  Each wave takes two rows at a time and issues the 1 KB chunks of
// both rows (8 KB each per step) with the matching 16-byte slices of x (L2-resident after
// the first waves) before it accumulates, so a wave has 16 weight loads in flight and no
// workgroup barrier.  Per-lane accumulation order is that of the LDS-staged kernel.
__global__ void __launch_bounds__(kGemvThreads)
gemv1_kernel(const uint16_t *__restrict__ W, const uint16_t *__restrict__ x, int N, int K,
             uint16_t *__restrict__ y) {
  int nblocks = gridDim.x;
  MOE_ARGS_FIRST(MOE_LIST("+s"(N), "+s"(K), "+s"(nblocks)), MOE_LIST("s"(W), "s"(x), "s"(y)));
  gemv1_rows(W, x + (threadIdx.x & (kWave - 1)) * 8, N, K, nblocks, y);
}

// ---------------------------------------------------------------- fused decode-step kernels
// One token.  Each removes a launch (about 4-5 us of dependent latency at batch 1) by doing
// a neighbouring step inside the projection kernel, with the same arithmetic and summation
// order as the separate kernels, so the results are bit-identical to them.  No kernel here
// waits for another workgroup: device-scope fences cost more than a launch on this part.
constexpr int kFusedMaxH = 8192;  // norm chunks per thread: up to 4
static_assert(kNormThreads == kGemvThreads, "the fused kernels run the norm and the GEMV in one workgroup");

// qkv_rope: r = x[row] (+ residual) -> residual_out (workgroup 0), xn = rmsnorm(r) in every
// workgroup's LDS, then the q/k/v projection with rows paired (i, i + hd/2) within a head,
// so the wave holding both outputs applies the rotary embedding (cos/sin of position pos0
// rounded to bf16) and writes q to q_out and k, v to the cache row pos0.  The first row
// pair's first 8 KB per row are in flight before the norm.
template <bool RES, int CH>
__global__ void __launch_bounds__(kNormThreads)
qkv_rope_kernel(const uint16_t *__restrict__ W, const uint16_t *__restrict__ x,
                const int64_t *__restrict__ x_row, int64_t x_rows, const uint16_t *__restrict__ res,
                const uint16_t *__restrict__ nw, float eps, int H, int nq, int nkv, int hd,
                const float *__restrict__ inv_freq, const int32_t *__restrict__ pos0, int64_t max_seq,
                uint16_t *__restrict__ res_out, uint16_t *__restrict__ q_out, uint16_t *__restrict__ kc,
                uint16_t *__restrict__ vc) {
  __shared__ __attribute__((aligned(16))) uint16_t s_x[kFusedMaxH];
  __shared__ float s_part[kNormThreads / kWave];
  int nblocks = gridDim.x;
  MOE_ARGS_FIRST(MOE_LIST("+s"(x_rows), "+s"(eps), "+s"(H), "+s"(nq), "+s"(nkv), "+s"(hd), "+s"(max_seq),
                          "+s"(nblocks)),
                 MOE_LIST("s"(W), "s"(x), "s"(x_row), "s"(res), "s"(nw), "s"(inv_freq), "s"(pos0),
                      "s"(res_out), "s"(q_out), "s"(kc), "s"(vc)));
  const int lane = threadIdx.x & (kWave - 1);
  const int gw = blockIdx.x * kGemvWaves + (threadIdx.x >> 6);
  const int nwv = nblocks * kGemvWaves;
  const int half = hd >> 1;
  const int pairs = (nq + 2 * nkv) * half;
  const int nchunk = H / 512;
  auto rows_of = [&](int p, const uint16_t *&w0, const uint16_t *&w1) {
    const int head = p / half, i = p - head * half;
    w0 = W + (size_t)(head * hd + i) * H + lane * 8;
    w1 = w0 + (size_t)half * H;
  };
  // The norm's loads (L2-resident, needed first) are issued before the first weight step,
  // so that waiting for them does not wait for the weights.
  int64_t row = x_row != nullptr ? *x_row : 0;
  row = row < 0 ? 0 : (row >= x_rows ? x_rows - 1 : row);  // ids outside the table clamp
  NormRegs<CH> g;
  norm_load<CH, RES>(g, x + (size_t)row * H, res, nw, H);
  // Unconditional (a wave past the last pair loads the last pair's rows and drops them): a
  // conditional load here would make every later wait count it as possibly not issued,
  // i.e. wait for the weights too.
  uint4 a[kGemv1Chunks], b[kGemv1Chunks];
  const uint16_t *w0 = W, *w1 = W;
  rows_of(gw < pairs ? gw : pairs - 1, w0, w1);
  gemv1_load8(a, w0, 0, nchunk);
  gemv1_load8(b, w1, 0, nchunk);
  __builtin_amdgcn_sched_barrier(0);  // keep the weight loads ahead of the norm arithmetic
  norm_finish<CH, RES>(g, eps, H, blockIdx.x == 0 ? res_out : nullptr, s_x, s_part);
  lds_barrier();
  const int pos = *pos0;
  const bool pos_ok = pos >= 0 && pos < max_seq;  // else the cache has no row (caller error)
  for (int p = gw; p < pairs; p += nwv) {
    const bool loaded = p == gw;
    if (!loaded) rows_of(p, w0, w1);
    float acc0, acc1;
    gemv1_pair(w0, w1, s_x + lane * 8, nchunk, a, b, loaded, acc0, acc1);
    wave_sum_pair(acc0, acc1);
    if (lane == 0) {
      const int head = p / half, i = p - head * half;
      const float y1 = bf16r(acc0), y2 = bf16r(acc1);
      float o1 = y1, o2 = y2;
      if (head < nq + nkv) {
        const float ang = (float)pos * inv_freq[i];
        const float co = bf16r(cosf(ang)), si = bf16r(sinf(ang));
        o1 = bf16r(y1 * co) + bf16r(-y2 * si);
        o2 = bf16r(y2 * co) + bf16r(y1 * si);
      }
      uint16_t *dst = nullptr;
      if (head < nq)
        dst = q_out + (size_t)head * hd;
      else if (pos_ok)
        dst = head < nq + nkv ? kc + ((size_t)(head - nq) * max_seq + pos) * hd
                              : vc + ((size_t)(head - nq - nkv) * max_seq + pos) * hd;
      if (dst != nullptr) {
        dst[i] = f32_to_bf16(o1);
        dst[i + half] = f32_to_bf16(o2);
      }
    }
  }
}

// (value, index) order of torch.argmax: NaN above every number (the first NaN wins), then
// the larger value, then the lower index.
__device__ __forceinline__ bool argmax_better(float v, int i, float bv, int bi) {
  const bool nv = v != v, nb = bv != bv;
  if (nv != nb) return nv;
  if (nv || v == bv) return i < bi;
  return v > bv;
}

__device__ __forceinline__ void argmax_wave(float &v, int &i) {
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(v, o, kWave);
    const int oi = __shfl_xor(i, o, kWave);
    if (argmax_better(ov, oi, v, i)) {
      v = ov;
      i = oi;
    }
  }
}

// head_logits: r = x + residual, xn = rmsnorm(r) per workgroup (the final norm), logits =
// W xn (bf16, rows (n, n + 1) per wave), and each workgroup's best (value, index) to cand.
template <bool RES, int CH>
__global__ void __launch_bounds__(kNormThreads)
head_logits_kernel(const uint16_t *__restrict__ W, const uint16_t *__restrict__ x,
                   const uint16_t *__restrict__ res, const uint16_t *__restrict__ nw, float eps, int N,
                   int K, uint16_t *__restrict__ logits, float *__restrict__ cand_v,
                   int32_t *__restrict__ cand_i) {
  __shared__ __attribute__((aligned(16))) uint16_t s_x[kFusedMaxH];
  __shared__ float s_part[kNormThreads / kWave];
  __shared__ float s_bv[kGemvWaves];
  __shared__ int s_bi[kGemvWaves];
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x >> 6;
  const int gw = blockIdx.x * kGemvWaves + wave;
  const int nwv = gridDim.x * kGemvWaves;
  const int nchunk = K / 512;
  NormRegs<CH> g;
  norm_load<CH, RES>(g, x, res, nw, K);
  uint4 a[kGemv1Chunks], b[kGemv1Chunks];
  const int f0 = gw * 2;
  {  // unconditional, as in qkv_rope_kernel (rows clamped to the last one)
    const int p0 = f0 < N ? f0 : N - 1;
    const int p1 = p0 + 1 < N ? p0 + 1 : p0;
    gemv1_load8(a, W + (size_t)p0 * K + lane * 8, 0, nchunk);
    gemv1_load8(b, W + (size_t)p1 * K + lane * 8, 0, nchunk);
  }
  __builtin_amdgcn_sched_barrier(0);  // keep the weight loads ahead of the norm arithmetic
  norm_finish<CH, RES>(g, eps, K, nullptr, s_x, s_part);
  lds_barrier();
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int n0 = f0; n0 < N; n0 += nwv * 2) {
    const int n1 = n0 + 1 < N ? n0 + 1 : n0;
    float acc0, acc1;
    gemv1_pair(W + (size_t)n0 * K + lane * 8, W + (size_t)n1 * K + lane * 8, s_x + lane * 8, nchunk,
               a, b, n0 == f0, acc0, acc1);
    wave_sum_pair(acc0, acc1);
    const float y0 = bf16r(acc0), y1 = bf16r(acc1);
    if (argmax_better(y0, n0, bv, bi)) {
      bv = y0;
      bi = n0;
    }
    if (n1 != n0 && argmax_better(y1, n1, bv, bi)) {
      bv = y1;
      bi = n1;
    }
    if (lane == 0) {
      logits[n0] = f32_to_bf16(acc0);
      if (n1 != n0) logits[n1] = f32_to_bf16(acc1);
    }
  }
  if (lane == 0) {
    s_bv[wave] = bv;
    s_bi[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kGemvWaves; ++w)
      if (argmax_better(s_bv[w], s_bi[w], bv, bi)) {
        bv = s_bv[w];
        bi = s_bi[w];
      }
    cand_v[blockIdx.x] = bv;
    cand_i[blockIdx.x] = bi;
  }
}

// One workgroup: the best of the n candidates is the token; when given,
// gen[*gen_ctr] = token (if the index is in [0, gen_cap)), *gen_ctr += 1, *pos += 1.
// (A second launch is cheaper here than a device-scope fence per workgroup of the head.)
__global__ void __launch_bounds__(kNormThreads)
argmax_finish_kernel(const float *__restrict__ cand_v, const int32_t *__restrict__ cand_i, int n,
                     int64_t *__restrict__ token, int64_t *__restrict__ gen, int64_t gen_cap,
                     int64_t *__restrict__ gen_ctr, int32_t *__restrict__ pos) {
  __shared__ float s_bv[kGemvWaves];
  __shared__ int s_bi[kGemvWaves];
  MOE_ARGS_FIRST(MOE_LIST("+s"(n), "+s"(gen_cap)),
                 MOE_LIST("s"(cand_v), "s"(cand_i), "s"(token), "s"(gen), "s"(gen_ctr), "s"(pos)));
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x >> 6;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int g = threadIdx.x; g < n; g += kNormThreads)
    if (argmax_better(cand_v[g], cand_i[g], bv, bi)) {
      bv = cand_v[g];
      bi = cand_i[g];
    }
  argmax_wave(bv, bi);
  if (lane == 0) {
    s_bv[wave] = bv;
    s_bi[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kGemvWaves; ++w)
      if (argmax_better(s_bv[w], s_bi[w], bv, bi)) {
        bv = s_bv[w];
        bi = s_bi[w];
      }
    *token = bi;
    if (gen_ctr != nullptr) {
      const int64_t c = *gen_ctr;
      if (gen != nullptr && c >= 0 && c < gen_cap) gen[c] = bi;
      *gen_ctr = c + 1;
    }
    if (pos != nullptr) *pos += 1;
  }
}

}  // namespace
}  // namespace moe

extern "C" int moe_add_rmsnorm_bf16(const void *x, const void *residual_in, const void *weight,
                                    float eps, int64_t T, int32_t H, void *residual_out,
                                    void *out, void *stream) {
  MOE_REQUIRE(T >= 0 && H > 0 && H % 8 == 0 && H <= moe::kNormThreads * moe::kNormMaxChunks * 8,
              "hidden size must be a positive multiple of 8 up to %d (got %d)",
              moe::kNormThreads * moe::kNormMaxChunks * 8, H);
  if (T == 0) return MOE_STATUS_OK;
  MOE_REQUIRE(x && weight && out, "null pointer");
  MOE_REQUIRE(((uintptr_t)x | (uintptr_t)weight | (uintptr_t)out | (uintptr_t)residual_in |
               (uintptr_t)residual_out) % 16 == 0,
              "tensors must be 16-byte aligned");
  // Chunks per thread: the smallest power of two with 256 threads x 8 values x CH >= H.
  const int chunks = (H + moe::kNormThreads * 8 - 1) / (moe::kNormThreads * 8);
  const bool r = residual_in != nullptr;
  auto kern = chunks <= 1 ? (r ? moe::add_rmsnorm_kernel<1, true> : moe::add_rmsnorm_kernel<1, false>)
            : chunks <= 2 ? (r ? moe::add_rmsnorm_kernel<2, true> : moe::add_rmsnorm_kernel<2, false>)
            : chunks <= 4 ? (r ? moe::add_rmsnorm_kernel<4, true> : moe::add_rmsnorm_kernel<4, false>)
                          : (r ? moe::add_rmsnorm_kernel<8, true> : moe::add_rmsnorm_kernel<8, false>);
  hipLaunchKernelGGL(kern, dim3((unsigned)T), dim3(moe::kNormThreads), 0, (hipStream_t)stream,
                     (const uint16_t *)x, (const uint16_t *)residual_in, (const uint16_t *)weight,
                     eps, H, (uint16_t *)residual_out, (uint16_t *)out);
  MOE_LAUNCH_CHECK();
  return MOE_STATUS_OK;
}

extern "C" int moe_rope_kv_bf16(const void *qkv, int64_t T, int32_t n_q_heads, int32_t n_kv_heads,
                                int32_t head_dim, const void *inv_freq_f32, const void *pos0_i32,
                                int64_t max_seq, void *q_out, void *k_cache, void *v_cache,
                                void *stream) {
  MOE_REQUIRE(T >= 0 && n_q_heads > 0 && n_kv_heads > 0 && max_seq > 0, "bad sizes");
  MOE_REQUIRE(head_dim > 0 && head_dim % 16 == 0 && head_dim / 2 <= moe::kRopeMaxHalf,
              "head dim must be a multiple of 16 up to %d (got %d)", 2 * moe::kRopeMaxHalf, head_dim);
  if (T == 0) return MOE_STATUS_OK;
  MOE_REQUIRE(qkv && inv_freq_f32 && pos0_i32 && q_out && k_cache && v_cache, "null pointer");
  MOE_REQUIRE(((uintptr_t)qkv | (uintptr_t)q_out | (uintptr_t)k_cache | (uintptr_t)v_cache) % 16 == 0,
              "q/k/v and cache tensors must be 16-byte aligned");
  hipLaunchKernelGGL(moe::rope_kv_kernel, dim3((unsigned)T), dim3(moe::kRopeThreads), 0,
                     (hipStream_t)stream, (const uint16_t *)qkv, n_q_heads, n_kv_heads, head_dim,
                     (const float *)inv_freq_f32, (const int32_t *)pos0_i32, max_seq,
                     (uint16_t *)q_out, (uint16_t *)k_cache, (uint16_t *)v_cache);
  MOE_LAUNCH_CHECK();
  return MOE_STATUS_OK;
}

extern "C" int moe_attention_bf16(const void *q, const void *k_cache, const void *v_cache, int64_t T,
                                  int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                                  const void *pos0_i32, int64_t max_seq, float scaling, void *out,
                                  void *stream) {
  MOE_REQUIRE(T >= 0 && n_q_heads > 0 && n_kv_heads > 0 && n_q_heads % n_kv_heads == 0,
              "query heads must be a multiple of the KV heads");
  MOE_REQUIRE(head_dim > 0 && head_dim <= moe::kAttnMaxHeadDim && moe::kAttnThreads % head_dim == 0 &&
                  head_dim % 8 == 0,
              "head dim must divide %d and be a multiple of 8 (got %d)", moe::kAttnThreads, head_dim);
  MOE_REQUIRE(max_seq > 0 && max_seq <= moe::kAttnMaxKeys, "max_seq must be in [1, %d]",
              moe::kAttnMaxKeys);
  if (T == 0) return MOE_STATUS_OK;
  MOE_REQUIRE(q && k_cache && v_cache && pos0_i32 && out, "null pointer");
  MOE_REQUIRE(((uintptr_t)q | (uintptr_t)k_cache | (uintptr_t)v_cache) % 16 == 0,
              "q and the KV cache must be 16-byte aligned");
  hipLaunchKernelGGL(moe::attention_kernel, dim3((unsigned)n_q_heads, (unsigned)T),
                     dim3(moe::kAttnThreads), 0, (hipStream_t)stream, (const uint16_t *)q,
                     (const uint16_t *)k_cache, (const uint16_t *)v_cache, n_q_heads, n_kv_heads,
                     head_dim, (const int32_t *)pos0_i32, max_seq, scaling, (uint16_t *)out);
  MOE_LAUNCH_CHECK();
  return MOE_STATUS_OK;
}

extern "C" int moe_gemv_bf16(const void *weight, const void *x, int64_t T, int32_t N, int32_t K,
                             void *y, void *stream) {
  MOE_REQUIRE(T >= 1 && T <= moe::kGemvMaxTokens, "gemv takes 1 to %d tokens (got %lld)",
              moe::kGemvMaxTokens, (long long)T);
  MOE_REQUIRE(N > 0 && K > 0 && K % 512 == 0 && K <= moe::kGemvMaxK,
              "K must be a positive multiple of 512 up to %d (got %d)", moe::kGemvMaxK, K);
  MOE_REQUIRE(weight && x && y, "null pointer");
  MOE_REQUIRE(((uintptr_t)weight | (uintptr_t)x) % 16 == 0, "weight and x must be 16-byte aligned");
  const int waves = (N + 1) / 2;
  int grid = (waves + moe::kGemvWaves - 1) / moe::kGemvWaves;
  const int cap = moe::device_cu_count() * 4;
  if (grid > cap) grid = cap;
  hipStream_t s = (hipStream_t)stream;
  const uint16_t *w = (const uint16_t *)weight, *xx = (const uint16_t *)x;
  uint16_t *yy = (uint16_t *)y;
  switch (T) {
    case 1: hipLaunchKernelGGL(moe::gemv1_kernel, dim3(grid), dim3(moe::kGemvThreads), 0, s, w, xx, N, K, yy); break;
    case 2: hipLaunchKernelGGL(moe::gemv_kernel<2>, dim3(grid), dim3(moe::kGemvThreads), 0, s, w, xx, N, K, yy); break;
    case 3: hipLaunchKernelGGL(moe::gemv_kernel<3>, dim3(grid), dim3(moe::kGemvThreads), 0, s, w, xx, N, K, yy); break;
    default: hipLaunchKernelGGL(moe::gemv_kernel<4>, dim3(grid), dim3(moe::kGemvThreads), 0, s, w, xx, N, K, yy); break;
  }
  MOE_LAUNCH_CHECK();
  return MOE_STATUS_OK;
}

namespace {
int gemv1_grid(int64_t waves) {
  int64_t grid = (waves + moe::kGemvWaves - 1) / moe::kGemvWaves;
  const int64_t cap = (int64_t)moe::device_cu_count() * 4;
  return (int)(grid > cap ? cap : grid);
}
}  // namespace

extern "C" int moe_qkv_rope_bf16(const void *weight, const void *x, const void *x_row_i64,
                                 int64_t x_rows, const void *residual, const void *norm_weight,
                                 float eps, int32_t H, int32_t n_q_heads, int32_t n_kv_heads,
                                 int32_t head_dim, const void *inv_freq_f32, const void *pos0_i32,
                                 int64_t max_seq, void *residual_out, void *q_out, void *k_cache,
                                 void *v_cache, void *stream) {
  MOE_REQUIRE(H > 0 && H % 512 == 0 && H <= moe::kFusedMaxH,
              "hidden size must be a positive multiple of 512 up to %d (got %d)", moe::kFusedMaxH, H);
  MOE_REQUIRE(n_q_heads > 0 && n_kv_heads > 0 && head_dim > 0 && head_dim % 2 == 0 && max_seq > 0 &&
                  x_rows > 0,
              "bad sizes");
  MOE_REQUIRE(weight && x && norm_weight && inv_freq_f32 && pos0_i32 && q_out && k_cache && v_cache,
              "null pointer");
  // Workgroup 0 writes residual_out while the others still read x, residual, the norm
  // weight and the projection weight.
  const int64_t hb = 2 * (int64_t)H;
  const int64_t wrows = (int64_t)(n_q_heads + 2 * n_kv_heads) * head_dim;
  MOE_REQUIRE(!moe::ranges_overlap(residual_out, hb, x, hb * x_rows) &&
                  !moe::ranges_overlap(residual_out, hb, residual, hb) &&
                  !moe::ranges_overlap(residual_out, hb, norm_weight, hb) &&
                  !moe::ranges_overlap(residual_out, hb, weight, hb * wrows),
              "residual_out must not overlap x, residual, norm_weight or the weight");
  MOE_REQUIRE(((uintptr_t)weight | (uintptr_t)x | (uintptr_t)residual | (uintptr_t)norm_weight |
               (uintptr_t)residual_out) % 16 == 0,
              "weight, x, residual and norm tensors must be 16-byte aligned");
  const int64_t pairs = (int64_t)(n_q_heads + 2 * n_kv_heads) * (head_dim / 2);
  // Norm chunks per thread: 2 for H <= 4096, else 4.
  const bool small = H <= moe::kNormThreads * 8 * 2;
  auto kern = residual ? (small ? moe::qkv_rope_kernel<true, 2> : moe::qkv_rope_kernel<true, 4>)
                       : (small ? moe::qkv_rope_kernel<false, 2> : moe::qkv_rope_kernel<false, 4>);
  hipLaunchKernelGGL(kern, dim3((unsigned)gemv1_grid(pairs)), dim3(moe::kNormThreads),
                     0, (hipStream_t)stream, (const uint16_t *)weight, (const uint16_t *)x,
                     (const int64_t *)x_row_i64, x_rows, (const uint16_t *)residual,
                     (const uint16_t *)norm_weight, eps, H, n_q_heads, n_kv_heads, head_dim,
                     (const float *)inv_freq_f32, (const int32_t *)pos0_i32, max_seq,
                     (uint16_t *)residual_out, (uint16_t *)q_out, (uint16_t *)k_cache,
                     (uint16_t *)v_cache);
  MOE_LAUNCH_CHECK();
  return MOE_STATUS_OK;
}

extern "C" int moe_head_argmax_bf16(const void *weight, const void *x, const void *residual,
                                    const void *norm_weight, float eps, int32_t N, int32_t K,
                                    void *logits, void *cand_ws, int64_t cand_ws_bytes,
                                    void *token_i64, void *gen_i64, int64_t gen_cap,
                                    void *gen_ctr_i64, void *pos_i32, void *stream) {
  MOE_REQUIRE(K > 0 && K % 512 == 0 && K <= moe::kFusedMaxH,
              "K must be a positive multiple of 512 up to %d (got %d)", moe::kFusedMaxH, K);
  MOE_REQUIRE(N > 0, "N must be positive");
  MOE_REQUIRE(weight && x && norm_weight && logits && cand_ws && token_i64, "null pointer");
  MOE_REQUIRE(cand_ws_bytes >= 8, "candidate workspace must hold at least one entry (8 bytes)");
  MOE_REQUIRE(((uintptr_t)weight | (uintptr_t)x | (uintptr_t)residual | (uintptr_t)norm_weight) % 16 == 0,
              "weight, x, residual and norm tensors must be 16-byte aligned");
  MOE_REQUIRE((uintptr_t)cand_ws % 4 == 0, "candidate workspace must be 4-byte aligned");
  int grid = gemv1_grid((N + 1) / 2);
  if (grid > cand_ws_bytes / 8) grid = (int)(cand_ws_bytes / 8);
  float *cand_v = (float *)cand_ws;
  int32_t *cand_i = (int32_t *)((char *)cand_ws + (size_t)grid * 4);
  hipStream_t s = (hipStream_t)stream;
  const bool small = K <= moe::kNormThreads * 8 * 2;
  auto kern = residual ? (small ? moe::head_logits_kernel<true, 2> : moe::head_logits_kernel<true, 4>)
                       : (small ? moe::head_logits_kernel<false, 2> : moe::head_logits_kernel<false, 4>);
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(moe::kNormThreads), 0, s,
                     (const uint16_t *)weight, (const uint16_t *)x, (const uint16_t *)residual,
                     (const uint16_t *)norm_weight, eps, N, K, (uint16_t *)logits, cand_v, cand_i);
  MOE_LAUNCH_CHECK();
  hipLaunchKernelGGL(moe::argmax_finish_kernel, dim3(1), dim3(moe::kNormThreads), 0, s, cand_v,
                     cand_i, grid, (int64_t *)token_i64, (int64_t *)gen_i64, gen_cap,
                     (int64_t *)gen_ctr_i64, (int32_t *)pos_i32);
  MOE_LAUNCH_CHECK();
  return MOE_STATUS_OK;
}
