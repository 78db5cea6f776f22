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
#include "common.h"

namespace moe {
namespace {

constexpr int kNormThreads = 256;
constexpr int kNormMaxChunks = 8;  // 8-value chunks per thread: H <= 16384

__device__ __forceinline__ float bf16r(float v) { return bf16_to_f32(f32_to_bf16(v)); }

__device__ __forceinline__ float block_sum(float v, float *s_part) {
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x >> 6;
  v = wave_sum(v);
  if (lane == 0) s_part[wave] = v;
  __syncthreads();
  float t = 0.0f;
  for (int w = 0; w < (int)(blockDim.x >> 6); ++w) t += s_part[w];
  __syncthreads();
  return t;
}

__global__ void __launch_bounds__(kNormThreads)
add_rmsnorm_kernel(const uint16_t *__restrict__ x, const uint16_t *__restrict__ res_in,
                   const uint16_t *__restrict__ w, float eps, int H,
                   uint16_t *__restrict__ res_out, uint16_t *__restrict__ out) {
  __shared__ float s_part[kNormThreads / kWave];
  const size_t base = (size_t)blockIdx.x * H;
  uint4 rv[kNormMaxChunks];
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < kNormMaxChunks; ++i) {
    const int c = (threadIdx.x + i * kNormThreads) * 8;
    if (c < H) {
      uint4 v = *reinterpret_cast<const uint4 *>(x + base + c);
      if (res_in != nullptr) {
        const uint4 r = *reinterpret_cast<const uint4 *>(res_in + base + c);
        const uint32_t a[4] = {v.x, v.y, v.z, v.w}, b[4] = {r.x, r.y, r.z, r.w};
        uint32_t o[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          o[j] = pack_bf16x2(bf16lo_to_f32(a[j]) + bf16lo_to_f32(b[j]),
                             bf16hi_to_f32(a[j]) + bf16hi_to_f32(b[j]));
        v = make_uint4(o[0], o[1], o[2], o[3]);
        if (res_out != nullptr) *reinterpret_cast<uint4 *>(res_out + base + c) = v;
      }
      rv[i] = v;
      const uint32_t a[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float lo = bf16lo_to_f32(a[j]), hi = bf16hi_to_f32(a[j]);
        ss += lo * lo + hi * hi;
      }
    }
  }
  const float inv = 1.0f / sqrtf(block_sum(ss, s_part) / (float)H + eps);
#pragma unroll
  for (int i = 0; i < kNormMaxChunks; ++i) {
    const int c = (threadIdx.x + i * kNormThreads) * 8;
    if (c < H) {
      const uint4 wv = *reinterpret_cast<const uint4 *>(w + c);
      const uint32_t a[4] = {rv[i].x, rv[i].y, rv[i].z, rv[i].w}, g[4] = {wv.x, wv.y, wv.z, wv.w};
      uint32_t o[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        o[j] = pack_bf16x2(bf16lo_to_f32(g[j]) * bf16r(bf16lo_to_f32(a[j]) * inv),
                           bf16hi_to_f32(g[j]) * bf16r(bf16hi_to_f32(a[j]) * inv));
      *reinterpret_cast<uint4 *>(out + base + c) = make_uint4(o[0], o[1], o[2], o[3]);
    }
  }
}

constexpr int kRopeThreads = 256;

// Token t (blockIdx.x) at position pos0 + t: q heads and k heads rotated pairwise (value i
// with i + hd/2), q to q_out [T, nq, hd], k and v to the cache rows [kv head][pos][hd].
__global__ void __launch_bounds__(kRopeThreads)
rope_kv_kernel(const uint16_t *__restrict__ qkv, int nq, int nkv, int hd,
               const float *__restrict__ inv_freq, const int32_t *__restrict__ pos0,
               int64_t max_seq, uint16_t *__restrict__ q_out, uint16_t *__restrict__ kc,
               uint16_t *__restrict__ vc) {
  const int t = blockIdx.x;
  const int pos = *pos0 + t;
  if (pos < 0 || pos >= max_seq) return;  // the cache has no row for it (caller error)
  const int half = hd >> 1;
  const int row = (nq + 2 * nkv) * hd;
  const uint16_t *src = qkv + (size_t)t * row;
  for (int idx = threadIdx.x; idx < (nq + nkv) * half; idx += kRopeThreads) {
    const int head = idx / half, i = idx - head * half;
    const uint16_t *hx = src + (size_t)head * hd;  // k heads follow the q heads
    const float x1 = bf16_to_f32(hx[i]), x2 = bf16_to_f32(hx[i + half]);
    const float ang = (float)pos * inv_freq[i];
    const float c = bf16r(cosf(ang)), s = bf16r(sinf(ang));
    const uint16_t o1 = f32_to_bf16(bf16r(x1 * c) + bf16r(-x2 * s));
    const uint16_t o2 = f32_to_bf16(bf16r(x2 * c) + bf16r(x1 * s));
    uint16_t *dst;
    if (head < nq)
      dst = q_out + ((size_t)t * nq + head) * hd;
    else
      dst = kc + ((size_t)(head - nq) * max_seq + pos) * hd;
    dst[i] = o1;
    dst[i + half] = o2;
  }
  const uint16_t *vsrc = src + (size_t)(nq + nkv) * hd;
  for (int idx = threadIdx.x; idx < nkv * hd; idx += kRopeThreads) {
    const int head = idx / hd, d = idx - head * hd;
    vc[((size_t)head * max_seq + pos) * hd + d] = vsrc[idx];
  }
}

constexpr int kAttnThreads = 256;
constexpr int kAttnMaxKeys = 8192;
constexpr int kAttnMaxHeadDim = 256;

// One workgroup per (query head, token): scores of keys 0 .. pos0 + t (causal), bf16 scores
// scaled in bf16, fp32 softmax rounded to bf16, then the bf16 probabilities times V with
// fp32 accumulation.
__global__ void __launch_bounds__(kAttnThreads)
attention_kernel(const uint16_t *__restrict__ q, const uint16_t *__restrict__ kc,
                 const uint16_t *__restrict__ vc, int nq, int nkv, int hd,
                 const int32_t *__restrict__ pos0, int64_t max_seq, float scaling,
                 uint16_t *__restrict__ out) {
  __shared__ float s_q[kAttnMaxHeadDim];
  __shared__ float s_p[kAttnMaxKeys];
  __shared__ float s_red[kAttnThreads / kWave];
  __shared__ float s_acc[kAttnThreads];
  const int h = blockIdx.x, t = blockIdx.y;
  const int kvh = h / (nq / nkv);
  // Keys 0 .. pos0 + t, bounded by the cache (a position past it is a caller error).
  const int nkeys = min(*pos0 + t + 1, (int)max_seq);
  const uint16_t *qr = q + ((size_t)t * nq + h) * hd;
  for (int d = threadIdx.x; d < hd; d += kAttnThreads) s_q[d] = bf16_to_f32(qr[d]);
  __syncthreads();
  const uint16_t *kbase = kc + (size_t)kvh * max_seq * hd;
  const uint16_t *vbase = vc + (size_t)kvh * max_seq * hd;
  float mx = -INFINITY;
  for (int j = threadIdx.x; j < nkeys; j += kAttnThreads) {
    const uint4 *kr = reinterpret_cast<const uint4 *>(kbase + (size_t)j * hd);
    float dot = 0.0f;
    for (int c = 0; c < hd / 8; ++c) {
      const uint4 kv = kr[c];
      const uint32_t a[4] = {kv.x, kv.y, kv.z, kv.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        dot = fmaf(s_q[8 * c + 2 * e], bf16lo_to_f32(a[e]), dot);
        dot = fmaf(s_q[8 * c + 2 * e + 1], bf16hi_to_f32(a[e]), dot);
      }
    }
    const float sc = bf16r(bf16r(dot) * scaling);
    s_p[j] = sc;
    mx = fmaxf(mx, sc);
  }
  // block max
  {
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x >> 6;
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, kWave));
    if (lane == 0) s_red[wave] = mx;
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
  sum = block_sum(sum, s_red);
  for (int j = threadIdx.x; j < nkeys; j += kAttnThreads) s_p[j] = bf16r(s_p[j] / sum);
  __syncthreads();
  // out[d] = sum_j p_j v_j[d]: thread (part, d) sums keys part, part + parts, ...
  const int parts = kAttnThreads / hd;  // hd divides kAttnThreads
  const int d = threadIdx.x % hd, part = threadIdx.x / hd;
  float acc = 0.0f;
  for (int j = part; j < nkeys; j += parts) acc = fmaf(s_p[j], bf16_to_f32(vbase[(size_t)j * hd + d]), acc);
  s_acc[threadIdx.x] = acc;
  __syncthreads();
  if (part == 0) {
    for (int p = 1; p < parts; ++p) acc += s_acc[p * hd + d];
    out[((size_t)t * nq + h) * hd + d] = f32_to_bf16(acc);
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
        wv[0][u] = *reinterpret_cast<const uint4 *>(w0 + cc * 512);
        wv[1][u] = *reinterpret_cast<const uint4 *>(w1 + cc * 512);
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
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const float v = wave_sum(acc[r][t]);
        if (lane == 0 && (r == 0 || n1 != n0)) y[(size_t)t * N + (r ? n1 : n0)] = f32_to_bf16(v);
      }
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
  hipLaunchKernelGGL(moe::add_rmsnorm_kernel, dim3((unsigned)T), dim3(moe::kNormThreads), 0,
                     (hipStream_t)stream, (const uint16_t *)x, (const uint16_t *)residual_in,
                     (const uint16_t *)weight, eps, H, (uint16_t *)residual_out, (uint16_t *)out);
  MOE_LAUNCH_CHECK();
  return MOE_STATUS_OK;
}

extern "C" int moe_rope_kv_bf16(const void *qkv, int64_t T, int32_t n_q_heads, int32_t n_kv_heads,
                                int32_t head_dim, const void *inv_freq_f32, const void *pos0_i32,
                                int64_t max_seq, void *q_out, void *k_cache, void *v_cache,
                                void *stream) {
  MOE_REQUIRE(T >= 0 && n_q_heads > 0 && n_kv_heads > 0 && head_dim > 0 && head_dim % 2 == 0 &&
                  max_seq > 0,
              "bad sizes");
  if (T == 0) return MOE_STATUS_OK;
  MOE_REQUIRE(qkv && inv_freq_f32 && pos0_i32 && q_out && k_cache && v_cache, "null pointer");
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
  MOE_REQUIRE(((uintptr_t)k_cache | (uintptr_t)v_cache) % 16 == 0, "KV cache must be 16-byte aligned");
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
    case 1: hipLaunchKernelGGL(moe::gemv_kernel<1>, dim3(grid), dim3(moe::kGemvThreads), 0, s, w, xx, N, K, yy); break;
    case 2: hipLaunchKernelGGL(moe::gemv_kernel<2>, dim3(grid), dim3(moe::kGemvThreads), 0, s, w, xx, N, K, yy); break;
    case 3: hipLaunchKernelGGL(moe::gemv_kernel<3>, dim3(grid), dim3(moe::kGemvThreads), 0, s, w, xx, N, K, yy); break;
    default: hipLaunchKernelGGL(moe::gemv_kernel<4>, dim3(grid), dim3(moe::kGemvThreads), 0, s, w, xx, N, K, yy); break;
  }
  MOE_LAUNCH_CHECK();
  return MOE_STATUS_OK;
}
