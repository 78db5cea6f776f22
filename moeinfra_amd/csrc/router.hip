// K2: gate linear + fp32 softmax + top-k + renormalise, one workgroup per token.
//
// Follows ExpertRouter.route_with_logits (engine/router.py:50-94):
//   logits = bf16(x . gate^T)          F.linear in the activation dtype  (:66-69)
//   p      = softmax(float(logits))    fp32                               (:81-84)
//   w, idx = topk(p, k)                descending                         (:86-90)
//   w     /= w.sum(-1)                                                    (:92)
// The dot products accumulate in fp32 (each thread a strided slice of H, then a
// butterfly reduction per wave and a fixed-order sum over the waves).  An optional fp32
// per-expert bias is added to float(logits) before the softmax (skewed-routing
// workloads).  Ties in p keep the lower index.
#include "common.h"

namespace moe {
namespace {

constexpr int kRouterThreads = 256;
constexpr int kRouterWaves = kRouterThreads / kWave;

// One workgroup per token: the 256 threads split H (8 values per thread per step, 16-byte
// loads of x and of every gate row), reduce within each wave and then across the four
// waves in a fixed order; wave 0 finishes the softmax and top-k.
template <int EMAX>
__global__ void __launch_bounds__(kRouterThreads)
router_topk_kernel(const uint16_t *__restrict__ x, const uint16_t *__restrict__ gate,
                   const float *__restrict__ bias, int64_t T, int H, int E, int k,
                   uint16_t *__restrict__ logits_out, float *__restrict__ w_out,
                   int64_t *__restrict__ idx_out, int32_t *__restrict__ idx32_out) {
  __shared__ float s_part[kRouterWaves][EMAX];
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid >> 6;
  const int64_t t = blockIdx.x;

  float acc[EMAX];
#pragma unroll
  for (int e = 0; e < EMAX; ++e) acc[e] = 0.0f;

  const uint16_t *xr = x + t * (int64_t)H;
  for (int c = tid * 8; c < H; c += kRouterThreads * 8) {
    const uint4 xv = *reinterpret_cast<const uint4 *>(xr + c);
    const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
    float xf[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      xf[2 * j] = bf16lo_to_f32(xw[j]);
      xf[2 * j + 1] = bf16hi_to_f32(xw[j]);
    }
#pragma unroll
    for (int e = 0; e < EMAX; ++e) {
      if (e < E) {
        const uint4 gv = *reinterpret_cast<const uint4 *>(gate + (int64_t)e * H + c);
        const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          acc[e] = fmaf(xf[2 * j], bf16lo_to_f32(gw[j]), acc[e]);
          acc[e] = fmaf(xf[2 * j + 1], bf16hi_to_f32(gw[j]), acc[e]);
        }
      }
    }
  }
#pragma unroll
  for (int e = 0; e < EMAX; ++e) {
    if (e < E) {
      const float v = wave_sum(acc[e]);
      if (lane == 0) s_part[wave][e] = v;
    }
  }
  __syncthreads();
  if (wave != 0) return;

  float p[EMAX];
  float m = -INFINITY;
#pragma unroll
  for (int e = 0; e < EMAX; ++e) {
    if (e < E) {
      float v = s_part[0][e];
#pragma unroll
      for (int w = 1; w < kRouterWaves; ++w) v += s_part[w][e];
      const uint16_t lb = f32_to_bf16(v);
      if (logits_out != nullptr && lane == e) logits_out[t * E + e] = lb;
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

  // Top-k by repeated arg-max (strict '>' keeps the lowest index among equals).
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
  if (lane < k) {
    float wv = 0.0f;
    int iv = 0;
    for (int j = 0; j < k; ++j)
      if (j == lane) {
        wv = topw[j];
        iv = topi[j];
      }
    w_out[t * k + lane] = wv / wsum;
    idx_out[t * k + lane] = iv;
    if (idx32_out != nullptr) idx32_out[t * k + lane] = iv;
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
  const dim3 g((unsigned)T), b(moe::kRouterThreads);
  hipStream_t s = (hipStream_t)stream;
  auto args = [&](auto kern) {
    hipLaunchKernelGGL(kern, g, b, 0, s, (const uint16_t *)x_bf16, (const uint16_t *)gate_bf16,
                       (const float *)bias_f32, T, H, E, k, (uint16_t *)logits_bf16,
                       (float *)weights_f32, (int64_t *)idx_i64, (int32_t *)idx_i32);
  };
  if (E <= 8)
    args(moe::router_topk_kernel<8>);
  else if (E <= 16)
    args(moe::router_topk_kernel<16>);
  else
    args(moe::router_topk_kernel<32>);
  MOE_LAUNCH_CHECK();
  return MOE_STATUS_OK;
}
