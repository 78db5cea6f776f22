// Residual add + RMSNorm of one row by a workgroup (MixtralRMSNorm on bf16 tensors, with
// the decoder layer's residual add in front): shared by the decoder kernels and the fused
// single-token MoE gate/up kernel, so that every caller with the same row length sums in
// the same order and produces the same bits.
#pragma once

#include "common.h"

namespace moe {
namespace {

constexpr int kNormThreads = 256;
constexpr int kNormMaxChunks = 8;  // 8-value chunks per thread: H <= 16384

__device__ __forceinline__ float bf16r(float v) { return bf16_to_f32(f32_to_bf16(v)); }

// Workgroup barrier that orders LDS only: a workgroup fence on all address spaces would
// also wait for the wave's outstanding global loads (s_waitcnt vmcnt(0)), which in the
// fused kernels are the weight rows still streaming in.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ float block_sum(float v, float *s_part) {
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x >> 6;
  float ws[1] = {v};
  lane_groups_reduce<false>(ws, kWave);
  if (lane == 0) s_part[wave] = ws[0];
  lds_barrier();
  float t = 0.0f;
  for (int w = 0; w < (int)(blockDim.x >> 6); ++w) t += s_part[w];
  lds_barrier();
  return t;
}

// One row of the residual add + RMSNorm, run by all kNormThreads threads of a workgroup:
// r = x (+ res) with one bf16 add (written to res_out when given), then
// out = bf16(w * bf16(r * inv)), inv = 1 / sqrt(mean(r^2) + eps) from fp32 statistics.
// Thread t takes the 8-value chunks (t + i * kNormThreads) * 8 for i < CH (chunks past H
// load the last chunk again, in bounds, and count for nothing), so every caller with the
// same H sums in the same order.  Split in two so that a caller can issue other loads
// between them: norm_load issues every load; norm_finish waits for them only (vmcnt is in
// order, so loads issued after norm_load are not waited for).  `out` may point to LDS.
template <int CH>
struct NormRegs {
  uint4 x[CH], r[CH], w[CH];
};

// RES: whether a residual is added (a compile-time choice, so that no load sits behind a
// branch, where the compiler would sink it past later loads).
template <int CH, bool RES>
__device__ __forceinline__ void norm_load(NormRegs<CH> &g, const uint16_t *x, const uint16_t *res,
                                          const uint16_t *w, int H) {
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    int c = (threadIdx.x + i * kNormThreads) * 8;
    c = c < H ? c : H - 8;
    g.w[i] = *reinterpret_cast<const uint4 *>(w + c);
    g.x[i] = *reinterpret_cast<const uint4 *>(x + c);
    if (RES) g.r[i] = *reinterpret_cast<const uint4 *>(res + c);
  }
}

// act: whether this thread takes part (all threads of the workgroup call it, for the
// barriers; threads with act false add nothing and store nothing; act must be true for
// exactly threads 0 .. kNormThreads-1, so the sums are those of a kNormThreads workgroup).
template <int CH, bool RES>
__device__ __forceinline__ void norm_finish(NormRegs<CH> &g, float eps, int H, uint16_t *res_out,
                                            uint16_t *out, float *s_part, bool act = true) {
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    if (!act) break;
    uint4 v = g.x[i];
    if (RES) {
      const uint32_t a[4] = {v.x, v.y, v.z, v.w}, b[4] = {g.r[i].x, g.r[i].y, g.r[i].z, g.r[i].w};
      uint32_t o[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        o[j] = pack_bf16x2(bf16lo_to_f32(a[j]) + bf16lo_to_f32(b[j]),
                           bf16hi_to_f32(a[j]) + bf16hi_to_f32(b[j]));
      v = make_uint4(o[0], o[1], o[2], o[3]);
    }
    g.x[i] = v;
    const uint32_t a[4] = {v.x, v.y, v.z, v.w};
    float t = ss;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float lo = bf16lo_to_f32(a[j]), hi = bf16hi_to_f32(a[j]);
      t += lo * lo + hi * hi;
    }
    ss = (threadIdx.x + i * kNormThreads) * 8 < H ? t : ss;
  }
  const float inv = 1.0f / sqrtf(block_sum(ss, s_part) / (float)H + eps);
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const int c = (threadIdx.x + i * kNormThreads) * 8;
    if (act && c < H) {
      const uint32_t a[4] = {g.x[i].x, g.x[i].y, g.x[i].z, g.x[i].w};
      const uint32_t gw[4] = {g.w[i].x, g.w[i].y, g.w[i].z, g.w[i].w};
      uint32_t o[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        o[j] = pack_bf16x2(bf16lo_to_f32(gw[j]) * bf16r(bf16lo_to_f32(a[j]) * inv),
                           bf16hi_to_f32(gw[j]) * bf16r(bf16hi_to_f32(a[j]) * inv));
      if (res_out != nullptr) *reinterpret_cast<uint4 *>(res_out + c) = g.x[i];
      *reinterpret_cast<uint4 *>(out + c) = make_uint4(o[0], o[1], o[2], o[3]);
    }
  }
}

// The same row by 2 kNormThreads threads for H <= 2 kNormThreads * 8 (the order of
// norm_finish<2>): thread t loads chunk t only, and thread kNormThreads + t hands its chunk's
// four squared pairs to thread t through LDS, which adds them after its own exactly as
// norm_finish<2> adds its second chunk.  The statistics and outputs are those of the
// kNormThreads form bit for bit, without the loads of a second chunk per thread or of
// chunks past H.
struct NormOneRegs {
  uint4 x, r, w;
};
template <bool RES>
__device__ __forceinline__ void norm_load_one(NormOneRegs &g, const uint16_t *x, const uint16_t *res,
                                              const uint16_t *w, int H) {
  int c = threadIdx.x * 8;
  c = c < H ? c : H - 8;
  g.w = *reinterpret_cast<const uint4 *>(w + c);
  g.x = *reinterpret_cast<const uint4 *>(x + c);
  if (RES) g.r = *reinterpret_cast<const uint4 *>(res + c);
}
template <bool RES>
__device__ __forceinline__ void norm_finish_one(NormOneRegs &g, float eps, int H, uint16_t *res_out,
                                                uint16_t *out, float *s_part,
                                                float (*s_sq)[4]) {
  const int tid = threadIdx.x;
  const int c = tid * 8;
  uint4 v = g.x;
  if (RES) {
    const uint32_t a[4] = {v.x, v.y, v.z, v.w}, b[4] = {g.r.x, g.r.y, g.r.z, g.r.w};
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      o[j] = pack_bf16x2(bf16lo_to_f32(a[j]) + bf16lo_to_f32(b[j]),
                         bf16hi_to_f32(a[j]) + bf16hi_to_f32(b[j]));
    v = make_uint4(o[0], o[1], o[2], o[3]);
  }
  g.x = v;
  float sq[4];
  {
    const uint32_t a[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float lo = bf16lo_to_f32(a[j]), hi = bf16hi_to_f32(a[j]);
      sq[j] = lo * lo + hi * hi;
    }
  }
  if (tid >= kNormThreads) {
#pragma unroll
    for (int j = 0; j < 4; ++j) s_sq[tid - kNormThreads][j] = sq[j];
  }
  lds_barrier();
  float ss = 0.0f;
  if (tid < kNormThreads) {
    float t = ss;
#pragma unroll
    for (int j = 0; j < 4; ++j) t += sq[j];
    ss = c < H ? t : ss;
    t = ss;
#pragma unroll
    for (int j = 0; j < 4; ++j) t += s_sq[tid][j];
    ss = c + kNormThreads * 8 < H ? t : ss;
  }
  const float inv = 1.0f / sqrtf(block_sum(ss, s_part) / (float)H + eps);
  if (c < H) {
    const uint32_t a[4] = {g.x.x, g.x.y, g.x.z, g.x.w};
    const uint32_t gw[4] = {g.w.x, g.w.y, g.w.z, g.w.w};
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      o[j] = pack_bf16x2(bf16lo_to_f32(gw[j]) * bf16r(bf16lo_to_f32(a[j]) * inv),
                         bf16hi_to_f32(gw[j]) * bf16r(bf16hi_to_f32(a[j]) * inv));
    if (res_out != nullptr) *reinterpret_cast<uint4 *>(res_out + c) = g.x;
    *reinterpret_cast<uint4 *>(out + c) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

template <int CH, bool RES>
__device__ __forceinline__ void rmsnorm_row(const uint16_t *x, const uint16_t *res, const uint16_t *w,
                                            float eps, int H, uint16_t *res_out, uint16_t *out,
                                            float *s_part) {
  NormRegs<CH> g;
  norm_load<CH, RES>(g, x, res, w, H);
  norm_finish<CH, RES>(g, eps, H, res_out, out, s_part);
}

}  // namespace
}  // namespace moe
