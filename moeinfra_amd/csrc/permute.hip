// K3: group (token, slot) pairs by expert with a counting sort that keeps token order.
//
// Same grouping as MoELayer._forward_tokens (model/moe_layer.py:150-185): experts in
// ascending id, and within an expert its tokens in ascending order (a boolean-mask
// gather visits tokens in order; a token never picks one expert twice).  Everything
// stays on the device: the reference's `unique().tolist()` and `mask.any()` host syncs
// become the `active` list and `counts` this kernel writes.
//
// One 1024-thread workgroup.  Pass 1 counts with LDS atomics.  Pass 2 walks the slots in
// 1024-slot chunks; the rank of a slot among equal-expert slots is a popcount of a wave
// ballot plus the totals of earlier waves and earlier chunks, so the order is stable.
#include "common.h"

namespace moe {
namespace {

constexpr int kPermThreads = 1024;
constexpr int kPermWaves = kPermThreads / kWave;

__global__ void __launch_bounds__(kPermThreads)
permute_kernel(const int32_t *__restrict__ idx, int64_t n_slots, int k, int E,
               int32_t *__restrict__ counts, int32_t *__restrict__ offsets,
               int32_t *__restrict__ perm_tok, int32_t *__restrict__ slot_pos,
               int32_t *__restrict__ active) {
  __shared__ int32_t s_count[MOE_MAX_EXPERTS];
  __shared__ int32_t s_base[MOE_MAX_EXPERTS];         // offsets[e] + rows already placed
  __shared__ int32_t s_wave[kPermWaves][MOE_MAX_EXPERTS];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid >> 6;
  if (tid < MOE_MAX_EXPERTS) s_count[tid] = 0;
  __syncthreads();

  // Ids outside [0, E) are never placed (the host validates them; this keeps LDS safe).
  for (int64_t s = tid; s < n_slots; s += kPermThreads) {
    const int e = idx[s];
    if ((unsigned)e < (unsigned)E) atomicAdd(&s_count[e], 1);
  }
  __syncthreads();

  if (tid == 0) {
    int run = 0, na = 0;
    for (int e = 0; e < E; ++e) {
      counts[e] = s_count[e];
      offsets[e] = run;
      s_base[e] = run;
      if (s_count[e] > 0) active[1 + na++] = e;
      run += s_count[e];
    }
    offsets[E] = run;
    active[0] = na;
    for (int e = na; e < E; ++e) active[1 + e] = -1;
  }
  __syncthreads();

  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int64_t c0 = 0; c0 < n_slots; c0 += kPermThreads) {
    const int64_t s = c0 + tid;
    int my_e = s < n_slots ? idx[s] : -1;
    if ((unsigned)my_e >= (unsigned)E) my_e = -1;
    int rank = 0;
    for (int e = 0; e < E; ++e) {
      const uint64_t b = __ballot(my_e == e);
      if (my_e == e) rank = __popcll(b & lt_mask);
      if (lane == 0) s_wave[wave][e] = __popcll(b);
    }
    __syncthreads();
    int pos = -1;
    if (my_e >= 0) {
      int before = 0;
      for (int w = 0; w < wave; ++w) before += s_wave[w][my_e];
      pos = s_base[my_e] + before + rank;
    }
    __syncthreads();  // everyone has read s_base before it advances
    if (tid < E) {
      int tot = 0;
      for (int w = 0; w < kPermWaves; ++w) tot += s_wave[w][tid];
      s_base[tid] += tot;
    }
    if (pos >= 0) perm_tok[pos] = (int32_t)(s / k);
    if (s < n_slots) slot_pos[s] = pos;  // -1 marks an id outside [0, E)
    __syncthreads();
  }
}

}  // namespace
}  // namespace moe

extern "C" int moe_permute(const void *idx_i32, int64_t T, int32_t k, int32_t E, void *counts,
                           void *offsets, void *perm_tok, void *slot_pos, void *active,
                           void *stream) {
  MOE_REQUIRE(T >= 0 && T <= (int64_t)1 << 26, "T out of range");
  MOE_REQUIRE(E >= 1 && E <= MOE_MAX_EXPERTS, "num_experts must be in [1, %d] (got %d)",
              MOE_MAX_EXPERTS, E);
  MOE_REQUIRE(k >= 1 && k <= E && k <= MOE_MAX_TOPK, "top-k must be in [1, min(E, %d)]",
              MOE_MAX_TOPK);
  MOE_REQUIRE(counts && offsets && active, "null device pointer");
  MOE_REQUIRE(T == 0 || (idx_i32 && perm_tok && slot_pos), "null device pointer");
  hipLaunchKernelGGL(moe::permute_kernel, dim3(1), dim3(moe::kPermThreads), 0, (hipStream_t)stream,
                     (const int32_t *)idx_i32, T * (int64_t)k, k, E, (int32_t *)counts,
                     (int32_t *)offsets, (int32_t *)perm_tok, (int32_t *)slot_pos,
                     (int32_t *)active);
  MOE_LAUNCH_CHECK();
  return MOE_STATUS_OK;
}
