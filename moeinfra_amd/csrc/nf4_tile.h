// Device helpers shared by the NF4 expert-FFN kernels (gfx950).
//
// NF4 byte -> bf16 pair lookup.  One v_perm_b32 builds the LDS byte address
// (byte << 8) | (replica << 2) and one ds_read_b32 returns
// {bf16(code[hi nibble]), bf16(code[lo nibble])} (value 2j in the low half).  The table
// has 64 replicas, one per lane, so lookups never bank-conflict: 256 x 64 x 4 B = 64 KB.
// A table may hold two codebooks: replicas 0-31 the first, 32-63 the second.
#pragma once

#include "common.h"

namespace moe {

struct ExpertTable {
  moe_nf4_expert_t e[MOE_MAX_EXPERTS];
};

struct Route {
  const int32_t *counts;
  const int32_t *offsets;
  const int32_t *perm_tok;
  const int32_t *active;
};

// Optional combine fused into the down projection: the last workgroup to finish computes
// out[t] from the y rows of token t's k slots (ascending expert order, bf16 destination),
// the work of the stand-alone combine kernel.
struct FusedCombine {
  const float *weights;     // [T, k]
  const int32_t *idx32;     // [T, k]
  const int32_t *slot_pos;  // [T*k]
  uint16_t *out;            // [T, H] (null: no fused combine)
  uint32_t *counter;        // zeroed before the launch
  int T;
  int k;
};

namespace {

constexpr int kFfnWaves = 4;
constexpr int kFfnThreads = kFfnWaves * kWave;
constexpr int kTableWords = 256 * 64;

__device__ __forceinline__ bf16x8 as_bf16x8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  return __builtin_bit_cast(bf16x8, make_uint4(a, b, c, d));
}
__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }
__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ uint32_t lds_lookup(const uint32_t *tbl, uint32_t byte_addr) {
  return *reinterpret_cast<const uint32_t *>(reinterpret_cast<const char *>(tbl) + byte_addr);
}

// Eight packed bytes (values 2j, 2j+1 per byte) -> eight bf16 pairs.  `lane_const` is the
// lane's replica byte offset (< 256); selector byte 1 takes packed byte j, byte 0 the
// replica offset, bytes 2-3 are zero.
__device__ __forceinline__ void lookup8(const uint32_t *tbl, uint2 q, uint32_t lane_const,
                                        uint32_t out[8]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    out[j] = lds_lookup(tbl, __builtin_amdgcn_perm(q.x, lane_const, 0x0c0c0400u + (j << 8)));
    out[4 + j] = lds_lookup(tbl, __builtin_amdgcn_perm(q.y, lane_const, 0x0c0c0400u + (j << 8)));
  }
}

// Loads the work item's codebooks and (re)builds the lookup table when they differ from
// the resident ones.  Must be called by all NT threads of the workgroup; acts as a barrier.
template <int NT = kFfnThreads>
__device__ __forceinline__ void ensure_table(uint32_t *tbl, uint32_t *s_raw, float *s_code,
                                             const float *code_lo, const float *code_hi,
                                             bool &built) {
  const int tid = threadIdx.x;
  uint32_t mine = 0;
  int diff = 0;
  if (tid < 32) {
    mine = __builtin_bit_cast(uint32_t, (tid < 16 ? code_lo : code_hi)[tid & 15]);
    diff = !built || mine != s_raw[tid];
  }
  if (__syncthreads_or(diff)) {
    if (tid < 32) {
      s_raw[tid] = mine;
      s_code[tid] = __builtin_bit_cast(float, mine);
    }
    __syncthreads();
    for (int i = tid; i < kTableWords; i += NT) {
      const int v = i >> 6;                   // packed byte value
      const int half = (i & 32) ? 16 : 0;     // replicas 32-63 use the second codebook
      tbl[i] = pack_bf16x2(s_code[half + (v >> 4)], s_code[half + (v & 15)]);
    }
    __syncthreads();
    built = true;
  }
}

__device__ __forceinline__ f32x4 mfma_block(bf16x8 a0, bf16x8 b0, bf16x8 a1, bf16x8 b1) {
  f32x4 t = {0.0f, 0.0f, 0.0f, 0.0f};
  t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, b0, t, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b1, t, 0, 0, 0);
}

__device__ __forceinline__ void scale_acc(f32x4 &acc, const f32x4 &t, float s) {
  acc[0] = fmaf(s, t[0], acc[0]);
  acc[1] = fmaf(s, t[1], acc[1]);
  acc[2] = fmaf(s, t[2], acc[2]);
  acc[3] = fmaf(s, t[3], acc[3]);
}

__device__ __forceinline__ float silu_f32(float v) { return v / (1.0f + expf(-v)); }

__device__ __forceinline__ uint16_t swiglu_bf16(float g, float u) {
  // bf16(bf16(silu(bf16(g))) * bf16(u)): the op sequence of F.silu(gate) * up on bf16 tensors.
  const float gb = bf16_to_f32(f32_to_bf16(g));
  const float ub = bf16_to_f32(f32_to_bf16(u));
  const float sb = bf16_to_f32(f32_to_bf16(silu_f32(gb)));
  return f32_to_bf16(sb * ub);
}

}  // namespace
}  // namespace moe
