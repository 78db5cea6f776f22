// Primitives of the NF4 decode GEMV on v_mfma_f32_4x4x4_16b_bf16 (gfx950), shared by the
// per-expert GEMV (expert_gemv4.hip) and the fused decode layer (decode_layer.hip).
//
// A wavefront streams tiles of 4 consecutive weight rows: lane l = 4*blk + j loads 16
// packed bytes of row j at byte 16*blk of each 256-byte segment, so one load instruction
// reads 4 rows x 256 contiguous bytes.  In the 4x4x4_16b MFMA, lane l holds B[block l/4]
// [k 0..3][n = l%4], A[block l/4][m = l%4][k 0..3] and receives D[block l/4][m 0..3]
// [n = l%4]; with the weights as B (n = row j) and the activations as A (m = token) the 16
// blocks are 16 independent K slices, and a butterfly over the 16 block lanes completes
// the dot products at the end of a tile.
#pragma once

#include "nf4_tile.h"

namespace moe {
namespace {

typedef __attribute__((__vector_size__(4 * sizeof(short)))) short s16x4;

constexpr int kStageVals = 512;  // values of one row per pipeline stage (256 packed bytes)

// One pipeline stage of a lane: 16 packed bytes per projection (values 32*blk .. +31 of
// the segment), the absmax of that half block, and the matching activations.  BC (one
// token): the lane holds only quarter j of the token's 64-byte activation chunk and the
// four lanes of a quad share the quarters through DPP broadcasts; otherwise the lane holds
// the whole chunk of its own token (row m = j of the MFMA A operand).
template <int NP, bool BC>
struct Stage4 {
  uint4 q[NP];
  float s[NP];
  uint4 xa[BC ? 1 : 4];
};

__device__ __forceinline__ s16x4 as_s16x4(uint32_t lo, uint32_t hi) {
  return __builtin_bit_cast(s16x4, make_uint2(lo, hi));
}

__device__ __forceinline__ uint32_t byte_of(const uint4 &q, int b) {
  const uint32_t w = b < 4 ? q.x : b < 8 ? q.y : b < 12 ? q.z : q.w;
  return (w >> (8 * (b & 3))) & 0xffu;
}

// DPP quad_perm [q,q,q,q]: every lane of a quad reads lane q of the quad.
template <int Q>
__device__ __forceinline__ uint32_t quad_bcast(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, Q * 0x55, 0xf, 0xf, false);
}
__device__ __forceinline__ uint32_t quad_bcast(uint32_t v, int q) {
  switch (q) {
    case 0: return quad_bcast<0>(v);
    case 1: return quad_bcast<1>(v);
    case 2: return quad_bcast<2>(v);
    default: return quad_bcast<3>(v);
  }
}

// A operand of MFMA i: activations 4i .. 4i+3 of the lane's 32-value chunk.
template <bool BC>
__device__ __forceinline__ s16x4 a_operand(const uint4 *xa, int i) {
  if (BC) {
    const uint32_t lo = (i & 1) ? xa[0].z : xa[0].x;
    const uint32_t hi = (i & 1) ? xa[0].w : xa[0].y;
    return as_s16x4(quad_bcast(lo, i >> 1), quad_bcast(hi, i >> 1));
  }
  const uint4 &xv = xa[i >> 1];
  return (i & 1) ? as_s16x4(xv.z, xv.w) : as_s16x4(xv.x, xv.y);
}

// B operand of MFMA i: packed bytes 2i and 2i+1 -> four bf16 code values.
template <bool SLOW>
__device__ __forceinline__ s16x4 b_operand(const uint4 &q, int i, const uint32_t *tbl,
                                           uint32_t lane_const, const float *slow_code) {
  uint32_t b0, b1;
  if (!SLOW) {
    const uint32_t wi = i < 2 ? q.x : i < 4 ? q.y : i < 6 ? q.z : q.w;
    const uint32_t sel = 0x0c0c0400u + ((uint32_t)(2 * (i & 1)) << 8);
    b0 = lds_lookup(tbl, __builtin_amdgcn_perm(wi, lane_const, sel));
    b1 = lds_lookup(tbl, __builtin_amdgcn_perm(wi, lane_const, sel + 0x100u));
  } else {
    const uint32_t v0 = byte_of(q, 2 * i), v1 = byte_of(q, 2 * i + 1);
    b0 = pack_bf16x2(slow_code[v0 >> 4], slow_code[v0 & 15u]);
    b1 = pack_bf16x2(slow_code[v1 >> 4], slow_code[v1 & 15u]);
  }
  return as_s16x4(b0, b1);
}

// Orders LDS writes of some lanes of a wave before LDS reads of other lanes of the same
// wave.  Lanes are separate threads to the compiler: without this, a store by one lane and
// a load of the same location by another are a race that the compiler may reorder (for
// example by forwarding the stored value to the storing lane and reading LDS early for the
// others).  Wavefront-scope release/acquire fences around a wave barrier; no s_barrier.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ float lanes_sum16(float v) {
  // Sum over the 16 lanes that share l % 4 (the block index occupies lane bits 2..5):
  // rotations by 4 and 8 within each 16-lane row (DPP), then the two cross-row pairs.
  v += dpp_mov<0x124>(v);  // row_ror:4
  v += dpp_mov<0x128>(v);  // row_ror:8
  v = op_xor16<false>(v);
  v = op_xor32<false>(v);
  return v;
}

}  // namespace
}  // namespace moe
