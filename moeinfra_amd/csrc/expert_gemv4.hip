// K4, decode form: NF4 expert GEMV for at most 4 tokens per expert, on
// v_mfma_f32_4x4x4_16b_bf16 (16 independent 4x4x4 blocks per instruction).
//
// Memory layout drives the design.  A wavefront streams a tile of 4 consecutive weight
// rows; lane l = 4*blk + j loads 16 packed bytes of row j at byte 16*blk of each 256-byte
// segment, so one load instruction reads 4 rows x 256 contiguous bytes (a contiguous
// stream per row -- measured at the copy rate on MI355X, where 16 rows x 32 B per
// instruction reach barely half of it).
//
// In the 4x4x4_16b MFMA, lane l holds B[block l/4][k 0..3][n = l%4], A[block l/4][m = l%4]
// [k 0..3] and receives D[block l/4][m 0..3][n = l%4].  With the weights as B (n = row j)
// and the activations as A (m = token), the 16 blocks are 16 independent K slices: the
// lane's 16 bytes (32 values, one half of an NF4 block) go through 8 MFMAs into a
// temporary that is scaled by the lane's single absmax and added to its accumulator.  At
// the end of a row tile a butterfly over the 16 block lanes completes the dot products.
//
// The codebook table (64 KB, see nf4_tile.h) is built once per workgroup from the first
// active expert, while the first weight loads are already in flight; a wave whose expert
// carries a different codebook switches to a per-nibble lookup in a private 16-entry
// table for that expert.
#include "gemv4_core.h"

namespace moe {
namespace {

// Streams `ntiles` consecutive 4-row tiles of expert `e` (starting at tile0) through a
// D-stage register pipeline and writes the tiles' outputs:
//   GATEUP: h[off + m][row] = swiglu(w1[row] . x[tok m], w3[row] . x[tok m])
//   !GATEUP: y[off + m][row] = w2[row] . h[off + m]
// `after_prologue` runs once the first D-1 stages are in flight (the kernel builds its
// lookup table there, overlapping the first loads).
template <bool GATEUP, int D, bool SLOW, bool BC, typename Hook>
__device__ __forceinline__ void stream_tiles(const moe_nf4_expert_t &ex, const uint16_t *act,
                                             int K, int R, const Route &rt, int e, int tile0,
                                             int ntiles, const uint32_t *tbl,
                                             const float *slow_code, uint16_t *h_out,
                                             float *y_out, Hook &&after_prologue) {
  constexpr int NP = GATEUP ? 2 : 1;
  const int lane = threadIdx.x & (kWave - 1);
  const int blk = lane >> 2;
  const int j = lane & 3;
  const int NS = K / kStageVals;
  const int cnt = rt.counts[e];
  const int off = rt.offsets[e];

  const size_t row_bytes = (size_t)(K >> 1);
  const size_t row_blocks = (size_t)(K >> 6);
  const size_t r0 = (size_t)tile0 * 4 + j;
  const uint8_t *wq[NP];
  const float *wa[NP];
  uint32_t lane_const[NP];
  if (GATEUP) {
    wq[0] = (const uint8_t *)ex.w1_packed + r0 * row_bytes + blk * 16;
    wa[0] = (const float *)ex.w1_absmax + r0 * row_blocks + (blk >> 1);
    wq[NP - 1] = (const uint8_t *)ex.w3_packed + r0 * row_bytes + blk * 16;
    wa[NP - 1] = (const float *)ex.w3_absmax + r0 * row_blocks + (blk >> 1);
    lane_const[0] = (uint32_t)(lane & 31) << 2;
    lane_const[NP - 1] = ((uint32_t)(lane & 31) << 2) | 128u;
  } else {
    wq[0] = (const uint8_t *)ex.w2_packed + r0 * row_bytes + blk * 16;
    wa[0] = (const float *)ex.w2_absmax + r0 * row_blocks + (blk >> 1);
    lane_const[0] = (uint32_t)lane << 2;
  }
  // Activation row of the lane's token m = j (A operand row): x rows are gathered
  // through perm_tok; h rows are already in expert order.  A lane whose token slot is
  // empty (j >= cnt) reads the expert's first row instead: row m of the MFMA result
  // depends only on row m of A, and rows m >= cnt are never stored, so no branch (which
  // would serialise the load pipeline) is needed.  With BC the lane reads quarter j of
  // the first token's chunk.
  const int jj = (!BC && j < cnt) ? j : 0;
  const int arow = GATEUP ? rt.perm_tok[off + jj] : off + jj;
  const uint16_t *ap = act + (size_t)arow * K + blk * 32 + (BC ? j * 8 : 0);
  const size_t tile_bytes = 4 * row_bytes;
  const size_t tile_blocks = 4 * row_blocks;

  // Past the last stage the (unused) prefetches read the lane's activations, which stay in
  // L2, instead of weight lines that the non-temporal loads have let go.
  bool past = false;
  auto load = [&](Stage4<NP, BC> &st, int t, int sg) {
    const uint8_t *dummy = reinterpret_cast<const uint8_t *>(ap + sg * kStageVals);
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      st.q[p] = ld_stream16(past ? dummy : wq[p] + t * tile_bytes + sg * 256);
      st.s[p] = past ? *reinterpret_cast<const float *>(dummy) : wa[p][t * tile_blocks + sg * 8];
    }
    const uint4 *px = reinterpret_cast<const uint4 *>(ap + sg * kStageVals);
#pragma unroll
    for (int i = 0; i < (BC ? 1 : 4); ++i) st.xa[i] = px[i];
  };

  f32x4 acc[NP];
#pragma unroll
  for (int p = 0; p < NP; ++p) acc[p] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  auto finish = [&](int t) {
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[p][i] = lanes_sum16(acc[p][i]);
    if (blk == 0) {
      const int row = (tile0 + t) * 4 + j;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        if (m < cnt) {
          if (GATEUP)
            h_out[(size_t)(off + m) * R + row] = swiglu_bf16(acc[0][m], acc[NP - 1][m]);
          else
            y_out[(size_t)(off + m) * R + row] = acc[0][m];
        }
      }
    }
#pragma unroll
    for (int p = 0; p < NP; ++p) acc[p] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  };

  // Eight 4x4x4 MFMAs per projection over the lane's 32 values, then one absmax scale.
  auto compute = [&](const Stage4<NP, BC> &st) {
    f32x4 t[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p) t[p] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const s16x4 a = a_operand<BC>(st.xa, i);
#pragma unroll
      for (int p = 0; p < NP; ++p)
        t[p] = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(
            a, b_operand<SLOW>(st.q[p], i, tbl, lane_const[p], slow_code + 16 * p), t[p], 0, 0, 0);
    }
#pragma unroll
    for (int p = 0; p < NP; ++p) scale_acc(acc[p], t[p], st.s[p]);
  };

  // Prefetches are unconditional (a branch around them would make the compiler wait
  // for the whole pipeline): past the last stage the load counter saturates and re-reads
  // the last stage, whose data is not used.
  const int total = ntiles * NS;
  Stage4<NP, BC> st[D];
  int lt = 0, ls = 0;  // next stage to load (tile, segment)
  auto advance = [&]() {
    if (++ls == NS) {
      ls = 0;
      ++lt;
    }
    if (lt == ntiles) {
      lt = ntiles - 1;
      ls = NS - 1;
      past = true;
    }
  };
  // The scheduling barriers keep the prologue's loads in stage order.  Left free, the
  // scheduler groups the weight loads first and the activation loads last, and since the
  // loop's wait counts must hold for the entry path too, every wait in the loop body then
  // assumes only a few younger loads in flight (measured: vmcnt(8) instead of ~25).
#pragma unroll
  for (int d = 0; d < D - 1; ++d) {
    load(st[d], lt, ls);
    advance();
    __builtin_amdgcn_sched_barrier(0);
  }
  after_prologue();
  int ct = 0, cs = 0;  // stage being consumed
  for (int s0 = 0; s0 < total; s0 += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      load(st[(d + D - 1) % D], lt, ls);
      advance();
      if (s0 + d < total) {
        compute(st[d]);
        if (++cs == NS) {
          finish(ct);
          cs = 0;
          ++ct;
        }
      }
    }
  }
}

template <bool GATEUP>
__device__ __forceinline__ const float *code_lo(const moe_nf4_expert_t &ex) {
  return (const float *)(GATEUP ? ex.w1_code : ex.w2_code);
}
template <bool GATEUP>
__device__ __forceinline__ const float *code_hi(const moe_nf4_expert_t &ex) {
  return (const float *)(GATEUP ? ex.w3_code : ex.w2_code);
}

__device__ void combine_tokens(const FusedCombine &fc, const float *y, int H, int64_t rows) {
  for (int t = 0; t < fc.T; ++t) {
    int ord[MOE_MAX_TOPK];
    int e_of[MOE_MAX_TOPK];
    for (int j = 0; j < fc.k; ++j) {
      ord[j] = j;
      e_of[j] = fc.idx32[t * fc.k + j];
    }
    for (int j = 1; j < fc.k; ++j) {
      const int cur = ord[j];
      int p = j - 1;
      while (p >= 0 && e_of[ord[p]] > e_of[cur]) {
        ord[p + 1] = ord[p];
        --p;
      }
      ord[p + 1] = cur;
    }
    for (int c = threadIdx.x * 4; c < H; c += kFfnThreads * 4) {
      float o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      for (int jj = 0; jj < fc.k; ++jj) {
        const int j = ord[jj];
        const int pos = fc.slot_pos[t * fc.k + j];
        if (pos < 0 || pos >= rows) continue;
        const float w = fc.weights[t * fc.k + j];
        const float4 yv4 = *reinterpret_cast<const float4 *>(y + (size_t)pos * H + c);
        const float yv[4] = {yv4.x, yv4.y, yv4.z, yv4.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float p = bf16_to_f32(f32_to_bf16(yv[i])) * w;
          o[i] = bf16_to_f32(f32_to_bf16(o[i] + p));
        }
      }
      *reinterpret_cast<uint2 *>(fc.out + (size_t)t * H + c) =
          make_uint2(pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3]));
    }
  }
}

template <bool GATEUP, int DB, int DN>
__global__ void __launch_bounds__(kFfnThreads, 2)
gemv4_kernel(const ExpertTable tab, const uint16_t *__restrict__ act, int H, int F, Route rt,
             uint16_t *__restrict__ h_out, float *__restrict__ y_out, FusedCombine fc,
             int64_t rows_total) {
  __shared__ __attribute__((aligned(16))) uint32_t s_tbl[kTableWords];
  __shared__ float s_code[32];
  __shared__ float s_slow[kFfnWaves][32];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid >> 6;
  const int K = GATEUP ? H : F;
  const int R = GATEUP ? F : H;
  const int tiles_e = R >> 2;
  const int n_active = rt.active[0];

  // The shared lookup table holds the codebooks of the first present active expert.
  int e0 = -1;
  for (int a = 0; a < n_active; ++a) {
    const int e = rt.active[1 + a];
    if ((GATEUP ? tab.e[e].w1_packed : tab.e[e].w2_packed) != nullptr) {
      e0 = e;
      break;
    }
  }
  // e0 < 0 (no present expert has tokens): no tile work, but the workgroup still takes
  // part in the completion count of a fused combine.
  const float *t_lo = e0 >= 0 ? code_lo<GATEUP>(tab.e[e0]) : nullptr;
  const float *t_hi = e0 >= 0 ? code_hi<GATEUP>(tab.e[e0]) : nullptr;
  const float t_mine = (e0 >= 0 && lane < 32) ? (lane < 16 ? t_lo : t_hi)[lane & 15] : 0.0f;

  // Every wave calls this exactly once (it contains workgroup barriers): inside its
  // first tile stream, after the first loads are issued, or at the end if it has no work.
  bool built = false;
  auto build_table = [&]() {
    if (built) return;
    built = true;
    if (tid < 32) s_code[tid] = t_mine;
    __syncthreads();
    for (int i = tid; i < kTableWords; i += kFfnThreads) {
      const int v = i >> 6;
      const int half = (i & 32) ? 16 : 0;
      s_tbl[i] = pack_bf16x2(s_code[half + (v >> 4)], s_code[half + (v & 15)]);
    }
    __syncthreads();
  };

  // Balanced contiguous range of the flattened (active expert, 4-row tile) list.
  const int64_t N = e0 >= 0 ? (int64_t)n_active * tiles_e : 0;
  const int64_t W = (int64_t)gridDim.x * kFfnWaves;
  const int64_t wid = (int64_t)blockIdx.x * kFfnWaves + wave;
  int64_t t = wid * N / W;
  const int64_t t_end = (wid + 1) * N / W;
  while (t < t_end) {
    const int ai = (int)(t / tiles_e);
    const int64_t seg_end = t_end < (int64_t)(ai + 1) * tiles_e ? t_end : (int64_t)(ai + 1) * tiles_e;
    const int e = rt.active[1 + ai];
    const moe_nf4_expert_t &ex = tab.e[e];
    const int tile0 = (int)(t - (int64_t)ai * tiles_e);
    const int ntiles = (int)(seg_end - t);
    t = seg_end;
    if ((GATEUP ? ex.w1_packed : ex.w2_packed) == nullptr) continue;  // absent expert
    // Codebook check against the table's (wave-uniform).
    float mine = 0.0f;
    int diff = 0;
    if (lane < 32) {
      mine = (lane < 16 ? code_lo<GATEUP>(ex) : code_hi<GATEUP>(ex))[lane & 15];
      diff = __builtin_bit_cast(uint32_t, mine) != __builtin_bit_cast(uint32_t, t_mine);
    }
    const bool slow = __any(diff);
    if (slow && lane < 32) s_slow[wave][lane] = mine;
    wave_lds_sync();  // the whole wave reads s_slow[wave] below
    const bool bc = rt.counts[e] == 1;
    const float *sc = s_slow[wave];
    if (!slow && bc)
      stream_tiles<GATEUP, DB, false, true>(ex, act, K, R, rt, e, tile0, ntiles, s_tbl, sc, h_out, y_out, build_table);
    else if (!slow)
      stream_tiles<GATEUP, DN, false, false>(ex, act, K, R, rt, e, tile0, ntiles, s_tbl, sc, h_out, y_out, build_table);
    else if (bc)
      stream_tiles<GATEUP, DB, true, true>(ex, act, K, R, rt, e, tile0, ntiles, s_tbl, sc, h_out, y_out, build_table);
    else
      stream_tiles<GATEUP, DN, true, false>(ex, act, K, R, rt, e, tile0, ntiles, s_tbl, sc, h_out, y_out, build_table);
  }
  build_table();

  if (!GATEUP && fc.out != nullptr) {
    __shared__ uint32_t s_last;
    __threadfence();  // publish this workgroup's y rows (device scope)
    __syncthreads();
    if (tid == 0) s_last = atomicAdd(fc.counter, 1u) == gridDim.x - 1;
    __syncthreads();
    if (s_last) {
      __threadfence();  // every other workgroup's y rows are visible now
      combine_tokens(fc, y_out, H, rows_total);
    }
  }
}

}  // namespace

bool gemv4_supported(int64_t max_tokens_per_expert, int32_t H, int32_t F) {
  return max_tokens_per_expert <= 4 && H % kStageVals == 0 && F % kStageVals == 0;
}

int launch_gemv4(const void *tab_ptr, const void *x, int32_t H, int32_t F, const void *route,
                 void *h_ws, void *ypart, int phases, int64_t active_max, int64_t rows_total,
                 const void *fused_combine, hipStream_t stream) {
  const ExpertTable &tab = *static_cast<const ExpertTable *>(tab_ptr);
  const Route &rt = *static_cast<const Route *>(route);
  FusedCombine fc{};
  if (fused_combine != nullptr) fc = *static_cast<const FusedCombine *>(fused_combine);
  const int64_t cap = (int64_t)device_cu_count() * 2;
  if (phases & 1) {
    int64_t g = (active_max * (F / 4) + kFfnWaves - 1) / kFfnWaves;
    if (g > cap) g = cap;
    hipLaunchKernelGGL((gemv4_kernel<true, 6, 4>), dim3((unsigned)g), dim3(kFfnThreads), 0, stream,
                       tab, (const uint16_t *)x, H, F, rt, (uint16_t *)h_ws, (float *)nullptr,
                       FusedCombine{}, rows_total);
    MOE_LAUNCH_CHECK();
  }
  if (phases & 2) {
    int64_t g = (active_max * (H / 4) + kFfnWaves - 1) / kFfnWaves;
    if (g > cap) g = cap;
    hipLaunchKernelGGL((gemv4_kernel<false, 8, 4>), dim3((unsigned)g), dim3(kFfnThreads), 0, stream,
                       tab, (const uint16_t *)h_ws, H, F, rt, (uint16_t *)nullptr, (float *)ypart,
                       fc, rows_total);
    MOE_LAUNCH_CHECK();
  }
  return MOE_STATUS_OK;
}

}  // namespace moe
