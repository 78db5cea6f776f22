// K4: grouped NF4 SwiGLU expert FFN (fused dequant, bf16 MFMA, fp32 accumulate) and
// K5: weighted combine, for gfx950.
//
// Reference semantics (ParshwaPatel-07/MoEInfra):
//   y_e(x) = w2( silu(w1 x) * (w3 x) )      transfer/nf4_reconstruct.py:152-155
//   out    = 0; for e ascending: out[mask_e] += y_e * w_e   model/moe_layer.py:147,172-191
//
// Weight tile mapping (both projections kernels).  A wavefront owns 16 weight rows.  In a
// v_mfma_f32_16x16x32_bf16, lane l = (n = l%16, g = l/16) supplies B[k in 8g..8g+7][n]
// and A[m = n][k in 8g..8g+7] and receives D[m = 4g+i][n].  The weights are B (one
// weight row per column n), the token activations are A (one token per row m).  For a
// 64-value NF4 block b of row n, lane (n, g) loads packed bytes 8g..8g+7 (values
// 16g..16g+15): the first four bytes feed one MFMA, the last four the next, so both
// MFMAs of a block see only that block and the block's absmax (one value per lane: the
// lane's row) scales the 4 accumulator values the lane holds.  A uses the same value
// order: lane (m, g) loads the 16 activations x[m][64b+16g .. +15].
//
// Packed byte -> bf16 pair: one v_perm_b32 builds the LDS byte address
// (byte << 8) | (replica << 2) and one ds_read_b32 returns
// {bf16(code[hi nibble]), bf16(code[lo nibble])}.  The table has 64 replicas (one per
// lane) so the lookups never bank-conflict: 256 x 64 x 4 B = 64 KB.  The gate/up kernel
// keeps w1's codebook in replicas 0-31 and w3's in 32-63 (both tables in the same 64 KB).
// A work item rebuilds the table only when its codebooks differ from the ones loaded.
//
// The code value is rounded to bf16 before the absmax scaling (the scaling happens in
// fp32 after the MFMA), so an effective weight is bf16(code)*absmax instead of
// bf16(code*absmax): a relative difference below 2^-8 per weight.
#include "nf4_tile.h"

namespace moe {
namespace {

// ----------------------------------------------------------------------------- pipeline
// Registers of one pipeline stage: U consecutive NF4 blocks of NP projections for the
// lane's weight row (8 packed bytes each), their absmax, and the activations of the
// lane's token row for MT token tiles.  A wave keeps D stages in flight: the loads of
// stage i+D-1 are issued before stage i is consumed.
template <int NP, int MT, int U>
struct Stage {
  uint2 q[NP][U];
  float s[NP][U];
  uint4 xa[MT][U][2];
};

// Activation rows of empty token slots point at a valid row: row m of an MFMA result
// depends only on row m of A and such rows are never stored, so the loads need no branch
// (a branch would make the compiler wait for the whole pipeline).
template <int NP, int MT, int U>
__device__ __forceinline__ void load_stage(Stage<NP, MT, U> &st, const uint8_t *const (&wq)[NP],
                                           const float *const (&wa)[NP],
                                           const uint16_t *const (&xr)[MT], int b) {
#pragma unroll
  for (int u = 0; u < U; ++u) {
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      st.q[p][u] = *reinterpret_cast<const uint2 *>(wq[p] + (size_t)(b + u) * 32);
      st.s[p][u] = wa[p][b + u];
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const uint4 *px = reinterpret_cast<const uint4 *>(xr[mt] + (size_t)(b + u) * 64);
      st.xa[mt][u][0] = px[0];
      st.xa[mt][u][1] = px[1];
    }
  }
}

template <int NP, int MT, int U>
__device__ __forceinline__ void compute_stage(const Stage<NP, MT, U> &st, const uint32_t *tbl,
                                              const uint32_t (&lane_const)[NP],
                                              f32x4 (&acc)[NP][MT]) {
#pragma unroll
  for (int u = 0; u < U; ++u) {
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      uint32_t l[8];
      lookup8(tbl, st.q[p][u], lane_const[p], l);
      const bf16x8 b0 = as_bf16x8(l[0], l[1], l[2], l[3]);
      const bf16x8 b1 = as_bf16x8(l[4], l[5], l[6], l[7]);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        scale_acc(acc[p][mt],
                  mfma_block(as_bf16x8(st.xa[mt][u][0]), b0, as_bf16x8(st.xa[mt][u][1]), b1),
                  st.s[p][u]);
    }
  }
}

// Streams blocks [b_lo, b_hi) of the lane's weight row(s) through the D-stage pipeline.
// Prefetches are unconditional: past the last full stage they re-read it (unused data).
template <int NP, int MT, int U, int D>
__device__ __forceinline__ void stream_blocks(const uint32_t *tbl, const uint8_t *const (&wq)[NP],
                                              const float *const (&wa)[NP],
                                              const uint16_t *const (&xr)[MT],
                                              const uint32_t (&lane_const)[NP], int b_lo,
                                              int b_hi, f32x4 (&acc)[NP][MT]) {
  const int ns = (b_hi - b_lo) / U;
  if (ns > 0) {
    Stage<NP, MT, U> st[D];
    const int last = b_lo + (ns - 1) * U;
    int bl = b_lo;  // next stage to load
#pragma unroll
    for (int d = 0; d < D - 1; ++d) {
      load_stage(st[d], wq, wa, xr, bl);
      bl = bl + U < last ? bl + U : last;
    }
    for (int s0 = 0; s0 < ns; s0 += D) {
#pragma unroll
      for (int d = 0; d < D; ++d) {
        load_stage(st[(d + D - 1) % D], wq, wa, xr, bl);
        bl = bl + U < last ? bl + U : last;
        if (s0 + d < ns) compute_stage(st[d], tbl, lane_const, acc);
      }
    }
  }
  for (int b = b_lo + ns * U; b < b_hi; ++b) {
    Stage<NP, MT, 1> t;
    load_stage(t, wq, wa, xr, b);
    compute_stage(t, tbl, lane_const, acc);
  }
}

// ----------------------------------------------------------------------------- gate/up
// A workgroup item is a group of 4/wpt consecutive 16-row tiles of one active expert's
// w1/w3; each tile is streamed by `wpt` waves that split H (wpt = 1: one wave streams
// the whole row tile and no reduction is needed).  After a fixed-order reduction of the
// K slices, the tile's rows of
//   h[off_e + r][row] = bf16( bf16(silu(bf16(g))) * bf16(u) )
// are written for the expert's rows r, in token tiles of 16*MT.
template <int MT, int U, int D>
__global__ void __launch_bounds__(kFfnThreads, 2)
gateup_kernel(const ExpertTable tab, const uint16_t *__restrict__ x, int H, int F, Route rt,
              uint16_t *__restrict__ h_ws, int wpt) {
  __shared__ __attribute__((aligned(16))) uint32_t s_tbl[kTableWords];
  __shared__ f32x4 s_red[kFfnWaves][2][MT][kWave];
  __shared__ uint32_t s_raw[32];
  __shared__ float s_code[32];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid >> 6;
  const int n = lane & 15;
  const int g = lane >> 4;
  const int NB = H >> 6;
  const int tpw = kFfnWaves / wpt;
  const int groups_e = (F >> 4) / tpw;
  const int n_groups = rt.active[0] * groups_e;
  const int ks = wave % wpt;
  const int b_lo = NB * ks / wpt;
  const int b_hi = NB * (ks + 1) / wpt;
  const uint32_t lc1 = (uint32_t)(lane & 31) << 2;
  const uint32_t lane_const[2] = {lc1, lc1 | 128u};
  bool built = false;

  for (int grp = blockIdx.x; grp < n_groups; grp += gridDim.x) {
    const int e = rt.active[1 + grp / groups_e];
    const moe_nf4_expert_t &ex = tab.e[e];
    if (ex.w1_packed == nullptr) continue;  // absent expert (uniform across the workgroup)
    ensure_table(s_tbl, s_raw, s_code, (const float *)ex.w1_code, (const float *)ex.w3_code,
                 built);

    const int row0 = ((grp % groups_e) * tpw + wave / wpt) << 4;
    const int cnt = rt.counts[e];
    const int off = rt.offsets[e];
    const size_t roff = (size_t)(row0 + n);
    const uint8_t *const wq[2] = {(const uint8_t *)ex.w1_packed + roff * (H >> 1) + g * 8,
                                  (const uint8_t *)ex.w3_packed + roff * (H >> 1) + g * 8};
    const float *const wa[2] = {(const float *)ex.w1_absmax + roff * NB,
                                (const float *)ex.w3_absmax + roff * NB};

    for (int tt = 0; tt < cnt; tt += 16 * MT) {
      const uint16_t *xr[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int r = tt + mt * 16 + n;
        const int tok = rt.perm_tok[off + (r < cnt ? r : 0)];
        xr[mt] = x + (size_t)tok * H + g * 16;
      }
      f32x4 acc[2][MT];
#pragma unroll
      for (int p = 0; p < 2; ++p)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[p][mt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

      stream_blocks<2, MT, U, D>(s_tbl, wq, wa, xr, lane_const, b_lo, b_hi, acc);

      if (wpt > 1) {
        if (ks > 0) {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            s_red[wave][0][mt][lane] = acc[0][mt];
            s_red[wave][1][mt][lane] = acc[1][mt];
          }
        }
        __syncthreads();
        if (ks == 0) {
          for (int w = 1; w < wpt; ++w) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
              const f32x4 gp = s_red[wave + w][0][mt][lane];
              const f32x4 up = s_red[wave + w][1][mt][lane];
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                acc[0][mt][i] += gp[i];
                acc[1][mt][i] += up[i];
              }
            }
          }
        }
      }
      if (ks == 0) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int r = tt + mt * 16 + g * 4 + i;
            if (r < cnt) {
              const float gb = bf16_to_f32(f32_to_bf16(acc[0][mt][i]));
              const float ub = bf16_to_f32(f32_to_bf16(acc[1][mt][i]));
              const float sb = bf16_to_f32(f32_to_bf16(silu_f32(gb)));
              h_ws[(size_t)(off + r) * F + row0 + n] = f32_to_bf16(sb * ub);
            }
          }
        }
      }
      if (wpt > 1) __syncthreads();
    }
  }
}

// ----------------------------------------------------------------------------- down
// A workgroup item is (active expert, group of 4/wpt consecutive 16-row tiles of w2,
// split sp of nsplit).  Each tile's K range (split sp) is streamed by `wpt` waves and
// reduced in LDS in a fixed order; the result is written as the fp32 partial sum
//   ypart[sp][off_e + r][row] = sum_{k in split sp} w2[row][k] * h[off_e + r][k].
template <int MT, int U, int D>
__global__ void __launch_bounds__(kFfnThreads, 2)
down_kernel(const ExpertTable tab, int H, int F, Route rt, const uint16_t *__restrict__ h_ws,
            float *__restrict__ ypart, int64_t rows_total, int nsplit, int wpt) {
  __shared__ __attribute__((aligned(16))) uint32_t s_tbl[kTableWords];
  __shared__ f32x4 s_red[kFfnWaves][MT][kWave];
  __shared__ uint32_t s_raw[32];
  __shared__ float s_code[32];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid >> 6;
  const int n = lane & 15;
  const int g = lane >> 4;
  const int NB = F >> 6;
  const int tpw = kFfnWaves / wpt;
  const int groups_e = (H >> 4) / tpw * nsplit;
  const int n_groups = rt.active[0] * groups_e;
  const int ks = wave % wpt;
  const uint32_t lane_const[1] = {(uint32_t)lane << 2};
  bool built = false;

  for (int grp = blockIdx.x; grp < n_groups; grp += gridDim.x) {
    const int e = rt.active[1 + grp / groups_e];
    const moe_nf4_expert_t &ex = tab.e[e];
    if (ex.w2_packed == nullptr) continue;  // absent expert (uniform across the workgroup)
    ensure_table(s_tbl, s_raw, s_code, (const float *)ex.w2_code, (const float *)ex.w2_code,
                 built);
    const int rem = grp % groups_e;
    const int sp = rem % nsplit;
    const int row0 = ((rem / nsplit) * tpw + wave / wpt) << 4;
    const int slice = sp * wpt + ks;
    const int nslice = nsplit * wpt;
    const int b_lo = NB * slice / nslice;
    const int b_hi = NB * (slice + 1) / nslice;
    const int cnt = rt.counts[e];
    const int off = rt.offsets[e];
    const size_t roff = (size_t)(row0 + n);
    const uint8_t *const wq[1] = {(const uint8_t *)ex.w2_packed + roff * (F >> 1) + g * 8};
    const float *const wa[1] = {(const float *)ex.w2_absmax + roff * NB};

    for (int tt = 0; tt < cnt; tt += 16 * MT) {
      const uint16_t *hr[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int r = tt + mt * 16 + n;
        hr[mt] = h_ws + (size_t)(off + (r < cnt ? r : 0)) * F + g * 16;
      }
      f32x4 acc[1][MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[0][mt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

      stream_blocks<1, MT, U, D>(s_tbl, wq, wa, hr, lane_const, b_lo, b_hi, acc);

      if (wpt > 1) {
        if (ks > 0) {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) s_red[wave][mt][lane] = acc[0][mt];
        }
        __syncthreads();
        if (ks == 0) {
          for (int w = 1; w < wpt; ++w) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
              const f32x4 yp = s_red[wave + w][mt][lane];
#pragma unroll
              for (int i = 0; i < 4; ++i) acc[0][mt][i] += yp[i];
            }
          }
        }
      }
      if (ks == 0) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int r = tt + mt * 16 + g * 4 + i;
            if (r < cnt) ypart[((size_t)sp * rows_total + off + r) * H + row0 + n] = acc[0][mt][i];
          }
        }
      }
      if (wpt > 1) __syncthreads();
    }
  }
}

// ----------------------------------------------------------------------------- combine
// Workgroup (t, c) combines columns [256c, 256c + 256) of token t; each thread owns 4
// consecutive columns.  One wave per workgroup: a 40-token layer then has 640 workgroups,
// enough loads in flight for the K-split planes' few megabytes.
constexpr int kCombineThreads = 64;
constexpr int kCombineCols = kCombineThreads * 4;

__global__ void __launch_bounds__(kCombineThreads)
combine_kernel(const float *__restrict__ ypart, int nsplit, int64_t rows_total,
               const float *__restrict__ wts, const int32_t *__restrict__ idx,
               const int32_t *__restrict__ slot_pos, int k, int H, uint16_t *__restrict__ out) {
  const int64_t t = blockIdx.x;
  const int c = blockIdx.y * kCombineCols + threadIdx.x * 4;
  if (c >= H) return;
  int ord[MOE_MAX_TOPK];
  int e_of[MOE_MAX_TOPK];
  for (int j = 0; j < k; ++j) {
    ord[j] = j;
    e_of[j] = idx[t * k + j];
  }
  // Ascending expert id (insertion sort; k is tiny).
  for (int j = 1; j < k; ++j) {
    const int cur = ord[j];
    int p = j - 1;
    while (p >= 0 && e_of[ord[p]] > e_of[cur]) {
      ord[p + 1] = ord[p];
      --p;
    }
    ord[p + 1] = cur;
  }
  const size_t split_stride = (size_t)rows_total * H;
  float o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int jj = 0; jj < k; ++jj) {
    const int j = ord[jj];
    const int pos = slot_pos[t * k + j];
    if (pos < 0 || pos >= rows_total) continue;
    const float w = wts[t * k + j];
    float4 y = *reinterpret_cast<const float4 *>(ypart + (size_t)pos * H + c);
#pragma unroll 4
    for (int s = 1; s < nsplit; ++s) {
      const float4 v = *reinterpret_cast<const float4 *>(ypart + s * split_stride + (size_t)pos * H + c);
      y.x += v.x;
      y.y += v.y;
      y.z += v.z;
      y.w += v.w;
    }
    const float yv[4] = {y.x, y.y, y.z, y.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float p = bf16_to_f32(f32_to_bf16(yv[i])) * w;  // bf16 expert output x fp32 weight
      o[i] = bf16_to_f32(f32_to_bf16(o[i] + p));            // bf16 destination
    }
  }
  *reinterpret_cast<uint2 *>(out + t * H + c) = make_uint2(pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3]));
}

// Single-expert helpers: identity routing tables and the split reduction.
__global__ void identity_route_kernel(int64_t T, int32_t *counts, int32_t *offsets,
                                      int32_t *perm_tok, int32_t *active) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < T) perm_tok[i] = (int32_t)i;
  if (i == 0) {
    counts[0] = (int32_t)T;
    offsets[0] = 0;
    offsets[1] = (int32_t)T;
    active[0] = T > 0 ? 1 : 0;
    active[1] = 0;
  }
}

__global__ void reduce_splits_kernel(const float *__restrict__ ypart, int nsplit, int64_t numel,
                                     uint16_t *__restrict__ y) {
  const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (i >= numel) return;
  float4 acc = *reinterpret_cast<const float4 *>(ypart + i);
  for (int s = 1; s < nsplit; ++s) {
    const float4 v = *reinterpret_cast<const float4 *>(ypart + (size_t)s * numel + i);
    acc.x += v.x;
    acc.y += v.y;
    acc.z += v.z;
    acc.w += v.w;
  }
  *reinterpret_cast<uint2 *>(y + i) = make_uint2(pack_bf16x2(acc.x, acc.y), pack_bf16x2(acc.z, acc.w));
}

// ----------------------------------------------------------------------------- host side
// An entry whose nine pointers are all null is an absent expert: the kernels skip any
// work item that names it (the caller must not route tokens to it).
int check_expert(const moe_nf4_expert_t &ex, int e) {
  if (!ex.w1_packed && !ex.w1_absmax && !ex.w1_code && !ex.w3_packed && !ex.w3_absmax &&
      !ex.w3_code && !ex.w2_packed && !ex.w2_absmax && !ex.w2_code)
    return MOE_STATUS_OK;
  MOE_REQUIRE(ex.w1_packed && ex.w1_absmax && ex.w1_code && ex.w3_packed && ex.w3_absmax &&
                  ex.w3_code && ex.w2_packed && ex.w2_absmax && ex.w2_code,
              "expert %d has a null pointer", e);
  MOE_REQUIRE(((uintptr_t)ex.w1_packed % 8) == 0 && ((uintptr_t)ex.w3_packed % 8) == 0 &&
                  ((uintptr_t)ex.w2_packed % 8) == 0,
              "expert %d: packed weights must be 8-byte aligned", e);
  MOE_REQUIRE(((uintptr_t)ex.w1_absmax % 4) == 0 && ((uintptr_t)ex.w3_absmax % 4) == 0 &&
                  ((uintptr_t)ex.w2_absmax % 4) == 0,
              "expert %d: absmax must be 4-byte aligned", e);
  return MOE_STATUS_OK;
}

int token_tiles_for(int64_t max_tokens_per_expert) { return max_tokens_per_expert <= 16 ? 1 : 2; }

}  // namespace

// Default number of cross-workgroup K splits of the down projection.  Inside a workgroup
// four waves already split each w2 tile's K range, which fills the chip at batch 1, so a
// single split (no partial sums to add in the combine) is the default.

bool gemv4_supported(int64_t max_tokens_per_expert, int32_t H, int32_t F);
bool expert_gemm_supported(int32_t H, int32_t F);
bool expert_gemm_splits_ok(int32_t F, int32_t nsplit);
bool expert_gemm_rows_ok(int64_t T, int64_t rows_total, int32_t H, int32_t F);
int expert_gemm_splits(int64_t rows, int64_t active, int32_t H, int32_t F);
int launch_expert_gemm(const void *tab, const void *x, int64_t T, int64_t rows_total,
                       int64_t active_max, int32_t H, int32_t F, const void *route, void *h_ws,
                       void *ypart, int32_t nsplit, int phases, hipStream_t stream);
// Average routed rows per expert from which a layer uses the batched GEMM.
constexpr int64_t kGemmMinRowsPerExpert = 32;

int launch_gemv4(const void *tab, const void *x, int32_t H, int32_t F, const void *route,
                 void *h_ws, void *ypart, int phases, int64_t active_max, int64_t rows_total,
                 const void *fused_combine, hipStream_t stream);
bool skinny_supported(int32_t H, int32_t F);
int launch_skinny(const void *tab, const void *x, int64_t T, int64_t rows_total, int32_t H,
                  int32_t F, const void *route, void *h_ws, void *ypart, int phases,
                  hipStream_t stream);
bool midbatch_supported(int32_t H, int32_t F, int32_t nsplit);
bool midbatch_rows_ok(int64_t T, int64_t rows_total, int32_t H, int32_t F);
int midbatch_splits(int64_t active_max, int32_t H, int32_t F);
int launch_midbatch(const void *tab, const void *x, int64_t T, int64_t rows_total, int32_t H,
                    int32_t F, const void *route, void *h_ws, void *ypart, int32_t nsplit,
                    int phases, hipStream_t stream);
bool mid_gateup_supported(int64_t T, int32_t k, int32_t E, int32_t H, int32_t F);
bool mid_down_supported(int64_t T, int32_t k, int32_t E, int32_t H, int32_t F);
int mid_down_parts(int32_t F);
int launch_mid_down(const void *tab, const void *h, int64_t T, int32_t k, int32_t H, int32_t F,
                    int32_t E, const void *route, void *ypart, int32_t parts, hipStream_t s);
int launch_mid_gateup(const void *tab, const void *x, int64_t T, int32_t k, int32_t H, int32_t F,
                      int32_t E, const void *route, void *h_ws, hipStream_t s,
                      const void *route_out);

// ypart planes a layer's down projection writes (the combine adds them): the streamed
// mid-batch kernels split K of the down projection over workgroups when few experts would
// leave CUs idle; every other path writes one plane.  Follows the path choice of
// launch_expert_ffn for a layer (T tokens, k slots, E experts).
int choose_nsplit(int64_t T, int32_t k, int32_t E, int32_t H, int32_t F) {
  const int64_t rows = T * k;
  const int64_t active_max = rows < E ? rows : E;
  if (T <= 0 || gemv4_supported(T, H, F)) return 1;
  if (mid_down_supported(T, k, E, H, F)) return mid_down_parts(F);
  if (rows >= kGemmMinRowsPerExpert * active_max && expert_gemm_supported(H, F) &&
      expert_gemm_rows_ok(T, rows, H, F))
    return expert_gemm_splits(rows, active_max, H, F);
  if (!midbatch_supported(H, F, 1) || !midbatch_rows_ok(T, rows, H, F)) return 1;
  return midbatch_splits(active_max, H, F);
}

bool mid_layer_supported(int64_t T, int32_t k, int32_t E, int32_t H, int32_t F);

// Gate/up of a mid-size layer with the routing and grouping in the same launch (every
// workgroup of launch_mid_gateup routing the tokens itself) or, with a null gate, only the
// grouping of a separate router launch's slots (idx32); route_out (a MidRouteOut) names the
// gate, the bias and the routing outputs, which workgroup 0 writes for the down projection
// and the combine.
int launch_mid_layer_gateup(const moe_nf4_expert_t *experts, int32_t E, const void *x, int64_t T,
                            int32_t k, int32_t H, int32_t F, void *h_ws, const void *route_out,
                            hipStream_t stream) {
  MOE_REQUIRE(E >= 1 && E <= MOE_MAX_EXPERTS, "num_experts must be in [1, %d]", MOE_MAX_EXPERTS);
  MOE_REQUIRE(experts && x && h_ws && route_out, "null pointer");
  MOE_REQUIRE(((uintptr_t)h_ws % 16) == 0, "h workspace must be 16-byte aligned");
  ExpertTable tab;
  for (int e = 0; e < MOE_MAX_EXPERTS; ++e) {
    if (e < E) {
      const int rc = check_expert(experts[e], e);
      if (rc != MOE_STATUS_OK) return rc;
      tab.e[e] = experts[e];
    } else {
      tab.e[e] = moe_nf4_expert_t{};
    }
  }
  return launch_mid_gateup(&tab, x, T, k, H, F, E, nullptr, h_ws, stream, route_out);
}

// phases: bit 0 = gate/up (x -> h), bit 1 = down (h -> ypart).  Up to 4 tokens per expert
// use the 4x4x4 MFMA GEMV (expert_gemv4.hip); more use the 16x16x32 tiles below.
int launch_expert_ffn(const moe_nf4_expert_t *experts, int32_t E, const void *x, int64_t T,
                      int32_t k, int32_t H, int32_t F, const int32_t *counts,
                      const int32_t *offsets, const int32_t *perm_tok, const int32_t *active,
                      void *h_ws, void *ypart, int32_t nsplit, int64_t max_tokens_per_expert,
                      int phases, hipStream_t stream, const FusedCombine *fused) {
  MOE_REQUIRE(E >= 1 && E <= MOE_MAX_EXPERTS, "num_experts must be in [1, %d]", MOE_MAX_EXPERTS);
  MOE_REQUIRE(H > 0 && H % 256 == 0, "hidden size must be a positive multiple of 256 (got %d)", H);
  MOE_REQUIRE(F > 0 && F % 256 == 0, "FFN size must be a positive multiple of 256 (got %d)", F);
  MOE_REQUIRE(nsplit >= 1 && nsplit <= 16, "nsplit must be in [1, 16]");
  MOE_REQUIRE(k >= 1 && k <= MOE_MAX_TOPK, "top-k must be in [1, %d]", MOE_MAX_TOPK);
  MOE_REQUIRE(T >= 0 && T * k <= 0x7fffffff, "T out of range");
  if (T == 0) return MOE_STATUS_OK;
  MOE_REQUIRE(experts && counts && offsets && perm_tok && active && h_ws, "null pointer");
  MOE_REQUIRE(!(phases & 1) || x != nullptr, "null activations");
  MOE_REQUIRE(!(phases & 2) || ypart != nullptr, "null ypart");
  MOE_REQUIRE(((uintptr_t)x % 16) == 0 && ((uintptr_t)h_ws % 16) == 0 &&
                  ((uintptr_t)ypart % 16) == 0,
              "x, h workspace and ypart must be 16-byte aligned");
  ExpertTable tab;
  for (int e = 0; e < MOE_MAX_EXPERTS; ++e) {
    if (e < E) {
      const int rc = check_expert(experts[e], e);
      if (rc != MOE_STATUS_OK) return rc;
      tab.e[e] = experts[e];
    } else {
      tab.e[e] = moe_nf4_expert_t{};
    }
  }
  const Route rt{counts, offsets, perm_tok, active};
  const int64_t rows_total = T * k;
  const int64_t active_max = rows_total < E ? rows_total : E;
  const int64_t wg_cap = (int64_t)device_cu_count() * 2;
  const int mt = token_tiles_for(max_tokens_per_expert);

  if (nsplit == 1 && gemv4_supported(max_tokens_per_expert, H, F))
    return launch_gemv4(&tab, x, H, F, &rt, h_ws, ypart, phases, active_max, rows_total, fused,
                        stream);
  // Mid-size batches (up to 64 tokens): gate/up on 16-row weight tiles of "virtual experts"
  // (<= 16 token rows of one expert) with each wave's K slice of the tokens in registers
  // (decode_layer.hip); the down projection takes the path chosen below.
  if ((phases & 1) && fused == nullptr && mid_gateup_supported(T, k, E, H, F)) {
    const int rc = launch_mid_gateup(&tab, x, T, k, H, F, E, &rt, h_ws, stream, nullptr);
    if (rc != MOE_STATUS_OK || !(phases & 2)) return rc;
    phases &= ~1;
  }
  // Its down projection: the same virtual experts over parts of 2048 values of F, when the
  // caller's plane count is that part count.
  if ((phases & 2) && fused == nullptr && mid_down_supported(T, k, E, H, F) &&
      nsplit == mid_down_parts(F))
    return launch_mid_down(&tab, h_ws, T, k, H, F, E, &rt, ypart, nsplit, stream);
  // Many tokens per expert on average: the LDS-staged GEMM streams each weight tile once per
  // 128 tokens (the per-tile kernels below re-stream it every 16 or 32 tokens).
  if (fused == nullptr && rows_total >= kGemmMinRowsPerExpert * active_max &&
      expert_gemm_supported(H, F) && expert_gemm_splits_ok(F, nsplit) &&
      expert_gemm_rows_ok(T, rows_total, H, F))
    return launch_expert_gemm(&tab, x, T, rows_total, active_max, H, F, &rt, h_ws, ypart, nsplit,
                              phases, stream);
  // Fewer: the mid-batch kernels stream each weight tile once per 32 tokens of its expert
  // (32x32x16 MFMA, 16-byte weight loads): the streamed form (whole-K waves, activations
  // through LDS, `nsplit` K splits of the down projection) where the shape allows, else the
  // K-split form with activations from L2.
  if (fused == nullptr && midbatch_supported(H, F, nsplit) && midbatch_rows_ok(T, rows_total, H, F))
    return launch_midbatch(&tab, x, T, rows_total, H, F, &rt, h_ws, ypart, nsplit, phases, stream);
  if (nsplit == 1 && fused == nullptr && skinny_supported(H, F) && rows_total <= 2048 &&
      T * (int64_t)H * 2 < ((int64_t)1 << 31) && rows_total * (int64_t)F * 2 < ((int64_t)1 << 31))
    return launch_skinny(&tab, x, T, rows_total, H, F, &rt, h_ws, ypart, phases, stream);
  MOE_REQUIRE(fused == nullptr, "a fused combine needs the small-batch GEMV path");
  const int wpt_gu = 1;  // a wave streams a whole w1/w3 row tile
  const int wpt_dn = 4;  // four waves split each w2 row tile's K range
  int64_t g1 = active_max * (F / 16) / (kFfnWaves / wpt_gu);
  if (g1 > wg_cap) g1 = wg_cap;
  int64_t g2 = active_max * (H / 16) / (kFfnWaves / wpt_dn) * nsplit;
  if (g2 > wg_cap) g2 = wg_cap;
  const dim3 blk(kFfnThreads);
  if (phases & 1) {
    if (mt == 1)
      hipLaunchKernelGGL((gateup_kernel<1, 2, 4>), dim3((unsigned)g1), blk, 0, stream, tab,
                         (const uint16_t *)x, H, F, rt, (uint16_t *)h_ws, wpt_gu);
    else
      hipLaunchKernelGGL((gateup_kernel<2, 2, 2>), dim3((unsigned)g1), blk, 0, stream, tab,
                         (const uint16_t *)x, H, F, rt, (uint16_t *)h_ws, wpt_gu);
    MOE_LAUNCH_CHECK();
  }
  if (phases & 2) {
    if (mt == 1)
      hipLaunchKernelGGL((down_kernel<1, 2, 4>), dim3((unsigned)g2), blk, 0, stream, tab, H, F,
                         rt, (const uint16_t *)h_ws, (float *)ypart, rows_total, nsplit, wpt_dn);
    else
      hipLaunchKernelGGL((down_kernel<2, 2, 3>), dim3((unsigned)g2), blk, 0, stream, tab, H, F,
                         rt, (const uint16_t *)h_ws, (float *)ypart, rows_total, nsplit, wpt_dn);
    MOE_LAUNCH_CHECK();
  }
  return MOE_STATUS_OK;
}

int launch_combine(const void *ypart, int32_t nsplit, const void *weights, const void *idx_i32,
                   const void *slot_pos, int64_t T, int32_t k, int32_t H, void *out,
                   hipStream_t stream) {
  MOE_REQUIRE(T >= 0 && T <= 0x7fffffff, "T out of range");
  MOE_REQUIRE(k >= 1 && k <= MOE_MAX_TOPK, "top-k must be in [1, %d]", MOE_MAX_TOPK);
  MOE_REQUIRE(H > 0 && H % 4 == 0, "hidden size must be a positive multiple of 4");
  MOE_REQUIRE(nsplit >= 1 && nsplit <= 16, "nsplit must be in [1, 16]");
  if (T == 0) return MOE_STATUS_OK;
  MOE_REQUIRE(ypart && weights && idx_i32 && slot_pos && out, "null device pointer");
  MOE_REQUIRE(((uintptr_t)ypart % 16) == 0 && ((uintptr_t)out % 8) == 0,
              "ypart must be 16-byte and out 8-byte aligned");
  const unsigned cgrid = (unsigned)((H + kCombineCols - 1) / kCombineCols);
  hipLaunchKernelGGL(combine_kernel, dim3((unsigned)T, cgrid), dim3(kCombineThreads), 0, stream,
                     (const float *)ypart, nsplit, T * k, (const float *)weights,
                     (const int32_t *)idx_i32, (const int32_t *)slot_pos, k, H, (uint16_t *)out);
  MOE_LAUNCH_CHECK();
  return MOE_STATUS_OK;
}

int launch_identity_route(int64_t T, int32_t *counts, int32_t *offsets, int32_t *perm_tok,
                          int32_t *active, hipStream_t stream) {
  const int64_t blocks = T > 0 ? (T + 255) / 256 : 1;
  hipLaunchKernelGGL(identity_route_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, T,
                     counts, offsets, perm_tok, active);
  MOE_LAUNCH_CHECK();
  return MOE_STATUS_OK;
}

int launch_reduce_splits(const float *ypart, int nsplit, int64_t numel, uint16_t *y,
                         hipStream_t stream) {
  if (numel == 0) return MOE_STATUS_OK;
  const int64_t blocks = (numel / 4 + 255) / 256;
  hipLaunchKernelGGL(reduce_splits_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, ypart,
                     nsplit, numel, y);
  MOE_LAUNCH_CHECK();
  return MOE_STATUS_OK;
}

}  // namespace moe

extern "C" int moe_expert_ffn_nf4(const moe_nf4_expert_t *experts, int32_t E, const void *x_bf16,
                                  int64_t T, int32_t k, int32_t H, int32_t F, const void *counts,
                                  const void *offsets, const void *perm_tok, const void *active,
                                  void *h_ws_bf16, void *ypart_f32, int32_t nsplit, void *stream) {
  return moe::launch_expert_ffn(experts, E, x_bf16, T, k, H, F, (const int32_t *)counts,
                                (const int32_t *)offsets, (const int32_t *)perm_tok,
                                (const int32_t *)active, h_ws_bf16, ypart_f32, nsplit, T, 3,
                                (hipStream_t)stream, nullptr);
}

extern "C" int moe_expert_gateup_nf4(const moe_nf4_expert_t *experts, int32_t E,
                                     const void *x_bf16, int64_t T, int32_t k, int32_t H,
                                     int32_t F, const void *counts, const void *offsets,
                                     const void *perm_tok, const void *active, void *h_ws_bf16,
                                     void *stream) {
  return moe::launch_expert_ffn(experts, E, x_bf16, T, k, H, F, (const int32_t *)counts,
                                (const int32_t *)offsets, (const int32_t *)perm_tok,
                                (const int32_t *)active, h_ws_bf16, nullptr, 1, T, 1,
                                (hipStream_t)stream, nullptr);
}

extern "C" int moe_expert_down_nf4(const moe_nf4_expert_t *experts, int32_t E, int64_t T,
                                   int32_t k, int32_t H, int32_t F, const void *counts,
                                   const void *offsets, const void *perm_tok, const void *active,
                                   const void *h_ws_bf16, void *ypart_f32, int32_t nsplit,
                                   void *stream) {
  return moe::launch_expert_ffn(experts, E, nullptr, T, k, H, F, (const int32_t *)counts,
                                (const int32_t *)offsets, (const int32_t *)perm_tok,
                                (const int32_t *)active, const_cast<void *>(h_ws_bf16),
                                ypart_f32, nsplit, T, 2, (hipStream_t)stream, nullptr);
}

extern "C" int moe_combine(const void *ypart_f32, int32_t nsplit, const void *weights_f32,
                           const void *idx_i32, const void *slot_pos, int64_t T, int32_t k,
                           int32_t H, void *out_bf16, void *stream) {
  return moe::launch_combine(ypart_f32, nsplit, weights_f32, idx_i32, slot_pos, T, k, H, out_bf16,
                             (hipStream_t)stream);
}
