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
#include "common.h"

namespace moe {
namespace {

constexpr int kFfnWaves = 4;
constexpr int kFfnThreads = kFfnWaves * kWave;
constexpr int kTableWords = 256 * 64;

struct ExpertTable {
  moe_nf4_expert_t e[MOE_MAX_EXPERTS];
};

struct Route {
  const int32_t *counts;
  const int32_t *offsets;
  const int32_t *perm_tok;
  const int32_t *active;
};

__device__ __forceinline__ bf16x8 as_bf16x8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  return __builtin_bit_cast(bf16x8, make_uint4(a, b, c, d));
}
__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

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
// the resident ones.  Must be called by every thread of the workgroup; acts as a barrier.
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
    for (int i = tid; i < kTableWords; i += kFfnThreads) {
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

// ----------------------------------------------------------------------------- gate/up
// Work item = (active expert, 16-row tile of w1/w3).  The four waves split H; the
// workgroup reduces the four partial sums in LDS in a fixed order and writes
//   h[off_e + r][row] = bf16( bf16(silu(bf16(g))) * bf16(u) )
// for the expert's rows r, in token tiles of 16*MT.
template <int MT, int U>
__global__ void __launch_bounds__(kFfnThreads, 2)
gateup_kernel(const ExpertTable tab, const uint16_t *__restrict__ x, int H, int F, Route rt,
              uint16_t *__restrict__ h_ws) {
  __shared__ __attribute__((aligned(16))) uint32_t s_tbl[kTableWords];
  __shared__ f32x4 s_red[kFfnWaves - 1][2][MT][kWave];
  __shared__ uint32_t s_raw[32];
  __shared__ float s_code[32];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid >> 6;
  const int n = lane & 15;
  const int g = lane >> 4;
  const int tiles = F >> 4;
  const int NB = H >> 6;
  const int b_lo = NB * wave / kFfnWaves;
  const int b_hi = NB * (wave + 1) / kFfnWaves;
  const uint32_t lane1 = (uint32_t)(lane & 31) << 2;
  const uint32_t lane3 = lane1 | 128u;
  const int n_items = rt.active[0] * tiles;
  bool built = false;

  for (int item = blockIdx.x; item < n_items; item += gridDim.x) {
    const int e = rt.active[1 + item / tiles];
    const int row0 = (item % tiles) << 4;
    const moe_nf4_expert_t &ex = tab.e[e];
    if (ex.w1_packed == nullptr) continue;  // absent expert (uniform across the workgroup)
    ensure_table(s_tbl, s_raw, s_code, (const float *)ex.w1_code, (const float *)ex.w3_code,
                 built);

    const int cnt = rt.counts[e];
    const int off = rt.offsets[e];
    const uint8_t *w1 = (const uint8_t *)ex.w1_packed + (size_t)(row0 + n) * (H >> 1) + g * 8;
    const uint8_t *w3 = (const uint8_t *)ex.w3_packed + (size_t)(row0 + n) * (H >> 1) + g * 8;
    const float *a1 = (const float *)ex.w1_absmax + (size_t)(row0 + n) * NB;
    const float *a3 = (const float *)ex.w3_absmax + (size_t)(row0 + n) * NB;

    for (int tt = 0; tt < cnt; tt += 16 * MT) {
      const uint16_t *xr[MT];
      bool ok[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int r = tt + mt * 16 + n;
        ok[mt] = r < cnt;
        const int tok = ok[mt] ? rt.perm_tok[off + r] : 0;
        xr[mt] = x + (size_t)tok * H + g * 16;
      }
      f32x4 acc1[MT], acc3[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        acc1[mt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        acc3[mt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      }

      int b = b_lo;
      for (; b + U <= b_hi; b += U) {
        uint2 q1[U], q3[U];
        float s1[U], s3[U];
        uint4 xa[U][MT][2];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          q1[u] = *reinterpret_cast<const uint2 *>(w1 + (size_t)(b + u) * 32);
          q3[u] = *reinterpret_cast<const uint2 *>(w3 + (size_t)(b + u) * 32);
          s1[u] = a1[b + u];
          s3[u] = a3[b + u];
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            if (ok[mt]) {
              const uint4 *p = reinterpret_cast<const uint4 *>(xr[mt] + (b + u) * 64);
              xa[u][mt][0] = p[0];
              xa[u][mt][1] = p[1];
            } else {
              xa[u][mt][0] = make_uint4(0, 0, 0, 0);
              xa[u][mt][1] = make_uint4(0, 0, 0, 0);
            }
          }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          uint32_t l1[8], l3[8];
          lookup8(s_tbl, q1[u], lane1, l1);
          lookup8(s_tbl, q3[u], lane3, l3);
          const bf16x8 b1a = as_bf16x8(l1[0], l1[1], l1[2], l1[3]);
          const bf16x8 b1b = as_bf16x8(l1[4], l1[5], l1[6], l1[7]);
          const bf16x8 b3a = as_bf16x8(l3[0], l3[1], l3[2], l3[3]);
          const bf16x8 b3b = as_bf16x8(l3[4], l3[5], l3[6], l3[7]);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            const bf16x8 x0 = as_bf16x8(xa[u][mt][0]);
            const bf16x8 x1 = as_bf16x8(xa[u][mt][1]);
            scale_acc(acc1[mt], mfma_block(x0, b1a, x1, b1b), s1[u]);
            scale_acc(acc3[mt], mfma_block(x0, b3a, x1, b3b), s3[u]);
          }
        }
      }
      for (; b < b_hi; ++b) {
        const uint2 q1 = *reinterpret_cast<const uint2 *>(w1 + (size_t)b * 32);
        const uint2 q3 = *reinterpret_cast<const uint2 *>(w3 + (size_t)b * 32);
        uint32_t l1[8], l3[8];
        lookup8(s_tbl, q1, lane1, l1);
        lookup8(s_tbl, q3, lane3, l3);
        const bf16x8 b1a = as_bf16x8(l1[0], l1[1], l1[2], l1[3]);
        const bf16x8 b1b = as_bf16x8(l1[4], l1[5], l1[6], l1[7]);
        const bf16x8 b3a = as_bf16x8(l3[0], l3[1], l3[2], l3[3]);
        const bf16x8 b3b = as_bf16x8(l3[4], l3[5], l3[6], l3[7]);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          uint4 xa0 = make_uint4(0, 0, 0, 0), xa1 = make_uint4(0, 0, 0, 0);
          if (ok[mt]) {
            const uint4 *p = reinterpret_cast<const uint4 *>(xr[mt] + b * 64);
            xa0 = p[0];
            xa1 = p[1];
          }
          scale_acc(acc1[mt], mfma_block(as_bf16x8(xa0), b1a, as_bf16x8(xa1), b1b), a1[b]);
          scale_acc(acc3[mt], mfma_block(as_bf16x8(xa0), b3a, as_bf16x8(xa1), b3b), a3[b]);
        }
      }

      // Fixed-order reduction of the four K slices, then the SwiGLU epilogue.
      if (wave > 0) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          s_red[wave - 1][0][mt][lane] = acc1[mt];
          s_red[wave - 1][1][mt][lane] = acc3[mt];
        }
      }
      __syncthreads();
      if (wave == 0) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          f32x4 gs = acc1[mt], us = acc3[mt];
#pragma unroll
          for (int w = 0; w < kFfnWaves - 1; ++w) {
            const f32x4 gp = s_red[w][0][mt][lane];
            const f32x4 up = s_red[w][1][mt][lane];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              gs[i] += gp[i];
              us[i] += up[i];
            }
          }
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int r = tt + mt * 16 + g * 4 + i;
            if (r < cnt) {
              const float gb = bf16_to_f32(f32_to_bf16(gs[i]));
              const float ub = bf16_to_f32(f32_to_bf16(us[i]));
              const float sb = bf16_to_f32(f32_to_bf16(silu_f32(gb)));
              h_ws[(size_t)(off + r) * F + row0 + n] = f32_to_bf16(sb * ub);
            }
          }
        }
      }
      __syncthreads();
    }
  }
}

// ----------------------------------------------------------------------------- down
// Work item = (active expert, 16-row tile of w2, K slice).  Writes the fp32 partial
//   ypart[ks][off_e + r][row] = sum over the slice of w2[row][k] * h[off_e + r][k].
template <int MT, int U>
__global__ void __launch_bounds__(kFfnThreads, 2)
down_kernel(const ExpertTable tab, int H, int F, Route rt, const uint16_t *__restrict__ h_ws,
            float *__restrict__ ypart, int64_t rows_total, int nsplit) {
  __shared__ __attribute__((aligned(16))) uint32_t s_tbl[kTableWords];
  __shared__ f32x4 s_red[kFfnWaves - 1][MT][kWave];
  __shared__ uint32_t s_raw[32];
  __shared__ float s_code[32];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid >> 6;
  const int n = lane & 15;
  const int g = lane >> 4;
  const int tiles = H >> 4;
  const int NB = F >> 6;
  const uint32_t lane2 = (uint32_t)lane << 2;
  const int per_expert = tiles * nsplit;
  const int n_items = rt.active[0] * per_expert;
  bool built = false;

  for (int item = blockIdx.x; item < n_items; item += gridDim.x) {
    const int e = rt.active[1 + item / per_expert];
    const int rem = item % per_expert;
    const int row0 = (rem / nsplit) << 4;
    const int ks = rem % nsplit;
    const moe_nf4_expert_t &ex = tab.e[e];
    if (ex.w2_packed == nullptr) continue;  // absent expert (uniform across the workgroup)
    ensure_table(s_tbl, s_raw, s_code, (const float *)ex.w2_code, (const float *)ex.w2_code,
                 built);

    const int kb0 = NB * ks / nsplit;
    const int kb1 = NB * (ks + 1) / nsplit;
    const int b_lo = kb0 + (kb1 - kb0) * wave / kFfnWaves;
    const int b_hi = kb0 + (kb1 - kb0) * (wave + 1) / kFfnWaves;
    const int cnt = rt.counts[e];
    const int off = rt.offsets[e];
    const uint8_t *w2 = (const uint8_t *)ex.w2_packed + (size_t)(row0 + n) * (F >> 1) + g * 8;
    const float *a2 = (const float *)ex.w2_absmax + (size_t)(row0 + n) * NB;

    for (int tt = 0; tt < cnt; tt += 16 * MT) {
      const uint16_t *hr[MT];
      bool ok[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int r = tt + mt * 16 + n;
        ok[mt] = r < cnt;
        hr[mt] = h_ws + (size_t)(off + (ok[mt] ? r : 0)) * F + g * 16;
      }
      f32x4 acc[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

      int b = b_lo;
      for (; b + U <= b_hi; b += U) {
        uint2 q[U];
        float s[U];
        uint4 xa[U][MT][2];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          q[u] = *reinterpret_cast<const uint2 *>(w2 + (size_t)(b + u) * 32);
          s[u] = a2[b + u];
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            if (ok[mt]) {
              const uint4 *p = reinterpret_cast<const uint4 *>(hr[mt] + (size_t)(b + u) * 64);
              xa[u][mt][0] = p[0];
              xa[u][mt][1] = p[1];
            } else {
              xa[u][mt][0] = make_uint4(0, 0, 0, 0);
              xa[u][mt][1] = make_uint4(0, 0, 0, 0);
            }
          }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          uint32_t l[8];
          lookup8(s_tbl, q[u], lane2, l);
          const bf16x8 ba = as_bf16x8(l[0], l[1], l[2], l[3]);
          const bf16x8 bb = as_bf16x8(l[4], l[5], l[6], l[7]);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
            scale_acc(acc[mt],
                      mfma_block(as_bf16x8(xa[u][mt][0]), ba, as_bf16x8(xa[u][mt][1]), bb), s[u]);
        }
      }
      for (; b < b_hi; ++b) {
        const uint2 q = *reinterpret_cast<const uint2 *>(w2 + (size_t)b * 32);
        uint32_t l[8];
        lookup8(s_tbl, q, lane2, l);
        const bf16x8 ba = as_bf16x8(l[0], l[1], l[2], l[3]);
        const bf16x8 bb = as_bf16x8(l[4], l[5], l[6], l[7]);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          uint4 xa0 = make_uint4(0, 0, 0, 0), xa1 = make_uint4(0, 0, 0, 0);
          if (ok[mt]) {
            const uint4 *p = reinterpret_cast<const uint4 *>(hr[mt] + (size_t)b * 64);
            xa0 = p[0];
            xa1 = p[1];
          }
          scale_acc(acc[mt], mfma_block(as_bf16x8(xa0), ba, as_bf16x8(xa1), bb), a2[b]);
        }
      }

      if (wave > 0) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) s_red[wave - 1][mt][lane] = acc[mt];
      }
      __syncthreads();
      if (wave == 0) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          f32x4 ys = acc[mt];
#pragma unroll
          for (int w = 0; w < kFfnWaves - 1; ++w) {
            const f32x4 yp = s_red[w][mt][lane];
#pragma unroll
            for (int i = 0; i < 4; ++i) ys[i] += yp[i];
          }
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int r = tt + mt * 16 + g * 4 + i;
            if (r < cnt) ypart[((size_t)ks * rows_total + off + r) * H + row0 + n] = ys[i];
          }
        }
      }
      __syncthreads();
    }
  }
}

// ----------------------------------------------------------------------------- combine
// One workgroup per token; each thread handles 4 consecutive columns per step.
constexpr int kCombineThreads = 256;

__global__ void __launch_bounds__(kCombineThreads)
combine_kernel(const float *__restrict__ ypart, int nsplit, int64_t rows_total,
               const float *__restrict__ wts, const int32_t *__restrict__ idx,
               const int32_t *__restrict__ slot_pos, int k, int H, uint16_t *__restrict__ out) {
  const int64_t t = blockIdx.x;
  int ord[MOE_MAX_TOPK];
  for (int j = 0; j < k; ++j) ord[j] = j;
  // Ascending expert id (insertion sort; k is tiny).
  for (int j = 1; j < k; ++j) {
    const int cur = ord[j];
    int p = j - 1;
    while (p >= 0 && idx[t * k + ord[p]] > idx[t * k + cur]) {
      ord[p + 1] = ord[p];
      --p;
    }
    ord[p + 1] = cur;
  }
  const size_t split_stride = (size_t)rows_total * H;
  for (int c = threadIdx.x * 4; c < H; c += kCombineThreads * 4) {
    float o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int jj = 0; jj < k; ++jj) {
      const int j = ord[jj];
      const int pos = slot_pos[t * k + j];
      if (pos < 0 || pos >= rows_total) continue;
      const float w = wts[t * k + j];
      float4 y = *reinterpret_cast<const float4 *>(ypart + (size_t)pos * H + c);
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

// Split of the down projection's K range so that small token counts still fill the chip.
int choose_nsplit(int64_t T, int32_t k, int32_t E, int32_t H) {
  const int64_t active_max = T * k < E ? T * k : E;
  const int64_t items = active_max * (H / 16);
  const int64_t target = 2048;
  int64_t s = items > 0 ? (target + items - 1) / items : 1;
  if (s < 1) s = 1;
  if (s > 8) s = 8;
  return (int)s;
}

int launch_expert_ffn(const moe_nf4_expert_t *experts, int32_t E, const void *x, int64_t T,
                      int32_t k, int32_t H, int32_t F, const int32_t *counts,
                      const int32_t *offsets, const int32_t *perm_tok, const int32_t *active,
                      void *h_ws, void *ypart, int32_t nsplit, int64_t max_tokens_per_expert,
                      hipStream_t stream) {
  MOE_REQUIRE(E >= 1 && E <= MOE_MAX_EXPERTS, "num_experts must be in [1, %d]", MOE_MAX_EXPERTS);
  MOE_REQUIRE(H > 0 && H % 256 == 0, "hidden size must be a positive multiple of 256 (got %d)", H);
  MOE_REQUIRE(F > 0 && F % 256 == 0, "FFN size must be a positive multiple of 256 (got %d)", F);
  MOE_REQUIRE(nsplit >= 1 && nsplit <= 16, "nsplit must be in [1, 16]");
  MOE_REQUIRE(T >= 0 && T * k <= 0x7fffffff, "T out of range");
  if (T == 0) return MOE_STATUS_OK;
  MOE_REQUIRE(experts && x && counts && offsets && perm_tok && active && h_ws && ypart,
              "null pointer");
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

  int64_t g1 = active_max * (F / 16);
  if (g1 > wg_cap) g1 = wg_cap;
  int64_t g2 = active_max * (H / 16) * nsplit;
  if (g2 > wg_cap) g2 = wg_cap;
  const dim3 blk(kFfnThreads);
  if (mt == 1) {
    hipLaunchKernelGGL((gateup_kernel<1, 4>), dim3((unsigned)g1), blk, 0, stream, tab,
                       (const uint16_t *)x, H, F, rt, (uint16_t *)h_ws);
    MOE_LAUNCH_CHECK();
    hipLaunchKernelGGL((down_kernel<1, 4>), dim3((unsigned)g2), blk, 0, stream, tab, H, F, rt,
                       (const uint16_t *)h_ws, (float *)ypart, rows_total, nsplit);
  } else {
    hipLaunchKernelGGL((gateup_kernel<2, 2>), dim3((unsigned)g1), blk, 0, stream, tab,
                       (const uint16_t *)x, H, F, rt, (uint16_t *)h_ws);
    MOE_LAUNCH_CHECK();
    hipLaunchKernelGGL((down_kernel<2, 2>), dim3((unsigned)g2), blk, 0, stream, tab, H, F, rt,
                       (const uint16_t *)h_ws, (float *)ypart, rows_total, nsplit);
  }
  MOE_LAUNCH_CHECK();
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
  hipLaunchKernelGGL(combine_kernel, dim3((unsigned)T), dim3(kCombineThreads), 0, stream,
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
  MOE_REQUIRE(k >= 1 && k <= MOE_MAX_TOPK, "top-k must be in [1, %d]", MOE_MAX_TOPK);
  return moe::launch_expert_ffn(experts, E, x_bf16, T, k, H, F, (const int32_t *)counts,
                                (const int32_t *)offsets, (const int32_t *)perm_tok,
                                (const int32_t *)active, h_ws_bf16, ypart_f32, nsplit, T,
                                (hipStream_t)stream);
}

extern "C" int moe_combine(const void *ypart_f32, int32_t nsplit, const void *weights_f32,
                           const void *idx_i32, const void *slot_pos, int64_t T, int32_t k,
                           int32_t H, void *out_bf16, void *stream) {
  return moe::launch_combine(ypart_f32, nsplit, weights_f32, idx_i32, slot_pos, T, k, H, out_bf16,
                             (hipStream_t)stream);
}
