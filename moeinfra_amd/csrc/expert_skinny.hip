// K4 for mid-size batches: the grouped NF4 SwiGLU expert FFN on v_mfma_f32_32x32x16_bf16,
// for a few to a few tens of tokens per expert, where the layer is bound by streaming the
// NF4 weights (every weight tile is read once per 32-token chunk of its expert).
//
//   gate/up:  h[off_e + r][f] = bf16(bf16(silu(bf16(w1_e x_t))) * bf16(w3_e x_t))[f]
//   down:     ypart[off_e + r][c] = sum_f w2_e[c][f] * h[off_e + r][f]        (fp32)
// for the rows r of every active expert e (token t = perm_tok[off_e + r]): the semantics
// of ReconstructedNF4Expert.forward (transfer/nf4_reconstruct.py:152-155) applied to the
// rows model/moe_layer.py:174-186 gathers.
//
// Tiling.  A workgroup item is (active expert, 32-row weight tile, 32-token chunk).  The
// workgroup's 8 waves split the reduction dimension: wave w streams NF4 blocks
// [w*NB/8, (w+1)*NB/8) of the tile's rows (NP = 2 streams for gate/up, w1 and w3; one for
// down, w2), and the waves' partial sums meet in LDS at the end of the item.
//
// MFMA layout.  In v_mfma_f32_32x32x16_bf16 lane l = 32*kg + i supplies B[k 8kg..8kg+7]
// [n = i] and A[m = i][k 8kg..8kg+7], and holds D[m][n = i] for m = 8*(v/4) + 4*kg + v%4
// in its register v.  The weights are B (n = weight row), the tokens A (m = token row).
// For NF4 block b a lane loads the 16 packed bytes 16*kg .. 16*kg+15 of its row's block,
// i.e. values 32*kg .. 32*kg+31, which are the K slices of four MFMAs (MFMA q takes values
// 32*kg + 8q .. +7); the lane's A operand is the same 32 values of its token (64 bytes).
// Every MFMA thus stays inside one 64-value block, and the block's absmax (one per lane:
// the lane's row) scales the MFMA result into the lane's 16 fp32 accumulators.  One load
// instruction reads 32 rows x 32 contiguous bytes at 16 bytes per lane, which streams as
// fast as whole-row loads on MI355X (16 bytes per lane is what matters; 8-byte lanes cap
// near 4.5 TB/s).
//
// Activations are read through a buffer descriptor bounded by the activation tensor: the
// lanes of token rows past the chunk's last row use an offset beyond the bound and receive
// zeros without a memory access.  The loads of a wave run kSkDepth blocks ahead of its
// MFMAs, across item boundaries (the next item's pointers are set up one item ahead).
#include "nf4_tile.h"

namespace moe {
namespace {

typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;

constexpr int kSkWaves = 8;
constexpr int kSkThreads = kSkWaves * kWave;
constexpr int kSkRows = 32;   // weight rows per item (MFMA columns)
constexpr int kSkToks = 32;   // token rows per item (MFMA rows)
constexpr int kSkDepth = 4;   // NF4 blocks in flight per wave
// Buffer-load offset that lies past any activation tensor this path accepts (< 2^31 B).
constexpr uint32_t kSkOob = 0x80000000u;
// Routed rows (T * k) the gate/up kernel keeps in LDS (their token ids).
constexpr int kSkMaxRows = 2048;
// ABS: the tile's absmax (all rows, all blocks) is staged in LDS per item, double
// buffered, with an odd row stride; these bound the blocks per row it holds and give the
// 16-byte chunk loads per thread that fill one buffer.
template <int NP>
constexpr int kSkAbsMaxNB = NP == 2 ? 64 : 224;
template <int NP>
constexpr int kSkAbsLoads = (NP * kSkRows * kSkAbsMaxNB<NP> / 4 + kSkThreads - 1) / kSkThreads;


// LDS-only barrier: orders the workgroup's LDS accesses without waiting for the waves'
// outstanding global loads (a workgroup fence on all address spaces would drain them).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Orders LDS stores of some lanes of a wave before LDS loads of other lanes of the same
// wave (wavefront-scope fences around a wave barrier; no s_barrier).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Four packed bytes (values 2j, 2j+1 per byte, j = 0..3) -> eight bf16 code values.
__device__ __forceinline__ bf16x8 lookup4(const uint32_t *tbl, uint32_t w, uint32_t lane_const) {
  uint32_t l[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) l[j] = lds_lookup(tbl, __builtin_amdgcn_perm(w, lane_const, 0x0c0c0400u + (j << 8)));
  return as_bf16x8(l[0], l[1], l[2], l[3]);
}

// Global-memory pointer types: loads through them stay global loads (a generic pointer
// becomes a flat load, which also counts against the LDS wait counter and would make the
// table lookups wait for the weight stream).
#define SK_GLOBAL __attribute__((address_space(1)))
typedef const SK_GLOBAL uint8_t *sk_gq_t;
typedef const SK_GLOBAL float *sk_ga_t;

// An item's streams: wave-uniform bases (scalar registers) of the tile's first row, to
// which every lane adds a constant offset (its row and half block), and the lane's
// activation offset.
template <int NP>
struct SkPtr {
  sk_gq_t wb[NP];  // packed bytes of the tile's first row
  sk_ga_t ab[NP];  // absmax of the tile's first row
  uint32_t aoff;   // byte offset of the lane's activations of block 0 (or past the bound)
};

template <int NP>
struct SkStage {
  u32x4 w[NP];
  float s[NP];
  u32x4 a[4];
};

// Lookup table (see nf4_tile.h) from two codebooks held in LDS, by the whole workgroup,
// between LDS-only barriers (the waves' outstanding weight loads stay in flight).
__device__ __forceinline__ void rebuild_table(uint32_t *tbl, const float *code_lo, const float *code_hi) {
  lds_barrier();  // every wave is done with the previous table
  for (int i = threadIdx.x; i < kTableWords; i += kSkThreads) {
    const int v = i >> 6;                              // packed byte value
    const float *c = (i & 32) ? code_hi : code_lo;     // replicas 32-63 use the second codebook
    tbl[i] = pack_bf16x2(c[v >> 4], c[v & 15]);
  }
  lds_barrier();
}

// Absmax modes: per block (4-byte load per lane and block), per group (a 16-byte load of
// four blocks per lane and group of four, kept in registers), or staged (the whole tile's
// absmax in LDS per item, loaded with contiguous 16-byte chunks by the workgroup).
enum SkAbs { kAbsBlock = 0, kAbsGroup = 1, kAbsStaged = 2 };

template <int NP, int D, int AM>
__global__ void __launch_bounds__(kSkThreads, 1)
skinny_kernel(const ExpertTable tab, const uint16_t *__restrict__ act, uint32_t act_bytes, int K,
              int NROWS, Route rt, int rows_total, uint16_t *__restrict__ h_out,
              float *__restrict__ y_out) {
  constexpr bool GATEUP = NP == 2;
  static_assert(D == 2 || D == 4, "pipeline depth");
  constexpr bool ABS = AM == kAbsStaged;
  static_assert(AM == kAbsBlock || D == 4, "absmax groups are four blocks");
  // Staged absmax needs every wave to own at least one group (K / 256 >= 8 groups): the
  // tile is loaded in each wave's last group, and a wave without groups would take a
  // second code path whose loads make the compiler drain the other waves' pipelines.
  // Staged: absmax of the current and the next item's tile, [buffer][stream][row][block].
  __shared__ float s_absb[ABS ? 2 : 1][NP][kSkRows][ABS ? kSkAbsMaxNB<NP> + 1 : 1];
  __shared__ __attribute__((aligned(16))) uint32_t s_tbl[kTableWords];
  // Cross-wave partial sums of one 16-token half of an item (registers v of one half).
  __shared__ float s_red[kSkWaves][NP][8][kWave];

  // Codebooks of every active expert: [0,16) w1 (down: w2), [16,32) w3 (down: w2).
  __shared__ float s_codes[MOE_MAX_EXPERTS][32];
  // Per active expert: id, rows, row offset, first item, 32-token chunks.
  __shared__ int s_ex[MOE_MAX_EXPERTS][5];
  __shared__ int s_ptok[GATEUP ? kSkMaxRows : 1];
  __shared__ int s_nitems;

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li32 = lane & 31;
  const int kg = lane >> 5;
  const int NB = K >> 6;
  const int tiles = NROWS / kSkRows;
  const size_t row_bytes = (size_t)(K >> 1);
  static_assert(MOE_MAX_EXPERTS <= kWave, "one lane per active expert");

  const int n_active = rt.active[0];
  if (n_active == 0) return;  // uniform over the grid, before any barrier
  if (wave == 0) {
    int e = 0, cnt = 0, items = 0, nch = 0;
    if (lane < n_active) {
      e = rt.active[1 + lane];
      // An absent expert (null pointers) gets no items; the caller routes no token to it.
      cnt = tab.e[e].w1_packed != nullptr ? rt.counts[e] : 0;
      nch = (cnt + kSkToks - 1) / kSkToks;
      items = nch * tiles;
    }
    int incl = items;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
      const int v = __shfl_up(incl, o);
      if (lane >= o) incl += v;
    }
    if (lane < n_active) {
      s_ex[lane][0] = e;
      s_ex[lane][1] = cnt;
      s_ex[lane][2] = rt.offsets[e];
      s_ex[lane][3] = incl - items;
      s_ex[lane][4] = nch;
    }
    if (lane == kWave - 1) s_nitems = incl;
  }
  if (GATEUP)
    for (int i = tid; i < rows_total; i += kSkThreads) s_ptok[i] = rt.perm_tok[i];
  for (int i = tid; i < n_active * 32; i += kSkThreads) {
    const moe_nf4_expert_t &ex = tab.e[rt.active[1 + (i >> 5)]];
    const int j = i & 15;
    float c = 0.0f;
    if (ex.w1_packed != nullptr) {
      if (GATEUP)
        c = ((const float *)((i & 16) ? ex.w3_code : ex.w1_code))[j];
      else
        c = ((const float *)ex.w2_code)[j];
    }
    s_codes[i >> 5][i & 31] = c;
  }
  __syncthreads();
  // One table for the launch when every present active expert holds the same codebooks
  // (the usual case); otherwise the table is rebuilt where an item's expert changes.
  int cb_diff = 0;
  {
    int a0 = 0;
    while (a0 + 1 < n_active && s_ex[a0][1] == 0) ++a0;
    for (int i = tid; i < n_active * 32; i += kSkThreads)
      if (s_ex[i >> 5][1] > 0)
        cb_diff |= __builtin_bit_cast(uint32_t, s_codes[i >> 5][i & 31]) !=
                   __builtin_bit_cast(uint32_t, s_codes[a0][i & 31]);
  }
  const bool per_item_table = __syncthreads_or(cb_diff) != 0;
  const int n_items = s_nitems;
  const int lo = (int)((int64_t)blockIdx.x * n_items / gridDim.x);
  const int hi = (int)((int64_t)(blockIdx.x + 1) * n_items / gridDim.x);
  if (lo >= hi) return;  // uniform over the workgroup

  // Item -> (active index, tile, chunk); wave-uniform.
  // LDS values read at wave-uniform addresses, moved to scalar registers.
  auto ex_field = [&](int a, int f) { return __builtin_amdgcn_readfirstlane(s_ex[a][f]); };
  auto decode = [&](int item, int &a, int &tile, int &ch) {
    const int sel = lane < n_active ? lane : 0;
    a = __popcll(__ballot(lane < n_active && s_ex[sel][3] <= item)) - 1;
    const int rem = item - ex_field(a, 3);
    const int nch = ex_field(a, 4);
    tile = rem / nch;
    ch = rem - tile * nch;
  };
  int tbl_a;
  {
    int tile, ch;
    decode(lo, tbl_a, tile, ch);
  }
  rebuild_table(s_tbl, s_codes[tbl_a], s_codes[tbl_a] + 16);

  const uint32_t lc = (uint32_t)li32 << 2;
  uint32_t lane_const[NP];
  if constexpr (GATEUP) {  // replicas 0-31 hold w1's codebook, 32-63 w3's
    lane_const[0] = lc;
    lane_const[1] = lc | 128u;
  } else {  // both halves hold w2's: spread the lanes over all 64 replicas
    lane_const[0] = lc | (kg ? 128u : 0u);
  }
  const __amdgpu_buffer_rsrc_t rsrc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(act), (short)0, (int)act_bytes, 0x00020000);

  // This wave's share of K: whole groups of D blocks (waves may differ by one group, or
  // own none when K is short; every wave takes part in every item's reduction).
  const int ngroups = NB / D;
  const int g0 = wave * ngroups / kSkWaves;
  const int ngrp = (wave + 1) * ngroups / kSkWaves - g0;
  const int k0 = g0 * D;
  const int bpw = ngrp * D;

  // Pointers of an item (LDS reads and address arithmetic only: no global load, so the
  // setup of the next item never waits on the weight loads in flight).
  auto set_ptrs = [&](SkPtr<NP> &P, int item) {
    int a, tile, ch;
    decode(item, a, tile, ch);
    const int e = ex_field(a, 0), cnt = ex_field(a, 1), off = ex_field(a, 2);
    const moe_nf4_expert_t &ex = tab.e[e];
    const size_t row0 = (size_t)tile * kSkRows;
    if constexpr (GATEUP) {
      P.wb[0] = (sk_gq_t)ex.w1_packed + row0 * row_bytes;
      P.wb[1] = (sk_gq_t)ex.w3_packed + row0 * row_bytes;
      P.ab[0] = (sk_ga_t)ex.w1_absmax + row0 * NB;
      P.ab[1] = (sk_ga_t)ex.w3_absmax + row0 * NB;
    } else {
      P.wb[0] = (sk_gq_t)ex.w2_packed + row0 * row_bytes;
      P.ab[0] = (sk_ga_t)ex.w2_absmax + row0 * NB;
    }
    const int r = ch * kSkToks + li32;
    uint32_t aoff = kSkOob;
    if (r < cnt) {
      const uint32_t arow = GATEUP ? (uint32_t)s_ptok[off + r] : (uint32_t)(off + r);
      aoff = (arow * (uint32_t)K + 32u * kg) * 2u;
    }
    P.aoff = aoff;
  };


  // Per-lane constant offsets: the lane's row and half block (bytes), its row's absmax.
  const uint32_t w_lane = (uint32_t)li32 * (uint32_t)row_bytes + 16u * kg;
  const uint32_t a_lane = (uint32_t)li32 * (uint32_t)NB;
  auto load = [&](SkStage<NP> &st, const SkPtr<NP> &Q, int b) {
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      st.w[p] = *reinterpret_cast<const SK_GLOBAL u32x4 *>(Q.wb[p] + (w_lane + (uint32_t)b * 32u));
      if (AM == kAbsBlock) st.s[p] = Q.ab[p][a_lane + (uint32_t)b];
    }
    const uint32_t ao = Q.aoff + (uint32_t)b * 128u;
#pragma unroll
    for (int q = 0; q < 4; ++q) st.a[q] = __builtin_amdgcn_raw_buffer_load_b128(rsrc, (int)(ao + 16u * q), 0, 0);
  };

  f32x16 acc[NP];
#pragma unroll
  for (int p = 0; p < NP; ++p)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[p][v] = 0.0f;

  // ABS: the tile's absmax, loaded by the whole workgroup as contiguous 16-byte chunks
  // (chunk c = (p * 32 + row) * NB/4 + j: blocks 4j .. 4j+3 of the row) and stored to one
  // of the two LDS buffers; `abuf` holds a thread's chunks between the two steps.
  const int nb4 = NB / 4;
  const int n_chunks = NP * kSkRows * nb4;
  f32x4 abuf[ABS ? kSkAbsLoads<NP> : 1];
  auto load_abs = [&](const SkPtr<NP> &Q) {
    if (ABS) {
#pragma unroll
      for (int i = 0; i < kSkAbsLoads<NP>; ++i) {
        int c = tid + kSkThreads * i;
        c = c < n_chunks ? c : n_chunks - 1;  // past the end: the last chunk again (unused)
        const int pr = c / nb4, j = c - pr * nb4;
        const sk_ga_t base = (NP == 2 && pr >= kSkRows) ? Q.ab[NP - 1] : Q.ab[0];
        abuf[i] = *reinterpret_cast<const SK_GLOBAL f32x4 *>(base + (uint32_t)((pr & (kSkRows - 1)) * NB + 4 * j));
      }
    }
  };
  auto store_abs = [&](int buf) {
    if (ABS) {
#pragma unroll
      for (int i = 0; i < kSkAbsLoads<NP>; ++i) {
        const int c = tid + kSkThreads * i;
        if (c < n_chunks) {
          const int pr = c / nb4, j = c - pr * nb4;
          float *dst = &s_absb[buf][pr >> 5][pr & (kSkRows - 1)][4 * j];
          dst[0] = abuf[i][0];
          dst[1] = abuf[i][1];
          dst[2] = abuf[i][2];
          dst[3] = abuf[i][3];
        }
      }
    }
  };
  int abuf_cur = 0;  // LDS buffer of the current item's absmax
  // Per group: the absmax of the group being consumed (ga_cur) and of the next one
  // (ga_nxt): 16 bytes of the lane's row of stream kg (NP = 2: lanes 32-63 hold w3's, the
  // other stream's value comes from lane l ^ 32) or of w2 (NP = 1).
  f32x4 ga_cur = {0.0f, 0.0f, 0.0f, 0.0f}, ga_nxt = ga_cur;
  auto load_ga = [&](const SkPtr<NP> &Q, int b) {
    if (AM == kAbsGroup) {
      const sk_ga_t base = (NP == 2 && kg) ? Q.ab[NP - 1] : Q.ab[0];
      ga_nxt = *reinterpret_cast<const SK_GLOBAL f32x4 *>(base + (a_lane + (uint32_t)b));
    }
  };
  auto compute = [&](const SkStage<NP> &st, int b) {
    float scl[NP];
    if (AM == kAbsGroup) {
      const float own = ga_cur[b & 3];
      if constexpr (NP == 2) {
        const float other = __shfl_xor(own, 32, kWave);
        scl[0] = kg ? other : own;
        scl[NP - 1] = kg ? own : other;
      } else {
        scl[0] = own;
      }
    } else {
#pragma unroll
      for (int p = 0; p < NP; ++p) scl[p] = ABS ? s_absb[abuf_cur][ABS ? p : 0][li32][ABS ? b : 0] : st.s[p];
    }
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      f32x16 t;
#pragma unroll
      for (int v = 0; v < 16; ++v) t[v] = 0.0f;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        t = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(st.a[q]), lookup4(s_tbl, st.w[p][q], lane_const[p]),
                                                     t, 0, 0, 0);
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[p][v] = fmaf(scl[p], t[v], acc[p][v]);
    }
  };

  // End of an item: the waves' partial sums meet in LDS (fixed wave order), and the
  // workgroup writes the item's output rows.
  auto finish = [&](int item) {
    int a, tile, ch;
    decode(item, a, tile, ch);
    const int cnt = s_ex[a][1], off = s_ex[a][2];
    const int nrow = min(kSkToks, cnt - ch * kSkToks);
#pragma unroll
    for (int h = 0; h < 2; ++h) {  // registers 8h .. 8h+7 hold token rows 16h .. 16h+15
      if (16 * h >= nrow) break;
      lds_barrier();  // the previous reads of s_red are done
#pragma unroll
      for (int v = 0; v < 8; ++v) {
        if (16 * h + 8 * (v >> 2) < nrow) {
#pragma unroll
          for (int p = 0; p < NP; ++p) s_red[wave][p][v][lane] = acc[p][8 * h + v];
        }
      }
      lds_barrier();
      {
        const int v = tid >> 6, l = tid & (kWave - 1);  // one entry per thread
        const int m = 16 * h + 8 * (v >> 2) + 4 * (l >> 5) + (v & 3);
        if (m < nrow) {
          float sum[NP];
#pragma unroll
          for (int p = 0; p < NP; ++p) {
            float sm = s_red[0][p][v][l];
#pragma unroll
            for (int w = 1; w < kSkWaves; ++w) sm += s_red[w][p][v][l];
            sum[p] = sm;
          }
          const size_t orow = (size_t)(off + ch * kSkToks + m);
          const int col = tile * kSkRows + (l & 31);
          if constexpr (GATEUP)
            h_out[orow * NROWS + col] = swiglu_bf16(sum[0], sum[1]);
          else
            y_out[orow * NROWS + col] = sum[0];
        }
      }
    }
  };

  // Stream: per item, ngrp groups of D blocks.  Every step loads the block D - 1 ahead of
  // the one it consumes; in the item's last group the loads move on to the next item's
  // first blocks (or, after the last item, re-read this item's last block, unused), chosen
  // by selects so that no branch surrounds a load.
  SkPtr<NP> P, Pn;
  set_ptrs(P, lo);
  Pn = P;
  if (lo + 1 < hi) set_ptrs(Pn, lo + 1);
  // Field-wise choice between two items' pointers (wave-uniform condition).
  auto pick = [&](bool c, const SkPtr<NP> &X, const SkPtr<NP> &Y) {
    SkPtr<NP> R;
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      R.wb[p] = c ? X.wb[p] : Y.wb[p];
      R.ab[p] = c ? X.ab[p] : Y.ab[p];
    }
    R.aoff = c ? X.aoff : Y.aoff;
    return R;
  };
  SkStage<NP> st[D];
  load_abs(P);
  store_abs(0);
  if (ABS) lds_barrier();  // the first item's absmax is visible to every wave
  if (ngrp > 0) {
    load_ga(P, k0);
    ga_cur = ga_nxt;
#pragma unroll
    for (int d = 0; d < D - 1; ++d) {
      load(st[d], P, k0 + d);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  for (int item = lo; item < hi; ++item) {
    const bool has_next = item + 1 < hi;
    for (int g = 0; g + 1 < ngrp; ++g) {
#pragma unroll
      for (int d = 0; d < D; ++d) {
        const int b = k0 + g * D + d + D - 1;
        if (d == 1) load_ga(P, b);  // the next group starts at the block loaded now
        load(st[(d + D - 1) % D], P, b);
        __builtin_amdgcn_sched_barrier(0);
        compute(st[d], k0 + g * D + d);
      }
      ga_cur = ga_nxt;
    }
    if (ngrp > 0) {
#pragma unroll
      for (int d = 0; d < D; ++d) {
        const SkPtr<NP> Q = pick(has_next, Pn, P);
        if (d == 0) {
          load_abs(Q);  // the next item's absmax, ahead of its first blocks
          load(st[D - 1], P, k0 + bpw - 1);
        } else {
          if (d == 1) load_ga(Q, has_next ? k0 : k0 + bpw - D);
          load(st[d - 1], Q, has_next ? k0 + d - 1 : k0 + bpw - 1);
        }
        __builtin_amdgcn_sched_barrier(0);
        compute(st[d], k0 + bpw - D + d);
      }
      ga_cur = ga_nxt;
      // Straight-line code after the loads: the wait for the absmax leaves the next
      // item's blocks in flight.  The other buffer was last read by the previous item.
      store_abs(abuf_cur ^ 1);
    }
    finish(item);  // its barriers also publish the next item's absmax
    abuf_cur ^= 1;
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[p][v] = 0.0f;
    if (has_next) {
      P = Pn;
      if (item + 2 < hi) set_ptrs(Pn, item + 2);
      if (per_item_table) {
        int a, tile, ch;
        decode(item + 1, a, tile, ch);
        if (a != tbl_a) {
          tbl_a = a;
          rebuild_table(s_tbl, s_codes[a], s_codes[a] + 16);
        }
      }
    }
  }
}

}  // namespace

// Shapes of the mid-batch path: 32-row tiles of every projection, at least one 64-value
// block per wave along K, and activation tensors addressable by a buffer descriptor.
bool skinny_supported(int32_t H, int32_t F) {
  return H % 128 == 0 && F % 128 == 0 && H >= 128 && F >= 128;
}

int launch_skinny(const void *tab_v, const void *x, int64_t T, int64_t rows_total, int32_t H,
                  int32_t F, const void *route_v, void *h_ws, void *ypart, int phases,
                  hipStream_t stream) {
  MOE_REQUIRE(skinny_supported(H, F), "shape not supported by the mid-batch expert kernels");
  MOE_REQUIRE(T * (int64_t)H * 2 < ((int64_t)1 << 31) && rows_total * (int64_t)F * 2 < ((int64_t)1 << 31) &&
                  rows_total <= kSkMaxRows,
              "activations too large for the mid-batch expert kernels");
  const ExpertTable &tab = *static_cast<const ExpertTable *>(tab_v);
  const Route &rt = *static_cast<const Route *>(route_v);
  const dim3 grid((unsigned)device_cu_count()), blk(kSkThreads);
  // Pipeline depth: 4 blocks when K splits into groups of four (Mixtral: 64 and 224
  // blocks), else 2.
  // Gate/up (two streams, at the register limit) loads absmax per group; down stages the
  // tile's absmax in LDS when a row's blocks fit.
  if (phases & 1) {
    const uint32_t xb = (uint32_t)(T * H * 2);
    if ((H / 64) % 4 == 0)
      hipLaunchKernelGGL((skinny_kernel<2, 4, kAbsGroup>), grid, blk, 0, stream, tab, (const uint16_t *)x, xb,
                         H, F, rt, (int)rows_total, (uint16_t *)h_ws, (float *)nullptr);
    else
      hipLaunchKernelGGL((skinny_kernel<2, 2, kAbsBlock>), grid, blk, 0, stream, tab, (const uint16_t *)x, xb,
                         H, F, rt, (int)rows_total, (uint16_t *)h_ws, (float *)nullptr);
    MOE_LAUNCH_CHECK();
  }
  if (phases & 2) {
    const uint32_t hb = (uint32_t)(rows_total * F * 2);
    if ((F / 64) % 4 == 0 && F / 64 <= kSkAbsMaxNB<1> && F / 256 >= kSkWaves)
      hipLaunchKernelGGL((skinny_kernel<1, 4, kAbsStaged>), grid, blk, 0, stream, tab, (const uint16_t *)h_ws,
                         hb, F, H, rt, (int)rows_total, (uint16_t *)nullptr, (float *)ypart);
    else if ((F / 64) % 4 == 0)
      hipLaunchKernelGGL((skinny_kernel<1, 4, kAbsGroup>), grid, blk, 0, stream, tab, (const uint16_t *)h_ws,
                         hb, F, H, rt, (int)rows_total, (uint16_t *)nullptr, (float *)ypart);
    else
      hipLaunchKernelGGL((skinny_kernel<1, 2, kAbsBlock>), grid, blk, 0, stream, tab, (const uint16_t *)h_ws,
                         hb, F, H, rt, (int)rows_total, (uint16_t *)nullptr, (float *)ypart);
    MOE_LAUNCH_CHECK();
  }
  return MOE_STATUS_OK;
}

}  // namespace moe
