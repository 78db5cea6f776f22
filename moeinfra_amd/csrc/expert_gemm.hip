// K4 for batches: grouped NF4 GEMM on the 16x16x32 bf16 MFMA with the activations staged
// in LDS, for many tokens per expert (prefill).
//
//   gate/up:  h[off_e + r][f] = bf16(bf16(silu(bf16(w1_e x_t))) * bf16(w3_e x_t))[f]
//   down:     ypart[off_e + r][c] = sum_f w2_e[c][f] * h[off_e + r][f]        (fp32)
// for the rows r of every active expert e (token t = perm_tok[off_e + r]), the semantics of
// ReconstructedNF4Expert.forward (transfer/nf4_reconstruct.py:152-155) applied to the rows
// model/moe_layer.py:174-186 gathers.
//
// Tiling.  A workgroup item is (active expert, 128-row token tile, weight tile): 8 waves,
// each owning 16 weight rows of NP = 2 B streams (gate/up: w1 and w3 rows; down: two
// 16-row tiles of w2, 128 rows apart), for all 128 tokens of the tile (eight 16-token
// MFMA tiles).  The K loop runs over 64-value NF4 blocks:
//  * the token tile's 128 x 64 activations are loaded cooperatively (one 16-byte load per
//    thread and half block), two blocks ahead, and staged in LDS (double buffer, 128-byte
//    rows whose 16-byte chunks are XOR-swizzled by the row, see a_swizzle);
//  * each lane's 8 packed bytes per stream and block come from a register ring 8 blocks
//    deep (the HBM latency), and are turned into bf16 operands by the 64 KB LDS table;
//  * per 16-token tile and stream, two MFMAs (K = 32 each) produce the block's partial
//    product, scaled by the row's absmax into the fp32 accumulator.
// The K order inside a block is the one of the per-expert kernels (expert_ffn.hip): lane
// (n, g) holds values 16g..16g+7 for the first MFMA and 16g+8..16g+15 for the second, for
// the weights (B, column n) and the activations (A, row n) alike.
#include "nf4_tile.h"

namespace moe {
namespace {

constexpr int kGemmWaves = 8;
constexpr int kGemmThreads = kGemmWaves * kWave;
constexpr int kGemmM = 128;             // tokens per item
constexpr int kGemmMT = kGemmM / 16;    // 16-token MFMA tiles per item
constexpr int kARowHalves = 64;         // LDS row stride of the activation tile, in bf16
constexpr int kGemmBDepth = 8;          // weight blocks in flight per wave
constexpr int kGemmADepth = 4;          // activation blocks in flight per thread
// The block loop is unrolled by kGemmBDepth from block 0, so b % kGemmADepth and b % 2 are
// those of the unrolled index: the activation registers and LDS buffers are then indexed
// statically (a dynamic index would make the compiler move the register array to LDS).
// Loads complete in issue order (vmcnt), so the wait for the activations of block b + 1
// also waits for every weight load issued before them: kGemmADepth - 1 blocks is the
// latency the loads of both operands get.
static_assert(kGemmBDepth % kGemmADepth == 0 && kGemmADepth % 2 == 0,
              "buffer indices must follow the unrolled index");

// Position of 16-byte chunk c (of 8) of activation-tile row r: c ^ a_swizzle(r & 15).
// gfx950 serves a 64-lane ds_read_b128 16 lanes per cycle, in the lane groups
// {0-3, 12-15, 20-27} and {4-11, 16-19, 28-31} (and the same + 32), over 64 four-byte
// banks.  The MFMA operand read has lane (n, g) fetch chunk 2g (then 2g + 1) of row n; with
// this swizzle the 16 lanes of every group cover 16 distinct (row parity, position) pairs,
// i.e. all 64 banks once.  The cooperative stores (8 lanes per cycle, one row) stay
// conflict-free for any swizzle.
__device__ __forceinline__ int a_swizzle(int r) { return ((r >> 1) & 3) | (((r + 4) >> 1) & 4); }

template <bool GATEUP>
__global__ void __launch_bounds__(kGemmThreads, 1)
expert_gemm_kernel(const ExpertTable tab, const uint16_t *__restrict__ act, int H, int F,
                   Route rt, uint16_t *__restrict__ h_out, float *__restrict__ y_out) {
  __shared__ __attribute__((aligned(16))) uint32_t s_tbl[kTableWords];
  __shared__ __attribute__((aligned(16))) uint16_t s_a[2][kGemmM * kARowHalves];
  __shared__ uint32_t s_raw[32];
  __shared__ float s_code[32];
  __shared__ int s_ex[MOE_MAX_EXPERTS][4];  // per active expert: id, rows, row offset, first item
  __shared__ int s_nitems;

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid >> 6;
  const int n = lane & 15;
  const int g = lane >> 4;
  const int K = GATEUP ? H : F;                  // reduction length
  const int NROWS = GATEUP ? F : H;              // weight rows (output columns)
  const int NB = K >> 6;                         // NF4 blocks per weight row
  const int WROWS = GATEUP ? 128 : 256;          // weight rows per item
  const int n_tiles = NROWS / WROWS;
  const uint32_t lc = (uint32_t)(lane & 31) << 2;
  // gate/up: replicas 0-31 hold w1's codebook, 32-63 w3's; down: both w2's.
  const uint32_t lane_const[2] = {lc, lc | 128u};
  bool built = false;

  // Items: for each active expert (ascending), its token tiles x weight tiles, the token
  // tile fastest so that concurrent items share weight tiles in L2.  Wave 0 stages the
  // active experts' ids, row counts, row offsets and first item indices in LDS once, so
  // that decoding an item is one LDS read and a ballot instead of a chain of global loads.
  static_assert(MOE_MAX_EXPERTS <= kWave, "one lane per active expert");
  const int n_active = rt.active[0];
  if (n_active == 0) return;  // uniform over the grid, before any barrier
  if (wave == 0) {
    int e = 0, cnt = 0, items = 0;
    if (lane < n_active) {
      e = rt.active[1 + lane];
      // An absent expert (all-null table entry) has no items.
      cnt = (GATEUP ? tab.e[e].w1_packed : tab.e[e].w2_packed) != nullptr ? rt.counts[e] : 0;
      items = ((cnt + kGemmM - 1) / kGemmM) * n_tiles;
    }
    int incl = items;  // inclusive prefix sum over the lanes
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
    }
    if (lane == kWave - 1) s_nitems = incl;
  }
  // Codebooks: when every active expert holds the codebooks of the first one (the usual
  // case: one NF4 codebook for all tensors), the table is built once for the launch;
  // otherwise it is checked per item.
  // The first present active expert supplies the reference codebooks; with none present
  // there is no item (uniform over the grid, before any barrier).
  int e0 = -1;
  for (int a = 0; a < n_active && e0 < 0; ++a) {
    const int e = rt.active[1 + a];
    if ((GATEUP ? tab.e[e].w1_packed : tab.e[e].w2_packed) != nullptr) e0 = e;
  }
  if (e0 < 0) return;
  int cb_diff = 0;
  {
    const float *lo0 = (const float *)(GATEUP ? tab.e[e0].w1_code : tab.e[e0].w2_code);
    const float *hi0 = (const float *)(GATEUP ? tab.e[e0].w3_code : tab.e[e0].w2_code);
    for (int i = tid; i < n_active * 32; i += kGemmThreads) {
      const int e = rt.active[1 + (i >> 5)], j = i & 15;
      if ((GATEUP ? tab.e[e].w1_packed : tab.e[e].w2_packed) == nullptr) continue;
      const float *lo = (const float *)(GATEUP ? tab.e[e].w1_code : tab.e[e].w2_code);
      const float *hi = (const float *)(GATEUP ? tab.e[e].w3_code : tab.e[e].w2_code);
      const float *x = (i & 16) ? hi : lo;
      const float *x0 = (i & 16) ? hi0 : lo0;
      cb_diff |= __builtin_bit_cast(uint32_t, x[j]) != __builtin_bit_cast(uint32_t, x0[j]);
    }
  }
  const bool per_item_table = __syncthreads_or(cb_diff) != 0;  // also publishes s_ex
  if (!per_item_table) {
    const moe_nf4_expert_t &ex0 = tab.e[e0];
    if (GATEUP)
      ensure_table<kGemmThreads>(s_tbl, s_raw, s_code, (const float *)ex0.w1_code, (const float *)ex0.w3_code, built);
    else
      ensure_table<kGemmThreads>(s_tbl, s_raw, s_code, (const float *)ex0.w2_code, (const float *)ex0.w2_code, built);
  }
  const int n_items = s_nitems;

  for (int item = blockIdx.x; item < n_items; item += gridDim.x) {
    // The item's expert: the last active expert whose first item is <= item.
    const int a = __popcll(__ballot(lane < n_active && s_ex[lane < n_active ? lane : 0][3] <= item)) - 1;
    const int e = s_ex[a][0], cnt = s_ex[a][1], off = s_ex[a][2];
    const int rem = item - s_ex[a][3];
    const int mtiles = (cnt + kGemmM - 1) / kGemmM;
    const int nt = rem / mtiles;
    const int mt_i = rem - nt * mtiles;
    const int m_base = mt_i * kGemmM;
    const moe_nf4_expert_t &ex = tab.e[e];
    if (per_item_table) {
      if (GATEUP)
        ensure_table<kGemmThreads>(s_tbl, s_raw, s_code, (const float *)ex.w1_code, (const float *)ex.w3_code, built);
      else
        ensure_table<kGemmThreads>(s_tbl, s_raw, s_code, (const float *)ex.w2_code, (const float *)ex.w2_code, built);
    }

    // Weight streams of this lane: row (row0 + n) of each stream.
    const int row0 = nt * WROWS + 16 * wave;
    const uint8_t *wq[2];
    const float *wa[2];
    if (GATEUP) {
      const size_t r = (size_t)(row0 + n);
      wq[0] = (const uint8_t *)ex.w1_packed + r * (K >> 1) + 8 * g;
      wq[1] = (const uint8_t *)ex.w3_packed + r * (K >> 1) + 8 * g;
      wa[0] = (const float *)ex.w1_absmax + r * NB;
      wa[1] = (const float *)ex.w3_absmax + r * NB;
    } else {
      const size_t r0 = (size_t)(row0 + n), r1 = r0 + 128;
      wq[0] = (const uint8_t *)ex.w2_packed + r0 * (K >> 1) + 8 * g;
      wq[1] = (const uint8_t *)ex.w2_packed + r1 * (K >> 1) + 8 * g;
      wa[0] = (const float *)ex.w2_absmax + r0 * NB;
      wa[1] = (const float *)ex.w2_absmax + r1 * NB;
    }
    // Activation loads of this thread: token-tile rows ar0 and ar0 + 64, 16 bytes at
    // half-block byte offset 16 * ac (one load per row and block).
    const int ac = tid & 7;
    const int ar0 = tid >> 3;  // 0..63
    const uint16_t *asrc[2];
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
      const int r = m_base + ar0 + 64 * h2;
      const int rr = r < cnt ? r : cnt - 1;  // rows past the expert's last repeat it (unused)
      const size_t src_row = GATEUP ? (size_t)rt.perm_tok[off + rr] : (size_t)(off + rr);
      asrc[h2] = act + src_row * K + 8 * ac;
    }

    // Rows ar0 and ar0 + 64 share the swizzle (64 is a multiple of 16).
    const int a_st = ar0 * kARowHalves + 8 * (ac ^ a_swizzle(ar0));
    u32x4 abuf[kGemmADepth][2];
    auto load_a = [&](u32x4 (&dst)[2], int b) {
      const int bb = b < NB ? b : NB - 1;  // past the end: the last block again (unused)
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2)
        dst[h2] = *reinterpret_cast<const u32x4 *>(asrc[h2] + (size_t)bb * 64);
    };
    auto store_a = [&](const u32x4 (&src)[2], int buf) {
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2)
        *reinterpret_cast<u32x4 *>(&s_a[buf][a_st + 64 * h2 * kARowHalves]) = src[h2];
    };
    // Operand reads of lane (n, g): chunks 2g and 2g + 1 of row n (+ 16 m).
    const int a_rd0 = n * kARowHalves + 8 * ((2 * g) ^ a_swizzle(n));
    const int a_rd1 = n * kARowHalves + 8 * ((2 * g + 1) ^ a_swizzle(n));
    uint2 bq[kGemmBDepth][2];
    auto load_b = [&](int slot, int b) {
      const int bb = b < NB ? b : NB - 1;
#pragma unroll
      for (int p = 0; p < 2; ++p) bq[slot][p] = *reinterpret_cast<const uint2 *>(wq[p] + (size_t)bb * 32);
    };
    // Absmax of blocks 4j..4j+3 as one 16-byte load per stream (rows hold NB % 4 == 0
    // values), two groups of four in registers: group j lives in slot j % 2.
    f32x4 bs4[2][2];
    auto load_s = [&](int slot, int b4) {
      const int bb = b4 < NB ? b4 : NB - 4;
#pragma unroll
      for (int p = 0; p < 2; ++p) bs4[slot][p] = *reinterpret_cast<const f32x4 *>(wa[p] + bb);
    };

    f32x4 acc[2][kGemmMT];
#pragma unroll
    for (int p = 0; p < 2; ++p)
#pragma unroll
      for (int m = 0; m < kGemmMT; ++m) acc[p][m] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // Prologue: activation block 0 to LDS, blocks 1..DA-1 in registers, weight blocks
    // 0..DB-2.
#pragma unroll
    for (int d = 0; d < kGemmADepth; ++d) load_a(abuf[d], d);
#pragma unroll
    for (int d = 0; d < kGemmBDepth - 1; ++d) load_b(d, d);
    load_s(0, 0);
    load_s(1, 4);
    store_a(abuf[0], 0);
    __syncthreads();

    for (int b0 = 0; b0 < NB; b0 += kGemmBDepth) {
#pragma unroll
      for (int d = 0; d < kGemmBDepth; ++d) {
        const int b = b0 + d;
        if (b < NB) {
          load_b((d + kGemmBDepth - 1) % kGemmBDepth, b + kGemmBDepth - 1);
          // Once the blocks of a group are done (block b = 4j + 4 starts), group j + 2
          // replaces it: four blocks ahead of its first use.
          if (d % 4 == 0 && b >= 4) load_s((d / 4 + 1) % 2, b + 4);
          load_a(abuf[d % kGemmADepth], b + kGemmADepth);  // block b's were stored at b-1
          const uint16_t *sa = s_a[d & 1];
          bf16x8 w0[2], w1[2];
#pragma unroll
          for (int p = 0; p < 2; ++p) {
            uint32_t l[8];
            lookup8(s_tbl, bq[d][p], lane_const[p], l);
            w0[p] = as_bf16x8(l[0], l[1], l[2], l[3]);
            w1[p] = as_bf16x8(l[4], l[5], l[6], l[7]);
          }
#pragma unroll
          for (int m = 0; m < kGemmMT; ++m) {
            const bf16x8 a0 = as_bf16x8(*reinterpret_cast<const u32x4 *>(sa + m * 16 * kARowHalves + a_rd0));
            const bf16x8 a1 = as_bf16x8(*reinterpret_cast<const u32x4 *>(sa + m * 16 * kARowHalves + a_rd1));
#pragma unroll
            for (int p = 0; p < 2; ++p) scale_acc(acc[p][m], mfma_block(a0, w0[p], a1, w1[p]), bs4[(d / 4) % 2][p][d % 4]);
          }
          // Block b+1's activations (loaded at block b+1-DA) to the other buffer.
          store_a(abuf[(d + 1) % kGemmADepth], (d + 1) & 1);
          __syncthreads();
        }
      }
    }

    // Epilogue: lane (n, g) holds rows 4g+i of each 16-token tile, column n of its streams.
#pragma unroll
    for (int m = 0; m < kGemmMT; ++m) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = m_base + m * 16 + 4 * g + i;
        if (r < cnt) {
          if (GATEUP) {
            h_out[(size_t)(off + r) * F + row0 + n] = swiglu_bf16(acc[0][m][i], acc[1][m][i]);
          } else {
            float *yrow = y_out + (size_t)(off + r) * H;
            yrow[row0 + n] = acc[0][m][i];
            yrow[row0 + 128 + n] = acc[1][m][i];
          }
        }
      }
    }
  }
}

}  // namespace

// The batched form of K4: gate/up (phases bit 0) and/or down (bit 1) with the LDS-staged
// GEMM.  Needs H % 256 == 0 (down tiles of 256 rows) and F % 256 == 0 (gate/up tiles of 128
// rows; absmax rows of a multiple of 4 blocks); writes ypart as one split.
bool expert_gemm_supported(int32_t H, int32_t F) { return H % 256 == 0 && F % 256 == 0; }

int launch_expert_gemm(const void *tab_v, const void *x, int32_t H, int32_t F, const void *route_v,
                       void *h_ws, void *ypart, int phases, hipStream_t stream) {
  MOE_REQUIRE(expert_gemm_supported(H, F), "shape not supported by the batched expert GEMM");
  const ExpertTable &tab = *static_cast<const ExpertTable *>(tab_v);
  const Route &rt = *static_cast<const Route *>(route_v);
  const dim3 grid((unsigned)device_cu_count()), blk(kGemmThreads);
  if (phases & 1) {
    hipLaunchKernelGGL(expert_gemm_kernel<true>, grid, blk, 0, stream, tab, (const uint16_t *)x, H,
                       F, rt, (uint16_t *)h_ws, (float *)nullptr);
    MOE_LAUNCH_CHECK();
  }
  if (phases & 2) {
    hipLaunchKernelGGL(expert_gemm_kernel<false>, grid, blk, 0, stream, tab, (const uint16_t *)h_ws,
                       H, F, rt, (uint16_t *)nullptr, (float *)ypart);
    MOE_LAUNCH_CHECK();
  }
  return MOE_STATUS_OK;
}

}  // namespace moe
