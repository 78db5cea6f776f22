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
//    thread and half block), two blocks ahead, and staged in LDS (double buffer, rows padded
//    to 144 bytes so that the 16-byte reads of 8 lanes hit distinct banks);
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
constexpr int kARowHalves = 72;         // LDS row stride of the activation tile, in bf16
constexpr int kGemmBDepth = 8;          // weight blocks in flight per wave
constexpr int kGemmADepth = 2;          // activation blocks in flight per thread

template <bool GATEUP>
__global__ void __launch_bounds__(kGemmThreads, 1)
expert_gemm_kernel(const ExpertTable tab, const uint16_t *__restrict__ act, int H, int F,
                   Route rt, uint16_t *__restrict__ h_out, float *__restrict__ y_out) {
  __shared__ __attribute__((aligned(16))) uint32_t s_tbl[kTableWords];
  __shared__ __attribute__((aligned(16))) uint16_t s_a[2][kGemmM * kARowHalves];
  __shared__ uint32_t s_raw[32];
  __shared__ float s_code[32];

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
  // tile fastest so that concurrent items share weight tiles in L2.
  int n_items = 0;
  const int n_active = rt.active[0];
  for (int a = 0; a < n_active; ++a) {
    const int cnt = rt.counts[rt.active[1 + a]];
    n_items += ((cnt + kGemmM - 1) / kGemmM) * n_tiles;
  }

  for (int item = blockIdx.x; item < n_items; item += gridDim.x) {
    int rem = item, a = 0, e = 0, cnt = 0, mtiles = 0;
    for (;;) {  // at most n_active steps
      e = rt.active[1 + a];
      cnt = rt.counts[e];
      mtiles = (cnt + kGemmM - 1) / kGemmM;
      if (rem < mtiles * n_tiles) break;
      rem -= mtiles * n_tiles;
      ++a;
    }
    const int nt = rem / mtiles;
    const int mt_i = rem - nt * mtiles;
    const int off = rt.offsets[e];
    const int m_base = mt_i * kGemmM;
    const moe_nf4_expert_t &ex = tab.e[e];
    if (GATEUP)
      ensure_table<kGemmThreads>(s_tbl, s_raw, s_code, (const float *)ex.w1_code, (const float *)ex.w3_code, built);
    else
      ensure_table<kGemmThreads>(s_tbl, s_raw, s_code, (const float *)ex.w2_code, (const float *)ex.w2_code, built);

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

    uint4 abuf[kGemmADepth][2];
    auto load_a = [&](uint4 (&dst)[2], int b) {
      const int bb = b < NB ? b : NB - 1;  // past the end: the last block again (unused)
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2)
        dst[h2] = *reinterpret_cast<const uint4 *>(asrc[h2] + (size_t)bb * 64);
    };
    auto store_a = [&](const uint4 (&src)[2], int buf) {
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2)
        *reinterpret_cast<uint4 *>(&s_a[buf][(ar0 + 64 * h2) * kARowHalves + 8 * ac]) = src[h2];
    };
    uint2 bq[kGemmBDepth][2];
    float bs[kGemmBDepth][2];
    auto load_b = [&](int slot, int b) {
      const int bb = b < NB ? b : NB - 1;
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        bq[slot][p] = *reinterpret_cast<const uint2 *>(wq[p] + (size_t)bb * 32);
        bs[slot][p] = wa[p][bb];
      }
    };

    f32x4 acc[2][kGemmMT];
#pragma unroll
    for (int p = 0; p < 2; ++p)
#pragma unroll
      for (int m = 0; m < kGemmMT; ++m) acc[p][m] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // Prologue: activation block 0 to LDS, block 1 in registers, weight blocks 0..D-2.
    load_a(abuf[0], 0);
    load_a(abuf[1], 1);
#pragma unroll
    for (int d = 0; d < kGemmBDepth - 1; ++d) load_b(d, d);
    store_a(abuf[0], 0);
    __syncthreads();

    for (int b0 = 0; b0 < NB; b0 += kGemmBDepth) {
#pragma unroll
      for (int d = 0; d < kGemmBDepth; ++d) {
        const int b = b0 + d;
        if (b < NB) {
          load_b((d + kGemmBDepth - 1) % kGemmBDepth, b + kGemmBDepth - 1);
          load_a(abuf[b & 1], b + 2);  // block b's registers were stored at block b-1
          const uint16_t *sa = s_a[b & 1];
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
            const uint4 *pa = reinterpret_cast<const uint4 *>(sa + (m * 16 + n) * kARowHalves + 16 * g);
            const bf16x8 a0 = as_bf16x8(pa[0]);
            const bf16x8 a1 = as_bf16x8(pa[1]);
#pragma unroll
            for (int p = 0; p < 2; ++p) scale_acc(acc[p][m], mfma_block(a0, w0[p], a1, w1[p]), bs[d][p]);
          }
          // Block b+1's activations (loaded at block b-1) to the other buffer.
          store_a(abuf[(b + 1) & 1], (b + 1) & 1);
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
// GEMM.  Needs H % 256 == 0 and F % 128 == 0; writes ypart as one split.
bool expert_gemm_supported(int32_t H, int32_t F) { return H % 256 == 0 && F % 128 == 0; }

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
