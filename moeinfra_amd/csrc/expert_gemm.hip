// K4 for batches: grouped NF4 GEMM on the 32x32x16 bf16 MFMA with the activations staged
// in LDS, for many tokens per expert (prefill).
//
//   gate/up:  h[off_e + r][f] = bf16(bf16(silu(bf16(w1_e x_t))) * bf16(w3_e x_t))[f]
//   down:     ypart[s][off_e + r][c] = sum_{f in K split s} w2_e[c][f] * h[off_e + r][f]   (fp32)
// for the rows r of every active expert e (token t = perm_tok[off_e + r]), the semantics of
// ReconstructedNF4Expert.forward (transfer/nf4_reconstruct.py:152-155) applied to the rows
// model/moe_layer.py:174-186 gathers.
//
// Work.  An item is (active expert, weight tile, K split, token tile), the token tile
// fastest: the items that share a weight tile are consecutive, and the persistent
// workgroups take them XCD by XCD (workgroup b runs on XCD b % 8, so b is renumbered to keep
// consecutive items on one XCD and its L2).  An item is 16 MFMAs per K step over all its
// waves' weight fragments (32 weight rows each) and token tiles (32 tokens each):
//  * large batches (>= 512 routed rows per expert): 256 tokens x 8 fragments, four waves
//    (one per SIMD) of 2 fragments x 8 token tiles;
//  * otherwise: 128 tokens x 16 fragments, eight waves (two per SIMD) of 2 fragments x 4
//    token tiles.
// Gate/up fragments pair w1 and w3 rows; down fragments are w2 row tiles.  Every lane holds
// 16 fp32 sums per (fragment, token tile).
//
// Weights. The B operand of the MFMA is the weight exactly as the reference materializes it
// before its matmul, bf16(code[nibble] * absmax) with an fp32 product (bitsandbytes'
// dequantize_4bit inside the Linear4bit built at transfer/nf4_reconstruct.py:57-114, which
// dequantizes the whole weight for more than one token): a 64 KB LDS table maps a packed byte
// to its two fp32 code values (ds_read_b64), the lane multiplies them by its row's block
// absmax and rounds to bf16. Lane l = 32 kg + i of fragment f holds row i of the fragment; per
// NF4 block it loads the 16 packed bytes 16 kg .. 16 kg + 15 of its row (values 32 kg .. 32 kg
// + 31), four 8-value K slices, one per MFMA step q.
//
// Activations.  The item's tokens x 64 bf16 tile of each block goes through LDS (128-byte
// rows, 16-byte pieces XOR-swizzled by the row); the A operand of step q for token row m is
// piece 4 kg + q of the row, the K slice the weight lanes hold.  The tiles arrive by LDS DMA
// (buffer loads into LDS: rows past the expert's count read zeros), two blocks ahead into
// three planes or, for 256-token tiles, one block ahead into two.  With two planes the
// workgroup meets at one LDS-only barrier per block, which leaves the weight loads in
// flight; with three, each wave waits only until every wave has issued its reads of the
// previous block (an LDS counter), so waves can drift up to a block apart.
#include "nf4_tile.h"

namespace moe {
namespace {

constexpr int kPairWords = 256 * 32 * 2;     // code-pair table: 256 bytes x 32 replicas x 8 B
constexpr uint32_t kGmOob = 0x80000000u;     // buffer offset past any accepted activation tensor

#define GM_GLOBAL __attribute__((address_space(1)))
#define GM_LDS __attribute__((address_space(3)))
typedef const GM_GLOBAL uint8_t *gm_gq_t;
typedef const GM_GLOBAL float *gm_ga_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef __attribute__((__vector_size__(2 * sizeof(float)))) float f32x2;

// s_waitcnt immediate that waits until at most n (< 64) vector memory loads are outstanding
// (gfx9 encoding: vmcnt[3:0] in bits 3:0, vmcnt[5:4] in bits 15:14; expcnt and lgkmcnt at
// their maxima, i.e. not waited for).
constexpr int gm_vmcnt(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// LDS-only barrier: orders the workgroup's LDS accesses without waiting for the waves'
// outstanding global loads (__syncthreads would wait for the whole weight ring).
__device__ __forceinline__ void gm_lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

}  // namespace

// Bounded waits of this device that gave up (lanes), read and cleared by
// moe_wait_timeouts(); zero unless a counting error or extreme wave drift occurred.
__device__ unsigned int g_wait_timeouts;

namespace {

// Waits until the workgroup counter *c reaches `target`.  The wait is bounded (~1 ms, far
// beyond a block's few microseconds): a counting error then gives wrong results instead of
// a wave that never ends, and the lanes that gave up are counted in g_wait_timeouts (a
// vector-memory atomic), which the layer tests require to stay zero.
__device__ __forceinline__ void gm_wait_ge(int *c, int target) {
  for (int i = 0; i < (1 << 14); ++i) {
    if (__hip_atomic_load(c, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) >= target) return;
    __builtin_amdgcn_s_sleep(1);
  }
  __hip_atomic_fetch_add(&g_wait_timeouts, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Position of 16-byte piece p in activation row r.  gfx950 serves a 64-lane ds_read_b128 16
// lanes per cycle, in the lane groups {0-3, 12-15, 20-27} and {4-11, 16-19, 28-31} (and the
// same + 32); the lanes of one group read one piece index of 16 rows whose (r & 1,
// (r >> 1) & 7) are distinct, so the swizzled positions cover all 64 banks once.
__device__ __forceinline__ int gm_pos(int r, int p) { return p ^ ((r >> 1) & 7); }

// Instruction order of one MFMA step of a wave with MT token tiles and NF fragments: 16
// MFMAs of the previous step; NF x 4 v_perm and LDS table reads and MT A-operand reads of
// this step; 12 NF VALU turning the table entries into bf16 weights.  The LDS reads go out
// between the first MFMAs, and the conversions, which wait for them, run under the remaining
// MFMAs instead of stalling in a row.
template <int MT, int NF>
__device__ __forceinline__ void gm_step_schedule() {
  constexpr int kMfma = 0x008, kValu = 0x002, kDsRead = 0x100;
  constexpr int kRest = MT * NF - 2 - NF - MT / 4;  // MFMAs under the conversions
  static_assert(MT * NF == 16 && MT % 4 == 0 && kRest > 0, "step shape");
  __builtin_amdgcn_sched_group_barrier(kMfma, 2, 0);
#pragma unroll
  for (int i = 0; i < NF; ++i) {
    __builtin_amdgcn_sched_group_barrier(kValu, 4, 0);
    __builtin_amdgcn_sched_group_barrier(kDsRead, 4, 0);
    __builtin_amdgcn_sched_group_barrier(kMfma, 1, 0);
  }
#pragma unroll
  for (int i = 0; i < MT / 4; ++i) {
    __builtin_amdgcn_sched_group_barrier(kDsRead, 4, 0);
    __builtin_amdgcn_sched_group_barrier(kMfma, 1, 0);
  }
#pragma unroll
  for (int i = 0; i < kRest; ++i) {
    __builtin_amdgcn_sched_group_barrier(kValu, (12 * NF + kRest - 1) / kRest, 0);
    __builtin_amdgcn_sched_group_barrier(kMfma, 1, 0);
  }
  __builtin_amdgcn_sched_barrier(0);
}

// Four packed bytes (values 2j, 2j+1 per byte) -> eight bf16 weights bf16(code * s).  The
// table entry of byte v for replica rep sits at byte (v << 8) | (rep << 3): {code[v >> 4],
// code[v & 15]}; `lc` is the lane's rep << 3.
__device__ __forceinline__ bf16x8 gm_dequant(const uint32_t *tbl, uint32_t w, uint32_t lc, float s) {
  uint32_t o[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t addr = __builtin_amdgcn_perm(w, lc, 0x0c0c0400u + (j << 8));
    const f32x2 c = *reinterpret_cast<const f32x2 *>(reinterpret_cast<const char *>(tbl) + addr);
    o[j] = pack_bf16x2(c[0] * s, c[1] * s);
  }
  return as_bf16x8(o[0], o[1], o[2], o[3]);
}

// bf16(bf16(silu(bf16(g))) * bf16(u)), the op order of F.silu(gate) * up on bf16 tensors,
// with silu(x) = x / (1 + e^-x) from the hardware's 2^x and reciprocal (about 1 ulp each in
// fp32, a few ulp for |x| in the tens) instead of an exactly rounded exp and division: the
// bf16 rounding of silu can then differ from the correctly rounded one by one bf16 ulp, for
// the values whose fp32 silu lies within a few fp32 ulp of a bf16 rounding boundary.  The
// batched products' fp32 sums already differ from a sequential sum by more than that.  Large
// negative x: 2^x overflows to inf, the reciprocal to 0, silu to -0, as the exact form.
__device__ __forceinline__ uint16_t gm_swiglu_bf16(float g, float u) {
  const uint32_t gu = pack_bf16x2(g, u);  // both rounded to bf16 in one conversion
  const float gb = __builtin_bit_cast(float, gu << 16);
  const float ub = __builtin_bit_cast(float, gu & 0xffff0000u);
  const float e = __builtin_amdgcn_exp2f(gb * -1.44269504088896341f);
  const float sb = bf16_to_f32(f32_to_bf16(gb * __builtin_amdgcn_rcpf(1.0f + e)));
  return f32_to_bf16(sb * ub);
}

// The DMA's inline asm names M0, a register the compiler reserves and sets before each of
// its own uses (this kernel has none besides the asm).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// W waves per workgroup (one workgroup per CU) and MT 32-token tiles per item: W = 4,
// MT = 4 (one wave per SIMD, 4 fragments each), W = 4, MT = 8 (one wave per SIMD, 2
// fragments against 8 token tiles: half the dequantization and weight loads per MFMA), both
// with the steps software-pipelined within the wave; or W = 8, MT = 4 (two waves per SIMD, 2
// fragments each, the other wave covering a wave's stalls).
template <bool GATEUP, int W, int MT, int NF, int BD>
__global__ void __launch_bounds__(W * 64, 1)
expert_gemm_kernel(const ExpertTable tab, const uint16_t *__restrict__ act, uint32_t act_bytes,
                   int K, int NROWS, Route rt, int rows_total, int nsplit,
                   uint16_t *__restrict__ h_out, float *__restrict__ y_out) {
  constexpr int kGmThreads = W * kWave;
  constexpr int kGmMT = MT;                            // 32-token MFMA tiles per item
  constexpr int kGmM = 32 * MT;                        // tokens per item
  constexpr int kGmPlane = kGmM * 128;                 // bytes of one block's activation tile
  constexpr int kGmNF = NF;                            // 32-row weight fragments per wave
  // NF4 blocks in flight per wave: the weight ring.  The block loop is unrolled by BD from
  // block 0, so ring slot b % BD is static; absmax comes per group of 4 blocks (K splits
  // hold whole groups); the activation plane is a runtime LDS offset.
  constexpr int kGmBDepth = BD;
  static_assert(BD % 4 == 0, "ring depth: whole absmax groups");
  // Activation planes: three (the DMA runs two blocks ahead) when they fit beside the 64 KB
  // table, else two (one block ahead).
  constexpr int kPlanes = MT == 8 ? 2 : 3;
  constexpr int kLA = kPlanes - 1;
  constexpr uint32_t kTblHi = (uint32_t)(kPlanes * kGmPlane) >> 16;  // table offset / 64 KB
  static_assert(kPlanes * kGmPlane < 65536 || (kPlanes * kGmPlane) % 65536 == 0, "table offset");
  // v_perm selector of a table address: byte 0 = lc's byte 0 (replica), byte 1 = the packed
  // byte (added per lookup), byte 2 = lc's byte 2 (table offset / 64 KB) or zero, byte 3 zero.
  constexpr uint32_t kTblSel = kTblHi ? 0x0c020400u : 0x0c0c0400u;
  constexpr int kRT = GATEUP ? kGmNF / 2 : kGmNF;      // 32-row tiles per wave
  constexpr int kRowsWave = 32 * kRT;                  // weight rows per wave
  constexpr int kRowsItem = W * kRowsWave;             // weight rows per item
  constexpr int kGmFill = kGmPlane / 16 / kGmThreads;  // 16-byte pieces per thread and block
  constexpr bool kPipe = W == 4 && MT * NF == 16;
  // With the DMA two blocks ahead (three planes) the waves meet through one LDS counter
  // instead of a barrier per block.  At block b's start a wave waits for its own share of
  // block b + 1's activations (issued a block earlier), then until every wave has issued
  // its reads of block b - 1 (a wave's count per block after its last step's reads):
  // those waves have passed block b - 1's start, so every share of block b's plane has
  // landed, and plane (b + 2) % 3 = (b - 1) % 3 is free for the DMA.  The first wave to pass
  // block b's start finds exactly b counts from each wave, so no wave gets more than a block
  // ahead and an early wave's counts never stand in for a late wave's.  Two planes (DMA one
  // block ahead) keep the barrier: a wave's share of the next plane lands only at its
  // block's end.
  constexpr bool kOneSided = kLA == 2;
  static_assert(((W == 4 && MT == 8 && NF == 2) || (W == 8 && MT == 4 && NF == 2) ||
                 (W == 4 && MT == 4 && NF == 4)) &&
                    kGmFill * kGmThreads * 16 == kGmPlane,
                "supported shapes");
  // The activation planes at LDS offset 0 (the DMA's M0 base stays small), then the table.
  __shared__ __attribute__((aligned(16))) uint8_t s_lds[kPlanes * kGmPlane + kPairWords * 4];
  uint32_t *const s_pair = reinterpret_cast<uint32_t *>(s_lds + kPlanes * kGmPlane);
  // Codebooks of every active expert: [0,16) w1 (down: w2), [16,32) w3 (down: w2).
  __shared__ float s_codes[MOE_MAX_EXPERTS][32];
  // Per active expert: id, rows, row offset, first item, token tiles.
  __shared__ int s_ex[MOE_MAX_EXPERTS][5];
  // Stream pointers of every active expert: gate/up w1, w3 packed, w1, w3 absmax; down w2
  // packed, w2 absmax.
  __shared__ const void *s_ptr[MOE_MAX_EXPERTS][4];
  __shared__ int s_nitems;
  // Three-plane shape: threads whose wave has issued the reads of its current block's plane
  // (counted over the item), in place of a barrier per block.
  __shared__ int s_rdone;

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 31;
  const int kg = lane >> 5;
  const int NB = K >> 6;
  const int NBp = NB / nsplit;            // blocks of one K split (a multiple of 4)
  const int wtiles = NROWS / kRowsItem;
  const uint32_t row_bytes = (uint32_t)(K >> 1);
  static_assert(MOE_MAX_EXPERTS <= kWave, "one lane per active expert");

  const int n_active = rt.active[0];
  if (n_active == 0) return;  // uniform over the grid, before any barrier
  if (wave == 0) {
    int e = 0, cnt = 0, items = 0, mtiles = 0;
    if (lane < n_active) {
      e = rt.active[1 + lane];
      // An absent expert (null pointers) gets no items; the caller routes no token to it.
      cnt = (GATEUP ? tab.e[e].w1_packed : tab.e[e].w2_packed) != nullptr ? rt.counts[e] : 0;
      mtiles = (cnt + kGmM - 1) / kGmM;
      items = mtiles * nsplit * wtiles;
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
      s_ex[lane][4] = mtiles;
      const moe_nf4_expert_t &ex = tab.e[e];
      if constexpr (GATEUP) {
        s_ptr[lane][0] = ex.w1_packed;
        s_ptr[lane][1] = ex.w3_packed;
        s_ptr[lane][2] = ex.w1_absmax;
        s_ptr[lane][3] = ex.w3_absmax;
      } else {
        s_ptr[lane][0] = ex.w2_packed;
        s_ptr[lane][1] = ex.w2_packed;
        s_ptr[lane][2] = ex.w2_absmax;
        s_ptr[lane][3] = ex.w2_absmax;
      }
    }
    if (lane == kWave - 1) s_nitems = incl;
  }
  for (int i = tid; i < n_active * 32; i += kGmThreads) {
    const moe_nf4_expert_t &ex = tab.e[rt.active[1 + (i >> 5)]];
    const int j = i & 15;
    float c = 0.0f;
    if ((GATEUP ? ex.w1_packed : ex.w2_packed) != nullptr) {
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
    for (int i = tid; i < n_active * 32; i += kGmThreads)
      if (s_ex[i >> 5][1] > 0)
        cb_diff |= __builtin_bit_cast(uint32_t, s_codes[i >> 5][i & 31]) !=
                   __builtin_bit_cast(uint32_t, s_codes[a0][i & 31]);
  }
  const bool per_item_table = __syncthreads_or(cb_diff) != 0;
  const int n_items = s_nitems;
  const int G = (int)gridDim.x;
  // Workgroups are dispatched to the 8 XCDs round-robin: renumber so that XCD x takes the
  // consecutive items [x G/8, (x + 1) G/8) of every round.
  const int vb = (G & 7) == 0 ? (int)(blockIdx.x & 7) * (G >> 3) + (int)(blockIdx.x >> 3)
                              : (int)blockIdx.x;
  if (vb >= n_items) return;  // uniform over the workgroup

  auto ex_field = [&](int a, int f) { return __builtin_amdgcn_readfirstlane(s_ex[a][f]); };
  // Item -> (active index, weight tile, split, token tile); wave-uniform.
  auto decode = [&](int item, int &a, int &wt, int &sp, int &mt) {
    const int sel = lane < n_active ? lane : 0;
    a = __popcll(__ballot(lane < n_active && s_ex[sel][3] <= item)) - 1;
    int rem = item - ex_field(a, 3);
    const int mtiles = ex_field(a, 4);
    const int q = rem / mtiles;
    mt = rem - q * mtiles;
    wt = q / nsplit;
    sp = q - wt * nsplit;
  };

  // Replica of the lane's table lookups per fragment: with one codebook in the table, lanes
  // l and l + 32 take different replicas (every half-wave covers all 32); with two
  // (gate/up, w1's differing from w3's), replicas 0-15 hold w1's and 16-31 w3's.
  constexpr int kStreams = GATEUP ? 2 : 1;
  uint32_t lc[kStreams];
  int tbl_a = -1;
  auto build_table = [&](int a) {
    gm_lds_barrier();  // every wave is done with the previous table
    for (int i = tid; i < 256 * 32; i += kGmThreads) {
      const int v = i >> 5;
      const float *c = s_codes[a] + ((i & 16) ? 16 : 0);
      *reinterpret_cast<f32x2 *>(&s_pair[2 * i]) = f32x2{c[v >> 4], c[v & 15]};
    }
    int two = 0;
    if (GATEUP && lane < 16)
      two = __builtin_bit_cast(uint32_t, s_codes[a][lane]) != __builtin_bit_cast(uint32_t, s_codes[a][16 + lane]);
    two = __ballot(two) != 0;
#pragma unroll
    for (int p = 0; p < kStreams; ++p)
      lc[p] = ((two ? (uint32_t)((lane & 15) | (p << 4)) : (uint32_t)(li ^ (kg << 4))) << 3) |
              (kTblHi << 16);
    gm_lds_barrier();
    tbl_a = a;
  };

  const __amdgpu_buffer_rsrc_t rsrc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(act), (short)0, (int)act_bytes, 0x00020000);

  // Activation fill by LDS DMA: for piece set j, wave w writes rows 8 W j + 8 w .. + 7 of a
  // plane with one 16-byte-per-lane buffer load; lane L lands at byte 16 L of the wave's
  // 1 KB, i.e. row fr = 8 W j + 8 w + L / 8 at position L % 8, so it loads the piece that
  // belongs there, gm_pos(fr, L % 8) (the swizzle is an involution; 8 W j leaves it alone).
  const int fr = 8 * wave + (lane >> 3);
  const uint32_t fsrc = 8u * (uint32_t)gm_pos(fr, lane & 7);
  // Lane's A operand: token row li of each 32-token tile, piece 4 kg + q.
  int a_lds[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) a_lds[q] = li * 128 + 16 * gm_pos(li, 4 * kg + q);
  // Fragment f's rows: gate/up stream f & 1, rows 32 (f >> 1) + i of the wave's; down rows
  // 32 f + i of the wave's.  Per block, 16 bytes at 32 b + 16 kg of the row; per group of 4
  // blocks, the row's 4 absmax values (one 16-byte load: a 4-byte load per block would
  // touch 32 rows' lines for 256 bytes).
  const uint32_t w_lane = (uint32_t)li * row_bytes + 16u * kg;
  const uint32_t s_lane = (uint32_t)li * (uint32_t)NB;
  const GM_LDS uint8_t *const s_a0 = (const GM_LDS uint8_t *)s_lds;
  const uint32_t s_a0_off = (uint32_t)(uintptr_t)s_a0;
  // Table reads address byte (v << 8) | (rep << 3) of the table.  Past 64 KB (two 32 KB
  // planes in front) the table's offset does not fit a ds_read's 16-bit immediate; the
  // v_perm that builds the address then inserts its high byte (from lc) instead.
  const GM_LDS char *const tbl = (const GM_LDS char *)s_lds + (kTblHi ? 0 : kPlanes * kGmPlane);

  f32x16 acc[kGmMT][kGmNF];
  u32x4 ring[kGmBDepth][kGmNF];
  f32x4 absc[kGmNF], absn[kGmNF];  // absmax of the current and the next group of 4 blocks

  for (int item = vb; item < n_items; item += G) {
    int a, wt, sp, mt;
    decode(item, a, wt, sp, mt);
    if (tbl_a < 0 || (per_item_table && a != tbl_a)) build_table(a);
    const int cnt = ex_field(a, 1), off = ex_field(a, 2);
    const uint32_t row0 = (uint32_t)(wt * kRowsItem + wave * kRowsWave);
    const uint32_t kb0 = (uint32_t)(sp * NBp);
    auto uptr = [&](int f) {
      const uint64_t v = (uint64_t)(uintptr_t)s_ptr[a][f];
      const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
      const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
      return (uint64_t)lo | ((uint64_t)hi << 32);
    };
    gm_gq_t wb[kGmNF];
    gm_ga_t ab[kGmNF];
#pragma unroll
    for (int f = 0; f < kGmNF; ++f) {
      const int s = GATEUP ? (f & 1) : 0;
      const uint32_t fr0 = row0 + 32u * (uint32_t)(GATEUP ? (f >> 1) : f);
      wb[f] = (gm_gq_t)(uintptr_t)uptr(s) + (fr0 * row_bytes + kb0 * 32u);
      ab[f] = (gm_ga_t)(uintptr_t)uptr(2 + s) + (fr0 * (uint32_t)NB + kb0);
    }
    // Rows past the expert's count read past the tensor (zeros).  The token ids of all rows
    // are loaded together (clamped to the last row, then masked): one round trip, where a
    // load behind a branch per row would wait for each in turn.
    uint32_t fo[kGmFill];
#pragma unroll
    for (int j = 0; j < kGmFill; ++j) {
      const int r = mt * kGmM + fr + 8 * W * j;
      const int rc = r < cnt ? r : cnt - 1;
      fo[j] = GATEUP ? (uint32_t)rt.perm_tok[off + rc] : (uint32_t)(off + rc);
    }
#pragma unroll
    for (int j = 0; j < kGmFill; ++j) {
      const int r = mt * kGmM + fr + 8 * W * j;
      fo[j] = r < cnt ? (fo[j] * (uint32_t)K + kb0 * 64u + fsrc) * 2u : kGmOob;
    }

    // Weights of block b and absmax of blocks b4..b4+3 (past the split's end: its last
    // block / group again, unused).
    auto load_b = [&](int slot, int b) {
      const uint32_t bo = w_lane + (uint32_t)(b < NBp ? b : NBp - 1) * 32u;
#pragma unroll
      for (int f = 0; f < kGmNF; ++f) ring[slot][f] = *reinterpret_cast<const GM_GLOBAL u32x4 *>(wb[f] + bo);
    };
    auto load_s = [&](f32x4 (&dst)[kGmNF], int b4) {
      const uint32_t so = s_lane + (uint32_t)(b4 < NBp ? b4 : NBp - 4);
#pragma unroll
      for (int f = 0; f < kGmNF; ++f) dst[f] = *reinterpret_cast<const GM_GLOBAL f32x4 *>(ab[f] + so);
    };
    // Activations of block b into the plane at LDS byte `plane`: kGmFill VMEM instructions
    // per thread.  Written as inline asm so that the compiler neither counts them nor makes
    // LDS reads wait for them (it cannot tell the planes apart); the explicit vmcnt waits
    // before the barriers count them.  M0 holds the wave's 1 KB destination.
    auto dma = [&](uint32_t plane, int b) {
      const uint32_t adv = (uint32_t)(b < NBp ? b : NBp - 1) * 128u;
#pragma unroll
      for (int j = 0; j < kGmFill; ++j) {
        const uint32_t dst = plane + (uint32_t)(8 * W * j + 8 * wave) * 128u;
        asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                     :
                     : "s"(dst), "v"(fo[j] + adv), "s"(rsrc)
                     : "m0");
      }
    };
    // One MFMA step: the A operands of the four token tiles and the table entries of the
    // four fragments' K slices (LDS), then the bf16 weights, then 16 MFMAs.
    struct Pre {
      u32x4 a[kGmMT];
      f32x2 c[kGmNF][4];
    };
    // Token tiles t >= live (wave-uniform: the tiles holding the item's rows; always kGmMT in
    // the pipelined forms, whose accumulators do not survive a branch around their MFMAs
    // without spilling) read no A operands and run no MFMAs: their sums stay zero and their
    // rows are past the expert's count.
    int live = kGmMT;
    auto issue = [&](Pre &P, const GM_LDS uint8_t *plane, const GM_LDS char *tb, int slot, int q) {
#pragma unroll
      for (int t = 0; t < kGmMT; ++t)
        if (t == 0 || kPipe || t < live)
          P.a[t] = *reinterpret_cast<const GM_LDS u32x4 *>(plane + a_lds[q] + t * 32 * 128);
#pragma unroll
      for (int f = 0; f < kGmNF; ++f)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t addr = __builtin_amdgcn_perm(ring[slot][f][q], lc[GATEUP ? (f & 1) : 0], kTblSel + (j << 8));
          P.c[f][j] = *reinterpret_cast<const GM_LDS f32x2 *>(tb + addr);
        }
    };
    auto convert = [&](const Pre &P, int slot, bf16x8 (&bv)[kGmNF]) {
#pragma unroll
      for (int f = 0; f < kGmNF; ++f) {
        const float sc = absc[f][slot & 3];  // block slot % 4 of its absmax group
        uint32_t o[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = pack_bf16x2(P.c[f][j][0] * sc, P.c[f][j][1] * sc);
        bv[f] = as_bf16x8(o[0], o[1], o[2], o[3]);
      }
    };
    auto mfmas = [&](const Pre &P, const bf16x8 (&bv)[kGmNF]) {
#pragma unroll
      for (int t = 0; t < kGmMT; ++t)
        if (t == 0 || kPipe || t < live) {
#pragma unroll
          for (int f = 0; f < kGmNF; ++f)
            acc[t][f] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(P.a[t]), bv[f], acc[t][f], 0, 0, 0);
        }
    };

#pragma unroll
    for (int t = 0; t < kGmMT; ++t)
#pragma unroll
      for (int f = 0; f < kGmNF; ++f)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[t][f][v] = 0.0f;
    // The step in flight: its operands, consumed one step later (zeros before block 0).
    Pre pc;
    bf16x8 bc[kGmNF];
#pragma unroll
    for (int t = 0; t < kGmMT; ++t) pc.a[t] = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int f = 0; f < kGmNF; ++f) bc[f] = as_bf16x8(0u, 0u, 0u, 0u);

    // Prologue: activations of blocks 0..kLA-1, weights of blocks 0..BDepth-2.  The previous
    // item's reads of every plane ended before its last barrier.
#pragma unroll
    for (int d = 0; d < kLA; ++d) dma(s_a0_off + d * kGmPlane, d);
#pragma unroll
    for (int d = 0; d < kGmBDepth - 1; ++d) load_b(d, d);
    load_s(absn, 0);  // moved to absc as block 0 starts
    // The prologue's activations landed (the weight loads issued after them may not).
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(gm_vmcnt(kGmNF * (kGmBDepth - 1)));
    if (kOneSided && threadIdx.x == 0) s_rdone = 0;
    gm_lds_barrier();

    // One block: the DMA of block b + kLA's activations into plane `dst`, block b + 3's
    // weights, and block b's four MFMA steps from plane `src` and the table.
    auto block = [&](uint32_t dst, const GM_LDS uint8_t *src, int d, int b) {
      if constexpr (kOneSided) {
        // Own share of block b + 1's activations: only block b - 1's weight loads were
        // issued after it.
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(gm_vmcnt(kGmNF));
        if (b > 0) gm_wait_ge(&s_rdone, kGmThreads * b);
        __builtin_amdgcn_sched_barrier(0);
      }
      // Issue order: absmax (at a group start), activations, weights.  The wait before the
      // barrier counts the loads issued after the activations it needs, so the absmax loads
      // go first: issued last, that count would also have to cover them.
      if (d % 4 == 0) {  // static: group b / 4 starts; its absmax was loaded 4 blocks ago
        // The loads that filled absn were issued before a block's activation DMA, whose
        // wait completed them.  Reading absn here, before this block's DMA is issued, puts
        // the compiler's own wait for them (it cannot count the DMA) where the hardware has
        // only the previous block's weight loads outstanding: a no-op, where further on it
        // would also wait for the DMA just issued.
#pragma unroll
        for (int f = 0; f < kGmNF; ++f) asm volatile("" ::"v"(absn[f]));
#pragma unroll
        for (int f = 0; f < kGmNF; ++f) absc[f] = absn[f];
        load_s(absn, b + 4);
      }
      __builtin_amdgcn_sched_barrier(0);
      dma(dst, b + kLA);
      load_b((d + kGmBDepth - 1) % kGmBDepth, b + kGmBDepth - 1);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if constexpr (kPipe) {
          Pre pn;
          bf16x8 bn[kGmNF];
          issue(pn, src, tbl, d, q);
          if (kOneSided && q == 3) {
            // After the block's last reads of its plane, as in the unpipelined step below.
            __builtin_amdgcn_sched_barrier(0);
            __hip_atomic_fetch_add(&s_rdone, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
            __builtin_amdgcn_sched_barrier(0);
          }
          mfmas(pc, bc);  // the previous step (for q = 0 the previous block's last)
          convert(pn, d, bn);
          pc = pn;
#pragma unroll
          for (int f = 0; f < kGmNF; ++f) bc[f] = bn[f];
          gm_step_schedule<MT, kGmNF>();
        } else {
          Pre p;
          bf16x8 bv[kGmNF];
          issue(p, src, tbl, d, q);
          if (kOneSided && q == 3) {
            // After the block's last reads of its plane (release: they complete first).  Every
            // lane adds 1 (the compiler folds the wave's adds into one ds_add of 64), so the
            // counts are threads: kGmThreads per block.
            __builtin_amdgcn_sched_barrier(0);
            __hip_atomic_fetch_add(&s_rdone, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
            __builtin_amdgcn_sched_barrier(0);
          }
          convert(p, d, bv);
          mfmas(p, bv);
        }
      }
      // Block b + 1's activations (issued kLA - 1 blocks earlier) must have landed for every
      // wave before the barrier.  Issued after them (sched_barriers keep the three groups in
      // order; the DMA is an asm statement no load moves across): with kLA = 1 block b's
      // weight loads (kGmNF); with kLA = 2 block b - 1's weight loads, then block b's absmax
      // loads if any, activations (kGmFill) and weights (kGmNF).  Waiting down to kGmNF,
      // resp. kGmFill + 2 kGmNF, completes exactly the loads up to those activations (with
      // block b's absmax loads present, block b - 1's weights too).
      if constexpr (!kOneSided) {
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(gm_vmcnt(kLA == 1 ? kGmNF : kGmFill + 2 * kGmNF));
        gm_lds_barrier();
      }
    };
    // An expert's last token tile is often partial (about half the experts of a 512-token
    // batch spill a few rows past 128).
    live = min(kGmMT, (cnt - mt * kGmM + 31) >> 5);
    int pb = 0;  // plane of block b: b % kPlanes
    for (int b0 = 0; b0 < NBp; b0 += kGmBDepth) {
#pragma unroll
      for (int d = 0; d < kGmBDepth; ++d) {
        if (BD == 4 || b0 + d < NBp) {  // a split (4 k blocks) may end inside a BD-block step
          // Plane (b + kLA) % kPlanes = (b - 1) % kPlanes was last read in block b - 1,
          // before the barrier.
          const int pd = pb == 0 ? kPlanes - 1 : pb - 1;
          block(s_a0_off + pd * kGmPlane, s_a0 + pb * kGmPlane, d, b0 + d);
          pb = pb == kPlanes - 1 ? 0 : pb + 1;
        }
      }
    }
    if constexpr (kPipe) mfmas(pc, bc);
    // Every wave's reads of the item's planes have ended before the next item's table,
    // counter reset and prologue DMA.
    if constexpr (kOneSided) gm_lds_barrier();

    // Lane l = 32 kg + i holds column i of each fragment for token rows
    // 32 t + 8 (v >> 2) + 4 kg + (v & 3) of the item's tile.  The stores go through a buffer
    // descriptor that spans the expert's cnt rows: a row past the expert's last is dropped by
    // the range check (which covers the per-lane offset, so the row goes there), instead of a
    // branch and 64-bit address arithmetic per value.
    {
      constexpr uint32_t kEs = GATEUP ? 2u : 4u;  // bytes per output value
      char *obase = GATEUP ? (char *)(h_out + (size_t)off * NROWS)
                           : (char *)(y_out + ((size_t)sp * rows_total + off) * NROWS);
      const __amdgpu_buffer_rsrc_t orsrc = __builtin_amdgcn_make_buffer_rsrc(
          obase, (short)0, (int)((uint32_t)cnt * (uint32_t)NROWS * kEs), 0x00020000);
      const uint32_t lane_off = ((uint32_t)(mt * kGmM + 4 * kg) * (uint32_t)NROWS + row0 + (uint32_t)li) * kEs;
      const uint32_t row_step = (uint32_t)NROWS * kEs;
#pragma unroll
      for (int t = 0; t < kGmMT; ++t) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const uint32_t o = lane_off + (uint32_t)(32 * t + 8 * (v >> 2) + (v & 3)) * row_step;
          if constexpr (GATEUP) {
#pragma unroll
            for (int r2 = 0; r2 < kRT; ++r2)
              __builtin_amdgcn_raw_buffer_store_b16(gm_swiglu_bf16(acc[t][2 * r2][v], acc[t][2 * r2 + 1][v]),
                                                    orsrc, (int)(o + 64u * r2), 0, 0);
          } else {
#pragma unroll
            for (int f = 0; f < kGmNF; ++f) {
              // Element by value: a bit cast of the vector element itself reads element 0.
              const float val = acc[t][f][v];
              __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, val), orsrc,
                                                    (int)(o + 128u * f), 0, 0);
            }
          }
        }
      }
    }
  }
  // The last item's DMAs past its end are still writing LDS: they must land before the
  // workgroup's LDS is released.
  __builtin_amdgcn_s_waitcnt(gm_vmcnt(0));
}
#pragma clang diagnostic pop

}  // namespace

// Kernel shape of a launch (waves, token tiles per item, fragments per wave, ring depth):
// 256-token items (W = 4, MT = 8) from 512 routed rows per active expert on average, else
// 128-token items with two waves per SIMD (W = 8, MT = 4).
struct GemmShape {
  int waves, mt, nf, bd;
  int64_t tokens() const { return 32 * mt; }
  int64_t down_rows() const { return 32LL * waves * nf; }
};
GemmShape gemm_shape(int64_t rows, int64_t active) {
  return active > 0 && rows >= 512 * active ? GemmShape{4, 8, 2, 4} : GemmShape{8, 4, 2, 4};
}

// The batched form of K4: gate/up (phases bit 0) and/or down (bit 1).  Gate/up items cover
// 16 W NF rows of F, down items 32 W NF rows of H (at most 512); the down projection splits
// K over `nsplit` ypart planes, each a whole number of 4-block absmax groups.
bool expert_gemm_supported(int32_t H, int32_t F) { return H % 512 == 0 && F % 256 == 0; }

bool expert_gemm_splits_ok(int32_t F, int32_t nsplit) {
  const int nb = F / 64;
  return nsplit >= 1 && nb % nsplit == 0 && (nb / nsplit) % 4 == 0;
}

// Activation tensors (x, h) and an expert's outputs (its h rows, its fp32 ypart rows of one
// split) are addressed with 32-bit buffer offsets below kGmOob.
bool expert_gemm_rows_ok(int64_t T, int64_t rows_total, int32_t H, int32_t F) {
  return T * (int64_t)H * 2 < (int64_t)kGmOob && rows_total * (int64_t)F * 2 < (int64_t)kGmOob &&
         rows_total * (int64_t)H * 4 < (int64_t)kGmOob;
}

// Down-projection splits for a layer of `rows` routed rows over `active` experts and a
// launch shape: the smallest power of two (up to kGmMaxSplits) that gives every CU
// kGmItemsPerCu items, when the shape allows it.  Routed counts vary around the average, so
// an expert's last token tile is often nearly empty but costs a whole item: several items
// per CU keep that from setting the launch's length.
#ifndef GM_ITEMS_PER_CU
#define GM_ITEMS_PER_CU 4
#endif
#ifndef GM_MAX_SPLITS
#define GM_MAX_SPLITS 8
#endif
static int gemm_splits_for(const GemmShape &g, int64_t rows, int64_t active, int32_t H, int32_t F) {
  const int64_t per = active > 0 ? (rows + active - 1) / active : 0;
  const int64_t m = g.tokens();
  const int64_t items = active * ((per + m - 1) / m) * (H / g.down_rows());
  const int64_t want = GM_ITEMS_PER_CU * (int64_t)device_cu_count();
  int s = 1;
  while (s < GM_MAX_SPLITS && items * s < want && expert_gemm_splits_ok(F, 2 * s)) s *= 2;
  return s;
}
int expert_gemm_splits(int64_t rows, int64_t active, int32_t H, int32_t F) {
  return gemm_splits_for(gemm_shape(rows, active), rows, active, H, F);
}

template <int W, int MT, int NF, int BD>
static int launch_gemm_shape(const ExpertTable &tab, const void *x, int64_t T, int64_t rows_total,
                             int32_t H, int32_t F, const Route &rt, void *h_ws, void *ypart,
                             int32_t nsplit, int phases, hipStream_t stream) {
  const dim3 grid((unsigned)device_cu_count()), blk(W * kWave);
  if (phases & 1) {
    hipLaunchKernelGGL((expert_gemm_kernel<true, W, MT, NF, BD>), grid, blk, 0, stream, tab,
                       (const uint16_t *)x, (uint32_t)(T * H * 2), H, F, rt, (int)rows_total, 1,
                       (uint16_t *)h_ws, (float *)nullptr);
    MOE_LAUNCH_CHECK();
  }
  if (phases & 2) {
    hipLaunchKernelGGL((expert_gemm_kernel<false, W, MT, NF, BD>), grid, blk, 0, stream, tab,
                       (const uint16_t *)h_ws, (uint32_t)(rows_total * F * 2), F, H, rt,
                       (int)rows_total, nsplit, (uint16_t *)nullptr, (float *)ypart);
    MOE_LAUNCH_CHECK();
  }
  return MOE_STATUS_OK;
}

static int check_gemm_args(int64_t T, int64_t rows_total, int32_t H, int32_t F, int32_t nsplit) {
  MOE_REQUIRE(expert_gemm_supported(H, F), "shape not supported by the batched expert GEMM");
  MOE_REQUIRE(expert_gemm_splits_ok(F, nsplit), "K split count not supported by the batched expert GEMM");
  MOE_REQUIRE(expert_gemm_rows_ok(T, rows_total, H, F), "activations too large for the batched expert GEMM");
  return MOE_STATUS_OK;
}

int launch_expert_gemm(const void *tab_v, const void *x, int64_t T, int64_t rows_total,
                       int64_t active_max, int32_t H, int32_t F, const void *route_v, void *h_ws,
                       void *ypart, int32_t nsplit, int phases, hipStream_t stream) {
  const int rc = check_gemm_args(T, rows_total, H, F, nsplit);
  if (rc != MOE_STATUS_OK) return rc;
  const ExpertTable &tab = *static_cast<const ExpertTable *>(tab_v);
  const Route &rt = *static_cast<const Route *>(route_v);
  const GemmShape g = gemm_shape(rows_total, active_max);
  if (g.mt == 8)
    return launch_gemm_shape<4, 8, 2, 4>(tab, x, T, rows_total, H, F, rt, h_ws, ypart, nsplit, phases, stream);
  return launch_gemm_shape<8, 4, 2, 4>(tab, x, T, rows_total, H, F, rt, h_ws, ypart, nsplit, phases, stream);
}

}  // namespace moe

// Reads (and with reset != 0 clears) the current device's count of bounded waits that gave
// up.  Synchronous with respect to the device: a diagnostic for tests, not for hot loops.
extern "C" int moe_wait_timeouts(int64_t *count, int32_t reset) {
  MOE_REQUIRE(count != nullptr, "null count");
  unsigned int v = 0;
  MOE_HIP_CHECK(hipMemcpyFromSymbol(&v, HIP_SYMBOL(moe::g_wait_timeouts), sizeof(v), 0,
                                    hipMemcpyDeviceToHost));
  if (reset) {
    const unsigned int zero = 0;
    MOE_HIP_CHECK(hipMemcpyToSymbol(HIP_SYMBOL(moe::g_wait_timeouts), &zero, sizeof(zero), 0,
                                    hipMemcpyHostToDevice));
  }
  *count = (int64_t)v;
  return MOE_STATUS_OK;
}
