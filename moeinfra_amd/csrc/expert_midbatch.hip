// K4 for mid-size batches, streamed form: the grouped NF4 SwiGLU expert FFN on
// v_mfma_f32_32x32x16_bf16 for a few to a few tens of tokens per expert, where a layer is
// bound by streaming the NF4 weights (each weight row is read once per 32-token chunk of its
// expert).
//
//   gate/up:  h[off_e + r][f] = bf16(bf16(silu(bf16(w1_e x_t))) * bf16(w3_e x_t))[f]
//   down:     ypart[s][off_e + r][c] = sum over f in K split s of w2_e[c][f] * h[off_e + r][f]
// for the rows r of every active expert e (token t = perm_tok[off_e + r]): the semantics of
// ReconstructedNF4Expert.forward (transfer/nf4_reconstruct.py:152-155) applied to the rows
// model/moe_layer.py:174-186 gathers; the combine adds the splits.
//
// Work.  A workgroup item is (active expert, 32-token chunk of its rows, K split, group of
// eight 32-row weight tiles).  Wave w owns tile 8g + w over the item's whole K range, so its
// sums are complete at the end of the item and no partial sum crosses waves.  Items are
// dealt to workgroups in contiguous ranges, ordered (expert, chunk, split, group) with the
// group fastest, so that concurrently running workgroups share activation rows in L2.  The
// down projection splits K into `nsplit` parts (separate ypart planes) so that a layer with
// few active experts still has work for every CU.
//
// Streams.  Each wave keeps kMbDepth NF4 blocks (16 bytes per lane per stream) in flight in
// a register ring that runs across item boundaries, and loads the absmax of a whole chunk
// (8 blocks of its row: 32 contiguous bytes per lane) with the chunk's activations.  The
// activations pass through LDS in chunks of kMbChunk blocks x 32 tokens, double buffered:
// the workgroup loads chunk q + 1 (four 16-byte pieces per thread) while it computes chunk
// q, stores it to the other buffer after the last block of chunk q and meets at one
// LDS-only barrier, which leaves the waves' weight loads in flight.  Chunk q + 1's loads are
// issued right after the weight load of block 8q + 7 (the ring's newest at that point), so
// waiting for them (loads complete in issue order) never waits for a weight block that is
// not due yet.
//
// MFMA layout.  In v_mfma_f32_32x32x16_bf16 lane l = 32*kg + i supplies B[k 8kg..8kg+7][n = i]
// and A[m = i][k 8kg..8kg+7], and holds D[m][n = i] for m = 8*(v/4) + 4*kg + v%4 in its
// register v.  The weights are B (n = weight row), the tokens A (m = token row).  For NF4
// block b a lane holds the 16 packed bytes 16*kg .. 16*kg+15 of its row's block (values
// 32*kg .. 32*kg+31), the K slices of four MFMAs (MFMA q takes values 32*kg + 8q .. +7); the
// A operand of MFMA q is piece 4*kg + q (16 bytes) of its token's 128-byte block row.  Every
// MFMA stays inside one 64-value block, and the block's absmax (one per lane: the lane's
// row) scales the MFMA result into the lane's 16 fp32 accumulators.
#include "nf4_tile.h"

namespace moe {
namespace {

typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;

constexpr int kMbWaves = 8;
constexpr int kMbThreads = kMbWaves * kWave;
constexpr int kMbRows = 32;     // weight rows per wave and item (MFMA columns)
constexpr int kMbToks = 32;     // token rows per chunk (MFMA rows)
constexpr int kMbDepth = 8;     // NF4 blocks in flight per wave
constexpr int kMbChunk = 8;     // blocks per activation chunk (one barrier per chunk)
static_assert(kMbDepth == kMbChunk, "the ring slot of a step is its block index in the chunk");
// LDS activation chunk: [block][token row][128 bytes]; a block plane is padded by one row
// so that consecutive planes start in opposite halves of the 64 banks.
constexpr int kMbPlane = kMbToks * 128 + 128;
constexpr int kMbChunkBytes = kMbChunk * kMbPlane;
// 16-byte pieces of one chunk per thread: thread t fills token rows wave + 8j (j < 4),
// block (lane / 8), piece (lane % 8).
constexpr int kMbFill = kMbToks * kMbChunk * 8 / kMbThreads;
static_assert(kMbFill == 4 && kMbToks == 8 * kMbFill, "fill layout");
constexpr int kMbMaxRows = 2048;  // routed rows whose token ids the gate/up kernel keeps in LDS
constexpr uint32_t kMbOob = 0x80000000u;  // buffer offset past any accepted activation tensor

#define MB_GLOBAL __attribute__((address_space(1)))
typedef const MB_GLOBAL uint8_t *mb_gq_t;
typedef const MB_GLOBAL float *mb_ga_t;

// LDS-only barrier: orders the workgroup's LDS accesses without waiting for the waves'
// outstanding global loads (a workgroup fence on all address spaces would drain them).
__device__ __forceinline__ void mb_lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Position of 16-byte piece p in token row r of a block plane: rows r and r + 1 sit in
// opposite bank halves, and the swizzle spreads the 16 lanes of one ds_read_b128 cycle
// over all 64 banks (gfx950 groups the lanes {0-3, 12-15, 20-27} and {4-11, 16-19, 28-31},
// and the same + 32; within each group the even and the odd rows take eight distinct
// values of (r >> 1) & 7).
__device__ __forceinline__ int mb_pos(int r, int p) { return p ^ ((r >> 1) & 7); }

// Four packed bytes (values 2j, 2j+1 per byte, j = 0..3) -> eight bf16 code values.
__device__ __forceinline__ bf16x8 mb_lookup4(const uint32_t *tbl, uint32_t w, uint32_t lane_const) {
  uint32_t l[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    l[j] = lds_lookup(tbl, __builtin_amdgcn_perm(w, lane_const, 0x0c0c0400u + (j << 8)));
  return as_bf16x8(l[0], l[1], l[2], l[3]);
}

// An item's streams: wave-uniform bases of the weight tile's first row at the item's first
// block, the lane's absmax pointer (its row, stream kg for gate/up) and the thread's four
// activation offsets of the item's chunk 0 (kMbOob for rows past the chunk).
template <int NP>
struct MbPtr {
  mb_gq_t wb[NP];
  mb_ga_t ab;
  uint32_t fo[kMbFill];
};

template <int NP>
struct MbStage {
  u32x4 w[NP];
};

template <int NP>
__global__ void __launch_bounds__(kMbThreads, 1)
midbatch_kernel(const ExpertTable tab, const uint16_t *__restrict__ act, uint32_t act_bytes,
                int K, int NROWS, Route rt, int rows_total, int nsplit,
                uint16_t *__restrict__ h_out, float *__restrict__ y_out) {
  constexpr bool GATEUP = NP == 2;
  __shared__ __attribute__((aligned(16))) uint32_t s_tbl[kTableWords];
  __shared__ __attribute__((aligned(16))) uint8_t s_ring[2][kMbChunkBytes];
  // Codebooks of every active expert: [0,16) w1 (down: w2), [16,32) w3 (down: w2).
  __shared__ float s_codes[MOE_MAX_EXPERTS][32];
  // Per active expert: id, rows, row offset, first item, 32-token chunks.
  __shared__ int s_ex[MOE_MAX_EXPERTS][5];
  __shared__ int s_ptok[GATEUP ? kMbMaxRows : 1];
  // Stream pointers of every active expert (packed, absmax): gate/up w1, w3; down w2.
  __shared__ const void *s_ptr[MOE_MAX_EXPERTS][2 * NP];
  __shared__ int s_nitems;

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li32 = lane & 31;
  const int kg = lane >> 5;
  const int NB = K >> 6;
  const int NBp = NB / nsplit;           // blocks of one K split (a multiple of kMbChunk)
  const int n_chunks = NBp / kMbChunk;   // activation chunks per item
  const int groups = NROWS / (kMbWaves * kMbRows);
  const uint32_t row_bytes = (uint32_t)(K >> 1);
  static_assert(MOE_MAX_EXPERTS <= kWave, "one lane per active expert");

  const int n_active = rt.active[0];
  if (n_active == 0) return;  // uniform over the grid, before any barrier
  if (wave == 0) {
    int e = 0, cnt = 0, items = 0, nch = 0;
    if (lane < n_active) {
      e = rt.active[1 + lane];
      // An absent expert (null pointers) gets no items; the caller routes no token to it.
      cnt = (GATEUP ? tab.e[e].w1_packed : tab.e[e].w2_packed) != nullptr ? rt.counts[e] : 0;
      nch = (cnt + kMbToks - 1) / kMbToks;
      items = nch * nsplit * groups;
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
      const moe_nf4_expert_t &ex = tab.e[e];
      if constexpr (GATEUP) {
        s_ptr[lane][0] = ex.w1_packed;
        s_ptr[lane][1] = ex.w3_packed;
        s_ptr[lane][2] = ex.w1_absmax;
        s_ptr[lane][3] = ex.w3_absmax;
      } else {
        s_ptr[lane][0] = ex.w2_packed;
        s_ptr[lane][1] = ex.w2_absmax;
      }
    }
    if (lane == kWave - 1) s_nitems = incl;
  }
  if (GATEUP)
    for (int i = tid; i < rows_total; i += kMbThreads) s_ptok[i] = rt.perm_tok[i];
  for (int i = tid; i < n_active * 32; i += kMbThreads) {
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
    for (int i = tid; i < n_active * 32; i += kMbThreads)
      if (s_ex[i >> 5][1] > 0)
        cb_diff |= __builtin_bit_cast(uint32_t, s_codes[i >> 5][i & 31]) !=
                   __builtin_bit_cast(uint32_t, s_codes[a0][i & 31]);
  }
  const bool per_item_table = __syncthreads_or(cb_diff) != 0;
  const int n_items = s_nitems;
  const int lo = (int)((int64_t)blockIdx.x * n_items / gridDim.x);
  const int hi = (int)((int64_t)(blockIdx.x + 1) * n_items / gridDim.x);
  if (lo >= hi) return;  // uniform over the workgroup

  // Item -> (active index, chunk, split, group); wave-uniform.
  auto ex_field = [&](int a, int f) { return __builtin_amdgcn_readfirstlane(s_ex[a][f]); };
  auto decode = [&](int item, int &a, int &ch, int &sp, int &g) {
    const int sel = lane < n_active ? lane : 0;
    a = __popcll(__ballot(lane < n_active && s_ex[sel][3] <= item)) - 1;
    int rem = item - ex_field(a, 3);
    const int per_chunk = nsplit * groups;
    ch = rem / per_chunk;
    rem -= ch * per_chunk;
    sp = rem / groups;
    g = rem - sp * groups;
  };
  int tbl_a;
  {
    int ch, sp, g;
    decode(lo, tbl_a, ch, sp, g);
  }
  // Lookup table (nf4_tile.h) from the item's two codebooks, by the whole workgroup, between
  // LDS-only barriers (the waves' outstanding weight loads stay in flight).
  auto build_table = [&](int a) {
    mb_lds_barrier();  // every wave is done with the previous table
    for (int i = tid; i < kTableWords; i += kMbThreads) {
      const int v = i >> 6;  // packed byte value
      const float *c = s_codes[a] + ((i & 32) ? 16 : 0);  // replicas 32-63: second codebook
      s_tbl[i] = pack_bf16x2(c[v >> 4], c[v & 15]);
    }
    mb_lds_barrier();
  };
  build_table(tbl_a);

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

  // Thread's fill pieces: rows wave + 8j, block fb, piece fp of every chunk; their LDS byte
  // offsets within a chunk buffer.
  const int fb = lane >> 3, fp = lane & 7;
  int fill_lds[kMbFill];
#pragma unroll
  for (int j = 0; j < kMbFill; ++j) {
    const int r = wave + 8 * j;
    fill_lds[j] = fb * kMbPlane + r * 128 + 16 * mb_pos(r, fp);
  }
  // Lane's A operand rows: token row li32, pieces 4*kg + q of each block plane.
  int a_lds[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) a_lds[q] = li32 * 128 + 16 * mb_pos(li32, 4 * kg + q);

  const uint32_t w_lane = (uint32_t)li32 * row_bytes + 16u * kg;
  auto set_ptrs = [&](MbPtr<NP> &P, int item) {
    int a, ch, sp, g;
    decode(item, a, ch, sp, g);
    const int cnt = ex_field(a, 1), off = ex_field(a, 2);
    const uint32_t row0 = (uint32_t)((g * kMbWaves + wave) * kMbRows);
    const uint32_t kb0 = (uint32_t)(sp * NBp);
    const uint32_t wofs = row0 * row_bytes + kb0 * 32u;
    // Wave-uniform LDS reads of the expert's pointers (no global load: the next item's
    // setup never waits for the weight loads in flight).
    auto uptr = [&](int f) {
      const uint64_t v = (uint64_t)(uintptr_t)s_ptr[a][f];
      // readfirstlane returns int: widen through uint32_t (no sign extension).
      const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
      const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
      return (uint64_t)lo | ((uint64_t)hi << 32);
    };
#pragma unroll
    for (int p = 0; p < NP; ++p) P.wb[p] = (mb_gq_t)(uintptr_t)uptr(p) + wofs;
    const uint64_t ab0 = uptr(NP), ab1 = uptr(2 * NP - 1);  // gate/up: w1, w3; down: w2, w2
    P.ab = (mb_ga_t)(uintptr_t)(kg ? ab1 : ab0) + (row0 + li32) * (uint32_t)NB + kb0;
#pragma unroll
    for (int j = 0; j < kMbFill; ++j) {
      const int r = ch * kMbToks + wave + 8 * j;
      uint32_t fo = kMbOob;
      if (r < cnt) {
        const uint32_t arow = GATEUP ? (uint32_t)s_ptok[off + r] : (uint32_t)(off + r);
        fo = (arow * (uint32_t)K + (kb0 + (uint32_t)fb) * 64u + 8u * fp) * 2u;
      }
      P.fo[j] = fo;
    }
  };

  auto load_w = [&](MbStage<NP> &st, const MbPtr<NP> &Q, int b) {
#pragma unroll
    for (int p = 0; p < NP; ++p)
      st.w[p] = *reinterpret_cast<const MB_GLOBAL u32x4 *>(Q.wb[p] + (w_lane + (uint32_t)b * 32u));
  };
  u32x4 fbuf[kMbFill];
  // Absmax of the lane's row for the 8 blocks of the current chunk (abs_cur) and of the
  // next one (abs_nxt, loaded with the next chunk's activations).
  f32x4 abs_cur[2], abs_nxt[2];
  auto load_fill = [&](const MbPtr<NP> &Q, int c) {
    const uint32_t adv = (uint32_t)c * (kMbChunk * 128u);
    // All lanes of a wave share row wave + 8j of piece set j, so a row past the chunk is a
    // wave-uniform skip: no load is issued for it (its LDS row keeps stale values, which
    // only reach MFMA rows that are never written out).
#pragma unroll
    for (int j = 0; j < kMbFill; ++j)
      if (__builtin_amdgcn_readfirstlane((int)(Q.fo[j] != kMbOob)))
        fbuf[j] = __builtin_amdgcn_raw_buffer_load_b128(rsrc, (int)(Q.fo[j] + adv), 0, 0);
#pragma unroll
    for (int h = 0; h < 2; ++h)
      abs_nxt[h] = *reinterpret_cast<const MB_GLOBAL f32x4 *>(Q.ab + (c * kMbChunk + 4 * h));
  };
  auto store_fill = [&](int buf) {
#pragma unroll
    for (int j = 0; j < kMbFill; ++j)
      *reinterpret_cast<u32x4 *>(&s_ring[buf][fill_lds[j]]) = fbuf[j];
  };

  f32x16 acc[NP];
#pragma unroll
  for (int p = 0; p < NP; ++p)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[p][v] = 0.0f;

  auto compute = [&](const MbStage<NP> &st, const uint8_t *plane, int d) {
    const float own = abs_cur[d >> 2][d & 3];
    float scl[NP];
    if constexpr (NP == 2) {
      const float other = __shfl_xor(own, 32, kWave);
      scl[0] = kg ? other : own;
      scl[1] = kg ? own : other;
    } else {
      scl[0] = own;
    }
    bf16x8 a[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) a[q] = as_bf16x8(*reinterpret_cast<const u32x4 *>(plane + a_lds[q]));
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      f32x16 t;
#pragma unroll
      for (int v = 0; v < 16; ++v) t[v] = 0.0f;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        t = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[q], mb_lookup4(s_tbl, st.w[p][q], lane_const[p]), t,
                                                     0, 0, 0);
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[p][v] = fmaf(scl[p], t[v], acc[p][v]);
    }
  };

  // End of an item: the wave's rows are complete; write them and clear the sums.
  auto finish = [&](int item) {
    int a, ch, sp, g;
    decode(item, a, ch, sp, g);
    const int cnt = ex_field(a, 1), off = ex_field(a, 2);
    const int col = (g * kMbWaves + wave) * kMbRows + li32;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int m = ch * kMbToks + 8 * (v >> 2) + 4 * kg + (v & 3);
      if (m < cnt) {
        const size_t orow = (size_t)(off + m);
        if constexpr (GATEUP)
          h_out[orow * NROWS + col] = swiglu_bf16(acc[0][v], acc[1][v]);
        else
          y_out[((size_t)sp * rows_total + orow) * NROWS + col] = acc[0][v];
      }
    }
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[p][v] = 0.0f;
  };

  // Stream.  P: the item being computed; Pn: the next one (P again after the last).
  MbPtr<NP> P, Pn;
  set_ptrs(P, lo);
  Pn = P;
  if (lo + 1 < hi) set_ptrs(Pn, lo + 1);
  MbStage<NP> st[kMbDepth];
  load_fill(P, 0);
#pragma unroll
  for (int d = 0; d < kMbDepth - 1; ++d) {
    load_w(st[d], P, d);
    __builtin_amdgcn_sched_barrier(0);
  }
  store_fill(0);
  abs_cur[0] = abs_nxt[0];
  abs_cur[1] = abs_nxt[1];
  mb_lds_barrier();
  int q = 0;  // chunk counter: buffer q & 1 holds the current chunk
  for (int item = lo; item < hi; ++item) {
    const bool has_next = item + 1 < hi;
    for (int c = 0; c < n_chunks; ++c) {
      // Source of the next chunk's blocks: this item's chunk c + 1, the next item's chunk
      // 0, or (after the last chunk of the last item) this chunk again, unused.
      const bool in_item = c + 1 < n_chunks;
      const int nc = in_item ? c + 1 : (has_next ? 0 : c);
      const MbPtr<NP> &Q = in_item ? P : Pn;
      const uint8_t *buf = s_ring[q & 1];
#pragma unroll
      for (int d = 0; d < kMbChunk; ++d) {
        if (d == 0) {
          load_w(st[kMbDepth - 1], P, c * kMbChunk + kMbChunk - 1);
          load_fill(Q, nc);
        } else {
          load_w(st[d - 1], Q, nc * kMbChunk + d - 1);
        }
        __builtin_amdgcn_sched_barrier(0);
        compute(st[d], buf + d * kMbPlane, d);
      }
      store_fill((q + 1) & 1);
      abs_cur[0] = abs_nxt[0];
      abs_cur[1] = abs_nxt[1];
      mb_lds_barrier();
      ++q;
    }
    finish(item);
    if (has_next) {
      P = Pn;
      if (item + 2 < hi) set_ptrs(Pn, item + 2);
      if (per_item_table) {
        int a, ch, sp, g;
        decode(item + 1, a, ch, sp, g);
        if (a != tbl_a) {
          tbl_a = a;
          build_table(a);
        }
      }
    }
  }
}

}  // namespace

// Shapes of the streamed mid-batch path: whole groups of eight 32-row tiles per projection,
// K splits of whole activation chunks, activation tensors addressable by a buffer descriptor.
bool midbatch_supported(int32_t H, int32_t F, int32_t nsplit) {
  return H % 512 == 0 && F % 512 == 0 && H >= 512 && F >= 512 && nsplit >= 1 &&
         (F / 64) % (kMbChunk * nsplit) == 0;
}

bool midbatch_rows_ok(int64_t T, int64_t rows_total, int32_t H, int32_t F) {
  return rows_total <= kMbMaxRows && T * (int64_t)H * 2 < ((int64_t)1 << 31) &&
         rows_total * (int64_t)F * 2 < ((int64_t)1 << 31);
}

// K splits of the down projection for a layer whose active experts are at most
// `active_max`: the smallest power of two that gives every CU two items, within the shape.
int midbatch_splits(int64_t active_max, int32_t H, int32_t F) {
  const int64_t want = 2 * (int64_t)device_cu_count();
  int s = 1;
  while (s < 4 && active_max * s * (H / (kMbWaves * kMbRows)) < want && midbatch_supported(H, F, 2 * s))
    s *= 2;
  return s;
}

int launch_midbatch(const void *tab_v, const void *x, int64_t T, int64_t rows_total, int32_t H,
                    int32_t F, const void *route_v, void *h_ws, void *ypart, int32_t nsplit,
                    int phases, hipStream_t stream) {
  MOE_REQUIRE(midbatch_supported(H, F, nsplit), "shape not supported by the streamed mid-batch kernels");
  MOE_REQUIRE(midbatch_rows_ok(T, rows_total, H, F),
              "activations too large for the streamed mid-batch kernels");
  const ExpertTable &tab = *static_cast<const ExpertTable *>(tab_v);
  const Route &rt = *static_cast<const Route *>(route_v);
  const dim3 grid((unsigned)device_cu_count()), blk(kMbThreads);
  if (phases & 1) {
    hipLaunchKernelGGL(midbatch_kernel<2>, grid, blk, 0, stream, tab, (const uint16_t *)x,
                       (uint32_t)(T * H * 2), H, F, rt, (int)rows_total, 1, (uint16_t *)h_ws,
                       (float *)nullptr);
    MOE_LAUNCH_CHECK();
  }
  if (phases & 2) {
    hipLaunchKernelGGL(midbatch_kernel<1>, grid, blk, 0, stream, tab, (const uint16_t *)h_ws,
                       (uint32_t)(rows_total * F * 2), F, H, rt, (int)rows_total, nsplit,
                       (uint16_t *)nullptr, (float *)ypart);
    MOE_LAUNCH_CHECK();
  }
  return MOE_STATUS_OK;
}

}  // namespace moe
