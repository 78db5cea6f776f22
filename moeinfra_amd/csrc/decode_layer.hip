// Decode MoE layer in two launches: routing fused into the NF4 gate/up GEMV, and the
// weighted combine fused into the NF4 down GEMV.  For T <= 4 tokens with T*k <= 8 routed
// slots and E <= 16 experts (Mixtral decode: T = 1, k = 2, E = 8).  The mid-size kernels
// (5 to 64 tokens, 16x16x32 MFMA) follow further down.
//
// Why: at batch 1 a Mixtral layer streams ~198 MB of NF4 weights; every extra kernel
// boundary costs about a microsecond, and any chain of dependent global loads before a
// wave's first weight load delays the whole stream by one memory round trip per link.
// Both kernels run one 8-wave workgroup per CU (one copy of the 64 KB codebook table per
// CU; the CU's waves share its items through an LDS counter).  So:
//
//  decode_gateup_kernel  every workgroup recomputes the routing of the <= 4 tokens (the
//    gate is 64 KB and stays in L2): logits = bf16(x . gate^T) with fp32 accumulation
//    (MFMA), fp32 softmax (+ optional per-expert bias), top-k (descending, ties keep the
//    lower index), renormalised weights, then the grouping of the T*k slots by expert
//    (engine/router.py:50-94, model/moe_layer.py:142-191).  The workgroup then streams
//    its share of the (active expert, 4-row tile) list of w1/w3 and writes
//    h = bf16(silu(bf16(w1 x)) * bf16(w3 x)) per routed row.  Workgroup 0 publishes the
//    routing outputs and a compact descriptor (DecodeRoute) for the down kernel.
//
//  decode_down_kernel  one descriptor load, then each workgroup owns whole 4-row tiles
//    of the output and runs them for every active expert, K split into parts that meet
//    in LDS; each expert's row value is rounded to bf16 (the expert's output dtype) and
//    the slots of each token are combined in ascending expert order,
//    o = bf16(o + bf16(y_e) * w_e) (model/moe_layer.py:147,187-191).
//
// Both kernels stream 4-row tiles through the register pipeline of the 4x4x4 MFMA GEMV
// (gemv4_core.h), with the NF4 codebook table in LDS.
#include <type_traits>

#include "gemv4_core.h"
#include "norm_row.h"

namespace moe {

constexpr int kDecMaxTokens = 4;
constexpr int kDecMaxSlots = 8;
constexpr int kDecMaxExperts = 16;
constexpr int kDecMaxTilesPerWg = 8;
// Both decode kernels run one 8-wave workgroup per CU: one copy of the 64 KB lookup table
// per CU, and the CU's waves share their items through an LDS counter.
constexpr int kDecWaves = 8;
constexpr int kDecThreads = kDecWaves * kWave;
// The down kernel splits K (= F) of every (tile, expert) into at most this many parts.
constexpr int kDecMaxKParts = 8;
// Items per workgroup whose sums the single-token gate/up path keeps in LDS until the end.
constexpr int kRawSlots = 32;
// Multi-token gate/up: the T tokens go to LDS once per workgroup when T * H fits this many
// values (32 KB; the Mixtral step, T = 4 and H = 4096, does).
constexpr int kXtMaxVals = kDecMaxTokens * 4096;


// Routing of one decode step, written by workgroup 0 of the gate/up kernel and read by
// the down kernel.  "Active" experts are those with at least one routed slot, in
// ascending expert order; slot s = t*k + j is the j-th choice of token t.
struct DecodeRoute {
  int32_t n_active;
  int32_t bc;     // every active expert has exactly one token
  int32_t slow1;  // an active expert's w1/w3 codebook differs from the first one's
  int32_t slow2;  // same for w2
  int32_t active[kDecMaxSlots];    // expert id of each active index
  int32_t counts[kDecMaxSlots];    // tokens of each active expert
  int32_t offsets[kDecMaxSlots];   // first h row of each active expert
  int32_t perm_tok[kDecMaxSlots];  // token of each h row
  int32_t slot_a[kDecMaxSlots];    // active index of each slot's expert
  int32_t slot_m[kDecMaxSlots];    // position of the slot's token within its expert's rows
  float slot_w[kDecMaxSlots];      // renormalised routing weight of each slot
  float code2[kDecMaxSlots][16];   // w2 codebook of each active expert
};
static_assert(sizeof(DecodeRoute) % 16 == 0, "descriptor is copied in 16-byte words");

// The post-attention residual add + RMSNorm in front of a single-token layer (the fused
// form of the decoder's norm kernel): x is then the un-normalised attention output,
// r = x + res goes to res_out (workgroup 0) and every workgroup normalises r itself, into
// LDS for the gate products and into its own row of xs for the expert stream.
struct DecodeNorm {
  const uint16_t *res;
  const uint16_t *w;
  float eps;
  uint16_t *res_out;
  uint16_t *xs;  // [gridDim.x][H]
};
constexpr int kDecNormMaxH = 8192;
constexpr int kDecNormChunks = kDecNormMaxH / (kNormThreads * 8);

// The fields of DecodeRoute before code2 (a wave's private copy in the gate/up kernel).
struct RouteHead {
  int32_t n_active, bc, slow1, slow2;
  int32_t active[kDecMaxSlots], counts[kDecMaxSlots], offsets[kDecMaxSlots];
  int32_t perm_tok[kDecMaxSlots], slot_a[kDecMaxSlots], slot_m[kDecMaxSlots];
  float slot_w[kDecMaxSlots];
};
static_assert(offsetof(DecodeRoute, code2) == sizeof(RouteHead), "DecodeRoute starts with RouteHead");
constexpr int kRouteHeadWords = (int)(sizeof(RouteHead) / 4);
constexpr int kRouteWords = (int)(sizeof(DecodeRoute) / 4);
static_assert(kRouteWords <= kDecThreads, "one descriptor word per thread");

namespace {

// Global-memory pointer types.  Pointers read back from LDS are generic to the compiler,
// and generic (flat) loads count against the LDS wait counter too, which would serialise
// the table lookups behind the weight stream; these casts keep the loads global.
#define MOE_GLOBAL __attribute__((address_space(1)))
typedef const MOE_GLOBAL uint8_t *gq_t;
typedef const MOE_GLOBAL float *ga_t;
typedef const MOE_GLOBAL uint16_t *gx_t;

typedef __attribute__((ext_vector_type(4))) unsigned int u32x4_t;
__device__ __forceinline__ uint4 ld_u4(const MOE_GLOBAL void *p) {
  const u32x4_t v = *static_cast<const MOE_GLOBAL u32x4_t *>(p);
  return make_uint4(v.x, v.y, v.z, v.w);
}
// The same load with the non-temporal hint (global_load_dwordx4 ... nt), for the weight
// and absmax streams, which a layer reads exactly once.  A single-pass read of 1 GB streams
// at ~7.0 TB/s this way on MI355X against ~6.1 TB/s with plain loads.
__device__ __forceinline__ uint4 ld_u4_nt(const MOE_GLOBAL void *p) {
  const u32x4_t v = __builtin_nontemporal_load(static_cast<const MOE_GLOBAL u32x4_t *>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// A pointer read from a wave-uniform address, kept in scalar registers (so that lanes can
// select among several such pointers without turning the reads into per-lane loads).
__device__ __forceinline__ const void *uniform_ptr(const void *const &field) {
  const uint64_t v = reinterpret_cast<uint64_t>(field);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return reinterpret_cast<const void *>(((uint64_t)hi << 32) | lo);
}

// Pointers of one pipeline item: NP weight streams (packed bytes and absmax of the lane's
// row, already offset to the item's first stage) and the lane's activation chunk.
template <int NP>
struct ItemPtr {
  gq_t wq[NP];
  ga_t wa[NP];
  gx_t ap;
  ga_t ab[NP];  // absmax of the item's first tile row at its first stage (aligned stream)
  // Activations staged in LDS (aligned stream, kXLds): the lane's 16-byte pieces of stage 0,
  // in 16-byte units from the staging buffer's base (four pieces per group of four token
  // rows, the lane's row of each group, or one quarter with BC); stage s adds 64 s.
  uint32_t xo[16];
};

// Where the aligned stream's activations come from.
constexpr int kXGlobal = 0;  // global memory, loaded with the stage's weights
constexpr int kXRegs = 1;    // registers, loaded once (one token for the whole stream)
constexpr int kXLds = 2;     // the workgroup's LDS copy of the tokens, read a stage ahead

// LDS copy of the T <= 4 tokens of a multi-token decode step: row t holds token t's H
// values as 16-byte pieces; piece i (0..3) of each 64-byte chunk sits at position
// i ^ (t & 3), so that the four lanes of a block, which read the same chunk of four
// different tokens (or four quarters of one token), hit four different bank groups.
typedef const __attribute__((address_space(3))) u32x4_t *lx_t;
__device__ __forceinline__ uint32_t xlds_piece(int t, int H, int piece) {
  return (uint32_t)(t * (H >> 3) + (piece & ~3) + ((piece & 3) ^ (t & 3)));
}

// Streams n_items items of nsq stages each (stage = 4 rows x 256 packed bytes per weight
// stream) through a D-stage register pipeline.  next_item(P) is called once per item, in
// order, and sets P to that item's pointers; finish(acc) receives each item's per-lane
// partial sums (before the cross-lane reduction), again in order; hook() runs once after
// the prologue loads are in flight (every wave calls it exactly once, also without work:
// it may contain workgroup barriers); slow_code() gives the private codebook of the item
// being consumed on the SLOW path and is called in order, once per item.
template <int NP, int D, bool SLOW, bool BC, typename ItemFn, typename FinishFn, typename Hook,
          typename SlowFn>
__device__ __forceinline__ void stream_items(int n_items, int nsq, ItemFn &&next_item,
                                             FinishFn &&finish, Hook &&hook, SlowFn &&slow_code,
                                             const uint32_t *tbl, const uint32_t (&lane_const)[NP],
                                             gq_t dummy) {
  const int total = n_items * nsq;
  if (total <= 0) {
    hook();
    return;
  }
  ItemPtr<NP> P;
  next_item(P);
  int lt = 0, ls = 0;  // next stage to load (item, stage)
  bool past = false;   // past the last stage: the (unused) loads read `dummy`, an L2-resident
                       // buffer, so that re-reads of streamed lines do not go back to HBM
  auto load = [&](Stage4<NP, BC> &st) {
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      st.q[p] = ld_u4_nt(past ? dummy + ls * 256 : P.wq[p] + ls * 256);
      st.s[p] = *(past ? (ga_t)(dummy + ls * 256) : P.wa[p] + ls * 8);
    }
    const gx_t px = P.ap + ls * kStageVals;
#pragma unroll
    for (int i = 0; i < (BC ? 1 : 4); ++i) st.xa[i] = ld_u4(px + 8 * i);
  };
  // Past the last stage the load position saturates and re-reads that stage (unused), so
  // the prefetches need no branch.
  auto advance = [&]() {
    if (++ls == nsq) {
      if (lt + 1 < n_items) {
        ++lt;
        ls = 0;
        next_item(P);
      } else {
        ls = nsq - 1;
        past = true;
      }
    }
  };

  f32x4 acc[NP];
#pragma unroll
  for (int p = 0; p < NP; ++p) acc[p] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  const float *sc = SLOW ? slow_code() : nullptr;
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
            a, b_operand<SLOW>(st.q[p], i, tbl, lane_const[p], sc + 16 * p), t[p], 0, 0, 0);
    }
#pragma unroll
    for (int p = 0; p < NP; ++p) scale_acc(acc[p], t[p], st.s[p]);
  };

  Stage4<NP, BC> st[D];
  // Scheduling barriers keep the prologue loads in stage order (the loop's wait counts
  // must also hold on entry; see expert_gemv4.hip).
#pragma unroll
  for (int d = 0; d < D - 1; ++d) {
    load(st[d]);
    advance();
    __builtin_amdgcn_sched_barrier(0);
  }
  hook();
  int ct = 0, cs = 0;  // item / stage being consumed
  for (int s0 = 0; s0 < total; s0 += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      load(st[(d + D - 1) % D]);
      advance();
      if (s0 + d < total) {
        compute(st[d]);
        if (++cs == nsq) {
          finish(acc);
#pragma unroll
          for (int p = 0; p < NP; ++p) acc[p] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
          cs = 0;
          ++ct;
          if (SLOW && ct < n_items) sc = slow_code();
        }
      }
    }
  }
}

// Aligned stream: every item has exactly NSQ stages (2 <= NSQ <= 8) and the register
// pipeline is DEPTH stages deep with DEPTH dividing NSQ, so unrolled step d always handles
// stage d of an item and buffer d % DEPTH.  That allows
//  * the item's absmax block (4 rows x 8*NSQ floats) to be fetched with one 16-byte load
//    per lane when the load side enters the item, and staged in the wave's LDS slot at
//    the item boundary, instead of one 4-byte load per lane and stage;
//  * with XREG (one token for the whole stream, single-token broadcast form), the
//    activation chunks of all NSQ stages to stay in registers, loaded once.
// Items come from grab() (wave-uniform item index, negative when none is left), taken one
// item ahead, so the waves of a workgroup can share a work counter; set_ptrs(P, item) sets
// the pointers of an item and finish(acc, item) receives its per-lane partial sums (before
// the cross-lane reduction).  Step d of an item issues the load of stage d + DEPTH - 1 of
// the stage sequence: stage d + DEPTH - 1 of this item, or stage d + DEPTH - 1 - NSQ of the
// next one (after the last item, a re-read of this item's stages, unused).  At most DEPTH
// stages per projection are in flight per wave: the depth sets the bytes a wave keeps
// outstanding.  With LA the table lookups of a stage are issued one step ahead of its
// products, so that their LDS latency overlaps the MFMAs.  hook() runs once after the
// prologue (every wave calls it exactly once, also without work).  `arow` is the absmax row
// stride (floats), `aslot` the wave's LDS slot (NP x kASlotFloats), `xbase` the lane's
// activation chunk of stage 0 (XREG only).  With BC the four MFMA result rows are the same
// token, and only row 0 of `acc` is accumulated (finish must read row 0 only).
// Per-wave absmax slot of one item: 4 rows of up to 64 floats, rows padded to 72 floats so
// that the four rows read in one instruction fall into different LDS banks.
constexpr int kASlotRow = 72;
constexpr int kASlotFloats = 4 * kASlotRow;

// The 16-level NF4 codebook (QLoRA; bitsandbytes' NF4 table, the `code` tensor of the quant
// state, transfer/nf4_reconstruct.py:48) as fp32: the decode kernels build their lookup
// table from these values and route experts whose codebooks differ to the per-nibble path.
constexpr float kNf4Code[16] = {
    -1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f,
    -0.28444138169288635f, -0.18477343022823334f, -0.09105003625154495f, 0.0f,
    0.07958029955625534f, 0.16093020141124725f, 0.24611230194568634f, 0.33791524242401123f,
    0.44070982933044434f, 0.5626170039176941f, 0.7229568362236023f, 1.0f};

#ifndef MOE_GATEUP_DEPTH
#define MOE_GATEUP_DEPTH 4
#endif
// Pipeline depth of the single-token gate/up stream (stages of both projections).
constexpr int kGateUpDepth = MOE_GATEUP_DEPTH;
#ifndef MOE_LOOKAHEAD
#define MOE_LOOKAHEAD 1
#endif
// Table lookups one stage ahead of the products in the aligned stream.
constexpr bool kLookahead = MOE_LOOKAHEAD != 0;

template <int NP, int NX>
struct StageQ {
  uint4 q[NP];
  uint4 xa[NX];
};
template <int NP>
struct StageQ<NP, 0> {
  uint4 q[NP];
};

// XREG activations from global memory or, for the fused-norm kernel, from LDS.
__device__ __forceinline__ uint4 ld_x(gx_t p) { return ld_u4(p); }
__device__ __forceinline__ uint4 ld_x(const uint16_t *lds_p) {
  return *reinterpret_cast<const uint4 *>(lds_p);
}

template <int NP, int NSQ, int DEPTH, bool BC, int XM, bool LA, int NG = 1, bool XFIX = false,
          typename GrabFn, typename PtrFn, typename FinishFn, typename Hook, typename XPtr>
__device__ __forceinline__ void stream_aligned(GrabFn &&grab, PtrFn &&set_ptrs,
                                               FinishFn &&finish, Hook &&hook,
                                               const uint32_t *tbl,
                                               const uint32_t (&lane_const)[NP], size_t arow,
                                               float *aslot, XPtr xbase, gq_t dummy) {
  static_assert(NSQ >= 2 && NSQ <= 8, "an item's absmax block must fit one load per lane");
  static_assert(DEPTH >= 2 && DEPTH <= NSQ && NSQ % DEPTH == 0, "depth must divide NSQ");
  static_assert(!LA || DEPTH >= 3, "lookahead needs depth >= 3");
  static_assert(XM != kXLds || LA, "LDS activations are read in the lookahead slot");
  static_assert(NG == 1 || (XM == kXLds && !BC && NG <= 4), "token groups: LDS activations");
  constexpr bool XREG = XM == kXRegs;
  constexpr bool XLDS = XM == kXLds;
  constexpr int NX = XREG ? 1 : (BC ? 1 : 4);
  constexpr int NXG = NX * NG;  // LDS activation pieces per lane and stage
  // First step that loads a stage of the next item.
  constexpr int kNext = NSQ - DEPTH + 1;
  const int lane = threadIdx.x & (kWave - 1);
  const int blk = lane >> 2;
  const int j = lane & 3;
  int cur = grab();
  if (cur < 0) {
    hook();
    return;
  }
  // This lane's absmax chunk: row a_row, floats a_col .. a_col+3 (lanes >= 8*NSQ idle).
  const bool a_act = lane < 8 * NSQ;
  const int a_row = a_act ? lane / (2 * NSQ) : 0;
  const int a_col = a_act ? 4 * (lane % (2 * NSQ)) : 0;

  ItemPtr<NP> P;
  set_ptrs(P, cur);
  uint4 abuf[NP];
  auto load_abs = [&]() {
#pragma unroll
    for (int p = 0; p < NP; ++p) abuf[p] = ld_u4_nt(P.ab[p] + a_row * arow + a_col);
  };
  auto store_abs = [&]() {
    if (a_act) {
#pragma unroll
      for (int p = 0; p < NP; ++p)
        *reinterpret_cast<uint4 *>(aslot + p * kASlotFloats + a_row * kASlotRow + a_col) = abuf[p];
    }
    wave_lds_sync();  // every lane reads chunks other lanes stored
  };
  uint4 xr[XREG ? NSQ : 1];
  if (XREG) {
#pragma unroll
    for (int sg = 0; sg < NSQ; ++sg) xr[sg] = ld_x(xbase + sg * kStageVals);
  }
  load_abs();
  auto load = [&](StageQ<NP, XM == kXGlobal ? NX : 0> &st, int sg) {
#pragma unroll
    for (int p = 0; p < NP; ++p) st.q[p] = ld_u4_nt(P.wq[p] + sg * 256);
    if constexpr (XM == kXGlobal) {
      const gx_t px = P.ap + sg * kStageVals;
#pragma unroll
      for (int i = 0; i < NX; ++i) st.xa[i] = ld_u4(px + 8 * i);
    }
  };
  // kXLds: the current stage's activations (xc), read from LDS right after the previous
  // stage's products have used the registers; xoc holds the current item's piece offsets
  // (P moves on to the next item at step kNext).  XFIX: every item reads the same rows, so
  // the first item's offsets serve all of them.
  uint4 xc[XLDS ? NXG : 1];
  uint32_t xoc[XLDS ? NXG : 1];
  auto lds_x = [&](uint4 (&dst)[XLDS ? NXG : 1], const uint32_t (&xo)[XLDS ? NXG : 1], int sg) {
    if constexpr (XLDS) {
      const lx_t xl = (lx_t)xbase;
#pragma unroll
      for (int i = 0; i < NXG; ++i) {
        const u32x4_t v = xl[xo[i] + 64 * sg];
        dst[i] = make_uint4(v.x, v.y, v.z, v.w);
      }
    }
  };
  if constexpr (XLDS) {
#pragma unroll
    for (int i = 0; i < NXG; ++i) xoc[i] = P.xo[i];
    lds_x(xc, xoc, 0);
  }
  StageQ<NP, XM == kXGlobal ? NX : 0> st[DEPTH];
#pragma unroll
  for (int d = 0; d < DEPTH - 1; ++d) {
    load(st[d], d);
    __builtin_amdgcn_sched_barrier(0);
  }
  store_abs();
  hook();
  // The next two items are known ahead, and the next item's pointers are set up at the
  // start of the current one: the work counter's and the LDS tables' latencies stay off
  // the step that switches the loads to the next item.
  int nxt = grab();
  int nxt2 = nxt >= 0 ? grab() : -1;
  ItemPtr<NP> Pn = P;
  if (nxt >= 0) set_ptrs(Pn, nxt);

  // Per projection p and token group g: acc[p * NG + g].
  f32x4 acc[NP * NG];
#pragma unroll
  for (int p = 0; p < NP * NG; ++p) acc[p] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  s16x4 bq[LA ? NP : 1][8];
  if (LA) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int p = 0; p < NP; ++p) bq[p][i] = b_operand<false>(st[0].q[p], i, tbl, lane_const[p], nullptr);
  }
  for (;;) {
#pragma unroll
    for (int d = 0; d < NSQ; ++d) {
      if (d == kNext) {
        if (nxt >= 0) {
          P = Pn;
          load_abs();
        } else {
          // Past the last item the loads re-read stages already streamed (unused): point
          // them at `dummy`, an L2-resident buffer, instead of lines that the non-temporal
          // loads have let go.
#pragma unroll
          for (int p = 0; p < NP; ++p) P.wq[p] = dummy + (lane >> 2) * 16;
        }
      }
      const int g = d + DEPTH - 1;  // stage sequence index of this step's load
      load(st[g % DEPTH], g < NSQ ? g : g - NSQ);
      __builtin_amdgcn_sched_barrier(0);  // this step's loads before its products
      const StageQ<NP, XM == kXGlobal ? NX : 0> &cs = st[d % DEPTH];
      const uint4 *xa;
      if constexpr (XM == kXGlobal)
        xa = cs.xa;
      else if constexpr (XREG)
        xa = &xr[d];
      else
        xa = xc;
      float scl[NP];
#pragma unroll
      for (int p = 0; p < NP; ++p) scl[p] = aslot[p * kASlotFloats + j * kASlotRow + 8 * d + (blk >> 1)];
      f32x4 t[NP * NG];
#pragma unroll
      for (int p = 0; p < NP * NG; ++p) t[p] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      if (LA) {
        // Stage d+1 is in buffer (d+1) % DEPTH (for d = NSQ-1: the next item's stage 0, or
        // a re-read of this item's when it is the last one).
        const StageQ<NP, XM == kXGlobal ? NX : 0> &ns = st[(d + 1) % DEPTH];
        s16x4 bn[LA ? NP : 1][8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
#pragma unroll
          for (int p = 0; p < NP; ++p) bn[p][i] = b_operand<false>(ns.q[p], i, tbl, lane_const[p], nullptr);
#pragma unroll
          for (int g = 0; g < NG; ++g) {
            const s16x4 a = a_operand<BC>(xa + g * NX, i);
#pragma unroll
            for (int p = 0; p < NP; ++p)
              t[p * NG + g] = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(a, bq[p][i], t[p * NG + g], 0, 0, 0);
          }
        }
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
          for (int p = 0; p < NP; ++p) bq[p][i] = bn[p][i];
        if constexpr (XLDS) {
          // Stage d + 1 of this item, or (d = NSQ - 1) stage 0 of the next one, whose
          // pointers P holds since step kNext (the current item's again after the last).
          if (d + 1 < NSQ) {
            lds_x(xc, xoc, d + 1);
          } else if (XFIX) {  // every item reads the same rows
            lds_x(xc, xoc, 0);
          } else {
            uint32_t xo_n[NXG];
#pragma unroll
            for (int i = 0; i < NXG; ++i) xo_n[i] = P.xo[i];
            lds_x(xc, xo_n, 0);
          }
        }
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const s16x4 a = a_operand<BC>(xa, i);
#pragma unroll
          for (int p = 0; p < NP; ++p)
            t[p] = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(
                a, b_operand<false>(cs.q[p], i, tbl, lane_const[p], nullptr), t[p], 0, 0, 0);
        }
      }
#pragma unroll
      for (int p = 0; p < NP; ++p) {
#pragma unroll
        for (int g = 0; g < NG; ++g) {
          if (BC)  // one token in every row: only row 0 is accumulated
            acc[p][0] = fmaf(scl[p], t[p][0], acc[p][0]);
          else
            scale_acc(acc[p * NG + g], t[p * NG + g], scl[p]);
        }
      }
    }
    finish(acc, cur);
#pragma unroll
    for (int p = 0; p < NP * NG; ++p) acc[p] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    if (nxt < 0) break;
    store_abs();
    if constexpr (XLDS && !XFIX) {
#pragma unroll
      for (int i = 0; i < NXG; ++i) xoc[i] = P.xo[i];
    }
    cur = nxt;
    nxt = nxt2;
    if (nxt >= 0) set_ptrs(Pn, nxt);
    nxt2 = nxt >= 0 ? grab() : -1;
  }
}

// 64 KB lookup table (see nf4_tile.h) from codebooks held in registers, by NT threads.
// Word 64*v + r holds the bf16 pair of packed byte v for replica r; replicas 0-31 use c_a,
// 32-63 use c_b, so four consecutive replicas hold the same word.  Store s (words 4s ..
// 4s+3, one 16-byte store) covers byte v = s/16 (high nibble v >> 4, low nibble v & 15)
// and replicas 4*(s%16) .. +3; thread tid makes stores s = tid + NT*r, r < 4096/NT, so its
// low nibble and replica half are fixed and its high nibble is tid/256 + (NT/256)*r.
template <int NT>
__device__ __forceinline__ void build_table_regs(uint32_t *tbl, const float (&c_a)[16],
                                                 const float (&c_b)[16]) {
  static_assert(NT % 256 == 0 && 4096 % NT == 0, "NT must be 256, 512, 1024, ...");
  constexpr int R = 4096 / NT;
  constexpr int HS = NT / 256;
  const int tid = threadIdx.x;
  const bool second = (tid & 8) != 0;  // replica 4*(tid%16) >= 32
  const int lo_nib = (tid >> 4) & 15;
  const int hi0 = tid >> 8;  // < HS
  // Selections on values (each array element read with a constant index), so that two
  // different codebooks never turn into a select between the arrays themselves.
  float lo_a = c_a[0], lo_b = c_b[0];
#pragma unroll
  for (int i = 1; i < 16; ++i) {
    const float va = c_a[i], vb = c_b[i];
    lo_a = i == lo_nib ? va : lo_a;
    lo_b = i == lo_nib ? vb : lo_b;
  }
  const float lo = second ? lo_b : lo_a;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float hi_a = c_a[HS * r], hi_b = c_b[HS * r];
#pragma unroll
    for (int h = 1; h < HS; ++h) {
      const float va = c_a[HS * r + h], vb = c_b[HS * r + h];
      hi_a = hi0 == h ? va : hi_a;
      hi_b = hi0 == h ? vb : hi_b;
    }
    const float hi = second ? hi_b : hi_a;
    const uint32_t w = pack_bf16x2(hi, lo);
    *reinterpret_cast<uint4 *>(tbl + 4 * (tid + NT * r)) = make_uint4(w, w, w, w);
  }
}

// Reductions over the 16 lanes of a DPP row (every lane of the row gets the result).
__device__ __forceinline__ float row_max16(float v) {
  v = fmaxf(v, dpp_mov<0xB1>(v));   // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp_mov<0x4E>(v));   // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp_mov<0x124>(v));  // row_ror:4
  v = fmaxf(v, dpp_mov<0x128>(v));  // row_ror:8
  return v;
}
__device__ __forceinline__ float row_sum16(float v) {
  v += dpp_mov<0xB1>(v);
  v += dpp_mov<0x4E>(v);
  v += dpp_mov<0x124>(v);
  v += dpp_mov<0x128>(v);
  return v;
}

// Routing of the T <= 4 tokens by one wave, lane (t = lane/16, e = lane%16) holding
// expert e of token t: fp32 sum of the NW waves' gate partials in wave order -> bf16
// logit (+ bias) -> fp32 softmax over the row -> top-k by k rounds of row arg-max (ties:
// the lowest expert index) -> weights renormalised by their sum in rank order.  Then the
// grouping of the T*k slots (s = t*k + j) by expert, ascending expert and ascending slot,
// written to `rh` (in LDS; the caller publishes it to the other waves).
struct RouteSummary {
  int n_active;      // wave-uniform
  bool bc;
  uint32_t present;  // bit x: expert x has a slot
};

// The per-token part of the routing, for tokens t0 + lane / 16 (those below T): lane
// (t, e) sums expert e's NW wave partials s_part[w][t0 + t][e] in wave order, and lane j
// of the row ends with choice j (expert my_win, renormalised weight my_wn), also stored at
// slot (t0 + t) * k + j of sl_e / sl_w.
struct RowRoute {
  int my_win;
  float my_wn;
  bool valid, taken;
};

template <int EMAX, int NW, int TD>
__device__ __forceinline__ RowRoute route_rows(int32_t *sl_e, float *sl_w,
                                               const float (*s_part)[TD][EMAX], int t0,
                                               const float *bias, int T, int E, int k,
                                               uint16_t *logits_out) {
  const int lane = threadIdx.x & (kWave - 1);
  const int t = t0 + (lane >> 4);
  const int e = lane & 15;
  const bool valid = t < T && e < E;
  float l = -INFINITY;
  if (valid) {
    float v = s_part[0][t][e];
#pragma unroll
    for (int w = 1; w < NW; ++w) v += s_part[w][t][e];
    const uint16_t lb = f32_to_bf16(v);
    if (logits_out != nullptr) logits_out[t * E + e] = lb;
    l = bf16_to_f32(lb);
    if (bias != nullptr) l = l + bias[e];
  }
  const float m = row_max16(l);
  const float pe = valid ? expf(l - m) : 0.0f;
  const float p = pe / row_sum16(pe);
  bool taken = false;
  float wsum = 0.0f, my_w = 0.0f;
  int my_win = 0;
  const int row = lane >> 4;
  for (int j = 0; j < k; ++j) {
    const bool cand = valid && !taken;
    const float best = row_max16(cand ? p : -1.0f);
    const uint64_t hit = __ballot(cand && p == best);
    const uint64_t any = __ballot(cand);
    int win = __builtin_ctzll(((hit >> (16 * row)) & 0xffffull) | 0x10000ull);  // row's lowest
    // No lane equal to the maximum (NaN weights): the lowest untaken expert, as a strict
    // '>' scan starting from "no choice yet" picks.
    if (win > 15) win = __builtin_ctzll(((any >> (16 * row)) & 0xffffull) | 0x10000ull);
    if (win > 15) win = 0;
    taken |= e == win;
    wsum += best;
    if (e == j) {  // lane j of the row keeps choice j
      my_win = win;
      my_w = best;
    }
  }
  const float my_wn = my_w / wsum;
  if (t < T && e < k) {
    sl_e[t * k + e] = my_win;
    sl_w[t * k + e] = my_wn;
  }
  return RowRoute{my_win, my_wn, valid, taken};
}

template <int EMAX, int NW>
__device__ __forceinline__ RouteSummary route_wave(RouteHead &rh, int32_t (&sl_e)[kDecMaxSlots],
                                           float (&sl_w)[kDecMaxSlots],
                                           const float (*s_part)[kDecMaxTokens][EMAX],
                                           const float *bias, int T, int E, int k,
                                           uint16_t *logits_out) {
  const int lane = threadIdx.x & (kWave - 1);
  const RowRoute rr = route_rows<EMAX, NW, kDecMaxTokens>(sl_e, sl_w, s_part, 0, bias, T, E, k,
                                                          logits_out);
  const int my_win = rr.my_win;
  const float my_wn = rr.my_wn;
  const bool valid = rr.valid, taken = rr.taken;
  if (T == 1) {
    // One token: its k slots have k distinct experts, so each active expert holds exactly
    // one slot, at the rank of its id among the chosen ones -- the same descriptor as the
    // general grouping below, without gathering the slots.
    const uint32_t present = (uint32_t)(__ballot(valid && taken) & 0xffffull);
    if (lane < k) {
      const int a = __builtin_popcount(present & ((1u << my_win) - 1u));
      rh.perm_tok[a] = 0;
      rh.slot_a[lane] = a;
      rh.slot_m[lane] = 0;
      rh.slot_w[lane] = my_wn;
      rh.active[a] = my_win;
      rh.counts[a] = 1;
      rh.offsets[a] = a;
    }
    if (lane == 0) {
      rh.n_active = k;
      rh.bc = 1;
    }
    wave_lds_sync();
    return RouteSummary{k, true, present};
  }
  // Grouping of the ns = T*k slots (slot s = t*k + j lives in lane 16*(s/k) + s%k): the
  // slot experts are gathered into scalars, then lane s < ns places its slot with a few
  // compares against them -- no loop over the experts, no LDS round trip.
  const int ns = T * k;
  int se[kDecMaxSlots];
  float sw[kDecMaxSlots];
  int stok[kDecMaxSlots];
  uint32_t present = 0;
  int tq = 0, jq = 0;  // token and choice of slot q
#pragma unroll
  for (int q = 0; q < kDecMaxSlots; ++q) {
    const int src = q < ns ? 16 * tq + jq : 0;
    se[q] = q < ns ? __builtin_amdgcn_readlane(my_win, src) : 0x7fff;
    sw[q] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_wn), src));
    stok[q] = tq;
    if (q < ns) present |= 1u << se[q];
    if (++jq == k) {
      jq = 0;
      ++tq;
    }
  }
  int my_e = se[0], my_tok = stok[0];
  float my_sw = sw[0];
#pragma unroll
  for (int q = 1; q < kDecMaxSlots; ++q)
    if (lane == q) {
      my_e = se[q];
      my_sw = sw[q];
      my_tok = stok[q];
    }
  int before = 0, same = 0, rank = 0;  // slots of smaller experts / of mine / of mine before me
#pragma unroll
  for (int q = 0; q < kDecMaxSlots; ++q) {
    before += se[q] < my_e ? 1 : 0;
    same += se[q] == my_e ? 1 : 0;
    rank += (se[q] == my_e && q < lane) ? 1 : 0;
  }
  const int my_a = __builtin_popcount(present & ((1u << my_e) - 1u));  // active index
  const int n_active = __builtin_popcount(present);
  const bool multi = __ballot(lane < ns && same > 1) != 0;
  if (lane < ns) {
    rh.perm_tok[before + rank] = my_tok;
    rh.slot_a[lane] = my_a;
    rh.slot_m[lane] = rank;
    rh.slot_w[lane] = my_sw;
    if (rank == 0) {  // the first slot of each expert describes it
      rh.active[my_a] = my_e;
      rh.counts[my_a] = same;
      rh.offsets[my_a] = before;
    }
  }
  if (lane == 0) {
    rh.n_active = n_active;
    rh.bc = multi ? 0 : 1;
  }
  wave_lds_sync();  // rh is read by every lane of the wave afterwards
  return RouteSummary{n_active, !multi, present};
}

template <int EMAX, bool NORM, bool N1 = false>
__global__ void __launch_bounds__(kDecThreads, 1)
decode_gateup_kernel(const ExpertTable tab, const uint16_t *__restrict__ x,
                     const uint16_t *__restrict__ gate, const float *__restrict__ bias, int T,
                     int H, int F, int E, int k, uint16_t *__restrict__ logits_out,
                     float *__restrict__ w_out, int64_t *__restrict__ idx_out,
                     DecodeRoute *__restrict__ route_out, uint16_t *__restrict__ h_out,
                     const DecodeNorm nrm) {
  __shared__ __attribute__((aligned(16))) uint32_t s_tbl[kTableWords];
  __shared__ float s_part[kDecWaves][kDecMaxTokens][EMAX];
  // Codebooks of every expert: [0,16) w1, [16,32) w3, [32,48) w2 ([48,64) repeats w2).
  __shared__ float s_code[EMAX][kWave];
  __shared__ const void *s_eptr[EMAX][4];  // w1_packed, w1_absmax, w3_packed, w3_absmax
  __shared__ __attribute__((aligned(16))) RouteHead s_rt;  // routing of the workgroup
  __shared__ int32_t s_sle[kDecMaxSlots];                    // slot experts
  __shared__ float s_slw[kDecMaxSlots];                      // slot weights
  __shared__ __attribute__((aligned(16))) uint8_t s_slowbits[16];  // per-expert codebook flags
  __shared__ __attribute__((aligned(16))) float s_aslot[kDecWaves][2 * kASlotFloats];
  __shared__ int32_t s_ticket;  // next item of the workgroup's range (single-token path)
  // Single-token path: per item of the workgroup, the per-lane sums of w1 and w3 (row
  // j = lane % 4 of the tile, block lane / 4).
  __shared__ float s_raw[kRawSlots][2][kWave];
  __shared__ uint8_t s_mine[kDecWaves][kRawSlots];  // the raw slots each wave filled
  // NORM or N1: the token the gate products and the single-token stream read (normalised
  // with NORM), and the norm's wave sums.
  __shared__ __attribute__((aligned(16))) uint16_t s_xn[NORM || N1 ? kDecNormMaxH : 8];
  __shared__ float s_npart[kDecWaves];
  __shared__ float s_nsq[N1 ? kNormThreads : 1][4];  // N1: the second half's squared pairs
  // Multi-token steps (no fused norm): the tokens, swizzled as xlds_piece describes.
  __shared__ uint4 s_xt[NORM || N1 ? 1 : kXtMaxVals / 8];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool wg0 = blockIdx.x == 0;
  if (tid == 0) s_ticket = 0;
  // NORM: the norm's loads (x, residual, weight; L2-resident) go first, so that waiting
  // for them does not wait for the gate rows issued after them.  N1 (H <= 4096): one chunk
  // per thread of the workgroup; otherwise threads 0..255 take up to four and the other
  // waves repeat loads (unused): no load behind a branch.  N1 without NORM (one token):
  // the token is copied into s_xn one 16-byte chunk per thread, and the gate products and
  // the stream read it there as they read the normalised token.
  NormRegs<N1 ? 1 : kDecNormChunks> ng;
  NormOneRegs n1;
  uint4 xcopy;  // N1 without NORM: this thread's chunk of the token (a plain register value)
  if (NORM) {
    if constexpr (N1)
      norm_load_one<true>(n1, x, nrm.res, nrm.w, H);
    else
      norm_load<kDecNormChunks, true>(ng, x, nrm.res, nrm.w, H);
    __builtin_amdgcn_sched_barrier(0);  // keep them ahead of the gate rows
  } else if constexpr (N1) {
    xcopy = *reinterpret_cast<const uint4 *>(x + (tid * 8 < H ? tid * 8 : H - 8));
    __builtin_amdgcn_sched_barrier(0);  // keep it ahead of the gate rows
  }
  // The token the expert stream reads: x, or this workgroup's row of normalised values.
  const uint16_t *xt = NORM ? nrm.xs + (size_t)blockIdx.x * H : x;

  // ---- gate products on the 4x4x4 MFMA: wave w takes the 128-value chunks c = w, w + 8,
  // ... of H; lane (b = lane/4, j = lane%4) holds values 8b .. 8b+7 of a chunk of token j
  // (A rows; tokens >= T repeat a valid row and are ignored) and of expert 4g + j (B
  // columns).  D[b][m][n] sums block b's slice for token m and expert 4g + n; a butterfly
  // over the 16 blocks completes the wave's partial sums.
  constexpr int G = EMAX / 4;                 // expert groups of four
  constexpr int CPR = EMAX <= 8 ? 4 : 2;      // chunks per load round
  const int lj = lane & 3;
  const int lb = lane >> 2;
  const int n_chunks = (H / 128 - wave + kDecWaves - 1) / kDecWaves;  // this wave's chunks
  // A wave without chunks (H < 1024) still issues its first round, on chunk 0 (in bounds,
  // unused): a load behind a branch would make every later wait count it as possibly
  // missing, i.e. wait for the loads issued after it too.
  const int wq = n_chunks > 0 ? wave : 0;
  const gx_t xrow = (gx_t)x + (size_t)(lj < T ? lj : T - 1) * H + (size_t)wq * 128 + 8 * lb;
  gx_t grow[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int e = 4 * g + lj;
    grow[g] = (gx_t)gate + (size_t)(e < E ? e : E - 1) * H + (size_t)wq * 128 + 8 * lb;
  }
  f32x4 gacc[G];
#pragma unroll
  for (int g = 0; g < G; ++g) gacc[g] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  uint4 xv[CPR], gv[CPR][G];
  auto load_round = [&](int c0) {
#pragma unroll
    for (int c = 0; c < CPR; ++c) {
      const int cc = c0 + c < n_chunks ? c0 + c : 0;  // past the end: chunk 0 again, unused
      if (!NORM && !N1) xv[c] = ld_u4(xrow + (size_t)cc * (128 * kDecWaves));
#pragma unroll
      for (int g = 0; g < G; ++g) gv[c][g] = ld_u4(grow[g] + (size_t)cc * (128 * kDecWaves));
    }
  };
  load_round(0);
  // Multi-token steps: this thread's pieces of the tokens for the LDS copy (stored before
  // the routing barrier).  Only T > 1 loads them; on the single-token path the compiler's
  // waits stay exact.
  const bool xlds = !NORM && !N1 && T > 1 && T * H <= kXtMaxVals;  // N1 runs one token only
  constexpr int kXtPer = kXtMaxVals / 8 / kDecThreads;  // pieces per thread at most
  uint4 xtv[kXtPer];
  if (xlds) {
#pragma unroll
    for (int r = 0; r < kXtPer; ++r) {
      const int q = tid + kDecThreads * r;
      if (q < T * (H >> 3)) xtv[r] = ld_u4((gx_t)x + (size_t)q * 8);
    }
  }
  // Metadata of experts wave + 8q (wave-uniform, so the table entries are scalar loads):
  // lane l < 16 reads w1 code[l], 16..31 w3 code[l-16], 32..63 w2 code[l & 15]; lane f < 4
  // keeps stream pointer f (w1_packed, w1_absmax, w3_packed, w3_absmax).
  constexpr int EPW = (EMAX + kDecWaves - 1) / kDecWaves;
  float cvw[EPW];
  const void *pvw[EPW];
#pragma unroll
  for (int q = 0; q < EPW; ++q) {
    const int e = wave + kDecWaves * q;
    const moe_nf4_expert_t &ex = tab.e[e < E ? e : E - 1];
    const void *c1 = uniform_ptr(ex.w1_code), *c3 = uniform_ptr(ex.w3_code);
    const void *c2 = uniform_ptr(ex.w2_code);
    const void *p1 = uniform_ptr(ex.w1_packed), *a1 = uniform_ptr(ex.w1_absmax);
    const void *p3 = uniform_ptr(ex.w3_packed), *a3 = uniform_ptr(ex.w3_absmax);
    const void *cp = lane < 16 ? c1 : lane < 32 ? c3 : c2;
    cvw[q] = ((ga_t)cp)[lane & 15];
    const int f = lane & 3;
    pvw[q] = f == 0 ? p1 : f == 1 ? a1 : f == 2 ? p3 : a3;
  }
  // ---- lookup table from the NF4 codebook constants, written while the loads above are
  // in flight.  Experts whose codebooks differ from these values take the per-nibble path.
  __builtin_amdgcn_sched_barrier(0);
  {
    float cst[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) cst[q] = kNf4Code[q];
    build_table_regs<kDecThreads>(s_tbl, cst, cst);
  }
  __builtin_amdgcn_sched_barrier(0);
  if (NORM) {
    // r = x + res (workgroup 0 writes it), xn = rmsnorm(r) with the sums of the 256-thread
    // norm kernel, into LDS (the single-token stream reads it there; other paths copy it to
    // the workgroup's xs row first).
    if constexpr (N1)
      norm_finish_one<true>(n1, nrm.eps, H, wg0 ? nrm.res_out : nullptr, s_xn, s_npart, s_nsq);
    else
      norm_finish<kDecNormChunks, true>(ng, nrm.eps, H, wg0 ? nrm.res_out : nullptr, s_xn, s_npart,
                                        tid < kNormThreads);
    lds_barrier();
  } else if constexpr (N1) {
    if (tid * 8 < H) *reinterpret_cast<uint4 *>(s_xn + tid * 8) = xcopy;
    lds_barrier();
  }
  for (int c0 = 0; c0 < n_chunks; c0 += CPR) {
    if (c0 > 0) {
      load_round(c0);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (NORM || N1) {  // this round's x chunks from LDS (T = 1)
#pragma unroll
      for (int c = 0; c < CPR; ++c) {
        const int cc = c0 + c < n_chunks ? c0 + c : 0;
        xv[c] = *reinterpret_cast<const uint4 *>(s_xn + (size_t)wq * 128 + 8 * lb +
                                                 (size_t)cc * (128 * kDecWaves));
      }
    }
#pragma unroll
    for (int c = 0; c < CPR; ++c) {
      if (c0 + c >= n_chunks) break;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const s16x4 av = h ? as_s16x4(xv[c].z, xv[c].w) : as_s16x4(xv[c].x, xv[c].y);
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const s16x4 bv = h ? as_s16x4(gv[c][g].z, gv[c][g].w) : as_s16x4(gv[c][g].x, gv[c][g].y);
          gacc[g] = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(av, bv, gacc[g], 0, 0, 0);
        }
      }
    }
  }
  // Butterfly over the blocks for the T token rows; lane j of block 0 writes the wave's
  // partial sums of experts 4g + j.
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int m = 0; m < kDecMaxTokens; ++m) {
      if (m < T) {
        const float v = lanes_sum16(gacc[g][m]);
        const int e = 4 * g + lj;
        if (lb == 0 && e < E) s_part[wave][m][e] = v;
      }
    }
  // Unconditional stores (clamped experts rewrite identical values), and each expert's
  // codebook check against the table's NF4 values: bit 0 when its w1 or w3 codebook
  // differs (lanes 0..31), bit 1 for w2 (lanes 32..47).
  float ref_f = kNf4Code[0];
#pragma unroll
  for (int q = 1; q < 16; ++q)
    if ((lane & 15) == q) ref_f = kNf4Code[q];
  const uint32_t ref = __builtin_bit_cast(uint32_t, ref_f);
#pragma unroll
  for (int q = 0; q < EPW; ++q) {
    const int e = wave + kDecWaves * q;
    const int ee = e < E ? e : E - 1;
    s_code[ee][lane] = cvw[q];
    s_eptr[ee][lane & 3] = pvw[q];
    const bool diff = __builtin_bit_cast(uint32_t, cvw[q]) != ref;
    const bool d1 = __ballot(lane < 32 && diff) != 0;
    const bool d2 = __ballot(lane >= 32 && lane < 48 && diff) != 0;
    if (lane == 0) s_slowbits[ee] = (uint8_t)((d1 ? 1 : 0) | (d2 ? 2 : 0));
  }
  if (xlds) {
#pragma unroll
    for (int r = 0; r < kXtPer; ++r) {
      const int q = tid + kDecThreads * r;
      const int t = q / (H >> 3);
      if (q < T * (H >> 3)) s_xt[xlds_piece(t, H, q - t * (H >> 3))] = xtv[r];
    }
  }
  // Gate sums, codebooks, stream pointers, the lookup table, the work counter and the token
  // copy are visible to every wave after this barrier.
  __syncthreads();

  // ---- routing and grouping by wave 0 (one wave, so that the SIMDs do not run the same
  // serial code eight times); the other waves wait at the barrier.
  const int ns = T * k;
  if (wave == 0) {
    // The codebook flags of all experts, as four words of four bytes.
    const uint4 fb = *reinterpret_cast<const uint4 *>(s_slowbits);
    const RouteSummary rs = route_wave<EMAX, kDecWaves>(s_rt, s_sle, s_slw, s_part, bias, T, E, k,
                                                        wg0 ? logits_out : nullptr);
    const uint32_t fw[4] = {(uint32_t)__builtin_amdgcn_readfirstlane(fb.x),
                            (uint32_t)__builtin_amdgcn_readfirstlane(fb.y),
                            (uint32_t)__builtin_amdgcn_readfirstlane(fb.z),
                            (uint32_t)__builtin_amdgcn_readfirstlane(fb.w)};
    uint32_t flags = 0;  // OR of the active experts' flags
#pragma unroll
    for (int x = 0; x < EMAX; ++x)
      if ((rs.present >> x) & 1u) flags |= (fw[x >> 2] >> (8 * (x & 3))) & 3u;
    if (lane == 0) {
      s_rt.slow1 = (flags & 1u) ? 1 : 0;
      s_rt.slow2 = (flags & 2u) ? 1 : 0;
    }
  }
  __syncthreads();
  const int u = __builtin_amdgcn_readfirstlane(s_rt.n_active);
  const bool bc = __builtin_amdgcn_readfirstlane(s_rt.bc) != 0;
  const bool slow1 = __builtin_amdgcn_readfirstlane(s_rt.slow1) != 0;
  if (wg0 && wave == 0) {
    const uint32_t *src = reinterpret_cast<const uint32_t *>(&s_rt);
    uint32_t *dst = reinterpret_cast<uint32_t *>(route_out);
    if (lane < kRouteHeadWords) dst[lane] = src[lane];
    for (int i = lane; i < kDecMaxSlots * 16; i += kWave) {
      const int a = i >> 4;
      route_out->code2[a][i & 15] = a < u ? s_code[s_rt.active[a]][32 + (i & 15)] : 0.0f;
    }
    if (lane < ns) {
      w_out[lane] = s_slw[lane];
      idx_out[lane] = s_sle[lane];
    }
  }

  // ---- w1/w3 stream over the workgroup's range of the (active expert, 4-row tile) items
  const int lanej = lane & 3;
  const int blk = lane >> 2;
  const int tiles_e = F >> 2;
  const int N = u * tiles_e;
  const int wlo = (int)((int64_t)blockIdx.x * N / gridDim.x);
  const int whi = (int)((int64_t)(blockIdx.x + 1) * N / gridDim.x);
  const int nsq = H / kStageVals;
  const size_t row_bytes = (size_t)(H >> 1);
  const size_t row_blocks = (size_t)(H >> 6);
  const uint32_t lane_const[2] = {(uint32_t)(lane & 31) << 2, ((uint32_t)(lane & 31) << 2) | 128u};

  // Pointers of item i = (active expert a, tile): rebuilt from the LDS tables.
  auto item_expert = [&](int i, int &tile) {
    int a = 0;
    while (i >= tiles_e) {  // at most u - 1 steps
      i -= tiles_e;
      ++a;
    }
    tile = i;
    return a;
  };
  auto set_ptrs = [&](ItemPtr<2> &P, int i) {
    int tile;
    const int a = item_expert(i, tile);
    const size_t row = (size_t)tile * 4 + lanej;
    const int e = s_rt.active[a];
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      P.wq[p] = (gq_t)s_eptr[e][2 * p] + row * row_bytes + blk * 16;
      P.wa[p] = (ga_t)s_eptr[e][2 * p + 1] + row * row_blocks + (blk >> 1);
      P.ab[p] = (ga_t)s_eptr[e][2 * p + 1] + (size_t)tile * 4 * row_blocks;
    }
    const int jj = (!bc && lanej < s_rt.counts[a]) ? lanej : 0;
    const int tok = s_rt.perm_tok[s_rt.offsets[a] + jj];
    P.ap = (gx_t)xt + (size_t)tok * H + blk * 32 + (bc ? lanej * 8 : 0);
    // The LDS copy: with BC quarter lanej of the token's chunk blk, else the whole chunk
    // of the lane's token row (the expert's first token again past its count).
#pragma unroll
    for (int i = 0; i < 16; ++i) P.xo[i] = xlds_piece(tok, H, 4 * blk + (bc ? lanej : (i & 3)));
  };
  // nrows: MFMA result rows that hold tokens (1 on the single-token path, whose other rows
  // are never accumulated).
  auto finish_item = [&](f32x4 (&ac)[2], int i, int nrows) {
#pragma unroll
    for (int p = 0; p < 2; ++p)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (q < nrows) ac[p][q] = lanes_sum16(ac[p][q]);
    if (blk == 0) {
      int tile;
      const int a = item_expert(i, tile);
      const int row = tile * 4 + lanej;
      const int cnt = s_rt.counts[a];
      const int off = s_rt.offsets[a];
#pragma unroll
      for (int m = 0; m < 4; ++m)
        if (m < cnt && m < nrows) h_out[(size_t)(off + m) * F + row] = swiglu_bf16(ac[0][m], ac[1][m]);
    }
  };
  auto hook = [&]() {};
  const bool slow = slow1;
  if (!slow && bc && nsq == 8 && T == 1) {
    // Single token: the workgroup's items are shared through the work counter.  With at
    // most kRawSlots items per workgroup, an item's per-lane sums go to LDS as they are (no
    // cross-lane reduction or SwiGLU in the stream), and after its stream each wave reduces
    // the items it streamed (blocks 0 to 15 in order) and writes h: no workgroup barrier
    // holds the waves that finish first.
    auto grab = [&]() -> int {
      int t = 0;
      if (lane == 0) t = __hip_atomic_fetch_add(&s_ticket, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      t = __builtin_amdgcn_readfirstlane(t) + wlo;
      return t < whi ? t : -1;
    };
    const gx_t xb = (gx_t)xt + blk * 32 + lanej * 8;
    const uint16_t *xl = s_xn + blk * 32 + lanej * 8;
    const int nit = whi - wlo;
    if (nit > kRawSlots) {
      auto finish1 = [&](f32x4 (&ac)[2], int i) { finish_item(ac, i, 1); };
      if (NORM || N1)
        stream_aligned<2, 8, kGateUpDepth, true, kXRegs, kLookahead>(
            grab, set_ptrs, finish1, hook, s_tbl, lane_const, row_blocks, s_aslot[wave], xl, (gq_t)gate);
      else
        stream_aligned<2, 8, kGateUpDepth, true, kXRegs, kLookahead>(
            grab, set_ptrs, finish1, hook, s_tbl, lane_const, row_blocks, s_aslot[wave], xb, (gq_t)gate);
      return;
    }
    int nmine = 0;  // wave-uniform
    auto finish_raw = [&](f32x4 (&ac)[2], int i) {
      s_raw[i - wlo][0][lane] = ac[0][0];
      s_raw[i - wlo][1][lane] = ac[1][0];
      if (lane == 0) s_mine[wave][nmine] = (uint8_t)(i - wlo);
      ++nmine;
    };
    if (NORM || N1)
      stream_aligned<2, 8, kGateUpDepth, true, kXRegs, kLookahead>(
          grab, set_ptrs, finish_raw, hook, s_tbl, lane_const, row_blocks, s_aslot[wave], xl, (gq_t)gate);
    else
      stream_aligned<2, 8, kGateUpDepth, true, kXRegs, kLookahead>(
          grab, set_ptrs, finish_raw, hook, s_tbl, lane_const, row_blocks, s_aslot[wave], xb, (gq_t)gate);
    wave_lds_sync();  // the wave's own raw slots, written by its other lanes
    for (int c = 0; c < nmine; c += kWave / 4) {  // lane 4 m + j: row j of the wave's item c + m
      const int m = c + (lane >> 2);
      if (m < nmine) {
        const int slot = s_mine[wave][m];
        const int j = lane & 3;
        float g = 0.0f, up = 0.0f;
#pragma unroll
        for (int b = 0; b < 16; ++b) {
          g += s_raw[slot][0][4 * b + j];
          up += s_raw[slot][1][4 * b + j];
        }
        int tile;
        const int a = item_expert(wlo + slot, tile);
        h_out[(size_t)s_rt.offsets[a] * F + tile * 4 + j] = swiglu_bf16(g, up);
      }
    }
    return;
  }
  if (!NORM && xlds && !slow && nsq == 8) {
    // Several tokens: the aligned stream over the workgroup's items, shared through the work
    // counter, with the activations read from the workgroup's LDS copy of the tokens.
    auto grab = [&]() -> int {
      int t = 0;
      if (lane == 0) t = __hip_atomic_fetch_add(&s_ticket, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      t = __builtin_amdgcn_readfirstlane(t) + wlo;
      return t < whi ? t : -1;
    };
    const uint16_t *xl = reinterpret_cast<const uint16_t *>(s_xt);
    if (bc) {
      auto finish1 = [&](f32x4 (&ac)[2], int i) { finish_item(ac, i, 1); };
      stream_aligned<2, 8, kGateUpDepth, true, kXLds, kLookahead>(
          grab, set_ptrs, finish1, hook, s_tbl, lane_const, row_blocks, s_aslot[wave], xl, (gq_t)gate);
    } else {
      auto finish4 = [&](f32x4 (&ac)[2], int i) { finish_item(ac, i, 4); };
      stream_aligned<2, 8, kGateUpDepth, false, kXLds, kLookahead>(
          grab, set_ptrs, finish4, hook, s_tbl, lane_const, row_blocks, s_aslot[wave], xl, (gq_t)gate);
    }
    return;
  }
  // Other shapes: each wave takes a contiguous part of the workgroup's range.
  if (NORM) {  // the stream reads the token from global memory: this workgroup's xs row
    for (int c = tid * 8; c < H; c += kDecThreads * 8)
      *reinterpret_cast<uint4 *>(const_cast<uint16_t *>(xt) + c) =
          *reinterpret_cast<const uint4 *>(s_xn + c);
    __syncthreads();
  }
  const int nw = whi - wlo;
  const int i0 = wlo + wave * nw / kDecWaves;
  const int n_items = wlo + (wave + 1) * nw / kDecWaves - i0;
  int li = i0 - 1;
  auto next_item = [&](ItemPtr<2> &P) { set_ptrs(P, ++li); };
  int ci = i0;
  auto finish = [&](f32x4 (&ac)[2]) { finish_item(ac, ci++, 4); };
  auto slow_code = [&]() -> const float * {
    int tile;
    return s_code[s_rt.active[item_expert(ci, tile)]];
  };
  if (!slow && bc)
    stream_items<2, 6, false, true>(n_items, nsq, next_item, finish, hook, slow_code, s_tbl, lane_const, (gq_t)gate);
  else if (!slow)
    stream_items<2, 4, false, false>(n_items, nsq, next_item, finish, hook, slow_code, s_tbl, lane_const, (gq_t)gate);
  else if (bc)
    stream_items<2, 6, true, true>(n_items, nsq, next_item, finish, hook, slow_code, s_tbl, lane_const, (gq_t)gate);
  else
    stream_items<2, 4, true, false>(n_items, nsq, next_item, finish, hook, slow_code, s_tbl, lane_const, (gq_t)gate);
}

__global__ void __launch_bounds__(kDecThreads, 1)
decode_down_kernel(const ExpertTable tab, const DecodeRoute *__restrict__ route,
                   const uint16_t *__restrict__ h, int T, int H, int F, int E, int k,
                   int tiles_per_wg, int kparts, uint16_t *__restrict__ out) {
  __shared__ __attribute__((aligned(16))) uint32_t s_tbl[kTableWords];
  __shared__ __attribute__((aligned(16))) DecodeRoute s_rt;
  // Partial sums of (tile, active expert, K part): 4 rows x 4 token rows.
  __shared__ float s_part[kDecMaxTilesPerWg][kDecMaxSlots][kDecMaxKParts][16];
  __shared__ const void *s_eptr[kDecMaxExperts][2];  // w2_packed, w2_absmax of every expert
  __shared__ __attribute__((aligned(16))) float s_aslot[kDecWaves][2 * kASlotFloats];
  __shared__ int32_t s_ticket;  // next unit of the workgroup (single-token path)

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // The descriptor and every expert's w2 pointers in one round trip.
  uint32_t rw = 0;
  if (tid < kRouteWords) rw = reinterpret_cast<const uint32_t *>(route)[tid];
  // Experts wave + 8q: wave-uniform table entries (scalar loads), lanes 0/1 keep
  // w2_packed / w2_absmax.
  constexpr int EPW = kDecMaxExperts / kDecWaves;
  const void *pk[EPW], *pa[EPW];
#pragma unroll
  for (int q = 0; q < EPW; ++q) {
    const int e = wave + kDecWaves * q;
    const moe_nf4_expert_t &ex = tab.e[e < E ? e : E - 1];
    pk[q] = uniform_ptr(ex.w2_packed);
    pa[q] = uniform_ptr(ex.w2_absmax);
  }
  if (tid == 0) s_ticket = 0;
  // Lookup table from the NF4 codebook constants, built while the loads are in flight; the
  // gate/up kernel flagged (slow2) active experts whose w2 codebook differs from them.
  {
    float cst[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) cst[q] = kNf4Code[q];
    build_table_regs<kDecThreads>(s_tbl, cst, cst);
  }
#pragma unroll
  for (int q = 0; q < EPW; ++q) {
    const int e = wave + kDecWaves * q;
    if (e < E && lane < 2) s_eptr[e][lane] = lane ? pa[q] : pk[q];
  }
  if (tid < kRouteWords) reinterpret_cast<uint32_t *>(&s_rt)[tid] = rw;
  __syncthreads();
  const int u = s_rt.n_active;

  const int lanej = lane & 3;
  const int blk = lane >> 2;
  const int r0 = blockIdx.x * tiles_per_wg;
  const int r_end = min(r0 + tiles_per_wg, H >> 2);
  const int ntl = r_end > r0 ? r_end - r0 : 0;
  const int NS = F / kStageVals;
  const int nsq = NS / kparts;  // stages per unit
  // Units: (active expert a, tile tl, K part kp), kp fastest, so that consecutive units
  // continue the same rows.
  const int n_units = u * ntl * kparts;
  const size_t row_bytes = (size_t)(F >> 1);
  const size_t row_blocks = (size_t)(F >> 6);
  const uint32_t lane_const[1] = {(uint32_t)lane << 2};
  const bool bc = s_rt.bc != 0;

  auto unit_fields = [&](int i, int &tl, int &kp) {
    kp = i % kparts;
    const int r = i / kparts;
    tl = r % ntl;
    return r / ntl;  // active index
  };
  auto set_ptrs = [&](ItemPtr<1> &P, int i) {
    int tl, kp;
    const int a = unit_fields(i, tl, kp);
    const int s_lo = kp * nsq;
    const size_t row = (size_t)(r0 + tl) * 4 + lanej;
    const int e = s_rt.active[a];
    P.wq[0] = (gq_t)s_eptr[e][0] + row * row_bytes + s_lo * 256 + blk * 16;
    P.wa[0] = (ga_t)s_eptr[e][1] + row * row_blocks + s_lo * 8 + (blk >> 1);
    P.ab[0] = (ga_t)s_eptr[e][1] + (size_t)(r0 + tl) * 4 * row_blocks + s_lo * 8;
    const int jj = (!bc && lanej < s_rt.counts[a]) ? lanej : 0;
    P.ap = (gx_t)h + (size_t)(s_rt.offsets[a] + jj) * F + (size_t)s_lo * kStageVals + blk * 32 +
           (bc ? lanej * 8 : 0);
  };
  // nrows: result rows to keep (1 when the stream accumulated row 0 only; the combine then
  // reads row 0, slot_m being 0 for every slot).
  auto finish_unit = [&](f32x4 (&ac)[1], int i, int nrows) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (q < nrows) ac[0][q] = lanes_sum16(ac[0][q]);
    if (blk == 0) {
      int tl, kp;
      const int a = unit_fields(i, tl, kp);
#pragma unroll
      for (int m = 0; m < 4; ++m)
        if (m < nrows) s_part[tl][a][kp][lanej * 4 + m] = ac[0][m];
    }
  };
  auto hook = [&]() {};
  const bool slow = s_rt.slow2 != 0;
  const int npairs = (ntl + 1) >> 1;
  if (!slow && nsq == 4) {
    // Units of two tiles (pair tp: tiles 2tp, 2tp+1) share the activation operand; the
    // workgroup's units are shared through the work counter.  With BC (every active expert
    // has one token) the lane holds a quarter of the token's chunk, else the whole chunk
    // of its token row.
    const int n_pu = u * npairs * kparts;
    auto pair_fields = [&](int i, int &tp, int &kp) {
      kp = i % kparts;
      const int r = i / kparts;
      tp = r % npairs;
      return r / npairs;  // active index
    };
    auto grab = [&]() -> int {
      int t = 0;
      if (lane == 0) t = __hip_atomic_fetch_add(&s_ticket, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      t = __builtin_amdgcn_readfirstlane(t);
      return t < n_pu ? t : -1;
    };
    auto set_ptrs2 = [&](ItemPtr<2> &P, int i) {
      int tp, kp;
      const int a = pair_fields(i, tp, kp);
      const int s_lo = kp * nsq;
      const int e = s_rt.active[a];
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int tl = min(2 * tp + q, ntl - 1);  // an odd last tile is read twice
        const size_t row = (size_t)(r0 + tl) * 4 + lanej;
        P.wq[q] = (gq_t)s_eptr[e][0] + row * row_bytes + s_lo * 256 + blk * 16;
        P.wa[q] = (ga_t)s_eptr[e][1] + row * row_blocks + s_lo * 8 + (blk >> 1);
        P.ab[q] = (ga_t)s_eptr[e][1] + (size_t)(r0 + tl) * 4 * row_blocks + s_lo * 8;
      }
      const int jj = (!bc && lanej < s_rt.counts[a]) ? lanej : 0;
      P.ap = (gx_t)h + (size_t)(s_rt.offsets[a] + jj) * F + (size_t)s_lo * kStageVals + blk * 32 +
             (bc ? lanej * 8 : 0);
#pragma unroll
      for (int i = 0; i < 16; ++i) P.xo[i] = 0;  // unused (activations from global memory)
    };
    // nrows: result rows that hold tokens (1 with BC, whose stream accumulates row 0 only).
    auto finish2 = [&](f32x4 (&ac)[2], int i, int nrows) {
      float v0[4], v1[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        if (m < nrows) {
          v0[m] = lanes_sum16(ac[0][m]);
          v1[m] = lanes_sum16(ac[1][m]);
        }
      }
      if (blk == 0) {
        int tp, kp;
        const int a = pair_fields(i, tp, kp);
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          if (m < nrows) {
            s_part[2 * tp][a][kp][lanej * 4 + m] = v0[m];
            if (2 * tp + 1 < ntl) s_part[2 * tp + 1][a][kp][lanej * 4 + m] = v1[m];
          }
        }
      }
    };
    const uint32_t lane_const2[2] = {(uint32_t)lane << 2, (uint32_t)lane << 2};
    if (bc) {
      auto fin = [&](f32x4 (&ac)[2], int i) { finish2(ac, i, 1); };
      stream_aligned<2, 4, 4, true, kXGlobal, kLookahead>(grab, set_ptrs2, fin, hook, s_tbl,
                                                       lane_const2, row_blocks, s_aslot[wave],
                                                       (gx_t)nullptr, (gq_t)h);
    } else {
      auto fin = [&](f32x4 (&ac)[2], int i) { finish2(ac, i, 4); };
      stream_aligned<2, 4, 4, false, kXGlobal, kLookahead>(grab, set_ptrs2, fin, hook, s_tbl,
                                                        lane_const2, row_blocks, s_aslot[wave],
                                                        (gx_t)nullptr, (gq_t)h);
    }
  } else {
    // Each wave takes a contiguous part of the units.
    const int i0 = wave * n_units / kDecWaves;
    const int n_items = (wave + 1) * n_units / kDecWaves - i0;
    int li = i0 - 1;
    auto next_item = [&](ItemPtr<1> &P) { set_ptrs(P, ++li); };
    int ci = i0;
    auto finish = [&](f32x4 (&ac)[1]) { finish_unit(ac, ci++, 4); };
    auto slow_code = [&]() -> const float * {
      int tl, kp;
      return s_rt.code2[unit_fields(ci, tl, kp)];
    };
    if (!slow && bc)
      stream_items<1, 8, false, true>(n_items, nsq, next_item, finish, hook, slow_code, s_tbl, lane_const, (gq_t)h);
    else if (!slow)
      stream_items<1, 8, false, false>(n_items, nsq, next_item, finish, hook, slow_code, s_tbl, lane_const, (gq_t)h);
    else if (bc)
      stream_items<1, 8, true, true>(n_items, nsq, next_item, finish, hook, slow_code, s_tbl, lane_const, (gq_t)h);
    else
      stream_items<1, 8, true, false>(n_items, nsq, next_item, finish, hook, slow_code, s_tbl, lane_const, (gq_t)h);
  }
  __syncthreads();

  // ---- combine: one thread per (tile, token, row); slots in ascending expert order; the
  // K parts of an expert are summed in part order.
  if (tid < ntl * T * 4) {
    const int tl = tid / (T * 4);
    const int rem = tid - tl * T * 4;
    const int t = rem >> 2;
    const int jr = rem & 3;
    int ord[kDecMaxSlots];
    for (int j = 0; j < k; ++j) {
      const int key = s_rt.slot_a[t * k + j];
      int p = j;
      while (p > 0 && s_rt.slot_a[t * k + ord[p - 1]] > key) {
        ord[p] = ord[p - 1];
        --p;
      }
      ord[p] = j;
    }
    float o = 0.0f;
    for (int jj = 0; jj < k; ++jj) {
      const int s = t * k + ord[jj];
      const int a = s_rt.slot_a[s];
      const int m = s_rt.slot_m[s];
      float y = s_part[tl][a][0][jr * 4 + m];
      for (int kp = 1; kp < kparts; ++kp) y += s_part[tl][a][kp][jr * 4 + m];
      const float pr = bf16_to_f32(f32_to_bf16(y)) * s_rt.slot_w[s];
      o = bf16_to_f32(f32_to_bf16(o + pr));
    }
    out[(size_t)t * H + (size_t)(r0 + tl) * 4 + jr] = f32_to_bf16(o);
  }
}

// Largest hidden size of the in-kernel routing of mid-size launches (the gate products'
// loads of one wave: at most four 128-value chunks).
constexpr int kMidMaxH = 4096;

// The routing a mid-size gate/up launch computes itself: the gate, the optional per-expert
// logit bias, and where workgroup 0 writes the router's outputs (logits may be null) and the
// grouping the down projection and the combine read (the layout of moe_permute: offsets
// [E + 1], active = {n, ids ascending}, slot_pos of every slot).  With a null gate and
// `parts` set, the launch routes from the gate products of a mid_gate_parts_kernel launch
// (parts); with both null it only groups the slots of a separate router launch (idx32).
struct MidRouteOut {
  const uint16_t *gate;
  const float *bias;
  uint16_t *logits;
  float *w;
  int64_t *idx64;
  int32_t *idx32;
  int32_t *counts;
  int32_t *offsets;
  int32_t *perm_tok;
  int32_t *slot_pos;
  int32_t *active;
  const float *parts;
};
constexpr int kMidMaxT = 16;
constexpr int kMidMaxSlots = kMidMaxT * 2;
constexpr int kMidGroupMaxSlots = 2 * kWave;  // slots the in-launch grouping takes
// How a mid-size gate/up launch gets its grouping: from the caller (Route), by routing the
// tokens itself, by grouping the slots of a separate router launch, or by routing from the
// gate products of a separate K-split launch.
constexpr int kRtExternal = 0, kRtRoute = 1, kRtGroup = 2, kRtParts = 3;
// The K-split gate products: [slice][token][expert] fp32, 8 slices of H/8 values (the waves'
// K slices of mid_gate_route), up to 64 tokens and 16 experts.
constexpr int kMidPartSlices = kDecWaves;
constexpr int kMidPartTokens = 64;
constexpr int kMidPartExperts = 16;
constexpr int64_t kMidPartsBytes = (int64_t)kMidPartSlices * kMidPartTokens * kMidPartExperts * 4;

// Grouping of ns <= 2 * kWave routed slots (slot s = t k + j routed to expert se) by expert,
// ascending expert then slot (the order of moe_permute), by one wave: lane l holds slots l
// and l + 64.  Fills s_cnt / s_off (rows and first row of every expert) and s_ptok (token
// of every grouped row); with `publish`, also writes counts, offsets [E + 1], active =
// {n, ids ascending}, slot_pos [ns] and perm_tok of ro.  Returns the grouped row of each of
// the lane's slots in pos.
__device__ __forceinline__ void mid_group(const int (&se)[2], int ns, int k, int E, int32_t *s_cnt,
                                          int32_t *s_off, int32_t *s_ptok, bool publish,
                                          const MidRouteOut &ro, int (&pos)[2]) {
  const int lane = threadIdx.x & (kWave - 1);
  const uint64_t lt = (1ull << lane) - 1ull;
  int run = 0, my_cnt = 0, my_off = 0;
  uint32_t present = 0;
  pos[0] = pos[1] = 0;
  for (int xe = 0; xe < E; ++xe) {
    const uint64_t m0 = __ballot(se[0] == xe), m1 = __ballot(se[1] == xe);
    const int c0 = __builtin_popcountll(m0);
    const int c = c0 + __builtin_popcountll(m1);
    if (se[0] == xe) pos[0] = run + __builtin_popcountll(m0 & lt);
    if (se[1] == xe) pos[1] = run + c0 + __builtin_popcountll(m1 & lt);
    if (lane == xe) {
      my_cnt = c;
      my_off = run;
    }
    if (c > 0) present |= 1u << xe;
    run += c;
  }
  if (lane < E) {
    s_cnt[lane] = my_cnt;
    s_off[lane] = my_off;
  }
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int sl = lane + kWave * h;
    if (sl < ns) s_ptok[pos[h]] = sl / k;
  }
  if (publish) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int sl = lane + kWave * h;
      if (sl < ns) {
        ro.slot_pos[sl] = pos[h];
        ro.perm_tok[pos[h]] = sl / k;
      }
    }
    if (lane < E) {
      ro.counts[lane] = my_cnt;
      ro.offsets[lane] = my_off;
    }
    if (lane == 0) {
      ro.offsets[E] = ns;
      ro.active[0] = __builtin_popcount(present);
    }
    // Active experts in ascending order: lane x writes its rank among the present ones.
    if (lane < E && ((present >> lane) & 1u))
      ro.active[1 + __builtin_popcount(present & ((1u << lane) - 1u))] = lane;
  }
}

// Offset (values) of lane group kq's 8-value pieces within a 64-value NF4 block in the
// 16x16x32 MFMA operands of the mid-size kernels ({0, 32, 16, 48}, see mid16_gateup_kernel).
__device__ __forceinline__ int m16_off(int kq) { return ((kq & 1) << 5) | ((kq >> 1) << 4); }

// Routing of T <= kMidMaxT tokens by one workgroup (the gate is small and stays in L2): the
// gate products into s_scratch (the waves' partials, kDecWaves x kMidMaxT x EMAX floats),
// then per-token routing (route_rows: slot experts and weights into s_sle / s_slw, logits
// [T][E] written when `logits` is not null).  `table` builds the lookup table while the gate
// loads are in flight.  Ends with a workgroup barrier.
//
// Gate products on the 16x16x32 MFMA (H = 1024 S): wave w takes values [w H/8, (w+1) H/8)
// of H, 4S MFMAs.  Lane l = 16 kq + n supplies token n's values (A rows; tokens >= T repeat
// token T - 1) and expert n's (B columns; experts >= E repeat expert E - 1) in the layout of
// the weight stream's activation operands (mid16_gateup_kernel: MFMA (s, j) takes values
// m16_off(kq) + 8 (j & 1) .. +7 of block 2s + (j >> 1) of the wave's slice), and ends with the
// wave's sum D[token 4 kq + r][expert n] in register r, stored as it is.  The token operands
// stay in xt for the stream.
template <int EMAX, int S, typename TableFn>
__device__ __forceinline__ void mid_gate_route(const uint16_t *__restrict__ x, int T, int H, int E,
                                               int k, const uint16_t *gate, const float *bias,
                                               uint16_t *logits, float *s_scratch, int32_t *s_sle,
                                               float *s_slw, bf16x8 (&xt)[S][4], TableFn &&table) {
  static_assert(EMAX <= 16, "one MFMA column per expert");
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15, kq = lane >> 4;
  const size_t k0 = (size_t)wave * (128 * S) + m16_off(kq);
  const gx_t xr = (gx_t)x + (size_t)(n < T ? n : T - 1) * H + k0;
  const gx_t gr = (gx_t)gate + (size_t)(n < E ? n : E - 1) * H + k0;
  // Every load goes out at once, then the table is built under them.
  bf16x8 ga[S][4];
#pragma unroll
  for (int sq = 0; sq < S; ++sq)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int o = 128 * sq + 64 * (j >> 1) + 8 * (j & 1);
      xt[sq][j] = as_bf16x8(ld_u4(xr + o));
      ga[sq][j] = as_bf16x8(ld_u4(gr + o));
    }
  __builtin_amdgcn_sched_barrier(0);
  table();
  __builtin_amdgcn_sched_barrier(0);
  f32x4 d = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int sq = 0; sq < S; ++sq)
#pragma unroll
    for (int j = 0; j < 4; ++j) d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xt[sq][j], ga[sq][j], d, 0, 0, 0);
  float(*s_part)[kMidMaxT][EMAX] = reinterpret_cast<float(*)[kMidMaxT][EMAX]>(s_scratch);
  if (n < E) {
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (4 * kq + r < T) s_part[wave][4 * kq + r][n] = d[r];
  }
  __syncthreads();
  // ---- per-token routing: wave w routes tokens 4w .. 4w+3 (workgroup 0 writes logits).
  if (4 * wave < T)
    route_rows<EMAX, kDecWaves, kMidMaxT>(s_sle, s_slw, s_part, 4 * wave, bias, T, E, k, logits);
  __syncthreads();
}

// Routing of the T <= kMidMaxT tokens of a mid-size launch in every workgroup
// (mid_gate_route), then the grouping of the T*k slots by expert into s_cnt / s_off / s_ptok
// (wave 0); workgroup 0 also writes the router's outputs and the grouping (MidRouteOut).
template <int EMAX, int S, typename TableFn>
__device__ __forceinline__ void mid_route(const uint16_t *__restrict__ x, int T, int H, int E,
                                          int k, const MidRouteOut &ro, float *s_scratch,
                                          int32_t *s_sle, float *s_slw, int32_t *s_cnt,
                                          int32_t *s_off, int32_t *s_ptok, bf16x8 (&xt)[S][4],
                                          TableFn &&table) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  mid_gate_route<EMAX, S>(x, T, H, E, k, ro.gate, ro.bias, blockIdx.x == 0 ? ro.logits : nullptr,
                       s_scratch, s_sle, s_slw, xt, table);
  // ---- grouping of the T k slots by expert (ascending expert, then slot), by wave 0;
  // workgroup 0 also writes the router's outputs.
  if (wave == 0) {
    const int ns = T * k;
    const int se[2] = {lane < ns ? s_sle[lane] : -1, -1};
    int pos[2];
    mid_group(se, ns, k, E, s_cnt, s_off, s_ptok, blockIdx.x == 0, ro, pos);
    if (blockIdx.x == 0 && lane < ns) {
      const int t = lane / k, j = lane - (lane / k) * k;
      ro.w[t * k + j] = s_slw[lane];
      ro.idx64[t * k + j] = se[0];
      ro.idx32[t * k + j] = se[0];
    }
  }
  __syncthreads();  // the grouping is visible; the gate partials are dead
}

// Gate/up of mid-size batches (5 to 64 tokens) on the 16x16x32 MFMA.  An active expert with
// cnt routed rows is ceil(cnt / 16) "virtual experts" of up to 16 consecutive rows; the
// workgroups are dealt to them by m16_share (the virtual experts of one expert side by side
// on one XCD, over the same tiles).  A workgroup takes its virtual expert's 16-row weight
// tiles one at a time, and wave w covers values [w H/8, (w+1) H/8) of every tile's K range, so each wave
// keeps its K slice of the expert's token rows in registers for the whole launch and no
// activation passes through LDS.  The eight partial sums of a tile meet in LDS (one
// LDS-only barrier per tile, two buffers), and 256 threads sum them in wave order and write
// h = bf16(silu(bf16(w1 x)) * bf16(w3 x)) (transfer/nf4_reconstruct.py:152-155 on the rows
// model/moe_layer.py:174-186 gathers).
//
// MFMA layout (v_mfma_f32_16x16x32_bf16): lane l = 16 kq + n supplies B[k in 8kq .. 8kq+7][n]
// and A[n][k in 8kq .. 8kq+7], and holds D[4 kq + r][n] in register r.  The weights are B
// (n: row of the tile), the tokens A.  Load s of a projection reads 16 rows x 64 bytes: lane
// l the 16 bytes 64s + 16kq of row n (two loads per 128-byte line, back to back).  The 64
// bytes are two NF4 blocks, 2s in lanes 0-31 and 2s+1 in lanes 32-63; two
// v_permlane32_swap (which exchange the upper half of the first operand with the lower
// half of the second) turn the lane's dwords d0..d3 into four MFMA operands that each lie
// in one block: {d0, d2} and {d1, d3} of lanes 0-31 hold block 2s, those of lanes 32-63
// block 2s+1.  Lane group kq of operand j covers block values kM16Off[kq] + 8 (j & 1) .. +7,
// and the A operand of MFMA (s, j) holds the same values of the lane's token row.  The
// absmax of a block (the lane's row) scales each pair of MFMA sums in fp32.
constexpr int kM16Rows = 16;  // rows of a virtual expert = weight rows of a tile

// Four packed bytes (values 2j, 2j+1 per byte) -> eight bf16 code values (B operand).
__device__ __forceinline__ bf16x8 m16_lookup(const uint32_t *tbl, uint32_t w, uint32_t lane_const) {
  uint32_t l[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    l[j] = lds_lookup(tbl, __builtin_amdgcn_perm(w, lane_const, 0x0c0c0400u + (j << 8)));
  return as_bf16x8(l[0], l[1], l[2], l[3]);
}

// The workgroup's share of a mid-size launch.  An active expert with cnt routed rows is
// nv = ceil(cnt / 16) virtual experts; a unit is (virtual expert, part) with `parts` parts
// of `tiles` tiles each.  The virtual experts of one expert (siblings) read the same weight
// tiles, so they are dealt together: expert e receives a budget of workgroups proportional to
// its units, cut into shares of nv workgroups, one per sibling, that take the same tile range
// of the same part.  Sibling workgroups are adjacent in an XCD-major numbering of the grid
// (workgroup b runs on XCD b mod 8), so they run side by side on one XCD and the siblings
// after the first find the tiles in that XCD's L2 rather than in HBM.  Workgroups past the
// last share get no tiles (t_lo == t_hi).  Requires V * parts <= gridDim.x (V = sum of nv)
// and nv = 0 on lanes >= E.
struct M16Share {
  int e, vj, part, t_lo, t_hi;
};
// Inclusive prefix sum over lanes 0 .. n-1 (n <= 64, wave-uniform; lanes >= n hold 0): a
// readlane per lane, which for the few experts here is shorter than a shuffle scan's chain
// of LDS permutes.
__device__ __forceinline__ int lanes_incl_scan(int v, int n) {
  const int lane = threadIdx.x & (kWave - 1);
  int acc = 0;
  for (int j = 0; j < n; ++j) {
    const int vj = __builtin_amdgcn_readlane(v, j);
    if (j <= lane) acc += vj;
  }
  return acc;
}

__device__ __forceinline__ M16Share m16_share(int nv, int parts, int tiles, int E) {
  const int lane = threadIdx.x & (kWave - 1);
  const int incl = lanes_incl_scan(nv, E);
  const int V = __builtin_amdgcn_readlane(incl, kWave - 1);
  const int G = gridDim.x, b = blockIdx.x;
  const int L = (G % 8 == 0) ? (b % 8) * (G / 8) + b / 8 : b;
  // 32-bit arithmetic throughout (G, V and parts are small; 64-bit division is a long
  // software sequence on the GPU).
  const uint32_t U = (uint32_t)V * (uint32_t)parts;
  // Shares of the lane's expert (>= parts when U <= G) and the workgroups they take.
  const int budget = nv > 0 ? (int)((uint32_t)G * (uint32_t)nv * (uint32_t)parts / U) : 0;
  const int shares = nv > 0 ? (int)((uint32_t)budget / (uint32_t)nv) : 0;
  const int used = nv * shares;
  const int end = lanes_incl_scan(used, E);
  const uint64_t past = __ballot(lane < E && end > L);
  M16Share r;
  if (past == 0) {  // an idle workgroup: no tiles (the first active expert keeps loads valid)
    r.e = __builtin_ctzll(__ballot(nv > 0));
    r.vj = r.part = r.t_lo = r.t_hi = 0;
    return r;
  }
  const int e = __builtin_ctzll(past);
  const int m = __builtin_amdgcn_readlane(nv, e);
  const int st = __builtin_amdgcn_readlane(shares, e);
  const int o = L - (__builtin_amdgcn_readlane(end, e) - __builtin_amdgcn_readlane(used, e));
  const int q = (int)((uint32_t)o / (uint32_t)m);  // the expert's share index; sibling o % m
  const int Q = (int)((uint32_t)st / (uint32_t)parts), R = st - Q * parts;
  int p, s, sp;  // parts < R take Q + 1 shares, the rest Q
  if (q < R * (Q + 1)) {
    p = (int)((uint32_t)q / (uint32_t)(Q + 1));
    s = q - p * (Q + 1);
    sp = Q + 1;
  } else {
    const int q2 = q - R * (Q + 1);
    p = R + (int)((uint32_t)q2 / (uint32_t)Q);
    s = q2 - (p - R) * Q;
    sp = Q;
  }
  r.e = e;
  r.vj = o - q * m;
  r.part = p;
  r.t_lo = (int)((uint32_t)s * (uint32_t)tiles / (uint32_t)sp);
  r.t_hi = (int)((uint32_t)(s + 1) * (uint32_t)tiles / (uint32_t)sp);
  return r;
}

// Gate products of up to 64 tokens for a mid-size layer, split over K so that no CU reads
// more than a slice: workgroup (token group tg of 16, slice ks) is one wave computing, for
// tokens 16 tg .. +15 and every expert, the sums over values [ks H/8, (ks+1) H/8) of H on the
// 16x16x32 MFMA in the operand layout of mid_gate_route (whose wave ks computes the same
// sums), into parts[ks][token][expert].  The mid-size gate/up launch adds the 8 slices in
// slice order and routes (kRtParts), as the routing inside the launch does for its waves.
template <int S>
__global__ void __launch_bounds__(kWave)
mid_gate_parts_kernel(const uint16_t *__restrict__ x, const uint16_t *__restrict__ gate, int T,
                      int H, int E, float *__restrict__ parts) {
  const int lane = threadIdx.x;
  const int ks = blockIdx.x % kMidPartSlices, tg = blockIdx.x / kMidPartSlices;
  const int n = lane & 15, kq = lane >> 4;
  const int t = 16 * tg + n;
  const size_t k0 = (size_t)ks * (128 * S) + m16_off(kq);
  const gx_t xr = (gx_t)x + (size_t)(t < T ? t : T - 1) * H + k0;
  const gx_t gr = (gx_t)gate + (size_t)(n < E ? n : E - 1) * H + k0;
  bf16x8 xa[S][4], ga[S][4];
#pragma unroll
  for (int sq = 0; sq < S; ++sq)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int o = 128 * sq + 64 * (j >> 1) + 8 * (j & 1);
      xa[sq][j] = as_bf16x8(ld_u4(xr + o));
      ga[sq][j] = as_bf16x8(ld_u4(gr + o));
    }
  f32x4 d = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int sq = 0; sq < S; ++sq)
#pragma unroll
    for (int j = 0; j < 4; ++j) d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[sq][j], ga[sq][j], d, 0, 0, 0);
  if (n < E) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int tt = 16 * tg + 4 * kq + r;
      if (tt < T) parts[((size_t)ks * kMidPartTokens + tt) * kMidPartExperts + n] = d[r];
    }
  }
}

template <int S, int EMAX, int RT>
__global__ void __launch_bounds__(kDecThreads, 1)
mid16_gateup_kernel(const ExpertTable tab, const uint16_t *__restrict__ x, int T, int H, int F,
                    int E, int k, const Route rt, const MidRouteOut ro,
                    uint16_t *__restrict__ h_out) {
  static_assert(S == 2 || S == 4, "H = 1024 S with S = 2 or 4");
  __shared__ __attribute__((aligned(16))) uint32_t s_tbl[kTableWords];
  // The waves' partial sums of a tile [buffer][wave][projection][4 lane + r]; before the
  // first tile (ROUTE) the waves' gate partials.
  __shared__ __attribute__((aligned(16))) float s_red[2][kDecWaves][2][kWave * 4];
  constexpr bool ROUTE = RT == kRtRoute;
  constexpr bool PARTS = RT == kRtParts;
  constexpr int kSlots = ROUTE ? kMidMaxSlots : PARTS ? kMidGroupMaxSlots : 1;
  __shared__ int32_t s_sle[kSlots];
  __shared__ float s_slw[kSlots];
  __shared__ int32_t s_cnt[RT != kRtExternal ? kWave : 1], s_off[RT != kRtExternal ? kWave : 1];
  __shared__ int32_t s_ptok[ROUTE ? kMidMaxSlots : RT != kRtExternal ? kMidGroupMaxSlots : 1];
  static_assert(!ROUTE || kDecWaves * kMidMaxT * EMAX * 4 <= (int)sizeof(s_red), "gate partials fit");
  static_assert(!PARTS || (kMidPartSlices * kMidPartTokens * EMAX * 4 <= (int)sizeof(s_red) &&
                           EMAX <= kMidPartExperts && kMidPartSlices == kDecWaves),
                "K-split gate products fit");

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // Lane e: expert e is resident (its table entry, read now, under the routing).
  const bool resident = lane < E && tab.e[lane < E ? lane : 0].w1_packed != nullptr;

  const int32_t *g_cnt = rt.counts, *g_off = rt.offsets, *g_ptok = rt.perm_tok;
  auto table_from_constants = [&]() {
    float cst[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) cst[q] = kNf4Code[q];
    build_table_regs<kDecThreads>(s_tbl, cst, cst);
  };
  // PARTS: the 8 slices' gate products of every token ([slice][token][expert], experts < EMAX)
  // are loaded first, so that they arrive while the table is built.
  constexpr int kPartQ = EMAX / 4;  // 16-byte pieces of a token's experts
  constexpr int kPartLoads = PARTS ? kMidPartSlices * kMidPartTokens * kPartQ / kDecThreads : 1;
  static_assert(!PARTS || kMidPartSlices * kMidPartTokens * kPartQ % kDecThreads == 0, "whole rounds");
  f32x4 pv[kPartLoads];
  if constexpr (PARTS) {
#pragma unroll
    for (int r = 0; r < kPartLoads; ++r) {
      const int i = tid + kDecThreads * r;
      const int q = i % kPartQ, t = (i / kPartQ) % kMidPartTokens, ks = i / (kPartQ * kMidPartTokens);
      pv[r] = t < T ? *reinterpret_cast<const f32x4 *>(
                          ro.parts + ((size_t)ks * kMidPartTokens + t) * kMidPartExperts + 4 * q)
                    : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
  }
  if constexpr (!ROUTE) table_from_constants();
  // ROUTE: every token's K slice of the wave (lane 16 kq + t: token t), loaded by the routing
  // in the layout of the activation operands below.
  bf16x8 xt[ROUTE ? S : 1][4];
  if constexpr (ROUTE) {
    mid_route<EMAX, S>(x, T, H, E, k, ro, &s_red[0][0][0][0], s_sle, s_slw, s_cnt, s_off, s_ptok,
                       xt, table_from_constants);
  }
  if constexpr (PARTS) {
    // The gate products into LDS ([slice][token][EMAX]; experts past E unused), then each
    // wave routes tokens 4w .. 4w+3 and 32 + 4w .. (route_rows adds the slices in slice
    // order), and wave 0 groups the slots; workgroup 0 publishes.
    float(*s_part)[kMidPartTokens][EMAX] =
        reinterpret_cast<float(*)[kMidPartTokens][EMAX]>(&s_red[0][0][0][0]);
#pragma unroll
    for (int r = 0; r < kPartLoads; ++r) {
      const int i = tid + kDecThreads * r;
      const int q = i % kPartQ, t = (i / kPartQ) % kMidPartTokens, ks = i / (kPartQ * kMidPartTokens);
      if (t < T) *reinterpret_cast<f32x4 *>(&s_part[ks][t][4 * q]) = pv[r];
    }
    __syncthreads();
    const bool wg0 = blockIdx.x == 0;
#pragma unroll
    for (int h = 0; h < kMidPartTokens / (4 * kDecWaves); ++h) {
      const int t0 = 4 * kDecWaves * h + 4 * wave;
      if (t0 < T)
        route_rows<EMAX, kMidPartSlices, kMidPartTokens>(s_sle, s_slw, s_part, t0, ro.bias, T, E, k,
                                                         wg0 ? ro.logits : nullptr);
    }
    __syncthreads();
    if (wave == 0) {
      const int ns = T * k;
      const int se[2] = {lane < ns ? s_sle[lane] : -1, lane + kWave < ns ? s_sle[lane + kWave] : -1};
      int pos[2];
      mid_group(se, ns, k, E, s_cnt, s_off, s_ptok, wg0, ro, pos);
      if (wg0) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int sl = lane + kWave * h;
          if (sl < ns) {
            ro.w[sl] = s_slw[sl];
            ro.idx64[sl] = se[h];
            ro.idx32[sl] = se[h];
          }
        }
      }
    }
    __syncthreads();
  }
  if constexpr (RT == kRtGroup) {  // the router's slots, grouped by wave 0
    if (wave == 0) {
      const int ns = T * k;
      const int se[2] = {lane < ns ? ro.idx32[lane] : -1, lane + kWave < ns ? ro.idx32[lane + kWave] : -1};
      int pos[2];
      mid_group(se, ns, k, E, s_cnt, s_off, s_ptok, blockIdx.x == 0, ro, pos);
    }
    __syncthreads();
  }
  if constexpr (RT != kRtExternal) {
    g_cnt = s_cnt;
    g_off = s_off;
    g_ptok = s_ptok;
  }

  // Virtual experts of every active expert (lane e holds expert e), counted in every wave.
  const int cnt = resident ? g_cnt[lane] : 0;
  const int off = lane < E ? g_off[lane] : 0;
  const int nv = (cnt + kM16Rows - 1) / kM16Rows;
  if (__ballot(nv > 0) == 0) return;  // uniform over the grid
  const M16Share sh = m16_share(nv, 1, F / kM16Rows, E);
  const int e = sh.e, vj = sh.vj;
  const int r0 = __builtin_amdgcn_readlane(off, e) + kM16Rows * vj;  // first h row
  const int n = min(kM16Rows, __builtin_amdgcn_readlane(cnt, e) - kM16Rows * vj);
  const int t_lo = sh.t_lo, t_hi = sh.t_hi;

  const moe_nf4_expert_t &ex = tab.e[e];
  const float *c1 = (const float *)uniform_ptr(ex.w1_code);
  const float *c3 = (const float *)uniform_ptr(ex.w3_code);
  const uint8_t *pk[2] = {(const uint8_t *)uniform_ptr(ex.w1_packed),
                          (const uint8_t *)uniform_ptr(ex.w3_packed)};
  const float *pa[2] = {(const float *)uniform_ptr(ex.w1_absmax),
                        (const float *)uniform_ptr(ex.w3_absmax)};

  // Stream pointers of the lane (row nl of a tile, bytes 16 kq of the wave's slice); the
  // first two tiles' loads go out before the activations' and the barrier below.
  const int nl = lane & 15, kq = lane >> 4;
  constexpr int kSlice = 128 * S;  // values of a wave's K slice (H / 8)
  const size_t row_bytes = (size_t)(H >> 1);
  const size_t row_blocks = (size_t)(H >> 6);
  const uint32_t lane_const[2] = {(uint32_t)(lane & 31) << 2, ((uint32_t)(lane & 31) << 2) | 128u};
  struct TileRegs {
    u32x4 w[2][S];
    f32x4 ab[2][S / 2];
  };
  auto load_w = [&](TileRegs &R, int t, int p, int s) {
    const size_t row = (size_t)t * kM16Rows + nl;
    R.w[p][s] = *reinterpret_cast<const MOE_GLOBAL u32x4 *>(
        (gq_t)pk[p] + row * row_bytes + (size_t)wave * (kSlice / 2) + 16 * kq + 64 * s);
  };
  auto load_ab = [&](TileRegs &R, int t) {
    const size_t row = (size_t)t * kM16Rows + nl;
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const ga_t ap = (ga_t)pa[p] + row * row_blocks + (size_t)wave * (2 * S);
#pragma unroll
      for (int q = 0; q < S / 2; ++q) R.ab[p][q] = *reinterpret_cast<const MOE_GLOBAL f32x4 *>(ap + 4 * q);
    }
  };
  auto load_tile = [&](TileRegs &R, int t) {
#pragma unroll
    for (int p = 0; p < 2; ++p)
#pragma unroll
      for (int s = 0; s < S; ++s) load_w(R, t, p, s);
    load_ab(R, t);
  };
  // Past the last tile the loads re-read it (L2, unused); a workgroup without tiles (more
  // workgroups than tiles) reads the expert's first tile and stops at the barrier.
  const int last = t_hi > t_lo ? t_hi - 1 : 0;
  TileRegs A, B;
  load_tile(A, min(t_lo, last));

  // The wave's K slice of the token rows, as A operands (s, j): lane (m = lane & 15, kq) holds
  // values m16_off(kq) + 8 (j & 1) .. +7 of block 2s + (j >> 1) of the slice of token row m
  // (the first row again past n).  With the routing in the launch, the routing's registers
  // hold every token's slice in this layout (lane 16 kq + t: token t): each lane takes its
  // row's from lane 16 kq + token in the same lane group, with no memory read.
  const int tok = g_ptok[r0 + (nl < n ? nl : 0)];
  bf16x8 xa[S][4];
  if constexpr (ROUTE) {
    const int src = (16 * kq + tok) << 2;  // byte address of the source lane
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const u32x4 v = __builtin_bit_cast(u32x4, xt[s][j]);
        u32x4 r;
#pragma unroll
        for (int q = 0; q < 4; ++q) r[q] = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)v[q]);
        xa[s][j] = as_bf16x8(r);
      }
  } else {
    const gx_t xrow = (gx_t)x + (size_t)tok * H + (size_t)wave * kSlice + m16_off(kq);
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
      for (int j = 0; j < 4; ++j) xa[s][j] = as_bf16x8(ld_u4(xrow + 128 * s + 64 * (j >> 1) + 8 * (j & 1)));
  }
  load_tile(B, min(t_lo + 1, last));

  // An expert whose w1 / w3 codebooks differ bitwise from the NF4 constants gets a table of
  // its own (replicas 0-31 w1, 32-63 w3).  LDS-only barriers: the weight loads stay in flight.
  float ref_f = kNf4Code[0];
#pragma unroll
  for (int q = 1; q < 16; ++q)
    if ((lane & 15) == q) ref_f = kNf4Code[q];
  const float cv = lane < 16 ? c1[lane & 15] : c3[lane & 15];
  const bool differ =
      __ballot(lane < 32 && __builtin_bit_cast(uint32_t, cv) != __builtin_bit_cast(uint32_t, ref_f)) != 0;
  if (differ) {
    float ca[16], cb[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      ca[q] = c1[q];
      cb[q] = c3[q];
    }
    lds_barrier();  // no wave still builds the constant table
    build_table_regs<kDecThreads>(s_tbl, ca, cb);
  }
  lds_barrier();
  if (t_lo >= t_hi) return;  // uniform over the workgroup

  int buf = 0;
  // Tile t from R (then tile t_next's loads into R); h rows written when `live`.  The steps
  // (projection p, load s) are software-pipelined: the table lookups of step i + 1 go out
  // before the MFMAs of step i.
  constexpr int kSteps = 2 * S;
  auto tile_step = [&](TileRegs &R, int t, int t_next, bool live) {
    // The slot's next load goes out only after its last use (the lookup addresses), so that
    // it can take the same registers: a load into other registers would need a copy at the
    // loop's back edge, which waits for it.  Slots 2j and 2j + 1 read the two halves of one
    // 128-byte line and go out together, after slot 2j + 1's last use: the L2 then serves
    // both from one fill (measured 2-4 % faster than one load per step).
    auto lookups = [&](int i, bf16x8 (&bo)[4]) {
      const int p = i / S, s = i % S;
      const u32x4 w = R.w[p][s];
      const auto lo = __builtin_amdgcn_permlane32_swap(w[0], w[2], false, false);
      const auto hi = __builtin_amdgcn_permlane32_swap(w[1], w[3], false, false);
      const uint32_t src[4] = {lo[0], hi[0], lo[1], hi[1]};
      uint32_t addr[4][4];
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          addr[q][j] = __builtin_amdgcn_perm(src[q], lane_const[p], 0x0c0c0400u + (j << 8));
      __builtin_amdgcn_sched_barrier(0);
      if (s & 1) {
        load_w(R, t_next, p, s - 1);
        load_w(R, t_next, p, s);
      }
#pragma unroll
      for (int q = 0; q < 4; ++q)
        bo[q] = as_bf16x8(lds_lookup(s_tbl, addr[q][0]), lds_lookup(s_tbl, addr[q][1]),
                          lds_lookup(s_tbl, addr[q][2]), lds_lookup(s_tbl, addr[q][3]));
    };
    f32x4 acc[2];
    acc[0] = acc[1] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    bf16x8 bc[4], bn[4];
    lookups(0, bc);
#pragma unroll
    for (int i = 0; i < kSteps; ++i) {
      const int p = i / S, s = i % S;
      if (i + 1 < kSteps) lookups(i + 1, bn);
      __builtin_amdgcn_sched_barrier(0);
      f32x4 ta = f32x4{0.0f, 0.0f, 0.0f, 0.0f}, tb = ta;
      ta = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[s][0], bc[0], ta, 0, 0, 0);
      ta = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[s][1], bc[1], ta, 0, 0, 0);
      tb = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[s][2], bc[2], tb, 0, 0, 0);
      tb = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[s][3], bc[3], tb, 0, 0, 0);
      const int ba = 2 * s;  // the blocks of load s: 2s (ta) and 2s + 1 (tb)
      scale_acc(acc[p], ta, R.ab[p][ba >> 2][ba & 3]);
      scale_acc(acc[p], tb, R.ab[p][(ba + 1) >> 2][(ba + 1) & 3]);
      if (i + 1 < kSteps) {
#pragma unroll
        for (int j = 0; j < 4; ++j) bc[j] = bn[j];
      }
    }
#pragma unroll
    for (int p = 0; p < 2; ++p) *reinterpret_cast<f32x4 *>(&s_red[buf][wave][p][lane * 4]) = acc[p];
    load_ab(R, t_next);
    lds_barrier();
    if (live && tid < kM16Rows * kM16Rows) {
      // Token row m, tile row c: D[m][c] is register m & 3 of lane 16 (m >> 2) + c.
      const int c = tid & 15, m = tid >> 4;
      const int idx = (16 * (m >> 2) + c) * 4 + (m & 3);
      float g = 0.0f, u = 0.0f;
#pragma unroll
      for (int w = 0; w < kDecWaves; ++w) {
        g += s_red[buf][w][0][idx];
        u += s_red[buf][w][1][idx];
      }
      if (m < n) h_out[(size_t)(r0 + m) * F + (size_t)t * kM16Rows + c] = swiglu_bf16(g, u);
    }
    buf ^= 1;
  };
  // An odd count ends with one more pass over the last tile whose h rows are not written.
  for (int t = t_lo; t < t_hi; t += 2) {
    tile_step(A, t, min(t + 2, last), true);
    tile_step(B, min(t + 1, last), min(t + 3, last), t + 1 < t_hi);
  }
}

// Down projection of mid-size batches on the 16x16x32 MFMA: virtual experts of up to 16 h
// rows, F split into parts of 2048 values (one fp32 ypart plane per part, which the combine
// adds in part order, model/moe_layer.py:186-191 after the expert's w2).  The workgroups are
// dealt to the (virtual expert, part) pairs by m16_share, each taking its share of the
// pair's 64-row output tiles one at a time; wave w covers values [256 w, 256 w + 256)
// of the part, so its slice of the expert's h rows stays in registers.  The tile is four
// 16-row MFMA column blocks, loaded and scaled as in mid16_gateup_kernel (two 64-byte loads
// per row of a block: four NF4 blocks); the eight waves' partial sums meet in LDS.
constexpr int kM16DownCols = 4;                      // 16-row column blocks of an output tile
constexpr int kM16DownTile = 16 * kM16DownCols;      // output rows of a tile
constexpr int kM16DownSlice = 256;                   // values of F of a wave's slice
constexpr int kM16DownPlane = kDecWaves * kM16DownSlice;  // values of F of a part (2048)
constexpr int kMidDownVals = kM16DownPlane;  // K values of one part (one ypart plane)

__global__ void __launch_bounds__(kDecThreads, 1)
mid16_down_kernel(const ExpertTable tab, const uint16_t *__restrict__ h, int H, int F, int E,
                  int parts, int rows_total, const Route rt, float *__restrict__ ypart) {
  __shared__ __attribute__((aligned(16))) uint32_t s_tbl[kTableWords];
  // Partial sums [buffer][wave][column block][r * 64 + lane] (16 floats of padding per block
  // spread the reads of one wave over all banks).
  constexpr int kPlane = 4 * kWave + 16;
  __shared__ float s_red[2][kDecWaves][kM16DownCols][kPlane];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // The counts, offsets and residency loads go out together (one round trip, under the
  // table build).
  const int cnt_raw = lane < E ? rt.counts[lane] : 0;
  const int off = lane < E ? rt.offsets[lane] : 0;
  const bool resident = lane < E && tab.e[lane < E ? lane : 0].w2_packed != nullptr;
  {
    float cst[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) cst[q] = kNf4Code[q];
    build_table_regs<kDecThreads>(s_tbl, cst, cst);
  }
  const int cnt = resident ? cnt_raw : 0;
  const int nv = (cnt + kM16Rows - 1) / kM16Rows;
  if (__ballot(nv > 0) == 0) return;  // uniform over the grid
  const M16Share sh = m16_share(nv, parts, H / kM16DownTile, E);
  const int e = sh.e, vj = sh.vj, kp = sh.part;
  const int r0 = __builtin_amdgcn_readlane(off, e) + kM16Rows * vj;  // first h row
  const int n = min(kM16Rows, __builtin_amdgcn_readlane(cnt, e) - kM16Rows * vj);
  const int t_lo = sh.t_lo, t_hi = sh.t_hi;

  const moe_nf4_expert_t &ex = tab.e[e];
  const float *c2 = (const float *)uniform_ptr(ex.w2_code);
  const uint8_t *pk = (const uint8_t *)uniform_ptr(ex.w2_packed);
  const float *pa = (const float *)uniform_ptr(ex.w2_absmax);

  const int nl = lane & 15, kq = lane >> 4;
  const int k0 = kp * kM16DownPlane + wave * kM16DownSlice;  // first value of the wave's slice
  const size_t row_bytes = (size_t)(F >> 1);
  const size_t row_blocks = (size_t)(F >> 6);
  // Both table halves hold w2's codebook: the lanes spread over all 64 replicas.
  const uint32_t lane_const = ((uint32_t)(lane & 31) << 2) | ((lane & 32) ? 128u : 0u);
  struct TileRegs {
    u32x4 w[kM16DownCols][2];
    f32x4 ab[kM16DownCols];
  };
  auto load_w = [&](TileRegs &R, int t, int cb, int s) {
    const size_t row = (size_t)t * kM16DownTile + 16 * cb + nl;
    R.w[cb][s] = *reinterpret_cast<const MOE_GLOBAL u32x4 *>(
        (gq_t)pk + row * row_bytes + (size_t)(k0 >> 1) + 16 * kq + 64 * s);
  };
  auto load_ab = [&](TileRegs &R, int t) {
#pragma unroll
    for (int cb = 0; cb < kM16DownCols; ++cb) {
      const size_t row = (size_t)t * kM16DownTile + 16 * cb + nl;
      R.ab[cb] = *reinterpret_cast<const MOE_GLOBAL f32x4 *>((ga_t)pa + row * row_blocks + (k0 >> 6));
    }
  };
  auto load_tile = [&](TileRegs &R, int t) {
#pragma unroll
    for (int cb = 0; cb < kM16DownCols; ++cb)
#pragma unroll
      for (int s = 0; s < 2; ++s) load_w(R, t, cb, s);
    load_ab(R, t);
  };
  // The first two tiles' loads go out before the h rows' and the barrier below (past the last
  // tile the loads re-read it; a workgroup without tiles reads the first and stops there).
  const int last = t_hi > t_lo ? t_hi - 1 : 0;
  TileRegs A, B;
  load_tile(A, min(t_lo, last));

  // The wave's slice of the h rows as A operands (s, j), laid out as in mid16_gateup_kernel.
  const gx_t hrow = (gx_t)h + (size_t)(r0 + (nl < n ? nl : 0)) * F + k0 + m16_off(kq);
  bf16x8 ha[2][4];
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int j = 0; j < 4; ++j) ha[s][j] = as_bf16x8(ld_u4(hrow + 128 * s + 64 * (j >> 1) + 8 * (j & 1)));
  load_tile(B, min(t_lo + 1, last));

  float ref_f = kNf4Code[0];
#pragma unroll
  for (int q = 1; q < 16; ++q)
    if ((lane & 15) == q) ref_f = kNf4Code[q];
  const float cv = c2[lane & 15];
  if (__ballot(lane < 16 && __builtin_bit_cast(uint32_t, cv) != __builtin_bit_cast(uint32_t, ref_f)) != 0) {
    float cc[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) cc[q] = c2[q];
    lds_barrier();  // no wave still builds the constant table
    build_table_regs<kDecThreads>(s_tbl, cc, cc);
  }
  lds_barrier();  // LDS only: the weight loads stay in flight
  if (t_lo >= t_hi) return;  // uniform over the workgroup

  int buf = 0;
  constexpr int kSteps = 2 * kM16DownCols;
  // Tile t from R (then tile t_next's loads into R); ypart rows written when `live`.  The
  // table lookups of step i + 1 go out before the MFMAs of step i.
  auto tile_step = [&](TileRegs &R, int t, int t_next, bool live) {
    // The next loads after the last use, the two halves of a 128-byte line together
    // (mid16_gateup_kernel).
    auto lookups = [&](int i, bf16x8 (&bo)[4]) {
      const int cb = i >> 1, s = i & 1;
      const u32x4 w = R.w[cb][s];
      const auto lo = __builtin_amdgcn_permlane32_swap(w[0], w[2], false, false);
      const auto hi = __builtin_amdgcn_permlane32_swap(w[1], w[3], false, false);
      const uint32_t src[4] = {lo[0], hi[0], lo[1], hi[1]};
      uint32_t addr[4][4];
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          addr[q][j] = __builtin_amdgcn_perm(src[q], lane_const, 0x0c0c0400u + (j << 8));
      __builtin_amdgcn_sched_barrier(0);
      if (s & 1) {
        load_w(R, t_next, cb, s - 1);
        load_w(R, t_next, cb, s);
      }
#pragma unroll
      for (int q = 0; q < 4; ++q)
        bo[q] = as_bf16x8(lds_lookup(s_tbl, addr[q][0]), lds_lookup(s_tbl, addr[q][1]),
                          lds_lookup(s_tbl, addr[q][2]), lds_lookup(s_tbl, addr[q][3]));
    };
    f32x4 acc[kM16DownCols];
#pragma unroll
    for (int cb = 0; cb < kM16DownCols; ++cb) acc[cb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    bf16x8 bc[4], bn[4];
    lookups(0, bc);
#pragma unroll
    for (int i = 0; i < kSteps; ++i) {
      const int cb = i >> 1, s = i & 1;
      if (i + 1 < kSteps) lookups(i + 1, bn);
      __builtin_amdgcn_sched_barrier(0);
      f32x4 ta = f32x4{0.0f, 0.0f, 0.0f, 0.0f}, tb = ta;
      ta = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ha[s][0], bc[0], ta, 0, 0, 0);
      ta = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ha[s][1], bc[1], ta, 0, 0, 0);
      tb = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ha[s][2], bc[2], tb, 0, 0, 0);
      tb = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ha[s][3], bc[3], tb, 0, 0, 0);
      scale_acc(acc[cb], ta, R.ab[cb][2 * s]);
      scale_acc(acc[cb], tb, R.ab[cb][2 * s + 1]);
      if (i + 1 < kSteps) {
#pragma unroll
        for (int j = 0; j < 4; ++j) bc[j] = bn[j];
      }
    }
#pragma unroll
    for (int cb = 0; cb < kM16DownCols; ++cb)
#pragma unroll
      for (int r = 0; r < 4; ++r) s_red[buf][wave][cb][r * kWave + lane] = acc[cb][r];
    load_ab(R, t_next);
    lds_barrier();
    if (live) {
      // Output row c of the tile, token rows m and m + 8: D[m][c % 16] of block c / 16 is
      // register m & 3 of lane 16 (m >> 2) + c % 16.
      const int c = tid & (kM16DownTile - 1);
#pragma unroll
      for (int hm = 0; hm < 2; ++hm) {
        const int m = (tid >> 6) + 8 * hm;
        const int idx = (m & 3) * kWave + 16 * (m >> 2) + (c & 15);
        float y = 0.0f;
#pragma unroll
        for (int w = 0; w < kDecWaves; ++w) y += s_red[buf][w][c >> 4][idx];
        if (m < n) ypart[((size_t)kp * rows_total + r0 + m) * H + (size_t)t * kM16DownTile + c] = y;
      }
    }
    buf ^= 1;
  };
  for (int t = t_lo; t < t_hi; t += 2) {
    tile_step(A, t, min(t + 2, last), true);
    tile_step(B, min(t + 1, last), min(t + 3, last), t + 1 < t_hi);
  }
}

}  // namespace

// One workgroup per CU: each owns ceil(tiles / CUs) 4-row output tiles of the down GEMV.
int decode_tiles_per_wg(int32_t H) {
  const int rt = H / 4;
  const int cap = device_cu_count();
  return (rt + cap - 1) / cap;
}

// K parts of the down GEMV (at most 8): F/512 / 4 when the F/512 stages split into parts of
// 4 (the single-token path's item), else the smallest divisor d of the stages that leaves
// at most 8 stages per part, else 1.
int decode_kparts(int32_t F) {
  const int ns = F / kStageVals;
  if (ns % 4 == 0 && ns / 4 <= kDecMaxKParts) return ns / 4;
  for (int d = 1; d <= kDecMaxKParts; ++d)
    if (ns % d == 0 && ns / d <= 8) return d;
  return 1;
}

bool decode_layer_supported(int64_t T, int32_t k, int32_t E, int32_t H, int32_t F) {
  return T >= 1 && T <= kDecMaxTokens && T * k <= kDecMaxSlots && E >= 1 &&
         E <= kDecMaxExperts && k >= 1 && k <= E && H % kStageVals == 0 &&
         F % kStageVals == 0 && H >= kStageVals && F >= kStageVals &&
         decode_tiles_per_wg(H) <= kDecMaxTilesPerWg;
}

int64_t decode_route_bytes() { return (int64_t)sizeof(DecodeRoute); }
int64_t mid_route_out_bytes() { return (int64_t)sizeof(MidRouteOut); }

// The mid-size path: up to 64 tokens, hidden size 2048 or 4096 (a wave's K slice of 256 or
// 512 values), F a multiple of 16, at most 32 experts.  At 64 tokens (Mixtral, ~16 rows per
// expert) it still measured ahead of the 32-row tiles of the streamed mid-batch kernels
// (uniform 278 against 281 us per layer, Zipf 216 against 238), at 32 and 40 tokens by
// 20-24 % (uniform 216 / 215 against 270 / 271).
constexpr int kMidMaxTokens = 64;

bool mid_gateup_supported(int64_t T, int32_t k, int32_t E, int32_t H, int32_t F) {
  return T >= 1 && T <= kMidMaxTokens && k >= 1 && E >= 1 && E <= kWave / 2 &&
         (H == 2048 || H == 4096) && F >= kM16Rows && F % kM16Rows == 0 &&
         T * (int64_t)H * 2 >= 2048 && (int64_t)E + T * k / kM16Rows + 1 <= device_cu_count();
}

// The same path with the routing and grouping in the kernel (every workgroup routes the
// tokens; workgroup 0 publishes the results): top-k <= 2 and at most 16 experts.
bool mid_layer_supported(int64_t T, int32_t k, int32_t E, int32_t H, int32_t F) {
  return mid_gateup_supported(T, k, E, H, F) && T <= kMidMaxT && k <= 2 && E <= 16 &&
         T * k <= kMidMaxSlots;
}

// With the grouping of a separate router launch's slots in the kernel: T * k <= 128.
bool mid_group_supported(int64_t T, int32_t k, int32_t E, int32_t H, int32_t F) {
  return mid_gateup_supported(T, k, E, H, F) && T * k <= kMidGroupMaxSlots;
}

// With the routing from a K-split gate-product launch: up to 64 tokens, top-k <= 2 and at
// most 16 experts (one MFMA column each).
bool mid_parts_supported(int64_t T, int32_t k, int32_t E, int32_t H, int32_t F) {
  return mid_group_supported(T, k, E, H, F) && T <= kMidPartTokens && k <= 2 &&
         E <= kMidPartExperts;
}
int64_t mid_parts_bytes() { return kMidPartsBytes; }

int launch_mid_gate_parts(const void *x, const void *gate, int64_t T, int32_t H, int32_t E,
                          void *parts, hipStream_t s) {
  MOE_REQUIRE(T >= 1 && T <= kMidPartTokens && E >= 1 && E <= kMidPartExperts &&
                  (H == 2048 || H == 4096),
              "shape not supported by the K-split gate products");
  MOE_REQUIRE(((uintptr_t)x | (uintptr_t)gate | (uintptr_t)parts) % 16 == 0,
              "x, gate and the partials must be 16-byte aligned");
  const dim3 grid((unsigned)(((T + 15) / 16) * kMidPartSlices)), blk(kWave);
  if (H == 4096)
    hipLaunchKernelGGL(mid_gate_parts_kernel<4>, grid, blk, 0, s, (const uint16_t *)x,
                       (const uint16_t *)gate, (int)T, H, E, (float *)parts);
  else
    hipLaunchKernelGGL(mid_gate_parts_kernel<2>, grid, blk, 0, s, (const uint16_t *)x,
                       (const uint16_t *)gate, (int)T, H, E, (float *)parts);
  MOE_LAUNCH_CHECK();
  return MOE_STATUS_OK;
}

// The mid-size down projection: F a multiple of 2048 (the parts), at most 16 parts (the
// combine's plane limit), H a multiple of the 64-row output tile.
// Every (virtual expert, part) pair needs a workgroup of its own: at most E + T k / 16
// virtual experts.
bool mid_down_supported(int64_t T, int32_t k, int32_t E, int32_t H, int32_t F) {
  return mid_gateup_supported(T, k, E, H, F) && F % kMidDownVals == 0 &&
         F / kMidDownVals <= 16 && H % kM16DownTile == 0 &&
         ((int64_t)E + T * k / kM16Rows) * (F / kMidDownVals) <= device_cu_count();
}
int mid_down_parts(int32_t F) { return F / kMidDownVals; }

int launch_mid_down(const void *tab_v, const void *h, int64_t T, int32_t k, int32_t H, int32_t F,
                    int32_t E, const void *route_v, void *ypart, int32_t parts, hipStream_t s) {
  MOE_REQUIRE(mid_down_supported(T, k, E, H, F) && parts == mid_down_parts(F),
              "shape not supported by the mid-size down projection");
  MOE_REQUIRE(((uintptr_t)h % 16) == 0, "h must be 16-byte aligned");
  const ExpertTable &tab = *static_cast<const ExpertTable *>(tab_v);
  const Route &rt = *static_cast<const Route *>(route_v);
  hipLaunchKernelGGL(mid16_down_kernel, dim3((unsigned)device_cu_count()), dim3(kDecThreads), 0, s,
                     tab, (const uint16_t *)h, H, F, E, parts, (int)(T * k), rt, (float *)ypart);
  MOE_LAUNCH_CHECK();
  return MOE_STATUS_OK;
}

int launch_mid_gateup(const void *tab_v, const void *x, int64_t T, int32_t k, int32_t H, int32_t F,
                      int32_t E, const void *route_v, void *h_ws, hipStream_t s,
                      const void *route_out) {
  const MidRouteOut ro = route_out ? *static_cast<const MidRouteOut *>(route_out) : MidRouteOut{};
  const int mode = route_out == nullptr ? kRtExternal
                   : ro.gate            ? kRtRoute
                   : ro.parts           ? kRtParts
                                        : kRtGroup;
  MOE_REQUIRE(mode == kRtExternal ? mid_gateup_supported(T, k, E, H, F)
                  : mode == kRtRoute ? mid_layer_supported(T, k, E, H, F)
                  : mode == kRtParts ? mid_parts_supported(T, k, E, H, F)
                                     : mid_group_supported(T, k, E, H, F),
              "shape not supported by the mid-size gate/up");
  MOE_REQUIRE(((uintptr_t)x % 16) == 0, "x must be 16-byte aligned");
  const ExpertTable &tab = *static_cast<const ExpertTable *>(tab_v);
  const Route rt = route_v ? *static_cast<const Route *>(route_v) : Route{};
  if (mode == kRtRoute) {
    MOE_REQUIRE(((uintptr_t)ro.gate % 16) == 0, "gate must be 16-byte aligned");
    MOE_REQUIRE(ro.w && ro.idx64, "null routing output");
  }
  if (mode != kRtExternal)
    MOE_REQUIRE(ro.idx32 && ro.counts && ro.offsets && ro.perm_tok && ro.slot_pos && ro.active,
                "null routing output");
  if (mode == kRtParts) {
    MOE_REQUIRE(ro.w && ro.idx64, "null routing output");
    MOE_REQUIRE(((uintptr_t)ro.parts % 16) == 0, "the gate partials must be 16-byte aligned");
  }
  const dim3 grid((unsigned)device_cu_count()), blk(kDecThreads);
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, grid, blk, 0, s, tab, (const uint16_t *)x, (int)T, H, F, E, k, rt, ro,
                       (uint16_t *)h_ws);
  };
  if (mode == kRtExternal)
    go(H == 4096 ? mid16_gateup_kernel<4, 8, kRtExternal> : mid16_gateup_kernel<2, 8, kRtExternal>);
  else if (mode == kRtGroup)
    go(H == 4096 ? mid16_gateup_kernel<4, 8, kRtGroup> : mid16_gateup_kernel<2, 8, kRtGroup>);
  else if (mode == kRtParts && E <= 8)
    go(H == 4096 ? mid16_gateup_kernel<4, 8, kRtParts> : mid16_gateup_kernel<2, 8, kRtParts>);
  else if (mode == kRtParts)
    go(H == 4096 ? mid16_gateup_kernel<4, 16, kRtParts> : mid16_gateup_kernel<2, 16, kRtParts>);
  else if (E <= 8)
    go(H == 4096 ? mid16_gateup_kernel<4, 8, kRtRoute> : mid16_gateup_kernel<2, 8, kRtRoute>);
  else
    go(H == 4096 ? mid16_gateup_kernel<4, 16, kRtRoute> : mid16_gateup_kernel<2, 16, kRtRoute>);
  MOE_LAUNCH_CHECK();
  return MOE_STATUS_OK;
}
int64_t decode_norm_bytes() { return (int64_t)sizeof(DecodeNorm); }

// Workgroups of the gate/up kernel: one per CU at most; each takes an even share of the
// (routed expert, 4-row tile) items, which its waves then share through an LDS counter
// (or split evenly, off the single-token path).
int64_t decode_gateup_groups(int64_t T, int32_t k, int32_t E, int32_t F) {
  const int64_t u_max = T * k < E ? T * k : E;
  const int64_t groups = (u_max * (F / 4) + kDecWaves - 1) / kDecWaves;
  const int64_t cap = device_cu_count();
  return groups < cap ? groups : cap;
}

// Gate/up (with routing) then down (with combine).  `ev`, when given, receives marks
// before the first kernel (twice: the routing has no launch of its own), between the two
// kernels and after the second.
int launch_decode_layer(const moe_nf4_expert_t *experts, int32_t E, const void *gate,
                        const void *bias, const void *x, int64_t T, int32_t H, int32_t F,
                        int32_t k, void *out, void *logits, void *weights, void *idx64,
                        void *route_ws, void *h_ws, hipStream_t s, hipEvent_t *ev,
                        const void *norm) {
  MOE_REQUIRE(decode_layer_supported(T, k, E, H, F), "shape not supported by the decode layer");
  MOE_REQUIRE(experts != nullptr, "null expert table");
  DecodeNorm nrm{};
  if (norm != nullptr) {
    nrm = *static_cast<const DecodeNorm *>(norm);
    MOE_REQUIRE(T == 1, "the fused norm takes one token (got %lld)", (long long)T);
    MOE_REQUIRE(H <= kDecNormMaxH, "the fused norm takes H <= %d (got %d)", kDecNormMaxH, H);
    MOE_REQUIRE(nrm.res && nrm.w && nrm.xs, "null norm pointer");
    MOE_REQUIRE(((uintptr_t)nrm.res | (uintptr_t)nrm.w | (uintptr_t)nrm.res_out |
                 (uintptr_t)nrm.xs) % 16 == 0,
                "norm tensors must be 16-byte aligned");
  }
  MOE_REQUIRE(((uintptr_t)x % 16) == 0 && ((uintptr_t)gate % 16) == 0,
              "x and gate must be 16-byte aligned");
  MOE_REQUIRE(((uintptr_t)route_ws % 16) == 0 && ((uintptr_t)h_ws % 16) == 0,
              "workspace regions must be 16-byte aligned");
  ExpertTable tab{};
  for (int e = 0; e < E; ++e) {
    const moe_nf4_expert_t &ex = experts[e];
    MOE_REQUIRE(ex.w1_packed && ex.w1_absmax && ex.w1_code && ex.w3_packed && ex.w3_absmax &&
                    ex.w3_code && ex.w2_packed && ex.w2_absmax && ex.w2_code,
                "expert %d is not resident (null pointer in its table entry)", e);
    tab.e[e] = ex;
  }
  const int64_t g1 = decode_gateup_groups(T, k, E, F);
  const int tpw = decode_tiles_per_wg(H);
  const int64_t g2 = (H / 4 + tpw - 1) / tpw;

  if (ev) MOE_HIP_CHECK(hipEventRecord(ev[0], s));
  if (ev) MOE_HIP_CHECK(hipEventRecord(ev[1], s));
  auto gateup = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3((unsigned)g1), dim3(kDecThreads), 0, s, tab,
                       (const uint16_t *)x, (const uint16_t *)gate, (const float *)bias, (int)T, H,
                       F, E, k, (uint16_t *)logits, (float *)weights, (int64_t *)idx64,
                       (DecodeRoute *)route_ws, (uint16_t *)h_ws, nrm);
  };
  const bool n1 = H <= 2 * kNormThreads * 8;  // the fused norm's one-chunk-per-thread form
  if (norm != nullptr && n1)
    gateup(E <= 8 ? decode_gateup_kernel<8, true, true> : decode_gateup_kernel<16, true, true>);
  else if (norm != nullptr)
    gateup(E <= 8 ? decode_gateup_kernel<8, true> : decode_gateup_kernel<16, true>);
  else if (T == 1 && n1)  // the token from the workgroup's LDS copy
    gateup(E <= 8 ? decode_gateup_kernel<8, false, true> : decode_gateup_kernel<16, false, true>);
  else
    gateup(E <= 8 ? decode_gateup_kernel<8, false> : decode_gateup_kernel<16, false>);
  MOE_LAUNCH_CHECK();
  if (ev) MOE_HIP_CHECK(hipEventRecord(ev[2], s));
  hipLaunchKernelGGL(decode_down_kernel, dim3((unsigned)g2), dim3(kDecThreads), 0, s, tab,
                     (const DecodeRoute *)route_ws, (const uint16_t *)h_ws, (int)T, H, F, E, k,
                     tpw, decode_kparts(F), (uint16_t *)out);
  MOE_LAUNCH_CHECK();
  if (ev) MOE_HIP_CHECK(hipEventRecord(ev[3], s));
  return MOE_STATUS_OK;
}

}  // namespace moe
