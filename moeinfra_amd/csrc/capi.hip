// C-ABI glue: error reporting, device info, workspace layout, and the composed
// entry points (whole MoE layer, single expert).
#include <stdarg.h>
#include <stdio.h>

#include <mutex>

#include "nf4_tile.h"

namespace moe {

int choose_nsplit(int64_t T, int32_t k, int32_t E, int32_t H, int32_t F);
int launch_expert_ffn(const moe_nf4_expert_t *experts, int32_t E, const void *x, int64_t T,
                      int32_t k, int32_t H, int32_t F, const int32_t *counts,
                      const int32_t *offsets, const int32_t *perm_tok, const int32_t *active,
                      void *h_ws, void *ypart, int32_t nsplit, int64_t max_tokens_per_expert,
                      int phases, hipStream_t stream, const FusedCombine *fused);
bool gemv4_supported(int64_t max_tokens_per_expert, int32_t H, int32_t F);
bool route_small_supported(int64_t T, int32_t k);
int launch_route_small(const void *x, const void *gate, const void *bias, int64_t T, int32_t H,
                       int32_t E, int32_t k, void *logits, void *w, void *idx64, void *idx32,
                       void *counts, void *offsets, void *perm_tok, void *slot_pos, void *active,
                       void *zero_word, hipStream_t stream);
int launch_combine(const void *ypart, int32_t nsplit, const void *weights, const void *idx_i32,
                   const void *slot_pos, int64_t T, int32_t k, int32_t H, void *out,
                   hipStream_t stream);
int launch_identity_route(int64_t T, int32_t *counts, int32_t *offsets, int32_t *perm_tok,
                          int32_t *active, hipStream_t stream);
int launch_reduce_splits(const float *ypart, int nsplit, int64_t numel, uint16_t *y,
                         hipStream_t stream);
bool decode_layer_supported(int64_t T, int32_t k, int32_t E, int32_t H, int32_t F);
bool mid_layer_supported(int64_t T, int32_t k, int32_t E, int32_t H, int32_t F);
bool mid_group_supported(int64_t T, int32_t k, int32_t E, int32_t H, int32_t F);
int launch_mid_layer_gateup(const moe_nf4_expert_t *experts, int32_t E, const void *x, int64_t T,
                            int32_t k, int32_t H, int32_t F, void *h_ws, const void *route_out,
                            hipStream_t stream);
// Mirrors the layout of MidRouteOut (decode_layer.hip): eleven pointers.
struct MidRouteArgs {
  const void *gate;
  const void *bias;
  void *logits, *w, *idx64, *idx32, *counts, *offsets, *perm_tok, *slot_pos, *active;
  const void *parts;
};
static_assert(sizeof(MidRouteArgs) == 12 * sizeof(void *), "MidRouteOut layout");
bool mid_parts_supported(int64_t T, int32_t k, int32_t E, int32_t H, int32_t F);
int64_t mid_parts_bytes();
int launch_mid_gate_parts(const void *x, const void *gate, int64_t T, int32_t H, int32_t E,
                          void *parts, hipStream_t s);
int64_t mid_route_out_bytes();
int64_t decode_route_bytes();
int launch_decode_layer(const moe_nf4_expert_t *experts, int32_t E, const void *gate,
                        const void *bias, const void *x, int64_t T, int32_t H, int32_t F,
                        int32_t k, void *out, void *logits, void *weights, void *idx64,
                        void *route_ws, void *h_ws, hipStream_t s, hipEvent_t *ev,
                        const void *norm);
// Mirrors the layout of DecodeNorm (decode_layer.hip).
struct DecodeNormArgs {
  const uint16_t *res;
  const uint16_t *w;
  float eps;
  uint16_t *res_out;
  uint16_t *xs;
};
int64_t decode_norm_bytes();

namespace {
thread_local char g_last_error[512] = "";

constexpr int kMaxDevices = 64;
int g_cu_count[kMaxDevices] = {0};
std::mutex g_cu_mutex;

constexpr int64_t kAlign = 256;
int64_t align_up(int64_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

// Byte offsets of the layer workspace regions.
struct LayerWs {
  int64_t idx32, counts, offsets, perm_tok, slot_pos, active, counter, droute, h, ypart,
      ypart_bytes, total;
  int nsplit;
};

// nsplit_override > 0 replaces the default number of down-projection ypart planes.
LayerWs layer_ws(int64_t T, int32_t k, int32_t E, int32_t H, int32_t F, int nsplit_override = 0) {
  LayerWs w{};
  const int64_t rows = T * k;
  w.nsplit = nsplit_override > 0 ? nsplit_override : choose_nsplit(T, k, E, H, F);
  int64_t o = 0;
  w.idx32 = o;    o = align_up(o + rows * 4);
  w.counts = o;   o = align_up(o + (int64_t)E * 4);
  w.offsets = o;  o = align_up(o + (int64_t)(E + 1) * 4);
  w.perm_tok = o; o = align_up(o + rows * 4);
  w.slot_pos = o; o = align_up(o + rows * 4);
  w.active = o;   o = align_up(o + (int64_t)(E + 1) * 4);
  w.counter = o;  o = align_up(o + 4);
  w.droute = o;   o = align_up(o + decode_route_bytes());
  w.h = o;        o = align_up(o + rows * (int64_t)F * 2);
  w.ypart = o;    o = align_up(o + (int64_t)w.nsplit * rows * H * 4);
  w.ypart_bytes = o - w.ypart;
  w.total = o;
  return w;
}

struct ExpertWs {
  int64_t counts, offsets, perm_tok, active, h, ypart, total;
  int nsplit;
};

ExpertWs expert_ws(int64_t T, int32_t H, int32_t F) {
  ExpertWs w{};
  w.nsplit = choose_nsplit(T, 1, 1, H, F);
  int64_t o = 0;
  w.counts = o;   o = align_up(o + 4);
  w.offsets = o;  o = align_up(o + 8);
  w.perm_tok = o; o = align_up(o + T * 4);
  w.active = o;   o = align_up(o + 8);
  w.h = o;        o = align_up(o + T * (int64_t)F * 2);
  w.ypart = o;    o = align_up(o + (int64_t)w.nsplit * T * H * 4);
  w.total = o;
  return w;
}

template <typename P>
P *at(void *base, int64_t off) {
  return reinterpret_cast<P *>(static_cast<char *>(base) + off);
}
}  // namespace

void set_error(const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof g_last_error, fmt, ap);
  va_end(ap);
}

int device_cu_count() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
  {
    std::lock_guard<std::mutex> lock(g_cu_mutex);
    if (g_cu_count[dev] > 0) return g_cu_count[dev];
  }
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    cus = 256;
  std::lock_guard<std::mutex> lock(g_cu_mutex);
  g_cu_count[dev] = cus;
  return cus;
}

}  // namespace moe

extern "C" const char *moe_last_error(void) { return moe::g_last_error; }

extern "C" int moe_version(void) { return 100; }

extern "C" int64_t moe_layer_workspace_bytes(int64_t T, int32_t k, int32_t E, int32_t H,
                                             int32_t F) {
  if (T < 0 || k < 1 || E < 1 || H < 1 || F < 1) return -1;
  return moe::layer_ws(T, k, E, H, F).total;
}

extern "C" int32_t moe_layer_down_splits(int64_t T, int32_t k, int32_t E, int32_t H, int32_t F) {
  if (T < 0 || k < 1 || E < 1 || H < 1 || F < 1) return -1;
  return moe::choose_nsplit(T, k, E, H, F);
}

namespace moe {
namespace {
// Decode batches (T <= 4, T*k <= 8, E <= 16) run the two-launch decode layer (routing in
// the gate/up kernel, combine in the down kernel).  Otherwise: router -> grouping ->
// gate/up -> down -> combine, with the fused routing + grouping kernel for T <= 16.
// `ev`, when given, receives hipEventRecord marks before the routing and after each of
// the three phases (route, gate/up, down + combine).
int layer_forward(const moe_nf4_expert_t *experts, int32_t E, const void *gate_bf16,
                  const void *bias_f32, const void *x_bf16, int64_t T, int32_t H, int32_t F,
                  int32_t k, void *out_bf16, void *logits_bf16, void *weights_f32, void *idx_i64,
                  void *workspace, int64_t workspace_bytes, hipStream_t s, hipEvent_t *ev,
                  int nsplit_override = 0) {
  MOE_REQUIRE(T >= 0 && k >= 1 && E >= 1 && H >= 1 && F >= 1, "bad sizes");
  if (T == 0) return MOE_STATUS_OK;
  MOE_REQUIRE(out_bf16 && weights_f32 && idx_i64, "null output pointer");
  const LayerWs w = layer_ws(T, k, E, H, F, nsplit_override);
  MOE_REQUIRE(workspace != nullptr && workspace_bytes >= w.total,
              "workspace too small: need %lld bytes, got %lld", (long long)w.total,
              (long long)workspace_bytes);
  MOE_REQUIRE(((uintptr_t)workspace % 256) == 0, "workspace must be 256-byte aligned");
  int32_t *idx32 = at<int32_t>(workspace, w.idx32);
  int32_t *counts = at<int32_t>(workspace, w.counts);
  int32_t *offsets = at<int32_t>(workspace, w.offsets);
  int32_t *perm_tok = at<int32_t>(workspace, w.perm_tok);
  int32_t *slot_pos = at<int32_t>(workspace, w.slot_pos);
  int32_t *active = at<int32_t>(workspace, w.active);
  uint32_t *counter = at<uint32_t>(workspace, w.counter);
  if (decode_layer_supported(T, k, E, H, F))
    return launch_decode_layer(experts, E, gate_bf16, bias_f32, x_bf16, T, H, F, k, out_bf16,
                               logits_bf16, weights_f32, idx_i64, at<void>(workspace, w.droute),
                               at<void>(workspace, w.h), s, ev, nullptr);
  if (ev) MOE_HIP_CHECK(hipEventRecord(ev[0], s));
  const bool mid = mid_layer_supported(T, k, E, H, F);
  // Above that size the mid-size gate/up groups the router's slots itself (no permute launch).
  const bool mid_group = !mid && mid_group_supported(T, k, E, H, F);
  const bool small = route_small_supported(T, k);
  int rc;
  if (mid) {
    MOE_REQUIRE(mid_route_out_bytes() == (int64_t)sizeof(MidRouteArgs), "MidRouteOut layout");
    // Routing and grouping inside the gate/up launch: events 0 and 1 back to back.
    if (ev) MOE_HIP_CHECK(hipEventRecord(ev[1], s));
    const MidRouteArgs ro{gate_bf16, bias_f32, logits_bf16, weights_f32, idx_i64, idx32, counts,
                          offsets, perm_tok, slot_pos, active, nullptr};
    rc = launch_mid_layer_gateup(experts, E, x_bf16, T, k, H, F, at<void>(workspace, w.h), &ro, s);
  } else if (mid_group && mid_parts_supported(T, k, E, H, F)) {
    // The gate products split over K by a small launch (no CU reads more than a slice of the
    // tokens and the gate), the routing and grouping in the gate/up launch.  The partials sit
    // at the start of the ypart region, which the down projection writes only after the
    // gate/up launch has read them.
    MOE_REQUIRE(w.ypart_bytes >= mid_parts_bytes(), "workspace too small for the gate partials");
    void *parts = at<void>(workspace, w.ypart);
    rc = launch_mid_gate_parts(x_bf16, gate_bf16, T, H, E, parts, s);
    if (rc == MOE_STATUS_OK) {
      if (ev) MOE_HIP_CHECK(hipEventRecord(ev[1], s));
      const MidRouteArgs ro{nullptr, bias_f32, logits_bf16, weights_f32, idx_i64, idx32, counts,
                            offsets, perm_tok, slot_pos, active, parts};
      rc = launch_mid_layer_gateup(experts, E, x_bf16, T, k, H, F, at<void>(workspace, w.h), &ro, s);
    }
  } else if (mid_group) {
    rc = moe_router_topk(x_bf16, gate_bf16, bias_f32, T, H, E, k, logits_bf16, weights_f32,
                         idx_i64, idx32, s);
    if (rc == MOE_STATUS_OK) {
      if (ev) MOE_HIP_CHECK(hipEventRecord(ev[1], s));
      const MidRouteArgs ro{nullptr, nullptr, nullptr, nullptr, nullptr, idx32, counts,
                            offsets, perm_tok, slot_pos, active, nullptr};
      rc = launch_mid_layer_gateup(experts, E, x_bf16, T, k, H, F, at<void>(workspace, w.h), &ro, s);
    }
  } else if (small) {
    rc = launch_route_small(x_bf16, gate_bf16, bias_f32, T, H, E, k, logits_bf16, weights_f32,
                            idx_i64, idx32, counts, offsets, perm_tok, slot_pos, active, counter,
                            s);
  } else {
    rc = moe_router_topk(x_bf16, gate_bf16, bias_f32, T, H, E, k, logits_bf16, weights_f32,
                         idx_i64, idx32, s);
    if (rc == MOE_STATUS_OK)
      rc = moe_permute(idx32, T, k, E, counts, offsets, perm_tok, slot_pos, active, s);
  }
  if (rc != MOE_STATUS_OK) return rc;
  if (!mid && !mid_group) {
    if (ev) MOE_HIP_CHECK(hipEventRecord(ev[1], s));
    rc = launch_expert_ffn(experts, E, x_bf16, T, k, H, F, counts, offsets, perm_tok, active,
                           at<void>(workspace, w.h), at<void>(workspace, w.ypart), w.nsplit, T, 1,
                           s, nullptr);
    if (rc != MOE_STATUS_OK) return rc;
  }
  if (ev) MOE_HIP_CHECK(hipEventRecord(ev[2], s));
  // The down projection can also fold the combine into its last workgroup (FusedCombine);
  // on MI355X the device-scope fences that needs cost more than the separate launch, so the
  // layer uses the stand-alone combine kernel.
  const bool fuse = false;
  const FusedCombine fc{(const float *)weights_f32, idx32, slot_pos, (uint16_t *)out_bf16, counter,
                        (int)T, k};
  rc = launch_expert_ffn(experts, E, nullptr, T, k, H, F, counts, offsets, perm_tok, active,
                         at<void>(workspace, w.h), at<void>(workspace, w.ypart), w.nsplit, T, 2,
                         s, fuse ? &fc : nullptr);
  if (rc != MOE_STATUS_OK) return rc;
  if (!fuse) {
    rc = launch_combine(at<void>(workspace, w.ypart), w.nsplit, weights_f32, idx32, slot_pos, T,
                        k, H, out_bf16, s);
    if (rc != MOE_STATUS_OK) return rc;
  }
  if (ev) MOE_HIP_CHECK(hipEventRecord(ev[3], s));
  return MOE_STATUS_OK;
}
}  // namespace
}  // namespace moe

extern "C" int moe_layer_forward_nf4(const moe_nf4_expert_t *experts, int32_t E,
                                     const void *gate_bf16, const void *bias_f32,
                                     const void *x_bf16, int64_t T, int32_t H, int32_t F,
                                     int32_t k, void *out_bf16, void *logits_bf16,
                                     void *weights_f32, void *idx_i64, void *workspace,
                                     int64_t workspace_bytes, void *stream) {
  return moe::layer_forward(experts, E, gate_bf16, bias_f32, x_bf16, T, H, F, k, out_bf16,
                            logits_bf16, weights_f32, idx_i64, workspace, workspace_bytes,
                            (hipStream_t)stream, nullptr);
}

extern "C" int moe_layer_forward_nf4_profiled(const moe_nf4_expert_t *experts, int32_t E,
                                              const void *gate_bf16, const void *bias_f32,
                                              const void *x_bf16, int64_t T, int32_t H,
                                              int32_t F, int32_t k, void *out_bf16,
                                              void *logits_bf16, void *weights_f32,
                                              void *idx_i64, void *workspace,
                                              int64_t workspace_bytes, void *const *events,
                                              void *stream) {
  MOE_REQUIRE(events != nullptr && events[0] && events[1] && events[2] && events[3],
              "four HIP events are required");
  hipEvent_t ev[4] = {(hipEvent_t)events[0], (hipEvent_t)events[1], (hipEvent_t)events[2],
                      (hipEvent_t)events[3]};
  return moe::layer_forward(experts, E, gate_bf16, bias_f32, x_bf16, T, H, F, k, out_bf16,
                            logits_bf16, weights_f32, idx_i64, workspace, workspace_bytes,
                            (hipStream_t)stream, ev);
}

extern "C" int64_t moe_expert_workspace_bytes(int64_t T, int32_t H, int32_t F) {
  if (T < 0 || H < 1 || F < 1) return -1;
  return moe::expert_ws(T, H, F).total;
}

extern "C" int moe_expert_swiglu_nf4(const moe_nf4_expert_t *expert, const void *x_bf16,
                                     int64_t T, int32_t H, int32_t F, void *y_bf16,
                                     void *workspace, int64_t workspace_bytes, void *stream) {
  MOE_REQUIRE(T >= 0 && T <= 0x7fffffff, "T out of range");
  MOE_REQUIRE(expert != nullptr, "null expert");
  if (T == 0) return MOE_STATUS_OK;
  MOE_REQUIRE(y_bf16 != nullptr && ((uintptr_t)y_bf16 % 8) == 0, "y must be 8-byte aligned");
  const moe::ExpertWs w = moe::expert_ws(T, H, F);
  MOE_REQUIRE(workspace != nullptr && workspace_bytes >= w.total,
              "workspace too small: need %lld bytes, got %lld", (long long)w.total,
              (long long)workspace_bytes);
  MOE_REQUIRE(((uintptr_t)workspace % 256) == 0, "workspace must be 256-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  int rc = moe::launch_identity_route(T, moe::at<int32_t>(workspace, w.counts),
                                      moe::at<int32_t>(workspace, w.offsets),
                                      moe::at<int32_t>(workspace, w.perm_tok),
                                      moe::at<int32_t>(workspace, w.active), s);
  if (rc != MOE_STATUS_OK) return rc;
  rc = moe::launch_expert_ffn(expert, 1, x_bf16, T, 1, H, F,
                              moe::at<int32_t>(workspace, w.counts),
                              moe::at<int32_t>(workspace, w.offsets),
                              moe::at<int32_t>(workspace, w.perm_tok),
                              moe::at<int32_t>(workspace, w.active),
                              moe::at<void>(workspace, w.h), moe::at<void>(workspace, w.ypart),
                              w.nsplit, T, 3, s, nullptr);
  if (rc != MOE_STATUS_OK) return rc;
  return moe::launch_reduce_splits(moe::at<float>(workspace, w.ypart), w.nsplit, T * (int64_t)H,
                                   (uint16_t *)y_bf16, s);
}

namespace {
// The single-token layer with the fused norm: the layer workspace at T = 1, then one row of
// normalised values per gate/up workgroup (at most one per CU).
int64_t norm_ws_rows_offset(int32_t k, int32_t E, int32_t H, int32_t F) {
  return moe::layer_ws(1, k, E, H, F).total;
}
}  // namespace

extern "C" int64_t moe_layer_norm_workspace_bytes(int32_t k, int32_t E, int32_t H, int32_t F) {
  if (k < 1 || E < 1 || H < 1 || F < 1) return -1;
  return moe::align_up(norm_ws_rows_offset(k, E, H, F) +
                       (int64_t)moe::device_cu_count() * H * 2);
}

extern "C" int moe_layer_forward_nf4_norm(const moe_nf4_expert_t *experts, int32_t E,
                                          const void *gate_bf16, const void *x_bf16,
                                          const void *residual_bf16, const void *norm_weight_bf16,
                                          float eps, int32_t H, int32_t F, int32_t k,
                                          void *residual_out_bf16, void *out_bf16,
                                          void *weights_f32, void *idx_i64, void *workspace,
                                          int64_t workspace_bytes, void *stream) {
  MOE_REQUIRE(k >= 1 && E >= 1 && H >= 1 && F >= 1, "bad sizes");
  MOE_REQUIRE(moe::decode_layer_supported(1, k, E, H, F),
              "shape not supported by the single-token decode layer");
  MOE_REQUIRE(experts && x_bf16 && residual_bf16 && norm_weight_bf16 && residual_out_bf16 &&
                  out_bf16 && weights_f32 && idx_i64 && gate_bf16,
              "null pointer");
  // Workgroup 0 writes residual_out while the others still read x, residual, the norm
  // weight and the gate; the down kernel writes out, which must not clobber residual_out.
  const int64_t hb = 2 * (int64_t)H;
  MOE_REQUIRE(!moe::ranges_overlap(residual_out_bf16, hb, x_bf16, hb) &&
                  !moe::ranges_overlap(residual_out_bf16, hb, residual_bf16, hb) &&
                  !moe::ranges_overlap(residual_out_bf16, hb, norm_weight_bf16, hb) &&
                  !moe::ranges_overlap(residual_out_bf16, hb, gate_bf16, hb * E),
              "residual_out must not overlap x, residual, norm_weight or the gate");
  MOE_REQUIRE(!moe::ranges_overlap(out_bf16, hb, residual_out_bf16, hb),
              "out must not overlap residual_out");
  const int64_t need = moe_layer_norm_workspace_bytes(k, E, H, F);
  MOE_REQUIRE(workspace != nullptr && workspace_bytes >= need,
              "workspace too small: need %lld bytes, got %lld", (long long)need,
              (long long)workspace_bytes);
  MOE_REQUIRE(((uintptr_t)workspace % 256) == 0, "workspace must be 256-byte aligned");
  static_assert(sizeof(moe::DecodeNormArgs) == 40, "DecodeNorm layout");
  MOE_REQUIRE(moe::decode_norm_bytes() == (int64_t)sizeof(moe::DecodeNormArgs), "DecodeNorm layout");
  const moe::LayerWs w = moe::layer_ws(1, k, E, H, F);
  moe::DecodeNormArgs nrm{(const uint16_t *)residual_bf16, (const uint16_t *)norm_weight_bf16, eps,
                          (uint16_t *)residual_out_bf16,
                          moe::at<uint16_t>(workspace, norm_ws_rows_offset(k, E, H, F))};
  return moe::launch_decode_layer(experts, E, gate_bf16, nullptr, x_bf16, 1, H, F, k, out_bf16,
                                  nullptr, weights_f32, idx_i64, moe::at<void>(workspace, w.droute),
                                  moe::at<void>(workspace, w.h), (hipStream_t)stream, nullptr, &nrm);
}

// ----------------------------------------------------------------- allocation-free layer
namespace moe {
namespace {
// The workspace of moe_layer_forward_nf4_noalloc.  Every device the library runs on holds
// its own copy, at its own address, until the process ends; in host code the name is a
// stand-in, so kernels get the device address from scratch_address().
static __device__ __align__(256) unsigned char scratch[MOE_NOALLOC_SCRATCH_BYTES];

void *g_scratch_addr[kMaxDevices] = {};
std::mutex g_scratch_mutex;

// Device address of `scratch` on the current device, looked up once per device.
int scratch_address(void **addr) {
  int dev = 0;
  MOE_HIP_CHECK(hipGetDevice(&dev));
  MOE_REQUIRE(dev >= 0 && dev < kMaxDevices, "device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_addr[dev] == nullptr) {
    void *p = nullptr;
    MOE_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    MOE_REQUIRE(p != nullptr && ((uintptr_t)p % 256) == 0, "scratch address lookup failed");
    g_scratch_addr[dev] = p;
  }
  *addr = g_scratch_addr[dev];
  return MOE_STATUS_OK;
}
}  // namespace
}  // namespace moe

// The layer's kernels write every workspace region they read (the descriptor, grouping
// arrays and h before their consumers, the completion word through the routing kernel), so
// nothing in the scratch has to start at zero and no memset is issued.
extern "C" int moe_layer_forward_nf4_noalloc(const moe_nf4_expert_t *experts, int32_t E,
                                             const void *gate_bf16, const void *bias_f32,
                                             const void *x_bf16, int64_t T, int32_t H,
                                             int32_t F, int32_t k, void *out_bf16,
                                             void *logits_bf16, void *weights_f32,
                                             void *idx_i64, void *stream) {
  MOE_REQUIRE(T >= 0 && k >= 1 && E >= 1 && H >= 1 && F >= 1, "bad sizes");
  if (T == 0) return MOE_STATUS_OK;
  // When the default layout (down-projection K splits over several ypart planes) does not
  // fit the scratch, one plane: the same results, fewer workgroups on the down projection.
  int nsplit = 0;
  int64_t need = moe::layer_ws(T, k, E, H, F).total;
  if (need > MOE_NOALLOC_SCRATCH_BYTES) {
    nsplit = 1;
    need = moe::layer_ws(T, k, E, H, F, 1).total;
  }
  MOE_REQUIRE(need <= MOE_NOALLOC_SCRATCH_BYTES,
              "layer needs %lld bytes of workspace, above the %lld-byte static scratch; call "
              "moe_layer_forward_nf4 with a workspace",
              (long long)need, (long long)MOE_NOALLOC_SCRATCH_BYTES);
  void *ws = nullptr;
  const int rc = moe::scratch_address(&ws);
  if (rc != MOE_STATUS_OK) return rc;
  return moe::layer_forward(experts, E, gate_bf16, bias_f32, x_bf16, T, H, F, k, out_bf16,
                            logits_bf16, weights_f32, idx_i64, ws, MOE_NOALLOC_SCRATCH_BYTES,
                            (hipStream_t)stream, nullptr, nsplit);
}
