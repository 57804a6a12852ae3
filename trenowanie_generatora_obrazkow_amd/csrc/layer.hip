// Whole-layer forward in one C call: the routed path of an inference step (router, dispatch, gate/up + SwiGLU,
// down + routing weight + scatter, combine) chained over the library's own entry points, with every intermediate
// carved out of one caller-provided workspace.  The same kernels run in the same order as when the five entry points
// are called one by one, so the outputs are identical; what the one call removes is the host work between them (a
// binding's per-call argument checks, output allocations and calls), which bounds small layers: a 512-token layer
// takes about 43 us of GPU time and about 80 us of host time when driven op by op from Python.
#include "../../include/hmoe.h"

#include <cstddef>
#include <cstdint>

namespace {

// The gate/up GEMM reads the routed rows as row-group tiles from this hidden width on (the dispatch writes them;
// 7% of the GEMM for M d 2 more bytes written), below it gathers the rows of x itself.
constexpr int64_t kTilesMinH = 4096;

size_t al256(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

struct FwdLayout {
  size_t logits, counts, starts, order, a_idx, inv, w_sorted, n_invalid, dws, tiles, act, y, total;
  size_t dws_bytes;
  bool tiles_on;
};

// Byte offsets of the intermediates; false for sizes no entry point accepts.
bool fwd_layout(int64_t T, int64_t d, int E, int k, int64_t h, FwdLayout& L) {
  if (T < 0 || d <= 0 || E <= 0 || k <= 0 || h <= 0 || k > E) return false;
  const int64_t M = T * k;
  const size_t tiles_bytes = hmoe_xs_tiles_bytes(M > 0 ? M : 1, E, d);
  L.tiles_on = h >= kTilesMinH && tiles_bytes > 0 && tiles_bytes < (static_cast<size_t>(1) << 31);
  L.dws_bytes = hmoe_dispatch_workspace_size(T, k, E);
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o += al256(bytes > 0 ? bytes : 1);
    return at;
  };
  L.logits = take(static_cast<size_t>(T) * static_cast<size_t>(E) * 4);  // the router's, when the caller has none
  L.counts = take(static_cast<size_t>(E) * 4);
  L.starts = take(static_cast<size_t>(E + 1) * 4);
  L.order = take(static_cast<size_t>(M) * 4);
  L.a_idx = take(static_cast<size_t>(M) * 4);
  L.inv = take(static_cast<size_t>(M) * 4);
  L.w_sorted = take(static_cast<size_t>(M) * 2);
  L.n_invalid = take(4);
  L.dws = take(L.dws_bytes);
  L.tiles = L.tiles_on ? take(tiles_bytes) : 0;
  L.act = take(static_cast<size_t>(M) * static_cast<size_t>(h) * 2);
  L.y = take(static_cast<size_t>(M) * static_cast<size_t>(d) * 2);
  L.total = o;
  return true;
}

}  // namespace

extern "C" {

size_t hmoe_moe_forward_workspace_size(int64_t T, int64_t d, int E, int k, int64_t h) {
  FwdLayout L;
  return fwd_layout(T, d, E, k, h, L) ? L.total : 0;
}

int hmoe_moe_forward(const void* x, int64_t ldx, const void* wr, const float* bias, const void* wgu, const void* wd,
                     int64_t T, int64_t d, int E, int k, int64_t h, int renorm, float scaling, void* out,
                     int32_t* topk_ids, float* topk_w, float* logits, void* workspace, size_t workspace_bytes,
                     hmoe_stream_t stream) {
  FwdLayout L;
  if (!fwd_layout(T, d, E, k, h, L)) return HMOE_ERR_ARG;
  if (T == 0) return HMOE_OK;
  if (!x || !wr || !wgu || !wd || !out || !topk_ids || !topk_w) return HMOE_ERR_ARG;
  if (!workspace || workspace_bytes < L.total) return HMOE_ERR_WORKSPACE;
  // the five entry points' own limits, checked before the first launch so that a refused call launches nothing
  auto mis16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) != 0; };
  if ((reinterpret_cast<uintptr_t>(workspace) & 255u) || mis16(x) || mis16(wr) || mis16(wgu) || mis16(wd) ||
      mis16(out) || ldx < d || ldx % 8)
    return HMOE_ERR_ARG;
  if (d % 8 || h % 8 || E > 256 || k > 16 || T * k >= (static_cast<int64_t>(1) << 31)) return HMOE_ERR_SHAPE;
  char* ws = static_cast<char*>(workspace);
  const int64_t M = T * k;
  auto* counts = reinterpret_cast<int32_t*>(ws + L.counts);
  auto* starts = reinterpret_cast<int32_t*>(ws + L.starts);
  auto* order = reinterpret_cast<int32_t*>(ws + L.order);
  auto* a_idx = reinterpret_cast<int32_t*>(ws + L.a_idx);
  auto* inv = reinterpret_cast<int32_t*>(ws + L.inv);
  auto* w_sorted = reinterpret_cast<uint16_t*>(ws + L.w_sorted);
  auto* n_invalid = reinterpret_cast<int32_t*>(ws + L.n_invalid);
  void* tiles = L.tiles_on ? ws + L.tiles : nullptr;
  void* act = ws + L.act;
  void* y = ws + L.y;
  // the logits go to the workspace when the caller keeps none: with more than 16 experts small token counts route
  // through them
  float* lg = logits ? logits : reinterpret_cast<float*>(ws + L.logits);
  int rc = hmoe_route_topk(x, ldx, wr, bias, T, d, E, k, renorm, scaling, lg, topk_ids, topk_w, stream);
  if (rc != HMOE_OK) return rc;
  rc = hmoe_dispatch_tiles(topk_ids, HMOE_DT_I32, topk_w, HMOE_DT_F32, T, k, E, L.tiles_on ? x : nullptr,
                           L.tiles_on ? ldx : 0, L.tiles_on ? d : 0, nullptr, tiles, counts, nullptr, starts, order,
                           a_idx, inv, w_sorted, n_invalid, ws + L.dws, L.dws_bytes, HMOE_DT_BF16, stream);
  if (rc != HMOE_OK) return rc;
  if (L.tiles_on)
    rc = hmoe_gate_up_swiglu_tiles(tiles, wgu, E, d, h, counts, HMOE_DT_I32, M, act, nullptr, HMOE_DT_BF16, stream);
  else
    rc = hmoe_gate_up_swiglu(x, ldx, a_idx, wgu, E, d, h, counts, HMOE_DT_I32, M, act, nullptr, HMOE_DT_BF16,
                             stream);
  if (rc != HMOE_OK) return rc;
  rc = hmoe_down_scatter(act, wd, E, h, d, counts, HMOE_DT_I32, M, w_sorted, order, y, nullptr, HMOE_DT_BF16,
                         stream);
  if (rc != HMOE_OK) return rc;
  return hmoe_combine(y, inv, T, k, d, out, HMOE_DT_BF16, stream);
}

}  // extern "C"

// The expert part for routing decided elsewhere (a model's own gate): hmoe_dispatch_tiles, hmoe_gate_up_swiglu(_tiles,
// _i8) and hmoe_down_scatter(_i8) over one workspace, in the order and with the choices of the op-by-op path.
namespace {

struct ExpLayout {
  size_t counts, starts, order, a_idx, w_sorted, dws, tiles, act, total;
  size_t dws_bytes;
  bool tiles_on;
};

bool exp_layout(int64_t T, int64_t d, int E, int k, int64_t h, int w_dtype, int dtype, ExpLayout& L) {
  if (T < 0 || d <= 0 || E <= 0 || k <= 0 || h <= 0) return false;
  const int64_t M = T * k;
  const size_t tiles_bytes = hmoe_xs_tiles_bytes(M > 0 ? M : 1, E, d);
  L.tiles_on = w_dtype == dtype && h >= kTilesMinH && tiles_bytes > 0 &&
               tiles_bytes < (static_cast<size_t>(1) << 31);
  L.dws_bytes = hmoe_dispatch_workspace_size(T, k, E);
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o += al256(bytes > 0 ? bytes : 1);
    return at;
  };
  L.counts = take(static_cast<size_t>(E) * 4);
  L.starts = take(static_cast<size_t>(E + 1) * 4);
  L.order = take(static_cast<size_t>(M) * 4);
  L.a_idx = take(static_cast<size_t>(M) * 4);
  L.w_sorted = take(static_cast<size_t>(M) * 2);
  L.dws = take(L.dws_bytes);
  L.tiles = L.tiles_on ? take(tiles_bytes) : 0;
  L.act = take(static_cast<size_t>(M) * static_cast<size_t>(h) * 2);
  L.total = o;
  return true;
}

}  // namespace

extern "C" {

size_t hmoe_moe_experts_workspace_size(int64_t T, int64_t d, int E, int k, int64_t h, int w_dtype, int dtype) {
  ExpLayout L;
  return exp_layout(T, d, E, k, h, w_dtype, dtype, L) ? L.total : 0;
}

int hmoe_moe_experts(const void* x, int64_t ldx, const void* topk_ids, int ids_dtype, const void* topk_w,
                     int topk_w_dtype, const void* wgu, const void* wgu_s, int wgu_s_dtype, const void* wd,
                     const void* wd_s, int wd_s_dtype, int w_dtype, int64_t T, int64_t d, int E, int k, int64_t h,
                     void* y, int32_t* inv_pos, int32_t* n_invalid, void* workspace, size_t workspace_bytes,
                     int dtype, hmoe_stream_t stream) {
  ExpLayout L;
  if (!exp_layout(T, d, E, k, h, w_dtype, dtype, L)) return HMOE_ERR_ARG;
  if (dtype != HMOE_DT_BF16 && dtype != HMOE_DT_F16) return HMOE_ERR_DTYPE;
  const bool i8 = w_dtype == HMOE_DT_I8;
  if (!i8 && w_dtype != dtype) return HMOE_ERR_DTYPE;
  if (i8 != (wgu_s != nullptr) || i8 != (wd_s != nullptr)) return HMOE_ERR_ARG;
  if (!workspace || workspace_bytes < L.total) return HMOE_ERR_WORKSPACE;
  // the GEMMs' limits, checked before the first launch so that a refused call launches nothing (an empty input
  // only runs the dispatch, which writes counts and n_invalid)
  auto mis16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) != 0; };
  if ((reinterpret_cast<uintptr_t>(workspace) & 255u) || mis16(x) || mis16(wgu) || mis16(wd) || mis16(y))
    return HMOE_ERR_ARG;
  if (T > 0 && (!x || !topk_ids || !topk_w || !wgu || !wd || !y || ldx < d || ldx % 8)) return HMOE_ERR_ARG;
  if (d % (i8 ? 16 : 8) || h % (i8 ? 16 : 8) || E > 1024 || T * k >= (static_cast<int64_t>(1) << 31))
    return HMOE_ERR_SHAPE;
  char* ws = static_cast<char*>(workspace);
  const int64_t M = T * k;
  auto* counts = reinterpret_cast<int32_t*>(ws + L.counts);
  auto* starts = reinterpret_cast<int32_t*>(ws + L.starts);
  auto* order = reinterpret_cast<int32_t*>(ws + L.order);
  auto* a_idx = reinterpret_cast<int32_t*>(ws + L.a_idx);
  auto* w_sorted = reinterpret_cast<uint16_t*>(ws + L.w_sorted);
  void* tiles = L.tiles_on ? ws + L.tiles : nullptr;
  void* act = ws + L.act;
  // the dispatch checks ids, weights, sizes and x first; an empty input stops after it (counts and n_invalid written)
  int rc = hmoe_dispatch_tiles(topk_ids, ids_dtype, topk_w, topk_w_dtype, T, k, E, L.tiles_on ? x : nullptr,
                               L.tiles_on ? ldx : 0, L.tiles_on ? d : 0, nullptr, tiles, counts, nullptr, starts, order,
                               a_idx, inv_pos, M > 0 ? w_sorted : nullptr, n_invalid, ws + L.dws, L.dws_bytes, dtype,
                               stream);
  if (rc != HMOE_OK || M == 0) return rc;
  if (L.tiles_on)
    rc = hmoe_gate_up_swiglu_tiles(tiles, wgu, E, d, h, counts, HMOE_DT_I32, M, act, nullptr, dtype, stream);
  else if (i8)
    rc = hmoe_gate_up_swiglu_i8(x, ldx, a_idx, wgu, wgu_s, wgu_s_dtype, E, d, h, counts, HMOE_DT_I32, M, act, dtype,
                                stream);
  else
    rc = hmoe_gate_up_swiglu(x, ldx, a_idx, wgu, E, d, h, counts, HMOE_DT_I32, M, act, nullptr, dtype, stream);
  if (rc != HMOE_OK) return rc;
  if (i8)
    return hmoe_down_scatter_i8(act, wd, wd_s, wd_s_dtype, E, h, d, counts, HMOE_DT_I32, M, w_sorted, order, y, dtype,
                                stream);
  return hmoe_down_scatter(act, wd, E, h, d, counts, HMOE_DT_I32, M, w_sorted, order, y, nullptr, dtype, stream);
}

}  // extern "C"
