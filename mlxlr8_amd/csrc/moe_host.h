// Host-side helpers shared by the C-ABI entry points: error reporting and per-device setup.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/moe_mi355x.h"
#include "moe_plan.h"

namespace moe {

// Record a message for moe_last_error() and return `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Build the E4M3 codebook table on the current device once (thread-safe).
int ensure_device_ready();

// Number of compute units of the current device (cached per device).
int device_cus();

// Bound of the fused decode blocks' cross-wave waits, in polls of their longest pause: the default
// (~50 ms) unless moe_set_wait_bound set another.  Passed to every fused launch.
constexpr int kDefaultWaitPolls = 1 << 14;
int wait_polls();

// Device address of the current device's 64 KB E4M3 code table (after ensure_device_ready), for
// kernels of other translation units.
const uint8_t* codebook_device_table();
// The same table as fp16 values (128 KB).
const uint16_t* codebook_f16_device_table();

// Router GEMV + route + dispatch plan for decode batches (router.hip).
int moe_router_fused_plan(const uint16_t* x, const float* w, const float* bias, int rows, int hidden, int experts,
                          float* logits, uint32_t* ids, float* scores, Plan* plan, int32_t* counter, hipStream_t s,
                          const uint16_t* attn = nullptr, const uint16_t* norm_w = nullptr, float eps = 0.0f,
                          uint16_t* h_out = nullptr, uint16_t* xn_out = nullptr);

// Sorted work order of the grouped entries (prefill.hip): moe_segment_table with ids outside
// [0, experts) clamped to the nearest valid expert (moe_segment_table skips them).
int segment_table_clamped(const uint32_t* ids, int n, int experts, int block_rows, int32_t* order, int32_t* counts,
                          int32_t* starts, int32_t* table, int capacity, int32_t* num_blocks, hipStream_t s);

// Fused K4 decode block (k4_layer.hip): route = 1 runs the router and plan on the device (slot 8 of
// every row = the shared expert, id 256), route = 0 uses the plan in the layer workspace, built
// beforehand from ids.  combine = 1 writes out (scores [rows, 8], residual), else per-slot values.
size_t k4_layer_workspace_bytes(int h, int m);
bool k4_layer_supported(int h, int m, bool route);
int k4_layer_check_alignment(const uint16_t* x, const uint16_t* residual, const uint16_t* const in_scale[3],
                             const uint16_t* const out_scale[3], const uint16_t* out, const uint16_t* values);
// The layer's residual add + RMSNorm folded into a one-row fused K4 launch (exlr8/fast_norm.py:20-28):
// h = T(x + residual) is written to the launch's residual argument and the normalised row to its
// x argument before either is read.
struct LayerNorm {
  const uint16_t* x;
  const uint16_t* residual;  // may be null (h = x)
  const uint16_t* w;
  float eps;
};
int k4_layer_run(const uint16_t* x, const uint16_t* residual, int rows, int route, const float* router_w,
                 const float* bias, uint32_t* ids, float* scores, const uint8_t* const packed[3],
                 const uint16_t* const in_scale[3], const uint16_t* const out_scale[3], int h, int m, int experts,
                 int combine, uint16_t* out, uint16_t* values, void* layer_ws, hipStream_t s,
                 const LayerNorm* norm = nullptr, int bits = 4);
// The layer workspace's plan (where a plan kernel writes it for route = 0).
Plan* k4_layer_plan(void* layer_ws);
// The fused block's work list for `units` units: 5 ints per item (kind, unit, a, b, c; see
// k4_layer.hip), in list order; returns the item count (items may be NULL to ask for it).
int k4_layer_item_list(int h, int m, int units, int route, int32_t* items, int capacity);
// The layer workspace's flag words (LayerFlag, layer_sync.h).
int32_t* k4_layer_flags(void* layer_ws, int h, int m);

// Fused joined-MXFP4 decode block for one token row (mx_layer.hip; hidden 6144, intermediate 2048,
// 256 routed experts + the shared expert 256): router, both projections of the nine slots and the
// combine in one launch.  `layer_ws`: mx_layer_workspace_bytes() bytes, zeroed once.
size_t mx_layer_workspace_bytes();
int32_t* mx_layer_flags(void* layer_ws);
// The flag words of the fused MXFP4 block inside a moe_mxfp4_workspace_bytes() workspace, and inside
// the allocation-free entry's per-device scratch.
int32_t* mx_workspace_flags(void* workspace, int h, int m);
int mx_scratch_flags(int32_t** flags);
int mx_layer_run(const uint16_t* x, const uint16_t* residual, const float* router_w, const float* bias, uint32_t* ids,
                 float* scores, const uint8_t* gu_codes, const uint8_t* gu_scales, const uint8_t* d_codes,
                 const uint8_t* d_scales, const uint16_t* unit, const uint16_t* out_gate, const uint16_t* out_up,
                 const uint16_t* in_down, const uint16_t* out_down, uint16_t* out, void* layer_ws, hipStream_t s);

}  // namespace moe

#define MOE_HIP(expr)                                                              \
  do {                                                                             \
    hipError_t e_ = (expr);                                                        \
    if (e_ != hipSuccess)                                                          \
      return ::moe::fail((int)e_, "%s failed: %s", #expr, hipGetErrorString(e_));  \
  } while (0)

#define MOE_ARG(cond, ...)                                       \
  do {                                                           \
    if (!(cond)) return ::moe::fail(MOE_EINVAL, __VA_ARGS__);    \
  } while (0)
