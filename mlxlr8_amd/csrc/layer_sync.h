// Cross-wave hand-over and routing shared by the fused decode blocks (K4 trellis and joined MXFP4):
// tagged 64-bit words, bounded waits, router items and the per-block routing into an LDS plan.
//
// Reference semantics (paths relative to the reference root):
//   logits = f32(x) @ W^T, sigmoid, bias-corrected top-8  exlr8/model.py:111-132,
//                                                          exlr8/metal/fast_router.metal:1-42
//
// The functions are templates over the launch's argument block, which provides x [rows, h] bf16,
// rows, h, router_w [256, h] fp32, bias [256], ids [rows, 9], scores [rows, 8] and a workspace `w`
// with `flags` (LayerFlag words) and `logit_part` ([rows][h / kRouterSlice][256] tagged words).
//
// Tagged words: a value another wave reads is stored as one 64-bit word (value, tag), the tag being
// the launch's epoch + 1; a consumer reloads until every word it needs carries the current tag.
// Waits are bounded: an exhausted wait sets the error word and the wave continues.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "moe_device.h"
#include "moe_plan.h"
#include "route.h"

namespace moe {

constexpr int kRouterSlice = 1024;  // router inputs per work item
constexpr int kMaxRouteHidden = 8192;  // hidden size limit of the fused router
// Workspace words of a fused block: LF_ERROR is set by a wave whose bounded wait ran out, LF_EXIT
// counts the blocks that left, LF_EPOCH tags the launch's words, LF_STALLED counts the launches
// that ended with LF_ERROR set (the last block to leave folds LF_ERROR into it and clears it; the
// host reads and resets it with moe_decode_status).
enum LayerFlag { LF_ERROR = 1, LF_EXIT = 2, LF_EPOCH = 3, LF_STALLED = 4, LF_COUNT = 8 };

// The lane index recomputed where it is used.  Code that runs rarely (router items, routing,
// finishes) uses it: with the plain index the compiler hoists their lane-derived addresses to the
// kernel's start, keeps them live across the decode loop and spills its registers to memory, and
// every reload in a latency-critical item then costs a memory round trip.
__device__ __forceinline__ int cold_lane() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

// ---------------------------------------------------------------- coherent and tagged words
__device__ __forceinline__ int ld_coh_i(const int32_t* p) {
  return __hip_atomic_load(const_cast<int32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ void st_coh_i(int32_t* p, int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ float ld_coh_f(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ uint64_t ld_tag(const uint64_t* p) {
  return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ void st_tag(uint64_t* p, float v, uint32_t tag) {
  __hip_atomic_store(p, (uint64_t)__float_as_uint(v) | ((uint64_t)tag << 32), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ bool has_tag(uint64_t w, uint32_t tag) { return (uint32_t)(w >> 32) == tag; }
__device__ __forceinline__ float tag_value(uint64_t w) { return __uint_as_float((uint32_t)w); }
template <class A>
__device__ __forceinline__ void set_error(const A& a) {
  if (lane_id() == 0) st_coh_i(a.w.flags + LF_ERROR, 1);
}
// One step of a bounded wait; false once the bound is exhausted (the error word is then set).
// The pause doubles from 64 clocks up to 64 * kMaxPauses: waiting waves must leave the memory
// system to the producers they wait for (hundreds of waves re-reading their inputs back to back
// starve them).  A wait on the critical path that only one wave per block makes (routing) uses a
// short pause; the bound on the total wait stays the same (~50 ms).  `a.wait_polls` is the bound
// in polls of the longest pause (kDefaultWaitPolls unless the host set another: moe_set_wait_bound).
template <int kMaxPauses = 64, class A>
__device__ __forceinline__ bool keep_waiting(const A& a, int& spins) {
  if (++spins >= a.wait_polls * (64 / kMaxPauses)) {
    set_error(a);
    return false;
  }
  const int pauses = spins < 6 ? min(1 << spins, kMaxPauses) : kMaxPauses;
  for (int k = 0; k < pauses; k++) __builtin_amdgcn_s_sleep(1);
  return true;
}
// The launch's exit, run by every thread of every block after its work: the last block to leave
// folds the error word into the stalled-launch count and clears it, resets LF_EXIT and advances
// the epoch.  Every wave's stores (an error word among them) are acknowledged before its block
// counts itself out, so the last block sees every error of the launch.  Returns whether this
// block was the last (its remaining resets are the caller's).
template <class A>
__device__ __forceinline__ bool leave_launch(const A& a, uint32_t epoch, int32_t& exit_last_lds) {
  release_stores();
  __syncthreads();
  if (threadIdx.x == 0)
    exit_last_lds = __hip_atomic_fetch_add(a.w.flags + LF_EXIT, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) + 1 ==
                    (int)gridDim.x;
  __syncthreads();
  const bool last = exit_last_lds != 0;
  if (last && threadIdx.x == 0) {
    if (ld_coh_i(a.w.flags + LF_ERROR) != 0) {
      st_coh_i(a.w.flags + LF_STALLED, ld_coh_i(a.w.flags + LF_STALLED) + 1);
      st_coh_i(a.w.flags + LF_ERROR, 0);
    }
    st_coh_i(a.w.flags + LF_EXIT, 0);
    st_coh_i(a.w.flags + LF_EPOCH, (int)(epoch + 1u == 0xFFFFFFFEu ? 0u : epoch + 1u));
  }
  return last;
}

// the lane's two words p[0], p[1] (a column pair) once both carry `tag`
template <int kMaxPauses = 64, class A>
__device__ __forceinline__ f32x2 ld_tag_pair(const A& a, const uint64_t* p, uint32_t tag) {
  uint64_t w0 = ld_tag(p), w1 = ld_tag(p + 1);
  int spins = 0;
  while (!__all(has_tag(w0, tag) && has_tag(w1, tag)) && keep_waiting<kMaxPauses>(a, spins)) {
    w0 = ld_tag(p);
    w1 = ld_tag(p + 1);
  }
  return f32x2{tag_value(w0), tag_value(w1)};
}
// ---------------------------------------------------------------- plan in LDS
// Each block holds the plan in LDS: per unit the expert id, the token count, the unit's token rows
// (3 bits each) and slots (7 bits each) packed, and (when the launch routes) the rows' scores.
// A routing launch computes it in every block; otherwise it is copied from the prebuilt plan.
struct PlanLds {
  int32_t units;
  int32_t ex[kMaxUnits], nt[kMaxUnits];
  uint32_t tok[kMaxUnits], sl0[kMaxUnits], sl1[kMaxUnits];
  float score[kMaxRows * 8];
};

// ---------------------------------------------------------------- router
// item r = e * S + j: partial logit of expert e over inputs [kRouterSlice j, kRouterSlice (j + 1))
// for every row, stored tagged at logit_part[(row * S + j) * 256 + e].
// The item in two halves: the loads of its weights and of row 0's inputs (issue), then the sums and
// stores (finish), so a wave can put other loads in flight between them.
constexpr int kRouterPer = kRouterSlice / 64;  // 16 inputs per lane
struct RouterLoads {
  f32x4 w[kRouterPer / 4];
  u32x4 x0[kRouterPer / 8];
};
template <class A>
__device__ __forceinline__ void router_item_issue(const A& a, int r, int S, RouterLoads& rl) {
  const int e = r / S, j = r - e * S;
  const int k0 = j * kRouterSlice + kRouterPer * cold_lane();
#pragma unroll
  for (int i = 0; i < kRouterPer / 4; i++)
    rl.w[i] = *reinterpret_cast<const f32x4*>(a.router_w + (int64_t)e * a.h + k0 + 4 * i);
#pragma unroll
  for (int i = 0; i < kRouterPer / 8; i++) rl.x0[i] = *reinterpret_cast<const u32x4*>(a.x + k0 + 8 * i);
}
template <class A>
__device__ __forceinline__ void router_item_finish(const A& a, int r, int S, uint32_t tag, const RouterLoads& rl) {
  const int e = r / S, j = r - e * S;
  const int lane = cold_lane();
  constexpr int kPer = kRouterPer;
  const int k0 = j * kRouterSlice + kPer * lane;
  for (int row = 0; row < a.rows; row++) {
    u32x4 xv[kPer / 8];
#pragma unroll
    for (int i = 0; i < kPer / 8; i++)
      xv[i] = row == 0 ? rl.x0[i] : *reinterpret_cast<const u32x4*>(a.x + (int64_t)row * a.h + k0 + 8 * i);
    const f32x4* w = rl.w;
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < kPer / 8; i++) {
      const f32x4 wa = w[2 * i], wb = w[2 * i + 1];
      acc = fmaf(bf16_to_f32((uint16_t)(xv[i].x & 0xFFFFu)), wa.x, acc);
      acc = fmaf(bf16_to_f32((uint16_t)(xv[i].x >> 16)), wa.y, acc);
      acc = fmaf(bf16_to_f32((uint16_t)(xv[i].y & 0xFFFFu)), wa.z, acc);
      acc = fmaf(bf16_to_f32((uint16_t)(xv[i].y >> 16)), wa.w, acc);
      acc = fmaf(bf16_to_f32((uint16_t)(xv[i].z & 0xFFFFu)), wb.x, acc);
      acc = fmaf(bf16_to_f32((uint16_t)(xv[i].z >> 16)), wb.y, acc);
      acc = fmaf(bf16_to_f32((uint16_t)(xv[i].w & 0xFFFFu)), wb.z, acc);
      acc = fmaf(bf16_to_f32((uint16_t)(xv[i].w >> 16)), wb.w, acc);
    }
    const float tot = wave_sum(acc);
    if (lane == 63) st_tag(a.w.logit_part + ((int64_t)row * S + j) * 256 + e, tot, tag);
  }
}
template <class A>
__device__ __forceinline__ void router_item(const A& a, int r, int S, uint32_t tag) {
  RouterLoads rl;
  router_item_issue(a, r, S, rl);
  router_item_finish(a, r, S, tag, rl);
}

// Routing of every row by one wave into its block's plan table: logits summed over their slices in
// slice order, bias-corrected top-8 per row, then the units -- the shared expert as unit 0 and the
// routed experts in first-appearance (slot) order.  Every block computes the same table from the
// same words; block 0 also stores ids and scores for the caller.
template <class A>
__device__ void route_block(const A& a, int S, uint32_t tag, PlanLds& T) {
  const int lane = cold_lane();
  __shared__ int32_t sid_lds[kMaxRows * kSlots];
  constexpr int kMaxS = kMaxRouteHidden / kRouterSlice;
  float bias[4];
#pragma unroll
  for (int i = 0; i < 4; i++) bias[i] = a.bias[lane + 64 * i];
  for (int row = 0; row < a.rows; row++) {
    const uint64_t* lp = a.w.logit_part + (int64_t)row * S * 256;
    int spins = 0;
    // every word of the lane's four experts in one round trip; while some are not yet current, a
    // sample (one word per lane spread over the row's slices) is polled before loading them again
    uint64_t wd[kMaxS][4];
    for (;;) {
#pragma unroll
      for (int j = 0; j < kMaxS; j++)
#pragma unroll
        for (int i = 0; i < 4; i++) wd[j][i] = ld_tag(lp + (int64_t)min(j, S - 1) * 256 + lane + 64 * i);
      bool ok = true;
#pragma unroll
      for (int j = 0; j < kMaxS; j++)
#pragma unroll
        for (int i = 0; i < 4; i++) ok = ok & has_tag(wd[j][i], tag);
      if (__all(ok)) break;
      bool live = true;
      for (;;) {
        if (__all(has_tag(ld_tag(lp + (lane * 24 + 7) % (S * 256)), tag))) break;
        if (!keep_waiting<4>(a, spins)) {
          live = false;
          break;
        }
      }
      if (!live) break;
    }
    RouteInput in;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      float v = 0.0f;
#pragma unroll
      for (int j = 0; j < kMaxS; j++)
        if (j < S) v += tag_value(wd[j][i]);
      in.logit[i] = v;
      in.bias[i] = bias[i];
    }
    route_select<false>(in, row, a.ids, a.scores, sid_lds, blockIdx.x == 0, T.score);
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  if (a.rows == 1) {
    // one row: unit 0 = the shared expert (slot 8), unit 1 + k = the row's expert of rank k (slot k)
    if (lane < kSlots) {
      const int u = lane < 8 ? lane + 1 : 0;
      T.ex[u] = lane < 8 ? min(max(sid_lds[lane], 0), 255) : 256;
      T.nt[u] = 1;
      T.tok[u] = 0u;
      T.sl0[u] = (uint32_t)lane;
      T.sl1[u] = 0u;
    }
    if (lane == 0) T.units = kSlots;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    return;
  }
  // Units.  Routed slot s' = 8 row + k is lane s' (global slot 9 row + k).  A row holds each expert
  // at most once, so a slot's position inside its unit is the number of earlier rows that chose the
  // same expert; the unit's first slot (position 0) leads it, and units are numbered in the order
  // of their leading slots.  Per-row expert bitmaps in LDS answer both questions in one pass over
  // the rows; the unit's rows and slots are then merged with LDS or (order-free).
  __shared__ uint32_t row_bits[kMaxRows][8];  // row r: bit e when expert e is in the row's top-8
  __shared__ uint8_t row_rank[kMaxRows][256];  // row r, expert e: its rank in the row (where set)
  const int n = a.rows * 8;
  const bool act = lane < n;
  const int row = lane >> 3, k = lane & 7;
  const int e = act ? min(max(sid_lds[row * kSlots + k], 0), 255) : 0;
  row_bits[lane >> 3][lane & 7] = 0u;
  for (int u = lane; u < kMaxUnits; u += 64) {
    T.tok[u] = 0u;
    T.sl0[u] = 0u;
    T.sl1[u] = 0u;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  if (act) {
    __hip_atomic_fetch_or(&row_bits[row][e >> 5], 1u << (e & 31), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    row_rank[row][e] = (uint8_t)k;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  int pos = 0, total = 0, first_row = row;
  for (int r = a.rows - 1; r >= 0; r--) {
    const int b = (int)((row_bits[r][e >> 5] >> (e & 31)) & 1u);
    total += b;
    pos += r < row ? b : 0;
    first_row = b ? r : first_row;
  }
  const int first_lane = first_row * 8 + row_rank[first_row][e];
  const uint64_t firsts = __ballot(act && pos == 0);
  const int unit = 1 + (int)__popcll(firsts & ((1ull << first_lane) - 1ull));
  if (act) {
    if (pos == 0) {
      T.ex[unit] = e;
      T.nt[unit] = total;
    }
    const uint32_t gs = (uint32_t)(row * kSlots + k);
    __hip_atomic_fetch_or(&T.tok[unit], (uint32_t)row << (3 * pos), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (pos < 4)
      __hip_atomic_fetch_or(&T.sl0[unit], gs << (7 * pos), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    else
      __hip_atomic_fetch_or(&T.sl1[unit], gs << (7 * (pos - 4)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  if (lane == 0) {
    uint32_t t0 = 0, z0 = 0, z1 = 0;
    for (int r = 0; r < a.rows; r++) {
      t0 |= (uint32_t)r << (3 * r);
      if (r < 4) z0 |= (uint32_t)(r * kSlots + 8) << (7 * r);
      else z1 |= (uint32_t)(r * kSlots + 8) << (7 * (r - 4));
    }
    T.ex[0] = 256;
    T.nt[0] = a.rows;
    T.tok[0] = t0;
    T.sl0[0] = z0;
    T.sl1[0] = z1;
    T.units = 1 + (int)__popcll(firsts);
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}
}  // namespace moe
