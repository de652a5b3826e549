// Bias-corrected top-8 routing of one token row by one wave (device code shared by the router
// kernel and the expert kernels that route in their prologue).
//
// Reference semantics (paths relative to the reference root):
//   s = v < 0 ? y : 1 - y, y = 1 / (1 + exp(|v|))        exlr8/metal/fast_router.metal:7-9
//   top-8 of s + bias, descending, ties -> lower id      exlr8/metal/fast_router.metal:13-34
//   score = s / (1e-20 + sum s_sel) * 2.5, slot 8 = 256  exlr8/metal/fast_router.metal:35-42
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "moe_device.h"
#include "moe_plan.h"

namespace moe {

__device__ __forceinline__ float router_sigmoid(float v) {
  const float y = 1.0f / (1.0f + expf(fabsf(v)));
  return v < 0.0f ? y : 1.0f - y;
}

// Order-preserving map of a float onto an unsigned key (larger float -> larger key).
__device__ __forceinline__ uint32_t float_key(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// One wave per row.  Lane l owns experts l, l+64, l+128, l+192.  COHERENT reads logits that
// other blocks of the same launch wrote (L2-bypassing loads).
//
// The row's logits and the bias as lane l holds them, loaded ahead of the selection so a caller
// can overlap the round trip with other work.
struct RouteInput {
  float logit[4], bias[4];
};
template <bool COHERENT = false>
__device__ __forceinline__ RouteInput route_load(const float* __restrict__ logits, const float* __restrict__ bias,
                                                 int row) {
  const int lane = lane_id();
  RouteInput in;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int e = lane + 64 * i;
    const float* lp = logits + (int64_t)row * 256 + e;
    in.logit[i] = COHERENT ? __hip_atomic_load(const_cast<float*>(lp), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM)
                           : *lp;
    in.bias[i] = bias[e];
  }
  return in;
}

template <bool COH_OUT = false>
__device__ __forceinline__ void route_select(const RouteInput& in, int row, uint32_t* __restrict__ ids,
                                             float* __restrict__ scores, int32_t* sid, bool store_global,
                                             float* score_lds = nullptr);

template <bool COHERENT = false>
__device__ __forceinline__ void route_row(const float* __restrict__ logits, const float* __restrict__ bias, int row,
                                          uint32_t* __restrict__ ids, float* __restrict__ scores,
                                          int32_t* sid = nullptr, bool store_global = true) {
  route_select(route_load<COHERENT>(logits, bias, row), row, ids, scores, sid, store_global);
}

// Largest value over the wave's lanes (valid in lane 63): the DPP steps of wave_sum with max.
// Lanes a broadcast step does not reach keep their value (max with 0, the unsigned identity).
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROW_MASK, 0xF, false);
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, dpp_u32<0xB1>(v));        // quad_perm [1,0,3,2]
  v = max(v, dpp_u32<0x4E>(v));        // quad_perm [2,3,0,1]
  v = max(v, dpp_u32<0x124>(v));       // row_ror:4
  v = max(v, dpp_u32<0x128>(v));       // row_ror:8
  v = max(v, dpp_u32<0x142, 0xA>(v));  // row_bcast:15 into rows 1 and 3
  v = max(v, dpp_u32<0x143, 0xC>(v));  // row_bcast:31 into rows 2 and 3
  return v;
}

// Selection of one row from its loaded logits.  The order is "descending choice, ties to the lower
// id" (a total order on (choice key, id)).  Each lane sorts its four candidates; then eight rounds
// each take the wave's largest head: a DPP max over the heads' choice keys, the owner lane found by
// ballot (a tie between lanes' heads -- equal choice keys -- goes to the lower id through a second
// max over the tied lanes' inverted ids), and the owner pops its head.  The winners come out in
// rank order, their sigmoid values and ids handed over by lane reads; the scores are summed in
// rank order.  COH_OUT: ids and scores are stored write-through (read by other CUs in the same
// launch).
template <bool COH_OUT>
__device__ __forceinline__ void route_select(const RouteInput& in, int row, uint32_t* __restrict__ ids,
                                             float* __restrict__ scores, int32_t* sid, bool store_global,
                                             float* score_lds) {
  const int lane = lane_id();
  float orig[4];
  uint32_t fk[4], id[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    id[i] = (uint32_t)(lane + 64 * i);
    orig[i] = router_sigmoid(in.logit[i]);
    fk[i] = float_key(orig[i] + in.bias[i]);
  }
  // the lane's candidates in descending order (a five-exchange network; ids are already ascending
  // within a lane, so "a before b" is fk[a] > fk[b] or equal keys with the lower id first)
  auto order = [&](int a, int b) {
    const bool swap = fk[b] > fk[a] || (fk[b] == fk[a] && id[b] < id[a]);
    const uint32_t tk = fk[a], ti = id[a];
    const float to = orig[a];
    fk[a] = swap ? fk[b] : fk[a];
    id[a] = swap ? id[b] : id[a];
    orig[a] = swap ? orig[b] : orig[a];
    fk[b] = swap ? tk : fk[b];
    id[b] = swap ? ti : id[b];
    orig[b] = swap ? to : orig[b];
  };
  order(0, 1);
  order(2, 3);
  order(0, 2);
  order(1, 3);
  order(1, 2);
  float sel[8];
  uint32_t win[8];
  uint32_t live = 4;  // candidates left in this lane (popped heads are replaced from the back)
#pragma unroll
  for (int r = 0; r < 8; r++) {
    const uint32_t head = live > 0 ? fk[0] : 0u;
    const uint32_t top = (uint32_t)__builtin_amdgcn_readlane((int)wave_max_u32(head), 63);
    const bool mine = live > 0 && head == top;
    uint64_t owners = __ballot(mine);
    if (__popcll(owners) > 1) {
      // equal choice keys in several lanes: the lowest id among them
      const uint32_t low = ~(uint32_t)__builtin_amdgcn_readlane((int)wave_max_u32(mine ? ~id[0] : 0u), 63);
      owners = __ballot(mine && id[0] == low);
    }
    const int owner = (int)__builtin_ctzll(owners);
    sel[r] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, orig[0]), owner));
    win[r] = (uint32_t)__builtin_amdgcn_readlane((int)id[0], owner);
    if (lane == owner) {
      fk[0] = fk[1];
      id[0] = id[1];
      orig[0] = orig[1];
      fk[1] = fk[2];
      id[1] = id[2];
      orig[1] = orig[2];
      fk[2] = fk[3];
      id[2] = id[3];
      orig[2] = orig[3];
      live--;
    }
  }
  if ((store_global || score_lds != nullptr) && lane < 9) {
    // every lane forms the same rank-ordered sum; lane i < 8 writes winner i, lane 8 the shared id
    float total = 1e-20f;
#pragma unroll
    for (int i = 0; i < 8; i++) total += sel[i];
    float mine = sel[0];
    uint32_t mid = win[0];
#pragma unroll
    for (int i = 1; i < 8; i++) {
      mine = lane == i ? sel[i] : mine;
      mid = lane == i ? win[i] : mid;
    }
    const float score = lane < 8 ? mine / total * 2.5f : 0.0f;
    const uint32_t idv = lane < 8 ? mid : 256u;
    if (score_lds != nullptr && lane < 8) score_lds[row * 8 + lane] = score;
    if (store_global) {
      if (COH_OUT) {
        if (lane < 8)
          __hip_atomic_store(scores + (int64_t)row * 8 + lane, score, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        __hip_atomic_store(ids + (int64_t)row * 9 + lane, idv, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      } else {
        if (lane < 8) scores[(int64_t)row * 8 + lane] = score;
        ids[(int64_t)row * 9 + lane] = idv;
      }
    }
  }
  if (sid != nullptr && lane < 9) {
    uint32_t mid = win[0];
#pragma unroll
    for (int i = 1; i < 8; i++) mid = lane == i ? win[i] : mid;
    sid[row * 9 + lane] = lane < 8 ? (int)mid : 256;
  }
}

}  // namespace moe
