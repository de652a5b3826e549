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

// Selection of one row from its loaded logits: a radix select on 40-bit keys (choice key << 8 |
// 255 - id).  Keys are unique, so "top 8 by descending choice, ties to the lower id" is exactly
// "the 8 largest keys".  Each bisection step counts candidates with wave-wide compare masks (no
// LDS round trip); the 8 winners are then ranked against each other and the scores summed in
// rank order.  COH_OUT: ids and scores are stored write-through (read by other CUs in the same
// launch).
template <bool COH_OUT>
__device__ __forceinline__ void route_select(const RouteInput& in, int row, uint32_t* __restrict__ ids,
                                             float* __restrict__ scores, int32_t* sid, bool store_global,
                                             float* score_lds) {
  const int lane = lane_id();
  float orig[4];
  uint32_t fk[4];
  uint64_t key[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int e = lane + 64 * i;
    orig[i] = router_sigmoid(in.logit[i]);
    const float choice = orig[i] + in.bias[i];
    fk[i] = float_key(choice);
    key[i] = ((uint64_t)fk[i] << 8) | (uint64_t)(255 - e);
  }
  // Bisection on the choice keys alone first (32-bit compares), each compare into its own mask so
  // the four compares of a step overlap: th = the 8th largest choice key.  Only when more than 8
  // keys reach th (a tie at the boundary) do the 8 id bits continue the bisection on full keys.
  uint32_t th = 0;
  for (int b = 31; b >= 0; b--) {
    const uint32_t cand = th | (1u << b);
    uint64_t m[4];
#pragma unroll
    for (int i = 0; i < 4; i++) m[i] = __builtin_amdgcn_uicmp(fk[i], cand, 35 /* unsigned >= */);
    int cnt = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) cnt += __popcll(m[i]);
    if (cnt >= 8) th = cand;
  }
  uint64_t thr = (uint64_t)th << 8;
  {
    int at = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) at += __popcll(__builtin_amdgcn_uicmp(fk[i], th, 35));
    if (at > 8) {
      for (int b = 7; b >= 0; b--) {
        const uint64_t cand = thr | (1ull << b);
        uint64_t m[4];
#pragma unroll
        for (int i = 0; i < 4; i++) m[i] = __builtin_amdgcn_uicmpl(key[i], cand, 35);
        int cnt = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) cnt += __popcll(m[i]);
        if (cnt >= 8) thr = cand;
      }
    }
  }
  // exactly 8 keys are >= thr.  The winners are packed into 8 LDS entries (position = winners in
  // earlier slots and lower lanes); lane l < 8 then ranks entry l against the other seven
  // (descending, keys are unique) and places its sigmoid score and id at that rank.
  __shared__ uint64_t wkey_lds[kMaxRows][8];
  __shared__ float worig_lds[kMaxRows][8];
  __shared__ float sel_lds[kMaxRows][8];
  __shared__ int id_lds[kMaxRows][8];
  const int rs = row & (kMaxRows - 1);
  uint64_t* wk = wkey_lds[rs];
  float* wo = worig_lds[rs];
  float* sel = sel_lds[rs];
  int* idl = id_lds[rs];
  int before = 0;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const uint64_t m = __ballot(key[i] >= thr);
    const int pos = before + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                                            __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
    if (key[i] >= thr) {
      wk[pos] = key[i];
      wo[pos] = orig[i];
    }
    before += __popcll(m);
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  if (lane < 8) {
    const uint64_t mine = wk[lane];
    int rank = 0;
#pragma unroll
    for (int j = 0; j < 8; j++) rank += wk[j] > mine ? 1 : 0;
    sel[rank] = wo[lane];
    idl[rank] = 255 - (int)(mine & 0xFFu);
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  if ((store_global || score_lds != nullptr) && lane < 9) {
    // every lane forms the same rank-ordered sum; lane i < 8 writes winner i, lane 8 the shared id
    float total = 1e-20f;
#pragma unroll
    for (int i = 0; i < 8; i++) total += sel[i];
    const float score = lane < 8 ? sel[lane] / total * 2.5f : 0.0f;
    const uint32_t id = lane < 8 ? (uint32_t)idl[lane] : 256u;
    if (score_lds != nullptr && lane < 8) score_lds[row * 8 + lane] = score;
    if (store_global) {
      if (COH_OUT) {
        if (lane < 8)
          __hip_atomic_store(scores + (int64_t)row * 8 + lane, score, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        __hip_atomic_store(ids + (int64_t)row * 9 + lane, id, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      } else {
        if (lane < 8) scores[(int64_t)row * 8 + lane] = score;
        ids[(int64_t)row * 9 + lane] = id;
      }
    }
  }
  if (sid != nullptr && lane < 9) sid[row * 9 + lane] = lane < 8 ? idl[lane] : 256;
}

}  // namespace moe
