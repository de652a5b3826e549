// Token -> expert dispatch plan for decode-sized batches (up to 8 token rows, 9 slots each).
//
// The reference appends the shared expert (id 256) to the routed top-8 (exlr8/model.py:407-408)
// and, for 2-4 rows, de-duplicates repeated experts so each expert's weights are read once
// (REUSE_ROWS in exlr8/metal/fast_decode_linear.metal:36-61).  Here every distinct expert of
// the batch becomes one "unit" that carries the list of token rows that selected it; the
// GEMV kernels stream each unit's weights once and apply them to all of its rows.
#pragma once
#include <stdint.h>

namespace moe {

constexpr int kMaxRows = 8;             // token rows per plan
constexpr int kSlots = 9;               // 8 routed + 1 shared
constexpr int kMaxUnits = kMaxRows * kSlots;

struct Plan {
  int32_t units;                        // number of distinct experts U
  int32_t rows;                         // token rows
  int32_t pad[2];
  int32_t expert[kMaxUnits];            // expert id of unit u
  int32_t ntok[kMaxUnits];              // rows that use unit u
  int32_t tok[kMaxUnits][kMaxRows];     // row index of the i-th user of unit u
  int32_t slot[kMaxUnits][kMaxRows];    // slot index row*9 + j of the i-th user of unit u
  int32_t slot_unit[kMaxUnits];         // unit of slot s
  int32_t slot_pos[kMaxUnits];          // position of slot s inside its unit's row list
};

// Build the plan from indices [rows, slots] in first-appearance order (serial; <= 72 slots).
// A unit holds at most `max_users` rows; further users of the same expert open a new unit,
// so the kernels' per-unit row arrays never overflow.  Ids outside 0..experts-1 are clamped
// to keep every weight access in bounds (callers validate ids beforehand).
// `unit_of_expert` (257 entries) must hold -1 on entry (see build_plan below).
__device__ inline void build_plan_serial(const uint32_t* idx, int rows, int slots, int experts, int max_users,
                                         Plan* plan, int32_t* unit_of_expert) {
  int units = 0;
  for (int s = 0; s < rows * slots; s++) {
    int e = (int)idx[s];
    if (e < 0) e = 0;
    if (e >= experts) e = experts - 1;
    if (e > 256) e = 256;
    int u = unit_of_expert[e];
    if (u < 0 || plan->ntok[u] >= max_users) {
      u = units++;
      unit_of_expert[e] = u;
      plan->expert[u] = e;
      plan->ntok[u] = 0;
    }
    int i = plan->ntok[u]++;
    plan->tok[u][i] = s / slots;
    plan->slot[u][i] = s;
    plan->slot_unit[s] = u;
    plan->slot_pos[s] = i;
  }
  plan->units = units;
  plan->rows = rows;
}

__device__ inline void build_plan(const uint32_t* idx, int rows, int slots, int experts, int max_users, Plan* plan,
                                  int32_t* unit_of_expert /* 257 */) {
  for (int e = 0; e < 257; e++) unit_of_expert[e] = -1;
  build_plan_serial(idx, rows, slots, experts, max_users, plan, unit_of_expert);
}

// Parallel plan build by one block (blockDim >= rows*slots, ids already in LDS `sid`), same result
// as build_plan: units in order of first appearance, each expert's users split into consecutive
// groups of `max_users`.  Pass 1: each slot finds its position among its expert's users and the
// slot that opens its group; pass 2: its unit is the number of group-opening slots before that.
// `open` is LDS scratch of kMaxUnits entries.  Every thread of the block must call this.
__device__ inline void build_plan_parallel(const int32_t* sid, int rows, int slots, int max_users, Plan* plan,
                                           int32_t* open) {
  const int n = rows * slots;
  const int s = threadIdx.x;
  int pos = 0, start = s, total = 0, e = 0;
  // no early exits: the LDS reads of the loops are independent and issue back to back
  if (s < n) {
    e = sid[s];
#pragma unroll 4
    for (int q = 0; q < n; q++) {
      const int m = sid[q] == e ? 1 : 0;
      pos += q < s ? m : 0;
      total += m;
    }
    const int want = (pos / max_users) * max_users;
    int seen = 0;
#pragma unroll 4
    for (int q = 0; q <= s; q++) {
      const int m = sid[q] == e ? 1 : 0;
      if (m && seen == want) start = q;
      seen += m;
    }
    open[s] = (pos % max_users) == 0;
  }
  __syncthreads();
  if (s < n) {
    int unit = 0;
#pragma unroll 4
    for (int q = 0; q < start; q++) unit += open[q];
    const int i = pos % max_users;
    if (i == 0) {
      plan->expert[unit] = e;
      const int left = total - pos;
      plan->ntok[unit] = left < max_users ? left : max_users;
    }
    plan->tok[unit][i] = s / slots;
    plan->slot[unit][i] = s;
    plan->slot_unit[s] = unit;
    plan->slot_pos[s] = i;
    if (s == 0) {
      int units = 0;
      for (int q = 0; q < n; q++) units += open[q];
      plan->units = units;
      plan->rows = rows;
    }
  }
}

}  // namespace moe
