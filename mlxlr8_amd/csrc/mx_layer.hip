// Fused joined-MXFP4 MoE block for one decode token on gfx950: router, shared expert, the eight
// routed experts and the weighted combine in ONE persistent launch.
//
// Reference semantics (paths relative to the reference root):
//   router   logits = f32(x) @ W^T, sigmoid, bias-corrected top-8   exlr8/model.py:111-132,
//                                                                    exlr8/metal/fast_router.metal:1-42
//   xh = H128(x * unit), shared by all slots                         exlr8/joined_mxfp4.py:96
//   gu = xh @ W_gate_up[e]^T (MXFP4, group 32 along K)               exlr8/joined_mxfp4.py:106-113
//   hidden = H128(swiglu_T(H(g)*og, H(u)*ou) * in_down)             exlr8/metal/joined_gate_finish.metal
//   v = hidden @ W_down[e]^T                                          exlr8/joined_mxfp4.py:121-130
//   finish: T(H128(v) * out_down), routed sum, shared, residual      exlr8/metal/fast_decode_finish_fused.metal
//
// MI355X design.
//   * Workers: one block of kMW waves per CU, every block resident at once (the launch checks
//     that one block fits a CU and launches one per CU).  Every weight row of the layer costs the
//     same bytes, so each wave owns a fixed share of every phase: no queue, no claims.
//   * Slots: a wave streams its weights as a sequence of 3 KB slots through one ring of kRing
//     slots held in registers.  A gate/up slot is one row (3 x 1 KB of e2m1 codes, 3 x 64 B of
//     e8m0 scales); a down slot is three consecutive rows (1 KB and 64 B each): the same 16 B and
//     1 B lane loads at the same offsets.  The wave's sequence is
//         [shared gate/up rows] [routed gate/up rows, unit 1 .. 8] [shared down slots]
//         [routed down slots, in unit order]
//     and loads run kRing slots ahead across the phase borders.  A row's arithmetic is that of the
//     three-launch path (mxfp4.hip): the same lane layout and order, so the same bits.
//   * Routing: waves first compute router items (partial logits over 1024-input slices), stage
//     xh in LDS and meet once; the block's first wave past that point routes the token into the
//     block's LDS plan while the others wait for it, the shared expert's first rows in flight.
//   * Hand-over by tagged words (value, launch tag): gate/up row results, down inputs, down row
//     results.  A consumer reloads until every word it needs is current; no wave waits for its
//     own stores, so the load ring never drains for a hand-over.
//   * Gate finish GF(u, c) (down inputs 128c .. 128c + 127 of unit u) is done by one designated
//     wave once its own rows of unit u + 1 are done, when the rows it reads are normally complete.
//     The combine of output block c (the down finish of all nine slots, their weighted sum, the
//     residual) is done by a designated wave after its own down slots.
//   * Progress: a wave waits only for results of earlier phases (router items before routing,
//     rows of unit u before GF(u, .), gate finishes before down slots, down slots before a
//     combine), all produced by waves that never wait for later ones; waits are bounded (an
//     exhausted wait sets the workspace's error word).
#include <hip/hip_runtime.h>

#include <mutex>

#include "layer_sync.h"
#include "moe_device.h"
#include "moe_host.h"

namespace moe {
namespace {

constexpr int kMW = 8;                  // waves per block
constexpr int kRing = 4;                // weight slots in flight per wave
constexpr int kH = 6144, kM = 2048;     // hidden, intermediate
constexpr int kGuRows = 2 * kM;         // gate rows [0, m), up rows [m, 2m)
constexpr int kDnSlots = kH / 3;        // down slots (three rows) per unit
constexpr int kRouted = 8;              // routed units; unit 0 is the shared expert
constexpr int kUnits = kRouted + 1;
constexpr int kGfPerUnit = kM / 128;    // gate finishes per unit
constexpr int kGfs = kUnits * kGfPerUnit;
constexpr int kCombines = kH / 128;     // output blocks
constexpr int kS = kH / kRouterSlice;   // router slices per expert
constexpr int kSharedExpert = 256;
static_assert(kH % 3 == 0 && kH % kRouterSlice == 0 && kH / 2 == 3 * 1024 && kM / 2 == 1024,
              "slot layout assumes gate/up rows of 3 KB and down rows of 1 KB");

struct MxLayerWs {
  int32_t* flags;        // LayerFlag words
  uint64_t* logit_part;  // [1][kS][256] tagged partial logits
  uint64_t* gu;          // [kUnits][kGuRows] tagged gate/up row results
  float* hid;            // [kUnits][kM] down inputs: complete once hid_cnt[u] == kGfPerUnit
  int32_t* hid_cnt;      // [kUnits] gate finishes done (reset by the launch's last block)
  uint64_t* dn;          // [kUnits][kH] tagged down row results
  size_t bytes;
};

struct MxLayerArgs {
  const uint16_t* x;         // [1, h] bf16: router and expert input
  const uint16_t* residual;  // [1, h] bf16
  int rows;                  // 1
  int h;
  const float* router_w;     // [256, h] fp32
  const float* bias;         // [256] fp32
  uint32_t* ids;             // out [1, 9]
  float* scores;             // out [1, 8]
  const uint8_t* gu_codes;   // [257][2m][h/2]
  const uint8_t* gu_scales;  // [257][2m][h/32]
  const uint8_t* d_codes;    // [257][h][m/2]
  const uint8_t* d_scales;   // [257][h][m/32]
  const uint16_t* unit;      // [h] fp16 (+-1)
  const uint16_t* out_gate;  // [257][m] fp16
  const uint16_t* out_up;    // [257][m]
  const uint16_t* in_down;   // [257][m]
  const uint16_t* out_down;  // [257][h]
  uint16_t* out;             // [1, h] bf16
  int wait_polls;            // bound of a cross-wave wait (moe_set_wait_bound)
  MxLayerWs w;
};

__device__ __forceinline__ int unit_expert(const PlanLds& T, int u) {
  return u == 0 ? kSharedExpert : min(max(__builtin_amdgcn_readfirstlane(T.ex[min(u, kMaxUnits - 1)]), 0), 255);
}

// Gate finish q = u * kGfPerUnit + c: the 256 gate/up results of column block c of unit u, as the
// three-launch path's gate/up finish computes them, stored as tagged down inputs.
__device__ void mx_gate_finish(const MxLayerArgs& a, int q, uint32_t tag, const PlanLds& T) {
  const int u = q / kGfPerUnit, c = q - u * kGfPerUnit;
  const int e = unit_expert(T, u);
  const int lane = cold_lane();
  const int col = 128 * c + 2 * lane;
  const int64_t si = (int64_t)e * kM + col;
  const uint32_t og = *reinterpret_cast<const uint32_t*>(a.out_gate + si);
  const uint32_t ou = *reinterpret_cast<const uint32_t*>(a.out_up + si);
  const uint32_t idn = *reinterpret_cast<const uint32_t*>(a.in_down + si);
  // the lane's gate pair and up pair, in one round trip per attempt
  const uint64_t* gp = a.w.gu + (int64_t)u * kGuRows + col;
  uint64_t w[4];
  int spins = 0;
  for (;;) {
    w[0] = ld_tag(gp);
    w[1] = ld_tag(gp + 1);
    w[2] = ld_tag(gp + kM);
    w[3] = ld_tag(gp + kM + 1);
    if (__all(has_tag(w[0], tag) && has_tag(w[1], tag) && has_tag(w[2], tag) && has_tag(w[3], tag)) ||
        !keep_waiting<8>(a, spins))
      break;
  }
  float g0 = tag_value(w[0]), g1 = tag_value(w[1]), u0 = tag_value(w[2]), u1 = tag_value(w[3]);
  hadamard128_wave(g0, g1);
  hadamard128_wave(u0, u1);
  auto lo = [](uint32_t v) { return f16_to_f32((uint16_t)(v & 0xFFFFu)); };
  auto hi = [](uint32_t v) { return f16_to_f32((uint16_t)(v >> 16)); };
  float h0 = swiglu_bf16(g0 * lo(og), u0 * lo(ou));
  float h1 = swiglu_bf16(g1 * hi(og), u1 * hi(ou));
  h0 *= lo(idn);
  h1 *= hi(idn);
  hadamard128_wave(h0, h1);
  // the down inputs (write-through), then -- once they are acknowledged -- the unit's counter
  __hip_atomic_store(reinterpret_cast<uint64_t*>(a.w.hid + (int64_t)u * kM + col),
                     (uint64_t)__float_as_uint(h0) | ((uint64_t)__float_as_uint(h1) << 32), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_SYSTEM);
  release_stores();
  if (lane == 0) __hip_atomic_fetch_add(a.w.hid_cnt + u, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Output block nb: the down finish of every slot (H128, out scale, bf16), the routed sum in slot
// order, the shared expert and the residual -- the three-launch path's combine, term for term.
__device__ void mx_combine(const MxLayerArgs& a, int nb, uint32_t tag, const PlanLds& T) {
  const int lane = cold_lane();
  const int col = 128 * nb + 2 * lane;
  uint64_t wd[kUnits][2];
  int spins = 0;
  for (;;) {
#pragma unroll
    for (int u = 0; u < kUnits; u++) {
      wd[u][0] = ld_tag(a.w.dn + (int64_t)u * kH + col);
      wd[u][1] = ld_tag(a.w.dn + (int64_t)u * kH + col + 1);
    }
    bool ok = true;
#pragma unroll
    for (int u = 0; u < kUnits; u++) ok = ok & has_tag(wd[u][0], tag) & has_tag(wd[u][1], tag);
    if (__all(ok) || !keep_waiting<8>(a, spins)) break;
    // one word per lane (lane l: unit l mod 9) until current, then the full reload
    const uint64_t* sp = a.w.dn + (int64_t)(lane % kUnits) * kH + 128 * nb + 2 * (lane / kUnits);
    while (!__all(has_tag(ld_tag(sp), tag)) && keep_waiting<8>(a, spins)) {
    }
  }
  // slot j < 8: routed unit j + 1; slot 8: the shared expert (unit 0)
  float y0[kUnits], y1[kUnits];
#pragma unroll
  for (int j = 0; j < kUnits; j++) {
    const int u = j < kRouted ? j + 1 : 0;
    float v0 = tag_value(wd[u][0]), v1 = tag_value(wd[u][1]);
    hadamard128_wave(v0, v1);
    const int64_t si = (int64_t)unit_expert(T, u) * kH + col;
    y0[j] = round_bf16(v0 * f16_to_f32(a.out_down[si]));
    y1[j] = round_bf16(v1 * f16_to_f32(a.out_down[si + 1]));
  }
  const uint32_t res = *reinterpret_cast<const uint32_t*>(a.residual + col);
  float t0 = y0[0] * T.score[0] + 0.0f, t1 = y1[0] * T.score[0] + 0.0f;
#pragma unroll
  for (int j = 1; j < kRouted; j++) {
    const float sc = T.score[j];
    t0 = (y0[j] * sc + 0.0f) + t0;
    t1 = (y1[j] * sc + 0.0f) + t1;
  }
  const float c0 = round_bf16(round_bf16(t0) + y0[kRouted]);
  const float c1 = round_bf16(round_bf16(t1) + y1[kRouted]);
  const uint32_t pk = (uint32_t)f32_to_bf16(bf16_to_f32((uint16_t)(res & 0xFFFFu)) + c0) |
                      ((uint32_t)f32_to_bf16(bf16_to_f32((uint16_t)(res >> 16)) + c1) << 16);
  *reinterpret_cast<uint32_t*>(a.out + col) = pk;
}

// The down input of unit u (kM values) copied into the block's LDS by one wave once the unit's
// gate finishes are all done.  The counter is polled by one lane; the values are then read with
// ordinary (cached) loads: nothing in this launch reads them before they are complete, so the
// first block of an XCD brings them into its L2 and the XCD's other blocks hit there (an input is
// read by every block that has down slots of its unit).
__device__ __forceinline__ void mx_stage_down_input(const MxLayerArgs& a, int u, float* dst) {
  int spins = 0;
  while (__builtin_amdgcn_readfirstlane(ld_coh_i(a.w.hid_cnt + u)) < kGfPerUnit && keep_waiting<8>(a, spins)) {
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  const int lane = cold_lane();
  const f32x4* src = reinterpret_cast<const f32x4*>(a.w.hid + (int64_t)u * kM);
  f32x4 v[kM / 256];
#pragma unroll
  for (int j = 0; j < kM / 256; j++) v[j] = src[lane + 64 * j];
#pragma unroll
  for (int j = 0; j < kM / 256; j++) reinterpret_cast<f32x4*>(dst)[lane + 64 * j] = v[j];
}

__global__ __launch_bounds__(kMW * 64) __attribute__((amdgpu_waves_per_eu(1)))
void mx_layer_kernel(MxLayerArgs a) {
  __shared__ __attribute__((aligned(16))) float xs[kH];
  __shared__ PlanLds plan_t;
  __shared__ int32_t route_state;  // 0 not started, 1 being computed, 2 ready
  __shared__ int32_t exit_last;
  __shared__ int32_t progress[kMW];  // slots done per wave (approximate, for issue priority)
  __shared__ __attribute__((aligned(16))) float hid_lds[kUnits][kM];  // down inputs the block uses
  __shared__ int32_t hid_state[kUnits];  // 0 not staged, 1 being staged, 2 ready

  const int lane = lane_id();
  const int wv = wave_id_uniform();
  const int G = (int)gridDim.x, WG = G * kMW;
  const int gw = (int)blockIdx.x * kMW + wv;
  if (threadIdx.x == 0) route_state = 0;
  if (threadIdx.x < kMW) progress[threadIdx.x] = 0;
  if (threadIdx.x < kUnits) hid_state[threadIdx.x] = 0;

  // ---- this wave's shares of every phase
  const int g_lo = (int)((int64_t)kGuRows * gw / WG), g_hi = (int)((int64_t)kGuRows * (gw + 1) / WG);
  const int ng = g_hi - g_lo;  // gate/up rows per unit
  // Down slots, ordered by when their inputs are complete (unit u's gate finishes follow the gate/up
  // rows of unit u + 1): the waves form four groups; group p takes a contiguous share of unit p's
  // slots, then the same share of unit p + 4's, and every wave ends with its share of the last
  // unit's -- whose inputs come last -- so no wave waits long for an input.
  const int grp = (int)((int64_t)4 * gw / WG);
  const int grp0 = (int)((int64_t)WG * grp / 4), grp_n = (int)((int64_t)WG * (grp + 1) / 4) - grp0;
  const int a_lo = (int)((int64_t)kDnSlots * (gw - grp0) / grp_n);
  const int na = (int)((int64_t)kDnSlots * (gw - grp0 + 1) / grp_n) - a_lo;
  const int c_lo = (int)((int64_t)kDnSlots * gw / WG), nc = (int)((int64_t)kDnSlots * (gw + 1) / WG) - c_lo;
  const int n1 = kUnits * ng;            // gate/up slots
  const int ns = n1 + 2 * na + nc;     // + down slots
  // Gate finishes and combines go to the block's first kMW / 2 waves.  Two waves share each SIMD
  // and the arbiter favours the older one: waves 0..3 end their gate/up rows ~4 us before 4..7,
  // so a finish there waits less for the rows it sums and delays no late wave's own rows (a
  // designated wave that was also a late one had held up the last unit's down inputs).
  const int ho = kMW / 2, hw = (int)blockIdx.x * ho + wv, HW = G * ho;
  const int gf_lo = wv < ho ? (int)((int64_t)kGfs * hw / HW) : 0;
  const int gf_hi = wv < ho ? (int)((int64_t)kGfs * (hw + 1) / HW) : 0;
  const int cb_lo = wv < ho ? (int)((int64_t)kCombines * hw / HW) : 0;
  const int cb_hi = wv < ho ? (int)((int64_t)kCombines * (hw + 1) / HW) : 0;

  // slot s -> (unit, first weight row); true for a gate/up slot
  auto slot_rows = [&](int s, int& u, int& row) {
    if (s < ng) {
      u = 0;
      row = g_lo + s;
      return true;
    }
    if (s < n1) {
      // (s - ng) / ng by subtraction: a uniform loop of at most eight scalar steps (an integer
      // division would take vector registers at the ring's busiest point)
      int k = 0, t = s - ng;
      while (t >= ng) {
        t -= ng;
        k++;
      }
      u = 1 + k;
      row = g_lo + t;
      return true;
    }
    const int t = s - n1;
    if (t < 2 * na) {
      const bool late = t >= na;
      u = late ? grp + 4 : grp;
      row = 3 * (a_lo + t - (late ? na : 0));
    } else {
      u = kRouted;
      row = 3 * (c_lo + t - 2 * na);
    }
    return false;
  };
  // the ring: loads of slot s into position j (slots past the wave's last re-read one small
  // region every wave reads, so they cost no HBM bytes; every load is unconditional)
  static_assert((uint64_t)(kSharedExpert + 1) * kGuRows * (kH / 2) < (1ull << 32) &&
                    (uint64_t)(kSharedExpert + 1) * kH * (kM / 2) < (1ull << 32),
                "weight offsets fit 32 bits");
  u32x4 wr[kRing][3];
  uint32_t sr[kRing][3];
  auto issue = [&](int j, int s) {
    int u, row;
    const bool gu = slot_rows(min(s, ns - 1), u, row);
    // uniform 32-bit offsets (scalar arithmetic; the largest, 257 experts of gate/up rows, fits)
    const uint32_t r = (uint32_t)unit_expert(plan_t, u) * (uint32_t)(gu ? kGuRows : kH) + (uint32_t)row;
    const uint32_t coff = s < ns ? r * (uint32_t)(gu ? kH / 2 : kM / 2) : 0u;
    const uint32_t soff = s < ns ? r * (uint32_t)(gu ? kH / 32 : kM / 32) : 0u;
    const uint8_t* cp = (gu ? a.gu_codes : a.d_codes) + coff;
    const uint8_t* sp = (gu ? a.gu_scales : a.d_scales) + soff;
#pragma unroll
    for (int i = 0; i < 3; i++) {
      wr[j][i] = load_stream16(cp + 1024 * i + 16 * lane);
      sr[j][i] = sp[64 * i + lane];
    }
  };

  // Issue priority from progress: the SIMD arbiter favours older waves, so without this the
  // block's first waves finish their rows well before its last ones, whose late rows then hold up
  // the gate finishes (and everything after them) of the last unit.  A wave behind its block's
  // mean runs at raised priority.
  auto balance = [&](int done) {
    if (lane == 0) __hip_atomic_store(&progress[wv], done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    int sum = 0;
#pragma unroll
    for (int k = 0; k < kMW; k++) sum += __hip_atomic_load(&progress[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (__builtin_amdgcn_readfirstlane(sum) > done * kMW)
      __builtin_amdgcn_s_setprio(1);
    else
      __builtin_amdgcn_s_setprio(0);
  };

  // ---- prologue: the launch tag, x, router items (their loads first: loads complete in order,
  // and routing gates everything else), then the shared expert's first slots
  const uint32_t epoch = (uint32_t)__builtin_amdgcn_readfirstlane(ld_coh_i(a.w.flags + LF_EPOCH));
  const uint32_t tag = epoch + 1u;
  constexpr int kPer = kH / 128 / kMW;
  static_assert(kPer * 128 * kMW == kH, "whole 128-blocks per wave");
  uint32_t xv[kPer], uv[kPer];
#pragma unroll
  for (int i = 0; i < kPer; i++) {
    const int c = (wv + i * kMW) * 128 + 2 * lane;
    xv[i] = *reinterpret_cast<const uint32_t*>(a.x + c);
    uv[i] = *reinterpret_cast<const uint32_t*>(a.unit + c);
  }
  __builtin_amdgcn_s_setprio(3);
  for (int r = wv * G + (int)blockIdx.x; r < 256 * kS; r += WG) router_item(a, r, kS, tag);
  if (ns > 0) {
#pragma unroll
    for (int j = 0; j < kRing; j++)
      if (j < ng) issue(j, j);
  }
  // xh = H128(x * unit) into LDS
#pragma unroll
  for (int i = 0; i < kPer; i++) {
    const int c = (wv + i * kMW) * 128 + 2 * lane;
    float v0 = bf16_to_f32((uint16_t)(xv[i] & 0xFFFFu)) * f16_to_f32((uint16_t)(uv[i] & 0xFFFFu));
    float v1 = bf16_to_f32((uint16_t)(xv[i] >> 16)) * f16_to_f32((uint16_t)(uv[i] >> 16));
    hadamard128_wave(v0, v1);
    *reinterpret_cast<f32x2*>(xs + c) = f32x2{v0, v1};
  }
  __syncthreads();

  // ---- the block's plan: the first wave here routes, the others wait for it
  {
    int old = 0;
    if (lane == 0) {
      int expected = 0;
      __hip_atomic_compare_exchange_strong(&route_state, &expected, 1, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_WORKGROUP);
      old = expected;
    }
    if (__builtin_amdgcn_readfirstlane(old) == 0) {
      route_block(a, kS, tag, plan_t);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
      if (lane == 0) __hip_atomic_store(&route_state, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    } else {
      while (__hip_atomic_load(&route_state, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) != 2)
        __builtin_amdgcn_s_sleep(1);
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    }
  }
  __builtin_amdgcn_s_setprio(0);
  if (ns > 0) {
#pragma unroll
    for (int j = 0; j < kRing; j++)
      if (j >= ng) issue(j, j);
  }

  // xh as the wave uses it: k = 2048 i + 32 lane + j in registers (read after routing, which
  // needs the registers)
  float xg[96];
#pragma unroll
  for (int i = 0; i < 3; i++)
#pragma unroll
    for (int jj = 0; jj < 8; jj++) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(xs + 2048 * i + 32 * lane + 4 * jj);
      xg[32 * i + 4 * jj] = v.x;
      xg[32 * i + 4 * jj + 1] = v.y;
      xg[32 * i + 4 * jj + 2] = v.z;
      xg[32 * i + 4 * jj + 3] = v.w;
    }

  // ---- gate/up slots; the designated gate finishes follow the wave's rows of the next unit
  int gf = gf_lo;
  for (int rb = 0; rb < n1; rb += kRing) {
#pragma unroll
    for (int j = 0; j < kRing; j++) {
      const int s = rb + j;
      if (s >= n1) break;
      int u, row;
      slot_rows(s, u, row);
      float acc = 0.0f;
#pragma unroll
      for (int i = 0; i < 3; i++) {
        const u32x4 w = wr[j][i];
        const float sc = e8m0_to_f32(sr[j][i]);
        acc = dot8_fp4(w.x, sc, xg + 32 * i, acc);
        acc = dot8_fp4(w.y, sc, xg + 32 * i + 8, acc);
        acc = dot8_fp4(w.z, sc, xg + 32 * i + 16, acc);
        acc = dot8_fp4(w.w, sc, xg + 32 * i + 24, acc);
      }
      issue(j, s + kRing);
      acc = wave_sum(acc);
      const float tot = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, acc), 63));
      if (lane == 0) st_tag(a.w.gu + (int64_t)u * kGuRows + row, tot, tag);
    }
    while (gf < gf_hi && rb + kRing >= (gf / kGfPerUnit + 2) * ng) {
      __builtin_amdgcn_s_setprio(3);
      mx_gate_finish(a, gf, tag, plan_t);
      gf++;
    }
    balance(rb + kRing);
  }
  for (; gf < gf_hi; gf++) {
    __builtin_amdgcn_s_setprio(3);
    mx_gate_finish(a, gf, tag, plan_t);
    __builtin_amdgcn_s_setprio(0);
  }

  // ---- down slots (three rows each); the down input is reloaded when the unit changes
  float xd[32];
  int cur = -1;
  for (int rb = n1 - n1 % kRing; rb < ns; rb += kRing) {
#pragma unroll
    for (int j = 0; j < kRing; j++) {
      const int s = rb + j;
      if (s < n1) continue;
      if (s >= ns) break;
      int u, row;
      slot_rows(s, u, row);
      if (u != cur) {
        // the unit's input: staged into LDS by the block's first wave to need it
        cur = u;
        const int k = min(max(u, 0), kUnits - 1);
        int old = 0;
        if (lane == 0) {
          int expected = 0;
          __hip_atomic_compare_exchange_strong(&hid_state[k], &expected, 1, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_WORKGROUP);
          old = expected;
        }
        if (__builtin_amdgcn_readfirstlane(old) == 0) {
          __builtin_amdgcn_s_setprio(3);
          mx_stage_down_input(a, k, hid_lds[k]);
          __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
          if (lane == 0) __hip_atomic_store(&hid_state[k], 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        } else {
          while (__hip_atomic_load(&hid_state[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) != 2)
            __builtin_amdgcn_s_sleep(1);
          __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        }
        const float* src = hid_lds[k] + 32 * cold_lane();
#pragma unroll
        for (int jj = 0; jj < 8; jj++) {
          const f32x4 v = *reinterpret_cast<const f32x4*>(src + 4 * jj);
          xd[4 * jj] = v.x;
          xd[4 * jj + 1] = v.y;
          xd[4 * jj + 2] = v.z;
          xd[4 * jj + 3] = v.w;
        }
      }
      float acc[3];
#pragma unroll
      for (int i = 0; i < 3; i++) {
        const u32x4 w = wr[j][i];
        const float sc = e8m0_to_f32(sr[j][i]);
        acc[i] = dot8_fp4(w.x, sc, xd, 0.0f);
        acc[i] = dot8_fp4(w.y, sc, xd + 8, acc[i]);
        acc[i] = dot8_fp4(w.z, sc, xd + 16, acc[i]);
        acc[i] = dot8_fp4(w.w, sc, xd + 24, acc[i]);
      }
      issue(j, s + kRing);
      float t[3];
#pragma unroll
      for (int i = 0; i < 3; i++) {
        const float v = wave_sum(acc[i]);
        t[i] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
      }
      const float mine = lane == 0 ? t[0] : (lane == 1 ? t[1] : t[2]);
      if (lane < 3) st_tag(a.w.dn + (int64_t)u * kH + row + lane, mine, tag);
    }
    balance(rb + kRing);
  }

  // ---- designated combines
  for (int nb = cb_lo; nb < cb_hi; nb++) {
    __builtin_amdgcn_s_setprio(3);
    mx_combine(a, nb, tag, plan_t);
    __builtin_amdgcn_s_setprio(0);
  }

  // the last block to leave reports a stalled wait, advances the epoch and resets the counters
  const bool last = leave_launch(a, epoch, exit_last);
  if (last && threadIdx.x < kUnits) st_coh_i(a.w.hid_cnt + threadIdx.x, 0);
  if (last) release_stores();
}

size_t mx_align(size_t v) { return (v + 255) & ~(size_t)255; }

MxLayerWs mx_layer_carve(void* base) {
  MxLayerWs w{};
  size_t off = 0;
  char* p = static_cast<char*>(base);
  auto take = [&](size_t bytes) { char* r = p ? p + off : nullptr; off += mx_align(bytes); return r; };
  w.flags = reinterpret_cast<int32_t*>(take(LF_COUNT * 4));
  w.logit_part = reinterpret_cast<uint64_t*>(take((size_t)kS * 256 * 8));
  w.gu = reinterpret_cast<uint64_t*>(take((size_t)kUnits * kGuRows * 8));
  w.hid = reinterpret_cast<float*>(take((size_t)kUnits * kM * 4));
  w.hid_cnt = reinterpret_cast<int32_t*>(take((size_t)kUnits * 4));
  w.dn = reinterpret_cast<uint64_t*>(take((size_t)kUnits * kH * 8));
  w.bytes = off;
  return w;
}

std::mutex g_fit_mutex;
int g_fit[64];  // per device: 0 unknown, 1 one block per CU fits, -1 it does not

}  // namespace

size_t mx_layer_workspace_bytes() { return mx_layer_carve(nullptr).bytes; }
int32_t* mx_layer_flags(void* layer_ws) { return mx_layer_carve(layer_ws).flags; }

int mx_layer_run(const uint16_t* x, const uint16_t* residual, const float* router_w, const float* bias, uint32_t* ids,
                 float* scores, const uint8_t* gu_codes, const uint8_t* gu_scales, const uint8_t* d_codes,
                 const uint8_t* d_scales, const uint16_t* unit, const uint16_t* out_gate, const uint16_t* out_up,
                 const uint16_t* in_down, const uint16_t* out_down, uint16_t* out, void* layer_ws, hipStream_t s) {
  auto misaligned = [](const void* p) { return ((uintptr_t)p & 3) != 0; };
  if (misaligned(x) || misaligned(residual) || misaligned(out) || misaligned(unit) || misaligned(out_gate) ||
      misaligned(out_up) || misaligned(in_down) || misaligned(out_down))
    return fail(MOE_EINVAL, "the MXFP4 decode block needs x, residual, out, unit and side-vector rows 4-byte aligned");
  int dev = 0;
  MOE_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= 64) return fail(MOE_ENOTSUP, "device index %d out of range", dev);
  {
    std::lock_guard<std::mutex> lock(g_fit_mutex);
    if (g_fit[dev] == 0) {
      int n = 0;
      MOE_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, mx_layer_kernel, kMW * 64, 0));
      g_fit[dev] = n >= 1 ? 1 : -1;
    }
    if (g_fit[dev] < 0) return fail(MOE_ENOTSUP, "the fused MXFP4 decode block does not fit a compute unit");
  }
  MxLayerArgs a{};
  a.x = x;
  a.residual = residual;
  a.rows = 1;
  a.h = kH;
  a.router_w = router_w;
  a.bias = bias;
  a.ids = ids;
  a.scores = scores;
  a.gu_codes = gu_codes;
  a.gu_scales = gu_scales;
  a.d_codes = d_codes;
  a.d_scales = d_scales;
  a.unit = unit;
  a.out_gate = out_gate;
  a.out_up = out_up;
  a.in_down = in_down;
  a.out_down = out_down;
  a.out = out;
  a.w = mx_layer_carve(layer_ws);
  a.wait_polls = wait_polls();
  const int grid = device_cus();
  hipLaunchKernelGGL(mx_layer_kernel, dim3(grid), dim3(kMW * 64), 0, s, a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail((int)e, "launch of the fused MXFP4 decode block failed: %s", hipGetErrorString(e));
  return MOE_OK;
}

}  // namespace moe
