// Resident joined-MXFP4 expert path on gfx950 (decode batches).
//
// Reference semantics (paths relative to the reference root):
//   xh = H128(x * unit), shared by all slots                  exlr8/joined_mxfp4.py:96
//   gu = xh @ W_gate_up[e]^T (MXFP4, group 32 along K)          exlr8/joined_mxfp4.py:106-113
//   hidden = H128(swiglu_T(H(g)*og, H(u)*ou) * in_down)        exlr8/metal/joined_gate_finish.metal
//   v = hidden @ W_down[e]^T                                     exlr8/joined_mxfp4.py:121-130
//   finish: T(H128(v) * out_down), routed sum, shared, residual exlr8/metal/fast_decode_finish_fused.metal
//   e2m1 codes, low nibble = even k; e8m0 scale 2^(s-127)        exlr8/metal/joined_gather_order*.metal
//
// MI355X design: HBM-bound GEMV.  Each wave owns a contiguous range of output rows; a lane holds
// the activations of its fixed K positions in VGPRs (K/64 floats), streams 16 B of codes per
// 32-wide group with coalesced dwordx4 loads, converts 2 codes per instruction with the hardware
// scaled FP4->f32 conversion (the e8m0 scale folded in, exact), and the row sum is one DPP
// reduction.  Completion counters hand 128-row blocks to the gate finish / combine, as in the
// K4 path.
#include <hip/hip_runtime.h>

#include <mutex>

#include "moe_device.h"
#include "moe_host.h"
#include "moe_plan.h"

namespace moe {

constexpr int kMxWaves = 8;
constexpr int kMxThreads = kMxWaves * 64;

enum MxMode { MX_GATEUP = 0, MX_DOWN_COMBINE = 1, MX_DOWN_VALUES = 2 };

struct MxArgs {
  const uint8_t* codes;        // [E][N][K/2]
  const uint8_t* scales;       // [E][N][K/32]
  int K, N;                    // input features, output rows per expert
  const uint32_t* ids;         // [slots] expert id per slot (row-major [rows, slots_per_row])
  int slots, slots_per_row;
  int experts;
  const uint16_t* x_bf16;      // GATEUP: [rows, K]
  const uint16_t* unit;        // GATEUP: [K] fp16 (+-1)
  const float* x_f32;          // DOWN: [slots, K] hidden
  float* rowout;               // [slots][N] fp32 row results (write-through)
  int32_t* counter_blk;        // [slots * N/128]
  int32_t* counter_grp;        // GATEUP: [slots * (N/2)/128]; DOWN: [N/128]
  const uint16_t* out_gate;    // [E][m]
  const uint16_t* out_up;      // [E][m]
  const uint16_t* in_down;     // [E][m]
  float* hidden;               // GATEUP output [slots][m]
  const uint16_t* out_down;    // [E][h]
  const float* scores;         // [rows][8]
  const uint16_t* residual;    // [rows][h]
  uint16_t* out;               // [rows][h]
  uint16_t* values;            // [slots][h]
};

__device__ __forceinline__ void st_wt(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ f32x2 ld_wt2(const float* p) {
  const uint64_t v = __hip_atomic_load(reinterpret_cast<uint64_t*>(const_cast<float*>(p)), __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_SYSTEM);
  return f32x2{__uint_as_float((uint32_t)v), __uint_as_float((uint32_t)(v >> 32))};
}
__device__ __forceinline__ int cnt_add(int32_t* c, int v) {
  int old = 0;
  if (lane_id() == 0) old = __hip_atomic_fetch_add(c, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  return __shfl(old, 0, 64);
}
__device__ __forceinline__ void cnt_reset(int32_t* c) {
  if (lane_id() == 0) __hip_atomic_store(c, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ int slot_expert(const MxArgs& a, int s) {
  int e = (int)a.ids[s];
  if (e < 0) e = 0;
  if (e >= a.experts) e = a.experts - 1;
  return e;
}

// KC = K / 2048 (16-byte chunks per lane per row): 3 for K = 6144 (gate/up), 1 for K = 2048 (down).
// down launches (K = 2048): kept within 128 VGPRs so two 8-wave blocks share a CU, and launched
// with that many blocks per CU (more rows in flight per CU)
#ifndef MOE_MX_DOWN_BPC
#define MOE_MX_DOWN_BPC 2
#endif
template <int MODE, int KC>
__global__ __launch_bounds__(kMxThreads) __attribute__((amdgpu_waves_per_eu(KC == 1 && MOE_MX_DOWN_BPC > 1 ? 4 : 1)))
void mx_gemv_kernel(MxArgs a) {
  __shared__ __attribute__((aligned(16))) float xs[2][KC * 2048];
  const int K = KC * 2048;
  const int N = a.N;
  const int64_t total = (int64_t)a.slots * N;
  const int G = gridDim.x;
  const int64_t r0 = total * blockIdx.x / G, r1 = total * (blockIdx.x + 1) / G;
  if (r0 >= r1) return;
  const int s0 = (int)(r0 / N);
  const int s1 = (int)((r1 - 1) / N);  // s1 <= s0 + 1 (host guarantees rows per block <= N)
  const int lane = lane_id(), wv = wave_id_in_block();
  // this wave's rows (row indices fit 32 bits: at most 72 slots x 6144 rows)
  const int w0 = (int)(r0 + (r1 - r0) * wv / kMxWaves), w1 = (int)(r0 + (r1 - r0) * (wv + 1) / kMxWaves);

  // Weight rows are streamed through a ring of D rows per wave (issued D rows ahead, so D row
  // loads are in flight while a row is reduced); the first D are issued before the activations
  // are staged.  Loads past the range re-read its last row, so the ring needs no branch.
  constexpr int D = KC == 3 ? 2 : 6;
  u32x4 wr[D][KC];
  uint32_t sr[D][KC];
  // experts of the block's (at most two) slots, read once (no scalar-load round trip per row)
  const int e_s0 = slot_expert(a, s0), e_s1 = slot_expert(a, s1);
  auto expert_of = [&](int s) { return s == s0 ? e_s0 : e_s1; };
  auto issue = [&](int j, int r) {
    const int rr = min(r, w1 - 1);
    const int s = rr / N, n = rr - s * N;
    const int e = expert_of(s);
    const uint8_t* crow = a.codes + ((int64_t)e * N + n) * (K / 2);
    const uint8_t* srow = a.scales + ((int64_t)e * N + n) * (K / 32);
#pragma unroll
    for (int i = 0; i < KC; i++) {
      wr[j][i] = load_stream16(crow + 1024 * i + 16 * lane);
      sr[j][i] = srow[64 * i + lane];
    }
  };
  if (w0 < w1) {
#pragma unroll
    for (int j = 0; j < D; j++) issue(j, w0 + j);
  }

  // ---- stage the activation rows of the (at most two) slots this block touches
  for (int q = 0; q <= s1 - s0; q++) {
    const int s = s0 + q;
    float* dst = xs[q];
    if (MODE == MX_GATEUP) {
      // H128(x_row * unit) for the slot's token row: the wave's K/128/waves blocks, all loads
      // issued before the first transform (one memory round trip)
      const int row = s / a.slots_per_row;
      constexpr int kPer = K / 128 / kMxWaves;
      static_assert(kPer * 128 * kMxWaves == K, "whole 128-blocks per wave");
      uint32_t xv[kPer], uv[kPer];
#pragma unroll
      for (int i = 0; i < kPer; i++) {
        const int c = (wv + i * kMxWaves) * 128 + 2 * lane;
        xv[i] = *reinterpret_cast<const uint32_t*>(a.x_bf16 + (int64_t)row * K + c);
        uv[i] = *reinterpret_cast<const uint32_t*>(a.unit + c);
      }
#pragma unroll
      for (int i = 0; i < kPer; i++) {
        const int c = (wv + i * kMxWaves) * 128 + 2 * lane;
        float v0 = bf16_to_f32((uint16_t)(xv[i] & 0xFFFFu)) * f16_to_f32((uint16_t)(uv[i] & 0xFFFFu));
        float v1 = bf16_to_f32((uint16_t)(xv[i] >> 16)) * f16_to_f32((uint16_t)(uv[i] >> 16));
        hadamard128_wave(v0, v1);
        *reinterpret_cast<f32x2*>(dst + c) = f32x2{v0, v1};
      }
    } else {
      for (int c = threadIdx.x * 4; c < K; c += kMxThreads * 4)
        *reinterpret_cast<f32x4*>(dst + c) = *reinterpret_cast<const f32x4*>(a.x_f32 + (int64_t)s * K + c);
    }
  }
  __syncthreads();

  float x[KC * 32];
  int cur = -1;
  int run_start = w0, buf_start = w0;
  float rbuf = 0.0f;
  for (int rb = w0; rb < w1; rb += D) {
#pragma unroll
    for (int j = 0; j < D; j++) {
      const int r = rb + j;
      if (r >= w1) break;
      const int s = r / N;
      const int n = r - s * N;
      if (s != cur) {
        cur = s;
        const float* src = xs[s - s0];
        // lane holds k = 2048*i + 32*lane + j (static register indices)
#pragma unroll
        for (int i = 0; i < KC; i++)
#pragma unroll
          for (int jj = 0; jj < 8; jj++) {
            const f32x4 v = *reinterpret_cast<const f32x4*>(src + 2048 * i + 32 * lane + 4 * jj);
            x[32 * i + 4 * jj] = v.x; x[32 * i + 4 * jj + 1] = v.y; x[32 * i + 4 * jj + 2] = v.z;
            x[32 * i + 4 * jj + 3] = v.w;
          }
      }
      const int e = expert_of(s);
      float acc = 0.0f;
#pragma unroll
      for (int i = 0; i < KC; i++) {
        const u32x4 w = wr[j][i];
        const float sc = e8m0_to_f32(sr[j][i]);
        acc = dot8_fp4(w.x, sc, x + 32 * i, acc);
        acc = dot8_fp4(w.y, sc, x + 32 * i + 8, acc);
        acc = dot8_fp4(w.z, sc, x + 32 * i + 16, acc);
        acc = dot8_fp4(w.w, sc, x + 32 * i + 24, acc);
      }
      issue(j, r + D);
      acc = wave_sum(acc);
      // row sums are gathered in one register (row r - buf_start in that lane) and stored with one
      // coalesced write-through store per 64 rows or block end: a store per row would put a
      // write acknowledgement in front of every later wait on the load ring
      const float tot = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, acc), 63));
      if (lane == r - buf_start) rbuf = tot;

      // close a run at the end of a 128-row block or of the wave's range
      const bool block_end = ((n & 127) == 127) || (r + 1 == w1);
      if (block_end || r - buf_start == 63) {
        if (lane <= r - buf_start) st_wt(a.rowout + buf_start + lane, rbuf);  // rowout index of row r is r
        buf_start = r + 1;
      }
      if (!block_end) continue;
      const int nb = n >> 7;
      const int run = r + 1 - run_start;
      run_start = r + 1;
      release_stores();
      if (MODE == MX_GATEUP) {
        // gate rows [0, m) and up rows [m, 2m): the 256 rows of column block b share one counter
        const int m = N / 2;
        const int b = nb % (m / 128);
        const int grp = s * (m / 128) + b;
        const int col = b * 128 + 2 * lane;
        const int64_t si = (int64_t)e * m + col;
        const uint32_t og = *reinterpret_cast<const uint32_t*>(a.out_gate + si);
        const uint32_t ou = *reinterpret_cast<const uint32_t*>(a.out_up + si);
        const uint32_t idn = *reinterpret_cast<const uint32_t*>(a.in_down + si);
        if (cnt_add(&a.counter_grp[grp], run) + run != 256) continue;
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        cnt_reset(&a.counter_grp[grp]);
        f32x2 g = ld_wt2(a.rowout + (int64_t)s * N + col);
        f32x2 u = ld_wt2(a.rowout + (int64_t)s * N + m + col);
        float g0 = g.x, g1 = g.y, u0 = u.x, u1 = u.y;
        hadamard128_wave(g0, g1);
        hadamard128_wave(u0, u1);
        auto lo = [](uint32_t v) { return f16_to_f32((uint16_t)(v & 0xFFFFu)); };
        auto hi = [](uint32_t v) { return f16_to_f32((uint16_t)(v >> 16)); };
        float h0 = swiglu_bf16(g0 * lo(og), u0 * lo(ou));
        float h1 = swiglu_bf16(g1 * hi(og), u1 * hi(ou));
        h0 *= lo(idn);
        h1 *= hi(idn);
        hadamard128_wave(h0, h1);
        *reinterpret_cast<f32x2*>(a.hidden + (int64_t)s * m + col) = f32x2{h0, h1};
      } else if (MODE == MX_DOWN_VALUES) {
        const int cb = s * (N / 128) + nb;
        if (cnt_add(&a.counter_blk[cb], run) + run != 128) continue;
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        cnt_reset(&a.counter_blk[cb]);
        const int col = nb * 128 + 2 * lane;
        f32x2 v = ld_wt2(a.rowout + (int64_t)s * N + col);
        float v0 = v.x, v1 = v.y;
        hadamard128_wave(v0, v1);
        const int64_t si = (int64_t)e * N + col;
        const uint32_t pk = (uint32_t)f32_to_bf16(v0 * f16_to_f32(a.out_down[si])) |
                            ((uint32_t)f32_to_bf16(v1 * f16_to_f32(a.out_down[si + 1])) << 16);
        *reinterpret_cast<uint32_t*>(a.values + (int64_t)s * N + col) = pk;
      } else {
        // per-slot bf16 value of this block, then the block's combine once every slot is done
        const int cb = s * (N / 128) + nb;
        if (cnt_add(&a.counter_blk[cb], run) + run != 128) continue;
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        cnt_reset(&a.counter_blk[cb]);
        const int col = nb * 128 + 2 * lane;
        f32x2 v = ld_wt2(a.rowout + (int64_t)s * N + col);
        float v0 = v.x, v1 = v.y;
        hadamard128_wave(v0, v1);
        const int64_t si = (int64_t)e * N + col;
        const uint64_t pk = (uint64_t)__float_as_uint(round_bf16(v0 * f16_to_f32(a.out_down[si]))) |
                            ((uint64_t)__float_as_uint(round_bf16(v1 * f16_to_f32(a.out_down[si + 1]))) << 32);
        __hip_atomic_store(reinterpret_cast<uint64_t*>(a.rowout + (int64_t)s * N + col), pk, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_SYSTEM);
        release_stores();
        if (cnt_add(&a.counter_grp[nb], 1) + 1 != a.slots) continue;
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        cnt_reset(&a.counter_grp[nb]);
        const int rows = a.slots / kSlots;
        for (int rr = 0; rr < rows; rr++) {
          f32x2 y[kSlots];
#pragma unroll
          for (int j = 0; j < kSlots; j++) y[j] = ld_wt2(a.rowout + (int64_t)(rr * kSlots + j) * N + col);
          const int64_t o = (int64_t)rr * N + col;
          const uint32_t res = *reinterpret_cast<const uint32_t*>(a.residual + o);
          float t0 = y[0].x * a.scores[rr * 8] + 0.0f, t1 = y[0].y * a.scores[rr * 8] + 0.0f;
#pragma unroll
          for (int j = 1; j < 8; j++) {
            const float sc = a.scores[rr * 8 + j];
            t0 = (y[j].x * sc + 0.0f) + t0;
            t1 = (y[j].y * sc + 0.0f) + t1;
          }
          const float c0 = round_bf16(round_bf16(t0) + y[8].x);
          const float c1 = round_bf16(round_bf16(t1) + y[8].y);
          const uint32_t pk2 = (uint32_t)f32_to_bf16(bf16_to_f32((uint16_t)(res & 0xFFFFu)) + c0) |
                               ((uint32_t)f32_to_bf16(bf16_to_f32((uint16_t)(res >> 16)) + c1) << 16);
          *reinterpret_cast<uint32_t*>(a.out + o) = pk2;
        }
      }
    }
  }
}

namespace {

size_t align_up(size_t v) { return (v + 255) & ~(size_t)255; }

struct MxWorkspace {
  int32_t* counter_blk;  // [72 * 48]
  int32_t* counter_grp;  // [72 * 16] / [48]
  float* rowout;         // [72][max(2m, h)]
  float* hidden;         // [72][m]
  Plan* plan;            // decode block: router plan (unused by the MXFP4 kernels)
  int32_t* router_counter;
  float* logits;         // [8][256]
  uint32_t* ids;         // [8][9]
  float* scores;         // [8][8]
  void* layer;           // the fused one-row decode block's region (mx_layer.hip)
  size_t bytes;
};

MxWorkspace mx_carve(void* base, int h, int m) {
  MxWorkspace w{};
  size_t off = 0;
  char* p = static_cast<char*>(base);
  auto take = [&](size_t bytes) { char* r = p ? p + off : nullptr; off += align_up(bytes); return r; };
  const int rowmax = 2 * m > h ? 2 * m : h;
  w.counter_blk = reinterpret_cast<int32_t*>(take((size_t)kMaxUnits * (rowmax / 128) * 4));
  w.counter_grp = reinterpret_cast<int32_t*>(take((size_t)kMaxUnits * (rowmax / 128) * 4));
  w.rowout = reinterpret_cast<float*>(take((size_t)kMaxUnits * rowmax * 4));
  w.hidden = reinterpret_cast<float*>(take((size_t)kMaxUnits * m * 4));
  w.plan = reinterpret_cast<Plan*>(take(sizeof(Plan)));
  w.router_counter = reinterpret_cast<int32_t*>(take(256));
  w.logits = reinterpret_cast<float*>(take((size_t)kMaxRows * 256 * 4));
  w.ids = reinterpret_cast<uint32_t*>(take((size_t)kMaxRows * kSlots * 4));
  w.scores = reinterpret_cast<float*>(take((size_t)kMaxRows * 8 * 4));
  w.layer = take(mx_layer_workspace_bytes());
  w.bytes = off;
  return w;
}

int mx_blocks(int64_t rows_total, int n) {
  int g = device_cus();
  if (g < 1) g = 1;
  if (g > 1024) g = 1024;
  // each block must span at most two slots: rows per block <= n
  const int64_t need = (rows_total + n - 1) / n;
  if (g < need) g = (int)need;
  return g;
}

// Argument checks of the MXFP4 decode MLP (no launch).
int mx_check(const uint16_t* x, const uint32_t* ids, int rows, int slots_per_row, const uint8_t* gu_codes,
             const uint8_t* gu_scales, const uint8_t* d_codes, const uint8_t* d_scales, int64_t experts,
             const uint16_t* unit, const uint16_t* out_gate, const uint16_t* out_up, const uint16_t* in_down,
             const uint16_t* out_down, int h, int m, const void* workspace, size_t workspace_bytes) {
  MOE_ARG(x && ids && gu_codes && gu_scales && d_codes && d_scales && unit && out_gate && out_up && in_down && out_down,
          "null pointer argument");
  MOE_ARG(h == 6144 && m == 2048, "this build's MXFP4 kernels are specialised for hidden 6144, intermediate 2048");
  MOE_ARG(rows >= 1 && slots_per_row >= 1 && slots_per_row <= kSlots && rows * slots_per_row <= kMaxUnits,
          "rows*slots must be in 1..%d", kMaxUnits);
  MOE_ARG(experts >= 1 && experts <= 257, "expert count must be in 1..257");
  MOE_ARG(workspace != nullptr, "workspace must not be NULL");
  const size_t need = mx_carve(nullptr, h, m).bytes;
  if (workspace_bytes < need) return fail(MOE_EWORKSPACE, "workspace too small: %zu < %zu", workspace_bytes, need);
  return MOE_OK;
}

// The MXFP4 decode MLP (gate/up GEMV + gate finish, down GEMV + values or combine) on a checked
// workspace.
int mx_launch(const uint16_t* x, const uint32_t* ids, const float* scores, const uint16_t* residual, int rows,
              int slots_per_row, const uint8_t* gu_codes, const uint8_t* gu_scales, const uint8_t* d_codes,
              const uint8_t* d_scales, int64_t experts, const uint16_t* unit, const uint16_t* out_gate,
              const uint16_t* out_up, const uint16_t* in_down, const uint16_t* out_down, int h, int m,
              uint16_t* values, uint16_t* out, void* workspace, hipStream_t s) {
  const MxWorkspace w = mx_carve(workspace, h, m);
  const int slots = rows * slots_per_row;

  MxArgs g{};
  g.codes = gu_codes; g.scales = gu_scales; g.K = h; g.N = 2 * m;
  g.ids = ids; g.slots = slots; g.slots_per_row = slots_per_row; g.experts = (int)experts;
  g.x_bf16 = x; g.unit = unit;
  g.rowout = w.rowout; g.counter_blk = w.counter_blk; g.counter_grp = w.counter_grp;
  g.out_gate = out_gate; g.out_up = out_up; g.in_down = in_down; g.hidden = w.hidden;
  hipLaunchKernelGGL((mx_gemv_kernel<MX_GATEUP, 3>), dim3(mx_blocks((int64_t)slots * 2 * m, 2 * m)), dim3(kMxThreads),
                     0, s, g);
  MOE_HIP(hipGetLastError());

  MxArgs d{};
  d.codes = d_codes; d.scales = d_scales; d.K = m; d.N = h;
  d.ids = ids; d.slots = slots; d.slots_per_row = slots_per_row; d.experts = (int)experts;
  d.x_f32 = w.hidden;
  d.rowout = w.rowout; d.counter_blk = w.counter_blk; d.counter_grp = w.counter_grp;
  d.out_down = out_down;
  const dim3 grid(mx_blocks((int64_t)slots * h, h) * MOE_MX_DOWN_BPC);
  if (out) {
    d.scores = scores; d.residual = residual; d.out = out;
    hipLaunchKernelGGL((mx_gemv_kernel<MX_DOWN_COMBINE, 1>), grid, dim3(kMxThreads), 0, s, d);
  } else {
    d.values = values;
    hipLaunchKernelGGL((mx_gemv_kernel<MX_DOWN_VALUES, 1>), grid, dim3(kMxThreads), 0, s, d);
  }
  MOE_HIP(hipGetLastError());
  return MOE_OK;
}

int mx_common(const uint16_t* x, const uint32_t* ids, const float* scores, const uint16_t* residual, int rows,
              int slots_per_row, const uint8_t* gu_codes, const uint8_t* gu_scales, const uint8_t* d_codes,
              const uint8_t* d_scales, int64_t experts, const uint16_t* unit, const uint16_t* out_gate,
              const uint16_t* out_up, const uint16_t* in_down, const uint16_t* out_down, int h, int m,
              uint16_t* values, uint16_t* out, void* workspace, size_t workspace_bytes, hipStream_t s) {
  int rc = mx_check(x, ids, rows, slots_per_row, gu_codes, gu_scales, d_codes, d_scales, experts, unit, out_gate,
                    out_up, in_down, out_down, h, m, workspace, workspace_bytes);
  if (rc) return rc;
  if (out) MOE_ARG(slots_per_row == kSlots && scores && residual, "the combined finish needs 9 slots, scores and residual");
  if ((rc = ensure_device_ready())) return rc;
  return mx_launch(x, ids, scores, residual, rows, slots_per_row, gu_codes, gu_scales, d_codes, d_scales, experts, unit,
                   out_gate, out_up, in_down, out_down, h, m, values, out, workspace, s);
}

// Zero two word ranges (counter regions) with one block.
__global__ __launch_bounds__(256) void zero_counters_kernel(int32_t* a, int na, int32_t* b, int nb) {
  for (int i = threadIdx.x; i < na; i += 256) a[i] = 0;
  for (int i = threadIdx.x; i < nb; i += 256) b[i] = 0;
}

}  // namespace
}  // namespace moe

// ---------------------------------------------------------------- allocation-free decode block
// moe_mxfp4_moe_decode_noalloc keeps its workspace in this fixed device array (one copy per GPU,
// held until the process ends).  Host code never passes the array's name to a kernel: the
// per-device address comes from hipGetSymbolAddress on the entry point's first call on a device.
constexpr size_t kScratchBytes = (size_t)4 << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace moe {
namespace {
std::mutex g_scratch_mutex;
void* g_scratch_addr[64];  // per device

int scratch_address(void** out) {
  int dev = 0;
  MOE_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= 64) return fail(MOE_ENOTSUP, "device index %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_addr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(e != hipSuccess ? (int)e : MOE_ENOTSUP, "hipGetSymbolAddress(scratch) failed: %s",
                  hipGetErrorString(e));
    g_scratch_addr[dev] = p;
  }
  *out = g_scratch_addr[dev];
  return MOE_OK;
}
}  // namespace

int32_t* mx_workspace_flags(void* workspace, int h, int m) {
  return mx_layer_flags(mx_carve(workspace, h > 0 ? h : 1, m > 0 ? m : 1).layer);
}
int mx_scratch_flags(int32_t** flags) {
  void* ws = nullptr;
  if (int rc = scratch_address(&ws)) return rc;
  *flags = mx_workspace_flags(ws, 6144, 2048);
  return MOE_OK;
}
}  // namespace moe

using namespace moe;

extern "C" {

size_t moe_mxfp4_workspace_bytes(int hidden, int intermediate) {
  return mx_carve(nullptr, hidden > 0 ? hidden : 1, intermediate > 0 ? intermediate : 1).bytes;
}

int moe_mxfp4_mlp(const uint16_t* x, const uint32_t* ids, int rows, int slots, const uint8_t* gate_up_codes,
                  const uint8_t* gate_up_scales, const uint8_t* down_codes, const uint8_t* down_scales,
                  int64_t experts, const uint16_t* unit, const uint16_t* out_gate, const uint16_t* out_up,
                  const uint16_t* in_down, const uint16_t* out_down, int hidden, int intermediate, uint16_t* values,
                  void* workspace, size_t workspace_bytes, moe_stream_t stream) {
  MOE_ARG(values != nullptr, "values must not be NULL");
  return mx_common(x, ids, nullptr, nullptr, rows, slots, gate_up_codes, gate_up_scales, down_codes, down_scales,
                   experts, unit, out_gate, out_up, in_down, out_down, hidden, intermediate, values, nullptr,
                   workspace, workspace_bytes, (hipStream_t)stream);
}

int moe_mxfp4_mlp_finish(const uint16_t* x, const uint32_t* ids, const float* scores, const uint16_t* residual,
                         int rows, const uint8_t* gate_up_codes, const uint8_t* gate_up_scales,
                         const uint8_t* down_codes, const uint8_t* down_scales, int64_t experts,
                         const uint16_t* unit, const uint16_t* out_gate, const uint16_t* out_up,
                         const uint16_t* in_down, const uint16_t* out_down, int hidden, int intermediate,
                         uint16_t* out, void* workspace, size_t workspace_bytes, moe_stream_t stream) {
  MOE_ARG(out != nullptr, "out must not be NULL");
  return mx_common(x, ids, scores, residual, rows, kSlots, gate_up_codes, gate_up_scales, down_codes, down_scales,
                   experts, unit, out_gate, out_up, in_down, out_down, hidden, intermediate, nullptr, out, workspace,
                   workspace_bytes, (hipStream_t)stream);
}

// Router GEMV + route + joined-MXFP4 MLP + combine for decode rows in one call on a checked
// workspace (every argument is validated before the first launch).  One token row runs the fused
// single-launch block (mx_layer.hip); more rows run the router kernel and the two GEMV launches.
static int mx_decode_block(const uint16_t* x, const uint16_t* residual, int rows, const float* router_w,
                           const float* bias, const uint8_t* gate_up_codes, const uint8_t* gate_up_scales,
                           const uint8_t* down_codes, const uint8_t* down_scales, int64_t experts, const uint16_t* unit,
                           const uint16_t* out_gate, const uint16_t* out_up, const uint16_t* in_down,
                           const uint16_t* out_down, int hidden, int intermediate, uint16_t* out, uint32_t* indices,
                           float* scores, void* workspace, size_t workspace_bytes, hipStream_t s,
                           bool clear_counters = false) {
  MOE_ARG(x && residual && router_w && bias && out && workspace, "null pointer argument");
  MOE_ARG(rows >= 1 && rows <= kMaxRows, "rows must be in 1..%d", kMaxRows);
  MOE_ARG(experts == 257, "the routed decode block needs 256 routed experts plus the shared expert (got %lld)",
          (long long)experts);
  MxWorkspace w = mx_carve(workspace, hidden > 0 ? hidden : 1, intermediate > 0 ? intermediate : 1);
  uint32_t* ids = indices ? indices : w.ids;
  float* sc = scores ? scores : w.scores;
  int rc = mx_check(x, ids, rows, kSlots, gate_up_codes, gate_up_scales, down_codes, down_scales, experts, unit,
                    out_gate, out_up, in_down, out_down, hidden, intermediate, workspace, workspace_bytes);
  if (rc) return rc;
  if ((rc = ensure_device_ready())) return rc;
  if (rows == 1)
    return mx_layer_run(x, residual, router_w, bias, ids, sc, gate_up_codes, gate_up_scales, down_codes, down_scales,
                        unit, out_gate, out_up, in_down, out_down, out, w.layer, s);
  if (clear_counters) {
    // counters that must start at zero: the router's arrival counter and the MLP's block and group
    // counters (a fill kernel, not a memset node, so the call can be captured in a graph)
    hipLaunchKernelGGL(zero_counters_kernel, dim3(1), dim3(256), 0, s, w.counter_blk,
                       (int)((reinterpret_cast<char*>(w.rowout) - reinterpret_cast<char*>(w.counter_blk)) / 4),
                       w.router_counter, 64);
    MOE_HIP(hipGetLastError());
  }
  rc = moe_router_fused_plan(x, router_w, bias, rows, hidden, 257, w.logits, ids, sc, w.plan, w.router_counter, s);
  if (rc) return rc;
  return mx_launch(x, ids, sc, residual, rows, kSlots, gate_up_codes, gate_up_scales, down_codes, down_scales,
                   experts, unit, out_gate, out_up, in_down, out_down, hidden, intermediate, nullptr, out, workspace,
                   s);
}

int moe_mxfp4_moe_decode(const uint16_t* x, const uint16_t* residual, int rows, const float* router_w,
                         const float* bias, const uint8_t* gate_up_codes, const uint8_t* gate_up_scales,
                         const uint8_t* down_codes, const uint8_t* down_scales, int64_t experts,
                         const uint16_t* unit, const uint16_t* out_gate, const uint16_t* out_up,
                         const uint16_t* in_down, const uint16_t* out_down, int hidden, int intermediate,
                         uint16_t* out, uint32_t* indices, float* scores, void* workspace, size_t workspace_bytes,
                         moe_stream_t stream) {
  return mx_decode_block(x, residual, rows, router_w, bias, gate_up_codes, gate_up_scales, down_codes, down_scales,
                         experts, unit, out_gate, out_up, in_down, out_down, hidden, intermediate, out, indices, scores,
                         workspace, workspace_bytes, (hipStream_t)stream);
}

// The decode block of moe_mxfp4_moe_decode with its workspace in the library's fixed per-device
// scratch array instead of a caller buffer: no allocation of any kind.  Shapes whose workspace
// exceeds the scratch are rejected.  Calls on one GPU share the scratch: overlapping calls race.
int moe_mxfp4_moe_decode_noalloc(const uint16_t* x, const uint16_t* residual, int rows, const float* router_w,
                                 const float* bias, const uint8_t* gate_up_codes, const uint8_t* gate_up_scales,
                                 const uint8_t* down_codes, const uint8_t* down_scales, int64_t experts,
                                 const uint16_t* unit, const uint16_t* out_gate, const uint16_t* out_up,
                                 const uint16_t* in_down, const uint16_t* out_down, int hidden, int intermediate,
                                 uint16_t* out, uint32_t* indices, float* scores, moe_stream_t stream) {
  MOE_ARG(hidden > 0 && intermediate > 0, "hidden and intermediate must be positive");
  const size_t need = mx_carve(nullptr, hidden, intermediate).bytes;
  if (need > kScratchBytes)
    return fail(MOE_ENOTSUP, "hidden %d / intermediate %d need %zu bytes of scratch; the fixed scratch holds %zu",
                hidden, intermediate, need, kScratchBytes);
  void* ws = nullptr;
  int rc = scratch_address(&ws);
  if (rc) return rc;
  return mx_decode_block(x, residual, rows, router_w, bias, gate_up_codes, gate_up_scales, down_codes, down_scales,
                         experts, unit, out_gate, out_up, in_down, out_down, hidden, intermediate, out, indices, scores,
                         ws, kScratchBytes, (hipStream_t)stream, true);
}

}  // extern "C"
