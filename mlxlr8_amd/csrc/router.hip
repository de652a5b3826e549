// Router for the MoE expert path on gfx950: fp32 gate GEMV, sigmoid, bias-corrected top-8.
//
// Reference semantics (paths relative to the reference root):
//   logits = f32(x) @ W^T with an fp32 weight          exlr8/dense.py:158-159, exlr8/model.py:367-370,406
//   s = v < 0 ? y : 1 - y, y = 1 / (1 + exp(|v|))        exlr8/metal/fast_router.metal:7-9
//   top-8 of s + bias, descending, ties -> lower id      exlr8/metal/fast_router.metal:13-34
//   score = s / (1e-20 + sum s_sel) * 2.5, slot 8 = 256  exlr8/metal/fast_router.metal:35-42
//
// MI355X design: one wave (64 lanes, 4 experts per lane) per token row; the arg-max of each
// of the 8 rounds is a 6-step butterfly over (value, id) pairs, so every lane learns the
// winner without a second pass.  For decode batches the same block also builds the
// token -> expert dispatch plan, so no route ever travels back to the host.
#include <hip/hip_runtime.h>

#include "moe_device.h"
#include "moe_host.h"
#include "moe_plan.h"
#include "route.h"

namespace moe {

// ---------------------------------------------------------------- logits, small batches
// One block per expert row; each thread covers hidden/256 inputs with 16-byte loads.
template <int R>
__global__ __launch_bounds__(256) void router_logits_small(const uint16_t* __restrict__ x,
                                                           const float* __restrict__ w, int rows, int hidden,
                                                           int experts, float* __restrict__ logits) {
  const int e = blockIdx.x;
  const float* __restrict__ we = w + (int64_t)e * hidden;
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; r++) acc[r] = 0.0f;
  for (int k = threadIdx.x * 4; k < hidden; k += 256 * 4) {
    const f32x4 wv = *reinterpret_cast<const f32x4*>(we + k);
#pragma unroll
    for (int r = 0; r < R; r++) {
      if (r < rows) {
        const u32x2 xv = *reinterpret_cast<const u32x2*>(x + (int64_t)r * hidden + k);
        acc[r] = fmaf(bf16_to_f32((uint16_t)(xv.x & 0xFFFFu)), wv.x, acc[r]);
        acc[r] = fmaf(bf16_to_f32((uint16_t)(xv.x >> 16)), wv.y, acc[r]);
        acc[r] = fmaf(bf16_to_f32((uint16_t)(xv.y & 0xFFFFu)), wv.z, acc[r]);
        acc[r] = fmaf(bf16_to_f32((uint16_t)(xv.y >> 16)), wv.w, acc[r]);
      }
    }
  }
  __shared__ float red[R][4];
  const int lane = lane_id(), wv = wave_id_in_block();
#pragma unroll
  for (int r = 0; r < R; r++) {
    const float v = wave_sum(acc[r]);
    if (lane == 63) red[r][wv] = v;
  }
  __syncthreads();
  if (threadIdx.x < R && (int)threadIdx.x < rows) {
    const int r = threadIdx.x;
    logits[(int64_t)r * experts + e] = (red[r][0] + red[r][1]) + (red[r][2] + red[r][3]);
  }
}

// ---------------------------------------------------------------- logits, prefill batches
// 16 rows x 16 experts per block on the fp32 matrix cores (v_mfma_f32_16x16x4_f32); the 16 waves
// split K into 16 chunks and the chunk tiles are summed in LDS in chunk order.  Which wave takes
// which chunk rotates with the block, so the blocks do not all read the same k offsets at once.
// Per 64-wide k step, lane l = 16 kk + r loads 16 consecutive k (32 B of x row r, 64 B of w row r)
// at 16 kk: a row's four lanes read whole 128 B lines.  MFMA i (0..15) takes element i, so its
// k-group kk covers k0 + 16 kk + i.
constexpr int kLogitWaves = 16;
__global__ __launch_bounds__(kLogitWaves * 64) void router_logits_mfma(const uint16_t* __restrict__ x,
                                                                      const float* __restrict__ w, int rows,
                                                                      int hidden, int experts,
                                                                      float* __restrict__ logits) {
  __shared__ f32x4 red[kLogitWaves][64];
  // 1-D grid of (expert blocks) x (row blocks).  Workgroups are dealt to the 8 XCDs in turn; when
  // the expert blocks split evenly over them, XCD x takes expert blocks [x n/8, (x+1) n/8) for
  // every row block (its slice of w stays in its L2, and the row block's x is read once per XCD)
  const int neb = (experts + 15) / 16;
  int bx, by;
  if (neb % 8 == 0) {
    const int per = neb / 8, j = blockIdx.x / 8;
    bx = (blockIdx.x % 8) * per + j % per;
    by = j / per;
  } else {
    bx = blockIdx.x % neb;
    by = blockIdx.x / neb;
  }
  const int r0 = by * 16, e0 = bx * 16;
  const int wv = wave_id_uniform(), lane = lane_id(), r = lane & 15, kk = lane >> 4;
  const int chunk = (wv + 5 * bx + 3 * by) % kLogitWaves;
  const int kq = hidden / kLogitWaves;  // a multiple of 64 (hidden % 1024 == 0)
  const uint16_t* __restrict__ xr = x + (int64_t)min(r0 + r, rows - 1) * hidden + chunk * kq + 16 * kk;
  const float* __restrict__ wr = w + (int64_t)min(e0 + r, experts - 1) * hidden + chunk * kq + 16 * kk;
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  // two 64-wide steps per batch: all of a batch's loads are issued before its MFMAs
  for (int k0 = 0; k0 < kq; k0 += 128) {
    u32x4 xv[2][2];
    f32x4 wvv[2][4];
#pragma unroll
    for (int b = 0; b < 2; b++) {
      const int k = min(k0 + 64 * b, kq - 64);  // past the end: re-read the last step (not used)
#pragma unroll
      for (int i = 0; i < 2; i++) xv[b][i] = *reinterpret_cast<const u32x4*>(xr + k + 8 * i);
#pragma unroll
      for (int i = 0; i < 4; i++) wvv[b][i] = *reinterpret_cast<const f32x4*>(wr + k + 4 * i);
    }
#pragma unroll
    for (int b = 0; b < 2; b++) {
      if (k0 + 64 * b < kq) {
#pragma unroll
        for (int i = 0; i < 16; i++) {
          const uint32_t xw = xv[b][i >> 3][(i >> 1) & 3];
          const float xa = bf16_to_f32((uint16_t)((i & 1) ? (xw >> 16) : (xw & 0xFFFFu)));
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xa, wvv[b][i >> 2][i & 3], acc, 0, 0, 0);
        }
      }
    }
  }
  red[chunk][lane] = acc;
  __syncthreads();
  if (wv == 0) {
    f32x4 t = red[0][lane];
#pragma unroll
    for (int i = 1; i < kLogitWaves; i++) t = t + red[i][lane];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int row = r0 + 4 * kk + i, e = e0 + r;  // D[4 kk + i][r]
      if (row < rows && e < experts) logits[(int64_t)row * experts + e] = t[i];
    }
  }
}

// ---------------------------------------------------------------- selection (route.h)

__global__ __launch_bounds__(64) void route_kernel(const float* __restrict__ logits, const float* __restrict__ bias,
                                                   int rows, uint32_t* __restrict__ ids, float* __restrict__ scores) {
  const int row = blockIdx.x;
  if (row < rows) route_row(logits, bias, row, ids, scores);
}

// logits per decode-router block: single-row launches use 4 (fewer, larger blocks dispatch
// faster); the 8-row kernel keeps one (its x rows already fill the registers)
template <int R>
struct RouterGroups {
  static constexpr int value = R == 1 ? 4 : 1;
};

// Decode batches in one launch: block e computes logit e of every row; the last block to finish
// routes all rows (one wave per row) and builds the token -> expert dispatch plan.  With a null
// counter only the logits (and the normalised rows) are produced.
// KI = hidden / 1024 when known at compile time (all loads of a block are then issued before the
// first multiply, one memory round trip), 0 for any multiple of 1024.
//
// NORM (KI > 0 only): the router input is RMSNorm(h), h = T(x + attn) (attn optional), computed
// in every block from the raw rows (each block holds whole rows, so it reduces the sum of squares
// itself); block r also stores row r's h (the layer residual) and normalised input for the
// expert kernels.  Same arithmetic as moe_residual_rmsnorm.
template <int R, int KI, bool NORM>
__global__ __launch_bounds__(256 * RouterGroups<R>::value) void router_decode_kernel(const uint16_t* __restrict__ x,
                                                            const float* __restrict__ w,
                                                            const float* __restrict__ bias, int rows, int hidden,
                                                            int experts, int max_users, float* logits,
                                                            uint32_t* ids, float* __restrict__ scores, Plan* plan,
                                                            int32_t* counter, const uint16_t* __restrict__ attn,
                                                            const uint16_t* __restrict__ norm_w, float eps,
                                                            uint16_t* __restrict__ h_out,
                                                            uint16_t* __restrict__ xn_out) {
  // kRouterGroups groups of 256 threads per block, group gi computing logit e
  constexpr int kRouterGroups = RouterGroups<R>::value;
  const int gi = (int)threadIdx.x >> 8, tx = (int)threadIdx.x & 255;
  const int e = (int)blockIdx.x * kRouterGroups + gi;
  const float* __restrict__ we = w + (int64_t)e * hidden;
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; r++) acc[r] = 0.0f;
  auto fma4 = [&](int r, const f32x4& wv, const u32x2& xv) {
    acc[r] = fmaf(bf16_to_f32((uint16_t)(xv.x & 0xFFFFu)), wv.x, acc[r]);
    acc[r] = fmaf(bf16_to_f32((uint16_t)(xv.x >> 16)), wv.y, acc[r]);
    acc[r] = fmaf(bf16_to_f32((uint16_t)(xv.y & 0xFFFFu)), wv.z, acc[r]);
    acc[r] = fmaf(bf16_to_f32((uint16_t)(xv.y >> 16)), wv.w, acc[r]);
  };
  if (KI > 0) {
    f32x4 wv[KI > 0 ? KI : 1];
    u32x2 xv[R][KI > 0 ? KI : 1];
#pragma unroll
    for (int i = 0; i < KI; i++) wv[i] = *reinterpret_cast<const f32x4*>(we + tx * 4 + i * 1024);
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
      for (int i = 0; i < KI; i++)
        if (r < rows) xv[r][i] = *reinterpret_cast<const u32x2*>(x + (int64_t)r * hidden + tx * 4 + i * 1024);
    if (NORM) {
      __shared__ float nred[kRouterGroups][R][4];
      u32x2 nw[KI > 0 ? KI : 1];
#pragma unroll
      for (int i = 0; i < KI; i++) nw[i] = *reinterpret_cast<const u32x2*>(norm_w + tx * 4 + i * 1024);
      auto lo = [](uint32_t v) { return bf16_to_f32((uint16_t)(v & 0xFFFFu)); };
      auto hi = [](uint32_t v) { return bf16_to_f32((uint16_t)(v >> 16)); };
      auto pk = [](float a, float b) { return (uint32_t)f32_to_bf16(a) | ((uint32_t)f32_to_bf16(b) << 16); };
      float ss[R];
#pragma unroll
      for (int r = 0; r < R; r++) {
        ss[r] = 0.0f;
#pragma unroll
        for (int i = 0; i < KI; i++)
          if (r < rows) {
            u32x2 av = u32x2{0, 0};
            if (attn) av = *reinterpret_cast<const u32x2*>(attn + (int64_t)r * hidden + tx * 4 + i * 1024);
            const float h0 = round_bf16(lo(xv[r][i].x) + lo(av.x)), h1 = round_bf16(hi(xv[r][i].x) + hi(av.x));
            const float h2 = round_bf16(lo(xv[r][i].y) + lo(av.y)), h3 = round_bf16(hi(xv[r][i].y) + hi(av.y));
            ss[r] = fmaf(h0, h0, ss[r]);
            ss[r] = fmaf(h1, h1, ss[r]);
            ss[r] = fmaf(h2, h2, ss[r]);
            ss[r] = fmaf(h3, h3, ss[r]);
            xv[r][i] = u32x2{pk(h0, h1), pk(h2, h3)};
          }
        const float v = wave_sum(ss[r]);
        if (lane_id() == 63) nred[gi][r][tx >> 6] = v;
      }
      __syncthreads();
#pragma unroll
      for (int r = 0; r < R; r++) {
        if (r < rows) {
          const float inv = 1.0f / sqrtf(((nred[gi][r][0] + nred[gi][r][1]) + (nred[gi][r][2] + nred[gi][r][3])) / (float)hidden + eps);
#pragma unroll
          for (int i = 0; i < KI; i++) {
            const u32x2 hv = xv[r][i];
            const u32x2 xn = u32x2{pk(round_bf16(lo(nw[i].x) * round_bf16(lo(hv.x) * inv)),
                                      round_bf16(hi(nw[i].x) * round_bf16(hi(hv.x) * inv))),
                                   pk(round_bf16(lo(nw[i].y) * round_bf16(lo(hv.y) * inv)),
                                      round_bf16(hi(nw[i].y) * round_bf16(hi(hv.y) * inv)))};
            if (e == r) {
              const int64_t off = (int64_t)r * hidden + tx * 4 + i * 1024;
              *reinterpret_cast<u32x2*>(h_out + off) = hv;
              *reinterpret_cast<u32x2*>(xn_out + off) = xn;
            }
            xv[r][i] = xn;
          }
        }
      }
    }
#pragma unroll
    for (int i = 0; i < KI; i++)
#pragma unroll
      for (int r = 0; r < R; r++)
        if (r < rows) fma4(r, wv[i], xv[r][i]);
  } else {
    for (int k = tx * 4; k < hidden; k += 256 * 4) {
      const f32x4 wv = *reinterpret_cast<const f32x4*>(we + k);
#pragma unroll
      for (int r = 0; r < R; r++)
        if (r < rows) fma4(r, wv, *reinterpret_cast<const u32x2*>(x + (int64_t)r * hidden + k));
    }
  }
  __shared__ float red[kRouterGroups][R][4];
  __shared__ int last;
  __shared__ int32_t sid[kMaxUnits];
  __shared__ int32_t open[kMaxUnits];
  const int lane = lane_id(), wv = wave_id_in_block();
#pragma unroll
  for (int r = 0; r < R; r++) {
    const float v = wave_sum(acc[r]);
    if (lane == 63) red[gi][r][tx >> 6] = v;
  }
  __syncthreads();
  if (tx < R && tx < rows) {
    const int r = tx;
    const float lg = (red[gi][r][0] + red[gi][r][1]) + (red[gi][r][2] + red[gi][r][3]);
    __hip_atomic_store(logits + (int64_t)r * 256 + e, lg, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  }
  // without a counter the routing is left to the expert kernels (they read the logits after
  // this launch ends)
  if (counter == nullptr) return;
  release_stores();
  __syncthreads();
  if (threadIdx.x == 0)
    last = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) == (int)gridDim.x - 1;
  __syncthreads();
  if (!last) return;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  (void)experts;  // routed ids are 0..255 plus the shared expert 256
  if (rows == 1) {
    // one row: slot s is unit s (the 8 routed ids are distinct and the shared id is 256), so the
    // routing lanes write the plan build_plan_parallel would build, without its passes
    if (wv == 0) {
      route_row<true>(logits, bias, 0, ids, scores, sid);
      const int lane = lane_id();
      if (lane < kSlots) {
        plan->expert[lane] = sid[lane];  // written by this lane in route_row
        plan->ntok[lane] = 1;
        plan->tok[lane][0] = 0;
        plan->slot[lane][0] = lane;
        plan->slot_unit[lane] = lane;
        plan->slot_pos[lane] = 0;
        if (lane == 0) {
          plan->units = kSlots;
          plan->rows = 1;
        }
      }
    }
  } else {
    for (int row = wv; row < rows; row += 4 * kRouterGroups) route_row<true>(logits, bias, row, ids, scores, sid);
    __syncthreads();
    build_plan_parallel(sid, rows, kSlots, max_users, plan, open);
  }
  if (threadIdx.x == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

int launch_router_logits(const uint16_t* x, const float* w, int rows, int hidden, int experts, float* logits,
                         hipStream_t s) {
  if (rows <= 1) {
    hipLaunchKernelGGL(router_logits_small<1>, dim3(experts), dim3(256), 0, s, x, w, rows, hidden, experts, logits);
  } else if (rows <= kMaxRows) {
    hipLaunchKernelGGL(router_logits_small<kMaxRows>, dim3(experts), dim3(256), 0, s, x, w, rows, hidden, experts,
                       logits);
  } else {
    const unsigned grid = (unsigned)((experts + 15) / 16) * (unsigned)((rows + 15) / 16);
    hipLaunchKernelGGL(router_logits_mfma, dim3(grid), dim3(kLogitWaves * 64), 0, s, x, w, rows, hidden, experts,
                       logits);
  }
  MOE_HIP(hipGetLastError());
  return MOE_OK;
}

// Router GEMV + route + dispatch plan for decode batches (used by moe_k4_moe_decode).  With
// norm_w, x is the raw layer input: the router (and the expert kernels, through xn_out) see
// RMSNorm(T(x + attn)), and h_out receives T(x + attn).
int moe_router_fused_plan(const uint16_t* x, const float* w, const float* bias, int rows, int hidden, int experts,
                          float* logits, uint32_t* ids, float* scores, Plan* plan, int32_t* counter, hipStream_t s,
                          const uint16_t* attn, const uint16_t* norm_w, float eps, uint16_t* h_out,
                          uint16_t* xn_out) {
  MOE_ARG(hidden > 0 && hidden % 1024 == 0, "router hidden size must be a positive multiple of 1024");
  MOE_ARG(rows >= 1 && rows <= kMaxRows, "decode routing handles 1..%d rows", kMaxRows);
  const int max_users = rows == 1 ? 1 : kMaxRows;
  const uint16_t* xin = x;
  const bool fused_norm = norm_w && hidden == 6144;
  if (norm_w && !fused_norm) {
    // other widths: normalise first, then route the normalised rows
    int rc = moe_residual_rmsnorm(x, attn, norm_w, rows, hidden, eps, h_out, xn_out, (moe_stream_t)s);
    if (rc) return rc;
    xin = xn_out;
  }
#define MOE_ROUTER_LAUNCH(R, KI, N)                                                                                 \
  hipLaunchKernelGGL((router_decode_kernel<R, KI, N>), dim3(256 / RouterGroups<R>::value),                       \
                     dim3(256 * RouterGroups<R>::value), 0, s,                                                        \
                     xin, w, bias, rows, hidden,                                                                      \
                     experts, max_users, logits, ids, scores, plan, counter, attn, norm_w, eps, h_out, xn_out)
  if (fused_norm && rows == 1)
    MOE_ROUTER_LAUNCH(1, 6, true);
  else if (fused_norm)
    MOE_ROUTER_LAUNCH(kMaxRows, 6, true);
  else if (rows == 1 && hidden == 6144)
    MOE_ROUTER_LAUNCH(1, 6, false);
  else if (rows == 1)
    MOE_ROUTER_LAUNCH(1, 0, false);
  else if (hidden == 6144)
    MOE_ROUTER_LAUNCH(kMaxRows, 6, false);
  else
    MOE_ROUTER_LAUNCH(kMaxRows, 0, false);
#undef MOE_ROUTER_LAUNCH
  MOE_HIP(hipGetLastError());
  return MOE_OK;
}

}  // namespace moe

using namespace moe;

extern "C" {

int moe_route_f32(const float* logits, const float* bias, int rows, uint32_t* indices, float* scores,
                  moe_stream_t stream) {
  MOE_ARG(logits && bias && indices && scores, "null pointer argument");
  MOE_ARG(rows >= 0, "rows must be non-negative");
  if (rows == 0) return MOE_OK;
  hipLaunchKernelGGL(route_kernel, dim3(rows), dim3(64), 0, (hipStream_t)stream, logits, bias, rows, indices, scores);
  MOE_HIP(hipGetLastError());
  return MOE_OK;
}

int moe_router_logits(const uint16_t* x, const float* w, int rows, int hidden, int experts, float* logits,
                      moe_stream_t stream) {
  MOE_ARG(x && w && logits, "null pointer argument");
  MOE_ARG(rows >= 0 && experts > 0, "rows must be non-negative and experts positive");
  MOE_ARG(hidden > 0 && hidden % 1024 == 0, "router hidden size must be a positive multiple of 1024");
  if (rows == 0) return MOE_OK;
  return launch_router_logits(x, w, rows, hidden, experts, logits, (hipStream_t)stream);
}

}  // extern "C"
