// Residual add + RMSNorm for decode rows (exlr8/fast_norm.py:20-28 residual_rms_pair,
// exlr8/metal/residual_rms.metal:18-90; model.py:376-384 for the unfused form):
//   h   = T(x + residual)                       (residual optional: h = x)
//   out = T(w * T(h * rsqrt(mean(h^2) + eps)))   T = bf16, the mean accumulated in fp32
// One block per row; every thread owns 8 consecutive elements (one 16 B load of each input).
#include "moe_device.h"
#include "moe_host.h"

namespace moe {
namespace {

typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float lo_bf16(uint32_t v) { return bf16_to_f32((uint16_t)(v & 0xFFFFu)); }
__device__ __forceinline__ float hi_bf16(uint32_t v) { return bf16_to_f32((uint16_t)(v >> 16)); }
__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  return (uint32_t)f32_to_bf16(a) | ((uint32_t)f32_to_bf16(b) << 16);
}

// block of 256 threads; n = 2048 * k for k <= 4 (8 elements per thread per 2048)
template <int K>
__global__ __launch_bounds__(256) void residual_rmsnorm_kernel(const uint16_t* __restrict__ x,
                                                               const uint16_t* __restrict__ residual,
                                                               const uint16_t* __restrict__ w, int n, float eps,
                                                               uint16_t* __restrict__ h_out,
                                                               uint16_t* __restrict__ out) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  // the weight row depends on nothing: its loads go out with the activations' (one round trip)
  u32x4v wv[K];
#pragma unroll
  for (int k = 0; k < K; k++) wv[k] = *reinterpret_cast<const u32x4v*>(w + k * 2048 + threadIdx.x * 8);
  u32x4v hv[K];
  float ss = 0.0f;
#pragma unroll
  for (int k = 0; k < K; k++) {
    const int64_t off = row * n + k * 2048 + threadIdx.x * 8;
    const u32x4v xv = *reinterpret_cast<const u32x4v*>(x + off);
    u32x4v rv = u32x4v{0, 0, 0, 0};
    if (residual) rv = *reinterpret_cast<const u32x4v*>(residual + off);
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const float a = round_bf16(lo_bf16(xv[j]) + lo_bf16(rv[j]));
      const float b = round_bf16(hi_bf16(xv[j]) + hi_bf16(rv[j]));
      ss = fmaf(a, a, ss);
      ss = fmaf(b, b, ss);
      hv[k][j] = pack_bf16(a, b);
    }
    if (h_out) *reinterpret_cast<u32x4v*>(h_out + off) = hv[k];
  }
  ss = wave_sum(ss);
  if (lane_id() == 63) red[wave_id_in_block()] = ss;
  __syncthreads();
  const float tot = (red[0] + red[1]) + (red[2] + red[3]);
  const float inv = 1.0f / sqrtf(tot / (float)n + eps);
#pragma unroll
  for (int k = 0; k < K; k++) {
    const int64_t off = row * n + k * 2048 + threadIdx.x * 8;
    u32x4v o;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      o[j] = pack_bf16(round_bf16(lo_bf16(wv[k][j]) * round_bf16(lo_bf16(hv[k][j]) * inv)),
                       round_bf16(hi_bf16(wv[k][j]) * round_bf16(hi_bf16(hv[k][j]) * inv)));
    }
    *reinterpret_cast<u32x4v*>(out + off) = o;
  }
}

}  // namespace
}  // namespace moe

using namespace moe;

extern "C" {

int moe_residual_rmsnorm(const uint16_t* x, const uint16_t* residual, const uint16_t* weight, int rows, int n,
                         float eps, uint16_t* h_out, uint16_t* out, moe_stream_t stream) {
  MOE_ARG(x && weight && out, "x, weight and out must not be NULL");
  MOE_ARG(rows >= 0, "rows must be non-negative");
  MOE_ARG(n > 0 && n % 2048 == 0 && n <= 8192, "normalised size must be a multiple of 2048 up to 8192 (got %d)", n);
  MOE_ARG(eps >= 0.0f, "epsilon must be non-negative");
  if (rows == 0) return MOE_OK;
  int rc = ensure_device_ready();
  if (rc) return rc;
  const hipStream_t s = (hipStream_t)stream;
  switch (n / 2048) {
    case 1: hipLaunchKernelGGL(residual_rmsnorm_kernel<1>, dim3(rows), dim3(256), 0, s, x, residual, weight, n, eps, h_out, out); break;
    case 2: hipLaunchKernelGGL(residual_rmsnorm_kernel<2>, dim3(rows), dim3(256), 0, s, x, residual, weight, n, eps, h_out, out); break;
    case 3: hipLaunchKernelGGL(residual_rmsnorm_kernel<3>, dim3(rows), dim3(256), 0, s, x, residual, weight, n, eps, h_out, out); break;
    default: hipLaunchKernelGGL(residual_rmsnorm_kernel<4>, dim3(rows), dim3(256), 0, s, x, residual, weight, n, eps, h_out, out); break;
  }
  MOE_HIP(hipGetLastError());
  return MOE_OK;
}

}  // extern "C"
