// Residual add + RMSNorm for decode rows (exlr8/fast_norm.py:20-28 residual_rms_pair,
// exlr8/metal/residual_rms.metal:18-90; model.py:376-384 for the unfused form):
//   h   = T(x + residual)                       (residual optional: h = x)
//   out = T(w * T(h * rsqrt(mean(h^2) + eps)))   T = bf16, the mean accumulated in fp32
// One block per row; every thread owns 8 consecutive elements (one 16 B load of each input).
#include "moe_device.h"
#include "moe_host.h"

namespace moe {
namespace {

// block of 256 threads; n = 2048 * k for k <= 4 (8 elements per thread per 2048)
template <int K>
__global__ __launch_bounds__(256) void residual_rmsnorm_kernel(const uint16_t* __restrict__ x,
                                                               const uint16_t* __restrict__ residual,
                                                               const uint16_t* __restrict__ w, int n, float eps,
                                                               uint16_t* __restrict__ h_out,
                                                               uint16_t* __restrict__ out) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  rms_u32x4 hv[K], wv[K];
  float ss = rms_row_sum<K>(x + row * n, residual ? residual + row * n : nullptr, w, K, (int)threadIdx.x, hv, wv,
                            h_out ? h_out + row * n : nullptr);
  ss = wave_sum(ss);
  if (lane_id() == 63) red[wave_id_in_block()] = ss;
  __syncthreads();
  rms_row_store<K>(hv, wv, K, (int)threadIdx.x, rms_inv(red, n, eps), out + row * n);
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
