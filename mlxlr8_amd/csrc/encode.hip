// Load-time conversion of K4 trellis experts to the joined-MXFP4 resident format on gfx950.
//
// Reference semantics (paths relative to the reference root), exlr8/joined_mxfp4.py:12-47 encode:
//   inner_e = decoded K4 matrix [in, out] of expert e (the trellis decode kernel)
//   gate/up: inner_e[k, :] *= float(in_scale[e, k] * unit[k]), unit = sign(in_scale_gate[0])
//   codes, scales = mx.quantize(inner_e^T, mode="mxfp4"): per output row, groups of 32 along k
//   gate_up = gate rows || up rows; down unscaled
//
// MXFP4 quantiser (OCP MX v1.0 conversion): shared exponent s = floor(log2 amax) - 2 (E2M1's
// largest exponent), clamped to the E8M0 range, byte s + 127 (0 for an all-zero group); element
// = sign | E2M1(|v| / 2^s), round to nearest, ties to the even code, saturating at 6.  MLX's own
// mx.quantize rounding cannot be checked here (MLX is not available); this is the published
// conversion.
//
// MI355X design: a load-time path, run once per layer: each expert's inner matrix is decoded to
// fp16 by the trellis decode kernel into a caller workspace, then one thread per (output row,
// 32-wide k group) reads its 32 values (adjacent threads take adjacent rows, so each of the 32
// reads is one coalesced line), quantises them and writes 16 code bytes and one scale byte.
#include <hip/hip_runtime.h>

#include "moe_device.h"
#include "moe_host.h"

namespace moe {
namespace {

// E2M1 code of a magnitude a = |v| / 2^s: nearest of 0, .5, 1, 1.5, 2, 3, 4, 6, ties to the even
// code, saturating (midpoints .25 .75 1.25 1.75 2.5 3.5 5)
__device__ __forceinline__ uint32_t e2m1_code(float a) {
  uint32_t c = 0;
  c += a > 0.25f;
  c += a >= 0.75f;
  c += a > 1.25f;
  c += a >= 1.75f;
  c += a > 2.5f;
  c += a >= 3.5f;
  c += a > 5.0f;
  return c;
}

// one thread per (row n of this projection, k group g); inner [in][out] fp16 of one expert
__global__ __launch_bounds__(256) void mx_quantize_kernel(const uint16_t* __restrict__ inner, int in_f, int out_f,
                                                          const uint16_t* __restrict__ in_scale,
                                                          const uint16_t* __restrict__ unit,
                                                          uint8_t* __restrict__ codes, uint8_t* __restrict__ scales) {
  const int n = blockIdx.x * 256 + threadIdx.x;
  const int g = blockIdx.y;
  if (n >= out_f) return;
  float v[32];
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 32; i++) {
    const int k = 32 * g + i;
    float x = f16_to_f32(inner[(int64_t)k * out_f + n]);
    if (in_scale) x *= f16_to_f32(in_scale[k]) * f16_to_f32(unit[k]);  // exact: unit is +-1
    v[i] = x;
    amax = fmaxf(amax, fabsf(x));
  }
  // floor(log2 amax) from the exponent field (amax below 2^-126 clamps to -127 either way)
  const int ebits = (int)((__float_as_uint(amax) >> 23) & 0xFFu);
  const int s = amax > 0.0f ? max(-127, min(127, ebits - 127 - 2)) : -127;
  uint32_t w[4];
#pragma unroll
  for (int q = 0; q < 4; q++) {
    uint32_t word = 0;
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const float x = v[8 * q + j];
      const uint32_t c = e2m1_code(__builtin_amdgcn_ldexpf(fabsf(x), -s)) | ((__float_as_uint(x) >> 31) << 3);
      word |= c << (4 * j);
    }
    w[q] = word;
  }
  const int64_t row = n;
  *reinterpret_cast<u32x4*>(codes + row * (in_f / 2) + 16 * g) = u32x4{w[0], w[1], w[2], w[3]};
  scales[row * (in_f / 32) + g] = (uint8_t)(s + 127);
}

}  // namespace
}  // namespace moe

using namespace moe;

extern "C" {

size_t moe_k4_to_mxfp4_workspace_bytes(int in_features, int out_features) {
  if (in_features <= 0 || out_features <= 0) return 0;
  return (size_t)in_features * out_features * sizeof(uint16_t);
}

int moe_k4_to_mxfp4(const void* packed, int64_t packed_bytes, int in_features, int out_features, int side,
                    const uint16_t* in_scale, const uint16_t* unit, uint8_t* codes, uint8_t* scales, int out_rows,
                    int row_offset, void* workspace, size_t workspace_bytes, moe_stream_t stream) {
  MOE_ARG(packed && codes && scales && workspace, "null pointer argument");
  MOE_ARG((in_scale == nullptr) == (unit == nullptr), "in_scale and unit are given together (gate/up) or not at all (down)");
  MOE_ARG(in_features > 0 && out_features > 0 && in_features % 128 == 0 && out_features % 128 == 0,
          "K4 dimensions must be positive multiples of 128 (got %d x %d)", in_features, out_features);
  MOE_ARG(side == 1 || side == 2, "sharded_side must be 1 (gate/up) or 2 (down)");
  MOE_ARG(row_offset >= 0 && out_rows >= row_offset + out_features,
          "rows %d..%d do not fit the %d-row destination", row_offset, row_offset + out_features, out_rows);
  MOE_ARG(((uintptr_t)codes % 16) == 0, "codes must be 16-byte aligned");
  const int64_t per_expert = (int64_t)in_features * out_features / 2;
  MOE_ARG(packed_bytes > 0 && packed_bytes % per_expert == 0,
          "packed size %lld is not a whole number of %d x %d K4 experts", (long long)packed_bytes, in_features,
          out_features);
  if (workspace_bytes < moe_k4_to_mxfp4_workspace_bytes(in_features, out_features))
    return fail(MOE_EWORKSPACE, "workspace too small: %zu < %zu bytes", workspace_bytes,
                moe_k4_to_mxfp4_workspace_bytes(in_features, out_features));
  int rc = ensure_device_ready();
  if (rc) return rc;
  const int64_t experts = packed_bytes / per_expert;
  uint16_t* inner = static_cast<uint16_t*>(workspace);
  const dim3 grid((unsigned)((out_features + 255) / 256), (unsigned)(in_features / 32));
  for (int64_t e = 0; e < experts; e++) {
    if ((rc = moe_trellis_decode_f16(packed, packed_bytes, 4, in_features, out_features, side, e, inner, stream)))
      return rc;
    const int64_t r0 = e * out_rows + row_offset;
    hipLaunchKernelGGL(mx_quantize_kernel, grid, dim3(256), 0, (hipStream_t)stream, inner, in_features, out_features,
                       in_scale ? in_scale + e * in_features : nullptr, unit, codes + r0 * (in_features / 2),
                       scales + r0 * (in_features / 32));
    MOE_HIP(hipGetLastError());
  }
  return MOE_OK;
}

}  // extern "C"
