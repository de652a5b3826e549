// Device-side building blocks shared by the MoE expert-path kernels (gfx950, wave64).
//
// Formats restated here (reference paths relative to the reference repository root):
//   * K4 trellis codewords: 16-bit windows of a circular MSB-first bitstream, 8 per 32-bit
//     word (exlr8/trellis.py:78-102; direct K4 form exlr8/metal/fast_decode_linear.metal:147-155).
//   * Codebook: MCG hash, IEEE half add, round to E4M3 (exlr8/trellis.py:43-50).
//   * Normalised 128-point Sylvester Hadamard (exlr8/trellis.py:67-75).
//   * Typed SwiGLU (exlr8/metal/fast_decode_common.metal:40-49).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace moe {

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef short i16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kInvSqrt128 = 0.08838834764831845f;

// ---------------------------------------------------------------- scalar formats
__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }
__device__ __forceinline__ float f16_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// ---------------------------------------------------------------- codebook
// Two codewords (low 16 bits of a and b) -> two E4M3 values as float.  The hash
// product is formed with 24-bit multiplies (full rate), the masks with one 3-input
// bit operation, the half add in fp16 and the E4M3 rounding by a round trip through
// the hardware fp8 (OCP e4m3) conversion, which rounds to nearest even.  All decoded
// magnitudes are below 4, so the conversion never saturates.
__device__ __forceinline__ uint32_t mcg_product(uint32_t cw) {
  // cw * 0xCBAC1FED mod 2^32 for cw < 2^16:  cw*0xAC1FED + ((cw*0xCB) << 24)
  return __umul24(cw, 0xAC1FEDu) + (__umul24(cw, 0xCBu) << 24);
}
__device__ __forceinline__ uint32_t mcg_halves(uint32_t cw) {
  return (mcg_product(cw) & 0x8FFF8FFFu) ^ 0x3B603B60u;
}
// returns the two E4M3 bytes (a in bits 0-7, b in bits 8-15)
__device__ __forceinline__ uint32_t decode_pair_fp8(uint32_t a, uint32_t b) {
  f16x2 ha = __builtin_bit_cast(f16x2, mcg_halves(a & 0xFFFFu));
  f16x2 hb = __builtin_bit_cast(f16x2, mcg_halves(b & 0xFFFFu));
  f16x2 s;
  s.x = ha.x + ha.y;
  s.y = hb.x + hb.y;
  i16x2 old = {0, 0};
  i16x2 f8 = __builtin_amdgcn_cvt_scalef32_pk_fp8_f16(old, s, 1.0f, false);
  return (uint32_t)__builtin_bit_cast(uint32_t, f8) & 0xFFFFu;
}
__device__ __forceinline__ f32x2 decode_pair_alu(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(decode_pair_fp8(a, b), 1.0f, false);
}
__device__ __forceinline__ float fp8_to_f32(uint32_t byte) { return __builtin_amdgcn_cvt_f32_fp8(byte, 0); }

// The E4M3 code table for all 65536 states (64 KB).  Filled once per device by
// moe_build_codebook_kernel; copied into LDS by the decode GEMVs.
extern __device__ uint8_t g_codebook_e4m3[65536];

// Cooperative copy of the 64 KB table into LDS (blockDim threads, 16 B each).
__device__ __forceinline__ void load_codebook_lds(uint8_t* lds) {
  const u32x4* src = reinterpret_cast<const u32x4*>(g_codebook_e4m3);
  u32x4* dst = reinterpret_cast<u32x4*>(lds);
  for (int i = threadIdx.x; i < 65536 / 16; i += blockDim.x) dst[i] = src[i];
}

// ---------------------------------------------------------------- K4 word decode
// Word w of a tile with its circular predecessor p holds 8 codewords (A.1 direct form):
//   slot 0..2 straddle p and w, slot 3..7 lie inside w.
// Slot s sits at tile row (lane%4)*2 + (s&1) + (s&2)*4 and column lane/4 + (s&4)*2.
// ALU_PAIRS selects how many codeword pairs are decoded arithmetically; the rest are
// looked up in the LDS table.  Pairs in ALU preference order: (7,3), (6,2), (5,1), (4,0).
template <int ALU_PAIRS>
__device__ __forceinline__ void decode_word(uint32_t w, uint32_t p, const uint8_t* tab, float f[8]) {
  const uint32_t a4 = __builtin_amdgcn_alignbit(p, w, 4);   // (slot6 | slot2 << 16)
  const uint32_t a8 = __builtin_amdgcn_alignbit(p, w, 8);   // (slot5 | slot1 << 16)
  const uint32_t a12 = __builtin_amdgcn_alignbit(p, w, 12); // (slot4 | slot0 << 16)
  const uint32_t pairs[4] = {w, a4, a8, a12};
  const int lo_slot[4] = {7, 6, 5, 4};
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const uint32_t v = pairs[q];
    if (q < ALU_PAIRS) {
      f32x2 r = decode_pair_alu(v, v >> 16);
      f[lo_slot[q]] = r.x;
      f[lo_slot[q] - 4] = r.y;
    } else {
      f[lo_slot[q]] = fp8_to_f32(tab[v & 0xFFFFu]);
      f[lo_slot[q] - 4] = fp8_to_f32(tab[v >> 16]);
    }
  }
}

// ---------------------------------------------------------------- wave-level H128
// 128 values held as 2 per lane (element i = 2*lane + j).  Normalised Sylvester order;
// the butterfly order differs from the reference's numpy loop only in float rounding.
__device__ __forceinline__ void hadamard128_wave(float& v0, float& v1) {
  float a = v0 + v1, b = v0 - v1;
  v0 = a; v1 = b;
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) {
    float o0 = __shfl_xor(v0, m, 64);
    float o1 = __shfl_xor(v1, m, 64);
    const bool hi = (lane & m) != 0;
    v0 = hi ? (o0 - v0) : (v0 + o0);
    v1 = hi ? (o1 - v1) : (v1 + o1);
  }
  v0 *= kInvSqrt128;
  v1 *= kInvSqrt128;
}

// ---------------------------------------------------------------- typed SwiGLU
__device__ __forceinline__ float swiglu_bf16(float gate, float up) {
  const float g = round_bf16(gate), u = round_bf16(up);
  const float tail = 1.0f / (1.0f + expf(fabsf(g)));
  const float sig = round_bf16(g < 0.0f ? tail : 1.0f - tail);
  return round_bf16(round_bf16(g * sig) * u);
}

// ---------------------------------------------------------------- wave reductions (DPP)
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_f32(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xF,
                                                                false));
}
// Sum over the 64 lanes; the total is valid in lane 63.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f32<0xB1>(v);        // quad_perm [1,0,3,2]
  v += dpp_f32<0x4E>(v);        // quad_perm [2,3,0,1]
  v += dpp_f32<0x124>(v);       // row_ror:4
  v += dpp_f32<0x128>(v);       // row_ror:8  -> every lane holds its row (16 lanes) sum
  v += dpp_f32<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3
  v += dpp_f32<0x143, 0xC>(v);  // row_bcast:31 into rows 2 and 3
  return v;
}

// ---------------------------------------------------------------- small wave helpers
__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave_id_in_block() { return threadIdx.x >> 6; }

}  // namespace moe
