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

#include <type_traits>
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

// ---------------------------------------------------------------- residual add + RMSNorm, one row
// (exlr8/fast_norm.py:20-28, exlr8/metal/residual_rms.metal:18-90)
//   h = T(x + residual), out = T(w * T(h * rsqrt(mean(h^2) + eps))), T = bf16, mean in fp32.
// Thread t of 256 owns elements 2048 k + 8 t .. + 7 for k < K; its square sum runs over them in
// that order.  The norm kernel and the fused K4 block both use these two steps, so their rows
// are the same bits.
typedef uint32_t rms_u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint32_t pack_bf16_pair(float a, float b) {
  return (uint32_t)f32_to_bf16(a) | ((uint32_t)f32_to_bf16(b) << 16);
}
template <int KMAX>
__device__ __forceinline__ float rms_row_sum(const uint16_t* __restrict__ x, const uint16_t* __restrict__ residual,
                                             const uint16_t* __restrict__ w, int K, int t,
                                             rms_u32x4 (&hv)[KMAX], rms_u32x4 (&wv)[KMAX],
                                             uint16_t* __restrict__ h_out) {
  // the weight row depends on nothing: its loads go out with the activations' (one round trip)
#pragma unroll
  for (int k = 0; k < KMAX; k++)
    if (k < K) wv[k] = *reinterpret_cast<const rms_u32x4*>(w + k * 2048 + t * 8);
  float ss = 0.0f;
#pragma unroll
  for (int k = 0; k < KMAX; k++) {
    if (k < K) {
      const int off = k * 2048 + t * 8;
      const rms_u32x4 xv = *reinterpret_cast<const rms_u32x4*>(x + off);
      rms_u32x4 rv = rms_u32x4{0, 0, 0, 0};
      if (residual) rv = *reinterpret_cast<const rms_u32x4*>(residual + off);
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const float a = round_bf16(bf16_to_f32((uint16_t)(xv[j] & 0xFFFFu)) + bf16_to_f32((uint16_t)(rv[j] & 0xFFFFu)));
        const float b = round_bf16(bf16_to_f32((uint16_t)(xv[j] >> 16)) + bf16_to_f32((uint16_t)(rv[j] >> 16)));
        ss = fmaf(a, a, ss);
        ss = fmaf(b, b, ss);
        hv[k][j] = pack_bf16_pair(a, b);
      }
      if (h_out) *reinterpret_cast<rms_u32x4*>(h_out + off) = hv[k];
    }
  }
  return ss;
}
// the four waves' sums red[0..3] -> 1 / rms
__device__ __forceinline__ float rms_inv(const float* red, int n, float eps) {
  const float tot = (red[0] + red[1]) + (red[2] + red[3]);
  return 1.0f / sqrtf(tot / (float)n + eps);
}
template <int KMAX>
__device__ __forceinline__ void rms_row_store(const rms_u32x4 (&hv)[KMAX], const rms_u32x4 (&wv)[KMAX], int K, int t,
                                              float inv, uint16_t* __restrict__ out) {
#pragma unroll
  for (int k = 0; k < KMAX; k++) {
    if (k < K) {
      rms_u32x4 o;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const float hl = bf16_to_f32((uint16_t)(hv[k][j] & 0xFFFFu)), hh = bf16_to_f32((uint16_t)(hv[k][j] >> 16));
        const float wl = bf16_to_f32((uint16_t)(wv[k][j] & 0xFFFFu)), wh = bf16_to_f32((uint16_t)(wv[k][j] >> 16));
        o[j] = pack_bf16_pair(round_bf16(wl * round_bf16(hl * inv)), round_bf16(wh * round_bf16(hh * inv)));
      }
      *reinterpret_cast<rms_u32x4*>(out + k * 2048 + t * 8) = o;
    }
  }
}
__device__ __forceinline__ float f16_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// ---------------------------------------------------------------- weight stream loads
// Expert weights are read once per call: their 16 B loads are marked non-temporal (streamed past
// the caches' reuse policy), which measured ~10% more HBM bandwidth on MI355X for a pure stream.
#ifndef MOE_NT_WEIGHTS
#define MOE_NT_WEIGHTS 1
#endif
__device__ __forceinline__ u32x4 load_stream16(const void* p) {
  if (MOE_NT_WEIGHTS) return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return *reinterpret_cast<const u32x4*>(p);
}

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
// The same table as fp16 values (128 KB), for decoders that keep it in LDS as fp16.
extern __device__ uint16_t g_codebook_f16[65536];

// Cooperative copy of the 64 KB table into LDS (blockDim threads, 16 B each), from the table of
// this translation unit or, in other ones, from its device address (codebook_device_table()).
// Copy of a table into LDS by THREADS threads (the block size): each thread issues its loads in
// batches of 8 x 16 B before storing them (one memory round trip per batch, 32 VGPRs).
template <int BYTES, int THREADS>
__device__ __forceinline__ void copy_table_lds(uint8_t* lds, const void* table) {
  const u32x4* src = reinterpret_cast<const u32x4*>(table);
  u32x4* dst = reinterpret_cast<u32x4*>(lds);
  constexpr int n = BYTES / 16;
  constexpr int per = (n + THREADS - 1) / THREADS;
  const int t = (int)threadIdx.x;
#pragma unroll
  for (int b = 0; b < per; b += 8) {
    u32x4 v[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const int i = (b + j) * THREADS + t;
      if (b + j < per && i < n) v[j] = src[i];
    }
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const int i = (b + j) * THREADS + t;
      if (b + j < per && i < n) dst[i] = v[j];
    }
  }
}
// Any block size (one 16 B load and store at a time).
template <int BYTES>
__device__ __forceinline__ void copy_table_lds_any(uint8_t* lds, const void* table) {
  const u32x4* src = reinterpret_cast<const u32x4*>(table);
  u32x4* dst = reinterpret_cast<u32x4*>(lds);
  for (int i = threadIdx.x; i < BYTES / 16; i += blockDim.x) dst[i] = src[i];
}
__device__ __forceinline__ void load_codebook_lds(uint8_t* lds, const uint8_t* table) {
  copy_table_lds_any<65536>(lds, table);
}
__device__ __forceinline__ void load_codebook_lds(uint8_t* lds) { load_codebook_lds(lds, g_codebook_e4m3); }
template <int THREADS>
__device__ __forceinline__ void load_codebook_lds_t(uint8_t* lds) { copy_table_lds<65536, THREADS>(lds, g_codebook_e4m3); }
template <int THREADS>
__device__ __forceinline__ void load_codebook16_lds(uint8_t* lds) {
  copy_table_lds<131072, THREADS>(lds, g_codebook_f16);
}

// ---------------------------------------------------------------- K4 word layout
// Word w of a tile with its circular predecessor p holds 8 codewords (A.1 direct form):
//   slot 0..2 straddle p and w, slot 3..7 lie inside w.
// Slot s sits at tile row (lane%4)*2 + (s&1) + (s&2)*4 and column lane/4 + (s&4)*2.

// ---------------------------------------------------------------- compile-time loop
// f(std::integral_constant<int, J>) for J = 0 .. N - 1, unrolled whatever the body's size.
template <int J, int N, class F>
__device__ __forceinline__ void static_for_from(F& f) {
  if constexpr (J < N) {
    f(std::integral_constant<int, J>{});
    static_for_from<J + 1, N>(f);
  }
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_from<0, N>(f);
}

// ---------------------------------------------------------------- K4 word -> fp16 MFMA operands
// The same word decode, producing the weights as fp16 pairs ready for a B fragment of
// v_mfma_f32_16x16x32_f16: q01 = (c0, c1), q23 = (c2, c3), q45 = (c4, c5), q67 = (c6, c7), where cs
// is the codeword of slot s.  Slots 0-3 are column lane/4 and slots 4-7 column lane/4 + 8 of the
// tile (rows as above), so each pair is two rows of one column.
//
// Arithmetic route, per codeword in half H of a register r (about 5 VALU ops):
//   t = (cw * 0xCBAC mod 2^16) << 16        one SDWA multiply reading the half directly
//   p = cw * 0x1FED + t = cw * 0xCBAC1FED   one v_mad_u32_u16 selecting the half
//   m = (p & 0x8FFF8FFF) ^ 0x3B603B60       one v_bitop3
//   f16(m.lo) + f16(m.hi)                   one SDWA fp16 add written into its half of the pair
// then E4M3 rounding by a round trip through the hardware fp8 conversions (two per pair).
// Table route: the E4M3 byte is read from LDS (one address op per codeword), two lookups meet in
// one register as [b0, 0, b1, 0], a byte permute joins two such pairs and two conversions widen
// them to fp16.  The split between routes is NALU arithmetic pairs per word (0..4), taken in the
// order q67, q23, q45, q01.
template <int H>
__device__ __forceinline__ uint32_t mcg_product_half(uint32_t r, uint32_t k_hi, uint32_t k_lo) {
  uint32_t t, p;
  asm volatile("v_mul_u32_u24_sdwa %0, %1, %2 dst_sel:WORD_1 dst_unused:UNUSED_PAD src0_sel:WORD_%3 src1_sel:DWORD"
               : "=v"(t)
               : "v"(r), "s"(k_hi), "n"(H));
  asm volatile("v_mad_u32_u16 %0, %1, %2, %3 op_sel:[%4,0,0,0]" : "=v"(p) : "v"(r), "s"(k_lo), "v"(t), "n"(H));
  return p;
}
// f16 pair (cw_x, cw_y) for codewords in half HX of rx and half HY of ry, before E4M3 rounding
template <int HX, int HY>
__device__ __forceinline__ uint32_t halves_sum_pair(uint32_t rx, uint32_t ry) {
  const uint32_t k_hi = 0xCBACu, k_lo = 0x1FEDu;
  const uint32_t mx = (mcg_product_half<HX>(rx, k_hi, k_lo) & 0x8FFF8FFFu) ^ 0x3B603B60u;
  const uint32_t my = (mcg_product_half<HY>(ry, k_hi, k_lo) & 0x8FFF8FFFu) ^ 0x3B603B60u;
  uint32_t s;
  asm volatile("v_add_f16_sdwa %0, %1, %1 dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:WORD_0 src1_sel:WORD_1"
               : "=v"(s)
               : "v"(mx));
  asm volatile("v_add_f16_sdwa %0, %1, %1 dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:WORD_0 src1_sel:WORD_1"
               : "+v"(s)
               : "v"(my));
  return s;
}
// An unconstrained register value: the fp8 conversions below write one half of their destination
// and keep the other, so the first one into a fresh register is given this instead of a zero
// (which would cost a copy).
__device__ __forceinline__ uint32_t scratch_reg() {
  uint32_t r;
  asm volatile("" : "=v"(r));
  return r;
}
__device__ __forceinline__ i16x2 as_i16x2(uint32_t v) { return __builtin_bit_cast(i16x2, v); }
// E4M3 rounding of one or two f16 pairs (round trip through fp8)
__device__ __forceinline__ f16x2 round_e4m3_pair(uint32_t s) {
  const uint32_t e = __builtin_bit_cast(
      uint32_t, __builtin_amdgcn_cvt_scalef32_pk_fp8_f16(as_i16x2(scratch_reg()), __builtin_bit_cast(f16x2, s), 1.0f, false));
  return __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(e, 1.0f, false);
}
__device__ __forceinline__ void round_e4m3_two(uint32_t sa, uint32_t sb, f16x2& fa, f16x2& fb) {
  i16x2 e = __builtin_amdgcn_cvt_scalef32_pk_fp8_f16(as_i16x2(scratch_reg()), __builtin_bit_cast(f16x2, sa), 1.0f, false);
  e = __builtin_amdgcn_cvt_scalef32_pk_fp8_f16(e, __builtin_bit_cast(f16x2, sb), 1.0f, true);
  fa = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(__builtin_bit_cast(uint32_t, e), 1.0f, false);
  fb = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(__builtin_bit_cast(uint32_t, e), 1.0f, true);
}
template <int H>
__device__ __forceinline__ uint32_t half_of(uint32_t r) {
  return H ? (r >> 16) : (r & 0xFFFFu);
}
// [tab[x], 0, tab[y], 0]
template <int HX, int HY>
__device__ __forceinline__ uint32_t lds_pair_bytes(const uint8_t* tab, uint32_t rx, uint32_t ry) {
  typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
  u16x2 r;
  r.x = tab[half_of<HX>(rx)];
  r.y = tab[half_of<HY>(ry)];
  return __builtin_bit_cast(uint32_t, r);
}
__device__ __forceinline__ void widen_two(uint32_t qa, uint32_t qb, f16x2& fa, f16x2& fb) {
  const uint32_t e = __builtin_amdgcn_perm(qb, qa, 0x06040200u);  // [qa.b0, qa.b2, qb.b0, qb.b2]
  fa = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(e, 1.0f, false);
  fb = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(e, 1.0f, true);
}
__device__ __forceinline__ f16x2 widen_one(uint32_t q) {
  return __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(__builtin_amdgcn_perm(q, q, 0x00000200u), 1.0f, false);
}

template <int NALU>
__device__ __forceinline__ void decode_word_f16(uint32_t w, uint32_t p, const uint8_t* tab, f16x2& q01, f16x2& q23,
                                                f16x2& q45, f16x2& q67) {
  const uint32_t a4 = __builtin_amdgcn_alignbit(p, w, 4);    // c6 | c2 << 16
  const uint32_t a8 = __builtin_amdgcn_alignbit(p, w, 8);    // c5 | c1 << 16
  const uint32_t a12 = __builtin_amdgcn_alignbit(p, w, 12);  // c4 | c0 << 16
  // pairs: q01 = (a12.hi, a8.hi), q23 = (a4.hi, w.hi), q45 = (a12.lo, a8.lo), q67 = (a4.lo, w.lo)
  if (NALU == 1) q67 = round_e4m3_pair(halves_sum_pair<0, 0>(a4, w));
  if (NALU >= 2) round_e4m3_two(halves_sum_pair<0, 0>(a4, w), halves_sum_pair<1, 1>(a4, w), q67, q23);
  if (NALU == 3) q45 = round_e4m3_pair(halves_sum_pair<0, 0>(a12, a8));
  if (NALU == 4) round_e4m3_two(halves_sum_pair<0, 0>(a12, a8), halves_sum_pair<1, 1>(a12, a8), q45, q01);
  if (NALU == 0) {
    widen_two(lds_pair_bytes<0, 0>(tab, a4, w), lds_pair_bytes<1, 1>(tab, a4, w), q67, q23);
    widen_two(lds_pair_bytes<0, 0>(tab, a12, a8), lds_pair_bytes<1, 1>(tab, a12, a8), q45, q01);
  } else if (NALU == 1) {
    widen_two(lds_pair_bytes<1, 1>(tab, a4, w), lds_pair_bytes<0, 0>(tab, a12, a8), q23, q45);
    q01 = widen_one(lds_pair_bytes<1, 1>(tab, a12, a8));
  } else if (NALU == 2) {
    widen_two(lds_pair_bytes<0, 0>(tab, a12, a8), lds_pair_bytes<1, 1>(tab, a12, a8), q45, q01);
  } else if (NALU == 3) {
    q01 = widen_one(lds_pair_bytes<1, 1>(tab, a12, a8));
  }
}

// ---------------------------------------------------------------- K4 piece -> fp16 MFMA operands
// Two consecutive words of one lane (w0's predecessor is `prior0`) decoded together, NE arithmetic
// pairs in w0 and NO in w1.  Every VALU result is needed about 16 clocks after issue, so the
// arithmetic route runs stage by stage over all of the two words' arithmetic codewords (ordered
// asm statements): a wave then always has independent work to issue.  q[i][j] receives word i's
// pair j as in decode_word_f16.
namespace piece_detail {
// pair kinds in arithmetic preference order: 0 = (c6,c7) = (a4.lo, w.lo), 1 = (c2,c3) = (a4.hi, w.hi),
// 2 = (c4,c5) = (a12.lo, a8.lo), 3 = (c0,c1) = (a12.hi, a8.hi); kind k fills q[i][kOut[k]]
constexpr int kOut[4] = {3, 1, 2, 0};
}  // namespace piece_detail

template <int H>
__device__ __forceinline__ uint32_t mul_hi16_shifted(uint32_t r, uint32_t k_hi) {
  uint32_t t;
  asm volatile("v_mul_u32_u24_sdwa %0, %1, %2 dst_sel:WORD_1 dst_unused:UNUSED_PAD src0_sel:WORD_%3 src1_sel:DWORD"
               : "=v"(t)
               : "v"(r), "s"(k_hi), "n"(H));
  return t;
}
template <int H>
__device__ __forceinline__ uint32_t mad_lo16(uint32_t r, uint32_t k_lo, uint32_t t) {
  uint32_t p;
  asm volatile("v_mad_u32_u16 %0, %1, %2, %3 op_sel:[%4,0,0,0]" : "=v"(p) : "v"(r), "s"(k_lo), "v"(t), "n"(H));
  return p;
}
__device__ __forceinline__ uint32_t add_halves_lo(uint32_t m) {
  uint32_t s;
  asm volatile("v_add_f16_sdwa %0, %1, %1 dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:WORD_0 src1_sel:WORD_1"
               : "=v"(s)
               : "v"(m));
  return s;
}
__device__ __forceinline__ void add_halves_hi(uint32_t& s, uint32_t m) {
  asm volatile("v_add_f16_sdwa %0, %1, %1 dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:WORD_0 src1_sel:WORD_1"
               : "+v"(s)
               : "v"(m));
}

// fp16 code table (128 KB of LDS, entry s at byte 2s): the byte offset of the codeword in half H of r
// is one SDWA shift, and two lookups meet in one register with a byte permute -- no fp8 widening.
template <int H>
__device__ __forceinline__ uint32_t tab16_off(uint32_t r) {
  uint32_t o;
  asm volatile("v_lshlrev_b32_sdwa %0, 1, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:WORD_%2"
               : "=v"(o)
               : "v"(r), "n"(H));
  return o;
}
__device__ __forceinline__ uint16_t tab16_at(const uint8_t* tab, uint32_t off) {
  return *reinterpret_cast<const uint16_t*>(tab + off);
}

// TAB16: `tab` is the fp16 table (else the 64 KB E4M3 byte table).
template <int NE, int NO, bool TAB16 = false>
__device__ __forceinline__ void decode_pair_words_f16(uint32_t w0, uint32_t w1, uint32_t prior0, const uint8_t* tab,
                                                      f16x2 (&q)[2][4]) {
  using piece_detail::kOut;
  const uint32_t w[2] = {w0, w1};
  const uint32_t pr[2] = {prior0, w0};
  uint32_t a4[2], a8[2], a12[2];
#pragma unroll
  for (int i = 0; i < 2; i++) {
    a4[i] = __builtin_amdgcn_alignbit(pr[i], w[i], 4);
    a8[i] = __builtin_amdgcn_alignbit(pr[i], w[i], 8);
    a12[i] = __builtin_amdgcn_alignbit(pr[i], w[i], 12);
  }
  auto nalu = [](int i) { return (i & 1) ? NO : NE; };
  auto xr = [&](int i, int k) { return (k & 2) ? a12[i] : a4[i]; };
  auto yr = [&](int i, int k) { return (k & 2) ? a8[i] : w[i]; };
  const uint32_t k_hi = 0xCBACu, k_lo = 0x1FEDu;

  // ---- table route for the pairs with k >= nalu(word): the byte lookups are issued first, and the
  // scheduling fences keep their use after the arithmetic route, which hides their latency
  uint32_t bx[2][4], by[2][4];
#pragma unroll
  for (int k = 0; k < 4; k++)
#pragma unroll
    for (int i = 0; i < 2; i++)
      if (k >= nalu(i)) {
        if (TAB16) {
          bx[i][k] = tab16_at(tab, (k & 1) ? tab16_off<1>(xr(i, k)) : tab16_off<0>(xr(i, k)));
          by[i][k] = tab16_at(tab, (k & 1) ? tab16_off<1>(yr(i, k)) : tab16_off<0>(yr(i, k)));
        } else {
          bx[i][k] = tab[(k & 1) ? (xr(i, k) >> 16) : (xr(i, k) & 0xFFFFu)];
          by[i][k] = tab[(k & 1) ? (yr(i, k) >> 16) : (yr(i, k) & 0xFFFFu)];
        }
      }
  __builtin_amdgcn_sched_barrier(0);

  // ---- arithmetic route, stage by stage over all (word, kind) pairs with k < nalu(word)
  uint32_t tx[2][4], ty[2][4], sm[2][4];
#pragma unroll
  for (int k = 0; k < 4; k++)
#pragma unroll
    for (int i = 0; i < 2; i++)
      if (k < nalu(i)) {
        if (k & 1) {
          tx[i][k] = mul_hi16_shifted<1>(xr(i, k), k_hi);
          ty[i][k] = mul_hi16_shifted<1>(yr(i, k), k_hi);
        } else {
          tx[i][k] = mul_hi16_shifted<0>(xr(i, k), k_hi);
          ty[i][k] = mul_hi16_shifted<0>(yr(i, k), k_hi);
        }
      }
#pragma unroll
  for (int k = 0; k < 4; k++)
#pragma unroll
    for (int i = 0; i < 2; i++)
      if (k < nalu(i)) {
        if (k & 1) {
          tx[i][k] = mad_lo16<1>(xr(i, k), k_lo, tx[i][k]);
          ty[i][k] = mad_lo16<1>(yr(i, k), k_lo, ty[i][k]);
        } else {
          tx[i][k] = mad_lo16<0>(xr(i, k), k_lo, tx[i][k]);
          ty[i][k] = mad_lo16<0>(yr(i, k), k_lo, ty[i][k]);
        }
      }
#pragma unroll
  for (int k = 0; k < 4; k++)
#pragma unroll
    for (int i = 0; i < 2; i++)
      if (k < nalu(i)) {
        tx[i][k] = (tx[i][k] & 0x8FFF8FFFu) ^ 0x3B603B60u;
        ty[i][k] = (ty[i][k] & 0x8FFF8FFFu) ^ 0x3B603B60u;
      }
#pragma unroll
  for (int k = 0; k < 4; k++)
#pragma unroll
    for (int i = 0; i < 2; i++)
      if (k < nalu(i)) sm[i][k] = add_halves_lo(tx[i][k]);
#pragma unroll
  for (int k = 0; k < 4; k++)
#pragma unroll
    for (int i = 0; i < 2; i++)
      if (k < nalu(i)) add_halves_hi(sm[i][k], ty[i][k]);
  // E4M3 rounding: consecutive arithmetic pairs share one fp8 register
  {
    int pend_i = -1, pend_k = -1;
#pragma unroll
    for (int k = 0; k < 4; k++)
#pragma unroll
      for (int i = 0; i < 2; i++)
        if (k < nalu(i)) {
          if (pend_i < 0) {
            pend_i = i;
            pend_k = k;
          } else {
            round_e4m3_two(sm[pend_i][pend_k], sm[i][k], q[pend_i][kOut[pend_k]], q[i][kOut[k]]);
            pend_i = -1;
          }
        }
    if (pend_i >= 0) q[pend_i][kOut[pend_k]] = round_e4m3_pair(sm[pend_i][pend_k]);
  }

  __builtin_amdgcn_sched_barrier(0);

  // ---- table route, fp16 entries: one permute per pair
  if (TAB16) {
#pragma unroll
    for (int k = 0; k < 4; k++)
#pragma unroll
      for (int i = 0; i < 2; i++)
        if (k >= nalu(i)) q[i][kOut[k]] = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(by[i][k], bx[i][k], 0x05040100u));
    return;
  }
  // ---- table route: [b_x, 0, b_y, 0] per pair, two pairs joined per permute, widened to fp16
  {
    uint32_t lb[2][4];
#pragma unroll
    for (int k = 0; k < 4; k++)
#pragma unroll
      for (int i = 0; i < 2; i++)
        if (k >= nalu(i)) lb[i][k] = bx[i][k] | (by[i][k] << 16);
    int pend_i = -1, pend_k = -1;
#pragma unroll
    for (int k = 0; k < 4; k++)
#pragma unroll
      for (int i = 0; i < 2; i++)
        if (k >= nalu(i)) {
          if (pend_i < 0) {
            pend_i = i;
            pend_k = k;
          } else {
            widen_two(lb[pend_i][pend_k], lb[i][k], q[pend_i][kOut[pend_k]], q[i][kOut[k]]);
            pend_i = -1;
          }
        }
    if (pend_i >= 0) q[pend_i][kOut[pend_k]] = widen_one(lb[pend_i][pend_k]);
  }
}

// ---------------------------------------------------------------- K3 piece -> fp16 MFMA operands
// A K3 tile is 24 words; lane piece m holds words 3m .. 3m + 2, i.e. the tile's codewords
// 32m .. 32m + 31.  Codeword i of a K-bit tile is the 16 bits of the circular MSB-first tile stream
// that end after its symbol, at bit (i + 1) K (exlr8/trellis.py:78-102, the generic window of
// exlr8/metal/trellis.metal:25-40).  With the piece's stream S = [predecessor word, words 0..2]
// (MSB first) codeword j of the piece ends at bit 3j + 35 of S: one funnel shift puts it in the
// low half of a register.  Its tile position is that of the K4 decoder's word j / 8, slot j % 8.
template <int J>
__device__ __forceinline__ uint32_t k3_window(const uint32_t (&S)[4]) {
  constexpr int E = 3 * J + 35, ws = (E - 16) / 32, we = (E - 1) / 32;
  if constexpr (ws == we) {
    constexpr int sh = 32 * we + 32 - E;  // 0 .. 16
    if constexpr (sh == 0) return S[we];
    else return S[we] >> sh;
  } else {
    return __builtin_amdgcn_alignbit(S[ws], S[we], 32 * ws + 64 - E);
  }
}
// q[i][p] = (c_2p, c_2p+1) of piece words R0 + i (i = 0, 1), as decode_pair_words_f16 gives them;
// the first NE (word R0) / NO (word R0 + 1) pairs by the arithmetic route, the rest from the
// E4M3 code table.
template <int NE, int NO, int R0>
__device__ __forceinline__ void decode_k3_pair_words(const uint32_t (&S)[4], const uint8_t* tab, f16x2 (&q)[2][4]) {
  uint32_t c[2][8];
  static_for<16>([&](auto jc) {
    constexpr int j = decltype(jc)::value;
    c[j / 8][j % 8] = k3_window<8 * R0 + j>(S);
  });
  auto nalu = [](int i) { return i ? NO : NE; };
  // table route first (its loads are then in flight during the arithmetic)
  uint32_t lb[2][4];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int p = 0; p < 4; p++)
      if (p >= nalu(i)) lb[i][p] = lds_pair_bytes<0, 0>(tab, c[i][2 * p], c[i][2 * p + 1]);
  uint32_t sm[2][4];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int p = 0; p < 4; p++)
      if (p < nalu(i)) sm[i][p] = halves_sum_pair<0, 0>(c[i][2 * p], c[i][2 * p + 1]);
  // E4M3 rounding, two arithmetic pairs per fp8 register; the table pairs widened two at a time
  {
    int pi = -1, pp = -1;
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
      for (int p = 0; p < 4; p++)
        if (p < nalu(i)) {
          if (pi < 0) {
            pi = i;
            pp = p;
          } else {
            round_e4m3_two(sm[pi][pp], sm[i][p], q[pi][pp], q[i][p]);
            pi = -1;
          }
        }
    if (pi >= 0) q[pi][pp] = round_e4m3_pair(sm[pi][pp]);
  }
  {
    int pi = -1, pp = -1;
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
      for (int p = 0; p < 4; p++)
        if (p >= nalu(i)) {
          if (pi < 0) {
            pi = i;
            pp = p;
          } else {
            widen_two(lb[pi][pp], lb[i][p], q[pi][pp], q[i][p]);
            pi = -1;
          }
        }
    if (pi >= 0) q[pi][pp] = widen_one(lb[pi][pp]);
  }
}

// The same decode as decode_pair_words_f16 with the fp16 table, written without scheduling fences:
// each table pair is two 16-bit LDS loads into the halves of one register, and the compiler
// interleaves the table and arithmetic routes of the two words freely.  Measured on MI355X in a
// register-fed quad loop: 14.0 codewords/clk/CU with NE = 1, NO = 2 (the fenced form: 12.0 at 2/2).
template <int NE, int NO>
__device__ __forceinline__ void decode_pair_words_h16(uint32_t w0, uint32_t w1, uint32_t prior0, const uint8_t* tab,
                                                      f16x2 (&q)[2][4]) {
  using piece_detail::kOut;
  const uint32_t w[2] = {w0, w1};
  const uint32_t pr[2] = {prior0, w0};
  uint32_t a4[2], a8[2], a12[2];
#pragma unroll
  for (int i = 0; i < 2; i++) {
    a4[i] = __builtin_amdgcn_alignbit(pr[i], w[i], 4);
    a8[i] = __builtin_amdgcn_alignbit(pr[i], w[i], 8);
    a12[i] = __builtin_amdgcn_alignbit(pr[i], w[i], 12);
  }
  auto nalu = [](int i) { return (i & 1) ? NO : NE; };
  auto xr = [&](int i, int k) { return (k & 2) ? a12[i] : a4[i]; };
  auto yr = [&](int i, int k) { return (k & 2) ? a8[i] : w[i]; };
#pragma unroll
  for (int k = 0; k < 4; k++)
#pragma unroll
    for (int i = 0; i < 2; i++)
      if (k >= nalu(i)) {
        const uint32_t ox = (k & 1) ? tab16_off<1>(xr(i, k)) : tab16_off<0>(xr(i, k));
        const uint32_t oy = (k & 1) ? tab16_off<1>(yr(i, k)) : tab16_off<0>(yr(i, k));
        f16x2 v;
        v.x = *reinterpret_cast<const _Float16*>(tab + ox);
        v.y = *reinterpret_cast<const _Float16*>(tab + oy);
        q[i][kOut[k]] = v;
      }
  const uint32_t k_hi = 0xCBACu, k_lo = 0x1FEDu;
  uint32_t sm[2][4];
#pragma unroll
  for (int k = 0; k < 4; k++)
#pragma unroll
    for (int i = 0; i < 2; i++)
      if (k < nalu(i)) {
        uint32_t tx, ty;
        if (k & 1) {
          tx = mad_lo16<1>(xr(i, k), k_lo, mul_hi16_shifted<1>(xr(i, k), k_hi));
          ty = mad_lo16<1>(yr(i, k), k_lo, mul_hi16_shifted<1>(yr(i, k), k_hi));
        } else {
          tx = mad_lo16<0>(xr(i, k), k_lo, mul_hi16_shifted<0>(xr(i, k), k_hi));
          ty = mad_lo16<0>(yr(i, k), k_lo, mul_hi16_shifted<0>(yr(i, k), k_hi));
        }
        tx = (tx & 0x8FFF8FFFu) ^ 0x3B603B60u;
        ty = (ty & 0x8FFF8FFFu) ^ 0x3B603B60u;
        sm[i][k] = add_halves_lo(tx);
        add_halves_hi(sm[i][k], ty);
      }
  int pend_i = -1, pend_k = -1;
#pragma unroll
  for (int k = 0; k < 4; k++)
#pragma unroll
    for (int i = 0; i < 2; i++)
      if (k < nalu(i)) {
        if (pend_i < 0) {
          pend_i = i;
          pend_k = k;
        } else {
          round_e4m3_two(sm[pend_i][pend_k], sm[i][k], q[pend_i][kOut[pend_k]], q[i][kOut[k]]);
          pend_i = -1;
        }
      }
  if (pend_i >= 0) q[pend_i][kOut[pend_k]] = round_e4m3_pair(sm[pend_i][pend_k]);
}

// ---------------------------------------------------------------- K4 storage and MFMA fragments
// Chunk of 8 tiles (256 K bytes at K bits: 1 KB at K4) of expert e, output block ob (128 columns),
// input tile tk of a packed projection with `it` input tiles and `obs` output blocks (side 1:
// gate/up order, side 2: down order); chunk_offset is its K4 byte offset
__device__ __forceinline__ uint64_t chunk_index(int side, uint64_t e, uint32_t ob, uint32_t tk, uint32_t it,
                                                uint32_t obs) {
  if (side == 2) return (((e * (it / 8u) + tk / 8u) * obs + ob) * 8u + tk % 8u);
  return ((e * obs + ob) * it + tk);
}
__device__ __forceinline__ uint64_t chunk_offset(int side, uint64_t e, uint32_t ob, uint32_t tk, uint32_t it,
                                                 uint32_t obs) {
  return chunk_index(side, e, ob, tk, it, obs) << 10;
}

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// four fp16 pairs -> one 8-wide MFMA operand
__device__ __forceinline__ f16x8 frag(f16x2 a, f16x2 b, f16x2 c, f16x2 d) {
  typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
  const f16x4 ab = __builtin_shufflevector(a, b, 0, 1, 2, 3), cd = __builtin_shufflevector(c, d, 0, 1, 2, 3);
  return __builtin_shufflevector(ab, cd, 0, 1, 2, 3, 4, 5, 6, 7);
}

// Accumulator guard for MFMAs mixed with the piece decoder's inline asm.  An MFMA keeps reading its
// accumulator input (SrcC) for several passes after issue; the compiler keeps its own VALU writes
// out of that window (and places the wait states an MFMA result needs before a VALU reads it), but
// it cannot see that an inline asm statement is a VALU write, and the register allocator may hand
// an asm statement a register that an MFMA issued just before still reads as SrcC.  Called with the
// results of each group of MFMAs right after issue: 16 wait states (longer than the SrcC read and
// the result latency of every fp16 MFMA used here), ordered after the MFMAs by the data dependence
// and before every later asm statement (asm volatile statements keep their order).
__device__ __forceinline__ void mfma_acc_guard(f32x4& a, f32x4& b) { asm volatile("s_nop 15" : "+v"(a), "+v"(b)); }
template <int N>
__device__ __forceinline__ void mfma_acc_guard(f32x4 (&acc)[N][2]) {
  static_assert(N == 1 || N == 2 || N == 4 || N == 8, "guard sizes");
  if constexpr (N == 1) {
    asm volatile("s_nop 15" : "+v"(acc[0][0]), "+v"(acc[0][1]));
  } else if constexpr (N == 2) {
    asm volatile("s_nop 15" : "+v"(acc[0][0]), "+v"(acc[0][1]), "+v"(acc[1][0]), "+v"(acc[1][1]));
  } else if constexpr (N == 4) {
    asm volatile("s_nop 15"
                 : "+v"(acc[0][0]), "+v"(acc[0][1]), "+v"(acc[1][0]), "+v"(acc[1][1]), "+v"(acc[2][0]),
                   "+v"(acc[2][1]), "+v"(acc[3][0]), "+v"(acc[3][1]));
  } else {
    asm volatile("s_nop 15"
                 : "+v"(acc[0][0]), "+v"(acc[0][1]), "+v"(acc[1][0]), "+v"(acc[1][1]), "+v"(acc[2][0]),
                   "+v"(acc[2][1]), "+v"(acc[3][0]), "+v"(acc[3][1]), "+v"(acc[4][0]), "+v"(acc[4][1]),
                   "+v"(acc[5][0]), "+v"(acc[5][1]), "+v"(acc[6][0]), "+v"(acc[6][1]), "+v"(acc[7][0]),
                   "+v"(acc[7][1]));
  }
}

// A operand of the K4 fp16 MFMAs: row r of a 16-row input tile -> (row half rh, position j inside
// the 8-wide k group), matching the B fragments decode_pair_words_f16 builds from a tile's words
__device__ __forceinline__ int a_rh(int r) { return (r >> 2) & 1; }
__device__ __forceinline__ int a_j(int r) { return 4 * ((r >> 1) & 1) + 2 * ((r >> 3) & 1) + (r & 1); }

// ---------------------------------------------------------------- wave-level H128
// 128 values held as 2 per lane (element i = 2*lane + j).  Normalised Sylvester order;
// the butterfly order differs from the reference's numpy loop only in float rounding.
// Lane bits 0..3 exchange inside a 16-lane row through DPP; a lane then computes own + partner
// (low half) or own - partner (high half): the high half's value is the negated butterfly
// (x - y = -(y - x) in round-to-nearest), and the sign is put back by the final scale.  Lane bits
// 4 and 5 use v_permlane16_swap / v_permlane32_swap, which place both values of a pair in one
// lane.  No LDS traffic; the values equal those of the lane-shuffle form bit for bit (a zero
// result is +0, as there).
template <int CTRL>
__device__ __forceinline__ float dpp_mov_f32(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
template <int K, int CTRL>
__device__ __forceinline__ void h128_row_stage(float& v0, float& v1, int lane) {
  const float s = __builtin_bit_cast(float, 0x3f800000 | ((lane << (31 - K)) & (int)0x80000000));
  v0 = __builtin_fmaf(dpp_mov_f32<CTRL>(v0), s, v0);
  v1 = __builtin_fmaf(dpp_mov_f32<CTRL>(v1), s, v1);
}
// v_permlane16_swap (odd 16-lane rows of a <-> even rows of b) and v_permlane32_swap (upper 32
// lanes of a <-> lower 32 lanes of b) on float pairs
__device__ __forceinline__ void swap16_f32(float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b),
                                                  false, false);
  const uint32_t r0 = r[0], r1 = r[1];
  a = __builtin_bit_cast(float, r0);
  b = __builtin_bit_cast(float, r1);
}
__device__ __forceinline__ void swap32_f32(float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b),
                                                  false, false);
  const uint32_t r0 = r[0], r1 = r[1];
  a = __builtin_bit_cast(float, r0);
  b = __builtin_bit_cast(float, r1);
}
__device__ __forceinline__ void hadamard128_wave(float& v0, float& v1) {
  float a = v0 + v1, b = v0 - v1;
  v0 = a;
  v1 = b;
  const int lane = threadIdx.x & 63;
  h128_row_stage<0, 0xB1>(v0, v1, lane);  // quad_perm [1,0,3,2]: lane ^ 1
  h128_row_stage<1, 0x4E>(v0, v1, lane);  // quad_perm [2,3,0,1]: lane ^ 2
  {
    // lane ^ 4: row_half_mirror (i -> 7 - i in each 8 lanes), then quad_perm [3,2,1,0]
    const float s = __builtin_bit_cast(float, 0x3f800000 | ((lane << 29) & (int)0x80000000));
    v0 = __builtin_fmaf(dpp_mov_f32<0x1B>(dpp_mov_f32<0x141>(v0)), s, v0);
    v1 = __builtin_fmaf(dpp_mov_f32<0x1B>(dpp_mov_f32<0x141>(v1)), s, v1);
  }
  h128_row_stage<3, 0x128>(v0, v1, lane);  // row_ror:8: lane ^ 8
  // lane ^ 16 and lane ^ 32.  After the first swap, lanes of row 0 hold rows 0 and 1 of v0 and
  // lanes of row 1 hold rows 0 and 1 of v1 (rows 2, 3 likewise); the pair sums and differences
  // come out in the same arrangement, so one 32-lane swap pairs rows 0 and 2 (1 and 3), and two
  // swaps in reverse order restore the layout.
  swap16_f32(v0, v1);
  a = v0 + v1;
  b = v0 - v1;
  swap32_f32(a, b);
  v0 = a + b;
  v1 = a - b;
  swap32_f32(v0, v1);
  swap16_f32(v0, v1);
  // sign of the row stages: -1 where lane bits 0..3 hold an odd number of ones
  const int sg = (__builtin_popcount(lane & 15) & 1) << 31;
  const float sc = __builtin_bit_cast(float, __builtin_bit_cast(int, kInvSqrt128) ^ sg);
  // fma with +0: a zero product comes out as +0 whatever the tracked sign
  v0 = __builtin_fmaf(v0, sc, 0.0f);
  v1 = __builtin_fmaf(v1, sc, 0.0f);
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

// ---------------------------------------------------------------- MXFP4 (e2m1 codes, e8m0 scales)
// 8 scaled fp4 codes of a 32-bit word -> 8 floats, accumulated against x[0..7]
__device__ __forceinline__ float dot8_fp4(uint32_t w, float scale, const float* x, float acc) {
  const f32x2 v0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, scale, 0);
  const f32x2 v1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, scale, 1);
  const f32x2 v2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, scale, 2);
  const f32x2 v3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, scale, 3);
  acc = fmaf(x[0], v0.x, acc);
  acc = fmaf(x[1], v0.y, acc);
  acc = fmaf(x[2], v1.x, acc);
  acc = fmaf(x[3], v1.y, acc);
  acc = fmaf(x[4], v2.x, acc);
  acc = fmaf(x[5], v2.y, acc);
  acc = fmaf(x[6], v3.x, acc);
  acc = fmaf(x[7], v3.y, acc);
  return acc;
}

// e8m0 block scale 2^(s-127) as a float (s = 0: 2^-127, a denormal)
__device__ __forceinline__ float e8m0_to_f32(uint32_t s) { return __uint_as_float(s == 0 ? 0x00400000u : s << 23); }

// ---------------------------------------------------------------- small wave helpers
__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave_id_in_block() { return threadIdx.x >> 6; }
// The same index as a wave-uniform (scalar) value, so that everything derived from it -- work
// ranges, loop bounds, segment ids -- lives in scalar registers and loops stay uniform.
// Publication of write-through stores to other CUs: wait until every earlier store of this wave
// is acknowledged (gfx9 counts stores in vmcnt; a workgroup-scope release emits no wait), then
// act as a compiler barrier.  Used before the counter atomic that hands the stored data over.
__device__ __forceinline__ void release_stores() {
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0), expcnt and lgkmcnt not waited on
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
}

// A value every lane holds equally (e.g. read from LDS), made wave-uniform for the compiler.
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ int wave_id_uniform() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

}  // namespace moe
