/*
 * CPU oracle for the exlr8 MoE expert path -- TEST INFRASTRUCTURE ONLY.
 *
 * This file restates, in plain C, the semantics of the reference operators that the
 * MI355X kernels replace.  It is used by tests/ (parity checker), by
 * __graft_entry__.smoke() (checker) and by bench.py's cpu_baseline leg (the timed CPU
 * port of the reference's --no-optimize operator chain).  Nothing in the product
 * (mlxlr8_amd/) may load it.
 *
 * Every function names the reference lines it follows (paths relative to the
 * reference repository root).  How each function is pinned:
 *   orc_round_e4m3        trellis.py:22-40      ties-to-even midpoints, +-448 saturation,
 *                                               signed zero (tests/test_trellis.py:48-57)
 *   orc_codebook          trellis.py:43-50      cb[0]=1.875 (tests/test_trellis.py:63);
 *                                               all 65536 entries against an independent
 *                                               integer-rounding restatement
 *                                               (tests/test_fast_decode.py:43-53)
 *   orc_decode_trellis    trellis.py:78-102     brute force: random k-bit symbols (k = 2, 3, 4) packed MSB-first
 *                                               (ponyexl3/ref/trellis.py:13-49), placed by the
 *                                               tensor-core map (ponyexl3/ref/perm.py:8-26)
 *                                               in both storage orders (trellis.metal:44-48)
 *   orc_hadamard128       trellis.py:67-75      explicit Sylvester matrix, self-inverse
 *   orc_route             fast_router.metal:1-42, model.py:111-132
 *                                               argsort-stable restatement and the special
 *                                               cases of tests/test_fast_router.py:14-33
 *   orc_router_logits     dense.py:158-159      float64 dot product (textbook)
 *   orc_k4_linear         trellis.py:172-196    dequantised public matrix times x in float64
 *   orc_mxfp4_linear      joined_gather_order_common.metal:29-45, joined_gather_order.metal:19-21
 *                                               e2m1/e8m0 closed forms times x in float64
 *   orc_swiglu_bf16       fast_decode_common.metal:40-49 (MLX-internal bf16 rounding of exp
 *                                               inside sigmoid is parity unpinned: MLX absent)
 *   orc_k4_moe / orc_mxfp4_moe  model.py:406-418, fast_decode_finish_fused.metal:24-63
 *   orc_residual_rmsnorm  residual_rms.metal:18-90 (rms_looped), model.py:376-384
 *   orc_segment_table     fast_prefill.py:19-46  brute-force counting on small inputs
 *   orc_mx_quantize_row / orc_k4_to_mxfp4  joined_mxfp4.py:12-47 (encode)
 *                                               orientation, fold and layout: the reference's
 *                                               tests/test_joined_mxfp4.py:44-58 structure
 *                                               (decode, x factor per input channel, quantise
 *                                               the transpose, gate||up rows); quantiser: every
 *                                               element within half an E2M1 step of its value,
 *                                               exact groups reproduced, zero and saturating
 *                                               groups.  The scale and rounding choice of MLX's
 *                                               mx.quantize(mode="mxfp4") is PARITY UNPINNED
 *                                               (MLX absent): this restates the OCP MX v1.0
 *                                               conversion (shared exponent floor(log2 amax) - 2,
 *                                               elements round-to-nearest-even, saturating at 6)
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------- scalar formats ---------------- */

static float f16_to_f32(uint16_t h) {
  uint32_t s = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1Fu, m = h & 0x3FFu, u;
  if (e == 0) {
    if (m == 0) { u = s; }
    else {  /* subnormal: m * 2^-24 */
      float v = (float)m * 5.9604644775390625e-08f;
      memcpy(&u, &v, 4); u |= s;
    }
  } else if (e == 31) { u = s | 0x7F800000u | (m << 13); }
  else { u = s | ((e + 112u) << 23) | (m << 13); }
  float f; memcpy(&f, &u, 4); return f;
}

/* float32 -> float16, round to nearest even (used only on exactly representable
   sums of two halves, and on fp16 side vectors). */
static uint16_t f32_to_f16(float f) {
  uint32_t u; memcpy(&u, &f, 4);
  uint32_t s = (u >> 16) & 0x8000u;
  uint32_t a = u & 0x7FFFFFFFu;
  if (a >= 0x7F800000u) return (uint16_t)(s | 0x7C00u | (a > 0x7F800000u ? 0x200u : 0));
  if (a >= 0x477FF000u) return (uint16_t)(s | 0x7C00u);           /* rounds to inf */
  if (a < 0x38800000u) {                                           /* subnormal / zero */
    float v; memcpy(&v, &a, 4);
    float q = v * 16777216.0f;                                     /* exact scaling by 2^24 */
    float r = nearbyintf(q);                                       /* RNE in default mode */
    return (uint16_t)(s | (uint32_t)r);
  }
  uint32_t mant = a & 0x7FFFFFu, exp = (a >> 23) - 112u;
  uint32_t h = (exp << 10) | (mant >> 13);
  uint32_t rem = mant & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
  return (uint16_t)(s | h);
}

static float bf16_to_f32(uint16_t b) { uint32_t u = (uint32_t)b << 16; float f; memcpy(&f, &u, 4); return f; }

static uint16_t f32_to_bf16(float f) {
  uint32_t u; memcpy(&u, &f, 4);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

uint16_t orc_f32_to_bf16(float f) { return f32_to_bf16(f); }
float orc_bf16_to_f32(uint16_t b) { return bf16_to_f32(b); }
uint16_t orc_f32_to_f16(float f) { return f32_to_f16(f); }
float orc_f16_to_f32(uint16_t h) { return f16_to_f32(h); }

/* E4M3 (OCP, finite) magnitudes: code c = 8e + f, f*2^-9 for e == 0, (8+f)*2^(e-10) otherwise.
   trellis.py:22-40: nearest level, ties to the even code, saturate at 448, keep the sign. */
static float e4m3_level(int c) { int e = c >> 3, f = c & 7; return e == 0 ? ldexpf((float)f, -9) : ldexpf((float)(8 + f), e - 10); }

float orc_round_e4m3(float v) {
  float m = fabsf(v);
  if (m > 448.0f || isnan(m)) m = 448.0f;
  /* upper = first level >= m (searchsorted left), clipped to 126 */
  int lo = 0, hi = 127;
  while (lo < hi) { int mid = (lo + hi) / 2; if (e4m3_level(mid) < m) lo = mid + 1; else hi = mid; }
  int upper = lo > 126 ? 126 : lo;
  int lower = upper - 1 < 0 ? 0 : upper - 1;
  float hd = e4m3_level(upper) - m, ld = m - e4m3_level(lower);
  int take_upper = (hd < ld) || (hd == ld && (upper & 1) == 0);
  return copysignf(e4m3_level(take_upper ? upper : lower), v);
}

/* trellis.py:43-50: codeword -> fp16 via the MCG hash, the IEEE half add, then E4M3 rounding. */
void orc_codebook(uint16_t* out) {
  for (uint32_t s = 0; s < 65536u; s++) {
    uint32_t w = ((s * 0xCBAC1FEDu) & 0x8FFF8FFFu) ^ 0x3B603B60u;
    float lo = f16_to_f32((uint16_t)(w & 0xFFFFu)), hi = f16_to_f32((uint16_t)(w >> 16));
    /* both operands have exponent fields in 12..15, so the float sum is exact and one
       rounding to half equals the IEEE half add */
    float sum = f16_to_f32(f32_to_f16(lo + hi));
    out[s] = f32_to_f16(orc_round_e4m3(sum));
  }
}

static float g_codebook_f32[65536];
static int g_codebook_ready = 0;
static void ensure_codebook(void) {
  if (g_codebook_ready) return;
#pragma omp critical(orc_cb)
  {
    if (!g_codebook_ready) {
      uint16_t* t = (uint16_t*)malloc(65536 * 2);
      orc_codebook(t);
      for (int i = 0; i < 65536; i++) g_codebook_f32[i] = f16_to_f32(t[i]);
      free(t);
      g_codebook_ready = 1;
    }
  }
}

/* ---------------- trellis geometry (trellis.py:78-102, trellis.metal:44-48) ---------------- */

/* byte offset of tile (tk, tn) of expert e; side 2 = input-block-major, else output-block-major */
static uint64_t tile_index(uint64_t e, uint32_t tk, uint32_t tn, uint32_t it, uint32_t ot, int side) {
  if (side == 2) return (((e * (it / 8) + tk / 8) * (ot / 8) + tn / 8) * 8 + tk % 8) * 8 + tn % 8;
  return ((e * (ot / 8) + tn / 8) * it + tk) * 8 + tn % 8;
}

/* codeword i (kernel order) of a tile holding 8k words, MSB-first circular bitstream */
static uint32_t tile_codeword(const uint32_t* w, int k, uint32_t i) {
  uint32_t nw = 8u * (uint32_t)k;
  uint32_t end = (i + 1u) * (uint32_t)k + 256u * (uint32_t)k;
  uint32_t last = (end - 1u) / 32u;
  uint64_t merged = ((uint64_t)w[(last - 1u) % nw] << 32) | (uint64_t)w[last % nw];
  return (uint32_t)(merged >> ((last + 1u) * 32u - end)) & 0xFFFFu;
}

/* kernel order (lane, slot) -> (row, col) inside the 16x16 tile */
static void tile_position(uint32_t i, uint32_t* r, uint32_t* c) {
  uint32_t lane = i / 8u, slot = i % 8u;
  *r = (lane % 4u) * 2u + (slot & 1u) + (slot & 2u) * 4u;
  *c = lane / 4u + (slot & 4u) * 2u;
}

/* codeword at input row `row`, output column `col` of expert e (returns the 16-bit state) */
uint32_t orc_codeword_at(const uint8_t* packed, int k, int in_f, int out_f, int side, int64_t e, int row, int col) {
  uint32_t it = (uint32_t)in_f / 16u, ot = (uint32_t)out_f / 16u;
  uint64_t t = tile_index((uint64_t)e, (uint32_t)row / 16u, (uint32_t)col / 16u, it, ot, side);
  const uint32_t* w = (const uint32_t*)(packed + t * 32u * (uint64_t)k);
  uint32_t lr = (uint32_t)row & 15u, lc = (uint32_t)col & 15u;
  /* inverse of tile_position */
  uint32_t lane = (lc & 7u) * 4u + ((lr & 7u) >> 1u);
  uint32_t slot = (lr & 1u) + ((lr & 8u) >> 2u) + ((lc & 8u) >> 1u);
  return tile_codeword(w, k, lane * 8u + slot);
}

int orc_check_format(int64_t nbytes, int k, int in_f, int out_f, int side) {
  if (k < 2 || k > 4) return -1;
  if (in_f <= 0 || out_f <= 0 || in_f % 128 || out_f % 128) return -2;
  if (side < 0 || side > 2) return -3;
  int64_t size = (int64_t)in_f * out_f * k / 8;
  if (nbytes == 0 || nbytes % size) return -4;
  return (int)(nbytes / size);
}

/* decode expert e to inner [in, out] float (trellis.py:78-102 for one matrix) */
void orc_decode_trellis(const uint8_t* packed, int k, int in_f, int out_f, int side, int64_t e, float* inner) {
  ensure_codebook();
  uint32_t it = (uint32_t)in_f / 16u, ot = (uint32_t)out_f / 16u;
#pragma omp parallel for schedule(static)
  for (int64_t tk = 0; tk < (int64_t)it; tk++) {
    for (uint32_t tn = 0; tn < ot; tn++) {
      uint64_t t = tile_index((uint64_t)e, (uint32_t)tk, tn, it, ot, side);
      const uint32_t* w = (const uint32_t*)(packed + t * 32u * (uint64_t)k);
      for (uint32_t i = 0; i < 256u; i++) {
        uint32_t r, c; tile_position(i, &r, &c);
        inner[((uint64_t)tk * 16u + r) * (uint64_t)out_f + tn * 16u + c] = g_codebook_f32[tile_codeword(w, k, i)];
      }
    }
  }
}

/* ---------------- Hadamard (trellis.py:67-75) ---------------- */
void orc_hadamard128(float* x, int64_t n) {
  const float scale = (float)(1.0 / sqrt(128.0));
  for (int64_t b = 0; b + 128 <= n; b += 128) {
    float* y = x + b;
    for (int bit = 1; bit < 128; bit <<= 1)
      for (int i = 0; i < 128; i++)
        if (!(i & bit)) { float a = y[i], c = y[i + bit]; y[i] = a + c; y[i + bit] = a - c; }
    for (int i = 0; i < 128; i++) y[i] *= scale;
  }
}

/* Accumulator of the router and K4 linear dot products: double for the oracle (the parity
   checker); the timed CPU baseline is the same code built with -DORC_ACC=float (fp32 accumulate,
   as the reference's own kernels). */
#ifndef ORC_ACC
#define ORC_ACC double
#endif

/* ---------------- router (model.py:111-132, fast_router.metal:1-42) ---------------- */
void orc_router_logits(const uint16_t* x_bf16, const float* w, int rows, int hidden, int experts, float* logits) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int r = 0; r < rows; r++)
    for (int e = 0; e < experts; e++) {
      ORC_ACC acc = 0;
      const uint16_t* xr = x_bf16 + (int64_t)r * hidden;
      const float* we = w + (int64_t)e * hidden;
      for (int k = 0; k < hidden; k++) acc += (ORC_ACC)bf16_to_f32(xr[k]) * (ORC_ACC)we[k];
      logits[(int64_t)r * experts + e] = (float)acc;
    }
}

static float router_sigmoid(float v) {
  float y = 1.0f / (1.0f + expf(fabsf(v)));
  return v < 0 ? y : 1.0f - y;
}

/* 256 experts, top-8 by descending (sigmoid + bias), ties to the lower id; slot 8 = shared 256 */
void orc_route(const float* logits, const float* bias, int rows, uint32_t* idx9, float* scores8) {
  for (int r = 0; r < rows; r++) {
    float orig[256], choice[256];
    for (int e = 0; e < 256; e++) { orig[e] = router_sigmoid(logits[(int64_t)r * 256 + e]); choice[e] = orig[e] + bias[e]; }
    float sel[8];
    for (int k = 0; k < 8; k++) {
      int best = -1;
      for (int e = 0; e < 256; e++)
        if (best < 0 || choice[e] > choice[best]) best = e;   /* strict > keeps the lower id on ties */
      idx9[(int64_t)r * 9 + k] = (uint32_t)best;
      sel[k] = orig[best];
      choice[best] = -INFINITY;
    }
    float total = 1e-20f;
    for (int k = 0; k < 8; k++) total += sel[k];
    for (int k = 0; k < 8; k++) scores8[(int64_t)r * 8 + k] = sel[k] / total * 2.5f;
    idx9[(int64_t)r * 9 + 8] = 256u;
  }
}

/* ---------------- typed SwiGLU (fast_decode_common.metal:40-49) ---------------- */
float orc_swiglu_bf16(float gate, float up) {
  float g = round_bf16(gate), u = round_bf16(up);
  float tail = 1.0f / (1.0f + expf(fabsf(g)));
  float sig = round_bf16(g < 0 ? tail : 1.0f - tail);
  return round_bf16(round_bf16(g * sig) * u);
}

/* ---------------- K4 trellis linear (trellis.py:172-196) ----------------
   y[out] = out_scale (*) H( H(x (*) in_scale) @ inner_e ), float32 side vectors, ORC_ACC dot.
   Returns the pre-cast float value; the caller applies the bf16 cast. */
static void k4_linear_one(const float* x, const uint8_t* packed, int k, int in_f, int out_f, int side,
                          int64_t e, const uint16_t* in_scale, const uint16_t* out_scale, float* y, float* tmp_in) {
  for (int i = 0; i < in_f; i++) tmp_in[i] = x[i] * f16_to_f32(in_scale[(int64_t)e * in_f + i]);
  orc_hadamard128(tmp_in, in_f);
  uint32_t it = (uint32_t)in_f / 16u, ot = (uint32_t)out_f / 16u;
  ORC_ACC* acc = (ORC_ACC*)calloc((size_t)out_f, sizeof(ORC_ACC));
  for (uint32_t tk = 0; tk < it; tk++)
    for (uint32_t tn = 0; tn < ot; tn++) {
      uint64_t t = tile_index((uint64_t)e, tk, tn, it, ot, side);
      const uint32_t* w = (const uint32_t*)(packed + t * 32u * (uint64_t)k);
      for (uint32_t i = 0; i < 256u; i++) {
        uint32_t r, c; tile_position(i, &r, &c);
        acc[tn * 16u + c] += (ORC_ACC)tmp_in[tk * 16u + r] * (ORC_ACC)g_codebook_f32[tile_codeword(w, k, i)];
      }
    }
  for (int o = 0; o < out_f; o++) y[o] = (float)acc[o];
  free(acc);
  orc_hadamard128(y, out_f);
  for (int o = 0; o < out_f; o++) y[o] *= f16_to_f32(out_scale[(int64_t)e * out_f + o]);
}

/* expert_linear over `slots` rows: x [slots, in] float, ids [slots], y [slots, out] float (pre-cast) */
void orc_k4_linear(const float* x, const uint32_t* ids, int slots, const uint8_t* packed, int k, int in_f, int out_f,
                   int side, const uint16_t* in_scale, const uint16_t* out_scale, float* y) {
  ensure_codebook();
#pragma omp parallel for schedule(dynamic)
  for (int s = 0; s < slots; s++) {
    float* tmp = (float*)malloc((size_t)in_f * sizeof(float));
    k4_linear_one(x + (int64_t)s * in_f, packed, k, in_f, out_f, side, ids[s], in_scale, out_scale, y + (int64_t)s * out_f, tmp);
    free(tmp);
  }
}

/* ---------------- MXFP4 (joined_gather_order_common.metal:29-45, joined_gather_order.metal:19-21) ---------------- */
static const float kE2M1[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
float orc_e2m1(uint32_t nib) { float v = kE2M1[nib & 7u]; return (nib & 8u) ? -v : v; }
float orc_e8m0(uint32_t s) { return s == 0 ? ldexpf(1.0f, -127) : ldexpf(1.0f, (int)s - 127); }

/* y[n] = sum_k x[k] * e2m1(code[n,k]) * 2^(s[n,k/32]-127); codes: 2 per byte, low nibble = even k */
static void mxfp4_linear_one(const float* x, const uint8_t* codes, const uint8_t* scales, int K, int N, float* y) {
  for (int n = 0; n < N; n++) {
    const uint8_t* c = codes + (int64_t)n * (K / 2);
    const uint8_t* s = scales + (int64_t)n * (K / 32);
    double acc = 0.0;
    for (int g = 0; g < K / 32; g++) {
      double part = 0.0;
      for (int j = 0; j < 32; j += 2) {
        uint8_t b = c[g * 16 + j / 2];
        part += (double)x[g * 32 + j] * orc_e2m1(b & 15u) + (double)x[g * 32 + j + 1] * orc_e2m1(b >> 4);
      }
      acc += part * (double)orc_e8m0(s[g]);
    }
    y[n] = (float)acc;
  }
}

/* ---------------- MXFP4 encode (joined_mxfp4.py:12-47) ---------------- */
/* E2M1 code of |a| (a = v / 2^s): nearest of 0, .5, 1, 1.5, 2, 3, 4, 6, ties to the even code, saturating */
static uint32_t e2m1_code(float a) {
  if (a <= 0.25f) return 0;
  if (a < 0.75f) return 1;
  if (a <= 1.25f) return 2;
  if (a < 1.75f) return 3;
  if (a <= 2.5f) return 4;
  if (a < 3.5f) return 5;
  if (a <= 5.0f) return 6;
  return 7;
}

/* One row of n values (n % 32 == 0) -> n/2 code bytes (low nibble = even k) and n/32 e8m0 scales.
 * Shared exponent s = floor(log2 amax) - 2 clamped to [-127, 127] (e8m0 byte s + 127; an all-zero
 * group gets byte 0); element code = sign | E2M1(|v| / 2^s). */
void orc_mx_quantize_row(const float* v, int n, uint8_t* codes, uint8_t* scales) {
  for (int g = 0; g < n / 32; g++) {
    const float* x = v + 32 * g;
    float amax = 0.0f;
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(x[i]));
    int s = -127;
    if (amax > 0.0f) {
      int ex;
      frexpf(amax, &ex);  /* amax = m 2^ex, m in [0.5, 1): floor(log2 amax) = ex - 1 */
      s = ex - 1 - 2;
      if (s < -127) s = -127;
      if (s > 127) s = 127;
    }
    scales[g] = (uint8_t)(s + 127);
    for (int i = 0; i < 32; i += 2) {
      uint32_t c[2];
      for (int j = 0; j < 2; j++) {
        const float xv = x[i + j];
        c[j] = e2m1_code(ldexpf(fabsf(xv), -s)) | (signbit(xv) ? 8u : 0u);
      }
      codes[16 * g + i / 2] = (uint8_t)(c[0] | (c[1] << 4));
    }
  }
}

/* Encode one projection of every expert: inner_e = decode(packed, e) [in, out]; gate/up (in_scale
 * non-null): inner_e[k, :] *= float(in_scale[e, k] * unit[k]); each output row n of inner_e^T is
 * quantised into codes[e][row_offset + n][in/2], scales[e][row_offset + n][in/32] of arrays with
 * out_rows rows per expert (gate at 0 and up at m of the joined gate_up; down at 0). */
void orc_k4_to_mxfp4(const uint8_t* packed, int in_f, int out_f, int side, int64_t experts, const uint16_t* in_scale,
                     const uint16_t* unit, uint8_t* codes, uint8_t* scales, int out_rows, int row_offset) {
  float* inner = (float*)malloc(sizeof(float) * (size_t)in_f * out_f);
  float* row = (float*)malloc(sizeof(float) * (size_t)in_f);
  for (int64_t e = 0; e < experts; e++) {
    orc_decode_trellis(packed, 4, in_f, out_f, side, e, inner);
    for (int n = 0; n < out_f; n++) {
      for (int k = 0; k < in_f; k++) {
        float v = inner[(int64_t)k * out_f + n];
        if (in_scale) v *= f16_to_f32(in_scale[e * in_f + k]) * f16_to_f32(unit[k]);
        row[k] = v;
      }
      const int64_t r = e * out_rows + row_offset + n;
      orc_mx_quantize_row(row, in_f, codes + r * (in_f / 2), scales + r * (in_f / 32));
    }
  }
  free(row);
  free(inner);
}

void orc_mxfp4_linear(const float* x, const uint32_t* ids, int slots, const uint8_t* codes, const uint8_t* scales,
                      int K, int N, float* y) {
#pragma omp parallel for schedule(dynamic)
  for (int s = 0; s < slots; s++)
    mxfp4_linear_one(x + (int64_t)s * K, codes + (int64_t)ids[s] * N * (K / 2), scales + (int64_t)ids[s] * N * (K / 32),
                     K, N, y + (int64_t)s * N);
}

/* ---------------- combine (model.py:415-418, fast_decode_finish_fused.metal:52-61) ---------------- */
static void combine_row(const float* y9 /* [9][h], bf16-valued */, const float* scores, const uint16_t* residual,
                        int h, uint16_t* out) {
  for (int c = 0; c < h; c++) {
    float total = y9[c] * scores[0] + 0.0f;
    for (int r = 1; r < 8; r++) total = (y9[(int64_t)r * h + c] * scores[r] + 0.0f) + total;
    float routed = round_bf16(total);
    float combined = round_bf16(routed + y9[(int64_t)8 * h + c]);
    out[c] = f32_to_bf16(bf16_to_f32(residual[c]) + combined);
  }
}

/* ---------------- full trellis MoE layer (A.5 cast points) ----------------
   k-bit experts (k = 2..4); x [rows, h] bf16, idx9 [rows, 9], scores8 [rows, 8], residual [rows, h]
   bf16 -> out [rows, h] bf16.  values (optional) receives the per-slot expert outputs [rows, 9, h]
   as bf16.  exlr8/experts.py:150-188 (reference chain) + exlr8/model.py:415-418. */
void orc_trellis_moe(int k, const uint16_t* x, const uint32_t* idx9, const float* scores8, const uint16_t* residual,
                     int rows, int h, int m, const uint8_t* pg, const uint8_t* pu, const uint8_t* pd,
                     const uint16_t* in_g, const uint16_t* out_g, const uint16_t* in_u, const uint16_t* out_u,
                     const uint16_t* in_d, const uint16_t* out_d, uint16_t* out, uint16_t* values) {
  ensure_codebook();
  int slots = rows * 9;
  float* y = (float*)malloc((size_t)slots * h * sizeof(float));
#pragma omp parallel for schedule(dynamic)
  for (int s = 0; s < slots; s++) {
    int r = s / 9;
    int64_t e = idx9[s];
    float* xf = (float*)malloc((size_t)h * sizeof(float));
    float* tmp = (float*)malloc((size_t)(h > m ? h : m) * sizeof(float));
    float* g = (float*)malloc((size_t)m * sizeof(float));
    float* u = (float*)malloc((size_t)m * sizeof(float));
    for (int i = 0; i < h; i++) xf[i] = bf16_to_f32(x[(int64_t)r * h + i]);
    k4_linear_one(xf, pg, k, h, m, 1, e, in_g, out_g, g, tmp);
    k4_linear_one(xf, pu, k, h, m, 1, e, in_u, out_u, u, tmp);
    for (int i = 0; i < m; i++) g[i] = orc_swiglu_bf16(g[i], u[i]);
    k4_linear_one(g, pd, k, m, h, 2, e, in_d, out_d, y + (int64_t)s * h, tmp);
    for (int i = 0; i < h; i++) y[(int64_t)s * h + i] = round_bf16(y[(int64_t)s * h + i]);
    free(xf); free(tmp); free(g); free(u);
  }
  if (values)
    for (int64_t i = 0; i < (int64_t)slots * h; i++) values[i] = f32_to_bf16(y[i]);
  for (int r = 0; r < rows; r++)
    combine_row(y + (int64_t)r * 9 * h, scores8 + (int64_t)r * 8, residual + (int64_t)r * h, h, out + (int64_t)r * h);
  free(y);
}

void orc_k4_moe(const uint16_t* x, const uint32_t* idx9, const float* scores8, const uint16_t* residual, int rows,
                int h, int m, const uint8_t* pg, const uint8_t* pu, const uint8_t* pd,
                const uint16_t* in_g, const uint16_t* out_g, const uint16_t* in_u, const uint16_t* out_u,
                const uint16_t* in_d, const uint16_t* out_d, uint16_t* out, uint16_t* values) {
  orc_trellis_moe(4, x, idx9, scores8, residual, rows, h, m, pg, pu, pd, in_g, out_g, in_u, out_u, in_d, out_d, out,
                  values);
}

/* ---------------- joined MXFP4 MoE layer (joined_mxfp4.py:90-165) ----------------
   gate_up codes [E, 2m, h/2], scales [E, 2m, h/32]; down codes [E, h, m/2], scales [E, h, m/32];
   unit [h] fp16 (+-1); out_g/out_u [E, m], in_d [E, m], out_d [E, h] fp16.
   Slots are taken expert by expert: each weight row is dequantised once (e2m1 x 2^(s-127), exact
   in double) and dotted in double with every slot of that expert, rows split over the threads. */
static double g_e2m1_d[16], g_e8m0_d[256];
static int g_mx_tables_ready = 0;
static void ensure_mx_tables(void) {
  if (g_mx_tables_ready) return;
  for (int i = 0; i < 16; i++) g_e2m1_d[i] = (double)orc_e2m1((uint32_t)i);
  for (int i = 0; i < 256; i++) g_e8m0_d[i] = (double)orc_e8m0((uint32_t)i);
  g_mx_tables_ready = 1;
}
static void dequant_row(const uint8_t* codes, const uint8_t* scales, int K, double* w) {
  for (int g = 0; g < K / 32; g++) {
    const double sc = g_e8m0_d[scales[g]];
    for (int j = 0; j < 16; j++) {
      const uint8_t b = codes[g * 16 + j];
      w[g * 32 + 2 * j] = g_e2m1_d[b & 15u] * sc;
      w[g * 32 + 2 * j + 1] = g_e2m1_d[b >> 4] * sc;
    }
  }
}
static double dot_d(const double* a, const double* b, int n) {
  double s = 0.0;
#pragma omp simd reduction(+ : s)
  for (int k = 0; k < n; k++) s += a[k] * b[k];
  return s;
}
/* y[j][n] = row n of the expert's matrix . x[j] for its `cnt` slot vectors x [cnt][K]; rows are
   dequantised in blocks of 32 per thread so each slot vector is read once per block */
static void mx_expert_rows(const uint8_t* codes, const uint8_t* scales, int K, int N, const double* x, int cnt,
                           float* y) {
  enum { RB = 32 };
#pragma omp parallel
  {
    double* w = (double*)malloc(sizeof(double) * (size_t)K * RB);
#pragma omp for schedule(dynamic)
    for (int n0 = 0; n0 < N; n0 += RB) {
      const int nr = N - n0 < RB ? N - n0 : RB;
      for (int r = 0; r < nr; r++)
        dequant_row(codes + (int64_t)(n0 + r) * (K / 2), scales + (int64_t)(n0 + r) * (K / 32), K, w + (int64_t)r * K);
      for (int j = 0; j < cnt; j++)
        for (int r = 0; r < nr; r++)
          y[(int64_t)j * N + n0 + r] = (float)dot_d(x + (int64_t)j * K, w + (int64_t)r * K, K);
    }
    free(w);
  }
}

void orc_mxfp4_moe(const uint16_t* x, const uint32_t* idx9, const float* scores8, const uint16_t* residual, int rows,
                   int h, int m, const uint8_t* gu_codes, const uint8_t* gu_scales, const uint8_t* d_codes,
                   const uint8_t* d_scales, const uint16_t* unit, const uint16_t* out_g, const uint16_t* out_u,
                   const uint16_t* in_d, const uint16_t* out_d, uint16_t* out, uint16_t* values) {
  const int slots = rows * 9;
  ensure_mx_tables();
  float* y = (float*)malloc((size_t)slots * h * sizeof(float));
  /* shared prep: xh = H128(x * unit) per token row */
  float* xh = (float*)malloc((size_t)rows * h * sizeof(float));
  for (int r = 0; r < rows; r++) {
    for (int i = 0; i < h; i++) xh[(int64_t)r * h + i] = bf16_to_f32(x[(int64_t)r * h + i]) * f16_to_f32(unit[i]);
    orc_hadamard128(xh + (int64_t)r * h, h);
  }
  uint32_t emax = 0;
  for (int s = 0; s < slots; s++) emax = idx9[s] > emax ? idx9[s] : emax;
  int* list = (int*)malloc(sizeof(int) * (size_t)slots);
  double* xs = (double*)malloc(sizeof(double) * (size_t)slots * h);
  float* gu = (float*)malloc(sizeof(float) * (size_t)slots * 2 * m);
  double* as = (double*)malloc(sizeof(double) * (size_t)slots * m);
  for (uint32_t e = 0; e <= emax; e++) {
    int cnt = 0;
    for (int s = 0; s < slots; s++)
      if (idx9[s] == e) list[cnt++] = s;
    if (!cnt) continue;
    for (int j = 0; j < cnt; j++)
      for (int i = 0; i < h; i++) xs[(int64_t)j * h + i] = (double)xh[(int64_t)(list[j] / 9) * h + i];
    mx_expert_rows(gu_codes + (int64_t)e * 2 * m * (h / 2), gu_scales + (int64_t)e * 2 * m * (h / 32), h, 2 * m, xs,
                   cnt, gu);
    for (int j = 0; j < cnt; j++) {
      float* g = gu + (int64_t)j * 2 * m;
      float* a = (float*)malloc(sizeof(float) * (size_t)m);
      orc_hadamard128(g, m);
      orc_hadamard128(g + m, m);
      for (int i = 0; i < m; i++) {
        float gv = g[i] * f16_to_f32(out_g[e * m + i]), uv = g[m + i] * f16_to_f32(out_u[e * m + i]);
        a[i] = orc_swiglu_bf16(gv, uv) * f16_to_f32(in_d[e * m + i]);
      }
      orc_hadamard128(a, m);
      for (int i = 0; i < m; i++) as[(int64_t)j * m + i] = (double)a[i];
      free(a);
    }
    float* v = (float*)malloc(sizeof(float) * (size_t)cnt * h);
    mx_expert_rows(d_codes + (int64_t)e * h * (m / 2), d_scales + (int64_t)e * h * (m / 32), m, h, as, cnt, v);
    for (int j = 0; j < cnt; j++) {
      float* vj = v + (int64_t)j * h;
      orc_hadamard128(vj, h);
      float* dst = y + (int64_t)list[j] * h;
      for (int i = 0; i < h; i++) dst[i] = round_bf16(vj[i] * f16_to_f32(out_d[e * h + i]));
    }
    free(v);
  }
  free(list); free(xs); free(gu); free(as); free(xh);
  if (values)
    for (int64_t i = 0; i < (int64_t)slots * h; i++) values[i] = f32_to_bf16(y[i]);
  for (int r = 0; r < rows; r++)
    combine_row(y + (int64_t)r * 9 * h, scores8 + (int64_t)r * 8, residual + (int64_t)r * h, h, out + (int64_t)r * h);
  free(y);
}

/* ---------------- residual + RMSNorm (residual_rms.metal:18-90) ----------------
   h = T(x + r); out = T(w * T(h * rsqrt(mean(h^2) + eps))).  r may be NULL (treated as 0). */
void orc_residual_rmsnorm(const uint16_t* x, const uint16_t* r, const uint16_t* w, int rows, int n, float eps,
                          uint16_t* h_out, uint16_t* out) {
  for (int row = 0; row < rows; row++) {
    double ss = 0.0;
    for (int i = 0; i < n; i++) {
      float hv = round_bf16(bf16_to_f32(x[(int64_t)row * n + i]) + (r ? bf16_to_f32(r[(int64_t)row * n + i]) : 0.0f));
      h_out[(int64_t)row * n + i] = f32_to_bf16(hv);
      ss += (double)hv * hv;
    }
    float inv = (float)(1.0 / sqrt(ss / n + (double)eps));
    for (int i = 0; i < n; i++) {
      float hv = bf16_to_f32(h_out[(int64_t)row * n + i]);
      out[(int64_t)row * n + i] = f32_to_bf16(bf16_to_f32(w[i]) * round_bf16(hv * inv));
    }
  }
}

/* ---------------- sorted work order (fast_prefill.py:19-46) ----------------
   Stable argsort of flat ids, then a block table of (expert, first, length) with
   `block_rows` rows per block.  Returns the number of valid blocks. */
int orc_segment_table(const uint32_t* ids, int n, int experts, int block_rows, int32_t* order,
                      int32_t* counts, int32_t* starts, int32_t* blk_expert, int32_t* blk_first, int32_t* blk_len) {
  for (int e = 0; e < experts; e++) counts[e] = 0;
  for (int i = 0; i < n; i++) counts[ids[i]]++;
  int acc = 0;
  for (int e = 0; e < experts; e++) { starts[e] = acc; acc += counts[e]; }
  int* fill = (int*)calloc((size_t)experts, sizeof(int));
  for (int i = 0; i < n; i++) { int e = (int)ids[i]; order[starts[e] + fill[e]++] = i; }
  free(fill);
  int b = 0;
  for (int e = 0; e < experts; e++)
    for (int f = 0; f < counts[e]; f += block_rows) {
      blk_expert[b] = e; blk_first[b] = starts[e] + f;
      blk_len[b] = counts[e] - f < block_rows ? counts[e] - f : block_rows;
      b++;
    }
  return b;
}

int orc_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
