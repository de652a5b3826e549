// K4 trellis expert path on gfx950: decode-fused GEMVs, gate finish, combine.
//
// Semantics follow the reference's resident K4 chain (paths relative to the reference root):
//   prep      xh = H128(x * in_scale[e])                 exlr8/metal/fast_decode_prep.metal
//   linear    inner = xh @ decode(packed_e)              exlr8/metal/fast_decode_linear.metal
//   gate fin. a = H128(swiglu_T(H(g)*og, H(u)*ou)*id)    exlr8/metal/fast_decode_gate_finish.metal
//   finish    T(H128(inner) * out_scale)                 exlr8/metal/fast_decode_finish.metal
//   combine   routed sum, shared, residual               exlr8/metal/fast_decode_finish_fused.metal
//
// MI355X design (not a translation of the Metal kernels):
//   * One persistent block of 16 waves per CU.  The 64 KB E4M3 code table lives in LDS once
//     per CU; every wave streams a static, contiguous range of 1 KB "chunks".
//   * A chunk is one 16-row input tile x 128 output columns (8 consecutive 128 B tiles).  Both
//     storage orders keep a chunk contiguous, so each wave load is one fully coalesced 1 KB
//     dwordx4 access.  Lane L holds 4 words of tile L/8 and owns output columns
//     16*(L/8) + L%8 and +8 for all 16 rows: no cross-lane reduction inside the k loop.
//   * Codewords are decoded by LDS table lookup or arithmetically (mix chosen at compile
//     time) and accumulated in fp32.
//   * Prep (scale + H128) is fused into the gate/up GEMV; the gate finish and the combine are
//     done by the last wave to finish a (unit, column block) / column block, detected with a
//     device-scope counter, so a layer is router + gate/up + down = few launches and the
//     partial sums are reduced in a fixed order (deterministic).
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>

#include <atomic>
#include <mutex>

#include "layer_sync.h"
#include "moe_device.h"
#include "moe_host.h"
#include "moe_plan.h"
#include "route.h"

#ifndef MOE_FOLD_NORM
#define MOE_FOLD_NORM 1
#endif

namespace moe {

__device__ uint8_t g_codebook_e4m3[65536];
__device__ uint16_t g_codebook_f16[65536];

// ============================================================== codebook

__global__ void build_codebook_kernel() {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;  // pair index, 32768 pairs
  if (i >= 32768u) return;
  const uint32_t a = 2u * i, b = 2u * i + 1u;
  const uint32_t bytes = decode_pair_fp8(a, b);
  g_codebook_e4m3[a] = (uint8_t)(bytes & 0xFFu);
  g_codebook_e4m3[b] = (uint8_t)(bytes >> 8);
  // widened one byte at a time (exact): element extraction from the packed fp8 -> f16 conversion
  // has been compiled into a store of the first element twice
  g_codebook_f16[a] = __builtin_bit_cast(uint16_t, (_Float16)fp8_to_f32(bytes & 0xFFu));
  g_codebook_f16[b] = __builtin_bit_cast(uint16_t, (_Float16)fp8_to_f32((bytes >> 8) & 0xFFu));
}

__global__ void copy_codebook_kernel(uint8_t* dst) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < 65536u) dst[i] = g_codebook_e4m3[i];
}

// ============================================================== plan

__global__ __launch_bounds__(128) void plan_kernel(const uint32_t* __restrict__ ids, int rows, int slots,
                                                    int experts, int max_users, Plan* plan) {
  __shared__ int32_t sid[kMaxUnits];
  __shared__ int32_t open[kMaxUnits];
  const int n = rows * slots;
  if ((int)threadIdx.x < n) {
    int e = (int)ids[threadIdx.x];
    if (e < 0) e = 0;
    if (e >= experts) e = experts - 1;
    if (e > 256) e = 256;
    sid[threadIdx.x] = e;
  }
  __syncthreads();
  build_plan_parallel(sid, rows, slots, max_users, plan, open);
}

// ============================================================== decode-only kernel

// Inner [in, out] fp16 of one expert (exlr8/metal/decode.metal semantics), decoded with the same
// device code as the GEMVs: thread = one 16 B piece (4 consecutive words of a tile), words
// decoded in pairs by decode_pair_words_f16.  Each block uses one of four arithmetic/table mixes,
// so a full decode exercises every route of the GEMV decoder.
template <int NE, int NO, bool T16 = false>
__device__ __forceinline__ void decode_piece_to_inner(const uint32_t* __restrict__ tw, int qg, const uint8_t* tab,
                                                      uint16_t* __restrict__ inner, int out_f, uint32_t row0,
                                                      uint32_t col0) {
  const u32x4 v = *reinterpret_cast<const u32x4*>(tw + 4 * qg);
  const uint32_t prior = tw[(4 * qg + 31) & 31];
#pragma unroll
  for (int h = 0; h < 2; h++) {
    f16x2 q[2][4];
    if (h == 0)
      decode_pair_words_f16<NE, NO, T16>(v.x, v.y, prior, tab, q);
    else
      decode_pair_words_f16<NE, NO, T16>(v.z, v.w, v.y, tab, q);
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
      for (int j = 0; j < 4; j++) {
        // word 2h+i, pair j: rows 2(2h+i) + 8*(j&1) + {0,1}, column qg + 8*(j>>1)
        const uint32_t r = row0 + 2 * (2 * h + i) + 8 * (j & 1), c = col0 + qg + 8 * (j >> 1);
        const uint32_t bits = __builtin_bit_cast(uint32_t, q[i][j]);
        inner[(int64_t)r * out_f + c] = (uint16_t)(bits & 0xFFFFu);
        inner[(int64_t)(r + 1) * out_f + c] = (uint16_t)(bits >> 16);
      }
  }
}

// T16: the blocks with odd index, decoded through the fp16 table (the even blocks, with T16 false,
// through the E4M3 byte table); the launch of the other kind leaves a block alone.
template <bool T16>
__global__ __launch_bounds__(1024) void trellis_decode_kernel(const uint32_t* __restrict__ packed, int in_f, int out_f,
                                                              int side, int64_t expert, uint16_t* __restrict__ inner) {
  if ((int)(blockIdx.x & 1) != (int)T16) return;
  __shared__ __attribute__((aligned(16))) uint8_t tab[T16 ? 131072 : 65536];
  if (T16)
    load_codebook16_lds<1024>(tab);
  else
    load_codebook_lds_t<1024>(tab);
  __syncthreads();
  const int64_t pieces = (int64_t)in_f * out_f / 32;  // 8 pieces per 256-weight tile
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= pieces) return;
  const uint32_t it = (uint32_t)in_f / 16u, ot = (uint32_t)out_f / 16u;
  const int64_t t = idx >> 3;
  const int qg = (int)(idx & 7);
  // tile t in row-major (tk, tn) order -> storage index of the side's layout
  const uint32_t tk = (uint32_t)(t / ot), tn = (uint32_t)(t % ot);
  const uint64_t e = (uint64_t)expert;
  const uint64_t tile = side == 2 ? ((((e * (it / 8u) + tk / 8u) * (ot / 8u) + tn / 8u) * 8u + tk % 8u) * 8u + tn % 8u)
                                  : (((e * (ot / 8u) + tn / 8u) * it + tk) * 8u + tn % 8u);
  const uint32_t* tw = packed + tile * 32u;
  // the mixes of the decoders in use (fused blocks 1/2, grouped GEMM 2/3) and every per-word count 0..4
  switch ((blockIdx.x >> 1) % 6) {
    case 0: decode_piece_to_inner<0, 0, T16>(tw, qg, tab, inner, out_f, 16u * tk, 16u * tn); break;
    case 1: decode_piece_to_inner<1, 2, T16>(tw, qg, tab, inner, out_f, 16u * tk, 16u * tn); break;
    case 2: decode_piece_to_inner<2, 2, T16>(tw, qg, tab, inner, out_f, 16u * tk, 16u * tn); break;
    case 3: decode_piece_to_inner<2, 3, T16>(tw, qg, tab, inner, out_f, 16u * tk, 16u * tn); break;
    case 4: decode_piece_to_inner<3, 1, T16>(tw, qg, tab, inner, out_f, 16u * tk, 16u * tn); break;
    default: decode_piece_to_inner<4, 4, T16>(tw, qg, tab, inner, out_f, 16u * tk, 16u * tn); break;
  }
}

// K3 tiles (24 words): thread = one lane's piece (words 3 qg .. 3 qg + 2, the previous lane's last
// word cyclically before them), decoded by decode_k3_pair_words, the fused block's K3 decoder, and
// placed as the K4 decoder's words 0..3.  Each block uses one arithmetic/table mix.
template <int NE, int NO>
__device__ __forceinline__ void decode_k3_piece_to_inner(const uint32_t* __restrict__ tw, int qg, const uint8_t* tab,
                                                         uint16_t* __restrict__ inner, int out_f, uint32_t row0,
                                                         uint32_t col0) {
  const uint32_t S[4] = {tw[(3 * qg + 23) % 24], tw[3 * qg], tw[3 * qg + 1], tw[3 * qg + 2]};
#pragma unroll
  for (int h = 0; h < 2; h++) {
    f16x2 q[2][4];
    if (h == 0)
      decode_k3_pair_words<NE, NO, 0>(S, tab, q);
    else
      decode_k3_pair_words<NE, NO, 2>(S, tab, q);
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const uint32_t r = row0 + 2 * (2 * h + i) + 8 * (j & 1), c = col0 + qg + 8 * (j >> 1);
        const uint32_t bits = __builtin_bit_cast(uint32_t, q[i][j]);
        inner[(int64_t)r * out_f + c] = (uint16_t)(bits & 0xFFFFu);
        inner[(int64_t)(r + 1) * out_f + c] = (uint16_t)(bits >> 16);
      }
  }
}
__global__ __launch_bounds__(1024) void trellis_decode_k3_kernel(const uint32_t* __restrict__ packed, int in_f, int out_f,
                                                                 int side, int64_t expert, uint16_t* __restrict__ inner) {
  __shared__ __attribute__((aligned(16))) uint8_t tab[65536];
  load_codebook_lds_t<1024>(tab);
  __syncthreads();
  const int64_t pieces = (int64_t)in_f * out_f / 32;  // 8 pieces per 256-weight tile
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= pieces) return;
  const uint32_t it = (uint32_t)in_f / 16u, ot = (uint32_t)out_f / 16u;
  const int64_t t = idx >> 3;
  const int qg = (int)(idx & 7);
  const uint32_t tk = (uint32_t)(t / ot), tn = (uint32_t)(t % ot);
  const uint64_t e = (uint64_t)expert;
  const uint64_t tile = side == 2 ? ((((e * (it / 8u) + tk / 8u) * (ot / 8u) + tn / 8u) * 8u + tk % 8u) * 8u + tn % 8u)
                                  : (((e * (ot / 8u) + tn / 8u) * it + tk) * 8u + tn % 8u);
  const uint32_t* tw = packed + tile * 24u;
  // the fused block's mix (MOE_LAYER3_ALU_EVEN / _ODD = 1 / 2) and every per-word count 0..4
  switch (blockIdx.x % 5) {
    case 0: decode_k3_piece_to_inner<1, 2>(tw, qg, tab, inner, out_f, 16u * tk, 16u * tn); break;
    case 1: decode_k3_piece_to_inner<0, 0>(tw, qg, tab, inner, out_f, 16u * tk, 16u * tn); break;
    case 2: decode_k3_piece_to_inner<2, 3>(tw, qg, tab, inner, out_f, 16u * tk, 16u * tn); break;
    case 3: decode_k3_piece_to_inner<4, 4>(tw, qg, tab, inner, out_f, 16u * tk, 16u * tn); break;
    default: decode_k3_piece_to_inner<3, 1>(tw, qg, tab, inner, out_f, 16u * tk, 16u * tn); break;
  }
}

// K2 / K3 tiles (8k words, exlr8/trellis.py:78-102): one thread per codeword.  Codeword i is the 16
// bits that end after its k-bit symbol in the tile's circular MSB-first bitstream; its weight is
// the E4M3 table entry widened to fp16 (exact), placed by the tensor-core position map.
__global__ __launch_bounds__(256) void trellis_decode_generic_kernel(const uint32_t* __restrict__ packed, int k,
                                                                      int in_f, int out_f, int side, int64_t expert,
                                                                      uint16_t* __restrict__ inner) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)in_f * out_f) return;
  const uint32_t it = (uint32_t)in_f / 16u, ot = (uint32_t)out_f / 16u;
  const int64_t t = idx >> 8;
  const uint32_t i = (uint32_t)(idx & 255);
  const uint32_t tk = (uint32_t)(t / ot), tn = (uint32_t)(t % ot);
  const uint64_t e = (uint64_t)expert;
  const uint64_t tile = side == 2 ? ((((e * (it / 8u) + tk / 8u) * (ot / 8u) + tn / 8u) * 8u + tk % 8u) * 8u + tn % 8u)
                                  : (((e * (ot / 8u) + tn / 8u) * it + tk) * 8u + tn % 8u);
  const uint32_t nw = 8u * (uint32_t)k;
  const uint32_t* tw = packed + tile * nw;
  const uint32_t end = (i + 1u) * (uint32_t)k + 256u * (uint32_t)k;
  const uint32_t last = (end - 1u) / 32u;
  const uint64_t merged = ((uint64_t)tw[(last - 1u) % nw] << 32) | (uint64_t)tw[last % nw];
  const uint32_t cw = (uint32_t)(merged >> ((last + 1u) * 32u - end)) & 0xFFFFu;
  const uint32_t lane = i / 8u, slot = i % 8u;
  const uint32_t r = (lane % 4u) * 2u + (slot & 1u) + (slot & 2u) * 4u, c = lane / 4u + (slot & 4u) * 2u;
  const _Float16 v = (_Float16)fp8_to_f32(g_codebook_e4m3[cw]);
  inner[(uint64_t)(16u * tk + r) * (uint64_t)out_f + 16u * tn + c] = __builtin_bit_cast(uint16_t, v);
}

// ============================================================== GEMV machinery

enum InMode { IN_PREP = 0, IN_DIRECT = 1 };
enum FinMode { FIN_GATE = 0, FIN_VALUES = 1, FIN_COMBINE = 2 };

// Decode GEMV (k4_mfma_kernel): per-word arithmetic pair counts (even, odd
// words) for single-token units (_1) and for units of up to kMaxRows tokens (_8), chosen by
// measurement on MI355X
#ifndef MOE_K4_ALU_EVEN_1
#define MOE_K4_ALU_EVEN_1 2
#endif
#ifndef MOE_K4_ALU_ODD_1
#define MOE_K4_ALU_ODD_1 2
#endif
#ifndef MOE_K4_ALU_EVEN_8
#define MOE_K4_ALU_EVEN_8 1
#endif
#ifndef MOE_K4_ALU_ODD_8
#define MOE_K4_ALU_ODD_8 2
#endif
// waves per block of the MFMA kernel for single-token units and for up to kMaxRows tokens (the
// latter needs more registers for its A fragments)
#ifndef MOE_K4_WAVES_1
#define MOE_K4_WAVES_1 16
#endif
#ifndef MOE_K4_WAVES_8
#define MOE_K4_WAVES_8 8
#endif
// the single-token gate/up GEMV runs 12 waves per block (3 per SIMD): measured faster than 16
// (47 vs 51 us) and than 8, with the fp16 table and the progress-based wave priority
#ifndef MOE_K4_WAVES_1_GU
#define MOE_K4_WAVES_1_GU 12
#endif
#ifndef MOE_K4_ALU_EVEN_1_DN
#define MOE_K4_ALU_EVEN_1_DN MOE_K4_ALU_EVEN_1
#endif
#ifndef MOE_K4_ALU_ODD_1_DN
#define MOE_K4_ALU_ODD_1_DN MOE_K4_ALU_ODD_1
#endif

// wave issue priority raised for waves that are behind on their range (measured per build)
#ifndef MOE_K4_PRIO
#define MOE_K4_PRIO 1
#endif

constexpr int kWaves = 16;            // waves per block (one block per CU)
constexpr int kThreads = kWaves * 64;
constexpr int kMaxBlocks = 256;
constexpr int kMaxWaves = kMaxBlocks * kWaves;
constexpr int kPartialStride = kMaxRows * 128;  // floats per (wave, visit)

struct GemvArgs {
  const uint8_t* packed[2];
  int nproj;
  int in_f, out_f, side;
  int x_per_slot;              // PREP: x row index = slot (else token row)
  const uint16_t* x_bf16;      // PREP: [rows or slots, in_f]
  const uint16_t* in_scale[2]; // PREP: [E, in_f]
  const float* x_f32;          // DIRECT: [slots, in_f]
  const Plan* plan;
  float* partial;              // [W][2][kMaxRows][128]
  int32_t* counter_seg;        // chunks completed per segment
  int32_t* counter_grp;        // segments completed per finish group
  float* yslot;                // COMBINE: bf16-rounded expert outputs [slot][out_f]
  const uint16_t* out_scale[2];
  const uint16_t* in_down;     // GATE
  float* down_xh;              // GATE output [slots, out_f]
  uint16_t* values;            // VALUES output [slots, out_f]
  const float* scores;         // COMBINE [rows, 8]
  const uint16_t* residual;    // COMBINE [rows, out_f]
  uint16_t* out;               // COMBINE [rows, out_f]
};

// Static split of n work units over nw waves: every wave takes `base` units and the first `rem`
// waves one more, so a wave's range start is a multiply-add (no division in the finish path).
struct Split {
  int base, rem;
  __device__ __forceinline__ int start(int w) const { return w * base + min(w, rem); }
  __device__ __forceinline__ bool nonempty(int w) const { return base > 0 || w < rem; }
  // the wave whose range holds unit c
  __device__ __forceinline__ int wave_of(int c) const {
    const int big = rem * (base + 1);
    return c < big ? c / (base + 1) : rem + (c - big) / base;
  }
};
__device__ __forceinline__ Split make_split(int n, int nw) { return Split{n / nw, n % nw}; }

// Cross-wave hand-off of partial sums inside one launch.  The XCDs' L2 caches are not coherent
// with each other, and an agent-scope release would write back a whole L2.  Partials are
// therefore stored write-through (system scope) and read back bypassing the L2; a
// workgroup-scope fence (wait for the stores' acknowledgement) orders them before the counter.
__device__ __forceinline__ void store_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ float load_coherent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ void store_coherent2(float* p, float a, float b) {
  const uint64_t v = (uint64_t)__float_as_uint(a) | ((uint64_t)__float_as_uint(b) << 32);
  __hip_atomic_store(reinterpret_cast<uint64_t*>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ f32x2 load_coherent2(const float* p) {
  const uint64_t v = __hip_atomic_load(reinterpret_cast<uint64_t*>(const_cast<float*>(p)), __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_SYSTEM);
  return f32x2{__uint_as_float((uint32_t)v), __uint_as_float((uint32_t)(v >> 32))};
}
__device__ __forceinline__ int counter_add(int32_t* c, int v) {
  int old = 0;
  if (lane_id() == 0) old = __hip_atomic_fetch_add(c, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  return __shfl(old, 0, 64);
}
__device__ __forceinline__ void counter_reset(int32_t* c) {
  if (lane_id() == 0) __hip_atomic_store(c, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Partial sums of one segment: the waves overlapping it and, for each, the visit that covers it.
struct SegWaves {
  int a;  // first work unit of the segment
  int wa, wb;
};
__device__ __forceinline__ SegWaves seg_waves(const Split& sp, int ups, int seg) {
  const int a = seg * ups;
  return SegWaves{a, sp.wave_of(a), sp.wave_of(a + ups - 1)};
}
// Load the partial pair of wave w for segment sw, token t, columns 2*lane, +1 (zero if the wave
// has no work there).
__device__ __forceinline__ f32x2 load_partial(const float* __restrict__ partial, const Split& sp, const SegWaves& sw,
                                              int w, int t, bool& ok) {
  ok = w <= sw.wb && sp.nonempty(w);
  const int visit = (sp.start(w) >= sw.a) ? 0 : 1;
  const int64_t idx = ok ? ((int64_t)w * 2 + visit) * kPartialStride + (int64_t)t * 128 + 2 * lane_id() : 0;
  return load_coherent2(partial + idx);
}

// Sum, in wave order, the partials of segment `seg` for token position `t` at columns
// 2*lane and 2*lane+1.  Work is partitioned in units (a chunk, or a quad of chunks); segment
// `seg` covers units [seg*ups, (seg+1)*ups) of `n` units split over `nw` waves.  Loads are
// issued in batches of 16 waves so one memory round trip covers a batch; empty wave ranges
// contribute nothing.
__device__ __forceinline__ void sum_partials(const float* __restrict__ partial, const Split& sp, int ups, int seg,
                                             int t, float& v0, float& v1) {
  const SegWaves sw = seg_waves(sp, ups, seg);
  v0 = 0.0f;
  v1 = 0.0f;
  for (int w0 = sw.wa; w0 <= sw.wb; w0 += 16) {
    f32x2 p[16];
    bool ok[16];
#pragma unroll
    for (int j = 0; j < 16; j++) p[j] = load_partial(partial, sp, sw, w0 + j, t, ok[j]);
#pragma unroll
    for (int j = 0; j < 16; j++) {
      if (ok[j]) { v0 += p[j].x; v1 += p[j].y; }
    }
  }
}
// The same for two segments at once (their loads share round trips).
__device__ __forceinline__ void sum_partials_pair(const float* __restrict__ partial, const Split& sp, int ups,
                                                  int seg_a, int seg_b, int t, f32x2& ra, f32x2& rb) {
  const SegWaves sa = seg_waves(sp, ups, seg_a), sb = seg_waves(sp, ups, seg_b);
  ra = f32x2{0.0f, 0.0f};
  rb = f32x2{0.0f, 0.0f};
  for (int k = 0; sa.wa + k <= sa.wb || sb.wa + k <= sb.wb; k += 12) {
    f32x2 pa[12], pb[12];
    bool oka[12], okb[12];
#pragma unroll
    for (int j = 0; j < 12; j++) {
      pa[j] = load_partial(partial, sp, sa, sa.wa + k + j, t, oka[j]);
      pb[j] = load_partial(partial, sp, sb, sb.wa + k + j, t, okb[j]);
    }
#pragma unroll
    for (int j = 0; j < 12; j++) {
      if (oka[j]) { ra.x += pa[j].x; ra.y += pa[j].y; }
      if (okb[j]) { rb.x += pb[j].x; rb.y += pb[j].y; }
    }
  }
}

// After a wave has stored the partials of one visit (`units` work units of segment `seg`):
// count them, and if this completes the segment reduce it and run the finish stage that the
// segment unlocks (gate finish, per-slot values, or the column-block combine).
template <int FM>
__device__ __forceinline__ void complete_visit(const GemvArgs& a, const Plan* __restrict__ P, int seg, int units,
                                               int ups, const Split& sp, int nproj, int U, int u, int ob, int e,
                                               int ntok) {
  const int lane = lane_id();
  const int col = ob * 128 + 2 * lane;
  release_stores();
  if (FM == FIN_GATE) {
    // gate and up of one column block are the adjacent segments 2*grp and 2*grp+1: one counter
    // covers both, and the wave that completes them reduces both and runs the gate finish
    const int grp = seg >> 1;
    if (counter_add(&a.counter_grp[grp], units) + units != 2 * ups) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    counter_reset(&a.counter_grp[grp]);
    // side vectors issued with the first partial loads (one round trip)
    const int64_t si = (int64_t)e * a.out_f + col;
    const uint32_t og = *reinterpret_cast<const uint32_t*>(a.out_scale[0] + si);
    const uint32_t ou = *reinterpret_cast<const uint32_t*>(a.out_scale[1] + si);
    const uint32_t idn = *reinterpret_cast<const uint32_t*>(a.in_down + si);
    auto lo = [](uint32_t v) { return f16_to_f32((uint16_t)(v & 0xFFFFu)); };
    auto hi = [](uint32_t v) { return f16_to_f32((uint16_t)(v >> 16)); };
    for (int t = 0; t < ntok; t++) {
      f32x2 g, uu;
      sum_partials_pair(a.partial, sp, ups, 2 * grp, 2 * grp + 1, t, g, uu);
      float g0 = g.x, g1 = g.y, u0 = uu.x, u1 = uu.y;
      hadamard128_wave(g0, g1);
      hadamard128_wave(u0, u1);
      float h0 = swiglu_bf16(g0 * lo(og), u0 * lo(ou));
      float h1 = swiglu_bf16(g1 * hi(og), u1 * hi(ou));
      h0 *= lo(idn);
      h1 *= hi(idn);
      hadamard128_wave(h0, h1);
      const int slot = P->slot[u][t];
      *reinterpret_cast<f32x2*>(a.down_xh + (int64_t)slot * a.out_f + col) = f32x2{h0, h1};
    }
    return;
  }
  if (counter_add(&a.counter_seg[seg], units) + units != ups) return;
  // this wave completed segment `seg`: reduce its partials once
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  counter_reset(&a.counter_seg[seg]);
  const int64_t si = (int64_t)e * a.out_f + col;
  const uint32_t osc = *reinterpret_cast<const uint32_t*>(a.out_scale[0] + si);  // with the partial loads
  const float os0 = f16_to_f32((uint16_t)(osc & 0xFFFFu)), os1 = f16_to_f32((uint16_t)(osc >> 16));
  if (FM == FIN_VALUES) {
    for (int t = 0; t < ntok; t++) {
      float v0, v1;
      sum_partials(a.partial, sp, ups, seg, t, v0, v1);
      hadamard128_wave(v0, v1);
      const int slot = P->slot[u][t];
      const uint32_t packed2 = (uint32_t)f32_to_bf16(v0 * os0) | ((uint32_t)f32_to_bf16(v1 * os1) << 16);
      *reinterpret_cast<uint32_t*>(a.values + (int64_t)slot * a.out_f + col) = packed2;
    }
  } else {
    // per-slot expert output of this column block: T(H128(inner) * out_scale)
    for (int t = 0; t < ntok; t++) {
      float v0, v1;
      sum_partials(a.partial, sp, ups, seg, t, v0, v1);
      hadamard128_wave(v0, v1);
      const int slot = P->slot[u][t];
      store_coherent2(a.yslot + (int64_t)slot * a.out_f + col, round_bf16(v0 * os0), round_bf16(v1 * os1));
    }
    release_stores();
    if (counter_add(&a.counter_grp[ob], 1) + 1 != U) return;
    // every unit of this column block is done: weighted routed sum, shared, residual
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    counter_reset(&a.counter_grp[ob]);
    for (int r = 0; r < P->rows; r++) {
      f32x2 y[kSlots];
#pragma unroll
      for (int j = 0; j < kSlots; j++) y[j] = load_coherent2(a.yslot + (int64_t)(r * kSlots + j) * a.out_f + col);
      float tot0 = y[0].x * a.scores[r * 8] + 0.0f, tot1 = y[0].y * a.scores[r * 8] + 0.0f;
#pragma unroll
      for (int j = 1; j < 8; j++) {
        const float sc = a.scores[r * 8 + j];
        tot0 = (y[j].x * sc + 0.0f) + tot0;
        tot1 = (y[j].y * sc + 0.0f) + tot1;
      }
      const float c0f = round_bf16(round_bf16(tot0) + y[8].x);
      const float c1f = round_bf16(round_bf16(tot1) + y[8].y);
      const int64_t o = (int64_t)r * a.out_f + col;
      const uint16_t* res = a.residual + o;
      const uint32_t packed2 = (uint32_t)f32_to_bf16(bf16_to_f32(res[0]) + c0f) |
                               ((uint32_t)f32_to_bf16(bf16_to_f32(res[1]) + c1f) << 16);
      *reinterpret_cast<uint32_t*>(a.out + o) = packed2;
    }
  }
}

// ============================================================== MFMA decode GEMV
//
// Work split: the (unit, output block, projection, quad) space is flattened and cut into one
// static contiguous range per wave; a segment is the run of quads of one (unit, output block,
// projection).  A quad is 4 chunks (64 input rows x 128 output columns).  The accumulation runs on
// the matrix cores (v_mfma_f32_16x16x32_f16), so the vector ALUs only decode.
//
//   * Lane l = 16g + n loads, for each of 4 sets s, the 16 B piece (tile 2s + n/8, word group n%8)
//     of chunk tk+g: 4 words = all 16 rows of output columns q = n%8 and q+8 of that tile.
//   * A word's 8 codewords become four fp16 pairs (c0,c1), (c2,c3), (c4,c5), (c6,c7) -- by LDS
//     table lookup or arithmetic decode (decode_word_f16).  Two words of a piece form one B
//     fragment (8 rows x 1 column) per output-column half h and row half rh, so a piece feeds
//     4 MFMAs; the 4 k-groups of the MFMA are the 4 chunks of the quad.
//   * A = x split into fp16 rows hi = f16(x) and lo = f16((x - hi) * 2^11) (x to ~22 bits), rows 2t
//     and 2t+1 for token row t of the unit; staged once per 128-row block in the wave's LDS slice
//     in A order.
//   * D[2t] + 2^-11 * D[2t+1] gives token t's fp32 dot products.

// The kernel body takes its LDS regions as distinct restrict pointers (table, the wave's A
// fragments), so the compiler knows they never alias.
template <int IM, int FM, int NT, int ALU_EVEN, int ALU_ODD, int WV>
__device__ __forceinline__ void k4_mfma_body(const GemvArgs& a, const Plan* __restrict__ P,
                                             const uint8_t* __restrict__ tab, _Float16* __restrict__ xw);

// Single-token units keep the code table as fp16 in LDS (128 KB; the lookups then need no fp8
// widening); batched units, whose A fragments need more LDS, keep the 64 KB E4M3 byte table.
template <int NT>
struct TableKind {
  static constexpr bool kF16 = NT == 1;
  static constexpr int kBytes = kF16 ? 131072 : 65536;
};

template <int IM, int FM, int NT, int ALU_EVEN, int ALU_ODD, int WV>
__global__ __launch_bounds__(WV * 64) void k4_mfma_kernel(GemvArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t tab[TableKind<NT>::kBytes];
  // per wave: A fragments for the two quads of the current 128-row block [Qb][rh][m][g][8]
  __shared__ __attribute__((aligned(16))) _Float16 xa[WV * 2 * 2 * (2 * NT) * 4 * 8];

  if (TableKind<NT>::kF16)
    load_codebook16_lds<WV * 64>(tab);
  else
    load_codebook_lds_t<WV * 64>(tab);
  __syncthreads();
  const int wv = wave_id_uniform();
  k4_mfma_body<IM, FM, NT, ALU_EVEN, ALU_ODD, WV>(a, a.plan, tab, xa + wv * (2 * 2 * (2 * NT) * 4 * 8));
}

template <int IM, int FM, int NT, int ALU_EVEN, int ALU_ODD, int WV>
__device__ __forceinline__ void k4_mfma_body(const GemvArgs& a, const Plan* __restrict__ P,
                                             const uint8_t* __restrict__ tab, _Float16* __restrict__ xw) {
  // plan fields are read as wave-uniform values (the plan may sit in LDS), so the work split and
  // the loop bounds stay scalar
  const int U = uniform(P->units);
  const int it = a.in_f / 16;
  const int ups = it / 4;  // quads per segment
  const int obs = a.out_f / 128;
  const int nproj = a.nproj;
  const int64_t nseg = (int64_t)U * obs * nproj;
  const int64_t nq = nseg * ups;
  const int nw = gridDim.x * WV;
  const int wave = blockIdx.x * WV + wave_id_uniform();
  const int lane = lane_id();
  const int g = lane >> 4, nn = lane & 15;
  // quad counts fit 32 bits (<= 72 units x 64 column blocks x 2 projections x 1024 quads)
  const Split sp = make_split((int)nq, nw);
  const int q_begin = sp.start(wave), q_end = sp.start(wave + 1);

  // this lane's 16 B inside a chunk: tile 2s + n/8 at +256 s, word group n%8
  const int lane_off = (nn >> 3) * 128 + (nn & 7) * 16;
  const int src_lane = (lane & 7) == 0 ? lane + 7 : lane - 1;

  int visit = 0;
  for (int c = q_begin; c < q_end; visit++) {
    const int seg = c / ups;
    const int tq0 = c % ups;
    const int tq1 = min(ups, tq0 + (q_end - c));
    const int proj = seg % nproj;
    const int ob = (seg / nproj) % obs;
    const int u = seg / (nproj * obs);
    const int e = uniform(P->expert[u]);
    const int ntok = uniform(P->ntok[u]);
    const uint8_t* __restrict__ base = a.packed[proj];

    f32x4 acc[4][2];
#pragma unroll
    for (int s4 = 0; s4 < 4; s4++)
#pragma unroll
      for (int h = 0; h < 2; h++) acc[s4][h] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // the lane's piece of set s4 in quad tq is at quad_ptr(tq) + 256 * s4
    auto quad_ptr = [&](int tq) {
      return base + chunk_offset(a.side, e, ob, 4 * tq + g, it, obs) + lane_off;
    };
    auto load_quad = [&](u32x4(&pc)[4], int tq) {
      const uint8_t* qp = quad_ptr(tq);
#pragma unroll
      for (int s4 = 0; s4 < 4; s4++) pc[s4] = load_stream16(qp + 256 * s4);
    };
    // x of one 128-row block for every token of the unit is fetched one block ahead of its use
    // (raw words in registers) and turned into A fragments when its block starts.
    // (unconditional loads -- positions past the unit's tokens re-read its last token -- so the
    // compiler can count them against the piece loads instead of draining the queue)
    uint32_t nx[NT], nsc = 0;
    f32x2 nxd[NT];
    // source rows of the unit's token positions (positions past ntok repeat the last token),
    // fixed for the visit and kept in scalar registers
    const uint16_t* xrow[NT];
    const float* xrowd[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) {
      const int tt = min(t, ntok - 1);
      if (IM == IN_PREP) {
        const int row = __builtin_amdgcn_readfirstlane(a.x_per_slot ? P->slot[u][tt] : P->tok[u][tt]);
        xrow[t] = a.x_bf16 + (int64_t)row * a.in_f + 2 * lane;
      } else {
        const int slot = __builtin_amdgcn_readfirstlane(P->slot[u][tt]);
        xrowd[t] = a.x_f32 + (int64_t)slot * a.in_f + 2 * lane;
      }
    }
    const uint16_t* scrow = IM == IN_PREP ? a.in_scale[proj] + (int64_t)e * a.in_f + 2 * lane : nullptr;
    auto fetch_block = [&](int blk) {
      if (IM == IN_PREP) {
        nsc = *reinterpret_cast<const uint32_t*>(scrow + blk * 128);
#pragma unroll
        for (int t = 0; t < NT; t++) nx[t] = *reinterpret_cast<const uint32_t*>(xrow[t] + blk * 128);
      } else {
#pragma unroll
        for (int t = 0; t < NT; t++) nxd[t] = *reinterpret_cast<const f32x2*>(xrowd[t] + blk * 128);
      }
    };
    auto stage_block = [&]() {
      // fetched block -> xh -> fp16 hi/lo A fragments in the wave's LDS slice
      float v0[NT], v1[NT];
#pragma unroll
      for (int t = 0; t < NT; t++) {
        if (t < ntok) {
          if (IM == IN_PREP) {
            v0[t] = bf16_to_f32((uint16_t)(nx[t] & 0xFFFFu)) * f16_to_f32((uint16_t)(nsc & 0xFFFFu));
            v1[t] = bf16_to_f32((uint16_t)(nx[t] >> 16)) * f16_to_f32((uint16_t)(nsc >> 16));
            hadamard128_wave(v0[t], v1[t]);
          } else {
            v0[t] = nxd[t].x;
            v1[t] = nxd[t].y;
          }
        }
      }
#pragma unroll
      for (int jj = 0; jj < 2; jj++) {
        const int el = 2 * lane + jj;  // row within the 128-row block
        const int qb = el >> 6, gg = (el >> 4) & 3, r = el & 15;
        const int base_off = (qb * 2 + a_rh(r)) * (2 * NT);
#pragma unroll
        for (int t = 0; t < NT; t++) {
          if (t < ntok) {
            float xv = jj ? v1[t] : v0[t];
            // materialise x in fp32 first: otherwise the compiler may fuse the Hadamard scale into
            // one of the two f16 conversions below and round hi differently in each of them
            asm volatile("" : "+v"(xv));
            const _Float16 hi = (_Float16)xv;
            // the remainder is stored scaled by 2^11 so it stays a normal fp16 (the matrix cores
            // flush fp16 denormals); the lo row of the product is scaled back by 2^-11 (exact)
            const _Float16 lo = (_Float16)((xv - (float)hi) * 2048.0f);
            xw[((base_off + 2 * t) * 4 + gg) * 8 + a_j(r)] = hi;
            xw[((base_off + 2 * t + 1) * 4 + gg) * 8 + a_j(r)] = lo;
          }
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };

    // One quad in flight per wave: each piece's registers are refilled with the next quad's
    // piece once the piece has been decoded.  The last quad re-reads itself (a cache hit), so the
    // prefetch needs no branch.
    const int tl = tq1 - 1;
    u32x4 pc[4];
    load_quad(pc, tq0);
    fetch_block(tq0 >> 1);
    for (int tq = tq0; tq < tq1; tq++) {
      if (MOE_K4_PRIO) {
        // issue priority from the wave's remaining share of its range: the SIMD's arbiter favours
        // older waves, so without this the waves of a SIMD finish one after another
        const int left = q_end - (c + (tq - tq0));
        switch (min(3, (4 * left) / (q_end - q_begin + 1))) {
          case 3: __builtin_amdgcn_s_setprio(3); break;
          case 2: __builtin_amdgcn_s_setprio(2); break;
          case 1: __builtin_amdgcn_s_setprio(1); break;
          default: __builtin_amdgcn_s_setprio(0); break;
        }
      }
      if (tq == tq0 || (tq & 1) == 0) {
        stage_block();
        fetch_block(min((tq >> 1) + 1, tl >> 1));
      }
      f16x8 A[2];
      const int m = nn;
      const bool live = m < 2 * ntok;
#pragma unroll
      for (int rh = 0; rh < 2; rh++) {
        A[rh] = live ? *reinterpret_cast<const f16x8*>(xw + ((((tq & 1) * 2 + rh) * (2 * NT) + m) * 4 + g) * 8)
                     : f16x8{0, 0, 0, 0, 0, 0, 0, 0};
      }
      const uint8_t* np = quad_ptr(min(tq + 1, tl));
      // predecessors of the pieces' first words (last word of the lane before, within the tile),
      // fetched for the whole quad at once
      uint32_t prior[4];
#pragma unroll
      for (int s4 = 0; s4 < 4; s4++) prior[s4] = (uint32_t)__shfl((int)pc[s4].w, src_lane, 64);
#pragma unroll
      for (int s4 = 0; s4 < 4; s4++) {
        const u32x4 v = pc[s4];
#pragma unroll
        for (int rh = 0; rh < 2; rh++) {
          // words 2rh, 2rh+1 = rows of row half rh; h = 0: slots (0,1),(2,3) ; h = 1: slots (4,5),(6,7)
          f16x2 q[2][4];  // [word][pair]: (c0,c1), (c2,c3), (c4,c5), (c6,c7)
          if (rh == 0)
            decode_pair_words_f16<ALU_EVEN, ALU_ODD, TableKind<NT>::kF16>(v.x, v.y, prior[s4], tab, q);
          else
            decode_pair_words_f16<ALU_EVEN, ALU_ODD, TableKind<NT>::kF16>(v.z, v.w, v.y, tab, q);
          if (rh == 1) pc[s4] = load_stream16(np + 256 * s4);
          const f16x8 b0 = frag(q[0][0], q[0][1], q[1][0], q[1][1]);
          const f16x8 b1 = frag(q[0][2], q[0][3], q[1][2], q[1][3]);
          acc[s4][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[rh], b0, acc[s4][0], 0, 0, 0);
          acc[s4][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[rh], b1, acc[s4][1], 0, 0, 0);
          mfma_acc_guard(acc[s4][0], acc[s4][1]);
        }
      }
    }

    // partials of this visit: token t = D rows 2t + 2t+1, held by lanes 16*(t/2) + n, regs 2(t%2), +1
    float* pw = a.partial + ((int64_t)wave * 2 + visit) * kPartialStride;
#pragma unroll
    for (int t = 0; t < NT; t++) {
      if (t < ntok && g == (t >> 1)) {
        const int r0 = 2 * (t & 1);
#pragma unroll
        for (int s4 = 0; s4 < 4; s4++)
#pragma unroll
          for (int h = 0; h < 2; h++) {
            const int col = 16 * (2 * s4 + (nn >> 3)) + (nn & 7) + 8 * h;
            store_coherent(pw + t * 128 + col, fmaf(acc[s4][h][r0 + 1], 1.0f / 2048.0f, acc[s4][h][r0]));
          }
      }
    }
    complete_visit<FM>(a, P, seg, tq1 - tq0, ups, sp, nproj, U, u, ob, e, ntok);
    c += tq1 - tq0;
  }
}

// ============================================================== host side

namespace {

struct DeviceState {
  bool ready = false;
  int cus = 0;
  const uint8_t* codebook = nullptr;
  const uint16_t* codebook16 = nullptr;
};
std::mutex g_mutex;
DeviceState g_devices[64];
thread_local char g_error[512];
thread_local hipEvent_t g_prof_events[4];

}  // namespace

// Record the armed profiling event `slot` on `s` (and disarm it).
static void prof_mark(int slot, hipStream_t s) {
  if (g_prof_events[slot]) {
    (void)hipEventRecord(g_prof_events[slot], s);
    g_prof_events[slot] = nullptr;
  }
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code;
}

int ensure_device_ready() {
  int dev = 0;
  MOE_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= 64) return fail(MOE_ENOTSUP, "device index %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_mutex);
  DeviceState& st = g_devices[dev];
  if (st.ready) return MOE_OK;
  MOE_HIP(hipDeviceGetAttribute(&st.cus, hipDeviceAttributeMultiprocessorCount, dev));
  void* table = nullptr;
  MOE_HIP(hipGetSymbolAddress(&table, HIP_SYMBOL(g_codebook_e4m3)));
  st.codebook = static_cast<const uint8_t*>(table);
  void* table16 = nullptr;
  MOE_HIP(hipGetSymbolAddress(&table16, HIP_SYMBOL(g_codebook_f16)));
  st.codebook16 = static_cast<const uint16_t*>(table16);
  hipLaunchKernelGGL(build_codebook_kernel, dim3(128), dim3(256), 0, 0);
  MOE_HIP(hipGetLastError());
  MOE_HIP(hipDeviceSynchronize());
  st.ready = true;
  return MOE_OK;
}

const uint8_t* codebook_device_table() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  return g_devices[dev].codebook;
}

const uint16_t* codebook_f16_device_table() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  return g_devices[dev].codebook16;
}

int device_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  return g_devices[dev].cus;
}

namespace {
std::atomic<int> g_wait_polls{0};  // 0: the default bound
// Takes the stalled-launch count out of a flag word (the host has waited for the stream).
__global__ void clear_word_kernel(int32_t* p) {
  __hip_atomic_store(p, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
}  // namespace

int wait_polls() {
  const int v = g_wait_polls.load(std::memory_order_relaxed);
  return v > 0 ? v : kDefaultWaitPolls;
}

// ---------------------------------------------------------------- workspace layout
namespace {

struct Workspace {
  Plan* plan;
  int32_t* counter_seg; // per-segment chunk counters (self-cleaning)
  int32_t* counter_grp; // per-group segment counters (self-cleaning)
  int32_t* router_counter;
  float* partial;       // [kMaxWaves][2][kPartialStride]
  float* yslot;         // [kMaxUnits][hidden]
  float* down_xh;       // [kMaxUnits][inter]
  float* logits;        // [kMaxRows][256]
  uint32_t* ids;        // [kMaxRows][9]
  float* scores;        // [kMaxRows][8]
  uint16_t* hrow;       // [kMaxRows][hidden] layer residual T(x + attn) (moe_k4_layer_decode)
  uint16_t* xnrow;      // [kMaxRows][hidden] normalised expert input (moe_k4_layer_decode)
  void* layer;          // the fused decode block's region (k4_layer.hip)
  size_t bytes;
};

constexpr size_t kCounters = 4096;

size_t align_up(size_t v) { return (v + 255) & ~(size_t)255; }

Workspace carve(void* base, int hidden, int inter) {
  Workspace w{};
  size_t off = 0;
  char* p = static_cast<char*>(base);
  auto take = [&](size_t bytes) { char* r = p ? p + off : nullptr; off += align_up(bytes); return r; };
  w.plan = reinterpret_cast<Plan*>(take(sizeof(Plan)));
  w.counter_seg = reinterpret_cast<int32_t*>(take(kCounters * 4));
  w.counter_grp = reinterpret_cast<int32_t*>(take(kCounters * 4));
  w.router_counter = reinterpret_cast<int32_t*>(take(256));
  w.partial = reinterpret_cast<float*>(take((size_t)kMaxWaves * 2 * kPartialStride * 4));
  w.yslot = reinterpret_cast<float*>(take((size_t)kMaxUnits * hidden * 4));
  w.down_xh = reinterpret_cast<float*>(take((size_t)kMaxUnits * inter * 4));
  w.logits = reinterpret_cast<float*>(take((size_t)kMaxRows * 256 * 4));
  w.ids = reinterpret_cast<uint32_t*>(take((size_t)kMaxRows * 9 * 4));
  w.scores = reinterpret_cast<float*>(take((size_t)kMaxRows * 8 * 4));
  w.hrow = reinterpret_cast<uint16_t*>(take((size_t)kMaxRows * hidden * 2));
  w.xnrow = reinterpret_cast<uint16_t*>(take((size_t)kMaxRows * hidden * 2));
  w.layer = take(k4_layer_workspace_bytes(hidden, inter));
  w.bytes = off;
  return w;
}

int grid_blocks() {
  int cus = device_cus();
  return cus < 1 ? 1 : (cus > kMaxBlocks ? kMaxBlocks : cus);
}

// Every wave's static chunk range must span at most two segments (the partial buffer holds two
// visits per wave), which holds when the number of waves is at least the number of segments.
template <int IM, int FM>
int launch_gemv(const GemvArgs& a, int max_ntok, int max_units, hipStream_t stream) {
  const int64_t nseg_max = (int64_t)max_units * (a.out_f / 128) * a.nproj;
  if (nseg_max > kMaxWaves)
    return fail(MOE_ENOTSUP, "too many (unit, column block) segments: %lld > %d", (long long)nseg_max, kMaxWaves);
  {
    // single-token launches: the gate/up GEMV (IN_PREP) and the down GEMV may use their own
    // wave count and decode mix
    constexpr int kWv1 = IM == IN_PREP ? MOE_K4_WAVES_1_GU : MOE_K4_WAVES_1;
    constexpr int kEven1 = IM == IN_PREP ? MOE_K4_ALU_EVEN_1 : MOE_K4_ALU_EVEN_1_DN;
    constexpr int kOdd1 = IM == IN_PREP ? MOE_K4_ALU_ODD_1 : MOE_K4_ALU_ODD_1_DN;
    const int WV = max_ntok <= 1 ? kWv1 : MOE_K4_WAVES_8;
    // 16 waves per CU (4 per SIMD: the decode's VALU results arrive 16 clocks after issue) when
    // two blocks fit a CU; a block with the 128 KB fp16 table has a CU to itself
    const bool f16_table = max_ntok <= 1 ? TableKind<1>::kF16 : TableKind<kMaxRows>::kF16;
    int mblocks = grid_blocks() * (WV < 16 && !f16_table ? 16 / WV : 1);
    // at least one wave per segment, so no wave's range spans more than two segments
    const int mneed = (int)((nseg_max + WV - 1) / WV);
    if (mblocks < mneed) mblocks = mneed;
    if (mblocks * WV > kMaxWaves)
      return fail(MOE_ENOTSUP, "too many waves for the partial buffer (%d)", mblocks * WV);
    if (max_ntok <= 1)
      hipLaunchKernelGGL((k4_mfma_kernel<IM, FM, 1, kEven1, kOdd1, kWv1>), dim3(mblocks), dim3(WV * 64), 0, stream, a);
    else
      hipLaunchKernelGGL((k4_mfma_kernel<IM, FM, kMaxRows, MOE_K4_ALU_EVEN_8, MOE_K4_ALU_ODD_8, MOE_K4_WAVES_8>),
                         dim3(mblocks), dim3(WV * 64), 0, stream, a);
  }
  MOE_HIP(hipGetLastError());
  return MOE_OK;
}

// Typed SwiGLU over bf16 arrays, eight elements (16 bytes) per lane and step: the activation
// between the separate gate/up and down expert linears (exlr8/experts.py:183).
// Each element is read before it is written by the same lane, so out may alias gate or up.
__global__ __launch_bounds__(256) void swiglu_bf16_kernel(const uint16_t* gate, const uint16_t* up, int64_t n,
                                                          uint16_t* out) {
  const int64_t vecs = n / 8;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t v = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; v < vecs; v += stride) {
    const u32x4 g = *(const u32x4*)(gate + v * 8), u = *(const u32x4*)(up + v * 8);
    u32x4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      o[j] = pack_bf16_pair(swiglu_bf16(bf16_to_f32((uint16_t)(g[j] & 0xFFFFu)), bf16_to_f32((uint16_t)(u[j] & 0xFFFFu))),
                            swiglu_bf16(bf16_to_f32((uint16_t)(g[j] >> 16)), bf16_to_f32((uint16_t)(u[j] >> 16))));
    *(u32x4*)(out + v * 8) = o;
  }
  if (blockIdx.x == 0 && threadIdx.x < n - vecs * 8) {
    const int64_t i = vecs * 8 + threadIdx.x;
    out[i] = f32_to_bf16(swiglu_bf16(bf16_to_f32(gate[i]), bf16_to_f32(up[i])));
  }
}

// K-bit trellis tensors: h * m * k / 8 bytes per expert
int check_trellis_k(int64_t bytes, int k, int in_f, int out_f, int64_t* experts) {
  MOE_ARG(in_f > 0 && out_f > 0 && in_f % 128 == 0 && out_f % 128 == 0,
          "trellis dimensions must be positive multiples of 128");
  const int64_t size = (int64_t)in_f * out_f * k / 8;
  MOE_ARG(bytes > 0 && bytes % size == 0, "packed byte count does not match the trellis dimensions");
  *experts = bytes / size;
  return MOE_OK;
}

int check_trellis(int64_t bytes, int in_f, int out_f, int64_t* experts) {
  MOE_ARG(in_f > 0 && out_f > 0 && in_f % 128 == 0 && out_f % 128 == 0,
          "trellis dimensions must be positive multiples of 128");
  const int64_t size = (int64_t)in_f * out_f / 2;
  MOE_ARG(bytes > 0 && bytes % size == 0, "packed byte count does not match the trellis dimensions");
  *experts = bytes / size;
  return MOE_OK;
}

}  // namespace

}  // namespace moe

using namespace moe;

extern "C" {

const char* moe_version(void) { return "mlxlr8_amd 0.1.0 (gfx950)"; }
const char* moe_last_error(void) { return g_error; }

int moe_init(void) { return ensure_device_ready(); }

int moe_codebook_e4m3(uint8_t* dst, moe_stream_t stream) {
  MOE_ARG(dst != nullptr, "dst must not be NULL");
  int rc = ensure_device_ready();
  if (rc) return rc;
  hipLaunchKernelGGL(copy_codebook_kernel, dim3(256), dim3(256), 0, (hipStream_t)stream, dst);
  MOE_HIP(hipGetLastError());
  return MOE_OK;
}

int moe_set_wait_bound(int polls) {
  MOE_ARG(polls >= 0, "the wait bound must be >= 0 polls (0 restores the default), got %d", polls);
  g_wait_polls.store(polls, std::memory_order_relaxed);
  return MOE_OK;
}

int moe_decode_status(const void* workspace, int kind, int hidden, int intermediate, int32_t* stalled,
                      moe_stream_t stream) {
  MOE_ARG(stalled != nullptr, "stalled must not be NULL");
  MOE_ARG(kind >= MOE_STATUS_K4 && kind <= MOE_STATUS_MXFP4_NOALLOC, "unknown workspace kind %d", kind);
  MOE_ARG(kind == MOE_STATUS_MXFP4_NOALLOC || workspace != nullptr, "workspace must not be NULL");
  MOE_ARG(kind != MOE_STATUS_K4 || (hidden > 0 && intermediate > 0), "hidden and intermediate must be positive");
  int rc = ensure_device_ready();
  if (rc) return rc;
  int32_t* flags = nullptr;
  void* ws = const_cast<void*>(workspace);
  if (kind == MOE_STATUS_K4) {
    flags = k4_layer_flags(carve(ws, hidden, intermediate).layer, hidden, intermediate);
  } else if (kind == MOE_STATUS_MXFP4) {
    flags = mx_workspace_flags(ws, hidden, intermediate);
  } else if ((rc = mx_scratch_flags(&flags))) {
    return rc;
  }
  const hipStream_t s = (hipStream_t)stream;
  int32_t v = 0;
  MOE_HIP(hipMemcpyAsync(&v, flags + LF_STALLED, sizeof(v), hipMemcpyDeviceToHost, s));
  MOE_HIP(hipStreamSynchronize(s));
  if (v != 0) {
    hipLaunchKernelGGL(clear_word_kernel, dim3(1), dim3(1), 0, s, flags + LF_STALLED);
    MOE_HIP(hipGetLastError());
  }
  *stalled = v;
  return MOE_OK;
}

int moe_k4_item_list(int hidden, int intermediate, int units, int route, int32_t* items, int capacity) {
  return k4_layer_item_list(hidden, intermediate, units, route, items, capacity);
}

int moe_profile_events(void** events, int count) {
  MOE_ARG(count >= 0 && count <= 4, "count must be in 0..4");
  for (int i = 0; i < 4; i++) g_prof_events[i] = (events && i < count) ? (hipEvent_t)events[i] : nullptr;
  return MOE_OK;
}

size_t moe_workspace_bytes(int hidden, int intermediate) {
  (void)hidden;
  return carve(nullptr, hidden > 0 ? hidden : 1, intermediate > 0 ? intermediate : 1).bytes;
}

int moe_trellis_decode_f16(const void* packed, int64_t packed_bytes, int k, int in_f, int out_f, int side,
                           int64_t expert, uint16_t* inner, moe_stream_t stream) {
  MOE_ARG(k >= 2 && k <= 4, "EXLR8 trellis width must be 2, 3, or 4 (got k=%d)", k);
  MOE_ARG(side >= 0 && side <= 2, "sharded_side must be 0, 1, or 2");
  MOE_ARG(packed && inner, "packed and inner must not be NULL");
  int64_t experts = 0;
  int rc = check_trellis(packed_bytes * 4 / k, in_f, out_f, &experts);  // same tile count as K4 bytes
  if (rc) return rc;
  MOE_ARG(packed_bytes % ((int64_t)in_f * out_f * k / 8) == 0, "packed byte count does not match the trellis dimensions");
  MOE_ARG(expert >= 0 && expert < experts, "expert %lld out of range (%lld experts)", (long long)expert,
          (long long)experts);
  rc = ensure_device_ready();
  if (rc) return rc;
  if (k == 3) {
    const int64_t pieces = (int64_t)in_f * out_f / 32;
    hipLaunchKernelGGL(trellis_decode_k3_kernel, dim3((unsigned)((pieces + 1023) / 1024)), dim3(1024), 0,
                       (hipStream_t)stream, (const uint32_t*)packed, in_f, out_f, side, expert, inner);
    MOE_HIP(hipGetLastError());
    return MOE_OK;
  }
  if (k != 4) {
    const int64_t n = (int64_t)in_f * out_f;
    hipLaunchKernelGGL(trellis_decode_generic_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, (const uint32_t*)packed, k, in_f, out_f, side, expert, inner);
    MOE_HIP(hipGetLastError());
    return MOE_OK;
  }
  const int64_t pieces = (int64_t)in_f * out_f / 32;
  const dim3 grid((unsigned)((pieces + 1023) / 1024));
  hipLaunchKernelGGL(trellis_decode_kernel<false>, grid, dim3(1024), 0, (hipStream_t)stream,
                     (const uint32_t*)packed, in_f, out_f, side, expert, inner);
  if (grid.x > 1)
    hipLaunchKernelGGL(trellis_decode_kernel<true>, grid, dim3(1024), 0, (hipStream_t)stream,
                       (const uint32_t*)packed, in_f, out_f, side, expert, inner);
  MOE_HIP(hipGetLastError());
  return MOE_OK;
}

static int validate_ws(void* workspace, size_t bytes, int hidden, int inter) {
  MOE_ARG(workspace != nullptr, "workspace must not be NULL");
  const size_t need = carve(nullptr, hidden, inter).bytes;
  if (bytes < need) return fail(MOE_EWORKSPACE, "workspace too small: %zu < %zu bytes", bytes, need);
  return MOE_OK;
}

int moe_swiglu_bf16(const uint16_t* gate, const uint16_t* up, int64_t n, uint16_t* out, moe_stream_t stream) {
  MOE_ARG(n >= 0, "element count must not be negative");
  if (n == 0) return MOE_OK;
  MOE_ARG(gate && up && out, "gate, up and out must not be NULL");
  MOE_ARG(((uintptr_t)gate | (uintptr_t)up | (uintptr_t)out) % 16 == 0, "bf16 arrays must be 16-byte aligned");
  int rc = ensure_device_ready();
  if (rc) return rc;
  const int64_t blocks = std::min<int64_t>(std::max<int64_t>((n / 8 + 255) / 256, 1), 4096);
  hipLaunchKernelGGL(swiglu_bf16_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, gate, up, n, out);
  MOE_HIP(hipGetLastError());
  return MOE_OK;
}

int moe_k4_expert_linear(const uint16_t* x, int x_per_slot, const uint32_t* ids, int rows, int slots,
                         const void* packed, int64_t packed_bytes, const uint16_t* in_scale,
                         const uint16_t* out_scale, int in_f, int out_f, int side, uint16_t* y, void* workspace,
                         size_t workspace_bytes, moe_stream_t stream) {
  MOE_ARG(x && ids && packed && in_scale && out_scale && y, "null pointer argument");
  MOE_ARG(rows >= 1 && slots >= 1 && slots <= kSlots && rows * slots <= kMaxUnits,
          "rows*slots must be in 1..%d with slots <= %d", kMaxUnits, kSlots);
  MOE_ARG(side >= 0 && side <= 2, "sharded_side must be 0, 1, or 2");
  int64_t experts = 0;
  int rc = check_trellis(packed_bytes, in_f, out_f, &experts);
  if (rc) return rc;
  const int wdim = out_f > in_f ? out_f : in_f;
  if ((rc = validate_ws(workspace, workspace_bytes, wdim, wdim))) return rc;
  if ((rc = ensure_device_ready())) return rc;
  Workspace w = carve(workspace, wdim, wdim);
  hipStream_t s = (hipStream_t)stream;
  const int max_users = (x_per_slot || rows == 1) ? 1 : kMaxRows;
  hipLaunchKernelGGL(plan_kernel, dim3(1), dim3(128), 0, s, ids, rows, slots, (int)(experts > 257 ? 257 : experts),
                     max_users, w.plan);
  MOE_HIP(hipGetLastError());
  GemvArgs a{};
  a.packed[0] = (const uint8_t*)packed;
  a.nproj = 1;
  a.in_f = in_f; a.out_f = out_f; a.side = side;
  a.x_per_slot = x_per_slot;
  a.x_bf16 = x;
  a.in_scale[0] = in_scale;
  a.plan = w.plan;
  a.partial = w.partial;
  a.counter_seg = w.counter_seg;
  a.counter_grp = w.counter_grp;
  a.out_scale[0] = out_scale;
  a.values = y;
  return launch_gemv<IN_PREP, FIN_VALUES>(a, max_users, rows * slots, s);
}

// The routed decode block in one fused launch: with norm_w, h = T(x + attn) (attn may be NULL) and
// the block runs on RMSNorm(h) with residual h; otherwise on x with `residual`.  Every argument is
// checked before the first launch.
static int k4_block(const uint16_t* x, const uint16_t* attn, const uint16_t* norm_w, float eps,
                    const uint16_t* residual, int rows, const float* router_w, const float* bias, const void* pg,
                    const void* pu, const void* pd, int64_t bytes, const uint16_t* in_g, const uint16_t* out_g,
                    const uint16_t* in_u, const uint16_t* out_u, const uint16_t* in_d, const uint16_t* out_d, int h,
                    int m, uint16_t* out, uint32_t* indices, float* scores, void* workspace, size_t workspace_bytes,
                    hipStream_t s, int bits = 4) {
  MOE_ARG(x && router_w && bias && out && pg && pu && pd && in_g && out_g && in_u && out_u && in_d && out_d,
          "null pointer argument");
  MOE_ARG(norm_w || residual, "null pointer argument");
  MOE_ARG(rows >= 1 && rows <= kMaxRows, "rows must be in 1..%d", kMaxRows);
  MOE_ARG(bits == 3 || bits == 4, "the decode block takes K3 or K4 experts (got k=%d)", bits);
  MOE_ARG(bits == 4 || !norm_w, "the fused residual + RMSNorm is built for K4 experts only");
  int64_t experts = 0;
  int rc = check_trellis_k(bytes, bits, h, m, &experts);
  if (rc) return rc;
  MOE_ARG(experts == 257, "the routed decode block needs 256 routed experts plus the shared expert (got %lld)",
          (long long)experts);
  MOE_ARG(k4_layer_supported(h, m, true),
          "hidden must be a multiple of 1024 up to 8192 (fused router) and intermediate a multiple of 128 (got %d, %d)",
          h, m);
  {
    const uint16_t* ins[3] = {in_g, in_u, in_d};
    const uint16_t* outs[3] = {out_g, out_u, out_d};
    if ((rc = k4_layer_check_alignment(norm_w ? nullptr : x, residual, ins, outs, out, nullptr))) return rc;
  }
  if ((rc = validate_ws(workspace, workspace_bytes, h, m))) return rc;
  if ((rc = ensure_device_ready())) return rc;
  Workspace w = carve(workspace, h, m);
  uint32_t* ids = indices ? indices : w.ids;
  float* sc = scores ? scores : w.scores;
  const uint16_t* xin = x;
  const uint16_t* res = residual;
  prof_mark(0, s);
  // one row: the residual add + RMSNorm runs at the start of the fused block (same bits as the
  // norm kernel); more rows: the norm kernel first
  LayerNorm ln{x, attn, norm_w, eps};
  const bool fold = MOE_FOLD_NORM && norm_w && rows == 1 && h % 2048 == 0;
  if (norm_w) {
    if (!fold && (rc = moe_residual_rmsnorm(x, attn, norm_w, rows, h, eps, w.hrow, w.xnrow, (moe_stream_t)s))) return rc;
    xin = w.xnrow;
    res = w.hrow;
  }
  const uint8_t* packed[3] = {(const uint8_t*)pg, (const uint8_t*)pu, (const uint8_t*)pd};
  const uint16_t* ins[3] = {in_g, in_u, in_d};
  const uint16_t* outs[3] = {out_g, out_u, out_d};
  prof_mark(1, s);
  rc = k4_layer_run(xin, res, rows, 1, router_w, bias, ids, sc, packed, ins, outs, h, m, 257, 1, out, nullptr,
                    w.layer, s, fold ? &ln : nullptr, bits);
  prof_mark(3, s);
  return rc;
}

static int k4_mlp_common(const uint16_t* x, const uint32_t* ids, const float* scores, const uint16_t* residual,
                         int rows, int slots, const void* pg, const void* pu, const void* pd, int64_t bytes,
                         const uint16_t* in_g, const uint16_t* out_g, const uint16_t* in_u, const uint16_t* out_u,
                         const uint16_t* in_d, const uint16_t* out_d, int h, int m, uint16_t* values, uint16_t* out,
                         void* workspace, size_t workspace_bytes, hipStream_t s, int bits = 4) {
  MOE_ARG(x && ids && pg && pu && pd && in_g && out_g && in_u && out_u && in_d && out_d, "null pointer argument");
  MOE_ARG(rows >= 1 && rows <= kMaxRows && slots >= 1 && slots <= kSlots,
          "rows must be in 1..%d and slots in 1..%d", kMaxRows, kSlots);
  MOE_ARG(bits == 3 || bits == 4, "the decode MLP takes K3 or K4 experts (got k=%d)", bits);
  int64_t experts = 0;
  int rc = check_trellis_k(bytes, bits, h, m, &experts);
  if (rc) return rc;
  MOE_ARG(experts >= 1, "no experts");
  MOE_ARG(k4_layer_supported(h, m, false), "hidden and intermediate must be multiples of 128 (got %d, %d)", h, m);
  if (out) MOE_ARG(slots == kSlots && scores && residual, "the combined finish needs 9 slots, scores and residual");
  {
    const uint16_t* ins[3] = {in_g, in_u, in_d};
    const uint16_t* outs[3] = {out_g, out_u, out_d};
    if ((rc = k4_layer_check_alignment(x, residual, ins, outs, out, values))) return rc;
  }
  if ((rc = validate_ws(workspace, workspace_bytes, h, m))) return rc;
  if ((rc = ensure_device_ready())) return rc;
  Workspace w = carve(workspace, h, m);
  const int max_users = rows == 1 ? 1 : kMaxRows;
  const int ecount = (int)(experts > 257 ? 257 : experts);
  hipLaunchKernelGGL(plan_kernel, dim3(1), dim3(128), 0, s, ids, rows, slots, ecount, max_users,
                     k4_layer_plan(w.layer));
  MOE_HIP(hipGetLastError());
  const uint8_t* packed[3] = {(const uint8_t*)pg, (const uint8_t*)pu, (const uint8_t*)pd};
  const uint16_t* ins[3] = {in_g, in_u, in_d};
  const uint16_t* outs[3] = {out_g, out_u, out_d};
  prof_mark(1, s);
  rc = k4_layer_run(x, residual, rows, 0, nullptr, nullptr, nullptr, const_cast<float*>(scores), packed, ins, outs, h,
                    m, ecount, out != nullptr, out, values, w.layer, s, nullptr, bits);
  prof_mark(3, s);
  return rc;
}

int moe_k4_mlp(const uint16_t* x, const uint32_t* ids, int rows, int slots, const void* packed_gate,
               const void* packed_up, const void* packed_down, int64_t packed_bytes, const uint16_t* in_gate,
               const uint16_t* out_gate, const uint16_t* in_up, const uint16_t* out_up, const uint16_t* in_down,
               const uint16_t* out_down, int hidden, int intermediate, uint16_t* values, void* workspace,
               size_t workspace_bytes, moe_stream_t stream) {
  MOE_ARG(values != nullptr, "values must not be NULL");
  return k4_mlp_common(x, ids, nullptr, nullptr, rows, slots, packed_gate, packed_up, packed_down, packed_bytes,
                       in_gate, out_gate, in_up, out_up, in_down, out_down, hidden, intermediate, values, nullptr,
                       workspace, workspace_bytes, (hipStream_t)stream);
}

int moe_k4_mlp_finish(const uint16_t* x, const uint32_t* ids, const float* scores, const uint16_t* residual, int rows,
                      const void* packed_gate, const void* packed_up, const void* packed_down, int64_t packed_bytes,
                      const uint16_t* in_gate, const uint16_t* out_gate, const uint16_t* in_up,
                      const uint16_t* out_up, const uint16_t* in_down, const uint16_t* out_down, int hidden,
                      int intermediate, uint16_t* out, void* workspace, size_t workspace_bytes,
                      moe_stream_t stream) {
  MOE_ARG(out != nullptr, "out must not be NULL");
  return k4_mlp_common(x, ids, scores, residual, rows, kSlots, packed_gate, packed_up, packed_down, packed_bytes,
                       in_gate, out_gate, in_up, out_up, in_down, out_down, hidden, intermediate, nullptr, out,
                       workspace, workspace_bytes, (hipStream_t)stream);
}

int moe_k4_moe_decode(const uint16_t* x, const uint16_t* residual, int rows, const float* router_w, const float* bias,
                      const void* packed_gate, const void* packed_up, const void* packed_down, int64_t packed_bytes,
                      const uint16_t* in_gate, const uint16_t* out_gate, const uint16_t* in_up,
                      const uint16_t* out_up, const uint16_t* in_down, const uint16_t* out_down, int hidden,
                      int intermediate, uint16_t* out, uint32_t* indices, float* scores, void* workspace,
                      size_t workspace_bytes, moe_stream_t stream) {
  return k4_block(x, nullptr, nullptr, 0.0f, residual, rows, router_w, bias, packed_gate, packed_up, packed_down,
                  packed_bytes, in_gate, out_gate, in_up, out_up, in_down, out_down, hidden, intermediate, out, indices,
                  scores, workspace, workspace_bytes, (hipStream_t)stream);
}

int moe_trellis_mlp(int k, const uint16_t* x, const uint32_t* ids, int rows, int slots, const void* packed_gate,
                    const void* packed_up, const void* packed_down, int64_t packed_bytes, const uint16_t* in_gate,
                    const uint16_t* out_gate, const uint16_t* in_up, const uint16_t* out_up, const uint16_t* in_down,
                    const uint16_t* out_down, int hidden, int intermediate, uint16_t* values, void* workspace,
                    size_t workspace_bytes, moe_stream_t stream) {
  MOE_ARG(values != nullptr, "values must not be NULL");
  return k4_mlp_common(x, ids, nullptr, nullptr, rows, slots, packed_gate, packed_up, packed_down, packed_bytes,
                       in_gate, out_gate, in_up, out_up, in_down, out_down, hidden, intermediate, values, nullptr,
                       workspace, workspace_bytes, (hipStream_t)stream, k);
}

int moe_trellis_mlp_finish(int k, const uint16_t* x, const uint32_t* ids, const float* scores,
                           const uint16_t* residual, int rows, const void* packed_gate, const void* packed_up,
                           const void* packed_down, int64_t packed_bytes, const uint16_t* in_gate,
                           const uint16_t* out_gate, const uint16_t* in_up, const uint16_t* out_up,
                           const uint16_t* in_down, const uint16_t* out_down, int hidden, int intermediate,
                           uint16_t* out, void* workspace, size_t workspace_bytes, moe_stream_t stream) {
  MOE_ARG(out != nullptr, "out must not be NULL");
  return k4_mlp_common(x, ids, scores, residual, rows, kSlots, packed_gate, packed_up, packed_down, packed_bytes,
                       in_gate, out_gate, in_up, out_up, in_down, out_down, hidden, intermediate, nullptr, out,
                       workspace, workspace_bytes, (hipStream_t)stream, k);
}

int moe_trellis_moe_decode(int k, const uint16_t* x, const uint16_t* residual, int rows, const float* router_w,
                           const float* bias, const void* packed_gate, const void* packed_up, const void* packed_down,
                           int64_t packed_bytes, const uint16_t* in_gate, const uint16_t* out_gate,
                           const uint16_t* in_up, const uint16_t* out_up, const uint16_t* in_down,
                           const uint16_t* out_down, int hidden, int intermediate, uint16_t* out, uint32_t* indices,
                           float* scores, void* workspace, size_t workspace_bytes, moe_stream_t stream) {
  return k4_block(x, nullptr, nullptr, 0.0f, residual, rows, router_w, bias, packed_gate, packed_up, packed_down,
                  packed_bytes, in_gate, out_gate, in_up, out_up, in_down, out_down, hidden, intermediate, out, indices,
                  scores, workspace, workspace_bytes, (hipStream_t)stream, k);
}

int moe_k4_layer_decode(const uint16_t* x, const uint16_t* attn, const uint16_t* norm_w, float eps, int rows,
                        const float* router_w, const float* bias, const void* packed_gate, const void* packed_up,
                        const void* packed_down, int64_t packed_bytes, const uint16_t* in_gate,
                        const uint16_t* out_gate, const uint16_t* in_up, const uint16_t* out_up,
                        const uint16_t* in_down, const uint16_t* out_down, int hidden, int intermediate,
                        uint16_t* out, uint32_t* indices, float* scores, void* workspace, size_t workspace_bytes,
                        moe_stream_t stream) {
  MOE_ARG(norm_w != nullptr, "null pointer argument");
  MOE_ARG(eps >= 0.0f, "epsilon must be non-negative");
  MOE_ARG(hidden % 2048 == 0 && hidden <= 8192, "layer width must be a multiple of 2048 up to 8192 (got %d)", hidden);
  return k4_block(x, attn, norm_w, eps, nullptr, rows, router_w, bias, packed_gate, packed_up, packed_down,
                  packed_bytes, in_gate, out_gate, in_up, out_up, in_down, out_down, hidden, intermediate, out, indices,
                  scores, workspace, workspace_bytes, (hipStream_t)stream);
}

}  // extern "C"
