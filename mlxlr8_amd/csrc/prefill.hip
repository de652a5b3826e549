// Joined-MXFP4 expert path for prefill chunks on gfx950: sorted-by-expert grouped GEMMs on the
// scaled MX MFMA (v_mfma_scale_f32_16x16x128_f8f6f4, activations fp8 x weights fp4).
//
// Reference semantics (paths relative to the reference root):
//   sorted work order: argsort of the flat expert ids, per-expert counts/starts and a block table
//     (expert, first, length)                                   exlr8/fast_prefill.py:19-46
//   xh = H128(x * unit) per token                                exlr8/joined_mxfp4.py:96
//   gu = xh @ W_gate_up[e]^T, grouped by expert (gather_qmm)     exlr8/joined_mxfp4.py:98-113
//   hidden = H128(swiglu_T(H(g)*og, H(u)*ou) * in_down)         exlr8/metal/joined_gate_finish.metal
//   v = hidden @ W_down[e]^T                                      exlr8/joined_mxfp4.py:121-134
//   value = T(H128(v) * out_down); out = T(T(sum_i value_i*score_i) + shared) + residual
//                                                                 exlr8/model.py:415-418
//
// MI355X design:
//   * Activations are split as x = hi + lo1 + lo2 with hi = f16(x) and the remainder in two fp8
//     (e4m3) terms, each with an e8m0 scale per 32 values (~20 significant bits in all: the bf16
//     casts of gate/up and of the values then flip as rarely as with fp32 activations).  hi runs on
//     the fp16 matrix cores (v_mfma_f32_16x16x32_f16) against the weights widened to fp16 in
//     registers (v_cvt_scalef32_pk_f16_fp4 applies the block scale; exact for e8m0 scales
//     114..140); lo1 and lo2 run on the scaled MX matrix cores (v_mfma_scale_f32_16x16x128_f8f6f4,
//     fp8 x MXFP4) with the resident codes and both block scales.  The scaled MX instruction keeps
//     only ~15 bits across its 128-product sums, ample for the < 2^-11 remainder but not for the
//     whole value; all terms go into one fp32 accumulator.
//   * Operand layout of the 16x16x128 scaled MFMA (measured on gfx950): lane l holds row/column
//     l%16; fp8 A bytes 0-15 are k = 16(l/16)+j and bytes 16-31 are k = 64+16(l/16)+j-16; fp4 B
//     nibble j (low nibble first) is k = 32(l/16)+j; lane l's scale byte scales k-block l/16.  The
//     fp16 MFMAs of a 128-wide k step reuse the lane's 32 widened weights: MFMA q (q = 0..3) maps
//     its k-group kg = l/16 to k = 32 kg + 8q + i, and the staged hi activations are read to match.
//   * A work item is (block of <= 64 sorted rows of one expert, output block): the weights of the
//     output block are streamed once per item with 16 B loads per lane; the item's activation
//     terms for one 128-wide k step are staged in LDS (double buffered) and shared by the 8 waves.
//   * The gate finish (both 128-column halves of an intermediate block are in one item) and the
//     down finish (H128 over the item's 128 output columns) run in the GEMM epilogues through LDS;
//     the gate epilogue writes the down GEMM's fp8 terms directly.
#include <hip/hip_runtime.h>

#include "moe_device.h"
#include "moe_host.h"

namespace moe {
namespace {

typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f16x8 pack_f16x8(f16x2 a, f16x2 b, f16x2 c, f16x2 d) {
  typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
  const f16x4 ab = __builtin_shufflevector(a, b, 0, 1, 2, 3), cd = __builtin_shufflevector(c, d, 0, 1, 2, 3);
  return __builtin_shufflevector(ab, cd, 0, 1, 2, 3, 4, 5, 6, 7);
}

constexpr int kPfItemRows = 64;  // sorted rows per GEMM work item (4 M-tiles of 16)
constexpr int kPfWaves = 8;      // waves per GEMM block
constexpr int kPfThreads = kPfWaves * 64;
constexpr int kPfRowBytes = 528; // LDS row stride of a staged k step: 256 B hi + 2 x 128 B lo + pad
constexpr int kPfLo = 2;         // fp8 remainder terms
constexpr int kPfMaxExperts = 1024;
constexpr size_t kPfMaxLds = 160 * 1024;  // LDS per workgroup on gfx950
#ifndef MOE_PF_MERGE_GATE
#define MOE_PF_MERGE_GATE 1
#endif
#ifndef MOE_PF_DOWN_TWO
#define MOE_PF_DOWN_TWO 1
#endif
#ifndef MOE_PF_MERGE_DOWN
#define MOE_PF_MERGE_DOWN 0
#endif

// ---------------------------------------------------------------- sorted work order
// One block of 1024 threads (16 waves).  Counting sort of the flat ids (stable: slots of one
// expert keep their order), per-expert counts and starts, and the block table of `block_rows`
// rows.  Wave w owns the contiguous slice [w n / 16, (w + 1) n / 16) of the ids: it counts its
// slice into its own histogram row, the rows are turned into per-wave write offsets, and each wave
// then places its slice in order (the rank among equal ids inside a 64-id chunk comes from
// matching the ids bit by bit with ballots), all waves at once.
// clamp: an id outside [0, experts) is taken as the nearest valid expert (the grouped MLP and
// linear entries, like the decode entries); otherwise it is skipped (moe_segment_table).
__global__ __launch_bounds__(1024) void segment_table_kernel(const uint32_t* __restrict__ ids, int n, int experts,
                                                             int block_rows, int32_t* __restrict__ order,
                                                             int32_t* __restrict__ counts,
                                                             int32_t* __restrict__ starts, int32_t* __restrict__ blk,
                                                             int cap, int32_t* __restrict__ nblk, int clamp) {
  __shared__ int32_t hist[16][kPfMaxExperts];  // per wave: counts, then write offsets
  __shared__ int32_t cnt[kPfMaxExperts], st[kPfMaxExperts], bst[kPfMaxExperts];
  __shared__ int32_t wsum[16];
  const int tid = threadIdx.x, lane = lane_id(), wv = wave_id_uniform();
  for (int i = tid; i < 16 * kPfMaxExperts; i += 1024) (&hist[0][0])[i] = 0;
  __syncthreads();
  const int s0 = (int)((int64_t)n * wv / 16), s1 = (int)((int64_t)n * (wv + 1) / 16);
  // ids outside [0, experts) are clamped or skipped (no position)
  auto id_at = [&](int i) {
    const uint32_t e = ids[i];
    return clamp ? (uint32_t)min(max((int)e, 0), experts - 1) : e;  // as the decode entries: signed id
  };
  for (int i = s0 + lane; i < s1; i += 64) {
    const uint32_t e = id_at(i);
    if (e < (uint32_t)experts) atomicAdd(&hist[wv][e], 1);
  }
  __syncthreads();
  // per expert: total, then the running offsets of the waves' slices (in wave order)
  for (int e = tid; e < experts; e += 1024) {
    int c = 0;
#pragma unroll
    for (int w = 0; w < 16; w++) c += hist[w][e];
    cnt[e] = c;
  }
  __syncthreads();
  // exclusive scans of the counts and of the per-expert block counts (experts <= 1024: one per thread)
  {
    const int c = tid < experts ? cnt[tid] : 0;
    const int b = tid < experts ? (c + block_rows - 1) / block_rows : 0;
    int ic = c, ib = b;  // inclusive wave scans
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int oc = __shfl_up(ic, d, 64), ob = __shfl_up(ib, d, 64);
      if (lane >= d) { ic += oc; ib += ob; }
    }
    if (lane == 63) wsum[wv] = ic;
    __syncthreads();
    int offc = 0;
    for (int w = 0; w < wv; w++) offc += wsum[w];
    __syncthreads();
    if (lane == 63) wsum[wv] = ib;
    __syncthreads();
    int offb = 0;
    for (int w = 0; w < wv; w++) offb += wsum[w];
    if (tid < experts) {
      const int start = offc + ic - c;
      st[tid] = start;
      bst[tid] = offb + ib - b;
      counts[tid] = c;
      starts[tid] = start;
      int run = start;
#pragma unroll
      for (int w = 0; w < 16; w++) {
        const int h = hist[w][tid];
        hist[w][tid] = run;
        run += h;
      }
    }
    if (tid == 1023) *nblk = offb + ib;
  }
  __syncthreads();
  // stable placement of each wave's slice, 64 ids at a time; ids are matched on 11 bits (valid ids
  // are < 1024, invalid ones are given the key 2047 and not placed)
  for (int c0 = s0; c0 < s1; c0 += 64) {
    const int i = c0 + lane;
    const uint32_t e = i < s1 ? id_at(i) : 0xFFFFFFFFu;
    const bool valid = e < (uint32_t)experts;
    const uint32_t key = valid ? e : 2047u;
    uint64_t same = __ballot(1);
#pragma unroll
    for (int bit = 0; bit < 11; bit++) {
      const bool on = (key >> bit) & 1u;
      const uint64_t bal = __ballot(on);
      same &= on ? bal : ~bal;
    }
    const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    const int rank = __popcll(same & below);
    if (valid) order[hist[wv][e] + rank] = i;
    __builtin_amdgcn_wave_barrier();
    if (valid && rank == 0) hist[wv][e] += __popcll(same);
    __builtin_amdgcn_wave_barrier();
  }
  // block table rows (expert, first, length)
  for (int e = tid; e < experts; e += 1024) {
    const int c = cnt[e];
    for (int f = 0, b = bst[e]; f < c; f += block_rows, b++) {
      if (b < cap) {
        blk[b] = e;
        blk[cap + b] = st[e] + f;
        blk[2 * cap + b] = min(block_rows, c - f);
      }
    }
  }
}

// ---------------------------------------------------------------- fp8 terms of activations
// 32 values held as 2 per lane by 16 lanes (one DPP row): max magnitude of the row.
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_f32<0xB1>(v));   // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp_f32<0x4E>(v));   // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp_f32<0x124>(v));  // row_ror:4
  v = fmaxf(v, dpp_f32<0x128>(v));  // row_ror:8
  return v;
}
// Split (v0, v1) of a 32-value group (the 16 lanes of a DPP row) into hi = f16 pair (returned as
// bits) and the remainder as kPfLo fp8 terms: lo[t] holds the term's two codes (bytes 0, 1) and
// scale[t] the group's e8m0 scale of term t (each term rounds the previous remainder).
__device__ __forceinline__ uint32_t hi_lo_terms(float v0, float v1, uint32_t (&lo)[kPfLo], uint32_t (&scale)[kPfLo]) {
  const _Float16 h0 = (_Float16)v0, h1 = (_Float16)v1;
  float r0 = v0 - (float)h0, r1 = v1 - (float)h1;  // exact
#pragma unroll
  for (int t = 0; t < kPfLo; t++) {
    const float amax = row16_max(fmaxf(fabsf(r0), fabsf(r1)));
    // scale 2^s with amax / 2^s in [128, 256): the e4m3 range (448) is never exceeded
    int s = 0;
    if (amax > 0.0f) s = (int)((__float_as_uint(amax) >> 23) & 0xFF) - 127 - 7;
    s = max(-127, min(127, s));
    const i16x2 old = {0, 0};
    const uint32_t codes =
        __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pk_fp8_f32(__builtin_amdgcn_ldexpf(r0, -s),
                                                                     __builtin_amdgcn_ldexpf(r1, -s),
                                                                     __builtin_bit_cast(int, old), false)) &
        0xFFFFu;
    lo[t] = codes;
    scale[t] = (uint32_t)(s + 127);
    const f32x2 d = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(codes, 1.0f, false);
    r0 -= __builtin_amdgcn_ldexpf(d.x, s);  // exact: the code is r0's rounding at this scale
    r1 -= __builtin_amdgcn_ldexpf(d.y, s);
  }
  return (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
}

// xh = H128(x * unit) of every token -> hi/lo terms.  One wave per (token, 128-block).
// xh_hi: [rows][K] fp16, xq: [kPfLo][rows][K] fp8 remainder terms, xs: [kPfLo][rows][K/32] e8m0.
__global__ __launch_bounds__(256) void prep_terms_kernel(const uint16_t* __restrict__ x,
                                                         const uint16_t* __restrict__ unit, int rows, int K,
                                                         uint16_t* __restrict__ xh_hi, uint8_t* __restrict__ xq,
                                                         uint8_t* __restrict__ xs) {
  const int64_t wid = (int64_t)blockIdx.x * 4 + wave_id_uniform();
  const int blocks = K / 128;
  if (wid >= (int64_t)rows * blocks) return;
  const int t = (int)(wid / blocks), b = (int)(wid % blocks);
  const int lane = lane_id();
  const int k0 = b * 128 + 2 * lane;
  const uint32_t xv = *reinterpret_cast<const uint32_t*>(x + (int64_t)t * K + k0);
  const uint32_t uv = *reinterpret_cast<const uint32_t*>(unit + k0);
  float v0 = bf16_to_f32((uint16_t)(xv & 0xFFFFu)) * f16_to_f32((uint16_t)(uv & 0xFFFFu));
  float v1 = bf16_to_f32((uint16_t)(xv >> 16)) * f16_to_f32((uint16_t)(uv >> 16));
  hadamard128_wave(v0, v1);
  uint32_t lo[kPfLo], sc[kPfLo];
  const uint32_t hi = hi_lo_terms(v0, v1, lo, sc);
  *reinterpret_cast<uint32_t*>(xh_hi + (int64_t)t * K + k0) = hi;
#pragma unroll
  for (int tt = 0; tt < kPfLo; tt++) {
    *reinterpret_cast<uint16_t*>(xq + ((int64_t)tt * rows + t) * K + k0) = (uint16_t)lo[tt];
    if ((lane & 15) == 0) xs[((int64_t)tt * rows + t) * (K / 32) + b * 4 + lane / 16] = (uint8_t)sc[tt];
  }
}

// ---------------------------------------------------------------- grouped GEMM machinery
struct PfGemm {
  // weights (MXFP4): codes [E][N][K/2], scales [E][N][K/32]
  const uint8_t* codes;
  const uint8_t* wscales;
  int K, N;
  // activation terms: ahi [arows][K] fp16, aq [kPfLo][arows][K] fp8 remainder terms,
  // as [kPfLo][arows][K/32] e8m0;
  // the row of sorted position p is rowmap ? rowmap[p] / rowdiv : p
  const uint16_t* ahi;
  const uint8_t* aq;
  const uint8_t* as;
  int64_t arows;
  const int32_t* rowmap;
  int rowdiv;
  // plan
  const int32_t* blk;  // [3][cap]
  int cap;
  const int32_t* nblk;
  const int32_t* order;  // sorted position -> slot
  // gate epilogue (N = 2m): hidden terms hhi [n][m] fp16, hq [kPfLo][n][m] fp8, hs [kPfLo][n][m/32]
  const uint16_t* out_gate;
  const uint16_t* out_up;
  const uint16_t* in_down;
  int m;
  uint16_t* hhi;
  uint8_t* hq;
  uint8_t* hs;
  int64_t nslots;
  // down epilogue: values [slots][N] bf16
  const uint16_t* out_down;
  uint16_t* values;
};

// Staging of one 128-wide k step of the item's activations: per row [256 B hi][128 B lo1][128 B lo2]
// at stride kPfRowBytes, and the row's 4 scales of each remainder term.
template <int MT>
struct PfStage {
  static constexpr int kBytes = MT * 16 * kPfRowBytes;
  static constexpr int kScaleBytes = MT * 16 * 4 * kPfLo;
};

// A k step's activation chunks in flight in registers: thread t holds chunks t + kPfThreads i
// (16 B each; MT * 16 rows x 32 chunks = MT chunks per thread) and at most one scale dword.
template <int MT>
struct PfFetch {
  i32x4 v[MT];
  uint32_t sc;
};
// Where a thread's chunks come from: chunk i is row r = t / 32 + 16 i of the item (t = thread) and
// chunk t % 32 of the row (0-15: hi, 16-23: lo1, 24-31: lo2); the addresses are fixed per item up
// to the k step offset, so they are formed once per item.
template <int MT>
struct PfSrc {
  const uint8_t* p[MT];  // chunk i at k step 0
  const uint8_t* sp;     // the thread's scale dword at k step 0
  int step;              // bytes per k step of the thread's chunks: 256 (hi) or 128 (lo)
};
template <int MT>
__device__ __forceinline__ void item_src(const PfGemm& a, const int64_t* rowidx, PfSrc<MT>& s) {
  constexpr int kPer = 16 + 8 * kPfLo;
  static_assert(MT * 16 * kPer == MT * kPfThreads, "one chunk per thread and M-tile");
  const int ch = (int)threadIdx.x % kPer;
  s.step = ch < 16 ? 256 : 128;
#pragma unroll
  for (int i = 0; i < MT; i++) {
    const int r = (int)threadIdx.x / kPer + i * (kPfThreads / kPer);
    if (ch < 16) {
      s.p[i] = reinterpret_cast<const uint8_t*>(a.ahi + rowidx[r] * a.K) + ch * 16;
    } else {
      const int t = (ch - 16) / 8, cc = (ch - 16) % 8;
      s.p[i] = a.aq + (t * a.arows + rowidx[r]) * a.K + cc * 16;
    }
  }
  const int c = min((int)threadIdx.x, MT * 16 * kPfLo - 1);
  const int r = c / kPfLo, t = c % kPfLo;
  s.sp = a.as + (t * a.arows + rowidx[r]) * (a.K / 32);
}
template <int MT>
__device__ __forceinline__ void fetch_k(const PfSrc<MT>& s, int ks, PfFetch<MT>& f) {
  const int off = ks * s.step;
#pragma unroll
  for (int i = 0; i < MT; i++) f.v[i] = *reinterpret_cast<const i32x4*>(s.p[i] + off);
  f.sc = *reinterpret_cast<const uint32_t*>(s.sp + ks * 4);
}
template <int MT>
__device__ __forceinline__ void put_k(const PfFetch<MT>& f, uint8_t* buf, uint8_t* sbuf) {
  constexpr int kPer = 16 + 8 * kPfLo;
#pragma unroll
  for (int i = 0; i < MT; i++) {
    const int c = threadIdx.x + i * kPfThreads;
    *reinterpret_cast<i32x4*>(buf + (c / kPer) * kPfRowBytes + (c % kPer) * 16) = f.v[i];
  }
  if ((int)threadIdx.x < MT * 16 * kPfLo) *reinterpret_cast<uint32_t*>(sbuf + threadIdx.x * 4) = f.sc;
}

// The item's rows: sorted positions [first, first + len), clamped into the item for the padding
// rows of the last M-tile (their results are discarded).
template <int MT>
__device__ __forceinline__ void item_rows(const PfGemm& a, int first, int len, int64_t* rowidx) {
  for (int r = threadIdx.x; r < MT * 16; r += kPfThreads) {
    const int p = first + min(r, len - 1);
    rowidx[r] = a.rowmap ? (int64_t)(a.rowmap[p] / a.rowdiv) : (int64_t)p;
  }
}

// One k step of the MFMAs: activations from the staged buffer, weights from (bw, bs).
template <int MT, int NT>
__device__ __forceinline__ void gemm_step(const uint8_t* ab, const uint8_t* sb, const i32x4 (&bw)[NT],
                                          const uint32_t (&bs)[NT], f32x4 (&acc)[MT][NT]) {
  const int lane = lane_id(), nn = lane & 15, g = lane >> 4;
  float wsc[NT];
#pragma unroll
  for (int j = 0; j < NT; j++) wsc[j] = __builtin_amdgcn_ldexpf(1.0f, (int)bs[j] - 127);
  // hi: 4 fp16 MFMAs per M-tile; the q-th reads k = 32 g + 8 q + i, i.e. the 8 codes of word q,
  // widened to fp16 with their block scale just before use
#pragma unroll
  for (int q = 0; q < 4; q++) {
    f16x8 bh[NT];
#pragma unroll
    for (int j = 0; j < NT; j++) {
      const uint32_t word = (uint32_t)bw[j][q];
      bh[j] = pack_f16x8(__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(word, wsc[j], 0),
                         __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(word, wsc[j], 1),
                         __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(word, wsc[j], 2),
                         __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(word, wsc[j], 3));
    }
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
      const f16x8 ah =
          *reinterpret_cast<const f16x8*>(ab + (mt * 16 + nn) * kPfRowBytes + (32 * g + 8 * q) * 2);
#pragma unroll
      for (int j = 0; j < NT; j++) acc[mt][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bh[j], acc[mt][j], 0, 0, 0);
    }
  }
#pragma unroll
  for (int mt = 0; mt < MT; mt++) {
    const uint8_t* rp = ab + (mt * 16 + nn) * kPfRowBytes;
    // remainder terms: one scaled MX MFMA each on the resident codes
#pragma unroll
    for (int t = 0; t < kPfLo; t++) {
      const i32x4 l0 = *reinterpret_cast<const i32x4*>(rp + 256 + 128 * t + 16 * g);
      const i32x4 l1 = *reinterpret_cast<const i32x4*>(rp + 256 + 128 * t + 64 + 16 * g);
      const i32x8 al = {l0.x, l0.y, l0.z, l0.w, l1.x, l1.y, l1.z, l1.w};
      const int asc = sb[((mt * 16 + nn) * kPfLo + t) * 4 + g];
#pragma unroll
      for (int j = 0; j < NT; j++) {
        const i32x8 bv = {bw[j].x, bw[j].y, bw[j].z, bw[j].w, 0, 0, 0, 0};
        acc[mt][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(al, bv, acc[mt][j], 0, 4, 0, asc, 0,
                                                                      (int)bs[j]);
      }
    }
  }
}

// One wave's NT column tiles (cols[j] .. +16) over all K for the item's MT M-tiles.  The weights
// and the activations are loaded D k steps ahead into rings of D register sets (set s % D holds
// step s); a step's activations go to LDS (double buffered) in the step before their use, after
// that step's MFMAs (D even).  The tiles' block scales for all k steps (16 rows x K/32 bytes per
// tile, one contiguous span in memory) are copied once per item into the wave's LDS region `wsl`
// with 16 B loads: a byte load per lane and k step from HBM costs about as much as the weights.
template <int MT, int NT, int MTMAX, int D>
__device__ __forceinline__ void gemm_item(const PfGemm& a, int e, const int (&cols)[NT], const int64_t* rowidx,
                                          uint8_t* abuf, uint8_t* sbuf, uint8_t* wsl, f32x4 (&acc)[MT][NT]) {
  static_assert(D % 2 == 0, "the LDS stage alternates with the step parity");
  const int lane = lane_id(), nn = lane & 15, g = lane >> 4;
  const int ksteps = a.K / 128, last = ksteps - 1;
#pragma unroll
  for (int mt = 0; mt < MT; mt++)
#pragma unroll
    for (int j = 0; j < NT; j++) acc[mt][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  const int sb = a.K / 32;  // scale bytes per weight row
#pragma unroll
  for (int j = 0; j < NT; j++) {
    const uint8_t* src = a.wscales + ((int64_t)e * a.N + cols[j]) * sb;
    uint8_t* dst = wsl + j * 16 * sb;
    for (int c = lane; c < sb; c += 64)  // 16 sb bytes = sb chunks of 16 B
      *reinterpret_cast<i32x4*>(dst + 16 * c) = *reinterpret_cast<const i32x4*>(src + 16 * c);
  }
  const uint8_t* wrow[NT];
  const uint8_t* srow[NT];
#pragma unroll
  for (int j = 0; j < NT; j++) {
    wrow[j] = a.codes + ((int64_t)e * a.N + cols[j] + nn) * (a.K / 2) + g * 16;
    srow[j] = wsl + (j * 16 + nn) * sb + g;
  }
  constexpr int kStage = PfStage<MTMAX>::kBytes, kSStage = PfStage<MTMAX>::kScaleBytes;
  auto load_w = [&](i32x4 (&bw)[NT], uint32_t (&bs)[NT], int ks) {
#pragma unroll
    for (int j = 0; j < NT; j++) {
      bw[j] = *reinterpret_cast<const i32x4*>(wrow[j] + ks * 64);
      bs[j] = srow[j][ks * 4];  // LDS; written above by this wave
    }
  };
  PfSrc<MT> src;
  item_src<MT>(a, rowidx, src);
  PfFetch<MT> f[D];
  i32x4 bw[D][NT];
  uint32_t bs[D][NT];
  fetch_k<MT>(src, 0, f[0]);
  put_k<MT>(f[0], abuf, sbuf);
#pragma unroll
  for (int d = 0; d < D; d++) load_w(bw[d], bs[d], min(d, last));
#pragma unroll
  for (int d = 1; d <= D; d++) fetch_k<MT>(src, min(d, last), f[d % D]);
  __syncthreads();
  for (int ks = 0; ks < ksteps; ks += D) {
#pragma unroll
    for (int u = 0; u < D; u++) {
      const int t = ks + u;  // block-uniform
      if (t < ksteps) {
        gemm_step<MT, NT>(abuf + (u & 1) * kStage, sbuf + (u & 1) * kSStage, bw[u], bs[u], acc);
        load_w(bw[u], bs[u], min(t + D, last));
        if (t + 1 < ksteps) put_k<MT>(f[(u + 1) % D], abuf + ((u + 1) & 1) * kStage, sbuf + ((u + 1) & 1) * kSStage);
        fetch_k<MT>(src, min(t + 1 + D, last), f[(u + 1) % D]);
        __syncthreads();
      }
    }
  }
}

// ---------------------------------------------------------------- gate/up GEMM + gate finish
// Item = (plan block b, intermediate blocks c NB .. c NB + NB - 1 of 128): for each block cb the
// gate columns [128 cb, +128) and the up columns [m + 128 cb, +128); wave w owns gate and up tile
// 16w of each block (tiles 2 bb, 2 bb + 1).  More blocks per item share each staged activation step
// among more weights.
template <int MT, int MTMAX, int NB>
__device__ __forceinline__ void gateup_item(const PfGemm& a, int e, int first, int len, int c, uint8_t* abuf, uint8_t* sbuf,
                                            uint8_t* wsl, int64_t* rowidx, float* ex) {
  const int w = wave_id_uniform(), lane = lane_id(), nn = lane & 15, g = lane >> 4;
  item_rows<MT>(a, first, len, rowidx);
  __syncthreads();
  int cols[2 * NB];
#pragma unroll
  for (int bb = 0; bb < NB; bb++) {
    cols[2 * bb] = 128 * (c * NB + bb) + 16 * w;
    cols[2 * bb + 1] = a.m + 128 * (c * NB + bb) + 16 * w;
  }
  f32x4 acc[MT][2 * NB];
  gemm_item<MT, 2 * NB, MTMAX, 2>(a, e, cols, rowidx, abuf, sbuf, wsl, acc);
  // epilogue per block and M-tile: gate/up tiles -> LDS [16][2][128] -> per row: H128, scale,
  // SwiGLU, in_down, H128
#pragma unroll
  for (int bb = 0; bb < NB; bb++) {
    const int cb = c * NB + bb;
    const int64_t si = (int64_t)e * a.m + 128 * cb + 2 * lane;
    const float og0 = f16_to_f32(a.out_gate[si]), og1 = f16_to_f32(a.out_gate[si + 1]);
    const float ou0 = f16_to_f32(a.out_up[si]), ou1 = f16_to_f32(a.out_up[si + 1]);
    const float id0 = f16_to_f32(a.in_down[si]), id1 = f16_to_f32(a.in_down[si + 1]);
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int r = 4 * g + i;
        ex[(r * 2 + 0) * 128 + 16 * w + nn] = acc[mt][2 * bb][i];
        ex[(r * 2 + 1) * 128 + 16 * w + nn] = acc[mt][2 * bb + 1][i];
      }
      __syncthreads();
#pragma unroll
      for (int rr = 0; rr < 2; rr++) {
        const int r = 2 * w + rr;  // 8 waves x 2 rows
        const int pr = mt * 16 + r;
        if (pr < len) {
          float g0 = ex[(r * 2) * 128 + 2 * lane], g1 = ex[(r * 2) * 128 + 2 * lane + 1];
          float u0 = ex[(r * 2 + 1) * 128 + 2 * lane], u1 = ex[(r * 2 + 1) * 128 + 2 * lane + 1];
          hadamard128_wave(g0, g1);
          hadamard128_wave(u0, u1);
          float h0 = swiglu_bf16(g0 * og0, u0 * ou0) * id0;
          float h1 = swiglu_bf16(g1 * og1, u1 * ou1) * id1;
          hadamard128_wave(h0, h1);
          uint32_t lo[kPfLo], sc[kPfLo];
          const uint32_t hi = hi_lo_terms(h0, h1, lo, sc);
          const int64_t p = first + pr;
          *reinterpret_cast<uint32_t*>(a.hhi + p * a.m + 128 * cb + 2 * lane) = hi;
#pragma unroll
          for (int t = 0; t < kPfLo; t++) {
            *reinterpret_cast<uint16_t*>(a.hq + (t * a.nslots + p) * a.m + 128 * cb + 2 * lane) = (uint16_t)lo[t];
            if (nn == 0) a.hs[(t * a.nslots + p) * (a.m / 32) + 4 * cb + g] = (uint8_t)sc[t];
          }
        }
      }
      __syncthreads();
    }
  }
}

// ---------------------------------------------------------------- down GEMM + value finish
// Item = (plan block b, output blocks ob NB .. ob NB + NB - 1 of 128); wave w owns tile 16w of each.
template <int MT, int MTMAX, int NB>
__device__ __forceinline__ void down_item(const PfGemm& a, int e, int first, int len, int ob, uint8_t* abuf, uint8_t* sbuf,
                                          uint8_t* wsl, int64_t* rowidx, float* ex) {
  const int w = wave_id_uniform(), lane = lane_id(), nn = lane & 15, g = lane >> 4;
  item_rows<MT>(a, first, len, rowidx);
  __syncthreads();
  int cols[NB];
#pragma unroll
  for (int bb = 0; bb < NB; bb++) cols[bb] = 128 * (ob * NB + bb) + 16 * w;
  f32x4 acc[MT][NB];
  gemm_item<MT, NB, MTMAX, 2>(a, e, cols, rowidx, abuf, sbuf, wsl, acc);
#pragma unroll
  for (int bb = 0; bb < NB; bb++) {
    const int cb = ob * NB + bb;
    const int64_t si = (int64_t)e * a.N + 128 * cb + 2 * lane;
    const float od0 = f16_to_f32(a.out_down[si]), od1 = f16_to_f32(a.out_down[si + 1]);
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
#pragma unroll
      for (int i = 0; i < 4; i++) ex[(4 * g + i) * 128 + 16 * w + nn] = acc[mt][bb][i];
      __syncthreads();
#pragma unroll
      for (int rr = 0; rr < 2; rr++) {
        const int r = 2 * w + rr;
        const int pr = mt * 16 + r;
        if (pr < len) {
          float v0 = ex[r * 128 + 2 * lane], v1 = ex[r * 128 + 2 * lane + 1];
          hadamard128_wave(v0, v1);
          const int slot = a.order[first + pr];
          const uint32_t pk = (uint32_t)f32_to_bf16(v0 * od0) | ((uint32_t)f32_to_bf16(v1 * od1) << 16);
          *reinterpret_cast<uint32_t*>(a.values + (int64_t)slot * a.N + 128 * cb + 2 * lane) = pk;
        }
      }
      __syncthreads();
    }
  }
}

// Grid: (plan blocks) x (output blocks per item).  Items of MTMIN..MTMAX M-tiles only (the others
// exit at once).  Dynamic LDS: double-buffered activation stage, its scale stage and the row map
// (the epilogue exchange reuses the stage), then per wave its tiles' weight scales.
template <int MTMIN, int MTMAX>
constexpr size_t pf_lds_bytes() {
  return 2 * PfStage<MTMAX>::kBytes + 2 * PfStage<MTMAX>::kScaleBytes + MTMAX * 16 * sizeof(int64_t);
}
// per wave: NT tiles x 16 rows x K/32 scale bytes
inline size_t pf_wscale_lds_bytes(int nt, int K) { return (size_t)kPfWaves * nt * 16 * (K / 32); }
// 128-column output blocks per item: two for the small items (activations re-staged half as often
// per weight byte), one for the large ones (register budget)
__host__ __device__ constexpr int pf_blocks_per_item(int mtmax) { return mtmax <= 2 ? 2 : 1; }
// LDS of the small and large GEMM kernels (GATE: gate/up, K = hidden; else down, K = intermediate)
inline size_t pf_small_lds(bool gate, int K) {
  return pf_lds_bytes<1, 2>() + pf_wscale_lds_bytes((gate ? 2 : 1) * pf_blocks_per_item(2), K);
}
inline size_t pf_large_lds(bool gate, int K) {
  return pf_lds_bytes<3, 4>() + pf_wscale_lds_bytes((gate ? 2 : 1) * pf_blocks_per_item(4), K);
}

template <bool GATE, int MTMIN, int MTMAX>
__device__ __forceinline__ void pf_gemm_body(const PfGemm& a, int bid) {
  extern __shared__ __attribute__((aligned(16))) uint8_t pf_lds[];
  uint8_t* abuf = pf_lds;
  uint8_t* sbuf = abuf + 2 * PfStage<MTMAX>::kBytes;
  int64_t* rowidx = reinterpret_cast<int64_t*>(sbuf + 2 * PfStage<MTMAX>::kScaleBytes);
  static_assert(2 * PfStage<1>::kBytes >= 16 * 2 * 128 * 4, "the epilogue exchange must fit in the stage");
  float* ex = reinterpret_cast<float*>(abuf);
  constexpr int kNB = pf_blocks_per_item(MTMAX), kNT = GATE ? 2 * kNB : kNB;
  uint8_t* wsl = pf_lds + pf_lds_bytes<MTMIN, MTMAX>() + wave_id_uniform() * kNT * 16 * (a.K / 32);
  const int outblocks = (GATE ? a.m : a.N) / (128 * kNB);
  // Workgroups are dealt to the 8 XCDs in turn.  Small items: the outblocks items of one plan block
  // go to one XCD, so its activation rows are read into one L2 (workgroup i -> plan block
  // 8 (i / 8 outblocks) + i % 8, output block (i % 8 outblocks) / 8).  Large items (the blocks of
  // the popular experts): consecutive plan blocks of an output block share an XCD and its weights.
  int b, ob;
  if (MTMAX <= 2) {
    const int grp = bid / (8 * outblocks), r = bid % (8 * outblocks);
    b = 8 * grp + r % 8;
    ob = r / 8;
  } else {
    b = bid / outblocks;
    ob = bid % outblocks;
  }
  if (b >= *a.nblk) return;
  const int e = a.blk[b], first = a.blk[a.cap + b], len = a.blk[2 * a.cap + b];
  const int mt = (len + 15) / 16;
  if (mt < MTMIN || mt > MTMAX) return;
#define PF_CASE(M)                                                                          \
  case M:                                                                                   \
    if (M >= MTMIN && M <= MTMAX) {                                                         \
      if (GATE)                                                                             \
        gateup_item<(M <= MTMAX ? M : 1), MTMAX, kNB>(a, e, first, len, ob, abuf, sbuf, wsl, rowidx, ex); \
      else                                                                                  \
        down_item<(M <= MTMAX ? M : 1), MTMAX, kNB>(a, e, first, len, ob, abuf, sbuf, wsl, rowidx, ex);     \
    }                                                                                       \
    break;
  switch (mt) {
    PF_CASE(1)
    PF_CASE(2)
    PF_CASE(3)
    PF_CASE(4)
    default: break;
  }
#undef PF_CASE
}

template <bool GATE, int MTMIN, int MTMAX>
__global__ __launch_bounds__(kPfThreads) void pf_gemm_kernel(PfGemm a) {
  pf_gemm_body<GATE, MTMIN, MTMAX>(a, (int)blockIdx.x);
}

// The down GEMM's small items (K = intermediate: 48 KB of LDS per block) held within 128 VGPRs so
// that two blocks share a CU.
__global__ __launch_bounds__(kPfThreads) __attribute__((amdgpu_waves_per_eu(4))) void pf_gemm_down_small_kernel(PfGemm a) {
  pf_gemm_body<false, 1, 2>(a, (int)blockIdx.x);
}

// Both item classes in one launch: the large items' workgroups first (`nlarge` of them, a multiple
// of 8 so that the small items keep their XCD mapping), so that the few long items of the popular
// experts start at once and the many small ones fill the machine around them, instead of running
// in a launch of their own after the small ones with most compute units idle.
template <bool GATE>
__global__ __launch_bounds__(kPfThreads) void pf_gemm_merged_kernel(PfGemm a, int nlarge) {
  if ((int)blockIdx.x < nlarge)
    pf_gemm_body<GATE, 3, 4>(a, (int)blockIdx.x);
  else
    pf_gemm_body<GATE, 1, 2>(a, (int)blockIdx.x - nlarge);
}

template <bool GATE>
int launch_pf_gemm(const PfGemm& a, hipStream_t s) {
  const int n128 = (GATE ? a.m : a.N) / 128;  // 128-column output blocks
  // whole groups of 8 plan blocks (b < *nblk <= cap is checked in the kernel)
  const unsigned groups = (unsigned)((a.cap + 7) / 8 * 8);
  const size_t small_lds = pf_small_lds(GATE, a.K), large_lds = pf_large_lds(GATE, a.K);
  if (small_lds > kPfMaxLds || large_lds > kPfMaxLds)
    return fail(MOE_EINVAL, "prefill GEMM needs %zu / %zu B of LDS (K = %d)", small_lds, large_lds, a.K);
  // dynamic LDS beyond 64 KB must be allowed explicitly (idempotent; cheap)
  MOE_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&pf_gemm_kernel<GATE, 1, 2>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)small_lds));
  MOE_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&pf_gemm_kernel<GATE, 3, 4>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)large_lds));
  const unsigned nsmall = groups * (n128 / pf_blocks_per_item(2)), nlarge = groups * (n128 / pf_blocks_per_item(4));
  if (GATE ? MOE_PF_MERGE_GATE : MOE_PF_MERGE_DOWN) {
    const size_t lds = small_lds > large_lds ? small_lds : large_lds;
    MOE_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&pf_gemm_merged_kernel<GATE>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    hipLaunchKernelGGL((pf_gemm_merged_kernel<GATE>), dim3(nlarge + nsmall), dim3(kPfThreads), lds, s, a, (int)nlarge);
    MOE_HIP(hipGetLastError());
    return MOE_OK;
  }
  if (!GATE && MOE_PF_DOWN_TWO) {
    MOE_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&pf_gemm_down_small_kernel),
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)small_lds));
    hipLaunchKernelGGL(pf_gemm_down_small_kernel, dim3(nsmall), dim3(kPfThreads), small_lds, s, a);
  } else {
    hipLaunchKernelGGL((pf_gemm_kernel<GATE, 1, 2>), dim3(nsmall), dim3(kPfThreads), small_lds, s, a);
  }
  MOE_HIP(hipGetLastError());
  hipLaunchKernelGGL((pf_gemm_kernel<GATE, 3, 4>), dim3(nlarge), dim3(kPfThreads), large_lds, s, a);
  MOE_HIP(hipGetLastError());
  return MOE_OK;
}

// ---------------------------------------------------------------- combine
// out[t] = T(T(sum_{i<8} value[9t+i] * score[t,i]) + value[9t+8]) + residual[t], the routed sum
// in the reference's order (value_0*s_0, then each next product added to the running sum).
// One block of 256 threads per row, 8 columns per thread per pass.
__global__ __launch_bounds__(256) void pf_combine_kernel(const uint16_t* __restrict__ values,
                                                         const float* __restrict__ scores,
                                                         const uint16_t* __restrict__ residual, int h,
                                                         uint16_t* __restrict__ out) {
  const int64_t r = blockIdx.x;
  float sc[8];
#pragma unroll
  for (int j = 0; j < 8; j++) sc[j] = scores[r * 8 + j];
  for (int c = threadIdx.x * 8; c < h; c += 256 * 8) {
    u32x4 y[9];
#pragma unroll
    for (int j = 0; j < 9; j++) y[j] = *reinterpret_cast<const u32x4*>(values + (r * 9 + j) * h + c);
    const u32x4 rv = *reinterpret_cast<const u32x4*>(residual + r * h + c);
    u32x4 o;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      float res2[2];
#pragma unroll
      for (int hh = 0; hh < 2; hh++) {
        auto val = [&](int j) { return bf16_to_f32((uint16_t)(hh ? (y[j][q] >> 16) : (y[j][q] & 0xFFFFu))); };
        float tot = val(0) * sc[0] + 0.0f;
#pragma unroll
        for (int j = 1; j < 8; j++) tot = (val(j) * sc[j] + 0.0f) + tot;
        const float comb = round_bf16(round_bf16(tot) + val(8));
        const float resv = bf16_to_f32((uint16_t)(hh ? (rv[q] >> 16) : (rv[q] & 0xFFFFu)));
        res2[hh] = resv + comb;
      }
      o[q] = (uint32_t)f32_to_bf16(res2[0]) | ((uint32_t)f32_to_bf16(res2[1]) << 16);
    }
    *reinterpret_cast<u32x4*>(out + r * h + c) = o;
  }
}

// ---------------------------------------------------------------- workspace
struct PfWorkspace {
  float* logits;      // [rows][256]
  uint32_t* ids;      // [rows][9]
  float* scores;      // [rows][8]
  int32_t* order;     // [n]
  int32_t* counts;    // [E]
  int32_t* starts;    // [E]
  int32_t* blk;       // [3][cap]
  int32_t* nblk;
  uint16_t* xhi;      // [rows][h] fp16
  uint8_t* xq;        // [kPfLo][rows][h] fp8 remainder terms
  uint8_t* xs;        // [kPfLo][rows][h/32]
  uint16_t* hhi;      // [n][m] fp16
  uint8_t* hq;        // [kPfLo][n][m] fp8 remainder terms
  uint8_t* hs;        // [kPfLo][n][m/32]
  uint16_t* values;   // [n][h]
  int cap;
  size_t bytes;
};

int pf_cap(int64_t n, int64_t experts) { return (int)(n / kPfItemRows + experts + 1); }

// n = rows * slots expert slots
PfWorkspace pf_carve(void* base, int rows, int slots, int h, int m, int64_t experts) {
  PfWorkspace w{};
  const int64_t n = (int64_t)rows * slots;
  w.cap = pf_cap(n, experts);
  size_t off = 0;
  char* p = static_cast<char*>(base);
  auto take = [&](size_t bytes) { char* r = p ? p + off : nullptr; off += (bytes + 255) & ~(size_t)255; return r; };
  w.logits = reinterpret_cast<float*>(take((size_t)rows * 256 * 4));
  w.ids = reinterpret_cast<uint32_t*>(take((size_t)n * 4));
  w.scores = reinterpret_cast<float*>(take((size_t)rows * 8 * 4));
  w.order = reinterpret_cast<int32_t*>(take((size_t)n * 4));
  w.counts = reinterpret_cast<int32_t*>(take((size_t)experts * 4));
  w.starts = reinterpret_cast<int32_t*>(take((size_t)experts * 4));
  w.blk = reinterpret_cast<int32_t*>(take((size_t)3 * w.cap * 4));
  w.nblk = reinterpret_cast<int32_t*>(take(4));
  w.xhi = reinterpret_cast<uint16_t*>(take((size_t)rows * h * 2));
  w.xq = reinterpret_cast<uint8_t*>(take((size_t)kPfLo * rows * h));
  w.xs = reinterpret_cast<uint8_t*>(take((size_t)kPfLo * rows * (h / 32)));
  w.hhi = reinterpret_cast<uint16_t*>(take((size_t)n * m * 2));
  w.hq = reinterpret_cast<uint8_t*>(take((size_t)kPfLo * n * m));
  w.hs = reinterpret_cast<uint8_t*>(take((size_t)kPfLo * n * (m / 32)));
  w.values = reinterpret_cast<uint16_t*>(take((size_t)n * h * 2));
  w.bytes = off;
  return w;
}

int launch_segment_table(const uint32_t* ids, int n, int experts, int block_rows, int32_t* order, int32_t* counts,
                         int32_t* starts, int32_t* blk, int cap, int32_t* nblk, hipStream_t s, int clamp) {
  hipLaunchKernelGGL(segment_table_kernel, dim3(1), dim3(1024), 0, s, ids, n, experts, block_rows, order, counts,
                     starts, blk, cap, nblk, clamp);
  MOE_HIP(hipGetLastError());
  return MOE_OK;
}

}  // namespace

// The segment table of the grouped MLP / linear entries: ids outside [0, experts) are clamped.
int segment_table_clamped(const uint32_t* ids, int n, int experts, int block_rows, int32_t* order, int32_t* counts,
                          int32_t* starts, int32_t* table, int capacity, int32_t* num_blocks, hipStream_t s) {
  return launch_segment_table(ids, n, experts, block_rows, order, counts, starts, table, capacity, num_blocks, s, 1);
}
}  // namespace moe

using namespace moe;

extern "C" {

int moe_combine_values(const uint16_t* values, const float* scores, const uint16_t* residual, int rows, int hidden,
                       uint16_t* out, moe_stream_t stream) {
  MOE_ARG(values && scores && residual && out, "null pointer argument");
  MOE_ARG(rows >= 1, "rows must be positive (got %d)", rows);
  MOE_ARG(hidden > 0 && hidden % 8 == 0, "hidden must be a positive multiple of 8 (got %d)", hidden);
  MOE_ARG((((uintptr_t)values | (uintptr_t)residual | (uintptr_t)out) & 15) == 0,
          "values, residual and out must be 16-byte aligned");
  int rc = ensure_device_ready();
  if (rc) return rc;
  hipLaunchKernelGGL(pf_combine_kernel, dim3(rows), dim3(256), 0, (hipStream_t)stream, values, scores, residual,
                     hidden, out);
  MOE_HIP(hipGetLastError());
  return MOE_OK;
}

int moe_segment_table(const uint32_t* ids, int n, int experts, int block_rows, int32_t* order, int32_t* counts,
                      int32_t* starts, int32_t* table, int capacity, int32_t* num_blocks, moe_stream_t stream) {
  MOE_ARG((ids && order) || n == 0, "null ids/order with n > 0");
  MOE_ARG(counts && starts && table && num_blocks, "null pointer argument");
  MOE_ARG(n >= 0, "n must be non-negative");
  MOE_ARG(experts >= 1 && experts <= kPfMaxExperts, "experts must be in 1..%d", kPfMaxExperts);
  MOE_ARG(block_rows >= 1, "block_rows must be positive");
  MOE_ARG(capacity >= (int64_t)n / block_rows + experts,
          "table capacity must be at least n / block_rows + experts (%lld)", (long long)n / block_rows + experts);
  int rc = ensure_device_ready();
  if (rc) return rc;
  return launch_segment_table(ids, n, experts, block_rows, order, counts, starts, table, capacity, num_blocks,
                              (hipStream_t)stream, 0);
}

size_t moe_mxfp4_prefill_workspace_bytes(int rows, int hidden, int intermediate, int64_t experts) {
  if (rows <= 0 || hidden <= 0 || intermediate <= 0 || experts <= 0) return 0;
  return pf_carve(nullptr, rows, kSlots, hidden, intermediate, experts).bytes;
}

size_t moe_mxfp4_grouped_mlp_workspace_bytes(int rows, int slots, int hidden, int intermediate, int64_t experts) {
  if (rows <= 0 || slots <= 0 || hidden <= 0 || intermediate <= 0 || experts <= 0) return 0;
  return pf_carve(nullptr, rows, slots, hidden, intermediate, experts).bytes;
}

}  // extern "C"

namespace moe {
namespace {

// Argument checks shared by the grouped MXFP4 entry points (all before any launch).
int mx_grouped_check(const uint16_t* x, const uint8_t* gate_up_codes, const uint8_t* gate_up_scales,
                     const uint8_t* down_codes, const uint8_t* down_scales, int64_t experts, const uint16_t* unit,
                     const uint16_t* out_gate, const uint16_t* out_up, const uint16_t* in_down,
                     const uint16_t* out_down, int rows, int slots, int hidden, int intermediate, const void* workspace,
                     size_t workspace_bytes, PfWorkspace* w) {
  MOE_ARG(x && gate_up_codes && gate_up_scales && down_codes && down_scales && unit && out_gate && out_up &&
              in_down && out_down,
          "null pointer argument");
  MOE_ARG(rows >= 1 && slots >= 1, "rows and slots must be positive (got %d, %d)", rows, slots);
  MOE_ARG(experts >= 1 && experts <= kPfMaxExperts, "experts must be in 1..%d (got %lld)", kPfMaxExperts,
          (long long)experts);
  MOE_ARG(hidden % 1024 == 0 && hidden > 0, "hidden must be a positive multiple of 1024 (got %d)", hidden);
  MOE_ARG(intermediate % 256 == 0 && intermediate > 0, "intermediate must be a positive multiple of 256 (got %d)",
          intermediate);
  MOE_ARG(pf_small_lds(true, hidden) <= kPfMaxLds && pf_large_lds(true, hidden) <= kPfMaxLds &&
              pf_small_lds(false, intermediate) <= kPfMaxLds && pf_large_lds(false, intermediate) <= kPfMaxLds,
          "hidden %d / intermediate %d too large for the prefill GEMM's LDS", hidden, intermediate);
  MOE_ARG(((uintptr_t)gate_up_scales | (uintptr_t)down_scales) % 16 == 0, "weight scale arrays must be 16-byte aligned");
  MOE_ARG(workspace != nullptr, "workspace must not be NULL");
  *w = pf_carve(const_cast<void*>(workspace), rows, slots, hidden, intermediate, experts);
  if (workspace_bytes < w->bytes)
    return fail(MOE_EWORKSPACE, "workspace too small: %zu < %zu bytes", workspace_bytes, w->bytes);
  return ensure_device_ready();
}

// Sorted grouped MXFP4 expert MLP of ids [rows, slots] (a row's slots share x [rows, hidden]):
// segment table, activation terms, gate/up GEMM + gate finish, down GEMM + value finish into
// values [rows * slots, hidden] bf16 (slot order).  An id outside [0, experts) is taken as the nearest
// valid expert, as in the decode entries.
int mx_grouped_body(const uint16_t* x, int rows, int slots, const uint32_t* ids, const uint8_t* gate_up_codes,
                    const uint8_t* gate_up_scales, const uint8_t* down_codes, const uint8_t* down_scales,
                    int64_t experts, const uint16_t* unit, const uint16_t* out_gate, const uint16_t* out_up,
                    const uint16_t* in_down, const uint16_t* out_down, int hidden, int intermediate, uint16_t* values,
                    const PfWorkspace& w, hipStream_t s) {
  const int n = rows * slots;
  int rc = launch_segment_table(ids, n, (int)experts, kPfItemRows, w.order, w.counts, w.starts, w.blk, w.cap, w.nblk,
                                s, 1);
  if (rc) return rc;
  // activation terms
  const int64_t pwaves = (int64_t)rows * (hidden / 128);
  hipLaunchKernelGGL(prep_terms_kernel, dim3((unsigned)((pwaves + 3) / 4)), dim3(256), 0, s, x, unit, rows, hidden,
                     w.xhi, w.xq, w.xs);
  MOE_HIP(hipGetLastError());
  // gate/up GEMM + gate finish -> hidden terms
  PfGemm g{};
  g.codes = gate_up_codes;
  g.wscales = gate_up_scales;
  g.K = hidden;
  g.N = 2 * intermediate;
  g.ahi = w.xhi;
  g.aq = w.xq;
  g.as = w.xs;
  g.arows = rows;
  g.rowmap = w.order;
  g.rowdiv = slots;
  g.blk = w.blk;
  g.cap = w.cap;
  g.nblk = w.nblk;
  g.order = w.order;
  g.out_gate = out_gate;
  g.out_up = out_up;
  g.in_down = in_down;
  g.m = intermediate;
  g.hhi = w.hhi;
  g.hq = w.hq;
  g.hs = w.hs;
  g.nslots = n;
  if ((rc = launch_pf_gemm<true>(g, s))) return rc;
  // down GEMM + value finish -> per-slot values
  PfGemm d{};
  d.codes = down_codes;
  d.wscales = down_scales;
  d.K = intermediate;
  d.N = hidden;
  d.ahi = w.hhi;
  d.aq = w.hq;
  d.as = w.hs;
  d.arows = n;
  d.rowmap = nullptr;
  d.rowdiv = 1;
  d.blk = w.blk;
  d.cap = w.cap;
  d.nblk = w.nblk;
  d.order = w.order;
  d.m = intermediate;
  d.out_down = out_down;
  d.values = values;
  return launch_pf_gemm<false>(d, s);
}

}  // namespace
}  // namespace moe

extern "C" {

int moe_mxfp4_grouped_mlp(const uint16_t* x, const uint32_t* ids, int rows, int slots, const uint8_t* gate_up_codes,
                          const uint8_t* gate_up_scales, const uint8_t* down_codes, const uint8_t* down_scales,
                          int64_t experts, const uint16_t* unit, const uint16_t* out_gate, const uint16_t* out_up,
                          const uint16_t* in_down, const uint16_t* out_down, int hidden, int intermediate,
                          uint16_t* values, void* workspace, size_t workspace_bytes, moe_stream_t stream) {
  MOE_ARG(ids && values, "null pointer argument");
  PfWorkspace w{};
  int rc = mx_grouped_check(x, gate_up_codes, gate_up_scales, down_codes, down_scales, experts, unit, out_gate, out_up,
                            in_down, out_down, rows, slots, hidden, intermediate, workspace, workspace_bytes, &w);
  if (rc) return rc;
  return mx_grouped_body(x, rows, slots, ids, gate_up_codes, gate_up_scales, down_codes, down_scales, experts, unit,
                         out_gate, out_up, in_down, out_down, hidden, intermediate, values, w, (hipStream_t)stream);
}

int moe_mxfp4_prefill(const uint16_t* x, const uint16_t* residual, int rows, const float* router_w,
                      const float* bias, const uint8_t* gate_up_codes, const uint8_t* gate_up_scales,
                      const uint8_t* down_codes, const uint8_t* down_scales, int64_t experts, const uint16_t* unit,
                      const uint16_t* out_gate, const uint16_t* out_up, const uint16_t* in_down,
                      const uint16_t* out_down, int hidden, int intermediate, uint16_t* out, uint32_t* indices,
                      float* scores, void* workspace, size_t workspace_bytes, moe_stream_t stream) {
  MOE_ARG(residual && router_w && bias && out, "null pointer argument");
  MOE_ARG(experts == 257, "the routed block needs 256 routed experts plus the shared expert (got %lld)",
          (long long)experts);
  PfWorkspace w{};
  int rc = mx_grouped_check(x, gate_up_codes, gate_up_scales, down_codes, down_scales, experts, unit, out_gate, out_up,
                            in_down, out_down, rows, kSlots, hidden, intermediate, workspace, workspace_bytes, &w);
  if (rc) return rc;
  hipStream_t s = (hipStream_t)stream;
  uint32_t* ids = indices ? indices : w.ids;
  float* sc = scores ? scores : w.scores;
  // routing: router GEMV, then top-8 + shared slot per row
  if ((rc = moe_router_logits(x, router_w, rows, hidden, 256, w.logits, stream))) return rc;
  if ((rc = moe_route_f32(w.logits, bias, rows, ids, sc, stream))) return rc;
  if ((rc = mx_grouped_body(x, rows, kSlots, ids, gate_up_codes, gate_up_scales, down_codes, down_scales, experts,
                            unit, out_gate, out_up, in_down, out_down, hidden, intermediate, w.values, w, s)))
    return rc;
  hipLaunchKernelGGL(pf_combine_kernel, dim3(rows), dim3(256), 0, s, w.values, sc, residual, hidden, out);
  MOE_HIP(hipGetLastError());
  return MOE_OK;
}

}  // extern "C"
