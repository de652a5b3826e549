// K4 trellis experts over sorted prefill rows on gfx950: grouped GEMMs with the trellis decoded
// next to the fp16 matrix cores, one weight stream per (expert block, column block).
//
// Reference semantics (paths relative to the reference root), exlr8/fast_prefill.py:188-211
// grouped_expert_mlp (values per slot; the caller combines):
//   sorted work order: argsort of the flat ids, per-expert blocks        fast_prefill.py:19-46
//   xh = H128(x * in_scale[e]) for gate and for up                        fast_prefill.py:87-97 (_prep)
//   inner = xh @ decode(packed[e]), fp32 dot                              fast_prefill.py:151-164 (_inner_sorted)
//   h = H128(swiglu_T(H128(g) * out_gate, H128(u) * out_up) * in_down)    fast_prefill.py:203-207 (gate_finish)
//   value = T(H128(h @ decode(down[e])) * out_down)                       fast_prefill.py:118-127 (_finish)
//
// MI355X design:
//   * Activations are split as x = hi + lo * 2^-11 with hi = f16(x) and lo = f16((x - hi) * 2^11)
//     (about 22 bits, the decode GEMV's split); both rows go through v_mfma_f32_16x16x32_f16
//     against the decoded fp16 weights (the codebook values are exact in fp16), so an M-tile of
//     16 A rows carries 8 tokens.  The prep and gate-finish kernels write the A operand directly
//     in the MFMA's k order (a_rh / a_j of the K4 tile rows), 256 B per row and 64-row quad.
//   * A work item is (block of <= 64 sorted rows of one expert, 256 output columns; 128 for the
//     last one when N % 256 == 128).  Each of the
//     8 waves owns one set of 2 tiles (32 columns): per 64-row quad it loads its 16 B piece of the
//     packed tiles, decodes it with the decode GEMV's piece decoder (LDS code table + arithmetic
//     route) and runs 4 MFMAs per M-tile; the quad's A rows of the item are staged in LDS once
//     for the 8 waves.  No split of K: every output is produced by one wave, no atomics.
//   * Items are classed by M-tiles (1, 2, 4, 8) so small experts pay no padded MFMAs; each class
//     is one persistent launch (the code table is loaded into LDS once per block).
//   * K2/K3 tiles (the K3 experts of the multi-token-prediction layer) take the same items and
//     MFMAs; a lane reads the 4-5 words of the circular tile stream that hold its 32 codewords
//     (the generic window of exlr8/metal/trellis.metal:25-40) and looks every codeword up in the
//     LDS table.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "moe_device.h"
#include "moe_host.h"

// arithmetic pairs per even / odd word of the piece decoder (the rest read the code table)
#ifndef MOE_KP_ALU_EVEN
#define MOE_KP_ALU_EVEN 2
#endif
// quads per staging step of the items of up to 16 rows (their two stages of two quads fit the
// launch's stage buffers)
#ifndef MOE_KP_PAIR
#define MOE_KP_PAIR 2
#endif
#ifndef MOE_KP_MERGED
#define MOE_KP_MERGED 1
#endif
#ifndef MOE_KP_ALU_ODD
#define MOE_KP_ALU_ODD 3
#endif

namespace moe {
namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr int kKpRows = 64;        // sorted rows per item
constexpr int kKpWaves = 8;
constexpr int kKpThreads = kKpWaves * 64;
constexpr int kKpRowQuad = 256;    // A bytes per (row, 64-row quad): [rh 2][hl 2][g 4][j 8] fp16
constexpr int kKpCols = 256;       // output columns per item

// A operand element (row p, input k, hl = 0 hi / 1 lo) -> fp16 index in the quad-ordered buffer
__device__ __forceinline__ int64_t kp_a_index(int64_t p, int nq, int k, int hl) {
  const int q = k >> 6, g = (k >> 4) & 3, r = k & 15;
  return ((((p * nq + q) * 2 + a_rh(r)) * 2 + hl) * 4 + g) * 8 + a_j(r);
}

// The pair (k, k + 1), k even, of one row: adjacent in the buffer (same 16-group, same row half,
// positions j and j + 1), so the two hi halves and the two lo halves go out as one 32-bit store each.
__device__ __forceinline__ void kp_store_a2(uint16_t* a, int64_t p, int nq, int k, float x0, float x1) {
  asm volatile("" : "+v"(x0), "+v"(x1));  // x in fp32 before both conversions
  const _Float16 h0 = (_Float16)x0, h1 = (_Float16)x1;
  const _Float16 l0 = (_Float16)((x0 - (float)h0) * 2048.0f), l1 = (_Float16)((x1 - (float)h1) * 2048.0f);
  *reinterpret_cast<uint32_t*>(a + kp_a_index(p, nq, k, 0)) =
      (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
  *reinterpret_cast<uint32_t*>(a + kp_a_index(p, nq, k, 1)) =
      (uint32_t)__builtin_bit_cast(uint16_t, l0) | ((uint32_t)__builtin_bit_cast(uint16_t, l1) << 16);
}

// ---------------------------------------------------------------- prep: xh for gate and up
// One wave per (sorted row p, run of kPrepBlocks 128-blocks, projection of nproj = 1 or 2):
// H128(x_row * in_scale[e]) -> A buffer, x_row = the slot's token row (x_per_slot = 0) or its own
// row.  The run's loads are all issued before the first block is transformed (a wave per block
// left each wave one load round trip with nothing to overlap it).
constexpr int kPrepBlocks = 8;
// 128-blocks per wave of the gate finish and the value finish (loads of the whole run first)
constexpr int kFinGateBlocks = 4, kFinValueBlocks = 8;
// Sorted rows placed by the segment table (ids outside [0, experts) clamped to the nearest expert).
__device__ __forceinline__ int64_t kp_placed(const int32_t* counts, const int32_t* starts, int experts) {
  return (int64_t)starts[experts - 1] + counts[experts - 1];
}
// The expert of a placed slot: its id clamped into [0, experts) exactly as the segment table placed it
// (a slot with an out-of-range id has a position, so its id must never index a side vector raw).
__device__ __forceinline__ int64_t kp_expert(const uint32_t* ids, int slot, int experts) {
  return min(max((int)ids[slot], 0), experts - 1);
}
// waves of the prep launch for n sorted rows
__host__ __device__ __forceinline__ int64_t kp_prep_waves(int64_t n, int K, int nproj) {
  return n * ((K / 128 + kPrepBlocks - 1) / kPrepBlocks) * nproj;
}

__global__ __launch_bounds__(256) void kp_prep_kernel(const uint16_t* __restrict__ x, const uint32_t* __restrict__ ids,
                                                      const int32_t* __restrict__ order, const int32_t* __restrict__ counts,
                                                      const int32_t* __restrict__ starts, int experts, int n, int slots, int K,
                                                      int nproj, int x_per_slot,
                                                      const uint16_t* __restrict__ in_gate,
                                                      const uint16_t* __restrict__ in_up, uint16_t* __restrict__ a_gate,
                                                      uint16_t* __restrict__ a_up) {
  const int64_t wid = (int64_t)blockIdx.x * 4 + wave_id_uniform();
  const int kbs = K / 128, kgs = (kbs + kPrepBlocks - 1) / kPrepBlocks, sh = nproj - 1;
  if (wid >= kp_prep_waves(n, K, nproj)) return;
  const int proj = (int)(wid & sh);
  const int kg = (int)((wid >> sh) % kgs);
  const int64_t p = (wid >> sh) / kgs;
  if (p >= kp_placed(counts, starts, experts)) return;
  const int slot = order[p];
  const int64_t e = kp_expert(ids, slot, experts);
  const int lane = lane_id();
  const int64_t xrow = x_per_slot ? slot : slot / slots;
  const uint16_t* xr = x + xrow * K;
  const uint16_t* sr = (proj ? in_up : in_gate) + e * K;
  uint32_t xv[kPrepBlocks], sv[kPrepBlocks];
#pragma unroll
  for (int i = 0; i < kPrepBlocks; i++) {
    const int k = min(kg * kPrepBlocks + i, kbs - 1) * 128 + 2 * lane;
    xv[i] = *reinterpret_cast<const uint32_t*>(xr + k);
    sv[i] = *reinterpret_cast<const uint32_t*>(sr + k);
  }
  uint16_t* a = proj ? a_up : a_gate;
#pragma unroll
  for (int i = 0; i < kPrepBlocks; i++) {
    const int kb = kg * kPrepBlocks + i;
    if (kb >= kbs) break;
    float v0 = bf16_to_f32((uint16_t)(xv[i] & 0xFFFFu)) * f16_to_f32((uint16_t)(sv[i] & 0xFFFFu));
    float v1 = bf16_to_f32((uint16_t)(xv[i] >> 16)) * f16_to_f32((uint16_t)(sv[i] >> 16));
    hadamard128_wave(v0, v1);
    kp_store_a2(a, p, K / 64, kb * 128 + 2 * lane, v0, v1);
  }
}

// ---------------------------------------------------------------- grouped GEMM
struct KpGemm {
  const uint8_t* codebook;    // device E4M3 code table (64 KB)
  const uint8_t* packed[2];   // per projection: [E] experts of K-bit tiles
  const uint16_t* a[2];       // per projection: A operand [n][K/64][256 B]
  int col_off[2];             // per projection: first column in `inner`
  int nproj, side, K, N;      // input / output features of one projection
  const int32_t* blk;         // plan [3][cap]: expert, first sorted row, length
  int cap;
  const int32_t* nblk;
  const int32_t* ent;         // item entries in launch order: 2 plan block + row half (kp_order_kernel)
  const int32_t* nent;
  int32_t* queue;             // this GEMM's claim counter (zeroed by kp_order_kernel)
  float* inner;               // [n][inner_stride] fp32
  int inner_stride;
  int bits;                   // trellis width K (2, 3 or 4)
};

// K2/K3: the 8 codewords of each of a lane's kernel-order tile lanes L0..L0+3 (L0 = 4 (nn & 7))
// are the 16-bit windows starting at stream bits b0 + j K, j = 0..31, of the circular tile
// stream (codeword i ends at bit (i + 1) K + 256 K, modulo 256 K), b0 = (8 L0 K + K - 16) mod
// 256 K.  The lane loads the words that hold bits b0 .. b0 + 31 K + 15.
template <int KB>
struct KpWords {
  static constexpr int kStream = (31 * KB + 16 + 31) / 32;  // 32-bit words of the lane's window
  uint32_t v[kStream + 1];                                   // from word b0 / 32 on (circular)
};

// The lane's two B fragments per row half rh (h = 0: slots 0-3, h = 1: slots 4-7 of each tile
// lane), in the order the K4 piece decoder gives them; o = b0 % 32.
template <int KB>
__device__ __forceinline__ void kp_generic_frags(const KpWords<KB>& p, int o, const uint8_t* __restrict__ tab,
                                                 f16x8 (&b)[2][2]) {
  constexpr int S = KpWords<KB>::kStream;
  uint32_t u[S];  // the stream from bit b0 on
#pragma unroll
  for (int k = 0; k < S; k++) u[k] = (uint32_t)(((((uint64_t)p.v[k]) << 32 | p.v[k + 1]) << o) >> 32);
  uint32_t q[4][2];  // [tile lane L0 + i][h]: the E4M3 bytes of 4 codewords
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int h = 0; h < 2; h++) {
      uint32_t pk = 0;
#pragma unroll
      for (int t = 0; t < 4; t++) {
        const int pos = (8 * i + 4 * h + t) * KB, wi = pos / 32, off = pos % 32;
        const uint32_t cw = off <= 16 ? (u[wi] >> (16 - off)) & 0xFFFFu
                                      : __builtin_amdgcn_alignbit(u[wi], u[min(wi + 1, S - 1)], 48 - off) & 0xFFFFu;
        pk |= (uint32_t)tab[cw] << (8 * t);
      }
      q[i][h] = pk;
    }
#pragma unroll
  for (int rh = 0; rh < 2; rh++)
#pragma unroll
    for (int h = 0; h < 2; h++)
      b[rh][h] = frag(__builtin_amdgcn_cvt_scalef32_pk_f16_fp8(q[2 * rh][h], 1.0f, false),
                      __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(q[2 * rh][h], 1.0f, true),
                      __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(q[2 * rh + 1][h], 1.0f, false),
                      __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(q[2 * rh + 1][h], 1.0f, true));
}

// One item: rows [first, first + len) of expert e (len <= 8 MT), projection proj, output columns
// [256 cb, +256).  `ab` holds the two A stages (at least MT * 8 * kKpRowQuad bytes each), `tab` the
// code table.  Every wave of the block runs it (it meets at block barriers).
// G quads share a staging step (one block barrier per G quads; a stage then holds G quads).
template <int MT, int KB, int G = 1>
__device__ __forceinline__ void kp_item(const KpGemm& a, const uint8_t* __restrict__ tab, uint8_t* ab0, uint8_t* ab1,
                                        int e, int first, int len, int proj, int cb) {
  static_assert(G == 1 || G == 2, "one or two quads per staging step");
  const int w = wave_id_uniform(), lane = lane_id(), nn = lane & 15, g = lane >> 4;
  const int nq = a.K / 64, it = a.K / 16, obs = a.N / 128;
  const int lane_off = (nn >> 3) * 128 + (nn & 7) * 16;
  const int src_lane = (lane & 7) == 0 ? lane + 7 : lane - 1;
  const int s4 = w & 3;
  // K2/K3: the lane's first window bit b0 within its tile, and the tile words it reads
  constexpr int kNw = 8 * KB;
  const int b0 = (8 * 4 * (nn & 7) * KB + KB - 16 + 256 * KB) % (256 * KB), bo = b0 & 31;
  int gw[KB == 4 ? 1 : KpWords<KB>::kStream + 1];
  if constexpr (KB != 4) {
#pragma unroll
    for (int k = 0; k <= KpWords<KB>::kStream; k++) gw[k] = (b0 / 32 + k) % kNw;
  }
  uint8_t* const abuf[2] = {ab0, ab1};
  // the last item of N % 256 == 128 has one column block: waves 4-7 then only stage A
  const bool active = 2 * cb + (w >> 2) < obs;
  const int ob = min(2 * cb + (w >> 2), obs - 1);
  using Piece = std::conditional_t<KB == 4, u32x4, KpWords<KB>>;
  const uint8_t* wbase = a.packed[proj] + (KB == 4 ? lane_off + 256 * s4 : 32 * KB * (2 * s4 + (nn >> 3)));
  auto piece = [&](int q) -> Piece {
    if constexpr (KB == 4) {
      return *reinterpret_cast<const u32x4*>(wbase + chunk_offset(a.side, e, ob, 4 * q + g, it, obs));
    } else {
      const uint32_t* t =
          reinterpret_cast<const uint32_t*>(wbase + chunk_index(a.side, e, ob, 4 * q + g, it, obs) * (256 * KB));
      Piece r;
#pragma unroll
      for (int k = 0; k <= KpWords<KB>::kStream; k++) r.v[k] = t[gw[k]];
      return r;
    }
  };
  // A staging: chunk c of the quad = row c / 16, 16 B part c % 16 ([rh][hl][g] of the row)
  constexpr int kChunks = MT * 8 * 16, kPer = (kChunks + kKpThreads - 1) / kKpThreads;
  const uint8_t* abase = reinterpret_cast<const uint8_t*>(a.a[proj]);
  auto fetch_a = [&](int q, i32x4 (&f)[kPer]) {
#pragma unroll
    for (int i = 0; i < kPer; i++) {
      const int c = min((int)threadIdx.x + i * kKpThreads, kChunks - 1);
      const int64_t p = first + min(c >> 4, len - 1);
      f[i] = *reinterpret_cast<const i32x4*>(abase + (p * nq + q) * kKpRowQuad + (c & 15) * 16);
    }
  };
  auto put_a = [&](const i32x4 (&f)[kPer], uint8_t* dst) {
#pragma unroll
    for (int i = 0; i < kPer; i++) {
      const int c = (int)threadIdx.x + i * kKpThreads;
      if (c < kChunks) {
        const int row = c >> 4, part = c & 15;  // part = (rh * 2 + hl) * 4 + g
        const int rh = part >> 3, hl = (part >> 2) & 1, gg = part & 3;
        const int m = 2 * (row & 7) + hl;
        *reinterpret_cast<i32x4*>(dst + (((row >> 3) * 2 + rh) * 16 + m) * 64 + gg * 16) = f[i];
      }
    }
  };
  f32x4 acc[MT][2];
#pragma unroll
  for (int mt = 0; mt < MT; mt++) acc[mt][0] = acc[mt][1] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  auto mfmas = [&](const uint8_t* ab, int rh, const f16x8& b0, const f16x8& b1) {
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
      const f16x8 av = *reinterpret_cast<const f16x8*>(ab + ((mt * 2 + rh) * 16 + nn) * 64 + g * 16);
      acc[mt][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, b0, acc[mt][0], 0, 0, 0);
      acc[mt][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, b1, acc[mt][1], 0, 0, 0);
    }
    mfma_acc_guard(acc);
  };
  auto quad = [&](const uint8_t* ab, const Piece& pc) {
    if (!active) return;
    if constexpr (KB == 4) {
      const uint32_t prior = (uint32_t)__shfl((int)pc.w, src_lane, 64);
#pragma unroll
      for (int rh = 0; rh < 2; rh++) {
        f16x2 qv[2][4];
        if (rh == 0)
          decode_pair_words_f16<MOE_KP_ALU_EVEN, MOE_KP_ALU_ODD>(pc.x, pc.y, prior, tab, qv);
        else
          decode_pair_words_f16<MOE_KP_ALU_EVEN, MOE_KP_ALU_ODD>(pc.z, pc.w, pc.y, tab, qv);
        mfmas(ab, rh, frag(qv[0][0], qv[0][1], qv[1][0], qv[1][1]), frag(qv[0][2], qv[0][3], qv[1][2], qv[1][3]));
      }
    } else {
      f16x8 bf[2][2];
      kp_generic_frags<KB>(pc, bo, tab, bf);
      mfmas(ab, 0, bf[0][0], bf[0][1]);
      mfmas(ab, 1, bf[1][0], bf[1][1]);
    }
  };
  i32x4 fa[kPer];
  if constexpr (G == 1) {
    fetch_a(0, fa);
    put_a(fa, abuf[0]);
    Piece pc0 = piece(0), pc1 = piece(min(1, nq - 1));
    fetch_a(min(1, nq - 1), fa);
    __syncthreads();
    for (int q = 0; q < nq; q += 2) {  // nq is even (K % 128 == 0)
      quad(abuf[0], pc0);
      pc0 = piece(min(q + 2, nq - 1));
      put_a(fa, abuf[1]);
      fetch_a(min(q + 2, nq - 1), fa);
      __syncthreads();
      quad(abuf[1], pc1);
      pc1 = piece(min(q + 3, nq - 1));
      if (q + 2 < nq) put_a(fa, abuf[0]);
      fetch_a(min(q + 3, nq - 1), fa);
      __syncthreads();
    }
  } else {
    // stage s holds quads 4i + 2s, 4i + 2s + 1 (QB bytes each); nq is even, so quads come in pairs
    constexpr int QB = MT * 8 * kKpRowQuad;
    i32x4 fb[kPer];
    fetch_a(0, fa);
    fetch_a(min(1, nq - 1), fb);
    put_a(fa, abuf[0]);
    put_a(fb, abuf[0] + QB);
    Piece p0 = piece(0), p1 = piece(min(1, nq - 1)), p2 = piece(min(2, nq - 1)), p3 = piece(min(3, nq - 1));
    fetch_a(min(2, nq - 1), fa);
    fetch_a(min(3, nq - 1), fb);
    __syncthreads();
    for (int q = 0; q < nq; q += 4) {
      quad(abuf[0], p0);
      quad(abuf[0] + QB, p1);
      p0 = piece(min(q + 4, nq - 1));
      p1 = piece(min(q + 5, nq - 1));
      if (q + 2 < nq) {
        put_a(fa, abuf[1]);
        put_a(fb, abuf[1] + QB);
      }
      fetch_a(min(q + 4, nq - 1), fa);
      fetch_a(min(q + 5, nq - 1), fb);
      __syncthreads();
      if (q + 2 < nq) {
        quad(abuf[1], p2);
        quad(abuf[1] + QB, p3);
      }
      p2 = piece(min(q + 6, nq - 1));
      p3 = piece(min(q + 7, nq - 1));
      if (q + 4 < nq) {
        put_a(fa, abuf[0]);
        put_a(fb, abuf[0] + QB);
      }
      fetch_a(min(q + 6, nq - 1), fa);
      fetch_a(min(q + 7, nq - 1), fb);
      __syncthreads();
    }
  }
  // D rows 4g + i of M-tile mt: rows 2t (hi) and 2t+1 (lo) of item row 8 mt + t, t = 2g + i/2
#pragma unroll
  for (int mt = 0; mt < MT; mt++)
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
      for (int tt = 0; tt < 2; tt++) {
        const int row = mt * 8 + 2 * g + tt;
        if (active && row < len) {
          const int col = a.col_off[proj] + ob * 128 + 16 * (2 * s4 + (nn >> 3)) + (nn & 7) + 8 * h;
          a.inner[(int64_t)(first + row) * a.inner_stride + col] =
              fmaf(acc[mt][h][2 * tt + 1], 1.0f / 2048.0f, acc[mt][h][2 * tt]);
        }
      }
}

// MT M-tiles (8 rows each) per item: items of 8 (MT - 1) < len <= 8 MT rows (MT = 1, 2, 4, 8);
// KB = trellis width
template <int MT, int KB>
__global__ __launch_bounds__(kKpThreads) void kp_gemm_kernel(KpGemm a) {
  __shared__ __attribute__((aligned(16))) uint8_t tab[65536];
  __shared__ __attribute__((aligned(16))) uint8_t abuf[2][MT * 8 * kKpRowQuad];
  load_codebook_lds(tab, a.codebook);
  __syncthreads();
  const int ncb = (a.N + kKpCols - 1) / kKpCols;
  const int nblk = *a.nblk;
  const int items = nblk * a.nproj * ncb;
  for (int item = blockIdx.x; item < items; item += gridDim.x) {
    const int cb = item % ncb, proj = (item / ncb) % a.nproj, b = item / (ncb * a.nproj);
    const int len = a.blk[2 * a.cap + b];
    if (len <= (MT / 2) * 8 || len > MT * 8) continue;  // another class
    kp_item<MT, KB>(a, tab, abuf[0], abuf[1], a.blk[b], a.blk[a.cap + b], len, proj, cb);
  }
}

// The GEMMs' item entries, largest first: plan blocks of 17..64 rows as entries of up to 32 rows
// (a block beyond 32 rows as two entries, its row halves: each row's sums are the same whatever
// rows share its tiles), then blocks of 9..16 rows, then of up to 8.  One block of 256 threads
// after the segment table; it also clears the two GEMMs' claim counters.
__global__ __launch_bounds__(256) void kp_order_kernel(const int32_t* __restrict__ blk, int cap,
                                                       const int32_t* __restrict__ nblk, int32_t* __restrict__ ent,
                                                       int32_t* __restrict__ nent, int32_t* __restrict__ queue) {
  __shared__ int32_t cnt[3], pos[3];
  if (threadIdx.x < 3) cnt[threadIdx.x] = pos[threadIdx.x] = 0;
  __syncthreads();
  const int nb = min(*nblk, cap);
  auto cls = [&](int len) { return len > 16 ? 0 : len > 8 ? 1 : 2; };
  for (int b = threadIdx.x; b < nb; b += 256) {
    const int len = blk[2 * cap + b];
    atomicAdd(&cnt[cls(len)], len > 32 ? 2 : 1);
  }
  __syncthreads();
  for (int b = threadIdx.x; b < nb; b += 256) {
    const int len = blk[2 * cap + b], c = cls(len);
    const int base = (c > 0 ? cnt[0] : 0) + (c > 1 ? cnt[1] : 0);
    const int at = base + atomicAdd(&pos[c], len > 32 ? 2 : 1);
    ent[at] = 2 * b;
    if (len > 32) ent[at + 1] = 2 * b + 1;
  }
  if (threadIdx.x == 0) {
    *nent = cnt[0] + cnt[1] + cnt[2];
    queue[0] = 0;
    queue[32] = 0;
  }
}

// Every item class in one persistent launch: the blocks claim items in entry order (largest first)
// from a counter, so blocks that finish the long items go on to the short ones and the launch has
// no class boundaries at which compute units wait for the last long item of a class.
template <int KB>
__global__ __launch_bounds__(kKpThreads) void kp_gemm_merged_kernel(KpGemm a) {
  __shared__ __attribute__((aligned(16))) uint8_t tab[65536];
  __shared__ __attribute__((aligned(16))) uint8_t abuf[2][4 * 8 * kKpRowQuad];
  // K2/K3 pieces hold more words: their registers allow one quad per step within 128 VGPRs
  constexpr int kPair = KB == 4 ? MOE_KP_PAIR : 1;
  load_codebook_lds(tab, a.codebook);
  const int ncb = (a.N + kKpCols - 1) / kKpCols, per = a.nproj * ncb;
  const int total = *a.nent * per;
  // The claimed item is handed to the block through the first word of the A stage, which no item
  // uses between its last barrier and the next item's staging: the block's LDS then stays at
  // 80 KB, so that two blocks fit a CU (a separate shared word would make it one).
  int32_t* claimed = reinterpret_cast<int32_t*>(&abuf[0][0]);
  for (;;) {
    if (threadIdx.x == 0) *claimed = __hip_atomic_fetch_add(a.queue, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    const int v = *claimed;
    __syncthreads();
    if (v >= total) break;
    const int en = a.ent[v / per], r = v % per;
    const int b = en >> 1, half = en & 1;
    const int cb = r % ncb, proj = r / ncb;
    const int len = a.blk[2 * a.cap + b];
    const int first = a.blk[a.cap + b] + 32 * half, n = half ? len - 32 : min(len, 32);
    if (n > 16)
      kp_item<4, KB>(a, tab, abuf[0], abuf[1], a.blk[b], first, n, proj, cb);
    else if (n > 8)
      kp_item<2, KB, kPair>(a, tab, abuf[0], abuf[0] + 2 * 8 * kKpRowQuad * kPair, a.blk[b], first, n, proj, cb);
    else
      kp_item<1, KB, kPair>(a, tab, abuf[0], abuf[0] + 8 * kKpRowQuad * kPair, a.blk[b], first, n, proj, cb);
  }
}

// ---------------------------------------------------------------- gate finish -> down A operand
// One wave per (sorted row p, run of kFinGateBlocks 128-column blocks of the intermediate); the
// decode GEMV's gate finish arithmetic.
__global__ __launch_bounds__(256) void kp_gate_finish_kernel(const float* __restrict__ inner, const uint32_t* __restrict__ ids,
                                                             const int32_t* __restrict__ order,
                                                             const int32_t* __restrict__ counts,
                                                             const int32_t* __restrict__ starts, int experts, int n, int m,
                                                             const uint16_t* __restrict__ out_gate,
                                                             const uint16_t* __restrict__ out_up,
                                                             const uint16_t* __restrict__ in_down,
                                                             uint16_t* __restrict__ a_down) {
  const int64_t wid = (int64_t)blockIdx.x * 4 + wave_id_uniform();
  const int cbs = m / 128, runs = (cbs + kFinGateBlocks - 1) / kFinGateBlocks;
  if (wid >= (int64_t)n * runs) return;
  const int64_t p = wid / runs;
  if (p >= kp_placed(counts, starts, experts)) return;
  const int run = (int)(wid % runs);
  const int64_t e = kp_expert(ids, order[p], experts);
  f32x2 gv[kFinGateBlocks], uv[kFinGateBlocks];
  uint32_t og[kFinGateBlocks], ou[kFinGateBlocks], idn[kFinGateBlocks];
#pragma unroll
  for (int i = 0; i < kFinGateBlocks; i++) {
    const int col = min(run * kFinGateBlocks + i, cbs - 1) * 128 + 2 * lane_id();
    gv[i] = *reinterpret_cast<const f32x2*>(inner + p * 2 * m + col);
    uv[i] = *reinterpret_cast<const f32x2*>(inner + p * 2 * m + m + col);
    og[i] = *reinterpret_cast<const uint32_t*>(out_gate + e * m + col);
    ou[i] = *reinterpret_cast<const uint32_t*>(out_up + e * m + col);
    idn[i] = *reinterpret_cast<const uint32_t*>(in_down + e * m + col);
  }
  auto lo = [](uint32_t v) { return f16_to_f32((uint16_t)(v & 0xFFFFu)); };
  auto hi = [](uint32_t v) { return f16_to_f32((uint16_t)(v >> 16)); };
#pragma unroll
  for (int i = 0; i < kFinGateBlocks; i++) {
    const int cb = run * kFinGateBlocks + i;
    if (cb >= cbs) break;
    float g0 = gv[i].x, g1 = gv[i].y, u0 = uv[i].x, u1 = uv[i].y;
    hadamard128_wave(g0, g1);
    hadamard128_wave(u0, u1);
    float h0 = swiglu_bf16(g0 * lo(og[i]), u0 * lo(ou[i]));
    float h1 = swiglu_bf16(g1 * hi(og[i]), u1 * hi(ou[i]));
    h0 *= lo(idn[i]);
    h1 *= hi(idn[i]);
    hadamard128_wave(h0, h1);
    kp_store_a2(a_down, p, m / 64, cb * 128 + 2 * lane_id(), h0, h1);
  }
}

// ---------------------------------------------------------------- value finish
// One wave per (sorted row p, run of kFinValueBlocks 128-column blocks): T(H128(inner) * out_down[e])
// -> values[slot].
__global__ __launch_bounds__(256) void kp_value_finish_kernel(const float* __restrict__ inner, const uint32_t* __restrict__ ids,
                                                              const int32_t* __restrict__ order,
                                                              const int32_t* __restrict__ counts,
                                                              const int32_t* __restrict__ starts, int experts, int n, int h,
                                                              const uint16_t* __restrict__ out_down,
                                                              uint16_t* __restrict__ values) {
  const int64_t wid = (int64_t)blockIdx.x * 4 + wave_id_uniform();
  const int hbs = h / 128, runs = (hbs + kFinValueBlocks - 1) / kFinValueBlocks;
  if (wid >= (int64_t)n * runs) return;
  const int64_t p = wid / runs;
  if (p >= kp_placed(counts, starts, experts)) return;
  const int run = (int)(wid % runs);
  const int slot = order[p];
  const int64_t e = kp_expert(ids, slot, experts);
  f32x2 v[kFinValueBlocks];
  uint32_t od[kFinValueBlocks];
#pragma unroll
  for (int i = 0; i < kFinValueBlocks; i++) {
    const int col = min(run * kFinValueBlocks + i, hbs - 1) * 128 + 2 * lane_id();
    v[i] = *reinterpret_cast<const f32x2*>(inner + p * h + col);
    od[i] = *reinterpret_cast<const uint32_t*>(out_down + e * h + col);
  }
#pragma unroll
  for (int i = 0; i < kFinValueBlocks; i++) {
    const int hb = run * kFinValueBlocks + i;
    if (hb >= hbs) break;
    float v0 = v[i].x, v1 = v[i].y;
    hadamard128_wave(v0, v1);
    const uint32_t pk = (uint32_t)f32_to_bf16(v0 * f16_to_f32((uint16_t)(od[i] & 0xFFFFu))) |
                        ((uint32_t)f32_to_bf16(v1 * f16_to_f32((uint16_t)(od[i] >> 16))) << 16);
    *reinterpret_cast<uint32_t*>(values + (int64_t)slot * h + hb * 128 + 2 * lane_id()) = pk;
  }
}

// ---------------------------------------------------------------- workspace
struct KpWorkspace {
  int32_t* order;   // [n]
  int32_t* counts;  // [E]
  int32_t* starts;  // [E]
  int32_t* blk;     // [3][cap]
  int32_t* nblk;
  uint16_t* a_gate; // [n][h/64][256 B]
  uint16_t* a_up;
  uint16_t* a_down; // [n][m/64][256 B]
  float* inner_gu;  // [n][2m]
  float* inner_d;   // [n][h]
  int32_t* ent;     // [2 cap] GEMM item entries, nent of them
  int32_t* nent;
  int32_t* queue;   // two claim counters, one 128 B line each
  int cap;
  size_t bytes;
};

KpWorkspace kp_carve(void* base, int64_t n, int h, int m, int64_t experts) {
  KpWorkspace w{};
  w.cap = (int)(n / kKpRows + experts + 1);
  size_t off = 0;
  char* p = static_cast<char*>(base);
  auto take = [&](size_t bytes) { char* r = p ? p + off : nullptr; off += (bytes + 255) & ~(size_t)255; return r; };
  w.order = reinterpret_cast<int32_t*>(take((size_t)n * 4));
  w.counts = reinterpret_cast<int32_t*>(take((size_t)experts * 4));
  w.starts = reinterpret_cast<int32_t*>(take((size_t)experts * 4));
  w.blk = reinterpret_cast<int32_t*>(take((size_t)3 * w.cap * 4));
  w.nblk = reinterpret_cast<int32_t*>(take(4));
  w.ent = reinterpret_cast<int32_t*>(take((size_t)2 * w.cap * 4));
  w.nent = reinterpret_cast<int32_t*>(take(4));
  w.queue = reinterpret_cast<int32_t*>(take(256));
  w.a_gate = reinterpret_cast<uint16_t*>(take((size_t)n * h * 4));
  w.a_up = reinterpret_cast<uint16_t*>(take((size_t)n * h * 4));
  w.a_down = reinterpret_cast<uint16_t*>(take((size_t)n * m * 4));
  w.inner_gu = reinterpret_cast<float*>(take((size_t)n * 2 * m * 4));
  w.inner_d = reinterpret_cast<float*>(take((size_t)n * h * 4));
  w.bytes = off;
  return w;
}

template <int KB>
int launch_kp_gemm_k(const KpGemm& g, hipStream_t s) {
  // persistent blocks, items strided over them.  The classes of up to 4 M-tiles fit two blocks per
  // CU (68-80 KB of LDS) and get 4 blocks per CU queued, so the CUs stay busy to the end of the
  // launch; the 8-tile class (96 KB) runs one block per CU.
  const int blocks = device_cus() > 0 ? device_cus() : 256;
  if (MOE_KP_MERGED) {
    hipLaunchKernelGGL((kp_gemm_merged_kernel<KB>), dim3(4 * blocks), dim3(kKpThreads), 0, s, g);
    MOE_HIP(hipGetLastError());
    return MOE_OK;
  }
  hipLaunchKernelGGL((kp_gemm_kernel<1, KB>), dim3(4 * blocks), dim3(kKpThreads), 0, s, g);
  MOE_HIP(hipGetLastError());
  hipLaunchKernelGGL((kp_gemm_kernel<2, KB>), dim3(4 * blocks), dim3(kKpThreads), 0, s, g);
  MOE_HIP(hipGetLastError());
  hipLaunchKernelGGL((kp_gemm_kernel<4, KB>), dim3(4 * blocks), dim3(kKpThreads), 0, s, g);
  MOE_HIP(hipGetLastError());
  hipLaunchKernelGGL((kp_gemm_kernel<8, KB>), dim3(blocks), dim3(kKpThreads), 0, s, g);
  MOE_HIP(hipGetLastError());
  return MOE_OK;
}

int launch_kp_gemm(const KpGemm& g, hipStream_t s) {
  if (g.bits == 4) return launch_kp_gemm_k<4>(g, s);
  if (g.bits == 3) return launch_kp_gemm_k<3>(g, s);
  return launch_kp_gemm_k<2>(g, s);
}

}  // namespace
}  // namespace moe

using namespace moe;

extern "C" {

size_t moe_k4_grouped_mlp_workspace_bytes(int rows, int slots, int hidden, int intermediate, int64_t experts) {
  if (rows <= 0 || slots <= 0 || hidden <= 0 || intermediate <= 0 || experts <= 0) return 0;
  return kp_carve(nullptr, (int64_t)rows * slots, hidden, intermediate, experts).bytes;
}

int moe_trellis_grouped_mlp(int k, const uint16_t* x, const uint32_t* ids, int rows, int slots,
                            const void* packed_gate, const void* packed_up, const void* packed_down,
                            int64_t packed_bytes, const uint16_t* in_gate, const uint16_t* out_gate,
                            const uint16_t* in_up, const uint16_t* out_up, const uint16_t* in_down,
                            const uint16_t* out_down, int hidden, int intermediate, uint16_t* values, void* workspace,
                            size_t workspace_bytes, moe_stream_t stream) {
  MOE_ARG(k >= 2 && k <= 4, "EXLR8 trellis width must be 2, 3, or 4 (got %d)", k);
  MOE_ARG(x && ids && packed_gate && packed_up && packed_down && in_gate && out_gate && in_up && out_up && in_down &&
              out_down && values && workspace,
          "null pointer argument");
  MOE_ARG(rows >= 1 && slots >= 1, "rows and slots must be positive");
  MOE_ARG(hidden > 0 && intermediate > 0 && hidden % 128 == 0 && intermediate % 128 == 0,
          "hidden and intermediate must be positive multiples of 128 (got %d, %d)", hidden, intermediate);
  const int64_t per = (int64_t)hidden * intermediate * k / 8;
  MOE_ARG(packed_bytes > 0 && packed_bytes % per == 0, "packed size %lld is not a whole number of K%d experts",
          (long long)packed_bytes, k);
  const int64_t experts = packed_bytes / per;
  MOE_ARG(experts <= 1024, "at most 1024 experts (got %lld)", (long long)experts);
  const int64_t n = (int64_t)rows * slots;
  MOE_ARG(n <= (int64_t)1 << 24, "too many slots (%lld)", (long long)n);
  const KpWorkspace w = kp_carve(workspace, n, hidden, intermediate, experts);
  if (workspace_bytes < w.bytes)
    return fail(MOE_EWORKSPACE, "workspace too small: %zu < %zu bytes", workspace_bytes, w.bytes);
  int rc = ensure_device_ready();
  if (rc) return rc;
  hipStream_t s = (hipStream_t)stream;
  // sorted work order in blocks of <= 64 rows (ids outside [0, experts) get no position)
  if ((rc = segment_table_clamped(ids, (int)n, (int)experts, kKpRows, w.order, w.counts, w.starts, w.blk, w.cap, w.nblk,
                                  (hipStream_t)stream)))
    return rc;
  hipLaunchKernelGGL(kp_order_kernel, dim3(1), dim3(256), 0, (hipStream_t)stream, w.blk, w.cap, w.nblk, w.ent, w.nent,
                     w.queue);
  MOE_HIP(hipGetLastError());
  const int64_t pw = kp_prep_waves(n, hidden, 2);
  hipLaunchKernelGGL(kp_prep_kernel, dim3((unsigned)((pw + 3) / 4)), dim3(256), 0, s, x, ids, w.order, w.counts, w.starts,
                     (int)experts, (int)n, slots, hidden, 2, 0, in_gate, in_up, w.a_gate, w.a_up);
  MOE_HIP(hipGetLastError());
  const uint8_t* table = codebook_device_table();
  if (!table) return fail(MOE_ENOTSUP, "code table not initialised on this device");
  KpGemm g{};
  g.codebook = table;
  g.packed[0] = static_cast<const uint8_t*>(packed_gate);
  g.packed[1] = static_cast<const uint8_t*>(packed_up);
  g.a[0] = w.a_gate;
  g.a[1] = w.a_up;
  g.col_off[0] = 0;
  g.col_off[1] = intermediate;
  g.nproj = 2;
  g.side = 1;
  g.K = hidden;
  g.N = intermediate;
  g.blk = w.blk;
  g.cap = w.cap;
  g.nblk = w.nblk;
  g.ent = w.ent;
  g.nent = w.nent;
  g.queue = w.queue;
  g.inner = w.inner_gu;
  g.inner_stride = 2 * intermediate;
  g.bits = k;
  if ((rc = launch_kp_gemm(g, s))) return rc;
  const int64_t fw = n * ((intermediate / 128 + kFinGateBlocks - 1) / kFinGateBlocks);
  hipLaunchKernelGGL(kp_gate_finish_kernel, dim3((unsigned)((fw + 3) / 4)), dim3(256), 0, s, w.inner_gu, ids, w.order,
                     w.counts, w.starts, (int)experts, (int)n, intermediate, out_gate, out_up, in_down, w.a_down);
  MOE_HIP(hipGetLastError());
  KpGemm d{};
  d.codebook = table;
  d.packed[0] = static_cast<const uint8_t*>(packed_down);
  d.a[0] = w.a_down;
  d.col_off[0] = 0;
  d.nproj = 1;
  d.side = 2;
  d.K = intermediate;
  d.N = hidden;
  d.blk = w.blk;
  d.cap = w.cap;
  d.nblk = w.nblk;
  d.ent = w.ent;
  d.nent = w.nent;
  d.queue = w.queue + 32;
  d.inner = w.inner_d;
  d.inner_stride = hidden;
  d.bits = k;
  if ((rc = launch_kp_gemm(d, s))) return rc;
  const int64_t vw = n * ((hidden / 128 + kFinValueBlocks - 1) / kFinValueBlocks);
  hipLaunchKernelGGL(kp_value_finish_kernel, dim3((unsigned)((vw + 3) / 4)), dim3(256), 0, s, w.inner_d, ids, w.order,
                     w.counts, w.starts, (int)experts, (int)n, hidden, out_down, values);
  MOE_HIP(hipGetLastError());
  return MOE_OK;
}

size_t moe_trellis_grouped_linear_workspace_bytes(int rows, int slots, int in_features, int out_features,
                                                  int64_t experts) {
  if (rows <= 0 || slots <= 0 || in_features <= 0 || out_features <= 0 || experts <= 0) return 0;
  return kp_carve(nullptr, (int64_t)rows * slots, max(in_features, out_features), 128, experts).bytes;
}

int moe_trellis_grouped_linear(int k, const uint16_t* x, int x_per_slot, const uint32_t* ids, int rows, int slots,
                               const void* packed, int64_t packed_bytes, const uint16_t* in_scale,
                               const uint16_t* out_scale, int in_features, int out_features, int side, uint16_t* y,
                               void* workspace, size_t workspace_bytes, moe_stream_t stream) {
  MOE_ARG(k >= 2 && k <= 4, "EXLR8 trellis width must be 2, 3, or 4 (got %d)", k);
  MOE_ARG(x && ids && packed && in_scale && out_scale && y && workspace, "null pointer argument");
  MOE_ARG(rows >= 1 && slots >= 1, "rows and slots must be positive");
  MOE_ARG(side == 1 || side == 2, "sharded_side must be 1 or 2 (got %d)", side);
  MOE_ARG(in_features > 0 && out_features > 0 && in_features % 128 == 0 && out_features % 128 == 0,
          "trellis dimensions must be positive multiples of 128 (got %d, %d)", in_features, out_features);
  const int64_t per = (int64_t)in_features * out_features * k / 8;
  MOE_ARG(packed_bytes > 0 && packed_bytes % per == 0, "packed size %lld is not a whole number of K%d experts",
          (long long)packed_bytes, k);
  const int64_t experts = packed_bytes / per;
  MOE_ARG(experts <= 1024, "at most 1024 experts (got %lld)", (long long)experts);
  const int64_t n = (int64_t)rows * slots;
  MOE_ARG(n <= (int64_t)1 << 24, "too many slots (%lld)", (long long)n);
  const KpWorkspace w = kp_carve(workspace, n, max(in_features, out_features), 128, experts);
  if (workspace_bytes < w.bytes)
    return fail(MOE_EWORKSPACE, "workspace too small: %zu < %zu bytes", workspace_bytes, w.bytes);
  int rc = ensure_device_ready();
  if (rc) return rc;
  hipStream_t s = (hipStream_t)stream;
  if ((rc = segment_table_clamped(ids, (int)n, (int)experts, kKpRows, w.order, w.counts, w.starts, w.blk, w.cap, w.nblk,
                                  (hipStream_t)stream)))
    return rc;
  hipLaunchKernelGGL(kp_order_kernel, dim3(1), dim3(256), 0, (hipStream_t)stream, w.blk, w.cap, w.nblk, w.ent, w.nent,
                     w.queue);
  MOE_HIP(hipGetLastError());
  const int64_t pw = kp_prep_waves(n, in_features, 1);
  hipLaunchKernelGGL(kp_prep_kernel, dim3((unsigned)((pw + 3) / 4)), dim3(256), 0, s, x, ids, w.order, w.counts, w.starts,
                     (int)experts, (int)n, slots, in_features, 1, x_per_slot ? 1 : 0, in_scale, in_scale, w.a_gate,
                     w.a_gate);
  MOE_HIP(hipGetLastError());
  const uint8_t* table = codebook_device_table();
  if (!table) return fail(MOE_ENOTSUP, "code table not initialised on this device");
  KpGemm g{};
  g.codebook = table;
  g.packed[0] = static_cast<const uint8_t*>(packed);
  g.a[0] = w.a_gate;
  g.col_off[0] = 0;
  g.nproj = 1;
  g.side = side;
  g.K = in_features;
  g.N = out_features;
  g.blk = w.blk;
  g.cap = w.cap;
  g.nblk = w.nblk;
  g.ent = w.ent;
  g.nent = w.nent;
  g.queue = w.queue;
  g.inner = w.inner_d;
  g.inner_stride = out_features;
  g.bits = k;
  if ((rc = launch_kp_gemm(g, s))) return rc;
  const int64_t vw = n * ((out_features / 128 + kFinValueBlocks - 1) / kFinValueBlocks);
  hipLaunchKernelGGL(kp_value_finish_kernel, dim3((unsigned)((vw + 3) / 4)), dim3(256), 0, s, w.inner_d, ids, w.order,
                     w.counts, w.starts, (int)experts, (int)n, out_features, out_scale, y);
  MOE_HIP(hipGetLastError());
  return MOE_OK;
}

int moe_k4_grouped_mlp(const uint16_t* x, const uint32_t* ids, int rows, int slots, const void* packed_gate,
                       const void* packed_up, const void* packed_down, int64_t packed_bytes, const uint16_t* in_gate,
                       const uint16_t* out_gate, const uint16_t* in_up, const uint16_t* out_up,
                       const uint16_t* in_down, const uint16_t* out_down, int hidden, int intermediate,
                       uint16_t* values, void* workspace, size_t workspace_bytes, moe_stream_t stream) {
  return moe_trellis_grouped_mlp(4, x, ids, rows, slots, packed_gate, packed_up, packed_down, packed_bytes, in_gate,
                                 out_gate, in_up, out_up, in_down, out_down, hidden, intermediate, values, workspace,
                                 workspace_bytes, stream);
}

}  // extern "C"
