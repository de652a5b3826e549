// Fused K4 trellis MoE block for decode batches (1..8 token rows) on gfx950: router, shared expert,
// routed experts and the weighted combine in ONE persistent launch.
//
// Reference semantics (paths relative to the reference root):
//   router   logits = f32(x) @ W^T, sigmoid, bias-corrected top-8  exlr8/model.py:111-132,
//                                                                   exlr8/metal/fast_router.metal:1-42
//   prep     xh = H128(x * in_scale[e])                             exlr8/metal/fast_decode_prep.metal
//   linear   inner = xh @ decode(packed_e)                          exlr8/metal/fast_decode_linear.metal
//   gate fin a = H128(swiglu_T(H(g) * og, H(u) * ou) * in_down)     exlr8/metal/fast_decode_gate_finish.metal
//   finish   T(H128(inner) * out_scale)                             exlr8/metal/fast_decode_finish.metal
//   combine  routed sum in slot order, shared, residual             exlr8/metal/fast_decode_finish_fused.metal:52-61
//
// MI355X design.
//   * Workers.  One block of kLW waves per CU; every wave takes work items from a queue until the
//     list is exhausted.  The codebook table enters LDS once per launch (the first item's loads are
//     already in flight while it is copied).
//   * Items.  A part is 2 quads (8 KB of K4 weights): 128 input rows x 128 output columns of one
//     (unit, projection, output block) -- exactly one H128 block of its input.  The list, in
//     dependency order (an item only ever waits for items before it):
//         [router] [GU(0)] [GU(1)] [GU(2)] [GF(0)] [GU(3)] [GF(1)] ... [GF(U-1)]
//         [D(0)] [D(1)] [D(2)] [D(3)] [DF(0)] [D(4)] [DF(1)] ... [DF(U-1)]
//     Unit 0 is the shared expert (it needs no routing, so its gate/up parts run beside the
//     router); GU(u) are unit u's gate/up parts, GF(u) its gate finishes (one per column block:
//     the down input), D(u) its down parts, DF(u) its down finishes (one per output block; the
//     last unit's also combine that output block of every row).  A finisher trails the parts it
//     sums by a few units.
//   * Routing.  Router items store partial logits over fixed input slices.  Each block's first
//     wave that reaches an item past GU(0) routes every row itself (top-8 into the block's LDS
//     plan table, the same in every block) while the block's other waves that need the table
//     wait on an LDS word: there is no plan hand-over between blocks.
//   * Queue.  The list is dealt round-robin over 8 sub-lists, one per XCD (block b serves sub-list
//     b mod 8); a wave claims its next item with one atomic on its sub-list's counter a whole item
//     ahead of use, so a wave that waited or finished something simply claims fewer items.  Any
//     number of resident blocks makes progress: the lowest unfinished item is always held by a
//     running wave and all its inputs come from lower items.
//   * Hand-over without counters or fences.  Every value another wave reads (router logit slices,
//     part partials, down inputs, slot outputs) is stored as one 64-bit word (value, tag), the tag
//     being the launch's epoch; a consumer reloads until every word it needs carries the current
//     tag.  Waits are bounded: an exhausted wait sets the error word and the wave continues.  The
//     epoch lives in the workspace and advances when the last block leaves, so a replayed launch
//     (the same arguments) never accepts its predecessor's words.  A stale word is mistaken for a
//     current one only if exactly a multiple of 2^32 - 1 launches separate them with the word never
//     rewritten in between.
//   * Deterministic reductions: a finisher sums its parts' partials in part order; part boundaries
//     depend only on the layer shape, so a token row gives the same bits alone or in an 8-row
//     batch.  Router logits are summed over fixed input slices in slice order.
//   * Per-wave pipeline: while quad 0 of an item is decoded, quad 1 streams in; while quad 1 is
//     decoded, quad 0 and the input block of the next item stream in.  Partial stores are never
//     waited for.
//   * Decode: the piece decoder of the GEMVs (fp16 code table for single-token launches, E4M3 byte
//     table for batches), fp16 MFMA with x split into hi and lo rows (k4_moe.hip).
#include <hip/hip_runtime.h>

#include "moe_device.h"
#include "moe_host.h"
#include "moe_plan.h"
#include "layer_sync.h"

namespace moe {

#ifndef MOE_LAYER_WAVES
#define MOE_LAYER_WAVES 12
#endif
// arithmetic codeword pairs per word (even, odd words of a piece) in the single-token decode
#ifndef MOE_LAYER_ALU_EVEN
#define MOE_LAYER_ALU_EVEN 1
#endif
#ifndef MOE_LAYER_ALU_ODD
#define MOE_LAYER_ALU_ODD 2
#endif

// arithmetic codeword pairs per word (even, odd words of a piece) in the K3 decode (1/2 measured
// on MI355X for the routed one-row block: 74.0 us against 75.7 for 2/2, 79.3 for 2/3, 74.3 for 1/1)
#ifndef MOE_LAYER3_ALU_EVEN
#define MOE_LAYER3_ALU_EVEN 1
#endif
#ifndef MOE_LAYER3_ALU_ODD
#define MOE_LAYER3_ALU_ODD 2
#endif

// longest pause (in 64-clock sleeps) of the finishes' and staging waits: they sit on the launch's
// final dependency chain, so a wait must not oversleep the value it waits for by long
#ifndef MOE_LAYER_WAIT
#define MOE_LAYER_WAIT 16
#endif
#ifndef MOE_LAYER_PRIO_UNITS
#define MOE_LAYER_PRIO_UNITS 2
#endif
// arithmetic pairs per even / odd word for batches (E4M3 byte table)
#ifndef MOE_LAYER8_ALU_EVEN
#define MOE_LAYER8_ALU_EVEN 1
#endif
#ifndef MOE_LAYER8_ALU_ODD
#define MOE_LAYER8_ALU_ODD 2
#endif
#ifndef MOE_LAYER_GS
#define MOE_LAYER_GS 1
#endif
constexpr int kLW = MOE_LAYER_WAVES;
constexpr int kXcds = 8;            // queue sub-lists
constexpr int kQueueStride = 32;    // ints between sub-list counters (one 128 B line each)
constexpr int kSumRound = 8;        // partial rows summed per round by the gate finishes
constexpr int kStraggle = 256;      // claims since a part's own after which it counts as behind

enum LayerFin { LFIN_VALUES = 0, LFIN_COMBINE = 1 };

struct LayerWs {
  Plan* plan;
  int32_t* flags;        // LayerFlag words
  int32_t* queue;        // [kXcds][kQueueStride] sub-list counters
  uint64_t* logit_part;  // [kMaxRows][h / kRouterSlice][256] tagged
  uint64_t* partial;     // [slot][3 (h/128)(m/128) parts][128] tagged
  uint64_t* down_xh;     // [slot][m] tagged
  uint64_t* yslot;       // [slot][h] tagged
  uint64_t* gsum;        // [unit][token][m / 128][2][group][128] tagged: the last units' group sums
  size_t bytes;
};

struct LayerArgs {
  const uint8_t* tab8;       // the device's E4M3 code table (64 KB)
  const uint16_t* tab16;     // the same table as fp16 (128 KB)
  const uint16_t* x;         // expert (and router) input [rows, h] bf16
  const uint16_t* residual;  // [rows, h] bf16 (combine)
  int rows;
  int bits;                  // trellis width of the experts (3 or 4)
  int route;                 // 1: router items + plan on the device; 0: plan prebuilt from ids
  const float* router_w;     // [256, h] fp32
  const float* bias;         // [256] fp32
  uint32_t* ids;             // route: out [rows, 9]
  float* scores;             // route: out [rows, 8]; else the caller's [rows, 8] (combine)
  const uint8_t* packed[3];  // gate, up (side 1), down (side 2)
  const uint16_t* in_scale[3];
  const uint16_t* out_scale[3];
  int h, m;
  int experts;               // experts per packed projection (ids are clamped below it)
  int fin;
  uint16_t* out;             // combine [rows, h]
  uint16_t* values;          // values [slots, h]
  // one row, norm_x set: the launch first forms the layer's residual add + RMSNorm itself,
  // h = T(norm_x + norm_res) into h_row (= residual) and the normalised row into x_row (= x)
  const uint16_t* norm_x;
  const uint16_t* norm_res;
  const uint16_t* norm_w;
  float eps;
  uint16_t* h_row;
  uint16_t* x_row;
  int wait_polls;            // bound of a cross-wave wait (moe_set_wait_bound)
  LayerWs w;
};

// Returns the unit count.  Every word is requested unconditionally (indices clamped into the
// arrays) so the loads issue back to back; units beyond the count are stored as empty.
__device__ __forceinline__ int load_plan(const Plan* P, PlanLds& T) {
  const int units = min(max(__builtin_amdgcn_readfirstlane(ld_coh_i(&P->units)), 1), kMaxUnits);
  const int lane = lane_id();
#pragma unroll
  for (int h = 0; h < 2; h++) {
    if (h == 1 && units <= 64) break;
    const int u = min(lane + 64 * h, kMaxUnits - 1);
    const bool ok = lane + 64 * h < units;
    const int ex = ld_coh_i(&P->expert[u]);
    const int nt = ld_coh_i(&P->ntok[u]);
    int tks[kMaxRows], sls[kMaxRows];
#pragma unroll
    for (int t = 0; t < kMaxRows; t++) {
      tks[t] = ld_coh_i(&P->tok[u][t]);
      sls[t] = ld_coh_i(&P->slot[u][t]);
    }
    uint32_t tp = 0, s0 = 0, s1 = 0;
#pragma unroll
    for (int t = 0; t < kMaxRows; t++) {
      tp |= (uint32_t)(tks[t] & 7) << (3 * t);
      if (t < 4) s0 |= (uint32_t)(sls[t] & 127) << (7 * t);
      else s1 |= (uint32_t)(sls[t] & 127) << (7 * (t - 4));
    }
    if (lane + 64 * h < kMaxUnits) {
      T.ex[u] = ok ? ex : 0;
      T.nt[u] = ok ? nt : 0;
      T.tok[u] = tp;
      T.sl0[u] = s0;
      T.sl1[u] = s1;
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  return units;
}
// Every field is clamped into range when read, so a plan that was never published (an exhausted
// wait) can give wrong results but no out-of-bounds access.
struct UnitInfo {
  int e, ntok;
  uint32_t tok, sl0, sl1;
  int rows;
  __device__ __forceinline__ int row(int t) const { return min((int)((tok >> (3 * t)) & 7u), rows - 1); }
  __device__ __forceinline__ int slot(int t) const {
    const int s = t < 4 ? (int)((sl0 >> (7 * t)) & 127u) : (int)((sl1 >> (7 * (t - 4))) & 127u);
    return min(s, kMaxUnits - 1);
  }
};
__device__ __forceinline__ UnitInfo unit_info(const PlanLds& T, int u, int experts, int rows) {
  u = min(max(u, 0), kMaxUnits - 1);
  UnitInfo i;
  i.rows = rows;
  i.e = min(max(__builtin_amdgcn_readfirstlane(T.ex[u]), 0), experts - 1);
  i.ntok = min(max(__builtin_amdgcn_readfirstlane(T.nt[u]), 0), kMaxRows);
  i.tok = (uint32_t)__builtin_amdgcn_readfirstlane((int)T.tok[u]);
  i.sl0 = (uint32_t)__builtin_amdgcn_readfirstlane((int)T.sl0[u]);
  i.sl1 = (uint32_t)__builtin_amdgcn_readfirstlane((int)T.sl1[u]);
  return i;
}

// ---------------------------------------------------------------- the item list
struct Items {
  int HB;     // h / 128: parts per gate/up segment, down output blocks
  int MB;     // m / 128: gate/up column blocks, parts per down segment
  int G;      // gate/up parts per unit: 2 * MB * HB
  int D;      // down parts per unit: HB * MB
  int R;      // router items
  int S;      // router slices per expert
  int NG;     // group sums per gate/up column block of the last unit (0: none)
  int route;
};
enum ItemKind { IT_GU = 0, IT_DOWN = 1, IT_ROUTER = 2, IT_GF = 3, IT_DF = 4, IT_NONE = 5, IT_GS = 6 };
struct Item {
  int kind, u, a, b, c;  // GU: a = output block, b = projection, c = part; DOWN: a = output block,
                         // c = part (input block); GF / DF: a = block; GS: a = block, b = group;
                         // ROUTER: a = item
};
// The list: [router R], then phase A, then phase B.
//   phase A: for the units 0..U-1, block b = GU(b), followed for b >= kLagG by GF(b - kLagG);
//            then GF of the last kLagG units, each unit's GF preceded by its group sums GS (their
//            parts are the list's last gate/up items, so their finishes head the launch's final
//            dependency chain: GS items sum the parts' rounds in parallel, and the GF then sums the
//            group sums in one round instead of HB / 8 rounds in sequence)
//   phase B: for the units 0..U-1, block b = D(b), followed for b >= kLagD by DF(b - kLagD);
//            then DF of the last units
// Unit 0 (the shared expert when routing) needs no plan, so its gate/up parts run beside the
// router.  A finisher comes kLag units after the parts it sums, so its inputs are normally complete
// when it is taken; the last unit's down finishes (the combine) close the list.
#ifndef MOE_LAYER_LAG_G
#define MOE_LAYER_LAG_G 2
#endif
#ifndef MOE_LAYER_LAG_D
#define MOE_LAYER_LAG_D 4
#endif
constexpr int kLagG = MOE_LAYER_LAG_G, kLagD = MOE_LAYER_LAG_D;
__host__ __device__ __forceinline__ int imin(int a, int b) { return a < b ? a : b; }
// The list's shape for a layer: hidden h, intermediate m, route = the launch routes itself.
__host__ __device__ __forceinline__ Items make_items(int h, int m, int route) {
  Items L;
  L.HB = h / 128;
  L.MB = m / 128;
  L.G = 2 * L.MB * L.HB;
  L.D = L.HB * L.MB;
  L.S = h / kRouterSlice;
  // group sums for the last kLagG units when their gate finishes then take one round (HB <= 8 kSumRound)
  L.NG = MOE_LAYER_GS && (L.HB + kSumRound - 1) / kSumRound <= kSumRound ? (L.HB + kSumRound - 1) / kSumRound : 0;
  L.R = route ? 256 * L.S : 0;
  L.route = route;
  return L;
}
// items that need no plan (the positions of GU(0) do not depend on the unit count)
__host__ __device__ __forceinline__ int pre_items(const Items& L) { return L.route ? L.R + L.G : 0; }
__host__ __device__ __forceinline__ int list_len(const Items& L, int U) {
  return (L.route ? L.R : 0) + U * (L.G + L.MB) + imin(U, kLagG) * L.NG * L.MB + U * (L.D + L.HB);
}
// position j inside a phase of U blocks of `big` part items, each followed after `lag` blocks by
// `small` finish items: sets (is_finish, unit, index inside the block); units count from 0
__host__ __device__ __forceinline__ void phase_at(int j, int U, int big, int small, int lag, bool& fin, int& unit,
                                                  int& r) {
  const int lead = imin(U, lag);  // blocks without a finish tail
  if (j < lead * big) {
    fin = false;
    unit = j / big;
    r = j - unit * big;
    return;
  }
  j -= lead * big;
  const int mid = U - lead;  // blocks with a finish tail
  if (j < mid * (big + small)) {
    const int k = j / (big + small), q = j - k * (big + small);
    if (q < big) {
      fin = false;
      unit = lead + k;
      r = q;
    } else {
      fin = true;
      unit = k;
      r = q - big;
    }
    return;
  }
  j -= mid * (big + small);
  fin = true;
  unit = mid + j / small;
  r = j - (unit - mid) * small;
}
__host__ __device__ __forceinline__ void set_gu(const Items& L, Item& it, int u, int r) {
  it.kind = IT_GU;
  it.u = u;
  it.a = r / (2 * L.HB);
  const int rem = r - it.a * 2 * L.HB;
  it.b = rem / L.HB;
  it.c = rem - it.b * L.HB;
}
__host__ __device__ __forceinline__ void set_down(const Items& L, Item& it, int u, int r) {
  it.kind = IT_DOWN;
  it.u = u;
  it.c = r / L.HB;
  it.a = r - it.c * L.HB;
}
__host__ __device__ __forceinline__ Item item_at(const Items& L, int j, int U) {
  Item it{IT_NONE, 0, 0, 0, 0};
  if (L.route) {
    // The first R + G positions hold the router items and GU(0) mixed in the ratio R : G within
    // every run of kXcds * kLW positions (one position per wave of eight blocks), so every block
    // starts with some router items: its waves that finish them route the block early.
    const int P = L.R + L.G;
    if (j < P) {
      constexpr int C = kXcds * kLW;
      const int c0 = j - j % C, c1 = imin(c0 + C, P);
      const int r0 = c0 * L.R / P, rc = c1 * L.R / P - r0;  // below 2^31: P <= 18432, R <= 2048
      const int o = j - c0;  // = 8 wave + sub-list for the first waves: wave < rc / 8 routes
      if (o < rc) {
        it.kind = IT_ROUTER;
        it.a = r0 + o;
        return it;
      }
      set_gu(L, it, 0, (c0 - r0) + (o - rc));
      return it;
    }
    j -= L.R;
  }
  bool fin;
  int unit, r;
  const int lenA = U * (L.G + L.MB), NU = imin(U, kLagG), NGS = L.NG * L.MB, tailA = lenA - NU * L.MB;
  if (j >= tailA && j < lenA + NU * NGS) {
    // per unit of the last NU: its group sums (block-major), then its gate finishes
    const int t = j - tailA, k = t / (NGS + L.MB), q = t - k * (NGS + L.MB);
    it.u = U - NU + k;
    if (q < NGS) {
      it.kind = IT_GS;
      it.a = q / L.NG;
      it.b = q - it.a * L.NG;
    } else {
      it.kind = IT_GF;
      it.a = q - NGS;
    }
    return it;
  }
  if (j < lenA) {
    phase_at(j, U, L.G, L.MB, kLagG, fin, unit, r);
    if (fin) {
      it.kind = IT_GF;
      it.u = unit;
      it.a = r;
    } else {
      set_gu(L, it, unit, r);
    }
    return it;
  }
  j -= lenA + NU * NGS;
  if (j < U * (L.D + L.HB)) {
    phase_at(j, U, L.D, L.HB, kLagD, fin, unit, r);
    if (fin) {
      it.kind = IT_DF;
      it.u = unit;
      it.a = r;
    } else {
      set_down(L, it, unit, r);
    }
  }
  return it;
}
__device__ __forceinline__ bool is_part(const Item& it) { return it.kind == IT_GU || it.kind == IT_DOWN; }

// ---------------------------------------------------------------- tables and LDS
// The code table in LDS: the 64 KB E4M3 byte table for every row count.  (The 128 KB fp16 form
// decodes no faster -- measured 28.1 vs 28.6 codewords/ns/CU in a register-fed loop -- and doubles
// the launch's start-up copy.)
template <int NT>
struct LTable {
  static constexpr bool kF16 = false;
  static constexpr int kBytes = kF16 ? 131072 : 65536;
};
constexpr int xa_halves(int nt) { return 2 * 2 * (2 * nt) * 4 * 8; }  // [qb][rh][m][g][8] fp16 per wave

__device__ __forceinline__ int part_count(const LayerArgs& a) { return 3 * (a.h / 128) * (a.m / 128); }
__device__ __forceinline__ uint64_t* part_ptr(const LayerArgs& a, int slot, int index) {
  return a.w.partial + ((int64_t)slot * part_count(a) + index) * 128;
}

// ---------------------------------------------------------------- one part: operands
// The wave's piece of quad qb (0, 1) of a part, K-bit tiles: 8 consecutive tiles (8K words each)
// per chunk; lane nn takes tile nn / 8 of the first two, piece nn % 8, and set s4 the next two.
// K4: 16 B pieces, sets at +256 B; K3: 12 B pieces, sets at +192 B.
template <int KB>
__device__ __forceinline__ const uint8_t* quad_ptr(const LayerArgs& a, const UnitInfo& ui, const Item& it, int qb) {
  const int lane = lane_id();
  const int g = lane >> 4, nn = lane & 15;
  const bool gu = it.kind == IT_GU;
  const int side = gu ? 1 : 2;
  const int in_f = gu ? a.h : a.m;
  const int it_tiles = in_f / 16, obs = gu ? a.m / 128 : a.h / 128;
  const uint8_t* base = a.packed[gu ? it.b : 2];
  return base + chunk_index(side, (uint64_t)ui.e, it.a, 8 * it.c + 4 * qb + g, it_tiles, obs) * (uint64_t)(256 * KB) +
         (nn >> 3) * (32 * KB) + (nn & 7) * (4 * KB);
}
template <int KB>
__device__ __forceinline__ void load_quad(u32x4 (&pc)[4], const uint8_t* qp) {
  if constexpr (KB == 4) {
#pragma unroll
    for (int s4 = 0; s4 < 4; s4++) pc[s4] = load_stream16(qp + 256 * s4);
  } else {
    static_assert(KB == 3, "the fused block decodes K3 and K4 tiles");
#pragma unroll
    for (int s4 = 0; s4 < 4; s4++) {
      const uint32_t* w = reinterpret_cast<const uint32_t*>(qp + 192 * s4);
      pc[s4] = u32x4{__builtin_nontemporal_load(w), __builtin_nontemporal_load(w + 1), __builtin_nontemporal_load(w + 2), 0u};
    }
  }
}
// The raw input block of a part, fetched ahead of its staging.
//   DPRE (one token): both kinds issue two 64-bit loads into r[0..1] and r[2..3] -- gate/up the
//     aligned 8 bytes holding the lane's bf16 x pair and those holding its in_scale pair (the
//     lane's half is picked at staging), down the two tagged down-input words.  Same loads, same
//     registers, same order: with kind-dependent register sets the compiler keeps the other
//     kind's words alive and copies them at the loop's joins, and a copy of a register still
//     loading waits for every memory operation issued since (the next part's quads included).
//   otherwise: gate/up the x pair of each token (r[t]) and the in_scale pair (r[NT]); down inputs
//     are loaded at staging.
template <int NT, bool DPRE>
struct InBlock {
  static_assert(!DPRE || NT == 1, "down inputs are fetched ahead for one token only");
  uint32_t r[DPRE ? 4 : NT + 1];
};
template <int NT, bool DPRE>
__device__ __forceinline__ void fetch_in(const LayerArgs& a, const UnitInfo& ui, const Item& it, InBlock<NT, DPRE>& in) {
  const int lane = lane_id();
  if (DPRE) {
    uint64_t w0, w1;
    if (it.kind == IT_GU) {
      // 8-byte words (x and in_scale rows are 8-byte aligned): lane l's pair is half l & 1 of word
      // l / 2 of the 128-element block
      const int blk = 128 * it.c;
      w0 = reinterpret_cast<const uint64_t*>(a.x + (int64_t)ui.row(0) * a.h + blk)[lane >> 1];
      w1 = reinterpret_cast<const uint64_t*>(a.in_scale[it.b] + (int64_t)ui.e * a.h + blk)[lane >> 1];
    } else {
      const uint64_t* p = a.w.down_xh + (int64_t)ui.slot(0) * a.m + 128 * it.c + 2 * lane;
      w0 = ld_tag(p);
      w1 = ld_tag(p + 1);
    }
    in.r[0] = (uint32_t)w0;
    in.r[1] = (uint32_t)(w0 >> 32);
    in.r[2] = (uint32_t)w1;
    in.r[3] = (uint32_t)(w1 >> 32);
  } else if (it.kind == IT_GU) {
    const int off = 128 * it.c + 2 * lane;
#pragma unroll
    for (int t = 0; t < NT; t++)
      in.r[t] = *reinterpret_cast<const uint32_t*>(a.x + (int64_t)ui.row(min(t, max(ui.ntok - 1, 0))) * a.h + off);
    in.r[NT] = *reinterpret_cast<const uint32_t*>(a.in_scale[it.b] + (int64_t)ui.e * a.h + off);
  }
}
// The lane's two words of a tagged block (ld_tag_pair), for a block that may not be written yet:
// while it is not, the wave polls one word of it (lane 0's) and loads the whole block again only
// once that word carries `tag`.  A waiting wave then requests 8 bytes per poll instead of the
// block's 1 KB: the waves waiting for one block poll the same lines, and their traffic slows the
// block's writer.  `known_missing`: the caller has just seen the block incomplete (skip the first
// full load).
template <int kMaxPauses, class A>
__device__ __forceinline__ f32x2 ld_tag_pair_sampled(const A& a, const uint64_t* p, uint32_t tag, bool known_missing) {
  if (!known_missing) {
    const uint64_t w0 = ld_tag(p), w1 = ld_tag(p + 1);
    if (__all(has_tag(w0, tag) && has_tag(w1, tag))) return f32x2{tag_value(w0), tag_value(w1)};
  }
  int spins = 0;
  for (;;) {
    uint64_t w = 0;
    if (lane_id() == 0) w = ld_tag(p);
    if ((uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(w >> 32)) == tag) break;
    if (!keep_waiting<kMaxPauses>(a, spins)) {
      // the bound ran out (the error word is set): the words as they are, without a second wait
      const uint64_t w0 = ld_tag(p), w1 = ld_tag(p + 1);
      return f32x2{tag_value(w0), tag_value(w1)};
    }
  }
  return ld_tag_pair<kMaxPauses>(a, p, tag);
}
// Largest value over the wave's lanes (valid in every lane after the read of lane 63).
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_f32<0xB1>(v));
  v = fmaxf(v, dpp_f32<0x4E>(v));
  v = fmaxf(v, dpp_f32<0x124>(v));
  v = fmaxf(v, dpp_f32<0x128>(v));
  v = fmaxf(v, dpp_f32<0x142, 0xA>(v));
  v = fmaxf(v, dpp_f32<0x143, 0xC>(v));
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
// A fragments of the part's 128 input rows (hi and lo fp16 rows per token) into the wave's LDS
// slice.  Down inputs are polled until they carry the launch's tag.
// A block whose values reach 2^15 (beyond what the fp16 hi row holds; the reference computes in
// fp32) is staged scaled by 2^-k so that its largest value stays below 2^15, and the part's
// partial sums are multiplied back by scale[t] = 2^k (powers of two: exact).  Other blocks keep
// scale 1 and bit-identical results.
template <int NT, bool DPRE>
__device__ __forceinline__ void stage_in(const LayerArgs& a, const UnitInfo& ui, const Item& it,
                                         const InBlock<NT, DPRE>& in, uint32_t tag, _Float16* __restrict__ xw,
                                         float (&scale)[NT]) {
  const int lane = lane_id();
  float v0[NT], v1[NT];
  uint32_t w[4] = {0u, 0u, 0u, 0u};
  if (DPRE) {
#pragma unroll
    for (int k = 0; k < 4; k++) w[k] = in.r[k];
  }
  if (it.kind == IT_GU) {
    const bool odd = (lane & 1) != 0;
    const uint32_t scw = DPRE ? (odd ? w[3] : w[2]) : in.r[NT];
    const float s0 = f16_to_f32((uint16_t)(scw & 0xFFFFu)), s1 = f16_to_f32((uint16_t)(scw >> 16));
#pragma unroll
    for (int t = 0; t < NT; t++) {
      if (t < ui.ntok) {
        const uint32_t xw2 = DPRE ? (odd ? w[1] : w[0]) : in.r[t];
        v0[t] = bf16_to_f32((uint16_t)(xw2 & 0xFFFFu)) * s0;
        v1[t] = bf16_to_f32((uint16_t)(xw2 >> 16)) * s1;
        hadamard128_wave(v0[t], v1[t]);
      }
    }
  } else {
    bool ready = true;
    if (DPRE) {
      ready = w[1] == tag && w[3] == tag;
      v0[0] = __uint_as_float(w[0]);
      v1[0] = __uint_as_float(w[2]);
    }
    if (!DPRE || !__all(ready)) {
#pragma unroll
      for (int t = 0; t < NT; t++) {
        if (t < ui.ntok) {
          const f32x2 hv = ld_tag_pair_sampled<MOE_LAYER_WAIT>(
              a, a.w.down_xh + (int64_t)ui.slot(t) * a.m + 128 * it.c + 2 * lane, tag, DPRE);
          v0[t] = hv.x;
          v1[t] = hv.y;
        }
      }
      // the (rare) polling path ends with nothing of its own outstanding: otherwise the compiler,
      // unsure whether a poll reload is still pending where the paths meet, waits for every memory
      // operation of the wave (the prefetched quads included) before the registers are reused
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    }
  }
#pragma unroll
  for (int t = 0; t < NT; t++) {
    scale[t] = 1.0f;
    if (t < ui.ntok) {
      const float big = fmaxf(fabsf(v0[t]), fabsf(v1[t]));
      if (__any(big >= 32768.0f)) {
        const float mx = wave_max(big);
        // floor(log2(mx)) from the exponent field (>= 15 here; inf and NaN give 128)
        const int e = (int)((__float_as_uint(mx) >> 23) & 0xFFu) - 127;
        const int k = min(e - 14, 120);
        v0[t] = ldexpf(v0[t], -k);
        v1[t] = ldexpf(v1[t], -k);
        scale[t] = ldexpf(1.0f, k);
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
      if (t < ui.ntok) {
        float xv = jj ? v1[t] : v0[t];
        // x is materialised in fp32 first so both conversions below see the same value
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
}
// Decode one quad held in pc (the pieces' predecessor words come from the neighbouring lane) and
// accumulate it on the matrix cores against the staged A fragments of quad qb.
template <int NT, int KB>
__device__ __forceinline__ void decode_quad(const u32x4 (&pc)[4], int qb, int ntok, const uint8_t* __restrict__ tab,
                                            const _Float16* __restrict__ xw, f32x4 (&acc)[4][2]) {
  const int lane = lane_id();
  const int g = lane >> 4, nn = lane & 15;
  const int src_lane = (lane & 7) == 0 ? lane + 7 : lane - 1;
  const bool live = nn < 2 * ntok;
  f16x8 A[2];
#pragma unroll
  for (int rh = 0; rh < 2; rh++)
    A[rh] = live ? *reinterpret_cast<const f16x8*>(xw + (((qb * 2 + rh) * (2 * NT) + nn) * 4 + g) * 8)
                 : f16x8{0, 0, 0, 0, 0, 0, 0, 0};
  uint32_t prior[4];
#pragma unroll
  for (int s4 = 0; s4 < 4; s4++) prior[s4] = (uint32_t)__shfl((int)(KB == 4 ? pc[s4].w : pc[s4].z), src_lane, 64);
#pragma unroll
  for (int s4 = 0; s4 < 4; s4++) {
    const u32x4 v = pc[s4];
#pragma unroll
    for (int rh = 0; rh < 2; rh++) {
      f16x2 q[2][4];
      if constexpr (KB == 3) {
        const uint32_t S[4] = {prior[s4], v.x, v.y, v.z};
        if (rh == 0)
          decode_k3_pair_words<MOE_LAYER3_ALU_EVEN, MOE_LAYER3_ALU_ODD, 0>(S, tab, q);
        else
          decode_k3_pair_words<MOE_LAYER3_ALU_EVEN, MOE_LAYER3_ALU_ODD, 2>(S, tab, q);
      } else {
        const uint32_t w0 = rh ? v.z : v.x, w1 = rh ? v.w : v.y, p0 = rh ? v.y : prior[s4];
        if (LTable<NT>::kF16)
          decode_pair_words_f16<MOE_LAYER_ALU_EVEN, MOE_LAYER_ALU_ODD, true>(w0, w1, p0, tab, q);
        else
          decode_pair_words_f16<MOE_LAYER8_ALU_EVEN, MOE_LAYER8_ALU_ODD, false>(w0, w1, p0, tab, q);
      }
      const f16x8 b0 = frag(q[0][0], q[0][1], q[1][0], q[1][1]);
      const f16x8 b1 = frag(q[0][2], q[0][3], q[1][2], q[1][3]);
      acc[s4][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[rh], b0, acc[s4][0], 0, 0, 0);
      acc[s4][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[rh], b1, acc[s4][1], 0, 0, 0);
      mfma_acc_guard(acc[s4][0], acc[s4][1]);
    }
  }
}
// The part's partial sums: token t = D rows 2t, 2t + 1, held by lanes 16 (t / 2) + n, registers
// 2 (t % 2), +1.  Tagged stores, never waited for.  One token: the 128 sums pass through the
// wave's LDS row `pst` so that every lane stores two columns with no branch around the stores
// (stores under a branch leave the compiler unsure how many are outstanding, and it then waits
// for all of them before the next part's staging).
template <int NT>
__device__ __forceinline__ void store_partials(const LayerArgs& a, const UnitInfo& ui, const Item& it,
                                               const f32x4 (&acc)[4][2], uint32_t tag, const Items& L,
                                               float* __restrict__ pst, const float (&scale)[NT]) {
  const int lane = lane_id();
  const int g = lane >> 4, nn = lane & 15;
  const int index = it.kind == IT_GU ? (it.b * L.MB + it.a) * L.HB + it.c : 2 * L.MB * L.HB + it.a * L.MB + it.c;
  if (NT == 1) {
    if (g == 0) {
#pragma unroll
      for (int s4 = 0; s4 < 4; s4++)
#pragma unroll
        for (int hh = 0; hh < 2; hh++)
          pst[16 * (2 * s4 + (nn >> 3)) + (nn & 7) + 8 * hh] =
              fmaf(acc[s4][hh][1], 1.0f / 2048.0f, acc[s4][hh][0]) * scale[0];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // lane l stores columns l and 64 + l: each store instruction writes 512 contiguous bytes (whole
    // lines; interleaved pairs would write every line in two halves)
    uint64_t* pw = part_ptr(a, ui.slot(0), index) + lane;
    st_tag(pw, pst[lane], tag);
    st_tag(pw + 64, pst[64 + lane], tag);
    return;
  }
#pragma unroll
  for (int t = 0; t < NT; t++) {
    if (t < ui.ntok && g == (t >> 1)) {
      uint64_t* pw = part_ptr(a, ui.slot(t), index);
      const int r0 = 2 * (t & 1);
#pragma unroll
      for (int s4 = 0; s4 < 4; s4++)
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
          const int col = 16 * (2 * s4 + (nn >> 3)) + (nn & 7) + 8 * hh;
          st_tag(pw + col, fmaf(acc[s4][hh][r0 + 1], 1.0f / 2048.0f, acc[s4][hh][r0]) * scale[t], tag);
        }
    }
  }
}

// ---------------------------------------------------------------- finishes
// Sums, for each of the K part rows p[k], of the partials of parts [0, n) (stride 128 words) for
// columns 2 lane, 2 lane + 1, in part order, once every word carries `tag`.  Rounds of B parts per
// row: every word of a round is requested before any is examined (indices clamped, not branched
// on, so the loads issue back to back).  A round that is not complete is waited for on a sample
// (one word per lane), so a waiting wave costs 512 B per poll instead of the round's, and loaded
// again.
template <int K, int B>
__device__ __forceinline__ void sum_parts(const LayerArgs& a, const uint64_t* const (&p)[K], int n, uint32_t tag,
                                          f32x2 (&s)[K]) {
  const int lane = cold_lane();
#pragma unroll
  for (int k = 0; k < K; k++) s[k] = f32x2{0.0f, 0.0f};
  int spins = 0;
  for (int i0 = 0; i0 < n; i0 += B) {
    uint64_t w[K][B][2];
    for (;;) {
#pragma unroll
      for (int k = 0; k < K; k++)
#pragma unroll
        for (int i = 0; i < B; i++) {
          const uint64_t* q = p[k] + (int64_t)min(i0 + i, n - 1) * 128 + 2 * lane;
          w[k][i][0] = ld_tag(q);
          w[k][i][1] = ld_tag(q + 1);
        }
      bool ok = true;
#pragma unroll
      for (int k = 0; k < K; k++)
#pragma unroll
        for (int i = 0; i < B; i++) ok = ok & (int)has_tag(w[k][i][0], tag) & (int)has_tag(w[k][i][1], tag);
      if (__all(ok)) break;
      bool live = true;
      for (;;) {
        const int k = K == 1 ? 0 : (lane >> 5) % K;
        const uint64_t* q = p[k] + (int64_t)min(i0 + (lane & 31) % B, n - 1) * 128 + (lane * 37 + 11) % 128;
        if (__all(has_tag(ld_tag(q), tag))) break;
        if (!keep_waiting<MOE_LAYER_WAIT>(a, spins)) {
          live = false;
          break;
        }
      }
      if (!live) break;
    }
    // a round's parts are summed on their own, then added: the sum of a round of kSumRound parts
    // is the same float whether this wave forms it or a group-sum item does
#pragma unroll
    for (int k = 0; k < K; k++) {
      float rx = 0.0f, ry = 0.0f;
#pragma unroll
      for (int i = 0; i < B; i++) {
        if (i0 + i < n) {
          rx += tag_value(w[k][i][0]);
          ry += tag_value(w[k][i][1]);
        }
      }
      s[k].x += rx;
      s[k].y += ry;
    }
  }
}

// Group sum g of projection k, column block ob, token t of grouped unit gi (0: the first of the
// last kLagG units): 128 tagged words; the groups of one (gi, t, ob, k) are consecutive.
__device__ __forceinline__ uint64_t* group_ptr(const LayerArgs& a, const Items& L, int gi, int t, int ob, int k,
                                               int g) {
  return a.w.gsum + (((((int64_t)gi * kMaxRows + t) * L.MB + ob) * 2 + k) * L.NG + g) * 128;
}

// Group sum g of column block ob of grouped unit gi (unit ui): its gate and up parts of round g,
// summed as a gate finish sums one round, for each token.
__device__ void group_sum(const LayerArgs& a, const UnitInfo& ui, int gi, int ob, int g, uint32_t tag,
                          const Items& L) {
  const int lane = cold_lane();
  const int i0 = g * kSumRound, n = min(kSumRound, L.HB - i0);
  for (int t = 0; t < ui.ntok; t++) {
    const int s = ui.slot(t);
    const uint64_t* rows[2] = {part_ptr(a, s, (0 * L.MB + ob) * L.HB + i0), part_ptr(a, s, (1 * L.MB + ob) * L.HB + i0)};
    f32x2 gu[2];
    sum_parts<2, kSumRound>(a, rows, n, tag, gu);
#pragma unroll
    for (int k = 0; k < 2; k++) {
      uint64_t* dst = group_ptr(a, L, gi, t, ob, k, g) + 2 * lane;
      st_tag(dst, gu[k].x, tag);
      st_tag(dst + 1, gu[k].y, tag);
    }
  }
}

// gate finish of column block ob of unit ui: the down input of each of its tokens (gi >= 0: grouped
// unit gi, whose rounds were summed by its group-sum items)
__device__ void gate_finish(const LayerArgs& a, const UnitInfo& ui, int ob, uint32_t tag, const Items& L, int gi) {
  const int lane = cold_lane();
  const int col = ob * 128 + 2 * lane;
  const int64_t si = (int64_t)ui.e * a.m + col;
  const uint32_t og = *reinterpret_cast<const uint32_t*>(a.out_scale[0] + si);
  const uint32_t ou = *reinterpret_cast<const uint32_t*>(a.out_scale[1] + si);
  const uint32_t idn = *reinterpret_cast<const uint32_t*>(a.in_scale[2] + si);
  auto lo = [](uint32_t v) { return f16_to_f32((uint16_t)(v & 0xFFFFu)); };
  auto hi = [](uint32_t v) { return f16_to_f32((uint16_t)(v >> 16)); };
  for (int t = 0; t < ui.ntok; t++) {
    const int s = ui.slot(t);
    const uint64_t* rows[2] = {part_ptr(a, s, (0 * L.MB + ob) * L.HB), part_ptr(a, s, (1 * L.MB + ob) * L.HB)};
    f32x2 gu[2];
    if (gi >= 0) {
      // the group sums of the unit's HB / kSumRound rounds, in one round
      const uint64_t* gs[2] = {group_ptr(a, L, gi, t, ob, 0, 0), group_ptr(a, L, gi, t, ob, 1, 0)};
      sum_parts<2, kSumRound>(a, gs, L.NG, tag, gu);
    } else {
      sum_parts<2, kSumRound>(a, rows, L.HB, tag, gu);
    }
    float g0 = gu[0].x, g1 = gu[0].y, u0 = gu[1].x, u1 = gu[1].y;
    hadamard128_wave(g0, g1);
    hadamard128_wave(u0, u1);
    float h0 = swiglu_bf16(g0 * lo(og), u0 * lo(ou));
    float h1 = swiglu_bf16(g1 * hi(og), u1 * hi(ou));
    h0 *= lo(idn);
    h1 *= hi(idn);
    hadamard128_wave(h0, h1);
    uint64_t* dst = a.w.down_xh + (int64_t)s * a.m + col;
    st_tag(dst, h0, tag);
    st_tag(dst + 1, h1, tag);
  }
}

// combine of output block ob over all rows (reference sum order, shared, residual); `score` is the
// rows' [rows, 8] scores (the block's plan table when the launch routes, else the caller's)
__device__ void combine_block(const LayerArgs& a, int ob, uint32_t tag, const float* score) {
  const int lane = cold_lane();
  const int col = ob * 128 + 2 * lane;
  for (int r = 0; r < a.rows; r++) {
    f32x2 y[kSlots];
    {
      uint64_t w[kSlots][2];
      int spins = 0;
      for (;;) {
#pragma unroll
        for (int j = 0; j < kSlots; j++) {
          const uint64_t* q = a.w.yslot + (int64_t)(r * kSlots + j) * a.h + col;
          w[j][0] = ld_tag(q);
          w[j][1] = ld_tag(q + 1);
        }
        bool ok = true;
#pragma unroll
        for (int j = 0; j < kSlots; j++) ok = ok & (int)has_tag(w[j][0], tag) & (int)has_tag(w[j][1], tag);
        if (__all(ok)) break;
        bool live = true;
        for (;;) {
          const uint64_t* q = a.w.yslot + (int64_t)(r * kSlots + lane % kSlots) * a.h + col;
          if (__all(has_tag(ld_tag(q), tag))) break;
          if (!keep_waiting<MOE_LAYER_WAIT>(a, spins)) {
            live = false;
            break;
          }
        }
        if (!live) break;
      }
#pragma unroll
      for (int j = 0; j < kSlots; j++) y[j] = f32x2{tag_value(w[j][0]), tag_value(w[j][1])};
    }
    float sc[8];
#pragma unroll
    for (int j = 0; j < 8; j++) sc[j] = score[r * 8 + j];
    float tot0 = y[0].x * sc[0] + 0.0f, tot1 = y[0].y * sc[0] + 0.0f;
#pragma unroll
    for (int j = 1; j < 8; j++) {
      tot0 = (y[j].x * sc[j] + 0.0f) + tot0;
      tot1 = (y[j].y * sc[j] + 0.0f) + tot1;
    }
    const float c0f = round_bf16(round_bf16(tot0) + y[8].x);
    const float c1f = round_bf16(round_bf16(tot1) + y[8].y);
    const int64_t o = (int64_t)r * a.h + col;
    const uint32_t res = *reinterpret_cast<const uint32_t*>(a.residual + o);
    const uint32_t packed2 = (uint32_t)f32_to_bf16(bf16_to_f32((uint16_t)(res & 0xFFFFu)) + c0f) |
                             ((uint32_t)f32_to_bf16(bf16_to_f32((uint16_t)(res >> 16)) + c1f) << 16);
    *reinterpret_cast<uint32_t*>(a.out + o) = packed2;
  }
}

// down finish of output block ob of unit ui: per-slot values, or the slot outputs for the combine
// (and, for the last unit, the combine of the block)
// The combine of output block ob for a one-row launch, by the last unit's down finish: `own`
// (slot `js`) is this unit's output, kept in registers (nothing else reads it), `res` the residual
// pair loaded earlier.  The other slots' words are normally complete; stale ones are waited for.
__device__ void combine_one_row(const LayerArgs& a, int col, int js, f32x2 own, uint32_t res, uint32_t tag,
                                const float* score) {
  const int lane = cold_lane();
  uint64_t w[kSlots][2];
#pragma unroll
  for (int j = 0; j < kSlots; j++) {
    const uint64_t* q = a.w.yslot + (int64_t)j * a.h + col;
    w[j][0] = ld_tag(q);
    w[j][1] = ld_tag(q + 1);
  }
  bool ok = true;
#pragma unroll
  for (int j = 0; j < kSlots; j++) ok = ok & (j == js || ((int)has_tag(w[j][0], tag) & (int)has_tag(w[j][1], tag)));
  int spins = 0;
  while (!__all(ok)) {
    bool live = true;
    for (;;) {
      const int j = lane % kSlots;
      const uint64_t* q = a.w.yslot + (int64_t)j * a.h + col;
      if (__all(j == js || has_tag(ld_tag(q), tag))) break;
      if (!keep_waiting<MOE_LAYER_WAIT>(a, spins)) {
        live = false;
        break;
      }
    }
#pragma unroll
    for (int j = 0; j < kSlots; j++) {
      const uint64_t* q = a.w.yslot + (int64_t)j * a.h + col;
      w[j][0] = ld_tag(q);
      w[j][1] = ld_tag(q + 1);
    }
    if (!live) break;
    ok = true;
#pragma unroll
    for (int j = 0; j < kSlots; j++) ok = ok & (j == js || ((int)has_tag(w[j][0], tag) & (int)has_tag(w[j][1], tag)));
  }
  f32x2 y[kSlots];
#pragma unroll
  for (int j = 0; j < kSlots; j++) y[j] = j == js ? own : f32x2{tag_value(w[j][0]), tag_value(w[j][1])};
  float tot0 = y[0].x * score[0] + 0.0f, tot1 = y[0].y * score[0] + 0.0f;
#pragma unroll
  for (int j = 1; j < 8; j++) {
    tot0 = (y[j].x * score[j] + 0.0f) + tot0;
    tot1 = (y[j].y * score[j] + 0.0f) + tot1;
  }
  const float c0f = round_bf16(round_bf16(tot0) + y[8].x);
  const float c1f = round_bf16(round_bf16(tot1) + y[8].y);
  const uint32_t packed2 = (uint32_t)f32_to_bf16(bf16_to_f32((uint16_t)(res & 0xFFFFu)) + c0f) |
                           ((uint32_t)f32_to_bf16(bf16_to_f32((uint16_t)(res >> 16)) + c1f) << 16);
  *reinterpret_cast<uint32_t*>(a.out + col) = packed2;
}

__device__ void down_finish(const LayerArgs& a, const UnitInfo& ui, int ob, bool last, uint32_t tag, const Items& L,
                            const float* score) {
  const int lane = cold_lane();
  const int col = ob * 128 + 2 * lane;
  const uint32_t osc = *reinterpret_cast<const uint32_t*>(a.out_scale[2] + (int64_t)ui.e * a.h + col);
  const float os0 = f16_to_f32((uint16_t)(osc & 0xFFFFu)), os1 = f16_to_f32((uint16_t)(osc >> 16));
  if (a.fin == LFIN_COMBINE && last && a.rows == 1 && ui.ntok == 1) {
    // The launch's last dependency chain ends here.  One row, one slot of this unit: its output
    // goes to the combine in registers (no store and read-back), and the residual is requested
    // before this block's down partials are waited for.
    const uint32_t res = *reinterpret_cast<const uint32_t*>(a.residual + col);
    const int js = min(max(ui.slot(0), 0), kSlots - 1);
    const uint64_t* rows[1] = {part_ptr(a, ui.slot(0), 2 * L.MB * L.HB + ob * L.MB)};
    f32x2 v[1];
    sum_parts<1, 16>(a, rows, L.MB, tag, v);
    float v0 = v[0].x, v1 = v[0].y;
    hadamard128_wave(v0, v1);
    combine_one_row(a, col, js, f32x2{round_bf16(v0 * os0), round_bf16(v1 * os1)}, res, tag, score);
    return;
  }
  for (int t = 0; t < ui.ntok; t++) {
    const int s = ui.slot(t);
    const uint64_t* rows[1] = {part_ptr(a, s, 2 * L.MB * L.HB + ob * L.MB)};
    f32x2 v[1];
    sum_parts<1, 16>(a, rows, L.MB, tag, v);
    float v0 = v[0].x, v1 = v[0].y;
    hadamard128_wave(v0, v1);
    if (a.fin == LFIN_VALUES) {
      const uint32_t packed2 = (uint32_t)f32_to_bf16(v0 * os0) | ((uint32_t)f32_to_bf16(v1 * os1) << 16);
      *reinterpret_cast<uint32_t*>(a.values + (int64_t)s * a.h + col) = packed2;
    } else {
      uint64_t* dst = a.w.yslot + (int64_t)s * a.h + col;
      st_tag(dst, round_bf16(v0 * os0), tag);
      st_tag(dst + 1, round_bf16(v1 * os1), tag);
    }
  }
  if (a.fin == LFIN_COMBINE && last) {
    release_stores();  // this wave's own slot outputs are read back by the combine
    combine_block(a, ob, tag, score);
  }
}

// Share k of SHARES of the code table (a power-of-two size) into LDS by one wave, in one batch:
// every load is issued (unconditionally, index clamped: a load under a branch is waited for
// before the next) before the first store.
template <int BYTES, int SHARES>
struct TableShare {
  static constexpr int n = BYTES / 16;
  static constexpr int per = ((n + SHARES - 1) / SHARES + 63) & ~63;
  static constexpr int kLoads = per / 64;
  u32x4 v[kLoads];
};
// The share's loads (issue) and its LDS stores (commit): every block walks the table from its own
// 1 KB offset, since all CUs reading the same lines at the same time would queue on the same L2
// channels
template <int BYTES, int SHARES>
__device__ __forceinline__ void copy_table_issue(TableShare<BYTES, SHARES>& t, const void* table, int k) {
  using T = TableShare<BYTES, SHARES>;
  const u32x4* src = reinterpret_cast<const u32x4*>(table);
  const int lane = lane_id();
  const int lo = k * T::per, hi = min(T::n, lo + T::per);
  const int rot = ((int)blockIdx.x * 97 * 64) & (T::n - 1);
#pragma unroll
  for (int j = 0; j < T::kLoads; j++) t.v[j] = src[(min(lo + 64 * j + lane, hi - 1) + rot) & (T::n - 1)];
}
template <int BYTES, int SHARES>
__device__ __forceinline__ void copy_table_commit(const TableShare<BYTES, SHARES>& t, uint8_t* lds, int k) {
  using T = TableShare<BYTES, SHARES>;
  u32x4* dst = reinterpret_cast<u32x4*>(lds);
  const int lane = lane_id();
  const int lo = k * T::per, hi = min(T::n, lo + T::per);
  const int rot = ((int)blockIdx.x * 97 * 64) & (T::n - 1);
#pragma unroll
  for (int j = 0; j < T::kLoads; j++) {
    const int i = lo + 64 * j + lane;
    if (i < hi) dst[(i + rot) & (T::n - 1)] = t.v[j];
  }
}

// ---------------------------------------------------------------- the kernel
// The layer shape of the GLM-5.3 experts.  A launch of that shape runs an instantiation with the
// shape known at compile time: the work list's divisions (item_at) are then by constants, and the
// reciprocals a runtime shape needs no longer occupy scalar registers across the part loop (where
// the compiler otherwise spills them and reloads them with v_readlane: ~100 fewer instructions
// per part).
constexpr int kGlmHidden = 6144, kGlmInter = 2048;
// NORM (one row): the launch first forms the layer's residual add + RMSNorm (a separate
// instantiation, so that the plain one keeps its start unchanged); GLM: the shape is kGlmHidden x kGlmInter
template <int NT, bool NORM, int KB, bool GLM>
__global__ __launch_bounds__(kLW * 64) void k4_layer_kernel(LayerArgs a) {
  constexpr bool kDPre = NT == 1;  // down inputs fetched ahead (registers allow it for one token)
  __shared__ __attribute__((aligned(16))) uint8_t tab[LTable<NT>::kBytes];
  __shared__ __attribute__((aligned(16))) _Float16 xa[kLW * xa_halves(NT)];
  __shared__ __attribute__((aligned(16))) float pst_all[NT == 1 ? kLW * 128 : 1];  // one token: partial rows
  __shared__ int32_t exit_last;

  const int wv = wave_id_uniform();
  _Float16* __restrict__ xw = xa + wv * xa_halves(NT);
  const int xcd = (int)(blockIdx.x % kXcds);
  int32_t* qc = a.w.queue + xcd * kQueueStride;
  const Items L = make_items(GLM ? kGlmHidden : a.h, GLM ? kGlmInter : a.m, a.route);
  const int pre = pre_items(L);
  // the launch's epoch (read once per block below) and its tag
  uint32_t epoch = 0, tag = 0;

  // A wave's first item is its index among the waves serving its sub-list (no atomic: thousands
  // of simultaneous claims on eight counters would serialise the start); the counter hands out the
  // items after those.
  const int xcd_waves = (((int)gridDim.x - xcd + kXcds - 1) / kXcds) * kLW;
  const int first_sub = ((int)blockIdx.x / kXcds) * kLW + wv;
  // A claim in two steps: the atomic is issued, its result is read later.  Reading it waits for
  // every earlier memory operation of the wave (loads and stores share one counter), so a claim
  // issued during an item is read only once the data it was issued behind is needed anyway.
  auto claim_issue = [&]() {
    int v = 0;
    if (lane_id() == 0) v = __hip_atomic_fetch_add(qc, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    return v;
  };
  auto claim_take = [&](int v) { return xcd_waves + __builtin_amdgcn_readfirstlane(v); };
  auto claim = [&]() { return claim_take(claim_issue()); };

  __shared__ PlanLds plan_t;
  __shared__ int32_t route_state;  // routing launches: 0 not started, 1 being computed, 2 ready
  bool have_plan = false;
  int units = 1;
  if (!a.route) {
    units = load_plan(a.w.plan, plan_t);
    have_plan = true;
  }
  const float* score = a.route ? plan_t.score : a.scores;
  // Unit 0 of a routing launch is the shared expert, known before routing: rows 0.., slots
  // 9 r + 8.  Its fields are formed where they are used (a unit record kept in a variable that the
  // lambdas share would live in private memory, and its loads would be flat loads, which wait for
  // every outstanding memory operation of the wave).
  auto unit_of = [&](int u) {
    if (u == 0 && a.route) {
      UnitInfo i;
      i.e = min(256, a.experts - 1);
      i.ntok = a.rows;
      i.rows = a.rows;
      uint32_t tok = 0, s0 = 0, s1 = 0;
      for (int t = 0; t < a.rows; t++) {
        tok |= (uint32_t)t << (3 * t);
        if (t < 4) s0 |= (uint32_t)(kSlots * t + 8) << (7 * t);
        else s1 |= (uint32_t)(kSlots * t + 8) << (7 * (t - 4));
      }
      i.tok = tok;
      i.sl0 = s0;
      i.sl1 = s1;
      return i;
    }
    return unit_info(plan_t, u, a.experts, a.rows);
  };
  // the item at sub-list position `sub`, if it is known without waiting (kind NONE otherwise); a
  // wave without the plan takes the block's table once it is complete in LDS, so a run of parts
  // goes on from the shared expert's parts into the routed ones without leaving its load pipeline
  auto resolve = [&](int sub, Item& it) {
    const int j = sub * kXcds + xcd;
    it = Item{IT_NONE, 0, 0, 0, 0};
    if (j < pre) {
      it = item_at(L, j, 1);
      return;
    }
    if (!have_plan &&
        __builtin_amdgcn_readfirstlane(__hip_atomic_load(&route_state, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) == 2) {
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
      units = min(max(__builtin_amdgcn_readfirstlane(plan_t.units), 1), kMaxUnits);
      have_plan = true;
    }
    if (have_plan && j < list_len(L, units)) it = item_at(L, j, units);
  };

  // A run of part items: pc / in hold the first item's quad 0 and input block on entry.  Each item
  // is staged, streams its quad 1 while quad 0 is decoded and the next part's quad 0 and input
  // block while quad 1 is decoded, then stores its partials.  A wave never waits while it holds
  // partials it has not stored (the only wait of the loop, a down part's staging, comes after the
  // previous part's stores), so the lowest unfinished item always makes progress.
  // Returns with `sub` at the first item that is not a part (or not yet known).
  u32x4 pc[4];
  InBlock<NT, kDPre> in;
  auto run_parts = [&](Item it, int& sub) {
    for (;;) {
      const UnitInfo ui = unit_of(it.u);
      __builtin_amdgcn_s_setprio(2);
      float scale[NT];
      stage_in<NT, kDPre>(a, ui, it, in, tag, xw, scale);
      // the last units' parts head the launch's final dependency chain (their gate finishes, their
      // down parts, the combine): they get issue priority over the other decoding waves
      if (have_plan && it.u >= units - MOE_LAYER_PRIO_UNITS)
        __builtin_amdgcn_s_setprio(1);
      else
        __builtin_amdgcn_s_setprio(0);
      u32x4 pn[4];
      load_quad<KB>(pn, quad_ptr<KB>(a, ui, it, 1));
      // the next item is claimed once this one can no longer wait (a claimed item is only started
      // by its claimer); the claim's round trip is hidden by quad 0
      const int claimed = claim_issue();
      f32x4 acc[4][2];
#pragma unroll
      for (int s4 = 0; s4 < 4; s4++)
#pragma unroll
        for (int hh = 0; hh < 2; hh++) acc[s4][hh] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      decode_quad<NT, KB>(pc, 0, ui.ntok, tab, xw, acc);
      const int nsub = claim_take(claimed);
      // A part whose sub-list has handed out more than kStraggle items since the part was claimed
      // (a sub-list serves ~32 blocks x 12 waves: about half that many claims in a part's first
      // quad) has fallen behind the waves around it, and finishes may be waiting for it: its
      // second quad runs at raised priority.
      if (nsub - sub > kStraggle) __builtin_amdgcn_s_setprio(2);
      Item nit;
      resolve(nsub, nit);
      // the next part's quad 0 and input block -- this part's again when the next item is not a
      // part (every load of the loop is unconditional: a load under a branch makes the compiler
      // wait for all outstanding memory operations before the next use)
      const bool more = is_part(nit);
      const Item pit = more ? nit : it;
      const UnitInfo pui = unit_of(pit.u);
      load_quad<KB>(pc, quad_ptr<KB>(a, pui, pit, 0));
      fetch_in<NT, kDPre>(a, pui, pit, in);
      decode_quad<NT, KB>(pn, 1, ui.ntok, tab, xw, acc);
      store_partials<NT>(a, ui, it, acc, tag, L, pst_all + (NT == 1 ? wv * 128 : 0), scale);
      sub = nsub;
      if (!more) return;
      it = nit;
    }
  };

  // The launch's epoch (every wave reads it: a router item stores tagged words before the table is
  // in LDS).
  epoch = (uint32_t)__builtin_amdgcn_readfirstlane(ld_coh_i(a.w.flags + LF_EPOCH));
  tag = epoch + 1u;
  // Start-up.  Routing is the launch's first dependency chain (router items -> logits -> top-8 ->
  // plan -> the routed experts' loads), the code table its first bulk copy.  A wave whose first
  // item is a router item issues that item's loads ahead of its table share and finishes the item
  // while the share is in flight; waves 1..kLW-1 then commit their shares and count them in
  // `tab_ready`; wave 0 copies no share and, when its first item is a router item, finishes it and
  // routes the block at once.  A wave waits for the whole table only when it is about to decode.
  // With the layer's norm folded in, router items read the normalised row, which exists only after
  // the block meets: that instantiation meets once after the norm and the table copy.
  __shared__ int32_t tab_ready;
  if (threadIdx.x == 0) {
    route_state = 0;
    tab_ready = 0;
  }
  __syncthreads();
  int sub = first_sub;
  Item first;
  resolve(sub, first);  // positions before the plan's need none
  const bool first_router = !NORM && first.kind == IT_ROUTER;
  RouterLoads rl;
  if (first_router) router_item_issue(a, first.a, L.S, rl);
  // The layer's residual add + RMSNorm (one row): waves 0..3 form the row's square sums exactly as
  // the norm kernel's four waves do, and after the block meets write h and the normalised row;
  // every block writes the same bits, so each block reads values its own stores put in its L2.
  // The norm's loads go out first, the table's next; the block meets once the row's sums are in,
  // then waves 0..3 store the rows while every wave writes its table share into LDS.
  if constexpr (NORM) {
    __shared__ float norm_red[4];
    rms_u32x4 nh[4], nw[4];
    float nss = 0.0f;
    if (wv < 4) nss = rms_row_sum<4>(a.norm_x, a.norm_res, a.norm_w, a.h / 2048, (int)threadIdx.x, nh, nw, nullptr);
    TableShare<LTable<NT>::kBytes, kLW> share;
    copy_table_issue(share, LTable<NT>::kF16 ? (const void*)a.tab16 : (const void*)a.tab8, wv);
    if (wv < 4) {
      nss = wave_sum(nss);
      if (lane_id() == 63) norm_red[wv] = nss;
    }
    __syncthreads();
    if (wv < 4) {
      const int K = a.h / 2048, t = (int)threadIdx.x;
#pragma unroll
      for (int k = 0; k < 4; k++)
        if (k < K) *reinterpret_cast<rms_u32x4*>(a.h_row + k * 2048 + t * 8) = nh[k];
      rms_row_store<4>(nh, nw, K, t, rms_inv(norm_red, a.h, a.eps), a.x_row);
    }
    copy_table_commit(share, tab, wv);
    __syncthreads();
  } else if (wv == 0) {
    // wave 0 copies no share: when its first item is a router item (the case for every block of a
    // routing launch at the GLM shape) it finishes the item and goes on to route the block at once
    if (first_router) {
      __builtin_amdgcn_s_setprio(3);
      router_item_finish(a, first.a, L.S, tag, rl);
      __builtin_amdgcn_s_setprio(0);
    }
  } else {
    TableShare<LTable<NT>::kBytes, kLW - 1> share;
    copy_table_issue(share, LTable<NT>::kF16 ? (const void*)a.tab16 : (const void*)a.tab8, wv - 1);
    if (first_router) {
      __builtin_amdgcn_s_setprio(3);
      router_item_finish(a, first.a, L.S, tag, rl);
      __builtin_amdgcn_s_setprio(0);
    }
    copy_table_commit(share, tab, wv - 1);
    // the share is in LDS (this wave's LDS stores complete in order) before it is counted
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    if (lane_id() == 0) __hip_atomic_fetch_add(&tab_ready, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  bool table_ok = NORM;
  // before a wave first decodes: every share of the table (waves 1..kLW-1) is in LDS
  auto wait_table = [&]() {
    if (table_ok) return;
    while (__builtin_amdgcn_readfirstlane(__hip_atomic_load(&tab_ready, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) <
           kLW - 1)
      __builtin_amdgcn_s_sleep(1);
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    table_ok = true;
  };
  // Router items first.  The block's first wave done with one routes at once, before it claims
  // anything: a wave that routes holds no claimed item and the block's other waves keep claiming,
  // so the router items it waits for are always taken.
  bool route_now = false;
  bool router_done = first_router;  // the first router item was finished during the table copy
  while (first.kind == IT_ROUTER) {
    if (!router_done) {
      __builtin_amdgcn_s_setprio(3);
      router_item(a, first.a, L.S, tag);
      __builtin_amdgcn_s_setprio(0);
    }
    router_done = false;
    if (!have_plan) {
      int old = 0;
      if (lane_id() == 0) {
        int expected = 0;
        __hip_atomic_compare_exchange_strong(&route_state, &expected, 1, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_WORKGROUP);
        old = expected;
      }
      route_now = __builtin_amdgcn_readfirstlane(old) == 0;
      if (route_now) break;
    }
    sub = claim();
    resolve(sub, first);
  }

  for (;;) {
    if (route_now || (!have_plan && sub * kXcds + xcd >= pre)) {
      // the block's plan table: the first wave to ask routes (route_now: it has already won the
      // right after its router items), a later one waits for it
      __builtin_amdgcn_s_setprio(3);
      int old = 0;
      if (!route_now && lane_id() == 0) {
        int expected = 0;
        __hip_atomic_compare_exchange_strong(&route_state, &expected, 1, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_WORKGROUP);
        old = expected;
      }
      old = __builtin_amdgcn_readfirstlane(old);
      if (old == 0) {
        route_block(a, L.S, tag, plan_t);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        if (lane_id() == 0) __hip_atomic_store(&route_state, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      } else {
        while (__hip_atomic_load(&route_state, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) != 2)
          __builtin_amdgcn_s_sleep(1);
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
      }
      units = min(max(__builtin_amdgcn_readfirstlane(plan_t.units), 1), kMaxUnits);
      have_plan = true;
      __builtin_amdgcn_s_setprio(0);
      if (route_now) {
        // the router item at `sub` is done: on to the next
        route_now = false;
        sub = claim();
        continue;
      }
    }
    const int j = sub * kXcds + xcd;
    const int U = have_plan ? units : 1;
    if (have_plan && j >= list_len(L, U)) break;
    const Item it = item_at(L, j, U);
    if (it.kind == IT_NONE) break;
    if (is_part(it)) {
      wait_table();
      const UnitInfo ui = unit_of(it.u);
      load_quad<KB>(pc, quad_ptr<KB>(a, ui, it, 0));
      fetch_in<NT, kDPre>(a, ui, it, in);
      // the run's first part waits for its operands here, so nothing is pending on entry: without
      // this the compiler merges the entry (input block just requested) into the loop's state and
      // waits for every outstanding operation at each part's staging
      __builtin_amdgcn_s_waitcnt(0);
      run_parts(it, sub);
      continue;
    }
    // items other than parts are short and latency-bound, and others wait for them: they run at
    // raised wave priority (the SIMD arbiter otherwise favours the older, decoding waves)
    __builtin_amdgcn_s_setprio(3);
    if (it.kind == IT_ROUTER) {
      router_item(a, it.a, L.S, tag);
    } else if (it.kind == IT_GF) {
      const int gi = it.u - (U - min(U, kLagG));
      gate_finish(a, unit_of(it.u), it.a, tag, L, L.NG > 0 ? gi : -1);
    } else if (it.kind == IT_GS) {
      group_sum(a, unit_of(it.u), it.u - (U - min(U, kLagG)), it.a, it.b, tag, L);
    } else if (it.kind == IT_DF) {
      down_finish(a, unit_of(it.u), it.a, it.u == U - 1, tag, L, score);
    }
    __builtin_amdgcn_s_setprio(0);
    sub = claim();
  }
  // the last block to leave reports a stalled wait, advances the epoch and resets the sub-list
  // counters
  const bool last = leave_launch(a, epoch, exit_last);
  if (last && threadIdx.x < kXcds) st_coh_i(a.w.queue + threadIdx.x * kQueueStride, 0);
  // a wave may end with its stores still in flight, and the next launch reads these words at its
  // start: they are acknowledged before the block ends
  if (last) release_stores();
}

// ---------------------------------------------------------------- host side
size_t layer_align(size_t v) { return (v + 255) & ~(size_t)255; }

LayerWs layer_carve(void* base, int h, int m) {
  LayerWs w{};
  size_t off = 0;
  char* p = static_cast<char*>(base);
  auto take = [&](size_t bytes) { char* r = p ? p + off : nullptr; off += layer_align(bytes); return r; };
  const int HB = h / 128, MB = m / 128;
  w.plan = reinterpret_cast<Plan*>(take(sizeof(Plan)));
  w.flags = reinterpret_cast<int32_t*>(take(LF_COUNT * 4));
  w.queue = reinterpret_cast<int32_t*>(take((size_t)kXcds * kQueueStride * 4));
  w.logit_part = reinterpret_cast<uint64_t*>(take((size_t)kMaxRows * 256 * (h / kRouterSlice + 1) * 8));
  w.partial = reinterpret_cast<uint64_t*>(take((size_t)kMaxUnits * 3 * HB * MB * 128 * 8));
  w.down_xh = reinterpret_cast<uint64_t*>(take((size_t)kMaxUnits * m * 8));
  w.yslot = reinterpret_cast<uint64_t*>(take((size_t)kMaxUnits * h * 8));
  w.gsum = reinterpret_cast<uint64_t*>(take((size_t)kLagG * kMaxRows * MB * 2 * kSumRound * 128 * 8));
  w.bytes = off;
  return w;
}

Plan* k4_layer_plan(void* layer_ws) { return layer_carve(layer_ws, 1024, 128).plan; }
int32_t* k4_layer_flags(void* layer_ws, int h, int m) { return layer_carve(layer_ws, h, m).flags; }

size_t k4_layer_workspace_bytes(int h, int m) {
  return layer_carve(nullptr, h > 0 ? h : 128, m > 0 ? m : 128).bytes;
}

// The fused block reads x and the side-vector rows 8 bytes at a time (one token) and residual,
// output and value rows 4 bytes at a time.
int k4_layer_check_alignment(const uint16_t* x, const uint16_t* residual, const uint16_t* const in_scale[3],
                             const uint16_t* const out_scale[3], const uint16_t* out, const uint16_t* values) {
  auto misaligned = [](const void* p, uintptr_t a) { return p != nullptr && ((uintptr_t)p & (a - 1)) != 0; };
  bool bad = misaligned(x, 8) || misaligned(residual, 4) || misaligned(out, 4) || misaligned(values, 4);
  for (int i = 0; i < 3; i++) bad = bad || misaligned(in_scale[i], 8) || misaligned(out_scale[i], 4);
  if (bad)
    return fail(MOE_EINVAL, "the K4 decode block needs x and side-vector rows 8-byte aligned and residual, "
                            "output and value rows 4-byte aligned");
  return MOE_OK;
}

int k4_layer_item_list(int h, int m, int units, int route, int32_t* items, int capacity) {
  if (!k4_layer_supported(h, m, route != 0) || units < 1 || units > kMaxUnits || capacity < 0)
    return fail(MOE_EINVAL, "no fused K4 item list for hidden %d, intermediate %d, %d units", h, m, units);
  const Items L = make_items(h, m, route != 0);
  const int n = list_len(L, units);
  if (items) {
    if (capacity < n) return fail(MOE_EINVAL, "the list has %d items (capacity %d)", n, capacity);
    for (int j = 0; j < n; j++) {
      // a launch resolves the positions before the plan's with one unit (it does not know the
      // count yet): they must not depend on it
      const Item it = j < pre_items(L) ? item_at(L, j, 1) : item_at(L, j, units);
      const Item full = item_at(L, j, units);
      if (it.kind != full.kind || it.u != full.u || it.a != full.a || it.b != full.b || it.c != full.c)
        return fail(MOE_EINVAL, "item %d depends on the unit count before the plan is known", j);
      int32_t* o = items + 5 * (int64_t)j;
      o[0] = it.kind;
      o[1] = it.u;
      o[2] = it.a;
      o[3] = it.b;
      o[4] = it.c;
    }
  }
  return n;
}

bool k4_layer_supported(int h, int m, bool route) {
  return h > 0 && m > 0 && h % (route ? kRouterSlice : 128) == 0 && m % 128 == 0 && h <= (route ? kMaxRouteHidden : 16384) &&
         m <= 16384;
}

// One launch of the fused block.  `workspace` is the layer region (zeroed once; the kernel leaves
// its counters clean and advances its epoch).
static int k4_layer_launch(LayerArgs a, void* workspace, hipStream_t s) {
  a.w = layer_carve(workspace, a.h, a.m);
  a.wait_polls = wait_polls();
  a.tab8 = codebook_device_table();
  a.tab16 = codebook_f16_device_table();
  if (!a.tab8 || !a.tab16) return fail(MOE_ENOTSUP, "code tables are not initialised on this device");
  // every sub-list (blockIdx mod kXcds) needs a block to serve it
  const int grid = device_cus() > kXcds ? device_cus() : kXcds;
  const bool glm = a.h == kGlmHidden && a.m == kGlmInter;
#define MOE_K4_LAUNCH(NT, NORM, KB)                                                                   \
  do {                                                                                                 \
    if (glm)                                                                                           \
      hipLaunchKernelGGL((k4_layer_kernel<NT, NORM, KB, true>), dim3(grid), dim3(kLW * 64), 0, s, a);  \
    else                                                                                               \
      hipLaunchKernelGGL((k4_layer_kernel<NT, NORM, KB, false>), dim3(grid), dim3(kLW * 64), 0, s, a); \
  } while (0)
  if (a.bits == 3) {
    if (a.norm_x) return fail(MOE_ENOTSUP, "the fused residual + RMSNorm is built for K4 experts only");
    if (a.rows <= 1)
      MOE_K4_LAUNCH(1, false, 3);
    else
      MOE_K4_LAUNCH(kMaxRows, false, 3);
  } else if (a.rows <= 1 && a.norm_x) {
    MOE_K4_LAUNCH(1, true, 4);
  } else if (a.rows <= 1) {
    MOE_K4_LAUNCH(1, false, 4);
  } else {
    MOE_K4_LAUNCH(kMaxRows, false, 4);
  }
#undef MOE_K4_LAUNCH
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail((int)e, "launch of the fused K4 block failed: %s", hipGetErrorString(e));
  return MOE_OK;
}

int k4_layer_run(const uint16_t* x, const uint16_t* residual, int rows, int route, const float* router_w,
                 const float* bias, uint32_t* ids, float* scores, const uint8_t* const packed[3],
                 const uint16_t* const in_scale[3], const uint16_t* const out_scale[3], int h, int m, int experts,
                 int combine, uint16_t* out, uint16_t* values, void* layer_ws, hipStream_t s, const LayerNorm* norm,
                 int bits) {
  if (bits != 3 && bits != 4) return fail(MOE_EINVAL, "the fused block decodes K3 and K4 experts (got k=%d)", bits);
  if (!k4_layer_supported(h, m, route != 0))
    return fail(MOE_ENOTSUP, "the fused K4 block needs hidden a multiple of %d%s and intermediate a multiple of 128 "
                "(got %d, %d)", route ? kRouterSlice : 128, route ? " up to 8192 (fused router)" : "", h, m);
  if (rows < 1 || rows > kMaxRows) return fail(MOE_EINVAL, "the fused K4 block takes 1..%d rows (got %d)", kMaxRows, rows);
  if (int rc = k4_layer_check_alignment(x, residual, in_scale, out_scale, out, values)) return rc;
  LayerArgs a{};
  a.x = x;
  a.residual = residual;
  a.rows = rows;
  a.bits = bits;
  a.route = route;
  a.router_w = router_w;
  a.bias = bias;
  a.ids = ids;
  a.scores = scores;
  for (int i = 0; i < 3; i++) {
    a.packed[i] = packed[i];
    a.in_scale[i] = in_scale[i];
    a.out_scale[i] = out_scale[i];
  }
  a.h = h;
  a.m = m;
  a.experts = experts;
  a.fin = combine ? LFIN_COMBINE : LFIN_VALUES;
  a.out = out;
  a.values = values;
  if (norm) {
    // x and residual are then the launch's outputs: the normalised row and h
    if (rows != 1 || !route || !norm->x || !norm->w || h % 2048 || h > 8192)
      return fail(MOE_EINVAL, "the fused residual + RMSNorm takes one routed row of width a multiple of 2048 up to 8192");
    a.norm_x = norm->x;
    a.norm_res = norm->residual;
    a.norm_w = norm->w;
    a.eps = norm->eps;
    a.h_row = const_cast<uint16_t*>(residual);
    a.x_row = const_cast<uint16_t*>(x);
  }
  return k4_layer_launch(a, layer_ws, s);
}

}  // namespace moe
