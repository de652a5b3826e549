/*
 * moe_mi355x.h -- C ABI of the MI355X (gfx950) MoE expert path for GLM-5.3-style layers.
 *
 * One shared library, libmoe_mi355x.so.  Every pointer argument is a DEVICE pointer owned by
 * the caller (for example a PyTorch tensor's data_ptr()); every launch is enqueued on the
 * caller's `stream` with no host synchronisation.  Scratch memory is passed in as an explicit,
 * caller-owned workspace whose size is given by moe_workspace_bytes(); it must be zero-filled
 * before its first use, and every successful call leaves it ready for the next call.  Calls
 * that share one workspace must not overlap.
 *
 * Return codes: 0 ok; negative = invalid argument (MOE_E*), message in moe_last_error();
 * positive = hipError_t of the failing HIP call.  No C++ exception crosses this boundary.
 *
 * Data types: bf16 and f16 are passed as uint16_t bit patterns; fp32 as float.
 * Shapes: hidden h, intermediate m, experts E (routed + shared, the shared expert last).
 * Alignment: activation rows (x) and per-expert side-vector rows are read 8 bytes at a time and
 * residual / output rows 4 bytes at a time; the K4 decode entries reject misaligned pointers.
 * Expert ids: every entry that takes caller ids (the decode entries moe_k4_mlp, moe_k4_mlp_finish,
 * moe_k4_expert_linear, moe_mxfp4_mlp, moe_mxfp4_mlp_finish and the grouped entries) clamps an id
 * outside [0, E), read as a signed 32-bit integer, to the nearest valid expert (a negative id to 0,
 * one >= E to E - 1) instead of failing: checking ids on the host would synchronise the stream.  Callers validate ids beforehand (the routed entries produce valid ids
 * themselves).  moe_segment_table alone skips such ids (see there).
 *
 * Each entry point names the reference interface it replaces (paths relative to the
 * reference repository root).
 */
#ifndef MOE_MI355X_H
#define MOE_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* moe_stream_t; /* hipStream_t */

enum {
  MOE_OK = 0,
  MOE_EINVAL = -1,     /* bad shape / format / argument */
  MOE_ENOTSUP = -2,    /* valid request outside what this build supports */
  MOE_EWORKSPACE = -3, /* workspace missing or too small */
};

/* Library version string and the last error message of the calling thread. */
const char* moe_version(void);
const char* moe_last_error(void);

/* Per-device setup (codebook table).  Called implicitly by every entry point; exposed so a
 * caller can pay the cost up front.  Acts on the current HIP device. */
int moe_init(void);

/* ---------------------------------------------------------------- fused decode blocks: status
 *
 * The one-launch decode blocks (moe_k4_moe_decode, moe_k4_layer_decode, moe_k4_mlp,
 * moe_k4_mlp_finish, and moe_mxfp4_moe_decode / its _noalloc twin for one row) run one persistent
 * block per compute unit whose waves hand results to each other through the workspace.  They need
 * all of their blocks resident together: run them with no other kernel occupying the device's
 * compute units (calls on several streams at once may stall each other).  Every cross-wave wait is
 * bounded; a launch in which a wait ran out still completes, but its outputs are unreliable, and
 * it is counted in the workspace.  The reference reports failure by raising
 * (exlr8/experts.py:158-159, exlr8/fast_decode.py:110-117); these counts are how a caller learns
 * of this failure without a host synchronisation per call. */
enum {
  MOE_STATUS_K4 = 0,             /* workspace of moe_workspace_bytes(hidden, intermediate) */
  MOE_STATUS_MXFP4 = 1,          /* workspace of moe_mxfp4_workspace_bytes(hidden, intermediate) */
  MOE_STATUS_MXFP4_NOALLOC = 2,  /* the current device's scratch of moe_mxfp4_moe_decode_noalloc */
};

/* Number of fused-block launches on `workspace` (of the given kind) in which a bounded wait ran out,
 * since the workspace was zeroed or the last call; resets the count.  Synchronises `stream` (the
 * stream the workspace's launches use).  No counterpart in the reference: it replaces the
 * reference's raised errors for this failure (see above). */
int moe_decode_status(const void* workspace, int kind, int hidden, int intermediate, int32_t* stalled,
                      moe_stream_t stream);

/* Bound of the fused blocks' cross-wave waits in polls of their longest pause (0 = the default,
 * about 50 ms); applies to launches made after the call, on every device.  No counterpart in the
 * reference: for tests that make waits give up on purpose and check moe_decode_status. */
int moe_set_wait_bound(int polls);

/* The fused K4 block's work list for a layer (hidden, intermediate) with `units` distinct experts
 * (1..72; route != 0: the launch routes, unit 0 = the shared expert), in list order: 5 int32 per
 * item (kind, unit, a, b, c) with kind 0 gate/up part (a = output block, b = projection 0 gate /
 * 1 up, c = input block), 1 down part (a = output block, c = input block), 2 router item (a = item),
 * 3 gate finish (a = column block), 4 down finish (a = output block; the last unit's also
 * combine), 6 group sum (a = column block, b = group).  Items are dealt round-robin over 8
 * sub-lists, one per XCD; an item waits only for items before it in this list, which is what
 * keeps the persistent launch from deadlocking.  Returns the item count (items may be NULL to ask
 * for it).  Host-only, no device work.  No counterpart in the reference: it exposes the schedule
 * for checks of that ordering. */
int moe_k4_item_list(int hidden, int intermediate, int units, int route, int32_t* items, int capacity);

/* Copy the 65536-entry E4M3 code table (one byte per 16-bit trellis state) to `dst`.
 * Replaces: exlr8/trellis.py:43-50 mcg_codebook (as E4M3 codes; exlr8/static_cache.py:11-26). */
int moe_codebook_e4m3(uint8_t* dst, moe_stream_t stream);

/* ---------------------------------------------------------------- router */

/* Sigmoid scores, bias-corrected top-8 (ties to the lower id), renormalised x2.5; slot 8 = 256.
 * logits [rows,256] f32, bias [256] f32 -> indices [rows,9] u32, scores [rows,8] f32.
 * Replaces: exlr8/fast_router.py:17-24 route (exlr8/metal/fast_router.metal:1-42);
 *           exlr8/model.py:111-132 route_experts + 407-408 shared-expert append. */
int moe_route_f32(const float* logits, const float* bias, int rows, uint32_t* indices, float* scores,
                  moe_stream_t stream);

/* Router GEMV: logits [rows,experts] = f32(x [rows,hidden] bf16) @ w [experts,hidden]^T.
 * Replaces: the gate call gate(x.astype(f32)) of exlr8/fast_router.py:34 / exlr8/model.py:406
 *           (DenseLinear format 6 with fp32 weight, exlr8/dense.py:158-159, exlr8/model.py:367-370). */
int moe_router_logits(const uint16_t* x, const float* w, int rows, int hidden, int experts, float* logits,
                      moe_stream_t stream);

/* ---------------------------------------------------------------- K4 trellis */

/* Decode expert `expert` of a packed trellis tensor to inner weights [in,out] as fp16 bits.
 * packed_bytes is the size of the whole tensor (all experts); k is 2, 3 or 4.
 * Replaces: exlr8/trellis.py:199-214 dequantize_trellis (inner part; exlr8/metal/decode.metal). */
int moe_trellis_decode_f16(const void* packed, int64_t packed_bytes, int k, int in_features, int out_features,
                           int side, int64_t expert, uint16_t* inner, moe_stream_t stream);

/* Selected-expert trellis linear: y[slot] = bf16(out_scale[e] * H(H(x_row * in_scale[e]) @ inner_e)).
 * ids [rows, slots] u32 (slots <= 9, rows*slots <= 72 per call); x [rows, in] bf16, or
 * [rows*slots, in] when x_per_slot != 0; in_scale [E,in], out_scale [E,out] f16; y [rows*slots,out] bf16.
 * Replaces: exlr8/trellis.py:172-196 expert_linear; exlr8/fast_decode.py:153-165 fast_expert_linear. */
int moe_k4_expert_linear(const uint16_t* x, int x_per_slot, const uint32_t* ids, int rows, int slots,
                         const void* packed, int64_t packed_bytes, const uint16_t* in_scale,
                         const uint16_t* out_scale, int in_features, int out_features, int side, uint16_t* y,
                         void* workspace, size_t workspace_bytes, moe_stream_t stream);

/* Typed SwiGLU of two bf16 arrays: out[i] = bf16(bf16(g * bf16(sigmoid(g))) * u) with g = gate[i],
 * u = up[i]; n elements, all three arrays 16-byte aligned (out may alias gate or up).
 * Replaces: the swiglu(gate, up) step between the expert linears of exlr8/experts.py:176-188
 *           (mlx_lm.models.activations.swiglu; typed as exlr8/metal/fast_decode_common.metal:40-49). */
int moe_swiglu_bf16(const uint16_t* gate, const uint16_t* up, int64_t n, uint16_t* out, moe_stream_t stream);

/* Expert MLP over selected experts: values [rows, slots, h] bf16 (gate/up side 1, down side 2,
 * typed SwiGLU, A.5 cast points).  Arguments as moe_k4_expert_linear; scale pairs per projection.
 * Replaces: exlr8/experts.py:150-188 ExpertLayer.__call__ (resident K4);
 *           exlr8/fast_decode.py:208-221 fast_expert_mlp. */
int moe_k4_mlp(const uint16_t* x, const uint32_t* ids, int rows, int slots, const void* packed_gate,
               const void* packed_up, const void* packed_down, int64_t packed_bytes, const uint16_t* in_gate,
               const uint16_t* out_gate, const uint16_t* in_up, const uint16_t* out_up, const uint16_t* in_down,
               const uint16_t* out_down, int hidden, int intermediate, uint16_t* values, void* workspace,
               size_t workspace_bytes, moe_stream_t stream);

/* Expert MLP plus weighted combine: out = bf16(residual + bf16(bf16(sum_i values_i*scores_i) + values_8)).
 * ids [rows,9] (slot 8 = shared expert), scores [rows,8] f32, residual/out [rows,h] bf16.
 * Replaces: exlr8/fast_decode.py:224-244 compiled_expert_mlp_finish (exlr8/metal/fast_decode_finish_fused.metal)
 *           and the combine of exlr8/model.py:415-418. */
int moe_k4_mlp_finish(const uint16_t* x, const uint32_t* ids, const float* scores, const uint16_t* residual, int rows,
                      const void* packed_gate, const void* packed_up, const void* packed_down, int64_t packed_bytes,
                      const uint16_t* in_gate, const uint16_t* out_gate, const uint16_t* in_up,
                      const uint16_t* out_up, const uint16_t* in_down, const uint16_t* out_down, int hidden,
                      int intermediate, uint16_t* out, void* workspace, size_t workspace_bytes, moe_stream_t stream);

/* Whole routed MoE block for decode batches: router GEMV, route, expert MLP and combine.
 * x/residual/out [rows,h] bf16 (rows <= 8 per call), router_w [256,h] f32, bias [256] f32;
 * indices/scores (optional, may be NULL) receive the routing [rows,9] u32 / [rows,8] f32.
 * Replaces: exlr8/fast_router.py:27-37 compiled_finish(...).call(x, residual). */
int moe_k4_moe_decode(const uint16_t* x, const uint16_t* residual, int rows, const float* router_w,
                      const float* bias, const void* packed_gate, const void* packed_up, const void* packed_down,
                      int64_t packed_bytes, const uint16_t* in_gate, const uint16_t* out_gate,
                      const uint16_t* in_up, const uint16_t* out_up, const uint16_t* in_down,
                      const uint16_t* out_down, int hidden, int intermediate, uint16_t* out, uint32_t* indices,
                      float* scores, void* workspace, size_t workspace_bytes, moe_stream_t stream);

/* The three decode entries above for K-bit trellis experts, k = 3 or 4 (k = 4 is the K4 entry
 * itself): the same fused block, arguments and workspace, with packed_bytes a multiple of
 * hidden * intermediate * k / 8.  A K3 tile is 24 words; each lane reads 12 B of it and takes its 32
 * codewords as the 16-bit windows that end every 3 bits of its stream (one funnel shift each).
 * K2 experts take the grouped entries (moe_trellis_grouped_mlp) at every row count.
 * Replaces: exlr8/fast_decode.py:208-221 fast_expert_mlp and :224-244 compiled_expert_mlp_finish with
 *           k = 3 (the multi-token-prediction layer's experts, exlr8/experts.py:86,170-173; the
 *           generic window of exlr8/metal/fast_decode_linear.metal:77-90), and
 *           exlr8/fast_router.py:27-37 compiled_finish for those experts. */
int moe_trellis_mlp(int k, const uint16_t* x, const uint32_t* ids, int rows, int slots, const void* packed_gate,
                    const void* packed_up, const void* packed_down, int64_t packed_bytes, const uint16_t* in_gate,
                    const uint16_t* out_gate, const uint16_t* in_up, const uint16_t* out_up, const uint16_t* in_down,
                    const uint16_t* out_down, int hidden, int intermediate, uint16_t* values, void* workspace,
                    size_t workspace_bytes, moe_stream_t stream);
int moe_trellis_mlp_finish(int k, const uint16_t* x, const uint32_t* ids, const float* scores,
                           const uint16_t* residual, int rows, const void* packed_gate, const void* packed_up,
                           const void* packed_down, int64_t packed_bytes, const uint16_t* in_gate,
                           const uint16_t* out_gate, const uint16_t* in_up, const uint16_t* out_up,
                           const uint16_t* in_down, const uint16_t* out_down, int hidden, int intermediate,
                           uint16_t* out, void* workspace, size_t workspace_bytes, moe_stream_t stream);
int moe_trellis_moe_decode(int k, const uint16_t* x, const uint16_t* residual, int rows, const float* router_w,
                           const float* bias, const void* packed_gate, const void* packed_up, const void* packed_down,
                           int64_t packed_bytes, const uint16_t* in_gate, const uint16_t* out_gate,
                           const uint16_t* in_up, const uint16_t* out_up, const uint16_t* in_down,
                           const uint16_t* out_down, int hidden, int intermediate, uint16_t* out, uint32_t* indices,
                           float* scores, void* workspace, size_t workspace_bytes, moe_stream_t stream);

/* Residual add + RMSNorm of decode rows: h = T(x + residual) (residual may be NULL: h = x),
 * out = T(w * T(h * rsqrt(mean(h^2) + eps))), T = bf16, x/residual/h_out/out [rows, n], w [n];
 * h_out may be NULL.  n a multiple of 2048 up to 8192.
 * Replaces: exlr8/fast_norm.py:20-28 residual_rms_pair (exlr8/metal/residual_rms.metal), and
 * exlr8/model.py:382-383 (h = x + r; mx.fast.rms_norm(h, post_norm, eps)). */
int moe_residual_rmsnorm(const uint16_t* x, const uint16_t* residual, const uint16_t* weight, int rows, int n,
                         float eps, uint16_t* h_out, uint16_t* out, moe_stream_t stream);

/* One decode layer's MoE half with its input norm: h = T(x + attn) (attn may be NULL: h = x),
 * xn = RMSNorm(h) (norm_w [h] bf16, eps), then the routed MoE block on xn with residual h:
 * out = T(h + r).  Shapes and side vectors as moe_k4_moe_decode; hidden a multiple of 2048 <= 8192.
 * One row: a single launch (the norm runs at the start of the fused block, same bits as
 * moe_residual_rmsnorm followed by moe_k4_moe_decode); more rows: the norm kernel, then the block.
 * Replaces: exlr8/model.py:382-418 (h = x + r; x = rms_norm(h, post_norm); MoE branch), the
 * layer body of a stack with no attention output. */
int moe_k4_layer_decode(const uint16_t* x, const uint16_t* attn, const uint16_t* norm_w, float eps, int rows,
                        const float* router_w, const float* bias, const void* packed_gate, const void* packed_up,
                        const void* packed_down, int64_t packed_bytes, const uint16_t* in_gate,
                        const uint16_t* out_gate, const uint16_t* in_up, const uint16_t* out_up,
                        const uint16_t* in_down, const uint16_t* out_down, int hidden, int intermediate,
                        uint16_t* out, uint32_t* indices, float* scores, void* workspace, size_t workspace_bytes,
                        moe_stream_t stream);

/* ---------------------------------------------------------------- joined MXFP4 */

/* Resident joined-MXFP4 experts: gate_up codes [E, 2m, h/2] (e2m1, low nibble = even k) with e8m0
 * scales [E, 2m, h/32]; down codes [E, h, m/2] + scales [E, h, m/32]; unit [h] fp16 (+-1);
 * out_gate/out_up/in_down [E, m], out_down [E, h] fp16.  This build: h = 6144, m = 2048.
 * values [rows*slots, h] bf16 (slots <= 9, rows*slots <= 72).
 * Replaces: exlr8/joined_mxfp4.py:143-147 JoinedMXFP4.slots (_inner, exlr8/joined_mxfp4.py:90-134). */
int moe_mxfp4_mlp(const uint16_t* x, const uint32_t* ids, int rows, int slots, const uint8_t* gate_up_codes,
                  const uint8_t* gate_up_scales, const uint8_t* down_codes, const uint8_t* down_scales,
                  int64_t experts, const uint16_t* unit, const uint16_t* out_gate, const uint16_t* out_up,
                  const uint16_t* in_down, const uint16_t* out_down, int hidden, int intermediate, uint16_t* values,
                  void* workspace, size_t workspace_bytes, moe_stream_t stream);

/* Joined-MXFP4 MLP plus the weighted combine with the shared expert and residual (rows <= 8).
 * Replaces: exlr8/joined_mxfp4.py:148-163 JoinedMXFP4.finish (exlr8/metal/joined_finish_sorted.metal,
 *           exlr8/metal/fast_decode_finish_fused.metal). */
int moe_mxfp4_mlp_finish(const uint16_t* x, const uint32_t* ids, const float* scores, const uint16_t* residual,
                         int rows, const uint8_t* gate_up_codes, const uint8_t* gate_up_scales,
                         const uint8_t* down_codes, const uint8_t* down_scales, int64_t experts,
                         const uint16_t* unit, const uint16_t* out_gate, const uint16_t* out_up,
                         const uint16_t* in_down, const uint16_t* out_down, int hidden, int intermediate,
                         uint16_t* out, void* workspace, size_t workspace_bytes, moe_stream_t stream);

/* Router GEMV + route (as moe_k4_moe_decode) + joined-MXFP4 MLP + combine for 1..8 decode rows in
 * one call; indices [rows, 9] and scores [rows, 8] may be NULL (kept in the workspace).  One row
 * runs as a single persistent launch (router, both projections of the nine slots and the combine;
 * one block per compute unit, all resident together); 2..8 rows as the router kernel and two GEMV
 * launches.  Given the same ids and scores both produce the same output bits.
 * Replaces: exlr8/fast_router.py:27-37 compiled_finish with the joined-MXFP4 experts
 *           (exlr8/joined_mxfp4.py:148-163 JoinedMXFP4.finish; exlr8/model.py:406-418). */
int moe_mxfp4_moe_decode(const uint16_t* x, const uint16_t* residual, int rows, const float* router_w,
                         const float* bias, const uint8_t* gate_up_codes, const uint8_t* gate_up_scales,
                         const uint8_t* down_codes, const uint8_t* down_scales, int64_t experts,
                         const uint16_t* unit, const uint16_t* out_gate, const uint16_t* out_up,
                         const uint16_t* in_down, const uint16_t* out_down, int hidden, int intermediate,
                         uint16_t* out, uint32_t* indices, float* scores, void* workspace, size_t workspace_bytes,
                         moe_stream_t stream);

/* Workspace bytes for the three MXFP4 decode entry points above. */
size_t moe_mxfp4_workspace_bytes(int hidden, int intermediate);

/* moe_mxfp4_moe_decode with no workspace argument and no allocation of any kind: the workspace is
 * the library's fixed per-GPU scratch array (4 MiB, held by each GPU the library runs on until the
 * process ends; its address is resolved on the first call on a device, so call moe_init() and this
 * entry once before capturing it in a graph).  For 2..8 rows its counters are cleared by a fill
 * kernel at the start of every call; one row needs no clearing (the single-launch block tags its
 * words per launch and leaves its counters at zero).  Shapes whose workspace exceeds the scratch are rejected with MOE_ENOTSUP.  Every
 * call on one GPU shares that GPU's scratch: calls that overlap on one GPU (several streams or
 * threads) race.
 * No counterpart in the reference: for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc). */
int moe_mxfp4_moe_decode_noalloc(const uint16_t* x, const uint16_t* residual, int rows, const float* router_w,
                                 const float* bias, const uint8_t* gate_up_codes, const uint8_t* gate_up_scales,
                                 const uint8_t* down_codes, const uint8_t* down_scales, int64_t experts,
                                 const uint16_t* unit, const uint16_t* out_gate, const uint16_t* out_up,
                                 const uint16_t* in_down, const uint16_t* out_down, int hidden, int intermediate,
                                 uint16_t* out, uint32_t* indices, float* scores, moe_stream_t stream);

/* ---------------------------------------------------------------- profiling */

/* Arm HIP events (hipEvent_t handles, NULL entries skipped) for the next K4 layer call made by
 * the calling thread: events[0] before the router, [1] before the gate/up GEMV, [2] before the
 * down GEMV, [3] after the down GEMV.  Used by bench.py to time each kernel on the stream it
 * runs on.  No counterpart in the reference (its benchmarks time whole model steps). */
int moe_profile_events(void** events, int count);

/* ---------------------------------------------------------------- prefill (sorted work order) */

/* Sorted work order of flat expert ids [n] (values < experts <= 1024): order [n] (sorted position
 * -> flat index, stable within an expert), counts/starts [experts], and the block table
 * table [3][capacity] = (expert, first sorted position, length <= block_rows), *num_blocks rows used;
 * capacity >= n / block_rows + experts.  Ids outside [0, experts) are skipped (no position).
 * Replaces: exlr8/fast_prefill.py:19-46 _segment_table / _plan (argsort + counts + block table). */
int moe_segment_table(const uint32_t* ids, int n, int experts, int block_rows, int32_t* order, int32_t* counts,
                      int32_t* starts, int32_t* table, int capacity, int32_t* num_blocks, moe_stream_t stream);

/* Model combine of per-slot expert values [rows, 9, hidden] bf16 (slot 8 = shared expert):
 * out[t] = T(T(sum_{i<8} values[t,i] * scores[t,i]) + values[t,8]) + residual[t] cast to bf16,
 * the routed sum accumulated in slot order in fp32.  16-byte aligned buffers; hidden % 8 == 0.
 * Replaces: exlr8/model.py:415-418 (the caller-side combine after ExpertLayer.__call__). */
int moe_combine_values(const uint16_t* values, const float* scores, const uint16_t* residual, int rows, int hidden,
                       uint16_t* out, moe_stream_t stream);

/* Prefill chunk through the joined-MXFP4 experts: router GEMV + route for `rows` rows, sorted
 * work order, grouped gate_up GEMM + gate finish, grouped down GEMM + value finish, weighted
 * combine with the shared expert and the residual.  Weights/side vectors as moe_mxfp4_mlp
 * (hidden a multiple of 1024, intermediate of 128); indices/scores optional outputs.
 * Workspace: moe_mxfp4_prefill_workspace_bytes(rows, hidden, intermediate, experts) (no zeroing).
 * Exact window: the grouped GEMMs widen the e2m1 weights to fp16 with their block scale, which is
 * exact only for e8m0 scale bytes 114..140 (the same holds for moe_mxfp4_grouped_mlp).  A caller
 * whose weights hold any scale outside that window must use the decode entries (moe_mxfp4_moe_decode,
 * moe_mxfp4_mlp: exact for every scale) in chunks of <= 8 rows; the Python layer checks the window
 * once per layer and does so.
 * Replaces: exlr8/joined_mxfp4.py:90-134,148-163 (JoinedMXFP4._inner with gather_qmm sorted RHS,
 * finish) for prefill rows, with the router of exlr8/model.py:111-132. */
int moe_mxfp4_prefill(const uint16_t* x, const uint16_t* residual, int rows, const float* router_w,
                      const float* bias, const uint8_t* gate_up_codes, const uint8_t* gate_up_scales,
                      const uint8_t* down_codes, const uint8_t* down_scales, int64_t experts, const uint16_t* unit,
                      const uint16_t* out_gate, const uint16_t* out_up, const uint16_t* in_down,
                      const uint16_t* out_down, int hidden, int intermediate, uint16_t* out, uint32_t* indices,
                      float* scores, void* workspace, size_t workspace_bytes, moe_stream_t stream);
size_t moe_mxfp4_prefill_workspace_bytes(int rows, int hidden, int intermediate, int64_t experts);

/* Sorted grouped joined-MXFP4 expert MLP for many rows: per-slot values [rows*slots, h] bf16 of
 * ids [rows, slots] (x [rows, h] bf16 shared by a row's slots) through the same segment table,
 * activation terms and MX-MFMA grouped GEMMs as moe_mxfp4_prefill, with no router and no combine.
 * An id outside [0, experts) is clamped to the nearest valid expert, as in the decode entries.
 * Weights/side vectors as moe_mxfp4_mlp; workspace: moe_mxfp4_grouped_mlp_workspace_bytes (no zeroing).
 * Replaces: exlr8/joined_mxfp4.py:98-134 _inner on the sorted-RHS gather_qmm branch (grouped, >= 1028
 * slots in the reference) and exlr8/joined_mxfp4.py:143-147 JoinedMXFP4.slots for prefill rows. */
int moe_mxfp4_grouped_mlp(const uint16_t* x, const uint32_t* ids, int rows, int slots, const uint8_t* gate_up_codes,
                          const uint8_t* gate_up_scales, const uint8_t* down_codes, const uint8_t* down_scales,
                          int64_t experts, const uint16_t* unit, const uint16_t* out_gate, const uint16_t* out_up,
                          const uint16_t* in_down, const uint16_t* out_down, int hidden, int intermediate,
                          uint16_t* values, void* workspace, size_t workspace_bytes, moe_stream_t stream);
size_t moe_mxfp4_grouped_mlp_workspace_bytes(int rows, int slots, int hidden, int intermediate, int64_t experts);

/* Grouped K4 expert MLP over many rows (prefill): values[slot] = T(out_down[e] * H(H(h) @ down_e))
 * with h = H(swiglu_T(gate, up) * in_down[e]), gate/up = out_scale * H(H(x * in_scale[e]) @ inner_e),
 * for ids [rows, slots] (flat ids < experts; x [rows, hidden] bf16 shared by a row's slots).
 * Slots are sorted by expert into blocks of <= 64 rows; every expert's weights are streamed once
 * per block and 256-column group.  values [rows*slots, hidden] bf16 in slot order; side vectors
 * and packed layouts as moe_k4_mlp; hidden and intermediate multiples of 128.
 * Workspace: moe_k4_grouped_mlp_workspace_bytes(rows, slots, hidden, intermediate, experts).
 * Replaces: exlr8/fast_prefill.py:188-211 grouped_expert_mlp (sorted block-table trellis GEMMs). */
int moe_k4_grouped_mlp(const uint16_t* x, const uint32_t* ids, int rows, int slots, const void* packed_gate,
                       const void* packed_up, const void* packed_down, int64_t packed_bytes, const uint16_t* in_gate,
                       const uint16_t* out_gate, const uint16_t* in_up, const uint16_t* out_up,
                       const uint16_t* in_down, const uint16_t* out_down, int hidden, int intermediate,
                       uint16_t* values, void* workspace, size_t workspace_bytes, moe_stream_t stream);
size_t moe_k4_grouped_mlp_workspace_bytes(int rows, int slots, int hidden, int intermediate, int64_t experts);

/* moe_k4_grouped_mlp for trellis width k = 2, 3 or 4 (packed_bytes / (hidden*intermediate*k/8)
 * experts; same workspace).  K2/K3 tiles are read through the generic circular window; this is
 * the expert MLP of K3 layers (the multi-token-prediction layer) at every row count.
 * Replaces: exlr8/fast_prefill.py:188-211 and exlr8/fast_decode.py:208-221 for k != 4
 * (exlr8/metal/trellis.metal:25-40 window extraction). */
int moe_trellis_grouped_mlp(int k, const uint16_t* x, const uint32_t* ids, int rows, int slots,
                            const void* packed_gate, const void* packed_up, const void* packed_down,
                            int64_t packed_bytes, const uint16_t* in_gate, const uint16_t* out_gate,
                            const uint16_t* in_up, const uint16_t* out_up, const uint16_t* in_down,
                            const uint16_t* out_down, int hidden, int intermediate, uint16_t* values, void* workspace,
                            size_t workspace_bytes, moe_stream_t stream);

/* One trellis projection y[slot] = T(out_scale[e] * H(H(x * in_scale[e]) @ inner_e)) for
 * ids [rows, slots] at width k = 2, 3 or 4, over the grouped sorted-expert kernel: x is
 * [rows, in] (a token row shared by its slots, x_per_slot = 0) or [rows*slots, in]; y
 * [rows*slots, out] bf16.  Side vectors [E, in] / [E, out] fp16; side 1 (gate/up) or 2 (down)
 * storage order.  An id outside [0, experts) is clamped to the nearest valid expert.
 * Workspace: moe_trellis_grouped_linear_workspace_bytes(rows, slots, in, out, experts).
 * Replaces: exlr8/trellis.py:172-196 expert_linear (and trellis.metal's generic window) for k != 4. */
int moe_trellis_grouped_linear(int k, const uint16_t* x, int x_per_slot, const uint32_t* ids, int rows, int slots,
                               const void* packed, int64_t packed_bytes, const uint16_t* in_scale,
                               const uint16_t* out_scale, int in_features, int out_features, int side, uint16_t* y,
                               void* workspace, size_t workspace_bytes, moe_stream_t stream);
size_t moe_trellis_grouped_linear_workspace_bytes(int rows, int slots, int in_features, int out_features,
                                                  int64_t experts);

/* ---------------------------------------------------------------- load-time conversion */

/* K4 trellis experts of one projection -> MXFP4 rows of the joined resident format: for every
 * expert e of `packed` (packed_bytes / (in*out/2) experts), inner_e = decoded [in, out] matrix;
 * gate/up (in_scale [E, in] and unit [in] fp16 given): inner_e[k, :] *= in_scale[e, k] * unit[k];
 * down: both NULL.  Row n of inner_e^T is quantised (groups of 32 along in, shared exponent
 * floor(log2 amax) - 2 as e8m0, E2M1 codes round-to-nearest-even, saturating; low nibble = even k)
 * into codes [E, out_rows, in/2] and scales [E, out_rows, in/32] at row row_offset + n (gate/up:
 * out_rows = 2 out, offsets 0 and out; down: out_rows = out, offset 0).  Workspace:
 * moe_k4_to_mxfp4_workspace_bytes(in, out) (one decoded expert).
 * Replaces: exlr8/joined_mxfp4.py:12-47 encode (one projection; mx.quantize(mode="mxfp4")). */
int moe_k4_to_mxfp4(const void* packed, int64_t packed_bytes, int in_features, int out_features, int side,
                    const uint16_t* in_scale, const uint16_t* unit, uint8_t* codes, uint8_t* scales, int out_rows,
                    int row_offset, void* workspace, size_t workspace_bytes, moe_stream_t stream);
size_t moe_k4_to_mxfp4_workspace_bytes(int in_features, int out_features);

/* ---------------------------------------------------------------- workspace */

/* Bytes of workspace needed by the decode entry points above for the given shape on the
 * current device (independent of rows up to 8). */
size_t moe_workspace_bytes(int hidden, int intermediate);

#ifdef __cplusplus
}
#endif

#endif /* MOE_MI355X_H */
