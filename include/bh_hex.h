/*
 * bh_hex.h: C ABI of the MI355X (gfx950) HEX fused-MoE library, libbh_hex.so.
 *
 * HEX ("Header-Encoded eXperts") stores each expert matrix W [out, in] as
 *   idx           uint32 [n, out, in / 32 * bits]  one little-endian bit stream per 32 inputs
 *   block_scale   uint8  [n, out, in / B]          fp8 e4m3 code per block of B inputs (32 or 128)
 *   expert_scale  float  [n]
 *   levels        float  [n, 2^bits]               the expert's own sorted level table
 *   W[e, o, i] = levels[e, code] * fp8(block_scale[e, o, i / B]) * expert_scale[e]
 * (reference layout: blackhole/anatomy/hex.py:21-31, runtime/blackhole_runtime/hex_ref.py:5-11).
 * fp8 codes decode by the kernels' formula: 0x7F / 0xFF give +-480, not NaN.
 *
 * Conventions for every entry point:
 *   - all pointers are device pointers (HIP), owned by the caller; the library keeps none of
 *     them after it returns and allocates no device memory (bh_hex_moe_glu_ids_noalloc uses a
 *     static device array of the library instead of a caller workspace);
 *   - strides are in elements; the innermost dimension of every tensor is contiguous;
 *   - work is enqueued on `stream` (a hipStream_t; NULL is the default stream) and nothing
 *     synchronises the host, so every entry point can be captured in a hipGraph;
 *   - the return value is a status code; bh_hex_last_error() gives the message of the last
 *     failing call on the calling thread. BH_HEX_ERR_VALUE corresponds to the reference's
 *     ValueError, BH_HEX_ERR_ASSERT to its AssertionError (width checks).
 * Calls that overlap on one stream are ordered; calls on different streams writing the same
 * output race, as any two kernels would.
 */
#ifndef BH_HEX_H
#define BH_HEX_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BH_HEX_ABI_VERSION 13

enum bh_hex_status {
  BH_HEX_OK = 0,
  BH_HEX_ERR_VALUE = 1,       /* bad argument or shape (reference: ValueError) */
  BH_HEX_ERR_ASSERT = 2,      /* width check (reference: AssertionError, hex_moe.py:289-290) */
  BH_HEX_ERR_HIP = 3,         /* the HIP runtime refused a launch */
  BH_HEX_ERR_UNSUPPORTED = 4  /* a dtype / bits / block combination this build has no kernel for */
};

enum bh_hex_dtype { BH_HEX_F32 = 0, BH_HEX_BF16 = 1, BH_HEX_F16 = 2, BH_HEX_I32 = 3, BH_HEX_I64 = 4 };

/* Association orders of the dequantized value (each product rounded once to float32):
 *   R  level * (fp8 * es)   torch/numpy source of truth   (blackhole/anatomy/hex.py:180-204, 116-123)
 *   D  (level * fp8) * es   the reference's dequant kernel (runtime/blackhole_runtime/hex_moe.py:163-164)
 *   T  bf16(level * fp8)    the operand of its fused kernel, no expert scale (hex_moe.py:105, 140) */
enum bh_hex_order { BH_HEX_ORDER_R = 0, BH_HEX_ORDER_D = 1, BH_HEX_ORDER_T = 2 };

/* One projection (gate_proj, up_proj or down_proj) of one tier: the HexTier part dict of
 * runtime/blackhole_runtime/hex_moe.py:174-198 after prepare(). */
typedef struct bh_hex_proj {
  const uint32_t* idx;          /* [n, out, in / 32 * bits]                         */
  const uint8_t* block_scale;   /* [n, out, in / block]                             */
  const float* expert_scale;    /* [n]                                              */
  const float* levels;          /* [n, 2^bits], contiguous                          */
  int64_t s_ie, s_in;           /* idx strides of dims 0 and 1                      */
  int64_t s_be, s_bn;           /* block_scale strides of dims 0 and 1              */
  int32_t block;                /* inputs per fp8 scale: in / block_scale.shape[-1],
                                   a multiple of 32 (the reference writes 32)       */
} bh_hex_proj;

/* Tile choice of the fused kernels (the config dict of hex_moe.py:264-283, CDNA4 terms):
 * block_m slots per expert block: 16, 32 or 64 select the decode kernels (weight-streaming,
 * an item's inputs split between workgroups), 128 the prefill kernels (one workgroup per
 * 128-slot block and tile of 256 weight rows; n_in must be a multiple of 128 and output rows
 * 16-byte aligned, otherwise BH_HEX_ERR_UNSUPPORTED). block_n, the output rows of one work item
 * of the decode kernels (16 per wave of a 16-wave workgroup), must be 256; k_split must be 1. */
typedef struct bh_hex_tile {
  int32_t block_m;
  int32_t block_n;
  int32_t k_split;
} bh_hex_tile;

/* Message of the last failing call on this thread ("" when none). */
const char* bh_hex_last_error(void);
int bh_hex_abi_version(void);

/* Dequantize one tier projection into a stacked output, one float per weight:
 *   out[expert_ids[e], row_off + o, i] = W[e, o, i] in association order `order`,
 * rounded to out_dtype (F32, BF16 or F16) to nearest even.
 * n experts of the tier, n_out rows, n_in inputs (a multiple of 32 and of the block).
 * Replaces _hex_dequant_kernel and its launch in dequant_all (hex_moe.py:154-168, 328-346) and
 * hex_dequant (blackhole/anatomy/hex.py:180-204) when expert_ids is the identity. */
int bh_hex_dequant(const bh_hex_proj* w, int32_t bits, int64_t n, int64_t n_out, int64_t n_in,
                   const int32_t* expert_ids, void* out, int32_t out_dtype, int64_t s_oe, int64_t s_on,
                   int64_t row_off, int32_t order, void* stream);

/* Softmax routing of router logits [T, E] (fp32, bf16 or f16; row stride s_lt): the k largest
 * probabilities in descending order (ties to the lower expert), optionally divided by their sum.
 * topk_w float [T, k]; topk_ids [T, k] in ids_dtype (I32 or I64).
 * Upstream of the plugin boundary: the statement of reaper/reaper_pipeline/moe.py:161-166
 * (softmax branch), as vLLM computes it before HexMoEMethod.apply (vllm_hex.py:239-240). */
int bh_hex_route_topk(const void* logits, int32_t logits_dtype, int64_t s_lt, int64_t T, int32_t E, int32_t k,
                      int32_t renormalize, float* topk_w, void* topk_ids, int32_t ids_dtype, void* stream);

/* Expert choice from router logits, as reaper/reaper_pipeline/moe.py:141-168 (route_from_logits)
 * states it for the models the reference serves:
 *   softmax branch: p = softmax(logits); the k largest p; divided by their sum if renormalize;
 *   sigmoid branch (scoring BH_HEX_SCORE_SIGMOID, or any correction_bias): s = sigmoid(logits),
 *     choice = s + correction_bias[e]; with n_group > 1 the experts form n_group groups of
 *     E / n_group consecutive ids, each group scores the sum of its two largest choices, only the
 *     topk_group best groups keep their experts (0: every group); the k largest choices; their
 *     weights are the unbiased s, divided by (their sum + 1e-20) if renormalize;
 *   then every weight times routed_scaling_factor.
 * Ties go to the lower expert (or group) id. Weights in descending order of choice. */
enum bh_hex_scoring { BH_HEX_SCORE_SOFTMAX = 0, BH_HEX_SCORE_SIGMOID = 1 };
typedef struct bh_hex_routing {
  int32_t scoring;                /* bh_hex_scoring                                          */
  int32_t renormalize;            /* norm_topk_prob                                          */
  int32_t n_group;                /* 1: no groups; at most 64, dividing E into groups of >= 2 */
  int32_t topk_group;             /* groups kept, 0..n_group (0: all)                        */
  float routed_scaling_factor;    /* 1.0 for none                                            */
  const float* correction_bias;   /* device float [E] or null (e_score_correction_bias)      */
} bh_hex_routing;

/* The choice above for logits [T, E] (F32, BF16 or F16; row stride s_lt): topk_w float [T, k],
 * topk_ids [T, k] in ids_dtype (I32 or I64). routing null: softmax, renormalised, no scaling.
 * E <= 1024, k <= min(E, 64). What vLLM's expert selection computes before
 * HexMoEMethod.apply (reaper/reaper_pipeline/moe.py:141-168). */
int bh_hex_route_select(const void* logits, int32_t logits_dtype, int64_t s_lt, int64_t T, int32_t E, int32_t k,
                        const bh_hex_routing* routing, float* topk_w, void* topk_ids, int32_t ids_dtype, void* stream);

/* Router logits and expert choice in one launch: logits[t, e] = sum_h x[t, h] w_router[e, h]
 * (the MoE block's gate linear, no bias) accumulated in float32 on the matrix cores, rounded to
 * x_dtype (BF16 or F16, the gate linear's output dtype) and written as float32 to logits
 * [T, E] (row stride s_lt), then the choice of bh_hex_route_select on them. x [T, H] and
 * w_router [E, H] in x_dtype with 16-byte aligned rows; H a multiple of 32. counters: int32
 * workspace of bh_hex_route_gemm_workspace(T) values, zero before the first call and left zero
 * by every call; calls sharing it must not overlap in time. Replaces the gate linear
 * (reaper/reaper_pipeline/moe.py:141, the router module) and the choice after it. */
int bh_hex_route_gemm(const void* x, int32_t x_dtype, int64_t s_xm, const void* w_router, int64_t s_we, int64_t T,
                      int32_t H, int32_t E, int32_t k, const bh_hex_routing* routing, float* logits, int64_t s_lt,
                      float* topk_w, void* topk_ids, int32_t ids_dtype, int32_t* counters, int64_t n_counters,
                      void* stream);
int64_t bh_hex_route_gemm_workspace(int64_t T);

/* Number of expert blocks align() produces: ceil(S / block_m) + min(n_experts, S). */
int64_t bh_hex_align_max_blocks(int64_t S, int32_t n_experts, int32_t block_m);

/* Stable counting sort of S slots by expert, each expert's run padded to block_m
 * (runtime/blackhole_runtime/hex_moe.py:201-222, align):
 *   sorted_ids int32 [max_blocks * block_m]: slot ids grouped by expert in slot order, S as padding
 *   expert_ids int32 [max_blocks]: the expert of each block, -1 past the last used block
 *   npp        int32 [1]: used blocks * block_m
 * ids (I32 or I64) outside [0, n_experts) are not placed. */
int bh_hex_align(const void* ids, int32_t ids_dtype, int64_t S, int32_t n_experts, int32_t block_m,
                 int32_t* sorted_ids, int32_t* expert_ids, int32_t* npp, void* stream);

/* bh_hex_align over the slots of one tier: slots whose expert has no entry in the tier's lookup
 * (lookup[e] < 0; int32 [n_experts], as HexTier.prepare builds it) are not placed either, so the
 * plan holds only this tier's blocks. Same outputs and max_blocks otherwise. With several tiers
 * the fused launches of a tier then walk only its own blocks. No counterpart in the reference,
 * which shares one plan between its tiers (hex_moe.py:318-324). */
int bh_hex_align_tier(const void* ids, int32_t ids_dtype, int64_t S, int32_t n_experts, const int32_t* lookup,
                      int32_t block_m, int32_t* sorted_ids, int32_t* expert_ids, int32_t* npp, void* stream);

/* int32 values of the workspace bh_hex_align_ws takes for S slots: ceil(S / 1024) * n_experts
 * above 4096 slots, 0 up to 4096; -1 for bad sizes. */
int64_t bh_hex_align_workspace(int64_t S, int32_t n_experts);

/* bh_hex_align (lookup null) or bh_hex_align_tier (lookup given), same outputs, with a caller
 * workspace of bh_hex_align_workspace(S, n_experts) int32 values (workspace_len of them; its
 * contents on entry do not matter). Above 4096 slots one workgroup per 1024-slot chunk counts
 * the chunk's slots per expert into it, so the placing workgroups read each chunk's prefix
 * instead of counting every slot before their chunk. Replaces the same reference function
 * (runtime/blackhole_runtime/hex_moe.py:201-222, align). */
int bh_hex_align_ws(const void* ids, int32_t ids_dtype, int64_t S, int32_t n_experts, const int32_t* lookup,
                    int32_t block_m, int32_t* workspace, int64_t workspace_len, int32_t* sorted_ids,
                    int32_t* expert_ids, int32_t* npp, void* stream);

/* One block per slot, no sorting (hex_moe.py:228-237, direct): sorted_ids[s * block_m] = s and S
 * elsewhere, expert_ids = ids as int32, npp = S * block_m. */
int bh_hex_direct(const void* ids, int32_t ids_dtype, int64_t S, int32_t block_m, int32_t* sorted_ids,
                  int32_t* expert_ids, int32_t* npp, void* stream);

/* The gate/up half of a SwiGLU expert layer over one tier, for every expert block of the plan:
 *   act[s, o] = silu(es_g * sum_i a[s] W_g[o, i]) * (es_u * sum_i a[s] W_u[o, i]),
 *   a[s] = x[s / a_div], s the slots of the block (rows >= num_slots are padding).
 * Blocks whose expert belongs to another tier (lookup[e] < 0) are skipped. x and act are
 * BF16 or F16 (x_dtype; act has the same dtype), x [T, n_in], act [num_slots, n_out].
 * Weights enter the bf16/f16 matrix cores as round(level); each 32-input block's partial sum is
 * multiplied by its fp8 scale in float32 and the expert scale is applied at the end.
 * Replaces _hex_moe_kernel with GLU=True and its launch (hex_moe.py:109-151, 286-301, 322). */
int bh_hex_moe_glu(const void* x, int32_t x_dtype, int64_t s_xm, void* act, int64_t s_am,
                   const bh_hex_proj* gate, const bh_hex_proj* up, int32_t bits, int64_t n_out, int64_t n_in,
                   const int32_t* sorted_ids, const int32_t* expert_ids, int64_t num_blocks, const int32_t* npp,
                   const int32_t* lookup, int32_t n_experts, int64_t num_slots, int32_t a_div,
                   const bh_hex_tile* tile, int32_t* counters, int64_t n_counters, float* partials,
                   int64_t n_partials, void* stream);

/* The down half over one tier: y[s, o] = (es_d * sum_i act[s, i] W_d[o, i]) * topk_w[s],
 * written to y [num_slots, n_out] (row stride s_ym) for the slots of every block of this tier's
 * experts, in y_dtype: F32, or act_dtype (rounded once per slot, as the reference's y in
 * x.dtype, hex_moe.py:316). Replaces _hex_moe_kernel with GLU=False, MUL_W=True
 * (hex_moe.py:324). */
int bh_hex_moe_down(const void* act, int32_t act_dtype, int64_t s_am, void* y, int32_t y_dtype, int64_t s_ym,
                    const bh_hex_proj* down, int32_t bits, int64_t n_out, int64_t n_in,
                    const int32_t* sorted_ids, const int32_t* expert_ids, int64_t num_blocks, const int32_t* npp,
                    const int32_t* lookup, int32_t n_experts, int64_t num_slots, const float* topk_w,
                    const bh_hex_tile* tile, int32_t* counters, int64_t n_counters, float* partials,
                   int64_t n_partials, void* stream);

/* bh_hex_moe_glu without a precomputed plan: the kernel derives the slot plan from the routing
 * ids itself (topk_ids [num_slots], I32 or I64), as align() with this tier's lookup would
 * (hex_moe.py:201-222): every workgroup sorts the slots by expert in LDS and keeps the blocks
 * its range needs, so no align launch precedes it. block_m 16, 32 or 64 (the decode kernels)
 * and at most 1024 slots; otherwise BH_HEX_ERR_UNSUPPORTED. The workspace is
 * bh_hex_moe_workspace(bh_hex_align_max_blocks(num_slots, n_experts, block_m), ...). Same
 * results as align + bh_hex_moe_glu. Replaces align and the first _hex_moe_kernel launch of
 * hex_moe_fused (hex_moe.py:201-222, 318-322). */
int bh_hex_moe_glu_ids(const void* x, int32_t x_dtype, int64_t s_xm, void* act, int64_t s_am,
                       const bh_hex_proj* gate, const bh_hex_proj* up, int32_t bits, int64_t n_out, int64_t n_in,
                       const void* topk_ids, int32_t ids_dtype, const int32_t* lookup, int32_t n_experts,
                       int64_t num_slots, int32_t a_div, const bh_hex_tile* tile, int32_t* counters,
                       int64_t n_counters, float* partials, int64_t n_partials, void* stream);

/* bh_hex_moe_glu_ids without a workspace argument: it allocates nothing and takes no caller
 * workspace. No counterpart in the reference; it is for callers that cannot allocate device
 * memory (code under hipGraph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Its counters and partial sums live in a static device array of this library (17 MiB per
 * device, held until the process ends): 2^18 counters and 2^22 partial floats, enough for
 * 16-slot blocks on every CU of an MI355X; a launch that needs more returns
 * BH_HEX_ERR_UNSUPPORTED (bh_hex_moe_workspace gives the needs). The first call on a device
 * looks the array up and clears its counters (a fill kernel on `stream`); every call leaves
 * them zero. All calls on one device share the array: calls that overlap in time on one device
 * (different streams, or different host threads) race. Same limits and results as
 * bh_hex_moe_glu_ids. */
int bh_hex_moe_glu_ids_noalloc(const void* x, int32_t x_dtype, int64_t s_xm, void* act, int64_t s_am,
                               const bh_hex_proj* gate, const bh_hex_proj* up, int32_t bits, int64_t n_out,
                               int64_t n_in, const void* topk_ids, int32_t ids_dtype, const int32_t* lookup,
                               int32_t n_experts, int64_t num_slots, int32_t a_div, const bh_hex_tile* tile,
                               void* stream);

/* bh_hex_moe_down with the plan derived from the routing ids in the kernel, as
 * bh_hex_moe_glu_ids (same limits and workspace). Replaces the second _hex_moe_kernel launch of
 * hex_moe_fused (hex_moe.py:324) together with the plan it reads. */
int bh_hex_moe_down_ids(const void* act, int32_t act_dtype, int64_t s_am, void* y, int32_t y_dtype, int64_t s_ym,
                        const bh_hex_proj* down, int32_t bits, int64_t n_out, int64_t n_in, const void* topk_ids,
                        int32_t ids_dtype, const int32_t* lookup, int32_t n_experts, int64_t num_slots,
                        const float* topk_w, const bh_hex_tile* tile, int32_t* counters, int64_t n_counters,
                        float* partials, int64_t n_partials, void* stream);

/* Device workspace that bh_hex_moe_glu (glu != 0) or bh_hex_moe_down needs for a plan of
 * num_blocks blocks of block_m slots over n_out x n_in projections on the current device:
 * *n_counters int32 arrival counters and *n_partials floats (16-byte aligned) of partial sums.
 * The counters must be zero before their first use; every call leaves them zero again, so one
 * workspace, sized for the largest call, can be kept and shared by calls of any shape. The
 * partials need no initial value. Calls that share a workspace must not overlap in time (one
 * stream, or ordered streams). No counterpart in the reference, whose Triton kernels need none:
 * the kernels split an item's inputs between workgroups, and the last workgroup to arrive adds
 * the others' partial sums. For block_m 128 both sizes are 0 (the prefill kernels need no
 * workspace; counters and partials may then be null). */
int bh_hex_moe_workspace(int64_t num_blocks, int64_t n_out, int64_t n_in, int32_t block_m, int32_t glu,
                         int64_t* n_counters, int64_t* n_partials);

/* out[t, h] = sum_j y[t * k + j, h] over the token's k slots, in float32, rounded once to
 * out_dtype (F32, BF16 or F16); y is F32, BF16 or F16 (y_dtype); slots whose id (topk_ids, I32
 * or I64) is outside [0, n_experts) contribute nothing. Replaces y.view(T, k, H).sum(1)
 * (hex_moe.py:325). */
int bh_hex_moe_reduce(const void* y, int32_t y_dtype, int64_t s_ym, const void* topk_ids, int32_t ids_dtype,
                      int32_t n_experts, int64_t T, int32_t k, int64_t H, void* out, int32_t out_dtype, int64_t s_ot,
                      void* stream);

/* The whole layer of one tier for a few tokens, as two matrix-vector launches (no plan, no
 * workspace): act[s, o] as bh_hex_moe_glu writes it for every slot s < T * k whose expert has
 * this tier (one wave per slot and output row; act [T * k, inter], row stride s_am, in x_dtype,
 * rows of other slots left unwritten), then
 *   out[t, h] = sum_j topk_w[t * k + j] * es_d * sum_i act[t * k + j, i] W_d[h, i]
 * over the token's slots of this tier, in float32, rounded once to out_dtype (= x_dtype): the
 * down projection, the top-k weight and the k-slot sum in one launch (one wave per token and
 * output row). Slots whose id (topk_ids, I32 or I64) is outside [0, n_experts) or has no
 * expert in this tier (lookup[id] < 0) contribute nothing. Weights enter as in bh_hex_moe_glu
 * (round(level) times activations in float32, each 32-input block's partial times its fp8
 * scale, the expert scale at the end). Limits: k <= 16, hidden <= 4096, inter <= 2048, widths
 * multiples of 32, T * k <= 65535; otherwise BH_HEX_ERR_UNSUPPORTED. Each weight row of
 * a routed expert is read once per slot that routes to it, so the launches suit batches of a few
 * tokens. Replaces, for such batches, align, the two _hex_moe_kernel launches and the sum of
 * hex_moe_fused (hex_moe.py:304-325). */
int bh_hex_moe_gemv(const void* x, int32_t x_dtype, int64_t s_xm, void* act, int64_t s_am, void* out,
                    int32_t out_dtype, int64_t s_om, const bh_hex_proj* gate, const bh_hex_proj* up,
                    const bh_hex_proj* down, int32_t bits, int64_t hidden, int64_t inter, const void* topk_ids,
                    int32_t ids_dtype, const float* topk_w, const int32_t* lookup, int32_t n_experts, int64_t T,
                    int32_t k, void* stream);

/* The GPTQ column sweep of the HEX producer, rounding onto each expert's level table, with the
 * table indices of the result: for each of n experts, w [n, out, in] float32 (the weights with dead
 * columns zeroed; overwritten: the sweep updates it), u [n, in, in] float32 the upper Cholesky
 * factor of the damped inverse Hessian, levels [n, n_levels] float32 sorted (8 or 16), scale
 * [n, out, in / scale_block] float32 the dequant scale of each scale block. Columns run in order in
 * sweep blocks of `block` (1..128): column c of a row is rounded to the level nearest to
 * clamp(w / s, -1, 1) (midpoints (a + b) / 2, a left search) times s; its error (w - q) / u[c, c]
 * updates the block's later columns (w -= err * u[c, c'], product and difference each rounded)
 * and, when the block ends, the later columns take w -= sum_k err_k u[k, c'] as one fused
 * multiply-add chain over the block in column order. Then q is multiplied by 0 in the columns
 * that dead [n, in] marks (null: none) and codes [n, out, in] (uint8) get the index of the level
 * nearest to clamp(q / s, -1, 1). Every operation is the reference's on the CPU, so q and codes
 * equal its output bit for bit on the same inputs. Replaces the sweep of
 * reaper/gpu_perf/gptq.py:62-83 (_solve) and table_indices (harness/blackhole_pipeline/pack.py:53-62). */
/* The HEX producer's block header (reaper/gpu_perf/headers.py:39-51, _blocks, non-shared scale;
 * harness/blackhole_pipeline/pack.py:77-86, expert_scale and block_codes) for w [n, out, in]
 * float32, in a multiple of block: expert_scale[e] = max(max|w| / 448, 1e-30); per block of
 * `block` inputs scale = fp8(min(amax / es, 448)) * es (1 where that is 0; fp8 = e4m3fn, round to
 * nearest even), codes (uint8, may be null) the e4m3fn code of min(scale / es, 448), xn (may be
 * null) clamp(w / scale, -1, 1) [n, out, in], and, when col_weight [n, in] is given, the k-means
 * weights wt [n, out, in] = col_weight[col] * scale^2 (headers.py:96-98). Divisions are IEEE, so
 * every output equals the reference's on the CPU bit for bit. */
int bh_hex_block_header(const float* w, int64_t n, int64_t out, int64_t in, int32_t block, const float* col_weight,
                        float* xn, float* scale, uint8_t* codes, float* wt, float* expert_scale, void* stream);

/* The weighted 1-D k-means of the HEX producer (reaper/gpu_perf/headers.py:66-83, fit_levels) for
 * n experts of S sampled values xs [n, S] with weights ws [n, S] (the caller draws the sample as
 * the reference does, from its CPU generator): the start is the quantile lo + w (hi - lo) of each
 * of n_levels ranks (q_lo, q_hi [n, n_levels]: the sorted sample at the floor and ceiling of the
 * rank; q_w [n_levels] the fractions), then `iters` Lloyd rounds (left midpoint search, each
 * level's sums in sample order, num / max(den, 1e-30) where den > 0, sort). levels [n, n_levels].
 * Equals the reference on the CPU bit for bit. One wave per expert. */
int bh_hex_fit_levels(const float* xs, const float* ws, int64_t n, int64_t S, int32_t n_levels, const float* q_lo,
                      const float* q_hi, const float* q_w, int32_t iters, float* levels, void* stream);

int bh_hex_gptq_sweep(float* w, const float* u, const float* levels, int32_t n_levels, const float* scale,
                      int32_t scale_block, const uint8_t* dead, int64_t n, int64_t out, int64_t in, int32_t block,
                      float* q, uint8_t* codes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* BH_HEX_H */
