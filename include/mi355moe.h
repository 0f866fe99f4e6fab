/*
 * mi355moe: the routed-MoE layer hot path of GLM-style EXL3 models on one AMD MI355X (gfx950), as a C ABI.
 *
 * Conventions (every entry point):
 *   - all tensor arguments are device pointers (hipMalloc'd or torch CUDA tensors); sizes are element counts;
 *   - work is enqueued on `stream` in order; nothing is allocated, nothing synchronizes with the host, so every
 *     call can be captured into a HIP graph;
 *   - return 0 on success, a positive MI355MOE_E* code when an argument is rejected (checked before anything is
 *     enqueued, so outputs are untouched), or a negative value when a launch failed (the HIP error, negated);
 *   - `workspace` is caller-owned device memory of at least the size the matching *_workspace_bytes function
 *     reports, zero-filled once before its first use; calls keep it in that state (counters return to zero).
 *     Calls that share one workspace must be stream-ordered (not concurrent).
 *
 * EXL3 weights of one layer (code/fork/docs/prod_exl3_reference.py:2048-2162): per expert e, gate/up
 * trellis int16 [K/16][N/16][64], suh fp16 [K], svh fp16 [N]; down trellis int16 [N/16][K/16][64], suh fp16 [N],
 * svh fp16 [K]. The kernels reach them through nine int64 pointer tables of n device addresses each, the same
 * tables production builds (prod_exl3_reference.py:1438-1487).
 */
#ifndef MI355MOE_H
#define MI355MOE_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MI355MOE_ABI_VERSION 2

enum {
    MI355MOE_OK = 0,
    MI355MOE_EINVAL = 1,       /* null pointer or bad flag */
    MI355MOE_ESHAPE = 2,       /* unsupported shape */
    MI355MOE_ELIMIT = 3,       /* beyond a documented limit (pairs, experts, topk) */
    MI355MOE_EWORKSPACE = 4,   /* workspace too small */
    MI355MOE_EDTYPE = 5,       /* unsupported dtype code */
    MI355MOE_EUNSUPPORTED = 6, /* a format variant this library does not implement (e.g. bits != 4) */
    MI355MOE_ESCRATCH = 7      /* needs more than the fixed scratch of mi355moe_moe_layer_noalloc */
};

/* dtype codes */
enum { MI355MOE_F32 = 0, MI355MOE_F16 = 1, MI355MOE_BF16 = 2, MI355MOE_I32 = 3, MI355MOE_I64 = 4 };

typedef struct mi355moe_exl3_layer {
    int64_t n;              /* local experts */
    int64_t hidden;         /* K, multiple of 256 */
    int64_t intermediate;   /* N, multiple of 128 */
    /* nine device int64 [n] tables; entry i = expert i's tensor address. EVERY entry of every table must be
     * 16-byte aligned (trellis words and scales are read with 16-byte loads). */
    const int64_t* gate_trellis;
    const int64_t* gate_suh;
    const int64_t* gate_svh;
    const int64_t* up_trellis;
    const int64_t* up_suh;
    const int64_t* up_svh;
    const int64_t* down_trellis;
    const int64_t* down_suh;
    const int64_t* down_svh;
    int64_t flags;          /* MI355MOE_LAYER_* bits */
} mi355moe_exl3_layer;

/* gate and up share one input rotation (w13_suh[:, 0] == w13_suh[:, 1], production's _exl3_shared_w13_suh,
 * code/fork/docs/prod_exl3_reference.py:2243-2245); the grouped prefill path requires it (:376) */
#define MI355MOE_LAYER_SHARED_W13_SUH 1
/* every expert of the layer has the same w13 suh (with MI355MOE_LAYER_SHARED_W13_SUH): the rotated gate/up input
 * does not depend on the expert, so the grouped path gathers one row per token instead of one per routed pair and
 * its gate/up GEMM reads A rows through the rows' tokens (the reference's TOKGATHER, code/fork/docs/OPT_MOE.md:14;
 * true of the real checkpoints' layers). Same results bit for bit; the flag only changes the schedule. */
#define MI355MOE_LAYER_UNIFORM_W13_SUH 2

int mi355moe_abi_version(void);
const char* mi355moe_strerror(int code);

/* W_q fp16 [k_tiles*16][n_tiles*16] from one 4-bit trellis int16 [k_tiles][n_tiles][64], bit for bit the
 * reference decode (replaces code/fork/kernels/exl3_format_ref.py:88-97 `unpack` and ExLlamaV3's `reconstruct`,
 * code/fork/tests/test_layout_equiv.py:1-46). n_tiles must be a multiple of 8. */
int mi355moe_exl3_dequant(const void* trellis, int64_t k_tiles, int64_t n_tiles, void* wq, hipStream_t stream);

/* The logistic sigmoid of the SwiGLU epilogues on n fp32 values (stage entry): variant 0 = the decode epilogue's
 * 1 / (1 + (float)exp(-(double)g)) with an IEEE division, E3's formula (code/fork/docs/ref/mia_exl3-fat-kernel/
 * exl3_fat_moe.cu:366-369); variant 1 = the grouped prefill epilogues' fp32 form (v_exp_f32 of the rounded
 * exponent with its residual, one v_rcp_f32), a few ulp from variant 0. g and out fp32 device arrays of n. */
int mi355moe_sigmoid(const float* g, int64_t n, int variant, float* out, hipStream_t stream);

/* Router logits fp32 [T][E] = x bf16 [T][K] (row stride x_stride) times W bf16 [E][K]^T, each the bf16 rounding
 * (through fp32, nearest even) of the float64 sum of the bf16 products, as F.linear(x, W).to(torch.float32)
 * returns it (code/fork/docs/BF16_GEMV.md:27,38; reference oracle (X.double() @ W.t()).to(bfloat16),
 * code/fork/tests/router_topk_agreement.py:82). K % 512 == 0, K <= 8192. */
int mi355moe_router_logits(const void* x, int64_t T, int64_t K, int64_t x_stride, const void* w, int64_t E,
                           float* logits, hipStream_t stream);

/* Sigmoid + bias top-k with renormalisation and routed scale: vLLM grouped_topk(logits, num_expert_group=1,
 * topk_group=1, topk, renormalize, routed_scaling_factor, e_score_correction_bias, scoring="sigmoid")
 * (code/fork/tests/router_topk_agreement.py:58-61; semantics code/fork/docs/ref/tf_glue.py:371-401).
 * ids int32 [T][topk], weights fp32 [T][topk]. bias may be NULL. E <= 1024, topk <= 32. */
int mi355moe_router_topk(const float* logits, int64_t T, int64_t E, const float* bias, int64_t topk,
                         float routed_scale, int renormalize, int32_t* topk_ids, float* topk_weights,
                         hipStream_t stream);

/* Token -> expert permutation of P = T*topk pairs (stage entry). Local ids by map_topk_to_local
 * (prod_exl3_reference.py:936-958, expert_map optional, NULL = identity), stable sorted position per pair
 * (code/fork/kernels/exl3.cu:742-775), counts and the row-segment table of eligible experts (0 < count <= R,
 * ceil(count/seg_rows) segments each, code/fork/kernels/exl3.cu:529-566).
 * Outputs: tok/pe/w16 indexed by sorted position, inv[j] = position of pair j, seg_* [s_cap], nseg [1],
 * counts [n+1] (last = sentinel). ids dtype I32/I64, weights F32/F16/BF16. */
int64_t mi355moe_route_workspace_bytes(int64_t P, int64_t n);
int mi355moe_route(const void* ids, int ids_dtype, const void* weights, int weights_dtype, int64_t T, int64_t topk,
                   const int64_t* expert_map, int64_t n_global, int64_t n, int64_t R, int64_t seg_rows,
                   int32_t* tok, uint16_t* w16, int32_t* pe, int32_t* inv, int32_t* seg_expert, int32_t* seg_row0,
                   int32_t* seg_rows_out, int64_t s_cap, int32_t* nseg, int32_t* counts, void* workspace,
                   size_t workspace_bytes, hipStream_t stream);

/* The e4m3 extension's routing plan (code/fork/overlay/glm53_moe_e4m3.py:450-477) on the device: the permutation
 * above (local ids by map_topk_to_local, pairs sorted by local id, stable, the sentinel pairs last) returned as its
 * row tables: per pair j, local[j] (n for a pair with no local expert) and its row pos[j]; per row p, row_token[p]
 * (int64), row_weight[p] (fp32) and row_expert[p] (n for the sentinel rows); counts int64 [n + 1]. */
int64_t mi355moe_route_rows_workspace_bytes(int64_t P, int64_t n);
int mi355moe_route_rows(const void* ids, int ids_dtype, const void* weights, int weights_dtype, int64_t T,
                        int64_t topk, const int64_t* expert_map, int64_t n_global, int64_t n, int32_t* local,
                        int32_t* pos, int64_t* row_token, float* row_weight, int32_t* row_expert, int64_t* counts,
                        void* workspace, size_t workspace_bytes, hipStream_t stream);

/* Input rotation (stage entry): out[pos] = fp16(H(fp16(x[tok[pos]] * suh[pe[pos]])) * r) for rows with pe >= 0
 * (code/fork/kernels/exl3.cu:321-349; E3 gather code/fork/docs/ref/mia_exl3-fat-kernel/exl3_fat_moe.cu:95-126).
 * x dtype F16 or BF16 [*, K] (row stride x_stride); out fp16 [P][K]. */
int mi355moe_rot_in(const void* x, int x_dtype, int64_t x_stride, int64_t K, const int32_t* tok, const int32_t* pe,
                    int64_t P, const int64_t* suh_table, void* out, hipStream_t stream);

/* Routed experts from router ids: the decode apply (code/fork/kernels/exl3.cpp:307-391 moe_forward_ids,
 * exl3.cpp:409-503 moe_forward_glue) and, for many pairs, the grouped prefill tier (E3,
 * code/fork/docs/prod_exl3_reference.py:1364-1435, code/fork/docs/ref/mia_exl3-fat-kernel/exl3_fat_moe.cu).
 * x F16/BF16 [T][K] (row stride x_stride), ids I32/I64 [T][topk], weights F32/F16/BF16 [T][topk], out [T][K] of
 * out_dtype (row stride out_stride) is WRITTEN (not accumulated). limit = the SwiGLU limit (0 = none).
 * Both paths add a token's per-pair contributions in slot order (fp32, deterministic) and write out_dtype.
 * Pairs P = T*topk <= 65536. */
enum { MI355MOE_PATH_AUTO = 0, MI355MOE_PATH_DECODE = 1, MI355MOE_PATH_PREFILL = 2 };
/* The automatic choice: the prefill path when P >= MI355MOE_PREFILL_MIN_PAIRS and the layer has
 * MI355MOE_LAYER_SHARED_W13_SUH, else the decode path (measured at 288 experts, hidden 4096, intermediate 1024: the
 * decode path is faster up to ~4,700 pairs, the grouped path beyond). */
#define MI355MOE_PREFILL_MIN_PAIRS 5120
int64_t mi355moe_moe_workspace_bytes(const mi355moe_exl3_layer* layer, int64_t T, int64_t topk);
int64_t mi355moe_moe_workspace_bytes_path(const mi355moe_exl3_layer* layer, int64_t T, int64_t topk, int path);

/* Stage mask of mi355moe_moe_forward_ids_ex: the same call split into its launches, so a caller can time or
 * test one of them (the reference's stage entry points, code/fork/kernels/exl3.cpp:130-220: route_prep, grouped,
 * gateup_epilogue, down_epilogue). A stage reads what the earlier stages of a call with the same arguments left in
 * the workspace. */
enum { MI355MOE_STAGE_ROUTE = 1, MI355MOE_STAGE_GATEUP = 2, MI355MOE_STAGE_DOWN = 4, MI355MOE_STAGE_COMBINE = 8,
       MI355MOE_STAGE_ALL = 15 };
int mi355moe_moe_forward_ids(const mi355moe_exl3_layer* layer, const void* x, int x_dtype, int64_t x_stride,
                             int64_t T, const void* ids, int ids_dtype, const void* weights, int weights_dtype,
                             int64_t topk, const int64_t* expert_map, int64_t n_global, float limit, void* out,
                             int out_dtype, int64_t out_stride, void* workspace, size_t workspace_bytes,
                             hipStream_t stream);
int mi355moe_moe_forward_ids_ex(const mi355moe_exl3_layer* layer, const void* x, int x_dtype, int64_t x_stride,
                                int64_t T, const void* ids, int ids_dtype, const void* weights, int weights_dtype,
                                int64_t topk, const int64_t* expert_map, int64_t n_global, float limit, void* out,
                                int out_dtype, int64_t out_stride, void* workspace, size_t workspace_bytes, int path,
                                int stages, hipStream_t stream);

/* mi355moe_moe_forward_ids_ex with an options mask (the reference's opt-in prefill knobs, code/fork/docs/
 * OPT_MOE.md:9-21, and its e4m3 numerics):
 *   MI355MOE_OPT_ACCUMULATE   out += the routed output instead of out = (the FOLD_SHARED knob: out holds the shared
 *                             experts' output, and the sum is added to it in fp32 with one rounding to out_dtype, so
 *                             the separate shared + routed add is not needed); both paths.
 *   MI355MOE_OPT_BF16_CONTRIB the grouped path keeps its per-pair down accumulators in bf16 (half the bytes of the
 *                             contribution buffer; the ACC=bf16 knob's traffic saving). The combine still applies
 *                             the rotation, svh and router weight in fp32 and adds a token's slots in slot order, so
 *                             the result stays deterministic; each contribution carries one bf16 rounding of its raw
 *                             accumulators (relative error about 2^-9 per element). No effect on the decode path.
 *   MI355MOE_OPT_E4M3         the trellis-sourced e4m3 numerics of mi355moe_e4m3_moe_forward_ids (grouped path
 *                             only: path DECODE is refused; hidden <= 4096).
 *   MI355MOE_OPT_DOWN16       with MI355MOE_OPT_E4M3: the down projection on fp16 operands (the e4m3 extension's
 *                             variant 16, code/fork/overlay/glm53_moe_e4m3.py:660-674 spec_proj16): the down input
 *                             h = fp16(H(float(a16) * suh_d) * r) times the fp16 W_q with fp32 sums.
 *   MI355MOE_OPT_PERSISTENT   the grouped path's gate/up and down tiles in one launch of one workgroup per compute
 *                             unit, ticket-ordered with per-segment dataflow counts (the reference's fused schedule,
 *                             code/fork/kernels/moe_e4m3.cu:867-897; item order: mi355moe_sched_item), whatever the
 *                             call's size, on the tile kind the call picks. Without the option the library takes
 *                             this schedule by itself in every numerics (the environment variable
 *                             MI355MOE_SCHED=separate turns that off). Applies when the call runs both stages
 *                             (MI355MOE_STAGE_GATEUP and MI355MOE_STAGE_DOWN) on the grouped path; results are
 *                             bit-identical to the separate launches. With MI355MOE_OPT_E4M3 (e4m3 down GEMM) the
 *                             workgroup finishing a segment's gate/up items quantises its down inputs in the launch.
 *                             The lag (in segments of one of its eight queues) is read from the environment variable
 *                             MI355MOE_SCHED_LAG (default 0 = all of a queue's gate/up items first).
 * Unknown bits: MI355MOE_EINVAL. Workspace sizes as mi355moe_moe_workspace_bytes_path (with MI355MOE_OPT_E4M3:
 * mi355moe_e4m3_moe_workspace_bytes). */
enum { MI355MOE_OPT_ACCUMULATE = 1, MI355MOE_OPT_BF16_CONTRIB = 2, MI355MOE_OPT_E4M3 = 4, MI355MOE_OPT_PERSISTENT = 8,
       MI355MOE_OPT_DOWN16 = 16 };

/* Item `ticket` of the one-launch schedule (MI355MOE_OPT_PERSISTENT) over `segments` row segments with gateup_items /
 * down_items column blocks per segment (intermediate / 128 and hidden / 256) and lag L = min(lag, segments) (lag 0:
 * segments): the gate/up items of segments 0 .. L - 1, then for r = 0, 1, ... the gate/up items of segment L + r
 * followed by the down items of segment r, then the down items of the last L segments
 * (code/fork/kernels/moe_e4m3.cu:867-872 and 931-959, make_job). *kind = 0 gate/up, 1 down, -1 past the last item;
 * *segment and *block name the tile. A host-side query (no device work): 0, or MI355MOE_EINVAL. */
int mi355moe_sched_item(int64_t ticket, int64_t segments, int64_t lag, int64_t gateup_items, int64_t down_items,
                        int* kind, int* segment, int* block);
int mi355moe_moe_forward_ids_opt(const mi355moe_exl3_layer* layer, const void* x, int x_dtype, int64_t x_stride,
                                 int64_t T, const void* ids, int ids_dtype, const void* weights, int weights_dtype,
                                 int64_t topk, const int64_t* expert_map, int64_t n_global, float limit, void* out,
                                 int out_dtype, int64_t out_stride, void* workspace, size_t workspace_bytes, int path,
                                 int stages, int options, hipStream_t stream);

/* The thin/fat split of a prefill-size call (production's E3 branch, code/fork/docs/prod_exl3_reference.py:1659-1679,
 * with the cap of code/fork/glm53_prefill_cap.py): experts routed at most thin_cap rows run on the decode kernels
 * (16-row segments, limit after SiLU), the others on the grouped kernels (256-row tiles, limit before SiLU); both
 * write per-pair contributions at the same sorted positions and every token's slots are summed in slot order, out
 * WRITTEN in out_dtype. thin_cap = 0: every expert on the grouped kernels. The layer needs
 * MI355MOE_LAYER_SHARED_W13_SUH. Arguments otherwise as mi355moe_moe_forward_ids. */
int64_t mi355moe_moe_split_workspace_bytes(const mi355moe_exl3_layer* layer, int64_t T, int64_t topk,
                                           int64_t thin_cap);
int mi355moe_moe_forward_ids_split(const mi355moe_exl3_layer* layer, const void* x, int x_dtype, int64_t x_stride,
                                   int64_t T, const void* ids, int ids_dtype, const void* weights, int weights_dtype,
                                   int64_t topk, const int64_t* expert_map, int64_t n_global, float limit, void* out,
                                   int out_dtype, int64_t out_stride, int64_t thin_cap, void* workspace,
                                   size_t workspace_bytes, hipStream_t stream);

/* The fused-experts op exllamav3_ext.exl3_moe (code/fork/docs/ref/xl_exl3_moe.cu:93-130, called by
 * prod_exl3_reference.py:1490-1537): hidden fp16 [B][K]; out fp32 [B][K] ACCUMULATED into; expert_count int64
 * [n+1] (last = sentinel bucket, ignored); token_sorted int64 [P]; weight_sorted fp16 [P]; experts with more
 * than max_rows (the temps' second dimension) rows are skipped, as the original kernel does; act_function 0
 * (SiLU) only; k_gate/k_up/k_down = 4 (bits) only; mcg flags must be 1 and mul1 flags 0 (the formats this
 * library decodes). P = 0 is a no-op. */
int64_t mi355moe_exl3_moe_workspace_bytes(const mi355moe_exl3_layer* layer, int64_t P);
int mi355moe_exl3_moe(const mi355moe_exl3_layer* layer, const void* hidden, int64_t B, float* out,
                      const int64_t* expert_count, const int64_t* token_sorted, const void* weight_sorted, int64_t P,
                      int64_t max_rows, int act_function, int k_gate, int k_up, int k_down, int gate_mcg,
                      int gate_mul1, int up_mcg, int up_mul1, int down_mcg, int down_mul1, float act_limit,
                      void* workspace, size_t workspace_bytes, hipStream_t stream);

/* The routed-expert output of one MoE layer from its hidden states, in one call: router logits x . W^T in fp32
 * (mi355moe_router_logits' bf16-rounded values) or given logits, sigmoid + bias top-k with renormalisation and routed scale
 * (mi355moe_router_topk), the token -> expert permutation, the expert GEMMs and the slot-order combine. Replaces the
 * routed part of the model's MoE block: the gate linear (code/fork/docs/BF16_GEMV.md:27,38), vLLM grouped_topk with
 * one group (code/fork/tests/router_topk_agreement.py:58-61) and FusedMoE.apply (code/fork/docs/
 * prod_exl3_reference.py:1788-1823). Exactly one of router_w (bf16 [E][hidden]; x must then be BF16 with
 * x_stride % 8 == 0 and hidden % 512 == 0, hidden <= 8192) and logits (fp32 [T][E]) is given; bias may be NULL.
 * The results equal those of the separate entry points chained, bit for bit. ids_out / weights_out (optional,
 * int32 / fp32 [T][topk]) receive the picks. E <= 1024, topk <= 32. */
int64_t mi355moe_moe_layer_workspace_bytes(const mi355moe_exl3_layer* layer, int64_t T, int64_t topk, int64_t E);
int mi355moe_moe_layer(const mi355moe_exl3_layer* layer, const void* x, int x_dtype, int64_t x_stride, int64_t T,
                       const void* router_w, const float* logits, int64_t E, const float* bias, int64_t topk,
                       float routed_scale, int renormalize, float limit, void* out, int out_dtype, int64_t out_stride,
                       int32_t* ids_out, float* weights_out, void* workspace, size_t workspace_bytes,
                       hipStream_t stream);

/* mi355moe_moe_layer without a workspace argument, for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid allocation); it has no counterpart in the reference.
 * The scratch is a fixed array of MI355MOE_NOALLOC_SCRATCH_BYTES in the library's device memory, one per GPU, held
 * until the process ends: enough for decode-size calls (T <= 64 tokens at top-8 with hidden 4096, intermediate 1024
 * and E <= 1024 router experts; mi355moe_moe_layer_workspace_bytes says what a shape needs). Larger calls return
 * MI355MOE_ESCRATCH before anything is enqueued. The call allocates nothing (no hipMalloc, no library allocation);
 * the first call on a GPU looks the array up and zeroes its control block on `stream`. Every call on one GPU shares
 * that GPU's array: calls that overlap on one GPU (concurrent streams, or concurrently replayed graphs) race. The
 * results equal mi355moe_moe_layer's bit for bit. */
#define MI355MOE_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)
int mi355moe_moe_layer_noalloc(const mi355moe_exl3_layer* layer, const void* x, int x_dtype, int64_t x_stride,
                               int64_t T, const void* router_w, const float* logits, int64_t E, const float* bias,
                               int64_t topk, float routed_scale, int renormalize, float limit, void* out,
                               int out_dtype, int64_t out_stride, int32_t* ids_out, float* weights_out,
                               hipStream_t stream);

/* ---------------------------------------------------------------- the grouped (E3) trio over row tables */

/* The three stages of the grouped fat-expert tier on caller-built device tables, the contract of
 * exl3_fat_moe_gather / _gateup / _down (code/fork/docs/ref/mia_exl3-fat-kernel/exl3_fat_moe.cuh:20-56), called by
 * apply_exl3_grouped_fat (code/fork/docs/prod_exl3_reference.py:1364-1435) with the tables of
 * build_grouped_fat_tables (:1316-1361): rows grouped by expert in a row buffer of rows_cap rows, row_token int64 /
 * row_expert int32 / row_weight fp16 per row, segments (seg_expert, seg_row0, seg_rows) of at most
 * mi355moe_e3_tile_rows() rows each, and the live counts num_rows / num_segs as int32 [1] device words (read by the
 * kernels, so the host never synchronises). h13 fp16 [rows_cap][K] and h2 fp16 [rows_cap][N] are the stages'
 * intermediates, in this library's staging order (k permuted within 16-element groups); they are only meant to be
 * passed from one stage to the next. Numerics: the E3 rounding points (gather fp16(H(fp16(x * suh)) * r); gate/up
 * with the limit before SiLU; down (H(acc) * r) * svh * w). The down stage ADDS each token's rows to out fp32
 * [tokens][out_stride] in row order (deterministic, no atomics; at most 32 rows per token); its workspace (size from
 * mi355moe_e3_down_workspace_bytes) holds the raw accumulators and the token row lists. Rows whose token is outside
 * [0, tokens) or whose expert is outside [0, n) are skipped; segment entries outside the row buffer are skipped. */
int64_t mi355moe_e3_tile_rows(void);
/* The row and segment tables of the fat experts (the contract of build_grouped_fat_tables, prod_exl3_reference.py:
 * 1316-1361) from the sorted pairs' counts int64 [n] (sentinel excluded), token_sorted int64 [rows_cap] and
 * weight_sorted fp16 [rows_cap]: the experts with more than cap pairs are laid out back to back in expert order (row
 * r of expert e = its sorted position counts-prefix(e) + (r - fat-prefix(e))), segments of at most tile rows (tile <=
 * mi355moe_e3_tile_rows(), max_segs >= ceil(rows_cap / tile) + n). Rows past num_rows get row_expert -1, token 0 and
 * weight 0. scratch: int32 [2 n]. */
int mi355moe_e3_fat_tables(const int64_t* counts, int64_t n, int64_t cap, const int64_t* token_sorted,
                           const void* weight_sorted, int64_t rows_cap, int64_t tile, int32_t* seg_expert,
                           int32_t* seg_row0, int32_t* seg_rows, int64_t max_segs, int32_t* num_segs,
                           int32_t* num_rows, int32_t* row_expert, int64_t* row_token, void* row_weight,
                           int32_t* scratch, hipStream_t stream);
int mi355moe_e3_gather(const void* x, int x_dtype, int64_t x_stride, int64_t tokens, int64_t K,
                       const int64_t* row_token, const int32_t* row_expert, int64_t rows_cap, int64_t n,
                       const int64_t* suh_table, void* h13, const int32_t* num_rows, hipStream_t stream);
int mi355moe_e3_gateup(const void* h13, int64_t rows_cap, int64_t K, int64_t N, int64_t n,
                       const int64_t* gate_trellis, const int64_t* up_trellis, const int64_t* gate_svh,
                       const int64_t* up_svh, const int64_t* down_suh, void* h2, const int32_t* seg_expert,
                       const int32_t* seg_row0, const int32_t* seg_rows, int64_t seg_cap, const int32_t* num_segs,
                       float act_limit, hipStream_t stream);
int64_t mi355moe_e3_down_workspace_bytes(int64_t rows_cap, int64_t K, int64_t tokens);
int mi355moe_e3_down(const void* h2, int64_t rows_cap, int64_t K, int64_t N, int64_t n, const int64_t* down_trellis,
                     const int64_t* down_svh, float* out, int64_t tokens, int64_t out_stride,
                     const int64_t* row_token, const void* row_weight, const int32_t* seg_expert,
                     const int32_t* seg_row0, const int32_t* seg_rows, int64_t seg_cap, const int32_t* num_segs,
                     void* workspace, size_t workspace_bytes, hipStream_t stream);

/* ---------------------------------------------------------------- the e4m3 extension's stages over row tables */

/* The stage contract of the e4m3 extension that the overlay's run() drives (code/fork/overlay/glm53_moe_e4m3.py:
 * 450-592; bindings code/fork/kernels/moe_e4m3.cu:3081-3096), with the trellis-sourced e4m3 numerics of
 * mi355moe_e4m3_moe_forward_ids. The stages exchange caller-owned buffers in the extension's formats:
 *   a8  uint8 [rows][K] and a8d uint8 [rows][N]: one e4m3 (OCP E4M3FN) code per element, the columns of every group
 *       of 16 stored in the order 0,1,8,9,2,3,10,11,4,5,12,13,6,7,14,15 (the extension's perm_pos / perm_cols
 *       layout, moe_e4m3.cu:18-21,150-156); asc / dsc fp32 [rows]: the rows' scales (q * s is the value);
 *   a16 fp16 [rows][N]: the SwiGLU output in plain column order;
 * and the row / segment tables of seg_tables (rows grouped by expert, segments of at most `tile` rows) with the live
 * counts num_segs / num_rows as int32 [1] device words (read by the kernels: no host synchronisation). Every buffer
 * pointer must be 16-byte aligned. K (hidden) <= 4096, N (intermediate) <= 4096, multiples of 256 and 128.
 *
 * seg_tables (moe_e4m3.cu:3062-3083): counts int64 [n], max_segs >= ceil(rows_cap / tile) + n, 16 <= tile <=
 *   mi355moe_e4m3_tile_rows() (the GEMMs take segments of at most that many rows).
 * gather2 (moe_e4m3.cu:2493-2534): routed pair j = (token j / topk, slot j % topk) with local expert local[j] (skipped
 *   unless 0 <= local[j] < n) writes a8 row pos[j] (pos[j] < a8_rows) and asc[pos[j]]: v = H(fp16(x) * suh) * r in
 *   fp32, s = amax|v| / 448 (1 if 0), q = e4m3(clamp(v / s)). A non-null out (fp32 or bf16 [T][out_stride]) is zeroed.
 * gather_tok (moe_e4m3.cu:2536-2571): the same quantisation for one row per token with the suh of expert 0 (valid
 *   when every expert shares its w13 suh): a8 row t, asc[t] for t < T <= a8_rows; out zeroed if non-null.
 * gateup (moe_e4m3.cu:2641-2676): a16 rows of the segments of chunk `chunk` of `nchunks` (equal shares of the
 *   num_segs segments) = fp16(silu(min(g, L)) * clamp(u, -L, L)) (the limit iff L != 0), g = H(acc_g * s) * r * svh_g,
 *   acc_g = the a8 row's codes times the gate weights rounded to e4m3, summed in fp32; u likewise.
 * actq (moe_e4m3.cu:2573-2600): the rows of the chunk's segments: v = H(float(a16) * suh_d[row_expert[r]]) * r,
 *   quantised as in gather2 into a8d row r and dsc[r].
 * down (moe_e4m3.cu:2678-2719): every token's rows of the chunk's segments, (H(acc_d * dsc) * r) * svh_d * row_weight,
 *   ADDED to out fp32 [tokens][out_stride] in row order (deterministic; at most 32 rows per token).
 * fused (moe_e4m3.cu:2721-2725): gateup, actq and down of every segment in one call, out fp32 or bf16 ADDED to.
 *   a8d / dsc (both or neither) and a16 receive the intermediates when non-null. variant bits:
 *   MI355MOE_E4M3_TOKEN_ROWS: a8 / asc hold one row per token (gather_tok) and row r reads row row_token[r];
 *   MI355MOE_E4M3_DOWN16: the down projection on fp16 operands (h = fp16(H(float(a16) * suh_d) * r) times the
 *   fp16 W_q, the extension's variant 16, spec_proj16 at glm53_moe_e4m3.py:660-664); a8d / dsc are not written;
 *   MI355MOE_E4M3_LEAN_MAINLOOP (the extension's +8192 schedule variant): accepted, same results.
 *   mi355moe_e4m3_fused runs gate/up and down as one ticket-ordered launch (MI355MOE_OPT_PERSISTENT's schedule) by
 *   itself where that choice applies (DOWN16, or the 64-row tiles) and seg_cap <= rows_cap; the lag comes from
 *   MI355MOE_SCHED_LAG. The reference's per-call lag / grid / sync arguments have no counterpart.
 * The stages that take a workspace share one size, mi355moe_e4m3_stage_workspace_bytes(rows_cap, K, N, tokens). */
enum { MI355MOE_E4M3_DOWN16 = 16, MI355MOE_E4M3_TOKEN_ROWS = 2048, MI355MOE_E4M3_LEAN_MAINLOOP = 8192 };
int64_t mi355moe_e4m3_tile_rows(void);
int mi355moe_e4m3_seg_tables(const int64_t* counts, int64_t n, int64_t tile, int64_t rows_cap, int32_t* seg_expert,
                             int32_t* seg_row0, int32_t* seg_rows, int64_t max_segs, int32_t* num_segs,
                             int32_t* num_rows, hipStream_t stream);
int mi355moe_e4m3_gather2(const void* x, int x_dtype, int64_t x_stride, int64_t T, int64_t K, const int32_t* local,
                          const int32_t* pos, int64_t topk, int64_t n, const int64_t* gate_suh, uint8_t* a8,
                          int64_t a8_rows, float* asc, void* out, int out_dtype, int64_t out_stride,
                          hipStream_t stream);
int mi355moe_e4m3_gather_tok(const void* x, int x_dtype, int64_t x_stride, int64_t T, int64_t K,
                             const int64_t* gate_suh, uint8_t* a8, int64_t a8_rows, float* asc, void* out,
                             int out_dtype, int64_t out_stride, hipStream_t stream);
int64_t mi355moe_e4m3_stage_workspace_bytes(int64_t rows_cap, int64_t K, int64_t N, int64_t tokens);
int mi355moe_e4m3_gateup(const uint8_t* a8, const float* asc, int64_t rows_cap, int64_t K, int64_t N, int64_t n,
                         const int64_t* gate_trellis, const int64_t* up_trellis, const int64_t* gate_svh,
                         const int64_t* up_svh, void* a16, const int32_t* seg_expert, const int32_t* seg_row0,
                         const int32_t* seg_rows, int64_t seg_cap, const int32_t* num_segs, float limit, int64_t chunk,
                         int64_t nchunks, void* workspace, size_t workspace_bytes, hipStream_t stream);
int mi355moe_e4m3_actq(const void* a16, int64_t rows_cap, int64_t N, const int32_t* row_expert, int64_t n,
                       const int64_t* down_suh, uint8_t* a8d, float* dsc, const int32_t* seg_row0,
                       const int32_t* seg_rows, int64_t seg_cap, const int32_t* num_segs, int64_t chunk,
                       int64_t nchunks, void* workspace, size_t workspace_bytes, hipStream_t stream);
int mi355moe_e4m3_down(const uint8_t* a8d, const float* dsc, int64_t rows_cap, int64_t K, int64_t N, int64_t n,
                       const int64_t* down_trellis, const int64_t* down_svh, float* out, int64_t tokens,
                       int64_t out_stride, const int64_t* row_token, const float* row_weight,
                       const int32_t* seg_expert, const int32_t* seg_row0, const int32_t* seg_rows, int64_t seg_cap,
                       const int32_t* num_segs, int64_t chunk, int64_t nchunks, void* workspace,
                       size_t workspace_bytes, hipStream_t stream);
int mi355moe_e4m3_fused(const uint8_t* a8, const float* asc, int64_t a8_rows, uint8_t* a8d, float* dsc, void* a16,
                        void* out, int out_dtype, int64_t tokens, int64_t out_stride, int64_t K, int64_t N, int64_t n,
                        const int64_t* gate_trellis, const int64_t* up_trellis, const int64_t* gate_svh,
                        const int64_t* up_svh, const int64_t* down_trellis, const int64_t* down_suh,
                        const int64_t* down_svh, const int64_t* row_token, const float* row_weight, int64_t rows_cap,
                        const int32_t* seg_expert, const int32_t* seg_row0, const int32_t* seg_rows, int64_t seg_cap,
                        const int32_t* num_segs, float limit, int variant, void* workspace, size_t workspace_bytes,
                        hipStream_t stream);

/* ---------------------------------------------------------------- e4m3 expert variant */

/* One layer of block-scaled e4m3 routed experts in vLLM's fp8 w8a8 block-quantised MoE layout (128x128 blocks):
 * the weight the GEMM sees is e4m3(w) * scale[block]. */
typedef struct mi355moe_fp8_layer {
    int64_t n, hidden, intermediate;
    const void* w13;        /* e4m3 [n][2*intermediate][hidden]: rows 0..I-1 gate, I..2I-1 up */
    const float* w13_scale; /* [n][2*intermediate/128][hidden/128] */
    const void* w2;         /* e4m3 [n][hidden][intermediate] */
    const float* w2_scale;  /* [n][hidden/128][intermediate/128] */
} mi355moe_fp8_layer;

/* Per-row dynamic e4m3 quantisation: s[r] = amax(|x[r]|) / 448 (1 if 0), q[r] = e4m3_rn(clamp(x[r] / s[r],
 * -448, 448)), IEEE divisions. Replaces the reference's activation quantisers gather_tok / actq
 * (code/fork/kernels/moe_e4m3.cu:152-176, :245-310, :440-488; spec glm53_moe_e4m3.py:648-652). x: F32, F16 or
 * BF16 [rows][x_stride]; q uint8 [rows][K]; K % 4 == 0. */
int mi355moe_fp8_quant_rows(const void* x, int x_dtype, int64_t rows, int64_t K, int64_t x_stride, void* q,
                            float* scale, hipStream_t stream);

/* Routed-expert output of a block-scaled e4m3 layer from router ids and weights (the e4m3 expert path,
 * code/fork/overlay/glm53_moe_e4m3.py:484-592 -> moe_e4m3.cu fused, :3081-3096): activations quantised per
 * token, SwiGLU a16 = fp16(silu(min(g, L)) * clamp(u, -L, L)) (iff L != 0), a16 requantised per row, down GEMM,
 * per-pair contributions w * y summed per token in slot order (fp32, deterministic), out WRITTEN in out_dtype
 * (out_stride even). hidden % 256 == 0, intermediate % 128 == 0, both <= 16384;
 * T * topk <= 65536.
 * stages: the MI355MOE_STAGE_* mask (ROUTE = permutation and input quantisation, GATEUP, DOWN = requantisation and
 * down GEMM, COMBINE = the slot-order sum into out). */
int64_t mi355moe_fp8_moe_workspace_bytes(const mi355moe_fp8_layer* layer, int64_t T, int64_t topk);
int mi355moe_fp8_moe_forward_ids(const mi355moe_fp8_layer* layer, const void* x, int x_dtype, int64_t x_stride,
                                 int64_t T, const void* ids, int ids_dtype, const void* weights, int weights_dtype,
                                 int64_t topk, const int64_t* expert_map, int64_t n_global, float limit, void* out,
                                 int out_dtype, int64_t out_stride, void* workspace, size_t workspace_bytes,
                                 int stages, hipStream_t stream);

/* The trellis-sourced e4m3 variant of the EXL3 experts (code/fork/overlay/glm53_moe_e4m3.py:484-592 run() over a
 * layer's EXL3 pointer tables; numerics spec_proj / spec_ffn, :654-674, DOWN16 off; kernels
 * code/fork/kernels/moe_e4m3.cu gather2 :245-310 and the fused GEMMs :576-1856): per pair row v = H(fp16(x) * suh)
 * * r in fp32, s = amax|v| / 448 (1 if 0), q = e4m3(clamp(v / s)); the gate and up GEMMs multiply q by the decoded
 * weights rounded to e4m3 (W_q of the 4-bit trellis) with fp32 sums, g = H(acc * s) * r * svh (same for u),
 * a16 = fp16(silu(min(g, L)) * clamp(u, -L, L)) (iff L != 0), the down input H(a16 * suh_d) * r quantized per row
 * the same way, the down GEMM likewise, y = H(acc * s_d) * r * svh_d, out[t] = sum over the token's slots of w * y
 * in slot order (fp32, deterministic), WRITTEN in out_dtype. Arguments and stages as mi355moe_moe_forward_ids_ex
 * (grouped 256-row tiles whatever T); the layer needs MI355MOE_LAYER_SHARED_W13_SUH (one quantized copy of the
 * input rows) and hidden <= 4096. */
int64_t mi355moe_e4m3_moe_workspace_bytes(const mi355moe_exl3_layer* layer, int64_t T, int64_t topk);
int mi355moe_e4m3_moe_forward_ids(const mi355moe_exl3_layer* layer, const void* x, int x_dtype, int64_t x_stride,
                                  int64_t T, const void* ids, int ids_dtype, const void* weights, int weights_dtype,
                                  int64_t topk, const int64_t* expert_map, int64_t n_global, float limit, void* out,
                                  int out_dtype, int64_t out_stride, void* workspace, size_t workspace_bytes,
                                  int stages, hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* MI355MOE_H */
