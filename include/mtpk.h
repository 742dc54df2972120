/* libmtpk — MI355X (gfx950) kernels for the MTP speculative-decode step: MXFP4 routed-expert
 * MoE, fused router top-k, argmax, greedy / rejection acceptance with rollback indices.
 *
 * C ABI: plain device pointers, element counts and a HIP stream handle (hipStream_t passed as
 * void*; NULL = the default stream). The caller owns every buffer; no entry point allocates or
 * synchronises, and the launch shape of each depends only on its size arguments, so every
 * call can be captured into a HIP graph. Return value: 0 on success, MTPK_EINVAL / MTPK_ENODEV
 * for a rejected call (nothing launched), or a positive hipError_t reported by the launch.
 * Reference paths below point into the reference engine's repository.
 */
#ifndef MTPK_H
#define MTPK_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MTPK_OK 0
#define MTPK_EINVAL (-1) /* argument outside the contract: shape, dtype, alignment, null */
#define MTPK_ENODEV (-2) /* no usable HIP device */
#define MTPK_ETOOBIG (-3) /* the call needs more scratch than the library's static buffer holds */

/* Element type codes used by the dtype arguments. */
#define MTPK_F32 0
#define MTPK_BF16 1
#define MTPK_I32 2
#define MTPK_I64 3
#define MTPK_U8 4

#define MTPK_MAX_EXPERTS 4096 /* local experts one MoE call may address */
#define MTPK_MAX_TOP_K 32     /* router_fused.MAX_TOP_K (router_fused.py:37) */
#define MTPK_MAX_ROUTER_EXPERTS 1024
#define MTPK_MOE_UNIT_TOKENS 16 /* token columns per MoE work unit (one MFMA N tile) */

/* Human-readable text for a status code (static storage). */
const char* mtpk_status_string(int status);

/* ABI revision of this header; bumped on any signature change. The library returns the value
 * it was built with, and the Python binding refuses a library whose value differs. */
#define MTPK_ABI_VERSION 4
int mtpk_abi_version(void);

/* ---------------------------------------------------------------- MXFP4 dequant
 * Replaces `mxfp4.dequant_mxfp4` (mxfp4.py:32-51) for device tensors; the in-kernel decode it
 * exposes is the one `mxfp4_gemv._dequant_tile`/`_e8m0` define (mxfp4_gemv.py:335-382).
 * packed u8 [rows, k/2] (low nibble = even element), scale u8 [rows, k/32] (e8m0) ->
 * out f32 [rows, k]. k % 32 == 0.
 * mode 0: exact fp32, fp4 * 2^(s-127), scale byte 0 -> +0.0, 255 -> +inf.
 * mode 1: the MoE kernels' in-register decode (hardware fp4 -> bf16 convert with the block
 *         scale folded in, `decode8`), widened to fp32; equal to mode 0 bit for bit for scale
 *         bytes 0..254 (byte 0 as +-0.0); byte 255 gives NaN for every code. */
int mtpk_dequant_mxfp4(const uint8_t* packed, const uint8_t* scale, int64_t rows, int64_t k,
                       int mode, float* out, void* stream);

/* Load-time precondition of the in-register decode: replaces `mxfp4_gemv.bw_scales_ok` /
 * `moe_hip.supports` (mxfp4_gemv.py:1761-1776, moe_hip.py:204-215). Counts, into *bad_count
 * (device int32, cleared by the call), the threads that found a 32-element block whose e8m0
 * scale is 255 and whose 16 packed bytes hold a nonzero-magnitude code: the one case where the
 * hardware convert (NaN) differs from the pinned decode (+-inf). Block b is packed bytes
 * [16 b, 16 b + 16) and scale byte b, so a whole [E, N, K/2] / [E, N, K/32] pair is scanned
 * as blocks = E * N * K / 32. Zero means every block decodes exactly. */
int mtpk_scale_scan(const uint8_t* packed, const uint8_t* scale, int64_t blocks,
                    int32_t* bad_count, void* stream);

/* ---------------------------------------------------------------- routed MXFP4 MoE
 * Weights in the `load_experts` layout (model.py:758-804): gate_up u8 [E, 2I, H/2] (rows
 * 0..I-1 gate, I..2I-1 up), gate_up_scale u8 [E, 2I, H/32], down u8 [E, H, I/2],
 * down_scale u8 [E, H, I/32]; E = expert_hi - expert_lo local experts. Routing is the flat
 * `(a_expert, a_weight)` of `_routed_fused` (model.py:3096-3100): assignment a = t*top_k + j,
 * a_expert int32|int64 global ids, a_weight f32|bf16. An assignment is live iff
 * expert_lo <= a_expert < expert_hi and a_weight != 0 (mxfp4_gemv.py:472-474); dead ones are
 * dropped on the GPU. x and out are bf16 or f32 [T, H] (row-major, contiguous). */

/* Upper bound on work units for `assignments` over `local_experts` (units of at most
 * MTPK_MOE_UNIT_TOKENS assignments of one expert). */
int64_t mtpk_moe_max_units(int64_t assignments, int64_t local_experts);

/* Bytes of workspace `mtpk_fused_moe` needs for these sizes (x_dtype = MTPK_BF16|MTPK_F32). */
int64_t mtpk_moe_workspace_bytes(int64_t tokens, int64_t top_k, int64_t local_experts,
                                 int64_t inter, int64_t hidden, int x_dtype);

/* Work-list build: replaces `mxfp4_gemv.bw_prep`/`_bw_prep_kernel` (mxfp4_gemv.py:1962-2029,
 * :2320-2376) and `moe_hip.prep` (moe_hip.py:268-285). Counting sort of live assignments by
 * local expert into sorted i32 [assignments] (expert-grouped; order inside one expert's run
 * is unspecified), units i32 [3*max_units] = (local expert, first position in sorted,
 * count <= MTPK_MOE_UNIT_TOKENS), n_units i32 [1]. One workgroup. max_units below
 * mtpk_moe_max_units(assignments, expert_hi - expert_lo) is MTPK_EINVAL (a shorter list would
 * drop live assignments); the same bound holds for `mtpk_moe_gate_up` and `mtpk_moe_down`. */
int mtpk_moe_prep(const void* a_expert, int expert_dtype, const void* a_weight, int weight_dtype,
                  int64_t assignments, int expert_lo, int expert_hi, int32_t* sorted,
                  int32_t* units, int64_t max_units, int32_t* n_units, void* stream);

/* gate_up + SiLU: replaces `_gate_up_silu_kernel` (mxfp4_gemv.py:441-493) and the C ABI
 * `moe_hip_gate_up` (moe_hip.hip:403-421). inter[a, n] = silu(gate_e[n].x_t) * (up_e[n].x_t)
 * for every live assignment a, written as `inter_planes` bf16 planes of [assignments, I]
 * (plane p at inter + p*assignments*I) whose sum is the fp32 value: 2 planes for bf16 x,
 * 3 for f32 x. `x_planes` holds x as bf16 planes [x_nplanes, T, H] (1 plane for bf16 x; f32 x
 * is first split by `mtpk_split_planes`). */
int mtpk_moe_gate_up(const uint16_t* x_planes, int x_nplanes, int64_t tokens, int64_t hidden,
                     const uint8_t* gate_up, const uint8_t* gate_up_scale, int64_t local_experts,
                     int64_t inter_dim, const int32_t* sorted, const int32_t* units,
                     const int32_t* n_units, int64_t max_units, int top_k, uint16_t* inter,
                     int inter_planes, int64_t assignments, void* stream);

/* down: replaces the projection half of `_down_combine_kernel` (mxfp4_gemv.py:496-542) and
 * `moe_hip_down` (moe_hip.hip:403-452). y f32 [assignments, H] = down_e . inter[a] for every
 * live assignment (rows of dead assignments are not written). */
int mtpk_moe_down(const uint16_t* inter, int inter_planes, int64_t assignments, int64_t inter_dim,
                  const uint8_t* down, const uint8_t* down_scale, int64_t local_experts,
                  int64_t hidden, const int32_t* sorted, const int32_t* units,
                  const int32_t* n_units, int64_t max_units, float* y, void* stream);

/* Largest token count `mtpk_fused_moe` serves with the direct pipeline below (no prep, no y,
 * no separate combine); wider batches take prep -> gate_up -> down -> combine. */
int mtpk_moe_direct_max_tokens(void);

/* gate_up + SiLU with one work unit per assignment, read straight from the routing (the
 * per-assignment form of `_gate_up_silu_kernel`, mxfp4_gemv.py:441-493, including its in-kernel
 * drop of unowned / zero-weight assignments at :472-474). Same output as `mtpk_moe_gate_up`;
 * inter planes are [tokens*top_k, I]. */
int mtpk_moe_gate_up_direct(const uint16_t* x_planes, int x_nplanes, int64_t tokens,
                            int64_t hidden, const uint8_t* gate_up, const uint8_t* gate_up_scale,
                            int64_t local_experts, int64_t inter_dim, const void* a_expert,
                            int expert_dtype, const void* a_weight, int weight_dtype, int top_k,
                            int expert_lo, int expert_hi, uint16_t* inter, int inter_planes,
                            void* stream);

/* down + weighted combine per token: replaces `_down_combine_kernel` (mxfp4_gemv.py:496-542).
 * out[t] = sum over t's live assignments of a_weight * (down_e . inter[a]), no atomics and no
 * dependence on scheduling; tokens with no live assignment get exact zeros. */
int mtpk_moe_down_combine(const uint16_t* inter, int inter_planes, int64_t inter_dim,
                          const uint8_t* down, const uint8_t* down_scale, int64_t local_experts,
                          int64_t hidden, const void* a_expert, int expert_dtype,
                          const void* a_weight, int weight_dtype, int64_t tokens, int top_k,
                          int expert_lo, int expert_hi, void* out, int out_dtype, void* stream);

/* Combine: replaces `bw_combine` / `_dedup_combine_kernel` (mxfp4_gemv.py:1187-1211,
 * :2240-2264). out[t, n] = sum_{j=0..top_k-1, live} a_weight[a] * y[a, n], in that fixed j
 * order (no atomics, bit-reproducible); tokens with no live assignment get exact zeros. */
int mtpk_moe_combine(const float* y, const void* a_expert, int expert_dtype, const void* a_weight,
                     int weight_dtype, int64_t tokens, int top_k, int64_t hidden, int expert_lo,
                     int expert_hi, void* out, int out_dtype, void* stream);

/* Combine of rows that already carry their routing weight: replaces `bw_combine` and
 * `bw_combine_glue` (mxfp4_gemv.py:2440-2488, kernels :2240-2312), whose y comes from a down
 * projection that applies the weight in its epilogue (moe_hip.hip:401, mxfp4_gemv.py:2232-2236).
 * out[t, n] = sum over t's live assignments (expert in [expert_lo, expert_hi) and a_weight != 0;
 * dead rows of y are never read, so y needs no zero fill) of y[t*top_k + j, n], in j order, in
 * f32; tokens with none get zeros. y f32 (16-byte aligned) or bf16 (8-byte aligned)
 * [tokens*top_k, hidden], hidden % 4 == 0. With shared != NULL the shared expert's term is
 * added as in mtpk_fused_moe_shared (routed sum, sigmoid(shared_gate[t * gate_stride]) and the
 * product each rounded to out_dtype, then the add); shared = NULL is `bw_combine`. */
int mtpk_moe_combine_rows(const void* y, int y_dtype, const void* a_expert, int expert_dtype,
                          const void* a_weight, int weight_dtype, int64_t tokens, int top_k,
                          int64_t hidden, int expert_lo, int expert_hi, const void* shared,
                          int shared_dtype, const void* shared_gate, int gate_dtype,
                          int64_t gate_stride, void* out, int out_dtype, void* stream);

/* f32 [n] -> `nplanes` bf16 planes [nplanes, n] whose sum is the input (2 planes: 16
 * significant bits; 3 planes: all 24). */
int mtpk_split_planes(const float* src, int64_t n, int nplanes, uint16_t* planes, void* stream);

/* The whole routed MoE in one call (prep, gate_up, down, combine, and the f32 split when
 * x is f32): the drop-in for `mxfp4_gemv.fused_moe` (mxfp4_gemv.py:1020-1122) and
 * `moe_hip.fused_moe_hip` (moe_hip.py:357-409). x_dtype = out_dtype = MTPK_BF16 | MTPK_F32.
 * workspace must hold mtpk_moe_workspace_bytes(...) bytes, 256-byte aligned. */
int mtpk_fused_moe(const void* x, int x_dtype, int64_t tokens, int64_t hidden,
                   const uint8_t* gate_up, const uint8_t* gate_up_scale, const uint8_t* down,
                   const uint8_t* down_scale, int64_t local_experts, int64_t inter_dim,
                   const void* a_expert, int expert_dtype, const void* a_weight, int weight_dtype,
                   int top_k, int expert_lo, int expert_hi, void* workspace,
                   int64_t workspace_bytes, void* out, void* stream);

/* ---------------------------------------------------------------- routed bf16 experts
 * The MTP draft layer's routed experts in the real checkpoint, which are dense bf16 while the
 * target layers' are MXFP4: replaces `mtp_dense_moe.grouped_moe` / `fused_moe`
 * (mtp_dense_moe.py:359-745). Same contract as mtpk_fused_moe with bf16 weights: gate_up
 * bf16 [local_experts, 2 I, H] (gate rows, then up rows), down bf16 [local_experts, H, I], x
 * bf16 [tokens, H] contiguous, a_expert / a_weight [tokens * top_k] (live: expert in
 * [expert_lo, expert_hi) and weight != 0), out bf16 [tokens, H] = sum over a token's live
 * assignments in j order of w * down(silu(gate x) * (up x)); tokens with none get zeros.
 * fp32 accumulation; the intermediate is kept as two bf16 planes (16 significant bits).
 * H and I multiples of 256, one expert's gate_up < 2^31 bytes. workspace: 256-byte aligned,
 * mtpk_moe_dense_workspace_bytes(...) bytes. */
int64_t mtpk_moe_dense_workspace_bytes(int64_t tokens, int64_t top_k, int64_t local_experts,
                                       int64_t inter, int64_t hidden);
int mtpk_moe_dense(const uint16_t* x, int64_t tokens, int64_t hidden, const uint16_t* gate_up,
                   const uint16_t* down, int64_t local_experts, int64_t inter_dim,
                   const void* a_expert, int expert_dtype, const void* a_weight, int weight_dtype,
                   int top_k, int expert_lo, int expert_hi, void* workspace,
                   int64_t workspace_bytes, uint16_t* out, void* stream);

/* mtpk_fused_moe plus the shared expert's term of the layer (`Model.moe`, model.py:2871-2872;
 * the reference's `bw_combine_glue`, mxfp4_gemv.py:2266-2312): out = routed + sigmoid(g_t) *
 * shared[t], with g_t = shared_gate[t * gate_stride] (the shared-gate column of the router
 * GEMM output) and shared [tokens, hidden] of shared_dtype. The routed sum, the sigmoid and the
 * product are each rounded to the output dtype before the add, as the unfused torch ops round
 * them, so both spellings give the same values. shared = NULL is mtpk_fused_moe. */
int mtpk_fused_moe_shared(const void* x, int x_dtype, int64_t tokens, int64_t hidden,
                          const uint8_t* gate_up, const uint8_t* gate_up_scale, const uint8_t* down,
                          const uint8_t* down_scale, int64_t local_experts, int64_t inter_dim,
                          const void* a_expert, int expert_dtype, const void* a_weight,
                          int weight_dtype, int top_k, int expert_lo, int expert_hi,
                          const void* shared, int shared_dtype, const void* shared_gate,
                          int gate_dtype, int64_t gate_stride, void* workspace,
                          int64_t workspace_bytes, void* out, void* stream);

/* `mtpk_fused_moe_shared` without a workspace argument: its scratch (work list, intermediate
 * planes, y) is the library's own file-scope device buffer of MTPK_MOE_STATIC_SCRATCH bytes, one
 * per GPU, held until the process ends. Nothing is allocated, so the call suits code that cannot
 * call hipMalloc (HIP graph capture, serving loops, harnesses that forbid allocation). No
 * counterpart in the reference: it exists for those callers. A call whose
 * mtpk_moe_workspace_bytes(...) exceeds the buffer returns MTPK_ETOOBIG and launches nothing
 * (bf16 activations at H = 4096, I = 1024, top-10 of 512 fit up to 256 tokens). Every call on a
 * GPU shares that GPU's buffer, which keeps the last call's contents (no call needs it cleared):
 * calls that overlap on one GPU (different streams or host threads) race. The other arguments
 * and the result are those of mtpk_fused_moe_shared. */
#define MTPK_MOE_STATIC_SCRATCH (64LL << 20)
int mtpk_fused_moe_static(const void* x, int x_dtype, int64_t tokens, int64_t hidden,
                          const uint8_t* gate_up, const uint8_t* gate_up_scale, const uint8_t* down,
                          const uint8_t* down_scale, int64_t local_experts, int64_t inter_dim,
                          const void* a_expert, int expert_dtype, const void* a_weight,
                          int weight_dtype, int top_k, int expert_lo, int expert_hi,
                          const void* shared, int shared_dtype, const void* shared_gate,
                          int gate_dtype, int64_t gate_stride, void* out, void* stream);

/* ---------------------------------------------------------------- whole MoE layer
 * Replaces the body of `Model.moe` (model.py:2800-2873): router GEMM (`router_gate`, the experts'
 * rows then the shared gate's row, as `fuse_moe_dense` concatenates them, model.py:913-928),
 * softmax top-k renormalised, routed MXFP4 experts, shared expert `swiglu_mlp` (model.py:638-649),
 * out = routed + sigmoid(shared gate) * shared with the rounding points of the torch chain
 * (`bw_combine_glue`, mxfp4_gemv.py:2266-2312). The router and the shared expert run inside the
 * routed layer's launches: (1) router + shared gate/up GEMM tiles, (2) top-k + the shared SiLU
 * product, (3) the shared down GEMM tiles beside the routed gate_up (tokens <= 4) or the work-list
 * prep, (4) routed down (+ combine). h, router_gate [router_rows, hidden], shared_gate_up
 * [2 shared_inter, hidden] and shared_down [hidden, shared_inter] are bf16; out bf16
 * [tokens, hidden]; tokens <= 256; hidden and shared_inter multiples of 256. top_w f32 /
 * top_i i32 [tokens, top_k] receive the routing when not null (else it stays in the workspace).
 * workspace: mtpk_moe_layer_workspace_bytes(...) bytes, 256-byte aligned. */
int64_t mtpk_moe_layer_workspace_bytes(int64_t tokens, int64_t hidden, int64_t router_rows,
                                       int64_t shared_inter, int top_k, int64_t local_experts,
                                       int64_t inter_dim);
int mtpk_moe_layer(const uint16_t* h, int64_t tokens, int64_t hidden, const uint16_t* router_gate,
                   int64_t router_rows, const uint16_t* shared_gate_up,
                   const uint16_t* shared_down, int64_t shared_inter, const uint8_t* gate_up,
                   const uint8_t* gate_up_scale, const uint8_t* down, const uint8_t* down_scale,
                   int64_t local_experts, int64_t inter_dim, int top_k, int expert_lo,
                   int expert_hi, float* top_w, int32_t* top_i, void* workspace,
                   int64_t workspace_bytes, void* out, void* stream);

/* mtpk_moe_layer followed by the residual form of the next RMSNorm, fused into the layer's last
 * launch (the `x, h = add_rmsnorm(x, moe_out, w)` that starts the next decoder layer, or the
 * final norm; model.py:587-604 with its residual add): sum_out = bf16(residual + out) and
 * normed_out = sum_out * rsqrt(mean(sum_out^2) + eps) * (1 + norm_w), bf16 [tokens, hidden],
 * each equal to mtpk_moe_layer's out followed by mtpk_rownorm's residual form bit for bit; the
 * layer output itself is not stored. tokens > mtpk_moe_direct_max_tokens() (the work-unit path)
 * and hidden 2048 or 4096; otherwise MTPK_EINVAL. */
int mtpk_moe_layer_add_norm(const uint16_t* h, int64_t tokens, int64_t hidden,
                            const uint16_t* router_gate, int64_t router_rows,
                            const uint16_t* shared_gate_up, const uint16_t* shared_down,
                            int64_t shared_inter, const uint8_t* gate_up,
                            const uint8_t* gate_up_scale, const uint8_t* down,
                            const uint8_t* down_scale, int64_t local_experts, int64_t inter_dim,
                            int top_k, int expert_lo, int expert_hi, float* top_w, int32_t* top_i,
                            void* workspace, int64_t workspace_bytes, const uint16_t* residual,
                            const uint16_t* norm_w, float eps, uint16_t* sum_out,
                            uint16_t* normed_out, void* stream);
/* 1 when `mtpk_moe_layer` accepts these operands (given a large enough workspace), else 0: the
 * same checks, run without a launch and without dereferencing a pointer (pointers are tested
 * for null and 16-byte alignment only). Lets a caller choose the unfused launches up front, as
 * `Model.moe` chooses between `fuse_moe_dense` and the separate ops (model.py:913-928). */
int mtpk_moe_layer_supported(const void* h, int64_t tokens, int64_t hidden, const void* router_gate,
                             int64_t router_rows, const void* shared_gate_up,
                             const void* shared_down, int64_t shared_inter, const void* gate_up,
                             const void* gate_up_scale, const void* down, const void* down_scale,
                             int64_t local_experts, int64_t inter_dim, int top_k, int expert_lo,
                             int expert_hi);

/* ---------------------------------------------------------------- router top-k
 * Replaces `router_fused.route` / `_fused_route_kernel` (router_fused.py:56-151) and the torch
 * chain in `Model.moe` (model.py:2840-2843). routing [tokens, >= experts_out] f32|bf16 with
 * row stride `row_stride` elements; softmax (fp32) over the first experts_out columns,
 * top_k largest (ties: lower expert index first), renormalised to sum 1.
 * top_w f32 [tokens, top_k], top_i i32|i64 [tokens, top_k], highest weight first. */
int mtpk_route_topk(const void* routing, int routing_dtype, int64_t tokens, int64_t row_stride,
                    int experts_out, int top_k, float* top_w, void* top_i, int index_dtype,
                    void* stream);

/* ---------------------------------------------------------------- argmax
 * Replaces `logits.argmax(-1)` of the verify step (graph_mtp.py:539-540) and of
 * `mtp.greedy_token` (mtp.py:640-658). logits f32|bf16 [rows, vocab] with row stride
 * `row_stride` elements; out_index i64 [rows] = first index of the row maximum (-0.0 ties
 * +0.0). `partials` is u64 scratch of mtpk_argmax_partials(rows, vocab) entries. */
int64_t mtpk_argmax_partials(int64_t rows, int64_t vocab);
int mtpk_argmax_rows(const void* logits, int dtype, int64_t rows, int64_t vocab,
                     int64_t row_stride, uint64_t* partials, int64_t* out_index, void* stream);

/* ---------------------------------------------------------------- greedy acceptance
 * Replaces `_accept_len` + `_commit_limit` + `_fixed_prefix_pack_index` (graph_mtp.py:440-474),
 * the accept-length tail of `verify_round_step` (graph_mtp.py:541-580) and
 * `LaneTables.update` (mtp_overlap.py:53-71), for B <= 1024 rows and t = k + 1 columns.
 * Inputs: step_argmax i64 [B, t] (row stride sa_stride), draft i64 [B, k] (row stride
 * draft_stride, e.g. token_matrix[:, 1:]), active u8 [B], pos i64 [B], budget i64 [B],
 * stops i64 [B, n_stops] padded with -1, conv_k1 = conv kernel width - 1.
 * forced_n i64 [B] (may be NULL): a row with forced_n > 0 accepts exactly min(forced_n, k)
 * drafts, unclamped by stops and budget, and its budget_left is budget - 1 (the forced
 * override of graph_verify_wide.py:196-200 and LaneTables.update, mtp_overlap.py:53-71).
 * Outputs (any may be NULL except accept_len):
 *   accept_len i64 [B]  commit-limited accept length a
 *   lengths i64 [B]     a + 1 on active rows, 1 on padding rows
 *   packed_src i64 [B*t], packed_cu i32 [B+1]   fixed-size prefix-pack gather map
 *   conv_idx i64 [B, conv_k1]   min(lengths + w, conv_k1 + t - 1)
 *   keep u8 [B, t]      active && s <= a
 *   bonus i64 [B]       step_argmax[j, a]
 *   next_pos i64 [B], budget_left i64 [B], live u8 [B]   lane-table update values
 *   hidden_src i64 [B]  j*t + a, the verify row whose hidden state seeds the next draft */
int mtpk_greedy_accept(const int64_t* step_argmax, int64_t sa_stride, const int64_t* draft,
                       int64_t draft_stride, const uint8_t* active, const int64_t* pos,
                       const int64_t* budget, const int64_t* stops, int n_stops,
                       const int64_t* forced_n, int batch, int t, int conv_k1, int64_t* accept_len, int64_t* lengths, int64_t* packed_src,
                       int32_t* packed_cu, int64_t* conv_idx, uint8_t* keep, int64_t* bonus,
                       int64_t* next_pos, int64_t* budget_left, uint8_t* live,
                       int64_t* hidden_src, void* stream);

/* The verify step's argmax and acceptance in two launches instead of three: mtpk_argmax_keys
 * writes the first-occurrence (value, index) keys of each row's vocabulary chunks, keys u64
 * [rows, chunks] with chunks = mtpk_argmax_partials(rows, vocab) / rows (the first kernel of
 * mtpk_argmax_rows); mtpk_greedy_accept_keys reduces row (b, s)'s keys (rows = batch * t, row
 * b * t + s), writes step_argmax[b * sa_stride + s] and then does what mtpk_greedy_accept does,
 * with the same outputs. batch * t <= 4096 (MTPK_EINVAL beyond). */
int mtpk_argmax_keys(const void* logits, int dtype, int64_t rows, int64_t vocab,
                     int64_t row_stride, uint64_t* keys, void* stream);
int mtpk_greedy_accept_keys(const uint64_t* keys, int64_t chunks, int64_t* step_argmax,
                            int64_t sa_stride, const int64_t* draft, int64_t draft_stride,
                            const uint8_t* active, const int64_t* pos, const int64_t* budget,
                            const int64_t* stops, int n_stops, const int64_t* forced_n, int batch,
                            int t, int conv_k1, int64_t* accept_len, int64_t* lengths, int64_t* packed_src,
                            int32_t* packed_cu, int64_t* conv_idx, uint8_t* keep, int64_t* bonus,
                            int64_t* next_pos, int64_t* budget_left, uint8_t* live,
                            int64_t* hidden_src, void* stream);

/* ---------------------------------------------------------------- round fill
 * The device half of `MTPVerifyRunner.fill` (graph_mtp.py:795-874): one launch unpacks a round's
 * staged rows into the captured round's static buffers. staging i64 [rows, 6 + w + n_stops],
 * w = max(t - 1, 1), one row per buffer row: token, position, budget, slot, forced count,
 * active (0 | 1), w forced ids, n_stops stop ids. lane_tables i32 [lanes, max_blocks] (every
 * lane's block table), hidden_cache [lanes, row_bytes] (each lane's seed row, any dtype).
 * Writes, per row j: token_matrix i64 [rows, t] = (token, 0, ...); pos, budget, slot_rows,
 * forced_n i64 [rows]; active u8 [rows]; forced_ids i64 [rows, w]; stops i64 [rows, n_stops];
 * block_table i32 [rows, max_blocks] = the slot's table on active rows, reserved_block on the
 * others; block_valid i32 [rows] = floor((pos + t + block_size - 1) / block_size); write_rows
 * i64 [rows, t] = block_table[j][q / block_size] * block_size + q mod block_size at
 * q = pos + s (floor division; -1 where q / block_size falls outside the table);
 * draft_hidden [rows, row_bytes] = hidden_cache[slot] (zeros for a slot outside [0, lanes));
 * pos_grid i64 [rows, t] and pos_steps i64 [t, rows] = pos + s; commit_slots i64 [rows] = slot
 * on active rows, -1 on the others. */
int mtpk_round_fill(const int64_t* staging, int64_t rows, int64_t t, int64_t n_stops,
                    const int32_t* lane_tables, int64_t lanes, int64_t max_blocks,
                    int64_t block_size, int32_t reserved_block, const void* hidden_cache,
                    int64_t row_bytes, int64_t* token_matrix, int64_t* pos, int64_t* budget,
                    int64_t* slot_rows, int64_t* forced_n, uint8_t* active, int64_t* forced_ids,
                    int64_t* stops, int32_t* block_table, int32_t* block_valid,
                    int64_t* write_rows, void* draft_hidden, int64_t* pos_grid,
                    int64_t* pos_steps, int64_t* commit_slots, void* stream);

/* The token a draft step feeds forward (`draft_round_step`'s forced override and column write,
 * graph_mtp.py:477-504): out[j * out_stride] = forced[j * forced_stride] when forced_n[j] > step,
 * else tok[j * tok_stride], for j < rows (out: the token matrix's column step + 1; forced: the
 * forced ids' column step). */
int mtpk_draft_feed(const int64_t* tok, int64_t tok_stride, const int64_t* forced_n,
                    const int64_t* forced, int64_t forced_stride, int64_t step, int64_t* out,
                    int64_t out_stride, int64_t rows, void* stream);

/* Rows through two index lists (the verify step's hidden-seed write-back,
 * `scatter_time_active_rows`, graph_mtp.py:578-579): for j < rows, dst row dst_idx[j] (of
 * dst_rows, dst_stride bytes apart) = src row src_idx[j] (of src_rows, src_stride bytes apart),
 * row_bytes each; j is skipped when either index lies outside its table (e.g. slot -1 of a
 * padding row). */
int mtpk_copy_rows(const void* src, int64_t src_rows, int64_t src_stride, const int64_t* src_idx,
                   void* dst, int64_t dst_rows, int64_t dst_stride, const int64_t* dst_idx,
                   int64_t rows, int64_t row_bytes, void* stream);

/* ---------------------------------------------------------------- rejection sampling
 * Sampling-mode acceptance for an MTP round at temperature T > 0. The reference engine has no
 * counterpart: it runs MTP rounds only for all-greedy batches (scheduler.py:1775-1793,
 * model.py:4197-4201); this follows Leviathan et al. 2023, Alg. 1. With p_i = softmax(target_i
 * / T) and q_i = softmax(draft_i / T): draft x_i is accepted iff u_accept[b,i] * q_i(x_i) <=
 * p_i(x_i); at the first rejection a token is drawn from norm(max(0, p_i - q_i)) (from p_i if
 * that is all zero), else the bonus is drawn from p_k. A draw from weights w with uniform r is
 * the smallest v with cumsum(w)[v] > r * sum(w) (the last positive index if rounding leaves
 * none). Inputs: target f32|bf16 [B, k+1, vocab] and draft [B, k, vocab], contiguous;
 * draft_tokens i64 [B, k]; u_accept f32 [B, k]; u_sample f32 [B].
 * Outputs: accept_len i64 [B]; token i64 [B] (the resampled or bonus token); emitted i64
 * [B, k+1] (may be NULL) = accepted drafts, then `token` repeated, which is a step_argmax for
 * mtpk_greedy_accept that yields the same accept length and every rollback index; margin f32
 * [B, k] (may be NULL) = p_i(x_i) - u_i q_i(x_i), >= 0 accepts. fp32 arithmetic, fixed
 * reduction order. `workspace` (16-byte aligned) of mtpk_rejection_workspace_bytes bytes. */
int64_t mtpk_rejection_workspace_bytes(int64_t batch, int k, int64_t vocab);
int mtpk_rejection_sample(const void* target, const void* draft, int dtype, int64_t batch, int k,
                          int64_t vocab, const int64_t* draft_tokens, const float* u_accept,
                          const float* u_sample, float temperature, void* workspace,
                          int64_t workspace_bytes, int64_t* accept_len, int64_t* token,
                          int64_t* emitted, float* margin, void* stream);

/* mtpk_rejection_sample followed by the round's acceptance outputs in the same launches: what
 * mtpk_greedy_accept gives with `emitted` as the step argmax (stop ids, budget, every rollback
 * index), here taken from the sampler's accept length a (the stop ids and the budget can only
 * shorten the accept below a, through the drafts), so no acceptance launch follows. No reference
 * counterpart (as mtpk_rejection_sample). Inputs as mtpk_rejection_sample, plus active u8 [B],
 * pos / budget i64 [B], stops i64 [B, n_stops], conv_k1; outputs as mtpk_greedy_accept
 * (accept_len, lengths, token, emitted required; the others may be NULL), B <= 1024. */
int mtpk_rejection_accept(const void* target, const void* draft, int dtype, int64_t batch, int k,
                          int64_t vocab, const int64_t* draft_tokens, const float* u_accept,
                          const float* u_sample, float temperature, void* workspace,
                          int64_t workspace_bytes, const uint8_t* active, const int64_t* pos,
                          const int64_t* budget, const int64_t* stops, int n_stops, int conv_k1,
                          int64_t* accept_len, int64_t* lengths, int64_t* packed_src,
                          int32_t* packed_cu, int64_t* conv_idx, uint8_t* keep, int64_t* bonus,
                          int64_t* next_pos, int64_t* budget_left, uint8_t* live,
                          int64_t* hidden_src, int64_t* token, int64_t* emitted, void* stream);

/* Temperature sampling of one token per row, the draft step's sampler in sampling mode (the
 * reference's draft step is greedy only: mtp.py:640-658). logits f32|bf16 [rows, vocab]
 * contiguous, u f32 [rows]; token i64 [rows] = inverse-CDF draw from softmax(logits / T). */
int64_t mtpk_sample_workspace_bytes(int64_t rows, int64_t vocab);
int mtpk_sample_rows(const void* logits, int dtype, int64_t rows, int64_t vocab, float temperature,
                     const float* u, void* workspace, int64_t workspace_bytes, int64_t* token,
                     void* stream);

/* ---------------------------------------------------------------- Gated DeltaNet recurrence
 * Gated delta-rule steps over a pool of fp32 recurrent states, replacing
 * `deltanet_fused.delta_rule_verify_exact` (deltanet_fused.py:1090-1176, kernel :274-398) in the
 * verify forward (`deltanet_verify_static`, graph_mtp.py:227-344) and the accepted-prefix replay
 * (`deltanet_verify_rollback_static`, graph_mtp.py:347-437). Per step, for row j and head h:
 *   S <- exp(g) S;  S <- S + k ((v - S^T k) beta)^T;  out = S^T q
 * state f32 [slots_total, heads, k_dim = 128, v_dim] contiguous; row j uses state slot slot[j]
 * (int64 [rows], NULL: slot j); rows must name distinct slots. A row whose slot lies outside
 * [0, slots_total) touches no state: its outputs are zeros and a commit leaves the pool as is. q, k f32 [rows, t, qk_heads, 128]
 * (q and k already l2-normalised, q scaled), head h reads q/k head h / (heads / qk_heads);
 * v f32 [rows, t, heads, v_dim]; g (log decay) and beta f32 [rows, t, heads]; all contiguous.
 * lengths == NULL (verify): t steps from the stored state, which is not written; out
 * f32 [rows, t, heads, v_dim] receives every step's output. lengths int64 [rows] (commit): row j
 * advances its slot in place by min(max(lengths[j], 0), t) steps; out may be NULL.
 * t >= 1 (steps run in order; prefill of a prompt is one call with t = its length),
 * k_dim 16, 32, 64 or 128, 1 <= v_dim <= 4096. */
int mtpk_delta_rule(float* state, int64_t slots_total, const int64_t* slot, int64_t rows, int64_t t,
                    int64_t heads, int64_t qk_heads, int64_t k_dim, int64_t v_dim, const float* q,
                    const float* k, const float* v, const float* g, const float* beta,
                    const int64_t* lengths, float* out, void* stream);

/* Verify-row preparation of a Gated DeltaNet layer, replacing the torch chain of
 * `deltanet_verify` (model.py:3738-3905) between the in-projection and the recurrence: proj
 * [batch * t, proj_stride] (model dtype f32|bf16; per row qkv [C], z [v_heads * v_dim],
 * b [v_heads], a [v_heads], C = 2 k_heads k_dim + v_heads v_dim); conv_state [slots, C,
 * conv_k - 1] and conv_w [C, conv_k] of the model dtype; slot i64 [batch]; a_log, dt_bias f32
 * [v_heads]. Step s of row b: x = silu(sum_j win[s + j] conv_w[c][j]) over the window [stored
 * columns | the t new qkv columns], rounded to the model dtype; q = l2norm(x_q) * q_scale,
 * k = l2norm(x_k) (l2norm(x) = x rsqrt(sum x^2 + eps)), v = x_v, all f32 [batch, t, heads,
 * dim]; beta = sigmoid(b), g = -exp(a_log) softplus(a + dt_bias), f32 [batch, t, v_heads].
 * Head dims <= 256, conv_k <= 9. conv_state has slots_total slots; a row whose slot lies
 * outside [0, slots_total) reads a zero window instead. */
int mtpk_deltanet_prep(const void* proj, int dtype, int64_t proj_stride, const void* conv_state,
                       const int64_t* slot, int64_t slots_total, const void* conv_w, const float* a_log,
                       const float* dt_bias, int64_t batch, int64_t t, int64_t k_heads,
                       int64_t k_dim, int64_t v_heads, int64_t v_dim, int64_t conv_k, float eps,
                       float q_scale, float* q, float* k, float* v, float* g, float* beta,
                       void* stream);

/* The commit's conv-window update (`deltanet_verify_rollback`, model.py:3907-3972): the window
 * of slot[b], conv_state[slot[b]] [channels, k1], becomes columns idx[b][0 .. k1) (i64, clamped
 * to [0, k1 + t - 1]) of [stored window | the t new raw columns proj[b * t + s][0 .. channels)].
 * In place; slots distinct; conv_state has slots_total slots, and a row whose slot lies
 * outside [0, slots_total) is skipped. */
int mtpk_conv_commit(void* conv_state, int dtype, const int64_t* slot, int64_t slots_total,
                     const void* proj,
                     int64_t proj_stride, const int64_t* idx, int64_t batch, int64_t channels,
                     int64_t k1, int64_t t, void* stream);

/* A DeltaNet layer's whole commit (`deltanet_verify_rollback`, model.py:3907-3972): the delta
 * rule's commit mode (mtpk_delta_rule with lengths, no outputs) and the conv-window update
 * (mtpk_conv_commit, conv_state of conv_slots_total slots) for the same rows and slots, in one
 * launch when k_dim is 128 and v_dim a multiple of 64 (the conv rows run as extra one-wave
 * workgroups beside the state stream), else as the two launches. The results are those of the
 * two calls. */
int mtpk_deltanet_commit(float* state, int64_t slots_total, const int64_t* slot, int64_t rows,
                         int64_t t, int64_t heads, int64_t qk_heads, int64_t k_dim, int64_t v_dim,
                         const float* q, const float* k, const float* v, const float* g,
                         const float* beta, const int64_t* lengths, void* conv_state,
                         int conv_dtype, int64_t conv_slots_total, const void* proj,
                         int64_t proj_stride, const int64_t* conv_idx, int64_t channels, int64_t k1,
                         void* stream);

/* ---------------------------------------------------------------- skinny bf16 GEMM
 * y[M, N] = x[M, K] . w[N, K]^T for M <= 256 token rows, bf16 in, fp32 accumulation: the
 * weight-bandwidth-bound linears of the MTP draft and verify steps (fc, q/k/v/o and DeltaNet
 * projections), the shared
 * expert and router of a decode or draft MoE layer (`swiglu_mlp`, model.py:638-649;
 * model.py:2811-2873) and the LM head (`greedy_token`, mtp.py:640-658). x, w contiguous,
 * 16-byte aligned; K a multiple of 256; N * K * 2 < 2^31.
 * epilogue 0: out = y, f32 or bf16 [M, N].
 * epilogue 1: rows [0, N/2) are gate and [N/2, N) up (the `load_experts` gate_up order):
 *             out[m, j] = silu(y[m, j]) * y[m, N/2 + j], [M, N/2]; N/2 a multiple of 16.
 * epilogue 2: out int64 [M] = first-occurrence argmax over n of bf16(y[m, n]) (the argmax of
 *             the bf16 logits epilogue 0 would store).
 * workspace: mtpk_gemm_workspace_bytes(m, n, k, epilogue) bytes (split-K partials or argmax
 * keys; 0 means none is needed). */
int64_t mtpk_gemm_workspace_bytes(int64_t m, int64_t n, int64_t k, int epilogue);
int mtpk_gemm_bf16(const uint16_t* x, int64_t m, int64_t k, const uint16_t* w, int64_t n,
                   int epilogue, void* out, int out_dtype, void* workspace,
                   int64_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------- row norms
 * One launch per normalisation of the verify / draft forward, in place of the torch op chains
 * of `rmsnorm` (model.py:587-604), the DeltaNet output norm (model.py:613-619), the DeltaNet
 * q/k L2 norm and `apply_rope` (model.py:631-635). kind 0: y = x*rsqrt(mean(x^2)+eps)*(1+w);
 * kind 1: y = x*rsqrt(mean(x^2)+eps)*w, times silu(gate) when gate is given; kind 2:
 * y = x*rsqrt(sum(x^2)+eps)*scale (w unused). Row r (of `rows`) is head r % heads_per_token of
 * token r / heads_per_token, read from x at token*x_token_stride + head*x_head_stride
 * (elements; the gate likewise). res (optional, contiguous [rows, dim], heads_per_token 1,
 * x contiguous): x is replaced by x + res in x's dtype, which is also written to sum_out.
 * rope_cos/rope_sin (optional, f32 [positions, rot_dim]) with rope_pos (i64 [tokens]):
 * rotate-half RoPE on the first rot_dim channels of y rounded to the output dtype (dim <= 512;
 * rot_dim a multiple of 16, or 2, 4 or 8). gather (optional, i64): output token r reads input
 * token gather[r * gather_stride] of the gather_rows tokens x holds (an embedding lookup by
 * token id, fused; an id outside [0, gather_rows) reads the nearest row). out: token r's
 * heads_per_token rows of dim at r * out_token_stride (0: packed, heads_per_token * dim), so two
 * calls can fill the halves of one concatenated row; the residual form takes no gather and a
 * packed out. dim a multiple of 8, <= 8192; bf16 strides multiples of 8 and pointers 16-byte
 * aligned. */
int mtpk_rownorm(const void* x, int x_dtype, int64_t x_token_stride, int64_t x_head_stride,
                 const void* res, int res_dtype, void* sum_out, const void* w, int w_dtype,
                 int kind, float eps, float scale, const void* gate, int gate_dtype,
                 int64_t gate_token_stride, int64_t gate_head_stride, const float* rope_cos,
                 const float* rope_sin, const int64_t* rope_pos, int rot_dim, void* out,
                 int out_dtype, int64_t rows, int heads_per_token, int dim, const int64_t* gather,
                 int64_t gather_stride, int64_t gather_rows, int64_t out_token_stride,
                 void* stream);

/* ---------------------------------------------------------------- paged verify attention
 * Causal GQA attention of t query rows per lane over a paged bf16 KV cache, replacing
 * `verify_attention_paged` (model.py:1120-1205; per row `paged_attn.decode_attention_paged`,
 * paged_attn.py) in the verify forward and the MTP layer's attention (`mtp._attn_rows`,
 * mtp.py:233-279, t = 1). q bf16 [batch, heads, t, head_dim] contiguous; k_pool bf16
 * [pool_rows, kv_heads, head_dim] and v_pool bf16 [pool_rows / 16, kv_heads, head_dim, 16] (V
 * transposed inside each 16-row block), both contiguous; block_table int32
 * [batch, table_stride]: lane b's position p is pool row block_table[b][p / 16] * 16 + p % 16;
 * base_pos int64 [batch]: query row s of lane b is at base_pos[b] + s and attends to positions
 * 0 .. base_pos[b] + s (q head h uses kv head h / (heads / kv_heads)). out bf16, q's shape.
 * head_dim 64, 128 or 256. fp32 scores and softmax, bf16 probabilities into the PV product.
 * n_split key splits per (lane, kv head) (mtpk_attention_splits picks one from the shape and a
 * host bound on the context, so that every workgroup is resident at once; 0 for a shape the
 * kernel does not take); n_split > 1 needs mtpk_attention_workspace_bytes of workspace. */
int mtpk_attention_splits(int64_t batch, int64_t t, int64_t heads, int64_t kv_heads,
                          int64_t head_dim, int64_t max_ctx);
int64_t mtpk_attention_workspace_bytes(int64_t batch, int64_t t, int64_t heads, int64_t kv_heads,
                                       int64_t head_dim, int n_split);
int mtpk_paged_attention(const uint16_t* q, int64_t batch, int64_t t, int64_t heads,
                         int64_t kv_heads, int64_t head_dim, const uint16_t* k_pool,
                         const uint16_t* v_pool, int64_t pool_rows, const int32_t* block_table,
                         int64_t table_stride, const int64_t* base_pos, float scale, int n_split,
                         void* workspace, int64_t workspace_bytes, uint16_t* out, void* stream);

/* mtpk_paged_attention with the query rows read, and the output rows written, at any row
 * strides, and the attention output gate applied in the epilogue (`model.py:2158-2290`:
 * `o_proj(out * sigmoid(gate))`). Element d of (lane b, q head h, step s) is at
 * b * strides[0] + h * strides[1] + s * strides[2] + d of q, gate and out (three int64 strides
 * each, multiples of 8 for q). gate may be NULL; with it, out = bf16(bf16(o) *
 * bf16(sigmoid(gate))), the rounding of the unfused bf16 torch ops. */
int mtpk_paged_attention_gated(const uint16_t* q, const int64_t* q_strides, const uint16_t* gate,
                               const int64_t* gate_strides, int64_t batch, int64_t t,
                               int64_t heads, int64_t kv_heads, int64_t head_dim,
                               const uint16_t* k_pool, const uint16_t* v_pool, int64_t pool_rows,
                               const int32_t* block_table, int64_t table_stride,
                               const int64_t* base_pos, float scale, int n_split, void* workspace,
                               int64_t workspace_bytes, uint16_t* out, const int64_t* out_strides,
                               void* stream);

/* This round's K and V rows into the paged caches (the cache writes of `attn_verify`,
 * model.py:3519-3577, graph_mtp.py:857-860, and `mtp.cache_target_rows`, mtp.py:440-485):
 * k, v bf16 rows (b, s) of kv_heads * head_dim values at row strides k_row_stride /
 * v_row_stride (elements, row = b * t + s), position base_pos[b] + s, pool row
 * block_table[b][pos / 16] * 16 + pos % 16 of k_pool [pool_rows, kv_heads, head_dim] and of
 * v_pool [pool_rows / 16, kv_heads, head_dim, 16] (the layout mtpk_paged_attention reads).
 * keep (optional, u8 [batch, t] at element strides keep_b, keep_s; a 0 stride broadcasts, as a
 * per-lane mask does): rows with 0 are not written. head_dim a multiple of 8. */
int mtpk_kv_write(const uint16_t* k, int64_t k_row_stride, const uint16_t* v, int64_t v_row_stride,
                  uint16_t* k_pool, uint16_t* v_pool, int64_t pool_rows, const int32_t* block_table,
                  int64_t table_stride, const int64_t* base_pos, const uint8_t* keep, int64_t keep_b,
                  int64_t keep_s, int64_t batch, int64_t t, int64_t kv_heads, int64_t head_dim,
                  void* stream);

/* Streaming-read probe (no reference counterpart: a measurement of the HBM read ceiling the MoE
 * weight streams are compared with). Reads bytes [0, bytes) of `base` with 16-byte loads,
 * `loads_in_flight` (4, 8 or 16) per thread per iteration, over `grid` workgroups of 256
 * threads; stores nothing (sink u32 [1024] is written only for a constant no input produces).
 * bytes <= 4 GiB - 32. */
int mtpk_probe_stream(const void* base, int64_t bytes, int grid, int loads_in_flight,
                      uint32_t* sink, void* stream);

/* ---------------------------------------------------------------- test probes
 * In-bounds probe of the compiler builtin this library's MoE relies on: one wave computes
 * d = A(16x32) * B(32x16) with v_mfma_f32_16x16x32_bf16 from per-lane operand registers
 * a_lanes/b_lanes bf16 [64, 8] and writes its four result registers per lane to d_lanes
 * f32 [64, 4]. The caller checks the lane layout against a host matmul. No counterpart in the
 * reference (it verifies a gfx950 instruction's register layout). */
int mtpk_probe_mfma_16x16x32(const uint16_t* a_lanes, const uint16_t* b_lanes, float* d_lanes,
                             void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MTPK_H */
