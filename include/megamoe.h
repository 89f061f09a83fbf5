/*
 * megamoe.h -- C ABI of the MI355X-native Mega-MoE hot path (libmegamoe.so).
 *
 * Every entry point is asynchronous on the given HIP stream, allocates
 * nothing, and returns 0 on success or a negative code (MM_E_*) on an
 * argument or launch error; mm_last_error() returns a thread-local message.
 * Device buffers are raw pointers. bf16 tensors are passed as uint16_t bit
 * patterns, row-major, with the leading strides given in elements.
 *
 * Routing metadata is computed on the device and never copied to the host:
 * the number of valid routes lives in offsets[num_experts] and every kernel
 * that consumes expert-major rows reads it there, so a forward or backward
 * pass issues no host synchronisation.
 *
 * Each declaration names the reference interface it replaces
 * (paths relative to the Mega-MoE-TD source tree).
 */
#ifndef MEGAMOE_H_
#define MEGAMOE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* mm_stream_t; /* == hipStream_t */

#define MM_OK 0
#define MM_E_ARG -1     /* bad shape / pointer / size argument */
#define MM_E_WS -2      /* workspace too small */
#define MM_E_LAUNCH -3  /* HIP launch error */

/* Activation kinds (MoEForwardConfig.activation, src/mega_moe/config.py:24-32). */
#define MM_ACT_SWIGLU 0
#define MM_ACT_SITUGLU 1
#define MM_ACT_CLAMP_SWIGLU 2

/*
 * Formats of the saved raw FC1 output (MoEForwardConfig.save_fc1_dtype,
 * src/mega_moe/config.py:178-186; src/mega_moe/ops/forward.py:625-651):
 *   BF16  the raw gate/up values.
 *   FP16  the same bf16 values stored as fp16 (exact within fp16 range).
 *   FP8   E4M3 (OCP "fn": max 448) of value * 448 / amax, with one fp32
 *         scale amax / 448 per row and per MM_FC1_SCALE_GROUP-column group
 *         (amax over the group's |bf16 values|, 1 for an all-zero group);
 *         scale table [rows, 2I / MM_FC1_SCALE_GROUP], gate groups then up
 *         groups; dequantized value = e4m3 * scale
 *         (kernels/fused_forward.py:893-942, kernels/mega_bwd.py:3185-3206).
 */
#define MM_FC1_BF16 0
#define MM_FC1_FP16 1
#define MM_FC1_FP8 2
#define MM_FC1_SCALE_GROUP 128

const char* mm_last_error(void);
int mm_version(void);

/* ---------------------------------------------------------------- routing */

/* Workspace bytes mm_route needs for `num_routes` routes and `num_experts`. */
size_t mm_route_workspace_bytes(int64_t num_routes, int32_t num_experts);

/*
 * Stable expert-major routing plan.
 * Replaces runtime/routing.py:621-768 (build_routing_plan: valid mask,
 * float32 stable argsort, histogram, offsets), the fused per-core helpers in
 * kernels/fused_forward.py:158-480, and build_route_to_send
 * (kernels/fc2_combine.py:508-529).
 *
 *   selected      [num_routes] int32 expert id per flat route (token*k + slot);
 *                 ids outside [0, num_experts) are dropped. 1 <= num_experts
 *                 <= 32768 (the large-bin-count range of runtime/routing.py:
 *                 246-416).
 *   routing_weights [num_routes] fp32 or NULL.
 *   counts        [E]     routes per expert.
 *   offsets       [E+1]   exclusive prefix of counts; offsets[E] = #valid.
 *   send_route    [num_routes] flat route id of expert-major row i (i < #valid).
 *   send_token    [num_routes] send_route[i] / top_k.
 *   route_to_send [num_routes] inverse of send_route, -1 for dropped routes.
 *   weight_perm   [num_routes] routing_weights[send_route[i]] or NULL.
 * Rows i >= #valid of the send tables are left unwritten.
 */
int mm_route(const int32_t* selected, int64_t num_routes, int32_t top_k,
             int32_t num_experts, const float* routing_weights,
             int32_t* counts, int32_t* offsets, int32_t* send_route,
             int32_t* send_token, int32_t* route_to_send, float* weight_perm,
             void* workspace, size_t workspace_bytes, mm_stream_t stream);

/*
 * mm_route without a workspace argument: the per-unit count table lives in
 * a library-owned device array of mm_route_noalloc_scratch_bytes() bytes
 * (4 MiB) per GPU, kept until the process ends. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). Same arguments, outputs and errors as mm_route; calls whose
 * mm_route_workspace_bytes(num_routes, num_experts) exceeds the scratch size
 * return MM_E_ARG (with E = 1024 that allows about 2 million routes). The
 * call allocates nothing. Every call on one GPU shares that GPU's array:
 * calls that overlap on one GPU (different streams) race.
 */
size_t mm_route_noalloc_scratch_bytes(void);

int mm_route_noalloc(const int32_t* selected, int64_t num_routes, int32_t top_k,
                     int32_t num_experts, const float* routing_weights,
                     int32_t* counts, int32_t* offsets, int32_t* send_route,
                     int32_t* send_token, int32_t* route_to_send,
                     float* weight_perm, mm_stream_t stream);

/* ---------------------------------------------------------------- permute */

/*
 * Dispatch on one GPU: out[i, :] = x[send_token[i], :] for i < offsets[E].
 * Replaces the dispatch leg of kernels/dispatch_fc1.py:365-509 and
 * kernels/fused_forward.py:1106-1158 (remote row stores become a local
 * gather); also serves the backward gather gco = dy[send_token]
 * (kernels/dispatch_fc2_bwd.py:197-213).
 */
int mm_permute(const uint16_t* x, int64_t ldx, const int32_t* send_token,
               const int32_t* offsets, int32_t num_experts, int64_t max_rows,
               int32_t hidden, uint16_t* out, int64_t ldo, mm_stream_t stream);

/* ---------------------------------------------------------- grouped GEMMs */

/* Workspace bytes any grouped-GEMM entry needs (tile lists). */
size_t mm_gemm_workspace_bytes(int64_t max_rows, int32_t num_experts);

/*
 * FC1 grouped GEMM with the gated activation fused into its epilogue.
 * Replaces kernels/dispatch_fc1.py:580-752 + kernels/weighted_swiglu.py:18-81
 * and the FC1 leg of kernels/fused_forward.py:551-1008.
 *
 *   gu[i, :]   = x[row(i), :] @ w1[e]          (fp32 accumulate, e = expert of row i)
 *   gate, up   = bf16(gu[:, :I]), bf16(gu[:, I:])
 *   act[i, j]  = bf16(act_fn(gate, up) * weight_perm[i])
 * row(i) = send_token[i] when send_token != NULL (fused dispatch gather),
 * else i. w1 is [E, H, 2I] contiguous (gate_up_weight). fc1_out
 * ([rows, 2I] = [gate | up] in fc1_format, row stride 2I elements) may be
 * NULL; MM_FC1_FP8 needs I % MM_FC1_SCALE_GROUP == 0 and fc1_scale
 * ([rows, 2I / MM_FC1_SCALE_GROUP] fp32), which is ignored otherwise.
 */
int mm_fc1_swiglu(const uint16_t* x, int64_t ldx, const int32_t* send_token,
                  const uint16_t* w1, const int32_t* offsets,
                  const float* weight_perm, int32_t num_experts,
                  int64_t max_rows, int32_t hidden, int32_t inter,
                  int32_t act_kind, float situ_beta, float situ_linear_beta,
                  float clamp_limit, uint16_t* act, void* fc1_out,
                  int32_t fc1_format, float* fc1_scale,
                  void* workspace, size_t workspace_bytes, mm_stream_t stream);

/*
 * Generic grouped "row" GEMM over expert-major rows:
 *   c[i, n] = sum_k a[row(i), k] * B_e(k, n),  e = expert of row i
 *   B_e(k, n) = b[e*b_se + n*b_sn + k*b_sk]   (one of b_sn, b_sk must be 1)
 * row(i) = a_rows[i] when a_rows != NULL, else i. Output bf16 [rows, N], ldc.
 * Replaces the FC2 GEMM (kernels/fc2_combine.py:139-213,
 * kernels/fused_forward.py:1161-1213), the FC2 dgrad
 * (kernels/dispatch_fc2_bwd.py:223-563) and the FC1 dgrad
 * (kernels/combine_fc1_bwd.py:114-247).
 */
int mm_grouped_gemm(const uint16_t* a, int64_t lda, const int32_t* a_rows,
                    const uint16_t* b, int64_t b_se, int64_t b_sn, int64_t b_sk,
                    const int32_t* offsets, int32_t num_experts,
                    int64_t max_rows, int32_t n, int32_t k, uint16_t* c,
                    int64_t ldc, void* workspace, size_t workspace_bytes,
                    mm_stream_t stream);

/*
 * Grouped weight-gradient GEMM with ragged K (the expert's rows):
 *   c[e, n1, n2] = sum_{i in rows(e)} p[prow(i), n1] * q[qrow(i), n2]
 * prow(i) = p_rows[i] if p_rows != NULL else i (same for q). Output bf16
 * [E, N1, N2] contiguous; experts with no rows get zeros. max_rows is the
 * row capacity (an upper bound of offsets[E]); it selects the tiling (a
 * persistent kernel bound by the output write when experts average <= 192
 * rows, 256 x 256 tiles over the ragged K otherwise). Every kernel reads
 * gathered rows (p_rows / q_rows) in place: the workspace arguments are
 * unused and mm_wgrad_workspace_bytes returns 0 (both kept for ABI
 * compatibility).
 * Replaces kernels/transposed_grouped_gemm.py:24-100 and the default
 * torch_npu grouped wgrad of ops/backward.py:85-94.
 */
size_t mm_wgrad_workspace_bytes(int64_t max_rows, int32_t num_experts,
                                int32_t n1, int32_t n2);

int mm_grouped_wgrad(const uint16_t* p, int64_t ldp, const int32_t* p_rows,
                     const uint16_t* q, int64_t ldq, const int32_t* q_rows,
                     const int32_t* offsets, int32_t num_experts,
                     int64_t max_rows, int32_t n1, int32_t n2, uint16_t* c,
                     void* workspace, size_t workspace_bytes,
                     mm_stream_t stream);

/* ---------------------------------------------------------------- combine */

/*
 * Top-k combine without atomics:
 *   out[t, :] = bf16( sum_{j<k, route_to_send[t*k+j] >= 0} fp32(y[route_to_send[t*k+j], :]) )
 * summed in slot order j = 0..k-1. Replaces _kernel_local_topk_reduce
 * (kernels/fc2_combine.py:447-505) and _reduce_topk_rows
 * (kernels/fused_forward.py:1319-1387); with y = dX it is the grad_hidden
 * reduce of kernels/combine_fc1_bwd.py:357-394.
 */
int mm_combine(const uint16_t* y, int64_t ldy, const int32_t* route_to_send,
               int64_t num_tokens, int32_t top_k, int32_t hidden,
               uint16_t* out, int64_t ldo, mm_stream_t stream);

/*
 * Backward top-k reduce and routing-weight gradient gather in one launch:
 *   grad_hidden = mm_combine(dx, route_to_send)  and
 *   grad_rw[r]  = float(dscale[route_to_send[r]]) or 0 for dropped routes,
 * the two outputs of mm_combine + mm_gather_route_grad on the FC1 dgrad rows.
 * Replaces the grad_hidden reduce and gate-channel gather of
 * kernels/combine_fc1_bwd.py:357-394.
 */
int mm_combine_bwd(const uint16_t* dx, int64_t ldx,
                   const int32_t* route_to_send, int64_t num_tokens,
                   int32_t top_k, int32_t hidden, uint16_t* grad_hidden,
                   int64_t ldo, const uint16_t* dscale, float* grad_rw,
                   mm_stream_t stream);

/*
 * Gather of the per-row routing-weight gradient back to [T, k] order:
 *   grad_rw[r] = float(dscale[route_to_send[r]]) or 0 for dropped routes.
 * Replaces the gate-channel gather of kernels/combine_fc1_bwd.py:357-394.
 */
int mm_gather_route_grad(const uint16_t* dscale, const int32_t* route_to_send,
                         int64_t num_routes, float* grad_rw, mm_stream_t stream);

/* ---------------------------------------------------------- SwiGLU bwd */

/*
 * Gated-activation backward per expert-major row i < offsets[E]:
 *   a = gate, b = up (from fc1_out [rows, 2I] in fc1_format, dequantized
 *       with fc1_scale for MM_FC1_FP8), dc = grad_act [rows, I],
 *   s = bf16(scale[i]) (the routing weight rounded to bf16, as the reference's
 *       saved recv_weights_sorted is; ops/_torch_forward.py:267)
 *   dAB[i] = bf16([dc*act'(a)*v(b)*s | dc*act(a)*v'(b)*s]),
 *   dscale[i] = bf16(sum_j act(a)*v(b)*dc).
 * Replaces kernel_swiglu_bwd (kernels/swiglu_bwd.py:15-83).
 */
int mm_swiglu_bwd(const uint16_t* grad_act, int64_t ld_ga,
                  const void* fc1_out, int64_t ld_fc1, int32_t fc1_format,
                  const float* fc1_scale, const float* scale,
                  const int32_t* offsets, int32_t num_experts,
                  int64_t max_rows, int32_t inter, int32_t act_kind,
                  float situ_beta, float situ_linear_beta, float clamp_limit,
                  uint16_t* dab, uint16_t* dscale, mm_stream_t stream);

/*
 * Activation recompute from the saved FC1 output (any fc1_format), per
 * expert-major row i < offsets[E]:
 *   act[i, j] = bf16(act_fn(gate, up) * weight_perm[i])
 * — the FC1 epilogue's formula, so for a bf16 save it reproduces the
 * forward's act bit for bit. Replaces the MOE_SAVED_RECOMPUTE act recompute
 * of kernels/mega_bwd.py:1414-1468 (_recompute_act_rows).
 */
int mm_gated_act(const void* fc1_out, int64_t ld_fc1, int32_t fc1_format,
                 const float* fc1_scale, const float* weight_perm,
                 const int32_t* offsets, int32_t num_experts, int64_t max_rows,
                 int32_t inter, int32_t act_kind, float situ_beta,
                 float situ_linear_beta, float clamp_limit, uint16_t* act,
                 int64_t ld_act, mm_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MEGAMOE_H_ */
