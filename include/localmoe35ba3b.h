/*
 * localmoe35ba3b.h - C ABI of the MI355X (gfx950) quantized MoE-FFN hot path.
 *
 * Every entry point takes raw device pointers, 64-bit sizes and a HIP stream
 * handle passed as `void *` (a `hipStream_t`; NULL is the legacy default
 * stream).  Launches are asynchronous and stream-ordered; no entry point
 * synchronises the device, allocates device memory or frees caller memory.
 * All validation happens on the host before any launch, so a non-zero status
 * means nothing was enqueued.
 *
 * Status codes map onto the exception types the Python operators raise:
 *   LM_OK      0  success
 *   LM_EINVAL  1  ValueError   (bad geometry, dtype, id range, ...)
 *   LM_ENOMEM  2  MemoryError  (a workspace or capacity bound is exceeded)
 *   LM_ELAUNCH 3  RuntimeError (the HIP runtime refused a launch)
 * lm_last_error() returns the message of the last failing call on the
 * calling host thread.
 *
 * Data formats (identical to the reference converter's artifact format):
 *   weights  q int8 [N, K] row-major (K contiguous), K % 128 == 0
 *   scales   s fp32 [N, K/128]: w[n, k] ~= q[n, k] * s[n, k/128]
 *   expert banks are [E, N, K] / [E, N, K/128] with arbitrary expert stride.
 *   activations are bf16 (LM_BF16) or fp16 (LM_FP16) row-major; a `dtype`
 *   argument names the activation type, and outputs are written in it, as
 *   the reference allocates its outputs in x.dtype.
 *
 * Indices that a kernel turns into addresses (expert ids, route positions,
 * tile-table rows, combine slots) are clamped into the ranges the call
 * states, so malformed routing data yields wrong values, never an access
 * outside the buffers described by the arguments.
 *
 * Reference citations are to heliosz616/LocalMoe35Ba3b (qwen35_deploy/...)
 * and to the Transformers 5.15.0 Qwen3_5Moe modeling file ("HF").
 */
#ifndef LOCALMOE35BA3B_H
#define LOCALMOE35BA3B_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LM_OK 0
#define LM_EINVAL 1
#define LM_ENOMEM 2
#define LM_ELAUNCH 3

#define LM_BF16 0
#define LM_FP16 1
#define LM_FP32 2

/* Library identification and the message of the last error on this thread. */
const char *lm_version(void);
const char *lm_last_error(void);

/* Offline weight quantizer: s = max(amax_g|w| / 127, 1e-30) per 128-wide K
 * group, q = clamp(round_half_even(w / s), -127, 127).  w fp32 [rows, k].
 * Replaces convert.quantize (convert.py:31-37). */
int lm_quantize_weight_g128(const float *w, int8_t *q, float *s,
                            int64_t rows, int64_t k, void *stream);

/* The 16-row tile layout of an int8 weight bank q [experts][n][k] (rows k
 * bytes apart, experts expert_stride bytes apart), for the prefill GEMMs:
 *   tiles[e * expert_stride + ((b * k/64 + s) * 1024) + 256 p + 16 r + j]
 *     = q[e][16 b + r][64 s + 16 p + j],   r < 16, p < 4, j < 16.
 * Each 16-row x 64-K block is 1 KB, its 16-byte pieces ordered piece-major,
 * so lane 16 p + r of a wave loads exactly its MFMA operand piece.
 * format LM_TILES_PLAIN stores the bytes as they are; LM_TILES_F16 stores
 * u = q + 128 and, within every 4-byte word, the bytes of k = 0, 2, 1, 3
 * (the form the fused layer's fp16 gate_up GEMM converts to fp16 q with one
 * mask, one byte permute and one packed subtraction per two weights; see
 * lm_moe_layer.gu_q_tiles).  tiles has q's size and expert stride;
 * n % 16 == 0, k % 64 == 0.  No counterpart in the reference (a re-layout of
 * convert.py's int8 format). */
#define LM_TILES_PLAIN 0
#define LM_TILES_F16 1
int lm_w8_tile_rows(const int8_t *q, int64_t experts, int64_t n, int64_t k,
                    int64_t expert_stride, int8_t *tiles, int format,
                    void *stream);

/* Dynamic activation quantization per row and 128-group:
 * s = max(amax, 1e-10) * (1/127), q = rint(x / s).  x [rows, k] (x_dtype).
 * Replaces w8a8.quantize / w8a8._quant (w8a8.py:8-22). */
int lm_act_quant_g128(const void *x, int x_dtype, int8_t *q, float *s,
                      int64_t rows, int64_t k, void *stream);

/* Dense W8A16: y[m, n] = sum_k x[m, k] * dtype(q[n, k] * s[n, k/128]),
 * fp32 accumulation, y in the activation dtype.  m <= 8 runs the HBM
 * streaming GEMV, larger m the MFMA GEMM.  large_tile only selects the
 * MFMA tile height.  Replaces int8.linear / int8._linear (int8.py:9-37). */
int lm_w8a16_linear(const void *x, const int8_t *q, const float *s, void *y,
                    int64_t m, int64_t n, int64_t k, int dtype, int large_tile,
                    void *stream);

/* Grouped W8A16 decode GEMV over a device descriptor table
 * table[e, 5] = {gate_up.q, gate_up.s, down.q, down.s, slot} (int64):
 * y[e, :] = x[shared ? 0 : e, :] . dequant(table[e, field..field+1])^T,
 * x and y of `dtype`.
 * Replaces int8.grouped_linear / int8._grouped_linear (int8.py:213-237). */
int lm_w8a16_grouped_gemv(const void *x, const int64_t *table, void *y,
                          int64_t experts, int64_t n, int64_t k, int field,
                          int shared, int dtype, void *stream);

/* Grouped W8A8 decode GEMV on pre-quantized activations (xq int8 [rows, k],
 * xs fp32 [rows, k/128]): int32 dot per 128-group, then
 * acc = acc + (float(p_g) * xs_g) * ws[n, g] in ascending g, no FMA;
 * y written in y_dtype.
 * Replaces w8a8._linear (w8a8.py:25-41). */
int lm_w8a8_grouped_gemv(const int8_t *xq, const float *xs,
                         const int64_t *table, void *y, int64_t experts,
                         int64_t n, int64_t k, int field, int shared,
                         int y_dtype, void *stream);

/* lm_act_quant_g128 fused into lm_w8a8_grouped_gemv; x and y of `dtype`.
 * Replaces w8a8.grouped_linear (w8a8.py:44-48). */
int lm_w8a8_grouped_linear(const void *x, const int64_t *table, void *y,
                           int64_t experts, int64_t n, int64_t k, int field,
                           int shared, int dtype, void *stream);

/* Exact int32 per-group partials p[m, n, g] = sum_{k in g} xq[m, k] * wq[n, k]
 * of the W8A8 GEMV inner product (the tl.dot of w8a8.py:37), computed by the
 * same device code as the GEMV.  Exposed so callers can check bit-exactness. */
int lm_w8a8_group_partials(const int8_t *xq, const int8_t *wq, int32_t *p,
                           int64_t m, int64_t n, int64_t k, void *stream);

/* Dense W8A8 decode linear for m <= 8 rows of x (`dtype`): per-row dynamic
 * quantization, int32 group dots, the w8a8.py:40 fp32 epilogue, y in dtype.
 * swiglu != 0 treats the n weight rows as [gate; up] halves and writes
 * y[m, n/2] = T(T(silu(gate)) * up) (HF:715, int8.py:182-184).
 * No reference counterpart as one call: it is w8a8.quantize + w8a8._linear
 * + the SwiGLU glue on one dense matrix. */
int lm_w8a8_linear(const void *x, const int8_t *q, const float *s, void *y,
                   int64_t m, int64_t n, int64_t k, int swiglu, int dtype,
                   void *stream);

/* W8A8 MFMA GEMM for any number of rows (int8 x int8 -> int32 MFMA with
 * the per-group fp32 rescale), on rows already quantized by
 * lm_act_quant_g128: xq int8 [m, k], xs fp32 [m, k/128]; weights q int8
 * [n, k], s fp32 [n, k/128]; y [m, n] in y_dtype (bf16 or fp16), or
 * [m, n/2] with swiglu as in lm_w8a8_linear.  Replaces w8a8._linear
 * (w8a8.py:25-41) applied to every row rather than row 0 only: exact int32 group partials, then
 * acc = acc + (f32(p) * xs) * ws in ascending group order, unfused, so the
 * output is bit-identical to the reference's for each row. */
int lm_w8a8_gemm(const int8_t *xq, const float *xs, const int8_t *q, const float *s,
                 void *y, int64_t m, int64_t n, int64_t k, int swiglu, int y_dtype,
                 void *stream);

/* SwiGLU glue in `dtype` T: h[r, c] = T(T(silu(gu[r, c])) * gu[r, half + c]).
 * Replaces `gate, up = gu.chunk(2, -1); silu(gate) * up`
 * (int8.py:182-184, prefill.py:77-78, gpu_routes.py:74-75). */
int lm_swiglu(const void *gu, void *h, int64_t rows, int64_t half, int dtype,
              void *stream);

/* Decode combine over the descriptor table, ascending table order:
 * acc = T(acc + T(v[e, c] * w[slot_e])), v and y of `dtype` T; w_dtype
 * LM_BF16, LM_FP16 or LM_FP32; slots clamped into [0, experts).
 * Replaces int8._ordered_reduce (int8.py:240-250). */
int lm_ordered_reduce(const void *v, const int64_t *table, const void *w,
                      int w_dtype, void *y, int64_t n, int64_t experts,
                      int dtype, void *stream);

/* Prefill combine: per token over its top_k routes in ascending expert order
 * acc = T(acc + T(v[ordered[t,i], c] * w[t, slots[t,i]])), v and y of
 * `dtype` T; routes clamped into [0, tokens * top_k), slots into [0, top_k).
 * Replaces prefill._reduce (prefill.py:37-49). */
int lm_routed_reduce(const void *v, const int64_t *ordered,
                     const int64_t *slots, const void *w, int w_dtype,
                     void *y, int64_t tokens, int64_t n, int64_t top_k,
                     int dtype, void *stream);

/* Device route plan of gpu_routes.plan + _table (gpu_routes.py:17-36,47-63):
 * stable sort of the flat ids by expert; pos[p] = token of the p-th sorted
 * route; table[max_tiles, 3] = (expert, start, stop) per bm-row tile with
 * surplus rows (0, 0, 0); ordered[t, i] = sorted position of token t's i-th
 * smallest-id route; slots = argsort(ids, dim=1, stable).  ids int64
 * [tokens, top_k] in [0, experts).  experts <= 256.  max_tiles must be
 * ceil(tokens*top_k / bm) + experts. */
int lm_route_plan(const int64_t *ids, int64_t tokens, int64_t top_k,
                  int64_t experts, int64_t bm, int64_t *pos, int64_t *table,
                  int64_t max_tiles, int64_t *ordered, int64_t *slots,
                  void *stream);

/* Host (CPU) route plan of routing.plan_routes (routing.py:5-20):
 * positions[2, R] = (sorted_route // top_k, sorted_route % top_k) and the
 * segments (expert, start, stop) of non-empty experts; *n_segments receives
 * their count (segments arrays need room for `experts`).  Returns LM_EINVAL
 * for an empty input or an out-of-range id. */
int lm_plan_routes_host(const int64_t *ids, int64_t tokens, int64_t top_k,
                        int64_t experts, int64_t *positions,
                        int64_t *seg_expert, int64_t *seg_start,
                        int64_t *seg_stop, int64_t *n_segments);

/* Host (CPU) twin of lm_route_plan for ids already on the host, the plan of
 * the reference's host-planned prefill (prefill.py:52-85): pos[R] = token of
 * the p-th route in stable expert order; table rows (expert, start, stop)
 * for the bm-row tiles of the non-empty experts only (*n_tiles of them, in
 * expert order; max_tiles >= cdiv(R, bm) + experts is the capacity);
 * ordered/slots as in lm_route_plan; *n_active = number of non-empty
 * experts.  Returns LM_EINVAL for an empty input or an out-of-range id. */
int lm_route_plan_host(const int64_t *ids, int64_t tokens, int64_t top_k,
                       int64_t experts, int64_t bm, int64_t *pos,
                       int64_t *table, int64_t max_tiles, int64_t *ordered,
                       int64_t *slots, int64_t *n_tiles, int64_t *n_active);

/* Routed grouped W8A16 GEMM over a tile table (MFMA): for each tile
 * (e, start, stop) rows r in [start, min(start+bm, stop)):
 * y[r, :] = x[gather ? pos[r] : r, :] . dequant(q[e], s[e])^T.
 * x [x_rows, k] and y [y_rows, n] of `dtype`; the bank holds `experts`
 * experts at the given strides (elements).  Table experts are clamped into
 * [0, experts), starts and stops into [0, y_rows] and gathered rows pos[r]
 * into [0, x_rows); without gather y_rows <= x_rows.  pos (gather) has
 * y_rows entries.  bm must equal the table's tile height (<= 128).
 * Replaces prefill._routed / gpu_routes._nonempty (prefill.py:12-34,
 * gpu_routes.py:39-44). */
int lm_routed_gemm_w8a16(const void *x, int64_t x_rows, const int8_t *q,
                         const float *s, int64_t experts,
                         int64_t q_expert_stride, int64_t s_expert_stride,
                         const int64_t *pos, const int64_t *table,
                         int64_t n_tiles, int64_t bm, void *y, int64_t y_rows,
                         int64_t n, int64_t k, int gather, int dtype,
                         void *stream);

/* lm_routed_gemm_w8a16 (gathered) on the gate_up bank with the SwiGLU glue
 * fused into the epilogue: h[r, c] = T(T(silu(gu[r, c])) * gu[r, n/2 + c]),
 * h is [h_rows, n/2].  Same result as prefill.py:75-78 without the [R, n]
 * intermediate. */
int lm_routed_gate_up_swiglu(const void *x, int64_t x_rows, const int8_t *q,
                             const float *s, int64_t experts,
                             int64_t q_expert_stride, int64_t s_expert_stride,
                             const int64_t *pos, const int64_t *table,
                             int64_t n_tiles, int64_t bm, void *h,
                             int64_t h_rows, int64_t n, int64_t k, int dtype,
                             void *stream);

/* HF Qwen3_5MoeTopKRouter (HF:768-776) with a fixed tie rule:
 * logits[t, e] = float(bf16(float(sum_k double(x[t,k]) * double(w[e,k]))))
 * (+ bias[e] if bias != NULL, fp32 add); ids = top_k experts by
 * (logit desc, expert id asc); p = fp32 softmax over all experts;
 * weights = bf16(p_sel / sum(p_sel)).  ids are written in selection order.
 * x, w bf16; logits fp32 [tokens, experts] (required); ids int64
 * [tokens, top_k]; weights bf16 [tokens, top_k].  experts <= 256,
 * top_k <= 16. */
int lm_router_topk(const void *x, const void *w, const float *bias,
                   float *logits, int64_t *ids, void *weights, int64_t tokens,
                   int64_t experts, int64_t hidden, int64_t top_k,
                   void *stream);

/* Qwen3_5MoeRMSNorm (HF:801-815): y = bf16(x * rsqrt(mean(x^2) + eps)
 * * (1 + w)); x, y bf16 [rows, n], w fp32 [n] (NULL = zeros). */
int lm_rmsnorm(const void *x, const float *w, void *y, int64_t rows,
               int64_t n, float eps, void *stream);

/* ---------------------------------------------------------------------
 * Fused MoE-FFN block of the synthetic stack (router + 256 routed experts
 * top-8 + shared expert + RMSNorm + residual; HF:779-798, 801-815, 866-875).
 * One layer's weights:
 *   router_w  bf16 [E, H]         shared_gate_w bf16 [H]
 *   norm_w    fp32 [H] or NULL    router_bias fp32 [E] or NULL
 *   gu_q int8 [E+1, 2I, H], gu_s fp32 [E+1, 2I, H/128]   (index E = shared)
 *   dn_q int8 [E+1, H, I],  dn_s fp32 [E+1, H, I/128]
 * h bf16 [tokens, H] is the residual stream, updated in place:
 *   h = bf16(h + bf16(routed + bf16(bf16(sigmoid(g)) * shared)))
 * Decode (tokens == 1) runs routed experts W8A8 (w8a8.py) and the shared
 * expert W8A16; prefill runs everything W8A16 (prefill.py / gpu_routes.py).
 * H = 2048, I = 512, E = 256, top_k = 8 are the supported geometry.
 * `workspace` is caller-owned device memory of lm_moe_workspace_bytes(),
 * reused by every later call on the same stream; every call writes each
 * workspace region before reading it, so its initial contents do not
 * matter (lm_moe_workspace_init zeroes all of it for callers that want a
 * defined state).  Calls sharing a workspace must not overlap. */
typedef struct lm_moe_layer {
  /* sizeof(lm_moe_layer) as the caller compiled it; calls refuse any other
   * value (LM_EINVAL), so a caller built against an older layout of this
   * struct is rejected instead of misread. */
  int64_t struct_size;
  const void *router_w;
  const float *router_bias;
  const void *shared_gate_w;
  const float *norm_w;
  const int8_t *gu_q;
  const float *gu_s;
  const int8_t *dn_q;
  const float *dn_s;
  int64_t gu_q_expert_stride; /* elements between experts of gu_q */
  int64_t gu_s_expert_stride;
  int64_t dn_q_expert_stride;
  int64_t dn_s_expert_stride;
  /* Optional copies of gu_q and dn_q in the 16-row tile layout of
   * lm_w8_tile_rows (same expert strides), which the prefill grouped GEMMs
   * read with contiguous 1 KB wave loads; NULL = they read gu_q / dn_q.
   * dn_q_tiles is in LM_TILES_PLAIN and leaves results bit-identical.
   * gu_q_tiles is in the format gu_q_tiles_format names: LM_TILES_PLAIN
   * leaves results bit-identical; with LM_TILES_F16 the prefill gate_up GEMM
   * runs on fp16 operands - exact fp16 copies of the normalized rows (a
   * power of two per row) times exact q - and applies each 128-group's
   * scale to the fp32 sums instead of rounding q * s to bf16 per weight
   * (int8.py:21): within the bf16 tolerance of the reference's arithmetic,
   * not bit-identical to it, and faster.  No counterpart in the reference:
   * a device-side cache of the bank (for callers that can spend the memory
   * of a second int8 copy). */
  const int8_t *gu_q_tiles;
  const int8_t *dn_q_tiles;
  int64_t gu_q_tiles_format; /* LM_TILES_PLAIN or LM_TILES_F16 */
} lm_moe_layer;

int64_t lm_moe_workspace_bytes(int64_t max_tokens, int64_t hidden,
                               int64_t inter, int64_t experts, int64_t top_k);
int lm_moe_workspace_init(void *workspace, int64_t bytes, void *stream);

/* Where a call on `tokens` rows leaves its intermediates in the workspace:
 * byte offset and size of one region, for tests and debugging (no
 * reference counterpart; the reference keeps these in separate torch
 * tensors, prefill.py:52-85, int8.py:155-210).  R = tokens * top_k.
 * Regions of every call:
 *   LM_WS_NORMED      bf16  [tokens, H]      RMSNorm output (router input)
 *   LM_WS_GATE        fp32  [tokens]         shared-expert gate logits
 *   LM_WS_IDS         int64 [tokens, top_k]  selected experts, selection order
 *   LM_WS_WEIGHTS     bf16  [tokens, top_k]  routing weights, same order
 *   LM_WS_HIDDEN      bf16  [R + tokens, I]  SwiGLU rows (routed, then shared)
 *   LM_WS_DOWN        bf16  [R + tokens, H]  down rows (routed, then shared)
 * of prefill calls (tokens > 1) only:
 *   LM_WS_ROUTE_ROWS  int32 [tokens, top_k]  expert-sorted row of each route
 *   LM_WS_ROUTER_APPROX fp32 [tokens, experts] approximate router logits A
 *                                            (bf16 MFMA, fp32 sums, before
 *                                            the bias); the selection takes
 *                                            |A - x.w_e| <= 2^-17 |x| |w_e|
 *   LM_WS_ROW_NORMS   fp32  [tokens]         |x| of each normalized row
 *   LM_WS_ROUTER_NORMS fp32 [experts]        |w_e| of each router row
 *   (after a chained call, LM_WS_NORMED, LM_WS_ROW_NORMS and
 *   LM_WS_ROUTER_NORMS hold the next layer's inputs instead)
 * of decode calls (tokens == 1) only, whose routed rows in LM_WS_HIDDEN and
 * LM_WS_DOWN are in combine order (ascending expert id, slot s = row s):
 *   LM_WS_ACT_Q       int8  [H]              w8a8.quantize of the normed row
 *   LM_WS_ACT_SCALES  fp32  [H/128]          its group scales
 *   LM_WS_SLOT_IDS    int32 [top_k]          expert of each combine slot
 *   LM_WS_SLOT_WEIGHTS fp32 [top_k]          its (bf16-valued) routing weight
 *   LM_WS_GATE_UP_ACC fp32  [top_k, 2I]      W8A8 epilogue sums of the routed
 *                                            gate_up rows (w8a8.py:40), before
 *                                            the bf16 rounding
 *   LM_WS_DOWN_ACC    fp32  [top_k, H]       the same for the down rows
 * Valid until the next call using the workspace. */
#define LM_WS_NORMED 0
#define LM_WS_GATE 1
#define LM_WS_IDS 2
#define LM_WS_WEIGHTS 3
#define LM_WS_ROUTE_ROWS 4
#define LM_WS_HIDDEN 5
#define LM_WS_DOWN 6
#define LM_WS_ACT_Q 7
#define LM_WS_ACT_SCALES 8
#define LM_WS_SLOT_IDS 9
#define LM_WS_SLOT_WEIGHTS 10
#define LM_WS_GATE_UP_ACC 11
#define LM_WS_DOWN_ACC 12
#define LM_WS_ROUTER_APPROX 13
#define LM_WS_ROW_NORMS 14
#define LM_WS_ROUTER_NORMS 15
int lm_moe_workspace_region(int64_t tokens, int region, int64_t *offset,
                            int64_t *bytes);

/* One MoE-FFN layer on `tokens` rows of h (decode path when tokens == 1).
 * If ids_out / weights_out are non-NULL the routing of this layer is copied
 * there (int32 [tokens, top_k] in selection order, bf16 [tokens, top_k]).
 * phase_events, if non-NULL, holds hipEvent_t handles recorded on `stream`
 * before each kernel phase and after the last one: 8 for prefill (norm+gate,
 * router logits, top-k, plan, gate_up, down, combine, end), 4 for decode
 * (router, gate_up, down, end). */
int lm_moe_layer_forward(const lm_moe_layer *layer, void *h, int64_t tokens,
                         int64_t hidden, int64_t inter, int64_t experts,
                         int64_t top_k, float eps, void *workspace,
                         int64_t workspace_bytes, int32_t *ids_out,
                         void *weights_out, void *const *phase_events,
                         void *stream);

/* lm_moe_layer_forward for consecutive layers of one prefill chunk on one
 * workspace (the stack loop of HF:866-875 applied layer after layer).  With
 * next != NULL, the call's last kernel (the combine) also does next's norm
 * work on the rows it has just written: RMSNorm with next->norm_w, next's
 * shared-gate logit, the norms of next's router rows and, when next's
 * gate_up tiles are LM_TILES_F16, the fp16 row copy - the same code and
 * order as next's own norm kernel, so the results are bit-identical to
 * unchained calls.  The next call, on the same rows, workspace, stream and
 * eps with layer == this call's next, passes input_normed = 1 and skips its
 * norm kernel; the library remembers, per workspace, which layer, token
 * count and eps the last prefill call prepared, and refuses input_normed = 1
 * otherwise (LM_EINVAL, before any launch).  After a call with next, the
 * LM_WS_NORMED and LM_WS_GATE regions hold next's inputs.  Decode calls (tokens == 1) ignore next and
 * input_normed.  phase_events as above (with input_normed the norm+gate
 * phase is empty).  No counterpart in the reference: it saves one kernel and
 * one read of the hidden rows per layer and chunk. */
int lm_moe_layer_forward_chain(const lm_moe_layer *layer,
                               const lm_moe_layer *next, int input_normed,
                               void *h, int64_t tokens, int64_t hidden,
                               int64_t inter, int64_t experts, int64_t top_k,
                               float eps, void *workspace,
                               int64_t workspace_bytes, int32_t *ids_out,
                               void *weights_out, void *const *phase_events,
                               void *stream);

/* lm_moe_layer_forward without a workspace argument: the call's workspace
 * is a device array inside the library (one per device, about 7.3 MB, held
 * until the process ends), so the call allocates nothing and takes no
 * scratch from the caller.  It may be captured in a HIP graph once
 * lm_moe_static_init() has run on the device.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory - code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc.  At most
 * lm_moe_static_max_tokens() (128) tokens per call (LM_ENOMEM beyond);
 * same results as lm_moe_layer_forward.  Every call on one device shares
 * that device's array: calls that overlap on a device (several streams or
 * host threads) race and must be serialized by the caller. */
int64_t lm_moe_static_max_tokens(void);
/* Resolves the device array of lm_moe_layer_forward_static on the current
 * device (once per device; later calls return at once).  Call it before
 * capturing static calls in a HIP graph: a static call on a device whose
 * array is not resolved yet resolves it itself when its stream is not
 * capturing, and is refused (LM_EINVAL) when it is.  The stream of a static
 * call must belong to the current device (LM_EINVAL otherwise). */
int lm_moe_static_init(void);
int lm_moe_layer_forward_static(const lm_moe_layer *layer, void *h,
                                int64_t tokens, int64_t hidden, int64_t inter,
                                int64_t experts, int64_t top_k, float eps,
                                int32_t *ids_out, void *weights_out,
                                void *const *phase_events, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* LOCALMOE35BA3B_H */
