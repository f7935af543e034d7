/* escha_hip — C ABI of the MI355X (gfx950) coded-projection engine.
 *
 * Drop-in boundary for escha-mlx's kernel layer (escha_mlx/msl.py): every
 * entry point takes device pointers and sizes, enqueues on the given HIP
 * stream (hipStream_t passed as void*, NULL = default stream), never
 * allocates, frees or synchronises (except esc_init, once per device), and
 * writes caller-allocated outputs.  Pointer arguments follow the reference's
 * tensors: code is the export's int16 stream viewed as little-endian uint32
 * [..., TK, TN, 8K] (escha_mlx/msl.py:1398-1401); f16 data travels as
 * uint16_t bit patterns.
 *
 * Return value: 0 on success, a negative ESC_E* code otherwise; the message
 * is then available from esc_last_error() (thread-local).  Preconditions the
 * reference raises ValueError for (escha_mlx/dense.py:170-242,
 * msl.py:1794-1823) are checked here and return ESC_EINVAL.
 */
#ifndef ESCHA_HIP_H
#define ESCHA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ESC_OK 0
#define ESC_EINVAL (-1)   /* shape / K / pointer precondition violated */
#define ESC_EHIP (-2)     /* the HIP runtime reported an error           */
#define ESC_ENOSPACE (-3) /* workspace smaller than the *_workspace size */
#define ESC_ETIMEOUT (-4) /* an earlier single-launch expert-path call on the
                             device gave up a bounded wait (NaN outputs)    */

/* ABI version (major*100 + minor). */
int esc_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* esc_last_error(void);

/* Build the 65,536-entry decode table on the current device (idempotent,
 * synchronous).  Called implicitly by the first table-decode entry point on
 * a device; call it explicitly before capturing a HIP graph.
 * Replaces the host-built table upload msl._lut_array (escha_mlx/msl.py:1074-1076). */
int esc_init(void);

/* code u32 [TK][TN][8K] -> w f16 [IC][OC] (bit-exact decode).
 * Mirrors msl.decode_tiles (escha_mlx/msl.py:1404-1421). */
int esc_decode_tiles(const uint32_t* code, int K, int IC, int OC, int use_lut, uint16_t* w,
                     void* stream);

/* xh = f16(H128(f32(rows) * rin[e]) * RS), rows f16 [m][IC]; rin f32 [E][IC]
 * gathered by row_expert [m], or rin [IC] when row_expert is NULL.
 * Mirrors msl.scaled_had / dense_scaled_had (escha_mlx/msl.py:1029-1047, 1481-1483). */
int esc_input_transform(const uint16_t* rows, const float* rin, const int32_t* row_expert, int m,
                        int IC, float rs, uint16_t* out, void* stream);

/* Element types of the rows esc_input_transform_typed reads. */
#define ESC_ROWS_F16 0
#define ESC_ROWS_BF16 1
#define ESC_ROWS_F32 2

/* esc_input_transform for rows of another element type: rows [m][IC] of
 * f16, bf16 or f32 (dtype ESC_ROWS_*), converted exactly to f32 before the
 * transform (no f16 rounding of the rows), xh f16 [m][IC] out.  f16 rows give
 * esc_input_transform's result.  Mirrors the reference's transform of
 * non-f16 rows, xr = rows.astype(f32) * rin; f16(H128(xr) * RS)
 * (escha_mlx/dense.py:287-292, escha_mlx/models/qwen3_5_moe.py:103-110). */
int esc_input_transform_typed(const void* rows, int dtype, const float* rin,
                              const int32_t* row_expert, int m, int IC, float rs, uint16_t* out,
                              void* stream);

/* y = f16((H128(mid) * RS) * rout[e]) [+ bias f16 [OC], added in f32].
 * Mirrors msl.scaled_had_out / dense_scaled_had_out (escha_mlx/msl.py:1050-1067, 1486-1488)
 * and the bias step of EschaLinear.__call__ (escha_mlx/dense.py:356-361). */
int esc_output_transform(const float* mid, const float* rout, const int32_t* row_expert,
                         const uint16_t* bias, int m, int OC, float rs, uint16_t* out,
                         void* stream);

/* mid f32 [M][OC] = xh f16 [M][IC] @ decode(code[row_expert[r]]), in the
 * reference kernels' exact float32 order (bit-reproducible).  code is
 * [E][TK][TN][8K], or [TK][TN][8K] with row_expert NULL (dense).
 * Mirrors msl.moe_gemv / dense_gemv with splits=1 (escha_mlx/msl.py:1424-1478, 1530-1538). */
int esc_gemv(const uint16_t* xh, const uint32_t* code, const int32_t* row_expert, int M, int K,
             int IC, int OC, int use_lut, float* mid, void* stream);

/* Tolerance-contract GEMV (split-K, reassociated float32 sum, deterministic):
 * same arguments and result shape as esc_gemv; ws = float workspace of
 * esc_gemv_fast_workspace(M, K, IC, OC) bytes; out f16 [M][OC] is the fused
 * output transform with rout ([E][OC] gathered by row_expert, or [OC]).
 * Replaces msl.moe_gemv + msl.scaled_had_out (escha_mlx/msl.py:1424, 1050). */
size_t esc_gemv_fast_workspace(int M, int K, int IC, int OC);
int esc_gemv_fast_out(const uint16_t* xh, const uint32_t* code, const int32_t* row_expert,
                      const float* rout, int M, int K, int IC, int OC, int use_lut, float rs,
                      uint16_t* out, void* ws, size_t ws_bytes, void* stream);

/* Row-blocked expert GEMM, bit-identical to esc_gemv per row.  xh
 * [n_rows+1][IC] with row n_rows all zeros (padding sink); rows_idx
 * [n_groups*R] (padding = n_rows); group_expert [n_groups] (-1 = skip);
 * mid [n_rows+1][OC].  R in {1,2,3,4,8,12,16}.
 * Mirrors msl.moe_gemm_rows (escha_mlx/msl.py:1366-1395). */
int esc_gemm_rows(const uint16_t* xh, const uint32_t* code, const int32_t* rows_idx,
                  const int32_t* group_expert, int n_groups, int R, int n_rows, int K, int IC,
                  int OC, int use_lut, float* mid, void* stream);

/* Dense row-blocked GEMM: group g owns rows [gR, gR+R); bit-identical to
 * esc_gemv.  R in {1,2,4,8,16}.  Mirrors msl.dense_gemm_rows /
 * dense_gemm_rows_direct (escha_mlx/msl.py:1785-1841). */
int esc_dense_gemm_rows(const uint16_t* xh, const uint32_t* code, int M, int R, int K, int IC,
                        int OC, int use_lut, float* mid, void* stream);

/* Dense rows with the output transform fused: out f16 [M][OC].  R in {1,2,4,8}.
 * Mirrors msl.dense_gemm_rows_direct_out (escha_mlx/msl.py:1844-1870). */
int esc_dense_gemm_rows_out(const uint16_t* xh, const uint32_t* code, const float* rout, int M,
                            int R, int K, int IC, int OC, int use_lut, float rs, uint16_t* out,
                            void* stream);

/* mid f32 [M][OC] = xh f16 [M][IC] @ decode(code [TK][TN][8K]) on the matrix
 * cores: for OC a multiple of 256, v_mfma_f32_16x16x32_f16 with the weights
 * decoded straight into A operands (16*NRB rows x 256 columns per workgroup,
 * NRB chosen per shape); otherwise v_mfma_f32_32x32x16_f16 on weights decoded
 * into LDS (256 rows x 128 columns per workgroup).
 * Decoded weights are bit-exact; the float32 sum is reassociated
 * (deterministic; tolerance contract).  use_lut is accepted for the call
 * surface: table and hash decode give identical weights.
 * Mirrors msl.dense_gemm_mat (escha_mlx/msl.py:1762-1782, source 1608-1708). */
int esc_gemm_mfma(const uint16_t* xh, const uint32_t* code, int M, int K, int IC, int OC,
                  int use_lut, float* mid, void* stream);

/* The many-row GEMM and its output transform in one step: y f16 [M][OC] =
 * (bias +) f16((H128(xh @ decode(code)) * rs) * rout), xh f16 [M][IC] already
 * input-transformed.  For OC a multiple of 256 the transform runs in the
 * epilogue of esc_gemm_mfma's kernel (no f32 mid; ws unused, the workspace
 * size is 0); otherwise esc_gemm_mfma into ws (esc_gemm_mfma_out_workspace
 * bytes, M * OC f32), then esc_output_transform.  Bit-identical to those two
 * calls; deterministic, reassociated float32 sum (tolerance contract).
 * Replaces EschaLinear's many-row path, self._output_rows(self._gemv(xh))
 * (escha_mlx/dense.py:356): msl.dense_gemm_mat then msl.dense_scaled_had_out
 * (escha_mlx/msl.py:1762-1782, 1486-1489). */
size_t esc_gemm_mfma_out_workspace(int M, int K, int IC, int OC);
int esc_gemm_mfma_out(const uint16_t* xh, const uint32_t* code, const float* rout,
                      const uint16_t* bias, int M, int K, int IC, int OC, float rs, uint16_t* y,
                      void* ws, size_t ws_bytes, void* stream);

/* The whole coded linear, y f16 [M][OC] = (bias +) f16((H128(xh @ W) * rs) *
 * rout) with xh = f16(H128(f32(x) * rin) * rs), x f16 [M][IC], rin f32 [IC],
 * rout f32 [OC], bias f16 [OC] or NULL (added in f32 after the f16 round).
 * M < 16: one launch (in-block input transform).  One row: with the table
 * decode and at least 16,384 units (kt x 256-column groups) the persistent
 * kernel (one workgroup per CU stages the table once, units split evenly
 * over its waves), otherwise the split-K GEMV by hash (packed dot2 on the
 * VALU; the decodes give the same weights); 2..15 rows: split-K by hash
 * whichever decode is asked for, the rows of a group (all rows, or two
 * groups when one would leave the GPU short of workgroups) sharing each
 * decoded weight on the matrix core.  The last split of each column group
 * sums the partials in fixed order and output-transforms.
 * M >= 16: input transform, then esc_gemm_mfma_out.  ws: esc_linear_workspace bytes, zero-filled before its
 * first use (its counters are left zero after every call); calls sharing one
 * ws must not overlap, and a ws moved to another shape is zero-filled again
 * (each shape's plan puts its counters where another's partials may lie).  Tolerance contract (reassociated float32 sum);
 * decoded weights bit-exact.
 * Replaces EschaLinear.__call__ (escha_mlx/dense.py:337-362). */
size_t esc_linear_workspace(int M, int K, int IC, int OC);
int esc_linear(const uint16_t* x, const float* rin, const uint32_t* code, const float* rout,
               const uint16_t* bias, int M, int K, int IC, int OC, int use_lut, float rs,
               uint16_t* y, void* ws, size_t ws_bytes, void* stream);

/* Two coded linears over the same rows x f16 [M][IC] in one dispatch:
 * y0 = esc_linear(x; rin0, code0, rout0, bias0, K0, OC0) and likewise y1
 * (K0 and K1 may differ), each bit-identical to its own esc_linear call.
 * M < 16: one launch whose workgroups run either projection's plan; M >= 16:
 * the two linears one after the other.  ws: esc_linear_pair_workspace bytes
 * (projection 0's esc_linear workspace, then projection 1's), zero-filled
 * before its first use.  Replaces dense.project_pair with msl.dense_gemm_pair
 * / dense_gemm_pair_out and the pair transforms (escha_mlx/dense.py:365-437,
 * escha_mlx/msl.py:1491-1527, 1873-1950): the gate/up and k/v projections. */
size_t esc_linear_pair_workspace(int M, int K0, int K1, int IC, int OC0, int OC1);
int esc_linear_pair(const uint16_t* x, int M, int IC, const float* rin0, const uint32_t* code0,
                    const float* rout0, const uint16_t* bias0, int K0, int OC0, const float* rin1,
                    const uint32_t* code1, const float* rout1, const uint16_t* bias1, int K1,
                    int OC1, int use_lut, float rs, uint16_t* y0, uint16_t* y1, void* ws,
                    size_t ws_bytes, void* stream);

/* n (1 to 4) coded linears of the same input rows x f16 [M][IC]:
 * y[i] = esc_linear(x; rin[i], code[i], rout[i], bias[i], K, OC[i]) for the
 * projections of one input (an attention block's q, k and v), all with the
 * same K.  code, rin, rout, bias (may be null, or hold nulls), OC and y are
 * host arrays of n entries (device pointers).  One row: every OC[i] a
 * multiple of 256, one persistent launch whose projections share one plan
 * (units per wave from their total), so each output is within the tolerance
 * contract of its own esc_linear call, not bit-identical to it.  2..15 rows:
 * one split-K launch whose workgroups run each projection's own esc_linear
 * plan (bit-identical to its own call) when the plans have one row-group
 * size, else one esc_linear call each; 16 rows and more: one esc_linear call
 * each.  ws: esc_linear_multi_workspace bytes, zero-filled before its first
 * use (its counters are left zero).  No counterpart in the reference, which
 * computes the three projections as separate EschaLinear calls
 * (escha_mlx/dense.py:337-362) and pairs two projections for several rows
 * (dense.py:365-437). */
size_t esc_linear_multi_workspace(int M, int n, int K, int IC, const int* OC);
int esc_linear_multi(const uint16_t* x, int M, int IC, int K, int n, const uint32_t* const* code,
                     const float* const* rin, const float* const* rout,
                     const uint16_t* const* bias, const int* OC, int use_lut, float rs,
                     uint16_t* const* y, void* ws, size_t ws_bytes, void* stream);

/* Dense GEMM for a few rows, tolerance contract: y f16 [M][OC] =
 * f16((H128(xh @ decode(code)) * rs) * rout), R rows (2, 4 or 8) per
 * workgroup share every decoded weight (one row per B column of
 * v_mfma_f32_16x16x32_f16); split-K partials in ws
 * (esc_gemm_rows_fast_workspace bytes), summed in fixed order.  Deterministic;
 * reassociated float32 sum.  The decode-once-per-R-rows policy of
 * msl.dense_gemm_rows_direct_out (escha_mlx/msl.py:1844-1870, used by
 * EschaLinear at 1 < M, R <= 8: escha_mlx/dense.py:346-355), split along K. */
size_t esc_gemm_rows_fast_workspace(int M, int R, int K, int IC, int OC);
int esc_gemm_rows_fast_out(const uint16_t* xh, const uint32_t* code, const float* rout, int M,
                           int R, int K, int IC, int OC, int use_lut, float rs, uint16_t* out,
                           void* ws, size_t ws_bytes, void* stream);

/* Sort rows by expert into R-row groups (integer only, on device).
 * rows_idx [n_groups*R], group_expert [n_groups].
 * Mirrors moe.build_groups (escha_mlx/moe.py:30-78). */
int esc_build_groups(const int32_t* row_expert, int m, int E, int R, int n_groups,
                     int32_t* rows_idx, int32_t* group_expert, void* stream);

/* Router: logits f32 [T][E] -> ids [T][k] (descending, ties -> lower id) and
 * scores f32 [T][k] (softmax over the k values).  E <= 1024, k <= 32.
 * Mirrors the routing of EschaSparseMoeBlock.__call__
 * (escha_mlx/models/qwen3_5_moe.py:257-263) in ref.moe_block's stable order
 * (escha_mlx/ref.py:326-331). */
int esc_route_topk(const float* logits, int T, int E, int top_k, int32_t* ids, float* scores,
                   void* stream);

/* h f16 [m][I] = f16(f16(g / (1 + exp(-g))) * u), gate = first half of gu f16 [m][2I].
 * Mirrors ref.swiglu (escha_mlx/ref.py:296-301) / models/qwen3_5_moe.py:221-223. */
int esc_swiglu(const uint16_t* gu, int m, int I, uint16_t* h, void* stream);

/* y f16 [T][H] = f16(sum over slots s in order of f32(d16[t*k+s]) * f32(f16(scores[t*k+s]))).
 * Mirrors the weighted segmented sum of _expert_path (escha_mlx/models/qwen3_5_moe.py:227-253). */
int esc_moe_combine(const uint16_t* d16, const float* scores, int T, int top_k, int H,
                    uint16_t* y, void* stream);

/* Dense w8a16 linear: y f16 [M][O] = f16(f32-accumulated x @ wf^T) with
 * wf = f16(f32(w8) * f32(scale)), w8 int8 [O][K] (one output channel per row),
 * scale f32 [O], x f16 [M][K]; K a multiple of 16 in [128, 8192].  Each weight is
 * rounded as the contract states; the float32 sum is reassociated (tolerance
 * contract, deterministic).  The contract of EschaQ8Linear
 * (escha_mlx/quant.py:1-30, CPU statement ref.w8a16, escha_mlx/ref.py:308-311):
 * the shared expert's gate/up/down and the vocabulary head. */
int esc_w8a16(const uint16_t* x, const int8_t* w8, const float* scale, int M, int K, int O,
              uint16_t* y, void* stream);

/* f16-weight linear without bias: y f16 [M][O] = f16(f32-accumulated x @ w^T),
 * w f16 [O][K], K a multiple of 8 in [64, 4096].  The router gate and the shared
 * expert gate of the MoE block (escha_mlx/models/qwen3_5_moe.py:259, 271;
 * ref.moe_block, escha_mlx/ref.py:324, 347). */
int esc_gemv_f16w(const uint16_t* x, const uint16_t* w, int M, int K, int O, uint16_t* y,
                  void* stream);

/* Shared-expert activation: hh f16 [m][I] = f16((g / (1 + exp(-g))) * u) in
 * float32 from the f16 gate and up outputs (escha_mlx/ref.py:345,
 * models/qwen3_5_moe.py:268). */
int esc_moe_shared_act(const uint16_t* g, const uint16_t* u, int m, int I, uint16_t* hh,
                       void* stream);

/* MoE block output: out f16 [m][H] = f16(f32(y) + f32(sh) * sigmoid(f32(shg))),
 * y the f16 routed sum, sh f16 [m][H] the shared expert's output, shg f16 [m]
 * the shared-expert gate logit (models/qwen3_5_moe.py:250-253, 270-272). */
int esc_moe_block_out(const uint16_t* y, const uint16_t* sh, const uint16_t* shg, int m, int H,
                      uint16_t* out, void* stream);

/* int8 embedding lookup: out f16 [T][K] = f16(f32(w8[ids[t]]) * f32(scale[ids[t]])),
 * w8 int8 [N][K] (K a multiple of 16), scale f32 [N], ids int32 [T]: the
 * dequantised rows of EschaQ8Embedding (escha_mlx/quant.py:253-266; the same
 * rounding as the w8a16 linear's weights).  An id outside [0, N) yields a row
 * of f16 NaN rather than a read outside the table. */
int esc_q8_embed(const int32_t* ids, int T, const int8_t* w8, const float* scale, int N, int K,
                 uint16_t* out, void* stream);

/* Routed-expert path for T tokens: y f16 [T][H] = f16(sum over the k slots,
 * in slot order, of f32(d16) * f32(f16(score))), where per (token, slot):
 * gate_up linear (H -> 2I, K_gu) -> swiglu -> down linear (I -> H, K_dn).
 * gu_code [E][H/16][2I/16][8K_gu], gu_rin [E][H], gu_rout [E][2I],
 * dn_code [E][I/16][H/16][8K_dn], dn_rin [E][I], dn_rout [E][H] (f32).
 * Tolerance contract (reassociated GEMV sums; decode bit-exact).  ws:
 * esc_moe_expert_path_workspace bytes, zero-filled before its first use (the
 * counters it holds are left zero by every call); calls sharing one ws must
 * not overlap, and a ws moved to another shape, or between this entry point
 * and esc_moe_expert_path_one_launch, is zero-filled again (each plan puts its
 * counters where another's partials may lie).  Shapes that run as one persistent launch (H or I not a
 * multiple of 512) hand work between workgroups with bounded waits: a
 * workgroup that gives up writes NaN outputs and raises a device-wide flag,
 * and the next call on the device that would take that launch returns
 * ESC_ETIMEOUT without running (the flag is read without a synchronisation;
 * esc_moe_status reads it at once).  use_lut: the decode table (the hash's
 * image, same outputs) where a kernel uses it; above 64 routed rows with at
 * least one row per expert the grouped GEMMs then run as one persistent
 * launch that stages the table once per CU.
 * Replaces EschaSparseMoeBlock._expert_path (escha_mlx/models/qwen3_5_moe.py:207-253). */
size_t esc_moe_expert_path_workspace(int T, int top_k, int E, int H, int I);
int esc_moe_expert_path(const uint16_t* x, const int32_t* ids, const float* scores, int T,
                        int top_k, int E, int H, int I, const uint32_t* gu_code,
                        const float* gu_rin, const float* gu_rout, int K_gu,
                        const uint32_t* dn_code, const float* dn_rin, const float* dn_rout,
                        int K_dn, int use_lut, uint16_t* y, void* ws, size_t ws_bytes,
                        void* stream);

/* esc_moe_expert_path as one persistent launch at every shape it takes
 * (T*top_k <= 64, top_k <= 32, H a multiple of 256 up to 7936, I a multiple
 * of 128; others return ESC_EINVAL): gate_up items, the SwiGLU hand-off,
 * down items and the slot combine in one dispatch, handing work between
 * workgroups with the bounded waits described above.  Same arguments,
 * workspace, outputs and tolerance contract as esc_moe_expert_path, which
 * takes this launch by itself only where H or I is not a multiple of 512 (at
 * the others two launches measured faster on MI355X).  No counterpart in the
 * reference as a separate call: it is the one-launch walk of the selected
 * experts' gate/up/down stacks, for callers that want one dispatch per
 * token-layer. */
int esc_moe_expert_path_one_launch(const uint16_t* x, const int32_t* ids, const float* scores,
                                   int T, int top_k, int E, int H, int I,
                                   const uint32_t* gu_code, const float* gu_rin,
                                   const float* gu_rout, int K_gu, const uint32_t* dn_code,
                                   const float* dn_rin, const float* dn_rout, int K_dn,
                                   int use_lut, uint16_t* y, void* ws, size_t ws_bytes,
                                   void* stream);

/* esc_moe_expert_path without allocation: the same computation and outputs
 * (the same kernels), with its scratch (partials, counters, down inputs) in a
 * file-scope device array of esc_moe_expert_path_static_max() bytes (4 MiB)
 * that each GPU holds until the process ends, instead of a caller workspace.
 * No counterpart in the reference: it is for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  The call itself allocates nothing: the array's device address
 * is looked up and its counter region zeroed by esc_init() (or by the first
 * call on a device, which launches a fill kernel and synchronises: a call on
 * a stream under graph capture before esc_init() on the device returns
 * ESC_EINVAL, so capturing callers run esc_init() first).  Shapes whose plan
 * needs more scratch are rejected with ESC_ENOSPACE (T * top_k <= 64 rows at
 * H = 2048, I = 512 fit).  Every call on a GPU shares that GPU's array: calls
 * that overlap on one GPU (concurrent streams, threads) race and must be
 * serialised by the caller.  The status flag of a bounded wait that gave up
 * sits in the counter region's last word, outside every shape's counters.
 * use_lut needs esc_init() on the device first. */
size_t esc_moe_expert_path_static_max(void);
int esc_moe_expert_path_static(const uint16_t* x, const int32_t* ids, const float* scores, int T,
                               int top_k, int E, int H, int I, const uint32_t* gu_code,
                               const float* gu_rin, const float* gu_rout, int K_gu,
                               const uint32_t* dn_code, const float* dn_rin,
                               const float* dn_rout, int K_dn, int use_lut, uint16_t* y,
                               void* stream);

/* One token-layer of routed experts for esc_moe_expert_path_layers (device
 * pointers; the same tensors esc_moe_expert_path takes). */
typedef struct {
  const uint16_t* x;
  const int32_t* ids;
  const float* scores;
  const uint32_t* gu_code;
  const float* gu_rin;
  const float* gu_rout;
  const uint32_t* dn_code;
  const float* dn_rin;
  const float* dn_rout;
  uint16_t* y;
} esc_moe_layer;

/* L independent token-layers of routed experts in one launch (throughput
 * mode: large items, the layers' work overlaps).  layers = device array of L
 * records; every layer has the same T, top_k, E, H, I, K_gu, K_dn.  ws must be
 * zero-filled before its first use (esc_moe_layers_workspace bytes); the call
 * leaves its counters zero.  No counterpart in the reference: it is the
 * steady-state form of EschaSparseMoeBlock._expert_path
 * (escha_mlx/models/qwen3_5_moe.py:207-253) for callers that hold several
 * independent token-layers at once (pipelined or multi-request decode). */
size_t esc_moe_layers_workspace(int L, int T, int top_k, int H, int I);
int esc_moe_expert_path_layers(const esc_moe_layer* layers, int L, int T, int top_k, int E, int H,
                               int I, int K_gu, int K_dn, void* ws, size_t ws_bytes,
                               void* stream);

/* Diagnostic: *host_flag = 1 if a one-launch expert path run with this
 * workspace, or any such run on the current device, hit its bounded wait
 * since the flags were last read (never expected: the kernel's work claiming
 * guarantees progress; the outputs of an item that gave up are NaN, never
 * stale values).  Reading clears both flags, so the next esc_moe_expert_path
 * call does not also return ESC_ETIMEOUT for it.  At shapes that
 * esc_moe_expert_path runs as two launches (H and I multiples of 512), only
 * the device-wide flag is read (a run of esc_moe_expert_path_one_launch sets
 * it).  Synchronises the stream.
 * No counterpart in the reference (its expert path has no cross-workgroup
 * hand-off). */
int esc_moe_status(const void* ws, size_t ws_bytes, int T, int top_k, int H, int I,
                   int32_t* host_flag, void* stream);

/* Test hook (no counterpart in the reference): the number of polls a wait of
 * the one persistent expert launch makes before giving up, for every later
 * call in the process; polls < 0 restores the default (2^18).  0 makes every
 * wait give up at once, so the failure reporting can be tested with kernels
 * that still run to their end. */
int esc_moe_set_spin_limit(int polls);

/* Decode-rate probe (measurement only; no counterpart in the reference): the
 * K=2 decode + dot2 loop of the expert GEMVs streamed by persistent
 * workgroups (waves_per_cu 16 or 32) over `code` (esc_decode_probe_words
 * words: every wave reads `steps` wave-steps of 1 KiB, steps a multiple of
 * 4, `prefetch` (1-3) steps ahead), with nt of every 8 step pairs decoded
 * from the table in LDS (nt in 0, 2, 3, 4, 5, 6, 8; nt > 0 needs 16 waves
 * per CU) and the rest by hash.  out: one float per lane (steps * 256 code
 * words per 64 outputs), each lane's sum of x * w over its weights with
 * fixed inputs x.  Bounds the rate of any kernel built on this decode. */
size_t esc_decode_probe_words(int steps, int waves_per_cu);
int esc_decode_probe(const uint32_t* code, int steps, int nt, int waves_per_cu, int prefetch,
                     float* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ESCHA_HIP_H */
