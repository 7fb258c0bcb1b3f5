/*
 * mlxturbo_amd: C ABI of the MI355X (gfx950) quantized-matmul hot path.
 *
 * Plain C: caller-owned device buffers, sizes in elements, an explicit HIP
 * stream (hipStream_t passed as void*, NULL = default stream), no
 * allocation of user-visible memory, no stream synchronisation, every output
 * element written.  Safe to call from several host threads on different
 * streams.
 *
 * Formats (MLX affine quantization, the format the reference's kernels read:
 * mlxturbo/fast_qmm.py:93-106, kernels/_steel_flat.py:1152-1256):
 *   w       uint32 [N, K*bits/32]   a little-endian bitstream per row: code k
 *                                   at bits [bits*k, bits*k + bits); for 4/8
 *                                   bits, code j of word i = element
 *                                   i*(32/bits)+j at bit bits*j
 *   scales  T [N, K/group_size]     T = the activation dtype
 *   biases  T [N, K/group_size]
 *   deq     T(float(s)*q + float(b)), rounded to nearest even
 * Gather banks add a leading expert dimension E.
 *
 * Status codes: 0 = ok; MQ_EINVAL (-1) = invalid argument (the caller raises
 * ValueError, as MLX does); MQ_EUNSUPPORTED (-2) = valid but not implemented
 * here (caller raises NotImplementedError); > 0 = a hipError_t.  The message
 * of the last non-zero status on the calling thread is in mq_last_error().
 */
#ifndef MLXTURBO_AMD_H
#define MLXTURBO_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MQ_OK 0
#define MQ_EINVAL (-1)
#define MQ_EUNSUPPORTED (-2)

/* dtype codes of x / scales / biases / out */
#define MQ_BFLOAT16 0
#define MQ_FLOAT16 1
#define MQ_FLOAT32 2

/* ABI version; bumped on any signature or contract change. */
int mq_version(void);

/* Message for the last non-zero status returned on this thread. */
const char* mq_last_error(void);

/* Number of kernel launches made by this process (all entry points).  The
 * counterpart of the reference's "fire" counters (mlxturbo/kernels/_fire.py:
 * 17-32) that prove a custom kernel actually ran. */
uint64_t mq_launch_count(void);

/*
 * Row identity across call widths (process-wide, default 0).  One-row
 * calls (M = 1) normally run their own kernel, whose sums are rounded in a
 * different order from the 2..32-row kernels': each row is within the
 * output tolerance of both, not bit-identical to the same row computed in
 * a wider call.  With on != 0, one-row calls run the 2..32-row kernel
 * family, so a row's result does not depend on how many rows the call has
 * (decode vs. speculative verify).  The reference keeps this property with
 * its opt-in small-M route: rows of an M = 2..8 call bit-identical to the
 * M = 1 call (kernels/qmv_small_m.py:289-307, dispatch.py:337-347).
 * Returns the previous setting.  Not for calls running concurrently with a
 * change of the setting.
 */
int mq_set_row_identity(int on);

/*
 * out[N, K] (T) = dequantize(w, scales, biases).
 * Replaces mx.dequantize(w, scales, biases, group_size, bits, mode="affine"),
 * the format definer the reference's fp32 references call
 * (bench/test_qmm_wide_shapes.py:35-42, kernels/moe_verify_gather.py:932).
 * bits in {2, 3, 4, 5, 6, 8} (a row is a little-endian bitstream of K codes:
 * kernels/_steel_flat.py:1158-1167, 1184-1254); group_size in {32, 64, 128};
 * dtype any of the three; w and out 16-byte aligned.
 */
int mq_dequantize(const uint32_t* w, const void* scales, const void* biases, void* out,
                  int64_t N, int64_t K, int group_size, int bits, int dtype, void* hip_stream);

/*
 * (wq, scales, biases) = quantize(w): MLX affine quantization of w[N, K]
 * (dtype T) into wq uint32 [N, K*bits/32] and scales/biases T [N, K/group_size].
 * Replaces mx.quantize(w, group_size, bits, mode="affine") as the reference
 * calls it at runtime (mlxturbo/rebit.py:119 requantizing a layer,
 * spec.py:428) and in its tests (kernels/moe_verify_gather.py:887).  Per
 * group, in float32: scale = max((max-min)/(2^bits-1), 1e-7), negative unless
 * |min| > |max|, snapped so the larger-magnitude edge is a code (scale =
 * edge / round(edge/scale) unless that rounds to 0); bias = that edge (0 when
 * it rounded to 0); code = clamp(round_half_even((w-bias)/scale)), NaN -> 0.
 * bits in {2, 3, 4, 5, 6, 8}; group_size in {32, 64, 128}; w and wq 16-byte
 * aligned (scales/biases too for 16-bit T).
 */
int mq_quantize(const void* w, uint32_t* wq, void* scales, void* biases, int64_t N, int64_t K,
                int group_size, int bits, int dtype, void* hip_stream);

/*
 * out[M, N] = x[M, K] . dequantize(w)^T       (transpose = 1)
 * Replaces mx.quantized_matmul(x, w, scales, biases, transpose=True,
 * group_size, bits, mode="affine") as called by the reference's route layer
 * (mlxturbo/kernels/dispatch.py:302-382, the stock() call at 317-327) and its
 * drop-ins fast_qmm (mlxturbo/fast_qmm.py:334-374), qmv_small_m
 * (kernels/qmv_small_m.py:289-335), qmv_wide_nocap (kernels/
 * qmv_wide_nocap.py:240-288) and qmm_wide (kernels/qmm_wide.py:456-502).
 * x and out are row-major with leading dimension K and N.
 * bits in {4, 8}; group_size in {32, 64, 128}; dtype bfloat16 or float16;
 * other widths, float32 and transpose = 0 return MQ_EUNSUPPORTED (the
 * reference never accelerates them; the Python layer composes mq_dequantize
 * and a GEMM for them, as the reference falls back to stock MLX).
 */
int mq_quantized_matmul(const void* x, const uint32_t* w, const void* scales,
                        const void* biases, void* out, int64_t M, int64_t N, int64_t K,
                        int group_size, int bits, int dtype, int transpose, void* hip_stream);

/*
 * Bytes of device workspace mq_quantized_matmul_ws can use for an M x N x K
 * problem (float partial sums when the K range is split over workgroups:
 * narrow matrices at prefill widths and at 5-64 rows), 0 when the chosen
 * plan needs none.
 * No counterpart in the reference (MLX allocates its own temporaries); it
 * is the sizing call of the entry point below.
 */
size_t mq_quantized_matmul_workspace_size(int64_t M, int64_t N, int64_t K, int group_size,
                                          int bits);

/*
 * mq_quantized_matmul with a caller-provided device workspace of
 * workspace_bytes bytes (16-byte aligned, may be NULL): when it holds
 * mq_quantized_matmul_workspace_size(M, N, K, group_size, bits) bytes, wide
 * problems may split K over workgroups and reduce the partials in a second
 * kernel (same results up to the order of the float sums), and 5-64 rows on
 * matrices of fewer than 640 16-row tiles run their K slices on separate
 * workgroups and add them in a second kernel (every 16 rows get the bits of
 * a 16-row call without the workspace).  Replaces the
 * same mx.quantized_matmul call as mq_quantized_matmul; calls sharing a
 * workspace must be ordered (one stream).
 */
int mq_quantized_matmul_ws(const void* x, const uint32_t* w, const void* scales,
                           const void* biases, void* out, int64_t M, int64_t N, int64_t K,
                           int group_size, int bits, int dtype, int transpose, void* workspace,
                           size_t workspace_bytes, void* hip_stream);

/*
 * Bytes of device workspace mq_gather_qmm needs for P index pairs.
 */
size_t mq_gather_qmm_workspace_size(int64_t P, int64_t M);

/*
 * out[p, M, N] = x[lhs[p], M, K] . dequantize(w[rhs[p]])^T   for p < P.
 * Replaces mx.gather_qmm(x, w, scales, biases, lhs_indices, rhs_indices,
 * transpose=True, group_size, bits, mode="affine", sorted_indices) as called
 * by mlx-lm's QuantizedSwitchLinear / SwitchGLU (fused.py:2389-2394,
 * 2402-2418, 3105-3116) and by the reference's decode/verify gather kernels
 * (kernels/moe_decode_fused.py:331-397, kernels/moe_verify_gather.py:453-875)
 * and prefill grouped GEMM (kernels/moe_grouped_gemm.py:913-1066).
 * x is [B, M, K]; w is [E, N, K*bits/32]; scales/biases [E, N, K/group_size];
 * lhs_indices may be NULL: then pair p reads x batch p / (P / B), which
 * requires B to divide P (B == P: the identity; B == P / top_k: tokens
 * (T, 1) broadcast against their expert indices (T, top_k), mlx-lm's
 * SwitchGLU call, with no index table); indices are int32 device arrays of
 * length P (the caller broadcasts them).  Pairs that
 * share an expert are computed together so each expert's weights are read
 * once per call.  sorted_indices = 1 promises rhs is non-decreasing.
 * workspace must hold mq_gather_qmm_workspace_size(P, M) bytes.
 */
int mq_gather_qmm(const void* x, const uint32_t* w, const void* scales, const void* biases,
                  const int32_t* lhs_indices, const int32_t* rhs_indices, void* out, int64_t P,
                  int64_t B, int64_t M, int64_t N, int64_t K, int64_t E, int group_size, int bits,
                  int dtype, int sorted_indices, void* workspace, size_t workspace_bytes,
                  void* hip_stream);

/*
 * mq_gather_qmm without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference (MLX
 * allocates its own temporaries).  The workspace is a static device array of
 * 4 MiB (MQ_GATHER_NOALLOC_SCRATCH_BYTES) that each GPU holds until the
 * process ends; it takes calls whose mq_gather_qmm_workspace_size(P, M) fits,
 * i.e. up to 261375 pairs, and larger ones return MQ_EINVAL.  The call
 * allocates nothing.  Every call on one GPU shares that GPU's array, so calls
 * that overlap on one GPU (other streams, other threads) race: order them,
 * e.g. on one stream.  Arguments and results are those of mq_gather_qmm.
 */
#define MQ_GATHER_NOALLOC_SCRATCH_BYTES ((size_t)4 << 20)
int mq_gather_qmm_noalloc(const void* x, const uint32_t* w, const void* scales,
                          const void* biases, const int32_t* lhs_indices,
                          const int32_t* rhs_indices, void* out, int64_t P, int64_t B, int64_t M,
                          int64_t N, int64_t K, int64_t E, int group_size, int bits, int dtype,
                          int sorted_indices, void* hip_stream);

/*
 * Segment tables of a MoE layer's prefill gathers, built once for a routing
 * and reused by every gather of the layer over it: the reference builds them
 * once per layer (`tables = _moe_gemm_tables(idx_s, E)`, fused.py:3290) and
 * passes them to the up, gate and down grouped GEMMs (fused.py:3294-3316,
 * kernels/moe_grouped_gemm.py:913-1066).  Pairs as for mq_gather_qmm
 * (lhs_indices NULL: pair p's x batch is p / (P / B)); rows M per pair.
 * tables must hold mq_gather_qmm_workspace_size(P, M) bytes and stay
 * untouched until the last mq_gather_qmm_tables call using them has run.
 * Prefill widths only (P * M >= 1024, E <= 2048, M <= 16), else
 * MQ_EUNSUPPORTED.  Enqueues two kernels.
 */
int mq_gather_tables(const int32_t* lhs_indices, const int32_t* rhs_indices, int64_t P,
                     int64_t B, int64_t M, int64_t E, void* tables, size_t tables_bytes,
                     void* hip_stream);

/*
 * mq_gather_qmm over tables from mq_gather_tables for the same rhs_indices,
 * lhs_indices validity (NULL, or the same table), P, M and E; x, B, N, K
 * and the bank may differ from the call that built them (a layer's gate /
 * up bank over the tokens, its down bank over the SwiGLU rows, B = P).
 * Results are those of mq_gather_qmm, bit for bit.  Runs the thin grouped
 * kernel only: calls that mq_gather_qmm would run on another kernel (more
 * than 96 rows per expert, K > 2048) return MQ_EUNSUPPORTED, and the caller
 * runs mq_gather_qmm.
 */
int mq_gather_qmm_tables(const void* x, const uint32_t* w, const void* scales,
                         const void* biases, const int32_t* lhs_indices,
                         const int32_t* rhs_indices, void* out, int64_t P, int64_t B, int64_t M,
                         int64_t N, int64_t K, int64_t E, int group_size, int bits, int dtype,
                         const void* tables, size_t tables_bytes, void* hip_stream);

/*
 * A prefill MoE layer's gate and up gathers and its SwiGLU in one launch,
 * over tables from mq_gather_tables (same conditions as
 * mq_gather_qmm_tables): out [P * M, N] = mq_swiglu of mq_gather_qmm_tables
 * on the gate bank and on the up bank (both of N x K), bit for bit, with
 * each gathered x tile read once for both banks.  The reference's prefill
 * layer runs the gate and up grouped GEMMs over its shared tables and then
 * the activation (fused.py:3294-3302, kernels/moe_grouped_gemm.py:
 * 913-1066); mlx-lm's SwitchGLU applies it as nn.silu(gate) * up.  Calls the
 * tables' kernel does not take return MQ_EUNSUPPORTED, and the caller makes
 * the three calls.
 */
int mq_gather_swiglu_tables(const void* x, const uint32_t* w_gate, const void* scales_gate,
                            const void* biases_gate, const uint32_t* w_up, const void* scales_up,
                            const void* biases_up, const int32_t* lhs_indices,
                            const int32_t* rhs_indices, void* out, int64_t P, int64_t B,
                            int64_t M, int64_t N, int64_t K, int64_t E, int group_size, int bits,
                            int dtype, const void* tables, size_t tables_bytes,
                            void* hip_stream);

/*
 * The decode MoE block's routing and fused gate+up+SiLU in one launch:
 * mq_moe_route(logits, idx, weights, T, E, top_k, x, sgw, sgate, K, dtype)
 * followed by mq_gather_glu(x [T, 1, K], gate bank, up bank, lhs NULL, rhs
 * idx, out [T * top_k, N], P = T * top_k, B = T, M = 1, ...), bit for bit:
 * every workgroup routes the tokens itself (the routing kernel's pieces) and
 * workgroup 0 writes idx / weights (and, with sgw, sgate) for the down
 * projection that follows (mq_gather_qmm_combine).  The reference runs its
 * decode route (kernels/moe_route_decode.py:151-327) and its fused decode
 * gate/up (kernels/moe_decode_fused.py:331-350) as separate dispatches.
 * Up to 64 pairs (T * top_k) over up to 512 experts; other calls return
 * MQ_EUNSUPPORTED and the caller makes the two calls.
 */
int mq_moe_glu_route(const void* x, const float* logits, const uint32_t* w_gate,
                     const void* scales_gate, const void* biases_gate, const uint32_t* w_up,
                     const void* scales_up, const void* biases_up, const void* sgw, int32_t* idx,
                     float* weights, void* sgate, void* out, int64_t T, int64_t top_k, int64_t N,
                     int64_t K, int64_t E, int group_size, int bits, int dtype,
                     void* hip_stream);

/*
 * The whole decode MoE block of T <= 8 tokens in one launch:
 * mq_moe_glu_route (x [T, K1], logits [T, E], gate / up banks [E, N1, K1]
 * -> idx, weights, sgate, h [T * top_k, N1]) followed by
 * mq_gather_qmm_combine(h, down bank [E, N2, N1], idx, weights, sgate,
 * shared [T, N2] -> out [T, N2]), bit for bit.  The down
 * projection starts behind a grid-wide arrival inside the launch (device-
 * scope stores of h and per-workgroup flags in a static device array of the
 * library), so calls that overlap on one GPU race; a stream's calls run in
 * order.  The reference runs its decode route (kernels/moe_route_decode.py:
 * 151-327), its fused decode gate/up and down (kernels/moe_decode_fused.py:
 * 331-397) and its combine with the shared expert (moe_route_decode.py:
 * 353-398) as separate dispatches.  sgw / sgate / shared are all given or
 * all NULL.  T = 1 .. 8, top_k <= 8, T * top_k <= 64, E <= 512; other
 * calls, tile configurations other than the decode gathers' (gate/up tiles
 * over 4 waves, or over 2 or 1 with the scale copy; down tiles on one
 * wave), or a grid that does not fit the device at once return
 * MQ_EUNSUPPORTED, and the caller makes the two calls.
 */
int mq_moe_block(const void* x, const float* logits, const uint32_t* w_gate,
                 const void* scales_gate, const void* biases_gate, const uint32_t* w_up,
                 const void* scales_up, const void* biases_up, const uint32_t* w_down,
                 const void* scales_down, const void* biases_down, const void* sgw,
                 const void* shared, int32_t* idx, float* weights, void* sgate, void* h,
                 void* out, int64_t T, int64_t top_k, int64_t N1, int64_t K1, int64_t N2,
                 int64_t E, int group_size, int bits, int dtype, void* hip_stream);

/*
 * The decode MoE layer of T <= 8 tokens with its routing given, in one
 * launch: mq_gather_glu(x [T, 1, K1], gate bank, up bank, lhs NULL, rhs idx
 * [T, top_k], h [T * top_k, N1], P = T * top_k, B = T, M = 1, ...) followed
 * by mq_gather_qmm_combine(h, down bank [E, N2, N1], idx, weights
 * [T, top_k] (float router weights), no shared expert -> out [T, N2]), bit
 * for bit, with mq_moe_block's grid-wide arrival (calls that overlap on
 * one GPU race).
 * The reference's decode layer runs its fused gate/up and its down kernel
 * with the combine as separate dispatches (kernels/moe_decode_fused.py:
 * 331-397, kernels/moe_combine.py:160-195; fused.py:2456-2492).  An expert
 * outside [0, E) gives a zero row.  mq_moe_block's limits (T <= 8,
 * top_k <= 8, T * top_k <= 64, E <= 512, tiles, grid), else
 * MQ_EUNSUPPORTED and the caller makes the two calls.
 */
int mq_moe_layer(const void* x, const int32_t* idx, const float* weights, const uint32_t* w_gate,
                 const void* scales_gate, const void* biases_gate, const uint32_t* w_up,
                 const void* scales_up, const void* biases_up, const uint32_t* w_down,
                 const void* scales_down, const void* biases_down, void* h, void* out,
                 int64_t T, int64_t top_k, int64_t N1, int64_t K1, int64_t N2, int64_t E,
                 int group_size, int bits, int dtype, void* hip_stream);

/*
 * out[i] = T(T(silu(gate[i])) * up[i]) for i < n, silu(g) = g / (1 + exp(-g))
 * in float, dtype bf16 or fp16: mlx-lm SwitchGLU's activation between the
 * gate / up and down gathers (`act = switch_mlp.activation(x_up, x_gate)` in
 * the reference's prefill path, fused.py:3302), one pass.
 */
int mq_swiglu(const void* gate, const void* up, void* out, int64_t n, int dtype,
              void* hip_stream);

/*
 * Fused MoE gate+up+SiLU at decode / verify widths:
 *   out[p, M, N] = silu(x[lhs[p]] . dequantize(w_gate[rhs[p]])^T)
 *                * (x[lhs[p]] . dequantize(w_up[rhs[p]])^T)
 * with both products summed in float, silu(g) = g / (1 + exp(-g)) and the
 * product rounded once to dtype.  Replaces kernels/moe_glu.py:145-168
 * (`fused_glu(x_pairs, idx_flat, gate_proj, up_proj)`) and
 * kernels/moe_decode_fused.py:331-350 (`gate_up(x, idx_flat, gate, up,
 * topk)`).  Arguments as mq_gather_qmm, with two banks of one shape
 * ([E, N, K*bits/32], scales/biases [E, N, K/group_size]); the workspace is
 * mq_gather_qmm_workspace_size(P, M) bytes.  P * M >= 1024 output rows
 * (prefill) returns MQ_EUNSUPPORTED: the caller composes two mq_gather_qmm
 * calls there, as the reference keeps its stock path outside decode.
 */
int mq_gather_glu(const void* x, const uint32_t* w_gate, const void* scales_gate,
                  const void* biases_gate, const uint32_t* w_up, const void* scales_up,
                  const void* biases_up, const int32_t* lhs_indices,
                  const int32_t* rhs_indices, void* out, int64_t P, int64_t B, int64_t M,
                  int64_t N, int64_t K, int64_t E, int group_size, int bits, int dtype,
                  void* workspace, size_t workspace_bytes, void* hip_stream);

/*
 * MoE down projection with the combine folded in, at decode widths:
 *   out[t, n] = T( sum_k weights[t*top_k + k] * y[t*top_k + k, n] ),
 *   y[p, n]   = T( x[p] . dequantize(w[rhs[p]])[n]^T )
 * i.e. mq_gather_qmm (x [T*top_k, K], one row per pair, lhs_indices NULL,
 * M = 1) followed by mq_moe_combine (inv NULL), bit for bit, in one launch;
 * with sgate and shared (dtype [T] and [T, N], both or neither) the shared
 * expert is merged as mq_moe_combine_shared does.  The reference runs the two
 * passes (kernels/moe_decode_fused.py:378-397 `down`, then
 * kernels/moe_combine.py:160-195 or moe_route_decode.py:353-398 `combine`);
 * its prefill path folds the router weight into the down projection's store
 * instead (fused.py:3304-3315).  weights float32 [T*top_k], out [T, N].
 * Up to 16 pairs (T * top_k <= 16), fewer where the gather tile splits K
 * over 2 or 4 waves (8 or 4 pairs: each workgroup takes the call's segments
 * in at most two rounds); other calls, and tile configurations this kernel
 * does not cover, return MQ_EUNSUPPORTED, and the caller runs mq_gather_qmm
 * + mq_moe_combine, which is faster there.  Out-of-range experts give y = 0.
 */
int mq_gather_qmm_combine(const void* x, const uint32_t* w, const void* scales,
                          const void* biases, const int32_t* rhs_indices, const float* weights,
                          const void* sgate, const void* shared, void* out, int64_t T,
                          int64_t top_k, int64_t N, int64_t K, int64_t E, int group_size,
                          int bits, int dtype, void* hip_stream);

/*
 * MoE combine epilogue: out[t, n] = sum_k w[t*top_k + k] * y[inv[t*top_k + k], n]
 * for t < rows, accumulated in float in k order and rounded once to dtype.
 * Replaces kernels/moe_combine.py:160-195 (`combine(y, inv, w, rows, top_k)`,
 * the unsort + router weight + top-k sum after the down projection,
 * fused._moe_fold_block combine mode, fused.py:3283-3316).
 * y is [y_rows, N] in expert order (dtype bf16 or fp16), inv int32
 * [rows*top_k] gives the row of y holding token t's k-th expert output
 * (NULL: row t*top_k + k, which requires y_rows >= rows*top_k); an inv entry
 * outside [0, y_rows) contributes nothing (as a zero router weight would), so
 * no index reads outside y.  w float32 [rows*top_k], out [rows, N].
 * N % 8 == 0, 1 <= top_k <= 64, y and out 16-byte aligned.
 */
int mq_moe_combine(const void* y, int64_t y_rows, const int32_t* inv, const float* w, void* out,
                   int64_t rows, int64_t top_k, int64_t N, int dtype, void* hip_stream);

/*
 * mq_moe_combine with the shared expert merged in, as the reference's decode
 * combine does (kernels/moe_route_decode.py:353-398 `combine`, kept off by
 * default there): out[t, n] = T(float(T(sum_k w[t*top_k + k] * y[inv[..], n]))
 * + float(T(sgate[t] * shared[t, n]))), with sgate (dtype [rows]) the
 * already-sigmoided shared-expert gate (mq_moe_route writes it) and shared
 * (dtype [rows, N], 16-byte aligned) the shared expert's output.  Other
 * arguments and limits as mq_moe_combine.
 */
int mq_moe_combine_shared(const void* y, int64_t y_rows, const int32_t* inv, const float* w,
                          const void* sgate, const void* shared, void* out, int64_t rows,
                          int64_t top_k, int64_t N, int dtype, void* hip_stream);

/*
 * MoE routing at decode / verify widths.  Replaces the reference's
 * kernels/moe_route_decode.py:269-327 (`route(logits, top_k, x, sgw)`, kept
 * off by default there; the stock path is argpartition + take_along_axis +
 * softmax(precise) + the shared-expert gate of _vendor/qwen4_exp.py).  For
 * each of `rows` rows of float32 logits [rows, E]: the top_k experts by value
 * in descending order (equal values: the smaller expert index first, as
 * torch.topk decides) into idx (int32 [rows, top_k]), and their softmax
 * weights into weights (float32 [rows, top_k]):
 *   w_j = exp(v_j - v_0) / sum_i exp(v_i - v_0),  summed in float in order.
 * With x (dtype [rows, H]), sgw (dtype [H]) and sgate (dtype [rows]) given,
 * also the shared expert's gate sgate[r] = sigmoid(T(sum_h x[r,h] sgw[h]))
 * (dot in float; sigmoid as MLX evaluates it in T: y = 1 / (1 + exp(|s|)),
 * s < 0 ? y : 1 - y, every operation rounded to T); pass all three NULL to
 * skip it.  E <= 1024 and top_k <= 64 (else MQ_EUNSUPPORTED); dtype bf16 or
 * fp16 when the gate is asked for.
 */
int mq_moe_route(const float* logits, int32_t* idx, float* weights, int64_t rows, int64_t E,
                 int64_t top_k, const void* x, const void* sgw, void* sgate, int64_t H, int dtype,
                 void* hip_stream);

#ifdef __cplusplus
}
#endif

#endif /* MLXTURBO_AMD_H */
