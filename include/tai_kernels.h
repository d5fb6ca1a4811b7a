/*
 * tai_kernels.h - C ABI of libtai_kernels.so, the gfx950 (MI355X) kernels that serve
 * the fused inference operators TorchAir lowers FX graphs onto.
 *
 * Conventions shared by every entry point
 *   - Plain device pointers and sizes; no framework types cross this boundary.
 *   - dtype codes are torch ScalarType codes, the same integers TorchAir's converters
 *     pass as dst_type / output_dtype (python/torchair/ge/_ge_graph.py:215,
 *     python/torchair/_ge_concrete_graph/ge_converter/custom/grouped_matmul.py:178-195).
 *   - The caller owns every buffer. The library never allocates device memory and never
 *     synchronises; every kernel is enqueued on `stream` (a hipStream_t), so a call may be
 *     captured into a hipGraph. Data-dependent sizes (sequence lengths, block tables,
 *     group lists) are read on the device, so a graph replay with new values is correct.
 *   - Return 0 on success; otherwise a TAI_ERR_* code, with a message in tai_last_error()
 *     (thread-local).
 *   - Entry points that need scratch memory take (workspace, ws_bytes) and export a
 *     *_workspace_size() query (the role of the reference's
 *     _npu_fused_infer_attention_score_get_max_workspace, python/torchair/_acl_concrete_graph/acl_graph.py:100-108).
 */
#ifndef TAI_KERNELS_H_
#define TAI_KERNELS_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* torch ScalarType codes */
#define TAI_DT_UINT8 0
#define TAI_DT_INT8 1
#define TAI_DT_INT16 2
#define TAI_DT_INT32 3
#define TAI_DT_INT64 4
#define TAI_DT_FP16 5
#define TAI_DT_FP32 6
#define TAI_DT_BF16 15
#define TAI_DT_NONE (-1)

#define TAI_OK 0
#define TAI_ERR_INVALID 1     /* bad argument (shape, dtype, null pointer) */
#define TAI_ERR_UNSUPPORTED 2 /* valid for the reference, not implemented here */
#define TAI_ERR_LAUNCH 3      /* HIP runtime error */
#define TAI_ERR_WORKSPACE 4   /* workspace smaller than *_workspace_size() */

/* Layout of the second GEMM operand. */
#define TAI_LAYOUT_KN 0 /* row-major [K, N] (N contiguous) */
#define TAI_LAYOUT_NK 1 /* row-major [N, K] (K contiguous): the transpose_x2 / weight.t() view */
/* [K, N] with the gate and up halves of a SwiGLU weight interleaved in 64-column blocks: column
   128t + j is gate column 64t + j for j < 64 and up column N/2 + 64t + j - 64 otherwise
   (tai_grouped_matmul_swiglu_quant only; tai_swiglu_pack_kn writes it) */
#define TAI_LAYOUT_KN_SWIGLU 2

/* Cache layouts of npu_scatter_pa_kv_cache (cache_mode). */
#define TAI_CACHE_NORM 0  /* [num_blocks, block_size, row]: a slot's row is contiguous */
#define TAI_CACHE_PA_NZ 1 /* [num_blocks, row_bytes / 32, block_size, 32 bytes] (FRACTAL_NZ) */

const char* tai_last_error(void);
int tai_abi_version(void);
/* Hash of the sources and build flags the library was compiled from. The Python loader refuses a
 * library whose id differs from the hash of the sources beside it (a stale build). */
const char* tai_build_id(void);
/* Measurement helper, no counterpart in the reference: reads read_bytes of src once (non-temporal
 * 16-byte loads) and then writes write_bytes to dst. Its known byte counts give the read-dominated
 * HBM rate that the benchmark compares read-heavy kernels with. Sizes: multiples of 16 bytes,
 * write_bytes <= read_bytes (the words written are copies of words read). */
int tai_calib_read_stream(const void* src, size_t read_bytes, void* dst, size_t write_bytes, void* stream);

/* ---------------------------------------------------------------------------------------
 * npu_dynamic_quant: symmetric per-row int8 quantisation.
 * Replaces ge.DynamicQuant emitted by
 *   python/torchair/_ge_concrete_graph/ge_converter/custom/npu_dynamic_quant.py:8-42
 *   (prototype third_party/ascend/include/ops/op_proto/inc/nn_quantize.h:47-56).
 * x: [rows, cols] of x_dtype (BF16/FP16/FP32). smooth_scales: NULL, [cols] or
 * [num_groups, cols] fp32. group_index: NULL or [num_groups] cumulative row ends
 * (index dtype INT32/INT64); row r uses smooth row g = first g with r < group_index[g].
 * y: [rows, cols] int8, scale: [rows] fp32.
 * ------------------------------------------------------------------------------------- */
int tai_dynamic_quant(const void* x, int x_dtype, int64_t rows, int64_t cols,
                      const float* smooth_scales, const void* group_index, int group_index_dtype,
                      int64_t num_groups, int8_t* y, float* scale, void* stream);

/* ---------------------------------------------------------------------------------------
 * npu_dynamic_quant with quant_mode "pertensor" or dst_type_max != 0 (symmetric) and
 * npu_dynamic_quant_asymmetric: ge.DynamicQuantV2 emitted by
 *   python/torchair/_ge_concrete_graph/ge_converter/custom/npu_dynamic_quant.py:21-25, 47-61
 *   (prototype third_party/ascend/include/ops/op_proto/inc/nn_quantize.h:77-85).
 * x, smooth_scales, group_index as for tai_dynamic_quant. Per row (per_tensor 0) or over the whole
 * input (per_tensor 1), of the smoothed values xs with maximum mx and minimum mn:
 *   symmetric:  scale = max(|mx|, |mn|) / q (q = dst_type_max, 127 when 0),
 *               y = clamp(rint(xs / scale), -128, 127);
 *   asymmetric: hi = max(mx, 0), lo = min(mn, 0), scale = (hi - lo) / 255,
 *               offset = -128 - lo / scale, y = clamp(rint(xs / scale + offset), -128, 127).
 * A zero range gives scale 0 (offset 0) and y 0. y: [rows, cols] int8; scale (and offset for the
 * asymmetric mode): [rows] fp32, or [1] per tensor. workspace: tai_dynamic_quant_v2_workspace_size.
 * ------------------------------------------------------------------------------------- */
size_t tai_dynamic_quant_v2_workspace_size(int64_t rows);
int tai_dynamic_quant_v2(const void* x, int x_dtype, int64_t rows, int64_t cols,
                         const float* smooth_scales, const void* group_index,
                         int group_index_dtype, int64_t num_groups, int symmetric, int per_tensor,
                         float dst_type_max, int8_t* y, float* scale, float* offset,
                         void* workspace, size_t ws_bytes, void* stream);

/* ---------------------------------------------------------------------------------------
 * npu_swiglu: y = silu(a) * b, a and b the first and second halves of x along one dimension;
 * x viewed as [outer, 2 * n, inner] (the split dimension in the middle), y as [outer, n, inner];
 * bf16 / fp16 / fp32 (dtype), fp32 arithmetic, one rounding to the dtype.
 * Replaces ge.SwiGlu emitted by
 *   python/torchair/_ge_concrete_graph/ge_converter/custom/npu_swiglu.py:4-14.
 * ------------------------------------------------------------------------------------- */
int tai_swiglu(const void* x, int dtype, int64_t outer, int64_t n, int64_t inner, void* y, void* stream);

/* ---------------------------------------------------------------------------------------
 * npu_dequant_swiglu_quant (quant_mode=1 dynamic, swiglu_mode=0, round_mode=0 rint).
 * Replaces ge.DequantSwigluQuant emitted by
 *   python/torchair/_ge_concrete_graph/ge_converter/custom/npu_dequant_swiglu_quant.py:5-47
 *   (prototype experiment_ops.h:3765-3812; meta
 *   python/torchair/_contrib/custom_torch_ops/auto_register_custom_torch_ops.py:155-191).
 * x: [rows, 2n] int32. weight_scale: [2n] fp32 or, with group_index, [num_groups, 2n].
 * activation_scale: NULL or [rows] fp32. bias: NULL or [2n] / [num_groups, 2n] of
 * bias_dtype (INT32 added before dequant; FP32 added after). quant_scale: NULL, [n] or
 * [num_groups, n] fp32. group_index: NULL or [num_groups] per-group row COUNTS (INT32/INT64);
 * rows past the total are written as y=0, scale=0.
 * y: [rows, n] int8, scale: [rows] fp32.
 * ------------------------------------------------------------------------------------- */
int tai_dequant_swiglu_quant(const int32_t* x, int64_t rows, int64_t n2,
                             const float* weight_scale, const float* activation_scale,
                             const void* bias, int bias_dtype, const float* quant_scale,
                             const void* group_index, int group_index_dtype, int64_t num_groups,
                             int activate_left, int8_t* y, float* scale, void* stream);
/* The same with quant_mode 0 (static, the converter's default, npu_dequant_swiglu_quant.py:26-28 ->
 * ge.DequantSwigluQuant quant_mode "static", experiment_ops.h:3765-3812): y = clamp(rint(h * quant_scale
 * + quant_offset)) with h the SwiGLU output, quant_scale / quant_offset (offset may be NULL) of G * n
 * entries, each operation rounded once; scale is written as 0. quant_mode 1 is the dynamic mode above
 * (quant_offset must be NULL). */
int tai_dequant_swiglu_quant_static(const int32_t* x, int64_t rows, int64_t n2,
                                    const float* weight_scale, const float* activation_scale,
                                    const void* bias, int bias_dtype, const float* quant_scale,
                                    const float* quant_offset, const void* group_index,
                                    int group_index_dtype, int64_t num_groups, int activate_left,
                                    int quant_mode, int8_t* y, float* scale, void* stream);
/* swiglu_mode 1 of the same op (experiment_ops.h:3786-3790: "odd-even blocking" with clamp_limit,
 * glu_alpha and glu_bias): output column j takes input columns 2j and 2j + 1 (after the dequantisation
 * and bias, as above); the activated one (2j with activate_left, else 2j + 1) is clamped to at most
 * clamp_limit, the other to [-clamp_limit, clamp_limit], and
 * h = g * sigmoid(glu_alpha * g) * (l + glu_bias), then quant_scale and the quant_mode's quantisation. */
int tai_dequant_swiglu_quant_clamped(const int32_t* x, int64_t rows, int64_t n2,
                                     const float* weight_scale, const float* activation_scale,
                                     const void* bias, int bias_dtype, const float* quant_scale,
                                     const float* quant_offset, const void* group_index,
                                     int group_index_dtype, int64_t num_groups, int activate_left,
                                     int quant_mode, float clamp_limit, float glu_alpha, float glu_bias,
                                     int8_t* y, float* scale, void* stream);

/* ---------------------------------------------------------------------------------------
 * npu_quant_matmul (W8A8): acc = x1 @ x2 with exact int32 accumulation, then
 *   out_dtype INT32: acc (+ int32 bias)
 *   out_dtype BF16/FP16/FP32: (acc [+ int32 bias]) * scale[n] * pertoken_scale[m] [+ fp32 bias]
 *   out_dtype INT8 (the converter's default, quantmatmul.py:91-92, 244-254): clamp(rint(
 *     (acc [+ int32 bias]) * scale[n] [+ offset[n]]), -128, 127), fp32 arithmetic in that order
 *     (scale as fp32 values; the fp32 result is held in the workspace)
 * Replaces ge.QuantBatchMatmulV3 emitted by
 *   python/torchair/_ge_concrete_graph/ge_converter/custom/quantmatmul.py:63-255
 *   (prototype third_party/ascend/include/ops/op_proto/inc/fusion_ops.h:440-451).
 * x1: [M, K] int8 row-major; x2: int8, layout x2_layout (TAI_LAYOUT_KN / _NK).
 * scale: [N] or [1] fp32 (scale_len 1 or N), may be NULL for INT32 output.
 * offset: NULL or [N] / [1] fp32 (offset_len), INT8 output only.
 * pertoken_scale: NULL or [M] fp32. bias: NULL or [N] of bias_dtype (INT32 or FP32).
 * out: [M, N] of out_dtype. workspace: tai_quant_matmul_workspace_size(M, K, N, out_dtype) bytes,
 * 16-byte aligned: for M <= 128 the int32 partials of a K split (summed exactly), for M >= 4096 (K a
 * multiple of 64, N of 256) room for an [N, K] copy of a [K, N] x2, which the call transposes into and
 * multiplies from (without that room the [K, N] kernel runs), for INT8 output the fp32 result.
 * ------------------------------------------------------------------------------------- */
size_t tai_quant_matmul_workspace_size(int64_t m, int64_t k, int64_t n, int out_dtype);
int tai_quant_matmul(const int8_t* x1, const int8_t* x2, int64_t m, int64_t k, int64_t n,
                     int x2_layout, const float* scale, int64_t scale_len, const float* offset,
                     int64_t offset_len, const float* pertoken_scale, const void* bias, int bias_dtype,
                     int out_dtype, void* out, void* workspace, size_t ws_bytes, void* stream);
/* Weight prepacking for tai_quant_matmul, no counterpart in the reference's interface (the NPU's
 * weights are cast to their own format at load time, npu_format_cast): a [K, N] int8 weight is
 * transposed once into [N, K] storage, which the GEMM reads as x2_layout TAI_LAYOUT_NK.
 * tai_quant_matmul_prepack_wanted says whether an M x K x N product takes that path (tall products, and
 * decode-sized ones of at most 128 rows, whose weight stream is contiguous per row in [N, K] storage).
 * The transpose needs k % 64 == 0 and n % 256 == 0. */
int tai_transpose_kn_to_nk(const int8_t* b, int64_t k, int64_t n, int8_t* out, void* stream);
int tai_quant_matmul_prepack_wanted(int64_t m, int64_t k, int64_t n);

/* ---------------------------------------------------------------------------------------
 * npu_grouped_matmul, int8 path with split_item 2/3 and group_type 0 (groups along M):
 * rows [off_e, off_{e+1}) of x multiply weight[e].
 * Replaces ge.GroupedMatmul emitted by
 *   python/torchair/_ge_concrete_graph/ge_converter/custom/grouped_matmul.py:210-365
 *   (prototype experiment_ops.h:3636-3662).
 * x: [m, k] int8. weight: [num_groups, k, n] (TAI_LAYOUT_KN) or [num_groups, n, k] (_NK).
 * group_list: [num_groups] int64 on the device; group_list_type 0 = cumulative row ends,
 * 1 = per-group counts. Rows past the last group end are written as zero.
 * scale: NULL or [num_groups, n] fp32; per_token_scale: NULL or [m] fp32;
 * bias: NULL or [num_groups, n] of bias_dtype (INT32 or FP32).
 * out: [m, n] of out_dtype (INT32, BF16, FP16, FP32).
 * ------------------------------------------------------------------------------------- */
size_t tai_grouped_matmul_workspace_size(int64_t m, int64_t n, int64_t num_groups);
int tai_grouped_matmul(const int8_t* x, const int8_t* weight, int64_t m, int64_t k, int64_t n,
                       int64_t num_groups, int w_layout, const int64_t* group_list,
                       int group_list_type, const float* scale, const float* per_token_scale,
                       const void* bias, int bias_dtype, int out_dtype, void* out,
                       void* workspace, size_t ws_bytes, void* stream);
/* The same product with its rows gathered, no counterpart in the reference's interface (it serves
 * the compiled graph's fusion of npu_moe_init_routing_v2 into the GEMM that consumes its expanded
 * rows, so those rows are never materialised): product row r reads row a_rows[r] of x [x_rows, k]
 * (indices are clamped to [0, x_rows)); a_rows: [m] int32 (tai_moe_init_routing_v2_rows writes it).
 * Workspace as tai_grouped_matmul_workspace_size(m, n, num_groups). */
int tai_grouped_matmul_gather(const int8_t* x, int64_t x_rows, const int32_t* a_rows,
                              const int8_t* weight, int64_t m, int64_t k, int64_t n, int64_t num_groups,
                              int w_layout, const int64_t* group_list, int group_list_type,
                              const float* scale, const float* per_token_scale, const void* bias,
                              int bias_dtype, int out_dtype, void* out, void* workspace, size_t ws_bytes,
                              void* stream);

/* No counterpart in the reference. tai_grouped_matmul without a workspace argument and without
 * any allocation, for callers that cannot allocate device memory (code under hipGraph capture,
 * tight serving loops, harnesses that forbid hipMalloc). Its scratch is a static device array of
 * tai_grouped_matmul_noalloc_max_scratch() bytes (1 MiB) per device, held until the process ends;
 * calls whose tai_grouped_matmul_workspace_size exceeds it fail with TAI_ERR_INVALID. Calls that
 * overlap on one device share that array and race. Same arguments and results otherwise. */
size_t tai_grouped_matmul_noalloc_max_scratch(void);
int tai_grouped_matmul_noalloc(const int8_t* x, const int8_t* weight, int64_t m, int64_t k, int64_t n,
                               int64_t num_groups, int w_layout, const int64_t* group_list,
                               int group_list_type, const float* scale, const float* per_token_scale,
                               const void* bias, int bias_dtype, int out_dtype, void* out, void* stream);

/* ---------------------------------------------------------------------------------------
 * npu_grouped_matmul_swiglu_quant_v2 (dequant_mode 0, quant_mode 0, int8 out): the grouped
 * W8A8 GEMM of the MoE gate_up projection fused with dequant_swiglu_quant. For expert e's rows:
 * d = (float(x @ weight[e]) * weight_scale[e, col]) * x_scale[row]; h = silu(d[:, :n/2]) *
 * d[:, n/2:]; y = per-row symmetric int8 of h, y_scale = max|h| / 127.
 * Replaces ge.GroupedMatmulSwigluQuantV2 emitted by
 *   python/torchair/_ge_concrete_graph/ge_converter/custom/grouped_matmul_swiglu_quant_v2.py:86-166
 *   (prototype fusion_ops.h:769-789).
 * x: [m, k] int8; weight: [num_groups, k, n] (_KN, or _KN_SWIGLU with gate / up interleaved) or
 * [num_groups, n, k] (_NK) int8; weight_scale: [num_groups, n] fp32 (unpermuted); x_scale: [m] fp32; y: [m, n/2] int8; y_scale: [m] fp32.
 * Needs k % 64 == 0 and (n / 2) % 256 (_KN) or % 128 (_NK) == 0; TAI_ERR_UNSUPPORTED otherwise.
 * ------------------------------------------------------------------------------------- */
size_t tai_grouped_matmul_swiglu_quant_workspace_size(int64_t m, int64_t n, int64_t num_groups);
/* The same op with its rows gathered, no counterpart in the reference's interface (the compiled graph's
 * fusion of the routing into the gate_up GEMM): product row r reads row a_rows[r] of x [x_rows, k]
 * (clamped to [0, x_rows)), as tai_grouped_matmul_gather. */
int tai_grouped_matmul_swiglu_quant_gather(const int8_t* x, int64_t x_rows, const int32_t* a_rows,
                                           const int8_t* weight, int64_t m, int64_t k, int64_t n,
                                           int64_t num_groups, int w_layout, const int64_t* group_list,
                                           int group_list_type, const float* weight_scale,
                                           const float* x_scale, int8_t* y, float* y_scale,
                                           void* workspace, size_t ws_bytes, void* stream);
/* Weight prepacking for tai_grouped_matmul_swiglu_quant, no counterpart in the reference's interface
 * (the NPU casts weights to its own format at load time, npu_format_cast): writes the
 * TAI_LAYOUT_KN_SWIGLU copy of a [rows, n] int8 weight (rows = num_groups * k; n % 128 == 0), whose
 * tiles then read each weight row's columns contiguously instead of as separate gate and up pieces. */
int tai_swiglu_pack_kn(const int8_t* w, int64_t rows, int64_t n, int8_t* out, void* stream);
int tai_grouped_matmul_swiglu_quant(const int8_t* x, const int8_t* weight, int64_t m, int64_t k,
                                    int64_t n, int64_t num_groups, int w_layout,
                                    const int64_t* group_list, int group_list_type,
                                    const float* weight_scale, const float* x_scale, int8_t* y,
                                    float* y_scale, void* workspace, size_t ws_bytes, void* stream);

/* ---------------------------------------------------------------------------------------
 * npu_grouped_matmul_finalize_routing (int8 x / w, fp32 out): the grouped W8A8 GEMM of the MoE
 * down projection fused with the weighted combine. Row r's dequantised product
 * v = float(x[r] @ w[e]) * scale[e] * pertoken_scale[r] (+ bias[e]) is added, times logit[r],
 * into y[row_index[r]]; rows of a token are summed in ascending r; shared_input rows (times
 * shared_input_weight) are added at rows [shared_input_offset, + shared_rows).
 * Replaces ge.GroupedMatmulFinalizeRouting emitted by
 *   python/torchair/_ge_concrete_graph/ge_converter/custom/grouped_matmul_finalize_routing.py:32-133
 *   (prototype fusion_ops.h:640-725).
 * scale: [num_groups, n] fp32; pertoken_scale, logit: NULL or [m] fp32; bias: NULL or
 * [num_groups, n] fp32; row_index: NULL (row r -> token r) or [m] INT32/INT64;
 * shared_input: NULL or [shared_rows, n] bf16; y: [output_bs, n] fp32 (every row written).
 * A token may gather at most 1024 rows (beyond that its row is NaN).
 * ------------------------------------------------------------------------------------- */
size_t tai_grouped_matmul_finalize_routing_workspace_size(int64_t m, int64_t n, int64_t num_groups,
                                                         int64_t output_bs);
int tai_grouped_matmul_finalize_routing(const int8_t* x, const int8_t* weight, int64_t m,
                                        int64_t k, int64_t n, int64_t num_groups, int w_layout,
                                        const int64_t* group_list, int group_list_type,
                                        const float* scale, const float* pertoken_scale,
                                        const float* bias, const float* logit,
                                        const void* row_index, int row_index_dtype,
                                        const void* shared_input, int64_t shared_rows,
                                        float shared_input_weight, int64_t shared_input_offset,
                                        int64_t output_bs, float* y, void* workspace,
                                        size_t ws_bytes, void* stream);

/* ---------------------------------------------------------------------------------------
 * npu_moe_gating_top_k: grouped top-k expert selection (DeepSeek-V3 "noaux_tc").
 * Replaces ge.MoeGatingTopK emitted by
 *   python/torchair/_ge_concrete_graph/ge_converter/custom/npu_moe_gating_top_k.py:4-22
 *   (prototype experiment_ops.h:3723-3764; meta auto_register_custom_torch_ops.py:103-114).
 * x: [t, e] of x_dtype; bias: NULL or [e] of bias_dtype. norm_type 0 softmax, 1 sigmoid;
 * group_select_mode 0 group max, 1 sum of the group's top two.
 * y: [t, k] x_dtype; expert_idx: [t, k] int32; out: [t, e] fp32 (written when out_flag).
 * ------------------------------------------------------------------------------------- */
int tai_moe_gating_top_k(const void* x, int x_dtype, int64_t t, int64_t e, int k,
                         const void* bias, int bias_dtype, int k_group, int group_count,
                         int group_select_mode, int renorm, int norm_type, int out_flag,
                         float routed_scaling_factor, float eps, void* y, int32_t* expert_idx,
                         float* out, void* stream);

/* ---------------------------------------------------------------------------------------
 * npu_moe_compute_expert_tokens: out[e] = the number of entries of the ascending sorted_experts
 * [n] int32 that are <= e, for e < num_experts (the end row of each expert, the cumulative
 * group_list of the legacy routing path).
 * Replaces ge.MoeComputeExpertTokens emitted by
 *   python/torchair/_ge_concrete_graph/ge_converter/custom/npu_moe_compute_expert_tokens.py:4-11
 *   (prototype experiment_ops.h:3550-3563).
 * ------------------------------------------------------------------------------------- */
int tai_moe_compute_expert_tokens(const int32_t* sorted_experts, int64_t n, int64_t num_experts,
                                  int32_t* out, void* stream);

/* ---------------------------------------------------------------------------------------
 * npu_moe_init_routing_v2 (dropless, drop_pad_mode 0, quant_mode -1).
 * Replaces ge.MoeInitRoutingV3 emitted by
 *   python/torchair/_ge_concrete_graph/ge_converter/custom/npu_moe_init_routing_v2.py:41-91
 *   (prototype experiment_ops.h:2138-2190).
 * Source slot p = token * k + j. Slots whose expert lies in [expert_start, expert_end)
 * are sorted stably by expert (ties: ascending p); the first `active_rows` of them are
 * materialised. expanded_x: [active_rows, h] (elem_bytes per element) with
 * expanded_x[i] = x[src(i) / k]. expanded_row_idx: [t*k] int32 -
 *   row_idx_type 0: indexed by p, the destination row of slot p (-1 when dropped);
 *   row_idx_type 1: indexed by destination row i, the source slot src(i) (-1 past the end).
 * expert_tokens: [expert_end - expert_start] int64, counts (type 1) or cumsum (type 0).
 * scale: NULL or [t] fp32 -> expanded_scale [active_rows] = scale[src(i) / k].
 * ------------------------------------------------------------------------------------- */
size_t tai_moe_init_routing_workspace_size(int64_t t, int k, int64_t num_experts);
int tai_moe_init_routing_v2(const void* x, int elem_bytes, int64_t t, int64_t h,
                            const int32_t* expert_idx, int k, const float* scale,
                            int64_t active_rows, int expert_start, int expert_end,
                            int expert_tokens_num_type, int row_idx_type, void* expanded_x,
                            int32_t* expanded_row_idx, int64_t* expert_tokens,
                            float* expanded_scale, void* workspace, size_t ws_bytes, void* stream);
/* The same routing without expanded_x, no counterpart in the reference's interface (the compiled
 * graph's fusion of the routing into the grouped GEMM that consumes its rows): a_rows [active_rows]
 * int32 = src(i) / k, the token row that expanded row i copies (0 past the routed total), for
 * tai_grouped_matmul_gather; expanded_row_idx, expert_tokens and expanded_scale as above. Workspace
 * as tai_moe_init_routing_workspace_size. */
int tai_moe_init_routing_v2_rows(int64_t t, const int32_t* expert_idx, int k, const float* scale,
                                 int64_t active_rows, int expert_start, int expert_end,
                                 int expert_tokens_num_type, int row_idx_type, int32_t* a_rows,
                                 int32_t* expanded_row_idx, int64_t* expert_tokens,
                                 float* expanded_scale, void* workspace, size_t ws_bytes, void* stream);

/* npu_moe_init_routing_v2 with drop_pad_mode 1 (experiment_ops.h:2160-2189 drop_pad_mode /
 * expert_capacity; converter .../custom/npu_moe_init_routing_v2.py:41-91): expert e of
 * [expert_start, expert_end) owns rows [e * capacity, (e + 1) * capacity) of expanded_x [E * capacity, h];
 * its slots, in slot order, fill them and the rest are dropped (expanded_row_idx -1). Unfilled rows are
 * zero. expert_tokens: every slot routed to the expert (count, or cumsum for type 0). expanded_scale
 * (with scale [t]): [E * capacity], 0 on unfilled rows. */
size_t tai_moe_init_routing_v2_droppad_workspace_size(int64_t t, int k, int64_t num_experts,
                                                      int64_t capacity);
int tai_moe_init_routing_v2_droppad(const void* x, int elem_bytes, int64_t t, int64_t h,
                                    const int32_t* expert_idx, int k, const float* scale,
                                    int64_t capacity, int expert_start, int expert_end,
                                    int expert_tokens_num_type, void* expanded_x,
                                    int32_t* expanded_row_idx, int64_t* expert_tokens,
                                    float* expanded_scale, void* workspace, size_t ws_bytes,
                                    void* stream);

/* quant_mode 0 (static) of npu_moe_init_routing_v2 (experiment_ops.h:2160-2189; scale / offset of
 * MoeInitRoutingV3 :2140-2158): y = clamp(rint(x * scale + offset), -128, 127) over [rows, cols] of
 * x_dtype (bf16 / fp16 / fp32), each operation rounded once. scale / offset (offset may be NULL): one
 * value (per_col 0) or cols values (per_col 1) for each of scale_groups groups; a row's group is
 * row / group_rows (group_rows > 0) or found in the cumulative group_ends of num_groups entries
 * (scale_groups 1: every row uses group 0). */
int tai_static_quant_rows(const void* x, int x_dtype, int64_t rows, int64_t cols, const float* scale,
                          const float* offset, int64_t scale_groups, int per_col, const void* group_ends,
                          int group_ends_dtype, int64_t num_groups, int64_t group_rows, int8_t* y,
                          void* stream);

/* ---------------------------------------------------------------------------------------
 * npu_moe_init_routing (legacy). Replaces ge.MoeInitRouting emitted by
 *   python/torchair/_ge_concrete_graph/ge_converter/custom/moe_init_routing.py:10-21
 *   (prototype experiment_ops.h:2112-2135).
 * row_idx: [t, k] int32 (conventionally arange(k*t).view(k, t).T). Slots p = token*k + j
 * are sorted stably by expert. Outputs (active_rows = min(active_num, t) * k rows):
 *   expanded_x[i] = x[row_idx_flat[src(i)] % t]; expanded_row_idx[row_idx_flat[src(i)]] = i;
 *   expanded_expert_idx[i] = expert of src(i).
 * ------------------------------------------------------------------------------------- */
int tai_moe_init_routing(const void* x, int elem_bytes, int64_t t, int64_t h,
                         const int32_t* row_idx, const int32_t* expert_idx, int k,
                         int64_t num_experts, int64_t active_rows, void* expanded_x,
                         int32_t* expanded_row_idx, int32_t* expanded_expert_idx,
                         void* workspace, size_t ws_bytes, void* stream);

/* ---------------------------------------------------------------------------------------
 * npu_moe_finalize_routing. Replaces ge.MoeFinalizeRouting(V2) emitted by
 *   python/torchair/_ge_concrete_graph/ge_converter/custom/npu_moe_finalize_routing.py:21-41
 *   (prototype experiment_ops.h:2196-2219).
 * y[t] = skip1[t] + skip2[t] + sum_j scales[t,j] * (expanded[src_to_dst[p(t,j)]] + bias[expert[t,j]])
 * with p(t,j) = j*t_rows + t for drop_pad_mode 0 and t*k + j for drop_pad_mode 2.
 * All row tensors share `dtype` (BF16/FP16/FP32); scales has scales_dtype; optional
 * inputs may be NULL (absent scales means 1). Accumulation is fp32.
 * ------------------------------------------------------------------------------------- */
int tai_moe_finalize_routing(const void* expanded, int dtype, int64_t t, int64_t h, int k,
                             const void* skip1, const void* skip2, const void* bias,
                             const void* scales, int scales_dtype, const int32_t* src_to_dst,
                             const int32_t* expert_for_source_row, int drop_pad_mode, void* y,
                             void* stream);

/* ---------------------------------------------------------------------------------------
 * npu_fused_infer_attention_score, paged decode (one query token per sequence, GQA).
 * Replaces ge.FusedInferAttentionScore emitted by
 *   python/torchair/_ge_concrete_graph/ge_converter/custom/fused_infer_attention_score.py:4-109
 *   and python/torchair/ops/_npu_fused_infer_attention_score.py:14-34 (prototype
 *   experiment_ops.h:3878-3965; output shape rules :160-374 of the latter file).
 * q: [b, hq, d] of dtype (TAI_DT_BF16 or TAI_DT_FP16; BSH with S=1 and BNSD with S=1 share this
 *   memory order). k_cache / v_cache / out: dtype, element (block, slot, kv_head, dim) at
 *   block*stride_block + slot*stride_slot + kv_head*stride_head + dim (elements).
 * block_table: [b, max_blocks] int32; seq_lens_kv: [b] int64 (device).
 * out: [b, hq, d]; lse: NULL or [b, hq] fp32 (natural-log logsumexp of scaled scores).
 * ------------------------------------------------------------------------------------- */
size_t tai_fia_paged_decode_workspace_size(int64_t b, int hq, int d, int64_t max_blocks,
                                           int block_size);
int tai_fia_paged_decode(const void* q, const void* k_cache, const void* v_cache,
                         int64_t stride_block, int64_t stride_slot, int64_t stride_head,
                         const int32_t* block_table, int64_t max_blocks,
                         const int64_t* seq_lens_kv, int64_t b, int hq, int hkv, int d, int dtype,
                         int block_size, float scale, void* out, float* lse, void* workspace,
                         size_t ws_bytes, void* stream);
/* The same with learnable_sink (npu_fused_infer_attention_score_v2, prototype
 * experiment_ops.h:3940): sink [hq] fp32, one logit per query head that joins each row's softmax max
 * and denominator without a value row (a sink of -inf adds nothing). Workspace as above. */
int tai_fia_paged_decode_sink(const void* q, const void* k_cache, const void* v_cache,
                              int64_t stride_block, int64_t stride_slot, int64_t stride_head,
                              const int32_t* block_table, int64_t max_blocks,
                              const int64_t* seq_lens_kv, int64_t b, int hq, int hkv, int d, int dtype,
                              int block_size, float scale, const float* sink, void* out, float* lse,
                              void* workspace, size_t ws_bytes, void* stream);
/* The same over int8 key / value caches with per-channel antiquant scales and no offsets
 * (key_antiquant_scale / value_antiquant_scale, mode 0; prototype experiment_ops.h:3922-3932):
 * k = k_cache * k_scale[h * d + c], v = v_cache * v_scale[h * d + c] (fp32, [hkv * d]). The pages the
 * lengths cover are widened to 16-bit values in the workspace, the query takes the key scale and the
 * merge the value scale. Caches are int8 with byte strides (multiples of 8). */
size_t tai_fia_paged_decode_kv8_workspace_size(int64_t b, int hq, int hkv, int d, int64_t max_blocks,
                                               int block_size);
int tai_fia_paged_decode_kv8(const void* q, const int8_t* k_cache, const int8_t* v_cache,
                             int64_t stride_block, int64_t stride_slot, int64_t stride_head,
                             const int32_t* block_table, int64_t max_blocks,
                             const int64_t* seq_lens_kv, int64_t b, int hq, int hkv, int d, int dtype,
                             int block_size, float scale, const float* k_scale, const float* v_scale,
                             void* out, float* lse, void* workspace, size_t ws_bytes, void* stream);

/* ---------------------------------------------------------------------------------------
 * npu_fused_infer_attention_score with query sequences (GQA prefill, chunked prefill over a paged
 * cache, multi-token decode). Replaces ge.FusedInferAttentionScore for S_q > 1, emitted by
 *   python/torchair/_ge_concrete_graph/ge_converter/custom/fused_infer_attention_score.py:4-109
 *   (pre_tokens / next_tokens / sparse_mode / block_table: prototype experiment_ops.h:3878-3965).
 * q / k / v / out: dtype (TAI_DT_BF16 or TAI_DT_FP16) with element (batch, pos, head, dim) at
 *   batch*sb + pos*ss + head*sh + dim (per-tensor strides, elements).
 * k / v, dense (block_table NULL): like q. Paged (block_table [b, max_blocks] int32 on the device):
 *   caches whose element (block, slot, kv_head, dim) sits at block*k_block_stride + slot*k_strides[1]
 *   + kv_head*k_strides[2] + dim (v likewise); token t of sequence b is at block
 *   block_table[b, t / block_size], slot t % block_size; block_size a multiple of 32; k_strides[0]
 *   is not used.
 * seq_lens_q / seq_lens_kv: NULL (full length) or [b] int64 on the device (required when paged).
 * Mask: query i (of len_q) sees kv j (of len_kv) when -pre_tokens <= j - i - off <= next_tokens,
 *   off = len_kv - len_q for mask_origin 1 (bottom-right: sparse_mode 3 causal is next_tokens 0,
 *   sparse_mode 4 band) and 0 for mask_origin 0 (top-left: sparse_mode 2 causal, sparse_mode 0
 *   band). pre / next of 2^31 - 1 or more are no bound. A query that sees nothing gets 0 and lse -inf.
 * Query rows at or past seq_lens_q[b] are written as zero.
 * lse: NULL or [b, hq, s_q] fp32.
 * ------------------------------------------------------------------------------------- */
int tai_fia_prefill(const void* q, const void* k, const void* v, int64_t b, int64_t s_q,
                    int64_t s_kv, int hq, int hkv, int d, int dtype, const int64_t* q_strides,
                    const int64_t* k_strides, const int64_t* v_strides,
                    const int64_t* out_strides, const int64_t* seq_lens_q,
                    const int64_t* seq_lens_kv, int mask_origin, int64_t pre_tokens,
                    int64_t next_tokens, const int32_t* block_table, int64_t max_blocks,
                    int block_size, int64_t k_block_stride, int64_t v_block_stride, float scale,
                    void* out, float* lse, void* workspace, size_t ws_bytes, void* stream);
/* Bytes of the prefill workspace: work-queue counters and the rescaling pass's item list, which the
 * call clears itself. */
size_t tai_fia_prefill_workspace_size(int64_t b, int64_t s_q, int hq, int hkv);

/* ---------------------------------------------------------------------------------------
 * npu_fused_infer_attention_score, general path (same reference interface: ge.FusedInferAttentionScore
 * emitted by python/torchair/_ge_concrete_graph/ge_converter/custom/fused_infer_attention_score.py:4-109;
 * atten_mask / sparse_mode / query_rope / key_rope: prototype experiment_ops.h:3878-3965):
 * an explicit attention mask (sparse_mode 0/1), an MLA latent cache in bf16 or fp16, or head dims
 * the tiled kernels do not take. One wave per query row; fp32 arithmetic throughout.
 * query = [q1 (dk1) | q2 (dk2)], key = [k1 (dk1) | k2 (dk2)], value = v (dv <= 512); all of dtype.
 * Strides are elements (batch, pos, head) for q1 / q2 / out; for k1 / k2 / v (batch, pos, kv head),
 * or with a block table (block, slot, kv head): token t of sequence b at block
 * block_table[b * max_blocks + t / block_size], slot t % block_size.
 * mask: NULL or bytes with element (batch, query, kv) at the given strides (0 to broadcast); nonzero
 * = masked out. The band rule of tai_fia_prefill (mask_origin, pre_tokens, next_tokens) applies too.
 * A query that sees nothing gets 0 and lse -inf; rows at or past seq_lens_q[b] are 0.
 * lse: NULL or [b, hq, s_q] fp32 (natural-log logsumexp of the scaled scores).
 * ------------------------------------------------------------------------------------- */
typedef struct tai_fia_general_args {
  int dtype;
  int dk1, dk2, dv;
  int64_t b, s_q, s_kv, hq, hkv;
  const void* q1;
  int64_t q1_strides[3];
  const void* q2;
  int64_t q2_strides[3];
  const void* k1;
  int64_t k1_strides[3];
  const void* k2;
  int64_t k2_strides[3];
  const void* v;
  int64_t v_strides[3];
  const int32_t* block_table;
  int64_t max_blocks;
  int64_t block_size;
  const int64_t* seq_lens_q;
  const int64_t* seq_lens_kv;
  const uint8_t* mask;
  int64_t mask_strides[3];
  int64_t mask_origin;
  int64_t pre_tokens, next_tokens;
  float scale;
  void* out;
  int64_t out_strides[3];
  float* lse;
  /* int8 key / value caches (kv_dtype = TAI_DT_INT8; 0 = the query's dtype), dequantised as
   * (x + offset) * scale: mode 0 per channel, fp32 [hkv * dk1] (key) / [hkv * dv] (value); mode 1 per
   * token, fp32 element (b, t) at b * tok_stride + t; mode 2 per cache slot of a paged cache, element
   * block * block_size + slot (the MLA latent scale layout). A null offset is 0. A second key part
   * (k2, the MLA rope key) stays in the query's dtype. Replaces the key/value
   * antiquant inputs of ge.FusedInferAttentionScore (experiment_ops.h:3922-3932). */
  int64_t kv_dtype;
  const float* k_scale;
  const float* k_offset;
  int64_t k_quant_mode;
  const float* v_scale;
  const float* v_offset;
  int64_t v_quant_mode;
  int64_t tok_stride;
  /* int8 attention_out (out_dtype = TAI_DT_INT8; 0 = the query's dtype): clamp(rint(o * out_scale +
   * out_offset), -128, 127), fp32 scale / offset of out_scale_len = 1 or hq * dv entries (channel
   * h * dv + d); a null offset is 0. Replaces quant_scale2 / quant_offset2 (experiment_ops.h:3943). */
  int64_t out_dtype;
  const float* out_scale;
  const float* out_offset;
  int64_t out_scale_len;
  /* pse_shift (NULL: none): a positional bias of the query's dtype added to the scaled scores,
   * softmax(scale * q.k + pse) (experiment_ops.h:3915 pse_shift; the converter passes pse_type 0,
   * fused_infer_attention_score.py:94-109); element (b, h, i, j) at the dot of (b, h, i, j) with
   * pse_strides (a stride 0 broadcasts). */
  const void* pse;
  int64_t pse_strides[4];
  /* shared prefix (k_prefix NULL: none; experiment_ops.h:3933-3935 key_shared_prefix /
   * value_shared_prefix / actual_shared_prefix_len): prefix_len[0] rows of k_prefix / v_prefix (query
   * dtype, element (t, kv head) at t * prefix_strides[0] + h * prefix_strides[1]) precede every
   * sequence's keys and values; a sequence then holds prefix_len + its own kv length positions, over
   * which the masks apply. With an int8 cache the prefix stays in the query's dtype and the antiquant
   * scales index the sequence's own positions. */
  const void* k_prefix;
  const void* v_prefix;
  int64_t k_prefix_strides[2];
  int64_t v_prefix_strides[2];
  const int64_t* prefix_len;
  int64_t prefix_cap;  /* rows the prefix tensors hold (prefix_len is clamped to it) */
  /* packed sequences (the TND / NTD layouts, _npu_fused_infer_attention_score.py:171-180, 227-239;
   * NULL: the batched layouts). q_cum: b cumulative query ends, sequence b owning packed query rows
   * [q_cum[b-1], q_cum[b]) (from 0 for b = 0) of the s_q rows; query / out element (t, h) at
   * t * strides[1] + h * strides[2] (strides[0] unused) and lse (t, h) at t * hq + h; rows past the
   * last end write zeros and lse -inf. kv_cum (dense keys and values only, NULL: per-batch rows at
   * strides[0]): the same for the s_kv packed key / value rows. */
  const int64_t* q_cum;
  const int64_t* kv_cum;
  /* int8 query (q_dtype = TAI_DT_INT8; 0 = the dtype's): query, key and value are int8 (kv_dtype int8,
   * no antiquant scales, one key part) and dtype names the output (fp16 / bf16). One fp32 each:
   * S = (float(q.k) * deq_scale1[0]) * scale; m, l = max S, sum exp(S - m);
   * P8 = clamp(rint(exp(S - m) * quant_scale1[0]), 0, 127); O = (float(P8.V) * deq_scale2[0]) / l,
   * both products exact int32 sums. Replaces dequant_scale1 / quant_scale1 / dequant_scale2 of
   * ge.FusedInferAttentionScore (experiment_ops.h:3888-3890). */
  int64_t q_dtype;
  const float* deq_scale1;
  const float* quant_scale1;
  const float* deq_scale2;
  /* learnable_sink (NULL: none; experiment_ops.h:3940): one fp32 logit per query head, in the domain of
   * the scaled scores, that joins the softmax denominator without a value row: softmax over
   * [scores, sink] with the sink's column dropped. Not with the int8 query. */
  const float* sink;
} tai_fia_general_args;
int tai_fia_general(const tai_fia_general_args* args, void* stream);
/* sizeof(tai_fia_general_args) as compiled into the library (no counterpart in the reference): a
 * binding that mirrors the struct (ctypes, cffi, JNI) checks its own layout against it at load. */
size_t tai_fia_general_args_size(void);

/* ---------------------------------------------------------------------------------------
 * npu_fused_infer_attention_score, MLA absorbed decode with an int8 latent cache
 * (query_rope/key_rope given, key_antiquant_mode 1 = per-token scale).
 * q_nope: [b, hq, dn] bf16, q_rope: [b, hq, dr] bf16.
 * ckv_cache: [num_blocks, block_size, dn] int8, ckv_scale: [num_blocks, block_size] fp32,
 * krope_cache: [num_blocks, block_size, dr] bf16. Latent c = int8 * scale is both key
 * (with k_rope appended) and value. out: [b, hq, dn] bf16; lse: NULL or [b, hq] fp32.
 * ------------------------------------------------------------------------------------- */
size_t tai_fia_mla_decode_workspace_size(int64_t b, int hq, int dn, int64_t max_blocks,
                                         int block_size);
int tai_fia_mla_decode(const void* q_nope, const void* q_rope, const int8_t* ckv_cache,
                       const float* ckv_scale, const void* krope_cache,
                       const int32_t* block_table, int64_t max_blocks,
                       const int64_t* seq_lens_kv, int64_t b, int hq, int dn, int dr,
                       int block_size, float scale, void* out, float* lse, void* workspace,
                       size_t ws_bytes, void* stream);

/* ---------------------------------------------------------------------------------------
 * npu_add_rms_norm: x = x1 + x2; y = x * rstd * gamma with rstd = 1/sqrt(mean(x^2) + eps).
 * Replaces ge.AddRmsNorm emitted by
 *   python/torchair/_ge_concrete_graph/ge_converter/custom/npu_add_rms_norm.py:4-13 (prototype nn_norm.h:50-58).
 * x1, x2, y, x_out: [rows, cols] of dtype (BF16/FP16/FP32); gamma: [cols] of dtype;
 * rstd: NULL or [rows] fp32; x_out: NULL or x1 + x2 rounded to dtype.
 * ------------------------------------------------------------------------------------- */
int tai_add_rms_norm(const void* x1, const void* x2, const void* gamma, int dtype, int64_t rows,
                     int64_t cols, float epsilon, void* y, float* rstd, void* x_out, void* stream);

/* ---------------------------------------------------------------------------------------
 * npu_add_rms_norm_dynamic_quant: add_rms_norm (+ beta), then symmetric per-row int8
 * quantisation of y (rounded to dtype) times smooth_scale1 (and, when y2 is given, times
 * smooth_scale2). Replaces ge.AddRmsNormDynamicQuant emitted by
 *   python/torchair/_ge_concrete_graph/ge_converter/custom/npu_add_rms_norm_dynamic_quant.py:8-21
 * and is the target of TorchAir's fusion pattern
 *   python/torchair/patterns/add_rms_norm_dynamic_quant.py:67-80.
 * beta, smooth_scale1/2: NULL or [cols]; y1/y2: [rows, cols] int8; scale1/2: [rows] fp32.
 * ------------------------------------------------------------------------------------- */
int tai_add_rms_norm_dynamic_quant(const void* x1, const void* x2, const void* gamma,
                                   const void* beta, const float* smooth_scale1,
                                   const float* smooth_scale2, int dtype, int64_t rows,
                                   int64_t cols, float epsilon, int8_t* y1, int8_t* y2,
                                   void* x_out, float* scale1, float* scale2, void* stream);

/* ---------------------------------------------------------------------------------------
 * npu_scatter_pa_kv_cache: writes token t's key / value rows into cache slot slot_mapping[t]
 * (slot = block * block_size + offset; negative slots are skipped).
 * Replaces ge.ScatterPaKvCache emitted by
 *   python/torchair/_ge_concrete_graph/ge_converter/custom/npu_scatter_pa_kv_cache.py:44-74
 *   (prototype experiment_ops.h:3963-4002).
 * key / value: [tokens, *] contiguous rows of key_row_bytes / value_row_bytes; caches in
 * TAI_CACHE_NORM or TAI_CACHE_PA_NZ layout; slot_mapping: [tokens] INT32/INT64.
 * ------------------------------------------------------------------------------------- */
int tai_scatter_pa_kv_cache(const void* key, const void* value, void* key_cache,
                            void* value_cache, const void* slot_mapping, int slot_dtype,
                            int64_t tokens, int64_t key_row_bytes, int64_t value_row_bytes,
                            int64_t num_blocks, int64_t block_size, int cache_mode, void* stream);

/* ---------------------------------------------------------------------------------------
 * npu_kv_rmsnorm_rope_cache: the MLA cache update. Per token: c_kv = rms_norm(kv[:dc]) *
 * gamma; k_rope = interleaved RoPE of kv[dc:] with cos / sin; both written to their caches at
 * the token's cache row. Replaces ge.KvRmsNormRopeCache emitted by
 *   python/torchair/_ge_concrete_graph/ge_converter/custom/npu_kv_rmsnorm_rope_cache.py:4-66
 *   (prototype experiment_ops.h:3677-3697; meta auto_register_custom_torch_ops.py:82-110).
 * kv: [tokens, dc + dr], cos / sin: [tokens, dr], gamma: [dc], all of dtype.
 * index: [tokens] int64 cache row (PA layouts, norm_rows = 0) or position inside the token's
 * batch (Norm layout: batch = token / seq, row = batch * norm_rows + index); negative skips.
 * k_cache: rows of dr (dtype, or int8 quantised with k_rope_scale [dr] (+ offset)).
 * ckv_cache: rows of dc (dtype, or int8): with c_kv_scale [dc] (+ offset) a static
 * per-channel quantisation round(v * scale + offset); with c_kv_token_scale (a [cache_rows]
 * fp32 cache) a per-token dynamic quantisation whose scale is stored there - the int8 latent
 * format tai_fia_mla_decode reads.
 * k_rope_out / c_kv_out: NULL or [tokens, dr] / [tokens, dc] of dtype.
 * ------------------------------------------------------------------------------------- */
int tai_kv_rmsnorm_rope_cache(const void* kv, const void* gamma, const void* cos, const void* sin,
                              const int64_t* index, int dtype, int64_t tokens, int64_t seq, int dc,
                              int dr, float epsilon, void* k_cache, int k_cache_dtype,
                              void* ckv_cache, int ckv_cache_dtype, int64_t cache_rows,
                              int64_t norm_rows, const float* k_rope_scale,
                              const float* k_rope_offset, const float* c_kv_scale,
                              const float* c_kv_offset, float* c_kv_token_scale, void* k_rope_out,
                              void* c_kv_out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TAI_KERNELS_H_ */
