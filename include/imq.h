/* imq.h -- C ABI of the gfx950 (MI355X) weight-only quantized Linear library (libimq.so).
 *
 * One entry point per kernel family of the reference's quantized-Linear hot path. The
 * reference has no C ABI: its operators are Python callables returned by lazy builders in
 * worker_quant.py. Each entry below names the operator it replaces (file:line in the
 * reference tree); the Python layer (infinitemodel_amd.worker_quant) keeps the reference's
 * operator signatures and calls these.
 *
 * Conventions
 *   - Pointers are device pointers owned by the caller (torch allocates every buffer).
 *   - Strides are in elements, except packed-weight row strides which are in BYTES.
 *   - x / y are bf16 unless stated otherwise.
 *   - scale / zero dtype codes: IMQ_DT_BF16, IMQ_DT_FP16, IMQ_DT_FP32.
 *   - `stream` is a hipStream_t passed as void* (torch.cuda.current_stream().cuda_stream).
 *   - Return 0 on success, IMQ_ERR_* (< 0) for rejected arguments, or a positive hipError_t
 *     when a launch fails. No call allocates, frees or synchronizes; all are re-entrant and
 *     keep no state between calls except a per-device immutable attribute cache (and, for
 *     imq_linear_w4_noalloc, the per-device address of its static scratch array). Scratch
 *     memory (split-K partials, MoE intermediates) is a caller-provided workspace argument,
 *     except in imq_linear_w4_noalloc.
 */
#ifndef IMQ_H
#define IMQ_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define IMQ_ABI_VERSION 8

#define IMQ_DT_BF16 0
#define IMQ_DT_FP16 1
#define IMQ_DT_FP32 2
#define IMQ_DT_I32 3 /* integer ids (imq_moe_experts_w4_ex idx_dtype) */
#define IMQ_DT_I64 4

/* MoE expert activations (imq_moe_experts_w4_ex) */
#define IMQ_ACT_SILU_GLU 0 /* gate_up rows [gate (I) | up (I)]: h = silu(gate) * up */
#define IMQ_ACT_GPTOSS 1   /* rows interleaved (gate 2i, up 2i+1): gpt-oss clamped GLU */

#define IMQ_OK 0
#define IMQ_ERR_INVALID (-1)     /* bad shape / stride / dtype / null pointer */
#define IMQ_ERR_UNSUPPORTED (-2) /* valid for the reference but not for this kernel family */
#define IMQ_ERR_ALIGN (-3)       /* pointer or stride not aligned as the kernel requires */
#define IMQ_ERR_SCRATCH (-4)     /* workspace need exceeds IMQ_NOALLOC_SCRATCH_BYTES */

int imq_abi_version(void);
const char* imq_strerror(int status);

/* ---- dequant: the reference dequant, bit-exact ----------------------------------------------
 * out[n, k] = R(R(q[n,k] - R(zero[n, k/G])) * R(scale[n, k/G])) for k < in_features, where R
 * rounds to out_dtype -- QuantLinear4._dequant (worker_quant.py:638-648).
 * qweight: u8 [N, K_pad/2], low nibble = even column. */
int imq_dequant_w4(const void* qweight, int64_t q_row_stride, const void* scale, int64_t s_stride_n,
                   int64_t s_stride_g, int s_dtype, const void* zero, int64_t z_stride_n,
                   int64_t z_stride_g, int z_dtype, int64_t N, int64_t in_features, int64_t group_size,
                   void* out, int64_t out_row_stride, int out_dtype, void* stream);

/* QuantLinear2._dequant (worker_quant.py:1652-1664); qweight u8 [N, K_pad/4], crumb i = col 4j+i. */
int imq_dequant_w2(const void* qweight, int64_t q_row_stride, const void* scale, int64_t s_stride_n,
                   int64_t s_stride_g, int s_dtype, const void* zero, int64_t z_stride_n,
                   int64_t z_stride_g, int z_dtype, int64_t N, int64_t in_features, int64_t group_size,
                   void* out, int64_t out_row_stride, int out_dtype, void* stream);

/* int8 naive weight `qweight.to(dt) * scale` rounded to out_dtype (worker_quant.py:439); the
 * scale is rounded to out_dtype first only when out_dtype is the scale's own dtype class
 * (callers choose out_dtype = torch's promoted dtype). qweight int8 [N, K]. */
int imq_dequant_w8(const void* qweight, int64_t q_row_stride, const void* scale, int64_t s_stride_n,
                   int s_dtype, int64_t N, int64_t K, void* out, int64_t out_row_stride, int out_dtype,
                   void* stream);

/* ---- RTN packers on the device, bit-identical to the host packers -------------------------------
 * pack_linear_int4 / pack_linear_int2 (shard_compile.py:50-94, == worker_quant.py:1588-1608 /
 * 1921-1944): W [N, in_features] (w_dtype: bf16 / fp16 / fp32, row stride in elements) ->
 * qweight u8 [N, K_pad * bits / 8] (row stride in bytes), scale and zero [N, ng] in w_dtype (row
 * stride sz_row_stride elements, groups contiguous). K_pad = ng * group_size; group_size 64, 128
 * or 256. fp32 min / max over each zero-padded group, IEEE division, round-half-even. */
int imq_pack_w4(const void* W, int64_t w_row_stride, int w_dtype, int64_t N, int64_t in_features,
                int64_t group_size, void* qweight, int64_t q_row_stride, void* scale, void* zero,
                int64_t sz_row_stride, void* stream);
int imq_pack_w2(const void* W, int64_t w_row_stride, int w_dtype, int64_t N, int64_t in_features,
                int64_t group_size, void* qweight, int64_t q_row_stride, void* scale, void* zero,
                int64_t sz_row_stride, void* stream);

/* pack_linear_int8 (shard_compile.py:170-178, == worker_quant.py:511-536): per-row symmetric in
 * W's own dtype; qweight int8 [N, K], scale [N, 1] in w_dtype. */
int imq_pack_w8(const void* W, int64_t w_row_stride, int w_dtype, int64_t N, int64_t K, void* qweight,
                int64_t q_row_stride, void* scale, int64_t s_stride_n, void* stream);

/* ---- fused dequant linear: y[M, N] = x[M, K_pad] @ dequant(W)^T, fp32 accumulate, bf16 out ---
 * Replaces the op returned by _w4a16_triton_op() (worker_quant.py:1079-1225: `_ksk` M==1 split-K
 * GEMV, `_k` M>1 tl.dot GEMM), called as op(x[M,Kpad] bf16, qweight, group, (scale, zero)).
 * K_pad = 2 * qweight columns; x must be zero beyond in_features (the module pads, 839-840).
 * Any M >= 1; the library picks the decode (MFMA line / skinny GEMV) or prefill (LDS-dequant MFMA
 * GEMM) kernel. Scale/zero are rounded to bf16 as _dequant(torch.bfloat16) does.
 *
 * workspace (optional, may be NULL): device memory of at least imq_linear_workspace_bytes(M, N,
 * K_pad) bytes, 16-byte aligned, contents need not be initialised. With it, prefill shapes whose
 * tiles do not fill the CUs split K across workgroups; a second launch sums the fp32 partials in
 * split order (deterministic). Calls that share a workspace must be ordered on one stream.
 * Without it (or when too small) K is not split. The bound covers the decode K-split kernels too
 * (4 < M <= 16; on line-tiled int2 weights also M 3..4 and the M <= 2 shapes too long in K for
 * the int2 line kernel). */
int64_t imq_linear_workspace_bytes(int64_t M, int64_t N, int64_t K_pad);

/* Workspace bytes imq_linear_w4 uses for exactly this call (the same arguments as imq_linear_w4,
 * without the pointers) on the current device: 0 when the kernels it picks keep every partial
 * inside the workgroup (the decode line and wave-split kernels), the fp32 partials of the K-split
 * or split-K plan otherwise; -1 for invalid sizes. imq_linear_workspace_bytes above is the
 * shape-only upper bound over the int4 / int2 / int8 families. No counterpart in the reference
 * (its Triton ops allocate internally). */
int64_t imq_linear_w4_workspace_bytes(int64_t M, int64_t K_pad, int64_t N, int64_t group_size,
                                      int64_t q_row_stride, int64_t x_row_stride, int64_t s_stride_n,
                                      int64_t s_stride_g, int s_dtype, int64_t z_stride_n,
                                      int64_t z_stride_g, int z_dtype);

int imq_linear_w4(const void* x, int64_t x_row_stride, int64_t M, int64_t K_pad, const void* qweight,
                  int64_t q_row_stride, const void* scale, int64_t s_stride_n, int64_t s_stride_g,
                  int s_dtype, const void* zero, int64_t z_stride_n, int64_t z_stride_g, int z_dtype,
                  int64_t N, int64_t group_size, void* y, int64_t y_row_stride, void* workspace,
                  int64_t workspace_bytes, void* stream);

/* ---- line-tiled packed weights ------------------------------------------------------------------
 * No counterpart in the reference: a device layout of the same bytes as a row-layout qweight
 * [N, row_bytes] (int4: row_bytes = K_pad / 2, int2: K_pad / 4, int8: K; N a multiple of 16,
 * row_bytes of 128), permuted in 16-byte pieces so that the decode kernels' full-line weight loads read 256
 * contiguous bytes per 16 lanes instead of 8 partial 128-byte lines. In 16-row tile t the 2 KiB
 * block of line-step l (bytes [128 l, 128 l + 128) of every row of the tile) sits at byte
 * 2048 (t row_bytes / 128 + l); its 16-byte slot 64 h + s (h 0..1, s 0..63) holds piece
 * 4 (((s >> 3) & 1) ^ h) + (s >> 4) of tile row 8 h + (s & 7).
 * imq_line_tile / imq_line_untile convert between the layouts, out of place (the tiled array is
 * dense: N * row_bytes bytes). imq_linear_w4_tiled / imq_linear_w2_tiled take the arguments of
 * imq_linear_w4 / imq_linear_w2 and give the same results, with qweight tiled (q_row_stride =
 * row_bytes; int4 groups of 128, int2 groups of 64); the decode line / wave-split / K-split kernels
 * and the prefill GEMMs read the layout, and a call none of them takes returns
 * IMQ_ERR_UNSUPPORTED. They serve the reference operators of imq_linear_w4 / _w2
 * (_w4a16_triton_op, worker_quant.py:1079-1225; _w2a16_triton_op, 1775-1918) for modules whose
 * weights were tiled once at load. */
int imq_line_tile(const void* q_rows, int64_t q_row_stride, int64_t N, int64_t row_bytes, void* q_tiled,
                  void* stream);
int imq_line_untile(const void* q_tiled, int64_t N, int64_t row_bytes, void* q_rows, int64_t q_row_stride,
                    void* stream);
int imq_linear_w4_tiled(const void* x, int64_t x_row_stride, int64_t M, int64_t K_pad, const void* qweight,
                        int64_t q_row_stride, const void* scale, int64_t s_stride_n, int64_t s_stride_g,
                        int s_dtype, const void* zero, int64_t z_stride_n, int64_t z_stride_g, int z_dtype,
                        int64_t N, int64_t group_size, void* y, int64_t y_row_stride, void* workspace,
                        int64_t workspace_bytes, void* stream);
int imq_linear_w2_tiled(const void* x, int64_t x_row_stride, int64_t M, int64_t K_pad, const void* qweight,
                        int64_t q_row_stride, const void* scale, int64_t s_stride_n, int64_t s_stride_g,
                        int s_dtype, const void* zero, int64_t z_stride_n, int64_t z_stride_g, int z_dtype,
                        int64_t N, int64_t group_size, void* y, int64_t y_row_stride, void* workspace,
                        int64_t workspace_bytes, void* stream);
/* int8 twin (imq_linear_w8's arguments; q_row_stride = K, K a multiple of 128): the decode line
 * and skinny kernels and both prefill GEMMs read the layout. Serves _w8a16_triton_op
 * (worker_quant.py:926-1057) for modules whose op serves every M. */
int imq_linear_w8_tiled(const void* x, int64_t x_row_stride, int64_t M, int64_t K, const void* qweight,
                        int64_t q_row_stride, const void* scale, int64_t s_stride_n, int s_dtype, int64_t N,
                        void* y, int64_t y_row_stride, void* workspace, int64_t workspace_bytes, void* stream);

/* int2 twin: replaces _w2a16_triton_op() (worker_quant.py:1775-1918: `_ksk2`, `_k2`).
 * K_pad = 4 * qweight columns. */
int imq_linear_w2(const void* x, int64_t x_row_stride, int64_t M, int64_t K_pad, const void* qweight,
                  int64_t q_row_stride, const void* scale, int64_t s_stride_n, int64_t s_stride_g,
                  int s_dtype, const void* zero, int64_t z_stride_n, int64_t z_stride_g, int z_dtype,
                  int64_t N, int64_t group_size, void* y, int64_t y_row_stride, void* workspace,
                  int64_t workspace_bytes, void* stream);

/* int8 per-row symmetric: y = bf16(scale[n] * sum_k x[m,k] * q[n,k]). Replaces
 * _w8a16_triton_op() (worker_quant.py:926-1057: `_ksk8`, `_k8`), op(x, qweight, scale). */
int imq_linear_w8(const void* x, int64_t x_row_stride, int64_t M, int64_t K, const void* qweight,
                  int64_t q_row_stride, const void* scale, int64_t s_stride_n, int s_dtype, int64_t N,
                  void* y, int64_t y_row_stride, void* workspace, int64_t workspace_bytes, void* stream);

/* ---- allocation-free int4 linear -----------------------------------------------------------------
 * No counterpart in the reference. For callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc): the same arguments,
 * kernels and results as imq_linear_w4 without the workspace arguments. The K-split / split-K
 * partials go to a static scratch array of IMQ_NOALLOC_SCRATCH_BYTES bytes that each GPU the
 * library runs on holds from the first call on that GPU until the process ends; nothing is
 * allocated or freed per call. Calls whose own workspace need (imq_linear_w4_workspace_bytes)
 * exceeds it return IMQ_ERR_SCRATCH before any launch. Every call on one GPU shares that GPU's array and
 * it keeps the last call's partials (they need no clearing: each call writes every partial it
 * reads), so calls that may overlap on one GPU (other streams, or unordered work) race: order
 * them on one stream. */
#define IMQ_NOALLOC_SCRATCH_BYTES (64ll << 20)

int imq_linear_w4_noalloc(const void* x, int64_t x_row_stride, int64_t M, int64_t K_pad,
                          const void* qweight, int64_t q_row_stride, const void* scale, int64_t s_stride_n,
                          int64_t s_stride_g, int s_dtype, const void* zero, int64_t z_stride_n,
                          int64_t z_stride_g, int z_dtype, int64_t N, int64_t group_size, void* y,
                          int64_t y_row_stride, void* stream);

/* ---- fused MoE experts (int4 g-wise, [E, N, K_pad/2] stacks) ----------------------------------
 * Per-row grouped GEMV: y[b, :] = x[b, :] @ dequant(W[eid[b]])^T for b < B (fp32 accumulate,
 * bf16 out). Replaces the op returned by _w4a16_moe_op() (worker_quant.py:1342-1495, `_mk`),
 * op(x[B,Kin], eid[B], q[E,N,Kpad/2], scale, zero, group, in_features). x is [B, K_pad] bf16
 * (zero beyond in_features); eid int32 [B]. */
int imq_moe_rows_w4(const void* x, int64_t x_row_stride, int64_t B, int64_t K_pad, const int32_t* eid,
                    int64_t E, const void* qweight, int64_t q_stride_e, int64_t q_row_stride,
                    const void* scale, int64_t s_stride_e, int64_t s_stride_n, int64_t s_stride_g,
                    const void* zero, int64_t z_stride_e, int64_t z_stride_n, int64_t z_stride_g,
                    int sz_dtype, int64_t N, int64_t group_size, void* y, int64_t y_row_stride,
                    void* stream);

/* Whole experts forward of one MoE layer (the patched experts.forward of
 * _install_fused_moe_forward, worker_quant.py:2131-2248, whose semantics are the transformers
 * eager experts loop): out[t] = sum_j w[t,j] * down_e( silu(gate) * up ), [gate | up] =
 * gate_up_e(x[t]), e = topk_idx[t,j].
 *   hidden bf16 [T, H_pad] (row stride; zero beyond H when H_pad > H), or rows of just H
 *   columns when H % 8 == 0 (read as zero past H); topk_idx int32 [T, k] contiguous, topk_w
 *   bf16 [T, k] contiguous, gate_up stack [E, 2I, H_pad/2] + s/z [E, 2I, ng1], down stack
 *   [E, H, I_pad/2] + s/z [E, H, ng2] (scale and zero share strides), out bf16 [T, H].
 *   workspace: device bytes >= imq_moe_workspace_bytes(T, k, E, H, I, G); contents need not be
 *   initialised; calls sharing a workspace must be stream-ordered. */
int64_t imq_moe_workspace_bytes(int64_t T, int64_t top_k, int64_t E, int64_t H, int64_t I,
                                int64_t group_size);
int imq_moe_experts_w4(const void* hidden, int64_t h_row_stride, int64_t T, int64_t H, int64_t top_k,
                       const int32_t* topk_idx, const void* topk_w, int64_t E,
                       const void* gu_q, int64_t gu_q_stride_e, int64_t gu_q_row_stride,
                       const void* gu_s, const void* gu_z, int64_t gu_sz_stride_e, int64_t gu_sz_stride_n,
                       int64_t I, const void* dn_q, int64_t dn_q_stride_e, int64_t dn_q_row_stride,
                       const void* dn_s, const void* dn_z, int64_t dn_sz_stride_e, int64_t dn_sz_stride_n,
                       int sz_dtype, int64_t group_size, void* out, int64_t out_row_stride,
                       void* workspace, int64_t workspace_bytes, void* stream);

/* imq_moe_experts_w4 generalized to the gpt-oss experts forward (_install_gptoss_fused_forward,
 * worker_quant.py:2280-2314) and to kernel-layout row padding:
 *   gu_K_pad / dn_K_pad: K of each projection as laid out in qweight / scale / zero -- a multiple
 *     of group_size, >= H (resp. I), dn_K_pad <= I_pad rounded up to 256; codes and scales of
 *     columns past in_features must be zero (a holder padded past the reference's K_pad).
 *   gu_bias [E, 2I] / dn_bias [E, H] (expert stride, unit row stride, bias_dtype), or NULL: added
 *     to the projection outputs before the activation / before the routing weight.
 *   act IMQ_ACT_SILU_GLU (alpha, limit unused) or IMQ_ACT_GPTOSS: gate = y[2i] + b (<= limit),
 *     up = y[2i+1] + b (clamped to [-limit, limit]), h = (up + 1) * gate * sigmoid(alpha * gate).
 *   out[t] = sum_j w[t,j] * (down_e(h) + dn_bias[e]), e = topk_idx[t,j]. Same workspace as
 *   imq_moe_experts_w4. gpt-oss experts are transpose-packed: gate_up [E, 2I, H_pad/2] with the
 *   interleaved rows, down [E, H, I_pad/2].
 *   topk_idx [T, k] contiguous of idx_dtype IMQ_DT_I32 or IMQ_DT_I64 (the int64 ids torch's top-k
 *   returns are read as they are, as the reference's MoE op reads them: no conversion launch). */
int imq_moe_experts_w4_ex(const void* hidden, int64_t h_row_stride, int64_t T, int64_t H, int64_t top_k,
                          const void* topk_idx, int idx_dtype, const void* topk_w, int64_t E,
                          const void* gu_q, int64_t gu_q_stride_e, int64_t gu_q_row_stride, int64_t gu_K_pad,
                          const void* gu_s, const void* gu_z, int64_t gu_sz_stride_e, int64_t gu_sz_stride_n,
                          int64_t I, const void* dn_q, int64_t dn_q_stride_e, int64_t dn_q_row_stride,
                          int64_t dn_K_pad, const void* dn_s, const void* dn_z, int64_t dn_sz_stride_e,
                          int64_t dn_sz_stride_n, int sz_dtype, int64_t group_size,
                          const void* gu_bias, int64_t gu_bias_stride_e, const void* dn_bias,
                          int64_t dn_bias_stride_e, int bias_dtype, int act, float alpha, float limit,
                          void* out, int64_t out_row_stride, void* workspace, int64_t workspace_bytes,
                          void* stream);

/* ---- measurement probes ---------------------------------------------------------------------
 * No counterpart in the reference: the hardware ceilings the hot-path kernels are measured
 * against (bench.py --config ceiling | stream | launch | mfma).
 *   imq_probe_stream: one read-only launch over nbuf buffers taken in order; `ptrs` is a device
 *     array of nbuf uint64 addresses (16-byte aligned), `n16s` a device array of nbuf int64 sizes
 *     in 16-byte words (buffers of 0 words are skipped), total_n16 their sum (sizes the grid).
 *     loads_per_lane U in {1, 2, 4, 8, 16} (a workgroup of 256 lanes reads 256 U words per chunk,
 *     the next chunk's loads issued before the current one's are consumed), at most wg_per_cu
 *     (1..32) workgroups per CU, nontemporal != 0 for non-temporal loads. Nothing is written.
 *   imq_probe_copy: dst[0:bytes) = src[0:bytes) (bytes a multiple of 16, both 16-byte aligned),
 *     U in {2, 4, 8} loads then U non-temporal stores per lane.
 *   imq_probe_empty: one empty kernel of `grid` workgroups of 64 lanes.
 *   imq_probe_mfma: cus * wg_per_cu workgroups of 4 waves, each wave running 4 independent
 *     accumulator chains of `iters` MFMAs: kind 0 = v_mfma_f32_32x32x16_bf16 (32768 flops each),
 *     kind 1 = v_mfma_f32_16x16x32_bf16 (16384 flops each).
 *   `sink`: device memory of at least imq_probe_sink_bytes() bytes (never written in practice). */
int64_t imq_probe_sink_bytes(void);
int imq_probe_stream(const void* ptrs, const void* n16s, int nbuf, int64_t total_n16, int loads_per_lane,
                     int wg_per_cu, int nontemporal, void* sink, int64_t sink_bytes, void* stream);
int imq_probe_copy(void* dst, const void* src, int64_t bytes, int loads_per_lane, int wg_per_cu, void* stream);
int imq_probe_empty(int grid, void* stream);
int imq_probe_mfma(int kind, int64_t iters, int wg_per_cu, void* sink, int64_t sink_bytes, void* stream);

/* GPTQ int2 solver (the calibrated int2 packer's quantization, after its Cholesky stage).
 *   imq_gptq_int2_params: the group search alone -- replaces gptq_pack.py:78-100 (_find_params):
 *       scale[r], zero[r] of rows Wg[r][0:cols) (fp32, row stride ldw) on the asymmetric 0..3 grid,
 *       the best of int(maxshrink * grid) range-shrink candidates by sum |dq - w|^2.4.
 *   imq_gptq_int2_solve: replaces gptq_pack.py:141-180 (_GPTQ.solve from its block loop): W
 *       [out][ldw] fp32 (dead columns zeroed; consumed: overwritten by the cross-block updates),
 *       Hinv [in_f][ldh] fp32 the upper Cholesky factor of the damped H^-1, blocks of blocksize
 *       (<= 128, a multiple of group_size, itself a multiple of 4) columns. Writes qweight
 *       [out][ldq] crumbs (byte j of a row = columns 4j..4j+3, lowest bits first; in_pad =
 *       ceil(in_f / group_size) * group_size, padded columns at the last group's rounded zero),
 *       scale / zero [out][ldsz] fp32 and, when dq is non-null, the dequantized weight
 *       dq [out][lddq] fp32. Workspace: imq_gptq_int2_workspace_bytes(out, blocksize).
 * float32 throughout, every operation rounded on its own, sums in a fixed order: reproducible
 * bit for bit on any device by a restatement with the same order. */
int64_t imq_gptq_int2_workspace_bytes(int64_t out, int64_t blocksize);
int imq_gptq_int2_params(const float* Wg, int64_t ldw, int64_t rows, int64_t cols, int grid, double maxshrink,
                         float* scale, float* zero, void* stream);
int imq_gptq_int2_solve(float* W, int64_t ldw, int64_t out, int64_t in_f, const float* Hinv, int64_t ldh,
                        int64_t group_size, int grid, double maxshrink, int64_t blocksize, uint8_t* qweight,
                        int64_t ldq, float* scale, float* zero, int64_t ldsz, float* dq, int64_t lddq,
                        void* workspace, int64_t workspace_bytes, void* stream);

/* ---- launch plans (no counterpart in the reference) -----------------------------------------
 * For test harnesses and tooling: the launch plan the dispatcher computes for a shape, from the
 * same host functions its launchers call, without a device (the device's LDS bytes per
 * workgroup and CU count are arguments). The CPU bounds model of the kernels' address ranges
 * checks its restated plans against these.
 *   in[10] = {M, K_pad (K for int8), group_size (0 for int8), N, q_row_stride (bytes),
 *             x_row_stride (elements), s_stride_n (elements), s_dtype, max_lds_bytes, cus};
 *             group strides are 1, the zero point's strides and dtype are the scale's.
 *   out[5] = {taken (1 when that kernel takes the call, else 0 and the rest 0), p1, p2, p3,
 *             LDS bytes per workgroup}:
 *     IMQ_PLAN_W4_LINE    int4 line kernel: p1 line-steps per wave, p2 waves
 *     IMQ_PLAN_W4_KSPLIT  int4 K-split kernel: p1 splits, p2 row tiles per workgroup,
 *                         p3 line-steps per split
 *     IMQ_PLAN_W4_WSPLIT  int4 wave-split kernel: p1 line-steps per wave, p2 waves
 *     IMQ_PLAN_W4_SKINNY  int4 skinny kernel: p1 K steps per wave per round, p2 waves
 *                         (taken whenever K_pad is a whole number of 128-code steps)
 *     IMQ_PLAN_W2_LINE    int2 line kernel: p1 line-steps per wave, p2 waves
 *     IMQ_PLAN_W2_KSPLIT  int2 K-split kernel: p1 splits, p2 row tiles per workgroup
 *     IMQ_PLAN_W8_LINE    int8 line kernel: p1 line-steps per wave, p2 waves
 *     IMQ_PLAN_GEMM       LDS-dequant GEMM: p1 tile rows, p2 tile columns, p3 K splits
 *     IMQ_PLAN_GEMM_RB    register-B GEMM (int4 with group_size, int8 when it is 0):
 *                         p1 32-row blocks per wave, p2 K splits
 * Returns IMQ_OK, or IMQ_ERR_INVALID for an unknown kind or a null pointer. */
#define IMQ_PLAN_W4_LINE 1
#define IMQ_PLAN_W4_KSPLIT 2
#define IMQ_PLAN_W4_WSPLIT 3
#define IMQ_PLAN_W4_SKINNY 4
#define IMQ_PLAN_W2_LINE 5
#define IMQ_PLAN_W2_KSPLIT 6
#define IMQ_PLAN_W8_LINE 7
#define IMQ_PLAN_GEMM 8
#define IMQ_PLAN_GEMM_RB 9
int imq_launch_plan(int kind, const int64_t* in, int64_t* out);

#ifdef __cplusplus
}
#endif

#endif /* IMQ_H */
