/*
 * ptb_amd.h -- C ABI of the MI355X (gfx950) kernels that execute the hot path of
 * PSAL-POSTECH/PyTorchSim-Triton-Backend's lowered kernels.
 *
 * The reference executes each lowered kernel as a RISC-V ELF whose generated C driver calls
 *   void <kernel>(int64_t rank, memref_desc*, ..., scalars..., gx, gy, gz, pidx, pidy, pidz)
 * once per grid program (reference: pytorchsim_triton_compiler/codegen/wrapper.py:37-51,
 * :126-277; memref descriptor :140-146; program loop :254-265).  Here one call covers the whole
 * grid: every entry point below takes caller-owned device pointers (bf16 carried as uint16 bits,
 * fp8 e4m3fn as uint8 bits, as contract/kernel_object.py:43-56 carries them), sizes, and a
 * hipStream_t passed as void* (NULL = the null stream).  Launches are asynchronous on that stream,
 * nothing is allocated, and there is no global mutable state, so entry points are thread-safe --
 * except ptb_attn_decode_bf16_noalloc, whose static per-device scratch is shared by every call on
 * a GPU (see there).
 *
 * An entry point whose output is empty returns 0 without looking at its pointers.
 * Return value: 0 on success; a negative PTB_ERR_* for an argument the library refuses before
 * launching anything (the role of the wrapper main's exit codes 2/3/4 at codegen/wrapper.py:191-250
 * and of contract/kernel_object.py:93-107 refuse_grid_past_bound); a positive value is the
 * hipError_t the HIP runtime reported for the launch.
 */
#ifndef PTB_AMD_H
#define PTB_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PTB_ABI_VERSION 1

#define PTB_OK 0
#define PTB_ERR_NULL (-1)        /* a required pointer is NULL */
#define PTB_ERR_SHAPE (-2)       /* a size is negative, zero where it may not be, or inconsistent */
#define PTB_ERR_ALIGN (-3)       /* a pointer or a row is not aligned for 128-bit access */
#define PTB_ERR_DTYPE (-4)       /* an unknown dtype code */
#define PTB_ERR_UNSUPPORTED (-5) /* a shape outside what the kernel implements (e.g. head_dim != 128) */
#define PTB_ERR_GRID (-6)        /* the launch would need a grid past the hardware's bound */
#define PTB_ERR_WORKSPACE (-7)   /* the caller's workspace is smaller than required */

#define PTB_DTYPE_BF16 0
#define PTB_DTYPE_F32 1
#define PTB_DTYPE_I32 2
#define PTB_DTYPE_I64 3
#define PTB_DTYPE_E4M3 4

#define PTB_ROLE_IN 0
#define PTB_ROLE_OUT 1
#define PTB_ROLE_INOUT 2

#define PTB_REDUCE_SUM 0
#define PTB_REDUCE_MAX 1

/* Library identity and status text. */
int ptb_abi_version(void);
const char* ptb_status_string(int status);

/* RMSNorm over rows: y[r,c] = bf16( (x[r,c] * rsqrt(sum_c x^2 / cols + eps)) * w[c] ), fp32 math,
 * one rounding at the store.  w is bf16 (w_dtype = PTB_DTYPE_BF16) or fp32 (PTB_DTYPE_F32).
 * Replaces: validation/pytorchsim/qwen3_8b_layer_prefill_2048x2048_bf16/00_..._gwdq6qer/
 *           pytorchsim_triton_compiler_fused__to_copy_add_mean_mul_pow_rsqrt_gwdq6qer_triton.py:17-60 */
int ptb_rmsnorm_bf16(const void* x, const void* w, int w_dtype, void* y, int64_t rows, int64_t cols,
                     float eps, void* stream);

/* fp32 RMSNorm over rows: y = (x * rsqrt(sum_c x^2 / cols + eps)) * w, fp32 in and out (no
 * rounding below fp32).  x, w, y 16-byte aligned, cols % 4 == 0.
 * Replaces: tests/cases/workloads/rmsnorm.py:44-54 (the row arm, output o). */
int ptb_rmsnorm_f32(const float* x, const float* w, float* y, int64_t rows, int64_t cols, float eps, void* stream);
/* The column arm of the same case: c[j] = rsqrt(sum_i x[i,j]^2 / rows + eps), fp32.
 * Replaces: tests/cases/workloads/rmsnorm.py:56-57 (output c). */
int ptb_col_rms_f32(const float* x, float* c, int64_t rows, int64_t cols, float eps, void* stream);

/* Row softmax: y = bf16( exp(x - max) / sum(exp(x - max)) ), max NaN-propagating, fp32 math.
 * Replaces: validation/pytorchsim/vector_softmax_2048x6144_bf16/00_..._sa7wwqqf/..._triton.py:17-68 */
int ptb_softmax_rows_bf16(const void* x, void* y, int64_t rows, int64_t cols, void* stream);

/* The same row softmax with the probabilities stored as fp32 (no rounding): the MoE router's
 * softmax over expert logits.
 * Replaces: validation/pytorchsim/layer_layer_decode_1x1024_bf16/16_..._qslpdpud/
 *           pytorchsim_triton_compiler_fused__softmax__to_copy_qslpdpud_triton.py:17-45 */
int ptb_softmax_rows_bf16_f32(const void* x, void* y, int64_t rows, int64_t cols, void* stream);

/* fp32 row softmax: y = exp(x - max) / sum(exp(x - max)), fp32 in and out, max NaN-propagating.
 * x, y 16-byte aligned, cols % 4 == 0.
 * Replaces: tests/cases/workloads/softmax.py:46-55 (rtol 1e-5, atol 1e-6 at :84). */
int ptb_softmax_rows_f32(const float* x, float* y, int64_t rows, int64_t cols, void* stream);

/* fp32 SiLU gate: out[t,j] = (g / (1 + exp(-g))) * u, g = gu[t, j], u = gu[t, inter + j], all fp32.
 * inter % 4 == 0, pointers 16-byte aligned.  The elementwise half of tests/cases/workloads/swiglu.py
 * (silu(gate) * up at :61-62); ptb_swiglu_f32 is the whole case. */
int ptb_silu_mul_f32(const float* gate_up, float* out, int64_t rows, int64_t inter, void* stream);

/* fp32 SwiGLU block: o[m,n] = silu(g) * u with g = (x . wg)[m,n], u = (x . wu)[m,n], x [m,k],
 * wg / wu [k,n] row-major, fp32 operands and accumulation, silu(g) = g / (1 + exp(-g)).
 * Replaces: tests/cases/workloads/swiglu.py:44-62 (rtol = atol = 1e-3 at :100). */
int ptb_swiglu_f32(const float* x, const float* wg, const float* wu, float* o, int64_t m, int64_t n, int64_t k,
                   void* stream);

/* SiLU gate: out[t,j] = bf16( (g / (1 + exp(-g))) * u ), g = gu[t, j], u = gu[t, inter + j].
 * Replaces: qwen3_8b_layer_prefill_2048x2048_bf16/10_..._ktzl5s2h/..._triton.py:17-36 */
int ptb_silu_mul_bf16(const void* gate_up, void* out, int64_t rows, int64_t inter, void* stream);

/* Head transpose: y[b, a, :] = x[a, b, :] for x of shape [d0, d1, inner] (exact copy).
 * [T,H,D] -> [H,T,D] replaces qwen3_8b_layer_prefill_2048x2048_bf16/05_..._ff5nvvqz_triton.py:17-27;
 * [H,T,D] -> [T,H,D] replaces 07_..._ei42assc_triton.py:17-27. */
int ptb_transpose_heads_bf16(const void* x, void* y, int64_t d0, int64_t d1, int64_t inner,
                             void* stream);
/* The same with x's rows of d1*inner elements ld elements apart (ld >= d1*inner, ld % 8 == 0): reads
 * the v part of a fused [T, q|k|v] projection output in place.  Replaces the same launch as above. */
int ptb_transpose_heads_ld_bf16(const void* x, int64_t ld, void* y, int64_t d0, int64_t d1, int64_t inner,
                                void* stream);

/* Per-(token, head) RMSNorm (eps) with weight w[head_dim], then rotate-half RoPE with fp32
 * cos/sin [tokens, head_dim], stored head-major: out[h, t, :].  x is [tokens, heads, head_dim].
 * Replaces: qwen3_8b_layer_prefill_2048x2048_bf16/02_..._mmis7ufj_triton.py:17-98 (H=32) and
 *           04_..._ll67ghqi_triton.py (H=8); with tokens = 1, qwen3_8b_layer_decode_1x<S>_bf16/
 *           02_..._twgfj5dp_triton.py:17-96 (cos/sin of the token's position, [1, head_dim]). */
int ptb_qk_norm_rope_bf16(const void* x, const void* w, const float* cos_t, const float* sin_t,
                          void* out, int64_t tokens, int64_t heads, int64_t head_dim, float eps,
                          void* stream);
/* The same with token t's heads starting at x + t*ld (ld >= heads*head_dim, ld % 8 == 0): reads the
 * q or k part of a fused [T, q|k|v] projection output in place.  Replaces the same launches. */
int ptb_qk_norm_rope_ld_bf16(const void* x, int64_t ld, const void* w, const float* cos_t, const float* sin_t,
                             void* out, int64_t tokens, int64_t heads, int64_t head_dim, float eps,
                             void* stream);

/* Whole-tensor reduction to one fp32: PTB_REDUCE_SUM (fp32 accumulation) or PTB_REDUCE_MAX
 * (NaN-propagating).  workspace must hold ptb_reduce_workspace_bytes(n) bytes.
 * Replaces: vector_sum_<R>x<C>_bf16/00_..._2y6fwkvp_triton.py and vector_max_<R>x<C>_bf16/
 *           00_..._q47252w4_triton.py. */
size_t ptb_reduce_workspace_bytes(int64_t n);
int ptb_reduce_bf16(const void* x, float* out, int64_t n, int op, void* workspace,
                    size_t workspace_bytes, void* stream);
/* The same reduction over fp32 elements (16-byte aligned).
 * Replaces: validation/pytorchsim/layer_layer_decode_1x1024_bf16/18_..._7gslrk5a/
 *           pytorchsim_triton_compiler_fused_sum_7gslrk5a_triton.py:17-38 (the MoE router's sum of
 *           its top-k weights). */
int ptb_reduce_f32(const float* x, float* out, int64_t n, int op, void* workspace,
                   size_t workspace_bytes, void* stream);

/* y = bf16(float(x) + s) elementwise.  Replaces vector_add1_<R>x<C>_bf16/00_..._du5rd5jd_triton.py. */
int ptb_add_scalar_bf16(const void* x, void* y, int64_t n, float s, void* stream);

/* out[i] = float(x[first + i]) + s into fp32, i < count (a slice of a bf16 tensor plus a constant).
 * Replaces vector_slice_<R>x<C>_bf16/00_..._fused__to_copy_add_slice_slnyinbt_triton.py:17-27
 * (first = 0, count = 1, s = 1). */
int ptb_slice_add_bf16(const void* x, float* out, int64_t first, int64_t count, float s, void* stream);

/* Dense GEMM, row-major: C[m,n] = bf16( sum_k A[m,k] * B[k,n] (+ float(R[m,n])) ), fp32 accumulation.
 * residual may be NULL.  Requires k % 64 == 0 and n % 8 == 0; m is free.  Operands are addressed
 * with 32-bit byte offsets: (k + 128) * n * 2 and 256 * k * 2 below 4 GiB and n <= 2^22, else
 * PTB_ERR_UNSUPPORTED.
 * Replaces: qwen3_8b_layer_prefill_2048x2048_bf16/01_..._fused_mm_ckb6aiys_triton.py:18-97 (and
 *           03, 09), the residual epilogues 08_..._utuycvlm_triton.py:18-99 and
 *           11_..._fjjozd2g_triton.py:18-66, and the gemm_<M>x<K>x<N>_bf16 bundle kernels. */
int ptb_gemm_bf16(const void* a, const void* b, const void* residual, void* c, int64_t m, int64_t n,
                  int64_t k, void* stream);

/* The same GEMM with a caller workspace for split-K: when the output's 64x128 tiles leave CUs idle
 * (and K >= 1024), K may be cut into 2, 4 or 8 slices (at least 256 deep, tiles x slices within the
 * CUs, as a fitted cost model of the workgroups' operand streaming and the partial traffic decides)
 * multiplied by separate workgroups into fp32 partials that a finish pass sums (+ residual) and
 * rounds once.  ptb_gemm_bf16_workspace_bytes is 0 for shapes that do not split; then
 * ptb_gemm_bf16_ws is ptb_gemm_bf16.  A split shape refuses a NULL workspace (PTB_ERR_NULL) or one
 * shorter than ptb_gemm_bf16_workspace_bytes (PTB_ERR_WORKSPACE).
 * Replaces: the same kernels as ptb_gemm_bf16 (the small M x N gemm_<M>x<K>x<N>_bf16 shapes). */
size_t ptb_gemm_bf16_workspace_bytes(int64_t m, int64_t n, int64_t k);
int ptb_gemm_bf16_ws(const void* a, const void* b, const void* residual, void* c, int64_t m, int64_t n, int64_t k,
                     void* workspace, size_t workspace_bytes, void* stream);

/* The gate_up GEMM with the SwiGLU gate fused into its epilogue: for A [m, k] and B [k, 2*inter]
 * (gate columns [0, inter), up columns [inter, 2*inter)), C [m, inter] = bf16( silu(g) * u ) with
 * g, u = bf16(A . B[:, j]) and bf16(A . B[:, inter + j]) and silu(g) = g / (1 + e^-g), fp32 --
 * bit for bit what ptb_gemm_bf16 followed by ptb_silu_mul_bf16 give, without the [m, 2*inter]
 * intermediate.  k % 64 == 0, inter % 128 == 0, 2 * inter <= 2^22 (and the ptb_gemm_bf16 offset
 * limits for n = 2 * inter).
 * Replaces: qwen3_8b_layer_prefill_2048x2048_bf16/09_..._fused__to_copy_add_mean_mm_mul_pow_rsqrt_5ojlpnva's
 *           gate_up product together with 10_..._fused__to_copy_mul_silu_slice_ktzl5s2h (the pair
 *           ptb_amd.qwen3's prefill layer launches back to back; the bundle's manifests keep them apart). */
int ptb_gemm_swiglu_bf16(const void* a, const void* b, void* c, int64_t m, int64_t inter, int64_t k, void* stream);

/* Per-row dynamic e4m3 quantisation of bf16 activations: scale[r] = max_c |x[r,c]| / 448,
 * xq[r,c] = e4m3fn(x[r,c] / scale[r]) (round to nearest even; an all-zero row gets scale 1).
 * Semantics: tests/cases/mechanism/ops/ops_fp8_e4m3_dot.py:41-44 (the e4m3 cast) and
 * tests/cases/workloads/int8_dequant_matmul.py:59-69 (per-token scale). */
int ptb_quant_rows_e4m3(const void* x, void* xq, float* scale, int64_t rows, int64_t cols,
                        void* stream);

/* Per-output-channel e4m3 quantisation of an fp32 weight W[k, n] (row-major):
 * scale[j] = max_i |W[i,j]| / 448, and the packed weight is stored transposed, wq_t[j, i] =
 * e4m3fn(W[i,j] / scale[j]) (K contiguous, the layout the fp8 GEMM streams). */
int ptb_quant_weight_e4m3(const float* w, void* wq_t, float* scale, int64_t k, int64_t n,
                          void* stream);

/* fp8-weight GEMM: C[m,n] = bf16( (sum_k aq[m,k] * wq_t[n,k]) * sa[m] * sw[n] ), e4m3 operands,
 * fp32 accumulation.  Requires k % 128 == 0 and n % 16 == 0, 256 * k below 4 GiB and n <= 2^22.
 * Semantics: tests/cases/mechanism/ops/ops_fp8_e4m3_dot.py:13-60 and
 *            tests/cases/workloads/int8_dequant_matmul.py:59-69 (scale epilogue). */
int ptb_gemm_fp8_scaled(const void* aq, const float* sa, const void* wq_t, const float* sw, void* c,
                        int64_t m, int64_t n, int64_t k, void* stream);


/* Flash-attention forward, head-major layout: q/o [batch*hq, seq, head_dim], k/v [batch*hkv, seq,
 * head_dim]; q head h reads kv head h / (hq / hkv).  Online softmax in fp32 with P rounded to bf16
 * before P.V; causal masks key > query.  head_dim must be 128 and seq a multiple of 128.
 * Replaces: validation/pytorchsim/attention_prefill_32x8x4096_bf16/00__prefill_kernel/
 *           _prefill_kernel_triton.py:4-44 (and qwen3_8b_layer_prefill_2048x2048_bf16/06__prefill_kernel). */
int ptb_flash_attn_fwd_bf16(const void* q, const void* k, const void* v, void* o, int64_t batch,
                            int64_t hq, int64_t hkv, int64_t seq, int64_t head_dim, float scale,
                            int causal, void* stream);
/* The same attention with O written token-major, o [batch, seq, hq, 128] (row t of batch b holds
 * every query head's output for token t), the layout the layer's output projection reads: the
 * separate head transpose after attention is not needed.
 * Replaces: 06__prefill_kernel together with 07_..._fused_clone_select_transpose_ei42assc of
 *           qwen3_8b_layer_prefill_2048x2048_bf16 (attention, then O -> [T, 32, 128]). */
int ptb_flash_attn_fwd_tokens_bf16(const void* q, const void* k, const void* v, void* o, int64_t batch,
                                   int64_t hq, int64_t hkv, int64_t seq, int64_t head_dim, float scale, int causal,
                                   void* stream);

/* The prefill layer's attention reading the fused projection in place: qkv is [batch*seq, ld] bf16
 * (ld >= (hq + 2*hkv)*128, ld % 8 == 0) holding each token's q (columns [0, hq*128)), k and v
 * (columns [(hq+hkv)*128, (hq+2*hkv)*128)); k is the k-norm + RoPE output [batch*hkv, seq, 128].
 * Each query row gets its per-head RMSNorm (qnorm_w [128] bf16, eps) and rotate-half RoPE (cos_t /
 * sin_t [seq, 128] fp32) in the kernel's prologue, v is read with row stride ld, and o is written
 * token-major [batch, seq, hq, 128]: bit-identical to ptb_qk_norm_rope_ld_bf16 (q) +
 * ptb_transpose_heads_ld_bf16 (v) + ptb_flash_attn_fwd_tokens_bf16, in one launch.
 * Replaces: qwen3_8b_layer_prefill_2048x2048_bf16/02_..._mmis7ufj_triton.py:17-98 (q-norm + RoPE),
 *           05_..._ff5nvvqz_triton.py:17-27 (v transpose), 06__prefill_kernel and
 *           07_..._fused_clone_select_transpose_ei42assc (O -> [T, 32, 128]). */
int ptb_flash_attn_fwd_qkv_bf16(const void* qkv, int64_t ld, const void* k, const void* qnorm_w, const float* cos_t,
                                const float* sin_t, float eps, void* o, int64_t batch, int64_t hq, int64_t hkv,
                                int64_t seq, int64_t head_dim, float scale, int causal, void* stream);

/* ---- single-token (decode) path: qwen3_8b_layer_decode_1x<S>_bf16 and attention_decode_* ---- */

/* out[0] = sum_i (float(x[i]) + float(y[i]))^2 in fp32; y may be NULL (then sum x^2).  One workgroup.
 * Replaces: qwen3_8b_layer_decode_1x<S>_bf16/00_..._fused__to_copy_mean_pow_3iwn5auz_triton.py:17-41 (x^2) and
 *           05_..._fused__to_copy_add_mean_pow_tcz6sl32_triton.py:17-43 ((x + a)^2). */
int ptb_sumsq_bf16(const void* x, const void* y, float* out, int64_t n, void* stream);

/* Matrix-vector products y[n] = bf16( sum_k xp[k] * W[k,n] ), W row-major [k, n] bf16, fp32
 * accumulation split over k; the fp32 partials live in a caller workspace of
 * ptb_gemv_workspace_bytes(k, n) bytes.  n % 8 == 0, W 16-byte aligned.
 *   ptb_gemv_bf16:          xp = x.
 *     Replaces decode 04_..._fused_add_select_transpose_view_vumxrjnr_triton.py:17-42 (o-projection).
 *   ptb_gemv_rmsnorm_bf16:  xp = ((x + add) * rsqrt(ss[0]/k + eps)) * g, all fp32; add may be NULL.
 *     ss may be NULL: then every workgroup forms sum((x + add)^2) over k itself (x, add 16-byte
 *     aligned), which saves the ptb_sumsq_bf16 launch a decode step otherwise makes before it.
 *     Replaces decode 01_..._fused__to_copy_add_mean_mm_mul_pow_rsqrt_ddfn4f75_triton.py:17-55 (q-projection)
 *     and 06_..._5gopcdje_triton.py:17-57 (gate/up projection after the post-attention norm).
 *   ptb_gemv_silu_bf16:     xp = silu(gate_up[k']) * gate_up[k + k'] (gate_up holds 2k values);
 *     y = bf16( sum + (res_a[n] + res_b[n]) ), res_a/res_b may be NULL.
 *     Replaces decode 07_..._fused__to_copy_add_mul_silu_slice_3d4ocw7y_triton.py:17-56 (down projection
 *     plus the residual). */
size_t ptb_gemv_workspace_bytes(int64_t k, int64_t n);
int ptb_gemv_bf16(const void* x, const void* w, void* y, int64_t k, int64_t n, void* workspace,
                  size_t workspace_bytes, void* stream);
int ptb_gemv_rmsnorm_bf16(const void* x, const void* add, const float* ss, const void* g, float eps,
                          const void* w, void* y, int64_t k, int64_t n, void* workspace,
                          size_t workspace_bytes, void* stream);
int ptb_gemv_silu_bf16(const void* gate_up, const void* w, const void* res_a, const void* res_b, void* y,
                       int64_t k, int64_t n, void* workspace, size_t workspace_bytes, void* stream);

/* The decode layer's gate/up and down projections with the gate/up finish pass folded into the down
 * projection's prologue (one launch fewer).  ptb_gemv_rmsnorm_parts_bf16 is ptb_gemv_rmsnorm_bf16's
 * partial pass alone: its fp32 partials stay in `parts` (ptb_gemv_workspace_bytes(k, n) bytes, 4-byte
 * aligned) and nothing is written to a y.  ptb_gemv_silu_parts_bf16 is ptb_gemv_silu_bf16 whose
 * gate_up vector is formed from such partials (gate_up_parts written by ptb_gemv_rmsnorm_parts_bf16
 * with k = gate_up_k and n = 2 * k) with the finish pass's own sums and rounding, so its y is bit for
 * bit that of ptb_gemv_rmsnorm_bf16 followed by ptb_gemv_silu_bf16; `workspace` is its own partials'
 * (ptb_gemv_workspace_bytes(k, n) bytes) and must not overlap gate_up_parts.
 * Replaces: decode 06_..._5gopcdje_triton.py:17-57 and 07_..._3d4ocw7y_triton.py:17-56 together. */
int ptb_gemv_rmsnorm_parts_bf16(const void* x, const void* add, const float* ss, const void* g, float eps,
                                const void* w, float* parts, int64_t k, int64_t n, size_t parts_bytes, void* stream);
int ptb_gemv_silu_parts_bf16(const float* gate_up_parts, int64_t gate_up_k, const void* w, const void* res_a,
                             const void* res_b, void* y, int64_t k, int64_t n, void* workspace,
                             size_t workspace_bytes, void* stream);

/* Decode attention for one query token: q, o [nkv, group, 128]; k, v [nkv, seq, 128] (nkv = batch *
 * kv heads; query head g of kv head h is row h*group + g).  Full softmax over the seq cached keys,
 * P rounded to bf16 before P.V, fp32 row sums.  group in {1,2,3,4,6,8}; q, k, v 16-byte aligned.
 * Workspace: ptb_attn_decode_workspace_bytes(nkv, group, seq) bytes, 16-byte aligned; 0 bytes (and
 * workspace may be NULL) when seq <= 256, which is a single launch.  seq below 2^30 (else
 * PTB_ERR_GRID).
 * Replaces: attention_decode_<HQ>x8x<S>_bf16/00__decode_kernel/_decode_kernel_triton.py:4-29 (and
 *           qwen3_8b_layer_decode_1x<S>_bf16/03__decode_kernel). */
size_t ptb_attn_decode_workspace_bytes(int64_t nkv, int64_t group, int64_t seq);
int ptb_attn_decode_bf16(const void* q, const void* k, const void* v, void* o, int64_t nkv, int64_t group,
                         int64_t seq, int64_t head_dim, float scale, void* workspace,
                         size_t workspace_bytes, void* stream);

/* Allocation-free decode attention: ptb_attn_decode_bf16 with its partial records in a static device
 * scratch of ptb_attn_decode_noalloc_max_bytes() bytes (16 MiB) instead of a caller workspace; no
 * allocation of any kind.  No counterpart in the reference: for callers that cannot allocate (code
 * under HIP graph capture, serving loops that forbid hipMalloc).  A shape whose workspace
 * (ptb_attn_decode_workspace_bytes) exceeds the scratch is refused with PTB_ERR_WORKSPACE.  Each GPU
 * holds its own scratch until the process ends, its address looked up on the first call on that
 * device; calls that overlap on one GPU share it and race. */
size_t ptb_attn_decode_noalloc_max_bytes(void);
int ptb_attn_decode_bf16_noalloc(const void* q, const void* k, const void* v, void* o, int64_t nkv, int64_t group,
                                 int64_t seq, int64_t head_dim, float scale, void* stream);

/* Decode attention with the query's per-head RMSNorm and rotate-half RoPE done in its prologue:
 * q is the q projection's raw output [nkv, group, 128]; each workgroup normalizes (qnorm_w [128]
 * bf16, eps) and rotates (cos_t / sin_t [128] fp32 of the token's position) its own query rows,
 * rounding them to bf16 exactly as ptb_qk_norm_rope_bf16 does, then attends as
 * ptb_attn_decode_bf16 (same workspace).  qnorm_w, cos_t, sin_t 16-byte aligned.
 * Replaces: qwen3_8b_layer_decode_1x<S>_bf16/02__decode_kernel (q-norm + RoPE) together with
 *           qwen3_8b_layer_decode_1x<S>_bf16/03__decode_kernel (attention). */
int ptb_attn_decode_qnorm_rope_bf16(const void* q, const void* qnorm_w, const float* cos_t, const float* sin_t,
                                    float eps, const void* k, const void* v, void* o, int64_t nkv, int64_t group,
                                    int64_t seq, int64_t head_dim, float scale, void* workspace,
                                    size_t workspace_bytes, void* stream);

/* ---- Qwen3-30B-A3B mixture-of-experts layer (validation/pytorchsim/layer_op_* and layer_layer_*).
 * Paths below are relative to validation/pytorchsim/; LOP_<op> = layer_op_<op>_1024x0_bf16 and
 * LL = layer_layer_prefill_1024x1024_bf16 (other token counts differ only in sizes).  Index
 * arguments are int64 (int32 where named); entries outside a table are bounds-checked and give
 * zeros where the reference would stop on a device_assert. */

/* Zero nbytes at out (a fill kernel, no memset: safe in captured graphs).
 * Replaces: LOP_gmm_gate_up/00_..._fused_new_zeros_q6uym5lr_triton.py:17-22 */
int ptb_fill_zero(void* out, int64_t nbytes, void* stream);

/* y[i] = (int32) x[i] (two's-complement wrap).
 * Replaces: LOP_gmm_gate_up/04_..._fused__to_copy_oeoxw6br_triton.py:17-23 */
int ptb_cast_i64_i32(const int64_t* x, int32_t* y, int64_t n, void* stream);

/* Inclusive prefix sum of n <= 8192 integers (x_dtype, y_dtype: PTB_DTYPE_I32 / _I64), into y0 and,
 * when not NULL, y1; int32 results wrap.
 * Replaces: LOP_gmm_gate_up/01_..._fused_cumsum_6fi3sv3v_triton.py:17-33, LOP_combine/01_..._fused_cumsum_
 *           qi2bfo64_triton.py:17-33, LL/08_..._fused__to_copy_cumsum_ggousx36_triton.py:17-35 */
int ptb_cumsum_int(const void* x, int x_dtype, void* y0, void* y1, int y_dtype, int64_t n, void* stream);

/* From inclusive group ends (int32 or int64, n <= 8192): starts[i] = ends[i-1] (0 for i = 0),
 * rows[i] = ends[i] - starts[i], nonempty[i] = #{j <= i : rows[j] > 0}; all int64.
 * Replaces: LOP_gmm_gate_up/02_..._fused__to_copy_cat_cumsum_gt_new_zeros_slice_sub_gnib2ocx_triton.py:17-57 */
int ptb_moe_group_table(const void* ends, int ends_dtype, int64_t n, int64_t* nonempty, int64_t* starts,
                        int64_t* rows, void* stream);

/* out[i] = #{r < n : x[r] <= i} as int32, i < m.
 * Replaces: LOP_gmm_gate_up/03_..._fused__to_copy_arange_le_sum_unsqueeze_j72wougd_triton.py:17-35 */
int ptb_count_le(const int64_t* x, int64_t n, int32_t* out, int64_t m, void* stream);

/* Expert histogram of r slot ids over e <= 1024 experts: counts[x] (and counts2[x] when not NULL)
 * = #{s : ids[s] == x}; cum[s*e + x] = #{s' <= s : ids[s'] == x}.
 * Replaces: LOP_combine/00_..._fused__to_copy_arange_cumsum_eq_sum_unsqueeze_view_dmnbvm2a_triton.py:17-54
 *           and LL/07_..._vrrn72ou (two count outputs) */
int ptb_moe_expert_count(const int64_t* ids, int64_t r, int64_t e, int64_t* counts, int64_t* counts2,
                         int64_t* cum, void* stream);

/* out[s] = cum[s*e + ids[s]] (each slot's 1-based rank within its expert; 0 if ids[s] is no expert).
 * Replaces: LOP_combine/02_..._fused__to_copy_arange_eq_mul_sum_unsqueeze_view_dmbn5ao4_triton.py:17-44 */
int ptb_moe_rank_select(const int64_t* cum, const int64_t* ids, int64_t r, int64_t e, int64_t* out, void* stream);

/* Stable sort of each of `rows` rows of e keys (key_dtype PTB_DTYPE_I64 or PTB_DTYPE_F32, values
 * the same dtype): values in order, indices = original positions (int64); floats order NaN above
 * +inf and -0 as +0.  Rows longer than 8192 need ptb_sort_workspace_bytes(rows, e) of workspace.
 * Replaces: LOP_dispatch/00__sort_kernel/_sort_kernel_triton.py:4-49 */
size_t ptb_sort_workspace_bytes(int64_t rows, int64_t e);
int ptb_sort_rows(const void* x, int key_dtype, void* values, int64_t* indices, int64_t rows, int64_t e,
                  int descending, void* workspace, size_t workspace_bytes, void* stream);

/* The k largest (largest != 0) or smallest of each row of e <= 1024 fp32 values, in order, ties to
 * the lowest position; indices int64.
 * Replaces: LOP_router_post/01__topk_kernel/_topk_kernel_triton.py:4-30 */
int ptb_topk_rows_f32(const float* x, int64_t rows, int64_t e, int64_t k, int largest, float* values,
                      int64_t* indices, void* stream);

/* out[s, :] = x[floor(slot[s] / k), :] for r slots (bf16 rows of c; the token index wraps from the
 * end when negative; rows with no such token are zeros).
 * Replaces: LOP_dispatch/01_..._fused_floor_divide_index_select_guslzqr3_triton.py:17-42 and
 *           LL/23_..._fused__to_copy_floor_divide_index_select_4hjjds7p */
int ptb_moe_gather_rows_bf16(const int64_t* slot, int64_t r, int64_t k, const void* x, int64_t t, int64_t c,
                             void* out, void* stream);

/* Each of `tokens` tokens' weighted sum of its k expert rows of y (yrows x c, bf16): slot s = t*k + j
 * of expert id = ids[s] sits at row ends[id] - counts[id] + rank[s] - 1.  w_dtype PTB_DTYPE_BF16: w
 * bf16, wsum NULL, out = bf16(sum); PTB_DTYPE_F32: weight w[s] / wsum[t] and, with h, out is updated
 * in place: out = bf16((h + out) + sum).  fp32 accumulation.
 * Replaces: LOP_combine/03_..._fused__to_copy_add_index_select_mul_sub_sum_unsqueeze_view_jskr7oe3_triton.py
 *           :17-54 and LL/27_..._fused__to_copy_add_div_index_select_mul_sub_sum_unsqueeze_view_pjwo6jhr
 *           _triton.py:17-63 */
int ptb_moe_combine_bf16(const int64_t* ids, const int64_t* ends, const int64_t* counts, const int64_t* rank,
                         const void* y, int64_t yrows, const void* w, int w_dtype, const float* wsum, const void* h,
                         void* out, int64_t tokens, int64_t k, int64_t e, int64_t c, void* stream);

/* Rows of k fp32 values: out_bf16[r, j] = bf16(x[r, j] / sum_j x[r, j]) (out_sum NULL), or
 * out_sum[r] = sum_j x[r, j] (out_bf16 NULL).
 * Replaces: LOP_router_post/02_..._fused__to_copy_div_sum_d4c5sb6k_triton.py:17-35 and
 *           LL/22_..._fused_sum_kon7yqsn_triton.py:17-34 */
int ptb_normalize_rows_f32(const float* x, int64_t rows, int64_t k, void* out_bf16, float* out_sum, void* stream);

/* y = bf16(float(a) + float(b)).
 * Replaces: LOP_residual/00_..._fused_add_dfgomnnn_triton.py:17-26 */
int ptb_add_bf16(const void* a, const void* b, void* y, int64_t n, void* stream);

/* Rotate-half RoPE without a norm: x, out [tokens, heads, 128] bf16, cos/sin [tokens, 128] fp32.
 * Replaces: LOP_rope_q/00_..._fused__to_copy_add_cat_mul_neg_slice_unsqueeze_4de5dxfe_triton.py:17-47
 *           (and rope_k) */
int ptb_rope_bf16(const void* x, const float* cos_t, const float* sin_t, void* out, int64_t tokens, int64_t heads,
                  int64_t head_dim, void* stream);

/* y = bf16( (x + a) * rsqrt(sum((x + a)^2) / cols + eps) * w ) per row, x + a in fp32 (a may be NULL).
 * Replaces: LL/18_..._fused__to_copy_add_mean_mul_pow_rsqrt_p5e5f5kj_triton.py:17-58 */
int ptb_rmsnorm_add_bf16(const void* x, const void* a, const void* w, void* y, int64_t rows, int64_t cols,
                         float eps, void* stream);

/* One token's normalised vector to each of its `rows` slots: out[s, :] = bf16( (x + a) *
 * rsqrt(ss[0] / cols + eps) * w ).
 * Replaces: layer_layer_decode_1x1024_bf16/19_..._fused__to_copy_add_floor_divide_index_select_mean_mul_pow_
 *           rsqrt_wkrpkilh_triton.py:17-60 */
int ptb_rms_broadcast_bf16(const void* x, const void* a, const float* ss, const void* w, void* out, int64_t rows,
                           int64_t cols, float eps, void* stream);

/* Grouped GEMM: for program p < nprog (<= 256), g = group[p] (int32): C[start[g] + i, :] =
 * bf16( A[start[g] + i, :] . B_g ) for i < rows[g], B_g the row-major [k, n] bf16 matrix at
 * b + g * weight_stride (nweights of them); A is [a_rows, k], C [a_rows, n]; start/rows hold ntab
 * int32 entries.  Entries that do not describe rows inside A or a weight inside B count as empty.
 * A group listed by several programs is computed once (with ntab <= 1024).  The groups' row ranges
 * must not overlap one another (the reference's tables, consecutive ranges of expert rows, never
 * do; overlapping ranges written with different weights have no defined result there either): the
 * launch sizes its grid for ceil(a_rows / 128) + nprog row tiles.  k % 64 == 0, n % 8 == 0.
 * Replaces: LOP_gmm_gate_up/05__grouped_mm_kernel/_grouped_mm_kernel_triton.py:4-46 (and gmm_down) */
int ptb_grouped_gemm_bf16(const void* a, const void* b, const int32_t* group, const int32_t* start,
                          const int32_t* rows, void* c, int64_t nprog, int64_t ntab, int64_t a_rows,
                          int64_t nweights, int64_t k, int64_t n, int64_t weight_stride, void* stream);
/* The same grouped GEMM with a caller workspace of ptb_grouped_gemm_workspace_bytes(nprog, a_rows,
 * k, n) bytes (16-byte aligned), non-zero when a_rows <= 16: a split-K GEMV pass over each
 * program's weight (every weight row read once per 4 rows of A) and a pass that sums the slices,
 * rounding once.  Same results contract and argument checks as ptb_grouped_gemm_bf16, which it
 * calls when the workspace query is 0 or the workspace is missing or short.
 * Replaces: the same grouped_mm kernels, at the decode shapes (layer_layer_decode_1x<S>_bf16/20, 22) */
size_t ptb_grouped_gemm_workspace_bytes(int64_t nprog, int64_t a_rows, int64_t k, int64_t n);
int ptb_grouped_gemm_bf16_ws(const void* a, const void* b, const int32_t* group, const int32_t* start,
                             const int32_t* rows, void* c, int64_t nprog, int64_t ntab, int64_t a_rows,
                             int64_t nweights, int64_t k, int64_t n, int64_t weight_stride, void* workspace,
                             size_t workspace_bytes, void* stream);

/* ---- spec-driven entry points: one per kernel family ----
 * The reference's generated driver calls a lowered kernel as
 *   <kernel>(1, &desc_0, ..., 1, &desc_n, scalars..., gx, gy, gz, pidx, pidy, pidz)
 * once per program, desc_i being a memref descriptor {allocated, aligned, offset, size, stride} per
 * tensor in spec order (reference: pytorchsim_triton_compiler/codegen/wrapper.py:37-51 declaration,
 * :140-146 descriptor, :126-277 main, program loop :254-265).  Each ptb_<family>_args entry takes
 * the same in one call: `args` the tensors in spec order as ptb_tensor descriptors, `ints` / `floats`
 * the family's integer and floating-point parameters in the order listed per entry (the kernel's
 * runtime scalars and the constexprs its compile baked in), and `grid` the launch grid.
 * Sizes come from the descriptors and must agree with the parameters (PTB_ERR_SHAPE otherwise, as
 * a wrong count `nargs` / `nints` / `nfloats`).  Every family runs its programs along x.  Where the
 * last int is `programs`, it is the program bound the kernel was compiled for (kernel.json's
 * grid_bound, else the spec's grid), the programs splitting the rows (or outputs) evenly; the other
 * families' bound follows from their shape.  A grid with gy or gz != 1, gx < 1 or gx past the bound
 * is refused with PTB_ERR_GRID (contract/kernel_object.py:93-107 refuse_grid_past_bound).  A grid
 * below the bound runs the programs it covers where they are blocks of whole rows (rmsnorm,
 * softmax, silu_mul, and flash_attn over whole batches); elsewhere it is PTB_ERR_UNSUPPORTED.  A
 * tensor must be flat (stride 1 when size > 1), and a written tensor must not have role
 * PTB_ROLE_IN. */
typedef struct ptb_tensor {
  void* allocated;  /* allocation base (not read) */
  void* aligned;    /* element 0 sits at aligned + offset * itemsize */
  int64_t offset;   /* in elements */
  int64_t size;     /* elements */
  int64_t stride;   /* 1 */
  int32_t dtype;    /* PTB_DTYPE_* */
  int32_t role;     /* PTB_ROLE_* */
} ptb_tensor;

/* args [x, w, y] (L2048/00's in_ptr0, in_ptr1, out_ptr1), x/y bf16 with w bf16 or fp32, or all
 * fp32; or, all fp32, [x, w, o, c] with the column arm c[cols] = rsqrt(mean over the rows the grid
 * covers of x^2 + eps); ints [rows (xnumel), cols (r0_numel), programs (, block)]; floats [eps].
 * Row-block families (rmsnorm, softmax, silu_mul, add_scalar) run the leading gx blocks of `block`
 * rows (elements) a program -- the kernel's XBLOCK when stated, else ceil(extent / programs).
 * Replaces: qwen3_8b_layer_prefill_2048x2048_bf16/00_..._gwdq6qer_triton.py:17-60 and
 *           tests/cases/workloads/rmsnorm.py:44-57 (both arms) */
int ptb_rmsnorm_args(const ptb_tensor* args, int nargs, const int64_t* ints, int nints, const double* floats,
                     int nfloats, const int32_t grid[3], void* stream);
/* args [x, y]: bf16 -> bf16, bf16 -> fp32 or fp32 -> fp32; ints [rows, cols, programs (, block)].
 * Replaces: vector_softmax_<R>x<C>_bf16/00_..._triton.py:17-68, layer_layer_decode_1x1024_bf16/16
 *           (fp32 out), tests/cases/workloads/softmax.py:46-55 */
int ptb_softmax_args(const ptb_tensor* args, int nargs, const int64_t* ints, int nints, const double* floats,
                     int nfloats, const int32_t grid[3], void* stream);
/* args [gate_up, out] (bf16 or fp32); ints [rows, inter, programs (, block of outputs)].
 * Replaces: qwen3_8b_layer_prefill_2048x2048_bf16/10_..._ktzl5s2h_triton.py:17-36 */
int ptb_silu_mul_args(const ptb_tensor* args, int nargs, const int64_t* ints, int nints, const double* floats,
                      int nfloats, const int32_t grid[3], void* stream);
/* args [A, B, C] or, with the residual epilogue, [R, A, B, C] (bf16); ints [M, N, K, programs]
 * (only the whole grid runs: a partial grid's tiles follow the caller's template order).
 * Replaces: qwen3_8b_layer_prefill_2048x2048_bf16/01_..._ckb6aiys_triton.py:18-97 (and 03, 09),
 *           08_..._utuycvlm_triton.py:18-99, 11_..._fjjozd2g_triton.py:18-66, gemm_<M>x<K>x<N>_bf16 */
int ptb_gemm_args(const ptb_tensor* args, int nargs, const int64_t* ints, int nints, const double* floats,
                  int nfloats, const int32_t grid[3], void* stream);
/* args [q, k, v, o] head-major bf16; ints [batch, HQ, HKV (HQ / G), S, D, CAUSAL]; floats [SCALE];
 * one program per (batch, query head).
 * Replaces: attention_prefill_<HQ>x<HKV>x<S>_bf16/00__prefill_kernel/_prefill_kernel_triton.py:4-44 */
int ptb_flash_attn_args(const ptb_tensor* args, int nargs, const int64_t* ints, int nints, const double* floats,
                        int nfloats, const int32_t grid[3], void* stream);
/* args [q, k, v, o] (+ a workspace descriptor of ptb_attn_decode_workspace_bytes bytes when
 * S > 256); ints [HKV, G, S, D]; floats [SCALE]; one program per kv head (only the whole grid).
 * Replaces: attention_decode_<HQ>x8x<S>_bf16/00__decode_kernel/_decode_kernel_triton.py:4-29 */
int ptb_attn_decode_args(const ptb_tensor* args, int nargs, const int64_t* ints, int nints, const double* floats,
                         int nfloats, const int32_t grid[3], void* stream);
/* args [x, w, cos, sin, out] (L2048/02's in_ptr0..3, out_ptr2); ints [tokens, heads, head_dim,
 * programs]; floats [eps]; only the whole grid.
 * Replaces: qwen3_8b_layer_prefill_2048x2048_bf16/02_..._mmis7ufj_triton.py:17-98 (and 04) */
int ptb_qk_norm_rope_args(const ptb_tensor* args, int nargs, const int64_t* ints, int nints, const double* floats,
                          int nfloats, const int32_t grid[3], void* stream);
/* args [x, y]; ints [d0, d1, inner, programs]: y[b, a, :] = x[a, b, :]; only the whole grid.
 * Replaces: qwen3_8b_layer_prefill_2048x2048_bf16/05_..._ff5nvvqz_triton.py:17-27 and 07_..._ei42assc */
int ptb_transpose_heads_args(const ptb_tensor* args, int nargs, const int64_t* ints, int nints,
                             const double* floats, int nfloats, const int32_t grid[3], void* stream);

/* args [x, out] or [x, y, out] (x, y bf16 [n], out fp32 [1]); ints [n, programs]; only the whole
 * grid.  Replaces: qwen3_8b_layer_decode_1x<S>_bf16/00_..._fused__to_copy_mean_pow_3iwn5auz_triton.py:17-41
 *           and 05_..._fused__to_copy_add_mean_pow_tcz6sl32_triton.py:17-43 */
int ptb_sumsq_args(const ptb_tensor* args, int nargs, const int64_t* ints, int nints, const double* floats,
                   int nfloats, const int32_t grid[3], void* stream);
/* ints [mode, k, n, extra, programs]; args, then a workspace descriptor of
 * ptb_gemv_workspace_bytes(k, n) bytes (any dtype):
 *   mode 0 (plain):   [x, W, y], extra 0
 *   mode 1 (RMSNorm): [x, (add,) ss, g, W, y], extra = 1 with add; floats [eps]
 *   mode 2 (silu):    [gate_up, W, (res_a, (res_b,)) y], extra = the residual count
 * W [k, n] row-major bf16; only the whole grid.
 * Replaces: gemm_1x2048x128_bf16/00_..._fused_mm_oyeae7au_triton.py:17-42 (the M = 1 mm template), decode
 *           04_..._vumxrjnr_triton.py:17-42, 01_..._ddfn4f75_triton.py:17-55, 06_..._5gopcdje_triton.py:17-57,
 *           07_..._3d4ocw7y_triton.py:17-56 of qwen3_8b_layer_decode_1x<S>_bf16 */
int ptb_gemv_args(const ptb_tensor* args, int nargs, const int64_t* ints, int nints, const double* floats,
                  int nfloats, const int32_t grid[3], void* stream);
/* args [x (bf16 or fp32), out fp32 [1]] + a workspace descriptor of ptb_reduce_workspace_bytes(n)
 * bytes; ints [n, op (PTB_REDUCE_SUM / PTB_REDUCE_MAX), programs]; only the whole grid.
 * Replaces: vector_sum_<R>x<C>_bf16/00_..._2y6fwkvp_triton.py, vector_max_<R>x<C>_bf16/00_..._q47252w4_triton.py,
 *           layer_layer_decode_1x<S>_bf16/18_..._fused_sum_7gslrk5a_triton.py:17-38 */
int ptb_reduce_args(const ptb_tensor* args, int nargs, const int64_t* ints, int nints, const double* floats,
                    int nfloats, const int32_t grid[3], void* stream);
/* args [x, y] bf16 [n]; ints [n, programs (, block)]; floats [s]; a partial grid covers its leading
 * blocks.  Replaces: vector_add1_<R>x<C>_bf16/00_..._du5rd5jd_triton.py */
int ptb_add_scalar_args(const ptb_tensor* args, int nargs, const int64_t* ints, int nints, const double* floats,
                        int nfloats, const int32_t grid[3], void* stream);
/* args [x bf16, out fp32 [count]]; ints [first, count, programs]; floats [s]; first + count within
 * x; only the whole grid.  Replaces: vector_slice_<R>x<C>_bf16/00_..._slnyinbt_triton.py:17-27 */
int ptb_slice_add_args(const ptb_tensor* args, int nargs, const int64_t* ints, int nints, const double* floats,
                       int nfloats, const int32_t grid[3], void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PTB_AMD_H */
