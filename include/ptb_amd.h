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
 * nothing is allocated, and there is no global mutable state, so entry points are thread-safe.
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

/* Row softmax: y = bf16( exp(x - max) / sum(exp(x - max)) ), max NaN-propagating, fp32 math.
 * Replaces: validation/pytorchsim/vector_softmax_2048x6144_bf16/00_..._sa7wwqqf/..._triton.py:17-68 */
int ptb_softmax_rows_bf16(const void* x, void* y, int64_t rows, int64_t cols, void* stream);

/* The same row softmax with the probabilities stored as fp32 (no rounding): the MoE router's
 * softmax over expert logits.
 * Replaces: validation/pytorchsim/layer_layer_decode_1x1024_bf16/16_..._qslpdpud/
 *           pytorchsim_triton_compiler_fused__softmax__to_copy_qslpdpud_triton.py:17-45 */
int ptb_softmax_rows_bf16_f32(const void* x, void* y, int64_t rows, int64_t cols, void* stream);

/* SiLU gate: out[t,j] = bf16( (g / (1 + exp(-g))) * u ), g = gu[t, j], u = gu[t, inter + j].
 * Replaces: qwen3_8b_layer_prefill_2048x2048_bf16/10_..._ktzl5s2h/..._triton.py:17-36 */
int ptb_silu_mul_bf16(const void* gate_up, void* out, int64_t rows, int64_t inter, void* stream);

/* Head transpose: y[b, a, :] = x[a, b, :] for x of shape [d0, d1, inner] (exact copy).
 * [T,H,D] -> [H,T,D] replaces qwen3_8b_layer_prefill_2048x2048_bf16/05_..._ff5nvvqz_triton.py:17-27;
 * [H,T,D] -> [T,H,D] replaces 07_..._ei42assc_triton.py:17-27. */
int ptb_transpose_heads_bf16(const void* x, void* y, int64_t d0, int64_t d1, int64_t inner,
                             void* stream);

/* Per-(token, head) RMSNorm (eps) with weight w[head_dim], then rotate-half RoPE with fp32
 * cos/sin [tokens, head_dim], stored head-major: out[h, t, :].  x is [tokens, heads, head_dim].
 * Replaces: qwen3_8b_layer_prefill_2048x2048_bf16/02_..._mmis7ufj_triton.py:17-98 (H=32) and
 *           04_..._ll67ghqi_triton.py (H=8); with tokens = 1, qwen3_8b_layer_decode_1x<S>_bf16/
 *           02_..._twgfj5dp_triton.py:17-96 (cos/sin of the token's position, [1, head_dim]). */
int ptb_qk_norm_rope_bf16(const void* x, const void* w, const float* cos_t, const float* sin_t,
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
 * residual may be NULL.  Requires k % 64 == 0 and n % 8 == 0; m is free.
 * Replaces: qwen3_8b_layer_prefill_2048x2048_bf16/01_..._fused_mm_ckb6aiys_triton.py:18-97 (and
 *           03, 09), the residual epilogues 08_..._utuycvlm_triton.py:18-99 and
 *           11_..._fjjozd2g_triton.py:18-66, and the gemm_<M>x<K>x<N>_bf16 bundle kernels. */
int ptb_gemm_bf16(const void* a, const void* b, const void* residual, void* c, int64_t m, int64_t n,
                  int64_t k, void* stream);

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
 * fp32 accumulation.  Requires k % 128 == 0 and n % 16 == 0.
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

/* Decode attention for one query token: q, o [nkv, group, 128]; k, v [nkv, seq, 128] (nkv = batch *
 * kv heads; query head g of kv head h is row h*group + g).  Full softmax over the seq cached keys,
 * P rounded to bf16 before P.V, fp32 row sums.  group in {1,2,3,4,6,8}; workspace of
 * ptb_attn_decode_workspace_bytes(nkv, group, seq) bytes.
 * Replaces: attention_decode_<HQ>x8x<S>_bf16/00__decode_kernel/_decode_kernel_triton.py:4-29 (and
 *           qwen3_8b_layer_decode_1x<S>_bf16/03__decode_kernel). */
size_t ptb_attn_decode_workspace_bytes(int64_t nkv, int64_t group, int64_t seq);
int ptb_attn_decode_bf16(const void* q, const void* k, const void* v, void* o, int64_t nkv, int64_t group,
                         int64_t seq, int64_t head_dim, float scale, void* workspace,
                         size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PTB_AMD_H */
