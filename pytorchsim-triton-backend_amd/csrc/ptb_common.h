// Shared device helpers for the gfx950 kernels: bf16/fp8 bit conversions, wave64 and block
// reductions, status handling.  Written for CDNA4 only (wave64, MFMA, 160 KB LDS).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ptb_amd.h"

// dma16 below clobbers m0 on purpose (its LDS base register); nothing else here uses m0.
#pragma clang diagnostic ignored "-Winline-asm"

#define PTB_EXPORT extern "C" __attribute__((visibility("default")))

namespace ptb {

constexpr int kWave = 64;

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(8))) int i32x8;
// 128-bit chunk as a native vector: arrays of these stay in registers (HIP's uint4 is a union
// struct, and private arrays of it are demoted to scratch or LDS).
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4v __attribute__((ext_vector_type(4)));

// bf16 bits -> fp32 (exact).
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float(uint32_t(b) << 16); }

// fp32 -> bf16 bits, round to nearest even (LLVM fptrunc; v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  __bf16 h = (__bf16)f;
  return __builtin_bit_cast(uint16_t, h);
}
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return uint32_t(f32_to_bf16(lo)) | (uint32_t(f32_to_bf16(hi)) << 16);
}

// silu's quotient g / b, b = 2^(-g log2 e) + 1 (>= 1, +inf or NaN), for g a bf16 value (the SwiGLU
// GEMM epilogue and silu_mul): the reciprocal, one correction of the quotient by its fma residual
// (Markstein), then the hardware's special-operand fixup (infinite or NaN operands, the sign of a
// zero).  Equal to the IEEE quotient for every bf16 value of g whose b is below 2^126 (checked on
// the device for all 65536 bf16 patterns of g); a larger b (g in about [-88.7, -87.3]) has a
// subnormal reciprocal, which v_rcp_f32 flushes to zero, so the caller divides those in IEEE
// arithmetic.  5 instructions where the IEEE sequence takes 9.
__device__ __forceinline__ float silu_quotient(float g, float b) {
  const float r = __builtin_amdgcn_rcpf(b);
  const float q0 = g * r;
  const float e = __builtin_fmaf(-b, q0, g);
  return __builtin_amdgcn_div_fixupf(__builtin_fmaf(e, r, q0), b, g);
}

// NaN-propagating max (triton's tl.maximum(..., PropagateNan.ALL)): NaN if either input is NaN.
// The IEEE 754-2019 maximum, which gfx950 executes as v_maximum3_f32 (three operands, so a chain of
// them takes two new values an instruction); it also orders -0 below +0.
__device__ __forceinline__ float max_nan(float a, float b) { return __builtin_elementwise_maximum(a, b); }

// NaN-propagating max of 8 values: four v_maximum3_f32.
__device__ __forceinline__ float max8_nan(const float (&f)[8]) {
  return max_nan(max_nan(max_nan(f[0], f[1]), max_nan(f[2], f[3])), max_nan(max_nan(f[4], f[5]), max_nan(f[6], f[7])));
}

// fp32 -> OCP e4m3fn bits with round-to-nearest-even, following torch's float8_e4m3fn cast:
// NaN stays NaN (0x7f), magnitudes that round past 448 become NaN, subnormals down to 2^-9.
__device__ __forceinline__ uint32_t f32_to_e4m3(float x) {
  uint32_t u = __float_as_uint(x);
  uint32_t sign = (u >> 24) & 0x80u;
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return sign | 0x7fu;              // NaN
  if (a > 0x43e80000u) return sign | 0x7fu;              // |x| > 464 rounds past 448 (or is inf)
  if (a < 0x3c800000u) {                                 // |x| < 2^-6: subnormal range, step 2^-9
    float m = __builtin_rintf(__uint_as_float(a) * 512.0f);  // exact scaling, RNE to integer
    return sign | uint32_t(m);                           // m == 8 is the smallest normal, 0x08
  }
  // normal: keep 3 mantissa bits, RNE on the 20 dropped bits
  uint32_t r = a + 0x7ffffu + ((a >> 20) & 1u);
  uint32_t e = (r >> 23) - 120u;                         // rebias 127 -> 7
  uint32_t m = (r >> 20) & 7u;
  return sign | (e << 3) | m;
}

// e4m3fn bits -> fp32 (exact).
__device__ __forceinline__ float e4m3_to_f32(uint32_t b) {
  uint32_t sign = (b & 0x80u) << 24;
  uint32_t e = (b >> 3) & 0xfu, m = b & 7u;
  if (e == 15u && m == 7u) return __uint_as_float(sign | 0x7fc00000u);
  float v = (e == 0u) ? float(m) * (1.0f / 512.0f) : __uint_as_float(((e + 120u) << 23) | (m << 20));
  return __uint_as_float(__float_as_uint(v) | sign);
}

// Cross-lane steps on the VALU, with no LDS round trip (a __shfl_xor is a ds_bpermute).  DPP moves
// within a 16-lane row: quad_perm [1,0,3,2] and [2,3,0,1] pair lanes l^1 and l^2; row_half_mirror
// (l <-> 7-l within 8) and row_mirror (l <-> 15-l) then pair quads and half-rows, whose lanes hold
// equal values by then, so every lane of the row ends with the full row result.  The permlane
// swaps (gfx950) exchange rows between two registers; handed the same value twice, the two results
// are v[l] and v[l^16] (or v[l^32]) in some order, and combining them with a commutative op gives
// every lane the same pair result.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_f32<0xb1>(v);
  v += dpp_f32<0x4e>(v);
  v += dpp_f32<0x141>(v);
  v += dpp_f32<0x140>(v);
  return v;
}
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_f32<0xb1>(v));
  v = fmaxf(v, dpp_f32<0x4e>(v));
  v = fmaxf(v, dpp_f32<0x141>(v));
  v = fmaxf(v, dpp_f32<0x140>(v));
  return v;
}
__device__ __forceinline__ float pair16_sum(float v) {   // v[l] + v[l ^ 16]
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float pair16_max(float v) {   // max(v[l], v[l ^ 16])
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair32_sum(float v) {   // v[l] + v[l ^ 32]
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float pair32_max(float v) {   // max(v[l], v[l ^ 32])
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// v[l ^ 8] within a 16-lane row (row_ror:8: rotating a row by 8 lanes is the xor-8 exchange).
__device__ __forceinline__ uint32_t xor8_u32(uint32_t v) {
  return uint32_t(__builtin_amdgcn_update_dpp(0, int(v), 0x128, 0xf, 0xf, false));
}

// wave64 reductions on the VALU (DPP within rows, then the two permlane swaps); every lane gets the
// result.  All 64 lanes take part.
template <class Op>
__device__ __forceinline__ float wave_reduce(float v, Op op) {
  v = op(v, dpp_f32<0xb1>(v));
  v = op(v, dpp_f32<0x4e>(v));
  v = op(v, dpp_f32<0x141>(v));
  v = op(v, dpp_f32<0x140>(v));
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = op(__uint_as_float(r[0]), __uint_as_float(r[1]));
  r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return op(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
struct AddOp {
  __device__ float operator()(float a, float b) const { return a + b; }
};
struct MaxNanOp {
  __device__ float operator()(float a, float b) const { return max_nan(a, b); }
};
struct MaxOp {
  __device__ float operator()(float a, float b) const { return fmaxf(a, b); }
};
__device__ __forceinline__ float wave_sum(float v) { return wave_reduce(v, AddOp()); }
__device__ __forceinline__ float wave_max_nan(float v) { return wave_reduce(v, MaxNanOp()); }
__device__ __forceinline__ float wave_absmax(float v) { return wave_reduce(v, MaxOp()); }

// Block reductions for blocks of NW waves; `red` is NW floats of LDS.  Every thread gets the result.
template <int NW>
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int w = threadIdx.x / kWave, l = threadIdx.x % kWave;
  if (l == 0) red[w] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int i = 0; i < NW; ++i) t += red[i];
  __syncthreads();
  return t;
}
template <int NW>
__device__ __forceinline__ float block_max_nan(float v, float* red) {
  v = wave_max_nan(v);
  const int w = threadIdx.x / kWave, l = threadIdx.x % kWave;
  if (l == 0) red[w] = v;
  __syncthreads();
  float t = red[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) t = max_nan(t, red[i]);
  __syncthreads();
  return t;
}

// Column C of an 8x8 block of 16-bit values held as 8 row vectors (row p = 8 values): the 8
// values of column C, one from each row, packed in row order.  Used to transpose 8x8 tiles in
// registers before a K-contiguous LDS store (v_perm / v_and_or per dword).
template <int C>
__device__ __forceinline__ u32x4 column8x8(const u32x4 (&r)[8]) {
  u32x4 o;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint32_t lo = r[2 * q][C / 2], hi = r[2 * q + 1][C / 2];
    o[q] = (C % 2 == 0) ? ((lo & 0xffffu) | (hi << 16)) : ((lo >> 16) | (hi & 0xffff0000u));
  }
  return o;
}

typedef int i32x4 __attribute__((ext_vector_type(4)));

// Buffer resource for raw byte-offset loads: reads at offsets >= bytes return 0.
__device__ __forceinline__ i32x4 make_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  i32x4 r;
  r[0] = int(uint32_t(a));
  r[1] = int(uint32_t(a >> 32) & 0xffffu);  // stride 0
  r[2] = int(bytes);                        // num_records
  r[3] = 0x00020000;                        // dword data format (gfx9 family)
  return r;
}

// 16 bytes per lane from global (buffer resource, byte offsets voff + soff) straight into LDS at
// lds_base + 16 * lane (buffer_load_dwordx4 ... lds, no VGPR staging); lds_base is wave-uniform.
// The compiler does not see the LDS write: callers order it with wait_vmcnt + a barrier.
__device__ __forceinline__ void dma16(i32x4 rsrc, uint32_t lds_base, uint32_t voff, uint32_t soff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :: "s"(lds_base), "v"(voff), "s"(rsrc), "s"(soff) : "memory", "m0");
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" :: "n"(N) : "memory");
}

__host__ __forceinline__ bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

__host__ __forceinline__ int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? PTB_OK : int(e);
}

}  // namespace ptb
