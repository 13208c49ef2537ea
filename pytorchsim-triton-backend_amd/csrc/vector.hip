// Vector-family kernels for gfx950: RMSNorm, row softmax, SiLU gate, head transposes, q/k-norm+RoPE,
// whole-tensor sum/max and add-scalar.  All are HBM-bound: each thread moves 128-bit chunks
// (8 bf16) with coalesced global_load_dwordx4 / global_store_dwordx4, math is fp32, and every
// output is rounded to bf16 exactly once, at the store.
#include "ptb_common.h"

using namespace ptb;

namespace {

constexpr int kBlock = 256;

__device__ __forceinline__ void unpack8(const u32x4& v, float* f) {
  f[0] = bf16_lo(v[0]); f[1] = bf16_hi(v[0]);
  f[2] = bf16_lo(v[1]); f[3] = bf16_hi(v[1]);
  f[4] = bf16_lo(v[2]); f[5] = bf16_hi(v[2]);
  f[6] = bf16_lo(v[3]); f[7] = bf16_hi(v[3]);
}
__device__ __forceinline__ u32x4 pack8(const float* f) {
  return u32x4{pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]),
               pack_bf16x2(f[6], f[7])};
}
// exp as the CDNA transcendental unit computes it: 2^(x * log2 e) (v_exp_f32).
__device__ __forceinline__ float exp_e(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }

// Team-wide reductions: a team is TPR consecutive threads of the block (64 = one wave, or the block).
template <int TPR>
__device__ __forceinline__ float team_sum(float v, float* red) {
  if constexpr (TPR == kWave) return wave_sum(v);
  else return block_sum<TPR / kWave>(v, red);
}
template <int TPR>
__device__ __forceinline__ float team_max(float v, float* red) {
  if constexpr (TPR == kWave) return wave_max_nan(v);
  else return block_max_nan<TPR / kWave>(v, red);
}

// ---------------------------------------------------------------- RMSNorm
// One team of TPR threads per row; each thread keeps VPT 8-element chunks of the row in registers,
// so x is read once and y written once.
template <int TPR, int VPT, bool WF32>
__global__ __launch_bounds__(kBlock) void rmsnorm_rows(const uint16_t* __restrict__ x,
                                                       const void* __restrict__ w,
                                                       uint16_t* __restrict__ y, int64_t rows,
                                                       int cols, float eps) {
  __shared__ float red[kBlock / kWave];
  constexpr int kTeams = kBlock / TPR;
  const int team = threadIdx.x / TPR, lt = threadIdx.x % TPR;
  const int64_t row = int64_t(blockIdx.x) * kTeams + team;
  const bool live = row < rows;
  const int chunks = cols >> 3;
  const u32x4* xr = reinterpret_cast<const u32x4*>(x + (live ? row : 0) * int64_t(cols));
  u32x4 v[VPT];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int c = lt + i * TPR;
    v[i] = (live && c < chunks) ? xr[c] : u32x4{0u, 0u, 0u, 0u};
    float f[8];
    unpack8(v[i], f);
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += f[e] * f[e];
  }
  ss = team_sum<TPR>(ss, red);
  const float r = 1.0f / sqrtf(ss / float(cols) + eps);
  if (!live) return;
  u32x4* yr = reinterpret_cast<u32x4*>(y + row * int64_t(cols));
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int c = lt + i * TPR;
    if (c >= chunks) continue;
    float f[8], wf[8];
    unpack8(v[i], f);
    if constexpr (WF32) {
      const f32x4v* wp = reinterpret_cast<const f32x4v*>(w) + 2 * c;
      const f32x4v a = wp[0], b = wp[1];
      wf[0] = a.x; wf[1] = a.y; wf[2] = a.z; wf[3] = a.w; wf[4] = b.x; wf[5] = b.y; wf[6] = b.z; wf[7] = b.w;
    } else {
      unpack8(reinterpret_cast<const u32x4*>(w)[c], wf);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = (f[e] * r) * wf[e];
    yr[c] = pack8(f);
  }
}

// Rows too long for registers: one block per row, two passes over global memory.
template <bool WF32>
__global__ __launch_bounds__(kBlock) void rmsnorm_rows_long(const uint16_t* __restrict__ x,
                                                            const void* __restrict__ w,
                                                            uint16_t* __restrict__ y, int cols, float eps) {
  __shared__ float red[kBlock / kWave];
  const int64_t row = blockIdx.x;
  const int chunks = cols >> 3;
  const u32x4* xr = reinterpret_cast<const u32x4*>(x + row * int64_t(cols));
  float ss = 0.f;
  for (int c = threadIdx.x; c < chunks; c += kBlock) {
    float f[8];
    unpack8(xr[c], f);
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += f[e] * f[e];
  }
  ss = block_sum<kBlock / kWave>(ss, red);
  const float r = 1.0f / sqrtf(ss / float(cols) + eps);
  u32x4* yr = reinterpret_cast<u32x4*>(y + row * int64_t(cols));
  for (int c = threadIdx.x; c < chunks; c += kBlock) {
    float f[8], wf[8];
    unpack8(xr[c], f);
    if constexpr (WF32) {
      const f32x4v* wp = reinterpret_cast<const f32x4v*>(w) + 2 * c;
      const f32x4v a = wp[0], b = wp[1];
      wf[0] = a.x; wf[1] = a.y; wf[2] = a.z; wf[3] = a.w; wf[4] = b.x; wf[5] = b.y; wf[6] = b.z; wf[7] = b.w;
    } else {
      unpack8(reinterpret_cast<const u32x4*>(w)[c], wf);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = (f[e] * r) * wf[e];
    yr[c] = pack8(f);
  }
}

// ---------------------------------------------------------------- softmax
// Eight results of chunk c of a row: one bf16 rounding each (OutT = uint16_t) or fp32 as computed.
template <typename OutT>
__device__ __forceinline__ void store8(OutT* __restrict__ yrow, int c, const float (&f)[8]) {
  if constexpr (sizeof(OutT) == 2) {
    reinterpret_cast<u32x4*>(yrow)[c] = pack8(f);
  } else {
    f32x4v* p = reinterpret_cast<f32x4v*>(yrow) + 2 * c;
    p[0] = f32x4v{f[0], f[1], f[2], f[3]};
    p[1] = f32x4v{f[4], f[5], f[6], f[7]};
  }
}

// f[e] / s for the 8 exponentials of a chunk, s a row's sum (s >= 1: the row's maximum contributes
// exp(0); NaN for a row holding a NaN) and r = 1/s correctly rounded.  q0 = f*r, then one fma
// correction of the quotient (Markstein), which rounds exactly as the IEEE quotient does while q0
// and the residual stay normal: every f >= 2^-64 (s <= 2^30, so q0 >= 2^-94).  A chunk holding a
// smaller f (exp of an argument below -44, zeros of -inf entries) takes the IEEE division.
__device__ __forceinline__ void div8_by_sum(float (&f)[8], float s, float r) {
  const float lo = fminf(fminf(fminf(f[0], f[1]), fminf(f[2], f[3])), fminf(fminf(f[4], f[5]), fminf(f[6], f[7])));
  if (__builtin_expect(lo < 0x1p-64f, 0)) {
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = f[e] / s;
    return;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float q0 = f[e] * r;
    f[e] = __builtin_fmaf(__builtin_fmaf(-s, q0, f[e]), r, q0);
  }
}

template <int TPR, int VPT, typename OutT>
__global__ __launch_bounds__(kBlock) void softmax_rows(const uint16_t* __restrict__ x,
                                                       OutT* __restrict__ y, int64_t rows, int cols) {
  __shared__ float red[kBlock / kWave];
  constexpr int kTeams = kBlock / TPR;
  const int team = threadIdx.x / TPR, lt = threadIdx.x % TPR;
  const int64_t row = int64_t(blockIdx.x) * kTeams + team;
  const bool live = row < rows;
  const int chunks = cols >> 3;
  const u32x4* xr = reinterpret_cast<const u32x4*>(x + (live ? row : 0) * int64_t(cols));
  u32x4 v[VPT];
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int c = lt + i * TPR;
    const bool in = live && c < chunks;
    v[i] = in ? xr[c] : u32x4{0u, 0u, 0u, 0u};
    if (in) {
      float f[8];
      unpack8(v[i], f);
      mx = max_nan(mx, max8_nan(f));
    }
  }
  mx = team_max<TPR>(mx, red);
  // the exponentials stay in registers between the sum and the stores
  float ex[VPT][8];
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int c = lt + i * TPR;
    unpack8(v[i], ex[i]);
#pragma unroll
    for (int e = 0; e < 8; ++e) ex[i][e] = exp_e(ex[i][e] - mx);
    if (live && c < chunks) {
#pragma unroll
      for (int e = 0; e < 8; ++e) s += ex[i][e];
    }
  }
  s = team_sum<TPR>(s, red);
  if (!live) return;
  const float r = 1.0f / s;
  OutT* yr = y + row * int64_t(cols);
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int c = lt + i * TPR;
    if (c >= chunks) continue;
    div8_by_sum(ex[i], s, r);
    store8(yr, c, ex[i]);
  }
}

template <typename OutT>
__global__ __launch_bounds__(kBlock) void softmax_rows_long(const uint16_t* __restrict__ x,
                                                            OutT* __restrict__ y, int cols) {
  __shared__ float red[kBlock / kWave];
  const int64_t row = blockIdx.x;
  const int chunks = cols >> 3;
  const u32x4* xr = reinterpret_cast<const u32x4*>(x + row * int64_t(cols));
  float mx = -INFINITY;
  for (int c = threadIdx.x; c < chunks; c += kBlock) {
    float f[8];
    unpack8(xr[c], f);
    mx = max_nan(mx, max8_nan(f));
  }
  mx = block_max_nan<kBlock / kWave>(mx, red);
  float s = 0.f;
  for (int c = threadIdx.x; c < chunks; c += kBlock) {
    float f[8];
    unpack8(xr[c], f);
#pragma unroll
    for (int e = 0; e < 8; ++e) s += exp_e(f[e] - mx);
  }
  s = block_sum<kBlock / kWave>(s, red);
  const float r = 1.0f / s;
  OutT* yr = y + row * int64_t(cols);
  for (int c = threadIdx.x; c < chunks; c += kBlock) {
    float f[8];
    unpack8(xr[c], f);
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = exp_e(f[e] - mx);
    div8_by_sum(f, s, r);
    store8(yr, c, f);
  }
}

// ---------------------------------------------------------------- SiLU gate
// Each thread handles kPer 8-element chunks of the output, strided by the grid for coalescing.
constexpr int kPer = 4;
__global__ __launch_bounds__(kBlock) void silu_mul(const uint16_t* __restrict__ gu, uint16_t* __restrict__ out,
                                                   int64_t total_chunks, int64_t inter_chunks) {
  const int64_t stride = int64_t(gridDim.x) * kBlock;
  int64_t idx = int64_t(blockIdx.x) * kBlock + threadIdx.x;
  u32x4 g[kPer], u[kPer];
  int64_t id[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    id[i] = idx + i * stride;
    if (id[i] < total_chunks) {
      // 32-bit division where the chunk count allows (a 64-bit one is a long instruction sequence)
      const int64_t r = total_chunks <= 0xffffffffll ? int64_t(uint32_t(id[i]) / uint32_t(inter_chunks))
                                                     : id[i] / inter_chunks;
      const int64_t c = id[i] - r * inter_chunks;
      const u32x4* src = reinterpret_cast<const u32x4*>(gu) + r * 2 * inter_chunks;
      g[i] = src[c];
      u[i] = src[inter_chunks + c];
    }
  }
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    if (id[i] >= total_chunks) continue;
    float fg[8], fu[8];
    unpack8(g[i], fg);
    unpack8(u[i], fu);
    float b[8], q[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      b[e] = exp_e(-fg[e]) + 1.0f;
      q[e] = silu_quotient(fg[e], b[e]);
    }
    // the IEEE division where a denominator reaches 2^126 (fmaxf skips a NaN b, whose quotient the
    // fixup already made NaN)
    const float bmax = fmaxf(fmaxf(fmaxf(b[0], b[1]), fmaxf(b[2], b[3])), fmaxf(fmaxf(b[4], b[5]), fmaxf(b[6], b[7])));
    if (__builtin_expect(bmax >= 0x1p126f, 0)) {
#pragma unroll
      for (int e = 0; e < 8; ++e) q[e] = fg[e] / b[e];
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) fg[e] = q[e] * fu[e];
    reinterpret_cast<u32x4*>(out)[id[i]] = pack8(fg);
  }
}

// ---------------------------------------------------------------- head transpose
__global__ __launch_bounds__(kBlock) void transpose_heads(const u32x4* __restrict__ x, u32x4* __restrict__ y,
                                                          int64_t d0, int64_t d1, int64_t ic, int64_t xa,
                                                          int64_t total) {
  const int64_t stride = int64_t(gridDim.x) * kBlock;
  int64_t idx = int64_t(blockIdx.x) * kBlock + threadIdx.x;
  u32x4 v[kPer];
  int64_t id[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    id[i] = idx + i * stride;
    if (id[i] < total) {
      // output chunk id -> (b, a, c) of y[d1, d0, ic]; source x[a, b, c], xa chunks between a rows
      const int64_t c = id[i] % ic, ba = id[i] / ic;
      const int64_t a = ba % d0, b = ba / d0;
      v[i] = x[a * xa + b * ic + c];
    }
  }
#pragma unroll
  for (int i = 0; i < kPer; ++i)
    if (id[i] < total) y[id[i]] = v[i];
}

// ---------------------------------------------------------------- q/k norm + RoPE + head transpose
// head_dim 128: 16 threads per (token, head) row, 8 elements each; the rotate-half partner of
// element r (r +- 64) lives 8 lanes away.
__global__ __launch_bounds__(kBlock) void qk_norm_rope(const uint16_t* __restrict__ x,
                                                       const uint16_t* __restrict__ w,
                                                       const float* __restrict__ cos_t,
                                                       const float* __restrict__ sin_t,
                                                       uint16_t* __restrict__ out, int64_t tokens,
                                                       int heads, int64_t ld, float eps) {
  constexpr int D = 128;
  const int64_t row = int64_t(blockIdx.x) * (kBlock / 16) + threadIdx.x / 16;  // = t * heads + h
  const int c = threadIdx.x % 16;
  const bool live = row < tokens * heads;
  const int64_t rr = live ? row : 0;
  const int64_t t = rr / heads, h = rr - t * heads;   // token t's heads start ld elements apart
  const u32x4 v = reinterpret_cast<const u32x4*>(x + t * ld + h * D)[c];
  float f[8];
  unpack8(v, f);
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss = fmaf(f[e], f[e], ss);
  ss = row16_sum(ss);
  u32x4 pv;
#pragma unroll
  for (int q = 0; q < 4; ++q) pv[q] = xor8_u32(v[q]);
  if (!live) return;
  float pf[8], wf[8], pw[8];
  unpack8(pv, pf);
  const int pc = c ^ 8;
  unpack8(reinterpret_cast<const u32x4*>(w)[c], wf);
  unpack8(reinterpret_cast<const u32x4*>(w)[pc], pw);
  const float r = 1.0f / sqrtf(ss / float(D) + eps);
  const f32x4v* cp = reinterpret_cast<const f32x4v*>(cos_t + t * D + c * 8);
  const f32x4v* sp = reinterpret_cast<const f32x4v*>(sin_t + t * D + c * 8);
  const f32x4v c0 = cp[0], c1 = cp[1], s0 = sp[0], s1 = sp[1];
  const float cs[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
  const float sn[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
  const bool first_half = c < 8;
  float o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float a = (f[e] * r) * wf[e];
    const float p = (pf[e] * r) * pw[e];
    const float rot = first_half ? -p : p;
    o[e] = fmaf(a, cs[e], rot * sn[e]);   // explicit fma: the fused decode-attention prologue matches
  }
  reinterpret_cast<u32x4*>(out + (h * tokens + t) * D)[c] = pack8(o);
}

// ---------------------------------------------------------------- whole-tensor sum / max
constexpr int kReduceBlocks = 1024;
// Eight consecutive elements (chunk c) as fp32: one 16-byte load of bf16, two of fp32.
__device__ __forceinline__ void load8(const uint16_t* __restrict__ x, int64_t c, float (&f)[8]) {
  unpack8(reinterpret_cast<const u32x4*>(x)[c], f);
}
__device__ __forceinline__ void load8(const float* __restrict__ x, int64_t c, float (&f)[8]) {
  const f32x4v* p = reinterpret_cast<const f32x4v*>(x) + 2 * c;
  const f32x4v a = p[0], b = p[1];
  f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w; f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
}
__device__ __forceinline__ float as_f32(uint16_t v) { return bf16_to_f32(v); }
__device__ __forceinline__ float as_f32(float v) { return v; }

template <int OP, typename InT>
__global__ __launch_bounds__(kBlock) void reduce_partial(const InT* __restrict__ x, int64_t n,
                                                         float* __restrict__ part) {
  __shared__ float red[kBlock / kWave];
  const int64_t chunks = n >> 3;
  const int64_t stride = int64_t(gridDim.x) * kBlock;
  float acc = OP == PTB_REDUCE_SUM ? 0.f : -INFINITY;
  for (int64_t c = int64_t(blockIdx.x) * kBlock + threadIdx.x; c < chunks; c += stride) {
    float f[8];
    load8(x, c, f);
    if constexpr (OP == PTB_REDUCE_SUM) {
#pragma unroll
      for (int e = 0; e < 8; ++e) acc += f[e];
    } else {
      acc = max_nan(acc, max8_nan(f));
    }
  }
  if (blockIdx.x == 0) {
    for (int64_t i = (chunks << 3) + threadIdx.x; i < n; i += kBlock) {
      const float f = as_f32(x[i]);
      acc = OP == PTB_REDUCE_SUM ? acc + f : max_nan(acc, f);
    }
  }
  acc = OP == PTB_REDUCE_SUM ? block_sum<kBlock / kWave>(acc, red) : block_max_nan<kBlock / kWave>(acc, red);
  if (threadIdx.x == 0) part[blockIdx.x] = acc;
}
// Inputs of at most kSmallReduce elements: one workgroup (64..1024 threads, a thread per 8 chunks
// of 8 elements) and one launch.  Each thread issues all its loads of a batch before it
// accumulates (slots past the end load the last chunk again and are skipped), so a batch costs
// one memory round trip.
constexpr int kSmallThreads = 1024;
constexpr int kSmallLoads = 8;
// measured (HIP-graph replay, bf16): one workgroup 3.2 us at 65536 elements and 4.1-4.2 at 98304
// against 4.3 for the two launches; beyond, one CU's loads and VALU work outgrow the second launch
constexpr int64_t kSmallReduce = 98304;
template <int OP, typename InT>
__global__ __launch_bounds__(kSmallThreads) void reduce_small(const InT* __restrict__ x, int64_t n,
                                                               float* __restrict__ out) {
  __shared__ float red[kSmallThreads / kWave];
  const int chunks = int(n >> 3), nt = int(blockDim.x), tid = int(threadIdx.x);
  float acc = OP == PTB_REDUCE_SUM ? 0.f : -INFINITY;
  for (int base = 0; base < chunks; base += nt * kSmallLoads) {
    float f[kSmallLoads][8];
#pragma unroll
    for (int i = 0; i < kSmallLoads; ++i) load8(x, min(base + i * nt + tid, chunks - 1), f[i]);
#pragma unroll
    for (int i = 0; i < kSmallLoads; ++i) {
      if (base + i * nt + tid < chunks) {
        if constexpr (OP == PTB_REDUCE_SUM) {
#pragma unroll
          for (int e = 0; e < 8; ++e) acc += f[i][e];
        } else {
          acc = max_nan(acc, max8_nan(f[i]));
        }
      }
    }
  }
  for (int64_t i = (int64_t(chunks) << 3) + tid; i < n; i += nt) {
    const float v = as_f32(x[i]);
    acc = OP == PTB_REDUCE_SUM ? acc + v : max_nan(acc, v);
  }
  acc = OP == PTB_REDUCE_SUM ? wave_sum(acc) : wave_max_nan(acc);
  if ((tid & 63) == 0) red[tid >> 6] = acc;
  __syncthreads();
  if (tid == 0) {
    float t = red[0];
    for (int w = 1; w < nt / kWave; ++w) t = OP == PTB_REDUCE_SUM ? t + red[w] : max_nan(t, red[w]);
    out[0] = t;
  }
}

template <int OP>
__global__ __launch_bounds__(kBlock) void reduce_final(const float* __restrict__ part, int np,
                                                       float* __restrict__ out) {
  __shared__ float red[kBlock / kWave];
  float acc = OP == PTB_REDUCE_SUM ? 0.f : -INFINITY;
  for (int i = threadIdx.x; i < np; i += kBlock) acc = OP == PTB_REDUCE_SUM ? acc + part[i] : max_nan(acc, part[i]);
  acc = OP == PTB_REDUCE_SUM ? block_sum<kBlock / kWave>(acc, red) : block_max_nan<kBlock / kWave>(acc, red);
  if (threadIdx.x == 0) out[0] = acc;
}

// ---------------------------------------------------------------- add scalar
__global__ __launch_bounds__(kBlock) void add_scalar(const uint16_t* __restrict__ x, uint16_t* __restrict__ y,
                                                     int64_t n, float s) {
  const int64_t chunks = n >> 3;
  const int64_t stride = int64_t(gridDim.x) * kBlock;
  for (int64_t c = int64_t(blockIdx.x) * kBlock + threadIdx.x; c < chunks; c += stride) {
    float f[8];
    unpack8(reinterpret_cast<const u32x4*>(x)[c], f);
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = f[e] + s;
    reinterpret_cast<u32x4*>(y)[c] = pack8(f);
  }
  if (blockIdx.x == 0)
    for (int64_t i = (chunks << 3) + threadIdx.x; i < n; i += kBlock) y[i] = f32_to_bf16(bf16_to_f32(x[i]) + s);
}

// out[i] = float(x[first + i]) + s into fp32, for a short run of elements.
__global__ __launch_bounds__(kBlock) void slice_add(const uint16_t* __restrict__ x, float* __restrict__ out,
                                                    int64_t count, float s) {
  for (int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x; i < count; i += int64_t(gridDim.x) * kBlock)
    out[i] = bf16_to_f32(x[i]) + s;
}

int grid_for(int64_t work, int64_t per_block, int64_t cap) {
  int64_t g = (work + per_block - 1) / per_block;
  if (g < 1) g = 1;
  return int(g > cap ? cap : g);
}

// Row-kernel dispatch shared by RMSNorm and softmax: returns the team size and chunks per thread.
bool row_shape(int cols, int* tpr, int* vpt) {
  const int chunks = cols / 8;
  if (chunks <= 64 * 4) {
    *tpr = 64;
    *vpt = chunks <= 64 ? 1 : (chunks <= 128 ? 2 : 4);
    return true;
  }
  if (chunks <= 256 * 8) {
    *tpr = 256;
    *vpt = chunks <= 512 ? 2 : (chunks <= 1024 ? 4 : 8);
    return true;
  }
  return false;
}

}  // namespace

PTB_EXPORT int ptb_rmsnorm_bf16(const void* x, const void* w, int w_dtype, void* y, int64_t rows,
                                int64_t cols, float eps, void* stream) {
  if (rows < 0 || cols <= 0 || cols > (int64_t(1) << 30)) return PTB_ERR_SHAPE;
  if (w_dtype != PTB_DTYPE_BF16 && w_dtype != PTB_DTYPE_F32) return PTB_ERR_DTYPE;
  if (rows == 0) return PTB_OK;
  if (!x || !w || !y) return PTB_ERR_NULL;
  if (cols % 8 || !aligned16(x) || !aligned16(y) || !aligned16(w)) return PTB_ERR_ALIGN;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int c = int(cols);
  int tpr, vpt;
  const bool wf = w_dtype == PTB_DTYPE_F32;
  if (row_shape(c, &tpr, &vpt)) {
    const int teams = kBlock / tpr;
    const int64_t blocks = (rows + teams - 1) / teams;
    if (blocks > 0x7fffffff) return PTB_ERR_GRID;
    const uint16_t* xi = static_cast<const uint16_t*>(x);
    uint16_t* yo = static_cast<uint16_t*>(y);
#define RMS_CASE(T, V)                                                                              \
  if (tpr == T && vpt == V) {                                                                       \
    if (wf) rmsnorm_rows<T, V, true><<<dim3(unsigned(blocks)), dim3(kBlock), 0, s>>>(xi, w, yo, rows, c, eps); \
    else rmsnorm_rows<T, V, false><<<dim3(unsigned(blocks)), dim3(kBlock), 0, s>>>(xi, w, yo, rows, c, eps); \
    return launch_status();                                                                         \
  }
    RMS_CASE(64, 1) RMS_CASE(64, 2) RMS_CASE(64, 4) RMS_CASE(256, 2) RMS_CASE(256, 4) RMS_CASE(256, 8)
#undef RMS_CASE
  }
  if (rows > 0x7fffffff) return PTB_ERR_GRID;
  if (wf) rmsnorm_rows_long<true><<<dim3(unsigned(rows)), dim3(kBlock), 0, s>>>(static_cast<const uint16_t*>(x), w, static_cast<uint16_t*>(y), c, eps);
  else rmsnorm_rows_long<false><<<dim3(unsigned(rows)), dim3(kBlock), 0, s>>>(static_cast<const uint16_t*>(x), w, static_cast<uint16_t*>(y), c, eps);
  return launch_status();
}

namespace {

template <typename OutT>
int softmax_launch(const void* x, void* y, int64_t rows, int64_t cols, void* stream) {
  if (rows < 0 || cols <= 0 || cols > (int64_t(1) << 30)) return PTB_ERR_SHAPE;
  if (rows == 0) return PTB_OK;
  if (!x || !y) return PTB_ERR_NULL;
  if (cols % 8 || !aligned16(x) || !aligned16(y)) return PTB_ERR_ALIGN;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int c = int(cols);
  const uint16_t* xi = static_cast<const uint16_t*>(x);
  OutT* yo = static_cast<OutT*>(y);
  int tpr, vpt;
  if (row_shape(c, &tpr, &vpt)) {
    // at most one workgroup per CU's worth of rows: a 256-thread team per row, so each lane holds
    // as few chunks as it can (the row's latency, not the throughput, sets the time)
    const int chunks = c / 8;
    if (rows <= 256 && chunks > 64) {
      tpr = 256;
      vpt = chunks <= 256 ? 1 : chunks <= 512 ? 2 : chunks <= 1024 ? 4 : 8;
    }
    const int teams = kBlock / tpr;
    const int64_t blocks = (rows + teams - 1) / teams;
    if (blocks > 0x7fffffff) return PTB_ERR_GRID;
#define SM_CASE(T, V)                                                                                 \
  if (tpr == T && vpt == V) {                                                                         \
    softmax_rows<T, V, OutT><<<dim3(unsigned(blocks)), dim3(kBlock), 0, s>>>(xi, yo, rows, c);      \
    return launch_status();                                                                           \
  }
    SM_CASE(64, 1) SM_CASE(64, 2) SM_CASE(64, 4) SM_CASE(256, 1) SM_CASE(256, 2) SM_CASE(256, 4) SM_CASE(256, 8)
#undef SM_CASE
  }
  if (rows > 0x7fffffff) return PTB_ERR_GRID;
  softmax_rows_long<OutT><<<dim3(unsigned(rows)), dim3(kBlock), 0, s>>>(xi, yo, c);
  return launch_status();
}

}  // namespace

PTB_EXPORT int ptb_softmax_rows_bf16(const void* x, void* y, int64_t rows, int64_t cols, void* stream) {
  return softmax_launch<uint16_t>(x, y, rows, cols, stream);
}

PTB_EXPORT int ptb_softmax_rows_bf16_f32(const void* x, void* y, int64_t rows, int64_t cols, void* stream) {
  return softmax_launch<float>(x, y, rows, cols, stream);
}

PTB_EXPORT int ptb_silu_mul_bf16(const void* gate_up, void* out, int64_t rows, int64_t inter, void* stream) {
  if (rows < 0 || inter <= 0) return PTB_ERR_SHAPE;
  if (rows == 0) return PTB_OK;
  if (!gate_up || !out) return PTB_ERR_NULL;
  if (inter % 8 || !aligned16(gate_up) || !aligned16(out)) return PTB_ERR_ALIGN;
  const int64_t total = rows * (inter / 8);
  const int g = grid_for(total, int64_t(kBlock) * kPer, 1 << 20);
  silu_mul<<<dim3(g), dim3(kBlock), 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t*>(gate_up), static_cast<uint16_t*>(out), total, inter / 8);
  return launch_status();
}

PTB_EXPORT int ptb_transpose_heads_ld_bf16(const void* x, int64_t ld, void* y, int64_t d0, int64_t d1,
                                           int64_t inner, void* stream) {
  if (d0 < 0 || d1 < 0 || inner <= 0) return PTB_ERR_SHAPE;
  if (d0 == 0 || d1 == 0) return PTB_OK;
  if (ld < d1 * inner) return PTB_ERR_SHAPE;
  if (!x || !y) return PTB_ERR_NULL;
  if (inner % 8 || ld % 8 || !aligned16(x) || !aligned16(y)) return PTB_ERR_ALIGN;
  const int64_t total = d0 * d1 * (inner / 8);
  const int g = grid_for(total, int64_t(kBlock) * kPer, 1 << 20);
  transpose_heads<<<dim3(g), dim3(kBlock), 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const u32x4*>(x), static_cast<u32x4*>(y), d0, d1, inner / 8, ld / 8, total);
  return launch_status();
}

PTB_EXPORT int ptb_transpose_heads_bf16(const void* x, void* y, int64_t d0, int64_t d1, int64_t inner,
                                        void* stream) {
  if (d0 < 0 || d1 < 0 || inner <= 0) return PTB_ERR_SHAPE;
  return ptb_transpose_heads_ld_bf16(x, d1 * inner, y, d0, d1, inner, stream);
}

PTB_EXPORT int ptb_qk_norm_rope_ld_bf16(const void* x, int64_t ld, const void* w, const float* cos_t,
                                        const float* sin_t, void* out, int64_t tokens, int64_t heads,
                                        int64_t head_dim, float eps, void* stream) {
  if (tokens < 0 || heads <= 0 || head_dim <= 0) return PTB_ERR_SHAPE;
  if (ld < heads * head_dim) return PTB_ERR_SHAPE;
  if (ld % 8) return PTB_ERR_ALIGN;
  if (head_dim != 128) return PTB_ERR_UNSUPPORTED;
  if (tokens == 0) return PTB_OK;
  if (!x || !w || !cos_t || !sin_t || !out) return PTB_ERR_NULL;
  if (!aligned16(x) || !aligned16(w) || !aligned16(cos_t) || !aligned16(sin_t) || !aligned16(out))
    return PTB_ERR_ALIGN;
  const int64_t rows = tokens * heads;
  if (rows == 0) return PTB_OK;
  const int64_t blocks = (rows + 15) / 16;
  if (blocks > 0x7fffffff || heads > 0x7fffffff) return PTB_ERR_GRID;
  qk_norm_rope<<<dim3(unsigned(blocks)), dim3(kBlock), 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w), cos_t, sin_t,
      static_cast<uint16_t*>(out), tokens, int(heads), ld, eps);
  return launch_status();
}

PTB_EXPORT int ptb_qk_norm_rope_bf16(const void* x, const void* w, const float* cos_t, const float* sin_t,
                                     void* out, int64_t tokens, int64_t heads, int64_t head_dim, float eps,
                                     void* stream) {
  if (tokens < 0 || heads <= 0 || head_dim <= 0) return PTB_ERR_SHAPE;
  return ptb_qk_norm_rope_ld_bf16(x, heads * head_dim, w, cos_t, sin_t, out, tokens, heads, head_dim, eps, stream);
}

PTB_EXPORT size_t ptb_reduce_workspace_bytes(int64_t n) {
  (void)n;
  return kReduceBlocks * sizeof(float);
}

namespace {

template <typename InT>
int reduce_launch(const InT* x, float* out, int64_t n, int op, void* workspace, size_t workspace_bytes,
                  void* stream) {
  if (!x || !out || !workspace) return PTB_ERR_NULL;
  if (n < 0) return PTB_ERR_SHAPE;
  if (op != PTB_REDUCE_SUM && op != PTB_REDUCE_MAX) return PTB_ERR_DTYPE;
  if (!aligned16(x) || !aligned16(workspace)) return PTB_ERR_ALIGN;
  if (workspace_bytes < ptb_reduce_workspace_bytes(n)) return PTB_ERR_WORKSPACE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (n <= kSmallReduce) {
    const int64_t per = (n / 8 + kSmallLoads - 1) / kSmallLoads;        // threads for one batch
    const int nt = int(per <= kWave ? kWave : per >= kSmallThreads ? kSmallThreads : (per + kWave - 1) / kWave * kWave);
    if (op == PTB_REDUCE_SUM)
      reduce_small<PTB_REDUCE_SUM, InT><<<dim3(1), dim3(nt), 0, s>>>(x, n, out);
    else
      reduce_small<PTB_REDUCE_MAX, InT><<<dim3(1), dim3(nt), 0, s>>>(x, n, out);
    return launch_status();
  }
  const int g = grid_for(n / 8, int64_t(kBlock) * 8, kReduceBlocks);
  float* part = static_cast<float*>(workspace);
  if (op == PTB_REDUCE_SUM) {
    reduce_partial<PTB_REDUCE_SUM, InT><<<dim3(g), dim3(kBlock), 0, s>>>(x, n, part);
    reduce_final<PTB_REDUCE_SUM><<<dim3(1), dim3(kBlock), 0, s>>>(part, g, out);
  } else {
    reduce_partial<PTB_REDUCE_MAX, InT><<<dim3(g), dim3(kBlock), 0, s>>>(x, n, part);
    reduce_final<PTB_REDUCE_MAX><<<dim3(1), dim3(kBlock), 0, s>>>(part, g, out);
  }
  return launch_status();
}

}  // namespace

PTB_EXPORT int ptb_reduce_bf16(const void* x, float* out, int64_t n, int op, void* workspace,
                               size_t workspace_bytes, void* stream) {
  return reduce_launch(static_cast<const uint16_t*>(x), out, n, op, workspace, workspace_bytes, stream);
}

PTB_EXPORT int ptb_reduce_f32(const float* x, float* out, int64_t n, int op, void* workspace,
                              size_t workspace_bytes, void* stream) {
  return reduce_launch(x, out, n, op, workspace, workspace_bytes, stream);
}

PTB_EXPORT int ptb_add_scalar_bf16(const void* x, void* y, int64_t n, float s, void* stream) {
  if (n < 0) return PTB_ERR_SHAPE;
  if (n == 0) return PTB_OK;
  if (!x || !y) return PTB_ERR_NULL;
  if (!aligned16(x) || !aligned16(y)) return PTB_ERR_ALIGN;
  const int g = grid_for(n / 8 + 1, int64_t(kBlock) * 4, 1 << 20);
  add_scalar<<<dim3(g), dim3(kBlock), 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t*>(x), static_cast<uint16_t*>(y), n, s);
  return launch_status();
}

PTB_EXPORT int ptb_slice_add_bf16(const void* x, float* out, int64_t first, int64_t count, float s, void* stream) {
  if (first < 0 || count < 0) return PTB_ERR_SHAPE;
  if (count == 0) return PTB_OK;
  if (!x || !out) return PTB_ERR_NULL;
  const int g = grid_for(count, kBlock, 1 << 16);
  slice_add<<<dim3(g), dim3(kBlock), 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t*>(x) + first, out, count, s);
  return launch_status();
}
