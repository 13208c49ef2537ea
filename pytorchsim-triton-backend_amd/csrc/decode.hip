// Single-token (decode) kernels on gfx950: sum of squares, matrix-vector products with the decode
// layer's fused prologues / epilogue, and flash-decoding attention over a KV cache.  All of them
// stream their big operand (the weight matrix, the K/V cache) from HBM once and are bound by HBM
// bandwidth, so they are built for bytes in flight; decode attention over more than 256 keys puts
// its dot products on the matrix cores only to keep the VALU work after each load short.
//
// GEMV, y[n] = sum_k xp[k] * W[k, n] with W row-major [K, N] (N contiguous), split over K:
//   pass 1: workgroup (column block of 512, K slice of `kb` rows); the slice's xp[k] (the fused
//           prologue: plain x, RMSNorm-scaled x or x+a, or silu(g)*u) goes to LDS first, then each
//           wave walks every fourth row, each lane owning 8 consecutive columns (one 16-byte load
//           per row, a wave covers 1 KB of the row), eight rows in flight; the four waves' sums
//           meet in LDS and the slice's fp32 partials go to the workspace [splits, N].
//   pass 2: y[n] = bf16(sum over splits (+ r1[n] + r2[n])), one rounding.
// Decode attention (one query token, G query heads per kv head, S cached keys, D = 128):
//   pass 1, more than 256 keys: one wave per (key range, kv head), 32-key steps through LDS, scores
//           and P.V on v_mfma_f32_16x16x32_bf16 with the head's G query rows as the N side (K and V
//           read once); an (acc, m, l) record per range (attn_decode_mfma below).
//   up to 256 keys, one pass: a workgroup per query row, teams of 256 threads each taking one 64-key
//           chunk (scores with 16 lanes per key, one 256-byte row, summed by DPP row moves; a
//           base-2 softmax over the chunk), met in LDS; the workgroup writes o itself.
//   pass 2 (more than one range): workgroup (kv head, query head): o = sum acc_r 2^(m_r-M) / sum l_r 2^(m_r-M), M = max m_r.
#include <algorithm>
#include <cmath>

#include <mutex>
#include <type_traits>

#include "ptb_common.h"

using namespace ptb;

namespace {

// ---------------------------------------------------------------------------------------------
// sum of squares

__global__ __launch_bounds__(1024) void sumsq_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ y,
                                                     float* __restrict__ out, int64_t n) {
  __shared__ float red[16];
  float s = 0.f;
  const int64_t n8 = n / 8;
  for (int64_t i = threadIdx.x; i < n8; i += blockDim.x) {
    const u32x4 a = reinterpret_cast<const u32x4*>(x)[i];
    u32x4 b = {0u, 0u, 0u, 0u};
    if (y) b = reinterpret_cast<const u32x4*>(y)[i];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float lo = bf16_lo(a[c]) + bf16_lo(b[c]);
      const float hi = bf16_hi(a[c]) + bf16_hi(b[c]);
      s = __builtin_fmaf(lo, lo, s);
      s = __builtin_fmaf(hi, hi, s);
    }
  }
  for (int64_t i = n8 * 8 + threadIdx.x; i < n; i += blockDim.x) {
    const float v = bf16_to_f32(x[i]) + (y ? bf16_to_f32(y[i]) : 0.f);
    s = __builtin_fmaf(v, v, s);
  }
  s = block_sum<16>(s, red);
  if (threadIdx.x == 0) out[0] = s;
}

// ---------------------------------------------------------------------------------------------
// GEMV

// kSiluParts: kSilu whose gate_up vector is still the fp32 partials [splits, 2K] of the GEMV that
// produces it (that GEMV's finish pass is done in this prologue, in the finish's own order and
// rounding, so the result is bit-identical to finishing it first).
enum GemvMode { kPlain = 0, kRms = 1, kSilu = 2, kSiluParts = 3 };

constexpr int kColBlock = 512;   // columns per workgroup: 64 lanes x 8
constexpr int kMaxKb = 512;      // rows per K slice (LDS prologue buffer)
constexpr int kGemvThreads = 256;

struct GemvSplit {
  int splits, kb;
};

__host__ __device__ inline GemvSplit gemv_split(int64_t k, int64_t n) {
  const int64_t cb = (n + kColBlock - 1) / kColBlock;
  int64_t splits = (1024 + cb - 1) / cb;                    // about four workgroups per CU
  splits = splits < 1 ? 1 : splits;
  const int64_t max_splits = (k + 31) / 32;                 // at least 32 rows a slice
  if (splits > max_splits) splits = max_splits;
  int64_t kb = (k + splits - 1) / splits;
  kb = (kb + 31) / 32 * 32;
  if (kb > kMaxKb) kb = kMaxKb;
  if (kb < 32) kb = 32;
  return GemvSplit{int((k + kb - 1) / kb), int(kb)};
}

// xp[k] for the fused prologues (reference decode layer, validation/pytorchsim/
// qwen3_8b_layer_decode_1x<S>_bf16): kPlain x[k] (04_..._vumxrjnr); kRms ((x[k] (+ add[k])) * r) * g[k]
// with r = 1/sqrt(ss/K + eps), all fp32 (01_..._ddfn4f75, 06_..._5gopcdje); kSilu silu(x[k]) * x[K+k]
// (07_..._3d4ocw7y).
template <int MODE>
__device__ __forceinline__ float prologue(const uint16_t* x, const uint16_t* add, const uint16_t* g, float r,
                                          int64_t k, int64_t K) {
  if constexpr (MODE == kPlain) {
    return bf16_to_f32(x[k]);
  } else if constexpr (MODE == kRms) {
    float v = bf16_to_f32(x[k]);
    if (add) v += bf16_to_f32(add[k]);
    return (v * r) * bf16_to_f32(g[k]);
  } else {
    const float gv = bf16_to_f32(x[k]);
    const float u = bf16_to_f32(x[K + k]);
    return (gv / (__builtin_amdgcn_exp2f(-gv * 1.4426950408889634f) + 1.f)) * u;
  }
}

// 16 bytes of a weight row.  A GEMV reads each weight once per call: with the non-temporal
// (streaming) cache policy the 4096x24576 RMSNorm-prologue GEMV measured 34.9 us against 38.3 us.
__device__ __forceinline__ u32x4 ld_stream(const uint16_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

// bf16(sum of part[.][n]) exactly as gemv_finish forms it (no residual): split group sg (the splits
// sp = sg mod 16) summed from 0 in split order, then the 16 groups in order from 0, one rounding.
// Sixteen loads are in flight a round.
__device__ __forceinline__ float finish_value(const float* __restrict__ part, int splits, int N, int n) {
  float acc[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) acc[j] = 0.f;
  for (int sp0 = 0; sp0 < splits; sp0 += 16) {
    float v[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) v[j] = part[int64_t(min(sp0 + j, splits - 1)) * N + n];
#pragma unroll
    for (int j = 0; j < 16; ++j)
      if (sp0 + j < splits) acc[j] += v[j];
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 16; ++j) s += acc[j];
  return bf16_to_f32(f32_to_bf16(s));
}

template <int MODE>
__global__ __launch_bounds__(kGemvThreads) void gemv_partial(const uint16_t* __restrict__ x,
                                                             const uint16_t* __restrict__ add,
                                                             const float* __restrict__ ss,
                                                             const uint16_t* __restrict__ g, float eps,
                                                             const uint16_t* __restrict__ W,
                                                             float* __restrict__ part, int K, int N, int kb,
                                                             const float* __restrict__ xparts, int xsplits) {
  __shared__ float xs[kMaxKb];
  __shared__ float red[4][kColBlock];
  __shared__ float xu[MODE == kSiluParts ? kMaxKb : 1];   // the up half, kSiluParts
  const int n0 = blockIdx.x * kColBlock;
  const int split = blockIdx.y;
  const int k0 = split * kb;
  const int rows = min(K - k0, kb);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = n0 + 8 * lane;
  const uint16_t* wp = W + int64_t(k0) * N + col;
  // the first eight rows' weights go out before the prologue, whose loads and reduction they overlap
  u32x4 v[8];
  if (col < N && wave + 28 < rows) {
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = ld_stream(wp + int64_t(wave + 4 * u) * N);
  }
  float r = 0.f;
  if constexpr (MODE == kRms) {
    float sv;
    if (ss) {
      sv = ss[0];
    } else {   // no sum of squares given: every workgroup forms sum (x + add)^2 over K itself (from L2)
      float t = 0.f;
      const int k8 = K / 8;
      for (int i = threadIdx.x; i < k8; i += kGemvThreads) {
        const u32x4 a = reinterpret_cast<const u32x4*>(x)[i];
        const u32x4 b = add ? reinterpret_cast<const u32x4*>(add)[i] : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const float lo = bf16_lo(a[c]) + bf16_lo(b[c]), hi = bf16_hi(a[c]) + bf16_hi(b[c]);
          t = __builtin_fmaf(lo, lo, t);
          t = __builtin_fmaf(hi, hi, t);
        }
      }
      for (int i = k8 * 8 + threadIdx.x; i < K; i += kGemvThreads) {
        const float v = bf16_to_f32(x[i]) + (add ? bf16_to_f32(add[i]) : 0.f);
        t = __builtin_fmaf(v, v, t);
      }
      sv = block_sum<kGemvThreads / kWave>(t, &red[0][0]);
    }
    r = 1.f / sqrtf(sv / float(K) + eps);
  }
  if constexpr (MODE == kSiluParts) {
    // gate (t < rows) and up (t >= rows) values of the slice, each finished from the partials
    for (int t = threadIdx.x; t < 2 * rows; t += kGemvThreads) {
      const bool up = t >= rows;
      const float v = finish_value(xparts, xsplits, 2 * K, up ? K + k0 + (t - rows) : k0 + t);
      if (up) xu[t - rows] = v;
      else xs[t] = v;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < rows; i += kGemvThreads) {
      const float gv = xs[i], u = xu[i];
      xs[i] = (gv / (__builtin_amdgcn_exp2f(-gv * 1.4426950408889634f) + 1.f)) * u;
    }
  } else {
    for (int i = threadIdx.x; i < rows; i += kGemvThreads) xs[i] = prologue<MODE>(x, add, g, r, k0 + i, K);
  }
  __syncthreads();

  float acc[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) acc[c] = 0.f;
  if (col < N) {
    int i = wave;
    for (; i + 28 < rows; i += 32) {
      if (i != wave) {   // the first eight rows are already loaded
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = ld_stream(wp + int64_t(i + 4 * u) * N);
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const float xv = xs[i + 4 * u];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          acc[2 * c] = __builtin_fmaf(xv, bf16_lo(v[u][c]), acc[2 * c]);
          acc[2 * c + 1] = __builtin_fmaf(xv, bf16_hi(v[u][c]), acc[2 * c + 1]);
        }
      }
    }
    for (; i < rows; i += 4) {
      const u32x4 v = ld_stream(wp + int64_t(i) * N);
      const float xv = xs[i];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        acc[2 * c] = __builtin_fmaf(xv, bf16_lo(v[c]), acc[2 * c]);
        acc[2 * c + 1] = __builtin_fmaf(xv, bf16_hi(v[c]), acc[2 * c + 1]);
      }
    }
  }
#pragma unroll
  for (int c = 0; c < 8; ++c) red[wave][8 * lane + c] = acc[c];
  __syncthreads();
  for (int c = threadIdx.x; c < kColBlock; c += kGemvThreads) {
    const int n = n0 + c;
    if (n < N) part[int64_t(split) * N + n] = (red[0][c] + red[1][c]) + (red[2][c] + red[3][c]);
  }
}

// 16 columns a workgroup, 16 split groups of 16 lanes: each lane sums every 16th split, eight of
// its loads in flight before the first add (the partials come from L2 or another XCD: latency,
// not bandwidth, bounds this; up to 128 splits cost one round trip)
constexpr int kFinCols = 16;
__global__ __launch_bounds__(256) void gemv_finish(const float* __restrict__ part, int splits, int N,
                                                   const uint16_t* __restrict__ r1, const uint16_t* __restrict__ r2,
                                                   uint16_t* __restrict__ y) {
  __shared__ float red[16][kFinCols];
  const int c = threadIdx.x % kFinCols, sg = threadIdx.x / kFinCols;
  const int n = blockIdx.x * kFinCols + c;
  float acc = 0.f;
  if (n < N) {
    for (int sp0 = sg; sp0 < splits; sp0 += 128) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int sp = sp0 + 16 * u;
        v[u] = part[int64_t(sp < splits ? sp : splits - 1) * N + n];
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) acc += sp0 + 16 * u < splits ? v[u] : 0.f;
    }
  }
  red[sg][c] = acc;
  __syncthreads();
  if (sg == 0 && n < N) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) s += red[i][c];
    if (r1) s += bf16_to_f32(r1[n]) + (r2 ? bf16_to_f32(r2[n]) : 0.f);
    y[n] = f32_to_bf16(s);
  }
}

// y == nullptr: the partial pass only, its partials left in ws for a consumer that finishes them
// (kSiluParts).  xparts / xsplits: kSiluParts' input partials.
template <int MODE>
int launch_gemv(const void* x, const void* add, const float* ss, const void* g, float eps, const void* w,
                const void* r1, const void* r2, void* y, int64_t k, int64_t n, void* ws, size_t ws_bytes,
                void* stream, const float* xparts = nullptr, int xsplits = 0) {
  if (k < 0 || n < 0) return PTB_ERR_SHAPE;
  if (n == 0) return PTB_OK;
  if ((MODE == kSiluParts ? !xparts : !x) || !w || (MODE == kRms && !g)) return PTB_ERR_NULL;
  if (!y && MODE != kRms) return PTB_ERR_NULL;
  if (MODE == kRms && !ss && (!aligned16(x) || (add && !aligned16(add)))) return PTB_ERR_ALIGN;
  if (k == 0) return PTB_ERR_UNSUPPORTED;
  if (k > 0x7fffffff || n > 0x7fffffff || k * n >= (int64_t(1) << 40)) return PTB_ERR_SHAPE;
  if (n % 8) return PTB_ERR_UNSUPPORTED;
  if (!aligned16(w)) return PTB_ERR_ALIGN;
  const GemvSplit sp = gemv_split(k, n);
  if (sp.splits > 65535) return PTB_ERR_GRID;
  if (!ws || ws_bytes < size_t(sp.splits) * size_t(n) * sizeof(float)) return PTB_ERR_WORKSPACE;
  if (reinterpret_cast<uintptr_t>(ws) & 3u) return PTB_ERR_ALIGN;
  hipStream_t s = static_cast<hipStream_t>(stream);
  float* part = static_cast<float*>(ws);
  const dim3 grid1(unsigned((n + kColBlock - 1) / kColBlock), unsigned(sp.splits));
  gemv_partial<MODE><<<grid1, dim3(kGemvThreads), 0, s>>>(
      static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(add), ss, static_cast<const uint16_t*>(g), eps,
      static_cast<const uint16_t*>(w), part, int(k), int(n), sp.kb, xparts, xsplits);
  if (!y) return launch_status();
  gemv_finish<<<dim3(unsigned((n + kFinCols - 1) / kFinCols)), dim3(256), 0, s>>>(
      part, sp.splits, int(n), static_cast<const uint16_t*>(r1), static_cast<const uint16_t*>(r2),
      static_cast<uint16_t*>(y));
  return launch_status();
}

// ---------------------------------------------------------------------------------------------
// grouped GEMV: the grouped GEMM when A has at most kGgMaxRows rows (the decode MoE: one token's k
// experts, a row each).  For each program p with g = group[p]: C[start[g] + i] = A[start[g] + i] @
// B[g] for i < rows[g].  Pass 1: workgroup (512-column block, 64-row K slice, program); as soon as
// g is known every lane issues its 16 weight loads of the slice (the slice stays in registers, read
// once however many rows the group has), then reads start/rows and A's slice into LDS, kGgRows rows
// at a time; fp32 partials per (program, slice, row).  Pass 2 sums the slices and rounds.

constexpr int kGgRows = 4;       // A rows a pass of FMAs over the register-held slice serves
constexpr int kGgMaxRows = 16;   // A rows at most: no program can have more
constexpr int kGgKb = 64;        // K rows per slice: 16 per wave, one 16-byte load each per lane

// Table checks as the MFMA path makes them: group in [0, ntab) and below nweights; rows > 0,
// start >= 0, start + rows <= a_rows.  An entry failing them is an empty program.
__device__ __forceinline__ bool gg_weight(int g, int ntab, int nweights) { return g >= 0 && g < ntab && g < nweights; }
__device__ __forceinline__ bool gg_rows(int s0, int nr, int a_rows) {
  return nr > 0 && s0 >= 0 && int64_t(s0) + nr <= a_rows;
}

__global__ __launch_bounds__(kGemvThreads) void ggemv_partial(const uint16_t* __restrict__ A,
                                                              const uint16_t* __restrict__ B,
                                                              const int32_t* __restrict__ grp,
                                                              const int32_t* gstart, const int32_t* grows, int ntab,
                                                              int nweights, int a_rows, int64_t sbg, int K, int N,
                                                              int splits, float* __restrict__ part) {
  __shared__ float xs[kGgRows][kGgKb];
  __shared__ float red[4][kGgRows][kColBlock];
  const int p = blockIdx.z, split = blockIdx.y, n0 = blockIdx.x * kColBlock;
  const int g = grp[p];
  if (!gg_weight(g, ntab, nweights)) return;   // uniform
  const int k0 = split * kGgKb, krows = min(K - k0, kGgKb);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = min(n0 + 8 * lane, N - 8);    // lanes past N repeat the last columns (not stored)
  // rows wave, wave + 4, ... of the slice; rows past K repeat the slice's last row (weight 0 below)
  const uint16_t* wp = B + int64_t(g) * sbg + int64_t(k0) * N + col;
  u32x4 v[kGgKb / 4];
#pragma unroll
  for (int u = 0; u < kGgKb / 4; ++u)
    v[u] = ld_stream(wp + int64_t(min(wave + 4 * u, krows - 1)) * N);
  // the first pass below runs even for an empty row range (it then stores nothing): an exit or a
  // guarded loop would let the compiler move the weight loads after the table reads and wait for
  // those first
  const int s0r = gstart[g], nr0 = grows[g];
  const bool has_rows = gg_rows(s0r, nr0, a_rows);
  const int nr = has_rows ? nr0 : 0, s0 = has_rows ? s0r : 0;
  int i0 = 0;
  do {
    const int rb = min(kGgRows, nr - i0);   // <= 0 for an empty range: no A row read, nothing stored
    for (int t = threadIdx.x; t < kGgRows * kGgKb; t += kGemvThreads) {
      const int r = t / kGgKb, kk = t % kGgKb;
      xs[r][kk] = (r < rb && kk < krows) ? bf16_to_f32(A[int64_t(s0 + i0 + r) * K + k0 + kk]) : 0.f;
    }
    __syncthreads();
    // the weights' unpacking stays here, after A's loads went out (hoisted out of the loop it
    // would wait for every weight load before A's loads)
#pragma unroll
    for (int u = 0; u < kGgKb / 4; ++u) __asm__ volatile("" : "+v"(v[u]));
    float acc[kGgRows][8];
#pragma unroll
    for (int r = 0; r < kGgRows; ++r)
#pragma unroll
      for (int c = 0; c < 8; ++c) acc[r][c] = 0.f;
#pragma unroll
    for (int u = 0; u < kGgKb / 4; ++u)
#pragma unroll
      for (int r = 0; r < kGgRows; ++r) {
        const float xv = xs[r][wave + 4 * u];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          acc[r][2 * c] = __builtin_fmaf(xv, bf16_lo(v[u][c]), acc[r][2 * c]);
          acc[r][2 * c + 1] = __builtin_fmaf(xv, bf16_hi(v[u][c]), acc[r][2 * c + 1]);
        }
      }
#pragma unroll
    for (int r = 0; r < kGgRows; ++r)
#pragma unroll
      for (int c = 0; c < 8; ++c) red[wave][r][8 * lane + c] = acc[r][c];
    __syncthreads();
    for (int t = threadIdx.x; t < kGgRows * kColBlock; t += kGemvThreads) {
      const int r = t / kColBlock, c = t - r * kColBlock, n = n0 + c;
      if (r < rb && n < N)
        part[((int64_t(p) * splits + split) * a_rows + i0 + r) * N + n] =
            (red[0][r][c] + red[1][r][c]) + (red[2][r][c] + red[3][r][c]);
    }
    __syncthreads();   // xs and red are refilled by the next rows
    i0 += kGgRows;
  } while (i0 < nr);
}

// Workgroup (program, 64 columns): C[start + i, n] = bf16(sum over slices) for the program's rows i;
// 4 slice groups of 64 lanes, each lane 8 slices in flight.
constexpr int kGgFinCols = 64;
__global__ __launch_bounds__(256) void ggemv_finish(const float* __restrict__ part, const int32_t* __restrict__ grp,
                                                    const int32_t* __restrict__ gstart,
                                                    const int32_t* __restrict__ grows, int ntab, int nweights,
                                                    int a_rows, int splits, int N, uint16_t* __restrict__ C) {
  __shared__ float red[4][kGgFinCols];
  const int p = blockIdx.y;
  const int g = grp[p];
  if (!gg_weight(g, ntab, nweights)) return;   // uniform
  const int s0 = gstart[g], nr = grows[g];
  if (!gg_rows(s0, nr, a_rows)) return;        // uniform
  const int c = threadIdx.x % kGgFinCols, sg = threadIdx.x / kGgFinCols;
  const int n = blockIdx.x * kGgFinCols + c;
  const int64_t sstride = int64_t(a_rows) * N;
  for (int i = 0; i < nr; ++i) {
    const float* base = part + (int64_t(p) * splits * a_rows + i) * N + min(n, N - 1);
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int sp0 = sg; sp0 < splits; sp0 += 32) {
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int sp = sp0 + 4 * u;
        acc[u] += sp < splits ? base[int64_t(min(sp, splits - 1)) * sstride] : 0.f;
      }
    }
    red[sg][c] = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
    __syncthreads();
    if (sg == 0 && n < N) C[int64_t(s0 + i) * N + n] = f32_to_bf16((red[0][c] + red[1][c]) + (red[2][c] + red[3][c]));
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------------------------
// decode attention

constexpr int kD = 128;
constexpr int kChunk = 64;          // keys per team step
constexpr int kTeam = 256;          // threads per 64-key chunk
constexpr int kMaxRecords = 256;    // key ranges per kv head that the merge pass combines

// The VALU form serves caches of at most kWaveMinSeq (256) keys in one pass: a workgroup per query
// row, T teams of 256 threads taking one 64-key chunk each (T = 1, 2 or 4 for up to 1, 2 or 4
// chunks; four teams are 1024 threads at 128 VGPRs a lane), merged in LDS.
inline int small_teams(int64_t seq) {
  const int64_t chunks = (seq + kChunk - 1) / kChunk;
  return chunks <= 1 ? 1 : chunks <= 2 ? 2 : 4;
}

// One record per (kv head, key range): acc[G][128], m[G], l[G], padded to 16 bytes.
constexpr int64_t record_floats(int64_t g) { return g * kD + ((2 * g + 3) & ~int64_t(3)); }

// One 64-key step of K and V into registers: lane (kj = tid/16, d8 = tid%16 of its team) holds
// dims 8*d8..+8 of keys kj, kj+16, kj+32, kj+48; keys past S repeat key S-1 (their scores are
// masked), so an idle team's loads stay in bounds too.
__device__ __forceinline__ void load_step(const uint16_t* __restrict__ kp, const uint16_t* __restrict__ vp, int key0,
                                          int S, int kj, int d8, u32x4 (&kr)[kChunk / 16],
                                          u32x4 (&vr)[kChunk / 16]) {
#pragma unroll
  for (int pass = 0; pass < kChunk / 16; ++pass) {
    const int key = min(key0 + pass * 16 + kj, S - 1);
    kr[pass] = *reinterpret_cast<const u32x4*>(kp + int64_t(key) * kD + 8 * d8);
  }
#pragma unroll
  for (int pass = 0; pass < kChunk / 16; ++pass) {
    const int key = min(key0 + pass * 16 + kj, S - 1);
    vr[pass] = *reinterpret_cast<const u32x4*>(vp + int64_t(key) * kD + 8 * d8);
  }
}

// One 16-byte query vector, dims 8*(qi%16).. of query head qi/16 (the layout of the q/k-norm
// kernel), with, for the fused q-norm + RoPE (qw given), its norm weights and the token's cos/sin.
struct QVec {
  u32x4 q, w, wp;
  f32x4v cs0, cs1, sn0, sn1;
};
__device__ __forceinline__ QVec load_qvec(const uint16_t* __restrict__ q, int qi, const uint16_t* __restrict__ qw,
                                          const float* __restrict__ qcos, const float* __restrict__ qsin) {
  QVec v;
  v.q = *reinterpret_cast<const u32x4*>(q + 8 * qi);
  const int qc = qi & 15;
  v.w = u32x4{0u, 0u, 0u, 0u};
  v.wp = v.w;
  v.cs0 = f32x4v{0.f, 0.f, 0.f, 0.f};
  v.cs1 = v.cs0;
  v.sn0 = v.cs0;
  v.sn1 = v.cs0;
  if (qw) {
    v.w = reinterpret_cast<const u32x4*>(qw)[qc];
    v.wp = reinterpret_cast<const u32x4*>(qw)[qc ^ 8];
    v.cs0 = reinterpret_cast<const f32x4v*>(qcos + 8 * qc)[0];
    v.cs1 = reinterpret_cast<const f32x4v*>(qcos + 8 * qc)[1];
    v.sn0 = reinterpret_cast<const f32x4v*>(qsin + 8 * qc)[0];
    v.sn1 = reinterpret_cast<const f32x4v*>(qsin + 8 * qc)[1];
  }
  return v;
}
// The vector's 8 values as fp32 (exact bf16 values).  With q-norm + RoPE: the q/k-norm kernel's
// arithmetic, rounded to bf16 as its output is; the sum of squares meets across the 16 lanes of
// the head (a 16-lane row), so all 16 lanes of a row call this together.
__device__ __forceinline__ void qvec_values(const QVec& v, int qi, bool norm, float qeps, float (&qf8)[8]) {
  const int qc = qi & 15;
  const u32x4 qv = v.q, wv = v.w, wp = v.wp;
  const f32x4v cs0 = v.cs0, cs1 = v.cs1, sn0 = v.sn0, sn1 = v.sn1;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    qf8[2 * e] = bf16_lo(qv[e]);
    qf8[2 * e + 1] = bf16_hi(qv[e]);
  }
  if (norm) {
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss = fmaf(qf8[e], qf8[e], ss);
    ss = row16_sum(ss);
    float pf[8], wf[8], pw[8];
    u32x4 pv;
#pragma unroll
    for (int e = 0; e < 4; ++e) pv[e] = xor8_u32(qv[e]);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      pf[2 * e] = bf16_lo(pv[e]);
      pf[2 * e + 1] = bf16_hi(pv[e]);
      wf[2 * e] = bf16_lo(wv[e]);
      wf[2 * e + 1] = bf16_hi(wv[e]);
      pw[2 * e] = bf16_lo(wp[e]);
      pw[2 * e + 1] = bf16_hi(wp[e]);
    }
    const float r = 1.0f / sqrtf(ss / float(kD) + qeps);
    const float cs[8] = {cs0.x, cs0.y, cs0.z, cs0.w, cs1.x, cs1.y, cs1.z, cs1.w};
    const float sn[8] = {sn0.x, sn0.y, sn0.z, sn0.w, sn1.x, sn1.y, sn1.z, sn1.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float a = (qf8[e] * r) * wf[e];
      const float pp = (pf[e] * r) * pw[e];
      const float rot = qc < 8 ? -pp : pp;
      qf8[e] = bf16_to_f32(f32_to_bf16(fmaf(a, cs[e], rot * sn[e])));
    }
  }
}

// Workgroup (query row kvh of kv head kvh / group) of T teams, team t on keys 64t .. 64t+63: scores
// t = (q.k) * scale*log2(e) with 16 lanes a key, a base-2 softmax over the chunk (m = max, p =
// 2^(t-m), l = sum of fp32 p) and acc = sum bf16(p) * v; the teams then meet in LDS (weights
// 2^(m_t - M)) and the workgroup writes o = bf16(acc / l).  G = 1 (one row a workgroup).
template <int G, int T>
__global__ __launch_bounds__(kTeam * T) void attn_decode_partial(const uint16_t* __restrict__ Q,
                                                                 const uint16_t* __restrict__ Kc,
                                                                 const uint16_t* __restrict__ Vc,
                                                                 uint16_t* __restrict__ O, int S, float c, int group,
                                                                 const uint16_t* __restrict__ qw,
                                                                 const float* __restrict__ qcos,
                                                                 const float* __restrict__ qsin, float qeps) {
  __shared__ float qs[G][kD];
  __shared__ float ts[T][G][kChunk];      // scores, then bf16-rounded p
  __shared__ float red[T][4][G][kD];
  __shared__ float mrun[T][G], lrun[T][G], alpha[T][G], wt[T][G], lfin[G];
  const int kvh = blockIdx.x;
  const int tid = threadIdx.x, team = tid / kTeam, ttid = tid % kTeam;
  const int lane = tid & 63, wave = ttid >> 6, d8 = lane & 15, kj = ttid >> 4;
  const uint16_t* q = Q + int64_t(kvh) * G * kD;                 // kvh: this workgroup's G query rows
  const uint16_t* kp = Kc + int64_t(kvh / group) * S * kD;       // of kv head kvh / group
  const uint16_t* vp = Vc + int64_t(kvh / group) * S * kD;
  const int key0 = team * kChunk;                                // this team's chunk

  // q's load goes out before the first step's K and V, so waiting for q does not wait for them:
  // 16 bytes a lane, lanes past the G*16 vectors repeat the last one (the same value, and no
  // branch for the load to sink into)
  const int qi = min(tid, G * kD / 8 - 1);
  const QVec qv = load_qvec(q, qi, qw, qcos, qsin);
  u32x4 kr[kChunk / 16], vr[kChunk / 16];
  load_step(kp, vp, key0, S, kj, d8, kr, vr);
  float qf8[8];
  qvec_values(qv, qi, qw != nullptr, qeps, qf8);
  // lanes past the G*16 vectors hold repeats (whose norms are not their head's): they do not store
  if (tid < G * kD / 8) {
#pragma unroll
    for (int e = 0; e < 8; ++e) qs[0][8 * qi + e] = qf8[e];
  }
  if (ttid < G) {
    mrun[team][ttid] = -INFINITY;
    lrun[team][ttid] = 0.f;
  }
  __syncthreads();
  // one team: q in registers; several (up to 1024 threads, 128 VGPRs a lane): q read from LDS
  float qf[T == 1 ? G : 1][8];
  if constexpr (T == 1) {
#pragma unroll
    for (int gi = 0; gi < G; ++gi)
#pragma unroll
      for (int e = 0; e < 8; ++e) qf[gi][e] = qs[gi][8 * d8 + e];
  }
  float acc[G][8];
#pragma unroll
  for (int gi = 0; gi < G; ++gi)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[gi][e] = 0.f;

  {
    const u32x4 (&kc)[kChunk / 16] = kr;
    const u32x4 (&vc)[kChunk / 16] = vr;

#pragma unroll
    for (int pass = 0; pass < kChunk / 16; ++pass) {
      const int j = pass * 16 + kj;
      float kf[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        kf[2 * e] = bf16_lo(kc[pass][e]);
        kf[2 * e + 1] = bf16_hi(kc[pass][e]);
      }
#pragma unroll
      for (int gi = 0; gi < G; ++gi) {
        float sc = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) sc = __builtin_fmaf(T == 1 ? qf[gi][e] : qs[gi][8 * d8 + e], kf[e], sc);
        sc = row16_sum(sc);
        if (d8 == 0) ts[team][gi][j] = (key0 + j < S) ? sc * c : -INFINITY;
      }
    }
    __syncthreads();

    // running softmax: 32 lanes per query head, 2 keys a lane; a chunk with no key left (an idle
    // team) keeps m = -inf, l = 0 and adds nothing
    for (int gi = ttid / 32; gi < G; gi += kTeam / 32) {
      const int l32 = ttid & 31;
      float mx = -INFINITY;
#pragma unroll
      for (int e = 0; e < kChunk / 32; ++e) mx = fmaxf(mx, ts[team][gi][l32 + 32 * e]);
      mx = pair16_max(row16_max(mx));
      const float mold = mrun[team][gi], mnew = fmaxf(mold, mx);
      const float mref = mnew == -INFINITY ? 0.f : mnew;
      float ls = 0.f;
#pragma unroll
      for (int e = 0; e < kChunk / 32; ++e) {
        const float p = __builtin_amdgcn_exp2f(ts[team][gi][l32 + 32 * e] - mref);
        ls += p;
        ts[team][gi][l32 + 32 * e] = bf16_to_f32(f32_to_bf16(p));
      }
      ls = pair16_sum(row16_sum(ls));
      if (l32 == 0) {
        const float a = __builtin_amdgcn_exp2f(mold - mref);
        alpha[team][gi] = a;
        mrun[team][gi] = mnew;
        lrun[team][gi] = __builtin_fmaf(lrun[team][gi], a, ls);
      }
    }
    __syncthreads();

#pragma unroll
    for (int gi = 0; gi < G; ++gi) {
      const float a = alpha[team][gi];
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[gi][e] *= a;
    }
#pragma unroll
    for (int pass = 0; pass < kChunk / 16; ++pass) {
      const int j = pass * 16 + kj;
      float vf[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        vf[2 * e] = bf16_lo(vc[pass][e]);
        vf[2 * e + 1] = bf16_hi(vc[pass][e]);
      }
#pragma unroll
      for (int gi = 0; gi < G; ++gi) {
        const float p = ts[team][gi][j];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[gi][e] = __builtin_fmaf(p, vf[e], acc[gi][e]);
      }
    }
  }

  // lanes l, l^16, l^32, l^48 hold the same dims; then each team's four waves meet in LDS
#pragma unroll
  for (int gi = 0; gi < G; ++gi)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[gi][e] = pair32_sum(pair16_sum(acc[gi][e]));
  if (lane < 16) {
#pragma unroll
    for (int gi = 0; gi < G; ++gi)
#pragma unroll
      for (int e = 0; e < 8; ++e) red[team][wave][gi][8 * d8 + e] = acc[gi][e];
  }
  if (tid < G) {   // the teams' weights: 2^(m_t - M), 0 for a team that saw no key
    float mm = mrun[0][tid];
#pragma unroll
    for (int t = 1; t < T; ++t) mm = fmaxf(mm, mrun[t][tid]);
    float ll = 0.f;
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const float w = T == 1 ? 1.f : __builtin_amdgcn_exp2f(mrun[t][tid] - mm);
      wt[t][tid] = w;
      ll = __builtin_fmaf(lrun[t][tid], w, ll);
    }
    lfin[tid] = ll;
  }
  __syncthreads();

  for (int i = tid; i < G * kD; i += kTeam * T) {
    const int gi = i / kD, d = i % kD;
    float o = 0.f;
#pragma unroll
    for (int t = 0; t < T; ++t)
      o = __builtin_fmaf(wt[t][gi], (red[t][0][gi][d] + red[t][1][gi][d]) + (red[t][2][gi][d] + red[t][3][gi][d]), o);
    O[(int64_t(kvh) * G + gi) * kD + d] = f32_to_bf16(o / lfin[gi]);
  }
}

// Workgroup (kv head, query head): o = sum acc_r 2^(m_r-M) / sum l_r 2^(m_r-M), M = max m_r, over
// the head's records.  The acc loads do not depend on the weights, so they go out with the (m, l)
// loads: lane (r, o4) holds 4 dims of records r, r+8, ..., up to 16 of them in flight, and a lane
// per record reads its m and l; one round trip covers up to 128 records.
template <int G>
__global__ __launch_bounds__(256) void attn_decode_merge(const float* __restrict__ part, uint16_t* __restrict__ O,
                                                         int nrec) {
  constexpr int kRec = int(record_floats(G));
  constexpr int kR = 256 / (kD / 4);    // 8 lanes per 4 output dims
  __shared__ float wl[kMaxRecords];
  __shared__ float red[2][4];
  __shared__ f32x4 msum[256];
  const int kvh = blockIdx.x, gi = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const float* recs = part + int64_t(kvh) * nrec * kRec;
  const int o4 = tid % (kD / 4), r = tid / (kD / 4);
  const float* base = recs + gi * kD + 4 * o4;
  f32x4 v[16];
#pragma unroll
  for (int u = 0; u < 16; ++u) v[u] = *reinterpret_cast<const f32x4*>(base + int64_t(min(r + u * kR, nrec - 1)) * kRec);
  const int r0 = min(tid, nrec - 1);
  const bool ok = tid < nrec;
  const float m = ok ? recs[int64_t(r0) * kRec + G * kD + gi] : -INFINITY;
  const float l = recs[int64_t(r0) * kRec + G * kD + G + gi];
  const float mw = wave_absmax(m);
  if (lane == 0) red[0][wave] = mw;
  __syncthreads();
  const float mm = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
  const float w = ok ? __builtin_amdgcn_exp2f(m - mm) : 0.f;
  if (ok) wl[tid] = w;
  const float lw = wave_sum(l * w);
  if (lane == 0) red[1][wave] = lw;
  __syncthreads();

  f32x4 sum = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int u = 0; u < 16; ++u) {
    const int s = r + u * kR;
    const float ws = s < nrec ? wl[s] : 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) sum[e] = __builtin_fmaf(ws, v[u][e], sum[e]);
  }
  for (int s0 = r + 16 * kR; s0 < nrec; s0 += 16 * kR) {   // more than 128 records
#pragma unroll
    for (int u = 0; u < 16; ++u) v[u] = *reinterpret_cast<const f32x4*>(base + int64_t(min(s0 + u * kR, nrec - 1)) * kRec);
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int s = s0 + u * kR;
      const float ws = s < nrec ? wl[s] : 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) sum[e] = __builtin_fmaf(ws, v[u][e], sum[e]);
    }
  }
  msum[tid] = sum;
  __syncthreads();
  if (tid < kD / 4) {
    f32x4 t = msum[tid];
#pragma unroll
    for (int rr = 1; rr < kR; ++rr) t += msum[rr * (kD / 4) + tid];
    const float lt = (red[1][0] + red[1][1]) + (red[1][2] + red[1][3]);
    uint16_t* out = O + (int64_t(kvh) * G + gi) * kD + 4 * tid;
#pragma unroll
    for (int e = 0; e < 4; ++e) out[e] = f32_to_bf16(t[e] / lt);
  }
}

// Decode attention on the matrix cores.  Workgroup = one wave = (key range, kv head); the range's
// `steps` steps of 32 keys run in turn, each step's K and V tiles moving HBM -> LDS with
// buffer_load ... lds (the next step's while this one computes; keys past S read as zero through
// the buffer range).  All G <= 16 query rows of the kv head are the N side of
// v_mfma_f32_16x16x32_bf16, so K and V are read once whatever G is:
//   S^T[key][q] = K Q^T: A = K (lane: key 16t + l%16, dims 32kk + 8(l/16) .. +7, from the K tile),
//   B = Q^T (lane: query l%16, the same dims; rows past G are zero); key tile t's accumulator leaves
//   lane l the scores of keys 16t + 4(l/16) + i (i < 4) of query l%16.
//   O^T[d][q] += V^T[d][key] P^T[key][q]: B = P^T straight from the score accumulators (k slot
//   8(l/16) + j is key 4(l/16) + j for j < 4 and 16 + 4(l/16) + j - 4 for j >= 4), A = V^T from two
//   ds_read_b64_tr_b16 of the V tile per 16 dims (a 16-lane group reads 4 keys x 16 dims).
// Online softmax in base 2 per step, as the reference's decode kernel per key block: t = (q.k) *
// scale*log2(e), m = running max, p = 2^(t - m), l = l*2^(m_old - m) + sum of fp32 p (each lane
// sums its own keys; the four lane groups add up at the end), acc = acc*2^(m_old - m) + bf16(p) V.
// One range writes o = bf16(acc / l) itself; more leave (acc, m, l) records for attn_decode_merge.
constexpr int kWKeys = 32;                   // keys per wave step
constexpr int kWTile = kWKeys * kD * 2;      // 8 KB: one step's K or V tile

typedef unsigned int u32x2v __attribute__((ext_vector_type(2)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
typedef __attribute__((address_space(3))) bf16x8 lds_bf16x8;

__device__ __forceinline__ bf16x8 lds_b128(uint32_t addr) {
  return *reinterpret_cast<const lds_bf16x8*>(size_t(addr));
}
__device__ __forceinline__ i16x4 lds_tr16(uint32_t addr) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(reinterpret_cast<lds_i16x4*>(size_t(addr)));
}

template <int G>
__global__ __launch_bounds__(64) void attn_decode_mfma(const uint16_t* __restrict__ Q, const uint16_t* __restrict__ Kc,
                                                       const uint16_t* __restrict__ Vc, uint16_t* __restrict__ O,
                                                       float* __restrict__ part, int S, float c, int steps,
                                                       const uint16_t* __restrict__ qw, const float* __restrict__ qcos,
                                                       const float* __restrict__ qsin, float qeps) {
  static_assert(G >= 1 && G <= 16, "the query rows fit the MFMA's N side");
  constexpr int kRec = int(record_floats(G));
  constexpr int kQVecs = G * kD / 8;         // 16-byte query vectors
  // two stages of (K tile, V tile), then the query rows as bf16 [16][128] (rows past G zero)
  __shared__ __attribute__((aligned(1024))) uint8_t smem[4 * kWTile + 16 * kD * 2];
  const int range = blockIdx.x, kvh = blockIdx.y, nrec = gridDim.x;
  const int lane = threadIdx.x, l16 = lane & 15, g4 = lane >> 4;
  const uint16_t* kp = Kc + int64_t(kvh) * S * kD;
  const uint16_t* vp = Vc + int64_t(kvh) * S * kD;
  const uint32_t lds0 = uint32_t(reinterpret_cast<uintptr_t>(smem));
  uint8_t* const qs = smem + 4 * kWTile;

  // DMA instruction i of a tile fills key rows 4i .. 4i+3: lane L writes row 4i + L/16, slot L%16,
  // so it fetches the chunk that belongs in that slot.  K row r keeps chunk c in slot c ^ (r & 15)
  // (a fragment read's 16 lanes take 16 rows); V row r keeps chunk c in slot c ^ (4 * (r & 3)) (a
  // transposing read's 16 lanes take 4 rows x 4 chunks).
  // Offsets stay in the VGPR operand (soffset 0), which the buffer range check covers.
  uint32_t koff[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int r = 4 * i + g4;
    koff[i] = uint32_t(r * 256 + ((l16 ^ (r & 15)) << 4));
  }
  const uint32_t vdma = uint32_t(g4 * 256 + ((l16 ^ (4 * g4)) << 4));
  auto issue = [&](int s, auto par) __attribute__((always_inline)) {
    constexpr int P = decltype(par)::value;
    const int key0 = (range * steps + s) * kWKeys;
    const uint32_t bytes = uint32_t(max(0, min(kWKeys, S - key0))) * uint32_t(kD * 2);
    i32x4 rk = make_rsrc(kp + int64_t(key0) * kD, bytes);
    i32x4 rv = make_rsrc(vp + int64_t(key0) * kD, bytes);
#pragma unroll
    for (int e = 0; e < 4; ++e) {   // wave-uniform values, kept in SGPRs as the instruction needs
      rk[e] = __builtin_amdgcn_readfirstlane(rk[e]);
      rv[e] = __builtin_amdgcn_readfirstlane(rv[e]);
    }
    const uint32_t st = lds0 + uint32_t(P * 2 * kWTile);
#pragma unroll
    for (int i = 0; i < 8; ++i)
      dma16(rk, __builtin_amdgcn_readfirstlane(st + i * 1024), koff[i], 0);
#pragma unroll
    for (int i = 0; i < 8; ++i)
      dma16(rv, __builtin_amdgcn_readfirstlane(st + kWTile + i * 1024), vdma + i * 1024, 0);
  };
  issue(0, std::integral_constant<int, 0>{});

  // the query rows into LDS (vector v at byte 16 v: row v / 16, dims 8 (v % 16) ..), zero past G;
  // the 16 lanes of a row hold one head's vectors, as qvec_values wants
  const uint16_t* q = Q + int64_t(kvh) * G * kD;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int v = lane + 64 * u;
    u32x4 packed = {0u, 0u, 0u, 0u};
    if (64 * u < kQVecs) {
      const int qi = min(v, kQVecs - 1);
      const QVec qv = load_qvec(q, qi, qw, qcos, qsin);
      float qf8[8];
      qvec_values(qv, qi, qw != nullptr, qeps, qf8);
      if (v < kQVecs) {
#pragma unroll
        for (int e = 0; e < 4; ++e) packed[e] = pack_bf16x2(qf8[2 * e], qf8[2 * e + 1]);
      }
    }
    *reinterpret_cast<u32x4*>(qs + 16 * v) = packed;
  }
  // B = Q^T fragments: query l16, dims 32kk + 8 g4 .. +7 (the wave's own LDS writes are done)
  bf16x8 qf[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk)
    qf[kk] = *reinterpret_cast<const bf16x8*>(qs + l16 * 256 + (4 * kk + g4) * 16);

  // V^T fragment reads: in-group lane 4 jj + qq supplies key 4 g4 + jj (16 more for the second
  // read), dims 16 dt + 4 qq .. +3 = chunk 2 dt + qq / 2, byte 8 (qq & 1) within it
  const int jj = l16 >> 2, qq = l16 & 3;
  uint32_t vrd[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt)
    vrd[dt] = uint32_t((4 * g4 + jj) * 256 + (((2 * dt + (qq >> 1)) ^ (4 * jj)) << 4) + (qq & 1) * 8);

  f32x4 acc[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, lsum = 0.f;

  auto step = [&](int s, auto par, auto more) __attribute__((always_inline)) {
    constexpr int P = decltype(par)::value;
    constexpr bool MORE = decltype(more)::value;
    // the next step's tiles go into the other stage, whose reads (the previous step's) are done
    if constexpr (MORE) issue(s + 1, std::integral_constant<int, 1 - P>{});
    const uint32_t st = lds0 + uint32_t(P * 2 * kWTile);
    wait_vmcnt<MORE ? 24 : 8>();   // this step's K tile has landed (its V tile may still be coming)
    f32x4 sacc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const bf16x8 kf = lds_b128(st + (16 * t + l16) * 256 + (((4 * kk + g4) ^ l16) << 4));
        sacc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qf[kk], sacc[t], 0, 0, 0);
      }
    const int key0 = (range * steps + s) * kWKeys;
    float tv[2][4];
    float mx = -INFINITY;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        tv[t][i] = key0 + 16 * t + 4 * g4 + i < S ? sacc[t][i] * c : -INFINITY;
        mx = fmaxf(mx, tv[t][i]);
      }
    mx = pair32_max(pair16_max(mx));
    const float mnew = fmaxf(m, mx);
    const float mref = mnew == -INFINITY ? 0.f : mnew;
    const float alpha = __builtin_amdgcn_exp2f(m - mref);
    m = mnew;
    float ps = 0.f;
    uint32_t pb[4];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int i = 0; i < 4; i += 2) {
        const float p0 = __builtin_amdgcn_exp2f(tv[t][i] - mref);
        const float p1 = __builtin_amdgcn_exp2f(tv[t][i + 1] - mref);
        ps += p0;
        ps += p1;
        pb[2 * t + i / 2] = pack_bf16x2(p0, p1);
      }
    lsum = __builtin_fmaf(lsum, alpha, ps);
    if (__builtin_amdgcn_ballot_w64(alpha != 1.f)) {
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) acc[dt] *= alpha;
    }
    const bf16x8 pf = __builtin_bit_cast(bf16x8, u32x4{pb[0], pb[1], pb[2], pb[3]});
    wait_vmcnt<MORE ? 16 : 0>();   // this step's V tile has landed
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const i16x4 lo = lds_tr16(st + kWTile + vrd[dt]);
      const i16x4 hi = lds_tr16(st + kWTile + vrd[dt] + 16 * 256);
      const bf16x8 vf = __builtin_bit_cast(bf16x8, i16x8(__builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7)));
      acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pf, acc[dt], 0, 0, 0);
    }
  };
  using P0 = std::integral_constant<int, 0>;
  using P1 = std::integral_constant<int, 1>;
  using More = std::true_type;
  using Last = std::false_type;
  int s = 0;
  for (; s + 2 < steps; s += 2) {
    step(s, P0{}, More{});
    step(s + 1, P1{}, More{});
  }
  if (s + 1 < steps) {
    step(s, P0{}, More{});
    step(s + 1, P1{}, Last{});
  } else {
    step(s, P0{}, Last{});
  }

  // lane l holds O^T[16 dt + 4 g4 + i][l16]; the query's l is the sum over its four lane groups
  lsum = pair32_sum(pair16_sum(lsum));
  if (l16 < G) {
    if (nrec == 1) {
      uint16_t* o = O + (int64_t(kvh) * G + l16) * kD + 4 * g4;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt)
        *reinterpret_cast<u32x2v*>(o + 16 * dt) =
            u32x2v{pack_bf16x2(acc[dt][0] / lsum, acc[dt][1] / lsum), pack_bf16x2(acc[dt][2] / lsum, acc[dt][3] / lsum)};
    } else {
      float* rec = part + (int64_t(kvh) * nrec + range) * kRec;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) *reinterpret_cast<f32x4*>(rec + l16 * kD + 16 * dt + 4 * g4) = acc[dt];
      if (g4 == 0) {
        rec[G * kD + l16] = m;
        rec[G * kD + G + l16] = lsum;
      }
    }
  }
}

// q-norm + RoPE fused into the prologue when qw is given (per-head weights [128], the token's
// cos / sin [128]): q is then the projection's raw output
struct QNorm {
  const uint16_t* w;
  const float* cos;
  const float* sin;
  float eps;
};

// The matrix-core form's cut of a kv head: `records` ranges of `steps` 32-key steps each (n steps in
// all): ceil(n / 48) steps a range below 256 steps, ceil(n / 64) from there, so a head has at most
// 64 ranges (the merge pass takes up to kMaxRecords).  Measured on MI355X (8 kv heads, graph
// replay), against one step a range: 4096 keys 10.63 -> 9.70 us, 8192 keys 16.0 -> 12.4 us, 16384
// keys 20.7 -> 18.6 us, G = 8 at 4096 keys 11.9 -> 10.2 us (fewer waves each stream more steps
// through the two stages, and the merge has fewer records).  Against the VALU form, at one step a
// range: 512 keys 6.98 -> 6.66 us, 4096 keys 11.46 -> 10.63 us, G = 8 at 4096 keys 15.2 -> 11.9 us.
// It serves caches of more than kWaveMinSeq keys.
constexpr int64_t kWaveMinSeq = 256;
struct WavePlan {
  int steps, records;
};
WavePlan wave_plan(int64_t seq) {
  const int64_t n = (seq + kWKeys - 1) / kWKeys;
  const int64_t steps = n < 256 ? (n + 47) / 48 : (n + 63) / 64;
  return {int(steps), int((n + steps - 1) / steps)};
}

template <int G>
void launch_attn_decode_mfma(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o, float* part,
                             int nkv, int seq, float c, const WavePlan& p, const QNorm& qn, hipStream_t s) {
  attn_decode_mfma<G><<<dim3(unsigned(p.records), unsigned(nkv)), dim3(64), 0, s>>>(
      q, k, v, o, part, seq, c, p.steps, qn.w, qn.cos, qn.sin, qn.eps);
  if (p.records > 1) attn_decode_merge<G><<<dim3(unsigned(nkv), unsigned(G)), dim3(256), 0, s>>>(part, o, p.records);
}

// The VALU form: one query row a workgroup, T teams (small_teams), o written in the same launch.
template <int T>
void launch_attn_decode_small(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o, int nkv, int group,
                              int seq, float c, const QNorm& qn, hipStream_t s) {
  attn_decode_partial<1, T><<<dim3(unsigned(nkv * group)), dim3(kTeam * T), 0, s>>>(q, k, v, o, seq, c, group, qn.w,
                                                                                      qn.cos, qn.sin, qn.eps);
}

}  // namespace

PTB_EXPORT int ptb_sumsq_bf16(const void* x, const void* y, float* out, int64_t n, void* stream) {
  if (n < 0) return PTB_ERR_SHAPE;
  if (!x || !out) return PTB_ERR_NULL;
  if (!aligned16(x) || (y && !aligned16(y))) return PTB_ERR_ALIGN;
  sumsq_kernel<<<dim3(1), dim3(1024), 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(y), out, n);
  return launch_status();
}

PTB_EXPORT size_t ptb_gemv_workspace_bytes(int64_t k, int64_t n) {
  if (k <= 0 || n <= 0) return 0;
  const GemvSplit sp = gemv_split(k, n);
  return size_t(sp.splits) * size_t(n) * sizeof(float);
}

PTB_EXPORT int ptb_gemv_bf16(const void* x, const void* w, void* y, int64_t k, int64_t n, void* workspace,
                             size_t workspace_bytes, void* stream) {
  return launch_gemv<kPlain>(x, nullptr, nullptr, nullptr, 0.f, w, nullptr, nullptr, y, k, n, workspace,
                             workspace_bytes, stream);
}

PTB_EXPORT int ptb_gemv_rmsnorm_bf16(const void* x, const void* add, const float* ss, const void* g, float eps,
                                     const void* w, void* y, int64_t k, int64_t n, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  return launch_gemv<kRms>(x, add, ss, g, eps, w, nullptr, nullptr, y, k, n, workspace, workspace_bytes, stream);
}

PTB_EXPORT int ptb_gemv_silu_bf16(const void* gate_up, const void* w, const void* res_a, const void* res_b, void* y,
                                  int64_t k, int64_t n, void* workspace, size_t workspace_bytes, void* stream) {
  if (res_b && !res_a) return PTB_ERR_NULL;
  return launch_gemv<kSilu>(gate_up, nullptr, nullptr, nullptr, 0.f, w, res_a, res_b, y, k, n, workspace,
                            workspace_bytes, stream);
}

PTB_EXPORT int ptb_gemv_rmsnorm_parts_bf16(const void* x, const void* add, const float* ss, const void* g, float eps,
                                           const void* w, float* parts, int64_t k, int64_t n, size_t parts_bytes,
                                           void* stream) {
  if (!parts) return PTB_ERR_NULL;
  return launch_gemv<kRms>(x, add, ss, g, eps, w, nullptr, nullptr, nullptr, k, n, parts, parts_bytes, stream);
}

PTB_EXPORT int ptb_gemv_silu_parts_bf16(const float* gate_up_parts, int64_t gate_up_k, const void* w, const void* res_a,
                                        const void* res_b, void* y, int64_t k, int64_t n, void* workspace,
                                        size_t workspace_bytes, void* stream) {
  if (res_b && !res_a) return PTB_ERR_NULL;
  if (gate_up_k <= 0 || gate_up_k > 0x7fffffff || k <= 0 || 2 * k > 0x7fffffff) return PTB_ERR_SHAPE;
  if (gate_up_parts && (reinterpret_cast<uintptr_t>(gate_up_parts) & 3u)) return PTB_ERR_ALIGN;
  // the producing GEMV's split of its K = gate_up_k rows, N = 2k columns
  const GemvSplit gs = gemv_split(gate_up_k, 2 * k);
  return launch_gemv<kSiluParts>(nullptr, nullptr, nullptr, nullptr, 0.f, w, res_a, res_b, y, k, n, workspace,
                                 workspace_bytes, stream, gate_up_parts, gs.splits);
}

PTB_EXPORT size_t ptb_attn_decode_workspace_bytes(int64_t nkv, int64_t group, int64_t seq) {
  if (nkv <= 0 || group <= 0 || seq <= 0 || seq >= (int64_t(1) << 30)) return 0;
  if (seq <= kWaveMinSeq) return 0;   // the VALU form's single launch
  const WavePlan w = wave_plan(seq);
  if (w.records == 1) return 0;
  return size_t(nkv * w.records * record_floats(group)) * sizeof(float);
}

static int attn_decode_entry(const void* q, const void* k, const void* v, void* o, int64_t nkv, int64_t group,
                             int64_t seq, int64_t head_dim, float scale, const QNorm& qn, void* workspace,
                             size_t workspace_bytes, void* stream) {
  if (nkv < 0 || group <= 0 || seq <= 0 || head_dim <= 0) return PTB_ERR_SHAPE;
  if (head_dim != kD) return PTB_ERR_UNSUPPORTED;
  if (group != 1 && group != 2 && group != 3 && group != 4 && group != 6 && group != 8) return PTB_ERR_UNSUPPORTED;
  if (!std::isfinite(scale)) return PTB_ERR_UNSUPPORTED;
  if (nkv == 0) return PTB_OK;
  if (!q || !k || !v || !o) return PTB_ERR_NULL;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v)) return PTB_ERR_ALIGN;
  // caches below 2^30 keys (256 GB of K per kv head): the kernels' key indices, ranges * steps * 32
  // included, stay within 32 bits
  if (nkv > 65535 || seq >= (int64_t(1) << 30) || nkv * seq * kD >= (int64_t(1) << 40)) return PTB_ERR_GRID;
  const size_t need = ptb_attn_decode_workspace_bytes(nkv, group, seq);
  if (need && (!workspace || workspace_bytes < need)) return PTB_ERR_WORKSPACE;
  if (need && !aligned16(workspace)) return PTB_ERR_ALIGN;
  const float c = scale * 1.4426950408889634f;
  auto qp = static_cast<const uint16_t*>(q), kp = static_cast<const uint16_t*>(k), vp = static_cast<const uint16_t*>(v);
  auto op = static_cast<uint16_t*>(o);
  float* ws = need ? static_cast<float*>(workspace) : nullptr;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (seq > kWaveMinSeq) {
    const WavePlan w = wave_plan(seq);
    switch (group) {
      case 1: launch_attn_decode_mfma<1>(qp, kp, vp, op, ws, int(nkv), int(seq), c, w, qn, s); break;
      case 2: launch_attn_decode_mfma<2>(qp, kp, vp, op, ws, int(nkv), int(seq), c, w, qn, s); break;
      case 3: launch_attn_decode_mfma<3>(qp, kp, vp, op, ws, int(nkv), int(seq), c, w, qn, s); break;
      case 4: launch_attn_decode_mfma<4>(qp, kp, vp, op, ws, int(nkv), int(seq), c, w, qn, s); break;
      case 6: launch_attn_decode_mfma<6>(qp, kp, vp, op, ws, int(nkv), int(seq), c, w, qn, s); break;
      default: launch_attn_decode_mfma<8>(qp, kp, vp, op, ws, int(nkv), int(seq), c, w, qn, s); break;
    }
    return launch_status();
  }
  switch (small_teams(seq)) {
    case 1: launch_attn_decode_small<1>(qp, kp, vp, op, int(nkv), int(group), int(seq), c, qn, s); break;
    case 2: launch_attn_decode_small<2>(qp, kp, vp, op, int(nkv), int(group), int(seq), c, qn, s); break;
    default: launch_attn_decode_small<4>(qp, kp, vp, op, int(nkv), int(group), int(seq), c, qn, s); break;
  }
  return launch_status();
}

PTB_EXPORT int ptb_attn_decode_bf16(const void* q, const void* k, const void* v, void* o, int64_t nkv, int64_t group,
                                    int64_t seq, int64_t head_dim, float scale, void* workspace,
                                    size_t workspace_bytes, void* stream) {
  return attn_decode_entry(q, k, v, o, nkv, group, seq, head_dim, scale, QNorm{nullptr, nullptr, nullptr, 0.f},
                           workspace, workspace_bytes, stream);
}

PTB_EXPORT int ptb_attn_decode_qnorm_rope_bf16(const void* q, const void* qnorm_w, const float* cos_t,
                                               const float* sin_t, float eps, const void* k, const void* v, void* o,
                                               int64_t nkv, int64_t group, int64_t seq, int64_t head_dim, float scale,
                                               void* workspace, size_t workspace_bytes, void* stream) {
  if (!qnorm_w || !cos_t || !sin_t) return PTB_ERR_NULL;
  if (!aligned16(qnorm_w) || !aligned16(cos_t) || !aligned16(sin_t)) return PTB_ERR_ALIGN;
  return attn_decode_entry(q, k, v, o, nkv, group, seq, head_dim, scale,
                           QNorm{static_cast<const uint16_t*>(qnorm_w), cos_t, sin_t, eps}, workspace,
                           workspace_bytes, stream);
}

// ---- allocation-free decode attention
// For callers that cannot allocate (code under HIP graph capture, serving loops that forbid
// hipMalloc): the partial records live in a file-scope device array instead of a caller workspace.
// Each GPU the library runs on holds its own copy of the array until the process ends; its address is
// looked up once per device (hipGetSymbolAddress, with that device current) and kept.  Every call on a
// GPU shares that GPU's array, so calls that overlap on one GPU race; nothing in it has to start at
// zero (each record is written before the merge pass reads it).
constexpr size_t kScratchBytes = size_t(16) << 20;   // 16 MiB: the records of up to 62 kv heads of 8 query rows at any cache length (at most 64 a head)
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices] = {};

int device_scratch(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return int(e);
  if (dev < 0 || dev >= kMaxScratchDevices) return PTB_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return int(e);
    if (!p) return PTB_ERR_NULL;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return PTB_OK;
}
}  // namespace

PTB_EXPORT size_t ptb_attn_decode_noalloc_max_bytes(void) { return kScratchBytes; }

PTB_EXPORT int ptb_attn_decode_bf16_noalloc(const void* q, const void* k, const void* v, void* o, int64_t nkv,
                                            int64_t group, int64_t seq, int64_t head_dim, float scale, void* stream) {
  const size_t need = ptb_attn_decode_workspace_bytes(nkv, group, seq);
  if (need > kScratchBytes) return PTB_ERR_WORKSPACE;   // past the static scratch's size
  void* ws = nullptr;
  if (need) {
    const int st = device_scratch(&ws);
    if (st != PTB_OK) return st;
  }
  return attn_decode_entry(q, k, v, o, nkv, group, seq, head_dim, scale, QNorm{nullptr, nullptr, nullptr, 0.f}, ws,
                           need ? kScratchBytes : 0, stream);
}

PTB_EXPORT size_t ptb_grouped_gemm_workspace_bytes(int64_t nprog, int64_t a_rows, int64_t k, int64_t n) {
  if (nprog <= 0 || a_rows <= 0 || a_rows > kGgMaxRows || k <= 0 || n < 8 || nprog > 65535) return 0;
  const int64_t splits = (k + kGgKb - 1) / kGgKb;
  return size_t(nprog * splits * a_rows * n) * sizeof(float);
}

PTB_EXPORT int ptb_grouped_gemm_bf16_ws(const void* a, const void* b, const int32_t* group, const int32_t* start,
                                        const int32_t* rows, void* c, int64_t nprog, int64_t ntab, int64_t a_rows,
                                        int64_t nweights, int64_t k, int64_t n, int64_t weight_stride,
                                        void* workspace, size_t workspace_bytes, void* stream) {
  const size_t need = ptb_grouped_gemm_workspace_bytes(nprog, a_rows, k, n);
  // the MFMA path for more rows (or no workspace); it also owns the argument checks below
  if (need == 0 || !workspace || workspace_bytes < need || (reinterpret_cast<uintptr_t>(workspace) & 15u))
    return ptb_grouped_gemm_bf16(a, b, group, start, rows, c, nprog, ntab, a_rows, nweights, k, n, weight_stride,
                                 stream);
  if (ntab < 0 || nweights < 0) return PTB_ERR_SHAPE;
  if (!a || !b || !group || !start || !rows || !c) return PTB_ERR_NULL;
  if (k % 64 || n % 8 || nprog > 256) return PTB_ERR_UNSUPPORTED;
  if (weight_stride < k * n || ntab > 0x7fffffff || nweights > 0x7fffffff || k > 0x7fffffff || n > 0x7fffffff)
    return PTB_ERR_SHAPE;
  if (!aligned16(a) || !aligned16(b) || !aligned16(c) || (weight_stride % 8)) return PTB_ERR_ALIGN;
  const int splits = int((k + kGgKb - 1) / kGgKb);
  if (splits > 65535) return PTB_ERR_GRID;
  hipStream_t s = static_cast<hipStream_t>(stream);
  float* part = static_cast<float*>(workspace);
  ggemv_partial<<<dim3(unsigned((n + kColBlock - 1) / kColBlock), unsigned(splits), unsigned(nprog)),
                  dim3(kGemvThreads), 0, s>>>(static_cast<const uint16_t*>(a), static_cast<const uint16_t*>(b), group,
                                              start, rows, int(ntab), int(nweights), int(a_rows), weight_stride, int(k),
                                              int(n), splits, part);
  ggemv_finish<<<dim3(unsigned((n + kGgFinCols - 1) / kGgFinCols), unsigned(nprog)), dim3(256), 0, s>>>(
      part, group, start, rows, int(ntab), int(nweights), int(a_rows), splits, int(n), static_cast<uint16_t*>(c));
  return launch_status();
}
