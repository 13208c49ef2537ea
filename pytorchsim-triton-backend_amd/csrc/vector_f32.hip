// fp32 forms of the vector family for gfx950: RMSNorm over rows (and the column arm of the same
// reference case), row softmax, the SiLU gate, and the two-matmul SwiGLU block.  These serve the
// reference's own fp32 workload cases (tests/cases/workloads/{rmsnorm,softmax,swiglu}.py), which
// hold inputs and outputs in fp32 with tolerances down to rtol 1e-5: nothing is rounded below fp32.
// Rows move as 128-bit chunks of 4 floats with coalesced loads and stores; reductions are wave DPP /
// permlane steps plus one LDS pass across waves.
#include "ptb_common.h"

using namespace ptb;

namespace {

constexpr int kBlock = 256;

__device__ __forceinline__ float exp_e(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }

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

// ---------------------------------------------------------------- RMSNorm over rows
// A team of TPR threads per row, VPT chunks of 4 per thread held in registers (one read, one write).
template <int TPR, int VPT>
__global__ __launch_bounds__(kBlock) void rmsnorm_rows_f32(const float* __restrict__ x, const float* __restrict__ w,
                                                           float* __restrict__ y, int64_t rows, int cols, float eps) {
  __shared__ float red[kBlock / kWave];
  constexpr int kTeams = kBlock / TPR;
  const int team = threadIdx.x / TPR, lt = threadIdx.x % TPR;
  const int64_t row = int64_t(blockIdx.x) * kTeams + team;
  const bool live = row < rows;
  const int chunks = cols >> 2;
  const f32x4v* xr = reinterpret_cast<const f32x4v*>(x + (live ? row : 0) * int64_t(cols));
  f32x4v v[VPT];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int c = lt + i * TPR;
    v[i] = (live && c < chunks) ? xr[c] : f32x4v{0.f, 0.f, 0.f, 0.f};
    ss += v[i].x * v[i].x + v[i].y * v[i].y + v[i].z * v[i].z + v[i].w * v[i].w;
  }
  ss = team_sum<TPR>(ss, red);
  const float r = 1.0f / sqrtf(ss / float(cols) + eps);
  if (!live) return;
  f32x4v* yr = reinterpret_cast<f32x4v*>(y + row * int64_t(cols));
  const f32x4v* wr = reinterpret_cast<const f32x4v*>(w);
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int c = lt + i * TPR;
    if (c >= chunks) continue;
    const f32x4v wv = wr[c];
    yr[c] = f32x4v{(v[i].x * r) * wv.x, (v[i].y * r) * wv.y, (v[i].z * r) * wv.z, (v[i].w * r) * wv.w};
  }
}

// Rows too long for registers: one block per row, two passes over the row.
__global__ __launch_bounds__(kBlock) void rmsnorm_rows_f32_long(const float* __restrict__ x, const float* __restrict__ w,
                                                                float* __restrict__ y, int cols, float eps) {
  __shared__ float red[kBlock / kWave];
  const int64_t row = blockIdx.x;
  const int chunks = cols >> 2;
  const f32x4v* xr = reinterpret_cast<const f32x4v*>(x + row * int64_t(cols));
  float ss = 0.f;
  for (int c = threadIdx.x; c < chunks; c += kBlock) {
    const f32x4v a = xr[c];
    ss += a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w;
  }
  ss = block_sum<kBlock / kWave>(ss, red);
  const float r = 1.0f / sqrtf(ss / float(cols) + eps);
  f32x4v* yr = reinterpret_cast<f32x4v*>(y + row * int64_t(cols));
  const f32x4v* wr = reinterpret_cast<const f32x4v*>(w);
  for (int c = threadIdx.x; c < chunks; c += kBlock) {
    const f32x4v a = xr[c], wv = wr[c];
    yr[c] = f32x4v{(a.x * r) * wv.x, (a.y * r) * wv.y, (a.z * r) * wv.z, (a.w * r) * wv.w};
  }
}

// ---------------------------------------------------------------- column arm: rsqrt(mean_i x[i,j]^2 + eps)
// 64 columns per workgroup, its 4 waves splitting the rows; each lane walks its column.
__global__ __launch_bounds__(kBlock) void col_rms_f32(const float* __restrict__ x, float* __restrict__ c,
                                                      int64_t rows, int64_t cols, float eps) {
  __shared__ float part[4][64];
  const int64_t j = int64_t(blockIdx.x) * 64 + (threadIdx.x & 63);
  const int slice = threadIdx.x >> 6;
  float ss = 0.f;
  if (j < cols)
    for (int64_t i = slice; i < rows; i += 4) {
      const float v = x[i * cols + j];
      ss += v * v;
    }
  part[slice][threadIdx.x & 63] = ss;
  __syncthreads();
  if (slice == 0 && j < cols) {
    const float s = (part[0][threadIdx.x] + part[1][threadIdx.x]) + (part[2][threadIdx.x] + part[3][threadIdx.x]);
    c[j] = 1.0f / sqrtf(s / float(rows) + eps);
  }
}

// ---------------------------------------------------------------- row softmax
template <int TPR, int VPT>
__global__ __launch_bounds__(kBlock) void softmax_rows_f32(const float* __restrict__ x, float* __restrict__ y,
                                                           int64_t rows, int cols) {
  __shared__ float red[kBlock / kWave];
  constexpr int kTeams = kBlock / TPR;
  const int team = threadIdx.x / TPR, lt = threadIdx.x % TPR;
  const int64_t row = int64_t(blockIdx.x) * kTeams + team;
  const bool live = row < rows;
  const int chunks = cols >> 2;
  const f32x4v* xr = reinterpret_cast<const f32x4v*>(x + (live ? row : 0) * int64_t(cols));
  f32x4v v[VPT];
  float m = -__builtin_inff();
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int c = lt + i * TPR;
    const bool in = live && c < chunks;
    v[i] = in ? xr[c] : f32x4v{0.f, 0.f, 0.f, 0.f};
    if (in) m = max_nan(m, max_nan(max_nan(v[i].x, v[i].y), max_nan(v[i].z, v[i].w)));
  }
  m = team_max<TPR>(m, red);
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int c = lt + i * TPR;
    if (!(live && c < chunks)) continue;
    v[i] = f32x4v{exp_e(v[i].x - m), exp_e(v[i].y - m), exp_e(v[i].z - m), exp_e(v[i].w - m)};
    s += (v[i].x + v[i].y) + (v[i].z + v[i].w);
  }
  s = team_sum<TPR>(s, red);
  if (!live) return;
  f32x4v* yr = reinterpret_cast<f32x4v*>(y + row * int64_t(cols));
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int c = lt + i * TPR;
    if (c >= chunks) continue;
    yr[c] = f32x4v{v[i].x / s, v[i].y / s, v[i].z / s, v[i].w / s};
  }
}

// Long rows: one block per row, three passes over the row.
__global__ __launch_bounds__(kBlock) void softmax_rows_f32_long(const float* __restrict__ x, float* __restrict__ y,
                                                                int cols) {
  __shared__ float red[kBlock / kWave];
  const int64_t row = blockIdx.x;
  const int chunks = cols >> 2;
  const f32x4v* xr = reinterpret_cast<const f32x4v*>(x + row * int64_t(cols));
  float m = -__builtin_inff();
  for (int c = threadIdx.x; c < chunks; c += kBlock) {
    const f32x4v a = xr[c];
    m = max_nan(m, max_nan(max_nan(a.x, a.y), max_nan(a.z, a.w)));
  }
  m = block_max_nan<kBlock / kWave>(m, red);
  float s = 0.f;
  for (int c = threadIdx.x; c < chunks; c += kBlock) {
    const f32x4v a = xr[c];
    s += (exp_e(a.x - m) + exp_e(a.y - m)) + (exp_e(a.z - m) + exp_e(a.w - m));
  }
  s = block_sum<kBlock / kWave>(s, red);
  f32x4v* yr = reinterpret_cast<f32x4v*>(y + row * int64_t(cols));
  for (int c = threadIdx.x; c < chunks; c += kBlock) {
    const f32x4v a = xr[c];
    yr[c] = f32x4v{exp_e(a.x - m) / s, exp_e(a.y - m) / s, exp_e(a.z - m) / s, exp_e(a.w - m) / s};
  }
}

// ---------------------------------------------------------------- SiLU gate
// out[r, j] = (g / (1 + exp(-g))) * u, g = gu[r, j], u = gu[r, inter + j]; 4 outputs per thread.
__global__ __launch_bounds__(kBlock) void silu_mul_f32(const float* __restrict__ gu, float* __restrict__ out,
                                                       int64_t rows, int64_t inter) {
  const int64_t q = inter >> 2;   // chunks per row
  const int64_t total = rows * q;
  for (int64_t t = int64_t(blockIdx.x) * kBlock + threadIdx.x; t < total; t += int64_t(gridDim.x) * kBlock) {
    const int64_t r = t / q, c = t - r * q;
    const f32x4v g = reinterpret_cast<const f32x4v*>(gu + r * 2 * inter)[c];
    const f32x4v u = reinterpret_cast<const f32x4v*>(gu + r * 2 * inter + inter)[c];
    reinterpret_cast<f32x4v*>(out + r * inter)[c] =
        f32x4v{(g.x / (1.0f + exp_e(-g.x))) * u.x, (g.y / (1.0f + exp_e(-g.y))) * u.y,
               (g.z / (1.0f + exp_e(-g.z))) * u.z, (g.w / (1.0f + exp_e(-g.w))) * u.w};
  }
}

// ---------------------------------------------------------------- SwiGLU block
// o = silu(x @ wg) * (x @ wu) for fp32 x [M, K], wg / wu [K, N]: 64x64 output tiles, 256 threads each
// owning a 4x4 block of both products, K in steps of 16 through LDS.  fp32 FMA (the operands are
// fp32; the reference case checks at rtol 1e-3).
constexpr int kSwT = 64, kSwK = 16;
__global__ __launch_bounds__(kBlock) void swiglu_f32(const float* __restrict__ x, const float* __restrict__ wg,
                                                     const float* __restrict__ wu, float* __restrict__ o, int M,
                                                     int N, int K) {
  __shared__ float xs[kSwK][kSwT + 4];
  __shared__ float gs[kSwK][kSwT];
  __shared__ float us[kSwK][kSwT];
  const int m0 = blockIdx.y * kSwT, n0 = blockIdx.x * kSwT;
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  float ag[4][4] = {}, au[4][4] = {};
  for (int k0 = 0; k0 < K; k0 += kSwK) {
    // x tile [64 rows][16 k] stored k-major; wg/wu tiles [16 k][64 n]
    for (int e = threadIdx.x; e < kSwT * kSwK; e += kBlock) {
      const int r = e / kSwK, kk = e % kSwK;
      const int gm = m0 + r, gk = k0 + kk;
      xs[kk][r] = (gm < M && gk < K) ? x[int64_t(gm) * K + gk] : 0.f;
      const int kr = e / kSwT, nn = e % kSwT;
      const int gk2 = k0 + kr, gn = n0 + nn;
      const bool ok = gk2 < K && gn < N;
      gs[kr][nn] = ok ? wg[int64_t(gk2) * N + gn] : 0.f;
      us[kr][nn] = ok ? wu[int64_t(gk2) * N + gn] : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < kSwK; ++kk) {
      float a[4], bg[4], bu[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = xs[kk][ty * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        bg[j] = gs[kk][tx * 4 + j];
        bu[j] = us[kk][tx * 4 + j];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          ag[i][j] = fmaf(a[i], bg[j], ag[i][j]);
          au[i][j] = fmaf(a[i], bu[j], au[i][j]);
        }
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int gm = m0 + ty * 4 + i;
    if (gm >= M) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int gn = n0 + tx * 4 + j;
      if (gn < N) {
        const float g = ag[i][j];
        o[int64_t(gm) * N + gn] = (g / (1.0f + exp_e(-g))) * au[i][j];
      }
    }
  }
}

bool aligned_rows(const void* p, int64_t cols) { return aligned16(p) && cols % 4 == 0; }

}  // namespace

PTB_EXPORT int ptb_rmsnorm_f32(const float* x, const float* w, float* y, int64_t rows, int64_t cols, float eps,
                               void* stream) {
  if (rows < 0 || cols <= 0 || cols > (int64_t(1) << 30)) return PTB_ERR_SHAPE;
  if (rows == 0) return PTB_OK;
  if (!x || !w || !y) return PTB_ERR_NULL;
  if (!aligned_rows(x, cols) || !aligned16(w) || !aligned16(y)) return PTB_ERR_ALIGN;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int chunks = int(cols / 4);
  const int c = int(cols);
  if (chunks <= 64 * 8) {                      // one wave per row, 4 rows a block
    const int64_t blocks = (rows + 3) / 4;
    if (blocks > 0x7fffffff) return PTB_ERR_GRID;
    const dim3 g = dim3(unsigned(blocks)), b = dim3(kBlock);
    if (chunks <= 64 * 2) rmsnorm_rows_f32<64, 2><<<g, b, 0, s>>>(x, w, y, rows, c, eps);
    else if (chunks <= 64 * 4) rmsnorm_rows_f32<64, 4><<<g, b, 0, s>>>(x, w, y, rows, c, eps);
    else rmsnorm_rows_f32<64, 8><<<g, b, 0, s>>>(x, w, y, rows, c, eps);
  } else {
    if (rows > 0x7fffffff) return PTB_ERR_GRID;
    const dim3 g = dim3(unsigned(rows)), b = dim3(kBlock);
    if (chunks <= kBlock * 8) rmsnorm_rows_f32<kBlock, 8><<<g, b, 0, s>>>(x, w, y, rows, c, eps);
    else rmsnorm_rows_f32_long<<<g, b, 0, s>>>(x, w, y, c, eps);
  }
  return launch_status();
}

PTB_EXPORT int ptb_col_rms_f32(const float* x, float* c, int64_t rows, int64_t cols, float eps, void* stream) {
  if (rows <= 0 || cols < 0) return PTB_ERR_SHAPE;
  if (cols == 0) return PTB_OK;
  if (!x || !c) return PTB_ERR_NULL;
  const int64_t blocks = (cols + 63) / 64;
  if (blocks > 0x7fffffff) return PTB_ERR_GRID;
  col_rms_f32<<<dim3(unsigned(blocks)), dim3(kBlock), 0, static_cast<hipStream_t>(stream)>>>(x, c, rows, cols, eps);
  return launch_status();
}

PTB_EXPORT int ptb_softmax_rows_f32(const float* x, float* y, int64_t rows, int64_t cols, void* stream) {
  if (rows < 0 || cols <= 0 || cols > (int64_t(1) << 30)) return PTB_ERR_SHAPE;
  if (rows == 0) return PTB_OK;
  if (!x || !y) return PTB_ERR_NULL;
  if (!aligned_rows(x, cols) || !aligned16(y)) return PTB_ERR_ALIGN;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int chunks = int(cols / 4);
  const int c = int(cols);
  if (chunks <= 64 * 8) {
    const int64_t blocks = (rows + 3) / 4;
    if (blocks > 0x7fffffff) return PTB_ERR_GRID;
    const dim3 g = dim3(unsigned(blocks)), b = dim3(kBlock);
    if (chunks <= 64 * 2) softmax_rows_f32<64, 2><<<g, b, 0, s>>>(x, y, rows, c);
    else if (chunks <= 64 * 4) softmax_rows_f32<64, 4><<<g, b, 0, s>>>(x, y, rows, c);
    else softmax_rows_f32<64, 8><<<g, b, 0, s>>>(x, y, rows, c);
  } else {
    if (rows > 0x7fffffff) return PTB_ERR_GRID;
    const dim3 g = dim3(unsigned(rows)), b = dim3(kBlock);
    if (chunks <= kBlock * 8) softmax_rows_f32<kBlock, 8><<<g, b, 0, s>>>(x, y, rows, c);
    else softmax_rows_f32_long<<<g, b, 0, s>>>(x, y, c);
  }
  return launch_status();
}

PTB_EXPORT int ptb_silu_mul_f32(const float* gate_up, float* out, int64_t rows, int64_t inter, void* stream) {
  if (rows < 0 || inter <= 0) return PTB_ERR_SHAPE;
  if (rows == 0) return PTB_OK;
  if (!gate_up || !out) return PTB_ERR_NULL;
  if (inter % 4 || !aligned16(gate_up) || !aligned16(out)) return PTB_ERR_ALIGN;
  const int64_t total = rows * (inter / 4);
  const int64_t blocks = std::min<int64_t>((total + kBlock - 1) / kBlock, 65536);
  silu_mul_f32<<<dim3(unsigned(blocks)), dim3(kBlock), 0, static_cast<hipStream_t>(stream)>>>(gate_up, out, rows,
                                                                                              inter);
  return launch_status();
}

PTB_EXPORT int ptb_swiglu_f32(const float* x, const float* wg, const float* wu, float* o, int64_t m, int64_t n,
                              int64_t k, void* stream) {
  if (m < 0 || n < 0 || k < 0) return PTB_ERR_SHAPE;
  if (m == 0 || n == 0) return PTB_OK;
  if (!x || !wg || !wu || !o) return PTB_ERR_NULL;
  if (m > 0x7fffffff || n > 0x7fffffff || k > 0x7fffffff) return PTB_ERR_SHAPE;
  const int64_t gx = (n + kSwT - 1) / kSwT, gy = (m + kSwT - 1) / kSwT;
  if (gx > 0x7fffffff || gy > 65535) return PTB_ERR_GRID;
  swiglu_f32<<<dim3(unsigned(gx), unsigned(gy)), dim3(kBlock), 0, static_cast<hipStream_t>(stream)>>>(
      x, wg, wu, o, int(m), int(n), int(k));
  return launch_status();
}
