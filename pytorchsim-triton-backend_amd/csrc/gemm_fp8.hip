// fp8 (OCP e4m3fn) weight GEMM on gfx950 plus its quantisers.
//
//   quant_rows   : per-row (per-token) dynamic quantisation of bf16 activations, scale = absmax/448
//   quant_weight : per-output-channel quantisation of an fp32 weight W[K,N], packed transposed as
//                  Wt[N,K] (K contiguous), which is how the GEMM streams it
//   gemm_fp8     : C[m,n] = bf16( (sum_k Aq[m,k] * Wt[n,k]) * sa[m] * sw[n] ), fp32 accumulation
//
// The GEMM uses v_mfma_f32_32x32x64_f8f6f4 (both operands e4m3, no block scales): a 256x256
// workgroup tile, K step 128, 4 waves of 128x128 (4x4 accumulators of 32x32).  Both operands are
// K-contiguous rows, so each stage is a plain copy into LDS (rows padded 128 -> 144 B, conflict-free
// 2 x 128-bit fragment reads); stages are double-buffered with one barrier per K step.
#include "ptb_common.h"

using namespace ptb;

namespace {

constexpr int BM = 256, BN = 256, BK = 128;  // BK in bytes (= fp8 elements)
constexpr int LDB = BK + 16;                 // padded LDS row, bytes
constexpr int kThreads = 256;
constexpr int kStageBytes = (BM + BN) * LDB;
constexpr int kGroupM = 8;

struct Slice {
  u32x4 a[8];
  u32x4 w[8];
};

__device__ __forceinline__ Slice gload(const uint8_t* const (&a_src)[8], const uint8_t* const (&w_src)[8], int k0) {
  Slice s;
#pragma unroll
  for (int p = 0; p < 8; ++p) s.a[p] = *reinterpret_cast<const u32x4*>(a_src[p] + k0);
#pragma unroll
  for (int p = 0; p < 8; ++p) s.w[p] = *reinterpret_cast<const u32x4*>(w_src[p] + k0);
  return s;
}

__device__ __forceinline__ void sstore(const Slice& s, uint8_t* a_dst, uint8_t* w_dst, int st) {
#pragma unroll
  for (int p = 0; p < 8; ++p) *reinterpret_cast<u32x4*>(a_dst + st * kStageBytes + p * 32 * LDB) = s.a[p];
#pragma unroll
  for (int p = 0; p < 8; ++p) *reinterpret_cast<u32x4*>(w_dst + st * kStageBytes + p * 32 * LDB) = s.w[p];
}

__device__ __forceinline__ i32x8 frag(const uint8_t* p) {
  const u32x4 lo = *reinterpret_cast<const u32x4*>(p);
  const u32x4 hi = *reinterpret_cast<const u32x4*>(p + 16);
  return i32x8{int(lo[0]), int(lo[1]), int(lo[2]), int(lo[3]), int(hi[0]), int(hi[1]), int(hi[2]), int(hi[3])};
}

__global__ __launch_bounds__(kThreads, 1) void gemm_fp8_kernel(
    const uint8_t* __restrict__ A, const float* __restrict__ SA, const uint8_t* __restrict__ W,
    const float* __restrict__ SW, uint16_t* __restrict__ C, int M, int N, int K, int tiles_m, int tiles_n) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[2 * kStageBytes];

  const int ntiles = tiles_m * tiles_n;
  int pid = blockIdx.x;
  if ((ntiles & 7) == 0) pid = (pid & 7) * (ntiles >> 3) + (pid >> 3);
  const int width = kGroupM * tiles_n;
  const int first_m = (pid / width) * kGroupM;
  const int gsize = min(tiles_m - first_m, kGroupM);
  const int tm = first_m + (pid % width) % gsize;
  const int tn = (pid % width) / gsize;
  const int m0 = tm * BM, n0 = tn * BN;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  const int chunk = tid & 7, lrow = tid >> 3;
  const uint8_t* a_src[8];
  const uint8_t* w_src[8];
#pragma unroll
  for (int p = 0; p < 8; ++p) {
    a_src[p] = A + int64_t(min(m0 + p * 32 + lrow, M - 1)) * K + chunk * 16;
    w_src[p] = W + int64_t(min(n0 + p * 32 + lrow, N - 1)) * K + chunk * 16;
  }
  uint8_t* const a_dst = smem + lrow * LDB + chunk * 16;
  uint8_t* const w_dst = smem + BM * LDB + lrow * LDB + chunk * 16;

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  // lane -> row/col lane % 32, K half (32 bytes) lane / 32
  const int fr = lane & 31, fk = (lane >> 5) * 32;
  const int a_off = (wm * 128 + fr) * LDB + fk;
  const int w_off = BM * LDB + (wn * 128 + fr) * LDB + fk;

  const int nk = K / BK;
  sstore(gload(a_src, w_src, 0), a_dst, w_dst, 0);
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const uint8_t* st = smem + (kt & 1) * kStageBytes;
    const bool more = kt + 1 < nk;
    Slice nxt;
    if (more) nxt = gload(a_src, w_src, (kt + 1) * BK);
#pragma unroll
    for (int ks = 0; ks < BK / 64; ++ks) {
      i32x8 fa[4], fw[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        fa[i] = frag(st + a_off + i * 32 * LDB + ks * 64);
        fw[i] = frag(st + w_off + i * 32 * LDB + ks * 64);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fa[i], fw[j], acc[i][j], 0, 0, 0, 0, 0, 0);
    }
    if (more) sstore(nxt, a_dst, w_dst, (kt + 1) & 1);
    __syncthreads();
  }

#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int col = n0 + wn * 128 + j * 32 + fr;
    const float sw = SW[min(col, N - 1)];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm * 128 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (row < M && col < N) C[int64_t(row) * N + col] = f32_to_bf16((acc[i][j][r] * SA[row]) * sw);
      }
    }
  }
}

// ---- per-row activation quantiser: one wave per row for rows up to 64*8*VPT elements
constexpr int kQBlock = 256;
template <int VPT>
__global__ __launch_bounds__(kQBlock) void quant_rows_kernel(const uint16_t* __restrict__ x, uint8_t* __restrict__ xq,
                                                             float* __restrict__ scale, int64_t rows, int cols) {
  const int64_t row = int64_t(blockIdx.x) * (kQBlock / kWave) + threadIdx.x / kWave;
  const int l = threadIdx.x % kWave;
  if (row >= rows) return;  // whole wave leaves together
  const int chunks = cols >> 3;
  const u32x4* xr = reinterpret_cast<const u32x4*>(x + row * int64_t(cols));
  u32x4 v[VPT];
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int c = l + i * kWave;
    v[i] = c < chunks ? xr[c] : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int q = 0; q < 4; ++q) amax = fmaxf(amax, fmaxf(fabsf(bf16_lo(v[i][q])), fabsf(bf16_hi(v[i][q]))));
  }
  amax = wave_absmax(amax);
  const float s = amax > 0.f ? amax / 448.0f : 1.0f;
  if (l == 0) scale[row] = s;
  uint2* qr = reinterpret_cast<uint2*>(xq + row * int64_t(cols));
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int c = l + i * kWave;
    if (c >= chunks) continue;
    uint32_t o[2] = {0u, 0u};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t b0 = f32_to_e4m3(bf16_lo(v[i][q]) / s), b1 = f32_to_e4m3(bf16_hi(v[i][q]) / s);
      o[q >> 1] |= (b0 | (b1 << 8)) << (16 * (q & 1));
    }
    qr[c] = make_uint2(o[0], o[1]);
  }
}

// Long rows: one block per row, the row held in registers (VPT chunks per thread).
template <int VPT>
__global__ __launch_bounds__(kQBlock) void quant_rows_block(const uint16_t* __restrict__ x, uint8_t* __restrict__ xq,
                                                            float* __restrict__ scale, int cols) {
  __shared__ float red[kQBlock / kWave];
  const int64_t row = blockIdx.x;
  const int chunks = cols >> 3;
  const u32x4* xr = reinterpret_cast<const u32x4*>(x + row * int64_t(cols));
  u32x4 v[VPT];
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int c = threadIdx.x + i * kQBlock;
    v[i] = c < chunks ? xr[c] : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int q = 0; q < 4; ++q) amax = fmaxf(amax, fmaxf(fabsf(bf16_lo(v[i][q])), fabsf(bf16_hi(v[i][q]))));
  }
  amax = wave_absmax(amax);
  if (threadIdx.x % kWave == 0) red[threadIdx.x / kWave] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float s = amax > 0.f ? amax / 448.0f : 1.0f;
  if (threadIdx.x == 0) scale[row] = s;
  uint2* qr = reinterpret_cast<uint2*>(xq + row * int64_t(cols));
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int c = threadIdx.x + i * kQBlock;
    if (c >= chunks) continue;
    uint32_t o[2] = {0u, 0u};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t b0 = f32_to_e4m3(bf16_lo(v[i][q]) / s), b1 = f32_to_e4m3(bf16_hi(v[i][q]) / s);
      o[q >> 1] |= (b0 | (b1 << 8)) << (16 * (q & 1));
    }
    qr[c] = make_uint2(o[0], o[1]);
  }
}

// ---- per-output-channel weight quantiser
// absmax over K of each column j of W[K,N]: block = 64 columns x 4 K-slices.
__global__ __launch_bounds__(256) void weight_absmax(const float* __restrict__ w, float* __restrict__ scale,
                                                     int64_t K, int64_t N) {
  __shared__ float red[4][64];
  const int64_t j = int64_t(blockIdx.x) * 64 + (threadIdx.x & 63);
  const int slice = threadIdx.x >> 6;
  float amax = 0.f;
  if (j < N)
    for (int64_t i = slice; i < K; i += 4) amax = fmaxf(amax, fabsf(w[i * N + j]));
  red[slice][threadIdx.x & 63] = amax;
  __syncthreads();
  if (slice == 0 && j < N) {
    const float m = fmaxf(fmaxf(red[0][threadIdx.x], red[1][threadIdx.x]), fmaxf(red[2][threadIdx.x], red[3][threadIdx.x]));
    scale[j] = m > 0.f ? m / 448.0f : 1.0f;
  }
}

// quantise + transpose through a 64x64 LDS tile: read W[i0:i0+64, j0:j0+64] along j, write
// Wt[j0:j0+64, i0:i0+64] along i.
__global__ __launch_bounds__(256) void weight_quant_t(const float* __restrict__ w, const float* __restrict__ scale,
                                                      uint8_t* __restrict__ wt, int64_t K, int64_t N) {
  __shared__ uint8_t tile[64][65];
  const int64_t i0 = int64_t(blockIdx.y) * 64, j0 = int64_t(blockIdx.x) * 64;
  const int tj = threadIdx.x & 63, ti = threadIdx.x >> 6;
  const int64_t j = j0 + tj;
  const float s = j < N ? scale[j] : 1.0f;
  for (int r = ti; r < 64; r += 4) {
    const int64_t i = i0 + r;
    tile[r][tj] = (i < K && j < N) ? uint8_t(f32_to_e4m3(w[i * N + j] / s)) : uint8_t(0);
  }
  __syncthreads();
  for (int r = ti; r < 64; r += 4) {
    const int64_t jj = j0 + r, ii = i0 + tj;
    if (jj < N && ii < K) wt[jj * K + ii] = tile[tj][r];
  }
}

}  // namespace

PTB_EXPORT int ptb_quant_rows_e4m3(const void* x, void* xq, float* scale, int64_t rows, int64_t cols, void* stream) {
  if (rows < 0 || cols <= 0 || cols > (int64_t(1) << 30)) return PTB_ERR_SHAPE;
  if (rows == 0) return PTB_OK;
  if (!x || !xq || !scale) return PTB_ERR_NULL;
  if (cols % 8 || !aligned16(x) || (reinterpret_cast<uintptr_t>(xq) & 7u)) return PTB_ERR_ALIGN;
  if (cols > kQBlock * 16 * 8) return PTB_ERR_UNSUPPORTED;
  if (rows == 0) return PTB_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int chunks = int(cols / 8);
  const int64_t blocks = (rows + 3) / 4;
  if (blocks > 0x7fffffff) return PTB_ERR_GRID;
  const uint16_t* xi = static_cast<const uint16_t*>(x);
  uint8_t* qo = static_cast<uint8_t*>(xq);
  if (chunks <= 64 * 8) {
    if (chunks <= 64 * 2)
      quant_rows_kernel<2><<<dim3(unsigned(blocks)), dim3(kQBlock), 0, s>>>(xi, qo, scale, rows, int(cols));
    else if (chunks <= 64 * 4)
      quant_rows_kernel<4><<<dim3(unsigned(blocks)), dim3(kQBlock), 0, s>>>(xi, qo, scale, rows, int(cols));
    else
      quant_rows_kernel<8><<<dim3(unsigned(blocks)), dim3(kQBlock), 0, s>>>(xi, qo, scale, rows, int(cols));
  } else {
    if (rows > 0x7fffffff) return PTB_ERR_GRID;
    const dim3 g = dim3(unsigned(rows)), b = dim3(kQBlock);
    if (chunks <= kQBlock * 4) quant_rows_block<4><<<g, b, 0, s>>>(xi, qo, scale, int(cols));
    else if (chunks <= kQBlock * 6) quant_rows_block<6><<<g, b, 0, s>>>(xi, qo, scale, int(cols));
    else if (chunks <= kQBlock * 8) quant_rows_block<8><<<g, b, 0, s>>>(xi, qo, scale, int(cols));
    else if (chunks <= kQBlock * 16) quant_rows_block<16><<<g, b, 0, s>>>(xi, qo, scale, int(cols));
    else return PTB_ERR_UNSUPPORTED;
  }
  return launch_status();
}

PTB_EXPORT int ptb_quant_weight_e4m3(const float* w, void* wq_t, float* scale, int64_t k, int64_t n, void* stream) {
  if (!w || !wq_t || !scale) return PTB_ERR_NULL;
  if (k <= 0 || n <= 0) return PTB_ERR_SHAPE;
  const int64_t gx = (n + 63) / 64, gy = (k + 63) / 64;
  if (gx > 0x7fffffff || gy > 65535) return PTB_ERR_GRID;
  hipStream_t s = static_cast<hipStream_t>(stream);
  weight_absmax<<<dim3(unsigned(gx)), dim3(256), 0, s>>>(w, scale, k, n);
  weight_quant_t<<<dim3(unsigned(gx), unsigned(gy)), dim3(256), 0, s>>>(w, scale, static_cast<uint8_t*>(wq_t), k, n);
  return launch_status();
}

PTB_EXPORT int ptb_gemm_fp8_scaled(const void* aq, const float* sa, const void* wq_t, const float* sw, void* c,
                                   int64_t m, int64_t n, int64_t k, void* stream) {
  if (m < 0 || n < 0 || k < 0) return PTB_ERR_SHAPE;
  if (m == 0 || n == 0) return PTB_OK;
  if (!aq || !sa || !wq_t || !sw || !c) return PTB_ERR_NULL;
  if (k == 0) return PTB_ERR_UNSUPPORTED;
  if (m > 0x7fffffff || n > 0x7fffffff || k > 0x7fffffff) return PTB_ERR_SHAPE;
  if (k % BK || n % 16) return PTB_ERR_UNSUPPORTED;
  if (!aligned16(aq) || !aligned16(wq_t) || (reinterpret_cast<uintptr_t>(c) & 1u)) return PTB_ERR_ALIGN;
  const int64_t tm = (m + BM - 1) / BM, tn = (n + BN - 1) / BN;
  if (tm * tn > 0x7fffffff) return PTB_ERR_GRID;
  gemm_fp8_kernel<<<dim3(unsigned(tm * tn)), dim3(kThreads), 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint8_t*>(aq), sa, static_cast<const uint8_t*>(wq_t), sw, static_cast<uint16_t*>(c),
      int(m), int(n), int(k), int(tm), int(tn));
  return launch_status();
}
