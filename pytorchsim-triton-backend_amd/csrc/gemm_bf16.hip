// bf16 GEMM on gfx950 matrix cores: C[M,N] = A[M,K] * B[K,N] (+ R[M,N]), all row-major, fp32
// accumulation, one bf16 rounding at the store.
//
// Workgroup tile 256x256, K step 64, 4 waves in a 2x2 arrangement, each wave owning a 128x128
// sub-tile as 4x4 v_mfma_f32_32x32x16_bf16 accumulators (256 fp32 per lane, held in AGPRs).
// Both operands are staged through LDS, double-buffered (2 x 72 KB of the 160 KB), with one barrier
// per K step: while the matrix cores work on stage s, the next K slice is already in flight from
// HBM into registers and is written to stage s^1 afterwards.
//
// MFMA wants every lane to hold 8 consecutive K values of one row (A) or one column (B).  A rows
// are K-contiguous already; B is N-contiguous, so each thread loads an 8(K) x 8(N) block of B with
// eight 128-bit loads and transposes it in registers (v_perm) before the 128-bit LDS stores.  LDS
// rows are padded to 72 elements (144 B), which makes both the fragment reads and the stores
// bank-conflict free.
//
// Tile order is XCD-aware: hardware hands workgroup i to XCD i % 8, so ids are remapped to give
// each XCD a contiguous range of tiles, walked in groups of 8 tile-rows for L2 reuse of B panels.
#include "ptb_common.h"

using namespace ptb;

namespace {

constexpr int BM = 256, BN = 256, BK = 64;
constexpr int LDK = BK + 8;                  // padded LDS row, bf16 elements
constexpr int kThreads = 256;
constexpr int kStageElems = (BM + BN) * LDK;  // one stage: A tile then transposed B tile
constexpr int kGroupM = 8;

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Column C of an 8x8 bf16 block held as 8 row vectors: 8 K-consecutive values of one column.
template <int C>
__device__ __forceinline__ u32x4 column(const u32x4 (&r)[8]) {
  u32x4 o;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint32_t lo = r[2 * q][C / 2], hi = r[2 * q + 1][C / 2];
    o[q] = (C % 2 == 0) ? ((lo & 0xffffu) | (hi << 16)) : ((lo >> 16) | (hi & 0xffff0000u));
  }
  return o;
}

template <int C>
__device__ __forceinline__ void store_columns(uint16_t* bs, const u32x4 (&r)[8]) {
  *reinterpret_cast<u32x4*>(bs + C * LDK) = column<C>(r);
  if constexpr (C + 1 < 8) store_columns<C + 1>(bs, r);
}

// One K slice of this thread's share: 8 A chunks (8 rows) and an 8x8 block of B.
struct Slice {
  u32x4 a[8];
  u32x4 b[8];
};

__device__ __forceinline__ Slice gload(const uint16_t* const (&a_src)[8], const uint16_t* b_src, int N,
                                       int k0) {
  Slice s;
#pragma unroll
  for (int p = 0; p < 8; ++p) s.a[p] = *reinterpret_cast<const u32x4*>(a_src[p] + k0);
#pragma unroll
  for (int p = 0; p < 8; ++p) s.b[p] = *reinterpret_cast<const u32x4*>(b_src + int64_t(k0 + p) * N);
  return s;
}

__device__ __forceinline__ void sstore(const Slice& s, uint16_t* a_dst, uint16_t* b_dst, int st) {
#pragma unroll
  for (int p = 0; p < 8; ++p) *reinterpret_cast<u32x4*>(a_dst + st * kStageElems + p * 32 * LDK) = s.a[p];
  store_columns<0>(b_dst + st * kStageElems, s.b);
}

template <bool RESID>
__global__ __launch_bounds__(kThreads, 1) void gemm_bf16_kernel(
    const uint16_t* __restrict__ A, const uint16_t* __restrict__ B, const uint16_t* __restrict__ R,
    uint16_t* __restrict__ C, int M, int N, int K, int tiles_m, int tiles_n) {
  __shared__ __attribute__((aligned(16))) uint16_t smem[2 * kStageElems];

  // ---- tile selection
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

  // ---- global -> register loaders (rows/cols past the edge are clamped; their results are
  //      never stored)
  const int a_chunk = tid & 7, a_row = tid >> 3;  // A: 8 chunks of 8 per 64-wide K row, 32 rows/pass
  const uint16_t* a_src[8];
#pragma unroll
  for (int p = 0; p < 8; ++p) a_src[p] = A + int64_t(min(m0 + p * 32 + a_row, M - 1)) * K + a_chunk * 8;
  const int b_kb = tid & 7, b_nb = tid >> 3;      // B: 8x8 block (k-block b_kb, n-block b_nb)
  const int b_n = min(n0 + b_nb * 8, N - 8);
  const uint16_t* b_src = B + int64_t(b_kb * 8) * N + b_n;
  uint16_t* const a_dst = smem + a_row * LDK + a_chunk * 8;
  uint16_t* const b_dst = smem + BM * LDK + (b_nb * 8) * LDK + b_kb * 8;

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  // fragment addressing: lane -> row/col (lane % 32), K half (lane / 32)
  const int fr = lane & 31, fk = (lane >> 5) * 8;
  const int a_off = (wm * 128 + fr) * LDK + fk;
  const int b_off = BM * LDK + (wn * 128 + fr) * LDK + fk;

  const int nk = K / BK;
  sstore(gload(a_src, b_src, N, 0), a_dst, b_dst, 0);
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const uint16_t* st = smem + (kt & 1) * kStageElems;
    const bool more = kt + 1 < nk;
    Slice nxt;
    if (more) nxt = gload(a_src, b_src, N, (kt + 1) * BK);
    bf16x8 fa[2][4], fb[2][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      fa[0][i] = *reinterpret_cast<const bf16x8*>(st + a_off + i * 32 * LDK);
      fb[0][i] = *reinterpret_cast<const bf16x8*>(st + b_off + i * 32 * LDK);
    }
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      const int cb = ks & 1;
      if (ks + 1 < BK / 16) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          fa[cb ^ 1][i] = *reinterpret_cast<const bf16x8*>(st + a_off + i * 32 * LDK + (ks + 1) * 16);
          fb[cb ^ 1][i] = *reinterpret_cast<const bf16x8*>(st + b_off + i * 32 * LDK + (ks + 1) * 16);
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[cb][i], fb[cb][j], acc[i][j], 0, 0, 0);
    }
    if (more) sstore(nxt, a_dst, b_dst, (kt + 1) & 1);
    __syncthreads();
  }

  // ---- epilogue: accumulator (i, j, r) of lane -> row 8*(r/4) + 4*(lane/32) + r%4, col lane%32
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int col = n0 + wn * 128 + j * 32 + fr;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm * 128 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (row < M && col < N) {
          const int64_t o = int64_t(row) * N + col;
          float v = acc[i][j][r];
          if constexpr (RESID) v = v + bf16_to_f32(R[o]);
          C[o] = f32_to_bf16(v);
        }
      }
    }
  }
}

}  // namespace

PTB_EXPORT int ptb_gemm_bf16(const void* a, const void* b, const void* residual, void* c, int64_t m,
                             int64_t n, int64_t k, void* stream) {
  if (m < 0 || n < 0 || k < 0) return PTB_ERR_SHAPE;
  if (m == 0 || n == 0) return PTB_OK;
  if (!a || !b || !c) return PTB_ERR_NULL;
  if (k == 0) return PTB_ERR_UNSUPPORTED;
  if (m > 0x7fffffff || n > 0x7fffffff || k > 0x7fffffff) return PTB_ERR_SHAPE;
  if (k % BK || n % 8) return PTB_ERR_UNSUPPORTED;
  if (!aligned16(a) || !aligned16(b) || !aligned16(c) || (residual && !aligned16(residual)))
    return PTB_ERR_ALIGN;
  const int64_t tm = (m + BM - 1) / BM, tn = (n + BN - 1) / BN;
  if (tm * tn > 0x7fffffff) return PTB_ERR_GRID;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(unsigned(tm * tn)), block(kThreads);
  if (residual)
    gemm_bf16_kernel<true><<<grid, block, 0, s>>>(static_cast<const uint16_t*>(a), static_cast<const uint16_t*>(b),
                                                   static_cast<const uint16_t*>(residual), static_cast<uint16_t*>(c),
                                                   int(m), int(n), int(k), int(tm), int(tn));
  else
    gemm_bf16_kernel<false><<<grid, block, 0, s>>>(static_cast<const uint16_t*>(a), static_cast<const uint16_t*>(b),
                                                    nullptr, static_cast<uint16_t*>(c), int(m), int(n), int(k),
                                                    int(tm), int(tn));
  return launch_status();
}
