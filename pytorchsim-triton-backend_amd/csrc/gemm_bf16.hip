// bf16 GEMM on gfx950 matrix cores: C[M,N] = A[M,K] * B[K,N] (+ R[M,N]), all row-major, fp32
// accumulation, one bf16 rounding at the store.
//
// Workgroup tile 256x256, K step 32, 4 waves in a 2x2 arrangement, each wave owning a 128x128
// sub-tile as 4x4 v_mfma_f32_32x32x16_bf16 accumulators (256 fp32 per lane, held in AGPRs).
//
// Operands move HBM -> LDS with buffer_load_dwordx4 ... lds (no VGPR staging) into a ring of four
// 32 KB LDS stages, three K steps ahead of the matrix cores, so two to three microseconds of memory
// latency stay hidden behind MFMA work.  Each stage holds the A tile [256 rows][32 k] and the B tile
// [32 k][256 n] in their global layouts, with 16-byte chunks XOR-swizzled per row so that every LDS
// read below is bank-conflict free:
//   A fragments (8 consecutive k of one row per lane) are plain 128-bit LDS reads;
//   B fragments (8 consecutive k of one column per lane, while B is N-contiguous) come from two
//   ds_read_b64_tr_b16 transposing reads: within each 16-lane group, lane 4j+q supplies row k+j,
//   columns n+4q..n+4q+3, and lane i receives rows k..k+3 of column n+i.
// Swizzles: A row m keeps chunk c in slot c ^ ((m >> 2) & 3); B row k keeps chunk c in slot
// c ^ (4 * (k & 3)), so the 4 rows x 4 chunks a half-wave reads land in 16 distinct bank groups.
// The fragments of the next 16-wide K slice are always read while the MFMAs of the current one
// run (the last slice of a step reads the first slice of the next stage, behind the barrier that
// publishes it), so LDS latency stays off the matrix cores' critical path.
// The MFMA is issued with B as its first operand, so each accumulator holds a 32x32 block of C^T:
// a lane's four consecutive registers are four consecutive columns of one row of C, stored (with
// the residual read) as one 8-byte access.
//
// Tile order is XCD-aware: hardware hands workgroup i to XCD i % 8, so ids are remapped to give
// each XCD a contiguous range of tiles, walked in groups of 8 tile-rows for L2 reuse.
#include "ptb_common.h"

using namespace ptb;



namespace {

constexpr int BM = 256, BN = 256, BK = 32;
constexpr int kThreads = 256;
#ifndef PTB_GEMM_STAGES
#define PTB_GEMM_STAGES 4
#endif
constexpr int kStages = PTB_GEMM_STAGES;  // LDS ring depth, 3..5 (32 KB each of the 160 KB)
static_assert(kStages >= 3 && kStages <= 5, "LDS ring of 3 to 5 stages");
constexpr int kABytes = BM * BK * 2;           // 16 KB: 256 rows x 64 B
constexpr int kBBytes = BK * BN * 2;           // 16 KB: 32 rows x 512 B
constexpr int kStageBytes = kABytes + kBBytes;  // 32 KB
constexpr int kGroupM = 8;
constexpr int kDmaPerStage = 8;                // buffer_load ... lds per wave per stage

typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

template <bool RESID>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1))) void gemm_bf16_kernel(
    const uint16_t* __restrict__ A, const uint16_t* __restrict__ B, const uint16_t* __restrict__ R,
    uint16_t* __restrict__ C, int M, int N, int K, int tiles_m, int tiles_n) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[kStages * kStageBytes];

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

  // ---- loaders: A tile rows past M read as zero (num_records); B columns past N are read from
  //      the next row or as zero, and only feed columns of C that are never stored
  const i32x4 rsrc_a = make_rsrc(A + int64_t(m0) * K, uint32_t(min(BM, M - m0)) * uint32_t(K) * 2u);
  const i32x4 rsrc_b = make_rsrc(B + n0, uint32_t((int64_t(K) * N - n0) * 2));
  // A: instruction t of this wave covers rows (4*wave+t)*16 .. +16; lane -> row l/4, slot l%4
  uint32_t a_voff[4], b_voff[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int row = (wave * 4 + t) * 16 + (lane >> 2);
    const int chunk = (lane & 3) ^ ((row >> 2) & 3);
    a_voff[t] = uint32_t(row * K + chunk * 8) * 2u;
    // B: instruction t covers k rows 2*(4*wave+t) + lane/32; lane -> slot lane%32
    const int k = 2 * (wave * 4 + t) + (lane >> 5);
    const int bchunk = (lane & 31) ^ (4 * (k & 3));
    b_voff[t] = uint32_t(k * N + bchunk * 8) * 2u;
  }
  const uint32_t lds0 = uint32_t(reinterpret_cast<uintptr_t>(smem));
  auto issue_stage = [&](int kt) {
    const uint32_t st = lds0 + uint32_t(kt % kStages) * kStageBytes;
    const uint32_t a_soff = uint32_t(kt * BK) * 2u;
    const uint32_t b_soff = uint32_t(kt * BK) * uint32_t(N) * 2u;
#pragma unroll
    for (int t = 0; t < 4; ++t)
      dma16(rsrc_a, __builtin_amdgcn_readfirstlane(st + (wave * 4 + t) * 1024), a_voff[t], a_soff);
#pragma unroll
    for (int t = 0; t < 4; ++t)
      dma16(rsrc_b, __builtin_amdgcn_readfirstlane(st + kABytes + (wave * 4 + t) * 1024), b_voff[t], b_soff);
  };

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  // ---- fragment addressing
  const int fr = lane & 31, h = lane >> 5;
  // A: row m (this lane's), chunk 2*ks + h, swizzled by (m >> 2) & 3
  int a_row_off[4], a_sw[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = wm * 128 + i * 32 + fr;
    a_row_off[i] = m * 64;
    a_sw[i] = (m >> 2) & 3;
  }
  // B (transposing reads): group g = lane/16 -> k half g/2, column half 16*(g%2); in-group lane
  // 4*jj + q supplies row 8h + 4r + jj (+16 ks), columns +4q..+4q+3
  const int g16 = (lane >> 4) & 1, l16 = lane & 15, jj = l16 >> 2, q = l16 & 3;
  int b_off[4][2];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int n = wn * 128 + j * 32 + 16 * g16 + 4 * q;
    const int chunk = n >> 3;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int k = 8 * h + 4 * r + jj;  // + 16*ks, which keeps k & 3
      b_off[j][r] = kABytes + k * 512 + ((chunk ^ (4 * (k & 3))) << 4) + (q & 1) * 8;
    }
  }

  // One K slice's fragments, read in 12 pieces (4 A reads, 8 B half-reads) so that the reads can
  // be spread between MFMAs.
  struct Slice {
    bf16x8 a[4];
    bf16x8 b[4];
    i16x4 blo[4];
  };
  auto read_piece = [&](const uint8_t* st, int ks, int p, Slice& f) {
    if (p < 4) {
      f.a[p] = *reinterpret_cast<const bf16x8*>(st + a_row_off[p] + (((2 * ks + h) ^ a_sw[p]) << 4));
    } else {
      const int j = (p - 4) >> 1, r = (p - 4) & 1;
      const i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(st + b_off[j][r] + ks * 16 * 512));
      if (r == 0) f.blo[j] = v;
      else f.b[j] = __builtin_bit_cast(bf16x8, i16x8{f.blo[j][0], f.blo[j][1], f.blo[j][2], f.blo[j][3], v[0], v[1], v[2], v[3]});
    }
  };
  auto mfma_one = [&](const Slice& f, int u) {
    const int i = u >> 2, j = u & 3;
    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.b[j], f.a[i], acc[i][j], 0, 0, 0);
  };
  // t-th of this wave's 8 DMA instructions of stage kt (4 for A, then 4 for B)
  auto dma_one = [&](int kt, int t) {
    const uint32_t st = lds0 + uint32_t(kt % kStages) * kStageBytes;
    if (t < 4)
      dma16(rsrc_a, __builtin_amdgcn_readfirstlane(st + (wave * 4 + t) * 1024), a_voff[t], uint32_t(kt * BK) * 2u);
    else
      dma16(rsrc_b, __builtin_amdgcn_readfirstlane(st + kABytes + (wave * 4 + t - 4) * 1024), b_voff[t - 4],
            uint32_t(kt * BK) * uint32_t(N) * 2u);
  };

  // The DMA stream runs kStages-1 stages ahead of the MFMAs and does not stop at the last K step:
  // stages past the end read zeros (num_records) into slots nobody reads any more, which keeps the
  // loop free of branches; everything is drained before the epilogue.
  const int nk = K / BK;
  for (int s = 0; s < kStages - 1; ++s) issue_stage(s);
  wait_vmcnt<(kStages - 2) * kDmaPerStage>();  // stage 0 landed (this wave's part)
  __syncthreads();                              // ... and everyone's
  Slice s0, s1;
#pragma unroll
  for (int p = 0; p < 12; ++p) read_piece(smem, 0, p, s0);

  // Each K step: slice 0's MFMAs with slice 1's reads folded in; the barrier publishing stage kt+1;
  // slice 1's MFMAs with the DMA of stage kt+3 and the reads of stage kt+1's slice 0 folded in.
  // sched_barrier(0) pins that interleave, so the matrix core is fed between memory instructions.
  for (int kt = 0; kt < nk; ++kt) {
    const uint8_t* st = smem + (kt % kStages) * kStageBytes;
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      mfma_one(s0, u);
      if (u < 12) read_piece(st, 1, u, s1);
      __builtin_amdgcn_sched_barrier(0);
    }
    // stage kt+1 landed; past this barrier no wave reads stage kt-1's slot, which takes kt+3
    wait_vmcnt<(kStages - 3) * kDmaPerStage>();
    __syncthreads();
    const uint8_t* nst = smem + ((kt + 1) % kStages) * kStageBytes;
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      mfma_one(s1, u);
      if (u < 8) dma_one(kt + kStages - 1, u);
      if (u >= 1 && u < 13) read_piece(nst, 0, u - 1, s0);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  wait_vmcnt<0>();

  // ---- epilogue: accumulator (i, j, r) of lane -> C row m0 + wm*128 + i*32 + lane%32,
  //      column n0 + wn*128 + j*32 + 8*(r/4) + 4*(lane/32) + r%4: 4 consecutive columns per r/4
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = m0 + wm * 128 + i * 32 + fr;
    if (row >= M) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int col = n0 + wn * 128 + j * 32 + 8 * g + 4 * h;
        if (col >= N) continue;  // N % 8 == 0: a 4-column group is all in or all out
        const int64_t o = int64_t(row) * N + col;
        float v0 = acc[i][j][4 * g], v1 = acc[i][j][4 * g + 1], v2 = acc[i][j][4 * g + 2], v3 = acc[i][j][4 * g + 3];
        if constexpr (RESID) {
          const u32x2 rr = *reinterpret_cast<const u32x2*>(R + o);
          v0 += bf16_lo(rr[0]);
          v1 += bf16_hi(rr[0]);
          v2 += bf16_lo(rr[1]);
          v3 += bf16_hi(rr[1]);
        }
        *reinterpret_cast<u32x2*>(C + o) = u32x2{pack_bf16x2(v0, v1), pack_bf16x2(v2, v3)};
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
  if (k % 64 || n % 8) return PTB_ERR_UNSUPPORTED;
  // buffer offsets are 32-bit: B and one 256-row panel of A must each stay under 4 GB
  if ((k + kStages * BK) * n * 2 >= (int64_t(1) << 32) || int64_t(BM) * k * 2 >= (int64_t(1) << 32))
    return PTB_ERR_UNSUPPORTED;
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
