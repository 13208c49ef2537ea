// fp8 (OCP e4m3fn) weight GEMM on gfx950 plus its quantisers.
//
//   quant_rows   : per-row (per-token) dynamic quantisation of bf16 activations, scale = absmax/448
//   quant_weight : per-output-channel quantisation of an fp32 weight W[K,N], packed transposed as
//                  Wt[N,K] (K contiguous), which is how the GEMM streams it
//   gemm_fp8     : C[m,n] = bf16( (sum_k Aq[m,k] * Wt[n,k]) * sa[m] * sw[n] ), fp32 accumulation
//
// The GEMM uses v_mfma_f32_32x32x64_f8f6f4 (both operands e4m3, no block scales): a 256xBN
// workgroup tile (BN = 256, or 128 when 256x256 tiles would leave CUs idle), 4 waves in a 2x2
// arrangement, each wave 128 x BN/2 as 32x32 accumulators.  Both operands are K-contiguous; a stage
// holds 128 bytes (= 128 K) of every tile row, so each row's DMA is one whole 128-byte line and the
// L2 serves one request per line (a 64-byte stage row costs the L2 a request slot for half a line:
// the request rate, not the bytes, bounded the 64-byte form).  Operands move HBM -> LDS with
// buffer_load_dwordx4 ... lds into a ring of NS stages (3 x 48 KB at BN = 128, 2 x 64 KB at
// BN = 256).  Within a row the eight 16-byte chunks sit XOR-swizzled by (row >> 1) & 7, so the
// 128-bit fragment reads (16 lanes a phase, 16 different rows) are bank-conflict free.  A stage is
// two MFMA K substeps of 64: substep 0's MFMAs run with substep 1's fragment reads folded in; the
// barrier that follows publishes the next stage and frees this one; substep 1's MFMAs then run with
// the reads of the next stage's substep 0.  The refill DMAs of a three-stage ring go into the slot
// the previous step freed and spread over both substeps (bunched into one substep they queue in the
// address unit and stall the MFMAs: config 4 85 -> 82 us); a two-stage ring refills the slot its
// own barrier frees, during substep 1.  MFMAs take W as the first operand, so accumulators hold C^T blocks and each lane
// stores 4 consecutive columns of a row of C at once.
#include <algorithm>
#include <type_traits>

#include "ptb_common.h"

using namespace ptb;

namespace {

constexpr int BM = 256, BK = 128;   // BK in bytes (= fp8 elements) per stage
constexpr int kThreads = 256;

typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

template <int BN>
struct Cfg {
  static constexpr int NS = BN == 256 ? 2 : 3;         // LDS ring depth
  static constexpr int WNT = BN / 64;                  // 32-wide column tiles per wave
  static constexpr int kABytes = BM * BK;              // 32 KB
  static constexpr int kWBytes = BN * BK;
  static constexpr int kStageBytes = kABytes + kWBytes;
  static constexpr int kDmaA = BM / 8 / 4;             // DMA instructions per wave per stage (8 rows each)
  static constexpr int kDmaW = BN / 8 / 4;
  static constexpr int kDma = kDmaA + kDmaW;
  static constexpr int kPieces = 2 * (4 + WNT);        // 128-bit fragment reads per wave per substep
  static constexpr int kMfma = 4 * WNT;                // MFMAs per wave per substep
};

template <int BN>
struct Frags {
  i32x8 a[4];
  i32x8 w[Cfg<BN>::WNT];
  u32x4 lo[4 + Cfg<BN>::WNT];
};

__device__ __forceinline__ int fp8_swz(int row) { return (row >> 1) & 7; }

template <int BN>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1))) void gemm_fp8_kernel(
    const uint8_t* __restrict__ A, const float* __restrict__ SA, const uint8_t* __restrict__ W,
    const float* __restrict__ SW, uint16_t* __restrict__ C, int M, int N, int K, int tiles_m, int tiles_n,
    int group_m) {
  using G = Cfg<BN>;
  constexpr int NS = G::NS;
  // stage kt+DIST refills the slot of stage kt+DIST-NS: with a three-stage ring that is stage kt-1,
  // freed by step kt-1's barrier, so the stage's DMAs spread over both substeps of step kt; with
  // two stages, stage kt's own slot, freed only by step kt's barrier (the DMAs go in substep 1)
  constexpr int DIST = NS > 2 ? NS - 1 : NS;
  constexpr bool kSpread = DIST < NS;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[NS * G::kStageBytes];

  const int ntiles = tiles_m * tiles_n;
  int pid = blockIdx.x;
  if ((ntiles & 7) == 0) pid = (pid & 7) * (ntiles >> 3) + (pid >> 3);
  const int width = group_m * tiles_n;
  const int first_m = (pid / width) * group_m;
  const int gsize = min(tiles_m - first_m, group_m);
  const int tm = first_m + (pid % width) % gsize;
  const int tn = (pid % width) / gsize;
  const int m0 = tm * BM, n0 = tn * BN;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  // the tile's row scales: one load a thread, issued ahead of the prologue's DMAs and held in a
  // register until the epilogue puts it in LDS, so the epilogue waits on no global load per
  // 32-row block (and nothing waits on this load before then)
  static_assert(BM == kThreads, "one row scale per thread");
  __shared__ float sa_tile[BM];
  const float sa_mine = SA[min(m0 + tid, M - 1)];

  // loaders: rows past M (A) or N (W) read as zero through num_records; stages past K read other
  // rows' bytes or zeros into slots nobody reads any more (the DMA stream runs ahead without a branch)
  const i32x4 rsrc_a = make_rsrc(A + int64_t(m0) * K, uint32_t(min(BM, M - m0)) * uint32_t(K));
  const i32x4 rsrc_w = make_rsrc(W + int64_t(n0) * K, uint32_t(min(BN, N - n0)) * uint32_t(K));
  // DMA instruction d of this wave covers rows 8*(kDma_op*wave + d) .. +8; lane -> row lane/8,
  // slot lane%8 holding chunk (lane%8) ^ swz(row)
  auto voff_of = [&](int row) { return uint32_t(row * K + (((lane & 7) ^ fp8_swz(row)) << 4)); };
  uint32_t a_voff[G::kDmaA], w_voff[G::kDmaW];
#pragma unroll
  for (int t = 0; t < G::kDmaA; ++t) a_voff[t] = voff_of((wave * G::kDmaA + t) * 8 + (lane >> 3));
#pragma unroll
  for (int t = 0; t < G::kDmaW; ++t) w_voff[t] = voff_of((wave * G::kDmaW + t) * 8 + (lane >> 3));
  // stg = kt % NS is a compile-time constant at every call (the main loop runs NS steps a trip), so
  // stage addresses are constants: scalar adds for the DMA bases, immediate offsets for the reads
  const uint32_t lds0 = uint32_t(reinterpret_cast<uintptr_t>(smem));
  const uint32_t wave_a = __builtin_amdgcn_readfirstlane(uint32_t(wave * G::kDmaA * 1024));
  const uint32_t wave_w = __builtin_amdgcn_readfirstlane(uint32_t(wave * G::kDmaW * 1024));
  auto dma_one = [&](int kt, int d, auto stg) __attribute__((always_inline)) {
    const uint32_t st = lds0 + uint32_t(decltype(stg)::value) * G::kStageBytes;
    const uint32_t soff = uint32_t(kt * BK);
    if (d < G::kDmaA)
      dma16(rsrc_a, st + wave_a + d * 1024, a_voff[d], soff);
    else
      dma16(rsrc_w, st + G::kABytes + wave_w + (d - G::kDmaA) * 1024, w_voff[d - G::kDmaA], soff);
  };

  f32x16 acc[4][G::WNT];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < G::WNT; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  // lane -> row (or column) lane % 32, K half (32 bytes = chunks 4ks + 2h, 4ks + 2h + 1) lane / 32
  const int fr = lane & 31, h = lane >> 5;
  int row_off[4 + G::WNT], row_sw[4 + G::WNT];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = wm * 128 + i * 32 + fr;
    row_off[i] = m * BK;
    row_sw[i] = fp8_swz(m);
  }
#pragma unroll
  for (int j = 0; j < G::WNT; ++j) {
    const int n = wn * (BN / 2) + j * 32 + fr;
    row_off[4 + j] = G::kABytes + n * BK;
    row_sw[4 + j] = fp8_swz(n);
  }
  // piece p of substep ks: operand row t = p / 2, half c = p % 2 (chunk 4ks + 2h + c)
  auto read_piece = [&](const uint8_t* st, int ks, int p, Frags<BN>& f) __attribute__((always_inline)) {
    const int t = p >> 1, c = p & 1;
    const u32x4 v = *reinterpret_cast<const u32x4*>(st + row_off[t] + (((4 * ks + 2 * h + c) ^ row_sw[t]) << 4));
    if (c == 0) {
      f.lo[t] = v;
    } else {
      const i32x8 x = i32x8{int(f.lo[t][0]), int(f.lo[t][1]), int(f.lo[t][2]), int(f.lo[t][3]),
                            int(v[0]), int(v[1]), int(v[2]), int(v[3])};
      if (t < 4) f.a[t] = x;
      else f.w[t - 4] = x;
    }
  };
  auto mfma_one = [&](const Frags<BN>& f, int u) __attribute__((always_inline)) {
    const int i = u / G::WNT, j = u % G::WNT;
    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(f.w[j], f.a[i], acc[i][j], 0, 0, 0, 0, 0, 0);
  };

  const int nk = K / BK;
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  using S2 = std::integral_constant<int, 2 % NS>;
#pragma unroll
  for (int d = 0; d < G::kDma; ++d) dma_one(0, d, S0{});
#pragma unroll
  for (int d = 0; d < G::kDma; ++d) dma_one(1, d, S1{});
  if constexpr (DIST > 2) {
#pragma unroll
    for (int d = 0; d < G::kDma; ++d) dma_one(2, d, S2{});
  }
  wait_vmcnt<(DIST - 1) * G::kDma>();   // stage 0 landed (this wave's part)
  __syncthreads();                    // ... and everyone's
  Frags<BN> f0, f1;
#pragma unroll
  for (int p = 0; p < G::kPieces; ++p) read_piece(smem, 0, p, f0);

  // Reads are issued in the order the MFMAs first use the operands (MFMA u multiplies A row block
  // u / WNT by W column block u % WNT): A0, W0 .. W(WNT-1), A1, A2, A3, two 128-bit pieces each,
  // two pieces per MFMA from the start of a substep, so the next substep's first MFMAs find their
  // operands landed instead of waiting on the LDS.  The refill DMAs spread over the whole substep.
  constexpr int U = G::kMfma, P = G::kPieces, D = G::kDma;
  constexpr int NPRE = [] {   // DMAs of stage kt+DIST issued before step kt's barrier
    int n = 0;
    for (int o = 0; o < D; ++o)
      if (kSpread && o * 2 * U / D < U) ++n;
    return n;
  }();
  auto piece_of = [](int q) constexpr {
    const int o = q >> 1;   // operand in first-use order
    const int t = o == 0 ? 0 : (o <= G::WNT ? 4 + (o - 1) : o - G::WNT);
    return 2 * t + (q & 1);
  };
  auto step = [&](int kt, auto stg) __attribute__((always_inline)) {
    constexpr int SI = decltype(stg)::value;   // kt % NS
    using Far = std::integral_constant<int, (SI + DIST) % NS>;
    const uint8_t* st = smem + SI * G::kStageBytes;
    // substep 0, with the reads of substep 1 of this stage (and, spread, the first of stage
    // kt+DIST's DMAs)
#pragma unroll
    for (int u = 0; u < U; ++u) {
      mfma_one(f0, u);
#pragma unroll
      for (int q = 2 * u; q < 2 * u + 2; ++q)
        if (q < P) read_piece(st, 1, piece_of(q), f1);
      if constexpr (kSpread) {
#pragma unroll
        for (int d = 0; d < D; ++d)
          if (d * 2 * U / D == u) dma_one(kt + DIST, d, Far{});
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // stage kt+1 landed (later stages' DMAs may still be in flight); past the barrier every wave
    // is done reading stage kt
    wait_vmcnt<(DIST - 2) * G::kDma + NPRE>();
    __syncthreads();
    const uint8_t* nst = smem + ((SI + 1) % NS) * G::kStageBytes;
    // substep 1, with the reads of the next stage's substep 0 and the refill DMA
#pragma unroll
    for (int u = 0; u < U; ++u) {
      mfma_one(f1, u);
#pragma unroll
      for (int q = 2 * u; q < 2 * u + 2; ++q)
        if (q < P) read_piece(nst, 0, piece_of(q), f0);
#pragma unroll
      for (int d = 0; d < D; ++d)
        if (kSpread ? d * 2 * U / D == U + u : d * U / D == u) dma_one(kt + DIST, d, Far{});
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  int kt = 0;
  for (; kt + NS <= nk; kt += NS) {
    step(kt, S0{});
    step(kt + 1, S1{});
    if constexpr (NS > 2) step(kt + 2, S2{});
  }
  if (kt < nk) step(kt, S0{});
  if constexpr (NS > 2) {
    if (kt + 1 < nk) step(kt + 1, S1{});
  }
  wait_vmcnt<0>();

  // accumulator (i, j, r) of lane holds C row m0 + wm*128 + i*32 + lane%32, columns
  // n0 + wn*BN/2 + j*32 + 8*(r/4) + 4*(lane/32) + r%4.  Each value is scaled, (acc * sa) * sw, and
  // rounded to bf16 where it sits, then the tile leaves through the LDS, which is free once every
  // DMA has landed and, past the barrier, no wave reads a stage: a wave writes one 32-row block of
  // its bf16 results into a private, padded region and reads it back 4 columns a lane, so each
  // store writes whole rows of its block (in the accumulator layout one store instruction writes
  // into each of 32 rows).  The region is the wave's own and LDS operations of a wave complete in
  // order, so no barrier separates its writes from its reads.  Rows past M and columns past N fall
  // outside the output's buffer resource (stores dropped), so the stores need no branches.
  sa_tile[tid] = sa_mine;
  // the weight scales of this lane's accumulator columns: 4 consecutive ones per (j, g)
  f32x4v swc[G::WNT][4];
#pragma unroll
  for (int j = 0; j < G::WNT; ++j)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int c = n0 + wn * (BN / 2) + j * 32 + 8 * g + 4 * h;
      swc[j][g] = *reinterpret_cast<const f32x4v*>(SW + (c < N ? c : 0));
    }
  __syncthreads();
  constexpr int WC = G::WNT * 32;       // columns of a wave's block
  constexpr int kPitch = WC * 2 + 16;   // bytes per staged bf16 row: rows start 4 banks apart
  constexpr int LPR = WC / 4;           // lanes per row, 4 columns each
  constexpr int RPI = 64 / LPR;         // rows per instruction
  static_assert(4 * 32 * kPitch <= NS * G::kStageBytes, "the staging regions fit in the ring's LDS");
  uint8_t* const stage = smem + wave * (32 * kPitch);
  const int rl = lane / LPR, c4 = lane % LPR;
  const int gcol = n0 + wn * (BN / 2) + 4 * c4;
  const __amdgpu_buffer_rsrc_t rsrc_c = __builtin_amdgcn_make_buffer_rsrc(
      C + int64_t(m0) * N, 0, uint32_t(min(BM, M - m0)) * uint32_t(N) * 2u, 0x00020000);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r0 = wm * 128 + i * 32 + rl;   // tile row of this lane's first stored row
    const float sa = sa_tile[wm * 128 + i * 32 + fr];
#pragma unroll
    for (int j = 0; j < G::WNT; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x4v w4 = swc[j][g];
        const float v0 = (acc[i][j][4 * g] * sa) * w4.x, v1 = (acc[i][j][4 * g + 1] * sa) * w4.y;
        const float v2 = (acc[i][j][4 * g + 2] * sa) * w4.z, v3 = (acc[i][j][4 * g + 3] * sa) * w4.w;
        *reinterpret_cast<u32x2*>(stage + fr * kPitch + (j * 32 + 8 * g + 4 * h) * 2) =
            u32x2{pack_bf16x2(v0, v1), pack_bf16x2(v2, v3)};
      }
    // every staged row of the block read back before the first store: the reads' latencies overlap
    u32x2 v[32 / RPI];
#pragma unroll
    for (int t = 0; t < 32 / RPI; ++t) v[t] = *reinterpret_cast<const u32x2*>(stage + (t * RPI + rl) * kPitch + c4 * 8);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < 32 / RPI; ++t) {
      const uint32_t off = gcol < N ? (uint32_t(r0 + t * RPI) * uint32_t(N) + uint32_t(gcol)) * 2u : 0x80000000u;
      __builtin_amdgcn_raw_buffer_store_b64(v[t], rsrc_c, off, 0, 0);
    }
  }
}

// ---- per-row activation quantiser
// Eight bf16 values of a row (one 128-bit chunk) to e4m3 with the row's scale s.  Exact form: the
// IEEE quotient x / s, then the bit-arithmetic RNE cast.  Fast form (rows whose absmax lies in
// [2^-100, FLT_MAX], so that s and r = 1 / s are normal fp32): the quotient as
// q0 = x * r, q = q0 + (x - q0 * s) * r (two FMAs) with x's sign, then v_cvt_pk_fp8_f32 (gfx950: OCP
// e4m3fn, round to nearest even).  On MI355X the fast form gives the exact form's byte for every bf16
// x with |x| <= amax and every bf16 amax in that range (2^31 pairs checked on the device), and the
// conversion instruction equals the bit-arithmetic cast for every fp32 input, NaN and infinity
// included; the exact form stays for rows outside the range.
__device__ __forceinline__ u32x2 quant8_exact(const u32x4& v, float s) {
  uint32_t o[2] = {0u, 0u};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint32_t b0 = f32_to_e4m3(bf16_lo(v[q]) / s), b1 = f32_to_e4m3(bf16_hi(v[q]) / s);
    o[q >> 1] |= (b0 | (b1 << 8)) << (16 * (q & 1));
  }
  return u32x2{o[0], o[1]};
}
__device__ __forceinline__ float quot(float x, float s, float r) {
  const float q0 = x * r;
  return __builtin_copysignf(__builtin_fmaf(__builtin_fmaf(-q0, s, x), r, q0), x);
}
__device__ __forceinline__ u32x2 quant8_fast(const u32x4& v, float s, float r) {
  uint32_t o[2];
#pragma unroll
  for (int w = 0; w < 2; ++w) {
    const uint32_t lo = v[2 * w], hi = v[2 * w + 1];
    int p = __builtin_amdgcn_cvt_pk_fp8_f32(quot(bf16_lo(lo), s, r), quot(bf16_hi(lo), s, r), 0, false);
    p = __builtin_amdgcn_cvt_pk_fp8_f32(quot(bf16_lo(hi), s, r), quot(bf16_hi(hi), s, r), p, true);
    o[w] = uint32_t(p);
  }
  return u32x2{o[0], o[1]};
}
__device__ __forceinline__ bool quant_fast_row(float amax) { return amax >= 0x1p-100f && amax <= 3.402823466e38f; }
// Non-zero when either bf16 of the word is a NaN (magnitude above 0x7f80 carries into its top bit).
__device__ __forceinline__ uint32_t nan_pair(uint32_t w) { return ((w & 0x7fff7fffu) + 0x007f007fu) & 0x80008000u; }
// The row's scale as torch computes it: absmax / 448, 1 for an all-zero row, and 1 for a row holding a
// NaN (its absmax is NaN, and NaN > 0 is false).
__device__ __forceinline__ float quant_scale(float amax, bool has_nan) {
  return (!has_nan && amax > 0.f) ? amax / 448.0f : 1.0f;
}

// One wave per row for rows up to 64*8*VPT elements, the row held in registers.
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
  uint32_t nan = 0u;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int c = l + i * kWave;
    v[i] = c < chunks ? __builtin_nontemporal_load(xr + c) : u32x4{0u, 0u, 0u, 0u};   // read once: streaming policy
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      amax = fmaxf(amax, fmaxf(fabsf(bf16_lo(v[i][q])), fabsf(bf16_hi(v[i][q]))));
      nan |= nan_pair(v[i][q]);
    }
  }
  amax = wave_absmax(amax);
  const bool has_nan = __ballot(nan != 0u) != 0ull;
  const float s = quant_scale(amax, has_nan);
  if (l == 0) scale[row] = s;
  u32x2* qr = reinterpret_cast<u32x2*>(xq + row * int64_t(cols));
  if (!has_nan && quant_fast_row(amax)) {   // uniform over the wave
    const float r = 1.0f / s;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int c = l + i * kWave;
      if (c < chunks) qr[c] = quant8_fast(v[i], s, r);
    }
  } else {
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int c = l + i * kWave;
      if (c < chunks) qr[c] = quant8_exact(v[i], s);
    }
  }
}

// Long rows: one block per row, the row held in registers (VPT chunks per thread).
template <int VPT>
__global__ __launch_bounds__(kQBlock) void quant_rows_block(const uint16_t* __restrict__ x, uint8_t* __restrict__ xq,
                                                            float* __restrict__ scale, int cols) {
  __shared__ float red[kQBlock / kWave];
  __shared__ int red_nan[kQBlock / kWave];
  const int64_t row = blockIdx.x;
  const int chunks = cols >> 3;
  const u32x4* xr = reinterpret_cast<const u32x4*>(x + row * int64_t(cols));
  u32x4 v[VPT];
  float amax = 0.f;
  uint32_t nan = 0u;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int c = threadIdx.x + i * kQBlock;
    v[i] = c < chunks ? __builtin_nontemporal_load(xr + c) : u32x4{0u, 0u, 0u, 0u};   // read once: streaming policy
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      amax = fmaxf(amax, fmaxf(fabsf(bf16_lo(v[i][q])), fabsf(bf16_hi(v[i][q]))));
      nan |= nan_pair(v[i][q]);
    }
  }
  amax = wave_absmax(amax);
  const bool wave_nan = __ballot(nan != 0u) != 0ull;
  if (threadIdx.x % kWave == 0) {
    red[threadIdx.x / kWave] = amax;
    red_nan[threadIdx.x / kWave] = wave_nan;
  }
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const bool has_nan = (red_nan[0] | red_nan[1] | red_nan[2] | red_nan[3]) != 0;
  const float s = quant_scale(amax, has_nan);
  if (threadIdx.x == 0) scale[row] = s;
  u32x2* qr = reinterpret_cast<u32x2*>(xq + row * int64_t(cols));
  if (!has_nan && quant_fast_row(amax)) {   // uniform over the block
    const float r = 1.0f / s;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int c = threadIdx.x + i * kQBlock;
      if (c < chunks) qr[c] = quant8_fast(v[i], s, r);
    }
  } else {
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int c = threadIdx.x + i * kQBlock;
      if (c < chunks) qr[c] = quant8_exact(v[i], s);
    }
  }
}

// ---- per-output-channel weight quantiser
// Column absmax of W[K,N] as the bits of |w|: non-negative floats order like their bit patterns, and
// a NaN's bits exceed every number's, so an unsigned max propagates NaN as torch's amax does (the
// scale of such a column is then 1, as `amax > 0` fails).  The bits collect in amax[N] (zeroed
// first) by one atomicMax per column and K slice.
__global__ __launch_bounds__(256) void fill_zero_u32(uint32_t* __restrict__ p, int64_t n) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i < n) p[i] = 0u;
}

// Block (64 columns, K slice of `rows` rows, a multiple of 16): lane l of wave v reads the 16 bytes of
// columns 4*(l % 16) .. +3 of rows k0 + 16*t + 4*v + l/16, eight loads in flight; the 16 row lanes
// sharing a column meet in LDS.  N % 4 == 0, W 16-byte aligned.
__global__ __launch_bounds__(256) void weight_absmax_part(const float* __restrict__ w, uint32_t* __restrict__ amax,
                                                          int64_t K, int64_t N, int64_t rows) {
  __shared__ uint32_t red[16][65];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int64_t c = int64_t(blockIdx.x) * 64 + 4 * (lane & 15);
  const int64_t k0 = int64_t(blockIdx.y) * rows, k1 = min(K, k0 + rows);
  const int rr = 4 * wv + (lane >> 4);
  uint32_t m[4] = {0u, 0u, 0u, 0u};
  if (c < N) {
    for (int64_t kb = k0; kb < k1; kb += 16 * 8) {
      f32x4v v[8];
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const int64_t k = kb + 16 * t + rr;
        v[t] = k < k1 ? *reinterpret_cast<const f32x4v*>(w + k * N + c) : f32x4v{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int t = 0; t < 8; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) m[e] = max(m[e], __float_as_uint(v[t][e]) & 0x7fffffffu);
    }
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) red[rr][4 * (lane & 15) + e] = m[e];
  __syncthreads();
  if (threadIdx.x < 64) {
    const int64_t j = int64_t(blockIdx.x) * 64 + threadIdx.x;
    uint32_t r = red[0][threadIdx.x];
#pragma unroll
    for (int i = 1; i < 16; ++i) r = max(r, red[i][threadIdx.x]);
    if (j < N) atomicMax(amax + j, r);
  }
}

__device__ __forceinline__ float weight_scale(uint32_t amax_bits) {
  const float m = __uint_as_float(amax_bits);
  return m > 0.f ? m / 448.0f : 1.0f;
}

// quantise + transpose: block (64 columns j, 256 rows i); each thread quantises 4 rows x 4 columns
// (four 16-byte row loads) into four dwords of 4 consecutive i, which meet in an LDS tile [j][i/4];
// then each wave stores 16 rows of Wt, 256 contiguous bytes a store instruction.  K % 4 == 0.
__global__ __launch_bounds__(256) void weight_quant_t(const float* __restrict__ w, const uint32_t* __restrict__ amax,
                                                      uint8_t* __restrict__ wt, int64_t K, int64_t N) {
  __shared__ uint32_t tile[64][65];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int64_t i0 = int64_t(blockIdx.y) * 256, j0 = int64_t(blockIdx.x) * 64;
  const int cq = lane & 15;
  const int64_t c = j0 + 4 * cq;
  float s[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) s[e] = c + e < N ? weight_scale(amax[c + e]) : 1.0f;
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int g = (lane >> 4) + 4 * wv + 16 * it;    // group of 4 consecutive rows
    f32x4v v[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t i = i0 + 4 * g + r;
      v[r] = (i < K && c < N) ? *reinterpret_cast<const f32x4v*>(w + i * N + c) : f32x4v{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      uint32_t q = 0u;
#pragma unroll
      for (int r = 0; r < 4; ++r) q |= f32_to_e4m3(v[r][e] / s[e]) << (8 * r);
      tile[4 * cq + e][g] = q;
    }
  }
  __syncthreads();
#pragma unroll 4
  for (int r = 0; r < 16; ++r) {
    const int jj = 16 * wv + r;
    const int64_t i = i0 + 4 * lane;
    if (j0 + jj < N && i < K) *reinterpret_cast<uint32_t*>(wt + (j0 + jj) * K + i) = tile[jj][lane];
  }
}

// the scales from the collected absmax bits, in place
__global__ __launch_bounds__(256) void weight_scales(uint32_t* __restrict__ amax, int64_t n) {
  const int64_t j = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (j < n) amax[j] = __float_as_uint(weight_scale(amax[j]));
}

// Any shape: absmax over K of each column by one block of 64 columns x 4 K-slices, then quantise +
// transpose through a 64x64 byte tile.
__global__ __launch_bounds__(256) void weight_absmax_any(const float* __restrict__ w, float* __restrict__ scale,
                                                         int64_t K, int64_t N) {
  __shared__ uint32_t red[4][64];
  const int64_t j = int64_t(blockIdx.x) * 64 + (threadIdx.x & 63);
  const int slice = threadIdx.x >> 6;
  uint32_t amax = 0u;
  if (j < N)
    for (int64_t i = slice; i < K; i += 4) amax = max(amax, __float_as_uint(w[i * N + j]) & 0x7fffffffu);
  red[slice][threadIdx.x & 63] = amax;
  __syncthreads();
  if (slice == 0 && j < N) {
    const uint32_t m = max(max(red[0][threadIdx.x], red[1][threadIdx.x]), max(red[2][threadIdx.x], red[3][threadIdx.x]));
    scale[j] = weight_scale(m);
  }
}

__global__ __launch_bounds__(256) void weight_quant_t_any(const float* __restrict__ w, const float* __restrict__ scale,
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
  const int64_t gx = (n + 63) / 64;
  if (gx > 0x7fffffff || (k + 63) / 64 > 65535) return PTB_ERR_GRID;
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint8_t* wt = static_cast<uint8_t*>(wq_t);
  if (n % 4 || k % 4 || !aligned16(w) || (reinterpret_cast<uintptr_t>(wq_t) & 3u)) {
    weight_absmax_any<<<dim3(unsigned(gx)), dim3(256), 0, s>>>(w, scale, k, n);
    weight_quant_t_any<<<dim3(unsigned(gx), unsigned((k + 63) / 64)), dim3(256), 0, s>>>(w, scale, wt, k, n);
    return launch_status();
  }
  // the column maxima split over K so that about 2048 blocks cover the chip: K slices of a
  // multiple of 16 rows; the scale array holds the absmax bits until the last launch
  uint32_t* amax = reinterpret_cast<uint32_t*>(scale);
  const int64_t want = std::max<int64_t>(1, std::min<int64_t>((2048 + gx - 1) / gx, (k + 127) / 128));
  const int64_t rows = ((k + want - 1) / want + 15) / 16 * 16;
  const int64_t gy = (k + rows - 1) / rows;
  fill_zero_u32<<<dim3(unsigned((n + 255) / 256)), dim3(256), 0, s>>>(amax, n);
  weight_absmax_part<<<dim3(unsigned(gx), unsigned(gy)), dim3(256), 0, s>>>(w, amax, k, n, rows);
  weight_quant_t<<<dim3(unsigned(gx), unsigned((k + 255) / 256)), dim3(256), 0, s>>>(w, amax, wt, k, n);
  weight_scales<<<dim3(unsigned((n + 255) / 256)), dim3(256), 0, s>>>(amax, n);
  return launch_status();
}

namespace {

int device_cus() {
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess) hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  return cus;
}

int fp8_check(const void* aq, const float* sa, const void* wq_t, const float* sw, void* c, int64_t m, int64_t n,
              int64_t k) {
  if (m < 0 || n < 0 || k < 0) return PTB_ERR_SHAPE;
  if (m == 0 || n == 0) return PTB_OK;
  if (!aq || !sa || !wq_t || !sw || !c) return PTB_ERR_NULL;
  if (k == 0) return PTB_ERR_UNSUPPORTED;
  if (m > 0x7fffffff || n > 0x7fffffff || k > 0x7fffffff) return PTB_ERR_SHAPE;
  if (k % 128 || n % 16) return PTB_ERR_UNSUPPORTED;
  if (int64_t(BM) * k >= (int64_t(1) << 32)) return PTB_ERR_UNSUPPORTED;  // 32-bit buffer offsets
  // a 256-row tile of C within 2^31 bytes: the epilogue's 32-bit store offsets, and the 0x80000000
  // that marks a column outside C, stay in range
  if (n > (int64_t(1) << 22)) return PTB_ERR_UNSUPPORTED;
  if (!aligned16(aq) || !aligned16(wq_t) || !aligned16(sw) || (reinterpret_cast<uintptr_t>(c) & 7u))
    return PTB_ERR_ALIGN;
  return 1;   // go on
}

}  // namespace

PTB_EXPORT int ptb_gemm_fp8_scaled(const void* aq, const float* sa, const void* wq_t, const float* sw, void* c,
                                   int64_t m, int64_t n, int64_t k, void* stream) {
  const int st = fp8_check(aq, sa, wq_t, sw, c, m, n, k);
  if (st <= 0) return st;
  // 256x256 tiles unless that leaves CUs idle, then 256x128
  const int64_t tm = (m + BM - 1) / BM;
  const bool wide = tm * ((n + 255) / 256) >= device_cus();
  const int bn = wide ? 256 : 128;
  const int64_t tn = (n + bn - 1) / bn;
  if (tm * tn > 0x7fffffff) return PTB_ERR_GRID;
  const dim3 grid(unsigned(tm * tn)), block(kThreads);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint8_t* a8 = static_cast<const uint8_t*>(aq);
  const uint8_t* w8 = static_cast<const uint8_t*>(wq_t);
  uint16_t* c16 = static_cast<uint16_t*>(c);
  // Tile order: ids are spread so that each XCD takes a contiguous range of tiles, walked in groups
  // of group_m tile-rows.  At 256x128 tiles a group of 4 rows makes an XCD's 32 resident tiles a 4x8
  // block, whose A and W panels (4 x 256 rows + 8 x 128 rows of K) are the fewest bytes its L2 must
  // fetch; 256x256 tiles keep groups of 8.
  const int group_m = wide ? 8 : 4;
  if (wide)
    gemm_fp8_kernel<256><<<grid, block, 0, s>>>(a8, sa, w8, sw, c16, int(m), int(n), int(k), int(tm), int(tn),
                                                group_m);
  else
    gemm_fp8_kernel<128><<<grid, block, 0, s>>>(a8, sa, w8, sw, c16, int(m), int(n), int(k), int(tm), int(tn),
                                                group_m);
  return launch_status();
}
