// bf16 GEMM on gfx950 matrix cores: C[M,N] = A[M,K] * B[K,N] (+ R[M,N]), all row-major, fp32
// accumulation, one bf16 rounding at the store.
//
// Workgroup tiles of 256x256, 256x192, 256x128, 128x128 or 64x128 (Shape below), 4 waves in a 2x2
// arrangement, each wave owning WM x WN v_mfma_f32_32x32x16_bf16 accumulators (256 fp32 per lane
// for 256x256 tiles, held in AGPRs).
//
// Operands move HBM -> LDS with buffer_load_dwordx4 ... lds (no VGPR staging).  256-row tiles stage
// 64 K columns at a time (a whole 128-byte line of every A row) -- 256x128 tiles in a ring of three
// slots, 256x256 and 256x192 tiles in rings of three A slots and two B slots (160 / 144 KB) -- and
// 128x128 and smaller tiles 32 columns in rings of four slots.  Each stage's DMAs run two (or three)
// stages ahead and spread over a whole K step's MFMAs, into the slots the previous step's barrier
// freed.  A and B keep their global layouts in LDS with 16-byte chunks XOR-swizzled per row, so
// every fragment read is bank-conflict free:
//   A fragments (8 consecutive k of one row per lane) are plain 128-bit LDS reads; row m keeps
//   chunk c in slot c ^ ((m >> 1) & 7) for 64-deep stages, c ^ ((m >> 2) & 3) for 32-deep ones;
//   B fragments (8 consecutive k of one column per lane, while B is N-contiguous) come from two
//   ds_read_b64_tr_b16 transposing reads; row k keeps chunk c in slot c ^ (4 * (k & 3)) (rows of
//   384 bytes: c ^ (4 * ((k >> 1) & 1))).
// The fragments of the next 16-wide K slice are read while the MFMAs of the current one run, and
// the main loop runs a whole number of ring turns a trip, so every slot address is a constant.
// The MFMA is issued with B as its first operand, so each accumulator holds a 32x32 block of C^T.
// The epilogue stages each wave's 32-row blocks of fp32 results through a private, padded LDS
// region (the rings are free by then) so that stores, and residual loads, cover whole rows; buffer
// resources drop rows and columns outside C.
//
// Modes: plain (+ residual), split-K into fp32 partials (splitk_finish sums them), SwiGLU (the gate
// and up columns of the same outputs meet in one wave; the epilogue stores silu(gate) * up) and
// grouped (the MoE grouped GEMM: a program table maps row tiles to weights).
//
// Tile order is XCD-aware: hardware hands workgroup i to XCD i % 8, so ids are remapped to give
// each XCD a contiguous range of tiles, walked in groups of 8 tile-rows for L2 reuse.
#include <algorithm>
#include <type_traits>

#include "ptb_common.h"

using namespace ptb;



namespace {

constexpr int kThreads = 256;
constexpr int kGroupM = 8;
// K past the end the DMA stream may address (the deepest ring: 4 stages of 32 or 2 of 64)
constexpr int kRunAhead = 128;
// Widest C (columns) the epilogue addresses: a 256-row tile of it stays within 2^31 bytes, so its
// 32-bit store offsets, and the 0x80000000 that marks a column outside C, stay in range.
constexpr int64_t kMaxOutCols = int64_t(1) << 22;

typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

// Tile shape: the 4 waves sit 2x2, each owning WM x WN blocks of 32x32, so the workgroup tile is
// BM = 64*WM rows by BN = 64*WN columns (256x256, 256x192, 256x128, 128x128 or 64x128).  A stage
// holds BK of K: 32 (a 64-byte piece of every A row; 128x128 and 64x128 tiles) in rings of 4 slots,
// or 64 (a whole 128-byte line of every A row: the L2 serves a request per line, and a half-line
// request costs a whole one) in rings of 3 slots (256x128 tiles) or of 3 A slots and 2 B slots
// (256x256, 256x192).  Stage
// kt + DIST, DIST = NSA - 1 = 2 or 3, refills the slots of stage kt-1, which the barrier of step
// kt-1 freed, so the stage's DMAs spread over all of step kt's MFMAs; with two B slots, its B part
// waits for the barrier of step kt and spreads over the slice after it.
template <int WM, int WN, int BKT>
struct Shape {
  static constexpr int BK = BKT;
  // A and B live in rings of their own: NSA and NSB slots.  256x256 and 256x192 tiles with 64-deep
  // stages have room for three A slots and two B slots only (160 / 144 KB), so their B ring
  // refills a slot only after the barrier that frees it (the "hybrid" schedule below); every other
  // ring is one slot deeper than its DMA distance.
  static constexpr bool kHybrid = BK == 64 && WM * WN >= 12;
  static constexpr int NSA = BK == 64 ? 3 : 4;
  static constexpr int NSB = kHybrid ? 2 : NSA;
  static constexpr int NS = NSA;
  static constexpr int DIST = NSA - 1;
  static constexpr int SPS = BK / 16;                    // 16-wide K slices per stage
  static constexpr int BM = 64 * WM, BN = 64 * WN;
  static constexpr int kRowBytes = BK * 2;               // bytes of an A row in a stage
  static constexpr int kChunks = BK / 8;                 // 16-byte chunks of an A row in a stage
  static constexpr int kABytes = BM * BK * 2;
  static constexpr int kBBytes = BK * BN * 2;
  static constexpr int kDmaA = kABytes / 4096;           // buffer_load ... lds per wave per stage
  static constexpr int kDmaB = kBBytes / 4096;
  static constexpr int kDma = kDmaA + kDmaB;
  static constexpr int kARowsPerKB = 1024 / kRowBytes;   // A rows per DMA instruction
  static constexpr int kMfma = WM * WN;                  // MFMAs per wave per 16-wide K slice
  static constexpr int kPieces = WM + 2 * WN;            // LDS reads per wave per K slice
  static constexpr int kBSlots = BN / 8;                 // 16-byte chunks per B row
  static constexpr int kSmemBytes = NSA * kABytes + NSB * kBBytes;
  static_assert(kSmemBytes <= 160 * 1024, "the rings fit the LDS");
  static_assert(kABytes % 4096 == 0 && kBBytes % 4096 == 0, "whole 1 KB DMA instructions per wave");
  static_assert(DIST == NS - 1 && DIST >= 2, "the DMA refills the slot freed a step earlier");
};
// A row m keeps chunk c in slot c ^ swz: 4 chunks (BK 32) rotate by (m >> 2) & 3, 8 chunks (BK 64)
// by (m >> 1) & 7; either way the 16 rows a 16-lane phase reads land in 16 distinct bank groups.
template <int BKT>
__device__ __forceinline__ int a_swz(int m) { return BKT == 64 ? (m >> 1) & 7 : (m >> 2) & 3; }
// B row k keeps chunk c in slot c ^ b_swz(k).  A transposing read takes 64 bytes of each of 4
// consecutive rows k0..k0+3 (k0 % 4 == 0) per 32 lanes.  Rows of 512 or 256 bytes all start at
// bank 0, so the rows shift by 64 bytes each: 4 * (k & 3).  Rows of 384 bytes (BN 192) start 32
// banks apart in turn, so only k0+2 and k0+3 shift, by 64 bytes: 4 * ((k >> 1) & 1).  Either way
// the 4 rows' 64 bytes take 64 distinct banks, and the XOR stays inside the row's chunks.
template <int BN>
__device__ __forceinline__ int b_swz(int k) { return BN == 192 ? 4 * ((k >> 1) & 1) : 4 * (k & 3); }

// Grouped mode (the MoE grouped GEMM): program p of the launch multiplies group g = grp[p]'s
// rows [gstart[g], gstart[g] + grows[g]) of A by weight g of B (row-major K x N at B + g*sbg) into
// the same rows of C.  A workgroup's linear tile index runs over every program's row tiles in
// program order (times the column tiles); the per-program tile counts are scanned in LDS, so
// workgroups past the last tile leave at once.  Table entries that do not describe rows inside A
// (or a weight inside B) count as empty.
struct Groups {
  const int32_t* grp;
  const int32_t* gstart;
  const int32_t* grows;
  int nprog, ntab, nweights, a_rows;
  int64_t sbg;
};
constexpr int kMaxPrograms = 256;
constexpr int kMaxDedupGroups = 1024;   // group tables up to this size have repeated programs skipped

// Split-K mode: workgroup (tile, blockIdx.y = s) multiplies K columns [s*kchunk, s*kchunk + kchunk)
// and stores its fp32 partial tile at part + s*M*N; splitk_finish sums the partials.
// SwiGLU mode (the gate_up GEMM with silu(gate) * up fused into its epilogue): B is [K, 2*I] with
// gate columns [0, I) and up columns [I, 2I); a 256x256 workgroup tile's B columns alternate in
// 32-wide blocks between gate and up columns of the same 128 output columns, so each wave's
// accumulator pairs (j even: gate, j + 1: up) cover the same outputs and the epilogue stores
// bf16(silu(bf16(gate)) * bf16(up)), as a separate silu_mul would compute it from the bf16 GEMM.
enum { kPlain = 0, kGrouped = 1, kSplit = 2, kSwiGLU = 3 };


// PERSIST (plain 256x256 tiles, no residual): one workgroup per CU walks the tiles
// blockIdx.x, blockIdx.x + gridDim.x, ...; the next tile's first stage goes out halfway through the
// current tile's epilogue, so its latency hides behind the stores (see the epilogue).
template <int WM, int WN, bool RESID, int MODE, int BKT = 32, bool PERSIST = false>
__global__ __launch_bounds__(kThreads, (WM * WN >= 12 ? 1 : 2)) void gemm_bf16_kernel(
    const uint16_t* __restrict__ A_in, const uint16_t* __restrict__ B_in, const uint16_t* __restrict__ R,
    uint16_t* __restrict__ C_in, int M_in, int N, int K, int tiles_m, int tiles_n, Groups gp,
    float* __restrict__ part, int kchunk) {
  using Sh = Shape<WM, WN, BKT>;
  constexpr int BM = Sh::BM, BN = Sh::BN, kABytes = Sh::kABytes;
  constexpr int BK = Sh::BK, NS = Sh::NS, DIST = Sh::DIST, NSA = Sh::NSA, NSB = Sh::NSB;
  constexpr bool kHybrid = Sh::kHybrid;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[Sh::kSmemBytes];

  // ---- tile selection: tile id -> (first row, first column); ids are spread so that each XCD
  //      takes a contiguous range of tiles, walked in groups of kGroupM tile-rows
  const int ntiles = tiles_m * tiles_n;
  auto tile_origin = [&](int id, int& tm0, int& tn0) __attribute__((always_inline)) {
    int pid = id;
    if ((ntiles & 7) == 0) pid = (pid & 7) * (ntiles >> 3) + (pid >> 3);
    const int width = kGroupM * tiles_n;
    const int first_m = (pid / width) * kGroupM;
    const int gsize = min(tiles_m - first_m, kGroupM);
    const int tm = first_m + (pid % width) % gsize;
    const int tn = (pid % width) / gsize;
    tm0 = tm * BM;
    tn0 = MODE == kSwiGLU ? tn * (BN / 2) : tn * BN;   // SwiGLU: the output (and gate) column base
  };
  const uint16_t* A = A_in;
  const uint16_t* B = B_in;
  uint16_t* C = C_in;
  int M = M_in, m0, n0;
  int Kl = K;    // the K columns this workgroup multiplies
  if constexpr (MODE == kGrouped) {
    __shared__ int pref[kMaxPrograms + 1];
    __shared__ int wsum[kThreads / 64];
    __shared__ int first_prog[kMaxDedupGroups];   // the first program listing each group
    const int t = threadIdx.x, l = t & 63, w = t >> 6;
    const bool dedup = gp.ntab <= kMaxDedupGroups;
    if (dedup)
      for (int i = t; i < gp.ntab; i += kThreads) first_prog[i] = kMaxPrograms;
    __syncthreads();
    const int gt = t < gp.nprog ? gp.grp[t] : -1;
    const bool in_table = gt >= 0 && gt < gp.ntab;
    if (dedup && in_table) atomicMin(&first_prog[gt], t);
    __syncthreads();
    // a program repeating an earlier program's group writes the same rows with the same values:
    // it takes no tiles, so repeats cannot push later programs' tiles past the grid
    int cnt = 0;
    if (in_table && (!dedup || first_prog[gt] == t)) {
      const int s0 = gp.gstart[gt], nr = gp.grows[gt];
      if (nr > 0 && s0 >= 0 && int64_t(s0) + nr <= gp.a_rows && gt < gp.nweights) cnt = (nr + BM - 1) / BM;
    }
    int v = cnt;   // inclusive scan over the 256 programs: within waves, then across the 4 waves
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int u = __shfl_up(v, off, 64);
      if (l >= off) v += u;
    }
    if (l == 63) wsum[w] = v;
    __syncthreads();
    for (int i = 0; i < w; ++i) v += wsum[i];
    pref[t + 1] = v;
    if (t == 0) pref[0] = 0;
    __syncthreads();
    const int total = pref[gp.nprog];
    const int tn = int(blockIdx.x) % tiles_n, mt_all = int(blockIdx.x) / tiles_n;
    if (mt_all >= total) return;   // uniform over the workgroup, before the pipeline starts
    int lo = 0, hi = gp.nprog;     // the last program p with pref[p] <= mt_all
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (pref[mid] <= mt_all) lo = mid;
      else hi = mid;
    }
    const int g = gp.grp[lo], mt = mt_all - pref[lo];
    const int first = gp.gstart[g] + mt * BM;
    M = min(BM, gp.grows[g] - mt * BM);
    A = A_in + int64_t(first) * K;
    C = C_in + int64_t(first) * N;
    B = B_in + int64_t(g) * gp.sbg;
    m0 = 0;
    n0 = tn * BN;
  } else {
    if constexpr (MODE == kSplit) {
      const int k0 = int(blockIdx.y) * kchunk;
      Kl = min(kchunk, K - k0);
      A = A_in + k0;
      B = B_in + int64_t(k0) * N;
    }
    tile_origin(blockIdx.x, m0, n0);
  }

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // ---- loaders: A tile rows past M read as zero (num_records); B columns past N are read from
  //      the next row or as zero, and only feed columns of C that are never stored
  const int koff = MODE == kSplit ? int(blockIdx.y) * kchunk : 0;   // this split's first K column
  auto make_rsrc_a = [&](int tm0) __attribute__((always_inline)) {
    return make_rsrc(A + int64_t(tm0) * K, uint32_t(int64_t(min(BM, M - tm0)) * K - koff) * 2u);
  };
  auto make_rsrc_b = [&](int tn0) __attribute__((always_inline)) {
    return make_rsrc(B + tn0, uint32_t((int64_t(K - koff) * N - tn0) * 2));
  };
  i32x4 rsrc_a = make_rsrc_a(m0);
  i32x4 rsrc_b = make_rsrc_b(n0);
  // A: instruction t of this wave covers rows kARowsPerKB*(kDmaA*wave + t) + lane/kChunks; lane ->
  //    slot lane%kChunks, holding chunk slot ^ a_swz(row)
  // B: instruction t covers the stage's 16-byte pieces 64*(kDmaB*wave + t) + lane in row-major order,
  //    piece i -> row i/kBSlots, slot i%kBSlots holding chunk slot ^ b_swz(row)
  uint32_t a_voff[Sh::kDmaA], b_voff[Sh::kDmaB];
#pragma unroll
  for (int t = 0; t < Sh::kDmaA; ++t) {
    const int row = (wave * Sh::kDmaA + t) * Sh::kARowsPerKB + lane / Sh::kChunks;
    const int chunk = (lane % Sh::kChunks) ^ a_swz<BKT>(row);
    a_voff[t] = uint32_t(row * K + chunk * 8) * 2u;
  }
#pragma unroll
  for (int t = 0; t < Sh::kDmaB; ++t) {
    const int piece = 64 * (wave * Sh::kDmaB + t) + lane;
    const int k = piece / Sh::kBSlots;
    const int bchunk = (piece % Sh::kBSlots) ^ b_swz<BN>(k);
    int bcol = bchunk * 8;
    if constexpr (MODE == kSwiGLU) {   // 32-wide block b: gate (b even) or up (b odd) of pair b / 2
      const int b = bchunk >> 2;
      bcol = ((b & 1) ? N / 2 : 0) + 32 * (b >> 1) + 8 * (bchunk & 3);
    }
    b_voff[t] = uint32_t(k * N + bcol) * 2u;
  }
  const uint32_t lds0 = uint32_t(reinterpret_cast<uintptr_t>(smem));
  const uint32_t wave_a = __builtin_amdgcn_readfirstlane(uint32_t(wave * Sh::kDmaA * 1024));
  const uint32_t wave_b = __builtin_amdgcn_readfirstlane(uint32_t(wave * Sh::kDmaB * 1024));
  // t-th of this wave's A (or B) DMA instructions of stage kt into A slot sa (B slot sb); the slots
  // are compile-time constants at every call (the main loop runs a whole number of ring turns a
  // trip), so the LDS addresses are constants plus scalar offsets and the fragment reads take them
  // as immediate offsets
  const uint32_t lds_b0 = lds0 + uint32_t(NSA * kABytes);
  auto dma_a = [&](int kt, int t, auto sa) __attribute__((always_inline)) {
    dma16(rsrc_a, lds0 + uint32_t(decltype(sa)::value) * kABytes + wave_a + t * 1024, a_voff[t],
          uint32_t(kt * BK) * 2u);
  };
  auto dma_b = [&](int kt, int t, auto sb) __attribute__((always_inline)) {
    dma16(rsrc_b, lds_b0 + uint32_t(decltype(sb)::value) * Sh::kBBytes + wave_b + t * 1024, b_voff[t],
          uint32_t(kt * BK) * uint32_t(N) * 2u);
  };
  // the t-th DMA of a stage, A first, then B
  auto dma_one = [&](int kt, int t, auto sa, auto sb) __attribute__((always_inline)) {
    if (t < Sh::kDmaA) dma_a(kt, t, sa);
    else dma_b(kt, t - Sh::kDmaA, sb);
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;
  using I4 = std::integral_constant<int, 4>;
  using I5 = std::integral_constant<int, 5>;

  f32x16 acc[WM][WN];

  // ---- fragment addressing
  const int fr = lane & 31, h = lane >> 5;
  // A: row m (this lane's), chunk 2*ks + h, swizzled by a_swz(m)
  int a_row_off[WM], a_sw[WM];
#pragma unroll
  for (int i = 0; i < WM; ++i) {
    const int m = wm * (BM / 2) + i * 32 + fr;
    a_row_off[i] = m * Sh::kRowBytes;
    a_sw[i] = a_swz<BKT>(m);
  }
  // B (transposing reads): group g = lane/16 -> k half g/2, column half 16*(g%2); in-group lane
  // 4*jj + q supplies row 8h + 4r + jj (+16 ks), columns +4q..+4q+3
  const int g16 = (lane >> 4) & 1, l16 = lane & 15, jj = l16 >> 2, q = l16 & 3;
  int b_off[WN][2];
#pragma unroll
  for (int j = 0; j < WN; ++j) {
    const int n = wn * (BN / 2) + j * 32 + 16 * g16 + 4 * q;
    const int chunk = n >> 3;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int k = 8 * h + 4 * r + jj;  // + 16*ks, which keeps k & 3
      b_off[j][r] = k * (2 * BN) + ((chunk ^ b_swz<BN>(k)) << 4) + (q & 1) * 8;
    }
  }

  // One K slice's fragments, read in kPieces pieces (WM A reads, 2*WN B half-reads) so that the
  // reads can be spread between MFMAs.
  struct Slice {
    bf16x8 a[WM];
    bf16x8 b[WN];
    i16x4 blo[WN];
  };
  auto read_piece = [&](const uint8_t* sta, const uint8_t* stb, int ks, int p, Slice& f) __attribute__((always_inline)) {
    if (p < WM) {
      f.a[p] = *reinterpret_cast<const bf16x8*>(sta + a_row_off[p] + (((2 * ks + h) ^ a_sw[p]) << 4));
    } else {
      const int j = (p - WM) >> 1, r = (p - WM) & 1;
      const i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(stb + b_off[j][r] + ks * 16 * 2 * BN));
      if (r == 0) f.blo[j] = v;
      else f.b[j] = __builtin_bit_cast(bf16x8, i16x8{f.blo[j][0], f.blo[j][1], f.blo[j][2], f.blo[j][3], v[0], v[1], v[2], v[3]});
    }
  };
  auto mfma_one = [&](const Slice& f, int u) __attribute__((always_inline)) {
    const int i = u / WN, j = u % WN;
    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.b[j], f.a[i], acc[i][j], 0, 0, 0);
  };

  // The DMA stream runs DIST stages ahead of the MFMAs and does not stop at the last K step:
  // stages past the end read zeros (num_records) into slots nobody reads any more, which keeps the
  // loop free of branches; everything is drained before the epilogue.
  constexpr int U = Sh::kMfma, P = Sh::kPieces, D = Sh::kDma, SPS = Sh::SPS;
  constexpr bool kOneReadPerMfma = P <= U;
  // stage kt+DIST's DMAs go out one every SLOTS/D MFMAs of step kt (bunched after the barrier they
  // would queue behind each other in the address unit and stall the MFMAs)
  constexpr int SLOTS = SPS * U;
  // Hybrid schedule (two B slots): stage kt+2's A DMAs spread over step kt before its barrier, into
  // the A slot step kt-1 freed; its B DMAs go into the B slot step kt's barrier frees, spread over
  // step kt's last slice (one per two MFMAs, against the A DMAs' one per six).  Splitting the B
  // DMAs between that slice and the next step's first MFMAs measured no faster.
  constexpr int NPRE = [] {   // DMAs of stage kt+DIST issued before step kt's barrier
    int n = 0;
    if (kHybrid) return Sh::kDmaA;
    for (int o = 0; o < D; ++o)
      if (o * SLOTS / D < (SPS - 1) * U) ++n;
    return n;
  }();
  const int nk = Kl / BK;
  const uint8_t* const smem_b = smem + NSA * kABytes;
  static_assert(!PERSIST || (WM == 4 && WN == 4 && BKT == 64 && !RESID && MODE == kPlain),
                "the persistent walk is for plain 256x256 tiles (the SwiGLU form has no registers to spare)");
  // stores of the epilogue's second half, issued after the next tile's stage-0 DMAs
  constexpr int kStoresAfter = (WM / 2) * 4 * (MODE == kSwiGLU ? WN / 2 : WN);
  int tile_id = blockIdx.x;
  bool pre0 = false;   // this tile's stage 0 went out during the previous tile's epilogue
  for (;;) {
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int j = 0; j < WN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  if (!pre0) {
#pragma unroll
    for (int t = 0; t < D; ++t) dma_one(0, t, I0{}, I0{});
  }
#pragma unroll
  for (int t = 0; t < D; ++t) dma_one(1, t, I1{}, std::integral_constant<int, 1 % NSB>{});
  if constexpr (DIST > 2) {
#pragma unroll
    for (int t = 0; t < D; ++t) dma_one(2, t, I2{}, std::integral_constant<int, 2 % NSB>{});
  }
  // stage 0 landed (this wave's part): after it went out, the stages above and, when it was
  // prefetched, the epilogue's last kStoresAfter stores (memory operations count down in order)
  if (pre0) wait_vmcnt<(DIST - 1) * D + (PERSIST ? kStoresAfter : 0)>();
  else wait_vmcnt<(DIST - 1) * D>();
  __syncthreads();                  // ... and everyone's
  Slice sl[2];
#pragma unroll
  for (int p = 0; p < P; ++p) read_piece(smem, smem_b, 0, p, sl[0]);

  // Each K step: slices 0 .. SPS-2, each with the next slice's reads and a share of the DMAs folded
  // in; the barrier that publishes stage kt+1 (and frees stage kt's slots); the last slice with the
  // rest of the DMAs and the reads of stage kt+1's slice 0 folded in.  sched_barrier(0) pins that
  // interleave, so the matrix core is fed between memory instructions.
  auto step = [&](int kt, auto sa, auto sb) __attribute__((always_inline)) {
    constexpr int SA = decltype(sa)::value, SB = decltype(sb)::value;   // kt % NSA, kt % NSB
    using FarA = std::integral_constant<int, (SA + DIST) % NSA>;
    using FarB = std::integral_constant<int, (SB + DIST) % NSB>;
    const uint8_t* sta = smem + SA * kABytes;
    const uint8_t* stb = smem_b + SB * Sh::kBBytes;
#pragma unroll
    for (int q = 0; q + 1 < SPS; ++q) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        mfma_one(sl[q & 1], u);
#pragma unroll
        for (int p = 0; p < P; ++p)
          if (kOneReadPerMfma ? p == u : (p >= u * P / U && p < (u + 1) * P / U)) read_piece(sta, stb, q + 1, p, sl[(q + 1) & 1]);
        if constexpr (kHybrid) {
#pragma unroll
          for (int o = 0; o < Sh::kDmaA; ++o)
            if (o * (SPS - 1) * U / Sh::kDmaA == q * U + u) dma_a(kt + DIST, o, FarA{});
        } else {
#pragma unroll
          for (int o = 0; o < D; ++o)
            if (o * SLOTS / D == q * U + u) dma_one(kt + DIST, o, FarA{}, FarB{});
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // stage kt+1 landed (later stages' DMAs may still be in flight); past this barrier no wave
    // reads stage kt
    wait_vmcnt<(DIST - 2) * D + NPRE>();
    __syncthreads();
    const uint8_t* nsta = smem + ((SA + 1) % NSA) * kABytes;
    const uint8_t* nstb = smem_b + ((SB + 1) % NSB) * Sh::kBBytes;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      mfma_one(sl[(SPS - 1) & 1], u);
      // the stage's remaining DMAs, and the next stage's first reads spread evenly
      if constexpr (kHybrid) {
#pragma unroll
        for (int o = 0; o < Sh::kDmaB; ++o)
          if (o * U / Sh::kDmaB == u) dma_b(kt + DIST, o, FarB{});   // into the B slot this barrier freed
      } else {
#pragma unroll
        for (int o = 0; o < D; ++o)
          if (o * SLOTS / D == (SPS - 1) * U + u) dma_one(kt + DIST, o, FarA{}, FarB{});
      }
#pragma unroll
      for (int p = 0; p < P; ++p)
        if (p >= u * P / U && p < (u + 1) * P / U) read_piece(nsta, nstb, 0, p, sl[0]);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // L steps a trip: a whole number of turns of both rings, so every slot is a constant
  constexpr int L = kHybrid ? 6 : NSA;
  auto stepc = [&](int k, auto i) __attribute__((always_inline)) {
    constexpr int I = decltype(i)::value;
    step(k, std::integral_constant<int, I % NSA>{}, std::integral_constant<int, I % NSB>{});
  };
  int kt = 0;
  for (; kt + L <= nk; kt += L) {
    stepc(kt, I0{});
    stepc(kt + 1, I1{});
    stepc(kt + 2, I2{});
    if constexpr (L > 3) stepc(kt + 3, I3{});
    if constexpr (L > 4) stepc(kt + 4, I4{});
    if constexpr (L > 5) stepc(kt + 5, I5{});
  }
  if (kt < nk) stepc(kt, I0{});
  if (kt + 1 < nk) stepc(kt + 1, I1{});
  if constexpr (L > 3) {
    if (kt + 2 < nk) stepc(kt + 2, I2{});
  }
  if constexpr (L > 4) {
    if (kt + 3 < nk) stepc(kt + 3, I3{});
  }
  if constexpr (L > 5) {
    if (kt + 4 < nk) stepc(kt + 4, I4{});
  }
  wait_vmcnt<0>();

  // the next tile of a persistent walk, and its stage-0 DMAs into A slot 0 and B slot 0 (free:
  // every DMA has landed and, past the epilogue's barrier, no wave reads a stage)
  const int next_id = tile_id + int(gridDim.x);
  const bool has_next = PERSIST && next_id < ntiles;
  int nm0 = 0, nn0 = 0;
  if (has_next) tile_origin(next_id, nm0, nn0);
  auto prefetch_next = [&]() __attribute__((always_inline)) {
    if (has_next) {
      rsrc_a = make_rsrc_a(nm0);
      rsrc_b = make_rsrc_b(nn0);
#pragma unroll
      for (int t = 0; t < D; ++t) dma_one(0, t, I0{}, I0{});
    }
  };

  // ---- epilogue: accumulator (i, j, r) of lane holds C row m0 + wm*BM/2 + i*32 + lane%32,
  //      column n0 + wn*BN/2 + j*32 + 8*(r/4) + 4*(lane/32) + r%4: 4 consecutive columns per r/4
  if constexpr (MODE == kSplit) {
#pragma unroll
    for (int i = 0; i < WM; ++i) {
      const int row = m0 + wm * (BM / 2) + i * 32 + fr;
      if (row >= M) continue;
#pragma unroll
      for (int j = 0; j < WN; ++j) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int col = n0 + wn * (BN / 2) + j * 32 + 8 * g + 4 * h;
          if (col >= N) continue;  // N % 8 == 0: a 4-column group is all in or all out
          *reinterpret_cast<f32x4v*>(part + int64_t(blockIdx.y) * M * N + int64_t(row) * N + col) =
              f32x4v{acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
        }
      }
    }
    return;
  }
  // Plain, grouped and SwiGLU tiles leave through the LDS, which is free now (every DMA has landed
  // and, past the barrier, no wave reads a stage): a wave writes one 32-row block of its results
  // (bf16; fp32 where a residual is still to be added, and in the persistent walk) (WJ 32-column
  // blocks; value(i, jj, g) gives
  // the 4 fp32 columns 8g + 4*(lane/32) .. +3 of
  // block jj for row lane%32) into a private, padded region and reads it back 4 columns a lane, so
  // each store writes whole rows of its block (in the accumulator layout one store instruction
  // writes 16 bytes into each of 32 rows, which took 12% of a 256x256 tile's time) and the
  // residual is read the same way.  The region is the wave's own and LDS operations of a wave
  // complete in order, so no barrier separates its writes from its reads.  Rows past M and columns
  // past `cols` fall outside the buffer resources (stores dropped, loads 0): no branches.
  __syncthreads();
  auto store_staged = [&](auto wj, auto value, uint16_t* out, int ldc, int cols, int col0) __attribute__((always_inline)) {
    constexpr int WJ = decltype(wj)::value;
    constexpr int WC = WJ * 32;           // columns of a wave's block
    // without a residual to add, each value is rounded to bf16 before it is staged (the rounding
    // the store would make anyway), halving the staged bytes; with one, the fp32 sum needs fp32.
    // The persistent walk keeps fp32 staging: its bf16 form needs registers it does not have
    // (632 bytes of spills)
    constexpr bool kF32Stage = RESID || PERSIST;
    constexpr int kEl = kF32Stage ? 4 : 2;   // bytes per staged value
    constexpr int kPitch = WC * kEl + 16; // bytes per staged row: rows start 4 banks apart
    constexpr int LPR = WC / 4;           // lanes per row, 4 columns each
    constexpr int RPI = 64 / LPR;         // rows per instruction (96 columns: 2 rows, 48 lanes)
    static_assert(32 % RPI == 0, "whole instructions per 32-row block");
    static_assert(4 * 32 * kPitch <= Sh::kSmemBytes, "the staging regions fit in the ring's LDS");
    // a persistent walk keeps A slot 0 and B slot 0 free for the next tile's first stage: waves 0-2
    // stage in A slots 1-2, wave 3 in B slot 1
    static_assert(!PERSIST || (3 * 32 * kPitch <= 2 * kABytes && 32 * kPitch <= Sh::kBBytes),
                  "the persistent staging regions fit beside the next tile's first stage");
    uint8_t* const stage = !PERSIST ? smem + wave * (32 * kPitch)
                           : wave < 3 ? smem + kABytes + wave * (32 * kPitch)
                                      : smem + NSA * kABytes + Sh::kBBytes;
    const bool lane_on = lane < RPI * LPR;     // lanes past the last whole row store nothing
    const int rl = lane_on ? lane / LPR : 0, c4 = lane % LPR;
    const int gcol = col0 + 4 * c4;
    const uint32_t tile_bytes = uint32_t(min(BM, M - m0)) * uint32_t(ldc) * 2u;
    const __amdgpu_buffer_rsrc_t rsrc_c =
        __builtin_amdgcn_make_buffer_rsrc(out + int64_t(m0) * ldc, 0, tile_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rsrc_r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(RESID ? R + int64_t(m0) * ldc : out), 0, tile_bytes,
                                          0x00020000);
#pragma unroll
    for (int i = 0; i < WM; ++i) {
      const int r0 = wm * (BM / 2) + i * 32 + rl;   // tile row of this lane's first row
      uint32_t voff[32 / RPI];
#pragma unroll
      for (int t = 0; t < 32 / RPI; ++t)
        voff[t] = lane_on && gcol < cols ? (uint32_t(r0 + t * RPI) * uint32_t(ldc) + uint32_t(gcol)) * 2u
                                         : 0x80000000u;
      u32x2 rr[32 / RPI];
      if constexpr (RESID) {   // issued before the staging writes so their latency overlaps them
#pragma unroll
        for (int t = 0; t < 32 / RPI; ++t) rr[t] = __builtin_amdgcn_raw_buffer_load_b64(rsrc_r, voff[t], 0, 0);
      }
#pragma unroll
      for (int jj = 0; jj < WJ; ++jj)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4v v = value(i, jj, g);
          if constexpr (kF32Stage)
            *reinterpret_cast<f32x4v*>(stage + fr * kPitch + (jj * 32 + 8 * g + 4 * h) * 4) = v;
          else
            *reinterpret_cast<u32x2*>(stage + fr * kPitch + (jj * 32 + 8 * g + 4 * h) * 2) =
                u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
        }
      // every staged row of the block read back before the first conversion: the reads' latencies
      // overlap instead of adding up pair by pair
      using Staged = std::conditional_t<kF32Stage, f32x4v, u32x2>;
      Staged sv[32 / RPI];
#pragma unroll
      for (int t = 0; t < 32 / RPI; ++t)
        sv[t] = *reinterpret_cast<const Staged*>(stage + (t * RPI + rl) * kPitch + c4 * 4 * kEl);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int t = 0; t < 32 / RPI; ++t) {
        u32x2 packed;
        if constexpr (kF32Stage) {
          f32x4v v = sv[t];
          if constexpr (RESID) {
            v[0] += bf16_lo(rr[t][0]);
            v[1] += bf16_hi(rr[t][0]);
            v[2] += bf16_lo(rr[t][1]);
            v[3] += bf16_hi(rr[t][1]);
          }
          packed = u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
        } else {
          packed = sv[t];
        }
        __builtin_amdgcn_raw_buffer_store_b64(packed, rsrc_c, voff[t], 0, 0);
      }
      if constexpr (PERSIST) {
        static_assert(32 / RPI * (WM - WM / 2) == kStoresAfter, "the prologue's wait counts these stores");
        if (i == WM / 2 - 1) prefetch_next();   // half the stores out: the next tile's stage 0
      }
    }
  };
  if constexpr (MODE == kSwiGLU) {
    // pair jp of this wave: gate acc[i][2jp], up acc[i][2jp+1] -> output columns
    // n0 + 32*(wn*WN/2 + jp) + 8*(r/4) + 4*(lane/32) + r%4 of C [M, N/2]
    store_staged(std::integral_constant<int, WN / 2>{}, [&](int i, int jp, int g) __attribute__((always_inline)) {
      float gv[4], uv[4], bv[4], q[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        gv[e] = bf16_to_f32(f32_to_bf16(acc[i][2 * jp][4 * g + e]));
        uv[e] = bf16_to_f32(f32_to_bf16(acc[i][2 * jp + 1][4 * g + e]));
        bv[e] = __builtin_amdgcn_exp2f(-gv[e] * 1.4426950408889634f) + 1.0f;
        q[e] = silu_quotient(gv[e], bv[e]);
      }
      // one test per four outputs for the rare denominators past 2^126 (fmaxf skips a NaN b, whose
      // quotient the fixup already made NaN)
      if (__builtin_expect(fmaxf(fmaxf(bv[0], bv[1]), fmaxf(bv[2], bv[3])) >= 0x1p126f, 0)) {
#pragma unroll
        for (int e = 0; e < 4; ++e) q[e] = gv[e] / bv[e];
      }
      f32x4v o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = q[e] * uv[e];
      return o;
    }, C, N / 2, N / 2, n0 + wn * (BN / 4));
  } else {
    store_staged(std::integral_constant<int, WN>{}, [&](int i, int j, int g) __attribute__((always_inline)) {
      return f32x4v{acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
    }, C, N, N, n0 + wn * (BN / 2));
  }
  if (!has_next) break;
  __syncthreads();   // every wave has read its staged rows back: the next stages may land there
  tile_id = next_id;
  m0 = nm0;
  n0 = nn0;
  pre0 = true;
  }   // tile walk
}

// 256x256 and 256x128 tiles take 64-deep stages (whole-line A requests), 128x128 tiles 32-deep
// ones.  For 256x256 tiles the 3 A + 2 B slot rings beat 32-deep stages in 4-slot rings (same box:
// 4096x4096x12288 314.6 -> 306.8 us, SwiGLU 2048x4096x24576 305.7 -> 297.8 us, 2048x4096x6144
// 89.7 -> 86.5 us).
template <int WM, int WN>
constexpr int kBKOf = WM * WN >= 8 ? 64 : 32;

int cu_count();

template <int WM, int WN>
int launch_gemm(const void* a, const void* b, const void* residual, void* c, int64_t m, int64_t n, int64_t k,
                hipStream_t s) {
  using Sh = Shape<WM, WN, kBKOf<WM, WN>>;
  const int64_t tm = (m + Sh::BM - 1) / Sh::BM, tn = (n + Sh::BN - 1) / Sh::BN;
  if (tm * tn > 0x7fffffff) return PTB_ERR_GRID;
  const dim3 grid(unsigned(tm * tn)), block(kThreads);
  const Groups none{nullptr, nullptr, nullptr, 0, 0, 0, 0, 0};
  if constexpr (WM == 4 && WN == 4) {
    // two or more rounds of 256x256 tiles: one workgroup per CU walks its tiles
    const int64_t cus = cu_count();
    if (!residual && tm * tn >= 2 * cus) {
      gemm_bf16_kernel<4, 4, false, kPlain, 64, true><<<dim3(unsigned(cus)), block, 0, s>>>(
          static_cast<const uint16_t*>(a), static_cast<const uint16_t*>(b), nullptr, static_cast<uint16_t*>(c),
          int(m), int(n), int(k), int(tm), int(tn), none, nullptr, 0);
      return launch_status();
    }
  }
  if (residual)
    gemm_bf16_kernel<WM, WN, true, kPlain, kBKOf<WM, WN>><<<grid, block, 0, s>>>(
        static_cast<const uint16_t*>(a), static_cast<const uint16_t*>(b), static_cast<const uint16_t*>(residual),
        static_cast<uint16_t*>(c), int(m), int(n), int(k), int(tm), int(tn), none, nullptr, 0);
  else
    gemm_bf16_kernel<WM, WN, false, kPlain, kBKOf<WM, WN>><<<grid, block, 0, s>>>(
        static_cast<const uint16_t*>(a), static_cast<const uint16_t*>(b), nullptr, static_cast<uint16_t*>(c), int(m),
        int(n), int(k), int(tm), int(tn), none, nullptr, 0);
  return launch_status();
}

int cu_count() {
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess) hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  return cus;
}

// Tile shape (wm x wn waves of 64x64 blocks: 4x4 = 256x256, 4x3 = 256x192, 4x2 = 256x128,
// 2x2 = 128x128, 1x2 = 64x128) and K split of a GEMM.
struct GemmPlan {
  int wm, wn, splits;
  int64_t kchunk;   // K columns per split
};

// Split-K cost model for 64x128 tiles, fitted to the bundle's 97 GEMM shapes with M >= 8 (each
// (tile, split) timed on MI355X by HIP-graph replay): a launch costs kLaunchUs; a workgroup streams
// its (64 + 128) x K/S operand bytes at min(kWgBpus, kChipBpus / workgroups); a split adds the
// finish launch and 8 bytes of partial traffic (written, then read) per output per slice.
constexpr double kLaunchUs = 2.5, kFinishUs = 1.5;
constexpr double kWgBpus = 90e3;       // bytes per us one workgroup streams
constexpr double kChipBpus = 25e6;     // L2 -> CU bytes per us over the chip
constexpr double kPartialBpus = 2.5e6;

// The largest tile that still gives every CU a tile: 256x256, else 256x128 (from 3/4 of the CUs:
// one round of them beats 1.5 rounds of 128x128 tiles, 8192x3072x768 48.6 -> 35.3 us); then
// 128x128 while its tiles cover 3/4 of the CUs (or 64x128 ones would need a second round); else
// 64x128 (column tiles stay 128 wide: the B swizzle spans 16 chunks), its K split S ways (S fills at
// most one round, slices at least 256 deep, K >= 1024) when the model above says the split pays:
// over those 97 shapes the model's plans run 1.13x faster (geometric mean) than one pass of
// 128x128 tiles or 128x128 splits, within 0.3% of the best measured plan.  Where 256x256 tiles
// leave CUs idle but 256x128 ones would need a second round, 256x192 tiles when one round of them
// covers more CUs (the fused q|k|v projection, 2048x4096x6144: 256 tiles against 192), else 256x256:
// a 256x256 workgroup moves ~1.4x the flops per CU of a 256x128 one, so one round of it beats two
// of the smaller.
GemmPlan gemm_plan(int64_t m, int64_t n, int64_t k, bool may_split) {
  const int64_t cus = cu_count();
  auto tiles = [&](int64_t bm, int64_t bn) { return ((m + bm - 1) / bm) * ((n + bn - 1) / bn); };
  const int64_t t256 = tiles(256, 256), t256x192 = tiles(256, 192), t256x128 = tiles(256, 128);
  const int64_t t128 = tiles(128, 128), t64 = tiles(64, 128);
  if (t256 < cus && t256x128 > cus && t256x192 <= cus && t256x192 > t256) return {4, 3, 1, k};
  if (t256 >= cus || t256x128 > cus) return {4, 4, 1, k};
  if (4 * t256x128 >= 3 * cus) return {4, 2, 1, k};
  if (4 * t128 >= 3 * cus || (t64 > cus && 2 * t128 >= cus)) return {2, 2, 1, k};
  int best_s = 1;
  double best_t = 0.0;
  for (int sp = 1; sp <= 8; sp *= 2) {
    if (sp > 1 && (!may_split || k < 1024 || k / sp < 256 || t64 * sp > cus)) continue;
    const double wgs = double(t64 * sp);
    const double rate = std::min(kWgBpus, kChipBpus / std::min(wgs, double(cus)));
    double t = kLaunchUs + double(k) / sp * (64 + 128) * 2 / rate;
    if (sp > 1) t += kFinishUs + sp * double(m) * double(n) * 8 / kPartialBpus;
    if (sp == 1 || t < best_t) {
      best_t = t;
      best_s = sp;
    }
  }
  if (best_s == 1) return {1, 2, 1, k};
  const int64_t kc = ((k + best_s - 1) / best_s + 63) / 64 * 64;
  return {1, 2, int((k + kc - 1) / kc), kc};
}

int launch_planned(const GemmPlan& p, const void* a, const void* b, const void* residual, void* c, int64_t m,
                   int64_t n, int64_t k, hipStream_t s) {
  if (p.wm == 4 && p.wn == 3) return launch_gemm<4, 3>(a, b, residual, c, m, n, k, s);
  if (p.wm == 4 && p.wn == 4) return launch_gemm<4, 4>(a, b, residual, c, m, n, k, s);
  if (p.wm == 4 && p.wn == 2) return launch_gemm<4, 2>(a, b, residual, c, m, n, k, s);
  if (p.wm == 2 && p.wn == 2) return launch_gemm<2, 2>(a, b, residual, c, m, n, k, s);
  return launch_gemm<1, 2>(a, b, residual, c, m, n, k, s);
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
  if ((k + kRunAhead) * n * 2 >= (int64_t(1) << 32) || int64_t(256) * k * 2 >= (int64_t(1) << 32) ||
      n > kMaxOutCols)
    return PTB_ERR_UNSUPPORTED;
  if (!aligned16(a) || !aligned16(b) || !aligned16(c) || (residual && !aligned16(residual)))
    return PTB_ERR_ALIGN;
  return launch_planned(gemm_plan(m, n, k, false), a, b, residual, c, m, n, k, static_cast<hipStream_t>(stream));
}

namespace {

// C = bf16(sum_s P[s] (+ R)), 4 consecutive elements per thread.
// Eight slices' loads go out before any is added (a plain loop waits for each in turn); the sum
// keeps the slice order, P_0 + P_1 + ... .
__global__ __launch_bounds__(256) void splitk_finish(const float* __restrict__ P, int splits, int64_t mn,
                                                     const uint16_t* __restrict__ R, uint16_t* __restrict__ C) {
  const int64_t q = (int64_t(blockIdx.x) * 256 + threadIdx.x) * 4;
  if (q >= mn) return;
  f32x4v acc = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < splits; s0 += 8) {
    f32x4v v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int sl = s0 + u < splits ? s0 + u : splits - 1;
      v[u] = *reinterpret_cast<const f32x4v*>(P + int64_t(sl) * mn + q);
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int sl = s0 + u;
      acc = sl == 0 ? v[u] : (sl < splits ? acc + v[u] : acc);
    }
  }
  if (R) {
    const u32x2 rr = *reinterpret_cast<const u32x2*>(R + q);
    acc.x += bf16_lo(rr[0]);
    acc.y += bf16_hi(rr[0]);
    acc.z += bf16_lo(rr[1]);
    acc.w += bf16_hi(rr[1]);
  }
  *reinterpret_cast<u32x2*>(C + q) = u32x2{pack_bf16x2(acc.x, acc.y), pack_bf16x2(acc.z, acc.w)};
}

}  // namespace

PTB_EXPORT size_t ptb_gemm_bf16_workspace_bytes(int64_t m, int64_t n, int64_t k) {
  if (m <= 0 || n <= 0 || k <= 0 || m > 0x7fffffff || n > 0x7fffffff || k > 0x7fffffff) return 0;
  const GemmPlan p = gemm_plan(m, n, k, true);
  if (p.splits < 2) return 0;
  return size_t(p.splits) * size_t(m) * size_t(n) * sizeof(float);
}

PTB_EXPORT int ptb_gemm_bf16_ws(const void* a, const void* b, const void* residual, void* c, int64_t m, int64_t n,
                                int64_t k, void* workspace, size_t workspace_bytes, void* stream) {
  if (m <= 0 || n <= 0 || k <= 0 || k % 64 || n % 8 || m > 0x7fffffff || n > 0x7fffffff || k > 0x7fffffff)
    return ptb_gemm_bf16(a, b, residual, c, m, n, k, stream);   // refused or trivial there
  const GemmPlan p = gemm_plan(m, n, k, true);
  if (p.splits < 2) return ptb_gemm_bf16(a, b, residual, c, m, n, k, stream);   // no split for this shape
  if (!a || !b || !c || !workspace) return PTB_ERR_NULL;
  if (workspace_bytes < ptb_gemm_bf16_workspace_bytes(m, n, k)) return PTB_ERR_WORKSPACE;
  using Sh = Shape<1, 2, kBKOf<1, 2>>;   // the split plans use 64x128 tiles
  if ((k + kRunAhead) * n * 2 >= (int64_t(1) << 32) || int64_t(Sh::BM) * k * 2 >= (int64_t(1) << 32))
    return PTB_ERR_UNSUPPORTED;
  if (!aligned16(a) || !aligned16(b) || !aligned16(c) || !aligned16(workspace) || (residual && !aligned16(residual)))
    return PTB_ERR_ALIGN;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t tm = (m + Sh::BM - 1) / Sh::BM, tn = (n + Sh::BN - 1) / Sh::BN;
  if (tm * tn > 0x7fffffff) return PTB_ERR_GRID;
  const Groups none{nullptr, nullptr, nullptr, 0, 0, 0, 0, 0};
  float* part = static_cast<float*>(workspace);
  const int splits = p.splits;
  const dim3 grid(unsigned(tm * tn), unsigned(splits));
  gemm_bf16_kernel<1, 2, false, kSplit, kBKOf<1, 2>><<<grid, dim3(kThreads), 0, s>>>(
        static_cast<const uint16_t*>(a), static_cast<const uint16_t*>(b), nullptr, nullptr, int(m), int(n), int(k),
        int(tm), int(tn), none, part, int(p.kchunk));
  const int64_t mn = m * n;
  splitk_finish<<<dim3(unsigned((mn / 4 + 255) / 256)), dim3(256), 0, s>>>(
      part, splits, mn, static_cast<const uint16_t*>(residual), static_cast<uint16_t*>(c));
  return launch_status();
}

PTB_EXPORT int ptb_gemm_swiglu_bf16(const void* a, const void* b, void* c, int64_t m, int64_t inter, int64_t k,
                                    void* stream) {
  if (m < 0 || inter < 0 || k < 0) return PTB_ERR_SHAPE;
  if (m == 0 || inter == 0) return PTB_OK;
  if (!a || !b || !c) return PTB_ERR_NULL;
  if (k == 0 || k % 64 || inter % 128) return PTB_ERR_UNSUPPORTED;
  const int64_t n = 2 * inter;
  if (m > 0x7fffffff || n > 0x7fffffff || k > 0x7fffffff) return PTB_ERR_SHAPE;
  if ((k + kRunAhead) * n * 2 >= (int64_t(1) << 32) || int64_t(256) * k * 2 >= (int64_t(1) << 32) ||
      n > kMaxOutCols)
    return PTB_ERR_UNSUPPORTED;
  if (!aligned16(a) || !aligned16(b) || !aligned16(c)) return PTB_ERR_ALIGN;
  const int64_t tm = (m + 255) / 256, tn = inter / 128;
  if (tm * tn > 0x7fffffff) return PTB_ERR_GRID;
  const Groups none{nullptr, nullptr, nullptr, 0, 0, 0, 0, 0};
  gemm_bf16_kernel<4, 4, false, kSwiGLU, kBKOf<4, 4>><<<dim3(unsigned(tm * tn)), dim3(kThreads), 0,
                                                        static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t*>(a), static_cast<const uint16_t*>(b), nullptr, static_cast<uint16_t*>(c), int(m),
      int(n), int(k), int(tm), int(tn), none, nullptr, 0);
  return launch_status();
}

PTB_EXPORT int ptb_grouped_gemm_bf16(const void* a, const void* b, const int32_t* group, const int32_t* start,
                                     const int32_t* rows, void* c, int64_t nprog, int64_t ntab, int64_t a_rows,
                                     int64_t nweights, int64_t k, int64_t n, int64_t weight_stride, void* stream) {
  if (nprog < 0 || ntab < 0 || a_rows < 0 || nweights < 0 || k < 0 || n < 0) return PTB_ERR_SHAPE;
  if (nprog == 0 || a_rows == 0 || n == 0) return PTB_OK;
  if (!a || !b || !group || !start || !rows || !c) return PTB_ERR_NULL;
  if (k == 0 || k % 64 || n % 8 || nprog > kMaxPrograms) return PTB_ERR_UNSUPPORTED;
  if (weight_stride < k * n || a_rows > 0x7fffffff || ntab > 0x7fffffff || nweights > 0x7fffffff) return PTB_ERR_SHAPE;
  if ((k + kRunAhead) * n * 2 >= (int64_t(1) << 32) || int64_t(128) * k * 2 >= (int64_t(1) << 32) ||
      n > kMaxOutCols)
    return PTB_ERR_UNSUPPORTED;
  if (!aligned16(a) || !aligned16(b) || !aligned16(c) || (weight_stride % 8)) return PTB_ERR_ALIGN;
  // a bound on the row tiles of every program together: each program's rows lie inside A
  const int64_t tn = (n + 127) / 128, tm_bound = (a_rows + 127) / 128 + nprog;
  if (tm_bound * tn > 0x7fffffff) return PTB_ERR_GRID;
  const Groups gp{group, start, rows, int(nprog), int(ntab), int(nweights), int(a_rows), weight_stride};
  gemm_bf16_kernel<2, 2, false, kGrouped><<<dim3(unsigned(tm_bound * tn)), dim3(kThreads), 0,
                                            static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t*>(a), static_cast<const uint16_t*>(b), nullptr, static_cast<uint16_t*>(c), 0, int(n),
      int(k), 0, int(tn), gp, nullptr, 0);
  return launch_status();
}
