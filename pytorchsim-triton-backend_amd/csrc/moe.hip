// Mixture-of-experts routing, bookkeeping and combine kernels for gfx950 (the Qwen3-30B-A3B layer
// of the validation bundle): fills and integer casts, scans over the expert table, the expert
// histogram with each slot's rank inside its expert, a stable key sort, top-k, the row gather
// that lays tokens out expert by expert, the weighted combine back to tokens, and the small
// elementwise / row kernels the layer launches around them.  Integer work is exact; floating
// point is fp32 with one rounding where the reference stores bf16.
//
// Indices read from memory are bounds-checked here: where the reference's kernels stop on a
// device_assert, these write zeros for the offending element instead of reading out of bounds.
#include "ptb_common.h"

#include <type_traits>

using namespace ptb;

namespace {

constexpr int kB = 256;

__device__ __forceinline__ void ld8(const uint16_t* __restrict__ p, float (&f)[8]) {
  const u32x4 v = *reinterpret_cast<const u32x4*>(p);
  f[0] = bf16_lo(v[0]); f[1] = bf16_hi(v[0]); f[2] = bf16_lo(v[1]); f[3] = bf16_hi(v[1]);
  f[4] = bf16_lo(v[2]); f[5] = bf16_hi(v[2]); f[6] = bf16_lo(v[3]); f[7] = bf16_hi(v[3]);
}
__device__ __forceinline__ void st8(uint16_t* __restrict__ p, const float (&f)[8]) {
  *reinterpret_cast<u32x4*>(p) = u32x4{pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]),
                                       pack_bf16x2(f[6], f[7])};
}
__device__ __forceinline__ void ld8f(const float* __restrict__ p, float (&f)[8]) {
  const f32x4v a = reinterpret_cast<const f32x4v*>(p)[0], b = reinterpret_cast<const f32x4v*>(p)[1];
  f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w; f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
}

// Python-style floor division of a by a positive divisor d.
__device__ __forceinline__ int64_t floordiv(int64_t a, int64_t d) {
  const int64_t q = a / d;
  return (a % d != 0 && a < 0) ? q - 1 : q;
}
// The index-wrap rule of the reference's gathers: i in [-n, 0) counts from the end; returns -1
// for anything still outside [0, n).
__device__ __forceinline__ int64_t wrap_index(int64_t i, int64_t n) {
  if (i < 0) i += n;
  return (i >= 0 && i < n) ? i : -1;
}

// ---------------------------------------------------------------- fill / cast
__global__ __launch_bounds__(kB) void fill_zero_u32(uint32_t* __restrict__ p, int64_t n) {
  for (int64_t i = int64_t(blockIdx.x) * kB + threadIdx.x; i < n; i += int64_t(gridDim.x) * kB) p[i] = 0u;
}
__global__ __launch_bounds__(kB) void fill_zero_u8(uint8_t* __restrict__ p, int64_t n) {
  for (int64_t i = int64_t(blockIdx.x) * kB + threadIdx.x; i < n; i += int64_t(gridDim.x) * kB) p[i] = 0u;
}
__global__ __launch_bounds__(kB) void cast_i64_i32(const int64_t* __restrict__ x, int32_t* __restrict__ y, int64_t n) {
  for (int64_t i = int64_t(blockIdx.x) * kB + threadIdx.x; i < n; i += int64_t(gridDim.x) * kB)
    y[i] = int32_t(uint32_t(uint64_t(x[i])));   // the low 32 bits, as a two's-complement cast
}

// ---------------------------------------------------------------- single-block scans
constexpr int kScanThreads = 1024, kScanPer = 8, kScanMax = kScanThreads * kScanPer;

// Exclusive prefix of the per-thread totals (int64) over the block: an inclusive scan within each
// wave (shift-up shuffles), then every wave adds the totals of the waves before it (one LDS pass,
// two barriers).  All kScanThreads threads call it; `s` holds at least one int64 per wave.
__device__ __forceinline__ int64_t block_exclusive_scan(int64_t t, int64_t* s) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int64_t v = t;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int64_t u = __shfl_up(v, off, 64);
    v += lane >= off ? u : 0;
  }
  if (lane == 63) s[w] = v;
  __syncthreads();
  int64_t before = 0;
  for (int i = 0; i < w; ++i) before += s[i];
  __syncthreads();   // s is reused by the caller's next scan
  return before + v - t;
}

template <typename InT, typename OutT>
__global__ __launch_bounds__(kScanThreads) void cumsum_block(const InT* __restrict__ x, OutT* __restrict__ y0,
                                                             OutT* __restrict__ y1, int n) {
  __shared__ int64_t s[kScanThreads];
  int64_t v[kScanPer];
  int64_t t = 0;
  const int base = threadIdx.x * kScanPer;
#pragma unroll
  for (int i = 0; i < kScanPer; ++i) {
    v[i] = base + i < n ? int64_t(x[base + i]) : 0;
    t += v[i];
  }
  int64_t run = block_exclusive_scan(t, s);
#pragma unroll
  for (int i = 0; i < kScanPer; ++i) {
    run += v[i];
    if (base + i < n) {
      y0[base + i] = OutT(run);
      if (y1) y1[base + i] = OutT(run);
    }
  }
}

// From inclusive group ends: starts[i] = ends[i-1] (0 for i = 0), rows[i] = ends[i] - starts[i],
// nonempty[i] = number of groups j <= i with rows[j] > 0.
template <typename InT>
__global__ __launch_bounds__(kScanThreads) void group_table_block(const InT* __restrict__ ends, int n,
                                                                  int64_t* __restrict__ nonempty,
                                                                  int64_t* __restrict__ starts,
                                                                  int64_t* __restrict__ rows) {
  __shared__ int64_t s[kScanThreads];
  int64_t f[kScanPer];
  int64_t t = 0;
  const int base = threadIdx.x * kScanPer;
#pragma unroll
  for (int i = 0; i < kScanPer; ++i) {
    const int j = base + i;
    f[i] = 0;
    if (j < n) {
      const int64_t st = j == 0 ? 0 : int64_t(ends[j - 1]);
      const int64_t r = int64_t(ends[j]) - st;
      starts[j] = st;
      rows[j] = r;
      f[i] = r > 0 ? 1 : 0;
    }
    t += f[i];
  }
  int64_t run = block_exclusive_scan(t, s);
#pragma unroll
  for (int i = 0; i < kScanPer; ++i) {
    run += f[i];
    if (base + i < n) nonempty[base + i] = run;
  }
}

// out[i] = number of r with x[r] <= i, for i < m: x staged through LDS in blocks of kB values.
__global__ __launch_bounds__(kB) void count_le(const int64_t* __restrict__ x, int64_t n, int32_t* __restrict__ out,
                                               int64_t m) {
  __shared__ int64_t xs[kB];
  const int64_t i = int64_t(blockIdx.x) * kB + threadIdx.x;
  int64_t c = 0;
  for (int64_t r0 = 0; r0 < n; r0 += kB) {
    const int64_t cnt = n - r0 < kB ? n - r0 : kB;
    if (threadIdx.x < cnt) xs[threadIdx.x] = x[r0 + threadIdx.x];
    __syncthreads();
    for (int j = 0; j < cnt; ++j) c += xs[j] <= i ? 1 : 0;
    __syncthreads();
  }
  if (i < m) out[i] = int32_t(c);
}

// ---------------------------------------------------------------- expert histogram and ranks
// Block b owns slots [64 b, 64 b + 64): it histograms the slots before its range (LDS atomics),
// then walks its own slots in order, so thread x carries the running count of expert x and
// writes cum[r, x] = #{r' <= r : ids[r'] == x} for its slots (a coalesced row of E counts).
// The block holding the last slot writes the totals.
constexpr int kSlotsPerBlock = 64;
__global__ __launch_bounds__(kB) void expert_count(const int64_t* __restrict__ ids, int64_t r, int e,
                                                   int64_t* __restrict__ counts, int64_t* __restrict__ counts2,
                                                   int64_t* __restrict__ cum) {
  __shared__ int hist[1024];
  __shared__ int64_t mine[kSlotsPerBlock];
  const int64_t r0 = int64_t(blockIdx.x) * kSlotsPerBlock;
  const int64_t left = r - r0;
  const int nr = int(left <= 0 ? 0 : (left < kSlotsPerBlock ? left : kSlotsPerBlock));
  for (int x = threadIdx.x; x < e; x += kB) hist[x] = 0;
  if (threadIdx.x < nr) mine[threadIdx.x] = ids[r0 + threadIdx.x];
  __syncthreads();
  for (int64_t q = threadIdx.x; q < r0; q += kB) {
    const int64_t id = ids[q];
    if (id >= 0 && id < e) atomicAdd(&hist[id], 1);
  }
  __syncthreads();
  const bool last = r0 + kSlotsPerBlock >= r;
  for (int x = threadIdx.x; x < e; x += kB) {
    int64_t run = hist[x];
    for (int j = 0; j < nr; ++j) {
      run += mine[j] == x ? 1 : 0;
      cum[(r0 + j) * e + x] = run;
    }
    if (last) {
      counts[x] = run;
      if (counts2) counts2[x] = run;
    }
  }
}

// out[s] = cum[s, ids[s]] (the slot's 1-based rank inside its expert), 0 when ids[s] is not an expert.
__global__ __launch_bounds__(kB) void rank_select(const int64_t* __restrict__ cum, const int64_t* __restrict__ ids,
                                                  int64_t r, int64_t e, int64_t* __restrict__ out) {
  const int64_t s = int64_t(blockIdx.x) * kB + threadIdx.x;
  if (s >= r) return;
  const int64_t id = ids[s];
  out[s] = (id >= 0 && id < e) ? cum[s * e + id] : 0;
}

// ---------------------------------------------------------------- stable key sort
// Keys become int64 with the same order: integers as they are, floats through their sign-magnitude
// bits (NaN as one canonical NaN above +inf, -0 as +0); descending order complements the keys.
// Ties keep the original position order, so (key, position) is a strict total order and the
// sorted result is unique.
__device__ __forceinline__ int64_t sort_key(const void* x, int64_t i, bool is_f32, bool desc) {
  int64_t k;
  if (is_f32) {
    const float v = static_cast<const float*>(x)[i];
    int32_t b = v != v ? 0x7FC00000 : (v == 0.f ? 0 : __float_as_int(v));
    b ^= (b >> 31) & 0x7FFFFFFF;
    k = int64_t(b);
  } else {
    k = static_cast<const int64_t*>(x)[i];
  }
  return desc ? ~k : k;
}
__device__ __forceinline__ void store_sorted(void* v, int64_t* idx, int64_t at, int64_t k, int32_t pos, bool is_f32,
                                             bool desc) {
  if (desc) k = ~k;
  if (is_f32) {
    int32_t b = int32_t(k);
    b ^= (b >> 31) & 0x7FFFFFFF;
    static_cast<float*>(v)[at] = __int_as_float(b);
  } else {
    static_cast<int64_t*>(v)[at] = k;
  }
  idx[at] = pos;
}
__device__ __forceinline__ bool key_less(int64_t ka, int32_t ia, int64_t kb, int32_t ib) {
  return (ka < kb) | ((ka == kb) & (ia < ib));   // bitwise: no short-circuit branches
}

// Rows of at most kRankSortMax keys: one workgroup per row, a key per thread in LDS; the stable
// position of key i is the number of keys ordered before it (smaller, or equal at a lower
// position), counted in one pass over the row's keys (the bitonic network's log^2 stages of
// barriers cost more than these few hundred compares).
constexpr int kRankSortMax = 256;
__global__ __launch_bounds__(kRankSortMax) void sort_rank(const void* __restrict__ x, int e, bool is_f32, bool desc,
                                                          void* __restrict__ v, int64_t* __restrict__ idx) {
  __shared__ int64_t ks[kRankSortMax];
  const int64_t row = blockIdx.x;
  const int i = threadIdx.x;
  const void* xr = is_f32 ? static_cast<const void*>(static_cast<const float*>(x) + row * e)
                          : static_cast<const void*>(static_cast<const int64_t*>(x) + row * e);
  const int64_t k = sort_key(xr, i < e ? i : e - 1, is_f32, desc);
  ks[i] = k;
  __syncthreads();
  if (i >= e) return;
  int rank = 0;
#pragma unroll 8
  for (int j = 0; j < e; ++j) {
    const int64_t o = ks[j];
    rank += int((o < k) | ((o == k) & (j < i)));
  }
  store_sorted(static_cast<uint8_t*>(v) + row * e * (is_f32 ? 4 : 8), idx + row * e, rank, k, i, is_f32, desc);
}

constexpr int kSortChunk = 8192;   // elements one workgroup sorts in LDS (96 KB)
constexpr int kSortThreads = 1024;

// Bitonic network over p = kSortThreads * R elements held R per thread (element g = tid*R + r):
// strides below R run in registers, the rest exchange through LDS.  Elements are unsigned words
// whose order is the wanted (key, position) order, so each step is one min / max.
// LDS slot of element g: one pad word after every 8, so the R = 8 words a thread writes (and the
// partner words it reads) fall in distinct banks across the wave.
__device__ __forceinline__ int lds_slot(int g) { return g + (g >> 3); }

template <typename W, int R>
__device__ __forceinline__ void bitonic_packed(W (&v)[R], W* lds, int p) {
  const int base = threadIdx.x * R;
  for (int size = 2; size <= p; size <<= 1) {
    // strides of size/2 .. R: partners in other threads, through LDS
    for (int stride = size >> 1; stride >= R; stride >>= 1) {
#pragma unroll
      for (int r = 0; r < R; ++r) lds[lds_slot(base + r)] = v[r];
      __syncthreads();
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int g = base + r;
        const W o = lds[lds_slot(g ^ stride)];
        const bool keep_min = ((g & stride) == 0) == ((g & size) == 0);
        const W lo = v[r] < o ? v[r] : o, hi = v[r] < o ? o : v[r];
        v[r] = keep_min ? lo : hi;
      }
      __syncthreads();
    }
    // strides below R: partners in this thread's registers (compile-time indices)
#pragma unroll
    for (int st = R / 2; st > 0; st >>= 1) {
      if (st < size) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
          if (r & st) continue;
          const bool up = ((base + r) & size) == 0;
          const W a = v[r], b = v[r | st];
          const W lo = a < b ? a : b, hi = a < b ? b : a;
          v[r] = up ? lo : hi;
          v[r | st] = up ? hi : lo;
        }
      }
    }
  }
}

// Sort one chunk of p (power of two, <= kSortChunk) elements of row blockIdx.x, chunk blockIdx.y.
// When the chunk's keys span a small enough range the (key, position) pair is packed into one
// 32-bit word (key range < 2^(32 - log2 p): expert ids) or one 64-bit word (range < 2^32: floats,
// int32-sized integers), and sorted as plain unsigned words in registers + LDS; any other int64
// keys take the general compare-exchange over separate key / position arrays.  final_out: write
// values + indices of the row, else (key, position) pairs to the workspace for the merge passes.
__global__ __launch_bounds__(kSortThreads) void sort_chunk(const void* __restrict__ x, int64_t e, int p, bool is_f32,
                                                           bool desc, bool final_out, void* __restrict__ v,
                                                           int64_t* __restrict__ idx, int64_t* __restrict__ wk,
                                                           int32_t* __restrict__ wi) {
  __shared__ __attribute__((aligned(16))) uint8_t lds_raw[kSortChunk * 12];   // >= (8192 + 1024) * 8 B packed
  __shared__ int64_t red_min[kSortThreads / kWave], red_max[kSortThreads / kWave];
  int64_t* key = reinterpret_cast<int64_t*>(lds_raw);
  int32_t* pos = reinterpret_cast<int32_t*>(lds_raw + kSortChunk * 8);
  const int64_t row = blockIdx.x, c0 = int64_t(blockIdx.y) * p;
  const void* xr = is_f32 ? static_cast<const void*>(static_cast<const float*>(x) + row * e)
                          : static_cast<const void*>(static_cast<const int64_t*>(x) + row * e);
  // keys (padding past e with the largest key) and their range over the chunk's live elements
  int64_t kmin = INT64_MAX, kmax = INT64_MIN;
  constexpr int kPer = kSortChunk / kSortThreads;   // every load of the chunk issued before the first use
  int64_t kk[kPer];
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    const int i = threadIdx.x + q * kSortThreads;
    const int64_t g = c0 + i;
    kk[q] = (i < p && g < e) ? sort_key(xr, g, is_f32, desc) : INT64_MAX;
  }
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    const int i = threadIdx.x + q * kSortThreads;
    if (i < p) {
      key[i] = kk[q];
      if (c0 + i < e) {
        kmin = kk[q] < kmin ? kk[q] : kmin;
        kmax = kk[q] > kmax ? kk[q] : kmax;
      }
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const int64_t a = __shfl_xor(kmin, off, kWave), b = __shfl_xor(kmax, off, kWave);
    kmin = a < kmin ? a : kmin;
    kmax = b > kmax ? b : kmax;
  }
  if (threadIdx.x % kWave == 0) {
    red_min[threadIdx.x / kWave] = kmin;
    red_max[threadIdx.x / kWave] = kmax;
  }
  __syncthreads();
  kmin = red_min[0];
  kmax = red_max[0];
  for (int w = 1; w < kSortThreads / kWave; ++w) {
    kmin = red_min[w] < kmin ? red_min[w] : kmin;
    kmax = red_max[w] > kmax ? red_max[w] : kmax;
  }
  int pbits = 0;
  while ((1 << pbits) < p) ++pbits;
  // range + 1 distinct key codes, one more for the padding: code = key - kmin, padding = range + 1
  const uint64_t range = kmax >= kmin ? uint64_t(kmax) - uint64_t(kmin) : 0;
  const int mode = (p >= kSortThreads && p % kSortThreads == 0)
                       ? (range + 1 < (uint64_t(1) << (32 - pbits)) ? 1 : (range + 1 < (uint64_t(1) << 32) ? 2 : 0))
                       : 0;
  const auto emit = [&](int i, int64_t k, int32_t ps) __attribute__((always_inline)) {
    const int64_t g = c0 + i;
    if (final_out) {
      if (g < e) store_sorted(static_cast<uint8_t*>(v) + row * e * (is_f32 ? 4 : 8), idx + row * e, g, k, ps, is_f32, desc);
    } else {
      wk[row * int64_t(gridDim.y) * p + g] = k;
      wi[row * int64_t(gridDim.y) * p + g] = ps;
    }
  };
  if (mode == 1 || mode == 2) {
    const int r_per = p / kSortThreads;   // 1 .. 8
    __syncthreads();                      // keys complete before the packed words overwrite them
    const auto run = [&](auto tag, auto rtag) __attribute__((always_inline)) {
      using W = decltype(tag);
      constexpr int R = decltype(rtag)::value;
      W w[R];
      const int shift = mode == 1 ? pbits : 32;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int i = threadIdx.x * R + r;
        const int64_t g = c0 + i;
        const uint64_t code = g < e ? uint64_t(key[i]) - uint64_t(kmin) : range + 1;
        w[r] = W((code << shift) | uint64_t(i));
      }
      __syncthreads();
      bitonic_packed<W, R>(w, reinterpret_cast<W*>(lds_raw), p);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int i = threadIdx.x * R + r;
        const uint64_t u = uint64_t(w[r]);
        const int32_t local = int32_t(u & ((uint64_t(1) << shift) - 1));
        const uint64_t code = u >> shift;
        const int64_t k = code > range ? INT64_MAX : int64_t(uint64_t(kmin) + code);
        emit(i, k, int32_t(c0 + local));
      }
    };
    const auto dispatch_r = [&](auto tag) __attribute__((always_inline)) {
      if (r_per == 1) run(tag, std::integral_constant<int, 1>{});
      else if (r_per == 2) run(tag, std::integral_constant<int, 2>{});
      else if (r_per == 4) run(tag, std::integral_constant<int, 4>{});
      else run(tag, std::integral_constant<int, 8>{});
    };
    if (mode == 1) dispatch_r(uint32_t{});
    else dispatch_r(uint64_t{});
    return;
  }
  for (int i = threadIdx.x; i < p; i += kSortThreads) pos[i] = int32_t(c0 + i);
  __syncthreads();
  for (int size = 2; size <= p; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int t = threadIdx.x; t < p / 2; t += kSortThreads) {
        const int lo = 2 * t - (t & (stride - 1));   // t with a zero bit inserted at `stride`
        const int hi = lo + stride;
        const bool up = (lo & size) == 0;
        const int64_t ka = key[lo], kb = key[hi];
        const int32_t ia = pos[lo], ib = pos[hi];
        if (key_less(kb, ib, ka, ia) == up) {
          key[lo] = kb; key[hi] = ka;
          pos[lo] = ib; pos[hi] = ia;
        }
      }
      __syncthreads();
    }
  }
  for (int i = threadIdx.x; i < p; i += kSortThreads) emit(i, key[i], pos[i]);
}

// One merge pass over runs of length run (a power of two): each element finds its place in the
// merged pair by a binary search of the other run.  Runs are contiguous ranges of positions and
// the left run's positions are all smaller, so equal keys of the left run come first.
__global__ __launch_bounds__(kB) void sort_merge(const int64_t* __restrict__ sk, const int32_t* __restrict__ si,
                                                 int64_t* __restrict__ dk, int32_t* __restrict__ di, int64_t total,
                                                 int64_t run) {
  const int64_t g = int64_t(blockIdx.x) * kB + threadIdx.x;
  if (g >= total) return;
  const int64_t pair = g / (2 * run), off = g - pair * 2 * run;
  const bool left = off < run;
  const int64_t base = pair * 2 * run;
  const int64_t other = left ? base + run : base;
  const int64_t k = sk[g];
  int64_t lo = 0, hi = run;   // count of elements in the other run ordered before this one
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    const int64_t ko = sk[other + mid];
    const bool before = left ? (ko < k) : (ko <= k);
    if (before) lo = mid + 1;
    else hi = mid;
  }
  const int64_t at = base + (left ? off : off - run) + lo;
  dk[at] = k;
  di[at] = si[g];
}

__global__ __launch_bounds__(kB) void sort_emit(const int64_t* __restrict__ sk, const int32_t* __restrict__ si,
                                                int64_t e, int64_t padded, bool is_f32, bool desc, void* __restrict__ v,
                                                int64_t* __restrict__ idx, int64_t rows) {
  const int64_t g = int64_t(blockIdx.x) * kB + threadIdx.x;
  if (g >= rows * e) return;
  const int64_t row = g / e, i = g - row * e;
  const int64_t at = row * padded + i;
  store_sorted(v, idx, g, sk[at], si[at], is_f32, desc);
}

// ---------------------------------------------------------------- top-k
// The reference's k rounds of "take the best, lowest position first, mark it spent (-inf for the
// largest, +inf for the smallest)".  Elements other than the spent value come out in order of value,
// larger first (smaller first for largest = false), equal values by lower position; a NaN, which
// the reference's comparisons leave to the backend, ranks after every number (for either
// direction) and NaNs among themselves by position (the 32-bit key below).  An element holding the
// spent value is never taken as itself: once the others are used up, every further round finds
// only spent values and reports (spent, position 0), as the reference's rounds do.
// order-preserving bits of a float: larger value, larger unsigned key
__device__ __forceinline__ uint32_t order_bits(float v) {
  const uint32_t u = __float_as_uint(v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
// The key of element v of a row searched for its largest (v already negated for smallest-k): a NaN
// gets 1, below every number's key and above 0, the key of taken, absent and spent (-inf) elements;
// -0 and +0 share a key, as they compare equal.
__device__ __forceinline__ uint32_t topk_key(float v) {
  return v != v ? 1u : (v == 0.f ? 0x80000000u : (v == -INFINITY ? 0u : order_bits(v)));
}

// One wave per row, the keys in LDS: element c's rank is the number of elements ordered before it
// (a larger key, or an equal key at a lower position); the elements of rank < k other than spent
// ones are the selected, in order, and ranks from the count of the others up to k report (spent, 0).
constexpr int kTopkMax = 1024;   // row length
constexpr int kTopkRows = kB / kWave;
__global__ __launch_bounds__(kB) void topk_rows(const float* __restrict__ x, int64_t rows, int e, int k, bool largest,
                                                float* __restrict__ vals, int64_t* __restrict__ idx) {
  __shared__ __attribute__((aligned(16))) uint32_t sk[kTopkRows][kTopkMax];
  const int w = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int64_t row = int64_t(blockIdx.x) * kTopkRows + w;
  if (row >= rows) return;   // a whole wave; no block barrier below
  uint32_t* r = sk[w];
  // smallest-k is largest-k of the negated values (negation reverses the order, keeps ties)
  const float sgn = largest ? 1.0f : -1.0f;
  const int e4 = (e + 3) & ~3;   // padded with key 0, which never ranks before a real element
  for (int c = lane; c < e4; c += kWave) r[c] = c < e ? topk_key(sgn * x[row * e + c]) : 0u;
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  const u32x4* r4 = reinterpret_cast<const u32x4*>(r);
  for (int c = lane; c < e; c += kWave) {
    const uint32_t v = r[c];
    int rank = 0;
#pragma unroll 8
    for (int q = 0; q < e4 / 4; ++q) {
      const u32x4 o = r4[q];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int j = 4 * q + t;
        rank += int((o[t] > v) | ((o[t] == v) & (j < c)));   // bitwise: no short-circuit branches
      }
    }
    if (v != 0u && rank < k) {
      vals[row * k + rank] = x[row * e + c];
      idx[row * k + rank] = c;
    }
  }
  int present = 0;   // elements other than spent ones: at most 1024, exact in the fp32 sum
  for (int c = lane; c < e; c += kWave) present += r[c] != 0u;
  present = int(wave_sum(float(present)));
  for (int n = present + lane; n < k; n += kWave) {
    vals[row * k + n] = largest ? -INFINITY : INFINITY;
    idx[row * k + n] = 0;
  }
}

// Top-k with k <= 64 of rows of at most 64*R elements: one wave per row with the row in registers
// (lane l holds elements l, l + 64, ...), every load in flight at once, then k rounds of a wave
// argmax over the elements not yet taken.  The 64-bit key (topk_key of the value, then the inverted
// position) makes a round's winner the largest value and, among equal values, the lowest position:
// the same selection and order as the rank kernel above.  Taken, absent and spent elements hold key
// 0, below every present one; a round whose winner is key 0 reports (spent, 0).
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return uint32_t(__builtin_amdgcn_update_dpp(0, int(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ void key_max(uint32_t& h, uint32_t& l, uint32_t oh, uint32_t ol) {
  const bool b = (oh > h) | ((oh == h) & (ol > l));
  h = b ? oh : h;
  l = b ? ol : l;
}
// Wave-wide max of the 64-bit keys (h, l); every lane gets it.  The permlane swaps move h and l by
// the same permutation, so each returned pair is one lane's key.
__device__ __forceinline__ void wave_key_max(uint32_t& h, uint32_t& l) {
  key_max(h, l, dpp_u32<0xb1>(h), dpp_u32<0xb1>(l));
  key_max(h, l, dpp_u32<0x4e>(h), dpp_u32<0x4e>(l));
  key_max(h, l, dpp_u32<0x141>(h), dpp_u32<0x141>(l));
  key_max(h, l, dpp_u32<0x140>(h), dpp_u32<0x140>(l));
  auto rh = __builtin_amdgcn_permlane16_swap(h, h, false, false);
  auto rl = __builtin_amdgcn_permlane16_swap(l, l, false, false);
  h = rh[0]; l = rl[0];
  key_max(h, l, rh[1], rl[1]);
  rh = __builtin_amdgcn_permlane32_swap(h, h, false, false);
  rl = __builtin_amdgcn_permlane32_swap(l, l, false, false);
  h = rh[0]; l = rl[0];
  key_max(h, l, rh[1], rl[1]);
}
template <int R>
__global__ __launch_bounds__(kB) void topk_rows_wave(const float* __restrict__ x, int64_t rows, int e, int k,
                                                     bool largest, float* __restrict__ vals,
                                                     int64_t* __restrict__ idx) {
  const int w = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int64_t row = int64_t(blockIdx.x) * kTopkRows + w;
  if (row >= rows) return;   // a whole wave; no block barrier below
  // smallest-k is largest-k of the negated values (negation reverses the order, keeps ties)
  const float sgn = largest ? 1.0f : -1.0f;
  const float* xr = x + row * e;
  float raw[R];
#pragma unroll
  for (int r = 0; r < R; ++r) raw[r] = xr[min(lane + kWave * r, e - 1)];
  uint32_t kh[R], kl[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const bool in = lane + kWave * r < e;
    kh[r] = in ? topk_key(sgn * raw[r]) : 0u;
    kl[r] = kh[r] != 0u ? ~uint32_t(lane + kWave * r) : 0u;
  }
  float outv = 0.f;
  int outi = 0;
  for (int n = 0; n < k; ++n) {
    uint32_t bh = kh[0], bl = kl[0];
#pragma unroll
    for (int r = 1; r < R; ++r) key_max(bh, bl, kh[r], kl[r]);
    wave_key_max(bh, bl);
    const int pos = bh != 0u ? int(~bl) : 0;   // only spent values left: (spent, 0)
    float mine = raw[0];   // the element at position pos, from the lane that holds it
#pragma unroll
    for (int r = 1; r < R; ++r) mine = pos / kWave == r ? raw[r] : mine;
    const float won = bh != 0u ? __shfl(mine, pos % kWave, kWave) : (largest ? -INFINITY : INFINITY);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const bool taken = lane + kWave * r == pos;
      kh[r] = taken ? 0u : kh[r];
      kl[r] = taken ? 0u : kl[r];
    }
    if (lane == n) {
      outv = won;
      outi = pos;
    }
  }
  if (lane < k) {
    vals[row * k + lane] = outv;
    idx[row * k + lane] = outi;
  }
}

// ---------------------------------------------------------------- token <-> slot data movement
// out[s, :] = x[floordiv(slot[s], k) (wrapped into [0, t)), :], 8 bf16 per thread.
__global__ __launch_bounds__(kB) void gather_rows(const int64_t* __restrict__ slot, int64_t r, int64_t k,
                                                  const uint16_t* __restrict__ x, int64_t t, int64_t c,
                                                  uint16_t* __restrict__ out) {
  const int64_t s = blockIdx.y;
  const int64_t ch = int64_t(blockIdx.x) * kB + threadIdx.x;
  if (s >= r || ch * 8 >= c) return;
  const int64_t src = wrap_index(floordiv(slot[s], k), t);
  u32x4 v{0u, 0u, 0u, 0u};
  if (src >= 0) v = *reinterpret_cast<const u32x4*>(x + src * c + ch * 8);
  *reinterpret_cast<u32x4*>(out + s * c + ch * 8) = v;
}

// Weighted sum of each token's k expert rows.  Slot s = tok*k + j of expert id = ids[s] sits at
// row ends[id] - counts[id] + rank[s] - 1 of y.  Weight: bf16 w[s] (wsum null), or fp32 w[s] /
// wsum[tok].  out = bf16(sum), or with a residual h: io = bf16((h + io) + sum).
__global__ __launch_bounds__(kB) void combine_rows(const int64_t* __restrict__ ids, const int64_t* __restrict__ ends,
                                                   const int64_t* __restrict__ counts, const int64_t* __restrict__ rank,
                                                   const uint16_t* __restrict__ y, int64_t yrows,
                                                   const void* __restrict__ w, bool w_f32,
                                                   const float* __restrict__ wsum, const uint16_t* __restrict__ h,
                                                   uint16_t* __restrict__ out, int64_t tokens, int k, int e,
                                                   int64_t c) {
  __shared__ int64_t srow[64];
  __shared__ float sw[64];
  const int64_t tok = blockIdx.y;
  if (threadIdx.x < k) {
    const int64_t s = tok * k + threadIdx.x;
    const int64_t id = wrap_index(ids[s], e);
    int64_t row = -1;
    if (id >= 0) row = wrap_index(ends[id] - counts[id] + rank[s] - 1, yrows);
    srow[threadIdx.x] = row;
    float wt;
    if (w_f32) wt = static_cast<const float*>(w)[s] / wsum[tok];
    else wt = bf16_to_f32(static_cast<const uint16_t*>(w)[s]);
    sw[threadIdx.x] = wt;
  }
  __syncthreads();
  const int64_t ch = int64_t(blockIdx.x) * kB + threadIdx.x;
  if (tok >= tokens || ch * 8 >= c) return;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  bool bad = false;
  for (int j = 0; j < k; ++j) {
    const int64_t row = srow[j];
    if (row < 0) {
      bad = true;
      continue;
    }
    float f[8];
    ld8(y + row * c + ch * 8, f);
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] += f[i] * sw[j];
  }
  uint16_t* o = out + tok * c + ch * 8;
  if (h) {
    float hv[8], iv[8];
    ld8(h + tok * c + ch * 8, hv);
    ld8(o, iv);
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = (hv[i] + iv[i]) + acc[i];
  }
  if (bad) {
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = 0.f;
  }
  st8(o, acc);
}

// ---------------------------------------------------------------- small row / elementwise kernels
// out[r, j] = bf16(x[r, j] / sum_j x[r, j]) (normalize) or out[r] = sum_j x[r, j] (row sum), fp32 x.
// Rows of up to 16 values: every load of the row in flight at once (slots past k reload the row's
// last value and add nothing), the sum in the same order as the plain loop.
__global__ __launch_bounds__(kB) void normalize_rows(const float* __restrict__ x, int64_t rows, int k,
                                                     uint16_t* __restrict__ out_bf16, float* __restrict__ out_sum) {
  const int64_t r = int64_t(blockIdx.x) * kB + threadIdx.x;
  if (r >= rows) return;
  if (k <= 16) {
    float v[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) v[j] = x[r * k + (j < k ? j : k - 1)];
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < 16; ++j) s += j < k ? v[j] : 0.f;
    if (out_sum) {
      out_sum[r] = s;
      return;
    }
#pragma unroll
    for (int j = 0; j < 16; ++j)
      if (j < k) out_bf16[r * k + j] = f32_to_bf16(v[j] / s);
    return;
  }
  float s = 0.f;
  for (int j = 0; j < k; ++j) s += x[r * k + j];
  if (out_sum) {
    out_sum[r] = s;
    return;
  }
  for (int j = 0; j < k; ++j) out_bf16[r * k + j] = f32_to_bf16(x[r * k + j] / s);
}

__global__ __launch_bounds__(kB) void add_bf16(const uint16_t* __restrict__ a, const uint16_t* __restrict__ b,
                                               uint16_t* __restrict__ y, int64_t n) {
  const int64_t chunks = n >> 3;
  for (int64_t i = int64_t(blockIdx.x) * kB + threadIdx.x; i < chunks; i += int64_t(gridDim.x) * kB) {
    float fa[8], fb[8];
    ld8(a + i * 8, fa);
    ld8(b + i * 8, fb);
#pragma unroll
    for (int j = 0; j < 8; ++j) fa[j] += fb[j];
    st8(y + i * 8, fa);
  }
  if (blockIdx.x == 0)
    for (int64_t i = (chunks << 3) + threadIdx.x; i < n; i += kB)
      y[i] = f32_to_bf16(bf16_to_f32(a[i]) + bf16_to_f32(b[i]));
}

// Rotate-half RoPE in place of layout: x, out [T, H, 128] bf16; cos, sin [T, 128] fp32.
// out[d] = x[d] cos[d] + r[d] sin[d], r = (-x[64:], x[:64]).  One thread per 8 elements.
__global__ __launch_bounds__(kB) void rope_rows(const uint16_t* __restrict__ x, const float* __restrict__ cs,
                                                const float* __restrict__ sn, uint16_t* __restrict__ out, int64_t tokens,
                                                int64_t heads) {
  const int64_t g = int64_t(blockIdx.x) * kB + threadIdx.x;   // chunk index: (t, h, c) with 16 chunks per row
  if (g >= tokens * heads * 16) return;
  const int c = int(g & 15);
  const int64_t rowi = g >> 4, t = rowi / heads;
  const uint16_t* xr = x + rowi * 128;
  float f[8], p[8], cv[8], sv[8];
  ld8(xr + c * 8, f);
  ld8(xr + (c ^ 8) * 8, p);
  ld8f(cs + t * 128 + c * 8, cv);
  ld8f(sn + t * 128 + c * 8, sv);
  const bool first = c < 8;
#pragma unroll
  for (int i = 0; i < 8; ++i) f[i] = f[i] * cv[i] + (first ? -p[i] : p[i]) * sv[i];
  st8(out + rowi * 128 + c * 8, f);
}

// y = bf16( (x + a) * rsqrt(sum((x + a)^2) / cols + eps) * w ) per row, x + a in fp32; a may be null.
__global__ __launch_bounds__(kB) void rmsnorm_add_rows(const uint16_t* __restrict__ x, const uint16_t* __restrict__ a,
                                                       const uint16_t* __restrict__ w, uint16_t* __restrict__ y,
                                                       int64_t cols, float eps) {
  __shared__ float red[kB / kWave];
  const int64_t row = blockIdx.x;
  const uint16_t* xr = x + row * cols;
  const uint16_t* ar = a ? a + row * cols : nullptr;
  float ss = 0.f;
  for (int64_t c = threadIdx.x * 8; c < cols; c += kB * 8) {
    float f[8], g[8];
    ld8(xr + c, f);
    if (ar) {
      ld8(ar + c, g);
#pragma unroll
      for (int i = 0; i < 8; ++i) f[i] += g[i];
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) ss += f[i] * f[i];
  }
  ss = block_sum<kB / kWave>(ss, red);
  const float r = 1.0f / sqrtf(ss / float(cols) + eps);
  for (int64_t c = threadIdx.x * 8; c < cols; c += kB * 8) {
    float f[8], g[8], wv[8];
    ld8(xr + c, f);
    if (ar) {
      ld8(ar + c, g);
#pragma unroll
      for (int i = 0; i < 8; ++i) f[i] += g[i];
    }
    ld8(w + c, wv);
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = (f[i] * r) * wv[i];
    st8(y + row * cols + c, f);
  }
}

// out[s, :] = bf16( (x + a) * rsqrt(ss / cols + eps) * w ) for every s < rows: one token's
// normalised vector copied to each of its slots (the single-token dispatch).
__global__ __launch_bounds__(kB) void rms_broadcast(const uint16_t* __restrict__ x, const uint16_t* __restrict__ a,
                                                    const float* __restrict__ ss, const uint16_t* __restrict__ w,
                                                    uint16_t* __restrict__ out, int64_t rows, int64_t cols, float eps) {
  const int64_t c = (int64_t(blockIdx.x) * kB + threadIdx.x) * 8;
  if (c >= cols) return;
  const float r = 1.0f / sqrtf(ss[0] / float(cols) + eps);
  float f[8], g[8], wv[8];
  ld8(x + c, f);
  ld8(a + c, g);
  ld8(w + c, wv);
#pragma unroll
  for (int i = 0; i < 8; ++i) f[i] = ((f[i] + g[i]) * r) * wv[i];
  for (int64_t s = 0; s < rows; ++s) st8(out + s * cols + c, f);
}

int blocks_for(int64_t n, int64_t per_block, int cap = 4096) {
  int64_t b = (n + per_block - 1) / per_block;
  if (b > cap) b = cap;
  return int(b < 1 ? 1 : b);
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

// ------------------------------------------------------------------------------ C ABI
PTB_EXPORT int ptb_fill_zero(void* out, int64_t nbytes, void* stream) {
  if (nbytes < 0) return PTB_ERR_SHAPE;
  if (nbytes == 0) return PTB_OK;
  if (!out) return PTB_ERR_NULL;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if ((reinterpret_cast<uintptr_t>(out) & 3u) == 0 && nbytes % 4 == 0)
    fill_zero_u32<<<blocks_for(nbytes / 4, kB), kB, 0, s>>>(static_cast<uint32_t*>(out), nbytes / 4);
  else
    fill_zero_u8<<<blocks_for(nbytes, kB), kB, 0, s>>>(static_cast<uint8_t*>(out), nbytes);
  return launch_status();
}

PTB_EXPORT int ptb_cast_i64_i32(const int64_t* x, int32_t* y, int64_t n, void* stream) {
  if (n < 0) return PTB_ERR_SHAPE;
  if (n == 0) return PTB_OK;
  if (!x || !y) return PTB_ERR_NULL;
  cast_i64_i32<<<blocks_for(n, kB), kB, 0, static_cast<hipStream_t>(stream)>>>(x, y, n);
  return launch_status();
}

PTB_EXPORT int ptb_cumsum_int(const void* x, int x_dtype, void* y0, void* y1, int y_dtype, int64_t n, void* stream) {
  if (n < 0 || n > kScanMax) return n < 0 ? PTB_ERR_SHAPE : PTB_ERR_UNSUPPORTED;
  if (n == 0) return PTB_OK;
  if (!x || !y0) return PTB_ERR_NULL;
  if ((x_dtype != PTB_DTYPE_I32 && x_dtype != PTB_DTYPE_I64) || (y_dtype != PTB_DTYPE_I32 && y_dtype != PTB_DTYPE_I64))
    return PTB_ERR_DTYPE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int m = int(n);
  if (x_dtype == PTB_DTYPE_I64 && y_dtype == PTB_DTYPE_I64)
    cumsum_block<int64_t, int64_t><<<1, kScanThreads, 0, s>>>(static_cast<const int64_t*>(x), static_cast<int64_t*>(y0),
                                                               static_cast<int64_t*>(y1), m);
  else if (x_dtype == PTB_DTYPE_I64)
    cumsum_block<int64_t, int32_t><<<1, kScanThreads, 0, s>>>(static_cast<const int64_t*>(x), static_cast<int32_t*>(y0),
                                                               static_cast<int32_t*>(y1), m);
  else if (y_dtype == PTB_DTYPE_I64)
    cumsum_block<int32_t, int64_t><<<1, kScanThreads, 0, s>>>(static_cast<const int32_t*>(x), static_cast<int64_t*>(y0),
                                                               static_cast<int64_t*>(y1), m);
  else
    cumsum_block<int32_t, int32_t><<<1, kScanThreads, 0, s>>>(static_cast<const int32_t*>(x), static_cast<int32_t*>(y0),
                                                               static_cast<int32_t*>(y1), m);
  return launch_status();
}

PTB_EXPORT int ptb_moe_group_table(const void* ends, int ends_dtype, int64_t n, int64_t* nonempty, int64_t* starts,
                                   int64_t* rows, void* stream) {
  if (n < 0 || n > kScanMax) return n < 0 ? PTB_ERR_SHAPE : PTB_ERR_UNSUPPORTED;
  if (n == 0) return PTB_OK;
  if (!ends || !nonempty || !starts || !rows) return PTB_ERR_NULL;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (ends_dtype == PTB_DTYPE_I32)
    group_table_block<int32_t><<<1, kScanThreads, 0, s>>>(static_cast<const int32_t*>(ends), int(n), nonempty, starts, rows);
  else if (ends_dtype == PTB_DTYPE_I64)
    group_table_block<int64_t><<<1, kScanThreads, 0, s>>>(static_cast<const int64_t*>(ends), int(n), nonempty, starts, rows);
  else
    return PTB_ERR_DTYPE;
  return launch_status();
}

PTB_EXPORT int ptb_count_le(const int64_t* x, int64_t n, int32_t* out, int64_t m, void* stream) {
  if (n < 0 || m < 0) return PTB_ERR_SHAPE;
  if (m == 0) return PTB_OK;
  if (!out || (n > 0 && !x)) return PTB_ERR_NULL;
  count_le<<<blocks_for(m, kB, 1 << 30), kB, 0, static_cast<hipStream_t>(stream)>>>(x, n, out, m);   // n may be 0
  return launch_status();
}

PTB_EXPORT int ptb_moe_expert_count(const int64_t* ids, int64_t r, int64_t e, int64_t* counts, int64_t* counts2,
                                    int64_t* cum, void* stream) {
  if (r < 0 || e <= 0) return PTB_ERR_SHAPE;
  if (e > 1024) return PTB_ERR_UNSUPPORTED;
  if (!counts || (r > 0 && (!ids || !cum))) return PTB_ERR_NULL;
  int64_t blocks = (r + kSlotsPerBlock - 1) / kSlotsPerBlock;
  if (blocks < 1) blocks = 1;
  if (blocks > 0x7fffffff) return PTB_ERR_GRID;
  expert_count<<<dim3(unsigned(blocks)), kB, 0, static_cast<hipStream_t>(stream)>>>(ids, r, int(e), counts, counts2, cum);
  return launch_status();
}

PTB_EXPORT int ptb_moe_rank_select(const int64_t* cum, const int64_t* ids, int64_t r, int64_t e, int64_t* out,
                                   void* stream) {
  if (r < 0 || e <= 0) return PTB_ERR_SHAPE;
  if (r == 0) return PTB_OK;
  if (!cum || !ids || !out) return PTB_ERR_NULL;
  rank_select<<<blocks_for(r, kB, 1 << 30), kB, 0, static_cast<hipStream_t>(stream)>>>(cum, ids, r, e, out);
  return launch_status();
}

PTB_EXPORT size_t ptb_sort_workspace_bytes(int64_t rows, int64_t e) {
  if (rows <= 0 || e <= kSortChunk) return 0;
  int64_t p = kSortChunk;
  while (p < e) p <<= 1;
  return size_t(rows) * size_t(p) * (8 + 4) * 2;
}

PTB_EXPORT int ptb_sort_rows(const void* x, int key_dtype, void* values, int64_t* indices, int64_t rows, int64_t e,
                             int descending, void* workspace, size_t workspace_bytes, void* stream) {
  if (rows < 0 || e < 0) return PTB_ERR_SHAPE;
  if (rows == 0 || e == 0) return PTB_OK;
  if (!x || !values || !indices) return PTB_ERR_NULL;
  if (key_dtype != PTB_DTYPE_I64 && key_dtype != PTB_DTYPE_F32) return PTB_ERR_DTYPE;
  if (e > (int64_t(1) << 30) || rows > 65535) return PTB_ERR_UNSUPPORTED;
  const bool f32 = key_dtype == PTB_DTYPE_F32, desc = descending != 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (e <= kRankSortMax) {
    sort_rank<<<dim3(unsigned(rows)), dim3(unsigned((e + kWave - 1) / kWave * kWave)), 0, s>>>(x, int(e), f32, desc,
                                                                                             values, indices);
    return launch_status();
  }
  if (e <= kSortChunk) {
    int p = 1;
    while (p < e) p <<= 1;
    sort_chunk<<<dim3(unsigned(rows), 1), 1024, 0, s>>>(x, e, p, f32, desc, true, values, indices, nullptr, nullptr);
    return launch_status();
  }
  if (workspace_bytes < ptb_sort_workspace_bytes(rows, e)) return PTB_ERR_WORKSPACE;
  if (!workspace || !al16(workspace)) return workspace ? PTB_ERR_ALIGN : PTB_ERR_NULL;
  int64_t p = kSortChunk;
  while (p < e) p <<= 1;
  const int64_t total = rows * p;
  int64_t* k0 = static_cast<int64_t*>(workspace);
  int64_t* k1 = k0 + total;
  int32_t* i0 = reinterpret_cast<int32_t*>(k1 + total);
  int32_t* i1 = i0 + total;
  sort_chunk<<<dim3(unsigned(rows), unsigned(p / kSortChunk)), 1024, 0, s>>>(x, e, kSortChunk, f32, desc, false,
                                                                           nullptr, nullptr, k0, i0);
  // merge runs within each row: rows are independent because p is a multiple of every run length
  for (int64_t run = kSortChunk; run < p; run <<= 1) {
    sort_merge<<<blocks_for(total, kB, 1 << 30), kB, 0, s>>>(k0, i0, k1, i1, total, run);
    int64_t* tk = k0; k0 = k1; k1 = tk;
    int32_t* ti = i0; i0 = i1; i1 = ti;
  }
  sort_emit<<<blocks_for(rows * e, kB, 1 << 30), kB, 0, s>>>(k0, i0, e, p, f32, desc, values, indices, rows);
  return launch_status();
}

PTB_EXPORT int ptb_topk_rows_f32(const float* x, int64_t rows, int64_t e, int64_t k, int largest, float* values,
                                 int64_t* indices, void* stream) {
  if (rows < 0 || e < 0 || k < 0) return PTB_ERR_SHAPE;
  if (rows == 0 || k == 0) return PTB_OK;
  if (!x || !values || !indices) return PTB_ERR_NULL;
  if (e > kTopkMax || k > e) return PTB_ERR_UNSUPPORTED;
  const int64_t blocks = (rows + kTopkRows - 1) / kTopkRows;
  if (blocks > 0x7fffffff) return PTB_ERR_GRID;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int ei = int(e), ki = int(k);
  const bool lg = largest != 0;
  if (k <= kWave) {   // the row in registers, k wave-argmax rounds
    if (e <= 64) topk_rows_wave<1><<<dim3(unsigned(blocks)), kB, 0, s>>>(x, rows, ei, ki, lg, values, indices);
    else if (e <= 128) topk_rows_wave<2><<<dim3(unsigned(blocks)), kB, 0, s>>>(x, rows, ei, ki, lg, values, indices);
    else if (e <= 256) topk_rows_wave<4><<<dim3(unsigned(blocks)), kB, 0, s>>>(x, rows, ei, ki, lg, values, indices);
    else if (e <= 512) topk_rows_wave<8><<<dim3(unsigned(blocks)), kB, 0, s>>>(x, rows, ei, ki, lg, values, indices);
    else topk_rows_wave<16><<<dim3(unsigned(blocks)), kB, 0, s>>>(x, rows, ei, ki, lg, values, indices);
  } else {
    topk_rows<<<dim3(unsigned(blocks)), kB, 0, s>>>(x, rows, ei, ki, lg, values, indices);
  }
  return launch_status();
}

PTB_EXPORT int ptb_moe_gather_rows_bf16(const int64_t* slot, int64_t r, int64_t k, const void* x, int64_t t,
                                        int64_t c, void* out, void* stream) {
  if (r < 0 || t < 0 || c < 0 || k <= 0) return PTB_ERR_SHAPE;
  if (r == 0 || c == 0) return PTB_OK;
  if (!slot || !x || !out) return PTB_ERR_NULL;
  if (c % 8 || !al16(x) || !al16(out)) return PTB_ERR_ALIGN;
  if (r > 65535) return PTB_ERR_GRID;
  const dim3 grid(unsigned((c / 8 + kB - 1) / kB), unsigned(r));
  gather_rows<<<grid, kB, 0, static_cast<hipStream_t>(stream)>>>(slot, r, k, static_cast<const uint16_t*>(x), t, c,
                                                                static_cast<uint16_t*>(out));
  return launch_status();
}

PTB_EXPORT int ptb_moe_combine_bf16(const int64_t* ids, const int64_t* ends, const int64_t* counts, const int64_t* rank,
                                    const void* y, int64_t yrows, const void* w, int w_dtype, const float* wsum,
                                    const void* h, void* out, int64_t tokens, int64_t k, int64_t e, int64_t c,
                                    void* stream) {
  if (tokens < 0 || k <= 0 || e <= 0 || c < 0 || yrows < 0) return PTB_ERR_SHAPE;
  if (tokens == 0 || c == 0) return PTB_OK;
  if (!ids || !ends || !counts || !rank || !y || !w || !out) return PTB_ERR_NULL;
  if (w_dtype == PTB_DTYPE_F32 ? !wsum : (w_dtype != PTB_DTYPE_BF16 || wsum)) return PTB_ERR_DTYPE;
  if (k > 64) return PTB_ERR_UNSUPPORTED;
  if (c % 8 || !al16(y) || !al16(out) || (h && !al16(h))) return PTB_ERR_ALIGN;
  if (tokens > 65535) return PTB_ERR_GRID;
  const dim3 grid(unsigned((c / 8 + kB - 1) / kB), unsigned(tokens));
  combine_rows<<<grid, kB, 0, static_cast<hipStream_t>(stream)>>>(
      ids, ends, counts, rank, static_cast<const uint16_t*>(y), yrows, w, w_dtype == PTB_DTYPE_F32, wsum,
      static_cast<const uint16_t*>(h), static_cast<uint16_t*>(out), tokens, int(k), int(e), c);
  return launch_status();
}

PTB_EXPORT int ptb_normalize_rows_f32(const float* x, int64_t rows, int64_t k, void* out_bf16, float* out_sum,
                                      void* stream) {
  if (rows < 0 || k <= 0) return PTB_ERR_SHAPE;
  if (rows == 0) return PTB_OK;
  if (!x || (!out_bf16 == !out_sum)) return PTB_ERR_NULL;
  normalize_rows<<<blocks_for(rows, kB, 1 << 30), kB, 0, static_cast<hipStream_t>(stream)>>>(
      x, rows, int(k), static_cast<uint16_t*>(out_bf16), out_sum);
  return launch_status();
}

PTB_EXPORT int ptb_add_bf16(const void* a, const void* b, void* y, int64_t n, void* stream) {
  if (n < 0) return PTB_ERR_SHAPE;
  if (n == 0) return PTB_OK;
  if (!a || !b || !y) return PTB_ERR_NULL;
  if (!al16(a) || !al16(b) || !al16(y)) return PTB_ERR_ALIGN;
  add_bf16<<<blocks_for(n / 8 + 1, kB, 8192), kB, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t*>(a), static_cast<const uint16_t*>(b), static_cast<uint16_t*>(y), n);
  return launch_status();
}

PTB_EXPORT int ptb_rope_bf16(const void* x, const float* cos_t, const float* sin_t, void* out, int64_t tokens,
                             int64_t heads, int64_t head_dim, void* stream) {
  if (tokens < 0 || heads < 0) return PTB_ERR_SHAPE;
  if (head_dim != 128) return PTB_ERR_UNSUPPORTED;
  if (tokens == 0 || heads == 0) return PTB_OK;
  if (!x || !cos_t || !sin_t || !out) return PTB_ERR_NULL;
  if (!al16(x) || !al16(out) || !al16(cos_t) || !al16(sin_t)) return PTB_ERR_ALIGN;
  rope_rows<<<blocks_for(tokens * heads * 16, kB, 1 << 30), kB, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t*>(x), cos_t, sin_t, static_cast<uint16_t*>(out), tokens, heads);
  return launch_status();
}

PTB_EXPORT int ptb_rmsnorm_add_bf16(const void* x, const void* a, const void* w, void* y, int64_t rows, int64_t cols,
                                    float eps, void* stream) {
  if (rows < 0 || cols <= 0) return PTB_ERR_SHAPE;
  if (rows == 0) return PTB_OK;
  if (!x || !w || !y) return PTB_ERR_NULL;
  if (cols % 8 || !al16(x) || !al16(w) || !al16(y) || (a && !al16(a))) return PTB_ERR_ALIGN;
  if (rows > 0x7fffffff) return PTB_ERR_GRID;
  rmsnorm_add_rows<<<dim3(unsigned(rows)), kB, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(a), static_cast<const uint16_t*>(w),
      static_cast<uint16_t*>(y), cols, eps);
  return launch_status();
}

PTB_EXPORT int ptb_rms_broadcast_bf16(const void* x, const void* a, const float* ss, const void* w, void* out,
                                      int64_t rows, int64_t cols, float eps, void* stream) {
  if (rows < 0 || cols <= 0) return PTB_ERR_SHAPE;
  if (rows == 0) return PTB_OK;
  if (!x || !a || !ss || !w || !out) return PTB_ERR_NULL;
  if (cols % 8 || !al16(x) || !al16(a) || !al16(w) || !al16(out)) return PTB_ERR_ALIGN;
  rms_broadcast<<<blocks_for(cols / 8, kB, 1 << 30), kB, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(a), ss, static_cast<const uint16_t*>(w),
      static_cast<uint16_t*>(out), rows, cols, eps);
  return launch_status();
}
