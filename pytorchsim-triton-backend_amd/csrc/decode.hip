// Single-token (decode) kernels on gfx950: sum of squares, matrix-vector products with the decode
// layer's fused prologues / epilogue, and flash-decoding attention over a KV cache.  All of them
// stream their big operand (the weight matrix, the K/V cache) from HBM once and are bound by HBM
// bandwidth, so they are built for bytes in flight, not for the matrix cores.
//
// GEMV, y[n] = sum_k xp[k] * W[k, n] with W row-major [K, N] (N contiguous), split over K:
//   pass 1: workgroup (column block of 512, K slice of `kb` rows); the slice's xp[k] (the fused
//           prologue: plain x, RMSNorm-scaled x or x+a, or silu(g)*u) goes to LDS first, then each
//           wave walks every fourth row, each lane owning 8 consecutive columns (one 16-byte load
//           per row, a wave covers 1 KB of the row), eight rows in flight; the four waves' sums
//           meet in LDS and the slice's fp32 partials go to the workspace [splits, N].
//   pass 2: y[n] = bf16(sum over splits (+ r1[n] + r2[n])), one rounding.
// Decode attention (one query token, G query heads per kv head, S cached keys, D = 128):
//   pass 1: workgroup (64-key chunk, kv head): scores t = (q.k) * scale*log2(e) with 16 lanes per
//           key (one 256-byte row), the chunk's softmax in base 2 (m = chunk max, p = 2^(t-m),
//           l = sum of fp32 p), acc = sum bf16(p) * v; (m, l, acc) to the workspace.
//   pass 2: merge the chunks of a kv head: m = max m_c, o = sum acc_c 2^(m_c-m) / sum l_c 2^(m_c-m).
#include <cmath>

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

enum GemvMode { kPlain = 0, kRms = 1, kSilu = 2 };

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

template <int MODE>
__global__ __launch_bounds__(kGemvThreads) void gemv_partial(const uint16_t* __restrict__ x,
                                                             const uint16_t* __restrict__ add,
                                                             const float* __restrict__ ss,
                                                             const uint16_t* __restrict__ g, float eps,
                                                             const uint16_t* __restrict__ W,
                                                             float* __restrict__ part, int K, int N, int kb) {
  __shared__ float xs[kMaxKb];
  __shared__ float red[4][kColBlock];
  const int n0 = blockIdx.x * kColBlock;
  const int split = blockIdx.y;
  const int k0 = split * kb;
  const int rows = min(K - k0, kb);
  float r = 0.f;
  if constexpr (MODE == kRms) r = 1.f / sqrtf(ss[0] / float(K) + eps);
  for (int i = threadIdx.x; i < rows; i += kGemvThreads) xs[i] = prologue<MODE>(x, add, g, r, k0 + i, K);
  __syncthreads();

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = n0 + 8 * lane;
  float acc[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) acc[c] = 0.f;
  if (col < N) {
    const uint16_t* wp = W + int64_t(k0) * N + col;
    int i = wave;
    for (; i + 28 < rows; i += 32) {
      u32x4 v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = *reinterpret_cast<const u32x4*>(wp + int64_t(i + 4 * u) * N);
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
      const u32x4 v = *reinterpret_cast<const u32x4*>(wp + int64_t(i) * N);
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

// 16 columns a workgroup, 16 split groups of 16 lanes: each lane sums every 16th split with its
// loads independent (the partials come from L2 or another XCD: latency, not bandwidth, bounds this)
constexpr int kFinCols = 16;
__global__ __launch_bounds__(256) void gemv_finish(const float* __restrict__ part, int splits, int N,
                                                   const uint16_t* __restrict__ r1, const uint16_t* __restrict__ r2,
                                                   uint16_t* __restrict__ y) {
  __shared__ float red[16][kFinCols];
  const int c = threadIdx.x % kFinCols, sg = threadIdx.x / kFinCols;
  const int n = blockIdx.x * kFinCols + c;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  if (n < N) {
    int sp = sg;
    for (; sp + 48 < splits; sp += 64) {
#pragma unroll
      for (int u = 0; u < 4; ++u) acc[u] += part[int64_t(sp + 16 * u) * N + n];
    }
    for (; sp < splits; sp += 16) acc[0] += part[int64_t(sp) * N + n];
  }
  red[sg][c] = (acc[0] + acc[1]) + (acc[2] + acc[3]);
  __syncthreads();
  if (sg == 0 && n < N) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) s += red[i][c];
    if (r1) s += bf16_to_f32(r1[n]) + (r2 ? bf16_to_f32(r2[n]) : 0.f);
    y[n] = f32_to_bf16(s);
  }
}

template <int MODE>
int launch_gemv(const void* x, const void* add, const float* ss, const void* g, float eps, const void* w,
                const void* r1, const void* r2, void* y, int64_t k, int64_t n, void* ws, size_t ws_bytes,
                void* stream) {
  if (k < 0 || n < 0) return PTB_ERR_SHAPE;
  if (n == 0) return PTB_OK;
  if (!x || !w || !y || (MODE == kRms && (!ss || !g))) return PTB_ERR_NULL;
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
      static_cast<const uint16_t*>(w), part, int(k), int(n), sp.kb);
  gemv_finish<<<dim3(unsigned((n + kFinCols - 1) / kFinCols)), dim3(256), 0, s>>>(
      part, sp.splits, int(n), static_cast<const uint16_t*>(r1), static_cast<const uint16_t*>(r2),
      static_cast<uint16_t*>(y));
  return launch_status();
}

// ---------------------------------------------------------------------------------------------
// decode attention

constexpr int kD = 128;
constexpr int kChunk = 64;       // keys per workgroup
constexpr int kAttnThreads = 256;

// workspace per (kv head, chunk): m[G], l[G], acc[G][128]
template <int G>
__global__ __launch_bounds__(kAttnThreads) void attn_decode_partial(const uint16_t* __restrict__ Q,
                                                                    const uint16_t* __restrict__ Kc,
                                                                    const uint16_t* __restrict__ Vc,
                                                                    float* __restrict__ ws, int S, float c) {
  __shared__ float qs[G][kD];
  __shared__ float ts[G][kChunk];          // scores, then bf16-rounded p
  __shared__ float red[4][G][kD];
  __shared__ float stat[G][2];
  const int chunk = blockIdx.x, kvh = blockIdx.y, nchunks = gridDim.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint16_t* q = Q + int64_t(kvh) * G * kD;
  const uint16_t* kp = Kc + int64_t(kvh) * S * kD;
  const uint16_t* vp = Vc + int64_t(kvh) * S * kD;
  const int key0 = chunk * kChunk;
  for (int i = tid; i < G * kD; i += kAttnThreads) qs[i / kD][i % kD] = bf16_to_f32(q[i]);
  __syncthreads();

  // every K and V load of the chunk goes out first (16 x 16 bytes a lane, 64 KB a workgroup in
  // flight): the kernel is bound by HBM latency x bandwidth, not by its few FMAs
  // scores: 16 lanes per key (8 dims each), 4 keys per wave, 16 keys per pass
  const int d8 = lane & 15;
  const int kj = tid >> 4;   // PV: 16 lanes per key, key kj of each pass
  u32x4 kreg[kChunk / 16], vreg[kChunk / 16];
#pragma unroll
  for (int pass = 0; pass < kChunk / 16; ++pass) {
    const int key = min(key0 + pass * 16 + wave * 4 + (lane >> 4), S - 1);
    kreg[pass] = *reinterpret_cast<const u32x4*>(kp + int64_t(key) * kD + 8 * d8);
  }
#pragma unroll
  for (int pass = 0; pass < kChunk / 16; ++pass) {
    const int key = min(key0 + pass * 16 + kj, S - 1);
    vreg[pass] = *reinterpret_cast<const u32x4*>(vp + int64_t(key) * kD + 8 * d8);
  }
#pragma unroll
  for (int pass = 0; pass < kChunk / 16; ++pass) {
    const int j = pass * 16 + wave * 4 + (lane >> 4);
    float kf[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      kf[2 * e] = bf16_lo(kreg[pass][e]);
      kf[2 * e + 1] = bf16_hi(kreg[pass][e]);
    }
#pragma unroll
    for (int gi = 0; gi < G; ++gi) {
      float s = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) s = __builtin_fmaf(qs[gi][8 * d8 + e], kf[e], s);
#pragma unroll
      for (int off = 8; off > 0; off >>= 1) s += __shfl_xor(s, off, 16);
      if (d8 == 0) ts[gi][j] = (key0 + j < S) ? s * c : -INFINITY;
    }
  }
  __syncthreads();

  // chunk softmax: 32 lanes per query head, 4 keys a lane
  for (int gi = tid / 32; gi < G; gi += kAttnThreads / 32) {
    const int l32 = tid & 31;
    float mx = -INFINITY;
#pragma unroll
    for (int e = 0; e < kChunk / 32; ++e) mx = fmaxf(mx, ts[gi][l32 + 32 * e]);
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 32));
    float ls = 0.f;
#pragma unroll
    for (int e = 0; e < kChunk / 32; ++e) {
      const float p = __builtin_amdgcn_exp2f(ts[gi][l32 + 32 * e] - mx);
      ls += p;
      ts[gi][l32 + 32 * e] = bf16_to_f32(f32_to_bf16(p));
    }
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) ls += __shfl_xor(ls, off, 32);
    if (l32 == 0) {
      stat[gi][0] = mx;
      stat[gi][1] = ls;
    }
  }
  __syncthreads();

  // acc[g][d] = sum_j p[g][j] v[j][d]: lane owns 8 dims of every 16th key
  float acc[G][8];
#pragma unroll
  for (int gi = 0; gi < G; ++gi)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[gi][e] = 0.f;
#pragma unroll
  for (int pass = 0; pass < kChunk / 16; ++pass) {
    const int j = pass * 16 + kj;
    float vf[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      vf[2 * e] = bf16_lo(vreg[pass][e]);
      vf[2 * e + 1] = bf16_hi(vreg[pass][e]);
    }
#pragma unroll
    for (int gi = 0; gi < G; ++gi) {
      const float p = ts[gi][j];
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[gi][e] = __builtin_fmaf(p, vf[e], acc[gi][e]);
    }
  }
  // lanes l, l^16, l^32, l^48 hold the same dims; then the four waves meet in LDS
#pragma unroll
  for (int gi = 0; gi < G; ++gi)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float a = acc[gi][e];
      a += __shfl_xor(a, 16, kWave);
      a += __shfl_xor(a, 32, kWave);
      acc[gi][e] = a;
    }
  if (lane < 16) {
#pragma unroll
    for (int gi = 0; gi < G; ++gi)
#pragma unroll
      for (int e = 0; e < 8; ++e) red[wave][gi][8 * d8 + e] = acc[gi][e];
  }
  __syncthreads();
  float* out = ws + (int64_t(kvh) * nchunks + chunk) * (G * (kD + 2));
  for (int i = tid; i < G * kD; i += kAttnThreads) {
    const int gi = i / kD, d = i % kD;
    out[2 * G + i] = (red[0][gi][d] + red[1][gi][d]) + (red[2][gi][d] + red[3][gi][d]);
  }
  if (tid < G) {
    out[tid] = stat[tid][0];
    out[G + tid] = stat[tid][1];
  }
}

// One workgroup per (kv head, query head): the chunk maxima reduce across the workgroup first,
// then each lane (one of the 128 dims) sums the chunks with independent loads.
template <int G>
__global__ __launch_bounds__(kD) void attn_decode_combine(const float* __restrict__ ws, uint16_t* __restrict__ O,
                                                          int nchunks) {
  __shared__ float red[2];
  const int kvh = blockIdx.x, gi = blockIdx.y, d = threadIdx.x;
  const float* base = ws + int64_t(kvh) * nchunks * (G * (kD + 2));
  constexpr int stride = G * (kD + 2);
  float m = -INFINITY;
  for (int ch = d; ch < nchunks; ch += kD) m = fmaxf(m, base[int64_t(ch) * stride + gi]);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, kWave));
  if ((d & 63) == 0) red[d >> 6] = m;
  __syncthreads();
  m = fmaxf(red[0], red[1]);
  float l[4] = {0.f, 0.f, 0.f, 0.f}, o[4] = {0.f, 0.f, 0.f, 0.f};
  int ch = 0;
  for (; ch + 3 < nchunks; ch += 4) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const float* p = base + int64_t(ch + u) * stride;
      const float w = __builtin_amdgcn_exp2f(p[gi] - m);
      l[u] = __builtin_fmaf(p[G + gi], w, l[u]);
      o[u] = __builtin_fmaf(p[2 * G + gi * kD + d], w, o[u]);
    }
  }
  for (; ch < nchunks; ++ch) {
    const float* p = base + int64_t(ch) * stride;
    const float w = __builtin_amdgcn_exp2f(p[gi] - m);
    l[0] = __builtin_fmaf(p[G + gi], w, l[0]);
    o[0] = __builtin_fmaf(p[2 * G + gi * kD + d], w, o[0]);
  }
  const float lt = (l[0] + l[1]) + (l[2] + l[3]), ot = (o[0] + o[1]) + (o[2] + o[3]);
  O[(int64_t(kvh) * G + gi) * kD + d] = f32_to_bf16(ot / lt);
}

template <int G>
void launch_attn_decode(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o, float* ws, int nkv,
                        int seq, float c, hipStream_t s) {
  const int nchunks = (seq + kChunk - 1) / kChunk;
  attn_decode_partial<G><<<dim3(unsigned(nchunks), unsigned(nkv)), dim3(kAttnThreads), 0, s>>>(q, k, v, ws, seq, c);
  attn_decode_combine<G><<<dim3(unsigned(nkv), unsigned(G)), dim3(kD), 0, s>>>(ws, o, nchunks);
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

PTB_EXPORT size_t ptb_attn_decode_workspace_bytes(int64_t nkv, int64_t group, int64_t seq) {
  if (nkv <= 0 || group <= 0 || seq <= 0) return 0;
  const int64_t nchunks = (seq + kChunk - 1) / kChunk;
  return size_t(nkv * nchunks * group * (kD + 2)) * sizeof(float);
}

PTB_EXPORT int ptb_attn_decode_bf16(const void* q, const void* k, const void* v, void* o, int64_t nkv, int64_t group,
                                    int64_t seq, int64_t head_dim, float scale, void* workspace,
                                    size_t workspace_bytes, void* stream) {
  if (nkv < 0 || group <= 0 || seq <= 0 || head_dim <= 0) return PTB_ERR_SHAPE;
  if (head_dim != kD) return PTB_ERR_UNSUPPORTED;
  if (!std::isfinite(scale)) return PTB_ERR_UNSUPPORTED;
  if (nkv == 0) return PTB_OK;
  if (!q || !k || !v || !o) return PTB_ERR_NULL;
  if (!aligned16(k) || !aligned16(v)) return PTB_ERR_ALIGN;
  if (nkv > 65535 || seq > 0x7fffffff || nkv * seq * kD >= (int64_t(1) << 40)) return PTB_ERR_GRID;
  if (!workspace || workspace_bytes < ptb_attn_decode_workspace_bytes(nkv, group, seq)) return PTB_ERR_WORKSPACE;
  if (reinterpret_cast<uintptr_t>(workspace) & 3u) return PTB_ERR_ALIGN;
  const float c = scale * 1.4426950408889634f;
  auto qp = static_cast<const uint16_t*>(q), kp = static_cast<const uint16_t*>(k), vp = static_cast<const uint16_t*>(v);
  auto op = static_cast<uint16_t*>(o);
  auto ws = static_cast<float*>(workspace);
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (group) {
    case 1: launch_attn_decode<1>(qp, kp, vp, op, ws, int(nkv), int(seq), c, s); break;
    case 2: launch_attn_decode<2>(qp, kp, vp, op, ws, int(nkv), int(seq), c, s); break;
    case 3: launch_attn_decode<3>(qp, kp, vp, op, ws, int(nkv), int(seq), c, s); break;
    case 4: launch_attn_decode<4>(qp, kp, vp, op, ws, int(nkv), int(seq), c, s); break;
    case 6: launch_attn_decode<6>(qp, kp, vp, op, ws, int(nkv), int(seq), c, s); break;
    case 8: launch_attn_decode<8>(qp, kp, vp, op, ws, int(nkv), int(seq), c, s); break;
    default: return PTB_ERR_UNSUPPORTED;
  }
  return launch_status();
}
