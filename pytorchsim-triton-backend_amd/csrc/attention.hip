// Causal / full GQA flash-attention forward on gfx950 matrix cores, head_dim 128, bf16 in/out.
//
// Layout (the reference's): q, o [B*HQ, S, 128]; k, v [B*HKV, S, 128]; query head h of batch b reads
// kv head b*HKV + h / (HQ/HKV).
//
// Workgroup = 4 waves = 128 query rows of one head (32 per wave); K/V blocks of 64 keys are staged
// in LDS, double-buffered (K as [key][d], V transposed to [d][key]).  Each wave computes the
// transposed score tile S^T = K Q^T (keys on the MFMA's M side, its 32 queries on the lanes), so a
// query's scores sit in one lane pair (lane, lane^32) and its softmax statistics need one cross-lane
// exchange per block.  The exponentials, rounded to bf16, are already laid out as the B operand of
// O^T += V^T P^T, so P never goes through LDS.  Online softmax follows the reference step by step:
// s = (q.k) * scale, masked entries -1e30, m_new = max(m, rowmax), alpha = exp(m - m_new),
// p = exp(s - m_new), l = l * alpha + rowsum(p), acc = acc * alpha + bf16(p) V, out = acc / l.
//
// Work order: q tiles heaviest-first (causal), and workgroup ids are spread so that each XCD serves
// one kv head group at a time (its K/V stay in that XCD's L2 while the group's query heads use them).
#include "ptb_common.h"

using namespace ptb;

namespace {

constexpr int D = 128;
constexpr int BQ = 128;            // query rows per workgroup
constexpr int BKV = 64;            // keys per block
constexpr int kThreads = 256;
constexpr int LDK = D + 8;         // K tile row (key) stride, elements: 272 B, conflict-free b128 reads
constexpr int LDV = BKV + 4;       // V^T tile row (d) stride, elements: 136 B, conflict-free b64 reads
constexpr int kKElems = BKV * LDK;
constexpr int kVElems = D * LDV;
constexpr int kStageElems = kKElems + kVElems;

typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

struct KV {
  u32x4 r[8];
};

// Threads 0..127 load an 8(key) x 8(d) block of V; threads 128..255 load 8 chunks of K.
__device__ __forceinline__ KV load_block(const uint16_t* __restrict__ kp, const uint16_t* __restrict__ vp, int key0,
                                         int tid) {
  KV x;
  if (tid < 128) {
    const int kb8 = tid & 7, db = tid >> 3;
    const uint16_t* src = vp + int64_t(key0 + kb8 * 8) * D + db * 8;
#pragma unroll
    for (int p = 0; p < 8; ++p) x.r[p] = *reinterpret_cast<const u32x4*>(src + p * D);
  } else {
    const int t = tid - 128;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int c = t + 128 * i;
      x.r[i] = *reinterpret_cast<const u32x4*>(kp + int64_t(key0 + (c >> 4)) * D + (c & 15) * 8);
    }
  }
  return x;
}

template <int C>
__device__ __forceinline__ void store_vt(uint16_t* vt, const u32x4 (&r)[8]) {
  const u32x4 col = column8x8<C>(r);
  *reinterpret_cast<u32x2*>(vt + C * LDV) = u32x2{col[0], col[1]};
  *reinterpret_cast<u32x2*>(vt + C * LDV + 4) = u32x2{col[2], col[3]};
  if constexpr (C + 1 < 8) store_vt<C + 1>(vt, r);
}

__device__ __forceinline__ void store_block(uint16_t* stage, const KV& x, int tid) {
  if (tid < 128) {
    const int kb8 = tid & 7, db = tid >> 3;
    store_vt<0>(stage + kKElems + (db * 8) * LDV + kb8 * 8, x.r);
  } else {
    const int t = tid - 128;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int c = t + 128 * i;
      *reinterpret_cast<u32x4*>(stage + (c >> 4) * LDK + (c & 15) * 8) = x.r[i];
    }
  }
}

__device__ __forceinline__ float exp_e(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }

__global__ __launch_bounds__(kThreads, 2) void flash_fwd_kernel(
    const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K, const uint16_t* __restrict__ V,
    uint16_t* __restrict__ O, int S, int hq, int hkv, int nkv, int nt, float scale, int causal) {
  __shared__ __attribute__((aligned(16))) uint16_t smem[2 * kStageElems];

  // ---- work decode: r enumerates (q tile heaviest-first, kv head); g = query head within group
  const int G = hq / hkv;
  const int total = nt * nkv * G;
  const int pid = blockIdx.x;
  int g, r;
  if ((total & 7) == 0 && ((total >> 3) % G) == 0) {
    const int x = pid & 7, j = pid >> 3;
    g = j % G;
    r = (j / G) * 8 + x;
  } else {
    g = pid % G;
    r = pid / G;
  }
  const int tile = causal ? nt - 1 - r / nkv : r / nkv;
  const int kvi = r % nkv;
  const int b = kvi / hkv, kvh = kvi % hkv;
  const int64_t bh = int64_t(b) * hq + kvh * G + g;
  const uint16_t* qp = Q + bh * S * D;
  const uint16_t* kp = K + int64_t(kvi) * S * D;
  const uint16_t* vp = V + int64_t(kvi) * S * D;
  uint16_t* op = O + bh * S * D;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = lane >> 5, fr = lane & 31;
  const int q0 = tile * BQ;
  const int qw0 = q0 + wave * 32;
  const int qi = qw0 + fr;  // this lane's query

  // Q fragments (B operand of S^T = K Q^T): 8 K-steps of 16 over d
  bf16x8 qf[8];
  {
    const uint16_t* src = qp + int64_t(qi) * D + h * 8;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) qf[kk] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(src + kk * 16));
  }

  f32x16 acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[i][e] = 0.f;
  float m_i = -1.0e30f, l_i = 0.f;

  const int nb = causal ? (q0 + BQ) / BKV : S / BKV;
  store_block(smem, load_block(kp, vp, 0, tid), tid);
  __syncthreads();

  for (int kb = 0; kb < nb; ++kb) {
    const uint16_t* st = smem + (kb & 1) * kStageElems;
    const bool more = kb + 1 < nb;
    KV nxt;
    if (more) nxt = load_block(kp, vp, (kb + 1) * BKV, tid);
    const int key0 = kb * BKV;
    // causal: skip blocks entirely above this wave's diagonal; mask the straddling one
    const bool live = !causal || key0 <= qw0 + 31;
    if (live) {
      const bool partial = causal && key0 + BKV - 1 > qw0;
      f32x16 sacc[2];
#pragma unroll
      for (int t2 = 0; t2 < 2; ++t2) {
#pragma unroll
        for (int e = 0; e < 16; ++e) sacc[t2][e] = 0.f;
        const uint16_t* krow = st + (t2 * 32 + fr) * LDK + h * 8;
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
          const bf16x8 kf = *reinterpret_cast<const bf16x8*>(krow + kk * 16);
          sacc[t2] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[kk], sacc[t2], 0, 0, 0);
        }
      }
      // scores: lane holds query qi, keys key0 + t2*32 + 8*(e/4) + 4*h + e%4
      float mloc = -1.0e30f;
#pragma unroll
      for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          float s = sacc[t2][e] * scale;
          if (partial) {
            const int key = key0 + t2 * 32 + 8 * (e >> 2) + 4 * h + (e & 3);
            if (key > qi) s = -1.0e30f;
          }
          sacc[t2][e] = s;
          mloc = fmaxf(mloc, s);
        }
      mloc = fmaxf(mloc, __shfl_xor(mloc, 32, kWave));
      const float m_new = fmaxf(m_i, mloc);
      const float alpha = exp_e(m_i - m_new);
      float lsum = 0.f;
      bf16x8 pf[2][2];
#pragma unroll
      for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const float p = exp_e(sacc[t2][e] - m_new);
          lsum += p;
          pf[t2][e >> 3][e & 7] = (__bf16)p;
        }
      l_i = l_i * alpha + lsum;  // per-lane partial over this lane's keys; halves combine at the end
      m_i = m_new;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][e] *= alpha;
      // O^T[d][q] += V^T[d][key] P^T[key][q]; K-step (t2, k16) covers keys t2*32 + k16*16 .. +16,
      // lane half h holding keys +4h..+4h+3 and +8+4h..+8+4h+3 (the score tile's own layout)
      const uint16_t* vt = st + kKElems;
#pragma unroll
      for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
        for (int k16 = 0; k16 < 2; ++k16) {
          const int kbase = t2 * 32 + k16 * 16 + 4 * h;
#pragma unroll
          for (int dt = 0; dt < 4; ++dt) {
            const uint16_t* vrow = vt + (dt * 32 + fr) * LDV + kbase;
            const u32x2 lo = *reinterpret_cast<const u32x2*>(vrow);
            const u32x2 hi = *reinterpret_cast<const u32x2*>(vrow + 8);
            const bf16x8 vf = __builtin_bit_cast(bf16x8, u32x4{lo[0], lo[1], hi[0], hi[1]});
            acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf[t2][k16], acc[dt], 0, 0, 0);
          }
        }
    }
    if (more) store_block(smem + ((kb + 1) & 1) * kStageElems, nxt, tid);
    __syncthreads();
  }

  const float l = l_i + __shfl_xor(l_i, 32, kWave);
  uint16_t* orow = op + int64_t(qi) * D;
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const int d0 = dt * 32 + 8 * g4 + 4 * h;
      const u32x2 w = u32x2{pack_bf16x2(acc[dt][4 * g4] / l, acc[dt][4 * g4 + 1] / l),
                            pack_bf16x2(acc[dt][4 * g4 + 2] / l, acc[dt][4 * g4 + 3] / l)};
      *reinterpret_cast<u32x2*>(orow + d0) = w;
    }
}

}  // namespace

PTB_EXPORT int ptb_flash_attn_fwd_bf16(const void* q, const void* k, const void* v, void* o, int64_t batch,
                                       int64_t hq, int64_t hkv, int64_t seq, int64_t head_dim, float scale,
                                       int causal, void* stream) {
  if (batch < 0 || hq <= 0 || hkv <= 0 || seq < 0 || head_dim <= 0) return PTB_ERR_SHAPE;
  if (hq % hkv) return PTB_ERR_SHAPE;
  if (head_dim != D) return PTB_ERR_UNSUPPORTED;
  if (batch == 0 || seq == 0) return PTB_OK;
  if (!q || !k || !v || !o) return PTB_ERR_NULL;
  if (seq % BQ) return PTB_ERR_UNSUPPORTED;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o)) return PTB_ERR_ALIGN;
  const int64_t nt = seq / BQ, nkv = batch * hkv;
  const int64_t total = nt * nkv * (hq / hkv);
  if (total > 0x7fffffff || seq > 0x7fffffff || batch * hq * seq > (int64_t(1) << 40)) return PTB_ERR_GRID;
  flash_fwd_kernel<<<dim3(unsigned(total)), dim3(kThreads), 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(v),
      static_cast<uint16_t*>(o), int(seq), int(hq), int(hkv), int(nkv), int(nt), scale, causal ? 1 : 0);
  return launch_status();
}
