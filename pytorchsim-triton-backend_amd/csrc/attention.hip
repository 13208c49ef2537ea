// Causal / full GQA flash-attention forward on gfx950 matrix cores, head_dim 128, bf16 in/out.
//
// Layout (the reference's): q, o [B*HQ, S, 128]; k, v [B*HKV, S, 128]; query head h of batch b reads
// kv head b*HKV + h / (HQ/HKV).
//
// Workgroup = 8 waves = 256 query rows of one head (32 per wave), one workgroup per CU, two waves
// per SIMD, when that gives at least two workgroups per CU (non-causal: one); otherwise either
// (causal, when the units fill at least 3/4 of the CUs) 8 waves over two 128-row tiles, a heavy one
// and its light complement, so every workgroup carries the same causal work, or 4 waves = 128 rows,
// two workgroups per CU.  Blocks of 64 keys move HBM -> LDS with buffer_load_dwordx4 ... lds (no VGPR
// staging) into two 32 KB stages, one block ahead, shared by all the workgroup's rows.  Both tiles
// keep their global [key][d] layout with the 16-byte chunks of each 256-byte row XOR-swizzled, so
// every LDS read is bank-conflict free:
//   K: chunk c of key row r sits in slot c ^ (r & 15); the 16 lanes of a 128-bit read take 16 keys.
//   V: chunk c of key row r sits in slot c ^ (4 * (r & 3)); V^T fragments come from
//      ds_read_b64_tr_b16 (within each 16-lane group lane 4j+q supplies key k+j, d n+4q..n+4q+3 and
//      lane i receives keys k..k+3 of d n+i), whose half-wave reads cover 4 keys x 4 chunks.
// Each wave computes the transposed score tile S^T = K Q^T (keys on the MFMA's M side, its 32
// queries on the lanes), so a query's 64 scores sit in one lane pair (lane, lane^32); the softmax
// statistics need one cross-lane exchange per block.  The K fragments of a block are read ahead of
// its MFMAs (four in flight), so LDS latency does not serialise the score MFMAs.  The exponentials,
// rounded to bf16, are already laid out as the B operand of O^T += V^T P^T, so P never goes
// through LDS.
//
// Online softmax, as the reference defines it (s = (q.k) * scale, masked entries excluded,
// p = exp(s - m), l sums the fp32 p, acc += bf16(p) V, out = acc / l), computed in base 2 with the
// scale folded in: t = (q.k) * scale*log2(e), p = 2^(t - m), one FMA and one v_exp_f32 per score.
// The running maximum m is raised only when a row's block maximum exceeds it by more than 2^8
// (any row of the wave: then acc and l are rescaled by 2^(m_old - m_new)); otherwise p <= 256 and
// acc, l carry the same factor, which cancels in acc / l.  The causal mask is applied only in the
// one 64-key block that straddles a wave's diagonal; blocks above it are skipped.
//
// Work order: q tiles heaviest-first (causal), and workgroup ids are spread so that each XCD serves
// one kv head group at a time (its K/V stay in that XCD's L2 while the group's query heads use them).
// When S is not a multiple of the tile height, the last tile's waves past S only keep the loads and
// barriers going (keys past S read as zero through the buffer range).
#include <cmath>
#include <type_traits>

#include "ptb_common.h"

using namespace ptb;

namespace {

constexpr int D = 128;
constexpr int BKV = 64;            // keys per block
constexpr int kTileBytes = BKV * D * 2;        // 16 KB: 64 key rows x 256 B
constexpr int kStageBytes = 2 * kTileBytes;    // K tile, then V tile
constexpr int kKPrefetch = 4;                  // K fragment reads kept ahead of the score MFMAs
constexpr float kRescaleLog2 = 8.f;            // raise m only when a block max exceeds it by 2^8

typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
typedef __attribute__((address_space(3))) bf16x8 lds_bf16x8;

__device__ __forceinline__ bf16x8 lds_read_b128(uint32_t addr) {
  return *reinterpret_cast<const lds_bf16x8*>(size_t(addr));
}

__device__ __forceinline__ i16x4 lds_read_tr(uint32_t addr) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(reinterpret_cast<lds_i16x4*>(size_t(addr)));
}

__device__ __forceinline__ bf16x8 join(i16x4 lo, i16x4 hi) {
  return __builtin_bit_cast(bf16x8, i16x8(__builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7)));
}

// A wave's online-softmax state for its 32 queries.
struct WaveState {
  f32x16 acc[4];   // O^T: d = 32*dt + 8*(r/4) + 4*h + r%4, query = lane%32
  float m;         // running maximum, log2 units (t = q.k * c)
  float l;         // this lane's partial row sum (the lane pair's two halves add up at the end)
};

// S^T (64 keys x 32 queries) = K Q^T for one wave: the lane holds query lane%32 and keys
// 32*t2 + 8*(e/4) + 4*(lane/32) + e%4 of the block.  All 16 K fragments are requested before the
// MFMAs that use them; the scheduling groups keep kKPrefetch reads in flight.
__device__ __forceinline__ void qk_step(f32x16 (&sacc)[2], const bf16x8 (&qf)[8], uint32_t k_tile,
                                        const uint32_t (&koff)[8]) {
#pragma unroll
  for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
    for (int e = 0; e < 16; ++e) sacc[t2][e] = 0.f;
  bf16x8 kf[2][8];
#pragma unroll
  for (int kk = 0; kk < 8; ++kk)
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2) kf[t2][kk] = lds_read_b128(k_tile + koff[kk] + t2 * 32 * 256);
#pragma unroll
  for (int kk = 0; kk < 8; ++kk)
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2)
      sacc[t2] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[t2][kk], qf[kk], sacc[t2], 0, 0, 0);
  __builtin_amdgcn_sched_group_barrier(0x100, kKPrefetch, 0);   // LDS reads
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);          // one MFMA
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);          // the next read
  }
}

// Online-softmax update from one S^T block; lim = query - key0 - 4*(lane/32) for the diagonal block.
template <bool MASK>
__device__ __forceinline__ void softmax_step(WaveState& w, f32x16 (&sacc)[2], bf16x8 (&pf)[2][2], float c,
                                             int lim) {
  if constexpr (MASK) {
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
      for (int e = 0; e < 16; ++e)
        if (32 * t2 + 8 * (e >> 2) + (e & 3) > lim) sacc[t2][e] = -INFINITY;
  }
  float mx = sacc[0][0];
#pragma unroll
  for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
    for (int e = 0; e < 16; ++e) mx = fmaxf(mx, sacc[t2][e]);
  mx = pair32_max(mx);
  const float mt = mx * c;
  if (__builtin_amdgcn_ballot_w64(mt > w.m + kRescaleLog2)) {
    const float m_new = fmaxf(w.m, mt);
    const float alpha = __builtin_amdgcn_exp2f(w.m - m_new);
    w.l *= alpha;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) w.acc[i][e] *= alpha;
    w.m = m_new;
  }
  const float nm = -w.m;
  float lsum = 0.f;
#pragma unroll
  for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[t2][e], c, nm));
      lsum += p;
      pf[t2][e >> 3][e & 7] = (__bf16)p;
    }
  w.l += lsum;
}

// O^T[d][q] += V^T[d][key] P^T[key][q]; K-step (t2, k16) covers keys 32*t2 + 16*k16 .. +16, lane
// half h holding keys +4h..+4h+3 and +8+4h..+8+4h+3 (the score tile's own layout).
__device__ __forceinline__ void pv_step(WaveState& w, const bf16x8 (&pf)[2][2], uint32_t v_tile,
                                        const uint32_t (&voff)[4]) {
#pragma unroll
  for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
    for (int k16 = 0; k16 < 2; ++k16)
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        const uint32_t a = v_tile + voff[dt] + (32 * t2 + 16 * k16) * 256;
        const i16x4 lo = lds_read_tr(a);
        const i16x4 hi = lds_read_tr(a + 8 * 256);
        w.acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(join(lo, hi), pf[t2][k16], w.acc[dt], 0, 0, 0);
      }
}

// The fused form's inputs (QKV = true): q and v are read in place from the [B*S, ld] output of a
// fused q|k|v projection (query head hd of token t at row b*S + t, columns hd*128 ..; kv head j's v
// at columns vcol + j*128 ..), and each q row gets its per-head RMSNorm (weight w, eps) and
// rotate-half RoPE (cos/sin [S, 128] fp32) in the prologue, with the fp32 operations of
// qk_norm_rope in the same order (the sum of squares chunk by chunk, then the same pairwise tree),
// so the result is bit-identical to the qk_norm_rope + transpose + attention launches.
struct QkvIn {
  const uint16_t* w;
  const float* cos;
  const float* sin;
  float eps;
  int ld;
  int vcol;
};

// 8 bf16 of a 16-byte word as fp32 (exact)
__device__ __forceinline__ void unpack8(const u32x4& v, float (&f)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(v[i] << 16);
    f[2 * i + 1] = __uint_as_float(v[i] & 0xffff0000u);
  }
}

// A wave's 32 query rows (row r at base + r*ld, 128 bf16 each), loaded as whole 128-byte halves of
// 8 rows per instruction: lane (r8, c8) = (lane / 8, lane % 8) receives v[4*p + t] = chunk 8*p + c8
// (d = 64*p + 8*c8 .. +7) of row 8*t + r8.  (Read straight in the MFMA fragment layout, one
// instruction would touch 32 rows.)
__device__ __forceinline__ void load_q_rows(const uint16_t* __restrict__ base, int64_t ld, int lane, u32x4 (&v)[8]) {
  const int r8 = lane >> 3, c8 = lane & 7;
#pragma unroll
  for (int p = 0; p < 2; ++p)
#pragma unroll
    for (int t = 0; t < 4; ++t)
      v[4 * p + t] = *reinterpret_cast<const u32x4*>(base + int64_t(8 * t + r8) * ld + 64 * p + 8 * c8);
}

// The rows of load_q_rows in the MFMA B-fragment layout: lane (fr, h) receives raw[kk] = chunk
// 2*kk + h (d = 16*kk + 8*h .. +7) of row fr.  Each half of the dims passes through the wave's own
// 4 KB LDS region (row-major, 16-byte chunk c of row r in slot c ^ ((r >> 1) & 7), so that the
// writes and the fragment reads are bank-conflict free).  A wave's LDS operations complete in
// order, so the region needs no barrier between its writes and reads, nor between the two halves.
__device__ __forceinline__ void q_rows_to_fragments(const u32x4 (&v)[8], uint8_t* region, int lane, u32x4 (&raw)[8]) {
  const int r8 = lane >> 3, c8 = lane & 7, fr = lane & 31, h = lane >> 5;
#pragma unroll
  for (int p = 0; p < 2; ++p) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int row = 8 * t + r8;
      *reinterpret_cast<u32x4*>(region + row * 128 + ((c8 ^ ((row >> 1) & 7)) << 4)) = v[4 * p + t];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
      raw[4 * p + j] = *reinterpret_cast<const u32x4*>(region + fr * 128 + (((2 * j + h) ^ ((fr >> 1) & 7)) << 4));
  }
}

// The fused form's per-head RMSNorm and rotate-half RoPE of the rows of load_q_rows (row 8*t + r8 at
// position pos0 + 8*t + r8), in place, with the fp32 operations of qk_norm_rope in the same order:
// each chunk's sum of squares by fma in element order, then the pairwise tree over the 16 chunks,
// (c, c^1), (c, c^2) and (c, c^4) across the lane's 8-lane group by DPP (quad_perm pairs, then
// row_half_mirror, whose partner quad holds one equal value per lane), then (c, c^8) within the
// lane, which holds both halves 8p + c8; chunk c is rotated against chunk c ^ 8, also in the lane.
// The fp32 cos/sin loads likewise cover 8 rows per instruction (a lane's 32 bytes in two halves).
__device__ __forceinline__ void qnorm_rope_rows(u32x4 (&v)[8], const QkvIn& in, int pos0, int lane) {
  const int r8 = lane >> 3, c8 = lane & 7;
  float w[2][8];
  unpack8(reinterpret_cast<const u32x4*>(in.w)[c8], w[0]);
  unpack8(reinterpret_cast<const u32x4*>(in.w)[8 + c8], w[1]);
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    float f[2][8], s[2];
    unpack8(v[t], f[0]);
    unpack8(v[4 + t], f[1]);
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      s[p] = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) s[p] = fmaf(f[p][e], f[p][e], s[p]);
      s[p] += dpp_f32<0xb1>(s[p]);
      s[p] += dpp_f32<0x4e>(s[p]);
      s[p] += dpp_f32<0x141>(s[p]);
    }
    const float ss = s[0] + s[1];
    const float r = 1.0f / sqrtf(ss / 128.f + in.eps);
    const int64_t pos = pos0 + 8 * t + r8;
    const float* cs = in.cos + pos * 128;
    const float* sn = in.sin + pos * 128;
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int d0 = 64 * p + 8 * c8;
      const f32x4v c0 = reinterpret_cast<const f32x4v*>(cs + d0)[0], c1 = reinterpret_cast<const f32x4v*>(cs + d0)[1];
      const f32x4v s0 = reinterpret_cast<const f32x4v*>(sn + d0)[0], s1 = reinterpret_cast<const f32x4v*>(sn + d0)[1];
      const float cv[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
      const float sv[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
      u32x4 o;
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        float y[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const float a = (f[p][e + u] * r) * w[p][e + u];
          const float q = (f[1 - p][e + u] * r) * w[1 - p][e + u];
          const float rot = p == 0 ? -q : q;
          y[u] = fmaf(a, cv[e + u], rot * sv[e + u]);
        }
        o[e / 2] = pack_bf16x2(y[0], y[1]);
      }
      v[4 * p + t] = o;
    }
  }
}

// WAVES = 8: 256 query rows per workgroup, one workgroup per CU; WAVES = 4: 128 rows, two per CU
// (more, smaller workgroups balance the causal triangle when there are few 256-row tiles).
template <int WAVES, bool QKV = false>
__global__ __launch_bounds__(64 * WAVES) __attribute__((amdgpu_waves_per_eu(2, 2))) void flash_fwd_kernel(
    const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K, const uint16_t* __restrict__ V,
    uint16_t* __restrict__ O, int S, int hq, int hkv, int nkv, int nt, float c, int negate, int causal,
    int o_tokens, QkvIn qin) {
  constexpr int BQ = 32 * WAVES;               // query rows per workgroup
  constexpr int kDmaT = 16 / WAVES;            // DMA instructions per wave per 16 KB tile
  __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * kStageBytes];

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
  const int kvi = r % nkv;
  const int b = kvi / hkv, kvh = kvi % hkv;
  const int64_t bh = int64_t(b) * hq + kvh * G + g;
  const uint16_t* qp = Q + bh * S * D;
  const uint16_t* kp = K + int64_t(kvi) * S * D;
  // V rows: D apart in [B*HKV, S, D], or ld apart in the fused projection output
  const int64_t vrow = QKV ? qin.ld : D;
  const uint16_t* vp = QKV ? V + int64_t(b) * S * qin.ld + qin.vcol + kvh * D : V + int64_t(kvi) * S * D;
  uint16_t* op = O + bh * S * D;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = lane >> 5, fr = lane & 31;
  // Rows of this wave, and the end of the workgroup's query range (its last key, when causal).
  // causal & 2 (8 waves; S a multiple of 128): work unit u pairs the 128-row tiles S/128 - 1 - u
  // (waves 0-3) and u (waves 4-7), so every unit carries the same causal work and each SIMD holds
  // one wave of the heavy tile beside one of the light tile; in the middle unit of an odd tile count
  // both are the same tile and waves 4-7 stay idle.  Otherwise tile r / nkv, heaviest-first.
  int qw0, qend;
  bool active;
  if (WAVES == 8 && (causal & 2)) {
    const int u = r / nkv, ta = S / 128 - 1 - u, half = wave >> 2;
    qw0 = (half ? u : ta) * 128 + (wave & 3) * 32;
    active = !half || u < ta;
    qend = (ta + 1) * 128;
  } else {
    const int tile = causal ? nt - 1 - r / nkv : r / nkv;
    qw0 = tile * BQ + wave * 32;
    active = qw0 < S;                  // S is a multiple of 32: a wave's rows are all in or all out
    qend = min(tile * BQ + BQ, S);
  }
  const int qi = qw0 + fr;             // this lane's query

  // ---- K/V loaders: instruction t of this wave fills key rows 4*(kDmaT*wave + t) .. +3 of a tile;
  //      lane L writes row L/16, slot L%16, so it fetches the chunk that belongs in that slot
  const uint32_t kv_bytes = uint32_t(S) * D * 2u;
  const i32x4 rsrc_k = make_rsrc(kp, kv_bytes);
  const i32x4 rsrc_v = make_rsrc(vp, uint32_t((int64_t(S) - 1) * vrow * 2 + D * 2));
  uint32_t k_voff[kDmaT], v_voff[kDmaT];
#pragma unroll
  for (int t = 0; t < kDmaT; ++t) {
    const int key = 4 * (kDmaT * wave + t) + (lane >> 4);
    const int slot = lane & 15;
    k_voff[t] = uint32_t(key * D + ((slot ^ (key & 15)) * 8)) * 2u;
    v_voff[t] = uint32_t(int64_t(key) * vrow + ((slot ^ (4 * (key & 3))) * 8)) * 2u;
  }
  const uint32_t lds0 = uint32_t(reinterpret_cast<uintptr_t>(smem));
  // par = kb & 1, a compile-time constant at every call, so stage addresses fold into the LDS
  // instructions' offset fields
  auto issue_block = [&](int kb, auto par) __attribute__((always_inline)) {
    const uint32_t st = lds0 + uint32_t(decltype(par)::value) * kStageBytes;
    const uint32_t soff = uint32_t(kb) * uint32_t(kTileBytes);
    const uint32_t soff_v = uint32_t(int64_t(kb) * BKV * vrow * 2);
#pragma unroll
    for (int t = 0; t < kDmaT; ++t)
      dma16(rsrc_k, __builtin_amdgcn_readfirstlane(st + (wave * kDmaT + t) * 1024), k_voff[t], soff);
#pragma unroll
    for (int t = 0; t < kDmaT; ++t)
      dma16(rsrc_v, __builtin_amdgcn_readfirstlane(st + kTileBytes + (wave * kDmaT + t) * 1024), v_voff[t],
            soff_v);
  };

  // ---- fragment addressing
  // K (A operand of S^T): key row 32*t2 + fr, chunk 2*kk + h in slot (2*kk + h) ^ (fr & 15)
  uint32_t koff[8];
  {
    const int s = h ^ (fr & 15);
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) koff[kk] = uint32_t(fr * 256 + (((2 * kk) ^ s) << 4));
  }
  // V^T (A operand of O^T): 16-lane group -> d half 16*g16; in-group lane 4*jj + q supplies key
  // base + 4h + jj, d 32*dt + 16*g16 + 4q .. +3 (chunk 4dt + 2g16 + q/2, byte 8*(q&1) within it)
  uint32_t voff[4];
  {
    const int g16 = (lane >> 4) & 1, l16 = lane & 15, jj = l16 >> 2, q = l16 & 3;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      const int chunk = 4 * dt + 2 * g16 + (q >> 1);
      voff[dt] = uint32_t((4 * h + jj) * 256 + ((chunk ^ (4 * jj)) << 4) + (q & 1) * 8);
    }
  }

  // ---- Q fragments (B operand of S^T = K Q^T): 8 K-steps of 16 over d; a negative scale is
  //      carried by Q's sign (exact in bf16) so that c > 0 and the max commutes with the scaling
  // the first K/V block's DMA goes out before the query loads: its latency overlaps theirs
  issue_block(0, std::integral_constant<int, 0>{});

  // the query rows pass through stage 1, which the first block leaves free; the barrier at the top
  // of that block (its fences wait for these LDS reads) comes before anything is loaded into it
  static_assert(WAVES * 4096 <= kStageBytes, "the query staging regions fit in one stage");
  bf16x8 qf[8];
  if (active) {
    const uint32_t flip = negate ? 0x80008000u : 0u;
    uint8_t* const qstage = smem + kStageBytes + wave * 4096;
    u32x4 v[8], raw[8];
    if constexpr (QKV) {
      load_q_rows(Q + (int64_t(b) * S + qw0) * qin.ld + (kvh * G + g) * D, qin.ld, lane, v);
      qnorm_rope_rows(v, qin, qw0, lane);
    } else {
      load_q_rows(qp + int64_t(qw0) * D, D, lane, v);
    }
    q_rows_to_fragments(v, qstage, lane, raw);
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) qf[kk] = __builtin_bit_cast(bf16x8, raw[kk] ^ flip);
  }

  WaveState w;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) w.acc[i][e] = 0.f;
  w.m = -INFINITY;
  w.l = 0.f;
  f32x16 sacc[2];
  bf16x8 pf[2][2];

  // causal: the workgroup needs keys up to its last row; a wave stops at the block holding its
  // diagonal (blocks past it are fully masked); inactive waves compute nothing
  const int nb = causal ? qend / BKV : S / BKV;
  const int last = !active ? -1 : causal ? (qw0 + 31) / BKV : nb - 1;
  auto block = [&](int kb, auto par) __attribute__((always_inline)) {
    constexpr int P = decltype(par)::value;
    wait_vmcnt<0>();
    __syncthreads();  // block kb landed (all waves); every wave is done with block kb-1's stage
    if (kb + 1 < nb) issue_block(kb + 1, std::integral_constant<int, 1 - P>{});
    if (kb <= last) {
      const uint32_t st = lds0 + uint32_t(P) * kStageBytes;
      qk_step(sacc, qf, st, koff);
      if (causal && kb == last)
        softmax_step<true>(w, sacc, pf, c, qi - kb * BKV - 4 * h);
      else
        softmax_step<false>(w, sacc, pf, c, 0);
      pv_step(w, pf, st + kTileBytes, voff);
    }
  };
  int kb = 0;
  for (; kb + 1 < nb; kb += 2) {   // two blocks a trip: the stage of each is a constant
    block(kb, std::integral_constant<int, 0>{});
    block(kb + 1, std::integral_constant<int, 1>{});
  }
  if (kb < nb) block(kb, std::integral_constant<int, 0>{});
  __syncthreads();   // every wave is done with the last block's stage: the LDS is free
  if (!active) return;

  const float l = pair32_sum(w.l);
  const float inv = 1.f / l;
  // The output tile leaves through the LDS, 64 of the 128 dims at a time: the lane holding query
  // row fr writes its 8 four-dim pieces into the wave's private, padded region, then each lane
  // reads 16 bytes of one row back, so a store instruction writes 8 rows' 128-byte segments (in
  // the accumulator layout it writes 8 bytes into each of 32 rows).  The region is the wave's own
  // and LDS operations of a wave complete in order, so no barrier separates its writes from its
  // reads.  O is [batch*hq, S, D] (head-major), or with o_tokens [batch, S, hq, D] (token-major).
  constexpr int kOPitch = 64 * 2 + 16;   // bytes per staged half row
  static_assert(WAVES * 32 * kOPitch <= 2 * kStageBytes, "the staging regions fit in the stages' LDS");
  uint8_t* const ostage = smem + wave * (32 * kOPitch);
  const int rl = lane >> 3, c8 = lane & 7;
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) {
#pragma unroll
    for (int dd = 0; dd < 2; ++dd)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int dt = 2 * hf + dd;
        *reinterpret_cast<u32x2*>(ostage + fr * kOPitch + (dd * 32 + 8 * g4 + 4 * h) * 2) =
            u32x2{pack_bf16x2(w.acc[dt][4 * g4] * inv, w.acc[dt][4 * g4 + 1] * inv),
                  pack_bf16x2(w.acc[dt][4 * g4 + 2] * inv, w.acc[dt][4 * g4 + 3] * inv)};
      }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int r = 8 * t + rl, q = qw0 + r;
      const u32x4 v = *reinterpret_cast<const u32x4*>(ostage + r * kOPitch + c8 * 16);
      uint16_t* orow = o_tokens ? O + ((int64_t(b) * S + q) * hq + (kvh * G + g)) * D : op + int64_t(q) * D;
      *reinterpret_cast<u32x4*>(orow + 64 * hf + 8 * c8) = v;
    }
  }
}

}  // namespace

// qin.w non-null: the fused form (q and v read from the projection output, q normalised in place)
static int flash_launch(const void* q, const void* k, const void* v, void* o, int64_t batch, int64_t hq, int64_t hkv,
                        int64_t seq, int64_t head_dim, float scale, int causal, int o_tokens, const QkvIn& qin,
                        void* stream) {
  if (batch < 0 || hq <= 0 || hkv <= 0 || seq < 0 || head_dim <= 0) return PTB_ERR_SHAPE;
  if (hq % hkv) return PTB_ERR_SHAPE;
  if (head_dim != D) return PTB_ERR_UNSUPPORTED;
  if (!std::isfinite(scale) || scale == 0.f) return PTB_ERR_UNSUPPORTED;
  if (batch == 0 || seq == 0) return PTB_OK;
  if (!q || !k || !v || !o) return PTB_ERR_NULL;
  if (seq % 128) return PTB_ERR_UNSUPPORTED;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o)) return PTB_ERR_ALIGN;
  const bool fused = qin.w != nullptr;
  const int64_t nkv = batch * hkv;
  // 256-row workgroups when there are at least two per CU (non-causal: one, since every workgroup
  // then carries the same work), else 128-row ones (two per CU)
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess) hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  const bool wide = ((seq + 255) / 256) * batch * hq >= (causal ? 2 : 1) * int64_t(cus);
  // causal with too few 256-row tiles: 256-row workgroups that each pair a heavy and a light 128-row
  // tile when those units fill at least 3/4 of the CUs in one round, else 128-row workgroups
  const int64_t units = (seq / 128 + 1) / 2 * batch * hq;
  const bool paired = causal && !wide && units <= cus && 4 * units >= 3 * int64_t(cus);
  const int64_t bq = wide ? 256 : 128;
  const int64_t nt = paired ? (seq / 128 + 1) / 2 : (seq + bq - 1) / bq;
  const int64_t total = nt * nkv * (hq / hkv);
  // K/V of one kv head are addressed through a 32-bit buffer range (v with its row stride)
  const int64_t vrow = fused ? qin.ld : D;
  if (total > 0x7fffffff || seq * vrow * 2 >= (int64_t(1) << 32) || batch * hq * seq > (int64_t(1) << 40))
    return PTB_ERR_GRID;
  const float c = std::fabs(scale) * 1.4426950408889634f;
  hipStream_t s = static_cast<hipStream_t>(stream);
  auto qp = static_cast<const uint16_t*>(q), kp = static_cast<const uint16_t*>(k), vp = static_cast<const uint16_t*>(v);
  auto op = static_cast<uint16_t*>(o);
  const int neg = scale < 0.f ? 1 : 0, cz = causal ? (paired ? 3 : 1) : 0;
  const unsigned grid = unsigned(total);
  if ((wide || paired) && fused)
    flash_fwd_kernel<8, true><<<grid, 512, 0, s>>>(qp, kp, vp, op, int(seq), int(hq), int(hkv), int(nkv), int(nt), c,
                                                   neg, cz, o_tokens, qin);
  else if (wide || paired)
    flash_fwd_kernel<8><<<grid, 512, 0, s>>>(qp, kp, vp, op, int(seq), int(hq), int(hkv), int(nkv), int(nt), c, neg,
                                             cz, o_tokens, qin);
  else if (fused)
    flash_fwd_kernel<4, true><<<grid, 256, 0, s>>>(qp, kp, vp, op, int(seq), int(hq), int(hkv), int(nkv), int(nt), c,
                                                   neg, cz, o_tokens, qin);
  else
    flash_fwd_kernel<4><<<grid, 256, 0, s>>>(qp, kp, vp, op, int(seq), int(hq), int(hkv), int(nkv), int(nt), c, neg,
                                             cz, o_tokens, qin);
  return launch_status();
}

PTB_EXPORT int ptb_flash_attn_fwd_bf16(const void* q, const void* k, const void* v, void* o, int64_t batch,
                                       int64_t hq, int64_t hkv, int64_t seq, int64_t head_dim, float scale,
                                       int causal, void* stream) {
  return flash_launch(q, k, v, o, batch, hq, hkv, seq, head_dim, scale, causal, 0, QkvIn{}, stream);
}

PTB_EXPORT int ptb_flash_attn_fwd_tokens_bf16(const void* q, const void* k, const void* v, void* o, int64_t batch,
                                              int64_t hq, int64_t hkv, int64_t seq, int64_t head_dim, float scale,
                                              int causal, void* stream) {
  return flash_launch(q, k, v, o, batch, hq, hkv, seq, head_dim, scale, causal, 1, QkvIn{}, stream);
}

PTB_EXPORT int ptb_flash_attn_fwd_qkv_bf16(const void* qkv, int64_t ld, const void* k, const void* qnorm_w,
                                           const float* cos_t, const float* sin_t, float eps, void* o,
                                           int64_t batch, int64_t hq, int64_t hkv, int64_t seq, int64_t head_dim,
                                           float scale, int causal, void* stream) {
  if (hq <= 0 || hkv <= 0 || ld < (hq + 2 * hkv) * D || ld > 0x7fffffff) return PTB_ERR_SHAPE;
  if (batch > 0 && seq > 0 && head_dim == D) {
    if (!qnorm_w || !cos_t || !sin_t) return PTB_ERR_NULL;
    if (ld % 8 || !aligned16(qnorm_w) || !aligned16(cos_t) || !aligned16(sin_t)) return PTB_ERR_ALIGN;
  }
  const QkvIn qin{static_cast<const uint16_t*>(qnorm_w), cos_t, sin_t, eps, int(ld), int((hq + hkv) * D)};
  return flash_launch(qkv, k, qkv, o, batch, hq, hkv, seq, head_dim, scale, causal, 1, qin, stream);
}
