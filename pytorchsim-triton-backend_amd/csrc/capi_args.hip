// Spec-driven entry points: one per kernel family, taking the kernel's tensors in spec order as
// memref-style descriptors, its integer and floating-point parameters, and the launch grid -- the
// call the reference's generated driver makes of a lowered kernel, program loop included
// (pytorchsim_triton_compiler/codegen/wrapper.py:37-51, :126-277).  Each entry checks the
// descriptors (count, dtype, size against the parameters, stride, role of the written tensors),
// refuses a grid past the family's program bound as contract/kernel_object.py:93-107 does, and then
// runs the typed entry point of include/ptb_amd.h over the programs the grid covers.  Host code
// only: no kernels live here.
#include <algorithm>

#include "ptb_common.h"

namespace {

int64_t itemsize(int dt) {
  switch (dt) {
    case PTB_DTYPE_BF16: return 2;
    case PTB_DTYPE_F32: return 4;
    case PTB_DTYPE_I32: return 4;
    case PTB_DTYPE_I64: return 8;
    case PTB_DTYPE_E4M3: return 1;
    default: return 0;
  }
}

struct View {
  void* p;
  int64_t n;
  int dt;
};

// One descriptor: flat (stride 1), a known dtype, a non-negative size; `written` tensors must not be
// declared read-only.
int view_of(const ptb_tensor& t, bool written, View& v) {
  const int64_t is = itemsize(t.dtype);
  if (is == 0) return PTB_ERR_DTYPE;
  if (t.size < 0 || t.offset < 0) return PTB_ERR_SHAPE;
  if (t.size > 1 && t.stride != 1) return PTB_ERR_UNSUPPORTED;
  if (written && t.role == PTB_ROLE_IN) return PTB_ERR_SHAPE;
  if (t.role != PTB_ROLE_IN && t.role != PTB_ROLE_OUT && t.role != PTB_ROLE_INOUT) return PTB_ERR_SHAPE;
  if (!t.aligned && t.size) return PTB_ERR_NULL;
  v.p = static_cast<uint8_t*>(t.aligned) + t.offset * is;
  v.n = t.size;
  v.dt = t.dtype;
  return PTB_OK;
}

// The grid a launch asks for against the family's program bound (programs along x only, as every
// family here runs its reference kernel's programs along one axis): gx in [1, bound], gy = gz = 1.
int grid_programs(const int32_t* grid, int64_t bound, int64_t& gx) {
  if (!grid) return PTB_ERR_NULL;
  if (grid[0] < 1 || grid[1] != 1 || grid[2] != 1 || grid[0] > bound) return PTB_ERR_GRID;
  gx = grid[0];
  return PTB_OK;
}

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Rows (or elements) per program: ints[at] when the caller states it (the kernel's XBLOCK), else
// the extent split evenly over the programs.  A program past the extent covers nothing.
int block_of(const int64_t* ints, int nints, int at, int64_t extent, int64_t programs, int64_t& block) {
  block = nints > at ? ints[at] : ceil_div(extent, programs);
  return block > 0 || extent == 0 ? PTB_OK : PTB_ERR_SHAPE;
}

#define PTB_TRY(expr)           \
  do {                          \
    const int st_ = (expr);     \
    if (st_ != PTB_OK) return st_; \
  } while (0)

}  // namespace

PTB_EXPORT int ptb_rmsnorm_args(const ptb_tensor* args, int nargs, const int64_t* ints, int nints,
                                const double* floats, int nfloats, const int32_t grid[3], void* stream) {
  if (!args || !ints || !floats) return PTB_ERR_NULL;
  if ((nargs != 3 && nargs != 4) || (nints != 3 && nints != 4) || nfloats != 1) return PTB_ERR_SHAPE;
  View x, w, y, c{nullptr, 0, 0};
  PTB_TRY(view_of(args[0], false, x));
  PTB_TRY(view_of(args[1], false, w));
  PTB_TRY(view_of(args[2], true, y));
  if (nargs == 4) PTB_TRY(view_of(args[3], true, c));
  const int64_t rows = ints[0], cols = ints[1], programs = ints[2];
  if (rows < 0 || cols <= 0 || programs <= 0) return PTB_ERR_SHAPE;
  if (x.n != rows * cols || y.n != x.n || w.n != cols || (nargs == 4 && c.n != cols)) return PTB_ERR_SHAPE;
  int64_t gx, block;
  PTB_TRY(grid_programs(grid, programs, gx));
  PTB_TRY(block_of(ints, nints, 3, rows, programs, block));
  const int64_t r = std::min(rows, gx * block);   // the row blocks the grid covers
  const float eps = float(floats[0]);
  if (x.dt == PTB_DTYPE_F32) {
    if (w.dt != PTB_DTYPE_F32 || y.dt != PTB_DTYPE_F32 || (nargs == 4 && c.dt != PTB_DTYPE_F32)) return PTB_ERR_DTYPE;
    PTB_TRY(ptb_rmsnorm_f32(static_cast<const float*>(x.p), static_cast<const float*>(w.p), static_cast<float*>(y.p),
                            r, cols, eps, stream));
    // the column arm (tests/cases/workloads/rmsnorm.py:56-57): c = rsqrt(mean over the rows of x^2 + eps)
    if (nargs == 4) return ptb_col_rms_f32(static_cast<const float*>(x.p), static_cast<float*>(c.p), r, cols, eps, stream);
    return PTB_OK;
  }
  if (nargs == 4) return PTB_ERR_DTYPE;   // the column arm exists in the fp32 case only
  if (x.dt != PTB_DTYPE_BF16 || y.dt != PTB_DTYPE_BF16) return PTB_ERR_DTYPE;
  if (w.dt != PTB_DTYPE_BF16 && w.dt != PTB_DTYPE_F32) return PTB_ERR_DTYPE;
  return ptb_rmsnorm_bf16(x.p, w.p, w.dt, y.p, r, cols, eps, stream);
}

PTB_EXPORT int ptb_softmax_args(const ptb_tensor* args, int nargs, const int64_t* ints, int nints,
                                const double* floats, int nfloats, const int32_t grid[3], void* stream) {
  (void)floats;
  if (!args || !ints) return PTB_ERR_NULL;
  if (nargs != 2 || (nints != 3 && nints != 4) || nfloats != 0) return PTB_ERR_SHAPE;
  View x, y;
  PTB_TRY(view_of(args[0], false, x));
  PTB_TRY(view_of(args[1], true, y));
  const int64_t rows = ints[0], cols = ints[1], programs = ints[2];
  if (rows < 0 || cols <= 0 || programs <= 0) return PTB_ERR_SHAPE;
  if (x.n != rows * cols || y.n != x.n) return PTB_ERR_SHAPE;
  int64_t gx, block;
  PTB_TRY(grid_programs(grid, programs, gx));
  PTB_TRY(block_of(ints, nints, 3, rows, programs, block));
  const int64_t r = std::min(rows, gx * block);
  if (x.dt == PTB_DTYPE_F32) {
    if (y.dt != PTB_DTYPE_F32) return PTB_ERR_DTYPE;
    return ptb_softmax_rows_f32(static_cast<const float*>(x.p), static_cast<float*>(y.p), r, cols, stream);
  }
  if (x.dt != PTB_DTYPE_BF16) return PTB_ERR_DTYPE;
  if (y.dt == PTB_DTYPE_BF16) return ptb_softmax_rows_bf16(x.p, y.p, r, cols, stream);
  if (y.dt == PTB_DTYPE_F32) return ptb_softmax_rows_bf16_f32(x.p, y.p, r, cols, stream);
  return PTB_ERR_DTYPE;
}

PTB_EXPORT int ptb_silu_mul_args(const ptb_tensor* args, int nargs, const int64_t* ints, int nints,
                                 const double* floats, int nfloats, const int32_t grid[3], void* stream) {
  (void)floats;
  if (!args || !ints) return PTB_ERR_NULL;
  if (nargs != 2 || (nints != 3 && nints != 4) || nfloats != 0) return PTB_ERR_SHAPE;
  View gu, out;
  PTB_TRY(view_of(args[0], false, gu));
  PTB_TRY(view_of(args[1], true, out));
  const int64_t rows = ints[0], inter = ints[1], programs = ints[2];
  if (rows < 0 || inter <= 0 || programs <= 0) return PTB_ERR_SHAPE;
  if (gu.n != 2 * rows * inter || out.n != rows * inter || gu.dt != out.dt) return PTB_ERR_SHAPE;
  int64_t gx, block;
  PTB_TRY(grid_programs(grid, programs, gx));
  PTB_TRY(block_of(ints, nints, 3, rows * inter, programs, block));
  const int64_t n = std::min(rows * inter, gx * block);   // outputs the grid covers
  if (n % inter) return PTB_ERR_UNSUPPORTED;             // a partial grid must end on a whole row
  if (gu.dt == PTB_DTYPE_F32)
    return ptb_silu_mul_f32(static_cast<const float*>(gu.p), static_cast<float*>(out.p), n / inter, inter, stream);
  if (gu.dt != PTB_DTYPE_BF16) return PTB_ERR_DTYPE;
  return ptb_silu_mul_bf16(gu.p, out.p, n / inter, inter, stream);
}

PTB_EXPORT int ptb_gemm_args(const ptb_tensor* args, int nargs, const int64_t* ints, int nints, const double* floats,
                             int nfloats, const int32_t grid[3], void* stream) {
  (void)floats;
  if (!args || !ints) return PTB_ERR_NULL;
  if ((nargs != 3 && nargs != 4) || nints != 4 || nfloats != 0) return PTB_ERR_SHAPE;
  const bool resid = nargs == 4;   // the residual epilogue kernels take the residual first
  View r{nullptr, 0, PTB_DTYPE_BF16}, a, b, c;
  if (resid) PTB_TRY(view_of(args[0], false, r));
  PTB_TRY(view_of(args[resid + 0], false, a));
  PTB_TRY(view_of(args[resid + 1], false, b));
  PTB_TRY(view_of(args[resid + 2], true, c));
  const int64_t m = ints[0], n = ints[1], k = ints[2], programs = ints[3];
  if (m < 0 || n < 0 || k < 0 || programs <= 0) return PTB_ERR_SHAPE;
  if (a.n != m * k || b.n != k * n || c.n != m * n || (resid && r.n != m * n)) return PTB_ERR_SHAPE;
  if (a.dt != PTB_DTYPE_BF16 || b.dt != PTB_DTYPE_BF16 || c.dt != PTB_DTYPE_BF16 || r.dt != PTB_DTYPE_BF16)
    return PTB_ERR_DTYPE;
  int64_t gx;
  PTB_TRY(grid_programs(grid, programs, gx));
  if (gx != programs) return PTB_ERR_UNSUPPORTED;   // a partial grid's tiles follow the caller's template order
  return ptb_gemm_bf16(a.p, b.p, resid ? r.p : nullptr, c.p, m, n, k, stream);
}

PTB_EXPORT int ptb_flash_attn_args(const ptb_tensor* args, int nargs, const int64_t* ints, int nints,
                                   const double* floats, int nfloats, const int32_t grid[3], void* stream) {
  if (!args || !ints || !floats) return PTB_ERR_NULL;
  if (nargs != 4 || nints != 6 || nfloats != 1) return PTB_ERR_SHAPE;
  View q, k, v, o;
  PTB_TRY(view_of(args[0], false, q));
  PTB_TRY(view_of(args[1], false, k));
  PTB_TRY(view_of(args[2], false, v));
  PTB_TRY(view_of(args[3], true, o));
  const int64_t batch = ints[0], hq = ints[1], hkv = ints[2], seq = ints[3], d = ints[4], causal = ints[5];
  if (batch < 0 || hq <= 0 || hkv <= 0 || seq < 0 || d <= 0 || hq % hkv) return PTB_ERR_SHAPE;
  if (q.n != batch * hq * seq * d || o.n != q.n || k.n != batch * hkv * seq * d || v.n != k.n) return PTB_ERR_SHAPE;
  if (q.dt != PTB_DTYPE_BF16 || k.dt != q.dt || v.dt != q.dt || o.dt != q.dt) return PTB_ERR_DTYPE;
  int64_t gx;   // one program per (batch, query head), as _prefill_kernel's grid
  PTB_TRY(grid_programs(grid, std::max<int64_t>(1, batch * hq), gx));
  if (gx % hq) return PTB_ERR_UNSUPPORTED;   // a partial grid must cover whole batches
  return ptb_flash_attn_fwd_bf16(q.p, k.p, v.p, o.p, gx / hq, hq, hkv, seq, d, float(floats[0]), causal ? 1 : 0,
                                 stream);
}

PTB_EXPORT int ptb_attn_decode_args(const ptb_tensor* args, int nargs, const int64_t* ints, int nints,
                                    const double* floats, int nfloats, const int32_t grid[3], void* stream) {
  if (!args || !ints || !floats) return PTB_ERR_NULL;
  if ((nargs != 4 && nargs != 5) || nints != 4 || nfloats != 1) return PTB_ERR_SHAPE;
  View q, k, v, o, ws{nullptr, 0, PTB_DTYPE_I32};
  PTB_TRY(view_of(args[0], false, q));
  PTB_TRY(view_of(args[1], false, k));
  PTB_TRY(view_of(args[2], false, v));
  PTB_TRY(view_of(args[3], true, o));
  if (nargs == 5) PTB_TRY(view_of(args[4], true, ws));   // the workspace, any dtype
  const int64_t nkv = ints[0], g = ints[1], seq = ints[2], d = ints[3];
  if (nkv < 0 || g <= 0 || seq <= 0 || d <= 0) return PTB_ERR_SHAPE;
  if (q.n != nkv * g * d || o.n != q.n || k.n != nkv * seq * d || v.n != k.n) return PTB_ERR_SHAPE;
  if (q.dt != PTB_DTYPE_BF16 || k.dt != q.dt || v.dt != q.dt || o.dt != q.dt) return PTB_ERR_DTYPE;
  int64_t gx;   // one program per kv head, as _decode_kernel's grid
  PTB_TRY(grid_programs(grid, std::max<int64_t>(1, nkv), gx));
  if (gx != std::max<int64_t>(1, nkv)) return PTB_ERR_UNSUPPORTED;
  return ptb_attn_decode_bf16(q.p, k.p, v.p, o.p, nkv, g, seq, d, float(floats[0]), ws.p,
                              size_t(ws.n * itemsize(ws.dt)), stream);
}

PTB_EXPORT int ptb_qk_norm_rope_args(const ptb_tensor* args, int nargs, const int64_t* ints, int nints,
                                     const double* floats, int nfloats, const int32_t grid[3], void* stream) {
  if (!args || !ints || !floats) return PTB_ERR_NULL;
  if (nargs != 5 || nints != 4 || nfloats != 1) return PTB_ERR_SHAPE;
  View x, w, c, s, o;
  PTB_TRY(view_of(args[0], false, x));
  PTB_TRY(view_of(args[1], false, w));
  PTB_TRY(view_of(args[2], false, c));
  PTB_TRY(view_of(args[3], false, s));
  PTB_TRY(view_of(args[4], true, o));
  const int64_t t = ints[0], h = ints[1], d = ints[2], programs = ints[3];
  if (t < 0 || h <= 0 || d <= 0 || programs <= 0) return PTB_ERR_SHAPE;
  if (x.n != t * h * d || o.n != x.n || w.n != d || c.n != t * d || s.n != c.n) return PTB_ERR_SHAPE;
  if (x.dt != PTB_DTYPE_BF16 || w.dt != x.dt || o.dt != x.dt || c.dt != PTB_DTYPE_F32 || s.dt != c.dt)
    return PTB_ERR_DTYPE;
  int64_t gx;   // programs over the (token, head) rows
  PTB_TRY(grid_programs(grid, programs, gx));
  if (gx != programs) return PTB_ERR_UNSUPPORTED;   // the head-major output keeps the full token stride
  return ptb_qk_norm_rope_bf16(x.p, w.p, static_cast<const float*>(c.p), static_cast<const float*>(s.p), o.p, t, h,
                               d, float(floats[0]), stream);
}

PTB_EXPORT int ptb_transpose_heads_args(const ptb_tensor* args, int nargs, const int64_t* ints, int nints,
                                        const double* floats, int nfloats, const int32_t grid[3], void* stream) {
  (void)floats;
  if (!args || !ints) return PTB_ERR_NULL;
  if (nargs != 2 || nints != 4 || nfloats != 0) return PTB_ERR_SHAPE;
  View x, y;
  PTB_TRY(view_of(args[0], false, x));
  PTB_TRY(view_of(args[1], true, y));
  const int64_t d0 = ints[0], d1 = ints[1], inner = ints[2], programs = ints[3];
  if (d0 < 0 || d1 < 0 || inner <= 0 || programs <= 0) return PTB_ERR_SHAPE;
  if (x.n != d0 * d1 * inner || y.n != x.n) return PTB_ERR_SHAPE;
  if (x.dt != PTB_DTYPE_BF16 || y.dt != x.dt) return PTB_ERR_DTYPE;
  int64_t gx;
  PTB_TRY(grid_programs(grid, programs, gx));
  if (gx != programs) return PTB_ERR_UNSUPPORTED;
  return ptb_transpose_heads_bf16(x.p, y.p, d0, d1, inner, stream);
}

namespace {

// The whole grid only: these families reduce over, or address, every element of their tensors.
int whole_grid(const int32_t* grid, int64_t programs) {
  int64_t gx;
  PTB_TRY(grid_programs(grid, programs, gx));
  return gx == programs ? PTB_OK : PTB_ERR_UNSUPPORTED;
}

// A trailing workspace descriptor (any dtype), written by the entry: its pointer and bytes.
int workspace_of(const ptb_tensor* args, int nargs, int at, void*& p, size_t& bytes) {
  p = nullptr;
  bytes = 0;
  if (nargs == at) return PTB_OK;
  if (nargs != at + 1) return PTB_ERR_SHAPE;
  View ws;
  PTB_TRY(view_of(args[at], true, ws));
  p = ws.p;
  bytes = size_t(ws.n * itemsize(ws.dt));
  return PTB_OK;
}

}  // namespace

PTB_EXPORT int ptb_sumsq_args(const ptb_tensor* args, int nargs, const int64_t* ints, int nints,
                              const double* floats, int nfloats, const int32_t grid[3], void* stream) {
  (void)floats;
  if (!args || !ints) return PTB_ERR_NULL;
  if ((nargs != 2 && nargs != 3) || nints != 2 || nfloats != 0) return PTB_ERR_SHAPE;
  View x, y{nullptr, 0, PTB_DTYPE_BF16}, out;
  PTB_TRY(view_of(args[0], false, x));
  if (nargs == 3) PTB_TRY(view_of(args[1], false, y));
  PTB_TRY(view_of(args[nargs - 1], true, out));
  const int64_t n = ints[0], programs = ints[1];
  if (n < 0 || programs <= 0) return PTB_ERR_SHAPE;
  if (x.n != n || (nargs == 3 && y.n != n) || out.n != 1) return PTB_ERR_SHAPE;
  if (x.dt != PTB_DTYPE_BF16 || y.dt != PTB_DTYPE_BF16 || out.dt != PTB_DTYPE_F32) return PTB_ERR_DTYPE;
  PTB_TRY(whole_grid(grid, programs));
  return ptb_sumsq_bf16(x.p, nargs == 3 ? y.p : nullptr, static_cast<float*>(out.p), n, stream);
}

PTB_EXPORT int ptb_gemv_args(const ptb_tensor* args, int nargs, const int64_t* ints, int nints, const double* floats,
                             int nfloats, const int32_t grid[3], void* stream) {
  if (!args || !ints) return PTB_ERR_NULL;
  if (nints != 5) return PTB_ERR_SHAPE;
  const int64_t mode = ints[0], k = ints[1], n = ints[2], extra = ints[3], programs = ints[4];
  if (k <= 0 || n <= 0 || programs <= 0) return PTB_ERR_SHAPE;
  // tensors before the workspace: plain [x, W, y]; rmsnorm [x, (add,) ss, g, W, y]; silu
  // [gate_up, W, (res_a, (res_b,)) y]
  int base;
  if (mode == 0 && extra == 0) base = 3;
  else if (mode == 1 && (extra == 0 || extra == 1)) base = 5 + int(extra);
  else if (mode == 2 && extra >= 0 && extra <= 2) base = 3 + int(extra);
  else return PTB_ERR_UNSUPPORTED;
  if (nargs < base || nfloats != (mode == 1 ? 1 : 0) || (mode == 1 && !floats)) return PTB_ERR_SHAPE;
  View v[6];
  for (int i = 0; i < base; ++i) PTB_TRY(view_of(args[i], i == base - 1, v[i]));
  void* ws;
  size_t ws_bytes;
  PTB_TRY(workspace_of(args, nargs, base, ws, ws_bytes));
  const View& y = v[base - 1];
  if (y.n != n || y.dt != PTB_DTYPE_BF16) return y.n != n ? PTB_ERR_SHAPE : PTB_ERR_DTYPE;
  PTB_TRY(whole_grid(grid, programs));
  if (mode == 0) {
    const View &x = v[0], &w = v[1];
    if (x.n != k || w.n != k * n) return PTB_ERR_SHAPE;
    if (x.dt != PTB_DTYPE_BF16 || w.dt != PTB_DTYPE_BF16) return PTB_ERR_DTYPE;
    return ptb_gemv_bf16(x.p, w.p, y.p, k, n, ws, ws_bytes, stream);
  }
  if (mode == 1) {
    const View& x = v[0];
    const View* add = extra ? &v[1] : nullptr;
    const View &ss = v[1 + extra], &g = v[2 + extra], &w = v[3 + extra];
    if (x.n != k || (add && add->n != k) || ss.n != 1 || g.n != k || w.n != k * n) return PTB_ERR_SHAPE;
    if (x.dt != PTB_DTYPE_BF16 || (add && add->dt != PTB_DTYPE_BF16) || ss.dt != PTB_DTYPE_F32 ||
        g.dt != PTB_DTYPE_BF16 || w.dt != PTB_DTYPE_BF16)
      return PTB_ERR_DTYPE;
    return ptb_gemv_rmsnorm_bf16(x.p, add ? add->p : nullptr, static_cast<const float*>(ss.p), g.p,
                                 float(floats[0]), w.p, y.p, k, n, ws, ws_bytes, stream);
  }
  const View &gu = v[0], &w = v[1];
  if (gu.n != 2 * k || w.n != k * n) return PTB_ERR_SHAPE;
  for (int i = 2; i < 2 + extra; ++i)
    if (v[i].n != n) return PTB_ERR_SHAPE;
  for (int i = 0; i < base; ++i)
    if (v[i].dt != PTB_DTYPE_BF16) return PTB_ERR_DTYPE;
  return ptb_gemv_silu_bf16(gu.p, w.p, extra > 0 ? v[2].p : nullptr, extra > 1 ? v[3].p : nullptr, y.p, k, n, ws,
                            ws_bytes, stream);
}

PTB_EXPORT int ptb_reduce_args(const ptb_tensor* args, int nargs, const int64_t* ints, int nints,
                               const double* floats, int nfloats, const int32_t grid[3], void* stream) {
  (void)floats;
  if (!args || !ints) return PTB_ERR_NULL;
  if ((nargs != 2 && nargs != 3) || nints != 3 || nfloats != 0) return PTB_ERR_SHAPE;
  View x, out;
  PTB_TRY(view_of(args[0], false, x));
  PTB_TRY(view_of(args[1], true, out));
  void* ws;
  size_t ws_bytes;
  PTB_TRY(workspace_of(args, nargs, 2, ws, ws_bytes));
  const int64_t n = ints[0], op = ints[1], programs = ints[2];
  if (n < 0 || programs <= 0) return PTB_ERR_SHAPE;
  if (op != PTB_REDUCE_SUM && op != PTB_REDUCE_MAX) return PTB_ERR_UNSUPPORTED;
  if (x.n != n || out.n != 1) return PTB_ERR_SHAPE;
  if (out.dt != PTB_DTYPE_F32) return PTB_ERR_DTYPE;
  PTB_TRY(whole_grid(grid, programs));
  if (x.dt == PTB_DTYPE_BF16)
    return ptb_reduce_bf16(x.p, static_cast<float*>(out.p), n, int(op), ws, ws_bytes, stream);
  if (x.dt == PTB_DTYPE_F32)
    return ptb_reduce_f32(static_cast<const float*>(x.p), static_cast<float*>(out.p), n, int(op), ws, ws_bytes,
                          stream);
  return PTB_ERR_DTYPE;
}

PTB_EXPORT int ptb_add_scalar_args(const ptb_tensor* args, int nargs, const int64_t* ints, int nints,
                                   const double* floats, int nfloats, const int32_t grid[3], void* stream) {
  if (!args || !ints || !floats) return PTB_ERR_NULL;
  if (nargs != 2 || (nints != 2 && nints != 3) || nfloats != 1) return PTB_ERR_SHAPE;
  View x, y;
  PTB_TRY(view_of(args[0], false, x));
  PTB_TRY(view_of(args[1], true, y));
  const int64_t n = ints[0], programs = ints[1];
  if (n < 0 || programs <= 0) return PTB_ERR_SHAPE;
  if (x.n != n || y.n != n) return PTB_ERR_SHAPE;
  if (x.dt != PTB_DTYPE_BF16 || y.dt != PTB_DTYPE_BF16) return PTB_ERR_DTYPE;
  int64_t gx, block;   // programs over blocks of elements: a partial grid covers its leading blocks
  PTB_TRY(grid_programs(grid, programs, gx));
  PTB_TRY(block_of(ints, nints, 2, n, programs, block));
  return ptb_add_scalar_bf16(x.p, y.p, std::min(n, gx * block), float(floats[0]), stream);
}

PTB_EXPORT int ptb_slice_add_args(const ptb_tensor* args, int nargs, const int64_t* ints, int nints,
                                  const double* floats, int nfloats, const int32_t grid[3], void* stream) {
  if (!args || !ints || !floats) return PTB_ERR_NULL;
  if (nargs != 2 || nints != 3 || nfloats != 1) return PTB_ERR_SHAPE;
  View x, out;
  PTB_TRY(view_of(args[0], false, x));
  PTB_TRY(view_of(args[1], true, out));
  const int64_t first = ints[0], count = ints[1], programs = ints[2];
  if (first < 0 || count < 0 || programs <= 0) return PTB_ERR_SHAPE;
  if (out.n != count || first + count > x.n) return PTB_ERR_SHAPE;
  if (x.dt != PTB_DTYPE_BF16 || out.dt != PTB_DTYPE_F32) return PTB_ERR_DTYPE;
  PTB_TRY(whole_grid(grid, programs));
  return ptb_slice_add_bf16(x.p, static_cast<float*>(out.p), first, count, float(floats[0]), stream);
}
