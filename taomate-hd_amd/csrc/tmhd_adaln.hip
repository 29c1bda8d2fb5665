// Row-wise bf16 RMSNorm / AdaLN-modulate / residual-gate ops of the DiT block
// around every attention call, for gfx950.  Reference: the "SOL" fused
// kernels of src/taomate_hd/inference/fused_kernels.py:221-255 (_modulate,
// _gate_add), 312-383 (_rms_norm, _rms_norm_modulate,
// _residual_gate_rms_norm_modulate) and their wrappers :636-671, 706-796,
// with the rounding helper _round_bf16 (:58-61) written R() below.
//
//   RMS       out = R((x * inv) * w)
//   RMS_MOD   n = R((x * inv) * w);  out = R(R(n * R(1 + scale[t])) + shift[t])
//   RES_MOD   h = R(res + R(gate[t] * branch));  hidden = h;
//             n = R((h * inv_h) * w);  out = R(R(n * R(1 + scale[t])) + shift[t])
//   MOD       out = R(R(x * R(1 + scale[t])) + shift[t])
//   GATE      out = R(res + R(gate[t] * branch))
// with t = index[row] selecting the table row and inv = 1 / sqrt(sum(x^2) /
// cols + eps).
//
// One wave per row, 4 rows per 256-thread block; the row stays in registers
// between the sum and the normalization.  Lane l holds 8-column chunks
// l, l + 64, l + 128, ...; the kernels are HBM-bound (rows read and written
// once, tables and weights hit in cache).
//
// Fixed where the reference leaves it to its compiler:
//   * sum of squares: per lane over its chunks in order, 8 columns each in
//     order, as a chain of fused multiply-adds; then a pairwise tree over the
//     64 lanes in lane order (lane ^ 1, ^ 2, ^ 4, ^ 8 by DPP, ^ 16, ^ 32);
//   * inverse RMS: correctly rounded division and square root.
// R() is gfx950's f32 -> bf16 conversion, which equals the reference's
// integer rounding on every value that reaches it here (the rounding
// self-check covers it).
#include <algorithm>

#include "tmhd_internal.h"

namespace tmhd {
namespace {

enum RowOp { kRms = 0, kRmsMod = 1, kResMod = 2, kMod = 3, kGate = 4 };

struct RowArgs {
  const uint16_t *x;  // value, or the residual of RES_MOD / GATE
  int64_t x_stride;
  const uint16_t *branch;
  int64_t branch_stride;
  const uint16_t *gate, *scale, *shift;
  int64_t gate_stride, scale_stride, shift_stride;
  const int64_t *index;
  int64_t table_rows;  // table indices are clamped to [0, table_rows)
  const uint16_t *weight;
  uint16_t *hidden;
  int64_t hidden_stride;
  uint16_t *out;
  int64_t out_stride;
  int64_t rows;
  int32_t cols;
  float eps;
};

__device__ __forceinline__ float lo_f32(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_f32(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xf, 0xf, false));
}

// pairwise tree over the 64 lanes in lane order; every lane gets the total
__device__ __forceinline__ float wave_sum_tree(float s) {
  s = s + dpp<0xb1>(s);   // lane ^ 1 (quad_perm 1,0,3,2)
  s = s + dpp<0x4e>(s);   // lane ^ 2 (quad_perm 2,3,0,1)
  s = s + dpp<0x141>(s);  // other quad of the 8 (half-row mirror)
  s = s + dpp<0x140>(s);  // other 8 of the 16 (row mirror)
  s = s + __shfl_xor(s, 16);
  s = s + __shfl_xor(s, 32);
  return s;
}

// AdaLN modulation of one packed pair of normalized values: R(R(n * R(1 + sc)) + sh)
__device__ __forceinline__ uint32_t modulate_pair(uint32_t n, uint32_t sc, uint32_t sh) {
  const uint32_t s1 = pack_bf16_rne(1.0f + lo_f32(sc), 1.0f + hi_f32(sc));
  const uint32_t m = pack_bf16_rne(lo_f32(n) * lo_f32(s1), hi_f32(n) * hi_f32(s1));
  return pack_bf16_rne(lo_f32(m) + lo_f32(sh), hi_f32(m) + hi_f32(sh));
}

// R(res + R(g * b)) on a packed pair
__device__ __forceinline__ uint32_t gate_add_pair(uint32_t res, uint32_t g, uint32_t b) {
  const uint32_t gb = pack_bf16_rne(lo_f32(g) * lo_f32(b), hi_f32(g) * hi_f32(b));
  return pack_bf16_rne(lo_f32(res) + lo_f32(gb), hi_f32(res) + hi_f32(gb));
}

template <int OP, int MAXCH>
__global__ void __launch_bounds__(256) row_kernel(const RowArgs a) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.rows) return;  // whole waves only: a row is one wave
  const int nch = a.cols >> 3;
  constexpr bool kTable = OP != kRms;
  constexpr bool kNorm = OP == kRms || OP == kRmsMod || OP == kResMod;
  const int64_t t = kTable ? min(max(a.index[row], (int64_t)0), a.table_rows - 1) : 0;
  i32x4 v[MAXCH];
#pragma unroll
  for (int i = 0; i < MAXCH; ++i) {
    const int c = lane + 64 * i;
    if (c < nch) v[i] = *(const i32x4 *)(a.x + row * a.x_stride + 8 * c);
  }
  if constexpr (OP == kResMod || OP == kGate) {
    i32x4 b[MAXCH];
#pragma unroll
    for (int i = 0; i < MAXCH; ++i) {
      const int c = lane + 64 * i;
      if (c < nch) b[i] = *(const i32x4 *)(a.branch + row * a.branch_stride + 8 * c);
    }
#pragma unroll
    for (int i = 0; i < MAXCH; ++i) {
      const int c = lane + 64 * i;
      if (c < nch) {
        const i32x4 g = *(const i32x4 *)(a.gate + t * a.gate_stride + 8 * c);
        i32x4 h;
#pragma unroll
        for (int e = 0; e < 4; ++e) h[e] = (int)gate_add_pair((uint32_t)v[i][e], (uint32_t)g[e], (uint32_t)b[i][e]);
        v[i] = h;
        if constexpr (OP == kGate)
          *(i32x4 *)(a.out + row * a.out_stride + 8 * c) = h;
        else  // the new residual stream, read again only after the attention and the MLP: a
              // non-temporal store keeps it from evicting `out`, which the next kernel reads at once
          __builtin_nontemporal_store(h, (i32x4 *)(a.hidden + row * a.hidden_stride + 8 * c));
      }
    }
    if constexpr (OP == kGate) return;
  }
  float inv = 1.0f;
  if constexpr (kNorm) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < MAXCH; ++i) {
      const int c = lane + 64 * i;
      if (c < nch) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float x = (e & 1) ? hi_f32((uint32_t)v[i][e >> 1]) : lo_f32((uint32_t)v[i][e >> 1]);
          s = (i == 0 && e == 0) ? x * x : __builtin_fmaf(x, x, s);
        }
      }
    }
    s = wave_sum_tree(s);
    inv = __fdiv_rn(1.0f, sqrt_rn(__fdiv_rn(s, (float)a.cols) + a.eps));
  }
#pragma unroll
  for (int i = 0; i < MAXCH; ++i) {
    const int c = lane + 64 * i;
    if (c < nch) {
      i32x4 o;
      i32x4 w, sc, sh;
      if constexpr (kNorm) w = *(const i32x4 *)(a.weight + 8 * c);
      if constexpr (kTable) {
        sc = *(const i32x4 *)(a.scale + t * a.scale_stride + 8 * c);
        sh = *(const i32x4 *)(a.shift + t * a.shift_stride + 8 * c);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        uint32_t n = (uint32_t)v[i][e];
        if constexpr (kNorm) {
          const uint32_t ww = (uint32_t)w[e];
          n = pack_bf16_rne((lo_f32(n) * inv) * lo_f32(ww), (hi_f32(n) * inv) * hi_f32(ww));
        }
        if constexpr (kTable) n = modulate_pair(n, (uint32_t)sc[e], (uint32_t)sh[e]);
        o[e] = (int)n;
      }
      *(i32x4 *)(a.out + row * a.out_stride + 8 * c) = o;
    }
  }
}

// SwiGLU over [rows][2 * half] (gate | up): out = R(R(g * sigmoid(g)) * u),
// sigmoid(g) = 1 / (1 + exp(-g)) with the accurate single-precision exp and a
// correctly rounded division.  8 columns per thread, grid-stride.
__global__ void __launch_bounds__(256) swiglu_kernel(const uint16_t *x, int64_t x_stride, uint16_t *out,
                                                     int64_t out_stride, int64_t rows, int32_t half) {
#pragma clang fp contract(off)
  const int64_t per_row = half >> 3;
  const int64_t total = rows * per_row;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / per_row, c = (i - r * per_row) * 8;
    const i32x4 g = *(const i32x4 *)(x + r * x_stride + c);
    const i32x4 u = *(const i32x4 *)(x + r * x_stride + half + c);
    i32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = (int)swiglu_pair((uint32_t)g[e], (uint32_t)u[e]);
    *(i32x4 *)(out + r * out_stride + c) = o;
  }
}

bool al16(const void *p) { return ((uintptr_t)p % 16) == 0; }

template <int OP>
int launch_rows(const RowArgs &a, void *stream, const char *what) {
  if (a.rows == 0) return TMHD_OK;
  const int nch = a.cols / 8;
  const dim3 grid((unsigned)((a.rows + 3) / 4)), block(256);
  hipStream_t s = (hipStream_t)stream;
  if (nch <= 64 * 4)
    hipLaunchKernelGGL((row_kernel<OP, 4>), grid, block, 0, s, a);
  else if (nch <= 64 * 8)
    hipLaunchKernelGGL((row_kernel<OP, 8>), grid, block, 0, s, a);
  else if (nch <= 64 * 12)  // the DiT's 5376 columns
    hipLaunchKernelGGL((row_kernel<OP, 12>), grid, block, 0, s, a);
  else
    hipLaunchKernelGGL((row_kernel<OP, 16>), grid, block, 0, s, a);
  return check_launch(what);
}

// Shared argument checks; `need` lists which pointers the op reads.
int check_rows(const char *what, const RowArgs &a, bool norm, bool table, bool branch, bool hidden) {
  if (a.rows < 0 || a.cols <= 0 || a.cols % 8 || a.cols > 8192)
    return set_error(TMHD_ERR_UNSUPPORTED, "%s: rows %lld cols %d (cols a multiple of 8 up to 8192)", what,
                     (long long)a.rows, a.cols);
  if (a.rows > ((int64_t)0x7fffffff - 3) * 4) return set_error(TMHD_ERR_UNSUPPORTED, "%s: too many rows", what);
  if (norm && !(a.eps >= 0.0f)) return set_error(TMHD_ERR_INVALID, "%s: eps must be >= 0", what);
  if (a.rows == 0) return TMHD_OK;
  bool ok = a.x && a.out && al16(a.x) && al16(a.out) && a.x_stride % 8 == 0 && a.out_stride % 8 == 0 &&
            a.x_stride >= a.cols && a.out_stride >= a.cols;
  if (norm) ok = ok && a.weight && al16(a.weight);
  if (table)
    ok = ok && a.index && a.table_rows > 0 && a.scale && a.shift && al16(a.scale) && al16(a.shift) && a.scale_stride % 8 == 0 &&
         a.shift_stride % 8 == 0 && a.scale_stride >= a.cols && a.shift_stride >= a.cols;
  if (branch)
    ok = ok && a.branch && a.gate && al16(a.branch) && al16(a.gate) && a.branch_stride % 8 == 0 &&
         a.gate_stride % 8 == 0 && a.branch_stride >= a.cols && a.gate_stride >= a.cols;
  if (hidden) ok = ok && a.hidden && al16(a.hidden) && a.hidden_stride % 8 == 0 && a.hidden_stride >= a.cols;
  if (!ok) return set_error(TMHD_ERR_INVALID, "%s: pointers and row strides must be 16-byte aligned rows", what);
  return -1;  // go on
}

}  // namespace
}  // namespace tmhd

using namespace tmhd;

extern "C" int tmhd_rms_norm(const void *x, int64_t x_stride, void *out, int64_t out_stride, const void *weight,
                             int64_t rows, int32_t cols, float eps, void *stream) {
  RowArgs a{};
  a.x = (const uint16_t *)x, a.x_stride = x_stride, a.out = (uint16_t *)out, a.out_stride = out_stride;
  a.weight = (const uint16_t *)weight, a.rows = rows, a.cols = cols, a.eps = eps;
  const int rc = check_rows("tmhd_rms_norm", a, true, false, false, false);
  return rc >= 0 ? rc : launch_rows<kRms>(a, stream, "tmhd_rms_norm");
}

extern "C" int tmhd_rms_norm_modulate(const void *x, int64_t x_stride, void *out, int64_t out_stride,
                                      const void *weight, const void *scale, int64_t scale_stride,
                                      const void *shift, int64_t shift_stride, const int64_t *index, int64_t table_rows,
                                      int64_t rows, int32_t cols, float eps, void *stream) {
  RowArgs a{};
  a.x = (const uint16_t *)x, a.x_stride = x_stride, a.out = (uint16_t *)out, a.out_stride = out_stride;
  a.weight = (const uint16_t *)weight, a.scale = (const uint16_t *)scale, a.scale_stride = scale_stride;
  a.shift = (const uint16_t *)shift, a.shift_stride = shift_stride, a.index = index;
  a.table_rows = table_rows, a.rows = rows, a.cols = cols, a.eps = eps;
  const int rc = check_rows("tmhd_rms_norm_modulate", a, true, true, false, false);
  return rc >= 0 ? rc : launch_rows<kRmsMod>(a, stream, "tmhd_rms_norm_modulate");
}

extern "C" int tmhd_residual_gate_rms_norm_modulate(const void *residual, int64_t residual_stride, const void *branch,
                                                    int64_t branch_stride, const void *gate, int64_t gate_stride,
                                                    const void *weight, const void *scale, int64_t scale_stride,
                                                    const void *shift, int64_t shift_stride, const int64_t *index,
                                                    int64_t table_rows, void *hidden, int64_t hidden_stride, void *out,
                                                    int64_t out_stride, int64_t rows, int32_t cols, float eps,
                                                    void *stream) {
  RowArgs a{};
  a.x = (const uint16_t *)residual, a.x_stride = residual_stride;
  a.branch = (const uint16_t *)branch, a.branch_stride = branch_stride;
  a.gate = (const uint16_t *)gate, a.gate_stride = gate_stride;
  a.weight = (const uint16_t *)weight, a.scale = (const uint16_t *)scale, a.scale_stride = scale_stride;
  a.shift = (const uint16_t *)shift, a.shift_stride = shift_stride, a.index = index, a.table_rows = table_rows;
  a.hidden = (uint16_t *)hidden, a.hidden_stride = hidden_stride, a.out = (uint16_t *)out, a.out_stride = out_stride;
  a.rows = rows, a.cols = cols, a.eps = eps;
  const int rc = check_rows("tmhd_residual_gate_rms_norm_modulate", a, true, true, true, true);
  return rc >= 0 ? rc : launch_rows<kResMod>(a, stream, "tmhd_residual_gate_rms_norm_modulate");
}

extern "C" int tmhd_modulate(const void *x, int64_t x_stride, void *out, int64_t out_stride, const void *scale,
                             int64_t scale_stride, const void *shift, int64_t shift_stride, const int64_t *index,
                             int64_t table_rows, int64_t rows, int32_t cols, void *stream) {
  RowArgs a{};
  a.x = (const uint16_t *)x, a.x_stride = x_stride, a.out = (uint16_t *)out, a.out_stride = out_stride;
  a.scale = (const uint16_t *)scale, a.scale_stride = scale_stride, a.shift = (const uint16_t *)shift;
  a.shift_stride = shift_stride, a.index = index, a.table_rows = table_rows, a.rows = rows, a.cols = cols;
  const int rc = check_rows("tmhd_modulate", a, false, true, false, false);
  return rc >= 0 ? rc : launch_rows<kMod>(a, stream, "tmhd_modulate");
}

extern "C" int tmhd_gate_add(const void *residual, int64_t residual_stride, const void *gate, int64_t gate_stride,
                             const void *branch, int64_t branch_stride, const int64_t *index, int64_t table_rows,
                             void *out, int64_t out_stride, int64_t rows, int32_t cols, void *stream) {
  RowArgs a{};
  a.x = (const uint16_t *)residual, a.x_stride = residual_stride;
  a.gate = (const uint16_t *)gate, a.gate_stride = gate_stride;
  a.branch = (const uint16_t *)branch, a.branch_stride = branch_stride, a.index = index, a.table_rows = table_rows;
  a.out = (uint16_t *)out, a.out_stride = out_stride, a.rows = rows, a.cols = cols;
  // the gate table is indexed like the modulation tables
  RowArgs chk = a;
  chk.scale = chk.shift = chk.gate, chk.scale_stride = chk.shift_stride = gate_stride;
  const int rc = check_rows("tmhd_gate_add", chk, false, true, true, false);
  return rc >= 0 ? rc : launch_rows<kGate>(a, stream, "tmhd_gate_add");
}

extern "C" int tmhd_swiglu(const void *x, int64_t x_stride, void *out, int64_t out_stride, int64_t rows, int32_t half,
                           void *stream) {
  const char *what = "tmhd_swiglu";
  if (rows < 0 || half <= 0 || half % 8)
    return set_error(TMHD_ERR_UNSUPPORTED, "%s: rows %lld half %d (a multiple of 8)", what, (long long)rows, half);
  if (rows == 0) return TMHD_OK;
  if (!x || !out || !al16(x) || !al16(out) || x_stride % 8 || out_stride % 8 || x_stride < 2 * (int64_t)half ||
      out_stride < half)
    return set_error(TMHD_ERR_INVALID, "%s: pointers and row strides must be 16-byte aligned rows", what);
  const int64_t total = rows * (half / 8);
  const int64_t blocks = std::min<int64_t>((total + 255) / 256, 256 * 64);
  hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t *)x, x_stride, (uint16_t *)out, out_stride, rows, half);
  return check_launch(what);
}
