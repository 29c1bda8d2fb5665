// Q/K RMSNorm + RoPE in place inside a merged [tokens, 3 * heads * head_dim]
// bf16 QKV projection, for gfx950.  Reference: fused_qkv_qk_norm_rope_ /
// _merged_qkv_preprocess_kernel, src/taomate_hd/inference/fused_kernels.py:
// 425-472 and 826-873, with its bf16 rounding helper _round_bf16 (:58-61).
//
// Work: one row = the head_dim channels of one (token, head, Q or K).  A
// group of head_dim / 8 lanes holds a row, 8 channels per lane as two pieces
// of 4 (8 bytes each): lane j < rotary / 8 holds channels 4j.. and
// rotary / 2 + 4j.., so both halves of its rotation pairs sit in the lane;
// the other lanes hold 8 consecutive channels of the unrotated tail.  A wave
// does 4 groups of 64 / (head_dim / 8) rows, loads all 4 before computing
// any, and computes the 4 rows' inverse RMS in one pass (one row per lane of
// each quad).  The kernel reads and writes the Q and K thirds of the buffer
// once; its instruction count is kept below what the HBM traffic takes.
//
// Fixed where the reference leaves it to its compiler:
//   * sum of squares: per lane over its 8 channels in the order above as a
//     chain of fused multiply-adds, then a pairwise tree over the row's lanes
//     in lane order (DPP: lane ^ 1, ^ 2, mirror within 8, mirror within 16,
//     which add the same pairs as the tree);
//   * inverse RMS: 1 / sqrt(variance + eps) with correctly rounded square
//     root and division.
// The bf16 rounding is gfx950's f32 -> bf16 conversion (round to nearest
// even).  It gives the reference's integer rounding (+ 0x7FFF + bit 16, low
// half cleared) for every non-NaN float and for every quiet NaN whose low 16
// bits are zero, the only NaNs that reach it here: arithmetic quiets NaNs and
// takes their payload from bf16 inputs, whose low 16 bits are zero.
#include <math.h>

#include "tmhd_internal.h"

namespace tmhd {
namespace {

using float2_t = float __attribute__((ext_vector_type(2)));

// Two floats to packed bf16, rounded to nearest even; and back.
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  const float2_t f = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2));
}
__device__ __forceinline__ float lo_f32(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_f32(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xf, 0xf, false));
}
constexpr int kQuadXor1 = 0xb1, kQuadXor2 = 0x4e, kHalfRowMirror = 0x141, kRowMirror = 0x140;

struct RopeArgs {
  uint16_t *qkv;
  int64_t row_stride;  // elements between tokens
  const uint16_t *qw, *kw;
  const uint16_t *cs;  // cos | sin rows
  int64_t cs_stride;
  const int64_t *pos;
  int64_t cs_rows;  // positions are clamped to [0, cs_rows)
  int32_t tokens, heads, rotary;
  float eps;
};

constexpr int kRopeUnroll = 4;  // row groups per wave; one per lane of a quad in the inverse RMS pass

template <int D>
__global__ void __launch_bounds__(256) qkv_norm_rope_kernel(const RopeArgs a) {
#pragma clang fp contract(off)
  constexpr int LPR = D / 8;     // lanes per row
  constexpr int RPW = 64 / LPR;  // rows per wave and group
  constexpr int U = kRopeUnroll;
  const int lane = threadIdx.x & 63, j = lane % LPR;
  const int two_h = 2 * a.heads;  // tokens * two_h is below 2^31 (host check)
  const int row0 = (blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * U * RPW + lane / LPR;
  const int half = a.rotary >> 1, rot_lanes = a.rotary >> 3;
  const bool rotates = j < rot_lanes;
  const int oa = rotates ? 4 * j : a.rotary + 8 * (j - rot_lanes);  // channel of piece A
  const int ob = rotates ? half + 4 * j : oa + 4;                   // channel of piece B
  uint16_t *ptr[U];
  bool live[U], is_k[U];
  int64_t pos[U];
  int token = row0 / two_h, rem = row0 - token * two_h;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (u) {
      rem += RPW;
      while (rem >= two_h) rem -= two_h, ++token;
    }
    live[u] = token < a.tokens;
    const int t = live[u] ? token : a.tokens - 1;  // lanes past the end compute a copy of the last row, unstored
    const int r = live[u] ? rem : two_h - 1;
    is_k[u] = r >= a.heads;
    ptr[u] = a.qkv + (int64_t)t * a.row_stride + (int64_t)r * D;
    if (a.rotary) pos[u] = a.pos[t];  // issued first: the cos / sin loads wait only for these
  }
  i32x2 xa[U], xb[U], ca[U], sa[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    xa[u] = *(const i32x2 *)(ptr[u] + oa);
    xb[u] = *(const i32x2 *)(ptr[u] + ob);
  }
  const i32x2 qwa = *(const i32x2 *)(a.qw + oa), qwb = *(const i32x2 *)(a.qw + ob);
  const i32x2 kwa = *(const i32x2 *)(a.kw + oa), kwb = *(const i32x2 *)(a.kw + ob);
  if (a.rotary) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t p = min(max(pos[u], (int64_t)0), a.cs_rows - 1);
      const uint16_t *crow = a.cs + p * a.cs_stride + (rotates ? 4 * j : 0);
      ca[u] = *(const i32x2 *)crow;
      sa[u] = *(const i32x2 *)(crow + half);
    }
  }

  float x[U][8], ss[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t w[4] = {(uint32_t)xa[u][0], (uint32_t)xa[u][1], (uint32_t)xb[u][0], (uint32_t)xb[u][1]};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[u][2 * e] = lo_f32(w[e]);
      x[u][2 * e + 1] = hi_f32(w[e]);
    }
    float s = x[u][0] * x[u][0];
#pragma unroll
    for (int e = 1; e < 8; ++e) s = __builtin_fmaf(x[u][e], x[u][e], s);
    s = s + dpp<kQuadXor1>(s);
    s = s + dpp<kQuadXor2>(s);
    s = s + dpp<kHalfRowMirror>(s);
    if (LPR == 16) s = s + dpp<kRowMirror>(s);
    ss[u] = s;
  }
  // lane q of each quad computes group q's inverse RMS, then each group reads it back
  const int q = lane & 3;
  const float sq = q == 0 ? ss[0] : q == 1 ? ss[1] : q == 2 ? ss[2] : ss[3];
  const float var = sq * (1.0f / D);  // exact: D is a power of two
  const float inv_q = __fdiv_rn(1.0f, __fsqrt_rn(var + a.eps));
  const float inv[U] = {dpp<0x00>(inv_q), dpp<0x55>(inv_q), dpp<0xaa>(inv_q), dpp<0xff>(inv_q)};

  const uint32_t qw[4] = {(uint32_t)qwa[0], (uint32_t)qwa[1], (uint32_t)qwb[0], (uint32_t)qwb[1]};
  const uint32_t kw[4] = {(uint32_t)kwa[0], (uint32_t)kwa[1], (uint32_t)kwb[0], (uint32_t)kwb[1]};
#pragma unroll
  for (int u = 0; u < U; ++u) {
    uint32_t nb[4];  // normalized, packed bf16: A pieces in 0-1, B in 2-3
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t w = is_k[u] ? kw[e] : qw[e];
      nb[e] = pack_bf16((x[u][2 * e] * inv[u]) * lo_f32(w), (x[u][2 * e + 1] * inv[u]) * hi_f32(w));
    }
    uint32_t out[4] = {nb[0], nb[1], nb[2], nb[3]};
    if (a.rotary) {
      // rotation pairs (A[e], B[e]): A' = A cos - B sin, B' = B cos + A sin, each
      // product and sum rounded to bf16 (rotate_half(n) = (-B, A))
      const uint32_t cw[2] = {(uint32_t)ca[u][0], (uint32_t)ca[u][1]};
      const uint32_t sw[2] = {(uint32_t)sa[u][0], (uint32_t)sa[u][1]};
      float oa_[4], ob_[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float na = (e & 1) ? hi_f32(nb[e >> 1]) : lo_f32(nb[e >> 1]);
        const float nbv = (e & 1) ? hi_f32(nb[2 + (e >> 1)]) : lo_f32(nb[2 + (e >> 1)]);
        const float c = (e & 1) ? hi_f32(cw[e >> 1]) : lo_f32(cw[e >> 1]);
        const float sn = (e & 1) ? hi_f32(sw[e >> 1]) : lo_f32(sw[e >> 1]);
        const uint32_t p1 = pack_bf16(na * c, nbv * sn);  // A cos, B sin
        const uint32_t p2 = pack_bf16(nbv * c, na * sn);  // B cos, A sin
        oa_[e] = lo_f32(p1) - hi_f32(p1);
        ob_[e] = lo_f32(p2) + hi_f32(p2);
      }
      if (rotates) {
        out[0] = pack_bf16(oa_[0], oa_[1]);
        out[1] = pack_bf16(oa_[2], oa_[3]);
        out[2] = pack_bf16(ob_[0], ob_[1]);
        out[3] = pack_bf16(ob_[2], ob_[3]);
      }
    }
    if (live[u]) {
      *(i32x2 *)(ptr[u] + oa) = i32x2{(int)out[0], (int)out[1]};
      *(i32x2 *)(ptr[u] + ob) = i32x2{(int)out[2], (int)out[3]};
    }
  }
}

}  // namespace
}  // namespace tmhd

extern "C" int tmhd_qkv_norm_rope(void *qkv, int32_t tokens, int32_t heads, int32_t head_dim, int64_t row_stride,
                                  const void *q_weight, const void *k_weight, const void *cos_sin,
                                  int64_t cos_sin_stride, int64_t cos_sin_rows, int32_t rotary_dim,
                                  const int64_t *positions, float eps, void *stream) {
  using namespace tmhd;
  const char *what = "tmhd_qkv_norm_rope";
  if (head_dim != 64 && head_dim != 128)
    return set_error(TMHD_ERR_UNSUPPORTED, "%s: head_dim %d (64 or 128)", what, head_dim);
  if (tokens < 0 || heads <= 0 || row_stride < (int64_t)3 * heads * head_dim)
    return set_error(TMHD_ERR_INVALID, "%s: tokens %d heads %d row_stride %lld", what, tokens, heads,
                     (long long)row_stride);
  if (rotary_dim < 0 || rotary_dim > head_dim || rotary_dim % 16)
    return set_error(TMHD_ERR_UNSUPPORTED, "%s: rotary_dim %d (a multiple of 16 up to head_dim)", what, rotary_dim);
  if (!(eps >= 0.0f)) return set_error(TMHD_ERR_INVALID, "%s: eps must be >= 0", what);
  if (tokens == 0) return TMHD_OK;
  if (!qkv || !q_weight || !k_weight || ((uintptr_t)qkv % 16) || row_stride % 8 || ((uintptr_t)q_weight % 16) ||
      ((uintptr_t)k_weight % 16))
    return set_error(TMHD_ERR_INVALID, "%s: qkv and weights must be 16-byte aligned rows", what);
  if (rotary_dim && (!cos_sin || !positions || ((uintptr_t)cos_sin % 16) || cos_sin_stride % 8 ||
                     cos_sin_stride < rotary_dim || cos_sin_rows <= 0))
    return set_error(TMHD_ERR_INVALID, "%s: cos_sin must be 16-byte aligned rows of >= rotary_dim", what);
  RopeArgs a{(uint16_t *)qkv, row_stride, (const uint16_t *)q_weight, (const uint16_t *)k_weight,
             (const uint16_t *)cos_sin, cos_sin_stride, positions, cos_sin_rows, tokens, heads, rotary_dim, eps};
  const int64_t rows = (int64_t)tokens * 2 * heads;
  const int rows_per_block = 4 * kRopeUnroll * (64 / (head_dim / 8));
  const int64_t blocks = (rows + rows_per_block - 1) / rows_per_block;
  if (rows > 0x7fffffff - rows_per_block) return set_error(TMHD_ERR_UNSUPPORTED, "%s: too many rows", what);
  hipStream_t s = (hipStream_t)stream;
  if (head_dim == 128)
    hipLaunchKernelGGL(qkv_norm_rope_kernel<128>, dim3((unsigned)blocks), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(qkv_norm_rope_kernel<64>, dim3((unsigned)blocks), dim3(256), 0, s, a);
  return check_launch(what);
}
