// Q/K RMSNorm + RoPE in place inside a merged [tokens, 3 * heads * head_dim]
// bf16 QKV projection, for gfx950.  Reference: fused_qkv_qk_norm_rope_ /
// _merged_qkv_preprocess_kernel, src/taomate_hd/inference/fused_kernels.py:
// 425-472 and 826-873, with its bf16 rounding helper _round_bf16 (:58-61).
//
// Work: one row = the head_dim channels of one (token, head, Q or K); a group
// of head_dim / 8 lanes holds a row, 8 channels (16 bytes) per lane, so a
// wave does 4 (D = 128) or 8 (D = 64) rows per group and loads its 4 groups
// before computing any (more bytes in flight).  The kernel is HBM-bound: it
// reads and writes the Q and K thirds of the buffer once.
//
// Fixed where the reference leaves it to its compiler:
//   * sum of squares: per lane over its 8 channels in order, then a butterfly
//     over the row's lanes (xor n/2 .. 1);
//   * inverse RMS: 1 / sqrt(variance + eps) with correctly rounded square
//     root and division.
#include <math.h>

#include "tmhd_internal.h"

namespace tmhd {
namespace {

// The reference's bf16 rounding on fp32 bits: + 0x7FFF + bit 16 (mod 2^32),
// low half cleared.
__device__ __forceinline__ float round_bf16(float x) {
  uint32_t u = __float_as_uint(x);
  u = (u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u;
  return __uint_as_float(u);
}

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

constexpr int kRopeUnroll = 4;  // row groups per wave, loaded before any is computed

template <int D>
__global__ void __launch_bounds__(256) qkv_norm_rope_kernel(const RopeArgs a) {
#pragma clang fp contract(off)
  constexpr int LPR = D / 8;     // lanes per row
  constexpr int RPW = 64 / LPR;  // rows per wave and group
  const int lane = threadIdx.x & 63, j = lane % LPR;
  const int64_t rows = (int64_t)a.tokens * 2 * a.heads;
  const int64_t first = ((int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * kRopeUnroll * RPW;
  uint16_t *ptr[kRopeUnroll];
  int tok[kRopeUnroll], prt[kRopeUnroll];
  bool live[kRopeUnroll];
  i32x4 raw[kRopeUnroll];
#pragma unroll
  for (int u = 0; u < kRopeUnroll; ++u) {
    const int64_t row = first + u * RPW + lane / LPR;
    live[u] = row < rows;
    const int64_t r = live[u] ? row : rows - 1;  // lanes past the end compute a copy of the last row, unstored
    const int token = (int)(r / (2 * a.heads));
    const int rem = (int)(r - (int64_t)token * 2 * a.heads);
    const int part = rem / a.heads, head = rem - part * a.heads;  // part 0: Q, 1: K
    tok[u] = token;
    prt[u] = part;
    ptr[u] = a.qkv + (int64_t)token * a.row_stride + (int64_t)part * a.heads * D + (int64_t)head * D + 8 * j;
    raw[u] = *(const i32x4 *)ptr[u];
  }
  const int half = a.rotary >> 1;
  const int c0 = 8 * j;
#pragma unroll
  for (int u = 0; u < kRopeUnroll; ++u) {
    float v[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[2 * e] = bf16_bits_to_f32((uint32_t)raw[u][e] & 0xffffu);
      v[2 * e + 1] = bf16_bits_to_f32((uint32_t)raw[u][e] >> 16);
    }
    float ss = v[0] * v[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) ss = ss + v[e] * v[e];
#pragma unroll
    for (int k = LPR / 2; k >= 1; k >>= 1) ss = ss + __shfl_xor(ss, k);
    const float variance = __fdiv_rn(ss, (float)D);
    const float inv = __fdiv_rn(1.0f, __fsqrt_rn(variance + a.eps));

    const i32x4 wraw = *(const i32x4 *)((prt[u] ? a.kw : a.qw) + 8 * j);
    float n[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      n[2 * e] = round_bf16((v[2 * e] * inv) * bf16_bits_to_f32((uint32_t)wraw[e] & 0xffffu));
      n[2 * e + 1] = round_bf16((v[2 * e + 1] * inv) * bf16_bits_to_f32((uint32_t)wraw[e] >> 16));
    }
    // the rotary span is a multiple of 16 channels, so a lane's 8 channels are
    // all rotated or all kept, and their partners sit in one other lane
    uint32_t packed[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      packed[e] = (__float_as_uint(n[2 * e]) >> 16) | (__float_as_uint(n[2 * e + 1]) & 0xffff0000u);
    const int plane = (lane - j) + (c0 < half ? j + half / 8 : j - half / 8);
    uint32_t pp[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) pp[e] = (uint32_t)__shfl((int)packed[e], c0 < a.rotary ? plane : lane);
    if (c0 < a.rotary) {
      const int64_t pos = min(max(a.pos[tok[u]], (int64_t)0), a.cs_rows - 1);
      const uint16_t *crow = a.cs + pos * a.cs_stride + (c0 % half);
      const i32x4 craw = *(const i32x4 *)crow;
      const i32x4 sraw = *(const i32x4 *)(crow + half);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t pw = pp[e >> 1], cw = (uint32_t)craw[e >> 1], sw = (uint32_t)sraw[e >> 1];
        const float paired = bf16_bits_to_f32((e & 1) ? (pw >> 16) : (pw & 0xffffu));
        const float rotated = c0 < half ? -paired : paired;
        const float cosv = round_bf16(bf16_bits_to_f32((e & 1) ? (cw >> 16) : (cw & 0xffffu)));
        const float sinv = round_bf16(bf16_bits_to_f32((e & 1) ? (sw >> 16) : (sw & 0xffffu)));
        n[e] = round_bf16(round_bf16(n[e] * cosv) + round_bf16(rotated * sinv));
      }
    }
    if (live[u]) {
      i32x4 out;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        out[e] = (int)((__float_as_uint(n[2 * e]) >> 16) | (__float_as_uint(n[2 * e + 1]) & 0xffff0000u));
      *(i32x4 *)ptr[u] = out;
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
  if (blocks > 0x7fffffff) return set_error(TMHD_ERR_UNSUPPORTED, "%s: too many rows", what);
  hipStream_t s = (hipStream_t)stream;
  if (head_dim == 128)
    hipLaunchKernelGGL(qkv_norm_rope_kernel<128>, dim3((unsigned)blocks), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(qkv_norm_rope_kernel<64>, dim3((unsigned)blocks), dim3(256), 0, s, a);
  return check_launch(what);
}
