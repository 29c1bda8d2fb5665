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
//     root (sqrt_rn) and division.
// The bf16 rounding is gfx950's f32 -> bf16 conversion (round to nearest
// even).  It gives the reference's integer rounding (+ 0x7FFF + bit 16, low
// half cleared) for every non-NaN float and for every quiet NaN whose low 16
// bits are zero, the only NaNs that reach it here: arithmetic quiets NaNs and
// takes their payload from bf16 inputs, whose low 16 bits are zero.
#include <math.h>

#include "tmhd_internal.h"

namespace tmhd {
namespace {

__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) { return pack_bf16_rne(lo, hi); }
__device__ __forceinline__ float lo_f32(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_f32(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xf, 0xf, false));
}
constexpr int kQuadXor1 = 0xb1, kQuadXor2 = 0x4e, kHalfRowMirror = 0x141, kRowMirror = 0x140;

struct RopeArgs {
  const uint16_t *src;
  uint16_t *dst;               // may equal src (in place)
  int64_t src_stride, dst_stride;  // elements between tokens
  const uint16_t *qw, *kw;     // kw for the rows of the second projection
  const uint16_t *cos, *sin;   // TABLE: cos = the cos | sin cache, sin unused
  int64_t cos_stride, sin_stride;
  const int64_t *pos;          // TABLE only
  int64_t cs_rows;             // TABLE only: positions are clamped to [0, cs_rows)
  int32_t tokens, heads, parts, rotary;  // parts: 2 = Q then K of each token, 1 = one projection
  float eps;
  // STAGE only: K rows of tokens [stage_row0, stage_row0 + stage_n) are also
  // written to slot row stage_dst + (t - stage_row0) of kslot (head stride kslot_hs)
  uint16_t *kslot;
  int64_t kslot_hs;
  int32_t stage_row0, stage_n, stage_dst;
  // SEND only: rows go to the Ulysses send buffer instead of back in place:
  // row (t, part p, head h) at ((dest * 3 + p) * tokens + t) * L + l (layout 0)
  // or ((dest * tokens + t) * 3 + p) * L + l (layout 1), dest = h / L, l = h % L
  uint16_t *send;
  int32_t send_local, send_layout;
};

constexpr int kRopeUnroll = 4;  // row groups per wave; one per lane of a quad in the inverse RMS pass

// TABLE: cos / sin of channel d at cos_sin[positions[t]][d % h] and [h + d % h]
// (the merged-projection form); otherwise at cos[t][d] and sin[t][d].
// NORM false: the rotation alone, applied to the input values (no RMSNorm).
// STAGE: the K rows of the staged token range also go to the slot.
// SEND: the rows go to the Ulysses send buffer (the source is left as it is).
template <int D, bool TABLE, bool NORM = true, bool STAGE = false, bool SEND = false>
__global__ void __launch_bounds__(256) qk_norm_rope_kernel(const RopeArgs a) {
#pragma clang fp contract(off)
  constexpr int LPR = D / 8;     // lanes per row
  constexpr int RPW = 64 / LPR;  // rows per wave and group
  constexpr int U = kRopeUnroll;
  const int lane = threadIdx.x & 63, j = lane % LPR;
  const int per_token = a.parts * a.heads;  // tokens * per_token is below 2^31 (host check)
  const int row0 = (blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * U * RPW + lane / LPR;
  const int half = a.rotary >> 1, rot_lanes = a.rotary >> 3;
  const bool rotates = j < rot_lanes;
  const int oa = rotates ? 4 * j : a.rotary + 8 * (j - rot_lanes);  // channel of piece A
  const int ob = rotates ? half + 4 * j : oa + 4;                   // channel of piece B
  int64_t src_off[U], dst_off[U];
  int tok[U], part_row[U];
  bool live[U], is_k[U];
  int64_t pos[U];
  int token = row0 / per_token, rem = row0 - token * per_token;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (u) {
      rem += RPW;
      while (rem >= per_token) rem -= per_token, ++token;
    }
    live[u] = token < a.tokens;
    const int t = live[u] ? token : a.tokens - 1;  // lanes past the end compute a copy of the last row, unstored
    const int r = live[u] ? rem : per_token - 1;
    tok[u] = t;
    part_row[u] = r;
    is_k[u] = r >= a.heads;
    src_off[u] = (int64_t)t * a.src_stride + (int64_t)r * D;
    if constexpr (SEND) {
      const int p = is_k[u] ? 1 : 0, h = r - p * a.heads;
      const int dest = h / a.send_local, l = h - dest * a.send_local;
      const int64_t row = a.send_layout == 0 ? (int64_t)(dest * 3 + p) * a.tokens + t
                                             : ((int64_t)dest * a.tokens + t) * 3 + p;
      dst_off[u] = (row * a.send_local + l) * D;
    } else {
      dst_off[u] = (int64_t)t * a.dst_stride + (int64_t)r * D;
    }
    if (TABLE && a.rotary) pos[u] = a.pos[t];  // issued first: the cos / sin loads wait only for these
  }
  i32x2 xa[U], xb[U], ca[U], sa[U], cb[U], sb[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    xa[u] = *(const i32x2 *)(a.src + src_off[u] + oa);
    xb[u] = *(const i32x2 *)(a.src + src_off[u] + ob);
  }
  i32x2 qwa{}, qwb{}, kwa{}, kwb{};
  if constexpr (NORM) {
    qwa = *(const i32x2 *)(a.qw + oa), qwb = *(const i32x2 *)(a.qw + ob);
    kwa = *(const i32x2 *)(a.kw + oa), kwb = *(const i32x2 *)(a.kw + ob);
  }
  if (a.rotary) {
    const int ph = rotates ? 4 * j : 0;  // lanes of the unrotated tail read a valid phase, unused
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (TABLE) {
        const int64_t p = min(max(pos[u], (int64_t)0), a.cs_rows - 1);
        const uint16_t *crow = a.cos + p * a.cos_stride + ph;
        ca[u] = *(const i32x2 *)crow;
        sa[u] = *(const i32x2 *)(crow + half);
      } else {
        const uint16_t *crow = a.cos + (int64_t)tok[u] * a.cos_stride + ph;
        const uint16_t *srow = a.sin + (int64_t)tok[u] * a.sin_stride + ph;
        ca[u] = *(const i32x2 *)crow;
        cb[u] = *(const i32x2 *)(crow + half);
        sa[u] = *(const i32x2 *)srow;
        sb[u] = *(const i32x2 *)(srow + half);
      }
    }
  }

  float x[U][8], ss[U];
#pragma unroll
  for (int u = 0; u < U && NORM; ++u) {
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
  float inv[U] = {1.0f, 1.0f, 1.0f, 1.0f};
  if constexpr (NORM) {
    const int q = lane & 3;
    const float sq = q == 0 ? ss[0] : q == 1 ? ss[1] : q == 2 ? ss[2] : ss[3];
    const float var = sq * (1.0f / D);  // exact: D is a power of two
    const float inv_q = __fdiv_rn(1.0f, sqrt_rn(var + a.eps));
    inv[0] = dpp<0x00>(inv_q), inv[1] = dpp<0x55>(inv_q), inv[2] = dpp<0xaa>(inv_q), inv[3] = dpp<0xff>(inv_q);
  }

  const uint32_t qw[4] = {(uint32_t)qwa[0], (uint32_t)qwa[1], (uint32_t)qwb[0], (uint32_t)qwb[1]};
  const uint32_t kw[4] = {(uint32_t)kwa[0], (uint32_t)kwa[1], (uint32_t)kwb[0], (uint32_t)kwb[1]};
#pragma unroll
  for (int u = 0; u < U; ++u) {
    uint32_t nb[4] = {(uint32_t)xa[u][0], (uint32_t)xa[u][1], (uint32_t)xb[u][0], (uint32_t)xb[u][1]};
    if constexpr (NORM) {  // normalized, packed bf16: A pieces in 0-1, B in 2-3
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t w = is_k[u] ? kw[e] : qw[e];
        nb[e] = pack_bf16((x[u][2 * e] * inv[u]) * lo_f32(w), (x[u][2 * e + 1] * inv[u]) * hi_f32(w));
      }
    }
    uint32_t out[4] = {nb[0], nb[1], nb[2], nb[3]};
    if (a.rotary) {
      // rotation pairs (A[e], B[e]): A' = A cos_A - B sin_A, B' = B cos_B + A sin_B,
      // each product and sum rounded to bf16 (rotate_half(n) = (-B, A))
      const uint32_t cwa[2] = {(uint32_t)ca[u][0], (uint32_t)ca[u][1]};
      const uint32_t swa[2] = {(uint32_t)sa[u][0], (uint32_t)sa[u][1]};
      const uint32_t cwb[2] = {(uint32_t)(TABLE ? ca : cb)[u][0], (uint32_t)(TABLE ? ca : cb)[u][1]};
      const uint32_t swb[2] = {(uint32_t)(TABLE ? sa : sb)[u][0], (uint32_t)(TABLE ? sa : sb)[u][1]};
      float oa_[4], ob_[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const auto half_of = [e](uint32_t wd) { return (e & 1) ? hi_f32(wd) : lo_f32(wd); };
        const float na = half_of(nb[e >> 1]), nbv = half_of(nb[2 + (e >> 1)]);
        const uint32_t p1 = pack_bf16(na * half_of(cwa[e >> 1]), nbv * half_of(swa[e >> 1]));  // A cos, B sin
        const uint32_t p2 = pack_bf16(nbv * half_of(cwb[e >> 1]), na * half_of(swb[e >> 1]));  // B cos, A sin
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
      uint16_t *const dst = SEND ? a.send : a.dst;
      *(i32x2 *)(dst + dst_off[u] + oa) = i32x2{(int)out[0], (int)out[1]};
      *(i32x2 *)(dst + dst_off[u] + ob) = i32x2{(int)out[2], (int)out[3]};
      if constexpr (STAGE) {
        const int i = tok[u] - a.stage_row0;
        if (is_k[u] && i >= 0 && i < a.stage_n) {
          uint16_t *row = a.kslot + (int64_t)(part_row[u] - a.heads) * a.kslot_hs + (int64_t)(a.stage_dst + i) * D;
          *(i32x2 *)(row + oa) = i32x2{(int)out[0], (int)out[1]};
          *(i32x2 *)(row + ob) = i32x2{(int)out[2], (int)out[3]};
        }
      }
    }
  }
}

int rope_rows_check(const RopeArgs &a, int head_dim, const char *what) {
  const int64_t rows = (int64_t)a.tokens * a.parts * a.heads;
  const int rows_per_block = 4 * kRopeUnroll * (64 / (head_dim / 8));
  if (rows > 0x7fffffff - rows_per_block) return set_error(TMHD_ERR_UNSUPPORTED, "%s: too many rows", what);
  return TMHD_OK;
}

int launch_rope(const RopeArgs &a, int head_dim, bool table, void *stream, const char *what, bool norm = true,
                bool stage = false, bool send = false) {
  if (int st = rope_rows_check(a, head_dim, what)) return st;
  const int64_t rows = (int64_t)a.tokens * a.parts * a.heads;
  const int rows_per_block = 4 * kRopeUnroll * (64 / (head_dim / 8));
  const dim3 grid((unsigned)((rows + rows_per_block - 1) / rows_per_block)), block(256);
  hipStream_t s = (hipStream_t)stream;
  if (send) {
    if (head_dim == 128)
      hipLaunchKernelGGL((qk_norm_rope_kernel<128, true, true, false, true>), grid, block, 0, s, a);
    else
      hipLaunchKernelGGL((qk_norm_rope_kernel<64, true, true, false, true>), grid, block, 0, s, a);
  } else if (stage) {
    if (head_dim == 128)
      hipLaunchKernelGGL((qk_norm_rope_kernel<128, true, true, true>), grid, block, 0, s, a);
    else
      hipLaunchKernelGGL((qk_norm_rope_kernel<64, true, true, true>), grid, block, 0, s, a);
  } else if (!norm) {
    if (head_dim == 128)
      hipLaunchKernelGGL((qk_norm_rope_kernel<128, false, false>), grid, block, 0, s, a);
    else
      hipLaunchKernelGGL((qk_norm_rope_kernel<64, false, false>), grid, block, 0, s, a);
  } else if (head_dim == 128 && table)
    hipLaunchKernelGGL((qk_norm_rope_kernel<128, true>), grid, block, 0, s, a);
  else if (head_dim == 128)
    hipLaunchKernelGGL((qk_norm_rope_kernel<128, false>), grid, block, 0, s, a);
  else if (table)
    hipLaunchKernelGGL((qk_norm_rope_kernel<64, true>), grid, block, 0, s, a);
  else
    hipLaunchKernelGGL((qk_norm_rope_kernel<64, false>), grid, block, 0, s, a);
  return check_launch(what);
}

bool aligned8(const void *p) { return ((uintptr_t)p % 8) == 0; }

}  // namespace
}  // namespace tmhd

namespace tmhd {
namespace {

// Arguments of the merged-projection form, validated; tokens == 0 leaves *a untouched
int qkv_rope_args(RopeArgs *a, void *qkv, int32_t tokens, int32_t heads, int32_t head_dim, int64_t row_stride,
                  const void *q_weight, const void *k_weight, const void *cos_sin, int64_t cos_sin_stride,
                  int64_t cos_sin_rows, int32_t rotary_dim, const int64_t *positions, float eps, const char *what) {
  if (head_dim != 64 && head_dim != 128)
    return set_error(TMHD_ERR_UNSUPPORTED, "%s: head_dim %d (64 or 128)", what, head_dim);
  if (tokens < 0 || heads <= 0 || row_stride < (int64_t)3 * heads * head_dim)
    return set_error(TMHD_ERR_INVALID, "%s: tokens %d heads %d row_stride %lld", what, tokens, heads,
                     (long long)row_stride);
  if (rotary_dim < 0 || rotary_dim > head_dim || rotary_dim % 8)
    return set_error(TMHD_ERR_UNSUPPORTED, "%s: rotary_dim %d (a multiple of 8 up to head_dim)", what, rotary_dim);
  if (!(eps >= 0.0f)) return set_error(TMHD_ERR_INVALID, "%s: eps must be >= 0", what);
  if (tokens == 0) return TMHD_OK;
  if (!qkv || !q_weight || !k_weight || !aligned8(qkv) || row_stride % 4 || !aligned8(q_weight) ||
      !aligned8(k_weight))
    return set_error(TMHD_ERR_INVALID, "%s: qkv rows and weights must be 8-byte aligned", what);
  if (rotary_dim && (!cos_sin || !positions || !aligned8(cos_sin) || cos_sin_stride % 4 ||
                     cos_sin_stride < rotary_dim || cos_sin_rows <= 0))
    return set_error(TMHD_ERR_INVALID, "%s: cos_sin must be 8-byte aligned rows of >= rotary_dim", what);
  *a = RopeArgs{(const uint16_t *)qkv, (uint16_t *)qkv, row_stride, row_stride, (const uint16_t *)q_weight,
                (const uint16_t *)k_weight, (const uint16_t *)cos_sin, nullptr, cos_sin_stride, 0, positions,
                cos_sin_rows, tokens, heads, 2, rotary_dim, eps, nullptr, 0, 0, 0, 0};
  return rope_rows_check(*a, head_dim, what);
}

}  // namespace
}  // namespace tmhd

extern "C" int tmhd_qkv_norm_rope(void *qkv, int32_t tokens, int32_t heads, int32_t head_dim, int64_t row_stride,
                                  const void *q_weight, const void *k_weight, const void *cos_sin,
                                  int64_t cos_sin_stride, int64_t cos_sin_rows, int32_t rotary_dim,
                                  const int64_t *positions, float eps, void *stream) {
  using namespace tmhd;
  const char *what = "tmhd_qkv_norm_rope";
  RopeArgs a{};
  if (int st = qkv_rope_args(&a, qkv, tokens, heads, head_dim, row_stride, q_weight, k_weight, cos_sin,
                             cos_sin_stride, cos_sin_rows, rotary_dim, positions, eps, what))
    return st;
  if (tokens == 0) return TMHD_OK;
  return launch_rope(a, head_dim, true, stream, what);
}

extern "C" int tmhd_qkv_norm_rope_stage(void *qkv, int32_t tokens, int32_t heads, int32_t head_dim,
                                        int64_t row_stride, const void *q_weight, const void *k_weight,
                                        const void *cos_sin, int64_t cos_sin_stride, int64_t cos_sin_rows,
                                        int32_t rotary_dim, const int64_t *positions, float eps, int32_t stage_row0,
                                        int32_t stage_n, void *k_slot, void *vt_slot, int64_t k_head_stride,
                                        int64_t vt_head_stride, int32_t vt_row_stride, int32_t dst, int32_t zero_to,
                                        void *stream) {
  using namespace tmhd;
  const char *what = "tmhd_qkv_norm_rope_stage";
  RopeArgs a{};
  if (int st = qkv_rope_args(&a, qkv, tokens, heads, head_dim, row_stride, q_weight, k_weight, cos_sin,
                             cos_sin_stride, cos_sin_rows, rotary_dim, positions, eps, what))
    return st;
  if (stage_row0 < 0 || stage_n < 0 || (int64_t)stage_row0 + stage_n > tokens)
    return set_error(TMHD_ERR_INVALID, "%s: staged rows [%d, %d) outside the %d tokens", what, stage_row0,
                     stage_row0 + stage_n, tokens);
  if ((uintptr_t)qkv % 16 || row_stride % 8)
    return set_error(TMHD_ERR_INVALID, "%s: qkv rows must be 16-byte aligned", what);
  uint16_t *const base = (uint16_t *)qkv;
  const int64_t width = (int64_t)heads * head_dim;
  // the slot arguments are those of tmhd_kv_pack over the K and V thirds (checked before any launch)
  if (int st = kv_pack(base + width, base + 2 * width, row_stride, head_dim, nullptr, stage_row0, stage_n, k_slot,
                       vt_slot, k_head_stride, vt_head_stride, vt_row_stride, dst, zero_to, heads, head_dim, stream,
                       false, true))
    return st;
  if (tokens > 0) {
    a.kslot = (uint16_t *)k_slot;
    a.kslot_hs = k_head_stride;
    a.stage_row0 = stage_row0;
    a.stage_n = stage_n;
    a.stage_dst = dst;
    if (int st = launch_rope(a, head_dim, true, stream, what, true, stage_n > 0)) return st;
  }
  return kv_pack(base + width, base + 2 * width, row_stride, head_dim, nullptr, stage_row0, stage_n, k_slot, vt_slot,
                 k_head_stride, vt_head_stride, vt_row_stride, dst, zero_to, heads, head_dim, stream, false, false);
}

extern "C" int tmhd_qk_norm_rope(const void *value, int32_t tokens, int32_t heads, int32_t head_dim,
                                 int64_t value_stride, void *out, int64_t out_stride, const void *weight,
                                 const void *cos, int64_t cos_stride, const void *sin, int64_t sin_stride,
                                 int32_t rotary_dim, float eps, void *stream) {
  using namespace tmhd;
  const char *what = "tmhd_qk_norm_rope";
  if (head_dim != 64 && head_dim != 128)
    return set_error(TMHD_ERR_UNSUPPORTED, "%s: head_dim %d (64 or 128)", what, head_dim);
  if (tokens < 0 || heads <= 0 || value_stride < (int64_t)heads * head_dim || out_stride < (int64_t)heads * head_dim)
    return set_error(TMHD_ERR_INVALID, "%s: tokens %d heads %d strides %lld / %lld", what, tokens, heads,
                     (long long)value_stride, (long long)out_stride);
  if (rotary_dim < 0 || rotary_dim > head_dim || rotary_dim % 8)
    return set_error(TMHD_ERR_UNSUPPORTED, "%s: rotary_dim %d (a multiple of 8 up to head_dim)", what, rotary_dim);
  if (!(eps >= 0.0f)) return set_error(TMHD_ERR_INVALID, "%s: eps must be >= 0", what);
  if (tokens == 0) return TMHD_OK;
  if (!value || !out || !weight || !aligned8(value) || !aligned8(out) || value_stride % 4 || out_stride % 4 ||
      !aligned8(weight))
    return set_error(TMHD_ERR_INVALID, "%s: value / out rows and the weight must be 8-byte aligned", what);
  if (rotary_dim && (!cos || !sin || !aligned8(cos) || !aligned8(sin) || cos_stride % 4 || sin_stride % 4 ||
                     cos_stride < rotary_dim || sin_stride < rotary_dim))
    return set_error(TMHD_ERR_INVALID, "%s: cos / sin must be 8-byte aligned rows of >= rotary_dim", what);
  if (out != value) {  // out-of-place: the two row sets must not overlap
    const char *v0 = (const char *)value, *o0 = (const char *)out;
    const int64_t vb = ((int64_t)(tokens - 1) * value_stride + (int64_t)heads * head_dim) * 2;
    const int64_t ob = ((int64_t)(tokens - 1) * out_stride + (int64_t)heads * head_dim) * 2;
    if (o0 < v0 + vb && v0 < o0 + ob)
      return set_error(TMHD_ERR_INVALID, "%s: out overlaps value (only exact in-place is allowed)", what);
  } else if (out_stride != value_stride) {
    return set_error(TMHD_ERR_INVALID, "%s: in place needs equal strides", what);
  }
  RopeArgs a{(const uint16_t *)value, (uint16_t *)out, value_stride, out_stride, (const uint16_t *)weight,
             (const uint16_t *)weight, (const uint16_t *)cos, (const uint16_t *)sin, cos_stride, sin_stride,
             nullptr, 0, tokens, heads, 1, rotary_dim, eps};
  return launch_rope(a, head_dim, false, stream, what);
}

extern "C" int tmhd_apply_rope(const void *value, int32_t tokens, int32_t heads, int32_t head_dim,
                               int64_t value_stride, void *out, int64_t out_stride, const void *cos,
                               int64_t cos_stride, const void *sin, int64_t sin_stride, int32_t rotary_dim,
                               void *stream) {
  using namespace tmhd;
  const char *what = "tmhd_apply_rope";
  if (head_dim != 64 && head_dim != 128)
    return set_error(TMHD_ERR_UNSUPPORTED, "%s: head_dim %d (64 or 128)", what, head_dim);
  if (tokens < 0 || heads <= 0 || value_stride < (int64_t)heads * head_dim || out_stride < (int64_t)heads * head_dim)
    return set_error(TMHD_ERR_INVALID, "%s: tokens %d heads %d strides %lld / %lld", what, tokens, heads,
                     (long long)value_stride, (long long)out_stride);
  if (rotary_dim < 0 || rotary_dim > head_dim || rotary_dim % 8)
    return set_error(TMHD_ERR_UNSUPPORTED, "%s: rotary_dim %d (a multiple of 8 up to head_dim)", what, rotary_dim);
  if (tokens == 0) return TMHD_OK;
  if (!value || !out || !aligned8(value) || !aligned8(out) || value_stride % 4 || out_stride % 4)
    return set_error(TMHD_ERR_INVALID, "%s: value / out rows must be 8-byte aligned", what);
  if (rotary_dim && (!cos || !sin || !aligned8(cos) || !aligned8(sin) || cos_stride % 4 || sin_stride % 4 ||
                     cos_stride < rotary_dim || sin_stride < rotary_dim))
    return set_error(TMHD_ERR_INVALID, "%s: cos / sin must be 8-byte aligned rows of >= rotary_dim", what);
  if (out != value) {
    const char *v0 = (const char *)value, *o0 = (const char *)out;
    const int64_t vb = ((int64_t)(tokens - 1) * value_stride + (int64_t)heads * head_dim) * 2;
    const int64_t ob = ((int64_t)(tokens - 1) * out_stride + (int64_t)heads * head_dim) * 2;
    if (o0 < v0 + vb && v0 < o0 + ob)
      return set_error(TMHD_ERR_INVALID, "%s: out overlaps value (only exact in-place is allowed)", what);
  } else if (out_stride != value_stride) {
    return set_error(TMHD_ERR_INVALID, "%s: in place needs equal strides", what);
  }
  RopeArgs a{(const uint16_t *)value, (uint16_t *)out, value_stride, out_stride, nullptr, nullptr,
             (const uint16_t *)cos, (const uint16_t *)sin, cos_stride, sin_stride, nullptr, 0, tokens, heads, 1,
             rotary_dim, 0.0f};
  return launch_rope(a, head_dim, false, stream, what, false);
}

extern "C" int tmhd_ulysses_qkv_norm_rope_send(const void *qkv, int64_t row_stride, int32_t tokens, int32_t heads,
                                              int32_t head_dim, const void *q_weight, const void *k_weight,
                                              const void *cos_sin, int64_t cos_sin_stride, int64_t cos_sin_rows,
                                              int32_t rotary_dim, const int64_t *positions, float eps,
                                              int32_t world, int32_t layout, void *out, void *stream) {
  using namespace tmhd;
  const char *what = "tmhd_ulysses_qkv_norm_rope_send";
  RopeArgs a{};
  if (int st = qkv_rope_args(&a, const_cast<void *>(qkv), tokens, heads, head_dim, row_stride, q_weight, k_weight,
                             cos_sin, cos_sin_stride, cos_sin_rows, rotary_dim, positions, eps, what))
    return st;
  // V rows and the zero padding heads come from the plain send (checked before any launch)
  if (int st = ulysses_send(qkv, row_stride, tokens, heads, head_dim, world, layout, out, 4, stream, true)) return st;
  if (tokens == 0) return TMHD_OK;
  a.dst = nullptr;
  a.send = (uint16_t *)out;
  a.send_local = (heads + world - 1) / world;
  a.send_layout = layout;
  if (int st = launch_rope(a, head_dim, true, stream, what, true, false, true)) return st;
  return ulysses_send(qkv, row_stride, tokens, heads, head_dim, world, layout, out, 4, stream, false);
}
