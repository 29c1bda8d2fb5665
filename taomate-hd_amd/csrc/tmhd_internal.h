// Internal helpers shared by the libtmhd HIP sources (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tmhd.h"

namespace tmhd {

using i32x2 = int __attribute__((ext_vector_type(2)));
using i32x4 = int __attribute__((ext_vector_type(4)));
using i32x16 = int __attribute__((ext_vector_type(16)));
using f32x4 = float __attribute__((ext_vector_type(4)));
using f32x16 = float __attribute__((ext_vector_type(16)));
using bf16x2 = __bf16 __attribute__((ext_vector_type(2)));
using bf16x8 = __bf16 __attribute__((ext_vector_type(8)));

// Records a formatted message for tmhd_last_error() and returns `status`.
int set_error(int status, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
// Checks hipGetLastError() after a launch; records it on failure.
int check_launch(const char *what);
// Compute units of the current device (cached per device; 0 if unknown).
int device_cus();
// tmhd_kv_pack with two switches: with_k false leaves the key rows of the
// data positions to the caller (zero positions are still cleared);
// check_only validates the arguments and launches nothing.
int kv_pack(const void *k, const void *v, int64_t token_stride, int64_t head_stride, const int32_t *rows,
            int32_t row0, int32_t n, void *k_slot, void *vt_slot, int64_t k_head_stride, int64_t vt_head_stride,
            int32_t vt_row_stride, int32_t dst, int32_t zero_to, int32_t heads, int32_t head_dim, void *stream,
            bool with_k, bool check_only);

// The Ulysses send layout of a merged QKV projection (tmhd_ulysses_qkv_send)
// for the parts whose bit is set in copy_parts (padded heads are always
// zeroed); check_only validates the arguments and launches nothing.
int ulysses_send(const void *qkv, int64_t row_stride, int32_t tokens, int32_t heads, int32_t head_dim,
                 int32_t world, int32_t layout, void *out, int32_t copy_parts, void *stream, bool check_only);

// bf16 bits -> fp32 (exact).
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// fp32 -> bf16 bits, round to nearest even (NaN kept quiet).
__host__ __device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
#if defined(__HIP_DEVICE_COMPILE__)
  uint32_t u = __float_as_uint(f);
#else
  uint32_t u;
  __builtin_memcpy(&u, &f, 4);
#endif
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// Two floats -> packed bf16 (lo in bits 0-15) with gfx950's conversion,
// round to nearest even.
__device__ __forceinline__ uint32_t pack_bf16_rne(float lo, float hi) {
  using f32x2_t = float __attribute__((ext_vector_type(2)));
  const f32x2_t f = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2));
}

// SwiGLU of one packed bf16 pair of gates and ups: R(R(g * sigmoid(g)) * u),
// sigmoid(g) = 1 / (1 + e^-g) in 12 instructions: e^-g = 2^t (1 + lo) with
// t = -g * log2(e) rounded and lo its rounding residual (log2(e) split into a
// float head and a tail, the residual of the head's product taken exactly with
// an FMA: Cody and Waite's argument reduction), 2^t from v_exp_f32, then the
// hardware reciprocal refined by one Newton step.  For every bf16 gate above
// -87.5 the SwiGLU output equals that of the correctly rounded division of
// 1 by 1 + expf(-g); below it both give outputs under 1e-36 in magnitude
// (this form returns 0 there: the reciprocal flushes denormals).  The input is
// clamped to [-128, 128] (NaN to -128), so that infinities and NaN never meet
// the correction: +inf gives 1, -inf and NaN give 0, and g * sigmoid(g) is then
// inf, NaN, NaN as with the division.
__device__ __forceinline__ float sigmoid_f32(float g) {
#pragma clang fp contract(off)
  constexpr float kLog2eHi = 1.44269502162933349609375f;                      // log2(e) rounded to float
  constexpr float kLog2eLoLn2 = 1.925963033500011e-08f * 0.6931471805599453f;  // (log2(e) - head) * ln 2
  constexpr float kLn2 = 0.6931471805599453f;
  const float gc = fminf(fmaxf(g, -128.0f), 128.0f);
  const float t = gc * -kLog2eHi;
  const float r1 = __builtin_fmaf(gc, -kLog2eHi, -t);            // exact: -gc * head - t
  const float lo = __builtin_fmaf(r1, kLn2, gc * -kLog2eLoLn2);  // (-gc log2(e) - t) ln 2
  float e = __builtin_amdgcn_exp2f(t);
  e = __builtin_fmaf(e, lo, e);  // 2^t e^lo to first order
  const float d = 1.0f + e;
  const float r = __builtin_amdgcn_rcpf(d);
  return fmaxf(__builtin_fmaf(__builtin_fmaf(-d, r, 1.0f), r, r), 0.0f);  // d = inf: NaN -> 0
}

// silu(gate) * up of two bf16 pairs, rounded as the reference rounds it
// (shared by the SwiGLU kernel and the GEMM's fused SwiGLU epilogue, so both
// give the same bits).
__device__ __forceinline__ uint32_t swiglu_pair(uint32_t g, uint32_t u) {
#pragma clang fp contract(off)
  const float g0 = __uint_as_float(g << 16), g1 = __uint_as_float(g & 0xffff0000u);
  const float s0 = sigmoid_f32(g0), s1 = sigmoid_f32(g1);
  const uint32_t act = pack_bf16_rne(g0 * s0, g1 * s1);
  return pack_bf16_rne(__uint_as_float(act << 16) * __uint_as_float(u << 16),
                       __uint_as_float(act & 0xffff0000u) * __uint_as_float(u & 0xffff0000u));
}

// Correctly rounded square root of x >= 0 (+inf and NaN pass through).  The
// hardware square root is within one ulp; the Tuckerman rounding test picks
// between it and its two neighbours s- < s < s+: sqrt(x) lies below the
// midpoint (s- + s) / 2 exactly when x - s- * s <= 0, and above (s + s+) / 2
// exactly when x - s * s+ > 0.  Both residuals are whole multiples of the
// squared spacing g^2 of the neighbours, while a midpoint's own residual is
// g^2 / 4, so the signs decide; each residual is one fused multiply-add,
// whose rounding keeps the sign.  Inputs below 2^-96 are scaled by 2^64 (and
// the root by 2^-32, both exact) so that g^2 stays above the subnormal range.
__device__ __forceinline__ float sqrt_rn(float x) {
  const bool tiny = x < 0x1p-96f;
  const float xs = tiny ? x * 0x1p64f : x;
  float s = __builtin_amdgcn_sqrtf(xs);
  if (s > 0.0f && s < __builtin_inff()) {
    const float sd = __uint_as_float(__float_as_uint(s) - 1u);
    const float su = __uint_as_float(__float_as_uint(s) + 1u);
    if (__builtin_fmaf(-sd, s, xs) <= 0.0f)
      s = sd;
    else if (__builtin_fmaf(-s, su, xs) > 0.0f)
      s = su;
  }
  return tiny ? s * 0x1p-32f : s;
}

// Slot position of token t inside the transposed value rows: swap the middle
// two 4-token chunks of each 16-token group (an involution).
__host__ __device__ __forceinline__ int vt_position(int t) {
  const int c = (t >> 2) & 3;
  const int pc = (c == 1) ? 2 : (c == 2) ? 1 : c;
  return (t & ~15) | (pc << 2) | (t & 3);
}

// Saturating round-to-nearest-even fp32 -> int8.
__device__ __forceinline__ int quant_rne_sat(float x) {
  float r = __builtin_rintf(x);
  r = fminf(fmaxf(r, -128.0f), 127.0f);
  return (int)r;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  return v;
}

constexpr int kMaxSeg = TMHD_MAX_SEGMENTS;

}  // namespace tmhd
