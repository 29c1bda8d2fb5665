// Selective W8A8 projection for gfx950: per-token dynamic INT8 activation
// quantization, per-output-channel INT8 weight quantization and the scaled
// INT8 GEMM with a bf16 epilogue (reference call sites:
// src/taomate_hd/inference/w8a8.py:67-73, 117-145, 175-179).
#include <math.h>

#include <type_traits>

#include <algorithm>

#include "tmhd_internal.h"

namespace tmhd {
namespace {

// ---------------------------------------------------------------------------
// Row quantization, one wave per row.  CH = 8-element chunks held per lane
// (one pass, row kept in registers); CH = 0 streams the row twice.
// WEIGHT selects the weight formula of _quantize_cutlass_w8a8_weight:
//   scale = max(amax / 127, 1e-12), q = clamp(rint(w / scale), -127, 127)
// otherwise the activation formula:
//   scale = amax / 127, q = sat_int8(rint(x * (127 / amax))), amax = 0 -> 0.
template <int CH, bool WEIGHT>
__global__ void __launch_bounds__(256) row_quant_kernel(int8_t *__restrict__ q, float *__restrict__ scale,
                                                        const uint16_t *__restrict__ x, int32_t rows, int32_t cols,
                                                        int64_t xs) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int nch = cols >> 3;
  const uint16_t *xr = x + (int64_t)row * xs;
  int8_t *qr = q + (int64_t)row * cols;
  float amax = 0.0f;
  i32x4 raw[CH > 0 ? CH : 1];
  if constexpr (CH > 0) {
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const int c = lane + 64 * j;
      raw[j] = c < nch ? *(const i32x4 *)(xr + c * 8) : i32x4{0, 0, 0, 0};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t w = (uint32_t)raw[j][e];
        amax = fmaxf(amax, fmaxf(fabsf(bf16_bits_to_f32(w & 0xffffu)), fabsf(bf16_bits_to_f32(w >> 16))));
      }
    }
  } else {
    for (int c = lane; c < nch; c += 64) {
      const i32x4 r = *(const i32x4 *)(xr + c * 8);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t w = (uint32_t)r[e];
        amax = fmaxf(amax, fmaxf(fabsf(bf16_bits_to_f32(w & 0xffffu)), fabsf(bf16_bits_to_f32(w >> 16))));
      }
    }
  }
  amax = wave_max(amax);
  float sc, inv;
  if constexpr (WEIGHT) {
    sc = fmaxf(__fdiv_rn(amax, 127.0f), 1e-12f);
    inv = 0.0f;
  } else {
    sc = __fdiv_rn(amax, 127.0f);
    inv = amax > 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
  }
  if (lane == 0) scale[row] = sc;
  auto qv = [&](float v) -> uint32_t {
    int r;
    if constexpr (WEIGHT) {
      r = (int)fminf(fmaxf(__builtin_rintf(__fdiv_rn(v, sc)), -127.0f), 127.0f);
    } else {
      r = quant_rne_sat(v * inv);
    }
    return (uint32_t)r & 0xffu;
  };
  auto emit = [&](int c, i32x4 r) {
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const uint32_t w0 = (uint32_t)r[e], w1 = (uint32_t)r[e + 2];
      lo |= qv(bf16_bits_to_f32(w0 & 0xffffu)) << (16 * e);
      lo |= qv(bf16_bits_to_f32(w0 >> 16)) << (16 * e + 8);
      hi |= qv(bf16_bits_to_f32(w1 & 0xffffu)) << (16 * e);
      hi |= qv(bf16_bits_to_f32(w1 >> 16)) << (16 * e + 8);
    }
    *(i32x2 *)(qr + c * 8) = i32x2{(int)lo, (int)hi};
  };
  if constexpr (CH > 0) {
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const int c = lane + 64 * j;
      if (c < nch) emit(c, raw[j]);
    }
  } else {
    for (int c = lane; c < nch; c += 64) emit(c, *(const i32x4 *)(xr + c * 8));
  }
}

template <bool WEIGHT>
int launch_row_quant(int8_t *q, float *scale, const void *x, int32_t rows, int32_t cols, int64_t xs, void *stream,
                     const char *what) {
  if (rows < 0 || cols <= 0 || cols % 8) return set_error(TMHD_ERR_UNSUPPORTED, "%s: cols %d must be a positive multiple of 8", what, cols);
  if (xs < cols || xs % 8) return set_error(TMHD_ERR_INVALID, "%s: row stride %lld", what, (long long)xs);
  if (!q || !scale || !x || ((uintptr_t)x % 16) || ((uintptr_t)q % 8))
    return set_error(TMHD_ERR_INVALID, "%s: null or misaligned pointer", what);
  if (rows == 0) return TMHD_OK;
  const int need = (cols / 8 + 63) / 64;
  const dim3 grid((rows + 3) / 4), block(256);
  hipStream_t s = (hipStream_t)stream;
  const uint16_t *xp = (const uint16_t *)x;
  if (need <= 1)
    hipLaunchKernelGGL((row_quant_kernel<1, WEIGHT>), grid, block, 0, s, q, scale, xp, rows, cols, xs);
  else if (need <= 2)
    hipLaunchKernelGGL((row_quant_kernel<2, WEIGHT>), grid, block, 0, s, q, scale, xp, rows, cols, xs);
  else if (need <= 4)
    hipLaunchKernelGGL((row_quant_kernel<4, WEIGHT>), grid, block, 0, s, q, scale, xp, rows, cols, xs);
  else if (need <= 8)
    hipLaunchKernelGGL((row_quant_kernel<8, WEIGHT>), grid, block, 0, s, q, scale, xp, rows, cols, xs);
  else if (need <= 10)
    hipLaunchKernelGGL((row_quant_kernel<10, WEIGHT>), grid, block, 0, s, q, scale, xp, rows, cols, xs);
  else if (need <= 16)
    hipLaunchKernelGGL((row_quant_kernel<16, WEIGHT>), grid, block, 0, s, q, scale, xp, rows, cols, xs);
  else
    hipLaunchKernelGGL((row_quant_kernel<0, WEIGHT>), grid, block, 0, s, q, scale, xp, rows, cols, xs);
  return check_launch(what);
}

// ---------------------------------------------------------------------------
// INT8 GEMM: C[m][n] = sum_k A[m][k] * B[n][k] with v_mfma_i32_32x32x32_i8.
// Workgroup tile 256 (m) x 256 (n), 8 waves as 4 (m) x 2 (n), each wave
// 64 x 128 (128 int32 accumulators per lane, two waves per SIMD).  The MFMA
// computes the transposed block D[n][m] = B-rows x A-rows, so a lane holds
// four consecutive n of one m and writes 4 bf16 (8 bytes) at a time.
// k-tiles of 64 stream through a 3-deep LDS ring filled by
// global_load_lds_dwordx4; the loop is unrolled by the ring depth so every
// LDS address is a compile-time slot.  LDS rows are 64 bytes (4 chunks);
// chunk c of row r sits at c ^ ((r >> 2) & 3), so the 16 lanes of one
// ds_read_b128 phase hit 16 distinct 16-byte bank groups.
constexpr int GBM = 256, GBN = 256, GBK = 64, GWAVES = 8, GRING = 3;
constexpr int GSTAGE = (GBM + GBN) * GBK;  // bytes per ring slot

struct GArgs {
  const int8_t *a;
  const int8_t *b;
  void *out;
  const float *as;
  const float *bs;
  const uint16_t *bias;
  int32_t m, n, k;
  int64_t lda, ldb, ldo;
  int32_t tm_count, tn_count;
  int32_t vec_ok;  // bs 16-byte and bias 8-byte aligned: vector loads of 4 columns
  int32_t st_ok;   // bf16 output rows 16-byte aligned: staged 16-byte stores
  // K split of the last, partial round (one-wave-per-SIMD kernel): tiles
  // [0, full) are whole; block t * nsplit + p of the split launch is k-range p
  // of tile full + t, whose int32 partial tile goes to ws (merged afterwards)
  int32_t full, nsplit;
  int32_t *ws;
};

// Tile (tm, tn) of logical tile L: 4 row tiles share each column sweep (L2
// reuse).  Measured on the 12,252-row projections: 4 beats 2, 6, 8, 16 and 48
// (about 3% against 8 on 5,120 x 13,824, 1.4% on the 5,376 x 28,672 FC1).
__device__ __forceinline__ void grouped_tile(int L, int tm_count, int tn_count, int &tm, int &tn) {
  constexpr int GROUP = 4;
  const int per_group = GROUP * tn_count;
  const int first_tm = (L / per_group) * GROUP;
  const int gsize = min(tm_count - first_tm, GROUP);
  tm = first_tm + (L % per_group) % gsize;
  tn = (L % per_group) / gsize;
}

// The dequantisation epilogue of one accumulator, the same operations in the
// same order as the GEMM's own epilogue: (float)acc * b_scale * a_scale (+ bias);
// rounded to bf16 by bf16_quad.
__device__ __forceinline__ float dequant_f32(int32_t acc, float bs, float as, bool has_bias, uint32_t bias_bits) {
#pragma clang fp contract(off)
  float t = (float)acc;
  t = t * bs;
  t = t * as;
  if (has_bias) t = t + bf16_bits_to_f32(bias_bits);
  return t;
}

// Four floats -> bf16 with gfx950's conversion (round to nearest even, two
// per instruction; the same bits as f32_to_bf16_bits for every non-NaN value).
__device__ __forceinline__ void bf16_quad(const float (&t)[4], uint16_t (&v)[4]) {
  const uint32_t p01 = pack_bf16_rne(t[0], t[1]), p23 = pack_bf16_rne(t[2], t[3]);
  v[0] = (uint16_t)p01, v[1] = (uint16_t)(p01 >> 16), v[2] = (uint16_t)p23, v[3] = (uint16_t)(p23 >> 16);
}

__device__ __forceinline__ int xcd_logical_id(int b, int G) {
  const int xcd = b & 7, pos = b >> 3, per = G >> 3, rem = G & 7;
  return xcd < rem ? xcd * (per + 1) + pos : rem * (per + 1) + (xcd - rem) * per + pos;
}

__device__ __forceinline__ void load_lds16(const void *gptr, void *lds) {
  __builtin_amdgcn_global_load_lds(gptr, (__attribute__((address_space(3))) void *)lds, 16, 0, 0);
}

template <bool RAW>
__global__ void __launch_bounds__(GWAVES * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
gemm_i8_kernel(const GArgs ga) {
#pragma clang fp contract(off)
  __shared__ __attribute__((aligned(1024))) char smem[GRING][GSTAGE];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, lr = lane & 31, g = lane >> 5;
  const int wm = w >> 1, wn = w & 1;  // wave tile: a rows [wm*64, +64), b rows [wn*128, +128)
  // grouped tile order: 8 row tiles share each column sweep (L2 reuse)
  const int L = xcd_logical_id(blockIdx.x, gridDim.x);
  constexpr int GROUP = 8;
  const int per_group = GROUP * ga.tn_count;
  const int grp = L / per_group;
  const int first_tm = grp * GROUP;
  const int gsize = min(ga.tm_count - first_tm, GROUP);
  const int tm = first_tm + (L % per_group) % gsize;
  const int tn = (L % per_group) / gsize;
  const int m0 = tm * GBM, n0 = tn * GBN;

  // loads: the a tile (256 rows x 64 B) and b tile are 16 wave loads each; wave w
  // loads blocks w and w + 8 of each (16 rows of 64 B per 1 KiB block)
  const int8_t *asrc[2];
  const int8_t *bsrc[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int blk = w + i * GWAVES, row = blk * 16 + (lane >> 2), ch = (lane & 3) ^ ((row >> 2) & 3);
    asrc[i] = ga.a + (int64_t)min(m0 + row, ga.m - 1) * ga.lda + ch * 16;
    bsrc[i] = ga.b + (int64_t)min(n0 + row, ga.n - 1) * ga.ldb + ch * 16;
  }
  auto issue = [&](int kt, char *slot) {
    const int k0 = kt * GBK;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      load_lds16(asrc[i] + k0, slot + (w + i * GWAVES) * 1024);
      load_lds16(bsrc[i] + k0, slot + GBM * GBK + (w + i * GWAVES) * 1024);
    }
  };
  // per-lane LDS byte offsets of the MFMA operands (k-step 0; k-step 1 flips chunk bit 1)
  const int arow0 = wm * 64 + lr, brow0 = wn * 128 + lr;
  const int aoff = arow0 * 64 + ((g ^ ((arow0 >> 2) & 3)) * 16);
  const int boff = GBM * GBK + brow0 * 64 + ((g ^ ((brow0 >> 2) & 3)) * 16);

  i32x16 acc[4][2];  // [n block][m block], D[n][m]
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

  auto compute = [&](const char *slot) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      // keep each k-step's operand reads next to its MFMAs (bounds register pressure)
      __builtin_amdgcn_sched_barrier(0);
      // chunk (2*ks + g) ^ sw == (g ^ sw) ^ (2*ks): k-step 1 toggles byte offset bit 5
      i32x4 av[2], bv[4];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int off = aoff + j * 32 * 64;
        av[j] = *(const i32x4 *)(slot + (off ^ (ks * 32)));
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int off = boff + i * 32 * 64;
        bv[i] = *(const i32x4 *)(slot + (off ^ (ks * 32)));
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bv[i], av[j], acc[i][j], 0, 0, 0);
    }
  };

  const int nk = ga.k / GBK;
  issue(0, smem[0]);
  if (nk > 1) issue(1, smem[1]);
  // iteration kt: stage kt ready (wait), everyone past iteration kt-1 (barrier),
  // refill the slot freed by kt-1 with stage kt+2, compute stage kt
  auto step = [&](int kt, char *cur, char *fill) {
    if (kt + 1 < nk)
      __builtin_amdgcn_s_waitcnt(0x0f74);  // vmcnt(4): stage kt+1's 4 loads may stay in flight
    else
      __builtin_amdgcn_s_waitcnt(0x0f70);
    __syncthreads();
    if (kt + 2 < nk) issue(kt + 2, fill);
    compute(cur);
    __builtin_amdgcn_sched_barrier(0);
  };
  // one exit only: the accumulators keep their registers across the unrolled steps
  int kt = 0;
  for (; kt + GRING <= nk; kt += GRING) {
    step(kt, smem[0], smem[2]);
    step(kt + 1, smem[1], smem[0]);
    step(kt + 2, smem[2], smem[1]);
  }
  if (kt < nk) step(kt, smem[0], smem[2]);
  if (kt + 1 < nk) step(kt + 1, smem[1], smem[0]);

  // epilogue: lane holds m = m-block base + lr; n = n-block base + 8u + 4g + (0..3)
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int m = m0 + wm * 64 + j * 32 + lr;
    if (m >= ga.m) continue;
    const float asm_ = RAW ? 0.0f : ga.as[m];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int n = n0 + wn * 128 + i * 32 + 8 * u + 4 * g;
        if (n >= ga.n) continue;
        if constexpr (RAW) {
          int32_t *op = (int32_t *)ga.out + (int64_t)m * ga.ldo + n;
          if (n + 3 < ga.n) {
            *(i32x4 *)op = i32x4{acc[i][j][4 * u], acc[i][j][4 * u + 1], acc[i][j][4 * u + 2], acc[i][j][4 * u + 3]};
          } else {
            for (int e = 0; e < 4 && n + e < ga.n; ++e) op[e] = acc[i][j][4 * u + e];
          }
        } else {
          uint16_t *op = (uint16_t *)ga.out + (int64_t)m * ga.ldo + n;
          uint16_t vals[4];
          float tv[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int nn = min(n + e, ga.n - 1);
            float t = (float)acc[i][j][4 * u + e];
            t = t * ga.bs[nn];
            t = t * asm_;
            if (ga.bias) t = t + bf16_bits_to_f32(ga.bias[nn]);
            tv[e] = t;
          }
          bf16_quad(tv, vals);
          if (n + 3 < ga.n) {
            *(i32x2 *)op = i32x2{(int)((uint32_t)vals[0] | ((uint32_t)vals[1] << 16)),
                                 (int)((uint32_t)vals[2] | ((uint32_t)vals[3] << 16))};
          } else {
            for (int e = 0; e < 4 && n + e < ga.n; ++e) op[e] = vals[e];
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// INT8 GEMM, one wave per SIMD: workgroup tile 256 (m) x 256 (n), 4 waves as
// 2 (m) x 2 (n), each wave 128 x 128 (64 blocks of 16 x 16, 256 int32
// accumulators per lane in AGPRs).  A 64-byte k-step reads 8 A and 8 B
// operands (ds_read_b128) for 64 v_mfma_i32_16x16x64_i8; the next k-step's
// reads are issued under the current one's MFMAs, one read per 4 MFMAs.
// The card is power-limited under this loop, and the 16 x 16 shape moves
// half the accumulator bytes per multiply-accumulate of the 32 x 32 one: on
// random int8 operands an MFMA-only stream settles at 4,085 TOPS against
// 3,430 for v_mfma_i32_32x32x32_i8 (1.96 against 1.63 GHz), and this kernel
// runs 7% faster with it than with the 32 x 32 shape at the same tiling.
// k moves in blocks of 128 bytes (two k-steps).  A block's operands sit in
// two ring units, one per 128-row half of the tile (rows of 128 bytes: whole
// cache lines, so each 1 KiB global_load_lds_dwordx4 touches 8 lines and
// every line is fetched once -- against 16 half-used lines per load with
// 64-byte rows, which measured 9% slower on the 12,252 x 5,120 x 13,824
// projection and the 12,252 x 5,376 x 28,672 FC1, with the load path's
// address unit stalled by the L1 27% of the time).  Units cycle through a
// 5-deep ring (5 x 32 KiB, all of the CU's LDS), 96 to 224 bytes of k ahead
// of their first read; a 3-deep ring of 64-byte stages (about 128 bytes
// ahead) was as fast as the 5-deep one, so the shorter lookahead costs
// nothing.
constexpr int HBM_ = 256, HBN = 256, HKD = 128, HWAVES = 4, HRING = 5;
constexpr int HUNIT = 2 * 128 * HKD;  // bytes of one ring unit: 128 rows of A, then of B

__device__ __forceinline__ void hload_lds16(const void *base, uint32_t off, uint32_t lds_addr) {
  asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "{m0}"(lds_addr) : "memory");
}

// GLU: the weight rows come in blocks of 256 (128 gate rows, then the 128
// matching up rows), so tile column c < 128 and c + 128 are the gate and up of
// one output column; the epilogue writes SwiGLU(gate, up) of the bf16
// projection, out[m][n0 / 2 + c] (ldo counts its columns).
template <bool RAW, bool SPLIT, bool GLU = false>
__global__ void __launch_bounds__(HWAVES * 64) __attribute__((amdgpu_waves_per_eu(1, 1)))
gemm_i8_wave128_kernel(const GArgs ga) {
#pragma clang fp contract(off)
  __shared__ __attribute__((aligned(1024))) char smem[HRING * HUNIT];
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char *)smem;
  const int tid = threadIdx.x, lane = tid & 63, lr = lane & 31, g = lane >> 5;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = w >> 1, wn = w & 1;  // wave tile: a rows [wm*128, +128), b rows [wn*128, +128)
  // whole tile, or (SPLIT) k-block range [d_begin, d_end) of a tile of the split round
  const int nd_all = ga.k / HKD;
  int L, part = 0, d_begin = 0, d_end = nd_all;
  if constexpr (SPLIT) {
    const int item = blockIdx.x / ga.nsplit;
    part = blockIdx.x - item * ga.nsplit;
    L = ga.full + item;
    d_begin = nd_all * part / ga.nsplit;
    d_end = nd_all * (part + 1) / ga.nsplit;
  } else {
    L = xcd_logical_id(blockIdx.x, gridDim.x);
  }
  int tm, tn;
  grouped_tile(L, ga.tm_count, ga.tn_count, tm, tn);
  const int m0 = tm * HBM_, n0 = tn * HBN;
  const int8_t *abase = ga.a + (int64_t)d_begin * HKD, *bbase = ga.b + (int64_t)d_begin * HKD;
  const int nd = d_end - d_begin;  // >= 1

  // Unit u = (k block u / 2, row half u % 2): rows [128 h, 128 h + 128) of the
  // A and the B tile over 128 bytes of k, in ring slot u % HRING (16 KiB of A,
  // then 16 KiB of B, rows of 128 bytes).  Chunk c of row r sits at
  // c ^ ((r >> 1) & 7), which keeps the operand reads free of bank conflicts
  // (their pattern is stated with the read offsets below).
  // Loads: a unit is 16 blocks of 1 KiB (8 rows x 128 bytes: whole cache
  // lines) per operand; wave w loads blocks w, w + 4, w + 8, w + 12 of each.
  // Lane: row 8 blk + lane / 8, physical chunk lane % 8, logical chunk
  // (lane % 8) ^ ((row >> 1) & 7) -- the same for all of the wave's blocks,
  // whose parity is w's.
  const int lch = (lane & 7) ^ ((4 * (w & 1) + (lane >> 4)) & 7);
  uint32_t aoff[2][4], boff[2][4];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = h * 128 + (w + 4 * i) * 8 + (lane >> 3);
      aoff[h][i] = (uint32_t)((int64_t)min(m0 + row, ga.m - 1) * ga.lda) + lch * 16;
      boff[h][i] = (uint32_t)((int64_t)min(n0 + row, ga.n - 1) * ga.ldb) + lch * 16;
    }
  // load n (0..7) of unit u: n < 4 A block w + 4 n, else B block w + 4 (n - 4).
  // Units past the last k block repeat it (in-bounds bytes into a slot nobody reads).
  auto load_one = [&](int u, int n) {
    const int j = min(u >> 1, nd - 1), h = u & 1, i = n & 3;
    const uint32_t dst = lds0 + (uint32_t)((u % HRING) * HUNIT) + (w + 4 * i) * 1024;
    if (n < 4)
      hload_lds16(abase + (int64_t)j * HKD, aoff[h][i], dst);
    else
      hload_lds16(bbase + (int64_t)j * HKD, boff[h][i], dst + HUNIT / 2);
  };
  // operand read offsets within a unit's operand part, k-step q (0..1) of the
  // block: 16x16x64 operand lane (i, g4) = lane % 16, lane / 16 holds 16 bytes
  // of row i (+ 16 per block) at logical chunk 4 q + g4.  A 16-byte read is
  // served for 32 consecutive lanes at a time from 128 4-byte banks: rows
  // i = 0..15 at two chunks, whose physical chunks under the swizzle fill all
  // 32 16-byte bank groups of the 4 row classes (row stride 128 bytes).
  const int li = lane & 15, lg = lane >> 4;
  uint32_t rdq[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) rdq[q] = (uint32_t)(li * HKD + (((4 * q + lg) ^ ((li >> 1) & 7)) * 16));
  auto rd = [&](uint32_t off) { return *(const i32x4 *)(smem + off); };

  i32x4 acc[8][8];  // [n block][m block], D[n][m]: lane (j, g4) holds n = 16 nb + 4 g4 + (0..3), m = 16 mb + j
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = i32x4{0, 0, 0, 0};

  // prologue: units 0..3 in flight; units 0 and 1 (k block 0) landed
#pragma unroll
  for (int u = 0; u < 4; ++u)
#pragma unroll
    for (int n = 0; n < 8; ++n) load_one(u, n);
  __builtin_amdgcn_s_waitcnt(0x0f70 | 16);  // vmcnt(16): units 2, 3 may stay in flight
  __syncthreads();
  i32x4 cur[16], nxt[16];
  // operand r of k-step q of k block d (ring position dm = d % HRING): r < 8
  // A block r from unit 2 d + wm, else B block r - 8 from unit 2 d + wn
  auto read_op = [&](int dm, int q, int r) -> i32x4 {
    if (r < 8) return rd((uint32_t)(((2 * dm + wm) % HRING) * HUNIT) + rdq[q] + r * 16 * HKD);
    return rd((uint32_t)(((2 * dm + wn) % HRING) * HUNIT + HUNIT / 2) + rdq[q] + (r - 8) * 16 * HKD);
  };
#pragma unroll
  for (int r = 0; r < 16; ++r) cur[r] = read_op(0, 0, r);

  // Epilogue operands: the column scales and bias of n-block i (the lane's
  // columns n = n0 + wn 128 + 16 i + 4 g4 + (0..3)) and the row scales of the
  // lane's 8 m-blocks.  The staged epilogue loads n-block i + 1's while it
  // converts n-block i; a tile that lies inside the matrix in n loads n-block
  // 0's and the row scales during its last k block, so that their latency
  // hides under its MFMAs.
  const bool early = !RAW && !SPLIT && ga.vec_ok && n0 + HBN <= ga.n;
  float asv[8];
  f32x4 bsc, bsn;
  i32x2 bic, bin;
  auto load_row_scales = [&]() {
#pragma unroll
    for (int j = 0; j < 8; ++j) asv[j] = ga.as[min(m0 + wm * 128 + j * 16 + li, ga.m - 1)];
  };
  // VEC: the whole tile lies inside the matrix in n and the scales and bias
  // are aligned for vector loads (`early`)
  auto load_cols = [&](auto vec_c, int i, f32x4 &bs, i32x2 &bi) {
    constexpr bool VEC = decltype(vec_c)::value;
    const int n = n0 + wn * 128 + i * 16 + 4 * lg;
    if (VEC || (ga.vec_ok && n + 3 < ga.n)) {
      bs = *(const f32x4 *)(ga.bs + n);
      bi = ga.bias ? *(const i32x2 *)(ga.bias + n) : i32x2{0, 0};
    } else {
      uint16_t bb[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int nn = min(n + e, ga.n - 1);
        bs[e] = ga.bs[nn];
        bb[e] = ga.bias ? ga.bias[nn] : 0;
      }
      bi = i32x2{(int)((uint32_t)bb[0] | ((uint32_t)bb[1] << 16)), (int)((uint32_t)bb[2] | ((uint32_t)bb[3] << 16))};
    }
  };

  // k block d at ring position dm: k-steps 0 and 1 of 64 MFMAs.  MODE 0:
  // unit 2 d + 4 is loaded under k-step 0 and unit 2 d + 5 under k-step 1, one
  // load per 8 MFMAs; one barrier, in front of k-step 1: behind it, units
  // 2 d + 2 and 2 d + 3 (block d + 1) have landed for k-step 1 to read ahead
  // from, and nobody reads block d's units any more (k-step 1's operands are
  // already in registers), so their slots take units 2 d + 5 and 2 d + 6.  The
  // last two blocks load no units (none are left): MODE 1 (next to last) waits
  // for all of its loads before the barrier; MODE 2 (last) reads nothing
  // ahead, needs no barrier, and loads the first epilogue operands.
  auto block = [&](auto dm_v, auto mode_c, int d) {
    constexpr int MODE = decltype(mode_c)::value;
    const int dm = dm_v, dn = (dm + 1) % HRING;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      if (q == 1 && MODE != 2) {
        if (MODE == 0)
          __builtin_amdgcn_s_waitcnt(0x0f70 | 8);  // vmcnt(8): unit 2 d + 4 may stay in flight
        else
          __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): block d + 1 has landed
        __syncthreads();
      }
      if constexpr (MODE == 2 && !RAW && !SPLIT)
        if (q == 0 && early) {
          load_row_scales();
          load_cols(std::true_type{}, 0, bsc, bic);
        }
#pragma unroll
      for (int idx = 0; idx < 64; ++idx) {
        if (idx % 4 == 0 && !(MODE == 2 && q == 1))
          nxt[idx / 4] = q == 0 ? read_op(dm, 1, idx / 4) : read_op(dn, 0, idx / 4);
        if (MODE == 0 && q == 0 && idx % 8 == 0) load_one(2 * d + 4, idx / 8);
        if (MODE == 0 && q == 1 && idx % 8 == 0) load_one(2 * d + 5, idx / 8);
        const int nb = idx >> 3, mb = idx & 7;
        acc[nb][mb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(cur[8 + nb], cur[mb], acc[nb][mb], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
      if (!(MODE == 2 && q == 1))
#pragma unroll
        for (int r = 0; r < 16; ++r) cur[r] = nxt[r];
    }
  };
  using M0 = std::integral_constant<int, 0>;
  int d = 0;
  for (; d + HRING <= nd - 2; d += HRING) {
    block(std::integral_constant<int, 0>{}, M0{}, d);
    block(std::integral_constant<int, 1>{}, M0{}, d + 1);
    block(std::integral_constant<int, 2>{}, M0{}, d + 2);
    block(std::integral_constant<int, 3>{}, M0{}, d + 3);
    block(std::integral_constant<int, 4>{}, M0{}, d + 4);
  }
  if (d < nd - 2) block(std::integral_constant<int, 0>{}, M0{}, d);
  if (d + 1 < nd - 2) block(std::integral_constant<int, 1>{}, M0{}, d + 1);
  if (d + 2 < nd - 2) block(std::integral_constant<int, 2>{}, M0{}, d + 2);
  if (d + 3 < nd - 2) block(std::integral_constant<int, 3>{}, M0{}, d + 3);
  // the last two blocks, at ring positions known at run time only
  if (nd >= 2) block((nd - 2) % HRING, std::integral_constant<int, 1>{}, nd - 2);
  block((nd - 1) % HRING, std::integral_constant<int, 2>{}, nd - 1);
  // every wave drains its loads before the workgroup ends
  __builtin_amdgcn_s_waitcnt(0x0f70);

  if constexpr (SPLIT) {
    // k-range of a split tile: the raw 256 x 256 int32 partial, row-major
    int32_t *wp = ga.ws + ((int64_t)(L - ga.full) * ga.nsplit + part) * (HBM_ * HBN);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int m = wm * 128 + j * 16 + li;
#pragma unroll
      for (int i = 0; i < 8; ++i) *(i32x4 *)(wp + m * HBN + wn * 128 + i * 16 + 4 * lg) = acc[i][j];
    }
    return;
  }

  if constexpr (!RAW) {
    if (ga.st_ok) {
      // bf16 tile through LDS: each wave stages its 128 x 128 outputs in rows
      // of 256 bytes whose 16-byte chunk c sits at c ^ stg_sw(row), then
      // writes 16 bytes per lane, 256-byte row segments.  A staging write (8
      // bytes per lane) covers 16 rows x 2 chunks, a read 2 rows x 16 chunks:
      // under the swizzle both meet every bank once.
      constexpr int ROWB = 128 * 2;
      static_assert(HWAVES * 128 * ROWB <= HRING * HUNIT, "staging fits the ring");
      auto stg_sw = [](int row) { return 2 * ((row >> 1) & 7); };
      __syncthreads();  // every wave is done with the ring
      const uint32_t wt = (uint32_t)(w * 128 * ROWB);
      if (!early) {
        load_row_scales();
        load_cols(std::false_type{}, 0, bsc, bic);
      }
      // n-blocks outermost, so that one block's column scales and converted
      // bias are live at a time (the next block's are in flight), and the
      // bias test outside the element loops (per element: convert, two
      // multiplies, the bias add, half a pack)
      auto stage_tile = [&](auto has_bias, auto vec_c) {
        constexpr bool HB = decltype(has_bias)::value;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          if (i < 7) load_cols(vec_c, i + 1, bsn, bin);
          float bf[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t bw = (uint32_t)bic[e >> 1];
            bf[e] = HB ? bf16_bits_to_f32((e & 1) ? (bw >> 16) : (bw & 0xffffu)) : 0.0f;
          }
          const int ch = 2 * i + (lg >> 1);  // 16-byte chunk of the lane's 4 columns
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            uint16_t vals[4];
            float tv[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              float t = (float)acc[i][j][e];
              t = t * bsc[e];
              t = t * asv[j];
              if constexpr (HB) t = t + bf[e];
              tv[e] = t;
            }
            bf16_quad(tv, vals);
            const int row = j * 16 + li;
            *(i32x2 *)(smem + wt + row * ROWB + (ch ^ stg_sw(row)) * 16 + (lg & 1) * 8) =
                i32x2{(int)((uint32_t)vals[0] | ((uint32_t)vals[1] << 16)),
                      (int)((uint32_t)vals[2] | ((uint32_t)vals[3] << 16))};
          }
          bsc = bsn;
          bic = bin;
        }
      };
      if (early) {
        if (ga.bias)
          stage_tile(std::true_type{}, std::true_type{});
        else
          stage_tile(std::false_type{}, std::true_type{});
      } else {
        if (ga.bias)
          stage_tile(std::true_type{}, std::false_type{});
        else
          stage_tile(std::false_type{}, std::false_type{});
      }
      if constexpr (GLU) {
        // gate halves sit in the staging rows of waves (wm, 0), up halves in
        // (wm, 1); each wave writes 64 of the tile's 256 output rows
        __syncthreads();
#pragma unroll
        for (int it = 0; it < 16; ++it) {
          const int r = w * 64 + it * 4 + (lane >> 4), c = lane & 15;
          const int wr = r >> 7, rr = r & 127;
          const uint32_t so = (uint32_t)(rr * ROWB + (c ^ stg_sw(rr)) * 16);
          const i32x4 gv = *(const i32x4 *)(smem + (uint32_t)((wr * 2) * 128 * ROWB) + so);
          const i32x4 uv = *(const i32x4 *)(smem + (uint32_t)((wr * 2 + 1) * 128 * ROWB) + so);
          i32x4 o;
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = (int)swiglu_pair((uint32_t)gv[e], (uint32_t)uv[e]);
          const int m = m0 + r, n = n0 / 2 + c * 8;
          if (m < ga.m) *(i32x4 *)((uint16_t *)ga.out + (int64_t)m * ga.ldo + n) = o;
        }
        return;
      }
#pragma unroll
      for (int it = 0; it < 32; ++it) {
        const int r = it * 4 + (lane >> 4), c = lane & 15;
        const i32x4 v = *(const i32x4 *)(smem + wt + r * ROWB + (c ^ stg_sw(r)) * 16);
        const int m = m0 + wm * 128 + r, n = n0 + wn * 128 + c * 8;
        if (m < ga.m && n < ga.n) {
          uint16_t *op = (uint16_t *)ga.out + (int64_t)m * ga.ldo + n;
          if (n + 7 < ga.n) {
            *(i32x4 *)op = v;
          } else {
            for (int e = 0; e < 8 && n + e < ga.n; ++e) op[e] = (uint16_t)((uint32_t)v[e >> 1] >> (16 * (e & 1)));
          }
        }
      }
      return;
    }
  }
  if constexpr (GLU) return;  // the GLU launcher always takes the staged path above
  // unstaged epilogue (bf16 rows not 16-byte aligned) and the raw int32 output
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    if constexpr (!RAW) load_cols(std::false_type{}, i, bsc, bic);
    const int n = n0 + wn * 128 + i * 16 + 4 * lg;
    if (n >= ga.n) continue;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int m = m0 + wm * 128 + j * 16 + li;
      if (m >= ga.m) continue;
      if constexpr (RAW) {
        int32_t *op = (int32_t *)ga.out + (int64_t)m * ga.ldo + n;
        if (n + 3 < ga.n) {
          *(i32x4 *)op = acc[i][j];
        } else {
          for (int e = 0; e < 4 && n + e < ga.n; ++e) op[e] = acc[i][j][e];
        }
      } else {
        const float asm_ = ga.as[m];
        uint16_t *op = (uint16_t *)ga.out + (int64_t)m * ga.ldo + n;
        uint16_t vals[4];
        float tv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float t = (float)acc[i][j][e];
          t = t * bsc[e];
          t = t * asm_;
          if (ga.bias) {
            const uint32_t bw = (uint32_t)bic[e >> 1];
            t = t + bf16_bits_to_f32((e & 1) ? (bw >> 16) : (bw & 0xffffu));
          }
          tv[e] = t;
        }
        bf16_quad(tv, vals);
        if (n + 3 < ga.n) {
          *(i32x2 *)op = i32x2{(int)((uint32_t)vals[0] | ((uint32_t)vals[1] << 16)),
                               (int)((uint32_t)vals[2] | ((uint32_t)vals[3] << 16))};
        } else {
          for (int e = 0; e < 4 && n + e < ga.n; ++e) op[e] = vals[e];
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// The last, partial round of 256 x 256 tiles when it holds at most an eighth
// of a round: each of its tiles runs as 8 sub-tiles of 64 (m) x 128 (n) over
// the whole of k, one workgroup each, so the round fills the CUs with no
// partial sums and no merge (the k split's int32 partials and their merge
// cost about twice the time).  4 waves as 2 (m) x 2 (n) of 32 x 64 (8 blocks
// of v_mfma_i32_16x16x64_i8).  k moves in blocks of 128 bytes, one ring unit
// each (64 rows of A, then 128 rows of B, rows of 128 bytes with chunk c of
// row r at c ^ ((r >> 1) & 7), as in the whole-tile kernel), 5 units deep;
// block d's loads fetch unit d + 3.  The epilogue stores straight from
// registers (the round is small) with the whole-tile kernel's arithmetic.
constexpr int SBM = 64, SBN = 128, SRING = 5;
constexpr int SUNIT = (SBM + SBN) * HKD;  // bytes of one ring unit
constexpr int SLOADS = SUNIT / 1024 / 4;  // 1 KiB wave loads per wave per unit
static_assert(SUNIT % 4096 == 0 && SRING * SUNIT <= 160 * 1024, "ring fits the LDS");

template <bool RAW>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
gemm_i8_sub_kernel(const GArgs ga) {
#pragma clang fp contract(off)
  __shared__ __attribute__((aligned(1024))) char smem[SRING * SUNIT];
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char *)smem;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = w >> 1, wn = w & 1;  // wave tile: a rows [wm*32, +32), b rows [wn*64, +64)
  // item L: sub-tile L % 8 of tile full + L / 8; the 8 sub-tiles of a tile are
  // consecutive logical ids, which run on one XCD (its L2 holds their panels)
  const int L = xcd_logical_id(blockIdx.x, gridDim.x);
  const int sub = L & 7;
  int tm, tn;
  grouped_tile(ga.full + (L >> 3), ga.tm_count, ga.tn_count, tm, tn);
  const int m0 = tm * HBM_ + (sub >> 1) * SBM, n0 = tn * HBN + (sub & 1) * SBN;
  if (m0 >= ga.m || n0 >= ga.n) return;  // the whole workgroup: no barrier is left waiting
  const int nd = ga.k / HKD;  // >= 1

  // Loads: block b (0..23) of a unit is 8 rows x 128 bytes: b < 8 the A rows
  // 8 b .., else the B rows 8 (b - 8) ..; wave w loads blocks w + 4 i.  Lane:
  // row 8 blk + lane / 8, physical chunk lane % 8, logical chunk
  // (lane % 8) ^ ((row >> 1) & 7), the same for all of the wave's blocks
  // (their parity is w's).
  const int lch = (lane & 7) ^ ((4 * (w & 1) + (lane >> 4)) & 7);
  uint32_t soff[SLOADS];
#pragma unroll
  for (int i = 0; i < SLOADS; ++i) {
    const int b = w + 4 * i;
    if (b < SBM / 8)
      soff[i] = (uint32_t)((int64_t)min(m0 + b * 8 + (lane >> 3), ga.m - 1) * ga.lda) + lch * 16;
    else
      soff[i] = (uint32_t)((int64_t)min(n0 + (b - SBM / 8) * 8 + (lane >> 3), ga.n - 1) * ga.ldb) + lch * 16;
  }
  // unit u (k block min(u, nd - 1): units past the last block repeat it, into
  // a slot nobody reads) into ring slot u % SRING
  auto load_unit = [&](int u) {
    const int64_t k0 = (int64_t)min(u, nd - 1) * HKD;
    const uint32_t dst = lds0 + (uint32_t)((u % SRING) * SUNIT);
#pragma unroll
    for (int i = 0; i < SLOADS; ++i) {
      const int b = w + 4 * i;
      hload_lds16((b < SBM / 8 ? ga.a : ga.b) + k0, soff[i], dst + b * 1024);
    }
  };
  // operand reads: 16x16x64 lane (i, g4) holds 16 bytes of row i at logical
  // chunk 4 q + g4 (k-step q of the block)
  const int li = lane & 15, lg = lane >> 4;
  uint32_t rdq[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) rdq[q] = (uint32_t)(li * HKD + (((4 * q + lg) ^ ((li >> 1) & 7)) * 16));
  // operand r of k-step q of unit u: r < 2 A block r, else B block r - 2
  auto read_op = [&](int u, int q, int r) -> i32x4 {
    const uint32_t base = (uint32_t)((u % SRING) * SUNIT) + rdq[q];
    if (r < 2) return *(const i32x4 *)(smem + base + (wm * 32 + 16 * r) * HKD);
    return *(const i32x4 *)(smem + base + SBM * HKD + (wn * 64 + 16 * (r - 2)) * HKD);
  };

  i32x4 acc[4][2];  // [n block][m block], D[n][m]: lane (j, g4) holds n = 16 nb + 4 g4 + (0..3), m = 16 mb + j
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = i32x4{0, 0, 0, 0};

  // prologue: units 0..2 in flight, unit 0 landed
  load_unit(0);
  load_unit(1);
  load_unit(2);
  __builtin_amdgcn_s_waitcnt(0x0f70 | (2 * SLOADS));  // units 1, 2 may stay in flight
  __syncthreads();
  i32x4 cur[6], nxt[6];
#pragma unroll
  for (int r = 0; r < 6; ++r) cur[r] = read_op(0, 0, r);
  // block d: k-step 0 loads unit d + 3 into the slot of unit d - 2 (every
  // wave is past block d - 2: the barrier of block d - 1) and reads k-step 1's
  // operands; k-step 1 waits for unit d + 1 (units d + 2 and d + 3 may stay in
  // flight), passes the barrier and reads block d + 1's first operands.
  for (int d = 0; d < nd; ++d) {
    load_unit(d + 3);
#pragma unroll
    for (int r = 0; r < 6; ++r) nxt[r] = read_op(d, 1, r);
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) acc[nb][mb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(cur[2 + nb], cur[mb], acc[nb][mb], 0, 0, 0);
    __builtin_amdgcn_s_waitcnt(0x0f70 | (2 * SLOADS));
    __syncthreads();
    if (d + 1 < nd)
#pragma unroll
      for (int r = 0; r < 6; ++r) cur[r] = read_op(d + 1, 0, r);
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) acc[nb][mb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(nxt[2 + nb], nxt[mb], acc[nb][mb], 0, 0, 0);
  }
  // every wave drains its loads before the workgroup ends
  __builtin_amdgcn_s_waitcnt(0x0f70);

  // epilogue straight from registers: 4 consecutive n of one m per lane
#pragma unroll
  for (int nb = 0; nb < 4; ++nb) {
    const int n = n0 + wn * 64 + nb * 16 + 4 * lg;
    if (n >= ga.n) continue;
    float bsv[4];
    uint16_t bbv[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int nn = min(n + e, ga.n - 1);
      bsv[e] = RAW ? 0.0f : ga.bs[nn];
      bbv[e] = (!RAW && ga.bias) ? ga.bias[nn] : 0;
    }
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      const int m = m0 + wm * 32 + mb * 16 + li;
      if (m >= ga.m) continue;
      if constexpr (RAW) {
        int32_t *op = (int32_t *)ga.out + (int64_t)m * ga.ldo + n;
        if (n + 3 < ga.n)
          *(i32x4 *)op = acc[nb][mb];
        else
          for (int e = 0; e < 4 && n + e < ga.n; ++e) op[e] = acc[nb][mb][e];
      } else {
        const float asm_ = ga.as[m];
        uint16_t vals[4];
        float tv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) tv[e] = dequant_f32(acc[nb][mb][e], bsv[e], asm_, ga.bias != nullptr, bbv[e]);
        bf16_quad(tv, vals);
        uint16_t *op = (uint16_t *)ga.out + (int64_t)m * ga.ldo + n;
        if (n + 3 < ga.n && ga.st_ok)
          *(i32x2 *)op = i32x2{(int)((uint32_t)vals[0] | ((uint32_t)vals[1] << 16)),
                               (int)((uint32_t)vals[2] | ((uint32_t)vals[3] << 16))};
        else
          for (int e = 0; e < 4 && n + e < ga.n; ++e) op[e] = vals[e];
      }
    }
  }
}

// Merge of the K-split GLU tiles: gate columns c .. c + 3 and up columns
// 128 + c .. of one row, each the sum of its partials, dequantised and
// rounded as the GEMM's epilogue does, then SwiGLU.  Block: 8 rows of one
// tile, 4 output columns per thread.
__global__ void __launch_bounds__(256) gemm_split_merge_glu_kernel(const GArgs ga) {
  const int item = blockIdx.x / (HBM_ / 8);
  const int r = (blockIdx.x % (HBM_ / 8)) * 8 + (threadIdx.x >> 5);
  const int c = (threadIdx.x & 31) * 4;
  int tm, tn;
  grouped_tile(ga.full + item, ga.tm_count, ga.tn_count, tm, tn);
  const int m = tm * HBM_ + r, n0 = tn * HBN;
  if (m >= ga.m) return;
  const int32_t *wp = ga.ws + (int64_t)item * ga.nsplit * (HBM_ * HBN) + r * HBN + c;
  i32x4 ag = *(const i32x4 *)wp, au = *(const i32x4 *)(wp + 128);
  for (int p = 1; p < ga.nsplit; ++p) {
    ag += *(const i32x4 *)(wp + (int64_t)p * (HBM_ * HBN));
    au += *(const i32x4 *)(wp + (int64_t)p * (HBM_ * HBN) + 128);
  }
  const float asm_ = ga.as[m];
  float tg[4], tu[4];
  uint16_t vg[4], vu[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int ng = n0 + c + e, nu = ng + 128;
    tg[e] = dequant_f32(ag[e], ga.bs[ng], asm_, ga.bias != nullptr, ga.bias ? ga.bias[ng] : 0u);
    tu[e] = dequant_f32(au[e], ga.bs[nu], asm_, ga.bias != nullptr, ga.bias ? ga.bias[nu] : 0u);
  }
  bf16_quad(tg, vg);
  bf16_quad(tu, vu);
  const uint32_t o0 = swiglu_pair((uint32_t)vg[0] | ((uint32_t)vg[1] << 16), (uint32_t)vu[0] | ((uint32_t)vu[1] << 16));
  const uint32_t o1 = swiglu_pair((uint32_t)vg[2] | ((uint32_t)vg[3] << 16), (uint32_t)vu[2] | ((uint32_t)vu[3] << 16));
  *(i32x2 *)((uint16_t *)ga.out + (int64_t)m * ga.ldo + n0 / 2 + c) = i32x2{(int)o0, (int)o1};
}

// Merge of the K-split tiles: the sum of each tile's nsplit int32 partials
// (exact), then the GEMM's epilogue.  Block: 4 rows of one tile, 4 columns
// per thread.
template <bool RAW>
__global__ void __launch_bounds__(256) gemm_split_merge_kernel(const GArgs ga) {
  const int item = blockIdx.x / (HBM_ / 4);
  const int r = (blockIdx.x % (HBM_ / 4)) * 4 + (threadIdx.x >> 6);
  const int c = (threadIdx.x & 63) * 4;
  int tm, tn;
  grouped_tile(ga.full + item, ga.tm_count, ga.tn_count, tm, tn);
  const int m = tm * HBM_ + r, n = tn * HBN + c;
  if (m >= ga.m || n >= ga.n) return;
  const int32_t *wp = ga.ws + (int64_t)item * ga.nsplit * (HBM_ * HBN) + r * HBN + c;
  i32x4 acc = *(const i32x4 *)wp;
  for (int p = 1; p < ga.nsplit; ++p) acc += *(const i32x4 *)(wp + (int64_t)p * (HBM_ * HBN));
  if constexpr (RAW) {
    int32_t *op = (int32_t *)ga.out + (int64_t)m * ga.ldo + n;
    if (n + 3 < ga.n)
      *(i32x4 *)op = acc;
    else
      for (int e = 0; e < 4 && n + e < ga.n; ++e) op[e] = acc[e];
  } else {
    const float asm_ = ga.as[m];
    uint16_t vals[4];
    float tv[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int nn = min(n + e, ga.n - 1);
      tv[e] = dequant_f32(acc[e], ga.bs[nn], asm_, ga.bias != nullptr, ga.bias ? ga.bias[nn] : 0u);
    }
    bf16_quad(tv, vals);
    uint16_t *op = (uint16_t *)ga.out + (int64_t)m * ga.ldo + n;
    if (n + 3 < ga.n)
      *(i32x2 *)op = i32x2{(int)((uint32_t)vals[0] | ((uint32_t)vals[1] << 16)),
                           (int)((uint32_t)vals[2] | ((uint32_t)vals[3] << 16))};
    else
      for (int e = 0; e < 4 && n + e < ga.n; ++e) op[e] = vals[e];
  }
}

// K split of the last, partial round of 256 x 256 tiles (all tiles when they
// fill less than half the CUs): its tiles' 128-byte k blocks are dealt to S
// parts, S up to CUs / tiles and at least 2 blocks per part, so that the
// round fills the CUs; the partials are merged by gemm_split_merge_kernel.
void gemm_split_plan(int32_t m, int32_t n, int32_t k, int &tail, int &parts) {
  tail = 0, parts = 1;
  const int cus = device_cus();
  if (cus <= 0 || m <= 0 || n <= 0 || k <= 0 || k % HKD) return;
  const int64_t tiles = (int64_t)((m + HBM_ - 1) / HBM_) * ((n + HBN - 1) / HBN);
  const int64_t t = tiles % cus;
  if (t == 0 || 2 * t > cus) return;
  const int64_t s = std::min<int64_t>(cus / t, (k / HKD) / 2);
  if (s < 2) return;
  tail = (int)t, parts = (int)s;
}

int64_t gemm_split_bytes(int tail, int parts) { return (int64_t)tail * parts * HBM_ * HBN * 4; }

template <bool RAW>
int launch_gemm(void *out, const int8_t *a, const int8_t *b, const float *as, const float *bs, const void *bias,
                int32_t m, int32_t n, int32_t k, int64_t lda, int64_t ldb, int64_t ldo, void *ws, int64_t ws_bytes,
                void *stream) {
  const char *what = RAW ? "tmhd_gemm_i8_i32" : "tmhd_gemm_w8a8";
  if (m < 0 || n <= 0 || k <= 0) return set_error(TMHD_ERR_INVALID, "%s: m %d n %d k %d", what, m, n, k);
  if (k % GBK) return set_error(TMHD_ERR_UNSUPPORTED, "%s: k %d must be a multiple of %d", what, k, GBK);
  if (!out || !a || !b || (!RAW && (!as || !bs))) return set_error(TMHD_ERR_INVALID, "%s: null pointer", what);
  if (((uintptr_t)a % 16) || ((uintptr_t)b % 16) || lda % 16 || ldb % 16 || lda < k || ldb < k || ldo < n)
    return set_error(TMHD_ERR_INVALID, "%s: operands must be 16-byte aligned rows with stride >= k", what);
  if (m == 0) return TMHD_OK;
  const int64_t tiles = (int64_t)((m + GBM - 1) / GBM) * ((n + GBN - 1) / GBN);
  GArgs ga{a, b, out, as, bs, (const uint16_t *)bias, m, n, k, lda, ldb, ldo, (m + GBM - 1) / GBM, (n + GBN - 1) / GBN,
           (int32_t)(((uintptr_t)bs % 16) == 0 && ((uintptr_t)bias % 8) == 0),
           (int32_t)(!RAW && ((uintptr_t)out % 16) == 0 && ldo % 8 == 0), (int32_t)tiles, 1, nullptr};
  const int64_t grid = tiles;
  // the one-wave-per-SIMD kernel takes 32-bit row offsets and whole 128-byte
  // k blocks; other shapes (k an odd multiple of 64) run the 8-wave kernel
  const bool wide = (int64_t)(m - 1) * lda + k < ((int64_t)1 << 32) &&
                    (int64_t)(n - 1) * ldb + k < ((int64_t)1 << 32);
  if (wide && k % HKD == 0) {
    // a last round of at most an eighth of the CUs' tiles runs as 64 x 128
    // sub-tiles over the whole of k (no workspace needed); a larger partial
    // round, up to half the CUs, is split along k into the workspace
    const int cus = device_cus();
    const int64_t last = cus > 0 ? tiles % cus : 0;
    if (last > 0 && 8 * last <= cus) {
      ga.full = (int32_t)(tiles - last);
      hipStream_t s = (hipStream_t)stream;
      if (ga.full > 0)
        hipLaunchKernelGGL((gemm_i8_wave128_kernel<RAW, false>), dim3((unsigned)ga.full), dim3(HWAVES * 64), 0, s, ga);
      hipLaunchKernelGGL((gemm_i8_sub_kernel<RAW>), dim3((unsigned)(last * 8)), dim3(256), 0, s, ga);
      return check_launch(what);
    }
    int tail = 0, parts = 1;
    gemm_split_plan(m, n, k, tail, parts);
    if (parts > 1 && ws && ((uintptr_t)ws % 16) == 0 && ws_bytes >= gemm_split_bytes(tail, parts)) {
      ga.full = (int32_t)(tiles - tail);
      ga.nsplit = parts;
      ga.ws = (int32_t *)ws;
    }
    hipStream_t s = (hipStream_t)stream;
    if (ga.full > 0)
      hipLaunchKernelGGL((gemm_i8_wave128_kernel<RAW, false>), dim3((unsigned)ga.full), dim3(HWAVES * 64), 0, s, ga);
    if (ga.nsplit > 1) {
      hipLaunchKernelGGL((gemm_i8_wave128_kernel<false, true>), dim3((unsigned)(tail * parts)), dim3(HWAVES * 64), 0,
                         s, ga);
      hipLaunchKernelGGL(gemm_split_merge_kernel<RAW>, dim3((unsigned)(tail * (HBM_ / 4))), dim3(256), 0, s, ga);
    }
  } else {
    hipLaunchKernelGGL(gemm_i8_kernel<RAW>, dim3((unsigned)grid), dim3(GWAVES * 64), 0, (hipStream_t)stream, ga);
  }
  return check_launch(what);
}

// The GEMM with the SwiGLU epilogue: out[m][n / 2] from gate / up rows
// interleaved in blocks of 128 (see the GLU kernel).  Only the one-wave-per-
// SIMD kernel and its k-split carry the GLU epilogue.
int launch_gemm_glu(void *out, const int8_t *a, const int8_t *b, const float *as, const float *bs, const void *bias,
                    int32_t m, int32_t n, int32_t k, int64_t lda, int64_t ldb, int64_t ldo, void *ws,
                    int64_t ws_bytes, void *stream) {
  const char *what = "tmhd_gemm_w8a8_swiglu_ws";
  if (m < 0 || n <= 0 || k <= 0) return set_error(TMHD_ERR_INVALID, "%s: m %d n %d k %d", what, m, n, k);
  if (k % HKD || n % 256)
    return set_error(TMHD_ERR_UNSUPPORTED, "%s: k %d (a multiple of %d), n %d (gate + up, a multiple of 256)", what,
                     k, HKD, n);
  if (!out || !a || !b || !as || !bs) return set_error(TMHD_ERR_INVALID, "%s: null pointer", what);
  if (((uintptr_t)a % 16) || ((uintptr_t)b % 16) || lda % 16 || ldb % 16 || lda < k || ldb < k || ldo < n / 2 ||
      ((uintptr_t)out % 16) || ldo % 8)
    return set_error(TMHD_ERR_INVALID, "%s: operands and output must be 16-byte aligned rows", what);
  if (m == 0) return TMHD_OK;
  if (!((int64_t)(m - 1) * lda + k < ((int64_t)1 << 32) && (int64_t)(n - 1) * ldb + k < ((int64_t)1 << 32)))
    return set_error(TMHD_ERR_UNSUPPORTED, "%s: operands beyond 32-bit row offsets", what);
  const int64_t tiles = (int64_t)((m + HBM_ - 1) / HBM_) * (n / HBN);
  GArgs ga{a, b, out, as, bs, (const uint16_t *)bias, m, n, k, lda, ldb, ldo, (m + HBM_ - 1) / HBM_, n / HBN,
           (int32_t)(((uintptr_t)bs % 16) == 0 && ((uintptr_t)bias % 8) == 0), 1, (int32_t)tiles, 1, nullptr};
  int tail = 0, parts = 1;
  gemm_split_plan(m, n, k, tail, parts);
  if (parts > 1 && ws && ((uintptr_t)ws % 16) == 0 && ws_bytes >= gemm_split_bytes(tail, parts)) {
    ga.full = (int32_t)(tiles - tail);
    ga.nsplit = parts;
    ga.ws = (int32_t *)ws;
  }
  hipStream_t s = (hipStream_t)stream;
  if (ga.full > 0)
    hipLaunchKernelGGL((gemm_i8_wave128_kernel<false, false, true>), dim3((unsigned)ga.full), dim3(HWAVES * 64), 0, s,
                       ga);
  if (ga.nsplit > 1) {
    hipLaunchKernelGGL((gemm_i8_wave128_kernel<false, true>), dim3((unsigned)(tail * parts)), dim3(HWAVES * 64), 0, s,
                       ga);
    hipLaunchKernelGGL(gemm_split_merge_glu_kernel, dim3((unsigned)(tail * (HBM_ / 8))), dim3(256), 0, s, ga);
  }
  return check_launch(what);
}

}  // namespace
}  // namespace tmhd

extern "C" int tmhd_token_quant_i8(int8_t *q, float *scale, const void *x, int32_t rows, int32_t cols,
                                   int64_t x_stride, void *stream) {
  return tmhd::launch_row_quant<false>(q, scale, x, rows, cols, x_stride, stream, "tmhd_token_quant_i8");
}

extern "C" int tmhd_weight_quant_i8(int8_t *q, float *scale, const void *w, int32_t n, int32_t k, void *stream) {
  return tmhd::launch_row_quant<true>(q, scale, w, n, k, k, stream, "tmhd_weight_quant_i8");
}

extern "C" int tmhd_gemm_w8a8(void *out, const int8_t *a, const int8_t *b, const float *a_scale,
                              const float *b_scale, const void *bias, int32_t m, int32_t n, int32_t k, int64_t lda,
                              int64_t ldb, int64_t ldo, void *stream) {
  return tmhd::launch_gemm<false>(out, a, b, a_scale, b_scale, bias, m, n, k, lda, ldb, ldo, nullptr, 0, stream);
}

extern "C" int tmhd_gemm_i8_i32(int32_t *out, const int8_t *a, const int8_t *b, int32_t m, int32_t n, int32_t k,
                                int64_t lda, int64_t ldb, int64_t ldo, void *stream) {
  return tmhd::launch_gemm<true>(out, a, b, nullptr, nullptr, nullptr, m, n, k, lda, ldb, ldo, nullptr, 0, stream);
}

extern "C" int64_t tmhd_gemm_split_workspace_bytes(int32_t m, int32_t n, int32_t k) {
  int tail = 0, parts = 1;
  tmhd::gemm_split_plan(m, n, k, tail, parts);
  return parts > 1 ? tmhd::gemm_split_bytes(tail, parts) : 0;
}

extern "C" int tmhd_gemm_w8a8_ws(void *out, const int8_t *a, const int8_t *b, const float *a_scale,
                                 const float *b_scale, const void *bias, int32_t m, int32_t n, int32_t k, int64_t lda,
                                 int64_t ldb, int64_t ldo, void *workspace, int64_t workspace_bytes, void *stream) {
  return tmhd::launch_gemm<false>(out, a, b, a_scale, b_scale, bias, m, n, k, lda, ldb, ldo, workspace,
                                  workspace_bytes, stream);
}

extern "C" int tmhd_gemm_i8_i32_ws(int32_t *out, const int8_t *a, const int8_t *b, int32_t m, int32_t n, int32_t k,
                                   int64_t lda, int64_t ldb, int64_t ldo, void *workspace, int64_t workspace_bytes,
                                   void *stream) {
  return tmhd::launch_gemm<true>(out, a, b, nullptr, nullptr, nullptr, m, n, k, lda, ldb, ldo, workspace,
                                 workspace_bytes, stream);
}

extern "C" int tmhd_gemm_w8a8_swiglu_ws(void *out, const int8_t *a, const int8_t *b, const float *a_scale,
                                        const float *b_scale, const void *bias, int32_t m, int32_t n, int32_t k,
                                        int64_t lda, int64_t ldb, int64_t ldo, void *workspace,
                                        int64_t workspace_bytes, void *stream) {
  return tmhd::launch_gemm_glu(out, a, b, a_scale, b_scale, bias, m, n, k, lda, ldb, ldo, workspace, workspace_bytes,
                               stream);
}
