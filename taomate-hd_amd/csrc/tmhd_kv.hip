// Slot packing (token-major K/V rows -> head-major slot) and the smooth-K
// INT8 quantization of the INT8-QK attention path.
#include <math.h>

#include "tmhd_internal.h"

namespace tmhd {
namespace {

constexpr int kTile = 64;

// ---------------------------------------------------------------------------
// tmhd_kv_pack: one workgroup = 64 slot positions of one head, D threads.
// Position p of the slot is: data row (p - dst) if dst <= p < dst + n,
// zero if dst + n <= p < zero_to, untouched otherwise.
// WITH_K false: the key rows of data positions are left to the caller (the
// staged norm + RoPE kernel writes them); zero positions are still cleared.
// Thread (dc, g) owns the 16-byte column chunk dc (columns 8 dc .. 8 dc + 7) of
// the 8 tokens stored at transposed positions 8 g .. 8 g + 7: it loads their 8
// key and value chunks, copies the keys, and transposes the 8 x 8 block of
// values in registers into 8 transposed rows of 8 positions. A wave's loads
// and stores are whole 128-byte lines; no LDS and no barrier.
template <int D, bool WITH_K = true>
__global__ void __launch_bounds__(D) kv_pack_kernel(const uint16_t *__restrict__ k, const uint16_t *__restrict__ v,
                                                    int64_t ts, int64_t hs, const int32_t *__restrict__ rows,
                                                    int32_t row0, int32_t n, uint16_t *__restrict__ ks,
                                                    uint16_t *__restrict__ vts, int64_t khs, int64_t vhs, int32_t vrs,
                                                    int32_t dst, int32_t zero_to, int32_t p_begin) {
  const int h = blockIdx.y;
  const int p0 = p_begin + blockIdx.x * kTile;
  const int dc = threadIdx.x >> 3, g = threadIdx.x & 7;
  int tok[8], kind[8];  // kind: 0 untouched, 1 data, 2 zero
  bool all = true, any = false;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    tok[e] = vt_position(g * 8 + e);
    const int p = p0 + tok[e];
    kind[e] = (p >= dst && p < dst + n) ? 1 : (p >= dst + n && p < zero_to) ? 2 : 0;
    all = all && kind[e] != 0;
    any = any || kind[e] != 0;
  }
  i32x4 kv[8], vv[8];
  if (n > 0) {
    // every load issued before any is used: indices are clamped into the
    // data rows and the values of other positions are dropped afterwards
    int64_t src[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int i = min(max(p0 + tok[e] - dst, 0), n - 1);
      src[e] = (int64_t)(rows ? rows[i] : row0 + i) * ts + (int64_t)h * hs + dc * 8;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if constexpr (WITH_K) kv[e] = *(const i32x4 *)(k + src[e]);
      vv[e] = *(const i32x4 *)(v + src[e]);
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e)
    if (n == 0 || kind[e] != 1) kv[e] = vv[e] = i32x4{0, 0, 0, 0};
  uint16_t *kout = ks + (int64_t)h * khs + dc * 8;
#pragma unroll
  for (int e = 0; e < 8; ++e)
    if (WITH_K ? kind[e] != 0 : kind[e] == 2) *(i32x4 *)(kout + (int64_t)(p0 + tok[e]) * D) = kv[e];
  if (!any) return;
  uint16_t *out = vts + (int64_t)h * vhs + (int64_t)(dc * 8) * vrs + p0 + g * 8;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    i32x4 w;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const uint32_t x = (uint32_t)vv[2 * m][j >> 1], y = (uint32_t)vv[2 * m + 1][j >> 1];
      w[m] = (int)((j & 1) ? (x >> 16) | (y & 0xffff0000u) : (x & 0xffffu) | (y << 16));
    }
    if (all) {
      *(i32x4 *)(out + (int64_t)j * vrs) = w;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (kind[e] != 0) out[(int64_t)j * vrs + e] = (uint16_t)((uint32_t)w[e >> 1] >> (16 * (e & 1)));
    }
  }
}

// ---------------------------------------------------------------------------
// Smooth-K mean.  Keys are summed exactly as int64 fixed point (x * 2^24,
// rounded to nearest even), so the sum does not depend on the order of the
// parallel reduction; mean = bf16(fp32(sum * 2^-24 / N)).
constexpr double kMeanFix = 16777216.0;  // 2^24

__global__ void zero_i64_kernel(int64_t *p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

__device__ __forceinline__ int64_t to_fixed(float x) {
  float y = x * 16777216.0f;
  y = fminf(fmaxf(y, -4.0e18f), 4.0e18f);
  return (int64_t)__builtin_rintf(y);
}

// Key segments of one launch: workgroups [blk0[i], blk0[i + 1]) of the grid's
// x dimension cover segment i (its own tokens, 256 per workgroup for the sums,
// TMHD_QUANT_BLOCK for the blocks).
struct KeySegs {
  const uint16_t *k[kMaxSeg];
  int64_t khs[kMaxSeg];
  int8_t *q8[kMaxSeg];
  int64_t q8hs[kMaxSeg];
  float *qs[kMaxSeg];
  int32_t qshs[kMaxSeg];
  int32_t tokens[kMaxSeg];
  int32_t blk0[kMaxSeg + 1];
  int32_t n;
};

__device__ __forceinline__ int key_seg(const KeySegs &a, int b) {
  int s = 0;
  while (s + 1 < a.n && b >= a.blk0[s + 1]) ++s;
  return s;
}

// Fixed-point column sums of one head's keys over 256 tokens per workgroup.
// Thread (c, r) reads 16-byte chunk c (8 channels) of rows t0 + r, t0 + r + RPI, ...
// (all its loads issued before any is used) and keeps 8 int64 partial sums;
// partials are combined in LDS and added to ws[h][d] with one 64-bit atomic per
// channel.  Values with |x| < 127 take the int32 conversion path; a chunk
// holding a larger value takes the int64 path (both give rint(x * 2^24) exactly).
template <int D>
__global__ void __launch_bounds__(256) k_sum_kernel(const KeySegs a, int64_t *__restrict__ ws) {
  constexpr int CPR = D / 8;      // 16-byte chunks per row
  constexpr int RPI = 256 / CPR;  // rows per pass
  constexpr int NP = 256 / RPI;   // passes per workgroup
  __shared__ long long part[RPI][D];
  const int h = blockIdx.y, tid = threadIdx.x, c = tid % CPR, r = tid / CPR;
  const int sg = key_seg(a, blockIdx.x);
  const int t0 = (blockIdx.x - a.blk0[sg]) * 256;
  const int n = min(a.tokens[sg] - t0, 256);
  const uint16_t *base = a.k[sg] + (int64_t)h * a.khs[sg] + (int64_t)t0 * D + c * 8;
  // every load issued before any is used: rows past the end re-read the last
  // row (in bounds) and are zeroed afterwards
  i32x4 raw[NP];
#pragma unroll
  for (int p = 0; p < NP; ++p) raw[p] = *(const i32x4 *)(base + (int64_t)min(p * RPI + r, n - 1) * D);
#pragma unroll
  for (int p = 0; p < NP; ++p)
    if (p * RPI + r >= n) raw[p] = i32x4{};
  long long acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0;
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    float x[8];
    float mx = 0.0f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[2 * e] = bf16_bits_to_f32((uint32_t)raw[p][e] & 0xffffu);
      x[2 * e + 1] = bf16_bits_to_f32((uint32_t)raw[p][e] >> 16);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf(x[e]));
    if (mx < 127.0f) {
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] += (long long)(int)__builtin_rintf(x[e] * 16777216.0f);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] += to_fixed(x[e]);
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) part[r][c * 8 + e] = acc[e];
  __syncthreads();
  if (tid < D) {
    long long sum = 0;
    for (int i = 0; i < RPI; ++i) sum += part[i][tid];
    atomicAdd((unsigned long long *)(ws + h * D + tid), (unsigned long long)sum);
  }
}

// ws[i] = sum over the given per-segment key sums (0 when none are given)
struct SumList {
  const int64_t *p[kMaxSeg];
  int32_t n;
};
__global__ void init_sum_kernel(int64_t *__restrict__ ws, const SumList l, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) {
    unsigned long long acc = 0;  // wrapping sum: the same as the atomics' (associative modulo 2^64)
    for (int s = 0; s < l.n; ++s) acc += (unsigned long long)l.p[s][i];
    ws[i] = (int64_t)acc;
  }
}

__global__ void k_mean_finalize_kernel(const int64_t *__restrict__ ws, uint16_t *__restrict__ mean, int n,
                                       double count) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) {
    const double m = __ddiv_rn((double)ws[i], count * kMeanFix);
    mean[i] = f32_to_bf16_bits((float)m);
  }
}

// ---------------------------------------------------------------------------
// Per-(head, 128-row block) symmetric INT8 quantization of x = src - mean:
//   amax = max |x| over the block's valid rows, scale = amax / 127,
//   q = sat_int8(rint(x * (127 / amax))) (amax = 0: scale 0, q 0).
// Rows in [nvalid, nwrite) are written as zero; every launched block writes
// its scale (0 for a block without valid rows).
template <int D, bool MEAN>
__device__ __forceinline__ void quant_block(const uint16_t *__restrict__ src, int64_t sts, int64_t shs,
                                            const int32_t *__restrict__ rows, int32_t row0,
                                            const uint16_t *__restrict__ mean, int32_t nvalid, int32_t nwrite,
                                            int8_t *__restrict__ q8, int64_t q8hs, float *__restrict__ qscale,
                                            int32_t qshs, int h, int blk) {
  constexpr int CPR = D / 8;          // 8-element chunks per row
  constexpr int RPI = 256 / CPR;      // rows per pass
  constexpr int NP = TMHD_QUANT_BLOCK / RPI;
  __shared__ float red[4];
  const int tid = threadIdx.x;
  const int ch = tid % CPR, r0 = tid / CPR;
  // All loads are issued before any is used (one memory round trip): the
  // mean as one 16-byte read, rows past nvalid re-read row nvalid - 1 (in
  // bounds; nvalid >= 1 for every launched block) and are zeroed afterwards.
  i32x4 mraw = {0, 0, 0, 0};
  if constexpr (MEAN) mraw = *(const i32x4 *)(mean + h * D + ch * 8);
  int rix[NP];
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int ic = min(blk * TMHD_QUANT_BLOCK + p * RPI + r0, nvalid - 1);
    rix[p] = rows ? rows[ic] : row0 + ic;
  }
  i32x4 raw[NP];
#pragma unroll
  for (int p = 0; p < NP; ++p) raw[p] = *(const i32x4 *)(src + (int64_t)rix[p] * sts + (int64_t)h * shs + ch * 8);
  float mf[8];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    mf[2 * e] = bf16_bits_to_f32((uint32_t)mraw[e] & 0xffffu);
    mf[2 * e + 1] = bf16_bits_to_f32((uint32_t)mraw[e] >> 16);
  }
  float x[NP][8];
  float amax = 0.0f;
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const bool valid = blk * TMHD_QUANT_BLOCK + p * RPI + r0 < nvalid;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t w = (uint32_t)raw[p][e];
      x[p][2 * e] = valid ? bf16_bits_to_f32(w & 0xffffu) - mf[2 * e] : 0.0f;
      x[p][2 * e + 1] = valid ? bf16_bits_to_f32(w >> 16) - mf[2 * e + 1] : 0.0f;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(x[p][e]));
  }
  amax = wave_max(amax);
  if ((tid & 63) == 0) red[tid >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float inv = amax > 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
  if (tid == 0) qscale[(int64_t)h * qshs + blk] = __fdiv_rn(amax, 127.0f);
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int i = blk * TMHD_QUANT_BLOCK + p * RPI + r0;
    if (i < nwrite) {
      uint32_t lo = 0, hi = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        lo |= ((uint32_t)quant_rne_sat(x[p][e] * inv) & 0xffu) << (8 * e);
        hi |= ((uint32_t)quant_rne_sat(x[p][4 + e] * inv) & 0xffu) << (8 * e);
      }
      *(i32x2 *)(q8 + (int64_t)h * q8hs + (int64_t)i * D + ch * 8) = i32x2{(int)lo, (int)hi};
    }
  }
}

template <int D>
__global__ void __launch_bounds__(256) block_quant_kernel(const uint16_t *__restrict__ src, int64_t sts, int64_t shs,
                                                          const int32_t *__restrict__ rows, int32_t row0,
                                                          const uint16_t *__restrict__ mean, int32_t nvalid,
                                                          int32_t nwrite, int8_t *__restrict__ q8, int64_t q8hs,
                                                          float *__restrict__ qscale, int32_t qshs) {
  if (mean)
    quant_block<D, true>(src, sts, shs, rows, row0, mean, nvalid, nwrite, q8, q8hs, qscale, qshs, blockIdx.y, blockIdx.x);
  else
    quant_block<D, false>(src, sts, shs, rows, row0, mean, nvalid, nwrite, q8, q8hs, qscale, qshs, blockIdx.y,
                          blockIdx.x);
}

// Every key segment's blocks in one launch (slot rows: token stride D); rows up
// to the 64-token tile padding are written.
template <int D>
__global__ void __launch_bounds__(256) key_block_quant_kernel(const KeySegs a, const uint16_t *__restrict__ mean) {
  const int sg = key_seg(a, blockIdx.x);
  const int nwrite = (a.tokens[sg] + kTile - 1) / kTile * kTile;
  quant_block<D, true>(a.k[sg], D, a.khs[sg], nullptr, 0, mean, a.tokens[sg], nwrite, a.q8[sg], a.q8hs[sg], a.qs[sg],
                       a.qshs[sg], blockIdx.y, blockIdx.x - a.blk0[sg]);
}

bool aligned(const void *p, int bytes) { return ((uintptr_t)p % bytes) == 0; }

template <int D>
int launch_block_quant(const uint16_t *src, int64_t sts, int64_t shs, const int32_t *rows, int32_t row0,
                       const uint16_t *mean, int32_t nvalid, int32_t nwrite, int8_t *q8, int64_t q8hs, float *qs,
                       int32_t qshs, int heads, hipStream_t s) {
  const int nblk = (nwrite + TMHD_QUANT_BLOCK - 1) / TMHD_QUANT_BLOCK;
  if (nblk == 0) return TMHD_OK;
  hipLaunchKernelGGL(block_quant_kernel<D>, dim3(nblk, heads), dim3(256), 0, s, src, sts, shs, rows, row0, mean,
                     nvalid, nwrite, q8, q8hs, qs, qshs);
  return check_launch("block_quant");
}

template <int D>
int smooth_quant(const tmhd_attn_args *a, const tmhd_qk_quant *qq, hipStream_t s) {
  const int H = a->heads;
  int64_t total = 0;
  for (int i = 0; i < a->n_segments; ++i) total += a->seg[i].tokens;
  // 1. exact key sums, 2. bf16 mean
  // one segment table for the key passes; workgroup ranges per pass
  KeySegs ks{}, sums{};
  SumList given{};
  ks.n = a->n_segments;
  for (int i = 0; i < a->n_segments; ++i) {
    const tmhd_kv_segment &sg = a->seg[i];
    ks.k[i] = (const uint16_t *)sg.k;
    ks.khs[i] = sg.k_head_stride;
    ks.q8[i] = qq->k_i8[i];
    ks.q8hs[i] = qq->k_head_stride[i];
    ks.qs[i] = qq->k_scale[i];
    ks.qshs[i] = qq->k_scale_head_stride[i];
    ks.tokens[i] = sg.tokens;
    if (qq->k_sum[i]) {  // exact sums given by the caller (tmhd_k_fixed_sum)
      given.p[given.n++] = qq->k_sum[i];
    } else {
      sums.k[sums.n] = ks.k[i];
      sums.khs[sums.n] = ks.khs[i];
      sums.tokens[sums.n++] = sg.tokens;
    }
  }
  auto ranges = [](KeySegs &t, int per) {
    t.blk0[0] = 0;
    for (int i = 0; i < t.n; ++i) t.blk0[i + 1] = t.blk0[i] + (t.tokens[i] + per - 1) / per;
    return t.blk0[t.n];
  };
  hipLaunchKernelGGL(init_sum_kernel, dim3((H * D + 255) / 256), dim3(256), 0, s, qq->mean_workspace, given, H * D);
  if (sums.n) hipLaunchKernelGGL(k_sum_kernel<D>, dim3(ranges(sums, 256), H), dim3(256), 0, s, sums, qq->mean_workspace);
  hipLaunchKernelGGL(k_mean_finalize_kernel, dim3((H * D + 255) / 256), dim3(256), 0, s, qq->mean_workspace,
                     qq->k_mean, H * D, (double)total);
  if (int st = check_launch("smooth-K mean")) return st;
  // 3. keys, every segment in one launch (rows up to the 64-token tile padding are written)
  const int nblk = ranges(ks, TMHD_QUANT_BLOCK);
  hipLaunchKernelGGL(key_block_quant_kernel<D>, dim3(nblk, H), dim3(256), 0, s, ks, (const uint16_t *)qq->k_mean);
  if (int st = check_launch("block_quant keys")) return st;
  // 4. queries (rows up to the 256-row workgroup padding are written)
  const int qcap = (a->lq + 255) / 256 * 256;
  return launch_block_quant<D>((const uint16_t *)a->q, a->q_token_stride, a->q_head_stride, a->q_rows, a->q_row0,
                               nullptr, a->lq, qcap, qq->q_i8, qq->q_head_stride, qq->q_scale,
                               qq->q_scale_head_stride, H, s);
}

}  // namespace
}  // namespace tmhd

namespace tmhd {

int kv_pack(const void *k, const void *v, int64_t token_stride, int64_t head_stride, const int32_t *rows,
            int32_t row0, int32_t n, void *k_slot, void *vt_slot, int64_t k_head_stride, int64_t vt_head_stride,
            int32_t vt_row_stride, int32_t dst, int32_t zero_to, int32_t heads, int32_t head_dim, void *stream,
            bool with_k, bool check_only) {
  if (head_dim != 64 && head_dim != 128) return set_error(TMHD_ERR_UNSUPPORTED, "kv_pack: head_dim %d", head_dim);
  if (n < 0 || dst < 0 || heads <= 0) return set_error(TMHD_ERR_INVALID, "kv_pack: n %d dst %d heads %d", n, dst, heads);
  const int end = max(dst + n, zero_to);
  const int p_begin = dst / kTile * kTile;
  const int p_end = (end + kTile - 1) / kTile * kTile;
  if (p_end > vt_row_stride || vt_row_stride % kTile || (int64_t)vt_row_stride * head_dim > vt_head_stride ||
      (int64_t)p_end * head_dim > k_head_stride)
    return set_error(TMHD_ERR_INVALID, "kv_pack: positions [%d, %d) exceed the slot (cap %d)", p_begin, p_end,
                     vt_row_stride);
  if ((n > 0 && (!k || !v)) || !k_slot || !vt_slot || !aligned(k_slot, 16) || !aligned(vt_slot, 16) ||
      (n > 0 && (!aligned(k, 16) || !aligned(v, 16))) || token_stride % 8 || head_stride % 8 || k_head_stride % 8 ||
      vt_head_stride % 8)
    return set_error(TMHD_ERR_INVALID, "kv_pack: pointers and strides must be 16-byte aligned");
  if (check_only || p_end == p_begin) return TMHD_OK;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((p_end - p_begin) / kTile, heads);
#define TMHD_PACK(DIM, WK)                                                                                      \
  hipLaunchKernelGGL((kv_pack_kernel<DIM, WK>), grid, dim3(DIM), 0, s, (const uint16_t *)k, (const uint16_t *)v, \
                     token_stride, head_stride, rows, row0, n, (uint16_t *)k_slot, (uint16_t *)vt_slot,          \
                     k_head_stride, vt_head_stride, vt_row_stride, dst, zero_to, p_begin)
  if (head_dim == 128 && with_k)
    TMHD_PACK(128, true);
  else if (head_dim == 128)
    TMHD_PACK(128, false);
  else if (with_k)
    TMHD_PACK(64, true);
  else
    TMHD_PACK(64, false);
#undef TMHD_PACK
  return check_launch("tmhd_kv_pack");
}

}  // namespace tmhd

extern "C" int tmhd_kv_pack(const void *k, const void *v, int64_t token_stride, int64_t head_stride,
                            const int32_t *rows, int32_t row0, int32_t n, void *k_slot, void *vt_slot,
                            int64_t k_head_stride, int64_t vt_head_stride, int32_t vt_row_stride, int32_t dst,
                            int32_t zero_to, int32_t heads, int32_t head_dim, void *stream) {
  return tmhd::kv_pack(k, v, token_stride, head_stride, rows, row0, n, k_slot, vt_slot, k_head_stride, vt_head_stride,
                       vt_row_stride, dst, zero_to, heads, head_dim, stream, true, false);
}

extern "C" int tmhd_qk_smooth_quant(const tmhd_attn_args *args, const tmhd_qk_quant *quant, void *stream) {
  using namespace tmhd;
  if (!args || !quant) return set_error(TMHD_ERR_INVALID, "smooth_quant: null arguments");
  const int D = args->head_dim;
  if (D != 64 && D != 128) return set_error(TMHD_ERR_UNSUPPORTED, "smooth_quant: head_dim %d", D);
  if (args->n_segments < 1 || args->n_segments > kMaxSeg || args->heads <= 0 || args->lq < 0)
    return set_error(TMHD_ERR_INVALID, "smooth_quant: bad segment count / heads / lq");
  if (!quant->k_mean || !quant->mean_workspace || !quant->q_i8 || !quant->q_scale)
    return set_error(TMHD_ERR_INVALID, "smooth_quant: null output buffers");
  if (!aligned(quant->k_mean, 16) || !aligned(quant->mean_workspace, 8))
    return set_error(TMHD_ERR_INVALID, "smooth_quant: k_mean must be 16-byte and mean_workspace 8-byte aligned");
  const int qcap = (args->lq + 255) / 256 * 256;
  if (quant->q_head_stride < (int64_t)qcap * D || quant->q_scale_head_stride < qcap / TMHD_QUANT_BLOCK ||
      !aligned(quant->q_i8, 16) || quant->q_head_stride % 16)
    return set_error(TMHD_ERR_INVALID, "smooth_quant: quantized query buffer below round_up(lq, 256) rows");
  if (args->lq > 0 && (!args->q || !aligned(args->q, 16) || args->q_token_stride % 8 || args->q_head_stride % 8))
    return set_error(TMHD_ERR_INVALID, "smooth_quant: query pointer/strides must be 16-byte aligned");
  for (int i = 0; i < args->n_segments; ++i) {
    const tmhd_kv_segment &sg = args->seg[i];
    if (quant->k_sum[i] && !aligned(quant->k_sum[i], 8))
      return set_error(TMHD_ERR_INVALID, "smooth_quant: segment %d key sums must be 8-byte aligned", i);
    const int64_t cap = ((int64_t)sg.tokens + kTile - 1) / kTile * kTile;
    if (sg.tokens <= 0 || !sg.k || !aligned(sg.k, 16) || sg.k_head_stride < cap * D || sg.k_head_stride % 8)
      return set_error(TMHD_ERR_INVALID, "smooth_quant: segment %d keys are not a slot", i);
    if (!quant->k_i8[i] || !quant->k_scale[i] || !aligned(quant->k_i8[i], 16) || quant->k_head_stride[i] < cap * D ||
        quant->k_head_stride[i] % 16 ||
        quant->k_scale_head_stride[i] < (sg.tokens + TMHD_QUANT_BLOCK - 1) / TMHD_QUANT_BLOCK)
      return set_error(TMHD_ERR_INVALID, "smooth_quant: segment %d quantized key buffers too small", i);
  }
  hipStream_t s = (hipStream_t)stream;
  return D == 128 ? smooth_quant<128>(args, quant, s) : smooth_quant<64>(args, quant, s);
}

extern "C" int tmhd_k_fixed_sum(const void *k, int64_t k_head_stride, int32_t tokens, int32_t heads, int32_t head_dim,
                                int64_t *sum, void *stream) {
  using namespace tmhd;
  if (head_dim != 64 && head_dim != 128) return set_error(TMHD_ERR_UNSUPPORTED, "k_fixed_sum: head_dim %d", head_dim);
  if (tokens <= 0 || heads <= 0 || k_head_stride < (int64_t)tokens * head_dim || k_head_stride % 8)
    return set_error(TMHD_ERR_INVALID, "k_fixed_sum: tokens %d heads %d head stride %lld", tokens, heads,
                     (long long)k_head_stride);
  if (!k || !sum || !aligned(k, 16) || !aligned(sum, 8))
    return set_error(TMHD_ERR_INVALID, "k_fixed_sum: keys must be 16-byte and sums 8-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  KeySegs t{};
  t.n = 1;
  t.k[0] = (const uint16_t *)k;
  t.khs[0] = k_head_stride;
  t.tokens[0] = tokens;
  t.blk0[0] = 0;
  t.blk0[1] = (tokens + 255) / 256;
  hipLaunchKernelGGL(zero_i64_kernel, dim3((heads * head_dim + 255) / 256), dim3(256), 0, s, sum, heads * head_dim);
  if (head_dim == 128)
    hipLaunchKernelGGL(k_sum_kernel<128>, dim3(t.blk0[1], heads), dim3(256), 0, s, t, sum);
  else
    hipLaunchKernelGGL(k_sum_kernel<64>, dim3(t.blk0[1], heads), dim3(256), 0, s, t, sum);
  return check_launch("tmhd_k_fixed_sum");
}
