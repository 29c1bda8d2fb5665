// Streaming attention forward for gfx950: softmax(q k^T * scale) v over a
// table of key/value segments held in slot format (see tmhd.h), no mask.
//
// Reference semantics: torch SDPA over the concatenated K/V parts in
// src/taomate_hd/streaming/attention_hook.py:100-115 (BF16 path) and the
// SageAttention call at :335-371 (INT8-QK path).  Attention without a mask is
// invariant to the order of keys, so segments are visited in place in table
// order and never concatenated.
//
// Work decomposition
//   workgroup = 4 waves = 128 query rows of one head; each wave owns 32 rows
//   and keeps them, their fp32 output accumulators and the online-softmax
//   state in registers (<= 256 VGPRs, two workgroups per CU, so two waves
//   share each SIMD and the hardware overlaps one wave's softmax with the
//   other's MFMAs).  Keys stream through LDS in 64-token tiles loaded with
//   global_load_lds_dwordx4 (no VGRP staging), double-buffered: the next
//   tile's loads are in flight while the current tile is computed.
//   Scores are computed transposed, S^T = K Q^T, with v_mfma_f32_32x32x16_bf16
//   (or v_mfma_i32_32x32x32_i8), so each lane holds 16 keys of one query
//   column; the same registers, converted to bf16, are directly the B operand
//   of O^T += V^T P^T.  The value slot layout (transposed, 4-token chunks
//   interleaved) makes the matching A operand one 16-byte LDS read.
//   LDS rows are XOR-swizzled per 16-byte chunk so that each 16-lane phase of
//   a ds_read_b128 touches 16 distinct 16-byte bank groups.
//   Online softmax works in log2 units with a lazy rescale: the running max
//   is only moved (and O, l rescaled) when a tile exceeds it by 2^8.
#include <math.h>

#include "tmhd_internal.h"

namespace tmhd {
namespace {

constexpr int kWaves = 8;
constexpr int kQW = 32;            // query rows per wave
constexpr int kBM = kWaves * kQW;  // query rows per workgroup
constexpr int kBN = 64;            // keys per tile
constexpr float kLazyRescale = 8.0f;
constexpr float kLog2e = 1.4426950408889634f;

struct Seg {
  const uint16_t *k;
  const uint16_t *vt;
  const int8_t *k8;
  const float *ks;
  int64_t khs;
  int64_t vhs;
  int32_t vrs;
  int32_t tokens;
  int32_t kshs;
  int32_t ntiles;
};

struct KArgs {
  const uint16_t *q;
  int64_t qts, qhs;
  const int32_t *q_rows;
  int32_t q_row0, lq;
  uint16_t *o;
  int64_t ots, ohs;
  const int32_t *o_rows;
  int32_t o_row0;
  const int8_t *q8;
  const float *qs;
  int64_t q8hs;
  int32_t qshs;
  int32_t heads, nqt;
  float c;  // softmax scale * log2(e)
  int32_t nseg;
  Seg seg[kMaxSeg];
};

__device__ __forceinline__ f32x16 mfma_bf16(i32x4 a, i32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

__device__ __forceinline__ i32x16 mfma_i8(i32x4 a, i32x4 b, i32x16 c) {
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  bf16x2 v = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, v);
}

// 16 bytes global -> LDS without a VGPR round trip.  `lds` is the wave's
// 1 KiB destination block; lane i's bytes land at lds + 16 * i.
__device__ __forceinline__ void load_lds16(const void *gptr, void *lds) {
  __builtin_amdgcn_global_load_lds(gptr, (__attribute__((address_space(3))) void *)lds, 16, 0, 0);
}

__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0f70); }  // vmcnt(0)

// Maps the linear workgroup id so that consecutive logical ids run on the same
// XCD (the hardware deals workgroups round-robin over the 8 XCDs).  Logical
// ids are head-major, so the workgroups that share one head's keys and values
// share that XCD's L2.
__device__ __forceinline__ int xcd_logical_id(int b, int G) {
  const int xcd = b & 7, pos = b >> 3, per = G >> 3, rem = G & 7;
  return xcd < rem ? xcd * (per + 1) + pos : rem * (per + 1) + (xcd - rem) * per + pos;
}

// Iterator over the (segment, tile) sequence of a call.
struct TileIt {
  int s, t;
  __device__ __forceinline__ void next(const KArgs &a) {
    if (++t >= a.seg[s].ntiles) {
      ++s;
      t = 0;
    }
  }
};

template <int D, bool I8>
__global__ void __launch_bounds__(kWaves * 64) __attribute__((amdgpu_waves_per_eu(2, 2))) attn_fwd_kernel(const KArgs a) {
  constexpr int KROW = I8 ? D : 2 * D;  // bytes per key row
  constexpr int KCPR = KROW / 16;       // 16-byte chunks per key row
  constexpr int KRP = 256 / KROW;       // key rows per 256 bytes (one bank sweep)
  constexpr int KT = kBN * KROW;        // key tile bytes
  constexpr int VT = D * kBN * 2;       // value tile bytes (D rows of 64 keys)
  constexpr int NKL = KT / 1024;           // 1 KiB wave loads per key tile
  constexpr int NVL = VT / 1024;
  constexpr int KWL = (NKL + kWaves - 1) / kWaves;  // per wave (some waves idle if NKL < waves)
  constexpr int VWL = (NVL + kWaves - 1) / kWaves;
  constexpr int QST = I8 ? D / 32 : D / 16;  // MFMA k-steps over head_dim
  constexpr int DB = D / 32;

  // K and V have separate double buffers: K runs one tile ahead of V
  __shared__ __attribute__((aligned(1024))) char kbuf[2][KT];
  __shared__ __attribute__((aligned(1024))) char vbuf[2][VT];

  // chunk swizzles: 16 consecutive rows (one 16-lane ds_read_b128 phase) hit
  // 16 distinct 16-byte positions modulo 256 bytes
  auto kswz = [](int row) { return (row / KRP) & (KCPR - 1); };
  auto vswz = [](int row) { return (row >> 1) & 7; };

  const int L = xcd_logical_id(blockIdx.x, gridDim.x);
  const int h = L / a.nqt;
  const int qt = L - h * a.nqt;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, lr = lane & 31, g = lane >> 5;
  const int ql = qt * kBM + w * kQW + lr;  // this lane's query column

  // ---- query operand (B operand of S^T = K Q^T), resident for the whole call
  i32x4 qv[QST];
  if (ql < a.lq) {
    if constexpr (I8) {
      const int8_t *p = a.q8 + (int64_t)h * a.q8hs + (int64_t)ql * D + g * 16;
#pragma unroll
      for (int st = 0; st < QST; ++st) qv[st] = *(const i32x4 *)(p + st * 32);
    } else {
      const int row = a.q_rows ? a.q_rows[ql] : a.q_row0 + ql;
      const uint16_t *p = a.q + (int64_t)row * a.qts + (int64_t)h * a.qhs + g * 8;
#pragma unroll
      for (int st = 0; st < QST; ++st) qv[st] = *(const i32x4 *)(p + st * 16);
    }
  } else {
#pragma unroll
    for (int st = 0; st < QST; ++st) qv[st] = i32x4{0, 0, 0, 0};
  }
  float qscale = 1.0f;
  if constexpr (I8) qscale = a.qs[(int64_t)h * a.qshs + (qt * kBM + w * kQW) / TMHD_QUANT_BLOCK];

  // per-lane byte offsets of this thread's tile loads (tile-invariant)
  uint32_t koff[KWL], vrow[VWL], vchk[VWL];
#pragma unroll
  for (int i = 0; i < KWL; ++i) {
    const int c = (w + i * kWaves) * 64 + lane, row = c / KCPR;
    koff[i] = row * KROW + ((c % KCPR) ^ kswz(row)) * 16;
  }
#pragma unroll
  for (int i = 0; i < VWL; ++i) {
    const int c = (w + i * kWaves) * 64 + lane, row = c >> 3;
    vrow[i] = row;
    vchk[i] = ((c & 7) ^ vswz(row)) * 16;
  }
  auto load_k = [&](TileIt it, int buf) {
    const Seg &S = a.seg[it.s];
    const char *base = I8 ? (const char *)(S.k8 + (int64_t)h * S.khs + (int64_t)it.t * kBN * D)
                          : (const char *)(S.k + (int64_t)h * S.khs + (int64_t)it.t * kBN * D);
#pragma unroll
    for (int i = 0; i < KWL; ++i)
      if (NKL % kWaves == 0 || w + i * kWaves < NKL)
        load_lds16(base + koff[i], &kbuf[buf][(w + i * kWaves) * 1024]);
  };
  auto load_v = [&](TileIt it, int buf) {
    const Seg &S = a.seg[it.s];
    const char *base = (const char *)(S.vt + (int64_t)h * S.vhs + it.t * kBN);
    const uint32_t rs = (uint32_t)S.vrs * 2;
#pragma unroll
    for (int i = 0; i < VWL; ++i)
      if (NVL % kWaves == 0 || w + i * kWaves < NVL)
        load_lds16(base + (vrow[i] * rs + vchk[i]), &vbuf[buf][(w + i * kWaves) * 1024]);
  };
  // S^T = K Q^T for the 64 keys of a tile: lane holds keys 32kb + 8(r/4) + 4g + r%4
  auto qk = [&](int buf, f32x16 (&sc)[2]) {
#pragma unroll
    for (int kb32 = 0; kb32 < 2; ++kb32) {
      const int krow = kb32 * 32 + lr;
      const char *kp = &kbuf[buf][krow * KROW];
      if constexpr (I8) {
        i32x16 ia;
#pragma unroll
        for (int r = 0; r < 16; ++r) ia[r] = 0;
#pragma unroll
        for (int st = 0; st < QST; ++st)
          ia = mfma_i8(*(const i32x4 *)(kp + ((2 * st + g) ^ kswz(krow)) * 16), qv[st], ia);
#pragma unroll
        for (int r = 0; r < 16; ++r) sc[kb32][r] = (float)ia[r];
      } else {
        f32x16 acc;
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
#pragma unroll
        for (int st = 0; st < QST; ++st)
          acc = mfma_bf16(*(const i32x4 *)(kp + ((2 * st + g) ^ kswz(krow)) * 16), qv[st], acc);
        sc[kb32] = acc;
      }
    }
  };
  auto mask_tail = [&](f32x16 (&sc)[2], int nvalid) {
#pragma unroll
    for (int kb32 = 0; kb32 < 2; ++kb32)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (kb32 * 32 + 8 * (r >> 2) + 4 * g + (r & 3) >= nvalid) sc[kb32][r] = -INFINITY;
  };
  auto tile_scale = [&](TileIt it) {
    float ct = a.c;
    if constexpr (I8) {
      const Seg &S = a.seg[it.s];
      // a zero-scale block must not turn a masked -inf logit into NaN
      ct = fmaxf(a.c * qscale * S.ks[(int64_t)h * S.kshs + (it.t * kBN) / TMHD_QUANT_BLOCK], 1e-30f);
    }
    return ct;
  };

  f32x16 o[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[db][r] = 0.0f;
  float mref = -INFINITY;
  float lsum = 0.0f;

  // ---- prologue: K(0), V(0), K(1) resident; S = scores of tile 0
  TileIt cur{0, 0}, n1 = cur, n2;
  n1.next(a);
  n2 = n1;
  if (n2.s < a.nseg) n2.next(a);
  load_k(cur, 0);
  load_v(cur, 0);
  if (n1.s < a.nseg) load_k(n1, 1);
  wait_vmem();
  __syncthreads();
  f32x16 sc[2];
  qk(0, sc);
  {
    const int nv = a.seg[0].tokens;
    if (nv < kBN) mask_tail(sc, nv);
  }
  __syncthreads();  // every wave is done with K(0) before K(2) overwrites it

  for (int j = 0;; ++j) {
    const int kb_cur = j & 1;
    const bool has1 = n1.s < a.nseg;
    const bool has2 = n2.s < a.nseg;
    if (has2) load_k(n2, kb_cur);        // K(j+2) into the buffer K(j) used
    if (has1) load_v(n1, kb_cur ^ 1);    // V(j+1) into the buffer V(j-1) used
    const float ct = tile_scale(cur);

    // online softmax of tile j (log2 units, lazy rescale)
    float m = sc[0][0];
#pragma unroll
    for (int r = 1; r < 16; ++r) m = fmaxf(m, sc[0][r]);
#pragma unroll
    for (int r = 0; r < 16; ++r) m = fmaxf(m, sc[1][r]);
    m = fmaxf(m, __shfl_xor(m, 32));
    const float cand = m * ct;
    if (__any(cand > mref + kLazyRescale)) {
      const float mn = fmaxf(mref, cand);
      const float alpha = (mref == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mref - mn);
      lsum *= alpha;
#pragma unroll
      for (int db = 0; db < DB; ++db) o[db] *= alpha;
      mref = mn;
    }
    const float nm = -mref;
    uint32_t pk[2][8];
    const bf16x2 ones = {(__bf16)1.0f, (__bf16)1.0f};
#pragma unroll
    for (int kb32 = 0; kb32 < 2; ++kb32) {
#pragma unroll
      for (int r = 0; r < 16; r += 2)
        pk[kb32][r >> 1] = pack_bf16x2(__builtin_amdgcn_exp2f(fmaf(sc[kb32][r], ct, nm)),
                                       __builtin_amdgcn_exp2f(fmaf(sc[kb32][r + 1], ct, nm)));
#pragma unroll
      for (int i = 0; i < 8; ++i)
        lsum = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pk[kb32][i]), ones, lsum, false);
    }
    // scores of tile j+1 (independent of the softmax above: overlappable).
    // Computed unconditionally so that this block stays one scheduling
    // region; after the last tile it reads a stale (in-bounds) buffer and
    // the result is dropped.
    f32x16 sn[2];
    qk(kb_cur ^ 1, sn);
    // O^T += V^T P^T for tile j, 16 keys per MFMA
#pragma unroll
    for (int kb32 = 0; kb32 < 2; ++kb32) {
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        const i32x4 pb = {(int)pk[kb32][4 * st], (int)pk[kb32][4 * st + 1], (int)pk[kb32][4 * st + 2],
                          (int)pk[kb32][4 * st + 3]};
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          const int vrow_ = db * 32 + lr;
          const i32x4 vv = *(const i32x4 *)(&vbuf[kb_cur][vrow_ * 128 + ((4 * kb32 + 2 * st + g) ^ vswz(vrow_)) * 16]);
          o[db] = mfma_bf16(vv, pb, o[db]);
        }
      }
    }
    if (!has1) break;
    {
      const int nv = a.seg[n1.s].tokens - n1.t * kBN;
      if (nv < kBN) mask_tail(sn, nv);
    }
    sc[0] = sn[0];
    sc[1] = sn[1];
    cur = n1;
    n1 = n2;
    if (has2) n2.next(a);
    wait_vmem();
    __syncthreads();
  }

  // ---- epilogue: O = O^T / l, written token-major (4 consecutive d per store)
  const float lt = lsum + __shfl_xor(lsum, 32);
  const float inv = 1.0f / lt;
  if (ql < a.lq) {
    const int row = a.o_rows ? a.o_rows[ql] : a.o_row0 + ql;
    uint16_t *op = a.o + (int64_t)row * a.ots + (int64_t)h * a.ohs + 4 * g;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        i32x2 pr = {(int)pack_bf16x2(o[db][4 * u] * inv, o[db][4 * u + 1] * inv),
                    (int)pack_bf16x2(o[db][4 * u + 2] * inv, o[db][4 * u + 3] * inv)};
        *(i32x2 *)(op + db * 32 + 8 * u) = pr;
      }
  }
}

bool aligned(const void *p, int bytes) { return ((uintptr_t)p % bytes) == 0; }

int build_kargs(const tmhd_attn_args *args, const tmhd_qk_quant *qq, bool i8, KArgs *k) {
  if (!args) return set_error(TMHD_ERR_INVALID, "attention: null args");
  const int D = args->head_dim;
  if (D != 64 && D != 128) return set_error(TMHD_ERR_UNSUPPORTED, "attention: head_dim %d (64 or 128)", D);
  if (args->heads <= 0 || args->lq < 0) return set_error(TMHD_ERR_INVALID, "attention: heads %d lq %d", args->heads, args->lq);
  if (args->n_segments < 1 || args->n_segments > kMaxSeg)
    return set_error(TMHD_ERR_INVALID, "attention: n_segments %d not in [1, %d]", args->n_segments, kMaxSeg);
  if (!(args->scale > 0.0f) || !isfinite(args->scale)) return set_error(TMHD_ERR_INVALID, "attention: scale must be > 0");
  if (!args->o || !aligned(args->o, 8) || args->o_token_stride % 4 || args->o_head_stride % 4)
    return set_error(TMHD_ERR_INVALID, "attention: output pointer/strides must be 8-byte aligned");
  if (!i8 && (!args->q || !aligned(args->q, 16) || args->q_token_stride % 8 || args->q_head_stride % 8))
    return set_error(TMHD_ERR_INVALID, "attention: query pointer/strides must be 16-byte aligned");
  const int nqt = (args->lq + kBM - 1) / kBM;
  *k = KArgs{};
  k->q = (const uint16_t *)args->q;
  k->qts = args->q_token_stride;
  k->qhs = args->q_head_stride;
  k->q_rows = args->q_rows;
  k->q_row0 = args->q_row0;
  k->lq = args->lq;
  k->o = (uint16_t *)args->o;
  k->ots = args->o_token_stride;
  k->ohs = args->o_head_stride;
  k->o_rows = args->o_rows;
  k->o_row0 = args->o_row0;
  k->heads = args->heads;
  k->nqt = nqt;
  k->c = args->scale * kLog2e;
  k->nseg = args->n_segments;
  if (i8) {
    if (!qq || !qq->q_i8 || !qq->q_scale || !aligned(qq->q_i8, 16) || qq->q_head_stride % 16)
      return set_error(TMHD_ERR_INVALID, "attention i8: bad quantized query buffers");
    if (qq->q_head_stride < (int64_t)nqt * kBM * D || qq->q_scale_head_stride < nqt * (kBM / TMHD_QUANT_BLOCK))
      return set_error(TMHD_ERR_INVALID, "attention i8: quantized query capacity below round_up(lq, 256)");
    k->q8 = qq->q_i8;
    k->qs = qq->q_scale;
    k->q8hs = qq->q_head_stride;
    k->qshs = qq->q_scale_head_stride;
  }
  for (int i = 0; i < args->n_segments; ++i) {
    const tmhd_kv_segment &sg = args->seg[i];
    const int64_t cap = ((int64_t)sg.tokens + kBN - 1) / kBN * kBN;
    if (sg.tokens <= 0) return set_error(TMHD_ERR_INVALID, "attention: segment %d has %d tokens", i, sg.tokens);
    if (!sg.k || !sg.vt || !aligned(sg.k, 16) || !aligned(sg.vt, 16))
      return set_error(TMHD_ERR_INVALID, "attention: segment %d pointers must be 16-byte aligned", i);
    if (sg.vt_row_stride % kBN || sg.vt_row_stride < cap || sg.vt_head_stride < (int64_t)D * sg.vt_row_stride ||
        sg.k_head_stride < cap * D || sg.vt_head_stride % 8 || sg.k_head_stride % 8)
      return set_error(TMHD_ERR_INVALID,
                       "attention: segment %d is not a slot (tokens %d, vt_row_stride %d, strides %lld/%lld)", i,
                       sg.tokens, sg.vt_row_stride, (long long)sg.k_head_stride, (long long)sg.vt_head_stride);
    Seg &S = k->seg[i];
    S.k = (const uint16_t *)sg.k;
    S.vt = (const uint16_t *)sg.vt;
    S.khs = sg.k_head_stride;
    S.vhs = sg.vt_head_stride;
    S.vrs = sg.vt_row_stride;
    S.tokens = sg.tokens;
    S.ntiles = (int)(cap / kBN);
    if (i8) {
      if (!qq->k_i8[i] || !qq->k_scale[i] || !aligned(qq->k_i8[i], 16) || qq->k_head_stride[i] < cap * D ||
          qq->k_head_stride[i] % 16 || qq->k_scale_head_stride[i] < (cap + TMHD_QUANT_BLOCK - 1) / TMHD_QUANT_BLOCK)
        return set_error(TMHD_ERR_INVALID, "attention i8: bad quantized key buffers for segment %d", i);
      S.k8 = qq->k_i8[i];
      S.ks = qq->k_scale[i];
      S.khs = qq->k_head_stride[i];
      S.kshs = qq->k_scale_head_stride[i];
    }
  }
  return TMHD_OK;
}

template <bool I8>
int launch_attn(const tmhd_attn_args *args, const tmhd_qk_quant *qq, void *stream) {
  KArgs k;
  int st = build_kargs(args, qq, I8, &k);
  if (st) return st;
  if (args->lq == 0) return TMHD_OK;
  const int64_t grid = (int64_t)k.nqt * k.heads;
  if (grid > 0x7fffffff) return set_error(TMHD_ERR_UNSUPPORTED, "attention: grid too large");
  hipStream_t s = (hipStream_t)stream;
  if (args->head_dim == 128)
    hipLaunchKernelGGL((attn_fwd_kernel<128, I8>), dim3((unsigned)grid), dim3(kWaves * 64), 0, s, k);
  else
    hipLaunchKernelGGL((attn_fwd_kernel<64, I8>), dim3((unsigned)grid), dim3(kWaves * 64), 0, s, k);
  return check_launch(I8 ? "tmhd_attn_fwd_i8qk" : "tmhd_attn_fwd_bf16");
}

}  // namespace
}  // namespace tmhd

extern "C" int tmhd_attn_fwd_bf16(const tmhd_attn_args *args, void *stream) {
  return tmhd::launch_attn<false>(args, nullptr, stream);
}

extern "C" int tmhd_attn_fwd_i8qk(const tmhd_attn_args *args, const tmhd_qk_quant *quant, void *stream) {
  return tmhd::launch_attn<true>(args, quant, stream);
}
