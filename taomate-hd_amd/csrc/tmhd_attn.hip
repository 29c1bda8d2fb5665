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
//   workgroup = 8 waves = 256 query rows of one head (one workgroup per CU,
//   two waves per SIMD); each wave owns 32 query rows and keeps them, their
//   fp32 output accumulators and the online-softmax state in registers
//   (<= 256 VGPRs).  Keys stream through LDS in 64-token tiles loaded with
//   global_load_lds_dwordx4 (no VGPR staging); K runs two tiles ahead of the
//   tile being finished and V one tile ahead, each double-buffered.
//   Scores are computed transposed, S^T = K Q^T, with v_mfma_f32_32x32x16_bf16
//   (or v_mfma_i32_32x32x32_i8), so each lane holds 16 keys of one query
//   column; the same registers, exponentiated and converted to bf16, are
//   directly the B operand of O^T += V^T P^T.  The value slot layout
//   (transposed, 4-token chunks interleaved) makes the matching A operand one
//   16-byte LDS read.  LDS rows are XOR-swizzled per 16-byte chunk so that
//   each 16-lane phase of a ds_read_b128 touches 16 distinct bank groups.
//
// Softmax in log2 units with a folded reference
//   BF16: the query is pre-scaled by scale*log2(e) (rounded to bf16 once) and
//   the score accumulator starts at -m (m = the column's running reference),
//   so the MFMA output is already the exponent: p = exp2(acc).
//   INT8: the int32 accumulator starts at 0x4B400000, so its bits read as the
//   float 1.5*2^23 + q.k exactly (|q.k| <= 127^2 * 128 < 2^22), and one FMA per
//   score applies the per-block dequantisation scale and -m.
//   The reference m only moves (and O, l are rescaled) when a tile's score
//   exceeds it by 2^8 (lazy rescale); P values stay <= 2^8.
//
// One loop iteration (tile j) is one basic block scheduled explicitly:
//   exp2 / pack / row-sum of P(j)        interleaved with QK(j+1)'s MFMAs,
//   max of S(j+1)                        interleaved with PV(j)'s MFMAs,
//   LDS operand reads issued two MFMAs ahead.
//   Rare work (partial tiles, rescale, segment switches) sits in branches
//   after the block.
#include <math.h>

#include <type_traits>

#include "tmhd_internal.h"

namespace tmhd {
namespace {

constexpr int kWaves = 8;
constexpr int kQW = 32;            // query rows per wave
constexpr int kBM = kWaves * kQW;  // query rows per workgroup
constexpr int kBN = 64;            // keys per tile
constexpr float kLazyRescale = 8.0f;
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kI8Magic = 0x4B400000;  // bits of 1.5 * 2^23
constexpr float kI8MagicF = 12582912.0f;

// sched_group_barrier instruction classes
constexpr int kSgMfma = 0x008;
constexpr int kSgValu = 0x002;
constexpr int kSgTrans = 0x400;
constexpr int kSgDsRead = 0x100;

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
  int32_t ntiles;  // sum of seg[].ntiles
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
// Issued as inline asm on purpose: the compiler's wait-count insertion cannot
// tell the destination block from the tiles being read and would place a
// vmcnt(0) wait in front of the next LDS read, serialising the prefetch.  The
// kernel itself waits (vmcnt(0) + barrier) before any read of a loaded tile;
// extra in-order vector-memory operations unknown to the compiler only make
// its own vmcnt waits stricter.
__device__ __forceinline__ void load_lds16(const void *gptr, void *lds) {
  const uint32_t m0v = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void *)lds;
  asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(gptr), "{m0}"(m0v) : "memory");
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

// Position of one head's tile stream: segment s, tile t of nt, with the
// segment's per-head base addresses.  All fields are wave-uniform (SGPRs).
struct Stream {
  int s, t, nt, tok;
  const char *kb;   // keys of tile 0 (bf16 or int8 rows)
  const char *vb;   // V^T row 0, token 0
  uint32_t vrs2;    // bytes per V^T row
  const float *ks;  // INT8: per-128-token key scales of this head
};

template <bool I8>
__device__ __forceinline__ void stream_set(Stream &S, const KArgs &a, int h, int s) {
  const Seg &G = a.seg[s];
  S.s = s;
  S.t = 0;
  S.nt = G.ntiles;
  S.tok = G.tokens;
  S.kb = I8 ? (const char *)(G.k8 + (int64_t)h * G.khs) : (const char *)(G.k + (int64_t)h * G.khs);
  S.vb = (const char *)(G.vt + (int64_t)h * G.vhs);
  S.vrs2 = (uint32_t)G.vrs * 2u;
  S.ks = I8 ? G.ks + (int64_t)h * G.kshs : nullptr;
}

// Next tile; the last tile of the last segment repeats (loads of a repeated
// tile are in-bounds and their results unused).
template <bool I8>
__device__ __forceinline__ void stream_next(Stream &S, const KArgs &a, int h) {
  if (++S.t >= S.nt) {
    if (S.s + 1 < a.nseg) {
      asm volatile("" ::: "memory");
      stream_set<I8>(S, a, h, S.s + 1);
    } else {
      S.t = S.nt - 1;
    }
  }
}

template <int D, bool I8>
__global__ void __launch_bounds__(kWaves * 64) __attribute__((amdgpu_waves_per_eu(2, 2))) attn_fwd_kernel(const KArgs a) {
  constexpr int KROW = I8 ? D : 2 * D;  // bytes per key row in memory
  constexpr int KCPR = KROW / 16;       // 16-byte chunks per key row
  constexpr int KRS = KROW + 16;        // LDS key row stride: one pad chunk, an odd number of chunks
  constexpr int KT = kBN * KRS;         // LDS key tile bytes
  constexpr int VRS = kBN * 2 + 16;     // LDS value row stride (64 keys + one pad chunk)
  constexpr int VT = D * VRS;           // LDS value tile bytes (D rows)
  constexpr int NKL = KT / 1024;        // 1 KiB wave loads per key tile
  constexpr int NVL = VT / 1024;
  static_assert(KT % 1024 == 0 && VT % 1024 == 0, "tiles are whole wave loads");
  constexpr int KWL = (NKL + kWaves - 1) / kWaves;  // per wave (some waves idle if NKL < waves)
  constexpr int VWL = (NVL + kWaves - 1) / kWaves;
  constexpr int QST = I8 ? D / 32 : D / 16;  // MFMA k-steps over head_dim
  constexpr int DB = D / 32;
  constexpr int NQK = 2 * QST;  // score MFMAs per tile
  constexpr int NPV = 4 * DB;   // output MFMAs per tile
  constexpr int LA = 4;         // LDS operand reads in flight ahead of their MFMA

  // four distinct LDS objects, so that the compiler can tell the tile being
  // loaded from the tiles being read (no vmcnt wait in front of the reads)
  __shared__ __attribute__((aligned(1024))) char kbuf0[KT];
  __shared__ __attribute__((aligned(1024))) char kbuf1[KT];
  __shared__ __attribute__((aligned(1024))) char vbuf0[VT];
  __shared__ __attribute__((aligned(1024))) char vbuf1[VT];
  auto kbuf = [&](int b) { return b ? kbuf1 : kbuf0; };
  auto vbuf = [&](int b) { return b ? vbuf1 : vbuf0; };

  // LDS layouts: a 16-lane ds_read_b128 phase reads one 16-byte chunk of 16
  // consecutive rows; those must fall on 16 distinct 16-byte positions modulo
  // 256 bytes.  Key and value rows are therefore padded to an odd number of
  // 16-byte chunks, and every operand read is one base register plus an
  // immediate offset.

  const int L = xcd_logical_id(blockIdx.x, gridDim.x);
  const int h = L / a.nqt;
  const int qt = L - h * a.nqt;
  const int tid = threadIdx.x, lane = tid & 63, lr = lane & 31, g = lane >> 5;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave index (uniform)
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
      for (int st = 0; st < QST; ++st) {
        const i32x4 raw = *(const i32x4 *)(p + st * 16);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t u = (uint32_t)raw[e];
          qv[st][e] = (int)pack_bf16x2(__uint_as_float(u << 16) * a.c, __uint_as_float(u & 0xffff0000u) * a.c);
        }
      }
    }
  } else {
#pragma unroll
    for (int st = 0; st < QST; ++st) qv[st] = i32x4{0, 0, 0, 0};
  }
  float cq = a.c;  // INT8: softmax scale * log2(e) * query block scale
  if constexpr (I8) cq = a.c * a.qs[(int64_t)h * a.qshs + (qt * kBM + w * kQW) / TMHD_QUANT_BLOCK];

  // per-lane LDS read offsets (bytes; k-step, 32-row half, buffer and db parts are immediates)
  const uint32_t kro = lr * KRS + g * 16;
  const uint32_t vro = lr * VRS + g * 16;

  // Tile loads.  LDS slot c (16 bytes) of a tile holds chunk c % (n + 1) of
  // row c / (n + 1) (n data chunks per row; the pad chunk repeats the row's
  // last chunk).  The per-lane offsets are recomputed at each load from the
  // lane id (kept opaque so they are not hoisted into registers that would
  // stay live across the scheduled block).
  auto slot_row_chunk = [&](int i, int n, int &row, int &chunk) {
    int l = lane;
    asm volatile("" : "+v"(l));
    const int c = (w + i * kWaves) * 64 + l;
    row = c / (n + 1);
    chunk = min(c - row * (n + 1), n - 1);
  };
  auto load_k = [&](const Stream &S, char *dst) {
    const char *base = S.kb + (int64_t)S.t * (kBN * KROW);
#pragma unroll
    for (int i = 0; i < KWL; ++i)
      if (NKL % kWaves == 0 || w + i * kWaves < NKL) {
        int row, chunk;
        slot_row_chunk(i, KCPR, row, chunk);
        load_lds16(base + (uint32_t)(row * KROW + chunk * 16), dst + (w + i * kWaves) * 1024);
      }
  };
  auto load_v = [&](const Stream &S, char *dst) {
    const char *base = S.vb + S.t * (kBN * 2);
#pragma unroll
    for (int i = 0; i < VWL; ++i)
      if (NVL % kWaves == 0 || w + i * kWaves < NVL) {
        int row, chunk;
        slot_row_chunk(i, 8, row, chunk);
        load_lds16(base + ((uint32_t)row * S.vrs2 + (uint32_t)chunk * 16), dst + (w + i * kWaves) * 1024);
      }
  };
  // INT8 key scale of a tile, read through the vector memory path (counted by
  // vmcnt, so the end-of-iteration wait covers it instead of an lgkmcnt wait
  // inside the scheduled block)
  auto load_ks = [&](const Stream &S) {
    int idx = S.t >> 1;  // 128-token quant blocks hold two tiles
    asm volatile("v_mov_b32 %0, %1" : "=v"(idx) : "s"(idx));
    return S.ks[idx];
  };

  // S^T = K Q^T for the 64 keys of a tile: lane holds keys 32kb + 8(r/4) + 4g + r%4
  auto qk = [&](const char *kb, const f32x16 &init, const i32x16 &init8, f32x16 (&sc)[2], float ct, float nb) {
    if constexpr (I8) {
      i32x16 ia[2] = {init8, init8};
#pragma unroll
      for (int kb32 = 0; kb32 < 2; ++kb32)
#pragma unroll
        for (int st = 0; st < QST; ++st)
          ia[kb32] = mfma_i8(*(const i32x4 *)(kb + kb32 * 32 * KRS + st * 32 + kro), qv[st], ia[kb32]);
#pragma unroll
      for (int kb32 = 0; kb32 < 2; ++kb32)
#pragma unroll
        for (int r = 0; r < 16; ++r) sc[kb32][r] = fmaf(__int_as_float(ia[kb32][r]), ct, nb);
    } else {
#pragma unroll
      for (int kb32 = 0; kb32 < 2; ++kb32) {
        sc[kb32] = init;
#pragma unroll
        for (int st = 0; st < QST; ++st)
          sc[kb32] = mfma_bf16(*(const i32x4 *)(kb + kb32 * 32 * KRS + st * 32 + kro), qv[st], sc[kb32]);
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
  auto lane_max = [](const f32x16 (&sc)[2]) {
    float m = fmaxf(sc[0][0], sc[0][1]);
#pragma unroll
    for (int r = 2; r < 16; r += 2) m = fmaxf(m, fmaxf(sc[0][r], sc[0][r + 1]));
#pragma unroll
    for (int r = 0; r < 16; r += 2) m = fmaxf(m, fmaxf(sc[1][r], sc[1][r + 1]));
    return m;
  };

  f32x16 o[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[db][r] = 0.0f;
  float lsum = 0.0f;
  f32x16 negm;  // BF16: -m in every element (the score accumulator's start value)
  i32x16 magic;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    negm[r] = 0.0f;
    magic[r] = kI8Magic;
  }

  // ---- prologue: K(0), V(0), K(1) resident; S = scores of tile 0
  Stream s0;
  stream_set<I8>(s0, a, h, 0);
  Stream sv = s0;  // V stream: tile j + 1 during iteration j
  stream_next<I8>(sv, a, h);
  Stream sk = sv;  // K stream: tile j + 2 during iteration j
  stream_next<I8>(sk, a, h);
  load_k(s0, kbuf(0));
  load_v(s0, vbuf(0));
  load_k(sv, kbuf(1));
  float ks_n = 0.0f, ks0 = 0.0f;  // INT8: key scale of tile j + 1
  if constexpr (I8) {
    ks0 = load_ks(s0);
    ks_n = load_ks(sv);
  }
  wait_vmem();
  __syncthreads();
  f32x16 sc[2];
  float mref;
  {
    const float ct0 = cq * ks0;
    qk(kbuf(0), negm, magic, sc, ct0, -kI8MagicF * ct0);
    if (s0.tok < kBN) mask_tail(sc, s0.tok);
    const float lm = lane_max(sc);
    mref = fmaxf(lm, __shfl_xor(lm, 32));
#pragma unroll
    for (int kb32 = 0; kb32 < 2; ++kb32) sc[kb32] -= mref;
    negm = -mref;
  }
  __syncthreads();  // every wave is done with K(0) before K(2) overwrites it

  const bf16x2 ones = {(__bf16)1.0f, (__bf16)1.0f};
  int j = 0;
  // iteration 0 loads K(2) and V(1)
  load_k(sk, kbuf(0));
  load_v(sv, vbuf(1));
  float ks_nn = 0.0f;  // INT8: key scale of tile j + 2
  if constexpr (I8) ks_nn = load_ks(sk);
  // One tile; B = j & 1 selects the buffers statically.  Returns false after the last tile.
  auto iter = [&](auto par) -> bool {
    constexpr int B = decltype(par)::value;
    const float ct_n = cq * ks_n;
    const float nb_n = -fmaf(kI8MagicF, ct_n, mref);

    // The block below is software-pipelined by hand in NS slots, fenced so
    // that the compiler keeps the order: slot i issues the LDS operand read of
    // MFMA i + LA, runs MFMA i and a fixed share of the VALU work.
    //   slots [0, NQK):  S(j+1) = K Q^T (key half kb32 = i / QST, k-step st),
    //                    under P(j) = exp2(S(j)) -> bf16 pairs and row sums;
    //   slots [NQK, NS): O^T += V^T P^T (kb32, st, db), under the row maxima
    //                    of S(j+1) (INT8: after its dequantisation).
    // After the last tile the score MFMAs read a stale in-bounds buffer and
    // their result is unused.
    constexpr int NS = NQK + NPV;
    constexpr int PPS = 16 / NQK;  // P pairs per score slot
    constexpr int MPS = 16 / NPV;  // max pairs per output slot
    auto read_op = [&](int i) -> i32x4 {
      if (i < NQK) {
        const int kb32 = i / QST, st = i % QST;
        return *(const i32x4 *)(kbuf(B ^ 1) + kb32 * 32 * KRS + st * 32 + kro);
      }
      const int pv = i - NQK, kb32 = pv / (2 * DB), st = (pv / DB) & 1, db = pv % DB;
      return *(const i32x4 *)(vbuf(B) + db * 32 * VRS + (4 * kb32 + 2 * st) * 16 + vro);
    };
    i32x4 ops[NS];
    i32x4 pkv[2][2];  // P(j) as bf16 pairs: [kb32][st] = keys 16 st .. of the half, 4 dwords
    float ts = 0.0f;
    f32x16 sn[2];
    i32x16 sni[2];
    float lm = -INFINITY;
#pragma unroll
    for (int i = 0; i < LA; ++i) ops[i] = read_op(i);
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      if (i + LA < NS) ops[i + LA] = read_op(i + LA);
      if (i < NQK) {
        const int kb32 = i / QST, st = i % QST;
        if constexpr (I8) {
          sni[kb32] = mfma_i8(ops[i], qv[st], st == 0 ? magic : sni[kb32]);
        } else {
          sn[kb32] = mfma_bf16(ops[i], qv[st], st == 0 ? negm : sn[kb32]);
        }
#pragma unroll
        for (int u = 0; u < PPS; ++u) {
          const int q = i * PPS + u, pk32 = q >> 3, r = (q & 7) * 2;
          const uint32_t pr =
              pack_bf16x2(__builtin_amdgcn_exp2f(sc[pk32][r]), __builtin_amdgcn_exp2f(sc[pk32][r + 1]));
          pkv[pk32][(q >> 2) & 1][q & 3] = (int)pr;
          ts = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pr), ones, ts, false);
        }
      } else {
        const int pv = i - NQK, kb32 = pv / (2 * DB), st = (pv / DB) & 1, db = pv % DB;
        o[db] = mfma_bf16(ops[i], pkv[kb32][st], o[db]);
#pragma unroll
        for (int u = 0; u < MPS; ++u) {
          const int q = pv * MPS + u, m32 = q >> 3, r = (q & 7) * 2;
          if constexpr (I8) {
            sn[m32][r] = fmaf(__int_as_float(sni[m32][r]), ct_n, nb_n);
            sn[m32][r + 1] = fmaf(__int_as_float(sni[m32][r + 1]), ct_n, nb_n);
          }
          lm = fmaxf(lm, fmaxf(sn[m32][r], sn[m32][r + 1]));
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    lsum += ts;

    if (++j >= a.ntiles) return false;
    // tile j (the new current tile) is the last, partial tile of its segment
    const int nv = sv.tok - sv.t * kBN;
    if (nv < kBN) {
      asm volatile("" ::: "memory");
      mask_tail(sn, nv);
      lm = lane_max(sn);
    }
    if (__any(lm > kLazyRescale)) {
      const float cm = fmaxf(lm, __shfl_xor(lm, 32));
      const float delta = fmaxf(cm, 0.0f);
      const float alpha = __builtin_amdgcn_exp2f(-delta);
      lsum *= alpha;
#pragma unroll
      for (int db = 0; db < DB; ++db) o[db] *= alpha;
#pragma unroll
      for (int kb32 = 0; kb32 < 2; ++kb32) sn[kb32] -= delta;
      mref += delta;
      negm = -mref;
    }
    sc[0] = sn[0];
    sc[1] = sn[1];
    ks_n = ks_nn;
    sv = sk;
    stream_next<I8>(sk, a, h);
    wait_vmem();
    __syncthreads();
    // K(j+3) into the buffer K(j+1) used, V(j+2) into the buffer V(j) used
    load_k(sk, kbuf(B ^ 1));
    load_v(sv, vbuf(B));
    if constexpr (I8) ks_nn = load_ks(sk);
    return true;
  };
  for (;;) {
    if (!iter(std::integral_constant<int, 0>{})) break;
    if (!iter(std::integral_constant<int, 1>{})) break;
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
    k->ntiles += S.ntiles;
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
