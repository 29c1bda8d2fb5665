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
//   workgroup = 4 waves = 256 query rows of one head, one workgroup per CU and
//   one wave per SIMD.  Each wave owns 64 query rows (two 32-row halves) and
//   keeps their query operands and fp32 output accumulators in AGPRs at fixed
//   registers, the score chain starts (BF16: -m per half) at fixed VGPRs
//   v[224:255], and the scores, probabilities and online-softmax state in
//   the other VGPRs.  Fixed registers keep the compiler from moving these
//   long-lived values around the loop.
//   Keys and values stream through LDS in 64-token tiles, triple-buffered
//   (tile t in buffer t % 3) and loaded with global_load_lds_dwordx4 (no
//   VGPR staging): K runs two tiles ahead of the tile being finished, V one.
//   Scores are computed transposed, S^T = K Q^T, with v_mfma_f32_32x32x16_bf16
//   (or v_mfma_i32_32x32x32_i8), so each lane holds 16 keys of one query
//   column; the same registers, exponentiated and converted to bf16, are
//   directly the B operand of O^T += V^T P^T.  The value slot layout
//   (transposed, 4-token chunks interleaved) makes the matching A operand one
//   16-byte LDS read.  LDS rows are padded to an odd number of 16-byte chunks
//   so that each 16-lane phase of a ds_read_b128 touches 16 distinct bank
//   groups and every operand read is one base register plus an immediate.
//
// Softmax in log2 units with a folded reference
//   BF16: the query is pre-scaled by scale*log2(e) (rounded to bf16 once) and
//   the score accumulator starts at -m (m = the column's running reference),
//   so the MFMA output is already the exponent: p = exp2(acc).
//   INT8: the int32 accumulator starts at the MFMA's inline constant 1/(2 pi),
//   bits 0x3E22F983, so its bits read as the float 0x1.45f306p-3 + q.k * 2^-26
//   exactly (the mantissa 0x22F983 = 2,292,099 exceeds |q.k| <= 128^3), and
//   one FMA per score applies the per-block dequantisation scale and -m.
//   The reference m only moves (and O, l are rescaled) when a tile's score
//   exceeds it by 2^8 (lazy rescale); P values stay <= 2^8.
//
// Pipeline: a tile is two 32-key sub-tiles; each sub-tile is one basic block
// of fenced slots, each slot one LDS operand read (issued four slots ahead)
// and two MFMAs (one per query half).  Issuing an MFMA holds the wave for
// about half of the MFMA's 32 cycles, so every MFMA is followed by its own
// share of the other work, spread by a compile-time plan that evens out the
// issue cycles between consecutive MFMAs:
//   exp2 / pack / row-sum of P(s)      under the score MFMAs of sub-tile s+1
//                                      and the first P.V MFMAs of sub-tile s,
//   scaling and row max of S(s+1)      under the later P.V MFMAs of sub-tile s,
//   the tile loads of the iteration    in the first sub-tile's slots.
// The last slots read the first operands of the next sub-tile.  Rare work
// (partial tiles, rescale, segment switches) sits in branches after the block.
// Scores of consecutive sub-tiles alternate between two register sets.
#include <math.h>

#include <mutex>
#include <type_traits>

#include "tmhd_internal.h"

// Scratch of tmhd_attn_fwd_bf16_noalloc: the key-range partials of a split
// last round, sized for one [256 rows][128 + 1] fp32 slot per CU of a
// 256-CU device (33,816,576 bytes, held by every device the library runs on
// until the process ends).  Host code reaches it only through the address
// hipGetSymbolAddress gives per device (static_scratch below).
static __device__ __align__(256) unsigned char scratch[256 * 256 * (128 + 1) * 4];

namespace tmhd {
namespace {

constexpr int kWaves = 4;
constexpr int kQW = 64;            // query rows per wave (two 32-row halves)
constexpr int kBM = kWaves * kQW;  // query rows per workgroup
constexpr int kBN = 64;            // keys per tile
constexpr float kLazyRescale = 8.0f;
constexpr float kLog2e = 1.4426950408889634f;
// INT8 score chain start: the inline constant 1/(2 pi) of the integer MFMA
// adds its bits, 0x3E22F983, to q.k; read as a float the sum is
// kI8MagicF + q.k * 2^-26 while |q.k| < 0x22F983
constexpr float kI8MagicF = 0x1.45f306p-3f;
constexpr float kI8Slope = 0x1p-26f;

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
  // Items (head, query tile) [0, full) run whole, one per workgroup; the
  // remaining ones run as nsplit key ranges each, whose partial results
  // (per workgroup: [kBM][D] normalised O, then [kBM] log2-sum-exp) go to ws.
  int32_t full, nsplit;
  float *ws;
  Seg seg[kMaxSeg];
};

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  bf16x2 v = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, v);
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

// Tile gt of the concatenated segments.
template <bool I8>
__device__ __forceinline__ void stream_seek(Stream &S, const KArgs &a, int h, int gt) {
  int s = 0;
  while (s + 1 < a.nseg && gt >= a.seg[s].ntiles) gt -= a.seg[s++].ntiles;
  stream_set<I8>(S, a, h, s);
  S.t = gt;
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

// ---- MFMA wrappers.  All MFMAs of the kernel are inline asm so that the
// query operands and the output accumulators can live in AGPRs (1 wave per
// SIMD, up to 512 registers) while scores and probabilities stay in VGPRs.
// The compiler does not see through the asm, so the hazards it would resolve
// for builtins are resolved by construction in the kernel:
//   * VALU write -> MFMA operand read needs 2 wait states: a P.V MFMA whose
//     P group was packed in front of the previous MFMA carries an s_nop 1;
//   * MFMA result -> VALU read (12 wait states for either MFMA): score results
//     are first read behind an s_nop 10 after the second output MFMA, which
//     names them so that no read moves above it; AGPR accumulators are read
//     only after mfma_drain();
//   * accvgpr write (rescale) -> MFMA accumulate: s_nop 2 after the rescale;
//   * the rescale itself reads each AGPR after mfma_drain();
//   * back-to-back accumulation into the same registers needs no wait states.
// Output registers of the first MFMA of a score chain are early-clobber, so
// they never overlap the operands.
// Query operand block qb (4 dwords per lane) lives in the fixed AGPRs
// a[128 + 4 qb, 128 + 4 qb + 3]; the score MFMAs name that range.
#define TMHD_QBLK(QB, LO, HI)                                                                                \
  case QB:                                                                                                   \
    asm volatile("" : "+{a[" #LO ":" #HI "]}"(q));                                                           \
    break;
__device__ __forceinline__ void qpin(int qb, i32x4 &q) {
  switch (qb) {
    TMHD_QBLK(0, 128, 131)
    TMHD_QBLK(1, 132, 135)
    TMHD_QBLK(2, 136, 139)
    TMHD_QBLK(3, 140, 143)
    TMHD_QBLK(4, 144, 147)
    TMHD_QBLK(5, 148, 151)
    TMHD_QBLK(6, 152, 155)
    TMHD_QBLK(7, 156, 159)
    TMHD_QBLK(8, 160, 163)
    TMHD_QBLK(9, 164, 167)
    TMHD_QBLK(10, 168, 171)
    TMHD_QBLK(11, 172, 175)
    TMHD_QBLK(12, 176, 179)
    TMHD_QBLK(13, 180, 183)
    TMHD_QBLK(14, 184, 187)
    TMHD_QBLK(15, 188, 191)
  }
}
#undef TMHD_QBLK
#define TMHD_QBLK(QB, LO, HI)                                                                                      \
  case QB:                                                                                                         \
    if (first && hf == 0)                                                                                          \
      asm("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %3" : "=&v"(d) : "v"(k), "{a[" #LO ":" #HI "]}"(q), "{v[224:239]}"(c)); \
    else if (first)                                                                                                \
      asm("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %3" : "=&v"(d) : "v"(k), "{a[" #LO ":" #HI "]}"(q), "{v[240:255]}"(c)); \
    else                                                                                                           \
      asm("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(d) : "v"(k), "{a[" #LO ":" #HI "]}"(q));                \
    break;
// S^T (+)= K Q^T for one k-step of query half hf: `first` starts the chain at
// c, which lives in v[224:239] (hf 0) or v[240:255] (hf 1).
__device__ __forceinline__ void qk_bf16(int qb, int hf, bool first, f32x16 &d, i32x4 k, const i32x4 &q,
                                        const f32x16 &c) {
  switch (qb) {
    TMHD_QBLK(0, 128, 131)
    TMHD_QBLK(1, 132, 135)
    TMHD_QBLK(2, 136, 139)
    TMHD_QBLK(3, 140, 143)
    TMHD_QBLK(4, 144, 147)
    TMHD_QBLK(5, 148, 151)
    TMHD_QBLK(6, 152, 155)
    TMHD_QBLK(7, 156, 159)
    TMHD_QBLK(8, 160, 163)
    TMHD_QBLK(9, 164, 167)
    TMHD_QBLK(10, 168, 171)
    TMHD_QBLK(11, 172, 175)
    TMHD_QBLK(12, 176, 179)
    TMHD_QBLK(13, 180, 183)
    TMHD_QBLK(14, 184, 187)
    TMHD_QBLK(15, 188, 191)
  }
}
#undef TMHD_QBLK
// Output accumulator block b (16 fp32 per lane) lives in the fixed AGPRs
// a[16b, 16b + 15] for the whole kernel: every asm that touches it names that
// range, so the compiler never moves it, and the rare rescale can address the
// registers by name.
#define TMHD_OBLK(B, LO, HI)                                                                         \
  case B:                                                                                            \
    if (fresh)                                                                                       \
      asm("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+{a[" #LO ":" #HI "]}"(o) : "v"(v), "v"(p)); \
    else                                                                                             \
      asm("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+{a[" #LO ":" #HI "]}"(o) : "v"(v), "v"(p));    \
    break;
__device__ __forceinline__ void pv(int b, bool fresh, f32x16 &o, i32x4 v, i32x4 p) {
  switch (b) {
    TMHD_OBLK(0, 0, 15)
    TMHD_OBLK(1, 16, 31)
    TMHD_OBLK(2, 32, 47)
    TMHD_OBLK(3, 48, 63)
    TMHD_OBLK(4, 64, 79)
    TMHD_OBLK(5, 80, 95)
    TMHD_OBLK(6, 96, 111)
    TMHD_OBLK(7, 112, 127)
  }
}
#undef TMHD_OBLK
// Declares block b as live in its AGPRs at this point (after C++ code wrote
// it, or before C++ code reads it).
#define TMHD_OPIN(B, LO, HI) \
  case B:                    \
    asm volatile("" : "+{a[" #LO ":" #HI "]}"(o)); \
    break;
__device__ __forceinline__ void opin(int b, f32x16 &o) {
  switch (b) {
    TMHD_OPIN(0, 0, 15)
    TMHD_OPIN(1, 16, 31)
    TMHD_OPIN(2, 32, 47)
    TMHD_OPIN(3, 48, 63)
    TMHD_OPIN(4, 64, 79)
    TMHD_OPIN(5, 80, 95)
    TMHD_OPIN(6, 96, 111)
    TMHD_OPIN(7, 112, 127)
  }
}
#undef TMHD_OPIN
// Declares the score chain start of query half hf as live in its VGPRs.
__device__ __forceinline__ void npin(int hf, f32x16 &c) {
  if (hf == 0)
    asm volatile("" : "+{v[224:239]}"(c));
  else
    asm volatile("" : "+{v[240:255]}"(c));
}
// o *= alpha for block b, in place in its AGPRs (read, multiply, write back).
#define TMHD_RS(N) "v_accvgpr_read_b32 %1, a" #N "\n\tv_mul_f32 %1, %1, %2\n\tv_accvgpr_write_b32 a" #N ", %1\n\t"
#define TMHD_RS4(A, B, C, D) TMHD_RS(A) TMHD_RS(B) TMHD_RS(C) TMHD_RS(D)
#define TMHD_ORS(B, LO, HI, R0, R1, R2, R3)                                                  \
  case B:                                                                                    \
    asm volatile(R0 R1 R2 R3 : "+{a[" #LO ":" #HI "]}"(o), "=&v"(t) : "v"(alpha) : "memory"); \
    break;
__device__ __forceinline__ void orescale(int b, f32x16 &o, float alpha) {
  float t;
  switch (b) {
    TMHD_ORS(0, 0, 15, TMHD_RS4(0, 1, 2, 3), TMHD_RS4(4, 5, 6, 7), TMHD_RS4(8, 9, 10, 11), TMHD_RS4(12, 13, 14, 15))
    TMHD_ORS(1, 16, 31, TMHD_RS4(16, 17, 18, 19), TMHD_RS4(20, 21, 22, 23), TMHD_RS4(24, 25, 26, 27),
             TMHD_RS4(28, 29, 30, 31))
    TMHD_ORS(2, 32, 47, TMHD_RS4(32, 33, 34, 35), TMHD_RS4(36, 37, 38, 39), TMHD_RS4(40, 41, 42, 43),
             TMHD_RS4(44, 45, 46, 47))
    TMHD_ORS(3, 48, 63, TMHD_RS4(48, 49, 50, 51), TMHD_RS4(52, 53, 54, 55), TMHD_RS4(56, 57, 58, 59),
             TMHD_RS4(60, 61, 62, 63))
    TMHD_ORS(4, 64, 79, TMHD_RS4(64, 65, 66, 67), TMHD_RS4(68, 69, 70, 71), TMHD_RS4(72, 73, 74, 75),
             TMHD_RS4(76, 77, 78, 79))
    TMHD_ORS(5, 80, 95, TMHD_RS4(80, 81, 82, 83), TMHD_RS4(84, 85, 86, 87), TMHD_RS4(88, 89, 90, 91),
             TMHD_RS4(92, 93, 94, 95))
    TMHD_ORS(6, 96, 111, TMHD_RS4(96, 97, 98, 99), TMHD_RS4(100, 101, 102, 103), TMHD_RS4(104, 105, 106, 107),
             TMHD_RS4(108, 109, 110, 111))
    TMHD_ORS(7, 112, 127, TMHD_RS4(112, 113, 114, 115), TMHD_RS4(116, 117, 118, 119),
             TMHD_RS4(120, 121, 122, 123), TMHD_RS4(124, 125, 126, 127))
  }
}
#undef TMHD_ORS
#undef TMHD_RS4
#undef TMHD_RS
// Wait states after the last MFMA that wrote an AGPR accumulator, before VALU
// code reads it (an 8-pass MFMA completes within 4 * 8 + 2 cycles).
__device__ __forceinline__ void mfma_drain() { asm volatile("s_nop 15\n\ts_nop 15\n\ts_nop 15" ::: "memory"); }

// 16 bytes per lane global -> LDS (saddr form: 64-bit uniform base, 32-bit
// per-lane offset); the wave's 64 lanes fill the 1 KiB LDS block at m0.
// Issued as inline asm on purpose: the compiler's wait-count insertion cannot
// tell the destination block from the tiles being read and would place a
// vmcnt(0) wait in front of the next LDS read, serialising the prefetch.  The
// kernel itself waits (vmcnt(0) + barrier) before any read of a loaded tile;
// extra in-order vector-memory operations unknown to the compiler only make
// its own vmcnt waits stricter.
__device__ __forceinline__ void load_lds16(const void *base, uint32_t off, uint32_t lds_addr) {
  asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "{m0}"(lds_addr) : "memory");
}

// Work plan of one sub-tile, fixed at compile time.  The sub-tile issues
// 2 * ns MFMAs (two per slot, one per query half); region r is the code in
// front of MFMA r.  Issuing an MFMA holds the wave for about 16 of the MFMA's
// 32 cycles, so each region has about 16 cycles for other instructions before
// the matrix core idles.  Units, with their issue cycles:
//   E(u): the two exp2 of pair u % 8 (keys 2q, 2q+1) of query half u / 8 of
//         the current sub-tile (8 each);
//   C(u): their bf16 pack and row-sum adds (4 each), at or after E(u) and at
//         least one MFMA before the P.V MFMA that reads the pack;
//   M(u): row maximum of pair u % 8, half u / 8 of the next sub-tile's
//         scores, after the score-read guard (costed 4);
//   L(n): tile load n (DMA and its LDS address, 8), in the first `lwin` regions;
//   X(u): the two exp2 of pair u of the NEXT sub-tile, for its first `nx` / 2
//         pairs of each half (16, after the score-read guard and the pair's M
//         unit), placed after every other unit: the regions of the last P.V
//         MFMAs hold little else, while the first regions of every sub-tile
//         are over budget; those pairs then have no E unit in their own
//         sub-tile.
// Every region starts with its share of the fixed work (the operand read of
// odd regions, the wait in front of each slot's first MFMA); each unit goes
// to the cheapest region of its window (the earliest on ties).
struct SlotPlan {
  int e[16], c[16], m[16], l[16], x[16];
};
constexpr int plan_put(int (&cost)[64], int lo, int hi, int c) {
  int best = lo;
  for (int i = lo + 1; i <= hi; ++i)
    if (cost[i] < cost[best]) best = i;
  cost[best] += c;
  return best;
}
constexpr int kGuardRegionOffset = 1;  // score-read guard in region 2 * nqk + 1
constexpr SlotPlan make_plan(int nqk, int npv, int db, int nld, int lwin, int nx) {
  SlotPlan s{};
  int cost[64] = {};
  const int ns = nqk + npv, nr = 2 * ns;
  auto early = [&](int u) { return (u & 7) < nx / 2; };  // exponentials computed by the previous sub-tile
  for (int u = 0; u < 16; ++u) s.x[u] = -1;
  for (int i = 0; i < ns; ++i) {
    cost[2 * i] += 4;
    cost[2 * i + 1] += 4;
  }
  cost[2 * nqk + kGuardRegionOffset] += 11;
  for (int q = 0; q < 4; ++q)
    for (int hf = 0; hf < 2; ++hf) {
      const int u = hf * 8 + q, dl = 2 * nqk + hf - 1;
      s.e[u] = early(u) ? -1 : plan_put(cost, 0, dl, 16);
      s.c[u] = plan_put(cost, early(u) ? 0 : s.e[u], dl, 12);
    }
  for (int q = 0; q < 8; ++q)
    for (int hf = 0; hf < 2; ++hf) s.m[hf * 8 + q] = plan_put(cost, 2 * nqk + 2, nr - 1, 4);
  for (int q = 4; q < 8; ++q)
    for (int hf = 0; hf < 2; ++hf) {
      const int u = hf * 8 + q, dl = 2 * (nqk + db) + hf - 1;
      s.e[u] = plan_put(cost, 0, dl, 16);
      s.c[u] = plan_put(cost, s.e[u], dl, 12);
    }
  for (int n = 0; n < 16; ++n) s.l[n] = n < nld ? plan_put(cost, 0, lwin - 1, 8) : -1;
  for (int u = 0; u < 16; ++u)
    if (early(u)) s.x[u] = plan_put(cost, 2 * nqk + 2, nr - 1, 16);
  return s;
}

// The orderings the sub-tile code relies on, checked at compile time:
// a pair's pack (with its row-sum adds) after its exponentials and by its
// P.V deadline; maxima and early exponentials after the score guard; loads
// inside their window.  An early pair's exponentials are carried into the
// sub-tile in the registers its X unit then rewrites with the next
// sub-tile's, so its pack and adds must precede every X unit, which the
// deadline before the guard ensures.
constexpr bool plan_valid(const SlotPlan &s, int nqk, int npv, int db, int nld, int lwin, int nx) {
  const int nr = 2 * (nqk + npv), guard = 2 * nqk + kGuardRegionOffset;
  for (int u = 0; u < 16; ++u) {
    const int hf = u >> 3, q = u & 7;
    const bool early = q < nx / 2;
    const int dl = q < 4 ? 2 * nqk + hf - 1 : 2 * (nqk + db) + hf - 1;
    if (early != (s.e[u] < 0) || s.c[u] < (early ? 0 : s.e[u]) || s.c[u] > dl) return false;
    if (s.m[u] <= guard || s.m[u] >= nr) return false;
    if (early != (s.x[u] >= 0) || (early && (s.x[u] <= guard || s.x[u] >= nr))) return false;
  }
  for (int n = 0; n < 16; ++n)
    if ((n < nld) != (s.l[n] >= 0) || s.l[n] >= lwin) return false;
  return true;
}

template <int D>
__global__ void __launch_bounds__(kWaves * 64) __attribute__((amdgpu_waves_per_eu(1, 1))) attn_fwd_kernel(const KArgs a) {
  constexpr int KROW = 2 * D;  // bytes per key row in memory
  constexpr int KCPR = KROW / 16;       // 16-byte chunks per key row
  constexpr int KRS = KROW + 16;        // LDS key row stride: one pad chunk, an odd number of chunks
  constexpr int KT = kBN * KRS;         // LDS key tile bytes
  constexpr int VRS = kBN * 2 + 16;     // LDS value row stride (64 keys + one pad chunk)
  constexpr int VT = D * VRS;           // LDS value tile bytes (D rows)
  constexpr int NKL = KT / 1024;        // 1 KiB wave loads per key tile
  constexpr int NVL = VT / 1024;
  static_assert(KT % 1024 == 0 && VT % 1024 == 0, "tiles are whole wave loads");
  constexpr int KWL = (NKL + kWaves - 1) / kWaves;  // per wave (the last round is partial)
  constexpr int VWL = (NVL + kWaves - 1) / kWaves;
  constexpr int QST = D / 16;  // MFMA k-steps over head_dim
  constexpr int DB = D / 32;
  constexpr int NQK = QST;     // score slots per 32-key sub-tile (one K operand, two MFMAs)
  constexpr int NPV = 2 * DB;  // output slots per sub-tile (one V operand, two MFMAs)
  constexpr int NS = NQK + NPV;
  constexpr int LA = NQK < 4 ? NQK : 4;  // LDS operand reads in flight ahead of their slot
  static_assert(LA <= NQK, "the reads prefetched for the next sub-tile are score-slot reads");
  static_assert(NS <= 32 && NPV >= 4, "slot plan bounds");

  // LDS: three K tiles, then three V tiles (tile t lives in buffer t % 3).  A
  // 16-lane ds_read_b128 phase reads one 16-byte chunk of 16 consecutive rows;
  // key and value rows are padded to an odd number of 16-byte chunks so those
  // fall on 16 distinct bank groups and every operand read is one base
  // register plus an immediate offset.
  __shared__ __attribute__((aligned(1024))) char smem[3 * KT + 3 * VT];
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char *)smem;

  // item L, whole or key-tile range [t_begin, t_begin + cnt) of part `part`
  int L, part = -1, t_begin = 0, cnt = a.ntiles;
  if ((int)blockIdx.x < a.full) {
    L = xcd_logical_id(blockIdx.x, a.full);
  } else {
    const int tb = blockIdx.x - a.full, item = tb / a.nsplit;
    L = a.full + item;
    part = tb - item * a.nsplit;
    t_begin = a.ntiles * part / a.nsplit;
    cnt = a.ntiles * (part + 1) / a.nsplit - t_begin;
  }
  const int h = L / a.nqt;
  const int qt = L - h * a.nqt;
  const int tid = threadIdx.x, lane = tid & 63, lr = lane & 31, g = lane >> 5;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave index (uniform)
  const int q0 = qt * kBM + w * kQW;                        // first query row of this wave

  // ---- query operands of both 32-row halves (B operands of S^T = K Q^T), pinned in AGPRs
  i32x4 qv[2][QST];
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) {
    const int ql = q0 + hf * 32 + lr;
    if (ql < a.lq) {
      const int row = a.q_rows ? a.q_rows[ql] : a.q_row0 + ql;
      const uint16_t *p = a.q + (int64_t)row * a.qts + (int64_t)h * a.qhs + g * 8;
#pragma unroll
      for (int st = 0; st < QST; ++st) {
        const i32x4 raw = *(const i32x4 *)(p + st * 16);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t u = (uint32_t)raw[e];
          qv[hf][st][e] =
              (int)pack_bf16x2(__uint_as_float(u << 16) * a.c, __uint_as_float(u & 0xffff0000u) * a.c);
        }
      }
    } else {
#pragma unroll
      for (int st = 0; st < QST; ++st) qv[hf][st] = i32x4{0, 0, 0, 0};
    }
  }
#pragma unroll
  for (int hf = 0; hf < 2; ++hf)
#pragma unroll
    for (int st = 0; st < QST; ++st) qpin(hf * QST + st, qv[hf][st]);

  // per-lane LDS read offsets from smem (bytes; k-step, key half, buffer and db parts are uniform/immediate)
  const uint32_t kro = lr * KRS + g * 16;
  const uint32_t vro = 3 * KT + lr * VRS + g * 16;

  // Tile loads.  LDS slot c (16 bytes) of a tile holds chunk c % (n + 1) of
  // row c / (n + 1) (n data chunks per row; the pad chunk repeats the row's
  // last chunk).  Per-lane source offsets: keys are tile-invariant; values
  // keep (row, chunk) packed and scale by the segment's row stride per load.
  uint32_t koff[KWL], vrc[VWL];
  // Wave w loads blocks w, w + 4, ...; in the last round the waves past the
  // tile's end repeat its last block (same bytes to the same place), so that
  // every wave issues the same, branch-free sequence.
  auto kblk = [&](int i) { return min(w + i * kWaves, NKL - 1); };
  auto vblk = [&](int i) { return min(w + i * kWaves, NVL - 1); };
#pragma unroll
  for (int i = 0; i < KWL; ++i) {
    const int c = kblk(i) * 64 + lane, row = c / (KCPR + 1), chunk = min(c - row * (KCPR + 1), KCPR - 1);
    koff[i] = row * KROW + chunk * 16;
  }
#pragma unroll
  for (int i = 0; i < VWL; ++i) {
    const int c = vblk(i) * 64 + lane, row = c / 9, chunk = min(c - row * 9, 7);
    vrc[i] = (uint32_t)row | ((uint32_t)chunk << 20);
  }
  // load n of a tile: K blocks first (n < KWL), then V blocks
  constexpr int NLD = KWL + VWL;
  static_assert(NLD <= 16, "slot plan bounds");
  // tile loads spread over the first NS regions (with the early exponentials in the last
  // regions, 0.7% faster than 1.5 NS in two same-box A/Bs, 2 NS 1.3% slower)
  // early exponentials: pairs 0..3 of each query half (same-box A/B at 768p, 6 runs each, against
  // pair 0 placed before the second E / C units: 8.098 -> 7.995 ms; pair 0 alone, placed last:
  // 8.036 ms; against no early units, pair 0 gave about 1%)
  constexpr int NX = 8;
  constexpr SlotPlan PL = make_plan(NQK, NPV, DB, NLD, NS, NX);  // sub-tiles with tile loads
  constexpr SlotPlan PN = make_plan(NQK, NPV, DB, 0, 1, NX);     // sub-tiles without
  static_assert(plan_valid(PL, NQK, NPV, DB, NLD, NS, NX) && plan_valid(PN, NQK, NPV, DB, 0, 1, NX),
                "slot plan orderings");
  // value source offsets for the V^T row stride of the current load segment
  uint32_t voff[VWL];
  auto set_voff = [&](uint32_t vrs2) {
#pragma unroll
    for (int i = 0; i < VWL; ++i) voff[i] = (vrc[i] & 0xfffffu) * vrs2 + ((vrc[i] >> 20) << 4);
  };
  auto load_one = [&](int n, const char *kbase, uint32_t kdst, const char *vbase, uint32_t vdst) {
    if (n < KWL)
      load_lds16(kbase, koff[n], kdst + kblk(n) * 1024);
    else
      load_lds16(vbase, voff[n - KWL], vdst + vblk(n - KWL) * 1024);
  };
  auto load_k = [&](const Stream &S, int buf) {
    const char *base = S.kb + (int64_t)S.t * (kBN * KROW);
#pragma unroll
    for (int i = 0; i < KWL; ++i) load_lds16(base, koff[i], lds0 + buf * KT + kblk(i) * 1024);
  };
  auto load_v = [&](const Stream &S, int buf) {
    const char *base = S.vb + S.t * (kBN * 2);
#pragma unroll
    for (int i = 0; i < VWL; ++i)
      load_lds16(base, (vrc[i] & 0xfffffu) * S.vrs2 + ((vrc[i] >> 20) << 4),
                 lds0 + 3 * KT + buf * VT + vblk(i) * 1024);
  };
  auto lds_read = [&](uint32_t off) { return *(const i32x4 *)(smem + off); };
  // valid keys of a stream's current tile (1 .. 64)
  auto tile_valid = [](const Stream &S) { return min(S.tok - S.t * kBN, kBN); };

  // keys of a 32-key sub-tile at or beyond nvalid (relative to the sub-tile) -> -inf
  // (element r of a lane holds key 8 (r / 4) + 4 g + r % 4; comparing the
  // constant part with nvalid - 4 g keeps no per-element constants in registers)
  auto mask_sub = [&](f32x16 (&s)[2], int nvalid) {
    const int t = nvalid - 4 * g;
#pragma unroll
    for (int hf = 0; hf < 2; ++hf)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (8 * (r >> 2) + (r & 3) >= t) s[hf][r] = -INFINITY;
  };
  auto sub_max = [](const f32x16 &s) {
    float m = fmaxf(s[0], s[1]);
#pragma unroll
    for (int r = 2; r < 16; r += 2) m = fmaxf(m, fmaxf(s[r], s[r + 1]));
    return m;
  };

  f32x16 o[2][DB];  // block hf * DB + db lives in AGPRs a[16 b, 16 b + 15]
#pragma unroll
  for (int hf = 0; hf < 2; ++hf)
#pragma unroll
    for (int db = 0; db < DB; ++db) {
#pragma unroll
      for (int r = 0; r < 16; ++r) o[hf][db][r] = 0.0f;
      opin(hf * DB + db, o[hf][db]);
    }
  float lsum[2] = {0.0f, 0.0f};
  float mref[2];   // running reference of each query half (log2 units)
  f32x16 negm[2];  // -mref in every element, the score accumulator start
  const f32x16 zero16 = {};

  // ---- prologue: K(0..2), V(0..1) resident; S = scores of sub-tile 0 (minus m)
  Stream t0, t1, t2, t3;
  stream_seek<false>(t0, a, h, t_begin);
  t1 = t0;
  stream_next<false>(t1, a, h);
  t2 = t1;
  stream_next<false>(t2, a, h);
  t3 = t2;
  stream_next<false>(t3, a, h);
  load_k(t0, 0);
  load_k(t1, 1);
  load_v(t0, 0);
  // valid keys of tiles j, j+1, j+2, j+3
  int nv0 = tile_valid(t0), nv1 = tile_valid(t1), nv2 = tile_valid(t2), nv3 = tile_valid(t3);
  wait_vmem();
  __syncthreads();
  // scores (minus m) of the current and the next sub-tile: sub-tiles alternate
  // between the two sets, so no copies are needed
  f32x16 sA[2], sB[2];
  {
#pragma unroll
    for (int st = 0; st < QST; ++st) {
      const i32x4 kv = lds_read(kro + st * 32);
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        if (st == 0) sA[hf] = zero16;
        qk_bf16(hf * QST + st, hf, false, sA[hf], kv, qv[hf][st], zero16);
      }
    }
    mfma_drain();
    if (nv0 < 32) mask_sub(sA, nv0);
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const float lm = sub_max(sA[hf]);
      mref[hf] = fmaxf(lm, __shfl_xor(lm, 32));
      sA[hf] -= mref[hf];
      negm[hf] = -mref[hf];
      npin(hf, negm[hf]);
    }
  }
  // load streams: K of tile j+3 and V of tile j+2, issued after the barrier of iteration j
  Stream sk = t3, sv = t2;
  // operands of the first slots of sub-tile (0, keys 32..63)
  i32x4 pre[LA];
#pragma unroll
  for (int i = 0; i < LA; ++i) pre[i] = lds_read(kro + 32 * KRS + i * 32);

  int j = 0, b0 = 0, b1 = 1, b2 = 2;  // LDS buffers of tiles j, j+1, j+2
  // exp2 of the first NX / 2 pairs of each query half of the next sub-tile's
  // scores (the X units of the slot plan; for sub-tile 0, here)
  float pe_early[16][2];
  auto early_exp = [&](f32x16 (&s)[2], int hf) {
#pragma unroll
    for (int u = 0; u < 16; ++u)
      if ((u & 7) < NX / 2 && (u >> 3) == hf) {
        pe_early[u][0] = __builtin_amdgcn_exp2f(s[hf][2 * (u & 7)]);
        pe_early[u][1] = __builtin_amdgcn_exp2f(s[hf][2 * (u & 7) + 1]);
      }
  };
  early_exp(sA, 0);
  early_exp(sA, 1);

  // One 32-key sub-tile, software-pipelined by hand in NS slots of two MFMAs
  // (one per query half), each MFMA fenced with the units the plan puts in
  // front of it so that the compiler keeps their order.  Slot i also issues
  // the LDS operand read of slot i + LA:
  //   slots [0, NQK):  scores of the next sub-tile, K rows at kb (k-step st = i);
  //   slots [NQK, NS): O^T += V^T P^T of the current sub-tile, V chunks at vb.
  // sc: scores (minus m) of the current sub-tile; sn: receives those of the
  // next.  nvs: valid keys of the next sub-tile (<= 0: none); live: the next
  // sub-tile exists.
  // With loads, the slots also issue the tile loads of the iteration.  pre:
  // the operands of the first LA slots, read by the previous sub-tile; on
  // return, those of the next sub-tile (K rows at kbn).
  auto sub_tile = [&](f32x16 (&sc)[2], f32x16 (&sn)[2], uint32_t kb, uint32_t vb, uint32_t kbn, i32x4 (&pre)[LA],
                      int nvs, bool live, auto loads_c, const char *lkb, uint32_t lkd, const char *lvb,
                      uint32_t lvd) {
    auto read_op = [&](int i) -> i32x4 {
      if (i < NQK) return lds_read(kb + i * 32);
      const int p = i - NQK, st = p / DB, db = p % DB;
      return lds_read(vb + db * 32 * VRS + 2 * st * 16);
    };
    i32x4 ops[NS];
    i32x4 pk[2][2];  // P as bf16 pairs: [query half][16-key step]
    float ts[2] = {0.0f, 0.0f};
    float lm[2] = {-INFINITY, -INFINITY};
#pragma unroll
    for (int i = 0; i < LA; ++i) ops[i] = pre[i];
    float pe[2][8][2];  // exponentials of the current sub-tile, between their E and C units
#pragma unroll
    for (int u = 0; u < 16; ++u)
      if ((u & 7) < NX / 2) {  // computed by the previous sub-tile (or the prologue)
        pe[u >> 3][u & 7][0] = pe_early[u][0];
        pe[u >> 3][u & 7][1] = pe_early[u][1];
      }
#pragma clang loop unroll(full)
    for (int r = 0; r < 2 * NS; ++r) {
      const int i = r >> 1, hr = r & 1;  // slot, query half of MFMA r
      constexpr bool loads = decltype(loads_c)::value;
      constexpr SlotPlan pl = loads ? PL : PN;
      if (hr == 1) {
        if (i + LA < NS)
          ops[i + LA] = read_op(i + LA);
        else
          pre[i + LA - NS] = lds_read(kbn + (i + LA - NS) * 32);
      }
      if (loads)
#pragma unroll
        for (int n = 0; n < NLD; ++n)
          if (pl.l[n] == r) load_one(n, lkb, lkd, lvb, lvd);
#pragma unroll
      for (int u = 0; u < 16; ++u)
        if (pl.e[u] == r) {
          const int hf = u >> 3, q = u & 7;
          pe[hf][q][0] = __builtin_amdgcn_exp2f(sc[hf][2 * q]);
          pe[hf][q][1] = __builtin_amdgcn_exp2f(sc[hf][2 * q + 1]);
          asm volatile("" : "+v"(pe[hf][q][0]), "+v"(pe[hf][q][1]));  // keeps them in this region
        }
#pragma unroll
      for (int u = 0; u < 16; ++u)
        if (pl.c[u] == r) {
          const int hf = u >> 3, q = u & 7;
          int pr = (int)pack_bf16x2(pe[hf][q][0], pe[hf][q][1]);
          ts[hf] += pe[hf][q][0];
          ts[hf] += pe[hf][q][1];
          asm volatile("" : "+v"(pr), "+v"(ts[hf]));  // keeps the pack and the row sum in this region
          pk[hf][q >> 2][q & 3] = pr;
        }
      if (r == 2 * NQK + kGuardRegionOffset) {
        // first reads of the next sub-tile's scores: at least 12 wait states
        // after the last score MFMA (the MFMA in front of this region and
        // these 10); naming the results keeps every read below
        asm volatile("s_nop 10" : "+v"(sn[0]), "+v"(sn[1]));
      }
#pragma unroll
      for (int u = 0; u < 16; ++u)
        if (pl.m[u] == r) {
          const int hf = u >> 3, rr = (u & 7) * 2;
          lm[hf] = fmaxf(lm[hf], fmaxf(sn[hf][rr], sn[hf][rr + 1]));
          asm volatile("" : "+v"(lm[hf]));  // keeps the row maximum in this region
        }
#pragma unroll
      for (int u = 0; u < 16; ++u)
        if (pl.x[u] == r) {
          const int hf = u >> 3, q = u & 7;
          pe_early[u][0] = __builtin_amdgcn_exp2f(sn[hf][2 * q]);
          pe_early[u][1] = __builtin_amdgcn_exp2f(sn[hf][2 * q + 1]);
          asm volatile("" : "+v"(pe_early[u][0]), "+v"(pe_early[u][1]));  // keeps them in this region
        }
      __builtin_amdgcn_sched_barrier(0);
      if (i < NQK) {
        qk_bf16(hr * QST + i, hr, i == 0, sn[hr], ops[i], qv[hr][i], negm[hr]);
      } else {
        const int p = i - NQK, st = p / DB, db = p % DB;
        // the P group read here was packed in the region in front of the previous MFMA
        bool fresh = false;
#pragma unroll
        for (int q = 4 * st; q < 4 * st + 4; ++q) fresh = fresh || pl.c[hr * 8 + q] >= r - 1;
        pv(hr * DB + db, fresh, o[hr][db], ops[i], pk[hr][st]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    lsum[0] += ts[0];
    lsum[1] += ts[1];
    if (!live) return;
    if (nvs < 32) {
      int nvo = nvs;  // opaque inside the branch: keeps the comparisons from being hoisted
      asm volatile("" : "+s"(nvo));
      mask_sub(sn, nvo);
      lm[0] = sub_max(sn[0]);
      lm[1] = sub_max(sn[1]);
      early_exp(sn, 0);  // of the masked scores
      early_exp(sn, 1);
    }
    if (__any(fmaxf(lm[0], lm[1]) > kLazyRescale)) {
      mfma_drain();
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const float cm = fmaxf(lm[hf], __shfl_xor(lm[hf], 32));
        const float delta = fmaxf(cm, 0.0f);
        const float alpha = __builtin_amdgcn_exp2f(-delta);
        lsum[hf] *= alpha;
#pragma unroll
        for (int db = 0; db < DB; ++db) orescale(hf * DB + db, o[hf][db], alpha);
        sn[hf] -= delta;
        mref[hf] += delta;
        early_exp(sn, hf);  // against the new reference
        negm[hf] = -mref[hf];
        npin(hf, negm[hf]);
      }
      asm volatile("s_nop 2" ::: "memory");
    }
  };

  // Iteration j: sub-tiles (j, keys 0..31) and (j, keys 32..63).  LDS holds
  // K(j), K(j+1) and V(j); the loads issued from its first sub-tile's slots
  // (K(j+2) over K(j-1), V(j+1) over V(j-2)) are waited for at its end.
  // tile loads issued from the slots of iteration j: K(j+2) and V(j+1)
  const char *lkb = t2.kb + (int64_t)t2.t * (kBN * KROW), *lvb = t1.vb + t1.t * (kBN * 2);
  uint32_t lvrs = t1.vrs2, lkd = lds0 + 2 * KT, lvd = lds0 + 3 * KT + 1 * VT;
  set_voff(lvrs);
  for (;;) {
    // P of keys 0..31 of tile j; scores of keys 32..63 of tile j come next
    sub_tile(sA, sB, kro + b0 * KT + 32 * KRS, vro + b0 * VT, kro + b1 * KT, pre, nv0 - 32, true, std::true_type{}, lkb,
             lkd, lvb, lvd);
    // P of keys 32..63 of tile j; scores of keys 0..31 of tile j+1 come next
    // (after the last tile they read a stale in-bounds buffer and are unused)
    const bool more = j + 1 < cnt;
    sub_tile(sB, sA, kro + b1 * KT, vro + b0 * VT + 4 * 16, kro + b1 * KT + 32 * KRS, pre, nv1, more, std::false_type{},
             lkb, lkd, lvb, lvd);
    if (!more) break;
    ++j;
    wait_vmem();     // this wave's loads of K(j+1), V(j) (tile numbers of the new j)
    __syncthreads();  // everyone's loads landed; K(j-1) and V(j-2) are free
    nv0 = nv1;
    nv1 = nv2;
    nv2 = nv3;
    const int bf = b0;  // buffers rotate: tile t lives in buffer t % 3
    b0 = b1;
    b1 = b2;
    b2 = bf;
    // K(j+2) over K(j-1) and V(j+1) over V(j-2), issued from the slots of the
    // first sub-tile of iteration j
    lkb = sk.kb + (int64_t)sk.t * (kBN * KROW);
    lkd = lds0 + b2 * KT;
    lvb = sv.vb + sv.t * (kBN * 2);
    if (sv.vrs2 != lvrs) {  // the value loads moved to a segment with another row stride
      lvrs = sv.vrs2;
      set_voff(lvrs);
    }
    lvd = lds0 + 3 * KT + b1 * VT;
    sv = sk;
    stream_next<false>(sk, a, h);
    nv3 = tile_valid(sk);
  }

  // ---- epilogue: O = O^T / l, written token-major (4 consecutive d per store).
  // The last iteration's tile loads (into buffers nobody reads) land before the
  // workgroup's LDS is released.
  wait_vmem();
  mfma_drain();
#pragma unroll
  for (int hf = 0; hf < 2; ++hf)
#pragma unroll
    for (int db = 0; db < DB; ++db) opin(hf * DB + db, o[hf][db]);
  if (part >= 0) {
    // key range of a split item: normalised partial O and its log2-sum-exp
    float *wo = a.ws + (int64_t)(blockIdx.x - a.full) * (kBM * D + kBM);
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const float lt = lsum[hf] + __shfl_xor(lsum[hf], 32);
      const float inv = 1.0f / lt;
      const int rl = w * kQW + hf * 32 + lr;  // row within the item
      if (q0 + hf * 32 + lr < a.lq) {
        float *op = wo + rl * D + 4 * g;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
          for (int u = 0; u < 4; ++u)
            *(f32x4 *)(op + db * 32 + 8 * u) = f32x4{o[hf][db][4 * u] * inv, o[hf][db][4 * u + 1] * inv,
                                                     o[hf][db][4 * u + 2] * inv, o[hf][db][4 * u + 3] * inv};
        if (g == 0) wo[kBM * D + rl] = mref[hf] + __log2f(lt);
      }
    }
    return;
  }
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) {
    const float lt = lsum[hf] + __shfl_xor(lsum[hf], 32);
    const float inv = 1.0f / lt;
    const int ql = q0 + hf * 32 + lr;
    if (ql < a.lq) {
      const int row = a.o_rows ? a.o_rows[ql] : a.o_row0 + ql;
      uint16_t *op = a.o + (int64_t)row * a.ots + (int64_t)h * a.ohs + 4 * g;
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          i32x2 pr = {(int)pack_bf16x2(o[hf][db][4 * u] * inv, o[hf][db][4 * u + 1] * inv),
                      (int)pack_bf16x2(o[hf][db][4 * u + 2] * inv, o[hf][db][4 * u + 3] * inv)};
          *(i32x2 *)(op + db * 32 + 8 * u) = pr;
        }
    }
  }
}

// ---- INT8-QK attention with two workgroups per CU (two waves per SIMD) ----
//
// The kernel above holds one wave per SIMD.  Issuing an MFMA blocks the
// issuing wave for about half of the MFMA's cycles, so a lone wave slips only
// a few VALU instructions under each MFMA; the INT8-QK sub-tile carries 24
// MFMAs (8 INT8 Q.K^T, 16 BF16 P.V) and about 160 softmax VALU instructions,
// more than fit, and the matrix cores idle.  A second wave on the SIMD issues
// while the first is blocked: measured on one MI355X, a mix of 24 MFMAs and
// 160 such VALU instructions costs 34.5 cycles per MFMA with two waves per
// SIMD against 46.2 with one (32.0 for the MFMAs alone).  A wave then has 256
// registers.  INT8 query operands take 32 per lane (BF16: 64), and with:
//   * all operands and accumulators in VGPRs (a kernel that touches AGPRs
//     gets them split 128 / 128, and the output accumulators alone fill 128);
//   * the score chains starting at the MFMA's inline constant 1/(2 pi), so
//     each int32 score reads as a float and is dequantised with the reference
//     folded in by one FMA (no conversion, no chain-start registers);
//   * one score buffer: the next sub-tile's scores are converted,
//     exponentiated and packed to bf16 under the current sub-tile's P.V
//     MFMAs, so only the packed probabilities (16 registers) are double-buffered;
//   * two LDS operand reads in flight instead of four;
//   * value tiles double-buffered (64.5 KiB of LDS per workgroup at head_dim
//     128, so two workgroups fit a CU)
// the loop fits 256 registers without spilling.  The exponentials are
// computed before the next sub-tile's row maximum is known; a sub-tile whose
// maximum exceeds the reference by more than 2^8 (lazy rescale), or that is
// partial (masked keys), is recomputed in a rare branch: its scores again
// from LDS, masked, the reference moved and O and l rescaled, then its
// probabilities against the new reference.  The work decomposition (256 query
// rows of one head per workgroup, 64 per wave), slot layouts, tile loads and
// split last round are those of the kernel above.
constexpr int kI8LA = 1;  // LDS operand reads in flight ahead of their slot
// the probabilities of a lane's 16 keys sum to at most 16 * 2^12 while every
// one is at most 2^12 (score at most 12 above the reference, log2 units)
constexpr float kRowSumBound = 16.0f * 4096.0f;

// Slot plan of one INT8 sub-tile.  Regions are as in make_plan; units:
//   M(u): conversion, dequantisation and row maximum of pair u % 8 (query half
//         u / 8) of the next sub-tile's scores (cost 20), after the score-read
//         guard;
//   E(u): its two exp2, in place (16), after M(u);
//   C(u): their bf16 pack and row-sum adds (12), after E(u) and after the
//         last P.V MFMA that reads the first pack group of the current
//         sub-tile (the new packs reuse those registers);
//   L(n): tile load n (8) in regions [lwlo, nr), the last ones, where the
//         packs have freed score registers for the load offsets.
struct SlotPlan8 {
  int m[16], e[16], c[16], l[16];
};
constexpr SlotPlan8 make_plan8(int nqk, int npv, int db, int nld, int lwlo) {
  SlotPlan8 s{};
  int cost[64] = {};
  const int ns = nqk + npv, nr = 2 * ns, guard = 2 * nqk + kGuardRegionOffset, cfree = 2 * (nqk + db);
  for (int i = 0; i < ns; ++i) {
    cost[2 * i] += 4;
    cost[2 * i + 1] += 4;
  }
  cost[guard] += 11;
  for (int n = 0; n < 16; ++n) s.l[n] = n < nld ? plan_put(cost, lwlo, nr - 1, 8) : -1;
  for (int q = 0; q < 8; ++q)
    for (int hf = 0; hf < 2; ++hf) s.m[hf * 8 + q] = plan_put(cost, guard + 1, nr - 1, 20);
  for (int q = 0; q < 8; ++q)
    for (int hf = 0; hf < 2; ++hf) s.e[hf * 8 + q] = plan_put(cost, s.m[hf * 8 + q], nr - 1, 16);
  for (int q = 0; q < 8; ++q)
    for (int hf = 0; hf < 2; ++hf) {
      const int u = hf * 8 + q;
      s.c[u] = plan_put(cost, s.e[u] > cfree ? s.e[u] : cfree, nr - 1, 12);
    }
  return s;
}
constexpr bool plan8_valid(const SlotPlan8 &s, int nqk, int npv, int db, int nld, int lwlo) {
  const int nr = 2 * (nqk + npv), guard = 2 * nqk + kGuardRegionOffset, cfree = 2 * (nqk + db);
  for (int u = 0; u < 16; ++u)
    if (s.m[u] <= guard || s.e[u] < s.m[u] || s.c[u] < s.e[u] || s.c[u] < cfree || s.c[u] >= nr) return false;
  for (int n = 0; n < 16; ++n)
    if ((n < nld) != (s.l[n] >= 0) || (n < nld && (s.l[n] < lwlo || s.l[n] >= nr))) return false;
  return true;
}

// S^T (+)= K Q^T for one 32-byte k-step, all in VGPRs; `first` starts the
// chain at the inline constant 1/(2 pi) (bits 0x3E22F983).  Volatile, like
// every MFMA of this kernel: the hazard waits in front of VALU reads of MFMA
// results (mfma_drain, the score guard) are volatile asm too, and only
// volatile asm keeps its order relative to them (a plain asm MFMA may be sunk
// below a drain that does not name its registers).
__device__ __forceinline__ void qk_i8z(bool first, i32x16 &d, i32x4 k, const i32x4 &q) {
  if (first)
    asm volatile("v_mfma_i32_32x32x32_i8 %0, %1, %2, 0.15915494309189532" : "=&v"(d) : "v"(k), "v"(q));
  else
    asm volatile("v_mfma_i32_32x32x32_i8 %0, %1, %2, %0" : "+v"(d) : "v"(k), "v"(q));
}
// O^T += V^T P^T with the accumulator in VGPRs (the packs are at least a
// sub-tile old, past the 2 wait states a VALU write needs).
__device__ __forceinline__ void pv_v(f32x16 &o, i32x4 v, i32x4 p) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(o) : "v"(v), "v"(p));
}

template <int D>
__global__ void __launch_bounds__(kWaves * 64) __attribute__((amdgpu_waves_per_eu(2, 2))) attn_i8_kernel(const KArgs a) {
  constexpr int KROW = D;            // bytes per int8 key row
  constexpr int KCPR = KROW / 16;    // 16-byte chunks per key row
  constexpr int KRS = KROW + 16;     // LDS key row stride (one pad chunk)
  constexpr int KT = kBN * KRS;      // LDS key tile bytes
  constexpr int VRS = kBN * 2 + 16;  // LDS value row stride
  constexpr int VT = D * VRS;        // LDS value tile bytes
  constexpr int NKL = KT / 1024;
  constexpr int NVL = VT / 1024;
  static_assert(KT % 1024 == 0 && VT % 1024 == 0, "tiles are whole wave loads");
  constexpr int KWL = (NKL + kWaves - 1) / kWaves;
  constexpr int VWL = (NVL + kWaves - 1) / kWaves;
  constexpr int QST = D / 32;  // INT8 k-steps over head_dim
  constexpr int DB = D / 32;
  constexpr int NQK = QST;
  constexpr int NPV = 2 * DB;
  constexpr int NS = NQK + NPV;
  constexpr int LA = kI8LA;
  static_assert(LA <= NQK && NS <= 32 && NPV >= 4, "slot plan bounds");

  // LDS: three K tiles (tile t in buffer t % 3), then two V tiles (t % 2),
  // then each lane's tile-load source offsets (8 words per lane)
  constexpr int TAB = 3 * KT + 2 * VT;
  __shared__ __attribute__((aligned(1024))) char smem[TAB + kWaves * 64 * 32];
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char *)smem;

  int L, part = -1, t_begin = 0, cnt = a.ntiles;
  if ((int)blockIdx.x < a.full) {
    L = xcd_logical_id(blockIdx.x, a.full);
  } else {
    const int tb = blockIdx.x - a.full, item = tb / a.nsplit;
    L = a.full + item;
    part = tb - item * a.nsplit;
    t_begin = a.ntiles * part / a.nsplit;
    cnt = a.ntiles * (part + 1) / a.nsplit - t_begin;
  }
  const int h = L / a.nqt;
  const int qt = L - h * a.nqt;
  const int tid = threadIdx.x, lane = tid & 63, lr = lane & 31, g = lane >> 5;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q0 = qt * kBM + w * kQW;

  // query operands of both 32-row halves (B operands of S^T = K Q^T)
  i32x4 qv[2][QST];
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) {
    const int ql = q0 + hf * 32 + lr;
    const int8_t *p = a.q8 + (int64_t)h * a.q8hs + (int64_t)ql * D + g * 16;
#pragma unroll
    for (int st = 0; st < QST; ++st) qv[hf][st] = ql < a.lq ? *(const i32x4 *)(p + st * 32) : i32x4{0, 0, 0, 0};
  }
  // softmax scale * log2(e) * query block scale (the wave's 64 rows lie in one 128-row block)
  const float cq = a.c * a.qs[(int64_t)h * a.qshs + q0 / TMHD_QUANT_BLOCK] * (1.0f / kI8Slope);

  const uint32_t kro = lr * KRS + g * 16;
  const uint32_t vro = 3 * KT + lr * VRS + g * 16;

  // per-lane source offsets of the tile loads, kept in LDS (the registers are
  // the loop's scarcest resource) and read at the start of each loading
  // sub-tile: keys tile-invariant; values for the V^T row stride of the
  // segment the loop's value loads are in, rewritten when that changes
  auto kblk = [&](int i) { return min(w + i * kWaves, NKL - 1); };
  auto vblk = [&](int i) { return min(w + i * kWaves, NVL - 1); };
  constexpr int NLD = KWL + VWL;
  static_assert(NLD <= 8, "eight offset words per lane");
  {
    uint32_t tab[8] = {};
#pragma unroll
    for (int i = 0; i < KWL; ++i) {
      const int c = kblk(i) * 64 + lane, row = c / (KCPR + 1), chunk = min(c - row * (KCPR + 1), KCPR - 1);
      tab[i] = row * KROW + chunk * 16;
    }
#pragma unroll
    for (int i = 0; i < VWL; ++i) tab[KWL + i] = 0;  // set by write_vtab once the streams are known
    *(i32x4 *)(smem + TAB + tid * 32) = i32x4{(int)tab[0], (int)tab[1], (int)tab[2], (int)tab[3]};
    *(i32x4 *)(smem + TAB + tid * 32 + 16) = i32x4{(int)tab[4], (int)tab[5], (int)tab[6], (int)tab[7]};
  }
  auto read_tab = [&](uint32_t (&t)[8]) {
    const i32x4 lo = *(const i32x4 *)(smem + TAB + tid * 32), hi = *(const i32x4 *)(smem + TAB + tid * 32 + 16);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      t[e] = (uint32_t)lo[e];
      t[4 + e] = (uint32_t)hi[e];
    }
  };
  // source offset of value load i for a V^T row stride of vrs2 bytes (row <
  // 128 and vrs2 < 2^24, which the launch checks, so it fits 32 bits)
  auto voff_of = [&](int i, uint32_t vrs2) {
    const int c = vblk(i) * 64 + lane, row = c / 9, chunk = min(c - row * 9, 7);
    return (uint32_t)row * vrs2 + (uint32_t)chunk * 16u;
  };
  // the lane's value offsets in the table, for row stride vrs2 (each lane
  // reads only its own words, so no barrier is needed)
  auto write_vtab = [&](uint32_t vrs2) {
#pragma unroll
    for (int i = 0; i < VWL; ++i) *(uint32_t *)(smem + TAB + tid * 32 + (KWL + i) * 4) = voff_of(i, vrs2);
  };
  // the tile loads go into the last NLD regions (at least the last 8); their
  // offsets are read from the table TABLEAD regions before the window
  constexpr int LWLO = 2 * NS - (NLD > 8 ? NLD : 8);
  constexpr int TABLEAD = 4;
  static_assert(LWLO >= TABLEAD, "room for the offset-table read");
  constexpr SlotPlan8 PL = make_plan8(NQK, NPV, DB, NLD, LWLO);
  constexpr SlotPlan8 PN = make_plan8(NQK, NPV, DB, 0, LWLO);
  static_assert(plan8_valid(PL, NQK, NPV, DB, NLD, LWLO) && plan8_valid(PN, NQK, NPV, DB, 0, LWLO),
                "slot plan orderings");
  auto load_one = [&](int n, const uint32_t (&t)[8], const char *kbase, uint32_t kdst, const char *vbase,
                      uint32_t vdst) {
    if (n < KWL)
      load_lds16(kbase, t[n], kdst + kblk(n) * 1024);
    else
      load_lds16(vbase, t[n], vdst + vblk(n - KWL) * 1024);
  };
  auto load_k = [&](const uint32_t (&t)[8], const Stream &S, int buf) {
    const char *base = S.kb + (int64_t)S.t * (kBN * KROW);
#pragma unroll
    for (int i = 0; i < KWL; ++i) load_lds16(base, t[i], lds0 + buf * KT + kblk(i) * 1024);
  };
  auto load_v = [&](const Stream &S, int buf) {
    const char *base = S.vb + S.t * (kBN * 2);
#pragma unroll
    for (int i = 0; i < VWL; ++i) load_lds16(base, voff_of(i, S.vrs2), lds0 + 3 * KT + buf * VT + vblk(i) * 1024);
  };
  auto load_ks = [&](const Stream &S) {
    int idx = S.t >> 1;  // 128-token quant blocks hold two tiles
    asm volatile("v_mov_b32 %0, %1" : "=v"(idx) : "s"(idx));
    return S.ks[idx];
  };
  auto lds_read = [&](uint32_t off) { return *(const i32x4 *)(smem + off); };
  auto tile_valid = [](const Stream &S) { return min(S.tok - S.t * kBN, kBN); };
  f32x16 o[2][DB];
#pragma unroll
  for (int hf = 0; hf < 2; ++hf)
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[hf][db][r] = 0.0f;
  float lsum[2] = {0.0f, 0.0f};
  float mref[2] = {0.0f, 0.0f};  // running reference of each query column (log2 units)
  i32x16 sn[2];                   // scores of the next sub-tile
  // scores live as the bits of floats in i32x16 (the MFMA writes int32
  // accumulators, converted in place)
  auto f = [](int bits) { return __int_as_float(bits); };
  // the wait states in front of VALU reads of MFMA results, naming the
  // registers read after them so that no read moves above the wait
  auto drain_scores = [&]() { asm volatile("s_nop 15\n\ts_nop 15\n\ts_nop 15" : "+v"(sn[0]), "+v"(sn[1])::"memory"); };
  auto drain_o = [&]() {
    mfma_drain();
#pragma unroll
    for (int hf = 0; hf < 2; ++hf)
#pragma unroll
      for (int db = 0; db < DB; ++db) asm volatile("" : "+v"(o[hf][db]));
  };
  auto sub_max = [&](const i32x16 &s) {
    float m = fmaxf(f(s[0]), f(s[1]));
#pragma unroll
    for (int r = 2; r < 16; r += 2) m = fmaxf(m, fmaxf(f(s[r]), f(s[r + 1])));
    return m;
  };


  // Rare path, and the first sub-tile: the scores of a 32-key sub-tile from
  // LDS (K rows at kb) into sn, dequantised against the reference, keys at or
  // beyond nvalid masked, the reference moved where a score exceeds it by
  // more than 2^8 (O and l rescaled; `first`: set to the sub-tile's maximum),
  // then the probabilities packed into pkn and their row sums added to l.
  auto full_softmax = [&](uint32_t kb, int nvalid, float ct, bool first, i32x4 (&pkn)[2][2]) {
#pragma unroll
    for (int st = 0; st < QST; ++st) {
      const i32x4 kv = lds_read(kb + st * 32);
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) qk_i8z(st == 0, sn[hf], kv, qv[hf][st]);
    }
    drain_scores();  // the score results, and every P.V accumulation in flight
    const int t = nvalid - 4 * g;  // element r of a lane holds key 8 (r / 4) + 4 g + r % 4
    float cm[2];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float x = fmaf(f(sn[hf][r]), ct, -fmaf(kI8MagicF, ct, mref[hf]));
        sn[hf][r] = __float_as_int(8 * (r >> 2) + (r & 3) >= t ? -INFINITY : x);
      }
      const float lm = sub_max(sn[hf]);
      cm[hf] = fmaxf(lm, __shfl_xor(lm, 32));
    }
    if (first) {
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        mref[hf] = cm[hf];  // the wave's first keys set the reference
#pragma unroll
        for (int r = 0; r < 16; ++r) sn[hf][r] = __float_as_int(f(sn[hf][r]) - cm[hf]);
      }
    } else if (__any(fmaxf(cm[0], cm[1]) > kLazyRescale)) {
      drain_o();
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const float delta = fmaxf(cm[hf], 0.0f);
        const float alpha = __builtin_amdgcn_exp2f(-delta);
        lsum[hf] *= alpha;
#pragma unroll
        for (int db = 0; db < DB; ++db) o[hf][db] *= alpha;
#pragma unroll
        for (int r = 0; r < 16; ++r) sn[hf][r] = __float_as_int(f(sn[hf][r]) - delta);
        mref[hf] += delta;
      }
      asm volatile("s_nop 2" ::: "memory");  // VALU writes of O before the next accumulation
    }
#pragma unroll
    for (int hf = 0; hf < 2; ++hf)
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const float e0 = __builtin_amdgcn_exp2f(f(sn[hf][2 * q])), e1 = __builtin_amdgcn_exp2f(f(sn[hf][2 * q + 1]));
        pkn[hf][q >> 2][q & 3] = (int)pack_bf16x2(e0, e1);
        lsum[hf] += e0;
        lsum[hf] += e1;
      }
  };

  // ---- prologue: K(0), K(1), V(0) resident; P of sub-tile 0
  Stream t0, t1, t2, t3;
  stream_seek<true>(t0, a, h, t_begin);
  t1 = t0;
  stream_next<true>(t1, a, h);
  t2 = t1;
  stream_next<true>(t2, a, h);
  t3 = t2;
  stream_next<true>(t3, a, h);
  write_vtab(t1.vrs2);  // the loop's first value loads are of tile 1
  __syncthreads();  // the offset table
  {
    uint32_t t[8];
    read_tab(t);
    load_k(t, t0, 0);
    load_k(t, t1, 1);
    load_v(t0, 0);
  }
  int nv0 = tile_valid(t0), nv1 = tile_valid(t1), nv2 = tile_valid(t2), nv3 = tile_valid(t3);
  float ks2 = load_ks(t2);
  float ks0 = load_ks(t0), ks1 = load_ks(t1);
  wait_vmem();
  __syncthreads();
  ks0 = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(ks0)));
  ks1 = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(ks1)));
  i32x4 pkA[2][2], pkB[2][2];  // packed probabilities of the current / next sub-tile, alternating
  full_softmax(kro, nv0, cq * ks0, true, pkA);
  Stream sk = t3, sv = t2;  // K of tile j+3 and V of tile j+2, issued after the barrier of iteration j
  i32x4 pre[LA];
#pragma unroll
  for (int i = 0; i < LA; ++i) pre[i] = lds_read(kro + 32 * KRS + i * 32);

  int j = 0, b0 = 0, b1 = 1, b2 = 2, vb = 0;  // K buffers of tiles j, j+1, j+2; V buffer of tile j

  // One 32-key sub-tile in NS slots of two MFMAs (one per query half), each
  // MFMA fenced with the units the plan puts in front of it:
  //   slots [0, NQK):  scores of the next sub-tile into sn, K rows at kb;
  //   slots [NQK, NS): O^T += V^T P^T of the current sub-tile (packs pk),
  //                    V chunks at vbo; under them the next sub-tile's
  //                    probabilities go into pkn.
  // Slot i issues the LDS operand read of slot i + LA; the last ones read the
  // first operands of the sub-tile after (K rows at kbn) into pre.
  auto sub_tile = [&](i32x4 (&pk)[2][2], i32x4 (&pkn)[2][2], uint32_t kb, uint32_t vbo, uint32_t kbn,
                      i32x4 (&pre)[LA], int nvs, float ctn, bool live, auto loads_c, const char *lkb, uint32_t lkd,
                      const char *lvb, uint32_t lvd) {
    const float nbn[2] = {-fmaf(kI8MagicF, ctn, mref[0]), -fmaf(kI8MagicF, ctn, mref[1])};
    auto read_op = [&](int i) -> i32x4 {
      if (i < NQK) return lds_read(kb + i * 32);
      const int p = i - NQK, st = p / DB, db = p % DB;
      return lds_read(vbo + db * 32 * VRS + 2 * st * 16);
    };
    i32x4 ops[NS];
    float ts[2] = {0.0f, 0.0f};
    constexpr bool loads = decltype(loads_c)::value;
    uint32_t tab[8];
#pragma unroll
    for (int i = 0; i < LA; ++i) ops[i] = pre[i];
#pragma clang loop unroll(full)
    for (int r = 0; r < 2 * NS; ++r) {
      const int i = r >> 1, hr = r & 1;
      constexpr SlotPlan8 pl = loads ? PL : PN;
      if (hr == 1) {
        if (i + LA < NS)
          ops[i + LA] = read_op(i + LA);
        else
          pre[i + LA - NS] = lds_read(kbn + (i + LA - NS) * 32);
      }
      if (loads && r == LWLO - TABLEAD) read_tab(tab);
      if (loads)
#pragma unroll
        for (int n = 0; n < NLD; ++n)
          if (pl.l[n] == r) load_one(n, tab, lkb, lkd, lvb, lvd);
      if (r == 2 * NQK + kGuardRegionOffset) {
        // first reads of the scores: at least 12 wait states after the last
        // score MFMA; naming them keeps every read below
        asm volatile("s_nop 10" : "+v"(sn[0]), "+v"(sn[1]));
      }
#pragma unroll
      for (int u = 0; u < 16; ++u)
        if (pl.m[u] == r) {
          const int hf = u >> 3, rr = (u & 7) * 2;
          sn[hf][rr] = __float_as_int(fmaf(f(sn[hf][rr]), ctn, nbn[hf]));
          sn[hf][rr + 1] = __float_as_int(fmaf(f(sn[hf][rr + 1]), ctn, nbn[hf]));
          asm volatile("" : "+v"(sn[hf][rr]), "+v"(sn[hf][rr + 1]));
        }
#pragma unroll
      for (int u = 0; u < 16; ++u)
        if (pl.e[u] == r) {
          const int hf = u >> 3, q = u & 7;
          sn[hf][2 * q] = __float_as_int(__builtin_amdgcn_exp2f(f(sn[hf][2 * q])));
          sn[hf][2 * q + 1] = __float_as_int(__builtin_amdgcn_exp2f(f(sn[hf][2 * q + 1])));
          asm volatile("" : "+v"(sn[hf][2 * q]), "+v"(sn[hf][2 * q + 1]));
        }
#pragma unroll
      for (int u = 0; u < 16; ++u)
        if (pl.c[u] == r) {
          const int hf = u >> 3, q = u & 7;
          int pr = (int)pack_bf16x2(f(sn[hf][2 * q]), f(sn[hf][2 * q + 1]));
          ts[hf] += f(sn[hf][2 * q]);
          ts[hf] += f(sn[hf][2 * q + 1]);
          asm volatile("" : "+v"(pr), "+v"(ts[hf]));
          pkn[hf][q >> 2][q & 3] = pr;
        }
      __builtin_amdgcn_sched_barrier(0);
      if (i < NQK) {
        qk_i8z(i == 0, sn[hr], ops[i], qv[hr][i]);
      } else {
        const int p = i - NQK, st = p / DB, db = p % DB;
        pv_v(o[hr][db], ops[i], pk[hr][st]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (!live) return;
    // a lane's 16 probabilities sum to at most 16 * 2^12 unless one exceeds
    // 2^12 (or overflowed): then, or for a partial sub-tile, recompute
    if (nvs < 32 || __any(!(fmaxf(ts[0], ts[1]) <= kRowSumBound))) {
      int nvo = nvs;  // opaque inside the branch: keeps the comparisons from being hoisted
      asm volatile("" : "+s"(nvo));
      full_softmax(kb, nvo, ctn, false, pkn);
      return;
    }
    lsum[0] += ts[0];
    lsum[1] += ts[1];
  };

  // tile loads issued from the slots of iteration j: K(j+2) and V(j+1)
  const char *lkb = t2.kb + (int64_t)t2.t * (kBN * KROW), *lvb = t1.vb + t1.t * (kBN * 2);
  uint32_t lvrs = t1.vrs2, lkd = lds0 + 2 * KT, lvd = lds0 + 3 * KT + 1 * VT;
  for (;;) {
    // P of keys 0..31 of tile j; scores of keys 32..63 of tile j
    sub_tile(pkA, pkB, kro + b0 * KT + 32 * KRS, vro + vb * VT, kro + b1 * KT, pre, nv0 - 32, cq * ks0, true,
             std::true_type{}, lkb, lkd, lvb, lvd);
    // P of keys 32..63 of tile j; scores of keys 0..31 of tile j+1 (after the
    // last tile they read a stale in-bounds buffer and are unused)
    const bool more = j + 1 < cnt;
    sub_tile(pkB, pkA, kro + b1 * KT, vro + vb * VT + 4 * 16, kro + b1 * KT + 32 * KRS, pre, nv1, cq * ks1, more,
             std::false_type{}, lkb, lkd, lvb, lvd);
    if (!more) break;
    ++j;
    wait_vmem();
    __syncthreads();
    nv0 = nv1;
    nv1 = nv2;
    nv2 = nv3;
    ks0 = ks1;
    ks1 = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(ks2)));  // uniform: keep it in an SGPR
    const int bf = b0;
    b0 = b1;
    b1 = b2;
    b2 = bf;
    vb ^= 1;
    lkb = sk.kb + (int64_t)sk.t * (kBN * KROW);
    lkd = lds0 + b2 * KT;
    lvb = sv.vb + sv.t * (kBN * 2);
    if (sv.vrs2 != lvrs) {  // the value loads moved to a segment with another row stride
      lvrs = sv.vrs2;
      write_vtab(lvrs);
    }
    lvd = lds0 + 3 * KT + (vb ^ 1) * VT;
    ks2 = load_ks(sk);
    sv = sk;
    stream_next<true>(sk, a, h);
    nv3 = tile_valid(sk);
  }

  // ---- epilogue (as the kernel above)
  wait_vmem();
  drain_o();
  if (part >= 0) {
    float *wo = a.ws + (int64_t)(blockIdx.x - a.full) * (kBM * D + kBM);
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const float lt = lsum[hf] + __shfl_xor(lsum[hf], 32);
      const float inv = 1.0f / lt;
      const int rl = w * kQW + hf * 32 + lr;
      if (q0 + hf * 32 + lr < a.lq) {
        float *op = wo + rl * D + 4 * g;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
          for (int u = 0; u < 4; ++u)
            *(f32x4 *)(op + db * 32 + 8 * u) = f32x4{o[hf][db][4 * u] * inv, o[hf][db][4 * u + 1] * inv,
                                                     o[hf][db][4 * u + 2] * inv, o[hf][db][4 * u + 3] * inv};
        if (g == 0) wo[kBM * D + rl] = mref[hf] + __log2f(lt);
      }
    }
    return;
  }
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) {
    const float lt = lsum[hf] + __shfl_xor(lsum[hf], 32);
    const float inv = 1.0f / lt;
    const int ql = q0 + hf * 32 + lr;
    if (ql < a.lq) {
      const int row = a.o_rows ? a.o_rows[ql] : a.o_row0 + ql;
      uint16_t *op = a.o + (int64_t)row * a.ots + (int64_t)h * a.ohs + 4 * g;
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          i32x2 pr = {(int)pack_bf16x2(o[hf][db][4 * u] * inv, o[hf][db][4 * u + 1] * inv),
                      (int)pack_bf16x2(o[hf][db][4 * u + 2] * inv, o[hf][db][4 * u + 3] * inv)};
          *(i32x2 *)(op + db * 32 + 8 * u) = pr;
        }
    }
  }
}

// Merge of split items: O = sum_p 2^(lse_p - lse) O_p with lse = log2 sum_p
// 2^lse_p (the partial O_p are normalised).  One thread per 4 columns of a
// row; item i of the split ones owns workspace blocks [i * nsplit, (i+1) * nsplit).
template <int D>
__global__ void __launch_bounds__(256) attn_merge_kernel(const KArgs a) {
  constexpr int CG = D / 4, RPB = 256 / CG;  // column groups per row, rows per block
  const int item = blockIdx.x / (kBM / RPB);
  const int rl = (blockIdx.x - item * (kBM / RPB)) * RPB + threadIdx.x / CG;
  const int cg = threadIdx.x % CG;
  const int L = a.full + item, h = L / a.nqt, qt = L - h * a.nqt;
  const int ql = qt * kBM + rl;
  if (ql >= a.lq) return;
  constexpr int64_t slot = kBM * D + kBM;
  const float *base = a.ws + (int64_t)item * a.nsplit * slot;
  float m = -INFINITY;
  for (int p = 0; p < a.nsplit; ++p) m = fmaxf(m, base[p * slot + kBM * D + rl]);
  float wsum = 0.0f;
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int p = 0; p < a.nsplit; ++p) {
    const float wp = __builtin_amdgcn_exp2f(base[p * slot + kBM * D + rl] - m);
    wsum += wp;
    acc += wp * *(const f32x4 *)(base + p * slot + rl * D + 4 * cg);
  }
  const float inv = 1.0f / wsum;
  const int row = a.o_rows ? a.o_rows[ql] : a.o_row0 + ql;
  uint16_t *op = a.o + (int64_t)row * a.ots + (int64_t)h * a.ohs + 4 * cg;
  *(i32x2 *)op = i32x2{(int)pack_bf16x2(acc[0] * inv, acc[1] * inv), (int)pack_bf16x2(acc[2] * inv, acc[3] * inv)};
}

bool aligned(const void *p, int bytes) { return ((uintptr_t)p % bytes) == 0; }

int64_t split_slot_bytes(int D) { return (int64_t)kBM * (D + 1) * 4; }

// Key ranges per remaining item: as many as fit the CUs the whole items leave
// free in the last round, at most 8, each at least 4 tiles long.
int choose_split(int items, int cus, int ntiles) {
  if (cus <= 0) return 1;
  const int rem = items % cus;
  if (rem == 0) return 1;
  int n = cus / rem;
  n = n < 8 ? n : 8;
  n = n < ntiles / 4 ? n : ntiles / 4;
  return n > 1 ? n : 1;
}

// The INT8-QK kernel's last round, over `slots` resident workgroups (two per
// CU): the rem items it holds run as n key ranges each, n (at most 8, each
// range at least 4 key tiles, rem * n within the workspace's max_parts)
// chosen to make the round shortest, ceil(rem * n / slots) sub-rounds of 1 / n
// of an item (the earliest n on ties).  A round that fills three quarters of
// the slots, as at 768p (1,920 items on 512 slots: 384), runs as 4 ranges in 3
// full sub-rounds, 0.75 of an item instead of 1; a round of at most half the
// slots gets the choose_split ranges.
int choose_split_i8(int items, int slots, int ntiles, int64_t max_parts) {
  if (slots <= 0) return 1;
  const int rem = items % slots;
  if (rem == 0) return 1;
  int best = 1;
  int64_t best_rounds = 1, best_n = 1;  // the round lasts best_rounds / best_n items
  for (int n = 2; n <= 8 && n <= ntiles / 4; ++n) {
    if ((int64_t)rem * n > max_parts) break;
    const int64_t rounds = ((int64_t)rem * n + slots - 1) / slots;
    if (rounds * best_n < best_rounds * n) {
      best = n;
      best_rounds = rounds;
      best_n = n;
    }
  }
  return best;
}

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
  if (args->split_workspace && (!aligned(args->split_workspace, 16) || args->split_workspace_bytes < 0))
    return set_error(TMHD_ERR_INVALID, "attention: split workspace must be 16-byte aligned");
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
    if (sg.vt_row_stride % kBN || sg.vt_row_stride < cap || sg.vt_row_stride >= (1 << 23) ||
        sg.vt_head_stride < (int64_t)D * sg.vt_row_stride ||
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
  const int64_t items = (int64_t)k.nqt * k.heads;
  if (items > 0x3fffffff) return set_error(TMHD_ERR_UNSUPPORTED, "attention: grid too large");
  // split the items of the last, partial round into key ranges when a workspace is given
  k.full = (int)items;
  k.nsplit = 1;
  int rem = 0;
  if (args->split_workspace) {
    // workgroups resident at once: one per CU (BF16), two per CU (INT8-QK)
    const int slots = (I8 ? 2 : 1) * device_cus();
    const int n = I8 ? choose_split_i8((int)items, slots, k.ntiles,
                                       args->split_workspace_bytes / split_slot_bytes(args->head_dim))
                     : choose_split((int)items, slots, k.ntiles);
    rem = n > 1 ? (int)(items % slots) : 0;
    if (n > 1 && args->split_workspace_bytes >= (int64_t)rem * n * split_slot_bytes(args->head_dim)) {
      k.full = (int)items - rem;
      k.nsplit = n;
      k.ws = (float *)args->split_workspace;
    } else {
      rem = 0;
    }
  }
  const unsigned grid = (unsigned)(k.full + (int64_t)rem * k.nsplit);
  hipStream_t s = (hipStream_t)stream;
  if (I8 && args->head_dim == 128)
    hipLaunchKernelGGL((attn_i8_kernel<128>), dim3(grid), dim3(kWaves * 64), 0, s, k);
  else if (I8)
    hipLaunchKernelGGL((attn_i8_kernel<64>), dim3(grid), dim3(kWaves * 64), 0, s, k);
  else if (args->head_dim == 128)
    hipLaunchKernelGGL((attn_fwd_kernel<128>), dim3(grid), dim3(kWaves * 64), 0, s, k);
  else
    hipLaunchKernelGGL((attn_fwd_kernel<64>), dim3(grid), dim3(kWaves * 64), 0, s, k);
  const char *what = I8 ? "tmhd_attn_fwd_i8qk" : "tmhd_attn_fwd_bf16";
  int st2 = check_launch(what);
  if (st2 || rem == 0) return st2;
  const unsigned mgrid = (unsigned)rem * (kBM / (256 / (args->head_dim / 4)));
  if (args->head_dim == 128)
    hipLaunchKernelGGL((attn_merge_kernel<128>), dim3(mgrid), dim3(256), 0, s, k);
  else
    hipLaunchKernelGGL((attn_merge_kernel<64>), dim3(mgrid), dim3(256), 0, s, k);
  return check_launch(what);
}

// Device address of `scratch` on the current device, looked up once per
// device (with that device current) and kept; nullptr with the error
// recorded if the lookup fails.
void *static_scratch(const char *what) {
  static std::mutex mu;
  static void *addr[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    set_error(TMHD_ERR_HIP, "%s: no current device", what);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (!addr[dev]) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      set_error(TMHD_ERR_HIP, "%s: scratch address on device %d: %s", what, dev, hipGetErrorString(e));
      return nullptr;
    }
    addr[dev] = p;
  }
  return addr[dev];
}

}  // namespace
}  // namespace tmhd

extern "C" int tmhd_attn_fwd_bf16_noalloc(const tmhd_attn_args *args, void *stream) {
  using namespace tmhd;
  const char *what = "tmhd_attn_fwd_bf16_noalloc";
  if (!args) return set_error(TMHD_ERR_INVALID, "%s: null args", what);
  if (args->split_workspace)
    return set_error(TMHD_ERR_INVALID, "%s: split_workspace must be NULL (the library's static scratch is used)",
                     what);
  KArgs k;
  if (int st = build_kargs(args, nullptr, false, &k)) return st;
  // any call's split needs at most one slot per CU of the device
  const int64_t need = (int64_t)device_cus() * split_slot_bytes(args->head_dim);
  if (need > (int64_t)sizeof(scratch))
    return set_error(TMHD_ERR_UNSUPPORTED, "%s: %lld bytes of split scratch on this device exceed the static %lld",
                     what, (long long)need, (long long)sizeof(scratch));
  void *ws = static_scratch(what);
  if (!ws) return TMHD_ERR_HIP;
  tmhd_attn_args a = *args;
  a.split_workspace = ws;
  a.split_workspace_bytes = (int64_t)sizeof(scratch);
  return launch_attn<false>(&a, nullptr, stream);
}

extern "C" int64_t tmhd_attn_split_workspace_bytes(int32_t head_dim) {
  if (head_dim != 64 && head_dim != 128) return 0;
  // the INT8-QK kernel runs two workgroups per CU, and its split round can
  // take up to three sub-rounds of them
  return 3 * 2 * (int64_t)tmhd::device_cus() * tmhd::split_slot_bytes(head_dim);
}

extern "C" int tmhd_attn_fwd_bf16(const tmhd_attn_args *args, void *stream) {
  return tmhd::launch_attn<false>(args, nullptr, stream);
}

extern "C" int tmhd_attn_fwd_i8qk(const tmhd_attn_args *args, const tmhd_qk_quant *quant, void *stream) {
  return tmhd::launch_attn<true>(args, quant, stream);
}
