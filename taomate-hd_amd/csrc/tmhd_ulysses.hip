// Ulysses sequence <-> heads layouts on each side of the all-to-alls that
// bracket the streaming attention, for gfx950.  Reference:
// src/taomate_hd/distributed/ulysses_layout.py:9-67 (_qkv_send,
// _attention_receive) and their callers, distributed/ulysses.py:113-212.
//
// A rank holds T tokens of the sequence and all H heads; the exchange gives
// it all U * T tokens of L = ceil(H / U) heads (zero-padded when U does not
// divide H).
//   send     merged QKV [T][3 H D] (row stride S)  ->  send buffer
//              layout 0 (the reference's): [U][3][T][L][D]
//              layout 1 (token-major):     [U][T][3][L][D]
//            chunk dest goes to rank dest; heads dest*L + l >= H are zero.
//            With layout 1 the received buffer [U][T][3][L][D] already is a
//            merged projection of the U*T tokens (row stride 3 L D), so the
//            hook reads its Q / K / V thirds in place and no receive copy runs.
//   receive  layout-0 QKV buffer [U][3][T][L][D] -> merged [U T][3][L][D]
//            (the reference's movedim + contiguous, ulysses.py:209-211);
//            attention output [U][T][L][D] from the heads -> sequence
//            exchange -> [T][H][D] (padded heads dropped).
// Every kernel is a 16-byte-per-lane copy: a block is 4 token rows of 64
// lanes, each lane striding over the L * D / 8 chunks of its (token, rank,
// part) row, so both sides stream whole rows and no index needs a division
// by a run-time value.
#include "tmhd_internal.h"

namespace tmhd {
namespace {

constexpr int kRowsPerBlock = 4;

struct SendArgs {
  const uint16_t *src;
  int64_t src_stride;  // elements between tokens of the merged projection
  uint16_t *dst;
  int32_t tokens, heads, local, world, layout;
  int32_t copy_parts;  // bit p: copy the real heads of part p (padded heads are always zeroed)
};

template <int D>
__global__ void __launch_bounds__(256) ulysses_send_kernel(const SendArgs a) {
  constexpr int CPH = D / 8;  // 16-byte chunks per head row
  const int t = blockIdx.x * kRowsPerBlock + threadIdx.y;
  if (t >= a.tokens) return;
  const int dp = blockIdx.y, dest = dp / 3, p = dp - 3 * dest;
  const int row_chunks = a.local * CPH;
  const int64_t row = a.layout == 0 ? (int64_t)dp * a.tokens + t : ((int64_t)dest * a.tokens + t) * 3 + p;
  i32x4 *out = (i32x4 *)(a.dst + row * row_chunks * 8);
  const bool copy = (a.copy_parts >> p) & 1;
  const uint16_t *in = a.src + (int64_t)t * a.src_stride + ((int64_t)p * a.heads + (int64_t)dest * a.local) * D;
  const int real = min(a.heads - dest * a.local, a.local) * CPH;  // chunks of real heads in this row
  for (int c = threadIdx.x; c < row_chunks; c += 64) {
    if (c >= real)
      out[c] = i32x4{0, 0, 0, 0};
    else if (copy)
      out[c] = *(const i32x4 *)(in + c * 8);
  }
}

struct RecvArgs {
  const uint16_t *src;
  uint16_t *dst;
  int64_t dst_token_stride, dst_head_stride;
  int32_t tokens, heads, local, world;
};

// layout-0 QKV receive: [U][3][T][L][D] -> dst row s*T + t, part p at p*L*D
template <int D>
__global__ void __launch_bounds__(256) ulysses_qkv_receive_kernel(const RecvArgs a) {
  constexpr int CPH = D / 8;
  const int t = blockIdx.x * kRowsPerBlock + threadIdx.y;
  if (t >= a.tokens) return;
  const int sp = blockIdx.y, s = sp / 3, p = sp - 3 * s;
  const int row_chunks = a.local * CPH;
  const i32x4 *in = (const i32x4 *)(a.src + ((int64_t)sp * a.tokens + t) * row_chunks * 8);
  i32x4 *out = (i32x4 *)(a.dst + ((int64_t)s * a.tokens + t) * a.dst_token_stride + (int64_t)p * a.local * D);
  for (int c = threadIdx.x; c < row_chunks; c += 64) out[c] = in[c];
}

// attention receive: [U][T][L][D] -> dst[t][s*L + l] for the real heads
template <int D>
__global__ void __launch_bounds__(256) ulysses_attention_receive_kernel(const RecvArgs a) {
  constexpr int CPH = D / 8;
  const int t = blockIdx.x * kRowsPerBlock + threadIdx.y;
  if (t >= a.tokens) return;
  const int s = blockIdx.y;
  const int real = min(a.heads - s * a.local, a.local) * CPH;
  const i32x4 *in = (const i32x4 *)(a.src + ((int64_t)s * a.tokens + t) * a.local * D);
  uint16_t *out = a.dst + (int64_t)t * a.dst_token_stride + (int64_t)s * a.local * a.dst_head_stride;
  for (int c = threadIdx.x; c < real; c += 64) {
    const int l = c / CPH, k = c - l * CPH;  // CPH is a power of two
    *(i32x4 *)(out + l * a.dst_head_stride + k * 8) = in[c];
  }
}

bool aligned16(const void *p) { return ((uintptr_t)p % 16) == 0; }

int check_world(int32_t tokens, int32_t heads, int32_t head_dim, int32_t world, const char *what) {
  if (head_dim != 64 && head_dim != 128)
    return set_error(TMHD_ERR_UNSUPPORTED, "%s: head_dim %d (64 or 128)", what, head_dim);
  if (tokens < 0 || heads <= 0 || world < 1 || world > 64)
    return set_error(TMHD_ERR_INVALID, "%s: tokens %d heads %d world %d (1..64)", what, tokens, heads, world);
  const int64_t local = (heads + world - 1) / world;
  if ((int64_t)world * 3 * tokens * local * head_dim / 8 > 0x7fffffff)
    return set_error(TMHD_ERR_UNSUPPORTED, "%s: buffer too large", what);
  if (((int64_t)tokens + kRowsPerBlock - 1) / kRowsPerBlock > 0x7fffffff)
    return set_error(TMHD_ERR_UNSUPPORTED, "%s: too many tokens", what);
  return TMHD_OK;
}

dim3 row_grid(int32_t tokens, int32_t y) {
  return dim3((unsigned)((tokens + kRowsPerBlock - 1) / kRowsPerBlock), (unsigned)y);
}

}  // namespace

// Shared with the norm + RoPE send (tmhd_rope.hip): validates and launches
// the plain send for the parts in copy_parts.
int ulysses_send(const void *qkv, int64_t row_stride, int32_t tokens, int32_t heads, int32_t head_dim,
                 int32_t world, int32_t layout, void *out, int32_t copy_parts, void *stream, bool check_only) {
  const char *what = "tmhd_ulysses_qkv_send";
  if (int st = check_world(tokens, heads, head_dim, world, what)) return st;
  if (layout != 0 && layout != 1) return set_error(TMHD_ERR_INVALID, "%s: layout %d (0 or 1)", what, layout);
  if (row_stride < (int64_t)3 * heads * head_dim)
    return set_error(TMHD_ERR_INVALID, "%s: row_stride %lld below 3 * heads * head_dim", what,
                     (long long)row_stride);
  if (tokens == 0) return TMHD_OK;
  if (!qkv || !out || !aligned16(qkv) || !aligned16(out) || row_stride % 8)
    return set_error(TMHD_ERR_INVALID, "%s: qkv rows and out must be 16-byte aligned", what);
  const int32_t local = (heads + world - 1) / world;
  const char *o0 = (const char *)out, *q0 = (const char *)qkv;
  const int64_t ob = (int64_t)world * 3 * tokens * local * head_dim * 2;
  const int64_t qb = ((int64_t)(tokens - 1) * row_stride + (int64_t)3 * heads * head_dim) * 2;
  if (o0 < q0 + qb && q0 < o0 + ob) return set_error(TMHD_ERR_INVALID, "%s: out overlaps qkv", what);
  if (check_only) return TMHD_OK;
  SendArgs a{(const uint16_t *)qkv, row_stride, (uint16_t *)out, tokens, heads, local, world, layout, copy_parts};
  const dim3 grid = row_grid(tokens, 3 * world), block(64, kRowsPerBlock);
  hipStream_t s = (hipStream_t)stream;
  if (head_dim == 128)
    hipLaunchKernelGGL(ulysses_send_kernel<128>, grid, block, 0, s, a);
  else
    hipLaunchKernelGGL(ulysses_send_kernel<64>, grid, block, 0, s, a);
  return check_launch(what);
}

}  // namespace tmhd

extern "C" int tmhd_ulysses_qkv_send(const void *qkv, int64_t row_stride, int32_t tokens, int32_t heads,
                                     int32_t head_dim, int32_t world, int32_t layout, void *out, void *stream) {
  return tmhd::ulysses_send(qkv, row_stride, tokens, heads, head_dim, world, layout, out, 7, stream, false);
}

extern "C" int tmhd_ulysses_qkv_receive(const void *recv, int32_t tokens, int32_t local_heads, int32_t head_dim,
                                        int32_t world, void *out, int64_t out_row_stride, void *stream) {
  using namespace tmhd;
  const char *what = "tmhd_ulysses_qkv_receive";
  if (local_heads <= 0 || world < 1 || world > 64)
    return set_error(TMHD_ERR_INVALID, "%s: local_heads %d world %d", what, local_heads, world);
  if (int st = check_world(tokens, local_heads * world, head_dim, world, what)) return st;
  if ((int64_t)world * tokens > 0x7fffffff) return set_error(TMHD_ERR_UNSUPPORTED, "%s: too many tokens", what);
  if (out_row_stride < (int64_t)3 * local_heads * head_dim)
    return set_error(TMHD_ERR_INVALID, "%s: out_row_stride below 3 * local_heads * head_dim", what);
  if (tokens == 0) return TMHD_OK;
  if (!recv || !out || !aligned16(recv) || !aligned16(out) || out_row_stride % 8)
    return set_error(TMHD_ERR_INVALID, "%s: buffers and out rows must be 16-byte aligned", what);
  const char *r0 = (const char *)recv, *o0 = (const char *)out;
  const int64_t rb = (int64_t)world * 3 * tokens * local_heads * head_dim * 2;
  const int64_t ob = (((int64_t)world * tokens - 1) * out_row_stride + (int64_t)3 * local_heads * head_dim) * 2;
  if (o0 < r0 + rb && r0 < o0 + ob) return set_error(TMHD_ERR_INVALID, "%s: out overlaps the received buffer", what);
  RecvArgs a{(const uint16_t *)recv, (uint16_t *)out, out_row_stride, 0, tokens, 0, local_heads, world};
  const dim3 grid = row_grid(tokens, 3 * world), block(64, kRowsPerBlock);
  hipStream_t s = (hipStream_t)stream;
  if (head_dim == 128)
    hipLaunchKernelGGL(ulysses_qkv_receive_kernel<128>, grid, block, 0, s, a);
  else
    hipLaunchKernelGGL(ulysses_qkv_receive_kernel<64>, grid, block, 0, s, a);
  return check_launch(what);
}

extern "C" int tmhd_ulysses_attention_receive(const void *recv, int32_t tokens, int32_t heads, int32_t head_dim,
                                              int32_t world, void *out, int64_t out_token_stride,
                                              int64_t out_head_stride, void *stream) {
  using namespace tmhd;
  const char *what = "tmhd_ulysses_attention_receive";
  if (int st = check_world(tokens, heads, head_dim, world, what)) return st;
  if (out_head_stride < head_dim || out_token_stride < (int64_t)(heads - 1) * out_head_stride + head_dim)
    return set_error(TMHD_ERR_INVALID, "%s: out strides %lld / %lld", what, (long long)out_token_stride,
                     (long long)out_head_stride);
  if (tokens == 0) return TMHD_OK;
  if (!recv || !out || !aligned16(recv) || !aligned16(out) || out_token_stride % 8 || out_head_stride % 8)
    return set_error(TMHD_ERR_INVALID, "%s: buffers and out rows must be 16-byte aligned", what);
  const int32_t local = (heads + world - 1) / world;
  const char *r0 = (const char *)recv, *o0 = (const char *)out;
  const int64_t rb = (int64_t)world * tokens * local * head_dim * 2;
  const int64_t ob = ((int64_t)(tokens - 1) * out_token_stride + (int64_t)(heads - 1) * out_head_stride + head_dim) * 2;
  if (o0 < r0 + rb && r0 < o0 + ob) return set_error(TMHD_ERR_INVALID, "%s: out overlaps the received buffer", what);
  RecvArgs a{(const uint16_t *)recv, (uint16_t *)out, out_token_stride, out_head_stride, tokens, heads, local, world};
  const dim3 grid = row_grid(tokens, world), block(64, kRowsPerBlock);
  hipStream_t s = (hipStream_t)stream;
  if (head_dim == 128)
    hipLaunchKernelGGL(ulysses_attention_receive_kernel<128>, grid, block, 0, s, a);
  else
    hipLaunchKernelGGL(ulysses_attention_receive_kernel<64>, grid, block, 0, s, a);
  return check_launch(what);
}
