/*
 * tmhd.h - C ABI of libtmhd.so, the gfx950 (MI355X) implementation of the
 * TaoMate-HD streaming KV-cache attention hook and its selective W8A8
 * projection.
 *
 * Every entry point takes plain device pointers, element strides and sizes,
 * plus the HIP stream (passed as void*) the work is ordered on.  The library
 * never allocates or frees device memory: scratch buffers are arguments.
 * Every entry point returns a tmhd_status; 0 means the work was enqueued.
 * tmhd_last_error() returns a message for the calling thread's last failure.
 *
 * Storage formats owned by this library
 * -------------------------------------
 *  Slot (one KV-cache block of one layer, "head-major"):
 *    k  : bf16 [H][cap][D]   row t of head h at k + h*k_head_stride + t*D
 *    vt : bf16 [H][D][cap]   value (h, t, d) at vt + h*vt_head_stride
 *                            + d*vt_row_stride + tmhd_vt_position(t)
 *    cap is a multiple of 64; rows in [tokens, round_up(tokens, 64)) are zero.
 *  tmhd_vt_position(t) swaps the middle two 4-token chunks of every 16-token
 *  group ((t & ~15) | perm[(t >> 2) & 3] << 2 | (t & 3), perm = {0,2,1,3}).
 *  This puts the 8 tokens one MFMA lane consumes for P.V next to each other.
 *
 *  Token-major tensors ([T][H][D], the hook's q/k/v/o) are addressed as
 *  base + row*token_stride + h*head_stride + d, with an optional int32 row
 *  list selecting rows.
 */
#ifndef TMHD_H
#define TMHD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TMHD_MAX_SEGMENTS 16
#define TMHD_KV_TILE 64
#define TMHD_QUANT_BLOCK 128

typedef enum tmhd_status {
  TMHD_OK = 0,
  TMHD_ERR_INVALID = 1,     /* bad pointer, shape, stride or alignment */
  TMHD_ERR_UNSUPPORTED = 2, /* valid but not implemented (e.g. head_dim) */
  TMHD_ERR_HIP = 3          /* a HIP launch failed */
} tmhd_status;

/* One key/value segment of an attention call, stored in slot format. */
typedef struct tmhd_kv_segment {
  const void *k;          /* bf16 slot keys */
  const void *vt;         /* bf16 slot values, transposed and interleaved */
  int64_t k_head_stride;  /* elements between heads of k (>= cap*D) */
  int64_t vt_head_stride; /* elements between heads of vt (>= D*cap) */
  int32_t vt_row_stride;  /* elements between d rows of vt (= cap; below 2^23) */
  int32_t tokens;         /* valid tokens, 0 < tokens <= cap */
} tmhd_kv_segment;

/* softmax(q k^T * scale) v over the concatenation of the segments; no mask. */
typedef struct tmhd_attn_args {
  const void *q;          /* bf16 token-major queries */
  int64_t q_token_stride; /* elements */
  int64_t q_head_stride;  /* elements */
  const int32_t *q_rows;  /* device row list of length lq, or NULL (entries must be valid rows) */
  int32_t q_row0;         /* first row when q_rows is NULL */
  int32_t lq;             /* query rows */
  void *o;                /* bf16 token-major output */
  int64_t o_token_stride;
  int64_t o_head_stride;
  const int32_t *o_rows;  /* device row list of length lq, or NULL (entries must be valid rows) */
  int32_t o_row0;
  int32_t heads;
  int32_t head_dim;       /* 64 or 128 */
  float scale;            /* softmax scale (head_dim ** -0.5 in the model) */
  int32_t n_segments;     /* 1..TMHD_MAX_SEGMENTS */
  tmhd_kv_segment seg[TMHD_MAX_SEGMENTS];
  /*
   * Optional scratch (NULL: none).  The work is one item per (head, 256-row
   * query tile); when the items do not fill the last round of workgroups the
   * device holds at once (one per CU for BF16, two per CU for INT8-QK), the
   * remaining items are split into key ranges whose partial results go here
   * and are merged by a second kernel on the same stream.  Without it
   * (or with fewer bytes than tmhd_attn_split_workspace_bytes) every item runs
   * whole.  Calls that share a workspace must be ordered (same stream).
   */
  void *split_workspace;
  int64_t split_workspace_bytes;
} tmhd_attn_args;

/*
 * Quantized operands of the INT8-QK attention (SageAttention-style).
 *   k_mean[h][d]   = bf16 mean of all keys of the call (all segments)
 *   Q block b of head h: rows [128b, 128b+128) of the call's queries
 *   K block b of segment s, head h: tokens [128b, 128b+128) of the segment
 *   scale = amax / 127, value = sat_int8(rint(x * (127 / amax))), amax = 0 -> 0
 *   with x = q for Q and x = k - k_mean for K (fp32).
 */
typedef struct tmhd_qk_quant {
  int8_t *q_i8;                 /* [H][q_cap][D], q_cap >= round_up(lq, 256) */
  float *q_scale;               /* [H][q_cap / 128] */
  int64_t q_head_stride;        /* elements of q_i8 between heads */
  int32_t q_scale_head_stride;  /* elements of q_scale between heads */
  int32_t reserved0;
  int8_t *k_i8[TMHD_MAX_SEGMENTS];      /* [H][cap][D] per segment */
  float *k_scale[TMHD_MAX_SEGMENTS];    /* [H][cap / 128] per segment */
  int64_t k_head_stride[TMHD_MAX_SEGMENTS];       /* elements */
  int32_t k_scale_head_stride[TMHD_MAX_SEGMENTS]; /* elements */
  uint16_t *k_mean;             /* bf16 [H][D] written by tmhd_qk_smooth_quant (16-byte aligned) */
  int64_t *mean_workspace;      /* int64 [H][D] scratch (8-byte aligned) */
  /* Optional, per segment: the exact fixed-point key sums of segment i from
   * tmhd_k_fixed_sum (int64 [H][D], 8-byte aligned), used in place of summing
   * its keys again; NULL: summed here.  The mean is the same bits either way. */
  const int64_t *k_sum[TMHD_MAX_SEGMENTS];
} tmhd_qk_quant;

/* Library identification: "tmhd <version> gfx950". */
const char *tmhd_version(void);
/* Message of the calling thread's last non-zero status ("" if none). */
const char *tmhd_last_error(void);

/*
 * BF16 streaming attention (serial-mode SDPA semantics).
 * Replaces torch SDPA in _sdpa_from_kv_parts,
 * src/taomate_hd/streaming/attention_hook.py:100-115, including the dense
 * K/V materialisation of _materialize_dense_kv_parts (:56-97): the segments
 * are read in place.
 */
int tmhd_attn_fwd_bf16(const tmhd_attn_args *args, void *stream);

/*
 * Bytes of split_workspace that let every attention call with this head_dim
 * on the current device split its last round, on either backend (six
 * [256][head_dim + 1] fp32 slots per CU: the INT8-QK split round can run up
 * to three sub-rounds of two workgroups per CU; 0 for an unsupported
 * head_dim).  Has no counterpart in the reference: the reference's SDPA /
 * SageAttention calls manage their own scratch.
 */
int64_t tmhd_attn_split_workspace_bytes(int32_t head_dim);

/*
 * tmhd_attn_fwd_bf16 that allocates nothing: args->split_workspace must be
 * NULL, and the key-range partials of a split last round go to a static
 * device array of the library (33,816,576 bytes per device: one
 * [256][head_dim + 1] fp32 slot for each CU of a device with up to 256 CUs;
 * a device with more CUs is refused with TMHD_ERR_UNSUPPORTED).  Same
 * results as tmhd_attn_fwd_bf16 with a workspace of
 * tmhd_attn_split_workspace_bytes, bit for bit.  Every call on one GPU
 * shares that array: calls ordered on one stream are safe, calls that
 * overlap on one GPU (other streams) race.  The first call on a device
 * looks up the array's address there.
 * Has no counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc).
 */
int tmhd_attn_fwd_bf16_noalloc(const tmhd_attn_args *args, void *stream);

/*
 * INT8-QK streaming attention: int8 Q.K^T (int32 accumulate) dequantised by
 * the per-block scales, fp32 online softmax, bf16 P.V with fp32 accumulate.
 * Replaces sageattn_qk_int8_pv_fp8_cuda_sm90 / sage_with_fused_value_padding,
 * src/taomate_hd/streaming/attention_hook.py:335-371 and
 * src/taomate_hd/inference/sage_value_padding.py:79-97.
 * The operands must have been produced by tmhd_qk_smooth_quant.
 */
int tmhd_attn_fwd_i8qk(const tmhd_attn_args *args, const tmhd_qk_quant *quant,
                       void *stream);

/*
 * K token-mean over every segment, then per-128-block INT8 quantization of
 * Q and of K - mean (formula above).  Replaces the k.mean(dim=1) and
 * per_thread_int8_triton step of
 * src/taomate_hd/inference/sage_value_padding.py:89-92.
 */
int tmhd_qk_smooth_quant(const tmhd_attn_args *args, const tmhd_qk_quant *quant,
                         void *stream);

/*
 * sum[h][d] = the exact fixed-point sum (rint(k * 2^24) as int64, wrapping)
 * over the `tokens` slot rows of head h, the per-segment term of the smooth-K
 * mean: a caller that keeps it for a segment whose keys do not change (a
 * cached block) passes it in tmhd_qk_quant.k_sum instead of having every call
 * sum those keys again.  No counterpart in the reference, which recomputes
 * k.mean over every key per call (src/taomate_hd/inference/sage_value_padding.py:89-92).
 */
int tmhd_k_fixed_sum(const void *k, int64_t k_head_stride, int32_t tokens, int32_t heads,
                     int32_t head_dim, int64_t *sum, void *stream);

/*
 * Copy `n` token-major K/V rows into a slot at token offset `dst`, then zero
 * slot rows [dst + n, zero_to).  Source row i is rows[i] (a device list whose
 * entries must be valid source rows; the kernel reads through them) or row0 + i.
 * Replaces the index_select staging and torch.cat commit of
 * src/taomate_hd/streaming/cache.py:273-296 and the dense copies of
 * src/taomate_hd/streaming/attention_hook.py:71-91.
 */
int tmhd_kv_pack(const void *k, const void *v, int64_t token_stride,
                 int64_t head_stride, const int32_t *rows, int32_t row0,
                 int32_t n, void *k_slot, void *vt_slot, int64_t k_head_stride,
                 int64_t vt_head_stride, int32_t vt_row_stride, int32_t dst,
                 int32_t zero_to, int32_t heads, int32_t head_dim, void *stream);

/*
 * Q/K RMSNorm + RoPE in place inside a merged bf16 QKV projection
 * qkv[tokens][row_stride] (Q, K, V of `heads` heads each, head_dim channels;
 * V is neither read nor written).  Per token and head, with x the Q (or K)
 * channels and w q_weight (or k_weight):
 *   n = bf16((x * (1 / sqrt(sum(x^2) / head_dim + eps))) * w)
 *   channel d < rotary_dim: bf16(bf16(n[d] * cos) + bf16(r[d] * sin)), where
 *   r[d] = -n[d + h] (d < h) or n[d - h] (d >= h), h = rotary_dim / 2, and
 *   cos / sin = cos_sin[p][d % h] / cos_sin[p][h + d % h] at p = positions[t]
 *   (clamped to [0, cos_sin_rows)); other channels keep n.
 * bf16() is round-to-nearest-even.  The sum of squares is fixed: the row's
 * channels are dealt to head_dim / 8 partials of 8 (partial j < rotary_dim / 8
 * takes channels 4j..4j+3 then h+4j..h+4j+3, the rest 8 consecutive channels
 * of the tail), each a chain of fused multiply-adds, added as a pairwise tree
 * in order.  The square root and division are correctly rounded.
 * Replaces fused_qkv_qk_norm_rope_ / _merged_qkv_preprocess_kernel,
 * src/taomate_hd/inference/fused_kernels.py:425-472, 824-873.
 * head_dim 64 or 128; rotary_dim a multiple of 8 up to head_dim; qkv rows,
 * weights and cos_sin rows 8-byte aligned.
 */
int tmhd_qkv_norm_rope(void *qkv, int32_t tokens, int32_t heads, int32_t head_dim,
                       int64_t row_stride, const void *q_weight, const void *k_weight,
                       const void *cos_sin, int64_t cos_sin_stride, int64_t cos_sin_rows,
                       int32_t rotary_dim, const int64_t *positions, float eps,
                       void *stream);

/*
 * tmhd_qkv_norm_rope followed by tmhd_kv_pack of the K and V thirds of tokens
 * [stage_row0, stage_row0 + stage_n) into a slot at row `dst` (zeroing slot
 * rows [dst + stage_n, zero_to)), with the same results, in one pass over Q
 * and K: the normalised, rotated K rows go to the slot as they are written
 * back, and only V is read again (for its transpose).  qkv rows must be
 * 16-byte aligned; the slot arguments are those of tmhd_kv_pack.  Replaces
 * the preprocessing of src/taomate_hd/inference/fused_kernels.py:824-873
 * together with the chunk's K/V staging copy in front of the hook
 * (src/taomate_hd/streaming/attention_hook.py:71-91, cache.py:273-296).
 */
int tmhd_qkv_norm_rope_stage(void *qkv, int32_t tokens, int32_t heads, int32_t head_dim,
                             int64_t row_stride, const void *q_weight, const void *k_weight,
                             const void *cos_sin, int64_t cos_sin_stride, int64_t cos_sin_rows,
                             int32_t rotary_dim, const int64_t *positions, float eps,
                             int32_t stage_row0, int32_t stage_n, void *k_slot, void *vt_slot,
                             int64_t k_head_stride, int64_t vt_head_stride, int32_t vt_row_stride,
                             int32_t dst, int32_t zero_to, void *stream);

/*
 * The same RMSNorm + RoPE on one projection value[tokens][heads][head_dim]
 * (row stride value_stride elements, heads * head_dim contiguous), written to
 * out (row stride out_stride; out == value with equal strides is in place,
 * any other overlap is refused), with one weight and per-token rotation
 * tables: channel d < rotary_dim uses cos[t][d] and sin[t][d] (row strides
 * cos_stride / sin_stride), r[d] as above.  Same fixed reduction order and
 * rounding.
 * Replaces fused_qk_norm_rope / _qk_norm_rope_kernel,
 * src/taomate_hd/inference/fused_kernels.py:385-422, 798-821.
 * head_dim 64 or 128; rotary_dim a multiple of 8 up to head_dim; rows 8-byte
 * aligned.
 */
int tmhd_qk_norm_rope(const void *value, int32_t tokens, int32_t heads, int32_t head_dim,
                      int64_t value_stride, void *out, int64_t out_stride,
                      const void *weight, const void *cos, int64_t cos_stride,
                      const void *sin, int64_t sin_stride, int32_t rotary_dim, float eps,
                      void *stream);

/*
 * The rotation alone, without the RMSNorm: out = R(R(x[d] * cos[t][d]) +
 * R(r[d] * sin[t][d])) for d < rotary_dim (r as above, on the input values),
 * x[d] for the other channels.  Same layout, tables and aliasing rules as
 * tmhd_qk_norm_rope.
 * Replaces fused_apply_rope / _rope_kernel,
 * src/taomate_hd/inference/fused_kernels.py:257-297, 673-692.
 */
int tmhd_apply_rope(const void *value, int32_t tokens, int32_t heads, int32_t head_dim,
                    int64_t value_stride, void *out, int64_t out_stride, const void *cos,
                    int64_t cos_stride, const void *sin, int64_t sin_stride, int32_t rotary_dim,
                    void *stream);

/*
 * Ulysses sequence <-> heads layouts (the all-to-all itself is the caller's).
 * A rank holds `tokens` (T) tokens of the sequence with all `heads` (H)
 * heads; after the exchange it holds all U*T tokens of L = ceil(H / U)
 * heads, heads H..U*L-1 being zero padding.  head_dim (D) 64 or 128; world
 * (U) 1..64; buffers and rows 16-byte aligned; outputs may not overlap inputs.
 *
 * tmhd_ulysses_qkv_send: merged projection qkv[T][3][H][D] (row stride
 * row_stride elements) -> the send buffer of the sequence -> heads exchange:
 *   layout 0: out[U][3][T][L][D]   the reference's layout
 *   layout 1: out[U][T][3][L][D]   token-major: the received buffer is then
 *             a merged projection of the U*T tokens (row stride 3*L*D) whose
 *             Q / K / V thirds the hook reads in place (no receive copy)
 * out[dest][part][t][l] = qkv[t][part][dest*L + l] (zero for padded heads).
 * Replaces qkv_send_layout / _qkv_send,
 * src/taomate_hd/distributed/ulysses_layout.py:9-41, as called by
 * merged_qkv_sequence_to_heads (ulysses.py:183-212).
 */
int tmhd_ulysses_qkv_send(const void *qkv, int64_t row_stride, int32_t tokens, int32_t heads,
                          int32_t head_dim, int32_t world, int32_t layout, void *out, void *stream);

/*
 * tmhd_qkv_norm_rope and tmhd_ulysses_qkv_send in one pass: the normalised,
 * rotated Q / K rows go straight into the send buffer (qkv itself is left
 * unchanged); V and the padding come from the plain send.  Same results as
 * the two calls in sequence, bit for bit.  Replaces fused_qkv_qk_norm_rope_
 * (fused_kernels.py:824-873) followed by merged_qkv_sequence_to_heads's send
 * layout (ulysses.py:183-212) in MiniMaxH3Attention.forward (layers.py:400-438).
 */
int tmhd_ulysses_qkv_norm_rope_send(const void *qkv, int64_t row_stride, int32_t tokens,
                                    int32_t heads, int32_t head_dim, const void *q_weight,
                                    const void *k_weight, const void *cos_sin,
                                    int64_t cos_sin_stride, int64_t cos_sin_rows,
                                    int32_t rotary_dim, const int64_t *positions, float eps,
                                    int32_t world, int32_t layout, void *out, void *stream);

/*
 * The received layout-0 buffer recv[U][3][T][L][D] (source rank, part, token,
 * local head) -> out[U*T][3][L][D], row s*T + t at out + (s*T + t) *
 * out_row_stride.  Replaces outputs.movedim(0, 1).contiguous() of
 * merged_qkv_sequence_to_heads (ulysses.py:209-211), in the merged-row form
 * the hook reads.
 */
int tmhd_ulysses_qkv_receive(const void *recv, int32_t tokens, int32_t local_heads,
                             int32_t head_dim, int32_t world, void *out,
                             int64_t out_row_stride, void *stream);

/*
 * The heads -> sequence direction: the received attention output
 * recv[U][T][L][D] (source rank s holds heads s*L..) -> out[t][h][d] at
 * out + t*out_token_stride + h*out_head_stride + d for h < heads (the
 * padded heads are dropped).  Replaces attention_receive_layout /
 * _attention_receive, ulysses_layout.py:44-67, as called by
 * heads_to_sequence (ulysses.py:113-138).
 */
int tmhd_ulysses_attention_receive(const void *recv, int32_t tokens, int32_t heads,
                                   int32_t head_dim, int32_t world, void *out,
                                   int64_t out_token_stride, int64_t out_head_stride,
                                   void *stream);

/*
 * Row-wise bf16 ops of the DiT block around each attention call: `rows`
 * rows of `cols` columns (row strides in elements), bf16 weight [cols],
 * bf16 tables scale / shift / gate [table_rows][*] read at row t =
 * index[row] (int64, clamped to [0, table_rows)).  With R() the bf16
 * round-to-nearest-even and inv = 1 / sqrt(sum(x^2) / cols + eps):
 *   tmhd_rms_norm:          out = R((x * inv) * w)
 *   tmhd_rms_norm_modulate: n = R((x * inv) * w),
 *                           out = R(R(n * R(1 + scale[t])) + shift[t])
 *   tmhd_residual_gate_rms_norm_modulate:
 *                           hidden = R(residual + R(gate[t] * branch)), then
 *                           out = the rms_norm_modulate of hidden
 *   tmhd_modulate:          out = R(R(x * R(1 + scale[t])) + shift[t])
 *   tmhd_gate_add:          out = R(residual + R(gate[t] * branch))
 * The sum of squares is fixed: the row's 8-column chunks are dealt to 64
 * partials (chunk c to partial c % 64), each a chain of fused multiply-adds
 * over its chunks in order, added as a pairwise tree in order; the square
 * root and divisions are correctly rounded.
 * Replace fused_rms_norm, fused_rms_norm_modulate,
 * fused_residual_gate_rms_norm_modulate, fused_modulate and fused_gate_add
 * with their kernels, src/taomate_hd/inference/fused_kernels.py:221-255,
 * 312-383, 636-671, 706-796.
 * cols a multiple of 8 up to 8192; pointers and row strides 16-byte aligned.
 */
int tmhd_rms_norm(const void *x, int64_t x_stride, void *out, int64_t out_stride,
                  const void *weight, int64_t rows, int32_t cols, float eps, void *stream);
int tmhd_rms_norm_modulate(const void *x, int64_t x_stride, void *out, int64_t out_stride,
                           const void *weight, const void *scale, int64_t scale_stride,
                           const void *shift, int64_t shift_stride, const int64_t *index,
                           int64_t table_rows, int64_t rows, int32_t cols, float eps,
                           void *stream);
int tmhd_residual_gate_rms_norm_modulate(const void *residual, int64_t residual_stride,
                                         const void *branch, int64_t branch_stride,
                                         const void *gate, int64_t gate_stride,
                                         const void *weight, const void *scale,
                                         int64_t scale_stride, const void *shift,
                                         int64_t shift_stride, const int64_t *index,
                                         int64_t table_rows, void *hidden,
                                         int64_t hidden_stride, void *out, int64_t out_stride,
                                         int64_t rows, int32_t cols, float eps, void *stream);
int tmhd_modulate(const void *x, int64_t x_stride, void *out, int64_t out_stride,
                  const void *scale, int64_t scale_stride, const void *shift,
                  int64_t shift_stride, const int64_t *index, int64_t table_rows, int64_t rows,
                  int32_t cols, void *stream);
int tmhd_gate_add(const void *residual, int64_t residual_stride, const void *gate,
                  int64_t gate_stride, const void *branch, int64_t branch_stride,
                  const int64_t *index, int64_t table_rows, void *out, int64_t out_stride,
                  int64_t rows, int32_t cols, void *stream);

/*
 * SwiGLU of x[rows][2 * half] (gate columns, then up columns; row stride
 * x_stride elements) into out[rows][half]: out = R(R(g * sigmoid(g)) * u),
 * sigmoid(g) = 1 / (1 + exp(-g)) in single precision (accurate exp,
 * correctly rounded division).  The reference's tl.sigmoid is its
 * compiler's, so agreement is within one bf16 ulp rather than bit-exact.
 * Replaces fused_swiglu / _swiglu_kernel,
 * src/taomate_hd/inference/fused_kernels.py:299-310, 694-704.
 * half a multiple of 8; pointers and row strides 16-byte aligned.
 */
int tmhd_swiglu(const void *x, int64_t x_stride, void *out, int64_t out_stride, int64_t rows,
                int32_t half, void *stream);

/*
 * No counterpart in the reference: a device self-check for deployments and
 * tests.  Runs every one of the 2^32 float bit patterns through the two
 * rounding helpers the norm + RoPE kernels depend on and adds the failures
 * to counts[0] (f32 -> bf16 conversion differing from the reference's
 * integer rounding, fused_kernels.py:58-61, on any non-NaN value or quiet NaN
 * with a zero low half) and counts[1] (square root not correctly rounded).
 * counts: two device uint64 the caller has zeroed; both stay 0 on a sound
 * device.  A few milliseconds on the stream.
 */
int tmhd_selfcheck_rounding(unsigned long long *counts, void *stream);

/*
 * Per-token dynamic symmetric INT8 quantization of a bf16 [rows][cols]
 * matrix (row stride x_stride elements): scale[m] = amax_m / 127,
 * q[m][k] = sat_int8(rint(x[m][k] * (127 / amax_m))), amax_m = 0 -> 0.
 * Replaces vLLM dynamic_scaled_int8_quant / scaled_int8_quant called at
 * src/taomate_hd/inference/w8a8.py:71 and :141.
 */
int tmhd_token_quant_i8(int8_t *q, float *scale, const void *x, int32_t rows,
                        int32_t cols, int64_t x_stride, void *stream);

/*
 * Static per-output-channel INT8 weight quantization of a bf16 [n][k]
 * weight: scale[r] = max(amax_r / 127, 1e-12),
 * q[r][c] = clamp(rint(w[r][c] / scale[r]), -127, 127).
 * Replaces _quantize_cutlass_w8a8_weight, src/taomate_hd/inference/w8a8.py:175-179.
 */
int tmhd_weight_quant_i8(int8_t *q, float *scale, const void *w, int32_t n,
                         int32_t k, void *stream);

/*
 * Scaled INT8 GEMM with a bf16 epilogue:
 *   acc[m][n] = sum_k a[m][k] * b[n][k]                  (exact int32)
 *   out[m][n] = bf16(float(acc) * b_scale[n] * a_scale[m] + bias[n])
 * evaluated in fp32 in that order (bias term skipped when bias is NULL).
 * a is row-major [m][k] (stride lda), b is the row-major [n][k] weight
 * (stride ldb), i.e. the [k][n] column-major operand of cutlass_scaled_mm.
 * Replaces vLLM cutlass_scaled_mm called at
 * src/taomate_hd/inference/w8a8.py:72 and :142-144.
 * k must be a multiple of 64 (a multiple of 128 takes the faster
 * one-wave-per-SIMD kernel); a, b rows 16-byte aligned.
 */
int tmhd_gemm_w8a8(void *out, const int8_t *a, const int8_t *b,
                   const float *a_scale, const float *b_scale,
                   const void *bias, int32_t m, int32_t n, int32_t k,
                   int64_t lda, int64_t ldb, int64_t ldo, void *stream);

/*
 * The same GEMM writing the raw int32 accumulators (no scales, no bias).
 * No counterpart in the reference: it exposes the accumulators that
 * cutlass_scaled_mm keeps internal, for exactness checks.
 */
int tmhd_gemm_i8_i32(int32_t *out, const int8_t *a, const int8_t *b, int32_t m,
                     int32_t n, int32_t k, int64_t lda, int64_t ldb,
                     int64_t ldo, void *stream);

/*
 * No counterpart in the reference (the caller-provided scratch of the two
 * GEMMs above).  When the 256 x 256 tiles leave a last round that fills at
 * most half of the CUs (or fill less than half in all), that round's tiles
 * are split along k into up to CUs / tiles parts of at least 256 bytes of k;
 * the parts' int32 partial tiles go to `workspace` and a second pass adds
 * them (exactly) and applies the same epilogue, so results are bit-identical
 * to the unsplit GEMM.  tmhd_gemm_split_workspace_bytes gives the bytes this
 * needs on the current device for the shape (0: no split); with a smaller or
 * null workspace the _ws calls run unsplit.  Partial tiles of calls that
 * overlap on one workspace race.  A last round of at most an eighth of the
 * CUs' tiles needs no workspace in these two GEMMs: it runs as 64 x 128
 * sub-tiles over the whole of k (bit-identical too), with or without one;
 * the SwiGLU GEMM below splits it along k.
 */
int64_t tmhd_gemm_split_workspace_bytes(int32_t m, int32_t n, int32_t k);
int tmhd_gemm_w8a8_ws(void *out, const int8_t *a, const int8_t *b, const float *a_scale,
                      const float *b_scale, const void *bias, int32_t m, int32_t n, int32_t k,
                      int64_t lda, int64_t ldb, int64_t ldo, void *workspace,
                      int64_t workspace_bytes, void *stream);
int tmhd_gemm_i8_i32_ws(int32_t *out, const int8_t *a, const int8_t *b, int32_t m, int32_t n,
                        int32_t k, int64_t lda, int64_t ldb, int64_t ldo, void *workspace,
                        int64_t workspace_bytes, void *stream);

/*
 * No counterpart in the reference as one call: FC1 of the DiT MLP followed by
 * SwiGLU (fused_kernels.py:694-704 applied to the W8A8 projection,
 * model/layers.py:525-534), without writing the [m][n] projection.  b holds
 * the n = 2 * f weight rows interleaved in blocks of 256: rows [256t,
 * 256t + 128) are gate rows [128t, 128t + 128) and rows [256t + 128,
 * 256t + 256) the matching up rows; b_scale (and bias) follow the same
 * order.  out[m][j] (j < n / 2, row stride ldo) = R(R(g * sigmoid(g)) * u)
 * of g, u = the bf16 projection values of tmhd_gemm_w8a8 for gate j and up j,
 * the SwiGLU of tmhd_swiglu: bit-identical to tmhd_gemm_w8a8 then
 * tmhd_swiglu on the de-interleaved projection.  n a multiple of 256, k of
 * 128; out 16-byte aligned rows; same optional split workspace as
 * tmhd_gemm_w8a8_ws.
 */
int tmhd_gemm_w8a8_swiglu_ws(void *out, const int8_t *a, const int8_t *b, const float *a_scale,
                             const float *b_scale, const void *bias, int32_t m, int32_t n,
                             int32_t k, int64_t lda, int64_t ldb, int64_t ldo, void *workspace,
                             int64_t workspace_bytes, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* TMHD_H */
