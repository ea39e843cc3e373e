/*
 * longctx100m_layer -- MI355X (gfx950) kernels around the attention of one
 * decoder layer's prefill share: RMSNorm (with the residual add fused), RoPE
 * and the SwiGLU gate.  Same library and conventions as longctx100m_attn.h
 * (device pointers, a hipStream_t passed as void*, LC_* status codes,
 * lc_last_error()).  The GEMMs of the layer are plain library GEMMs
 * (hipBLASLt through the caller) and are not part of this ABI.
 *
 * Tensors are row-major.  A "row" is one token: x [rows, cols] for RMSNorm and
 * SwiGLU, [tokens, heads, head_dim] for RoPE (batch folded into tokens: every
 * row of a batch shares the position table of its token index).
 * Arithmetic is fp32; bf16 results are rounded to nearest even at the same
 * points the reference rounds (noted per entry).
 */
#ifndef LONGCTX100M_LAYER_H
#define LONGCTX100M_LAYER_H

#include <stddef.h>
#include <stdint.h>

#include "longctx100m_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* RMSNorm, replacing RmsNorm::forward (rust/longctx100m-model/src/model.rs:53-62;
 * src/longctx100m/model.py:114-118):
 *   h   = x (+ residual, rounded to dtype, when residual != NULL)
 *   out = dtype(dtype(h * 1/sqrt(mean(h^2) + eps)) * weight)
 * h is written to residual_out when that pointer is non-NULL: the decoder's
 * residual stream x + attn(x), model.rs:387-393, computed once.  x, residual,
 * residual_out and out are [rows, cols], each with its own row stride in
 * elements (>= cols, a multiple of 8; residual_out_stride is read only when
 * residual_out is set); weight is [cols].  cols must be a multiple of 8 and
 * <= 16384; pointers 16-byte aligned.  (ABI version 2 added
 * residual_out_stride.) */
int lc_rmsnorm(int32_t dtype, int64_t rows, int32_t cols, float eps, const void* x,
               int64_t x_stride, const void* residual, int64_t residual_stride,
               void* residual_out, int64_t residual_out_stride, const void* weight, void* out,
               int64_t out_stride, void* stream);

/* RoPE scaling profile (rust/longctx100m-model/src/rope.rs:15-99; config
 * rope_scaling).  type: 0 default, 1 linear, 2 llama3. */
typedef struct lc_rope {
  int32_t head_dim; /* even, <= 256 */
  int32_t type;
  double theta;
  double factor;                           /* linear, llama3 */
  double low_freq_factor;                  /* llama3 */
  double high_freq_factor;                 /* llama3 */
  double original_max_position_embeddings; /* llama3 */
  double attention_factor;                 /* llama3 (scales cos only, rope.rs:109-114) */
} lc_rope_t;

/* Inverse frequencies of rope.rs:15-99 on the host (fp32, head_dim / 2 values)
 * and the cosine factor; validation messages are rope.rs's texts. */
int lc_rope_inv_freq(const lc_rope_t* rope, float* inv_freq, float* cos_factor);

/* Position table for tokens pos0 .. pos0 + tokens - 1 (rope.rs:101-114):
 * table [tokens, 2, head_dim / 2] fp32 holding cos(f) * cos_factor and sin(f)
 * with f = position * inv_freq (position scaled by 1/factor for the linear
 * profile). */
int lc_rope_table(const lc_rope_t* rope, int64_t tokens, int64_t pos0, float* table,
                  void* stream);

/* Rotate-half RoPE (rope.rs:116-127): for each [token, head] row of src,
 *   dst[:h] = x1 * cos - x2 * sin,  dst[h:] = x2 * cos + x1 * sin   (h = head_dim / 2)
 * in fp32, rounded to dtype.  src rows may be strided (e.g. the q or k columns
 * of a fused QKV projection: src_token_stride elements between tokens, heads
 * contiguous); dst is contiguous [tokens, heads, head_dim].  dst may equal src
 * when src is contiguous. */
int lc_rope_apply(int32_t dtype, int64_t tokens, int32_t heads, int32_t head_dim,
                  const float* table, const void* src, int64_t src_token_stride, void* dst,
                  void* stream);

/* SwiGLU gate (model.rs:323-327; src/longctx100m/model.py SwiGLU):
 *   out = dtype(dtype(silu(gate)) * up),  silu(g) = g / (1 + exp(-g)) in fp32.  gate and up are [rows, cols] with row
 * strides (e.g. the two halves of one fused gate/up projection); out is
 * contiguous [rows, cols].  cols must be a multiple of 8. */
int lc_swiglu(int32_t dtype, int64_t rows, int32_t cols, const void* gate, int64_t gate_stride,
              const void* up, int64_t up_stride, void* out, void* stream);

/* One token through a bias-free linear layer, replacing candle's Linear
 * forward at M = 1 (rust/longctx100m-model/src/model.rs:64-76, the q/k/v/o
 * projections :99-102, the MLP :290-292) and the LM head matmul (:670-674)
 * in the decode step:
 *   y[n] = dtype( sum_k w[n * w_stride + k] * x[k] ),  n < rows, k < cols
 * with fp32 accumulation.  bf16 only; cols and w_stride multiples of 8,
 * w_stride >= cols, w and x 16-byte aligned.  For more tokens use a GEMM. */
int lc_gemv(int32_t dtype, int64_t rows, int32_t cols, const void* w, int64_t w_stride,
            const void* x, void* y, void* stream);

/* lc_gemv with the row operation before it or after it folded in, so that one
 * launch does what the decode step of a decoder layer otherwise spreads over
 * a norm, a projection and a RoPE / SwiGLU / cast launch.  Every result is
 * bit-identical to the unfused sequence of this library's entry points (same
 * fp32 operations, same reduction orders, bf16 rounding at the same points).
 * The composed reference ops: RmsNorm::forward (model.rs:53-62) with the
 * decoder's residual add (:387-393), the attention output cast to the model
 * dtype, Linear (:64-76), rotate-half RoPE of q and k (rope.rs:116-127) with
 * the token's k and v appended to the KV cache, and SwiGLU (:323-327).
 *
 * Input forms (the bf16 vector the projection multiplies):
 *   LC_GEMV_IN_BF16     x is bf16 [cols], as lc_gemv;
 *   LC_GEMV_IN_F32      x is fp32 [cols], rounded to bf16 (nearest even) first;
 *   LC_GEMV_IN_RMSNORM  x is bf16 [cols]; the vector is lc_rmsnorm of the one
 *                       row x (+ residual) with norm_weight and eps, and
 *                       x + residual is written to residual_out when that is
 *                       set (cols <= 4096; residual_out must not overlap x or
 *                       residual: one workgroup writes it while the others
 *                       still read them).
 * Output forms:
 *   LC_GEMV_OUT_PLAIN     y [rows], as lc_gemv;
 *   LC_GEMV_OUT_SWIGLU    rows = 2 I (gate rows, then up rows, as one fused
 *                         gate/up weight): y [I] = lc_swiglu(gate, up) of the
 *                         two bf16 halves of the product;
 *   LC_GEMV_OUT_ROPE_QKV  rows = (q_heads + 2 kv_heads) head_dim (one fused
 *                         q/k/v weight): y [q_heads head_dim] = lc_rope_apply
 *                         of the q part, k_out [kv_heads head_dim] = that of
 *                         the k part, v_out [kv_heads head_dim] = the v part;
 *                         rope_row is one token's row of lc_rope_table
 *                         ([2, head_dim / 2] fp32), head_dim a multiple of 16
 *                         and <= 256 (as lc_rope_apply).  k_out and v_out may be the token's rows
 *                         of a KV cache.
 * bf16 weights only; cols and w_stride multiples of 8, w_stride >= cols; w,
 * x, residual, residual_out and norm_weight 16-byte aligned, rope_row 4-byte,
 * y, k_out and v_out 2-byte aligned. */
#define LC_GEMV_IN_BF16 0
#define LC_GEMV_IN_F32 1
#define LC_GEMV_IN_RMSNORM 2
#define LC_GEMV_OUT_PLAIN 0
#define LC_GEMV_OUT_SWIGLU 1
#define LC_GEMV_OUT_ROPE_QKV 2

typedef struct lc_gemv_fused {
  int32_t in_form;
  int32_t out_form;
  /* LC_GEMV_IN_RMSNORM */
  const void* residual;    /* bf16 [cols] or NULL */
  void* residual_out;      /* bf16 [cols] or NULL (needs residual) */
  const void* norm_weight; /* bf16 [cols] */
  float eps;
  /* LC_GEMV_OUT_ROPE_QKV */
  int32_t q_heads;
  int32_t kv_heads;
  int32_t head_dim;
  const float* rope_row;
  void* k_out; /* bf16 [kv_heads * head_dim] */
  void* v_out; /* bf16 [kv_heads * head_dim] */
} lc_gemv_fused_t;

int lc_gemv_fused(const lc_gemv_fused_t* f, int64_t rows, int32_t cols, const void* w,
                  int64_t w_stride, const void* x, void* y, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LONGCTX100M_LAYER_H */
