// C-ABI entry points of the decoder-layer row kernels (include/longctx100m_layer.h).
//
// The RoPE inverse frequencies are computed here on the host in fp32, as a
// literal restatement of rust/longctx100m-model/src/rope.rs:15-99 (candle's
// affine(mul, add) is x * (float)mul + (float)add on an fp32 tensor), so the
// table kernel multiplies exactly the values the reference multiplies.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "longctx100m_layer.h"
#include "kernels.h"

// The reference rounds after every tensor op; keep the host arithmetic unfused.
#pragma clang fp contract(off)

namespace {

using lc::hip_error;
using lc::set_error;

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_dtype(int32_t dtype) {
  if (dtype != LC_DTYPE_F32 && dtype != LC_DTYPE_BF16)
    return set_error(LC_ERR_UNSUPPORTED, "unsupported dtype %d", dtype);
  return LC_OK;
}

// Row strides must keep every 8-element chunk 16-byte aligned.
bool stride_ok(int64_t stride, int64_t min) { return stride >= min && stride % 8 == 0; }

}  // namespace

extern "C" {

int lc_rmsnorm(int32_t dtype, int64_t rows, int32_t cols, float eps, const void* x,
               int64_t x_stride, const void* residual, int64_t residual_stride,
               void* residual_out, int64_t residual_out_stride, const void* weight, void* out,
               int64_t out_stride, void* stream) {
  if (int rc = check_dtype(dtype)) return rc;
  if (rows < 0 || cols <= 0 || cols % 8 != 0 || cols > 16384)
    return set_error(LC_ERR_INVALID, "rmsnorm needs rows >= 0 and 0 < cols <= 16384, cols %% 8 == 0");
  if (!x || !weight || !out) return set_error(LC_ERR_INVALID, "null pointer argument");
  if (residual_out && !residual)
    return set_error(LC_ERR_INVALID, "residual_out needs a residual input");
  if (!stride_ok(x_stride, cols) || !stride_ok(out_stride, cols) ||
      (residual && !stride_ok(residual_stride, cols)) ||
      (residual_out && !stride_ok(residual_out_stride, cols)))
    return set_error(LC_ERR_INVALID, "row strides must be >= cols and multiples of 8 elements");
  if (!aligned16(x) || !aligned16(weight) || !aligned16(out) ||
      (residual && !aligned16(residual)) || (residual_out && !aligned16(residual_out)))
    return set_error(LC_ERR_INVALID, "rmsnorm pointers must be 16-byte aligned");
  if (!(eps >= 0.f)) return set_error(LC_ERR_INVALID, "eps must be non-negative");
  hipError_t e = lc::launch_rmsnorm(dtype, rows, cols, eps, x, x_stride, residual,
                                    residual_stride, residual_out, residual_out_stride, weight,
                                    out, out_stride, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? LC_OK : hip_error(e, "rmsnorm launch");
}

int lc_rope_inv_freq(const lc_rope_t* rope, float* inv_freq, float* cos_factor) {
  if (!rope || !inv_freq || !cos_factor) return set_error(LC_ERR_INVALID, "null pointer argument");
  const int dim = rope->head_dim;
  if (dim <= 0 || dim % 2 != 0 || dim > 256)
    return set_error(LC_ERR_INVALID, "head dimension must be even for rotary embeddings");
  if (!(rope->theta > 0.0)) return set_error(LC_ERR_INVALID, "rope theta must be positive");
  const int half = dim / 2;
  // inv = exp(arange(half) * (-2 ln theta / dim))   (rope.rs:15-22)
  const float mul = (float)(-2.0 * std::log(rope->theta) / (double)dim);
  for (int i = 0; i < half; ++i) inv_freq[i] = std::exp((float)i * mul + 0.0f);
  *cos_factor = 1.0f;
  switch (rope->type) {
    case 0:
      return LC_OK;
    case 1:  // linear: positions / factor (rope.rs:33-40); the table applies it
      if (!(rope->factor > 0.0))
        return set_error(LC_ERR_INVALID, "rope scaling factor must be positive");
      return LC_OK;
    case 2: {  // llama3 (rope.rs:41-96), step for step in fp32
      const double low = rope->low_freq_factor, high = rope->high_freq_factor;
      const double original = rope->original_max_position_embeddings;
      if (!(low > 0.0) || !(high > low) || !(original > 0.0))
        return set_error(LC_ERR_INVALID, "invalid llama3 RoPE scaling values");
      if (!(rope->attention_factor > 0.0))
        return set_error(LC_ERR_INVALID, "llama3 attention_factor must be positive");
      const double factor = rope->factor > 0.0 ? rope->factor : 1.0;
      const double two_pi = 2.0 * M_PI;
      const float low_wavelen = (float)(original / low);
      const float high_wavelen = (float)(original / high);
      for (int i = 0; i < half; ++i) {
        const float inv = inv_freq[i];
        // wavelength = inv.affine(2*pi, 0).div(&inv)   (rope.rs:70)
        const float wavelength = (inv * (float)two_pi + 0.0f) / inv;
        const float scaled = inv * (float)(1.0 / factor) + 0.0f;
        const float smooth = (1.0f / wavelength) * (float)(original / (high - low)) +
                             (float)(-(low / (high - low)));
        const float mid = (smooth * -1.0f + 1.0f) * scaled + smooth * inv;
        float r = wavelength > low_wavelen ? scaled : inv;
        if (wavelength >= high_wavelen && wavelength <= low_wavelen) r = mid;
        inv_freq[i] = r;
      }
      *cos_factor = (float)rope->attention_factor;
      return LC_OK;
    }
    default:
      return set_error(LC_ERR_INVALID, "unsupported RoPE type %d", rope->type);
  }
}

int lc_rope_table(const lc_rope_t* rope, int64_t tokens, int64_t pos0, float* table,
                  void* stream) {
  float inv[128];
  float cos_factor = 1.0f;
  if (int rc = lc_rope_inv_freq(rope, inv, &cos_factor)) return rc;
  if (tokens < 0 || pos0 < 0) return set_error(LC_ERR_INVALID, "tokens and pos0 must be >= 0");
  if (!table) return set_error(LC_ERR_INVALID, "null pointer argument");
  const bool linear = rope->type == 1;
  const float pos_scale = linear ? (float)(1.0 / rope->factor) : 1.0f;
  hipError_t e = lc::launch_rope_table(inv, rope->head_dim / 2, cos_factor, linear, pos_scale,
                                       tokens, pos0, table, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? LC_OK : hip_error(e, "rope table launch");
}

int lc_rope_apply(int32_t dtype, int64_t tokens, int32_t heads, int32_t head_dim,
                  const float* table, const void* src, int64_t src_token_stride, void* dst,
                  void* stream) {
  if (int rc = check_dtype(dtype)) return rc;
  if (tokens < 0 || heads <= 0)
    return set_error(LC_ERR_INVALID, "rope needs tokens >= 0 and heads > 0");
  if (head_dim <= 0 || head_dim % 16 != 0 || head_dim > 256)
    return set_error(LC_ERR_UNSUPPORTED, "rope kernel needs head_dim %% 16 == 0 and <= 256");
  if (!table || !src || !dst) return set_error(LC_ERR_INVALID, "null pointer argument");
  if (!stride_ok(src_token_stride, (int64_t)heads * head_dim))
    return set_error(LC_ERR_INVALID, "src token stride must be >= heads*head_dim, a multiple of 8");
  if (!aligned16(table) || !aligned16(src) || !aligned16(dst))
    return set_error(LC_ERR_INVALID, "rope pointers must be 16-byte aligned");
  if (dst == src && src_token_stride != (int64_t)heads * head_dim)
    return set_error(LC_ERR_INVALID, "in-place rope needs a contiguous source");
  hipError_t e = lc::launch_rope_apply(dtype, tokens, heads, head_dim, table, src,
                                       src_token_stride, dst, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? LC_OK : hip_error(e, "rope apply launch");
}

int lc_swiglu(int32_t dtype, int64_t rows, int32_t cols, const void* gate, int64_t gate_stride,
              const void* up, int64_t up_stride, void* out, void* stream) {
  if (int rc = check_dtype(dtype)) return rc;
  if (rows < 0 || cols <= 0 || cols % 8 != 0)
    return set_error(LC_ERR_INVALID, "swiglu needs rows >= 0 and cols > 0, cols %% 8 == 0");
  if (!gate || !up || !out) return set_error(LC_ERR_INVALID, "null pointer argument");
  if (!stride_ok(gate_stride, cols) || !stride_ok(up_stride, cols))
    return set_error(LC_ERR_INVALID, "row strides must be >= cols and multiples of 8 elements");
  if (!aligned16(gate) || !aligned16(up) || !aligned16(out))
    return set_error(LC_ERR_INVALID, "swiglu pointers must be 16-byte aligned");
  hipError_t e = lc::launch_swiglu(dtype, rows, cols, gate, gate_stride, up, up_stride, out,
                                   static_cast<hipStream_t>(stream));
  return e == hipSuccess ? LC_OK : hip_error(e, "swiglu launch");
}

int lc_gemv(int32_t dtype, int64_t rows, int32_t cols, const void* w, int64_t w_stride,
            const void* x, void* y, void* stream) {
  if (int rc = check_dtype(dtype)) return rc;
  if (dtype != LC_DTYPE_BF16) return set_error(LC_ERR_UNSUPPORTED, "gemv supports bf16 only");
  if (rows < 0 || cols <= 0 || cols % 8 != 0)
    return set_error(LC_ERR_INVALID, "gemv needs rows >= 0 and cols > 0, cols %% 8 == 0");
  if (!w || !x || !y) return set_error(LC_ERR_INVALID, "null pointer argument");
  if (!stride_ok(w_stride, cols))
    return set_error(LC_ERR_INVALID, "row strides must be >= cols and multiples of 8 elements");
  if (!aligned16(w) || !aligned16(x))
    return set_error(LC_ERR_INVALID, "gemv w and x must be 16-byte aligned");
  if (rows == 0) return LC_OK;
  hipError_t e = lc::launch_gemv_bf16(rows, cols, w, w_stride, x, y,
                                      static_cast<hipStream_t>(stream));
  return e == hipSuccess ? LC_OK : hip_error(e, "gemv launch");
}

int lc_gemv_fused(const lc_gemv_fused_t* f, int64_t rows, int32_t cols, const void* w,
                  int64_t w_stride, const void* x, void* y, void* stream) {
  if (!f) return set_error(LC_ERR_INVALID, "null pointer argument");
  if (rows < 0 || cols <= 0 || cols % 8 != 0)
    return set_error(LC_ERR_INVALID, "gemv needs rows >= 0 and cols > 0, cols %% 8 == 0");
  if (!w || !x || !y) return set_error(LC_ERR_INVALID, "null pointer argument");
  if (!stride_ok(w_stride, cols))
    return set_error(LC_ERR_INVALID, "row strides must be >= cols and multiples of 8 elements");
  if (!aligned16(w) || !aligned16(x))
    return set_error(LC_ERR_INVALID, "gemv w and x must be 16-byte aligned");
  if (reinterpret_cast<uintptr_t>(y) & 1u)
    return set_error(LC_ERR_INVALID, "gemv y must be 2-byte aligned");
  switch (f->in_form) {
    case LC_GEMV_IN_BF16:
    case LC_GEMV_IN_F32:
      break;
    case LC_GEMV_IN_RMSNORM:
      if (cols > 4096)
        return set_error(LC_ERR_INVALID, "the folded rmsnorm needs cols <= 4096");
      if (!f->norm_weight) return set_error(LC_ERR_INVALID, "rmsnorm needs norm_weight");
      if (f->residual_out && !f->residual)
        return set_error(LC_ERR_INVALID, "residual_out needs a residual input");
      if (!aligned16(f->norm_weight) || (f->residual && !aligned16(f->residual)) ||
          (f->residual_out && !aligned16(f->residual_out)))
        return set_error(LC_ERR_INVALID, "rmsnorm pointers must be 16-byte aligned");
      if (!(f->eps >= 0.f)) return set_error(LC_ERR_INVALID, "eps must be non-negative");
      if (f->residual_out) {  // written by one workgroup while the others read x and residual
        const auto lo = reinterpret_cast<uintptr_t>(f->residual_out);
        const auto hi = lo + 2 * (uintptr_t)cols;
        auto overlaps = [&](const void* p) {
          const auto b = reinterpret_cast<uintptr_t>(p);
          return b < hi && lo < b + 2 * (uintptr_t)cols;
        };
        if (overlaps(x) || overlaps(f->residual))
          return set_error(LC_ERR_INVALID, "residual_out must not overlap x or residual");
      }
      break;
    default:
      return set_error(LC_ERR_INVALID, "unknown gemv input form %d", f->in_form);
  }
  switch (f->out_form) {
    case LC_GEMV_OUT_PLAIN:
      break;
    case LC_GEMV_OUT_SWIGLU:
      if (rows % 4 != 0)
        return set_error(LC_ERR_INVALID, "the swiglu form needs rows (2 x intermediate) %% 4 == 0");
      break;
    case LC_GEMV_OUT_ROPE_QKV:
      if (f->q_heads <= 0 || f->kv_heads <= 0 || f->head_dim <= 0 || f->head_dim % 16 != 0 ||
          f->head_dim > 256)
        return set_error(LC_ERR_INVALID, "rope form needs heads > 0 and head_dim %% 16 == 0, <= 256");
      if (rows != (int64_t)(f->q_heads + 2 * (int64_t)f->kv_heads) * f->head_dim)
        return set_error(LC_ERR_INVALID, "rope form needs rows = (q_heads + 2 kv_heads) head_dim");
      if (!f->rope_row || !f->k_out || !f->v_out)
        return set_error(LC_ERR_INVALID, "rope form needs rope_row, k_out and v_out");
      if ((reinterpret_cast<uintptr_t>(f->rope_row) & 3u) ||
          (reinterpret_cast<uintptr_t>(f->k_out) & 1u) || (reinterpret_cast<uintptr_t>(f->v_out) & 1u))
        return set_error(LC_ERR_INVALID, "rope_row must be 4-byte and k_out, v_out 2-byte aligned");
      break;
    default:
      return set_error(LC_ERR_INVALID, "unknown gemv output form %d", f->out_form);
  }
  {
    // Every workgroup reads x, residual and residual_out's sources while
    // others write their output rows, so no output may share bytes with them.
    struct Range {
      uintptr_t lo, hi;
    };
    auto range = [](const void* p, size_t bytes) {
      const auto b = reinterpret_cast<uintptr_t>(p);
      return Range{b, p ? b + bytes : b};
    };
    auto meet = [](Range a, Range b) { return a.lo < b.hi && b.lo < a.hi; };
    const size_t xb = (size_t)cols * (f->in_form == LC_GEMV_IN_F32 ? 4 : 2);
    const Range ins[3] = {range(x, xb), range(f->residual, 2 * (size_t)cols),
                          range(f->residual_out, 2 * (size_t)cols)};
    size_t yn = (size_t)rows;  // bf16 elements of y
    if (f->out_form == LC_GEMV_OUT_SWIGLU) yn = (size_t)rows / 2;
    if (f->out_form == LC_GEMV_OUT_ROPE_QKV) yn = (size_t)f->q_heads * f->head_dim;
    const size_t kvn = (size_t)f->kv_heads * f->head_dim;
    const bool rope = f->out_form == LC_GEMV_OUT_ROPE_QKV;
    const Range outs[3] = {range(y, 2 * yn), range(rope ? f->k_out : nullptr, 2 * kvn),
                           range(rope ? f->v_out : nullptr, 2 * kvn)};
    for (const Range& o : outs)
      for (const Range& i : ins)
        if (meet(o, i))
          return set_error(LC_ERR_INVALID,
                           "gemv outputs must not overlap x, residual or residual_out");
  }
  if (rows == 0) return LC_OK;
  hipError_t e = lc::launch_gemv_fused(
      f->in_form, f->out_form, rows, cols, w, w_stride, x, y, f->residual, f->residual_out,
      f->norm_weight, f->eps, f->q_heads, f->kv_heads, f->head_dim, f->rope_row, f->k_out,
      f->v_out, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? LC_OK : hip_error(e, "gemv launch");
}

}  // extern "C"
