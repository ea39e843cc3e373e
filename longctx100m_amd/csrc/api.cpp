// C-ABI entry points of liblongctx100m_attn (declared in include/longctx100m_attn.h).
//
// Host-side mirror of the reference's ring-attention module
// (rust/longctx100m-model/src/ring_attention.rs): argument validation with
// the reference's messages (rs:148-171), the in-process ring emulation over
// KV shards held in HBM (hop h visits owner (rank - h) mod world, rs:191-225),
// the two-pass backward (rs:367-460) and the host-pointer forms a CPU-tensor
// caller binds.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <limits>
#include <string>
#include <vector>

#include "longctx100m_attn.h"
#include "kernels.h"

namespace {
thread_local std::string g_last_error;
}  // namespace

namespace lc {

int set_error(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int hip_error(hipError_t e, const char* where) {
  return set_error(LC_ERR_HIP, "%s: %s", where, hipGetErrorString(e));
}

}  // namespace lc

namespace {

using lc::hip_error;
using lc::set_error;

#define LC_TRY_HIP(expr, where)                \
  do {                                         \
    hipError_t e_ = (expr);                    \
    if (e_ != hipSuccess) return hip_error(e_, where); \
  } while (0)

size_t dtype_size(int dtype) { return dtype == LC_DTYPE_BF16 ? 2 : 4; }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Checks common to every shape: mirrors the reference's shape errors.
// Every flag bit this library defines; any other bit is rejected, so that a
// stray or uninitialised flags word cannot select a mode by accident.
constexpr uint32_t kKnownFlags = LC_FLAG_PRECISE | LC_FLAG_ACCUMULATE;

int check_shape(const lc_attn_shape_t* s) {
  if (s == nullptr) return set_error(LC_ERR_INVALID, "null shape argument");
  if (s->batch <= 0 || s->heads_q <= 0 || s->heads_kv <= 0 || s->head_dim <= 0 ||
      s->q_tokens < 0 || s->kv_tokens < 0)
    return set_error(LC_ERR_INVALID, "q, k, v must have shape [batch, tokens, heads, head_dim]");
  if (s->heads_q % s->heads_kv != 0)
    return set_error(LC_ERR_INVALID, "heads_q (%d) must be a multiple of heads_kv (%d)",
                     s->heads_q, s->heads_kv);
  if (s->dtype != LC_DTYPE_F32 && s->dtype != LC_DTYPE_BF16)
    return set_error(LC_ERR_UNSUPPORTED, "unsupported dtype %d", s->dtype);
  if (s->head_dim > 256)
    return set_error(LC_ERR_UNSUPPORTED, "head_dim %d > 256 is not supported", s->head_dim);
  if (s->flags & ~kKnownFlags)
    return set_error(LC_ERR_INVALID, "unknown flag bits 0x%x", s->flags & ~kKnownFlags);
  return LC_OK;
}

lc::Problem make_problem(const lc_attn_shape_t* s, const lc_attn_mask_t* m) {
  lc::Problem p;
  p.B = s->batch;
  p.Nq = s->q_tokens;
  p.Nk = s->kv_tokens;
  p.Hq = s->heads_q;
  p.Hkv = s->heads_kv;
  p.D = s->head_dim;
  p.dtype = s->dtype;
  p.precise = (s->flags & LC_FLAG_PRECISE) != 0;
  p.accumulate = false;  // read by lc_attn_fwd_shard alone
  p.q_pos0 = m ? m->q_pos0 : 0;
  p.k_pos0 = m ? m->k_pos0 : 0;
  p.valid = (m && m->valid_length >= 0) ? m->valid_length : std::numeric_limits<int64_t>::max();
  p.causal = m ? m->causal != 0 : true;
  p.scale = static_cast<float>(std::pow(static_cast<double>(p.D), -0.5));
  return p;
}

bool use_mfma(const lc::Problem& p, const void* q, const void* k, const void* v,
              const void* dout) {
  return lc::mfma_supported(p) && aligned16(q) && aligned16(k) && aligned16(v) &&
         (dout == nullptr || aligned16(dout));
}

// Whether any (query, key) pair of the shard pair is unmasked.
bool pair_active(const lc::Problem& p) {
  if (p.Nq == 0 || p.Nk == 0) return false;
  return lc::key_end_for(p, p.Nq) > 0;
}

// Rows of the streamed operand per launch of the d=128 kernels.  Every
// workgroup of a head streams the same tiles (K/V in the forward and dQ,
// Q/dO in dK/dV), and L2 serves them to the workgroups of an XCD only while
// those stay within a few hundred tiles of each other; over a longer range
// they drift apart and the tiles come from HBM again (measured on the
// forward at 1M keys: 16x the memory traffic).  A longer shard therefore runs
// as sub-shards of this many rows: the forward LSE-merges each into the
// running (o, m, l) in its epilogue, as the ring merges its hops; dQ, dK and
// dV accumulate anyway.
constexpr int64_t kStreamChunk = 65536;

int fwd_shard(const lc::Problem& p, const void* q, const void* k, const void* v, float* o,
              float* m, float* l, hipStream_t st) {
  hipError_t e = hipSuccess;
  if (use_mfma(p, q, k, v, nullptr) && p.D == 128) {
    if (p.Nk <= kStreamChunk) {
      e = lc::launch_fwd128(p, q, k, v, o, m, l, st, -1, p.accumulate);
    } else {
      const size_t row_bytes = (size_t)p.Hkv * p.D * 2;  // bf16 K/V row
      bool first = true;
      for (int64_t c0 = 0; c0 < p.Nk && e == hipSuccess; c0 += kStreamChunk) {
        lc::Problem pc = p;
        pc.Nk = (int)std::min<int64_t>(kStreamChunk, p.Nk - c0);
        pc.k_pos0 = p.k_pos0 + c0;
        if (!pair_active(pc)) continue;  // the running state is unchanged
        const char* kc = static_cast<const char*>(k) + c0 * row_bytes;
        const char* vc = static_cast<const char*>(v) + c0 * row_bytes;
        e = lc::launch_fwd128(pc, q, kc, vc, o, m, l, st, p.Nk, p.accumulate || !first);
        first = false;
      }
    }
  } else if (use_mfma(p, q, k, v, nullptr)) {
    e = lc::launch_fwd_mfma(p, q, k, v, o, m, l, st);
  } else {
    e = lc::launch_fwd_generic(p, q, k, v, o, m, l, st);
  }
  if (e != hipSuccess) return hip_error(e, "lc_attn_fwd_shard launch");
  return LC_OK;
}

int bwd_shard(const lc::Problem& p, const void* q, const void* k, const void* v, const void* dout,
              const float* lse2, const float* delta, float* dq, float* dk, float* dv,
              hipStream_t st) {
  const bool mf = use_mfma(p, q, k, v, dout);
  const bool d128 = p.D == 128;
  if (dq != nullptr) {
    hipError_t e = hipSuccess;
    if (!mf) {
      e = lc::launch_bwd_dq_generic(p, q, k, v, dout, lse2, delta, dq, st);
    } else if (!d128) {
      e = lc::launch_bwd_dq_mfma(p, q, k, v, dout, lse2, delta, dq, st);
    } else if (p.Nk <= kStreamChunk) {
      e = lc::launch_dq128(p, q, k, v, dout, lse2, delta, dq, st);
    } else {  // key sub-shards
      const size_t row_bytes = (size_t)p.Hkv * p.D * 2;
      for (int64_t c0 = 0; c0 < p.Nk && e == hipSuccess; c0 += kStreamChunk) {
        lc::Problem pc = p;
        pc.Nk = (int)std::min<int64_t>(kStreamChunk, p.Nk - c0);
        pc.k_pos0 = p.k_pos0 + c0;
        if (!pair_active(pc)) continue;
        e = lc::launch_dq128(pc, q, static_cast<const char*>(k) + c0 * row_bytes,
                             static_cast<const char*>(v) + c0 * row_bytes, dout, lse2, delta, dq,
                             st, p.Nk);
      }
    }
    if (e != hipSuccess) return hip_error(e, "lc_attn_bwd_shard dq launch");
  }
  if (dk != nullptr) {
    hipError_t e = hipSuccess;
    if (!mf) {
      e = lc::launch_bwd_dkdv_generic(p, q, k, v, dout, lse2, delta, dk, dv, st);
    } else if (!d128) {
      e = lc::launch_bwd_dkdv_mfma(p, q, k, v, dout, lse2, delta, dk, dv, st);
    } else if (p.Nq <= kStreamChunk) {
      e = lc::launch_dkdv128(p, q, k, v, dout, lse2, delta, dk, dv, st);
    } else {  // query sub-shards
      const size_t row_bytes = (size_t)p.Hq * p.D * 2;
      for (int64_t c0 = 0; c0 < p.Nq && e == hipSuccess; c0 += kStreamChunk) {
        lc::Problem pc = p;
        pc.Nq = (int)std::min<int64_t>(kStreamChunk, p.Nq - c0);
        pc.q_pos0 = p.q_pos0 + c0;
        if (!pair_active(pc)) continue;
        e = lc::launch_dkdv128(pc, static_cast<const char*>(q) + c0 * row_bytes, k, v,
                               static_cast<const char*>(dout) + c0 * row_bytes, lse2 + c0,
                               delta + c0, dk, dv, st, p.Nq);
      }
    }
    if (e != hipSuccess) return hip_error(e, "lc_attn_bwd_shard dk/dv launch");
  }
  return LC_OK;
}

// dS sharing (d = 128 on the bf16 MFMA path, dQ and dK/dV both requested, a
// workspace given): the dK/dV kernel stores the dS it forms and the dQ
// kernel reads it back, so dQ costs one GEMM instead of three (S, dP and dQ).
// The workspace holds the dS of one chunk of query rows at a time; chunks are
// multiples of 256 rows (half a dQ workgroup of 512; a workgroup past the
// chunk's end leaves its waves idle) of at most kStreamChunk rows.
// Returns the chunk's row count, 0 when the shape or workspace does not allow
// it.
int64_t ds_chunk_rows(const lc::Problem& p, size_t ws_bytes) {
  const int64_t nkb = (p.Nk + 31) / 32;
  const size_t per_tile = (size_t)p.B * p.Hq * nkb * lc::kDsBlockBytes;  // 32 query rows
  if (per_tile == 0) return 0;
  int64_t rows = (int64_t)(ws_bytes / per_tile) * 32;
  rows = std::min<int64_t>(rows, kStreamChunk);
  rows = rows >= p.Nq ? p.Nq : rows / 256 * 256;
  return rows;
}

// The dS of min(Nq, kStreamChunk) query rows, or, when that exceeds
// LC_BWD_DS_WORKSPACE_CAP, of the largest multiple of 256 rows within the cap
// (0 when not even 256 rows fit: such shards run the recomputing kernels).
size_t ds_workspace_bytes(const lc::Problem& p) {
  const size_t per_tile = (size_t)p.B * p.Hq * ((p.Nk + 31) / 32) * lc::kDsBlockBytes;
  const int64_t rows = std::min<int64_t>(p.Nq, kStreamChunk);
  const size_t full = per_tile * (size_t)((rows + 31) / 32);
  if (full <= LC_BWD_DS_WORKSPACE_CAP) return full;
  const size_t capped_rows = LC_BWD_DS_WORKSPACE_CAP / per_tile * 32 / 256 * 256;
  return capped_rows == 0 ? 0 : per_tile * (capped_rows / 32);
}

bool ds_path(const lc::Problem& p, const void* q, const void* k, const void* v, const void* dout) {
  return p.D == 128 && use_mfma(p, q, k, v, dout);
}

int bwd_shard_ds(const lc::Problem& p, int64_t chunk, const void* q, const void* k, const void* v,
                 const void* dout, const float* lse2, const float* delta, float* dq, float* dk,
                 float* dv, uint16_t* ds, hipStream_t st) {
  const size_t qrow_bytes = (size_t)p.Hq * p.D * 2;  // bf16 Q / dO row
  const size_t krow_bytes = (size_t)p.Hkv * p.D * 2;
  const int nkb = (p.Nk + 31) / 32;
  for (int64_t c0 = 0; c0 < p.Nq; c0 += chunk) {
    lc::Problem pc = p;
    pc.Nq = (int)std::min<int64_t>(chunk, p.Nq - c0);
    pc.q_pos0 = p.q_pos0 + c0;
    if (!pair_active(pc)) continue;
    hipError_t e = lc::launch_dkdv128(pc, static_cast<const char*>(q) + c0 * qrow_bytes, k, v,
                                      static_cast<const char*>(dout) + c0 * qrow_bytes, lse2 + c0,
                                      delta + c0, dk, dv, st, p.Nq, ds);
    if (e != hipSuccess) return hip_error(e, "lc_attn_bwd_shard_ws dk/dv launch");
    const int nqt = (pc.Nq + 31) / 32;
    float* dqc = dq + c0 * p.Hq * p.D;
    for (int64_t k0 = 0; k0 < p.Nk && e == hipSuccess; k0 += kStreamChunk) {  // key sub-shards
      lc::Problem pk = pc;
      pk.Nk = (int)std::min<int64_t>(kStreamChunk, p.Nk - k0);
      pk.k_pos0 = p.k_pos0 + k0;
      if (!pair_active(pk)) continue;
      e = lc::launch_dqds128(pk, static_cast<const char*>(k) + k0 * krow_bytes,
                             ds + (k0 / 32) * 1024, nqt, nkb, dqc, st, p.Nk, p.Nq);
    }
    if (e != hipSuccess) return hip_error(e, "lc_attn_bwd_shard_ws dq launch");
  }
  return LC_OK;
}

// ---- ring descriptors ---------------------------------------------------------

int check_ring(const lc_ring_desc_t* d) {
  if (d == nullptr) return set_error(LC_ERR_INVALID, "null ring descriptor");
  if (d->world <= 0 || d->rank < 0 || d->rank >= d->world)
    return set_error(LC_ERR_INVALID, "rank %d out of range for world_size %d", d->rank,
                     d->world);
  if (d->batch <= 0 || d->heads_q <= 0 || d->heads_kv <= 0 || d->head_dim <= 0 ||
      d->local_tokens < 0)
    return set_error(LC_ERR_INVALID, "q, k, v must have shape [batch, tokens, heads, head_dim]");
  if (d->heads_q % d->heads_kv != 0)
    return set_error(LC_ERR_INVALID, "q, k, v shard shapes must match");
  if (d->block_q <= 0 || d->block_k <= 0)
    return set_error(LC_ERR_INVALID, "block_q and block_k must be positive");
  if (d->local_tokens == 0) return set_error(LC_ERR_INVALID, "local_tokens must be positive");
  if (d->valid_length >= 0 &&
      !(0 < d->valid_length && d->valid_length <= (int64_t)d->world * d->local_tokens))
    return set_error(LC_ERR_INVALID, "valid_length must be within the padded distributed sequence");
  if (d->valid_length < -1) return set_error(LC_ERR_INVALID, "valid_length must be -1 (None) or positive");
  if (d->q_position_start < -1)
    return set_error(LC_ERR_INVALID, "q_position_start must be -1 (None) or non-negative");
  if (d->dtype != LC_DTYPE_F32 && d->dtype != LC_DTYPE_BF16)
    return set_error(LC_ERR_UNSUPPORTED, "unsupported dtype %d", d->dtype);
  if (d->head_dim > 256)
    return set_error(LC_ERR_UNSUPPORTED, "head_dim %d > 256 is not supported", d->head_dim);
  if (d->flags & ~kKnownFlags)
    return set_error(LC_ERR_INVALID, "unknown flag bits 0x%x", d->flags & ~kKnownFlags);
  if (d->flags & LC_FLAG_ACCUMULATE)
    return set_error(LC_ERR_INVALID, "LC_FLAG_ACCUMULATE applies to lc_attn_fwd_shard only");
  return LC_OK;
}

lc::Problem ring_problem(const lc_ring_desc_t* d, int64_t q_pos0, int64_t k_pos0) {
  lc_attn_shape_t s{d->batch, d->local_tokens, d->local_tokens, d->heads_q,
                    d->heads_kv, d->head_dim,  d->dtype,        d->flags};
  lc_attn_mask_t m{q_pos0, k_pos0, d->valid_length, d->causal, 0};
  return make_problem(&s, &m);
}

size_t round_up(size_t x) { return (x + 255) & ~size_t(255); }

// The running fp32 output; m and l are carried in the caller's outputs.
size_t fwd_ws_bytes(const lc_ring_desc_t* d) {
  const size_t n_o = (size_t)d->batch * d->local_tokens * d->heads_q * d->head_dim;
  return round_up(n_o * 4);
}

size_t bwd_ws_bytes(const lc_ring_desc_t* d) {
  const size_t n_q = (size_t)d->batch * d->local_tokens * d->heads_q * d->head_dim;
  const size_t n_k = (size_t)d->batch * d->local_tokens * d->heads_kv * d->head_dim;
  const size_t n_s = (size_t)d->batch * d->heads_q * d->local_tokens;
  return round_up(n_q * 4) + 2 * round_up(n_k * 4) + 2 * round_up(n_s * 4);
}

int check_ptrs(const void* const* arr, int world, const char* what) {
  if (arr == nullptr) return set_error(LC_ERR_INVALID, "null %s pointer array", what);
  for (int i = 0; i < world; ++i)
    if (arr[i] == nullptr) return set_error(LC_ERR_INVALID, "null %s[%d]", what, i);
  return LC_OK;
}

// Device buffer owned for the duration of a host-pointer call.
struct DevBuf {
  void* p = nullptr;
  DevBuf() = default;
  DevBuf(const DevBuf&) = delete;
  DevBuf& operator=(const DevBuf&) = delete;
  ~DevBuf() {
    if (p) (void)hipFree(p);
  }
  hipError_t alloc(size_t bytes) { return hipMalloc(&p, bytes ? bytes : 1); }
};

}  // namespace

extern "C" {

const char* lc_last_error(void) { return g_last_error.c_str(); }

int32_t lc_abi_version(void) { return 2; }

int lc_attn_fwd_shard(const lc_attn_shape_t* shape, const lc_attn_mask_t* mask, const void* q,
                      const void* k, const void* v, float* o, float* m, float* l, void* stream) {
  if (int rc = check_shape(shape)) return rc;
  if (!q || !k || !v || !o || !m || !l) return set_error(LC_ERR_INVALID, "null pointer argument");
  if (mask && mask->valid_length < -1)
    return set_error(LC_ERR_INVALID, "valid_length must be -1 (None) or non-negative");
  lc::Problem p = make_problem(shape, mask);
  p.accumulate = (shape->flags & LC_FLAG_ACCUMULATE) != 0;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (p.Nq == 0) return LC_OK;
  if (!pair_active(p)) {  // accumulate: alpha = 1, p = 0 leave the running state as it is
    if (p.accumulate) return LC_OK;
    hipError_t e = lc::launch_init_state(p.B, p.Nq, p.Hq, p.D, o, m, l, st);
    return e == hipSuccess ? LC_OK : hip_error(e, "lc_attn_fwd_shard init");
  }
  return fwd_shard(p, q, k, v, o, m, l, st);
}

size_t lc_attn_decode_workspace_bytes(const lc_attn_shape_t* shape) {
  if (check_shape(shape) != LC_OK) return 0;
  const lc::Problem p = make_problem(shape, nullptr);
  return lc::decode_supported(p) ? round_up(lc::decode_workspace_bytes(p)) : 0;
}

int lc_attn_decode(const lc_attn_shape_t* shape, const lc_attn_mask_t* mask, const void* q,
                   const void* k, const void* v, float* o, float* m, float* l, void* workspace,
                   size_t workspace_bytes, void* stream) {
  if (int rc = check_shape(shape)) return rc;
  if (!q || !k || !v || !o || !m || !l) return set_error(LC_ERR_INVALID, "null pointer argument");
  if (shape->flags & LC_FLAG_ACCUMULATE)
    return set_error(LC_ERR_INVALID, "LC_FLAG_ACCUMULATE applies to lc_attn_fwd_shard only");
  if (mask && mask->valid_length < -1)
    return set_error(LC_ERR_INVALID, "valid_length must be -1 (None) or non-negative");
  const lc::Problem p = make_problem(shape, mask);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (p.Nq == 0) return LC_OK;
  if (!pair_active(p)) {
    hipError_t e = lc::launch_init_state(p.B, p.Nq, p.Hq, p.D, o, m, l, st);
    return e == hipSuccess ? LC_OK : hip_error(e, "lc_attn_decode init");
  }
  if (!lc::decode_supported(p) || !aligned16(q) || !aligned16(k) || !aligned16(v) ||
      !aligned16(o))
    return fwd_shard(p, q, k, v, o, m, l, st);  // the blockwise kernels, no workspace
  const size_t need = round_up(lc::decode_workspace_bytes(p));
  if (workspace == nullptr || workspace_bytes < need)
    return set_error(LC_ERR_WORKSPACE, "decode workspace of %zu bytes is smaller than %zu",
                     workspace_bytes, need);
  if (!aligned16(workspace))  // the split kernel stores 16-byte vectors of partials
    return set_error(LC_ERR_INVALID, "decode workspace must be 16-byte aligned");
  hipError_t e = lc::launch_decode128(p, q, k, v, o, m, l, workspace, st);
  return e == hipSuccess ? LC_OK : hip_error(e, "lc_attn_decode launch");
}

int lc_attn_decode_static(const lc_attn_shape_t* shape, const lc_attn_mask_t* mask, const void* q,
                          const void* k, const void* v, float* o, float* m, float* l,
                          void* stream) {
  if (int rc = check_shape(shape)) return rc;
  if (!q || !k || !v || !o || !m || !l) return set_error(LC_ERR_INVALID, "null pointer argument");
  if (shape->flags & LC_FLAG_ACCUMULATE)
    return set_error(LC_ERR_INVALID, "LC_FLAG_ACCUMULATE applies to lc_attn_fwd_shard only");
  if (mask && mask->valid_length < -1)
    return set_error(LC_ERR_INVALID, "valid_length must be -1 (None) or non-negative");
  const lc::Problem p = make_problem(shape, mask);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (p.Nq == 0) return LC_OK;
  if (!pair_active(p)) {
    hipError_t e = lc::launch_init_state(p.B, p.Nq, p.Hq, p.D, o, m, l, st);
    return e == hipSuccess ? LC_OK : hip_error(e, "lc_attn_decode_static init");
  }
  if (!lc::decode_supported(p) || !aligned16(q) || !aligned16(k) || !aligned16(v) ||
      !aligned16(o))
    return fwd_shard(p, q, k, v, o, m, l, st);  // the blockwise kernels use no scratch
  const size_t need = round_up(lc::decode_workspace_bytes(p));
  if (need > lc::kDecodeStaticScratchBytes)
    return set_error(LC_ERR_WORKSPACE,
                     "decode needs %zu bytes of scratch, more than the static maximum of %zu; "
                     "use lc_attn_decode with a workspace",
                     need, lc::kDecodeStaticScratchBytes);
  void* scratch = nullptr;
  LC_TRY_HIP(lc::decode_static_scratch(st, &scratch), "lc_attn_decode_static scratch address");
  hipError_t e = lc::launch_decode128(p, q, k, v, o, m, l, scratch, st);
  return e == hipSuccess ? LC_OK : hip_error(e, "lc_attn_decode_static launch");
}

int lc_attn_merge(const lc_attn_shape_t* shape, float* o_run, float* m_run, float* l_run,
                  const float* o_part, const float* m_part, const float* l_part, void* out,
                  void* stream) {
  if (int rc = check_shape(shape)) return rc;
  if (!o_run || !m_run || !l_run || !o_part || !m_part || !l_part)
    return set_error(LC_ERR_INVALID, "null pointer argument");
  if (shape->q_tokens == 0) return LC_OK;
  hipError_t e = lc::launch_merge(shape->batch, shape->q_tokens, shape->heads_q, shape->head_dim,
                                  o_run, m_run, l_run, o_part, m_part, l_part, out, shape->dtype,
                                  static_cast<hipStream_t>(stream));
  return e == hipSuccess ? LC_OK : hip_error(e, "lc_attn_merge launch");
}

int lc_attn_init_state(const lc_attn_shape_t* shape, float* o_run, float* m_run, float* l_run,
                       void* stream) {
  if (int rc = check_shape(shape)) return rc;
  if (!o_run || !m_run || !l_run) return set_error(LC_ERR_INVALID, "null pointer argument");
  if (shape->q_tokens == 0) return LC_OK;
  hipError_t e = lc::launch_init_state(shape->batch, shape->q_tokens, shape->heads_q,
                                       shape->head_dim, o_run, m_run, l_run,
                                       static_cast<hipStream_t>(stream));
  return e == hipSuccess ? LC_OK : hip_error(e, "lc_attn_init_state launch");
}

int lc_attn_cast(const float* src, void* dst, int64_t n, int32_t dtype, void* stream) {
  if (dtype != LC_DTYPE_F32 && dtype != LC_DTYPE_BF16)
    return set_error(LC_ERR_UNSUPPORTED, "unsupported dtype %d", dtype);
  if (n < 0) return set_error(LC_ERR_INVALID, "negative element count");
  if (n == 0) return LC_OK;
  if (!src || !dst) return set_error(LC_ERR_INVALID, "null pointer argument");
  hipError_t e = lc::launch_cast(src, dst, n, dtype, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? LC_OK : hip_error(e, "lc_attn_cast launch");
}

int lc_attn_bwd_preprocess(const lc_attn_shape_t* shape, const void* out, const void* dout,
                           const float* m, const float* l, float* delta, float* lse2,
                           void* stream) {
  if (int rc = check_shape(shape)) return rc;
  if (!out || !dout || !m || !l || !delta || !lse2)
    return set_error(LC_ERR_INVALID, "null pointer argument");
  if (shape->q_tokens == 0) return LC_OK;
  hipError_t e = lc::launch_bwd_preprocess(shape->batch, shape->q_tokens, shape->heads_q,
                                           shape->head_dim, shape->dtype, out, dout, m, l, delta,
                                           lse2, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? LC_OK : hip_error(e, "lc_attn_bwd_preprocess launch");
}

int lc_attn_bwd_shard(const lc_attn_shape_t* shape, const lc_attn_mask_t* mask, const void* q,
                      const void* k, const void* v, const void* dout, const float* lse2,
                      const float* delta, float* dq_acc, float* dk_acc, float* dv_acc,
                      void* stream) {
  if (int rc = check_shape(shape)) return rc;
  if (!q || !k || !v || !dout || !lse2 || !delta)
    return set_error(LC_ERR_INVALID, "null pointer argument");
  if ((dk_acc == nullptr) != (dv_acc == nullptr))
    return set_error(LC_ERR_INVALID, "dk_acc and dv_acc must both be set or both be NULL");
  if (mask && mask->valid_length < -1)
    return set_error(LC_ERR_INVALID, "valid_length must be -1 (None) or non-negative");
  const lc::Problem p = make_problem(shape, mask);
  if (!pair_active(p)) return LC_OK;
  return bwd_shard(p, q, k, v, dout, lse2, delta, dq_acc, dk_acc, dv_acc,
                   static_cast<hipStream_t>(stream));
}

size_t lc_attn_bwd_shard_workspace_bytes(const lc_attn_shape_t* shape) {
  if (check_shape(shape) != LC_OK) return 0;
  const lc::Problem p = make_problem(shape, nullptr);
  if (p.D != 128 || !lc::mfma_supported(p)) return 0;
  return ds_workspace_bytes(p);
}

int lc_attn_bwd_shard_ws(const lc_attn_shape_t* shape, const lc_attn_mask_t* mask, const void* q,
                         const void* k, const void* v, const void* dout, const float* lse2,
                         const float* delta, float* dq_acc, float* dk_acc, float* dv_acc,
                         void* workspace, size_t workspace_bytes, void* stream) {
  if (int rc = check_shape(shape)) return rc;
  if (!q || !k || !v || !dout || !lse2 || !delta)
    return set_error(LC_ERR_INVALID, "null pointer argument");
  if ((dk_acc == nullptr) != (dv_acc == nullptr))
    return set_error(LC_ERR_INVALID, "dk_acc and dv_acc must both be set or both be NULL");
  if (mask && mask->valid_length < -1)
    return set_error(LC_ERR_INVALID, "valid_length must be -1 (None) or non-negative");
  if (workspace == nullptr && workspace_bytes != 0)
    return set_error(LC_ERR_INVALID, "workspace is NULL but workspace_bytes is not 0");
  const lc::Problem p = make_problem(shape, mask);
  if (!pair_active(p)) return LC_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dq_acc && dk_acc && workspace && (reinterpret_cast<uintptr_t>(workspace) & 255) == 0 &&
      ds_path(p, q, k, v, dout)) {
    const int64_t chunk = ds_chunk_rows(p, workspace_bytes);
    if (chunk > 0)
      return bwd_shard_ds(p, chunk, q, k, v, dout, lse2, delta, dq_acc, dk_acc, dv_acc,
                          static_cast<uint16_t*>(workspace), st);
  }
  return bwd_shard(p, q, k, v, dout, lse2, delta, dq_acc, dk_acc, dv_acc, st);
}

size_t lc_ring_fwd_workspace_bytes(const lc_ring_desc_t* desc) {
  if (check_ring(desc) != LC_OK) return 0;
  return fwd_ws_bytes(desc);
}

size_t lc_ring_bwd_workspace_bytes(const lc_ring_desc_t* desc) {
  if (check_ring(desc) != LC_OK) return 0;
  return bwd_ws_bytes(desc);
}

size_t lc_ring_bwd_ds_workspace_bytes(const lc_ring_desc_t* desc) {
  if (check_ring(desc) != LC_OK) return 0;
  const size_t base = bwd_ws_bytes(desc);
  const int64_t rn = (int64_t)desc->rank * desc->local_tokens;
  const int64_t q_pos0 = desc->q_position_start >= 0 ? desc->q_position_start : rn;
  const lc::Problem pd = ring_problem(desc, rn, rn);
  if (q_pos0 != rn || !pair_active(pd) || pd.D != 128 || !lc::mfma_supported(pd)) return base;
  return base + ds_workspace_bytes(pd);
}

int lc_ring_fwd_with_stats(const lc_ring_desc_t* d, const void* const* qs, const void* const* ks,
                           const void* const* vs, void* out, float* m, float* l, void* workspace,
                           size_t workspace_bytes, void* stream) {
  if (int rc = check_ring(d)) return rc;
  if (int rc = check_ptrs(qs, d->world, "q")) return rc;
  if (int rc = check_ptrs(ks, d->world, "k")) return rc;
  if (int rc = check_ptrs(vs, d->world, "v")) return rc;
  if (!out || !m || !l || !workspace) return set_error(LC_ERR_INVALID, "null pointer argument");
  if (workspace_bytes < fwd_ws_bytes(d))
    return set_error(LC_ERR_WORKSPACE, "workspace of %zu bytes is smaller than the %zu required",
                     workspace_bytes, fwd_ws_bytes(d));
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int n = d->local_tokens;
  const size_t n_o = (size_t)d->batch * n * d->heads_q * d->head_dim;
  float* o_run = static_cast<float*>(workspace);
  const int64_t q_pos0 = d->q_position_start >= 0 ? d->q_position_start : (int64_t)d->rank * n;

  // Hops with at least one unmasked pair; the others leave the reference's
  // (m, l, acc) unchanged (alpha = 1, p = 0 in rs:36-53).
  std::vector<int> owners;
  for (int hop = 0; hop < d->world; ++hop) {
    const int owner = ((d->rank - hop) % d->world + d->world) % d->world;
    if (pair_active(ring_problem(d, q_pos0, (int64_t)owner * n))) owners.push_back(owner);
  }
  if (owners.empty()) {
    LC_TRY_HIP(lc::launch_init_state(d->batch, n, d->heads_q, d->head_dim, o_run, m, l, st),
               "lc_ring_fwd_with_stats init");
    LC_TRY_HIP(lc::launch_cast(o_run, out, (int64_t)n_o, d->dtype, st), "lc_ring_fwd_with_stats cast");
    return LC_OK;
  }
  // The first hop writes (o_run, m, l); every later hop LSE-merges its result
  // into them in the forward's epilogue (the weights of lc_attn_merge), the
  // reference's (m, l, acc) state carried from hop to hop (rs:195-225).
  for (size_t i = 0; i < owners.size(); ++i) {
    const int owner = owners[i];
    lc::Problem p = ring_problem(d, q_pos0, (int64_t)owner * n);
    p.accumulate = i > 0;
    if (int rc = fwd_shard(p, qs[d->rank], ks[owner], vs[owner], o_run, m, l, st)) return rc;
  }
  LC_TRY_HIP(lc::launch_cast(o_run, out, (int64_t)n_o, d->dtype, st), "lc_ring_fwd_with_stats cast");
  return LC_OK;
}

int lc_ring_bwd(const lc_ring_desc_t* d, const void* const* qs, const void* const* ks,
                const void* const* vs, const void* const* outs, const float* const* ms,
                const float* const* ls, const void* const* grad_outs, void* dq, void* dk,
                void* dv, void* workspace, size_t workspace_bytes, void* stream) {
  if (int rc = check_ring(d)) return rc;
  if (int rc = check_ptrs(qs, d->world, "q")) return rc;
  if (int rc = check_ptrs(ks, d->world, "k")) return rc;
  if (int rc = check_ptrs(vs, d->world, "v")) return rc;
  if (int rc = check_ptrs(outs, d->world, "outs")) return rc;
  if (int rc = check_ptrs(reinterpret_cast<const void* const*>(ms), d->world, "ms")) return rc;
  if (int rc = check_ptrs(reinterpret_cast<const void* const*>(ls), d->world, "ls")) return rc;
  if (int rc = check_ptrs(grad_outs, d->world, "grad_outs")) return rc;
  if (!dq || !dk || !dv || !workspace) return set_error(LC_ERR_INVALID, "null pointer argument");
  if (workspace_bytes < bwd_ws_bytes(d))
    return set_error(LC_ERR_WORKSPACE, "workspace of %zu bytes is smaller than the %zu required",
                     workspace_bytes, bwd_ws_bytes(d));
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int n = d->local_tokens;
  const int r = d->rank;
  const size_t n_q = (size_t)d->batch * n * d->heads_q * d->head_dim;
  const size_t n_k = (size_t)d->batch * n * d->heads_kv * d->head_dim;
  const size_t n_s = (size_t)d->batch * d->heads_q * n;
  char* w = static_cast<char*>(workspace);
  float* dq_acc = reinterpret_cast<float*>(w);
  w += round_up(n_q * 4);
  float* dk_acc = reinterpret_cast<float*>(w);
  w += round_up(n_k * 4);
  float* dv_acc = reinterpret_cast<float*>(w);
  w += round_up(n_k * 4);
  float* delta = reinterpret_cast<float*>(w);
  w += round_up(n_s * 4);
  float* lse2 = reinterpret_cast<float*>(w);

  LC_TRY_HIP(lc::launch_fill_zero(dq_acc, (int64_t)n_q, st), "lc_ring_bwd zero");
  LC_TRY_HIP(lc::launch_fill_zero(dk_acc, (int64_t)n_k, st), "lc_ring_bwd zero");
  LC_TRY_HIP(lc::launch_fill_zero(dv_acc, (int64_t)n_k, st), "lc_ring_bwd zero");

  // The diagonal pair (this rank's queries against this rank's keys) is hop 0
  // of both passes: pass 1 takes its dK/dV, pass 2 its dQ, with the same
  // positions when q_position_start is the default.  Given workspace beyond
  // bwd_ws_bytes, both come from one dS-sharing run of that pair (the dK/dV
  // kernel stores dS, dQ is formed from it) instead of two recomputing runs.
  const int64_t q_pos0 = d->q_position_start >= 0 ? d->q_position_start : (int64_t)r * n;
  const lc::Problem pd = ring_problem(d, (int64_t)r * n, (int64_t)r * n);
  int64_t ds_chunk = 0;
  uint16_t* ds = nullptr;
  if (q_pos0 == (int64_t)r * n && pair_active(pd) &&
      ds_path(pd, qs[r], ks[r], vs[r], grad_outs[r]) && workspace_bytes > bwd_ws_bytes(d) &&
      (reinterpret_cast<uintptr_t>(workspace) & 255) == 0) {  // dS blocks as in _ws
    ds = reinterpret_cast<uint16_t*>(static_cast<char*>(workspace) + bwd_ws_bytes(d));
    ds_chunk = ds_chunk_rows(pd, workspace_bytes - bwd_ws_bytes(d));
  }
  if (ds_chunk > 0) {
    LC_TRY_HIP(lc::launch_bwd_preprocess(d->batch, n, d->heads_q, d->head_dim, d->dtype, outs[r],
                                         grad_outs[r], ms[r], ls[r], delta, lse2, st),
               "lc_ring_bwd preprocess");
    if (int rc = bwd_shard_ds(pd, ds_chunk, qs[r], ks[r], vs[r], grad_outs[r], lse2, delta,
                              dq_acc, dk_acc, dv_acc, ds, st))
      return rc;
  }

  // Pass 1 (rs:367-416): local KV fixed, query owners rank, rank-1, ...;
  // query positions owner*n + i.
  bool pass1_stats = false;  // delta / lse2 hold another owner's statistics
  for (int hop = 0; hop < d->world; ++hop) {
    const int qo = ((r - hop) % d->world + d->world) % d->world;
    if (qo == r && ds_chunk > 0) continue;  // done above
    const lc::Problem p = ring_problem(d, (int64_t)qo * n, (int64_t)r * n);
    if (!pair_active(p)) continue;
    pass1_stats = true;
    LC_TRY_HIP(lc::launch_bwd_preprocess(d->batch, n, d->heads_q, d->head_dim, d->dtype, outs[qo],
                                         grad_outs[qo], ms[qo], ls[qo], delta, lse2, st),
               "lc_ring_bwd preprocess");
    if (int rc = bwd_shard(p, qs[qo], ks[r], vs[r], grad_outs[qo], lse2, delta, nullptr, dk_acc,
                           dv_acc, st))
      return rc;
  }

  // Pass 2 (rs:418-460): local Q fixed with positions q_position_start
  // (default rank*n) + i, KV owners rank, rank-1, ...
  if (ds_chunk == 0 || pass1_stats)
    LC_TRY_HIP(lc::launch_bwd_preprocess(d->batch, n, d->heads_q, d->head_dim, d->dtype, outs[r],
                                         grad_outs[r], ms[r], ls[r], delta, lse2, st),
               "lc_ring_bwd preprocess");
  for (int hop = 0; hop < d->world; ++hop) {
    const int owner = ((r - hop) % d->world + d->world) % d->world;
    if (owner == r && ds_chunk > 0) continue;  // done above
    const lc::Problem p = ring_problem(d, q_pos0, (int64_t)owner * n);
    if (!pair_active(p)) continue;
    if (int rc = bwd_shard(p, qs[r], ks[owner], vs[owner], grad_outs[r], lse2, delta, dq_acc,
                           nullptr, nullptr, st))
      return rc;
  }

  LC_TRY_HIP(lc::launch_cast(dq_acc, dq, (int64_t)n_q, d->dtype, st), "lc_ring_bwd cast");
  LC_TRY_HIP(lc::launch_cast(dk_acc, dk, (int64_t)n_k, d->dtype, st), "lc_ring_bwd cast");
  LC_TRY_HIP(lc::launch_cast(dv_acc, dv, (int64_t)n_k, d->dtype, st), "lc_ring_bwd cast");
  return LC_OK;
}

int lc_ring_fwd_with_stats_host(const lc_ring_desc_t* d, const void* const* qs,
                                const void* const* ks, const void* const* vs, void* out, float* m,
                                float* l) {
  if (int rc = check_ring(d)) return rc;
  if (int rc = check_ptrs(qs, d->world, "q")) return rc;
  if (int rc = check_ptrs(ks, d->world, "k")) return rc;
  if (int rc = check_ptrs(vs, d->world, "v")) return rc;
  if (!out || !m || !l) return set_error(LC_ERR_INVALID, "null pointer argument");
  const int W = d->world;
  const size_t es = dtype_size(d->dtype);
  const size_t q_bytes = (size_t)d->batch * d->local_tokens * d->heads_q * d->head_dim * es;
  const size_t kv_bytes = (size_t)d->batch * d->local_tokens * d->heads_kv * d->head_dim * es;
  const size_t s_bytes = (size_t)d->batch * d->heads_q * d->local_tokens * 4;
  std::vector<DevBuf> kb(W), vb(W);
  DevBuf qb, ob, mb, lb, wb;
  std::vector<const void*> dqs(W, nullptr), dks(W), dvs(W);
  LC_TRY_HIP(qb.alloc(q_bytes), "hipMalloc");
  LC_TRY_HIP(hipMemcpy(qb.p, qs[d->rank], q_bytes, hipMemcpyHostToDevice), "hipMemcpy");
  for (int i = 0; i < W; ++i) {
    dqs[i] = qb.p;  // only this rank's queries are read
    LC_TRY_HIP(kb[i].alloc(kv_bytes), "hipMalloc");
    LC_TRY_HIP(vb[i].alloc(kv_bytes), "hipMalloc");
    LC_TRY_HIP(hipMemcpy(kb[i].p, ks[i], kv_bytes, hipMemcpyHostToDevice), "hipMemcpy");
    LC_TRY_HIP(hipMemcpy(vb[i].p, vs[i], kv_bytes, hipMemcpyHostToDevice), "hipMemcpy");
    dks[i] = kb[i].p;
    dvs[i] = vb[i].p;
  }
  const size_t ws = fwd_ws_bytes(d);
  LC_TRY_HIP(ob.alloc(q_bytes), "hipMalloc");
  LC_TRY_HIP(mb.alloc(s_bytes), "hipMalloc");
  LC_TRY_HIP(lb.alloc(s_bytes), "hipMalloc");
  LC_TRY_HIP(wb.alloc(ws), "hipMalloc");
  if (int rc = lc_ring_fwd_with_stats(d, dqs.data(), dks.data(), dvs.data(), ob.p,
                                      static_cast<float*>(mb.p), static_cast<float*>(lb.p), wb.p,
                                      ws, nullptr))
    return rc;
  LC_TRY_HIP(hipDeviceSynchronize(), "lc_ring_fwd_with_stats_host");
  LC_TRY_HIP(hipMemcpy(out, ob.p, q_bytes, hipMemcpyDeviceToHost), "hipMemcpy");
  LC_TRY_HIP(hipMemcpy(m, mb.p, s_bytes, hipMemcpyDeviceToHost), "hipMemcpy");
  LC_TRY_HIP(hipMemcpy(l, lb.p, s_bytes, hipMemcpyDeviceToHost), "hipMemcpy");
  return LC_OK;
}

int lc_ring_bwd_host(const lc_ring_desc_t* d, const void* const* qs, const void* const* ks,
                     const void* const* vs, const void* const* outs, const float* const* ms,
                     const float* const* ls, const void* const* grad_outs, void* dq, void* dk,
                     void* dv) {
  if (int rc = check_ring(d)) return rc;
  if (int rc = check_ptrs(qs, d->world, "q")) return rc;
  if (int rc = check_ptrs(ks, d->world, "k")) return rc;
  if (int rc = check_ptrs(vs, d->world, "v")) return rc;
  if (int rc = check_ptrs(outs, d->world, "outs")) return rc;
  if (int rc = check_ptrs(reinterpret_cast<const void* const*>(ms), d->world, "ms")) return rc;
  if (int rc = check_ptrs(reinterpret_cast<const void* const*>(ls), d->world, "ls")) return rc;
  if (int rc = check_ptrs(grad_outs, d->world, "grad_outs")) return rc;
  if (!dq || !dk || !dv) return set_error(LC_ERR_INVALID, "null pointer argument");
  const int W = d->world;
  const size_t es = dtype_size(d->dtype);
  const size_t q_bytes = (size_t)d->batch * d->local_tokens * d->heads_q * d->head_dim * es;
  const size_t kv_bytes = (size_t)d->batch * d->local_tokens * d->heads_kv * d->head_dim * es;
  const size_t s_bytes = (size_t)d->batch * d->heads_q * d->local_tokens * 4;
  std::vector<DevBuf> bufs(7 * W);
  std::vector<const void*> p_q(W), p_k(W), p_v(W), p_o(W), p_g(W);
  std::vector<const float*> p_m(W), p_l(W);
  for (int i = 0; i < W; ++i) {
    const void* src[7] = {qs[i], ks[i], vs[i], outs[i], grad_outs[i], ms[i], ls[i]};
    const size_t sz[7] = {q_bytes, kv_bytes, kv_bytes, q_bytes, q_bytes, s_bytes, s_bytes};
    for (int j = 0; j < 7; ++j) {
      DevBuf& b = bufs[7 * i + j];
      LC_TRY_HIP(b.alloc(sz[j]), "hipMalloc");
      LC_TRY_HIP(hipMemcpy(b.p, src[j], sz[j], hipMemcpyHostToDevice), "hipMemcpy");
    }
    p_q[i] = bufs[7 * i].p;
    p_k[i] = bufs[7 * i + 1].p;
    p_v[i] = bufs[7 * i + 2].p;
    p_o[i] = bufs[7 * i + 3].p;
    p_g[i] = bufs[7 * i + 4].p;
    p_m[i] = static_cast<const float*>(bufs[7 * i + 5].p);
    p_l[i] = static_cast<const float*>(bufs[7 * i + 6].p);
  }
  DevBuf dqb, dkb, dvb, wb;
  LC_TRY_HIP(dqb.alloc(q_bytes), "hipMalloc");
  LC_TRY_HIP(dkb.alloc(kv_bytes), "hipMalloc");
  LC_TRY_HIP(dvb.alloc(kv_bytes), "hipMalloc");
  // With room for the diagonal pair's dS the backward shares it between the
  // dK/dV and dQ kernels; when that allocation fails, the base workspace
  // runs the recomputing kernels instead.
  size_t ws = lc_ring_bwd_ds_workspace_bytes(d);
  if (ws > bwd_ws_bytes(d) && wb.alloc(ws) != hipSuccess) {
    (void)hipGetLastError();  // the failed allocation's status; nothing was allocated
    wb.p = nullptr;
    ws = bwd_ws_bytes(d);
  }
  if (wb.p == nullptr) LC_TRY_HIP(wb.alloc(ws), "hipMalloc");
  if (int rc = lc_ring_bwd(d, p_q.data(), p_k.data(), p_v.data(), p_o.data(), p_m.data(),
                           p_l.data(), p_g.data(), dqb.p, dkb.p, dvb.p, wb.p, ws, nullptr))
    return rc;
  LC_TRY_HIP(hipDeviceSynchronize(), "lc_ring_bwd_host");
  LC_TRY_HIP(hipMemcpy(dq, dqb.p, q_bytes, hipMemcpyDeviceToHost), "hipMemcpy");
  LC_TRY_HIP(hipMemcpy(dk, dkb.p, kv_bytes, hipMemcpyDeviceToHost), "hipMemcpy");
  LC_TRY_HIP(hipMemcpy(dv, dvb.p, kv_bytes, hipMemcpyDeviceToHost), "hipMemcpy");
  return LC_OK;
}

int lc_reference_causal_attention_host(int32_t batch, int32_t tokens, int32_t heads_q,
                                       int32_t heads_kv, int32_t head_dim, int32_t dtype,
                                       const void* q, const void* k, const void* v, int32_t causal,
                                       int64_t valid_length, void* out) {
  lc_ring_desc_t d{};
  d.world = 1;
  d.rank = 0;
  d.batch = batch;
  d.local_tokens = tokens;
  d.heads_q = heads_q;
  d.heads_kv = heads_kv;
  d.head_dim = head_dim;
  d.dtype = dtype;
  d.flags = 0;
  d.causal = causal;
  d.block_q = 64;
  d.block_k = 128;
  d.valid_length = valid_length;
  d.q_position_start = -1;
  if (!q || !k || !v || !out) return set_error(LC_ERR_INVALID, "null pointer argument");
  if (int rc = check_ring(&d)) return rc;
  const void* qs[1] = {q};
  const void* ks[1] = {k};
  const void* vs[1] = {v};
  std::vector<float> m((size_t)batch * heads_q * tokens), l(m.size());
  return lc_ring_fwd_with_stats_host(&d, qs, ks, vs, out, m.data(), l.data());
}

}  // extern "C"
