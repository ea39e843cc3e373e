// Internal launcher interface between the C-ABI host code (api.cpp) and the
// HIP kernel translation units.  Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lc {

// One (query shard x KV shard) problem after validation.
struct Problem {
  int B, Nq, Nk, Hq, Hkv, D;
  int dtype;  // 0 = f32, 1 = bf16
  bool precise;
  int64_t q_pos0, k_pos0;
  int64_t valid;  // INT64_MAX when the reference's valid_length is None
  bool causal;
  float scale;      // D^-1/2
  bool accumulate;  // forward: LSE-merge into the running (o, m, l) instead of writing them
};

// Index of the exclusive end of the keys that any query of [q_begin, q_end)
// can see, clipped to [0, Nk].
inline int64_t key_end_for(const Problem& p, int64_t q_end) {
  int64_t kend = p.Nk;
  if (p.causal) {
    const int64_t last_q = p.q_pos0 + q_end - 1;
    if (last_q - p.k_pos0 + 1 < kend) kend = last_q - p.k_pos0 + 1;
  }
  if (p.valid - p.k_pos0 < kend) kend = p.valid - p.k_pos0;
  return kend < 0 ? 0 : kend;
}

// True when the bf16 MFMA kernels implement this problem.
bool mfma_supported(const Problem& p);

// head_dim 128: swizzled direct-to-LDS tiles (fwd128.hip, bwd128.hip).
// The forward can run on a sub-shard of the keys: k and v point at its first
// key, p.Nk and p.k_pos0 describe the sub-shard, kv_rows is the key count of
// the whole shard (the batch stride of K and V; -1: p.Nk), and accumulate
// merges the result into the running (o, m, l) with the weights of
// lc_attn_merge instead of overwriting them (launch_fwd_mfma and
// launch_fwd_generic take it from p.accumulate).
hipError_t launch_fwd128(const Problem& p, const void* q, const void* k, const void* v, float* o,
                         float* m, float* l, hipStream_t s, int64_t kv_rows = -1,
                         bool accumulate = false);
// The backward can run on a sub-shard too (results accumulate into dq, dk,
// dv anyway): dQ on a key sub-shard (k, v at its first key, k_rows = keys of
// the whole shard), dK/dV on a query sub-shard (q, dout, lse2, delta at its
// first query, q_rows = queries of the whole shard).  -1: p's own count.
hipError_t launch_dq128(const Problem& p, const void* q, const void* k, const void* v,
                        const void* dout, const float* lse2, const float* delta, float* dq,
                        hipStream_t s, int64_t k_rows = -1);
hipError_t launch_dkdv128(const Problem& p, const void* q, const void* k, const void* v,
                          const void* dout, const float* lse2, const float* delta, float* dk,
                          float* dv, hipStream_t s, int64_t q_rows = -1, uint16_t* ds = nullptr);
// dS sharing: launch_dkdv128 with ds set also writes every dS block it forms
// (ceil(Nq/32) x ceil(Nk/32) blocks of 2 KB per (batch, query head), layout
// in bwd128.hip); launch_dqds128 then adds dQ = scale dS K from those blocks
// for the same problem, or for a key sub-shard of it: k and ds at the
// sub-shard's first key (ds + (c0 / 32) * 1024), ds_nkb the row length of the
// whole shard, k_rows / q_rows the batch strides.
constexpr size_t kDsBlockBytes = 2048;
hipError_t launch_dqds128(const Problem& p, const void* k, const uint16_t* ds, int ds_nqt,
                          int ds_nkb, float* dq, hipStream_t s, int64_t k_rows = -1,
                          int64_t q_rows = -1);

// head_dim 64 (and 128 on request): register-staged tiles (fwd_mfma.hip, bwd_mfma.hip).
hipError_t launch_fwd_mfma(const Problem& p, const void* q, const void* k, const void* v, float* o,
                           float* m, float* l, hipStream_t s);
hipError_t launch_fwd_generic(const Problem& p, const void* q, const void* k, const void* v,
                              float* o, float* m, float* l, hipStream_t s);

hipError_t launch_bwd_dq_mfma(const Problem& p, const void* q, const void* k, const void* v,
                              const void* dout, const float* lse2, const float* delta, float* dq,
                              hipStream_t s);
hipError_t launch_bwd_dkdv_mfma(const Problem& p, const void* q, const void* k, const void* v,
                                const void* dout, const float* lse2, const float* delta, float* dk,
                                float* dv, hipStream_t s);
hipError_t launch_bwd_dq_generic(const Problem& p, const void* q, const void* k, const void* v,
                                 const void* dout, const float* lse2, const float* delta,
                                 float* dq, hipStream_t s);
hipError_t launch_bwd_dkdv_generic(const Problem& p, const void* q, const void* k, const void* v,
                                   const void* dout, const float* lse2, const float* delta,
                                   float* dk, float* dv, hipStream_t s);

// Row-wise helpers.  rows = B * N * H, row r = ((b * N) + t) * H + h.
hipError_t launch_merge(int B, int N, int H, int D, float* o_run, float* m_run, float* l_run,
                        const float* o_part, const float* m_part, const float* l_part, void* out,
                        int out_dtype, hipStream_t s);
hipError_t launch_init_state(int B, int N, int H, int D, float* o, float* m, float* l,
                             hipStream_t s);
hipError_t launch_cast(const float* src, void* dst, int64_t n, int dtype, hipStream_t s);
hipError_t launch_fill_zero(float* dst, int64_t n, hipStream_t s);
hipError_t launch_bwd_preprocess(int B, int N, int H, int D, int dtype, const void* out,
                                 const void* dout, const float* m, const float* l, float* delta,
                                 float* lse2, hipStream_t s);

// Split-KV decode attention (decode.hip): bf16, D = 128, Nq * Hq / Hkv <= 16.
bool decode_supported(const Problem& p);
int decode_splits(const Problem& p);
size_t decode_workspace_bytes(const Problem& p);
hipError_t launch_decode128(const Problem& p, const void* q, const void* k, const void* v,
                            float* o, float* m, float* l, void* ws, hipStream_t s);
// Bytes of decode.hip's file-scope device array that stands in for the
// workspace of lc_attn_decode_static, and that array's address on the
// device of stream st (the current device for a null stream; looked up once
// per device; allocates nothing).
constexpr size_t kDecodeStaticScratchBytes = size_t(16) << 20;
hipError_t decode_static_scratch(hipStream_t st, void** ptr);

// Decoder-layer row kernels (layer.hip).
hipError_t launch_rmsnorm(int dtype, int64_t rows, int cols, float eps, const void* x,
                          int64_t xs, const void* res, int64_t rs, void* res_out, int64_t ros,
                          const void* w, void* out, int64_t os, hipStream_t s);
hipError_t launch_rope_table(const float* inv, int half, float cos_factor, bool linear,
                             float pos_scale, int64_t tokens, int64_t pos0, float* table,
                             hipStream_t s);
hipError_t launch_rope_apply(int dtype, int64_t tokens, int heads, int head_dim,
                             const float* table, const void* src, int64_t sts, void* dst,
                             hipStream_t s);
// y[n] = bf16(sum_k w[n][k] x[k]) for a bf16 [n, k] row-major w (row stride
// ws elements), bf16 x [k]; k % 8 == 0, ws % 8 == 0, 16-byte aligned (gemv.hip).
hipError_t launch_gemv_bf16(int64_t n, int k, const void* w, int64_t ws, const void* x, void* y,
                            hipStream_t s);
// lc_gemv_fused's launch (forms as LC_GEMV_IN_* / LC_GEMV_OUT_*).
hipError_t launch_gemv_fused(int in_form, int out_form, int64_t rows, int cols, const void* w,
                             int64_t ws, const void* x, void* y, const void* res, void* res_out,
                             const void* nw, float eps, int q_heads, int kv_heads, int head_dim,
                             const float* rope, void* k_out, void* v_out, hipStream_t s);
hipError_t launch_swiglu(int dtype, int64_t rows, int cols, const void* g, int64_t gs,
                         const void* u, int64_t us, void* out, hipStream_t s);

// Error reporting shared by the C-ABI translation units: set the calling
// thread's lc_last_error() text and return the code.
int set_error(int code, const char* fmt, ...);
int hip_error(hipError_t e, const char* where);

}  // namespace lc
