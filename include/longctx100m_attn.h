/*
 * longctx100m_attn -- MI355X (gfx950) exact causal ring attention, one rank's share.
 *
 * C ABI of the drop-in for the reference's ring-attention path
 * (rust/longctx100m-model/src/ring_attention.rs, re-exported at
 * rust/longctx100m-model/src/lib.rs:16-19).  Plain pointers and sizes only.
 *
 * Conventions
 *   - Tensor layouts are the reference's: q/k/v/out/dq/dk/dv are contiguous
 *     row-major [B, tokens, heads, head_dim] (ring_attention.rs:109,153-154);
 *     the softmax statistics m and l are fp32 [B, heads, tokens]
 *     (the reference's [B, H, n, 1], ring_attention.rs:185-186).
 *   - m is the row max of the masked scaled scores (natural-log units) and
 *     l = sum exp(s - m); a row with no valid key has m = -inf, l = 0, out = 0.
 *   - Optional integers use -1 for None (valid_length, q_position_start).
 *   - Device entry points take device pointers and a hipStream_t (passed as
 *     void*; NULL = the default stream), enqueue work and return without
 *     synchronising.  They allocate nothing: scratch comes from a caller-owned
 *     workspace sized by the *_workspace_bytes queries.
 *   - *_host entry points take host pointers, allocate device buffers for the
 *     call, run on the current device, synchronise and free before returning.
 *   - Every entry returns 0 on success or a nonzero LC_ERR_* code; the
 *     message of the last failure on the calling thread is lc_last_error().
 *     Validation messages are the reference's texts
 *     (ring_attention.rs:148-171, ring_attention.py:78-101).
 *   - GQA is native: heads_q % heads_kv == 0 and query head h reads KV head
 *     h / (heads_q / heads_kv), the map the reference's callers build with
 *     repeat_interleave (model.rs:85-94); dk/dv are summed over each group.
 */
#ifndef LONGCTX100M_ATTN_H
#define LONGCTX100M_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum lc_dtype { LC_DTYPE_F32 = 0, LC_DTYPE_BF16 = 1 };

enum lc_status {
  LC_OK = 0,
  LC_ERR_INVALID = 1,     /* argument rejected (message = reference text) */
  LC_ERR_HIP = 2,         /* a HIP runtime call failed */
  LC_ERR_UNSUPPORTED = 3, /* shape/dtype this build does not implement */
  LC_ERR_WORKSPACE = 4    /* workspace too small */
};

/* Flags for lc_attn_shape_t.flags. */
#define LC_FLAG_PRECISE 1u /* bf16 inputs: use the fp32-math kernels instead of bf16 MFMA */
#define LC_FLAG_ACCUMULATE 2u /* lc_attn_fwd_shard: merge into the running (o, m, l) */

/* One (query shard x KV shard) problem. */
typedef struct lc_attn_shape {
  int32_t batch;     /* B */
  int32_t q_tokens;  /* tokens of the query shard */
  int32_t kv_tokens; /* tokens of the KV shard */
  int32_t heads_q;   /* query heads */
  int32_t heads_kv;  /* KV heads (heads_q % heads_kv == 0) */
  int32_t head_dim;  /* D */
  int32_t dtype;     /* enum lc_dtype of q/k/v/out/dout */
  uint32_t flags;    /* LC_FLAG_* */
} lc_attn_shape_t;

/* Global positions and masking of one shard pair (ring_attention.rs:57-106):
 * query i sits at q_pos0 + i, key j at k_pos0 + j, and the pair is masked when
 * (causal && key > query) || (valid_length >= 0 && key >= valid_length). */
typedef struct lc_attn_mask {
  int64_t q_pos0;
  int64_t k_pos0;
  int64_t valid_length; /* -1 = None */
  int32_t causal;
  int32_t reserved;
} lc_attn_mask_t;

/* ---- per-shard device kernels (the ring's building blocks) ------------------ */

/* One ring hop's forward: attention of the query shard over one KV shard
 * (online softmax over the shard, rs:57-106 / rs:15-55).  Writes the shard's
 * normalised partial output o [B, q_tokens, heads_q, D] fp32 and its
 * statistics m, l [B, heads_q, q_tokens] fp32.
 * With LC_FLAG_ACCUMULATE in shape->flags, o, m and l hold a running state
 * (an earlier hop's result, or lc_attn_init_state's) and the hop's result is
 * merged into it in place with lc_attn_merge's weights: the reference's
 * (m, l, acc) state carried from hop to hop (rs:195-225), with no partial
 * buffers and no merge pass.  A pair with no unmasked key leaves the state
 * as it is.  lc_attn_decode, lc_attn_decode_static and the ring descriptor
 * reject the flag (LC_ERR_INVALID); the backward, merge, init and cast entry
 * points ignore it. */
int lc_attn_fwd_shard(const lc_attn_shape_t* shape, const lc_attn_mask_t* mask, const void* q,
                      const void* k, const void* v, float* o, float* m, float* l, void* stream);

/* Split-KV decode: the same outputs as lc_attn_fwd_shard for a query shard of
 * a few tokens against a long KV shard (a decode step over a KV cache).  For
 * bf16, head_dim 128 and q_tokens * heads_q / heads_kv <= 16 the key range of
 * each (batch, KV head) is split over many one-wave workgroups that stream the
 * cache, and a second kernel merges the splits by log-sum-exp; it needs a
 * 16-byte-aligned workspace of lc_attn_decode_workspace_bytes(shape) bytes
 * (LC_ERR_WORKSPACE if smaller, LC_ERR_INVALID if misaligned).  Other shapes run
 * the lc_attn_fwd_shard kernels (workspace unused; the size query returns 0).
 * No counterpart in the reference, whose generation loops recompute the whole
 * prefill for every new token (src/longctx100m/distributed_infer.py:185-219,
 * rust/longctx100m-model/src/bin/infer.rs:96-106); callers that keep a KV cache
 * use it in place of that recomputation. */
size_t lc_attn_decode_workspace_bytes(const lc_attn_shape_t* shape);
int lc_attn_decode(const lc_attn_shape_t* shape, const lc_attn_mask_t* mask, const void* q,
                   const void* k, const void* v, float* o, float* m, float* l, void* workspace,
                   size_t workspace_bytes, void* stream);

/* lc_attn_decode without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  The
 * split partials live in a file-scope device array of
 * LC_DECODE_STATIC_SCRATCH_BYTES bytes that each GPU the library runs on
 * holds until the process ends; the call allocates nothing.  Shapes whose
 * lc_attn_decode_workspace_bytes exceeds that size are rejected with
 * LC_ERR_WORKSPACE (use lc_attn_decode).  Every call on one GPU shares its
 * array, so calls that overlap on one GPU (concurrent streams or threads)
 * race; calls ordered on a stream do not.  The array used is that of the
 * stream's device (the current device for a null stream).  Results equal
 * lc_attn_decode's. */
#define LC_DECODE_STATIC_SCRATCH_BYTES ((size_t)16 << 20)
int lc_attn_decode_static(const lc_attn_shape_t* shape, const lc_attn_mask_t* mask,
                          const void* q, const void* k, const void* v, float* o, float* m,
                          float* l, void* stream);

/* Log-sum-exp merge of a partial (o_part, m_part, l_part) into the running
 * state (o_run, m_run, l_run), in place -- the carried (m, l, acc) state of
 * the reference's hop loop (rs:195-225).  If out != NULL the merged result is
 * also written to out [B, q_tokens, heads_q, D] in shape->dtype (the
 * finalize of rs:227-231). */
int lc_attn_merge(const lc_attn_shape_t* shape, float* o_run, float* m_run, float* l_run,
                  const float* o_part, const float* m_part, const float* l_part, void* out,
                  void* stream);

/* Sets the running state to "no key seen": o = 0, m = -inf, l = 0
 * (ring_attention.rs:185-187). */
int lc_attn_init_state(const lc_attn_shape_t* shape, float* o_run, float* m_run, float* l_run,
                       void* stream);

/* Casts n fp32 values to dtype (fp32 -> bf16 rounds to nearest even). */
int lc_attn_cast(const float* src, void* dst, int64_t n, int32_t dtype, void* stream);

/* Backward preprocess: delta = rowsum(dout * out) with out in its own dtype
 * (ring_attention.py:314,337; rs:382) and lse2 = log2-domain log-sum-exp
 * m*log2(e) + log2(max(l, FLT_MIN)) (+inf where m = -inf), both
 * [B, heads_q, q_tokens] fp32. */
int lc_attn_bwd_preprocess(const lc_attn_shape_t* shape, const void* out, const void* dout,
                           const float* m, const float* l, float* delta, float* lse2,
                           void* stream);

/* One ring hop's backward for a (query shard, KV shard) pair, recomputing P
 * from the saved statistics (rs:383-409 and rs:433-454):
 *   dq_acc [B, q_tokens, heads_q, D]   += dS K * scale       (NULL = skip)
 *   dk_acc [B, kv_tokens, heads_kv, D] += dS^T Q * scale     (NULL = skip)
 *   dv_acc [B, kv_tokens, heads_kv, D] += P^T dO             (with dk_acc)
 * All accumulators are fp32. */
int lc_attn_bwd_shard(const lc_attn_shape_t* shape, const lc_attn_mask_t* mask, const void* q,
                      const void* k, const void* v, const void* dout, const float* lse2,
                      const float* delta, float* dq_acc, float* dk_acc, float* dv_acc,
                      void* stream);

/* The same hop backward with a caller-owned workspace, replacing the same
 * reference lines (rs:383-409 and rs:433-454) when one rank computes both
 * dQ and dK/dV of a shard pair, as a ring that sends dK/dV back does.  With
 * dq_acc, dk_acc and dv_acc all set, d = 128 on the bf16 MFMA path and a
 * 256-byte-aligned workspace, the dK/dV kernel stores dS (bf16) in the
 * workspace and dQ is computed from it, without recomputing the scores.  The
 * workspace holds the dS of a chunk of query rows at a time (2 bytes per
 * query row, key and query head): lc_attn_bwd_shard_workspace_bytes returns
 * the size for chunks of min(q_tokens, 65,536) rows, or, when that exceeds
 * LC_BWD_DS_WORKSPACE_CAP (32 GiB, the full size at 32,768 x 32,768 tokens
 * and 16 heads), the size for the largest multiple of 256 rows within the
 * cap, and 0 when not even 256 rows fit (very long KV shards: the
 * recomputing kernels then run, as without a workspace).  A smaller
 * workspace runs smaller chunks (multiples of 256 rows); every chunk streams
 * the whole KV shard and updates dK/dV once more.  With no usable
 * workspace, or other shapes, this is lc_attn_bwd_shard.  Results agree with
 * lc_attn_bwd_shard up to fp32 summation order. */
#define LC_BWD_DS_WORKSPACE_CAP ((size_t)32 << 30)
size_t lc_attn_bwd_shard_workspace_bytes(const lc_attn_shape_t* shape);
int lc_attn_bwd_shard_ws(const lc_attn_shape_t* shape, const lc_attn_mask_t* mask, const void* q,
                         const void* k, const void* v, const void* dout, const float* lse2,
                         const float* delta, float* dq_acc, float* dk_acc, float* dv_acc,
                         void* workspace, size_t workspace_bytes, void* stream);

/* ---- emulated ring (one GPU, ordered loop over KV shards in HBM) ------------ */

/* Ring geometry: world equal shards of local_tokens tokens. */
typedef struct lc_ring_desc {
  int32_t world;
  int32_t rank;
  int32_t batch;
  int32_t local_tokens;
  int32_t heads_q;
  int32_t heads_kv;
  int32_t head_dim;
  int32_t dtype;
  uint32_t flags;
  int32_t causal;
  int32_t block_q; /* accepted as in the reference; must be > 0; tiles are the kernel's own */
  int32_t block_k;
  int64_t valid_length;     /* -1 = None */
  int64_t q_position_start; /* -1 = None (defaults to rank * local_tokens) */
} lc_ring_desc_t;

size_t lc_ring_fwd_workspace_bytes(const lc_ring_desc_t* desc);
size_t lc_ring_bwd_workspace_bytes(const lc_ring_desc_t* desc);
/* Workspace for lc_ring_bwd that also holds the dS of the diagonal pair
 * (this rank's queries against its own keys, hop 0 of both of the
 * reference's passes, rs:367-416 and rs:418-460): lc_ring_bwd_workspace_bytes
 * plus lc_attn_bwd_shard_workspace_bytes of that pair, when the pair takes
 * the d = 128 bf16 MFMA path and q_position_start is None (or rank *
 * local_tokens, so both passes see the pair at the same positions);
 * otherwise the same as lc_ring_bwd_workspace_bytes.  At world = 1 (the
 * dense attention of model.rs:223-252) the diagonal pair is the whole
 * backward. */
size_t lc_ring_bwd_ds_workspace_bytes(const lc_ring_desc_t* desc);

/* ring_causal_attention_forward_with_stats (ring_attention.rs:139-233) on
 * device pointers: qs/ks/vs hold `world` shard pointers in rank order; hop h
 * attends the KV shard of owner (rank - h) mod world.  Hops whose keys are all
 * masked are skipped (they leave the reference's state unchanged).  Outputs
 * out [B,n,Hq,D] (dtype), m and l [B,Hq,n] fp32. */
int lc_ring_fwd_with_stats(const lc_ring_desc_t* desc, const void* const* qs,
                           const void* const* ks, const void* const* vs, void* out, float* m,
                           float* l, void* workspace, size_t workspace_bytes, void* stream);

/* ring_causal_attention_backward (ring_attention.rs:281-475) on device
 * pointers: outs/ms/ls/grad_outs hold every rank's forward output,
 * statistics and upstream gradient.  Returns this rank's dq [B,n,Hq,D] and
 * dk, dv [B,n,Hkv,D] in dtype.  Pass 1 uses query positions owner*n + i and
 * pass 2 uses q_position_start (default rank*n) + i, as the reference does
 * (rs:377, rs:419).  The workspace needs lc_ring_bwd_workspace_bytes; with
 * more (up to lc_ring_bwd_ds_workspace_bytes) and 256-byte alignment, the
 * diagonal pair's dK/dV and dQ come from one dS-sharing run (the dK/dV kernel stores dS in the extra
 * bytes, the dQ kernel reads it) instead of a recomputing run of each, with
 * the same results up to fp32 summation order.  The host form below uses
 * the larger workspace when it can allocate it. */
int lc_ring_bwd(const lc_ring_desc_t* desc, const void* const* qs, const void* const* ks,
                const void* const* vs, const void* const* outs, const float* const* ms,
                const float* const* ls, const void* const* grad_outs, void* dq, void* dk,
                void* dv, void* workspace, size_t workspace_bytes, void* stream);

/* Host-pointer forms of the two reference signatures (what a CPU-tensor
 * caller such as the candle backend binds).  Synchronous. */
int lc_ring_fwd_with_stats_host(const lc_ring_desc_t* desc, const void* const* qs,
                                const void* const* ks, const void* const* vs, void* out, float* m,
                                float* l);
int lc_ring_bwd_host(const lc_ring_desc_t* desc, const void* const* qs, const void* const* ks,
                     const void* const* vs, const void* const* outs, const float* const* ms,
                     const float* const* ls, const void* const* grad_outs, void* dq, void* dk,
                     void* dv);

/* reference_causal_attention (ring_attention.rs:237-270): dense attention of
 * one [B,T,H,D] sequence, computed as a one-rank ring.  Host pointers. */
int lc_reference_causal_attention_host(int32_t batch, int32_t tokens, int32_t heads_q,
                                       int32_t heads_kv, int32_t head_dim, int32_t dtype,
                                       const void* q, const void* k, const void* v, int32_t causal,
                                       int64_t valid_length, void* out);

/* ---- misc ------------------------------------------------------------------- */

const char* lc_last_error(void);
int32_t lc_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* LONGCTX100M_ATTN_H */
