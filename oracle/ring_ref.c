/*
 * CPU restatement of longctx100m's exact causal ring attention.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity oracle and the timed CPU
 * baseline.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it; the product path (longctx100m_amd) never does.
 *
 * It follows the reference's candle implementation step by step:
 *   - online_update          rust/longctx100m-model/src/ring_attention.rs:15-55
 *   - tiled_update (masks)   ring_attention.rs:57-106
 *   - forward_with_stats     ring_attention.rs:139-233 (validation :148-171,
 *                            hop order :194-225, finalize :227-232)
 *   - dense oracle           ring_attention.rs:237-270
 *   - two-pass backward      ring_attention.rs:281-475 (pass 1 :370-416,
 *                            pass 2 :419-460)
 * and the Python twin's bf16 rule (upcast to fp32 before every matmul,
 * src/longctx100m/ring_attention.py:17,28,310-314): callers hand this file
 * fp32 arrays that already hold the upcast values.
 *
 * Layouts match the reference: q/k/v/out/dq/dk/dv are [B, n, H, D] row-major,
 * the statistics m and l are [B, H, n] (the reference's [B, H, n, 1]).
 * Arithmetic is fp32 with the same block_q x block_k tiling, so the rounding
 * sequence differs from candle's only inside the GEMM reduction order.
 * Parallelised with OpenMP over (batch, head, block); each output element is
 * still accumulated in the reference's order.
 */
#include <float.h>
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static __thread char g_err[256];

static int fail(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return 1;
}

const char* ref_last_error(void) { return g_err; }

/* invalid = (causal && k_pos > q_pos) || (valid && k_pos >= valid_length)
 * (ring_attention.rs:79-91, ring_attention.py:42-50) */
static inline int is_invalid(long long qp, long long kp, int causal, long long valid) {
  if (causal && kp > qp) return 1;
  if (valid >= 0 && kp >= valid) return 1;
  return 0;
}

/* Shared argument checks of ring_attention.rs:148-171. */
static int check_args(int world, int rank, int B, int n, int H, int D, int block_q, int block_k,
                      long long valid) {
  if (rank < 0 || rank >= world)
    return fail("rank %d out of range for world_size %d", rank, world);
  if (B <= 0 || H <= 0 || D <= 0)
    return fail("q, k, v must have shape [batch, tokens, heads, head_dim]");
  if (block_q <= 0 || block_k <= 0) return fail("block_q and block_k must be positive");
  if (n <= 0) return fail("local_tokens must be positive");
  if (valid >= 0 && !(0 < valid && valid <= (long long)world * n))
    return fail("valid_length must be within the padded distributed sequence");
  return 0;
}

#define IDX(b, t, h, d) ((((size_t)(b) * n + (t)) * H + (h)) * D + (d))
#define SIDX(b, h, t) (((size_t)(b) * H + (h)) * n + (t))

/*
 * ring_causal_attention_forward_with_stats (ring_attention.rs:139-233).
 * qs/ks/vs: world pointers, each [B, n, H, D] fp32.  valid_length and
 * q_position_start use -1 for None.  Outputs out [B,n,H,D], m and l [B,H,n].
 */
int ref_ring_fwd_with_stats(int world, int rank, int B, int n, int H, int D,
                            const float* const* qs, const float* const* ks, const float* const* vs,
                            int causal, int block_q, int block_k, long long valid_length,
                            long long q_position_start, float* out, float* m_out, float* l_out) {
  if (check_args(world, rank, B, n, H, D, block_q, block_k, valid_length)) return 1;
  const float scale = (float)pow((double)D, -0.5);
  const long long q0 = q_position_start >= 0 ? q_position_start : (long long)rank * n;
  const float* q = qs[rank];
  const int nqb = (n + block_q - 1) / block_q;
  int bad_alloc = 0;

#pragma omp parallel
  {
    float* acc = (float*)malloc(sizeof(float) * (size_t)block_q * D);
    float* mm = (float*)malloc(sizeof(float) * block_q);
    float* ll = (float*)malloc(sizeof(float) * block_q);
    float* sc = (float*)malloc(sizeof(float) * (size_t)block_q * block_k);
    if (!acc || !mm || !ll || !sc) {
#pragma omp atomic write
      bad_alloc = 1;
    } else {
#pragma omp for collapse(3) schedule(dynamic, 1)
      for (int b = 0; b < B; ++b)
        for (int h = 0; h < H; ++h)
          for (int qb = 0; qb < nqb; ++qb) {
            const int qs0 = qb * block_q;
            const int qn = (qs0 + block_q <= n ? block_q : n - qs0);
            for (int i = 0; i < qn; ++i) {
              mm[i] = -INFINITY;
              ll[i] = 0.f;
            }
            memset(acc, 0, sizeof(float) * (size_t)qn * D);
            int owner = rank;
            for (int hop = 0; hop < world; ++hop) {
              const float* k = ks[owner];
              const float* v = vs[owner];
              const long long kstart = (long long)owner * n;
              for (int off = 0; off < n; off += block_k) {
                const int kn = (off + block_k <= n ? block_k : n - off);
                /* online_update (ring_attention.rs:15-55) */
                for (int i = 0; i < qn; ++i) {
                  const float* qr = q + IDX(b, qs0 + i, h, 0);
                  float* srow = sc + (size_t)i * kn;
                  float bm = -INFINITY;
                  for (int j = 0; j < kn; ++j) {
                    const float* kr = k + IDX(b, off + j, h, 0);
                    float dot = 0.f;
                    for (int d = 0; d < D; ++d) dot += qr[d] * kr[d];
                    float s = dot * scale;
                    if (is_invalid(q0 + qs0 + i, kstart + off + j, causal, valid_length))
                      s = -INFINITY;
                    srow[j] = s;
                    if (s > bm) bm = s;
                  }
                  const float new_m = mm[i] > bm ? mm[i] : bm;
                  const int all_masked = (new_m == -INFINITY);
                  const float alpha = all_masked ? 0.f : expf(mm[i] - new_m);
                  float psum = 0.f;
                  float* ar = acc + (size_t)i * D;
                  for (int d = 0; d < D; ++d) ar[d] *= alpha;
                  for (int j = 0; j < kn; ++j) {
                    const float p = all_masked ? 0.f : expf(srow[j] - new_m);
                    psum += p;
                    if (p != 0.f) {
                      const float* vr = v + IDX(b, off + j, h, 0);
                      for (int d = 0; d < D; ++d) ar[d] += p * vr[d];
                    }
                  }
                  ll[i] = alpha * ll[i] + psum;
                  mm[i] = new_m;
                }
              }
              owner = (owner + world - 1) % world; /* ring_attention.rs:223 */
            }
            /* finalize: out = acc / max(l, FLT_MIN) (ring_attention.rs:227) */
            for (int i = 0; i < qn; ++i) {
              const float den = ll[i] > FLT_MIN ? ll[i] : FLT_MIN;
              float* o = out + IDX(b, qs0 + i, h, 0);
              for (int d = 0; d < D; ++d) o[d] = acc[(size_t)i * D + d] / den;
              m_out[SIDX(b, h, qs0 + i)] = mm[i];
              l_out[SIDX(b, h, qs0 + i)] = ll[i];
            }
          }
    }
    free(acc);
    free(mm);
    free(ll);
    free(sc);
  }
  if (bad_alloc) return fail("out of host memory");
  return 0;
}

/*
 * reference_causal_attention (ring_attention.rs:237-270): dense fp32
 * softmax(q k^T * d^-1/2 + mask) v on [B, T, H, D].  Rows whose keys are all
 * masked produce NaN in the reference (softmax of an all -inf row); here they
 * produce NaN as well.
 */
int ref_dense_attention(int B, int T, int H, int D, const float* q, const float* k, const float* v,
                        int causal, long long valid_length, float* out) {
  if (B <= 0 || T <= 0 || H <= 0 || D <= 0)
    return fail("q, k, v must have shape [batch, tokens, heads, head_dim]");
  const int n = T;
  const float scale = (float)pow((double)D, -0.5);
#pragma omp parallel
  {
    float* row = (float*)malloc(sizeof(float) * (size_t)T);
#pragma omp for collapse(3) schedule(dynamic, 4)
    for (int b = 0; b < B; ++b)
      for (int h = 0; h < H; ++h)
        for (int i = 0; i < T; ++i) {
          float mx = -INFINITY;
          for (int j = 0; j < T; ++j) {
            float dot = 0.f;
            for (int d = 0; d < D; ++d) dot += q[IDX(b, i, h, d)] * k[IDX(b, j, h, d)];
            float s = dot * scale;
            if ((causal && j > i) || (valid_length >= 0 && j >= valid_length)) s = -INFINITY;
            row[j] = s;
            if (s > mx) mx = s;
          }
          float sum = 0.f;
          for (int j = 0; j < T; ++j) {
            row[j] = expf(row[j] - mx);
            sum += row[j];
          }
          float* o = out + IDX(b, i, h, 0);
          for (int d = 0; d < D; ++d) o[d] = 0.f;
          for (int j = 0; j < T; ++j) {
            const float p = row[j] / sum;
            for (int d = 0; d < D; ++d) o[d] += p * v[IDX(b, j, h, d)];
          }
        }
    free(row);
  }
  return 0;
}

/* prob = exp(s - m) with m == -inf -> 0, divided by max(l, FLT_MIN)
 * (ring_attention.rs:393-402, :443-450). */
static inline float prob_of(float s, float m, float l) {
  if (m == -INFINITY) return 0.f;
  const float p = expf(s - m);
  return p / (l > FLT_MIN ? l : FLT_MIN);
}

/*
 * ring_causal_attention_backward (ring_attention.rs:281-475).
 * outs/ms/ls/gos: every rank's forward output ([B,n,H,D], already in fp32),
 * statistics ([B,H,n]) and upstream gradient.  Returns this rank's dq, dk, dv.
 * Pass 1 keeps this rank's KV fixed and visits query owners rank, rank-1, ...
 * with q positions owner*n + i (rs:377; q_position_start is not used there).
 * Pass 2 keeps this rank's Q fixed, with q positions q_position_start (default
 * rank*n) + i, and visits KV owners rank, rank-1, ... (rs:419-460).
 */
int ref_ring_bwd(int world, int rank, int B, int n, int H, int D, const float* const* qs,
                 const float* const* ks, const float* const* vs, const float* const* outs,
                 const float* const* ms, const float* const* ls, const float* const* gos,
                 int causal, int block_q, int block_k, long long valid_length,
                 long long q_position_start, float* dq, float* dk, float* dv) {
  if (check_args(world, rank, B, n, H, D, block_q, block_k, valid_length)) return 1;
  const float scale = (float)pow((double)D, -0.5);
  const int nqb = (n + block_q - 1) / block_q;
  const int nkb = (n + block_k - 1) / block_k;
  const float* kl = ks[rank];
  const float* vl = vs[rank];
  int bad_alloc = 0;

  /* Pass 1: dk, dv of the local KV shard.  One task per (b, h, k-block); each
   * task walks hops then q-blocks, which is the order in which the reference
   * adds into a given dk/dv block (rs:371-411). */
#pragma omp parallel
  {
    float* delta = (float*)malloc(sizeof(float) * block_q);
    float* pr = (float*)malloc(sizeof(float) * (size_t)block_q * block_k);
    float* ds = (float*)malloc(sizeof(float) * (size_t)block_q * block_k);
    if (!delta || !pr || !ds) {
#pragma omp atomic write
      bad_alloc = 1;
    } else {
#pragma omp for collapse(3) schedule(dynamic, 1)
      for (int b = 0; b < B; ++b)
        for (int h = 0; h < H; ++h)
          for (int kb = 0; kb < nkb; ++kb) {
            const int ks0 = kb * block_k;
            const int kn = (ks0 + block_k <= n ? block_k : n - ks0);
            for (int j = 0; j < kn; ++j) {
              memset(dk + IDX(b, ks0 + j, h, 0), 0, sizeof(float) * D);
              memset(dv + IDX(b, ks0 + j, h, 0), 0, sizeof(float) * D);
            }
            int qo = rank;
            for (int hop = 0; hop < world; ++hop) {
              const float* rq = qs[qo];
              const float* rgo = gos[qo];
              const float* ro = outs[qo];
              const float* rm = ms[qo];
              const float* rl = ls[qo];
              const long long qpos0 = (long long)qo * n;
              for (int qs0 = 0; qs0 < n; qs0 += block_q) {
                const int qn = (qs0 + block_q <= n ? block_q : n - qs0);
                for (int i = 0; i < qn; ++i) {
                  float s = 0.f;
                  for (int d = 0; d < D; ++d)
                    s += rgo[IDX(b, qs0 + i, h, d)] * ro[IDX(b, qs0 + i, h, d)];
                  delta[i] = s;
                }
                for (int i = 0; i < qn; ++i) {
                  const float mi = rm[SIDX(b, h, qs0 + i)];
                  const float li = rl[SIDX(b, h, qs0 + i)];
                  for (int j = 0; j < kn; ++j) {
                    float dot = 0.f, dpd = 0.f;
                    for (int d = 0; d < D; ++d) {
                      dot += rq[IDX(b, qs0 + i, h, d)] * kl[IDX(b, ks0 + j, h, d)];
                      dpd += rgo[IDX(b, qs0 + i, h, d)] * vl[IDX(b, ks0 + j, h, d)];
                    }
                    float s = dot * scale;
                    if (is_invalid(qpos0 + qs0 + i, (long long)rank * n + ks0 + j, causal,
                                   valid_length))
                      s = -INFINITY;
                    const float p = prob_of(s, mi, li);
                    pr[i * kn + j] = p;
                    ds[i * kn + j] = p * (dpd - delta[i]);
                  }
                }
                for (int j = 0; j < kn; ++j) {
                  float* dkr = dk + IDX(b, ks0 + j, h, 0);
                  float* dvr = dv + IDX(b, ks0 + j, h, 0);
                  for (int d = 0; d < D; ++d) {
                    float sk = 0.f, sv = 0.f;
                    for (int i = 0; i < qn; ++i) {
                      sk += ds[i * kn + j] * rq[IDX(b, qs0 + i, h, d)];
                      sv += pr[i * kn + j] * rgo[IDX(b, qs0 + i, h, d)];
                    }
                    dkr[d] += sk * scale;
                    dvr[d] += sv;
                  }
                }
              }
              qo = (qo + world - 1) % world;
            }
          }
    }
    free(delta);
    free(pr);
    free(ds);
  }
  if (bad_alloc) return fail("out of host memory");

  /* Pass 2: dq of the local Q shard (rs:419-460). */
  const long long qps = q_position_start >= 0 ? q_position_start : (long long)rank * n;
  const float* q = qs[rank];
  const float* go = gos[rank];
  const float* oh = outs[rank];
  const float* m = ms[rank];
  const float* l = ls[rank];
#pragma omp parallel
  {
    float* delta = (float*)malloc(sizeof(float) * block_q);
    float* ds = (float*)malloc(sizeof(float) * (size_t)block_q * block_k);
    if (!delta || !ds) {
#pragma omp atomic write
      bad_alloc = 1;
    } else {
#pragma omp for collapse(3) schedule(dynamic, 1)
      for (int b = 0; b < B; ++b)
        for (int h = 0; h < H; ++h)
          for (int qb = 0; qb < nqb; ++qb) {
            const int qs0 = qb * block_q;
            const int qn = (qs0 + block_q <= n ? block_q : n - qs0);
            for (int i = 0; i < qn; ++i) {
              memset(dq + IDX(b, qs0 + i, h, 0), 0, sizeof(float) * D);
              float s = 0.f;
              for (int d = 0; d < D; ++d)
                s += go[IDX(b, qs0 + i, h, d)] * oh[IDX(b, qs0 + i, h, d)];
              delta[i] = s;
            }
            int owner = rank;
            for (int hop = 0; hop < world; ++hop) {
              const float* kc = ks[owner];
              const float* vc = vs[owner];
              const long long kpos0 = (long long)owner * n;
              for (int ks0 = 0; ks0 < n; ks0 += block_k) {
                const int kn = (ks0 + block_k <= n ? block_k : n - ks0);
                for (int i = 0; i < qn; ++i) {
                  const float mi = m[SIDX(b, h, qs0 + i)];
                  const float li = l[SIDX(b, h, qs0 + i)];
                  for (int j = 0; j < kn; ++j) {
                    float dot = 0.f, dpd = 0.f;
                    for (int d = 0; d < D; ++d) {
                      dot += q[IDX(b, qs0 + i, h, d)] * kc[IDX(b, ks0 + j, h, d)];
                      dpd += go[IDX(b, qs0 + i, h, d)] * vc[IDX(b, ks0 + j, h, d)];
                    }
                    float s = dot * scale;
                    if (is_invalid(qps + qs0 + i, kpos0 + ks0 + j, causal, valid_length))
                      s = -INFINITY;
                    const float p = prob_of(s, mi, li);
                    ds[i * kn + j] = p * (dpd - delta[i]);
                  }
                }
                for (int i = 0; i < qn; ++i) {
                  float* dqr = dq + IDX(b, qs0 + i, h, 0);
                  for (int d = 0; d < D; ++d) {
                    float s = 0.f;
                    for (int j = 0; j < kn; ++j) s += ds[i * kn + j] * kc[IDX(b, ks0 + j, h, d)];
                    dqr[d] += s * scale;
                  }
                }
              }
              owner = (owner + world - 1) % world;
            }
          }
    }
    free(delta);
    free(ds);
  }
  if (bad_alloc) return fail("out of host memory");
  return 0;
}

/* Number of OpenMP threads the oracle will use (for the baseline report). */
int ref_num_threads(void) {
  int t = 1;
#pragma omp parallel
  {
#pragma omp single
    {
#ifdef _OPENMP
      extern int omp_get_num_threads(void);
      t = omp_get_num_threads();
#endif
    }
  }
  return t;
}
