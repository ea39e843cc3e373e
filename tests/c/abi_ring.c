/*
 * A C caller of liblongctx100m_attn: binds include/longctx100m_attn.h the way
 * a non-Python FFI (such as the reference's Rust crate) would, with
 * plain pointers and the host-pointer entry points of the reference's ring
 * signatures (ring_attention.rs:139-233 and :281-475).
 *
 *   abi_ring validate   argument checks only (no GPU needed): ABI version,
 *                       the reference's validation texts (rs:148-171)
 *   abi_ring config1    BASELINE config 1 (world 2, fp32, Hq 9 / Hkv 3, d 64,
 *                       512 tokens per rank, Q/K/V/dO ~ N(0,1)): forward and
 *                       backward of both ranks through the library, checked
 *                       against the C restatement oracle/ring_ref.c (test
 *                       infrastructure, linked here only as the checker) at
 *                       the fp32 bar of 1e-5 norm-relative
 *   abi_ring customop3  the exact call sequence of the candle CustomOp3 that
 *                       replaces the dense attention of model.rs:223-252
 *                       (longctx100m_amd/rust/amd_attn.rs): one rank, GQA
 *                       (Hq 8 / Hkv 2), d 128, bf16 host buffers of 700
 *                       tokens; cpu_fwd = lc_ring_fwd_with_stats_host keeping
 *                       m and l, bwd = lc_ring_bwd_host with the op's output,
 *                       the saved m and l and a bf16 upstream gradient; checked
 *                       against the C restatement at the bf16 bar of 2e-2
 *
 * Prints one line per check and "abi_ring: ok" at the end; exit status 0 on
 * success.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "longctx100m_attn.h"

/* oracle/ring_ref.c */
int ref_ring_fwd_with_stats(int world, int rank, int B, int n, int H, int D,
                            const float* const* qs, const float* const* ks, const float* const* vs,
                            int causal, int block_q, int block_k, long long valid_length,
                            long long q_position_start, float* out, float* m_out, float* l_out);
int ref_ring_bwd(int world, int rank, int B, int n, int H, int D, const float* const* qs,
                 const float* const* ks, const float* const* vs, const float* const* outs,
                 const float* const* ms, const float* const* ls, const float* const* gos,
                 int causal, int block_q, int block_k, long long valid_length,
                 long long q_position_start, float* dq, float* dk, float* dv);

static int failures = 0;

static void check(int ok, const char* what) {
  printf("%s: %s\n", ok ? "pass" : "FAIL", what);
  if (!ok) ++failures;
}

static void check_msg(int rc, int want_rc, const char* want_msg) {
  char what[256];
  snprintf(what, sizeof what, "rc %d message \"%s\"", want_rc, want_msg);
  check(rc == want_rc && strcmp(lc_last_error(), want_msg) == 0, what);
  if (rc != want_rc || strcmp(lc_last_error(), want_msg) != 0)
    printf("  got rc %d message \"%s\"\n", rc, lc_last_error());
}

static lc_ring_desc_t desc(int world, int rank, int n, int hq, int hkv, int d) {
  lc_ring_desc_t r;
  memset(&r, 0, sizeof r);
  r.world = world;
  r.rank = rank;
  r.batch = 1;
  r.local_tokens = n;
  r.heads_q = hq;
  r.heads_kv = hkv;
  r.head_dim = d;
  r.dtype = LC_DTYPE_F32;
  r.causal = 1;
  r.block_q = 64;
  r.block_k = 128;
  r.valid_length = -1;
  r.q_position_start = -1;
  return r;
}

static int validate(void) {
  check(lc_abi_version() == 2, "lc_abi_version() == 2");
  float x = 0.f;
  const void* p[2] = {&x, &x};
  float* fp = &x;
  lc_ring_desc_t d = desc(2, 2, 8, 4, 2, 64);
  check(lc_ring_fwd_workspace_bytes(&d) == 0, "workspace query rejects a bad descriptor");
  check_msg(lc_ring_fwd_with_stats_host(&d, p, p, p, &x, fp, fp), LC_ERR_INVALID,
            "rank 2 out of range for world_size 2");
  d = desc(2, 0, 8, 4, 2, 64);
  d.block_k = 0;
  check_msg(lc_ring_fwd_with_stats_host(&d, p, p, p, &x, fp, fp), LC_ERR_INVALID,
            "block_q and block_k must be positive");
  d = desc(2, 0, 8, 4, 2, 64);
  d.valid_length = 17;
  check_msg(lc_ring_fwd_with_stats_host(&d, p, p, p, &x, fp, fp), LC_ERR_INVALID,
            "valid_length must be within the padded distributed sequence");
  d = desc(2, 0, 8, 4, 3, 64);
  const float* fps[2] = {fp, fp};
  check_msg(lc_ring_bwd_host(&d, p, p, p, p, fps, fps, p, &x, &x, &x), LC_ERR_INVALID,
            "q, k, v shard shapes must match");
  d = desc(2, 0, 8, 4, 2, 64);
  check_msg(lc_ring_fwd_with_stats_host(&d, NULL, p, p, &x, fp, fp), LC_ERR_INVALID,
            "null q pointer array");
  return 0;
}

/* splitmix64 + Box-Muller: N(0, 1) values from a seed */
static uint64_t sm_state;
static uint64_t splitmix64(void) {
  uint64_t z = (sm_state += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
static double uniform01(void) { return ((splitmix64() >> 11) + 0.5) * (1.0 / 9007199254740992.0); }
static void fill_normal(float* x, size_t n) {
  for (size_t i = 0; i < n; i += 2) {
    const double r = sqrt(-2.0 * log(uniform01())), t = 6.283185307179586 * uniform01();
    x[i] = (float)(r * cos(t));
    if (i + 1 < n) x[i + 1] = (float)(r * sin(t));
  }
}

/* [n, hkv, d] -> [n, hkv * g, d], head h reading KV head h / g (model.rs:85-94) */
static float* expand_heads(const float* x, int n, int hkv, int g, int d) {
  float* y = malloc(sizeof(float) * (size_t)n * hkv * g * d);
  for (int t = 0; t < n; ++t)
    for (int h = 0; h < hkv * g; ++h)
      memcpy(y + ((size_t)t * hkv * g + h) * d, x + ((size_t)t * hkv + h / g) * d, sizeof(float) * d);
  return y;
}

static double norm_rel(const float* a, const float* b, size_t n) {
  double num = 0.0, den = 0.0;
  for (size_t i = 0; i < n; ++i) {
    const double e = fabs((double)a[i] - (double)b[i]), r = fabs((double)b[i]);
    if (e > num) num = e;
    if (r > den) den = r;
  }
  return den > 0 ? num / den : num;
}

static int config1(void) {
  enum { W = 2, N = 512, HQ = 9, HKV = 3, D = 64, G = HQ / HKV };
  const size_t nq = (size_t)N * HQ * D, nk = (size_t)N * HKV * D, ns = (size_t)HQ * N;
  float *q[W], *k[W], *v[W], *go[W], *ke[W], *ve[W];
  sm_state = 20251202u;
  for (int r = 0; r < W; ++r) {
    q[r] = malloc(nq * 4);
    k[r] = malloc(nk * 4);
    v[r] = malloc(nk * 4);
    go[r] = malloc(nq * 4);
    fill_normal(q[r], nq);
    fill_normal(k[r], nk);
    fill_normal(v[r], nk);
    fill_normal(go[r], nq);
    ke[r] = expand_heads(k[r], N, HKV, G, D);
    ve[r] = expand_heads(v[r], N, HKV, G, D);
  }
  float *out[W], *m[W], *l[W], *rout[W], *rm[W], *rl[W];
  for (int r = 0; r < W; ++r) {
    out[r] = malloc(nq * 4);
    m[r] = malloc(ns * 4);
    l[r] = malloc(ns * 4);
    rout[r] = malloc(nq * 4);
    rm[r] = malloc(ns * 4);
    rl[r] = malloc(ns * 4);
    lc_ring_desc_t d = desc(W, r, N, HQ, HKV, D);
    int rc = lc_ring_fwd_with_stats_host(&d, (const void* const*)q, (const void* const*)k,
                                         (const void* const*)v, out[r], m[r], l[r]);
    if (rc) {
      printf("FAIL: lc_ring_fwd_with_stats_host rank %d: %s\n", r, lc_last_error());
      return 1;
    }
    rc = ref_ring_fwd_with_stats(W, r, 1, N, HQ, D, (const float* const*)q,
                                 (const float* const*)ke, (const float* const*)ve, 1, 64, 128, -1,
                                 -1, rout[r], rm[r], rl[r]);
    if (rc) {
      printf("FAIL: oracle forward rank %d\n", r);
      return 1;
    }
    char what[128];
    const double e = norm_rel(out[r], rout[r], nq);
    snprintf(what, sizeof what, "config 1 rank %d out norm-rel %.2e <= 1e-5", r, e);
    check(e <= 1e-5, what);
    const double el = norm_rel(l[r], rl[r], ns);
    snprintf(what, sizeof what, "config 1 rank %d l norm-rel %.2e <= 1e-5", r, el);
    check(el <= 1e-5, what);
  }
  for (int r = 0; r < W; ++r) {
    float* dq = malloc(nq * 4);
    float* dk = malloc(nk * 4);
    float* dv = malloc(nk * 4);
    float* rdq = malloc(nq * 4);
    float* rdk = malloc(nq * 4);
    float* rdv = malloc(nq * 4);
    lc_ring_desc_t d = desc(W, r, N, HQ, HKV, D);
    int rc = lc_ring_bwd_host(&d, (const void* const*)q, (const void* const*)k,
                              (const void* const*)v, (const void* const*)out,
                              (const float* const*)m, (const float* const*)l,
                              (const void* const*)go, dq, dk, dv);
    if (rc) {
      printf("FAIL: lc_ring_bwd_host rank %d: %s\n", r, lc_last_error());
      return 1;
    }
    rc = ref_ring_bwd(W, r, 1, N, HQ, D, (const float* const*)q, (const float* const*)ke,
                      (const float* const*)ve, (const float* const*)rout,
                      (const float* const*)rm, (const float* const*)rl, (const float* const*)go,
                      1, 64, 128, -1, -1, rdq, rdk, rdv);
    if (rc) {
      printf("FAIL: oracle backward rank %d\n", r);
      return 1;
    }
    /* the GQA gradient of a KV head is the sum over its query-head group */
    float* sdk = calloc(nk, 4);
    float* sdv = calloc(nk, 4);
    for (int t = 0; t < N; ++t)
      for (int h = 0; h < HQ; ++h)
        for (int j = 0; j < D; ++j) {
          sdk[((size_t)t * HKV + h / G) * D + j] += rdk[((size_t)t * HQ + h) * D + j];
          sdv[((size_t)t * HKV + h / G) * D + j] += rdv[((size_t)t * HQ + h) * D + j];
        }
    char what[128];
    const double eq = norm_rel(dq, rdq, nq), ek = norm_rel(dk, sdk, nk), ev = norm_rel(dv, sdv, nk);
    snprintf(what, sizeof what, "config 1 rank %d dq %.2e dk %.2e dv %.2e <= 1e-5", r, eq, ek, ev);
    check(eq <= 1e-5 && ek <= 1e-5 && ev <= 1e-5, what);
    free(dq), free(dk), free(dv), free(rdq), free(rdk), free(rdv), free(sdk), free(sdv);
  }
  return 0;
}

/* bf16 <-> fp32: round to nearest even, as torch and candle's half crate do */
static uint16_t to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
static float from_bf16(uint16_t b) {
  const uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}
/* N(0,1) values rounded to bf16: the bits for the library, the values for the oracle */
static void fill_bf16(uint16_t* bits, float* vals, size_t n) {
  fill_normal(vals, n);
  for (size_t i = 0; i < n; ++i) {
    bits[i] = to_bf16(vals[i]);
    vals[i] = from_bf16(bits[i]);
  }
}

static int customop3(void) {
  enum { T = 700, HQ = 8, HKV = 2, D = 128, G = HQ / HKV };
  const size_t nq = (size_t)T * HQ * D, nk = (size_t)T * HKV * D, ns = (size_t)HQ * T;
  uint16_t *qb = malloc(nq * 2), *kb = malloc(nk * 2), *vb = malloc(nk * 2), *gb = malloc(nq * 2);
  float *qf = malloc(nq * 4), *kf = malloc(nk * 4), *vf = malloc(nk * 4), *gf = malloc(nq * 4);
  sm_state = 20260723u;
  fill_bf16(qb, qf, nq);
  fill_bf16(kb, kf, nk);
  fill_bf16(vb, vf, nk);
  fill_bf16(gb, gf, nq);
  /* CausalAttention::cpu_fwd: desc(1, 0, dims, hkv, bf16, causal, 64, 128, None, None) */
  lc_ring_desc_t d = desc(1, 0, T, HQ, HKV, D);
  d.dtype = LC_DTYPE_BF16;
  uint16_t* out = malloc(nq * 2);
  float *m = malloc(ns * 4), *l = malloc(ns * 4);
  const void* pq[1] = {qb};
  const void* pk[1] = {kb};
  const void* pv[1] = {vb};
  int rc = lc_ring_fwd_with_stats_host(&d, pq, pk, pv, out, m, l);
  if (rc) {
    printf("FAIL: cpu_fwd lc_ring_fwd_with_stats_host: %s\n", lc_last_error());
    return 1;
  }
  /* CausalAttention::bwd: ring_causal_attention_backward(&[(q, k, v)], 0, &[res], &[m], &[l],
   * &[grad]) -> lc_ring_bwd_host with the op's own output and the saved statistics */
  uint16_t *dqb = malloc(nq * 2), *dkb = malloc(nk * 2), *dvb = malloc(nk * 2);
  const void* po[1] = {out};
  const float* pm[1] = {m};
  const float* pl[1] = {l};
  const void* pg[1] = {gb};
  rc = lc_ring_bwd_host(&d, pq, pk, pv, po, pm, pl, pg, dqb, dkb, dvb);
  if (rc) {
    printf("FAIL: bwd lc_ring_bwd_host: %s\n", lc_last_error());
    return 1;
  }
  /* the oracle on the same bf16 values, KV heads expanded (model.rs:85-94) */
  float* ke = expand_heads(kf, T, HKV, G, D);
  float* ve = expand_heads(vf, T, HKV, G, D);
  float *rout = malloc(nq * 4), *rm = malloc(ns * 4), *rl = malloc(ns * 4);
  const float* oq[1] = {qf};
  const float* ok[1] = {ke};
  const float* ov[1] = {ve};
  if (ref_ring_fwd_with_stats(1, 0, 1, T, HQ, D, oq, ok, ov, 1, 64, 128, -1, -1, rout, rm, rl)) {
    printf("FAIL: oracle forward\n");
    return 1;
  }
  float* outf = malloc(nq * 4);
  for (size_t i = 0; i < nq; ++i) outf[i] = from_bf16(out[i]);
  char what[160];
  const double eo = norm_rel(outf, rout, nq), el = norm_rel(l, rl, ns), em = norm_rel(m, rm, ns);
  snprintf(what, sizeof what, "customop3 fwd out %.2e <= 2e-2, m %.2e l %.2e <= 1e-4", eo, em, el);
  check(eo <= 2e-2 && em <= 1e-4 && el <= 1e-4, what);
  /* the backward's delta uses the forward output in the input dtype (py:314) */
  float* routb = malloc(nq * 4);
  for (size_t i = 0; i < nq; ++i) routb[i] = from_bf16(to_bf16(rout[i]));
  float *rdq = malloc(nq * 4), *rdk = malloc(nq * 4), *rdv = malloc(nq * 4);
  const float* oo[1] = {routb};
  const float* om[1] = {rm};
  const float* ol[1] = {rl};
  const float* og[1] = {gf};
  if (ref_ring_bwd(1, 0, 1, T, HQ, D, oq, ok, ov, oo, om, ol, og, 1, 64, 128, -1, -1, rdq, rdk,
                   rdv)) {
    printf("FAIL: oracle backward\n");
    return 1;
  }
  float *sdk = calloc(nk, 4), *sdv = calloc(nk, 4);
  for (int t = 0; t < T; ++t)
    for (int h = 0; h < HQ; ++h)
      for (int j = 0; j < D; ++j) {
        sdk[((size_t)t * HKV + h / G) * D + j] += rdk[((size_t)t * HQ + h) * D + j];
        sdv[((size_t)t * HKV + h / G) * D + j] += rdv[((size_t)t * HQ + h) * D + j];
      }
  float *dqf = malloc(nq * 4), *dkf = malloc(nk * 4), *dvf = malloc(nk * 4);
  for (size_t i = 0; i < nq; ++i) dqf[i] = from_bf16(dqb[i]);
  for (size_t i = 0; i < nk; ++i) {
    dkf[i] = from_bf16(dkb[i]);
    dvf[i] = from_bf16(dvb[i]);
  }
  const double eq = norm_rel(dqf, rdq, nq), ek = norm_rel(dkf, sdk, nk), ev = norm_rel(dvf, sdv, nk);
  snprintf(what, sizeof what, "customop3 bwd dq %.2e dk %.2e dv %.2e <= 2e-2", eq, ek, ev);
  check(eq <= 2e-2 && ek <= 2e-2 && ev <= 2e-2, what);
  return 0;
}

int main(int argc, char** argv) {
  const char* mode = argc > 1 ? argv[1] : "validate";
  int rc = 0;
  if (strcmp(mode, "validate") == 0)
    rc = validate();
  else if (strcmp(mode, "config1") == 0)
    rc = config1();
  else if (strcmp(mode, "customop3") == 0)
    rc = customop3();
  else {
    fprintf(stderr, "usage: abi_ring validate|config1|customop3\n");
    return 2;
  }
  if (rc || failures) {
    printf("abi_ring: FAILED (%d checks)\n", failures);
    return 1;
  }
  printf("abi_ring: ok\n");
  return 0;
}
