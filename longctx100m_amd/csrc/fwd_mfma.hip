// Blockwise causal forward of one (query shard x KV shard) ring hop on bf16
// MFMA (gfx950 v_mfma_f32_16x16x32_bf16, fp32 accumulation).
//
// Semantics: the reference's tiled online-softmax update over one KV shard
// (rust/longctx100m-model/src/ring_attention.rs:15-106, the inner body of the
// hop loop at :195-219) followed by its finalize (:227): the workgroup emits
// the shard-local normalised output o = acc / l and the statistics (m, l),
// which lc_attn_merge folds into the ring's running state.
//
// Layout of the work:
//   workgroup = 4 waves = 128 queries of one (batch, query head); wave = 32
//   queries.  Q^T stays in VGPRs as the MFMA B operand.  KV tiles of 64 keys
//   are staged in LDS: K row-major (A operand of S^T = K Q^T) and V transposed
//   (A operand of O^T = V^T P^T).  Computing S^T rather than S puts all of a
//   lane's scores in one query column (query = lane % 16), so the row max is
//   per-lane plus two cross-lane steps, the row sum stays lane-partial until
//   the end, and the S^T accumulator layout is directly the B operand of the
//   PV product (lane-group g holds keys 4g..4g+3 and 16+4g..16+4g+3 of each
//   32-key step; V^T is read with the same key order).
//   The causal mask is applied only on tiles that straddle the diagonal (or
//   the valid_length / shard tail); tiles beyond every query are never
//   visited.  GQA: query head h reads KV head h / (Hq / Hkv).
#include "common.h"
#include "kernels.h"
#include "stage.h"

namespace lc {
namespace {

template <int D>
struct FwdCfg {
  static constexpr int kThreads = 256;
  static constexpr int kWaves = 4;
  static constexpr int kQW = 32;           // queries per wave
  static constexpr int BM = kWaves * kQW;  // queries per workgroup
  static constexpr int BN = 64;            // keys per tile
  static constexpr int KP = D + 8;         // LDS pitch of K rows (bf16)
  static constexpr int VP = BN + 8;        // LDS pitch of V^T rows (bf16)
  static constexpr int KS = D / 32;        // MFMA k-steps over head_dim
  static constexpr int DB = D / 16;        // 16-wide head_dim blocks
};

struct FwdArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  float* o;
  float* m;
  float* l;
  int Nq, Nk, Hq, Hkv, group, n_qtiles;
  int64_t q_pos0, k_pos0, valid;
  int causal;
  int accumulate;  // merge into the running (o, m, l) instead of writing them
  float sl2;       // scale * log2(e)
};

template <int D>
__global__ __launch_bounds__(256, 2) void fwd_mfma_kernel(FwdArgs a) {
  using C = FwdCfg<D>;
  __shared__ __attribute__((aligned(16))) uint16_t k_lds[C::BN * C::KP];
  __shared__ __attribute__((aligned(16))) uint16_t vt_lds[D * C::VP];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int c = lane & 15;
  const int g = lane >> 4;

  const int L = xcd_remap(blockIdx.x, gridDim.x);
  const int qt = a.n_qtiles - 1 - (L % a.n_qtiles);  // long (late) query tiles first
  const int bh = L / a.n_qtiles;
  const int h = bh % a.Hq;
  const int b = bh / a.Hq;
  const int hk = h / a.group;

  const int64_t qs = (int64_t)a.Hq * D;   // token stride of q / o
  const int64_t ks = (int64_t)a.Hkv * D;  // token stride of k / v
  const uint16_t* qbase = a.q + (int64_t)b * a.Nq * qs + (int64_t)h * D;
  const uint16_t* kbase = a.k + (int64_t)b * a.Nk * ks + (int64_t)hk * D;
  const uint16_t* vbase = a.v + (int64_t)b * a.Nk * ks + (int64_t)hk * D;

  const int q0 = qt * C::BM;
  const int qw0 = q0 + wave * C::kQW;

  // Q^T as the B operand: lane holds query (16*nb + c), head dims 32*kk + 8g..+7.
  bf16x8 qreg[2][C::KS];
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int row = qw0 + 16 * nb + c;
#pragma unroll
    for (int kk = 0; kk < C::KS; ++kk) {
      uint4 val = make_uint4(0u, 0u, 0u, 0u);
      if (row < a.Nq) val = *reinterpret_cast<const uint4*>(qbase + (int64_t)row * qs + 32 * kk + 8 * g);
      qreg[nb][kk] = __builtin_bit_cast(bf16x8, val);
    }
  }

  // Keys any query of this workgroup can see.
  const int q_end = min(q0 + C::BM, a.Nq);
  int64_t kend = a.Nk;
  if (a.causal) kend = min(kend, a.q_pos0 + q_end - a.k_pos0);
  kend = min(kend, a.valid - a.k_pos0);
  const int ntiles = kend > 0 ? (int)((kend + C::BN - 1) / C::BN) : 0;

  const int64_t wq_first = a.q_pos0 + qw0;
  const int64_t wq_last = wq_first + C::kQW - 1;

  f32x4 o[C::DB][2];
#pragma unroll
  for (int db = 0; db < C::DB; ++db) o[db][0] = o[db][1] = f32x4{0.f, 0.f, 0.f, 0.f};
  float mrun[2] = {-INFINITY, -INFINITY};
  float lsum[2] = {0.f, 0.f};

  RowStager<C::BN, D, C::KP, C::kThreads> kst;
  TransStager<C::BN, D, C::VP, C::kThreads> vst;
  if (ntiles > 0) {
    kst.load(kbase, ks, 0, a.Nk, tid);
    vst.load(vbase, ks, 0, a.Nk, tid);
  }

  for (int j = 0; j < ntiles; ++j) {
    __syncthreads();
    kst.store(k_lds, tid);
    vst.store(vt_lds, tid);
    __syncthreads();
    if (j + 1 < ntiles) {
      kst.load(kbase, ks, (j + 1) * C::BN, a.Nk, tid);
      vst.load(vbase, ks, (j + 1) * C::BN, a.Nk, tid);
    }
    const int key0 = j * C::BN;
    const int64_t kp_first = a.k_pos0 + key0;
    const int64_t kp_last = kp_first + C::BN - 1;
    if (qw0 >= a.Nq) continue;                      // wave past the shard tail
    if (a.causal && kp_first > wq_last) continue;   // every key after every query
    const bool need_mask = (a.causal && kp_last > wq_first) || kp_last >= a.valid ||
                           key0 + C::BN > a.Nk;

    // S^T = K Q^T : s[mb][nb][i] = S^T[key 16mb+4g+i][query 16nb+c]
    f32x4 s[4][2];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) s[mb][0] = s[mb][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < C::KS; ++kk) {
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        const bf16x8 ka =
            *reinterpret_cast<const bf16x8*>(k_lds + (16 * mb + c) * C::KP + 32 * kk + 8 * g);
        s[mb][0] = mfma16x16x32(ka, qreg[0][kk], s[mb][0]);
        s[mb][1] = mfma16x16x32(ka, qreg[1][kk], s[mb][1]);
      }
    }

    if (need_mask) {
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
          const int64_t qp = wq_first + 16 * nb + c;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int key = key0 + 16 * mb + 4 * g + i;
            const int64_t kp = a.k_pos0 + key;
            if (key >= a.Nk || (a.causal && kp > qp) || kp >= a.valid) s[mb][nb][i] = -INFINITY;
          }
        }
    }

    // Online softmax in the log2 domain (p = 2^(s*scale*log2e - m2)).
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      float mx = s[0][nb][0];
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int i = 0; i < 4; ++i) mx = fmaxf(mx, s[mb][nb][i]);
      mx = group4_max(mx);
      const float mnew = fmaxf(mrun[nb], mx * a.sl2);
      const float muse = (mnew == -INFINITY) ? 0.f : mnew;  // rows with no key yet: p = alpha = 0
      const float alpha = fast_exp2(mrun[nb] - muse);
      mrun[nb] = mnew;
      lsum[nb] *= alpha;
#pragma unroll
      for (int db = 0; db < C::DB; ++db) o[db][nb] *= alpha;
      float ps = 0.f;
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float p = fast_exp2(fmaf(s[mb][nb][i], a.sl2, -muse));
          ps += p;
          s[mb][nb][i] = p;
        }
      lsum[nb] += ps;
    }

    // O^T += V^T P^T over the tile's two 32-key steps.
#pragma unroll
    for (int kk = 0; kk < C::BN / 32; ++kk) {
      const bf16x8 pb0 = pack_bf16x8(s[2 * kk][0], s[2 * kk + 1][0]);
      const bf16x8 pb1 = pack_bf16x8(s[2 * kk][1], s[2 * kk + 1][1]);
#pragma unroll
      for (int db = 0; db < C::DB; ++db) {
        const uint16_t* vr = vt_lds + (16 * db + c) * C::VP + 32 * kk + 4 * g;
        const bf16x8 va = concat_bf16x4(*reinterpret_cast<const bf16x4*>(vr),
                                         *reinterpret_cast<const bf16x4*>(vr + 16));
        o[db][0] = mfma16x16x32(va, pb0, o[db][0]);
        o[db][1] = mfma16x16x32(va, pb1, o[db][1]);
      }
    }
  }

  // Epilogue: o = acc / l, m in natural-log units, l as the reference defines it.
  // accumulate: LSE-merge (o, m, l) into the running state of the row.
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const float lt = group4_sum(lsum[nb]);
    const int row = qw0 + 16 * nb + c;
    if (row < a.Nq) {
      const float inv = lt > 0.f ? 1.f / lt : 0.f;
      const float mnat = (mrun[nb] == -INFINITY) ? -INFINITY : mrun[nb] * kLn2;
      float* orow = a.o + (((int64_t)b * a.Nq + row) * a.Hq + h) * D;
      const int64_t si = ((int64_t)b * a.Hq + h) * a.Nq + row;
      float wa = 0.f, wb = inv, mo = mnat, lo = lt;
      if (a.accumulate) {
        const MergeW w = merge_weights(a.m[si], a.l[si], mnat, lt);
        wa = w.wa;
        wb = w.wb * inv;
        mo = w.m;
        lo = w.l;
      }
#pragma unroll
      for (int db = 0; db < C::DB; ++db) {
        f32x4* dst = reinterpret_cast<f32x4*>(orow + 16 * db + 4 * g);
        *dst = a.accumulate ? *dst * wa + o[db][nb] * wb : o[db][nb] * wb;
      }
      if (g == 0) {
        a.m[si] = mo;
        a.l[si] = lo;
      }
    }
  }
}

}  // namespace

bool mfma_supported(const Problem& p) {
  return p.dtype == 1 && !p.precise && (p.D == 64 || p.D == 128);
}

hipError_t launch_fwd_mfma(const Problem& p, const void* q, const void* k, const void* v, float* o,
                           float* m, float* l, hipStream_t s) {
  FwdArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.o = o;
  a.m = m;
  a.l = l;
  a.Nq = p.Nq;
  a.Nk = p.Nk;
  a.Hq = p.Hq;
  a.Hkv = p.Hkv;
  a.group = p.Hq / p.Hkv;
  a.q_pos0 = p.q_pos0;
  a.k_pos0 = p.k_pos0;
  a.valid = p.valid;
  a.causal = p.causal ? 1 : 0;
  a.accumulate = p.accumulate ? 1 : 0;
  a.sl2 = p.scale * kLog2e;
  if (p.D == 128) {
    a.n_qtiles = (p.Nq + FwdCfg<128>::BM - 1) / FwdCfg<128>::BM;
    const int nwg = a.n_qtiles * p.Hq * p.B;
    hipLaunchKernelGGL(fwd_mfma_kernel<128>, dim3(nwg), dim3(256), 0, s, a);
  } else if (p.D == 64) {
    a.n_qtiles = (p.Nq + FwdCfg<64>::BM - 1) / FwdCfg<64>::BM;
    const int nwg = a.n_qtiles * p.Hq * p.B;
    hipLaunchKernelGGL(fwd_mfma_kernel<64>, dim3(nwg), dim3(256), 0, s, a);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace lc
