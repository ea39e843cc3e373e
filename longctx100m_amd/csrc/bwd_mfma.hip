// Recomputation backward of one (query shard x KV shard) ring hop on bf16
// MFMA (gfx950 v_mfma_f32_16x16x32_bf16, fp32 accumulation).
//
// Semantics (rust/longctx100m-model/src/ring_attention.rs:383-409 and
// :433-454; src/longctx100m/ring_attention.py:338-357, :373-391):
//   P  = exp(s - m) / max(l, FLT_MIN)  (0 where the row saw no key)
//      = 2^(s*scale*log2e - lse2) with lse2 from lc_attn_bwd_preprocess
//   dS = P * (dO V^T - delta),  delta = rowsum(dO * O)
//   dQ += dS K * scale,  dK += dS^T Q * scale,  dV += P^T dO
//
// Two kernels, neither using atomics (each output element has one owner per
// launch, so results are deterministic and the accumulators are updated with
// plain read-modify-write):
//   * dq kernel  -- Q-stationary: workgroup = 4 waves x 32 queries of one
//     query head.  Q^T and dO^T stay in VGPRs; 64-key tiles of K (rows), V
//     (rows) and K^T are staged in LDS.  S^T = K Q^T, dP^T = V dO^T,
//     dQ^T += K^T dS^T.
//   * dkdv kernel -- KV-stationary: workgroup = 4 waves x 32 keys of one KV
//     head; it walks every query head of the GQA group, so the group-sum of
//     dK/dV happens in registers.  K^T and V^T stay in VGPRs; 32-query tiles
//     of Q, dO (rows), Q^T and dO^T are staged in LDS.  S = Q K^T,
//     dP = dO V^T, dV^T += dO^T P, dK^T += Q^T dS.
// The C-layout of each score product is reused directly as the B operand of
// the following product (see fwd_mfma.hip for the lane map).
#include "common.h"
#include "kernels.h"
#include "stage.h"

namespace lc {
namespace {

struct BwdArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* dout;
  const float* lse2;
  const float* delta;
  float* dq;
  float* dk;
  float* dv;
  int B, Nq, Nk, Hq, Hkv, group, n_tiles;
  int64_t q_pos0, k_pos0, valid;
  int causal;
  float sl2;    // scale * log2(e)
  float scale;  // D^-1/2
};

// ---------------------------------------------------------------- dQ kernel --

template <int D>
struct DqCfg {
  static constexpr int kThreads = 256;
  static constexpr int kQW = 32;
  static constexpr int BM = 4 * kQW;  // queries per workgroup
  static constexpr int BN = 64;       // keys per tile
  static constexpr int KP = D + 8;
  static constexpr int TP = BN + 8;
  static constexpr int KS = D / 32;
  static constexpr int DB = D / 16;
};

template <int D>
__global__ __launch_bounds__(256, 1) void bwd_dq_kernel(BwdArgs a) {
  using C = DqCfg<D>;
  __shared__ __attribute__((aligned(16))) uint16_t k_lds[C::BN * C::KP];
  __shared__ __attribute__((aligned(16))) uint16_t v_lds[C::BN * C::KP];
  __shared__ __attribute__((aligned(16))) uint16_t kt_lds[D * C::TP];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int c = lane & 15;
  const int g = lane >> 4;

  const int L = xcd_remap(blockIdx.x, gridDim.x);
  const int qt = a.n_tiles - 1 - (L % a.n_tiles);
  const int bh = L / a.n_tiles;
  const int h = bh % a.Hq;
  const int b = bh / a.Hq;
  const int hk = h / a.group;

  const int64_t qs = (int64_t)a.Hq * D;
  const int64_t ks = (int64_t)a.Hkv * D;
  const uint16_t* qbase = a.q + (int64_t)b * a.Nq * qs + (int64_t)h * D;
  const uint16_t* obase = a.dout + (int64_t)b * a.Nq * qs + (int64_t)h * D;
  const uint16_t* kbase = a.k + (int64_t)b * a.Nk * ks + (int64_t)hk * D;
  const uint16_t* vbase = a.v + (int64_t)b * a.Nk * ks + (int64_t)hk * D;

  const int q0 = qt * C::BM;
  const int qw0 = q0 + wave * C::kQW;

  bf16x8 qreg[2][C::KS], doreg[2][C::KS];
  float lse[2], dl[2];
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int row = qw0 + 16 * nb + c;
    const bool ok = row < a.Nq;
#pragma unroll
    for (int kk = 0; kk < C::KS; ++kk) {
      uint4 x = make_uint4(0u, 0u, 0u, 0u), y = x;
      if (ok) {
        x = *reinterpret_cast<const uint4*>(qbase + (int64_t)row * qs + 32 * kk + 8 * g);
        y = *reinterpret_cast<const uint4*>(obase + (int64_t)row * qs + 32 * kk + 8 * g);
      }
      qreg[nb][kk] = __builtin_bit_cast(bf16x8, x);
      doreg[nb][kk] = __builtin_bit_cast(bf16x8, y);
    }
    const int64_t si = ((int64_t)b * a.Hq + h) * a.Nq + row;
    lse[nb] = ok ? a.lse2[si] : INFINITY;
    dl[nb] = ok ? a.delta[si] : 0.f;
  }

  const int q_end = min(q0 + C::BM, a.Nq);
  int64_t kend = a.Nk;
  if (a.causal) kend = min(kend, a.q_pos0 + q_end - a.k_pos0);
  kend = min(kend, a.valid - a.k_pos0);
  const int ntiles = kend > 0 ? (int)((kend + C::BN - 1) / C::BN) : 0;

  const int64_t wq_first = a.q_pos0 + qw0;
  const int64_t wq_last = wq_first + C::kQW - 1;

  f32x4 acc[C::DB][2];
#pragma unroll
  for (int db = 0; db < C::DB; ++db) acc[db][0] = acc[db][1] = f32x4{0.f, 0.f, 0.f, 0.f};

  RowStager<C::BN, D, C::KP, C::kThreads> kst, vst;
  TransStager<C::BN, D, C::TP, C::kThreads> ktst;
  if (ntiles > 0) {
    kst.load(kbase, ks, 0, a.Nk, tid);
    vst.load(vbase, ks, 0, a.Nk, tid);
    ktst.load(kbase, ks, 0, a.Nk, tid);
  }

  for (int j = 0; j < ntiles; ++j) {
    __syncthreads();
    kst.store(k_lds, tid);
    vst.store(v_lds, tid);
    ktst.store(kt_lds, tid);
    __syncthreads();
    if (j + 1 < ntiles) {
      kst.load(kbase, ks, (j + 1) * C::BN, a.Nk, tid);
      vst.load(vbase, ks, (j + 1) * C::BN, a.Nk, tid);
      ktst.load(kbase, ks, (j + 1) * C::BN, a.Nk, tid);
    }
    const int key0 = j * C::BN;
    const int64_t kp_first = a.k_pos0 + key0;
    const int64_t kp_last = kp_first + C::BN - 1;
    if (qw0 >= a.Nq) continue;
    if (a.causal && kp_first > wq_last) continue;
    const bool need_mask = (a.causal && kp_last > wq_first) || kp_last >= a.valid ||
                           key0 + C::BN > a.Nk;

    // S^T = K Q^T and dP^T = V dO^T: [key 16mb+4g+i][query 16nb+c]
    f32x4 s[4][2], dp[4][2];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
      s[mb][0] = s[mb][1] = dp[mb][0] = dp[mb][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < C::KS; ++kk) {
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        const bf16x8 ka =
            *reinterpret_cast<const bf16x8*>(k_lds + (16 * mb + c) * C::KP + 32 * kk + 8 * g);
        const bf16x8 va =
            *reinterpret_cast<const bf16x8*>(v_lds + (16 * mb + c) * C::KP + 32 * kk + 8 * g);
        s[mb][0] = mfma16x16x32(ka, qreg[0][kk], s[mb][0]);
        s[mb][1] = mfma16x16x32(ka, qreg[1][kk], s[mb][1]);
        dp[mb][0] = mfma16x16x32(va, doreg[0][kk], dp[mb][0]);
        dp[mb][1] = mfma16x16x32(va, doreg[1][kk], dp[mb][1]);
      }
    }

#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        const int64_t qp = wq_first + 16 * nb + c;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float x = s[mb][nb][i];
          if (need_mask) {
            const int key = key0 + 16 * mb + 4 * g + i;
            const int64_t kp = a.k_pos0 + key;
            if (key >= a.Nk || (a.causal && kp > qp) || kp >= a.valid) x = -INFINITY;
          }
          const float p = fast_exp2(fmaf(x, a.sl2, -lse[nb]));
          s[mb][nb][i] = p * (dp[mb][nb][i] - dl[nb]);  // dS^T
        }
      }

    // dQ^T += K^T dS^T
#pragma unroll
    for (int kk = 0; kk < C::BN / 32; ++kk) {
      const bf16x8 b0 = pack_bf16x8(s[2 * kk][0], s[2 * kk + 1][0]);
      const bf16x8 b1 = pack_bf16x8(s[2 * kk][1], s[2 * kk + 1][1]);
#pragma unroll
      for (int db = 0; db < C::DB; ++db) {
        const uint16_t* kr = kt_lds + (16 * db + c) * C::TP + 32 * kk + 4 * g;
        const bf16x8 ka = concat_bf16x4(*reinterpret_cast<const bf16x4*>(kr),
                                         *reinterpret_cast<const bf16x4*>(kr + 16));
        acc[db][0] = mfma16x16x32(ka, b0, acc[db][0]);
        acc[db][1] = mfma16x16x32(ka, b1, acc[db][1]);
      }
    }
  }

#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int row = qw0 + 16 * nb + c;
    if (row < a.Nq && ntiles > 0) {
      float* dst = a.dq + (((int64_t)b * a.Nq + row) * a.Hq + h) * D + 4 * g;
#pragma unroll
      for (int db = 0; db < C::DB; ++db) {
        f32x4* p = reinterpret_cast<f32x4*>(dst + 16 * db);
        *p = *p + acc[db][nb] * a.scale;
      }
    }
  }
}

// -------------------------------------------------------------- dK/dV kernel --

template <int D>
struct DkvCfg {
  static constexpr int kThreads = 256;
  static constexpr int kKW = 32;      // keys per wave
  static constexpr int BN = 4 * kKW;  // keys per workgroup
  static constexpr int BM = 32;       // queries per tile
  static constexpr int MB = BM / 16;  // 16-query blocks per tile
  static constexpr int QP = D + 8;
  static constexpr int TP = BM + 8;
  static constexpr int KS = D / 32;
  static constexpr int DB = D / 16;
};

template <int D>
__global__ __launch_bounds__(256, 1) void bwd_dkdv_kernel(BwdArgs a) {
  using C = DkvCfg<D>;
  __shared__ __attribute__((aligned(16))) uint16_t q_lds[C::BM * C::QP];
  __shared__ __attribute__((aligned(16))) uint16_t o_lds[C::BM * C::QP];
  __shared__ __attribute__((aligned(16))) uint16_t qt_lds[D * C::TP];
  __shared__ __attribute__((aligned(16))) uint16_t ot_lds[D * C::TP];
  __shared__ __attribute__((aligned(16))) float lse_lds[C::BM];
  __shared__ __attribute__((aligned(16))) float dl_lds[C::BM];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int c = lane & 15;
  const int g = lane >> 4;

  const int L = xcd_remap(blockIdx.x, gridDim.x);
  const int kt = L % a.n_tiles;  // early keys see the most queries: dispatched first
  const int bh = L / a.n_tiles;
  const int hk = bh % a.Hkv;
  const int b = bh / a.Hkv;

  const int64_t qs = (int64_t)a.Hq * D;
  const int64_t ks = (int64_t)a.Hkv * D;
  const uint16_t* kbase = a.k + (int64_t)b * a.Nk * ks + (int64_t)hk * D;
  const uint16_t* vbase = a.v + (int64_t)b * a.Nk * ks + (int64_t)hk * D;

  const int k0 = kt * C::BN;
  const int kw0 = k0 + wave * C::kKW;

  // K^T and V^T as B operands: lane holds key (16*nb + c), dims 32*kk + 8g..+7.
  bf16x8 kreg[2][C::KS], vreg[2][C::KS];
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int row = kw0 + 16 * nb + c;
#pragma unroll
    for (int kk = 0; kk < C::KS; ++kk) {
      uint4 x = make_uint4(0u, 0u, 0u, 0u), y = x;
      if (row < a.Nk) {
        x = *reinterpret_cast<const uint4*>(kbase + (int64_t)row * ks + 32 * kk + 8 * g);
        y = *reinterpret_cast<const uint4*>(vbase + (int64_t)row * ks + 32 * kk + 8 * g);
      }
      kreg[nb][kk] = __builtin_bit_cast(bf16x8, x);
      vreg[nb][kk] = __builtin_bit_cast(bf16x8, y);
    }
  }

  f32x4 dk[C::DB][2], dv[C::DB][2];
#pragma unroll
  for (int db = 0; db < C::DB; ++db)
    dk[db][0] = dk[db][1] = dv[db][0] = dv[db][1] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Queries that can see any key of this workgroup.
  const int64_t kp_wg_first = a.k_pos0 + k0;
  int qstart = 0;
  if (a.causal) {
    const int64_t first = kp_wg_first - a.q_pos0;
    qstart = first <= 0 ? 0 : (first >= a.Nq ? a.Nq : (int)first);
  }
  qstart = (qstart / C::BM) * C::BM;
  const bool any_valid_key = kp_wg_first < a.valid && k0 < a.Nk;
  const int ntq = any_valid_key ? (a.Nq - qstart + C::BM - 1) / C::BM : 0;
  const int nsteps = ntq * a.group;

  const int64_t wk_first = a.k_pos0 + kw0;
  const int64_t wk_last = wk_first + C::kKW - 1;

  RowStager<C::BM, D, C::QP, C::kThreads> qst, ost;
  TransStager<C::BM, D, C::TP, C::kThreads> qtst, otst;
  float lse_pre = INFINITY, dl_pre = 0.f;

  auto load_step = [&](int step) {
    const int hq = hk * a.group + step / ntq;
    const int qrow0 = qstart + (step % ntq) * C::BM;
    const uint16_t* qb = a.q + (int64_t)b * a.Nq * qs + (int64_t)hq * D;
    const uint16_t* ob = a.dout + (int64_t)b * a.Nq * qs + (int64_t)hq * D;
    qst.load(qb, qs, qrow0, a.Nq, tid);
    ost.load(ob, qs, qrow0, a.Nq, tid);
    qtst.load(qb, qs, qrow0, a.Nq, tid);
    otst.load(ob, qs, qrow0, a.Nq, tid);
    if (tid < C::BM) {
      const int row = qrow0 + tid;
      const int64_t si = ((int64_t)b * a.Hq + hq) * a.Nq + row;
      lse_pre = row < a.Nq ? a.lse2[si] : INFINITY;
      dl_pre = row < a.Nq ? a.delta[si] : 0.f;
    }
  };

  if (nsteps > 0) load_step(0);
  for (int step = 0; step < nsteps; ++step) {
    __syncthreads();
    qst.store(q_lds, tid);
    ost.store(o_lds, tid);
    qtst.store(qt_lds, tid);
    otst.store(ot_lds, tid);
    if (tid < C::BM) {
      lse_lds[tid] = lse_pre;
      dl_lds[tid] = dl_pre;
    }
    __syncthreads();
    const int qrow0 = qstart + (step % ntq) * C::BM;
    if (step + 1 < nsteps) load_step(step + 1);

    const int64_t qp_first = a.q_pos0 + qrow0;
    const int64_t qp_last = qp_first + C::BM - 1;
    if (kw0 >= a.Nk) continue;
    if (a.causal && wk_first > qp_last) continue;
    const bool need_mask = (a.causal && wk_last > qp_first) || wk_last >= a.valid ||
                           kw0 + C::kKW > a.Nk;

    // S = Q K^T, dP = dO V^T: [query 16mb+4g+i][key 16nb+c]
    f32x4 s[C::MB][2], dp[C::MB][2];
#pragma unroll
    for (int mb = 0; mb < C::MB; ++mb)
      s[mb][0] = s[mb][1] = dp[mb][0] = dp[mb][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < C::KS; ++kk) {
#pragma unroll
      for (int mb = 0; mb < C::MB; ++mb) {
        const bf16x8 qa =
            *reinterpret_cast<const bf16x8*>(q_lds + (16 * mb + c) * C::QP + 32 * kk + 8 * g);
        const bf16x8 oa =
            *reinterpret_cast<const bf16x8*>(o_lds + (16 * mb + c) * C::QP + 32 * kk + 8 * g);
        s[mb][0] = mfma16x16x32(qa, kreg[0][kk], s[mb][0]);
        s[mb][1] = mfma16x16x32(qa, kreg[1][kk], s[mb][1]);
        dp[mb][0] = mfma16x16x32(oa, vreg[0][kk], dp[mb][0]);
        dp[mb][1] = mfma16x16x32(oa, vreg[1][kk], dp[mb][1]);
      }
    }

#pragma unroll
    for (int mb = 0; mb < C::MB; ++mb) {
      const f32x4 lse4 = *reinterpret_cast<const f32x4*>(lse_lds + 16 * mb + 4 * g);
      const f32x4 dl4 = *reinterpret_cast<const f32x4*>(dl_lds + 16 * mb + 4 * g);
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        const int key = kw0 + 16 * nb + c;
        const int64_t kp = a.k_pos0 + key;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float x = s[mb][nb][i];
          if (need_mask) {
            const int64_t qp = qp_first + 16 * mb + 4 * g + i;
            if (key >= a.Nk || (a.causal && kp > qp) || kp >= a.valid) x = -INFINITY;
          }
          const float p = fast_exp2(fmaf(x, a.sl2, -lse4[i]));
          s[mb][nb][i] = p;                             // P
          dp[mb][nb][i] = p * (dp[mb][nb][i] - dl4[i]);  // dS
        }
      }
    }

    // dV^T += dO^T P, dK^T += Q^T dS over the tile's two 32-query steps.
#pragma unroll
    for (int kk = 0; kk < C::BM / 32; ++kk) {
      const bf16x8 p0 = pack_bf16x8(s[2 * kk][0], s[2 * kk + 1][0]);
      const bf16x8 p1 = pack_bf16x8(s[2 * kk][1], s[2 * kk + 1][1]);
      const bf16x8 d0 = pack_bf16x8(dp[2 * kk][0], dp[2 * kk + 1][0]);
      const bf16x8 d1 = pack_bf16x8(dp[2 * kk][1], dp[2 * kk + 1][1]);
#pragma unroll
      for (int db = 0; db < C::DB; ++db) {
        const uint16_t* orow = ot_lds + (16 * db + c) * C::TP + 32 * kk + 4 * g;
        const uint16_t* qrow = qt_lds + (16 * db + c) * C::TP + 32 * kk + 4 * g;
        const bf16x8 oa = concat_bf16x4(*reinterpret_cast<const bf16x4*>(orow),
                                         *reinterpret_cast<const bf16x4*>(orow + 16));
        const bf16x8 qa = concat_bf16x4(*reinterpret_cast<const bf16x4*>(qrow),
                                         *reinterpret_cast<const bf16x4*>(qrow + 16));
        dv[db][0] = mfma16x16x32(oa, p0, dv[db][0]);
        dv[db][1] = mfma16x16x32(oa, p1, dv[db][1]);
        dk[db][0] = mfma16x16x32(qa, d0, dk[db][0]);
        dk[db][1] = mfma16x16x32(qa, d1, dk[db][1]);
      }
    }
  }

  if (nsteps == 0) return;
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int row = kw0 + 16 * nb + c;
    if (row < a.Nk) {
      const int64_t off = (((int64_t)b * a.Nk + row) * a.Hkv + hk) * D + 4 * g;
#pragma unroll
      for (int db = 0; db < C::DB; ++db) {
        f32x4* pk = reinterpret_cast<f32x4*>(a.dk + off + 16 * db);
        f32x4* pv = reinterpret_cast<f32x4*>(a.dv + off + 16 * db);
        *pk = *pk + dk[db][nb] * a.scale;
        *pv = *pv + dv[db][nb];
      }
    }
  }
}

BwdArgs make_args(const Problem& p, const void* q, const void* k, const void* v, const void* dout,
                  const float* lse2, const float* delta) {
  BwdArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.dout = static_cast<const uint16_t*>(dout);
  a.lse2 = lse2;
  a.delta = delta;
  a.dq = a.dk = a.dv = nullptr;
  a.B = p.B;
  a.Nq = p.Nq;
  a.Nk = p.Nk;
  a.Hq = p.Hq;
  a.Hkv = p.Hkv;
  a.group = p.Hq / p.Hkv;
  a.n_tiles = 0;
  a.q_pos0 = p.q_pos0;
  a.k_pos0 = p.k_pos0;
  a.valid = p.valid;
  a.causal = p.causal ? 1 : 0;
  a.sl2 = p.scale * kLog2e;
  a.scale = p.scale;
  return a;
}

}  // namespace

hipError_t launch_bwd_dq_mfma(const Problem& p, const void* q, const void* k, const void* v,
                              const void* dout, const float* lse2, const float* delta, float* dq,
                              hipStream_t s) {
  BwdArgs a = make_args(p, q, k, v, dout, lse2, delta);
  a.dq = dq;
  if (p.D == 128) {
    a.n_tiles = (p.Nq + DqCfg<128>::BM - 1) / DqCfg<128>::BM;
    hipLaunchKernelGGL(bwd_dq_kernel<128>, dim3(a.n_tiles * p.Hq * p.B), dim3(256), 0, s, a);
  } else if (p.D == 64) {
    a.n_tiles = (p.Nq + DqCfg<64>::BM - 1) / DqCfg<64>::BM;
    hipLaunchKernelGGL(bwd_dq_kernel<64>, dim3(a.n_tiles * p.Hq * p.B), dim3(256), 0, s, a);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_bwd_dkdv_mfma(const Problem& p, const void* q, const void* k, const void* v,
                                const void* dout, const float* lse2, const float* delta, float* dk,
                                float* dv, hipStream_t s) {
  BwdArgs a = make_args(p, q, k, v, dout, lse2, delta);
  a.dk = dk;
  a.dv = dv;
  if (p.D == 128) {
    a.n_tiles = (p.Nk + DkvCfg<128>::BN - 1) / DkvCfg<128>::BN;
    hipLaunchKernelGGL(bwd_dkdv_kernel<128>, dim3(a.n_tiles * p.Hkv * p.B), dim3(256), 0, s, a);
  } else if (p.D == 64) {
    a.n_tiles = (p.Nk + DkvCfg<64>::BN - 1) / DkvCfg<64>::BN;
    hipLaunchKernelGGL(bwd_dkdv_kernel<64>, dim3(a.n_tiles * p.Hkv * p.B), dim3(256), 0, s, a);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace lc
