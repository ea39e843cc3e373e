// Blockwise causal forward of one ring hop for head_dim 128 on bf16 MFMA
// (gfx950 v_mfma_f32_16x16x32_bf16, fp32 accumulation).
//
// Semantics: the reference's tiled online-softmax update over one KV shard
// (rust/longctx100m-model/src/ring_attention.rs:15-106, the body of the hop
// loop at :195-219) and its finalize (:227).  The workgroup emits the shard's
// normalised output o = acc / l and statistics (m, l); lc_attn_merge folds
// them into the ring's running state.
//
// Work split: workgroup = 4 waves x 32 queries of one (batch, query head).
// Q^T lives in VGPRs as the MFMA B operand.  64-key tiles of K and V are
// double-buffered in LDS as swizzled row-major tiles (tile128.h), filled by
// direct global->LDS loads one tile ahead; one barrier per tile.
//   S^T = K Q^T   A = K rows (ds_read_b128)
//   O^T += V^T P^T  A = V^T (ds_read_b64_tr_b16 from the same V tile),
//                   B = P^T straight from the S^T accumulators
// Computing S^T puts each lane's scores in a single query column (query =
// lane % 16): the row max is per-lane plus two cross-lane steps, the row sum
// stays lane-partial until the epilogue.  The mask is applied only on tiles
// that straddle the diagonal, valid_length or the shard tail (a separate,
// branch-free instantiation of the tile body).  GQA: query head h reads KV
// head h / (Hq / Hkv).
//
// Lazy rescaling: a row's reference maximum (log2 domain) is only raised when
// a tile's maximum exceeds it by more than kRescaleSlack, so the O^T *= alpha
// pass is skipped on almost every tile (p stays <= 2^kRescaleSlack, exact in
// the fp32 accumulators).  The true row maximum is tracked separately and the
// epilogue converts l to it, so m and l are exactly the reference's
// statistics (max of the masked scaled scores and sum exp(s - m)).
#include "common.h"
#include "kernels.h"
#include "tile128.h"

#include <type_traits>

namespace lc {
namespace {

constexpr int D = 128;
constexpr int kWaves = 4;
constexpr int kQW = 32;             // queries per wave
constexpr int BM = kWaves * kQW;    // queries per workgroup
constexpr int BN = 64;              // keys per tile
constexpr int KS = D / 32;          // MFMA k-steps over head_dim
constexpr int DB = D / 16;          // 16-wide head_dim blocks
constexpr int kTileBytes = BN * t128::kRowBytes;
constexpr float kRescaleSlack = 8.0f;  // log2 units

struct Fwd128Args {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  float* o;
  float* m;
  float* l;
  int Nq, Nk, Hq, Hkv, group, n_qtiles;
  int64_t q_pos0, k_pos0, valid;
  int causal;
  float sl2;  // scale * log2(e)
};

__global__ __launch_bounds__(256, 2) void fwd128_kernel(Fwd128Args a) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[2][2][kTileBytes];  // [buf][K,V]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int c = lane & 15;
  const int g = lane >> 4;

  const int L = xcd_remap(blockIdx.x, gridDim.x);
  const int qt = a.n_qtiles - 1 - (L % a.n_qtiles);  // long query tiles first
  const int bh = L / a.n_qtiles;
  const int h = bh % a.Hq;
  const int b = bh / a.Hq;
  const int hk = h / a.group;

  const int64_t qs = (int64_t)a.Hq * D;
  const int64_t ks = (int64_t)a.Hkv * D;
  const uint16_t* qbase = a.q + (int64_t)b * a.Nq * qs + (int64_t)h * D;
  const uint16_t* kbase = a.k + (int64_t)b * a.Nk * ks + (int64_t)hk * D;
  const uint16_t* vbase = a.v + (int64_t)b * a.Nk * ks + (int64_t)hk * D;

  const int q0 = qt * BM;
  const int qw0 = q0 + wave * kQW;

  const int q_end = min(q0 + BM, a.Nq);
  int64_t kend = a.Nk;
  if (a.causal) kend = min(kend, a.q_pos0 + q_end - a.k_pos0);
  kend = min(kend, a.valid - a.k_pos0);
  const int ntiles = kend > 0 ? (int)((kend + BN - 1) / BN) : 0;

  t128::RowLoader<BN, kWaves> ld;
  ld.init(ks, wave, lane);
  if (ntiles > 0) {
    ld.load<true>(kbase, ks, 0, a.Nk, smem[0][0], wave, lane);
    ld.load<true>(vbase, ks, 0, a.Nk, smem[0][1], wave, lane);
  }

  // Q^T operand: lane holds query 16*nb + c, head dims 32*kk + 8g .. +7.
  bf16x8 qreg[2][KS];
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int row = min(qw0 + 16 * nb + c, a.Nq - 1);
#pragma unroll
    for (int kk = 0; kk < KS; ++kk)
      qreg[nb][kk] = *reinterpret_cast<const bf16x8*>(qbase + (int64_t)row * qs + 32 * kk + 8 * g);
  }

  // Loop-invariant LDS byte offsets.
  int koff[KS];
#pragma unroll
  for (int kk = 0; kk < KS; ++kk) koff[kk] = t128::row_chunk_off(c, 4 * kk + g);
  int voff[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) voff[db] = t128::tr_off(0, 16 * db, lane);

  const int64_t wq_first = a.q_pos0 + qw0;
  const int64_t wq_last = wq_first + kQW - 1;

  f32x4 o[DB][2];
#pragma unroll
  for (int db = 0; db < DB; ++db) o[db][0] = o[db][1] = f32x4{0.f, 0.f, 0.f, 0.f};
  float mrun[2] = {-INFINITY, -INFINITY};   // reference maximum of p (log2 units)
  float mtrue[2] = {-INFINITY, -INFINITY};  // exact running maximum (log2 units)
  float lsum[2] = {0.f, 0.f};

  // One tile: S^T = K Q^T, mask (MASKED only), online softmax, O^T += V^T P^T.
  // For the mask, key k of the tile and query column q of the wave are
  // invalid when (causal && k - q > cthr) || k >= kmax, with
  // cthr = (q_pos0 + qw0) - (k_pos0 + key0) and kmax the first key index past
  // Nk / valid_length, both relative to the tile.
  auto tile = [&](auto masked_tag, const uint8_t* kt, const uint8_t* vt, int cthr, int kmax) {
    constexpr bool MASKED = decltype(masked_tag)::value;
    f32x4 s[4][2];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) s[mb][0] = s[mb][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        const bf16x8 ka = *reinterpret_cast<const bf16x8*>(kt + koff[kk] + mb * 16 * t128::kRowBytes);
        s[mb][0] = mfma16x16x32(ka, qreg[0][kk], s[mb][0]);
        s[mb][1] = mfma16x16x32(ka, qreg[1][kk], s[mb][1]);
      }
    }
    if constexpr (MASKED) {
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int nb = 0; nb < 2; ++nb)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int kr = 16 * mb + 4 * g + i;
            const bool bad = (a.causal && kr - (16 * nb + c) > cthr) || kr >= kmax;
            s[mb][nb][i] = bad ? -INFINITY : s[mb][nb][i];
          }
    }
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      float mx = s[0][nb][0];
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int i = 0; i < 4; ++i) mx = fmaxf(mx, s[mb][nb][i]);
      mx = group4_max(mx) * a.sl2;
      mtrue[nb] = fmaxf(mtrue[nb], mx);
      const bool raise = mx > mrun[nb] + kRescaleSlack;
      if (__any(raise)) {
        const float mnew = raise ? mx : mrun[nb];
        const float alpha = raise ? fast_exp2(mrun[nb] - mnew) : 1.f;  // mrun = -inf: 0
        mrun[nb] = mnew;
        lsum[nb] *= alpha;
#pragma unroll
        for (int db = 0; db < DB; ++db) o[db][nb] *= alpha;
      }
      const float muse = (mrun[nb] == -INFINITY) ? 0.f : mrun[nb];  // no key yet: p = 0
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
#pragma unroll
    for (int kk = 0; kk < BN / 32; ++kk) {
      const bf16x8 pb0 = pack_bf16x8(s[2 * kk][0], s[2 * kk + 1][0]);
      const bf16x8 pb1 = pack_bf16x8(s[2 * kk][1], s[2 * kk + 1][1]);
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const uint8_t* p = vt + voff[db] + kk * 32 * t128::kRowBytes;
        const bf16x8 va = concat_bf16x4(t128::ds_read_tr(p), t128::ds_read_tr(p + 16 * t128::kRowBytes));
        o[db][0] = mfma16x16x32(va, pb0, o[db][0]);
        o[db][1] = mfma16x16x32(va, pb1, o[db][1]);
      }
    }
  };

  for (int j = 0; j < ntiles; ++j) {
    t128::wait_vmem();
    __syncthreads();
    if (j + 1 < ntiles) {
      const int nbuf = (j + 1) & 1;
      ld.load<true>(kbase, ks, (j + 1) * BN, a.Nk, smem[nbuf][0], wave, lane);
      ld.load<true>(vbase, ks, (j + 1) * BN, a.Nk, smem[nbuf][1], wave, lane);
    }
    const int key0 = j * BN;
    const int64_t kp_first = a.k_pos0 + key0;
    const int64_t kp_last = kp_first + BN - 1;
    if (qw0 >= a.Nq) continue;                     // wave past the shard tail
    if (a.causal && kp_first > wq_last) continue;  // every key after every query
    const uint8_t* kt = smem[j & 1][0];
    const uint8_t* vt = smem[j & 1][1];
    if ((a.causal && kp_last > wq_first) || kp_last >= a.valid || key0 + BN > a.Nk) {
      const int64_t ct = wq_first - kp_first;
      const int cthr = (int)(ct < -4096 ? -4096 : (ct > 4096 ? 4096 : ct));
      const int64_t km = min((int64_t)(a.Nk - key0), a.valid - kp_first);
      const int kmax = (int)(km < 0 ? 0 : (km > BN ? BN : km));
      tile(std::true_type{}, kt, vt, cthr, kmax);
    } else {
      tile(std::false_type{}, kt, vt, 0, BN);
    }
  }

  // Epilogue: o = acc / l; m in natural-log units; l as the reference defines it.
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const float lt = group4_sum(lsum[nb]);  // relative to mrun
    const int row = qw0 + 16 * nb + c;
    if (row < a.Nq) {
      const float inv = lt > 0.f ? 1.f / lt : 0.f;
      const float ltrue = lt > 0.f ? lt * fast_exp2(mrun[nb] - mtrue[nb]) : 0.f;
      float* orow = a.o + (((int64_t)b * a.Nq + row) * a.Hq + h) * D;
#pragma unroll
      for (int db = 0; db < DB; ++db)
        *reinterpret_cast<f32x4*>(orow + 16 * db + 4 * g) = o[db][nb] * inv;
      if (g == 0) {
        const int64_t si = ((int64_t)b * a.Hq + h) * a.Nq + row;
        a.m[si] = (mtrue[nb] == -INFINITY) ? -INFINITY : mtrue[nb] * kLn2;
        a.l[si] = ltrue;
      }
    }
  }
}

}  // namespace

hipError_t launch_fwd128(const Problem& p, const void* q, const void* k, const void* v, float* o,
                         float* m, float* l, hipStream_t s) {
  if (p.D != D) return hipErrorInvalidValue;
  Fwd128Args a;
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
  a.n_qtiles = (p.Nq + BM - 1) / BM;
  a.q_pos0 = p.q_pos0;
  a.k_pos0 = p.k_pos0;
  a.valid = p.valid;
  a.causal = p.causal ? 1 : 0;
  a.sl2 = p.scale * kLog2e;
  hipLaunchKernelGGL(fwd128_kernel, dim3(a.n_qtiles * p.Hq * p.B), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace lc
