// Recomputation backward of one ring hop for head_dim 128 on bf16 MFMA
// (gfx950 v_mfma_f32_16x16x32_bf16, fp32 accumulation).
//
// Semantics (rust/longctx100m-model/src/ring_attention.rs:383-409 and
// :433-454; src/longctx100m/ring_attention.py:338-357, :373-391):
//   P  = exp(s - m) / max(l, FLT_MIN) (0 where the row saw no key)
//      = 2^(s*scale*log2e - lse2), lse2 from lc_attn_bwd_preprocess
//   dS = P * (dO V^T - delta),  delta = rowsum(dO * O)
//   dQ += dS K * scale,  dK += dS^T Q * scale,  dV += P^T dO
//
// Two kernels without atomics (one owner per output element per launch, so
// results are deterministic):
//   dq128   Q-stationary, 4 waves x 32 queries.  Q^T, dO^T in VGPRs; 64-key
//           tiles of K and V double-buffered in LDS.
//             S^T = K Q^T, dP^T = V dO^T   (A = K, V rows: ds_read_b128)
//             dQ^T += K^T dS^T             (A = K^T: ds_read_b64_tr_b16)
//   dkdv128 KV-stationary, 4 waves x 32 keys of one KV head, walking every
//           query head of the GQA group (group sum in registers).  K^T, V^T
//           in VGPRs; 64-query tiles of Q, dO, LSE and delta double-buffered
//           in LDS.
//             S = Q K^T, dP = dO V^T       (A = Q, dO rows)
//             dV^T += dO^T P, dK^T += Q^T dS  (A = dO^T, Q^T: transposed reads)
// Tiles are swizzled row-major and filled by direct global->LDS loads
// (tile128.h); each score accumulator's C layout is reused as the B operand
// of the following product.
#include "common.h"
#include "kernels.h"
#include "tile128.h"

#include <type_traits>

namespace lc {
namespace {

constexpr int D = 128;
constexpr int KS = D / 32;
constexpr int DB = D / 16;

struct Bwd128Args {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* dout;
  const float* lse2;
  const float* delta;
  float* dq;
  float* dk;
  float* dv;
  int Nq, Nk, Hq, Hkv, group, n_tiles;
  int64_t q_pos0, k_pos0, valid;
  int causal;
  float sl2;    // scale * log2(e)
  float scale;  // D^-1/2
};

// ------------------------------------------------------------------- dQ --

constexpr int kDqQW = 32;
constexpr int kDqBM = 4 * kDqQW;  // queries per workgroup
constexpr int kDqBN = 64;         // keys per tile
constexpr int kDqTile = kDqBN * t128::kRowBytes;

__global__ __launch_bounds__(256, 2) void dq128_kernel(Bwd128Args a) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[2][2][kDqTile];  // [buf][K,V]

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

  const int q0 = qt * kDqBM;
  const int qw0 = q0 + wave * kDqQW;

  const int q_end = min(q0 + kDqBM, a.Nq);
  int64_t kend = a.Nk;
  if (a.causal) kend = min(kend, a.q_pos0 + q_end - a.k_pos0);
  kend = min(kend, a.valid - a.k_pos0);
  const int ntiles = kend > 0 ? (int)((kend + kDqBN - 1) / kDqBN) : 0;
  if (ntiles == 0) return;  // nothing visible: dQ gets no contribution

  t128::RowLoader<kDqBN, 4> ld;
  ld.init(ks, wave, lane);
  ld.load<true>(kbase, ks, 0, a.Nk, smem[0][0], wave, lane);
  ld.load<true>(vbase, ks, 0, a.Nk, smem[0][1], wave, lane);

  bf16x8 qreg[2][KS], doreg[2][KS];
  float lse[2], dl[2];
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int row = min(qw0 + 16 * nb + c, a.Nq - 1);
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      qreg[nb][kk] = *reinterpret_cast<const bf16x8*>(qbase + (int64_t)row * qs + 32 * kk + 8 * g);
      doreg[nb][kk] = *reinterpret_cast<const bf16x8*>(obase + (int64_t)row * qs + 32 * kk + 8 * g);
    }
    const int64_t si = ((int64_t)b * a.Hq + h) * a.Nq + row;
    lse[nb] = a.lse2[si];
    dl[nb] = a.delta[si];
  }

  int roff[KS];
#pragma unroll
  for (int kk = 0; kk < KS; ++kk) roff[kk] = t128::row_chunk_off(c, 4 * kk + g);
  int toff[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) toff[db] = t128::tr_off(0, 16 * db, lane);

  const int64_t wq_first = a.q_pos0 + qw0;
  const int64_t wq_last = wq_first + kDqQW - 1;

  f32x4 acc[DB][2];
#pragma unroll
  for (int db = 0; db < DB; ++db) acc[db][0] = acc[db][1] = f32x4{0.f, 0.f, 0.f, 0.f};

  // One tile, per 32-key half (kk2): S^T = K Q^T and dP^T = V dO^T for keys
  // 32*kk2 + [16mb+4g+i] x query 16nb+c, then dQ^T += K^T dS^T.  Mask (MASKED
  // only): key k of the tile / query q of the wave are invalid when
  // (causal && k - q > cthr) || k >= kmax.
  auto tile = [&](auto masked_tag, const uint8_t* kt, const uint8_t* vt, int cthr, int kmax) {
    constexpr bool MASKED = decltype(masked_tag)::value;
#pragma unroll
    for (int kk2 = 0; kk2 < kDqBN / 32; ++kk2) {
      f32x4 s[2][2], dp[2][2];
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
        s[mb][0] = s[mb][1] = dp[mb][0] = dp[mb][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) {
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) {
          const int off = roff[kk] + (2 * kk2 + mb) * 16 * t128::kRowBytes;
          const bf16x8 ka = *reinterpret_cast<const bf16x8*>(kt + off);
          const bf16x8 va = *reinterpret_cast<const bf16x8*>(vt + off);
          s[mb][0] = mfma16x16x32(ka, qreg[0][kk], s[mb][0]);
          s[mb][1] = mfma16x16x32(ka, qreg[1][kk], s[mb][1]);
          dp[mb][0] = mfma16x16x32(va, doreg[0][kk], dp[mb][0]);
          dp[mb][1] = mfma16x16x32(va, doreg[1][kk], dp[mb][1]);
        }
      }
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int nb = 0; nb < 2; ++nb)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            float x = s[mb][nb][i];
            if constexpr (MASKED) {
              const int kr = 32 * kk2 + 16 * mb + 4 * g + i;
              const bool bad = (a.causal && kr - (16 * nb + c) > cthr) || kr >= kmax;
              x = bad ? -INFINITY : x;
            }
            const float p = fast_exp2(fmaf(x, a.sl2, -lse[nb]));
            s[mb][nb][i] = p * (dp[mb][nb][i] - dl[nb]);  // dS^T
          }
      const bf16x8 b0 = pack_bf16x8(s[0][0], s[1][0]);
      const bf16x8 b1 = pack_bf16x8(s[0][1], s[1][1]);
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const uint8_t* p = kt + toff[db] + kk2 * 32 * t128::kRowBytes;
        const bf16x8 ka = concat_bf16x4(t128::ds_read_tr(p), t128::ds_read_tr(p + 16 * t128::kRowBytes));
        acc[db][0] = mfma16x16x32(ka, b0, acc[db][0]);
        acc[db][1] = mfma16x16x32(ka, b1, acc[db][1]);
      }
    }
  };

  for (int j = 0; j < ntiles; ++j) {
    t128::wait_vmem();
    __syncthreads();
    if (j + 1 < ntiles) {
      const int nbuf = (j + 1) & 1;
      ld.load<true>(kbase, ks, (j + 1) * kDqBN, a.Nk, smem[nbuf][0], wave, lane);
      ld.load<true>(vbase, ks, (j + 1) * kDqBN, a.Nk, smem[nbuf][1], wave, lane);
    }
    const int key0 = j * kDqBN;
    const int64_t kp_first = a.k_pos0 + key0;
    const int64_t kp_last = kp_first + kDqBN - 1;
    if (qw0 >= a.Nq) continue;
    if (a.causal && kp_first > wq_last) continue;
    const uint8_t* kt = smem[j & 1][0];
    const uint8_t* vt = smem[j & 1][1];
    if ((a.causal && kp_last > wq_first) || kp_last >= a.valid || key0 + kDqBN > a.Nk) {
      const int64_t ct = wq_first - kp_first;
      const int cthr = (int)(ct < -4096 ? -4096 : (ct > 4096 ? 4096 : ct));
      const int64_t km = min((int64_t)(a.Nk - key0), a.valid - kp_first);
      const int kmax = (int)(km < 0 ? 0 : (km > kDqBN ? kDqBN : km));
      tile(std::true_type{}, kt, vt, cthr, kmax);
    } else {
      tile(std::false_type{}, kt, vt, 0, kDqBN);
    }
  }

#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int row = qw0 + 16 * nb + c;
    if (row < a.Nq) {
      float* dst = a.dq + (((int64_t)b * a.Nq + row) * a.Hq + h) * D + 4 * g;
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        f32x4* p = reinterpret_cast<f32x4*>(dst + 16 * db);
        *p = *p + acc[db][nb] * a.scale;
      }
    }
  }
}

// ---------------------------------------------------------------- dK/dV --

constexpr int kKvKW = 32;
constexpr int kKvBN = 4 * kKvKW;  // keys per workgroup
constexpr int kKvBM = 32;         // queries per tile
constexpr int kKvTile = kKvBM * t128::kRowBytes;

typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ f32x16 mfma32x32x16(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Byte offset of a transposed read for the 32x32x16 A operand X^T (X = a
// [32 x 128] Q or dO tile; k index = query row, m index = column), column
// block 0 and k-half p: lane l receives X[row(l/32, p, t)][l%32] in slot t,
// with row(h, p, t) = 4h + p + 2(t%2) + 8(t/2).  The four rows read in one
// cycle (lanes 0-31 or 32-63) then have distinct swz(r) / 4, so the 4 rows x
// 4 chunks land on 16 distinct chunks (no bank conflict).  Column block dblk
// is offset ^ (64 * dblk) (the block index occupies chunk bits 2-3 alone);
// rows 16 .. 31 are offset + 16 * kRowBytes (swz depends on r % 16).
__device__ __forceinline__ int tr32_off(int p, int lane) {
  const int G = lane >> 4, i = lane & 15, t = i >> 2;
  const int col = 16 * (G & 1) + 4 * (i & 3);
  const int r = 4 * (G >> 1) + p + 2 * (t & 1) + 8 * (t >> 1);
  return r * t128::kRowBytes + 16 * ((col >> 3) ^ t128::swz(r)) + 2 * (col & 7);
}

// Hides a value from loop-invariant code motion, so offsets derived from it
// by an XOR are formed next to their use instead of occupying registers.
__device__ __forceinline__ int opaque(int x) {
  asm volatile("" : "+v"(x));
  return x;
}

// dK/dV with v_mfma_f32_32x32x16_bf16: one 32x32 score block per wave and
// query tile, so half the MFMA instructions of the 16x16x32 form.
//   S = Q K^T, dP = dO V^T    A = Q, dO rows (ds_read_b128), B = K^T (VGPRs),
//                             V^T (rows of the V tile)
//   dV^T += dO^T P, dK^T += Q^T dS   A = dO^T, Q^T (transposed reads),
//                             B = P, dS straight from the score accumulators
// Score element v of lane l: query 8(v/4) + 4(l/32) + v%4, key l%32.  As a B
// operand, k-step u (queries 16u .. 16u+15) takes, in slot 4p + t, element
// 8u + 4(t/2) + 2(t%2) + p, i.e. query 16u + row(h, p, t) of tr32_off.
__global__ __launch_bounds__(256, 2) void dkdv128_kernel(Bwd128Args a) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[2][2][kKvTile];  // [buf][Q,dO]
  __shared__ __attribute__((aligned(1024))) uint8_t v_lds[kKvBN * t128::kRowBytes];
  __shared__ __attribute__((aligned(16))) float stat[2][2][64];           // [buf][lse2,delta]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int kc = lane & 31;  // key column of the wave's 32 keys
  const int h = lane >> 5;

  const int L = xcd_remap(blockIdx.x, gridDim.x);
  const int kt = L % a.n_tiles;  // early keys see the most queries: dispatched first
  const int bh = L / a.n_tiles;
  const int hk = bh % a.Hkv;
  const int b = bh / a.Hkv;

  const int64_t qs = (int64_t)a.Hq * D;
  const int64_t ks = (int64_t)a.Hkv * D;
  const uint16_t* kbase = a.k + (int64_t)b * a.Nk * ks + (int64_t)hk * D;
  const uint16_t* vbase = a.v + (int64_t)b * a.Nk * ks + (int64_t)hk * D;

  const int k0 = kt * kKvBN;
  const int kw0 = k0 + wave * kKvKW;

  // Queries that can see any key of this workgroup.
  const int64_t kp_wg_first = a.k_pos0 + k0;
  int qstart = 0;
  if (a.causal) {
    const int64_t first = kp_wg_first - a.q_pos0;
    qstart = first <= 0 ? 0 : (first >= a.Nq ? a.Nq : (int)first);
  }
  qstart = (qstart / kKvBM) * kKvBM;
  const bool any_valid_key = kp_wg_first < a.valid && k0 < a.Nk;
  const int ntq = any_valid_key ? (a.Nq - qstart + kKvBM - 1) / kKvBM : 0;
  const int nsteps = ntq * a.group;
  if (nsteps == 0) return;  // no visible (query, key) pair: no contribution

  t128::RowLoader<kKvBM, 4> ld;
  ld.init(qs, wave, lane);
  auto issue = [&](int hq, int qrow0, int buf) {
    const uint16_t* qb = a.q + (int64_t)b * a.Nq * qs + (int64_t)hq * D;
    const uint16_t* ob = a.dout + (int64_t)b * a.Nq * qs + (int64_t)hq * D;
    ld.load(qb, qs, qrow0, a.Nq, smem[buf][0], wave, lane);
    ld.load(ob, qs, qrow0, a.Nq, smem[buf][1], wave, lane);
    const int64_t sbase = ((int64_t)b * a.Hq + hq) * a.Nq;
    if (wave == 0) t128::load_f32x64(a.lse2 + sbase, qrow0, a.Nq, stat[buf][0], lane);
    if (wave == 1) t128::load_f32x64(a.delta + sbase, qrow0, a.Nq, stat[buf][1], lane);
  };
  const int hq0 = hk * a.group;
  issue(hq0, qstart, 0);

  // K^T as the B operand in VGPRs: lane l holds key kw0 + l%32, dims 16t + 8h .. +7.
  bf16x8 kreg[D / 16];
  {
    const int row = min(kw0 + kc, a.Nk - 1);
#pragma unroll
    for (int t = 0; t < D / 16; ++t)
      kreg[t] = *reinterpret_cast<const bf16x8*>(kbase + (int64_t)row * ks + 16 * t + 8 * h);
  }
  {
    t128::RowLoader<kKvBN, 4> vld;
    vld.init(ks, wave, lane);
    vld.load(vbase, ks, k0, a.Nk, v_lds, wave, lane);
  }

  // Row l%32 of a Q/dO tile, dims 16t + 8h .. +7, is roff0 ^ (32 t); the
  // wave's V rows are the same offsets in the wave's part of the V tile.
  const int roff0 = t128::row_chunk_off(kc, h);
  const int voff0 = roff0 + wave * kKvKW * t128::kRowBytes;
  const int toff0 = tr32_off(0, lane), toff1 = tr32_off(1, lane);
  f32x16 dk[4], dv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) dk[i] = dv[i] = f32x16{};

  const int64_t wk_first = a.k_pos0 + kw0;
  const int64_t wk_last = wk_first + kKvKW - 1;

  // One query tile as a stream of 32 MFMA steps j, each with its operands
  // fetched from LDS two steps ahead (A[j&1], B[j&1]):
  //   j  0- 7  S    += Q[:, 16t..]  K^T            (t = j)
  //   j  8-15  dP   += dO[:, 16t..] V^T            (t = j - 8)
  //   j 16-23  dV^T += dO^T P       (u, dblk) = ((j-16)/4, (j-16)%4)
  //   j 24-31  dK^T += Q^T dS       (u, dblk) = ((j-24)/4, (j-24)%4)
  // P = exp2(S sl2 - lse2) is formed on the VALU during the dP steps, and
  // dS = P (dP - delta) during the dV steps, beside the running MFMAs.
  auto tile = [&](auto masked_tag, int buf, int cthr, int kmax, int qmax) {
    constexpr bool MASKED = decltype(masked_tag)::value;
    const uint8_t* qt_ = smem[buf][0];
    const uint8_t* ot_ = smem[buf][1];
    const float* lse_ = stat[buf][0];
    const float* dlt_ = stat[buf][1];
    const int ro = opaque(roff0), vo = opaque(voff0);
    const int to0 = opaque(toff0), to1 = opaque(toff1);
    auto ld = [](const uint8_t* p) { return *reinterpret_cast<const bf16x8*>(p); };
    auto fetch = [&](int j, bf16x8& A, bf16x8& B) {
      if (j < 8) {
        A = ld(qt_ + (ro ^ (32 * j)));
      } else if (j < 16) {
        A = ld(ot_ + (ro ^ (32 * (j - 8))));
        B = ld(v_lds + (vo ^ (32 * (j - 8))));
      } else {
        const uint8_t* src = j < 24 ? ot_ : qt_;
        const int i = (j - 16) & 7;
        const int o0 = (to0 ^ (64 * (i & 3))) + (i >> 2) * 16 * t128::kRowBytes;
        const int o1 = (to1 ^ (64 * (i & 3))) + (i >> 2) * 16 * t128::kRowBytes;
        A = concat_bf16x4(t128::ds_read_tr(src + o0), t128::ds_read_tr(src + o1));
      }
    };
    int kq = 0, qlim = 0;
    bool kbad = false;
    if constexpr (MASKED) {
      kq = opaque(kc - 4 * h);
      qlim = opaque(qmax - 4 * h);
      kbad = kc >= kmax;
    }
    f32x16 sv, dpv;
    bf16x8 A[2], B[2], pb[2], db[2];
    f32x4 st[2];  // lse2 / delta quads, loaded two steps before use
    fetch(0, A[0], B[0]);
    fetch(1, A[1], B[1]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      const int sl = j & 1;
      if (j < 8) {
        sv = mfma32x32x16(A[sl], kreg[j], j == 0 ? f32x16{} : sv);
      } else if (j < 16) {
        dpv = mfma32x32x16(A[sl], B[sl], j == 8 ? f32x16{} : dpv);
      } else if (j < 24) {
        const int i = j - 16;
        dv[i & 3] = mfma32x32x16(A[sl], pb[i >> 2], dv[i & 3]);
      } else {
        const int i = j - 24;
        dk[i & 3] = mfma32x32x16(A[sl], db[i >> 2], dk[i & 3]);
      }
      if (j + 2 < 32) fetch(j + 2, A[sl], B[sl]);
      // statistics: lse2 quad w at j = 7 + 2w, delta quad w at j = 16 + 2w
      if (j >= 7 && j <= 13 && (j & 1)) {
        const int w = (j - 7) >> 1;
        st[w & 1] = *reinterpret_cast<const f32x4*>(&lse_[8 * w + 4 * h]);
      }
      if (j >= 16 && j <= 22 && !(j & 1)) {
        const int w = (j - 16) >> 1;
        st[w & 1] = *reinterpret_cast<const f32x4*>(&dlt_[8 * w + 4 * h]);
      }
      // P for elements 2k, 2k+1 at j = 9 + k
      if (j >= 9 && j <= 16) {
        const int k = j - 9;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const int v = 2 * k + e, w = v >> 2, r = v & 3;
          float x = sv[v];
          if constexpr (MASKED) {
            // query 4h + (8w + r) against key kc: the per-lane parts are kq, qlim
            const int qo = 8 * w + r;
            const bool bad = kbad || (a.causal && kq > cthr + qo) || qo >= qlim;
            x = bad ? -INFINITY : x;
          }
          sv[v] = fast_exp2(fmaf(x, a.sl2, -st[w & 1][r]));
        }
      }
      // dS for elements 2k, 2k+1 at j = 18 + k
      if (j >= 18 && j <= 25) {
        const int k = j - 18;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const int v = 2 * k + e, w = v >> 2, r = v & 3;
          dpv[v] = sv[v] * (dpv[v] - st[w & 1][r]);
        }
      }
      // Packed bf16 B operands (slot 4p + t <- element 8u + 4(t/2) + 2(t%2) + p)
      if (j == 12 || j == 16) {
        const int u = (j - 12) >> 2;
        pb[u] = pack_bf16x8(f32x4{sv[8 * u], sv[8 * u + 2], sv[8 * u + 4], sv[8 * u + 6]},
                            f32x4{sv[8 * u + 1], sv[8 * u + 3], sv[8 * u + 5], sv[8 * u + 7]});
      }
      if (j == 21 || j == 25) {
        const int u = (j - 21) >> 2;
        db[u] = pack_bf16x8(f32x4{dpv[8 * u], dpv[8 * u + 2], dpv[8 * u + 4], dpv[8 * u + 6]},
                            f32x4{dpv[8 * u + 1], dpv[8 * u + 3], dpv[8 * u + 5], dpv[8 * u + 7]});
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  int cur_q = qstart;                  // step being computed
  int nxt_hq = hq0, nxt_q = qstart;    // step being prefetched
  for (int step = 0; step < nsteps; ++step) {
    t128::wait_vmem();
    __syncthreads();
    nxt_q += kKvBM;
    if (nxt_q >= a.Nq) {
      nxt_q = qstart;
      ++nxt_hq;
    }
    if (step + 1 < nsteps) issue(nxt_hq, nxt_q, (step + 1) & 1);
    const int qrow0 = cur_q;
    cur_q += kKvBM;
    if (cur_q >= a.Nq) cur_q = qstart;
    const int64_t qp_first = a.q_pos0 + qrow0;
    const int64_t qp_last = qp_first + kKvBM - 1;
    if (kw0 >= a.Nk) continue;
    if (a.causal && wk_first > qp_last) continue;
    const int buf = step & 1;
    if ((a.causal && wk_last > qp_first) || wk_last >= a.valid || kw0 + kKvKW > a.Nk ||
        qrow0 + kKvBM > a.Nq) {
      const int64_t ct = qp_first - wk_first;
      const int cthr = (int)(ct < -4096 ? -4096 : (ct > 4096 ? 4096 : ct));
      const int64_t km = min((int64_t)(a.Nk - kw0), a.valid - wk_first);
      const int kmax = (int)(km < 0 ? 0 : (km > kKvKW ? kKvKW : km));
      const int qmax = min(a.Nq - qrow0, kKvBM);
      tile(std::true_type{}, buf, cthr, kmax, qmax);
    } else {
      tile(std::false_type{}, buf, 0, kKvKW, kKvBM);
    }
  }

  // dK^T / dV^T element v of lane l: key kw0 + l%32, dim 32*dblk + 8(v/4) + 4h + v%4.
  const int row = kw0 + kc;
  if (row < a.Nk) {
    const int64_t off = (((int64_t)b * a.Nk + row) * a.Hkv + hk) * D;
#pragma unroll
    for (int dblk = 0; dblk < 4; ++dblk)
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const int d0 = 32 * dblk + 8 * w + 4 * h;
        f32x4* pk = reinterpret_cast<f32x4*>(a.dk + off + d0);
        f32x4* pv = reinterpret_cast<f32x4*>(a.dv + off + d0);
        const f32x4 k4 = {dk[dblk][4 * w], dk[dblk][4 * w + 1], dk[dblk][4 * w + 2], dk[dblk][4 * w + 3]};
        const f32x4 v4 = {dv[dblk][4 * w], dv[dblk][4 * w + 1], dv[dblk][4 * w + 2], dv[dblk][4 * w + 3]};
        *pk = *pk + k4 * a.scale;
        *pv = *pv + v4;
      }
  }
}

Bwd128Args make_args(const Problem& p, const void* q, const void* k, const void* v,
                     const void* dout, const float* lse2, const float* delta) {
  Bwd128Args a;
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.dout = static_cast<const uint16_t*>(dout);
  a.lse2 = lse2;
  a.delta = delta;
  a.dq = a.dk = a.dv = nullptr;
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

hipError_t launch_dq128(const Problem& p, const void* q, const void* k, const void* v,
                        const void* dout, const float* lse2, const float* delta, float* dq,
                        hipStream_t s) {
  if (p.D != D) return hipErrorInvalidValue;
  Bwd128Args a = make_args(p, q, k, v, dout, lse2, delta);
  a.dq = dq;
  a.n_tiles = (p.Nq + kDqBM - 1) / kDqBM;
  hipLaunchKernelGGL(dq128_kernel, dim3(a.n_tiles * p.Hq * p.B), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_dkdv128(const Problem& p, const void* q, const void* k, const void* v,
                          const void* dout, const float* lse2, const float* delta, float* dk,
                          float* dv, hipStream_t s) {
  if (p.D != D) return hipErrorInvalidValue;
  Bwd128Args a = make_args(p, q, k, v, dout, lse2, delta);
  a.dk = dk;
  a.dv = dv;
  a.n_tiles = (p.Nk + kKvBN - 1) / kKvBN;
  hipLaunchKernelGGL(dkdv128_kernel, dim3(a.n_tiles * p.Hkv * p.B), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace lc
