// Recomputation backward of one ring hop for head_dim 128 on bf16 MFMA
// (gfx950 v_mfma_f32_32x32x16_bf16, fp32 accumulation).
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
//           query head of the GQA group (group sum in registers).  K^T in
//           VGPRs, the workgroup's V rows in LDS (negated once, so that
//           the dP accumulator runs from delta to delta - dP); 32-query
//           tiles of Q, dO, LSE and delta double-buffered in LDS.
//             S = Q K^T, dP = dO V^T       (A = Q, dO rows)
//             dV^T += dO^T P, dK^T += Q^T dS  (A = dO^T, Q^T: transposed reads)
// and, when one caller wants dQ and dK/dV of the same shard pair and gives a
// workspace, a dS-sharing pair: dkdv128 also stores its dS (bf16), and
//   dqds128 Q-stationary like dq128, but dQ^T += K^T dS^T with dS read back
//           (one GEMM instead of three; HBM-bound on the dS read).
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
  int64_t q_rows, k_rows;  // rows of the whole shards (batch strides; Nq, Nk: this launch's part)
  int64_t q_pos0, k_pos0, valid;
  int causal;
  float sl2;    // scale * log2(e)
  float scale;  // D^-1/2
  // dS exchange blocks (dkdv128 writes them when ds is set, dqds128 reads
  // them): ds_nqt query tiles x ds_nkb key blocks per (batch, query head).
  uint16_t* ds;
  int ds_nqt, ds_nkb;
};

// dS exchange layout.  dS (bf16, unscaled) of query tile qt (32 queries) and
// key block kb (32 keys) of head (b, hq) is a 2 KB block at element
// ((((b * Hq + hq) * nqt + qt) * nkb + kb) * 1024.  The dK/dV lane (key c,
// half h = lane / 32) holds k-step u of its dS B operand as 8 bf16: queries
// 16u + row(h, p, t) of tr32_off in slot 4p + t.  It stores them at byte
//   1024 u + 16 (ds_slot(c, h) ^ 8u)
// of the block, so one wave instruction writes 1 KB contiguously.  The dQ
// kernel reads the blocks back with transposed LDS reads (the key becomes the
// k index): the 16-byte slots of one transposed read (fixed key bits 0, 2, 4,
// varying bits 1, 3, the half and u) fall on 16 distinct slots modulo 256
// bytes, so the reads are free of bank conflicts.
__device__ __forceinline__ int ds_slot(int key, int half) {
  return ((key >> 1) & 1) | (((key >> 3) & 1) << 1) | (half << 2) | ((key & 1) << 3) |
         (((key >> 2) & 1) << 4) | (((key >> 4) & 1) << 5);
}
constexpr int kDsBlockElems = 1024;
constexpr int kDsBlockKeys = 32;  // keys per exchange block (= dK/dV keys per wave)

// ------------------------------------------------------------------- dQ --

constexpr int kDqQW = 32;
constexpr int kDqBM = 4 * kDqQW;  // queries per workgroup
constexpr int kDqBN = 64;         // keys per tile
constexpr int kDqTile = kDqBN * t128::kRowBytes;

// dQ with v_mfma_f32_32x32x16_bf16: each lane holds one query (lane % 32)
// of the wave's 32, so LSE and delta are one register each.  One 64-key tile
// is a stream of 48 MFMA steps j with LDS operands fetched two steps ahead:
//   j  0-15  S^T  = K Q^T      (mb, t) = (j % 2, j / 2)       A = K rows
//   j 16-31  dP^T = V dO^T     (mb, t) = ((j-16) / 8, (j-16) % 8), A = V rows
//   j 32-47  dQ^T += K^T dS^T  (u, dblk) = ((j-32) / 4, (j-32) % 4),
//                              A = K^T (transposed reads of the K tile)
// with P formed on the VALU during the dP steps and dS = P (dP - delta)
// during j 25-28 (keys 0-31) and 33-36 (keys 32-63).  The three phases are
// separate fully unrolled loops (one 48-step loop exceeds the unroller's
// limit, and a rolled loop would index the score arrays dynamically).  Score element v of
// block mb: key 32mb + 8(v/4) + 4(lane/32) + v%4.
__global__ __launch_bounds__(256, 2) void dq128_kernel(Bwd128Args a) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[2][2][kDqTile];  // [buf][K,V]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int kc = lane & 31;  // this lane's query within the wave
  const int hh = lane >> 5;

  const int L = xcd_remap(blockIdx.x, gridDim.x);
  const int qt = a.n_tiles - 1 - (L % a.n_tiles);
  const int bh = L / a.n_tiles;
  const int h = bh % a.Hq;
  const int b = bh / a.Hq;
  const int hk = h / a.group;

  const int64_t qs = (int64_t)a.Hq * D;
  const int64_t ks = (int64_t)a.Hkv * D;
  const uint16_t* qbase = a.q + (int64_t)b * a.q_rows * qs + (int64_t)h * D;
  const uint16_t* obase = a.dout + (int64_t)b * a.q_rows * qs + (int64_t)h * D;
  const uint16_t* kbase = a.k + (int64_t)b * a.k_rows * ks + (int64_t)hk * D;
  const uint16_t* vbase = a.v + (int64_t)b * a.k_rows * ks + (int64_t)hk * D;

  const int q0 = qt * kDqBM;
  const int qw0 = q0 + wave * kDqQW;

  const int q_end = min(q0 + kDqBM, a.Nq);
  int64_t kend = a.Nk;
  if (a.causal) kend = min(kend, a.q_pos0 + q_end - a.k_pos0);
  kend = min(kend, a.valid - a.k_pos0);
  const int ntiles = kend > 0 ? (int)((kend + kDqBN - 1) / kDqBN) : 0;
  if (ntiles == 0) return;  // nothing visible: dQ gets no contribution

  const uint32_t smem_lds = t128::lds_addr(smem);
  t128::RowLoader<kDqBN, 4> ld;
  ld.init(ks, wave, lane);
  ld.load(kbase, ks, 0, a.Nk, smem_lds, wave, lane);
  ld.load(vbase, ks, 0, a.Nk, smem_lds + kDqTile, wave, lane);

  // Q^T, dO^T as B operands: lane holds query qw0 + kc, dims 16t + 8hh .. +7.
  bf16x8 qreg[D / 16], doreg[D / 16];
  float lse, dl;
  {
    const int row = min(qw0 + kc, a.Nq - 1);
#pragma unroll
    for (int t = 0; t < D / 16; ++t) {
      qreg[t] = *reinterpret_cast<const bf16x8*>(qbase + (int64_t)row * qs + 16 * t + 8 * hh);
      doreg[t] = *reinterpret_cast<const bf16x8*>(obase + (int64_t)row * qs + 16 * t + 8 * hh);
    }
    const int64_t si = ((int64_t)b * a.Hq + h) * a.q_rows + row;
    lse = a.lse2[si];
    dl = a.delta[si];
  }

  const int roff0 = t128::row_chunk_off(kc, hh);  // row 32mb + kc, dims 16t + 8hh: ^ (32 t)
  const int toff0 = t128::tr32_off(0, lane), toff1 = t128::tr32_off(1, lane);

  const int64_t wq_first = a.q_pos0 + qw0;
  const int64_t wq_last = wq_first + kDqQW - 1;

  f32x16 acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[i] = f32x16{};

  // Mask (MASKED only): key idx + 4hh of the tile and query kc are invalid
  // when (causal && idx + 4hh - kc > cthr) || idx + 4hh >= kmax.
  auto tile = [&](auto masked_tag, const uint8_t* kt, const uint8_t* vt, int cthr, int kmax) {
    constexpr bool MASKED = decltype(masked_tag)::value;
    const int ro = opaque(roff0);
    const int to0 = opaque(toff0), to1 = opaque(toff1);
    int kq = 0, klim = 0;
    if constexpr (MASKED) {
      kq = opaque(4 * hh - kc);
      klim = opaque(kmax - 4 * hh);
    }
    auto fetch = [&](int j) {
      if (j < 16) {
        return *reinterpret_cast<const bf16x8*>(kt + ((ro ^ (32 * (j >> 1))) + (j & 1) * 32 * t128::kRowBytes));
      } else if (j < 32) {
        const int i = j - 16;
        return *reinterpret_cast<const bf16x8*>(vt + ((ro ^ (32 * (i & 7))) + (i >> 3) * 32 * t128::kRowBytes));
      } else {
        const int i = j - 32;
        const int o0 = (to0 ^ (64 * (i & 3))) + (i >> 2) * 16 * t128::kRowBytes;
        const int o1 = (to1 ^ (64 * (i & 3))) + (i >> 2) * 16 * t128::kRowBytes;
        return concat_bf16x4(t128::ds_read_tr(kt + o0), t128::ds_read_tr(kt + o1));
      }
    };
    f32x16 sv[2], dpv[2];
    bf16x8 A[2], dsb[4];
    // P for scores 4k .. 4k+3 (k = 0..7)
    auto probs = [&](int k) {
#pragma unroll
      for (int e = 4 * k; e < 4 * k + 4; ++e) {
        const int mb = e >> 4, v = e & 15;
        float x = sv[mb][v];
        if constexpr (MASKED) {
          const int idx = 32 * mb + 8 * (v >> 2) + (v & 3);
          const bool bad = (a.causal && kq > cthr - idx) || idx >= klim;
          x = bad ? -INFINITY : x;
        }
        sv[mb][v] = fast_exp2(fmaf(x, a.sl2, -lse));
      }
    };
    // dS for scores 4k .. 4k+3 of block mb (k = 0..3); packed at k = 3
    auto dscore = [&](int mb, int k) {
#pragma unroll
      for (int e = 4 * k; e < 4 * k + 4; ++e) dpv[mb][e] = sv[mb][e] * (dpv[mb][e] - dl);
      if (k == 3) {
#pragma unroll
        for (int u2 = 0; u2 < 2; ++u2) {
          const int e0 = 8 * u2;
          dsb[2 * mb + u2] = pack_bf16x8(
              f32x4{dpv[mb][e0], dpv[mb][e0 + 2], dpv[mb][e0 + 4], dpv[mb][e0 + 6]},
              f32x4{dpv[mb][e0 + 1], dpv[mb][e0 + 3], dpv[mb][e0 + 5], dpv[mb][e0 + 7]});
        }
      }
    };
    A[0] = fetch(0);
    A[1] = fetch(1);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < 16; ++j) {  // S^T
      sv[j & 1] = mfma32x32x16(A[j & 1], qreg[j >> 1], j < 2 ? f32x16{} : sv[j & 1]);
      A[j & 1] = fetch(j + 2);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {  // dP^T, P, dS of keys 0-31
      dpv[i >> 3] = mfma32x32x16(A[i & 1], doreg[i & 7], (i & 7) == 0 ? f32x16{} : dpv[i >> 3]);
      A[i & 1] = fetch(16 + i + 2);
      if (i >= 1 && i <= 8) probs(i - 1);
      if (i >= 9 && i <= 12) dscore(0, i - 9);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {  // dQ^T, dS of keys 32-63
      acc[i & 3] = mfma32x32x16(A[i & 1], dsb[i >> 2], acc[i & 3]);
      if (i + 2 < 16) A[i & 1] = fetch(32 + i + 2);
      if (i >= 1 && i <= 4) dscore(1, i - 1);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  for (int j = 0; j < ntiles; ++j) {
    t128::wait_vmem();
    __syncthreads();
    if (j + 1 < ntiles) {
      const uint32_t nb = smem_lds + ((j + 1) & 1) * 2 * kDqTile;
      ld.load(kbase, ks, (j + 1) * kDqBN, a.Nk, nb, wave, lane);
      ld.load(vbase, ks, (j + 1) * kDqBN, a.Nk, nb + kDqTile, wave, lane);
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

  // dQ^T element v of lane l: query qw0 + kc, dim 32*dblk + 8(v/4) + 4hh + v%4.
  const int row = qw0 + kc;
  if (row < a.Nq) {
    float* dst = a.dq + (((int64_t)b * a.q_rows + row) * a.Hq + h) * D;
#pragma unroll
    for (int d = 0; d < 4; ++d)
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        f32x4* p = reinterpret_cast<f32x4*>(dst + 32 * d + 8 * w + 4 * hh);
        const f32x4 v4 = {acc[d][4 * w], acc[d][4 * w + 1], acc[d][4 * w + 2], acc[d][4 * w + 3]};
        *p = *p + v4 * a.scale;
      }
  }
}

// ------------------------------------------------- dQ from stored dS --

// dQ^T += K^T dS^T with dS read back from the exchange blocks dkdv128 wrote
// for the same (query shard, KV shard) pair: no score recomputation, one
// GEMM.  Workgroup = 16 waves x 32 queries of one (batch, query head); 64-key
// tiles of K (shared, LDS DMA) and each wave's two dS blocks of the tile
// (its own, LDS DMA), one barrier per tile.  The more waves share each K tile,
// the fewer bytes cross into LDS per MFMA: per 32k x 32k x 16-head hop four
// waves took 6.4 ms, eight 5.9 ms, sixteen (dS one tile ahead instead of two)
// ~0.25 ms less again.
//   A = K^T (transposed reads of the K tile, tr32_off), B = dS^T (transposed
//   reads of the dS blocks, same key order)
// Column j of the accumulator is query qw0 + ds_query(j): the transposed read
// hands lane c of a 16-lane group element c % 4 of the 8-byte chunk c / 4 of
// a stored row, and a stored row of half h holds queries 16u + row(h, p, t).
// A tile block that dkdv128 skipped (keys past the shard or, causal, after
// every query of the wave) is replaced by zeros; inside a written block every
// masked score already has dS = 0.
constexpr int kDsWaveBytes = 2 * 2 * kDsBlockElems;  // a wave's two blocks of one tile
constexpr int kDsStages = 2;  // dS tiles in LDS: the one in use and one in flight
constexpr int kDsNW = 16;     // waves per workgroup (4 per SIMD: <= 128 VGPRs)
constexpr int kDsBM = kDsNW * kDqQW;  // queries per workgroup

__device__ __forceinline__ int ds_query(int j) {
  const int c = j & 15, cb = j >> 4;
  return 16 * (c >> 3) + 4 * cb + ((c >> 2) & 1) + 2 * (c & 1) + 8 * ((c >> 1) & 1);
}

// LDS: K double-buffered and dS in kDsStages buffers, both one tile ahead (the
// dS stream comes from HBM): 160 KB, one workgroup per CU.
__global__ __launch_bounds__(64 * kDsNW, 1) void dqds128_kernel(Bwd128Args a) {
  __shared__ __attribute__((aligned(1024))) uint8_t kbuf[2][kDqTile];
  __shared__ __attribute__((aligned(1024))) uint8_t dsbuf[kDsStages][kDsNW][kDsWaveBytes];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int kc = lane & 31;
  const int hh = lane >> 5;

  const int L = xcd_remap(blockIdx.x, gridDim.x);
  const int qt = a.n_tiles - 1 - (L % a.n_tiles);
  const int bh = L / a.n_tiles;
  const int h = bh % a.Hq;
  const int b = bh / a.Hq;
  const int hk = h / a.group;

  const int64_t ks = (int64_t)a.Hkv * D;
  const uint16_t* kbase = a.k + (int64_t)b * a.k_rows * ks + (int64_t)hk * D;

  const int q0 = qt * kDsBM;
  const int qw0 = q0 + wave * kDqQW;

  const int q_end = min(q0 + kDsBM, a.Nq);
  int64_t kend = a.Nk;
  if (a.causal) kend = min(kend, a.q_pos0 + q_end - a.k_pos0);
  kend = min(kend, a.valid - a.k_pos0);
  const int ntiles = kend > 0 ? (int)((kend + kDqBN - 1) / kDqBN) : 0;
  if (ntiles == 0) return;
  int nt_w = 0;
  if (qw0 < a.Nq) {
    int64_t kw = kend;
    if (a.causal) kw = min(kw, a.q_pos0 + min(qw0 + kDqQW, a.Nq) - a.k_pos0);
    nt_w = kw > 0 ? (int)((kw + kDqBN - 1) / kDqBN) : 0;
  }
  const int nkb = (a.Nk + kDsBlockKeys - 1) / kDsBlockKeys;  // this launch's key blocks
  // The wave's row of exchange blocks (only formed when the wave has tiles).
  const uint16_t* dsrow = nt_w > 0
      ? a.ds + (((int64_t)b * a.Hq + h) * a.ds_nqt + qw0 / kDqQW) * a.ds_nkb * kDsBlockElems
      : a.ds;

  const uint32_t kbuf_lds = t128::lds_addr(kbuf);
  const uint32_t ds_lds = t128::lds_addr(dsbuf) + wave * kDsWaveBytes;
  t128::RowLoader<kDqBN, kDsNW> ld;
  ld.init(ks, wave, lane);
  // dS of tile j (blocks 2j, 2j+1) as four DMA instructions (none for a tile
  // the wave does not compute); a missing block 2j+1 (past the keys) re-reads
  // block 2j, and its operand is zeroed below.
  auto load_ds = [&](int j) {
    if (j >= nt_w) return;
    const int nb = min(2, nkb - 2 * j);
    const uint16_t* src = dsrow + (int64_t)(2 * j) * kDsBlockElems;
    const uint32_t dst = ds_lds + (j % kDsStages) * kDsNW * kDsWaveBytes;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int si = i < 2 * nb ? i : i - 2;
      t128::dma_b128_nt(src + si * (kDsBlockElems / 2), 16u * lane, dst + i * 1024);
    }
  };
  ld.load(kbase, ks, 0, a.Nk, kbuf_lds, wave, lane);
  load_ds(0);

  // B operand read of k-step 0, k-half 0: lane (group G, index i) addresses
  // row key(hh, 0, t) of half G % 2, chunk g = i % 4 (u = g / 2, byte 8 (g % 2)).
  int dsoff0;
  {
    const int i = lane & 15, t = i >> 2, g = i & 3, u = g >> 1, cb = (lane >> 4) & 1;
    dsoff0 = u * 1024 + 16 * ((t | (cb << 2) | (hh << 4)) | (u << 3)) + 8 * (g & 1);
  }
  const int toff0 = t128::tr32_off(0, lane), toff1 = t128::tr32_off(1, lane);
  const int64_t wq_last = a.q_pos0 + qw0 + kDqQW - 1;

  f32x16 acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[i] = f32x16{};

  for (int j = 0; j < ntiles; ++j) {
    t128::wait_vmem();  // K_j and dS_j
    __syncthreads();
    if (j + 1 < ntiles)
      ld.load(kbase, ks, (j + 1) * kDqBN, a.Nk, kbuf_lds + ((j + 1) & 1) * kDqTile, wave, lane);
    load_ds(j + 1);
    if (j >= nt_w) continue;
    const uint8_t* kt = kbuf[j & 1];
    const uint8_t* dt = dsbuf[j % kDsStages][wave];
    // block 2j + 1 was not written by dkdv128: past the keys, or after every query
    const int64_t k1 = (int64_t)j * kDqBN + kDsBlockKeys;
    const bool skip1 = k1 >= a.Nk || (a.causal && a.k_pos0 + k1 > wq_last);
    const int so0 = opaque(dsoff0), so1 = so0 ^ 128;
    const int to0 = opaque(toff0), to1 = opaque(toff1);
    bf16x8 B[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int ko = (u >> 1) * 2 * kDsBlockElems + (u & 1) * 512;
      B[u] = concat_bf16x4(t128::ds_read_tr(dt + so0 + ko), t128::ds_read_tr(dt + so1 + ko));
    }
    if (skip1) B[2] = B[3] = bf16x8{};
    auto fetch = [&](int i) {  // K^T of keys 16(i/4) .., dims 32 (i%4) ..
      const int o0 = (to0 ^ (64 * (i & 3))) + (i >> 2) * 16 * t128::kRowBytes;
      const int o1 = (to1 ^ (64 * (i & 3))) + (i >> 2) * 16 * t128::kRowBytes;
      return concat_bf16x4(t128::ds_read_tr(kt + o0), t128::ds_read_tr(kt + o1));
    };
    bf16x8 A[2] = {fetch(0), fetch(1)};
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      acc[i & 3] = mfma32x32x16(A[i & 1], B[i >> 2], acc[i & 3]);
      if (i + 2 < 16) A[i & 1] = fetch(i + 2);
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // dQ^T element v of lane l: query qw0 + ds_query(l % 32), dim 32 dblk + 8(v/4) + 4hh + v%4.
  const int row = qw0 + ds_query(kc);
  if (nt_w > 0 && row < a.Nq) {
    float* dst = a.dq + (((int64_t)b * a.q_rows + row) * a.Hq + h) * D;
#pragma unroll
    for (int d = 0; d < 4; ++d)
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        f32x4* p = reinterpret_cast<f32x4*>(dst + 32 * d + 8 * w + 4 * hh);
        const f32x4 v4 = {acc[d][4 * w], acc[d][4 * w + 1], acc[d][4 * w + 2], acc[d][4 * w + 3]};
        *p = *p + v4 * a.scale;
      }
  }
}

// ---------------------------------------------------------------- dK/dV --

constexpr int kKvKW = 32;
constexpr int kKvBN = 4 * kKvKW;  // keys per workgroup
constexpr int kKvBM = 32;         // queries per tile
constexpr int kKvTile = kKvBM * t128::kRowBytes;

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
  const uint16_t* kbase = a.k + (int64_t)b * a.k_rows * ks + (int64_t)hk * D;
  const uint16_t* vbase = a.v + (int64_t)b * a.k_rows * ks + (int64_t)hk * D;

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
    const uint16_t* qb = a.q + (int64_t)b * a.q_rows * qs + (int64_t)hq * D;
    const uint16_t* ob = a.dout + (int64_t)b * a.q_rows * qs + (int64_t)hq * D;
    ld.load(qb, qs, qrow0, a.Nq, t128::lds_addr(smem) + buf * 2 * kKvTile, wave, lane);
    ld.load(ob, qs, qrow0, a.Nq, t128::lds_addr(smem) + (buf * 2 + 1) * kKvTile, wave, lane);
    const int64_t sbase = ((int64_t)b * a.Hq + hq) * a.q_rows;
    if (wave == 0) t128::load_f32x64(a.lse2 + sbase, qrow0, a.Nq, t128::lds_addr(stat) + buf * 512, lane);
    if (wave == 1) t128::load_f32x64(a.delta + sbase, qrow0, a.Nq, t128::lds_addr(stat) + buf * 512 + 256, lane);
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
    vld.load(vbase, ks, k0, a.Nk, t128::lds_addr(v_lds), wave, lane);
  }
  // K^T is in VGPRs from here on.  Without this wait the compiler (which
  // cannot tell how many vector memory operations the loop's waits leave
  // pending) would wait for the K loads before each S step, i.e. for every
  // load and store issued before that point.
  t128::wait_vmem();
  // V enters dP = dO V^T negated, so that the dP accumulator can start at
  // delta and end at delta - dP: dS = P (dP - delta) = -(P (delta - dP)).
  // Each wave negates the 32 rows it reads (written by every wave's DMA).
  __syncthreads();
  {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    uint8_t* vw = v_lds + wave * kKvKW * t128::kRowBytes + lane * 16;
#pragma unroll
    for (int i = 0; i < kKvKW * t128::kRowBytes / 1024; ++i) {
      u32x4* p = reinterpret_cast<u32x4*>(vw + i * 1024);
      *p = *p ^ 0x80008000u;
    }
  }

  // Row l%32 of a Q/dO tile, dims 16t + 8h .. +7, is roff0 ^ (32 t); the
  // wave's V rows are the same offsets in the wave's part of the V tile.
  const int roff0 = t128::row_chunk_off(kc, h);
  const int voff0 = roff0 + wave * kKvKW * t128::kRowBytes;
  const int toff0 = t128::tr32_off(0, lane), toff1 = t128::tr32_off(1, lane);
  f32x16 dk[4], dv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) dk[i] = dv[i] = f32x16{};

  const int64_t wk_first = a.k_pos0 + kw0;
  const int64_t wk_last = wk_first + kKvKW - 1;

  // One query tile as a stream of 32 MFMA steps j, each with its operands
  // fetched from LDS two steps ahead (A[j&1], B[j&1]):
  //   j  0- 7  S    += Q[:, 16t..]  K^T            (t = j)
  //   j  8-15  E    += dO[:, 16t..] (-V)^T         (t = j - 8), E = delta at j = 8
  //   j 16-23  dV^T += dO^T P       (u, dblk) = ((j-16)/4, (j-16)%4)
  //   j 24-31  dK^T += Q^T dS       (u, dblk) = ((j-24)/4, (j-24)%4)
  // P = exp2(S sl2 - lse2) is formed on the VALU during the E steps, and
  // dS = P (dP - delta) = -(P E) during the dV steps, beside the running
  // MFMAs: the V tile holds -V, so E ends at delta - dP (one multiply per
  // element instead of a subtraction and a multiply).
  bf16x8 ds_keep[2];  // the last tile's packed dS (both k-steps), stored at the next step's top
  auto tile = [&](auto masked_tag, int buf, int cthr, int kmax, int qmax) {
    constexpr bool MASKED = decltype(masked_tag)::value;
    const uint8_t* qt_ = &smem[0][0][0];
    const uint8_t* ot_ = &smem[0][1][0];
    const float* lse_ = stat[buf][0];
    const float* dlt_ = stat[buf][1];
    // The buffer offset (a multiple of 16 KB) is folded into the per-lane
    // bases: the swizzle XORs change only bits 5-7 of an offset below 8 KB.
    const int bo = buf * 2 * kKvTile;
    const int ro = opaque(roff0 + bo), vo = opaque(voff0);
    const int to0 = opaque(toff0 + bo), to1 = opaque(toff1 + bo);
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
    f32x16 sv, dpv, dinit;
    bf16x8 A[2], B[2], pb[2], db[2];
    f32x4 st[2];  // lse2 quads, loaded two steps before use
    fetch(0, A[0], B[0]);
    fetch(1, A[1], B[1]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      const int sl = j & 1;
      if (j < 8) {
        sv = mfma32x32x16(A[sl], kreg[j], j == 0 ? f32x16{} : sv);
      } else if (j < 16) {
        dpv = mfma32x32x16(A[sl], B[sl], j == 8 ? dinit : dpv);
      } else if (j < 24) {
        const int i = j - 16;
        dv[i & 3] = mfma32x32x16(A[sl], pb[i >> 2], dv[i & 3]);
      } else {
        const int i = j - 24;
        dk[i & 3] = mfma32x32x16(A[sl], db[i >> 2], dk[i & 3]);
      }
      if (j + 2 < 32) fetch(j + 2, A[sl], B[sl]);
      // statistics: lse2 quad w at j = 7 + 2w; delta (all four quads) at j = 5
      if (j >= 7 && j <= 13 && (j & 1)) {
        const int w = (j - 7) >> 1;
        st[w & 1] = *reinterpret_cast<const f32x4*>(&lse_[8 * w + 4 * h]);
      }
      if (j == 5) {  // delta of the lane's 16 queries, the dP accumulator's start
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const f32x4 d4 = *reinterpret_cast<const f32x4*>(&dlt_[8 * w + 4 * h]);
#pragma unroll
          for (int r = 0; r < 4; ++r) dinit[4 * w + r] = d4[r];
        }
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
          const int v = 2 * k + e;
          dpv[v] = -(sv[v] * dpv[v]);
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
      // k-step u of dS to the exchange block right after its pack, so that the
      // store has read its data long before the registers are reused
      if (j == 31) {  // stored at the next step's top
        ds_keep[0] = db[0];
        ds_keep[1] = db[1];
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  int cur_q = qstart, cur_hq = hq0;    // step being computed
  int nxt_hq = hq0, nxt_q = qstart;    // step being prefetched
  // dS stores: a tile's dS is stored at the top of the next step, after that
  // step's tile loads, so the wait for those loads at the following top does
  // not include the stores (vector memory operations complete in issue order,
  // and the stores take longer): they have two steps to complete.
  bool stored = false;  // this step's top issued the two dS stores (after its loads)
  int64_t pend = -1;    // exchange block of ds_keep, not yet stored
  auto store_ds = [&](int64_t blkid) {
    const int dsl = ds_slot(opaque(kc), opaque(h));
    typedef __attribute__((address_space(1))) bf16x8 gbl_bf16x8;  // global, not flat
    uint8_t* blk = reinterpret_cast<uint8_t*>(a.ds + (int64_t)blkid * kDsBlockElems);
    __builtin_nontemporal_store(ds_keep[0], (gbl_bf16x8*)(blk + 16 * dsl));
    __builtin_nontemporal_store(ds_keep[1], (gbl_bf16x8*)(blk + 1024 + 16 * (dsl ^ 8)));
  };
  for (int step = 0; step < nsteps; ++step) {
    if (stored)
      t128::wait_vmem_but<2>();  // the tile loads, not the stores issued after them
    else
      t128::wait_vmem();
    __syncthreads();
    stored = false;
    nxt_q += kKvBM;
    if (nxt_q >= a.Nq) {
      nxt_q = qstart;
      ++nxt_hq;
    }
    if (step + 1 < nsteps) issue(nxt_hq, nxt_q, (step + 1) & 1);
    if (pend >= 0) {  // the previous tile's dS, after the loads
      store_ds(pend);
      stored = true;
      pend = -1;
    }
    const int qrow0 = cur_q, hq_c = cur_hq;
    cur_q += kKvBM;
    if (cur_q >= a.Nq) {
      cur_q = qstart;
      ++cur_hq;
    }
    const int64_t qp_first = a.q_pos0 + qrow0;
    const int64_t qp_last = qp_first + kKvBM - 1;
    if (kw0 >= a.Nk) continue;
    if (a.causal && wk_first > qp_last) continue;
    const int buf = step & 1;
    const int64_t dsblk = a.ds == nullptr ? -1
        : (((int64_t)b * a.Hq + hq_c) * a.ds_nqt + qrow0 / kKvBM) * a.ds_nkb + kw0 / kKvKW;
    pend = dsblk;
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
  if (pend >= 0) store_ds(pend);

  // dK^T / dV^T element v of lane l: key kw0 + l%32, dim 32*dblk + 8(v/4) + 4h + v%4.
  const int row = kw0 + kc;
  if (row < a.Nk) {
    const int64_t off = (((int64_t)b * a.k_rows + row) * a.Hkv + hk) * D;
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
  a.q_rows = p.Nq;
  a.k_rows = p.Nk;
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
  a.ds = nullptr;
  a.ds_nqt = a.ds_nkb = 0;
  return a;
}

}  // namespace

hipError_t launch_dq128(const Problem& p, const void* q, const void* k, const void* v,
                        const void* dout, const float* lse2, const float* delta, float* dq,
                        hipStream_t s, int64_t k_rows) {
  if (p.D != D) return hipErrorInvalidValue;
  Bwd128Args a = make_args(p, q, k, v, dout, lse2, delta);
  if (k_rows >= 0) a.k_rows = k_rows;
  a.dq = dq;
  a.n_tiles = (p.Nq + kDqBM - 1) / kDqBM;
  hipLaunchKernelGGL(dq128_kernel, dim3(a.n_tiles * p.Hq * p.B), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_dkdv128(const Problem& p, const void* q, const void* k, const void* v,
                          const void* dout, const float* lse2, const float* delta, float* dk,
                          float* dv, hipStream_t s, int64_t q_rows, uint16_t* ds) {
  if (p.D != D) return hipErrorInvalidValue;
  Bwd128Args a = make_args(p, q, k, v, dout, lse2, delta);
  if (q_rows >= 0) a.q_rows = q_rows;
  a.dk = dk;
  a.dv = dv;
  if (ds != nullptr) {
    a.ds = ds;
    a.ds_nqt = (p.Nq + kKvBM - 1) / kKvBM;
    a.ds_nkb = (p.Nk + kDsBlockKeys - 1) / kDsBlockKeys;
  }
  a.n_tiles = (p.Nk + kKvBN - 1) / kKvBN;
  hipLaunchKernelGGL(dkdv128_kernel, dim3(a.n_tiles * p.Hkv * p.B), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_dqds128(const Problem& p, const void* k, const uint16_t* ds, int ds_nqt,
                          int ds_nkb, float* dq, hipStream_t s, int64_t k_rows, int64_t q_rows) {
  if (p.D != D) return hipErrorInvalidValue;
  Bwd128Args a = make_args(p, nullptr, k, nullptr, nullptr, nullptr, nullptr);
  if (k_rows >= 0) a.k_rows = k_rows;
  if (q_rows >= 0) a.q_rows = q_rows;
  a.dq = dq;
  a.ds = const_cast<uint16_t*>(ds);
  a.ds_nqt = ds_nqt;
  a.ds_nkb = ds_nkb;
  a.n_tiles = (p.Nq + kDsBM - 1) / kDsBM;
  hipLaunchKernelGGL(dqds128_kernel, dim3(a.n_tiles * p.Hq * p.B), dim3(64 * kDsNW), 0, s, a);
  return hipGetLastError();
}

}  // namespace lc
