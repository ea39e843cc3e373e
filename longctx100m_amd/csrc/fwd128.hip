// Blockwise causal forward of one ring hop for head_dim 128 on bf16 MFMA
// (gfx950 v_mfma_f32_32x32x16_bf16, fp32 accumulation).
//
// Semantics: the reference's tiled online-softmax update over one KV shard
// (rust/longctx100m-model/src/ring_attention.rs:15-106, the body of the hop
// loop at :195-219) and its finalize (:227).  The workgroup emits the shard's
// normalised output o = acc / l and statistics (m, l); lc_attn_merge folds
// them into the ring's running state.
//
// Work split: workgroup = NW waves x 32 queries of one (batch, query head),
// two waves per SIMD.  Q^T lives in VGPRs as the MFMA B operand; 64-key
// tiles of K and V live in LDS as swizzled row-major tiles (tile128.h),
// filled by LDS DMA.  Moving a tile into LDS costs SIMD cycles in proportion
// to its bytes, so a hop whose keys all precede its queries (no causal
// diagonal) runs NW = 8 (256 queries share each tile, one workgroup per CU:
// half the DMA per MFMA); a hop that straddles the diagonal runs NW = 4 (two
// workgroups per CU), whose shorter query range wastes less of each
// workgroup's tile walk on waves that have no key left to see.
//   S^T = K Q^T     A = K rows (ds_read_b128), B = Q^T
//   O^T += V^T P^T  A = V^T (transposed reads of the V tile),
//                   B = P^T straight from the S^T accumulators
// Each lane's scores and outputs belong to one query (lane % 32); the two
// lanes l, l ^ 32 share a query and split its keys, so a row maximum is a
// per-lane maximum plus one permlane32 swap, and the row sum stays
// lane-partial until the epilogue.
//
// Software pipeline: iteration j issues the MFMAs of S^T for tile j + 1 and,
// beside them on the VALU, the softmax of tile j (whose scores the previous
// iteration produced), then O^T += V_j^T P_j^T.  K therefore runs one tile
// ahead of V: iteration j loads K tile j + 2 and V tile j + 1 into the
// buffers iteration j - 1 finished with (two buffers each, one barrier per
// tile).  LDS operands of every MFMA are fetched two MFMAs ahead.  The mask
// is applied only on tiles that straddle the diagonal, valid_length or the
// shard tail (a separate instantiation of the iteration).  GQA: query head h
// reads KV head h / (Hq / Hkv).
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
constexpr int kQW = 32;             // queries per wave
constexpr int BN = 64;              // keys per tile
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
  int64_t kv_bstride;  // elements between batches of K and V
  int causal;
  int accumulate;  // merge into the running (o, m, l) instead of writing them
  float sl2;       // scale * log2(e)
};

template <int NW>
__global__ __launch_bounds__(64 * NW, 8 / NW) void fwd128_kernel(Fwd128Args a) {
  constexpr int kWaves = NW;
  constexpr int BM = kWaves * kQW;  // queries per workgroup
  __shared__ __attribute__((aligned(1024))) uint8_t kbuf[2][kTileBytes];
  __shared__ __attribute__((aligned(1024))) uint8_t vbuf[2][kTileBytes];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int kc = lane & 31;  // this lane's query within the wave
  const int hh = lane >> 5;  // which half of each 8-key group the lane holds

  const int L = xcd_remap(blockIdx.x, gridDim.x);
  const int qt = a.n_qtiles - 1 - (L % a.n_qtiles);  // long query tiles first
  const int bh = L / a.n_qtiles;
  const int hq = bh % a.Hq;
  const int b = bh / a.Hq;
  const int hk = hq / a.group;

  const int64_t qs = (int64_t)a.Hq * D;
  const int64_t ks = (int64_t)a.Hkv * D;
  const uint16_t* qbase = a.q + (int64_t)b * a.Nq * qs + (int64_t)hq * D;
  const uint16_t* kbase = a.k + (int64_t)b * a.kv_bstride + (int64_t)hk * D;
  const uint16_t* vbase = a.v + (int64_t)b * a.kv_bstride + (int64_t)hk * D;

  const int q0 = qt * BM;
  const int qw0 = q0 + wave * kQW;

  // Key tiles the workgroup loads, and the prefix of them this wave computes
  // (every tile with a key visible to one of its queries).
  const int q_end = min(q0 + BM, a.Nq);
  int64_t kend = a.Nk;
  if (a.causal) kend = min(kend, a.q_pos0 + q_end - a.k_pos0);
  kend = min(kend, a.valid - a.k_pos0);
  const int ntiles = kend > 0 ? (int)((kend + BN - 1) / BN) : 0;
  int nt_w = 0;
  if (qw0 < a.Nq) {
    int64_t kw = kend;
    if (a.causal) kw = min(kw, a.q_pos0 + min(qw0 + kQW, a.Nq) - a.k_pos0);
    nt_w = kw > 0 ? (int)((kw + BN - 1) / BN) : 0;
  }

  t128::RowLoader<BN, kWaves> ld;
  ld.init(ks, wave, lane);
  if (ntiles > 0) {
    ld.load(kbase, ks, 0, a.Nk, t128::lds_addr(kbuf), wave, lane);
    ld.load(vbase, ks, 0, a.Nk, t128::lds_addr(vbuf), wave, lane);
  }
  if (ntiles > 1) ld.load(kbase, ks, BN, a.Nk, t128::lds_addr(kbuf) + kTileBytes, wave, lane);

  // Q^T as B operand: lane holds query qw0 + kc, head dims 16t + 8hh .. +7.
  bf16x8 qreg[D / 16];
  {
    const int row = min(qw0 + kc, a.Nq - 1);
#pragma unroll
    for (int t = 0; t < D / 16; ++t)
      qreg[t] = *reinterpret_cast<const bf16x8*>(qbase + (int64_t)row * qs + 16 * t + 8 * hh);
  }

  // LDS offsets of the lane's operand fragments, computed once and kept in
  // registers (the swizzle XORs would otherwise be redone on every tile):
  //   K row 32mb + kc, dims 16t + 8hh: koff[t] + mb * 32 rows;
  //   V^T, PV step i: voff0/1[i % 4] + (i / 4) * 16 rows.
  const int roff0 = t128::row_chunk_off(kc, hh);
  const int toff0 = t128::tr32_off(0, lane), toff1 = t128::tr32_off(1, lane);
  int koff[8], voff0[4], voff1[4];
#pragma unroll
  for (int t = 0; t < 8; ++t) koff[t] = opaque(roff0 ^ (32 * t));
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    voff0[u] = opaque(toff0 ^ (64 * u));
    voff1[u] = opaque(toff1 ^ (64 * u));
  }
  const int64_t wq_first = a.q_pos0 + qw0;

  f32x16 o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = f32x16{};
  float mrun = -INFINITY;   // reference maximum of p (log2 units), shared by the lane pair
  float mtrue = -INFINITY;  // exact running maximum (log2 units)
  float lsum = 0.f;         // lane-partial sum of p relative to mrun

  auto kread = [&](const uint8_t* kt, int i) {  // S step i: t = i / 2, mb = i % 2
    return *reinterpret_cast<const bf16x8*>(kt + koff[i >> 1] + (i & 1) * 32 * t128::kRowBytes);
  };
  auto vread = [&](const uint8_t* vt, int i) {  // PV step i: u = i / 4, dblk = i % 4
    const int o0 = voff0[i & 3] + (i >> 2) * 16 * t128::kRowBytes;
    const int o1 = voff1[i & 3] + (i >> 2) * 16 * t128::kRowBytes;
    return concat_bf16x4(t128::ds_read_tr(vt + o0), t128::ds_read_tr(vt + o1));
  };

  // S^T of tile 0 (no softmax to overlap yet).
  auto scores_only = [&](const uint8_t* kt, f32x16 (&s)[2]) {
    bf16x8 A[2] = {kread(kt, 0), kread(kt, 1)};
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      s[i & 1] = mfma32x32x16(A[i & 1], qreg[i >> 1], i < 2 ? f32x16{} : s[i & 1]);
      if (i + 2 < 16) A[i & 1] = kread(kt, i + 2);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Iteration j: S^T(j+1) -> sn (HAS_NEXT) beside the softmax of sc = S^T(j),
  // then O^T += V_j^T P_j^T.  Mask (MASKED only): key idx + 4hh of the tile
  // and query kc are invalid when (causal && idx + 4hh - kc > cthr) ||
  // idx + 4hh >= kmax, idx = 32mb + 8w + r the compile-time part.
  auto iteration = [&](auto masked_tag, auto next_tag, const uint8_t* kt, const uint8_t* vt,
                       f32x16 (&sc)[2], f32x16 (&sn)[2], int cthr, int kmax) {
    constexpr bool MASKED = decltype(masked_tag)::value;
    constexpr bool HAS_NEXT = decltype(next_tag)::value;
    int kq = 0, klim = 0;
    if constexpr (MASKED) {
      kq = opaque(4 * hh - kc);
      klim = opaque(kmax - 4 * hh);
    }
    bf16x8 A[2], B[2], pb[4];
    if constexpr (HAS_NEXT) {
      A[0] = kread(kt, 0);
      A[1] = kread(kt, 1);
    }
    float pmax = -INFINITY, muse = 0.f;
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if constexpr (HAS_NEXT) {
        sn[i & 1] = mfma32x32x16(A[i & 1], qreg[i >> 1], i < 2 ? f32x16{} : sn[i & 1]);
        if (i + 2 < 16) A[i & 1] = kread(kt, i + 2);
      }
      if (i < 4) {  // mask and maximum, 8 scores per step
#pragma unroll
        for (int e = 8 * i; e < 8 * i + 8; ++e) {
          const int mb = e >> 4, v = e & 15;
          float x = sc[mb][v];
          if constexpr (MASKED) {
            const int idx = 32 * mb + 8 * (v >> 2) + (v & 3);
            const bool bad = (a.causal && kq > cthr - idx) || idx >= klim;
            x = bad ? -INFINITY : x;
            sc[mb][v] = x;
          }
          pmax = fmaxf(pmax, x);
        }
      }
      if (i == 7) {  // row maximum of the pair; rare rescale of the running state
        const float mx = xor32_max(pmax) * a.sl2;
        mtrue = fmaxf(mtrue, mx);
        const bool raise = mx > mrun + kRescaleSlack;
        if (__any(raise)) {
          const float mnew = raise ? mx : mrun;
          const float alpha = raise ? fast_exp2(mrun - mnew) : 1.f;  // mrun = -inf: 0
          mrun = mnew;
          lsum *= alpha;
#pragma unroll
          for (int d = 0; d < 4; ++d) o[d] *= alpha;
        }
        muse = (mrun == -INFINITY) ? 0.f : mrun;  // no key yet: p = 0
      }
      if (i >= 8) {  // p = exp2(s sl2 - muse), 4 scores per step
#pragma unroll
        for (int e = 4 * (i - 8); e < 4 * (i - 8) + 4; ++e) {
          const int mb = e >> 4, v = e & 15;
          const float pv = fast_exp2(fmaf(sc[mb][v], a.sl2, -muse));
          lsum += pv;
          sc[mb][v] = pv;
        }
      }
      if (i == 11 || i == 15) {  // P^T B operands of keys 32mb .. 32mb+31
        const int mb = (i - 11) >> 2;
#pragma unroll
        for (int u2 = 0; u2 < 2; ++u2) {
          const int e0 = 8 * u2;
          pb[2 * mb + u2] = pack_bf16x8(
              f32x4{sc[mb][e0], sc[mb][e0 + 2], sc[mb][e0 + 4], sc[mb][e0 + 6]},
              f32x4{sc[mb][e0 + 1], sc[mb][e0 + 3], sc[mb][e0 + 5], sc[mb][e0 + 7]});
        }
      }
      if (i == 14) B[0] = vread(vt, 0);
      if (i == 15) B[1] = vread(vt, 1);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      o[i & 3] = mfma32x32x16(B[i & 1], pb[i >> 2], o[i & 3]);
      if (i + 2 < 16) B[i & 1] = vread(vt, i + 2);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // One pipeline stage: barrier, loads for later tiles, iteration j.
  auto stage = [&](int j, f32x16 (&sc)[2], f32x16 (&sn)[2]) {
    t128::wait_vmem();
    __syncthreads();
    if (j + 2 < ntiles) ld.load(kbase, ks, (j + 2) * BN, a.Nk, t128::lds_addr(kbuf) + (j & 1) * kTileBytes, wave, lane);
    if (j + 1 < ntiles) ld.load(vbase, ks, (j + 1) * BN, a.Nk, t128::lds_addr(vbuf) + ((j + 1) & 1) * kTileBytes, wave, lane);
    if (j >= nt_w) return;
    const uint8_t* kt = kbuf[(j + 1) & 1];
    const uint8_t* vt = vbuf[j & 1];
    const int key0 = j * BN;
    const int64_t kp_first = a.k_pos0 + key0;
    const int64_t kp_last = kp_first + BN - 1;
    const bool next = j + 1 < nt_w;
    if ((a.causal && kp_last > wq_first) || kp_last >= a.valid || key0 + BN > a.Nk) {
      const int64_t ct = wq_first - kp_first;
      const int cthr = (int)(ct < -4096 ? -4096 : (ct > 4096 ? 4096 : ct));
      const int64_t km = min((int64_t)(a.Nk - key0), a.valid - kp_first);
      const int kmax = (int)(km < 0 ? 0 : (km > BN ? BN : km));
      if (next)
        iteration(std::true_type{}, std::true_type{}, kt, vt, sc, sn, cthr, kmax);
      else
        iteration(std::true_type{}, std::false_type{}, kt, vt, sc, sn, cthr, kmax);
    } else {
      if (next)
        iteration(std::false_type{}, std::true_type{}, kt, vt, sc, sn, 0, BN);
      else
        iteration(std::false_type{}, std::false_type{}, kt, vt, sc, sn, 0, BN);
    }
  };

  f32x16 sa[2], sb[2];
  t128::wait_vmem();
  __syncthreads();
  if (nt_w > 0) scores_only(kbuf[0], sa);
  for (int j = 0; j < ntiles; j += 2) {
    stage(j, sa, sb);
    if (j + 1 < ntiles) stage(j + 1, sb, sa);
  }

  // Epilogue: o = acc / l; m in natural-log units; l as the reference defines it.
  // accumulate: LSE-merge (o, m, l) into the running state of the row.
  const float lt = xor32_sum(lsum);  // relative to mrun
  const int row = qw0 + kc;
  if (row < a.Nq) {
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    const float ltrue = lt > 0.f ? lt * fast_exp2(mrun - mtrue) : 0.f;
    const float mnat = (mtrue == -INFINITY) ? -INFINITY : mtrue * kLn2;
    float* orow = a.o + (((int64_t)b * a.Nq + row) * a.Hq + hq) * D;
    const int64_t si = ((int64_t)b * a.Hq + hq) * a.Nq + row;
    float wa = 0.f, wb = inv, mo = mnat, lo = ltrue;
    if (a.accumulate) {
      const MergeW w = merge_weights(a.m[si], a.l[si], mnat, ltrue);
      wa = w.wa;
      wb = w.wb * inv;
      mo = w.m;
      lo = w.l;
    }
#pragma unroll
    for (int d = 0; d < 4; ++d)
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        f32x4* dst = reinterpret_cast<f32x4*>(orow + 32 * d + 8 * w + 4 * hh);
        const f32x4 v4 = {o[d][4 * w], o[d][4 * w + 1], o[d][4 * w + 2], o[d][4 * w + 3]};
        *dst = a.accumulate ? *dst * wa + v4 * wb : v4 * wb;
      }
    if (hh == 0) {
      a.m[si] = mo;
      a.l[si] = lo;
    }
  }
}

}  // namespace

hipError_t launch_fwd128(const Problem& p, const void* q, const void* k, const void* v, float* o,
                         float* m, float* l, hipStream_t s, int64_t kv_rows, bool accumulate) {
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
  // No causal diagonal in this launch: every key precedes every query.
  const bool full = !p.causal || p.k_pos0 + p.Nk - 1 <= p.q_pos0;
  const int bm = (full ? 8 : 4) * kQW;
  a.n_qtiles = (p.Nq + bm - 1) / bm;
  a.q_pos0 = p.q_pos0;
  a.k_pos0 = p.k_pos0;
  a.valid = p.valid;
  a.kv_bstride = (kv_rows < 0 ? p.Nk : kv_rows) * (int64_t)p.Hkv * D;
  a.causal = p.causal ? 1 : 0;
  a.accumulate = accumulate ? 1 : 0;
  a.sl2 = p.scale * kLog2e;
  if (full)
    hipLaunchKernelGGL(fwd128_kernel<8>, dim3(a.n_qtiles * p.Hq * p.B), dim3(512), 0, s, a);
  else
    hipLaunchKernelGGL(fwd128_kernel<4>, dim3(a.n_qtiles * p.Hq * p.B), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace lc
