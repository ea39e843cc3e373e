// fp32-math attention kernels for any head_dim <= 256 and fp32 or bf16
// inputs.  They carry the reference's exact arithmetic (fp32 scores, fp32
// probabilities, fp32 accumulation; bf16 inputs are upcast on load, the
// Python twin's rule at src/longctx100m/ring_attention.py:17,28) and serve the
// fp32 path, LC_FLAG_PRECISE, and head dims the MFMA kernels do not take.
//
// Mapping: four adjacent lanes own one query (forward, dQ) or one key (dK/dV);
// lane `sub` holds head dims sub, sub+4, sub+8, ...; dot products are reduced
// with two xor-shuffles.  The streamed operand is staged in LDS as fp32,
// 32 rows per tile.
//   forward: online softmax exactly as online_update
//            (rust/longctx100m-model/src/ring_attention.rs:15-55), one
//            32-key block at a time.
//   dQ     : rs:433-454 (pass 2 of the reference backward).
//   dK/dV  : rs:383-409 (pass 1), summed over the GQA group in registers.
#include "common.h"
#include "kernels.h"

namespace lc {
namespace {

constexpr int kRows = 64;  // queries (or keys) per workgroup, 4 lanes each
constexpr int kTile = 32;  // streamed rows per LDS tile

struct GenArgs {
  const void* q;
  const void* k;
  const void* v;
  const void* dout;
  const float* lse2;
  const float* delta;
  float* o;
  float* m;
  float* l;
  float* dq;
  float* dk;
  float* dv;
  int B, Nq, Nk, Hq, Hkv, D, group, n_tiles;
  int64_t q_pos0, k_pos0, valid;
  int causal;
  int accumulate;  // forward: merge into the running (o, m, l) instead of writing them
  float scale;
};

__device__ __forceinline__ bool masked(const GenArgs& a, int key, int64_t kp, int64_t qp) {
  return key >= a.Nk || (a.causal && kp > qp) || kp >= a.valid;
}

__device__ __forceinline__ float reduce4(float x) {
  x += __shfl_xor(x, 1, 64);
  x += __shfl_xor(x, 2, 64);
  return x;
}

template <typename T>
__device__ __forceinline__ void stage_rows(float* dst, const T* base, int64_t stride, int row0,
                                           int nrows, int D, int tid) {
  for (int idx = tid; idx < kTile * D; idx += 256) {
    const int r = idx / D;
    const int d = idx - r * D;
    const int row = row0 + r;
    dst[idx] = row < nrows ? load_f32(base + (int64_t)row * stride + d) : 0.f;
  }
}

template <typename T, int DPL>
__global__ __launch_bounds__(256) void fwd_generic_kernel(GenArgs a) {
  extern __shared__ float smem[];
  float* ksm = smem;
  float* vsm = smem + kTile * a.D;
  const int tid = threadIdx.x;
  const int r = tid >> 2;
  const int sub = tid & 3;
  const int qt = blockIdx.x % a.n_tiles;
  const int bh = blockIdx.x / a.n_tiles;
  const int h = bh % a.Hq;
  const int b = bh / a.Hq;
  const int hk = h / a.group;
  const int D = a.D;
  const int row = qt * kRows + r;
  const bool ok = row < a.Nq;

  const int64_t qs = (int64_t)a.Hq * D, ks = (int64_t)a.Hkv * D;
  const T* qb = static_cast<const T*>(a.q) + (int64_t)b * a.Nq * qs + (int64_t)h * D;
  const T* kb = static_cast<const T*>(a.k) + (int64_t)b * a.Nk * ks + (int64_t)hk * D;
  const T* vb = static_cast<const T*>(a.v) + (int64_t)b * a.Nk * ks + (int64_t)hk * D;

  float qv[DPL], acc[DPL];
#pragma unroll
  for (int j = 0; j < DPL; ++j) {
    const int d = sub + 4 * j;
    qv[j] = (ok && d < D) ? load_f32(qb + (int64_t)row * qs + d) : 0.f;
    acc[j] = 0.f;
  }
  float m = -INFINITY, l = 0.f;
  const int64_t qp = a.q_pos0 + row;

  const int q_end = min(qt * kRows + kRows, a.Nq);
  int64_t kend = a.Nk;
  if (a.causal) kend = min(kend, a.q_pos0 + q_end - a.k_pos0);
  kend = min(kend, a.valid - a.k_pos0);
  const int ntiles = kend > 0 ? (int)((kend + kTile - 1) / kTile) : 0;

  for (int t = 0; t < ntiles; ++t) {
    __syncthreads();
    stage_rows(ksm, kb, ks, t * kTile, a.Nk, D, tid);
    stage_rows(vsm, vb, ks, t * kTile, a.Nk, D, tid);
    __syncthreads();
    float sc[kTile];
    float bm = -INFINITY;
#pragma unroll
    for (int j = 0; j < kTile; ++j) {
      float part = 0.f;
#pragma unroll
      for (int jj = 0; jj < DPL; ++jj) {
        const int d = sub + 4 * jj;
        if (d < D) part += qv[jj] * ksm[j * D + d];
      }
      part = reduce4(part);
      float s = part * a.scale;
      const int key = t * kTile + j;
      if (masked(a, key, a.k_pos0 + key, qp)) s = -INFINITY;
      sc[j] = s;
      bm = fmaxf(bm, s);
    }
    const float mnew = fmaxf(m, bm);
    const bool all_masked = (mnew == -INFINITY);
    const float alpha = all_masked ? 0.f : expf(m - mnew);
#pragma unroll
    for (int jj = 0; jj < DPL; ++jj) acc[jj] *= alpha;
    float psum = 0.f;
#pragma unroll
    for (int j = 0; j < kTile; ++j) {
      const float p = all_masked ? 0.f : expf(sc[j] - mnew);
      psum += p;
#pragma unroll
      for (int jj = 0; jj < DPL; ++jj) {
        const int d = sub + 4 * jj;
        if (d < D) acc[jj] += p * vsm[j * D + d];
      }
    }
    l = alpha * l + psum;
    m = mnew;
  }

  // accumulate: LSE-merge (o, m, l) into the running state of the row, with
  // the arithmetic of lc_attn_merge on the normalised partial.
  if (ok) {
    const float den = l > kFltMin ? l : kFltMin;
    float* orow = a.o + (((int64_t)b * a.Nq + row) * a.Hq + h) * D;
    const int64_t si = ((int64_t)b * a.Hq + h) * a.Nq + row;
    MergeW w{};
    if (a.accumulate) w = merge_weights(a.m[si], a.l[si], m, l);
#pragma unroll
    for (int jj = 0; jj < DPL; ++jj) {
      const int d = sub + 4 * jj;
      if (d < D) orow[d] = a.accumulate ? orow[d] * w.wa + (acc[jj] / den) * w.wb : acc[jj] / den;
    }
    if (sub == 0) {
      a.m[si] = a.accumulate ? w.m : m;
      a.l[si] = a.accumulate ? w.l : l;
    }
  }
}

template <typename T, int DPL>
__global__ __launch_bounds__(256) void dq_generic_kernel(GenArgs a) {
  extern __shared__ float smem[];
  float* ksm = smem;
  float* vsm = smem + kTile * a.D;
  const int tid = threadIdx.x;
  const int r = tid >> 2;
  const int sub = tid & 3;
  const int qt = blockIdx.x % a.n_tiles;
  const int bh = blockIdx.x / a.n_tiles;
  const int h = bh % a.Hq;
  const int b = bh / a.Hq;
  const int hk = h / a.group;
  const int D = a.D;
  const int row = qt * kRows + r;
  const bool ok = row < a.Nq;
  const float sl2 = a.scale * kLog2e;

  const int64_t qs = (int64_t)a.Hq * D, ks = (int64_t)a.Hkv * D;
  const T* qb = static_cast<const T*>(a.q) + (int64_t)b * a.Nq * qs + (int64_t)h * D;
  const T* ob = static_cast<const T*>(a.dout) + (int64_t)b * a.Nq * qs + (int64_t)h * D;
  const T* kb = static_cast<const T*>(a.k) + (int64_t)b * a.Nk * ks + (int64_t)hk * D;
  const T* vb = static_cast<const T*>(a.v) + (int64_t)b * a.Nk * ks + (int64_t)hk * D;

  float qv[DPL], dov[DPL], acc[DPL];
#pragma unroll
  for (int j = 0; j < DPL; ++j) {
    const int d = sub + 4 * j;
    const bool in = ok && d < D;
    qv[j] = in ? load_f32(qb + (int64_t)row * qs + d) : 0.f;
    dov[j] = in ? load_f32(ob + (int64_t)row * qs + d) : 0.f;
    acc[j] = 0.f;
  }
  const int64_t si = ((int64_t)b * a.Hq + h) * a.Nq + row;
  const float lse = ok ? a.lse2[si] : INFINITY;
  const float dl = ok ? a.delta[si] : 0.f;
  const int64_t qp = a.q_pos0 + row;

  const int q_end = min(qt * kRows + kRows, a.Nq);
  int64_t kend = a.Nk;
  if (a.causal) kend = min(kend, a.q_pos0 + q_end - a.k_pos0);
  kend = min(kend, a.valid - a.k_pos0);
  const int ntiles = kend > 0 ? (int)((kend + kTile - 1) / kTile) : 0;

  for (int t = 0; t < ntiles; ++t) {
    __syncthreads();
    stage_rows(ksm, kb, ks, t * kTile, a.Nk, D, tid);
    stage_rows(vsm, vb, ks, t * kTile, a.Nk, D, tid);
    __syncthreads();
#pragma unroll 4
    for (int j = 0; j < kTile; ++j) {
      float ps = 0.f, pd = 0.f;
#pragma unroll
      for (int jj = 0; jj < DPL; ++jj) {
        const int d = sub + 4 * jj;
        if (d < D) {
          ps += qv[jj] * ksm[j * D + d];
          pd += dov[jj] * vsm[j * D + d];
        }
      }
      ps = reduce4(ps);
      pd = reduce4(pd);
      const int key = t * kTile + j;
      float p = 0.f;
      if (!masked(a, key, a.k_pos0 + key, qp)) p = fast_exp2(ps * sl2 - lse);
      const float ds = p * (pd - dl);
#pragma unroll
      for (int jj = 0; jj < DPL; ++jj) {
        const int d = sub + 4 * jj;
        if (d < D) acc[jj] += ds * ksm[j * D + d];
      }
    }
  }

  if (ok && ntiles > 0) {
    float* dst = a.dq + (((int64_t)b * a.Nq + row) * a.Hq + h) * D;
#pragma unroll
    for (int jj = 0; jj < DPL; ++jj) {
      const int d = sub + 4 * jj;
      if (d < D) dst[d] += acc[jj] * a.scale;
    }
  }
}

template <typename T, int DPL>
__global__ __launch_bounds__(256) void dkdv_generic_kernel(GenArgs a) {
  extern __shared__ float smem[];
  float* qsm = smem;
  float* osm = smem + kTile * a.D;
  float* lsm = smem + 2 * kTile * a.D;
  float* dsm = lsm + kTile;
  const int tid = threadIdx.x;
  const int r = tid >> 2;
  const int sub = tid & 3;
  const int kt = blockIdx.x % a.n_tiles;
  const int bh = blockIdx.x / a.n_tiles;
  const int hk = bh % a.Hkv;
  const int b = bh / a.Hkv;
  const int D = a.D;
  const int key = kt * kRows + r;
  const bool ok = key < a.Nk;
  const float sl2 = a.scale * kLog2e;

  const int64_t qs = (int64_t)a.Hq * D, ks = (int64_t)a.Hkv * D;
  const T* kb = static_cast<const T*>(a.k) + (int64_t)b * a.Nk * ks + (int64_t)hk * D;
  const T* vb = static_cast<const T*>(a.v) + (int64_t)b * a.Nk * ks + (int64_t)hk * D;

  float kv[DPL], vv[DPL], dka[DPL], dva[DPL];
#pragma unroll
  for (int j = 0; j < DPL; ++j) {
    const int d = sub + 4 * j;
    const bool in = ok && d < D;
    kv[j] = in ? load_f32(kb + (int64_t)key * ks + d) : 0.f;
    vv[j] = in ? load_f32(vb + (int64_t)key * ks + d) : 0.f;
    dka[j] = dva[j] = 0.f;
  }
  const int64_t kp = a.k_pos0 + key;

  const int64_t kp_first = a.k_pos0 + (int64_t)kt * kRows;
  int qstart = 0;
  if (a.causal) {
    const int64_t first = kp_first - a.q_pos0;
    qstart = first <= 0 ? 0 : (first >= a.Nq ? a.Nq : (int)first);
  }
  qstart = (qstart / kTile) * kTile;
  const bool any_valid = kp_first < a.valid && kt * kRows < a.Nk;
  const int ntq = any_valid ? (a.Nq - qstart + kTile - 1) / kTile : 0;

  for (int hh = 0; hh < a.group; ++hh) {
    const int hq = hk * a.group + hh;
    const T* qb = static_cast<const T*>(a.q) + (int64_t)b * a.Nq * qs + (int64_t)hq * D;
    const T* ob = static_cast<const T*>(a.dout) + (int64_t)b * a.Nq * qs + (int64_t)hq * D;
    for (int t = 0; t < ntq; ++t) {
      const int qrow0 = qstart + t * kTile;
      __syncthreads();
      stage_rows(qsm, qb, qs, qrow0, a.Nq, D, tid);
      stage_rows(osm, ob, qs, qrow0, a.Nq, D, tid);
      if (tid < kTile) {
        const int row = qrow0 + tid;
        const int64_t si = ((int64_t)b * a.Hq + hq) * a.Nq + row;
        lsm[tid] = row < a.Nq ? a.lse2[si] : INFINITY;
        dsm[tid] = row < a.Nq ? a.delta[si] : 0.f;
      }
      __syncthreads();
#pragma unroll 4
      for (int i = 0; i < kTile; ++i) {
        float ps = 0.f, pd = 0.f;
#pragma unroll
        for (int jj = 0; jj < DPL; ++jj) {
          const int d = sub + 4 * jj;
          if (d < D) {
            ps += kv[jj] * qsm[i * D + d];
            pd += vv[jj] * osm[i * D + d];
          }
        }
        ps = reduce4(ps);
        pd = reduce4(pd);
        const int64_t qp = a.q_pos0 + qrow0 + i;
        float p = 0.f;
        if (!masked(a, key, kp, qp)) p = fast_exp2(ps * sl2 - lsm[i]);
        const float ds = p * (pd - dsm[i]);
#pragma unroll
        for (int jj = 0; jj < DPL; ++jj) {
          const int d = sub + 4 * jj;
          if (d < D) {
            dka[jj] += ds * qsm[i * D + d];
            dva[jj] += p * osm[i * D + d];
          }
        }
      }
    }
  }

  if (ok && ntq > 0) {
    const int64_t off = (((int64_t)b * a.Nk + key) * a.Hkv + hk) * D;
#pragma unroll
    for (int jj = 0; jj < DPL; ++jj) {
      const int d = sub + 4 * jj;
      if (d < D) {
        a.dk[off + d] += dka[jj] * a.scale;
        a.dv[off + d] += dva[jj];
      }
    }
  }
}

GenArgs make_args(const Problem& p) {
  GenArgs a{};
  a.B = p.B;
  a.Nq = p.Nq;
  a.Nk = p.Nk;
  a.Hq = p.Hq;
  a.Hkv = p.Hkv;
  a.D = p.D;
  a.group = p.Hq / p.Hkv;
  a.q_pos0 = p.q_pos0;
  a.k_pos0 = p.k_pos0;
  a.valid = p.valid;
  a.causal = p.causal ? 1 : 0;
  a.accumulate = p.accumulate ? 1 : 0;
  a.scale = p.scale;
  return a;
}

// Chooses <input type, dims per lane> for a kernel family.
#define LC_GENERIC_DISPATCH(KERNEL, A, P, SMEM, GRID, STREAM)                               \
  do {                                                                                      \
    const bool bf = (P).dtype == 1;                                                         \
    const int d = (P).D;                                                                    \
    if (d <= 8) {                                                                           \
      if (bf) hipLaunchKernelGGL((KERNEL<uint16_t, 2>), GRID, dim3(256), SMEM, STREAM, A);  \
      else hipLaunchKernelGGL((KERNEL<float, 2>), GRID, dim3(256), SMEM, STREAM, A);        \
    } else if (d <= 32) {                                                                   \
      if (bf) hipLaunchKernelGGL((KERNEL<uint16_t, 8>), GRID, dim3(256), SMEM, STREAM, A);  \
      else hipLaunchKernelGGL((KERNEL<float, 8>), GRID, dim3(256), SMEM, STREAM, A);        \
    } else if (d <= 64) {                                                                   \
      if (bf) hipLaunchKernelGGL((KERNEL<uint16_t, 16>), GRID, dim3(256), SMEM, STREAM, A); \
      else hipLaunchKernelGGL((KERNEL<float, 16>), GRID, dim3(256), SMEM, STREAM, A);       \
    } else if (d <= 128) {                                                                  \
      if (bf) hipLaunchKernelGGL((KERNEL<uint16_t, 32>), GRID, dim3(256), SMEM, STREAM, A); \
      else hipLaunchKernelGGL((KERNEL<float, 32>), GRID, dim3(256), SMEM, STREAM, A);       \
    } else {                                                                                \
      if (bf) hipLaunchKernelGGL((KERNEL<uint16_t, 64>), GRID, dim3(256), SMEM, STREAM, A); \
      else hipLaunchKernelGGL((KERNEL<float, 64>), GRID, dim3(256), SMEM, STREAM, A);       \
    }                                                                                       \
  } while (0)

}  // namespace

hipError_t launch_fwd_generic(const Problem& p, const void* q, const void* k, const void* v,
                              float* o, float* m, float* l, hipStream_t s) {
  if (p.D > 256) return hipErrorInvalidValue;
  GenArgs a = make_args(p);
  a.q = q;
  a.k = k;
  a.v = v;
  a.o = o;
  a.m = m;
  a.l = l;
  a.n_tiles = (p.Nq + kRows - 1) / kRows;
  const size_t smem = sizeof(float) * 2 * kTile * p.D;
  const dim3 grid(a.n_tiles * p.Hq * p.B);
  LC_GENERIC_DISPATCH(fwd_generic_kernel, a, p, smem, grid, s);
  return hipGetLastError();
}

hipError_t launch_bwd_dq_generic(const Problem& p, const void* q, const void* k, const void* v,
                                 const void* dout, const float* lse2, const float* delta,
                                 float* dq, hipStream_t s) {
  if (p.D > 256) return hipErrorInvalidValue;
  GenArgs a = make_args(p);
  a.q = q;
  a.k = k;
  a.v = v;
  a.dout = dout;
  a.lse2 = lse2;
  a.delta = delta;
  a.dq = dq;
  a.n_tiles = (p.Nq + kRows - 1) / kRows;
  const size_t smem = sizeof(float) * 2 * kTile * p.D;
  const dim3 grid(a.n_tiles * p.Hq * p.B);
  LC_GENERIC_DISPATCH(dq_generic_kernel, a, p, smem, grid, s);
  return hipGetLastError();
}

hipError_t launch_bwd_dkdv_generic(const Problem& p, const void* q, const void* k, const void* v,
                                   const void* dout, const float* lse2, const float* delta,
                                   float* dk, float* dv, hipStream_t s) {
  if (p.D > 256) return hipErrorInvalidValue;
  GenArgs a = make_args(p);
  a.q = q;
  a.k = k;
  a.v = v;
  a.dout = dout;
  a.lse2 = lse2;
  a.delta = delta;
  a.dk = dk;
  a.dv = dv;
  a.n_tiles = (p.Nk + kRows - 1) / kRows;
  const size_t smem = sizeof(float) * (2 * kTile * p.D + 2 * kTile);
  const dim3 grid(a.n_tiles * p.Hkv * p.B);
  LC_GENERIC_DISPATCH(dkdv_generic_kernel, a, p, smem, grid, s);
  return hipGetLastError();
}

}  // namespace lc
