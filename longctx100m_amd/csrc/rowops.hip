// Row-wise, HBM-bound kernels of the ring: log-sum-exp merge of a hop's
// partial into the running state, state init, the backward preprocess
// (delta and log2-domain LSE), casts and fills.
//
// Row r of a [B, N, H, D] tensor is ((b * N) + t) * H + h; its statistics
// live at (b * H + h) * N + t of the [B, H, N] arrays.
#include "common.h"
#include "kernels.h"

namespace lc {
namespace {

__device__ __forceinline__ int64_t stat_index(int64_t row, int N, int H) {
  const int64_t h = row % H;
  const int64_t bt = row / H;
  const int64_t t = bt % N;
  const int64_t b = bt / N;
  return (b * H + h) * N + t;
}

// Pass 1 of the merge: output rows.  One thread per 4 consecutive elements
// when D % 4 == 0 (else per element); statistics are only read here.
template <int VEC>
__global__ void merge_rows_kernel(int64_t rows, int N, int H, int D, float* o_run,
                                  const float* m_run, const float* l_run, const float* o_part,
                                  const float* m_part, const float* l_part, void* out,
                                  int out_dtype) {
  const int per_row = D / VEC;
  const int64_t total = rows * per_row;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = idx / per_row;
    const int col = (int)(idx - row * per_row) * VEC;
    const int64_t si = stat_index(row, N, H);
    const MergeW w = merge_weights(m_run[si], l_run[si], m_part[si], l_part[si]);
    const int64_t e = row * D + col;
    float vals[VEC];
    if constexpr (VEC == 4) {
      const f32x4 a = *reinterpret_cast<const f32x4*>(o_run + e);
      const f32x4 b = *reinterpret_cast<const f32x4*>(o_part + e);
      const f32x4 r = a * w.wa + b * w.wb;
      *reinterpret_cast<f32x4*>(o_run + e) = r;
      vals[0] = r[0];
      vals[1] = r[1];
      vals[2] = r[2];
      vals[3] = r[3];
    } else {
      vals[0] = o_run[e] * w.wa + o_part[e] * w.wb;
      o_run[e] = vals[0];
    }
    if (out != nullptr) {
      if (out_dtype == 1) {
        uint16_t* dst = static_cast<uint16_t*>(out) + e;
#pragma unroll
        for (int i = 0; i < VEC; ++i) dst[i] = f32_to_bf16(vals[i]);
      } else {
        float* dst = static_cast<float*>(out) + e;
#pragma unroll
        for (int i = 0; i < VEC; ++i) dst[i] = vals[i];
      }
    }
  }
}

// Pass 2 of the merge: statistics, after every output row has read them.
__global__ void merge_stats_kernel(int64_t n, float* m_run, float* l_run, const float* m_part,
                                   const float* l_part) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const MergeW w = merge_weights(m_run[i], l_run[i], m_part[i], l_part[i]);
    m_run[i] = w.m;
    l_run[i] = w.l;
  }
}

__global__ void init_state_kernel(int64_t n_o, int64_t n_s, float* o, float* m, float* l) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_o;
       i += (int64_t)gridDim.x * blockDim.x) {
    o[i] = 0.f;
    if (i < n_s) {
      m[i] = -INFINITY;
      l[i] = 0.f;
    }
  }
}

__global__ void fill_zero_kernel(int64_t n, float* dst) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    dst[i] = 0.f;
}

template <typename T>
__global__ void cast_kernel(int64_t n, const float* src, T* dst) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    store_from_f32(dst + i, src[i]);
}

// fp32 -> bf16, eight elements per lane: two 16-byte loads, one 16-byte store
// (n8 = n / 8; both pointers 16-byte aligned).  Same rounding as cast_kernel.
__global__ void cast_bf16x8_kernel(int64_t n8, const f32x4* src, uint4* dst) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n8;
       i += (int64_t)gridDim.x * blockDim.x) {
    const f32x4 a = src[2 * i], b = src[2 * i + 1];
    uint4 r;
    r.x = (uint32_t)f32_to_bf16(a[0]) | ((uint32_t)f32_to_bf16(a[1]) << 16);
    r.y = (uint32_t)f32_to_bf16(a[2]) | ((uint32_t)f32_to_bf16(a[3]) << 16);
    r.z = (uint32_t)f32_to_bf16(b[0]) | ((uint32_t)f32_to_bf16(b[1]) << 16);
    r.w = (uint32_t)f32_to_bf16(b[2]) | ((uint32_t)f32_to_bf16(b[3]) << 16);
    dst[i] = r;
  }
}

// delta = rowsum(dout * out) over D (both in the input dtype, upcast to fp32),
// lse2 = m*log2(e) + log2(max(l, FLT_MIN)), +inf where m = -inf so that
// 2^(s*log2e - lse2) = 0 for rows that saw no key.  A group of 16 lanes owns
// a row at a time.  Workgroups walk the [B, N, H, D] rows in memory order
// (kPreRows consecutive rows each, group g rows g, g + kPreGroups, ...), so the
// reads stream whole DRAM pages; the 4-byte statistics writes land on
// [B, H, N] lines that the neighbouring workgroups complete in L2.  Small
// workgroups (128 threads, one row per lane group) measured 7-11% faster than
// 256 threads with four rows per group, with caches cold or warm.  VEC:
// elements per 16-byte load (row bytes a multiple of 16, pointers aligned), or
// 1 for the scalar path.
constexpr int kPreThreads = 128;
constexpr int kPreGroups = kPreThreads / 16;
constexpr int kPreRows = 8;

template <typename T, int VEC>
__global__ __launch_bounds__(kPreThreads) void bwd_preprocess_kernel(int64_t rows, int N, int H,
                                                                     int D, const T* out,
                                                                     const T* dout, const float* m,
                                                                     const float* l, float* delta,
                                                                     float* lse2) {
  constexpr int kPer = kPreRows / kPreGroups;  // rows per lane group
  static_assert(kPer * kPreGroups == kPreRows, "rows split evenly over the lane groups");
  const int sub = threadIdx.x & 15;
  const int g = threadIdx.x >> 4;
  const int64_t r0 = (int64_t)blockIdx.x * kPreRows + g;
  float acc[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) acc[i] = 0.f;
  if constexpr (VEC == 1) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int64_t row = min(r0 + kPreGroups * i, rows - 1);
      for (int d = sub; d < D; d += 16) acc[i] += load_f32(out + row * D + d) * load_f32(dout + row * D + d);
    }
  } else {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    const int nc = D / VEC;  // 16-byte chunks per row
    for (int c = sub; c < nc; c += 16) {
      u32x4 ov[kPer], gv[kPer];
#pragma unroll
      for (int i = 0; i < kPer; ++i) {  // every load of the pass issued before use; read once
        const int64_t off = min(r0 + kPreGroups * i, rows - 1) * D + (int64_t)c * VEC;
        ov[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(out + off));
        gv[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(dout + off));
      }
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const T* oe = reinterpret_cast<const T*>(&ov[i]);
        const T* ge = reinterpret_cast<const T*>(&gv[i]);
#pragma unroll
        for (int j = 0; j < VEC; ++j) acc[i] += load_f32(oe + j) * load_f32(ge + j);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) acc[i] += __shfl_xor(acc[i], off, 64);
    const int64_t row = r0 + kPreGroups * i;
    if (sub == 0 && row < rows) {
      const int64_t si = stat_index(row, N, H);
      const float mi = m[si];
      const float li = l[si];
      delta[si] = acc[i];
      lse2[si] = (mi == -INFINITY) ? INFINITY : mi * kLog2e + log2f(li > kFltMin ? li : kFltMin);
    }
  }
}

inline dim3 grid_for(int64_t n, int threads = 256) {
  int64_t blocks = (n + threads - 1) / threads;
  if (blocks > 65536) blocks = 65536;
  if (blocks < 1) blocks = 1;
  return dim3((unsigned)blocks);
}

}  // namespace

hipError_t launch_merge(int B, int N, int H, int D, float* o_run, float* m_run, float* l_run,
                        const float* o_part, const float* m_part, const float* l_part, void* out,
                        int out_dtype, hipStream_t s) {
  const int64_t rows = (int64_t)B * N * H;
  if (D % 4 == 0) {
    hipLaunchKernelGGL(merge_rows_kernel<4>, grid_for(rows * (D / 4)), dim3(256), 0, s, rows, N,
                       H, D, o_run, m_run, l_run, o_part, m_part, l_part, out, out_dtype);
  } else {
    hipLaunchKernelGGL(merge_rows_kernel<1>, grid_for(rows * D), dim3(256), 0, s, rows, N, H, D,
                       o_run, m_run, l_run, o_part, m_part, l_part, out, out_dtype);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(merge_stats_kernel, grid_for(rows), dim3(256), 0, s, rows, m_run, l_run,
                     m_part, l_part);
  return hipGetLastError();
}

hipError_t launch_init_state(int B, int N, int H, int D, float* o, float* m, float* l,
                             hipStream_t s) {
  const int64_t n_s = (int64_t)B * N * H;
  const int64_t n_o = n_s * D;
  hipLaunchKernelGGL(init_state_kernel, grid_for(n_o), dim3(256), 0, s, n_o, n_s, o, m, l);
  return hipGetLastError();
}

hipError_t launch_cast(const float* src, void* dst, int64_t n, int dtype, hipStream_t s) {
  const bool vec = n % 8 == 0 && (reinterpret_cast<uintptr_t>(src) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(dst) & 15) == 0;
  if (dtype == 1 && vec)
    hipLaunchKernelGGL(cast_bf16x8_kernel, grid_for(n / 8), dim3(256), 0, s, n / 8,
                       reinterpret_cast<const f32x4*>(src), static_cast<uint4*>(dst));
  else if (dtype == 1)
    hipLaunchKernelGGL(cast_kernel<uint16_t>, grid_for(n), dim3(256), 0, s, n, src,
                       static_cast<uint16_t*>(dst));
  else
    hipLaunchKernelGGL(cast_kernel<float>, grid_for(n), dim3(256), 0, s, n, src,
                       static_cast<float*>(dst));
  return hipGetLastError();
}

hipError_t launch_fill_zero(float* dst, int64_t n, hipStream_t s) {
  hipLaunchKernelGGL(fill_zero_kernel, grid_for(n), dim3(256), 0, s, n, dst);
  return hipGetLastError();
}

hipError_t launch_bwd_preprocess(int B, int N, int H, int D, int dtype, const void* out,
                                 const void* dout, const float* m, const float* l, float* delta,
                                 float* lse2, hipStream_t s) {
  const int64_t rows = (int64_t)B * N * H;
  if (rows == 0) return hipSuccess;
  const int64_t blocks = (rows + kPreRows - 1) / kPreRows;
  if (blocks * kPreThreads > 0xffffffffLL) return hipErrorInvalidValue;  // 32-bit grid size
  const dim3 grid((unsigned)blocks), block(kPreThreads);
  const bool vec = ((reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(dout)) & 15) == 0;
  if (dtype == 1) {
    const uint16_t* o = static_cast<const uint16_t*>(out);
    const uint16_t* g = static_cast<const uint16_t*>(dout);
    if (vec && D % 8 == 0)
      hipLaunchKernelGGL((bwd_preprocess_kernel<uint16_t, 8>), grid, block, 0, s, rows, N, H, D, o,
                         g, m, l, delta, lse2);
    else
      hipLaunchKernelGGL((bwd_preprocess_kernel<uint16_t, 1>), grid, block, 0, s, rows, N, H, D, o,
                         g, m, l, delta, lse2);
  } else {
    const float* o = static_cast<const float*>(out);
    const float* g = static_cast<const float*>(dout);
    if (vec && D % 4 == 0)
      hipLaunchKernelGGL((bwd_preprocess_kernel<float, 4>), grid, block, 0, s, rows, N, H, D, o, g,
                         m, l, delta, lse2);
    else
      hipLaunchKernelGGL((bwd_preprocess_kernel<float, 1>), grid, block, 0, s, rows, N, H, D, o, g,
                         m, l, delta, lse2);
  }
  return hipGetLastError();
}

}  // namespace lc
