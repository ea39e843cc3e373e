// Matrix-vector product of a bf16 row-major weight with one bf16 token, for
// the decode step's projections (candle Linear without bias at M = 1:
// rust/longctx100m-model/src/model.rs:64-76 and the LM head :670-674).
//   y[n] = bf16( sum_k W[n][k] x[k] ),  fp32 accumulation
// Bound by the weight read (2 bytes per weight, read once).  A workgroup
// owns kRows rows and splits their length over its kSplit waves (enough waves
// in flight for the 4096-row projections too); each lane strides its part in
// 16-byte chunks, kUnroll chunks per row per round, so kRows x kUnroll loads
// of 16 bytes are in flight per lane.  A butterfly over each wave and an LDS
// sum over the waves give the row totals.
#include "common.h"
#include "kernels.h"

namespace lc {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kRows = 4;
constexpr int kUnroll = 4;
constexpr int kSplit = 4;  // waves per workgroup, each over 1/kSplit of the row

__device__ __forceinline__ float bf16_lo(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }

__device__ __forceinline__ float dot8(const uint4& w, const uint4& x, float acc) {
  acc = fmaf(bf16_lo(w.x), bf16_lo(x.x), acc);
  acc = fmaf(bf16_hi(w.x), bf16_hi(x.x), acc);
  acc = fmaf(bf16_lo(w.y), bf16_lo(x.y), acc);
  acc = fmaf(bf16_hi(w.y), bf16_hi(x.y), acc);
  acc = fmaf(bf16_lo(w.z), bf16_lo(x.z), acc);
  acc = fmaf(bf16_hi(w.z), bf16_hi(x.z), acc);
  acc = fmaf(bf16_lo(w.w), bf16_lo(x.w), acc);
  acc = fmaf(bf16_hi(w.w), bf16_hi(x.w), acc);
  return acc;
}

__global__ __launch_bounds__(64 * kSplit) void gemv_bf16_kernel(int64_t n, int k,
                                                                 const uint16_t* w, int64_t ws,
                                                                 const uint16_t* x, uint16_t* y) {
  __shared__ float part[kSplit][kRows];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t row0 = (int64_t)blockIdx.x * kRows;
  const int nch = k / 8;  // 16-byte chunks per row
  const int per = (nch + kSplit - 1) / kSplit;
  const int cb = wave * per;
  const int ce = min(nch, cb + per);
  const uint4* xv = reinterpret_cast<const uint4*>(x);
  const uint4* wr[kRows];
#pragma unroll
  for (int r = 0; r < kRows; ++r) {
    const int64_t row = row0 + r < n ? row0 + r : n - 1;  // tail rows re-read the last one
    wr[r] = reinterpret_cast<const uint4*>(w + row * ws);
  }
  float acc[kRows] = {};
  for (int c0 = cb; c0 < ce; c0 += 64 * kUnroll) {
    uint4 xc[kUnroll], wc[kRows][kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int c = c0 + 64 * u + lane;
      const bool in = c < ce;
      xc[u] = in ? xv[c] : uint4{0, 0, 0, 0};
#pragma unroll
      for (int r = 0; r < kRows; ++r) {  // weights stream once per token: non-temporal
        const u32x4 v = in ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(&wr[r][c]))
                           : u32x4{0, 0, 0, 0};
        wc[r][u] = uint4{v[0], v[1], v[2], v[3]};
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
#pragma unroll
      for (int r = 0; r < kRows; ++r) acc[r] = dot8(wc[r][u], xc[u], acc[r]);
  }
#pragma unroll
  for (int r = 0; r < kRows; ++r)
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) acc[r] += __shfl_xor(acc[r], off);
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < kRows; ++r) part[wave][r] = acc[r];
  }
  __syncthreads();
  if (threadIdx.x < kRows && row0 + threadIdx.x < n) {
    float v = 0.f;
#pragma unroll
    for (int i = 0; i < kSplit; ++i) v += part[i][threadIdx.x];
    y[row0 + threadIdx.x] = f32_to_bf16(v);
  }
}

}  // namespace

hipError_t launch_gemv_bf16(int64_t n, int k, const void* w, int64_t ws, const void* x, void* y,
                            hipStream_t s) {
  const int64_t grid = (n + kRows - 1) / kRows;
  hipLaunchKernelGGL(gemv_bf16_kernel, dim3((unsigned)grid), dim3(64 * kSplit), 0, s, n, k,
                     static_cast<const uint16_t*>(w), ws, static_cast<const uint16_t*>(x),
                     static_cast<uint16_t*>(y));
  return hipGetLastError();
}

}  // namespace lc
