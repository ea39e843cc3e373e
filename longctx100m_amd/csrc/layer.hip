// Row kernels around one decoder layer's attention (gfx950): RMSNorm with the
// residual add fused, the RoPE position table and rotate-half RoPE, and the
// SwiGLU gate.  All are HBM-bound streams: 16-byte vector loads and stores,
// fp32 arithmetic, bf16 rounding at the points the reference rounds.
//
//   RMSNorm  rust/longctx100m-model/src/model.rs:53-62 (decoder use :387-393)
//   RoPE     rust/longctx100m-model/src/rope.rs:101-127
//   SwiGLU   rust/longctx100m-model/src/model.rs:323-327
#include "common.h"
#include "kernels.h"

// Each product and sum rounds on its own, as the reference's tensor ops do:
// no contraction into fused multiply-adds in this file (the build also passes
// -ffp-contract=off for it; sums of squares use an explicit fmaf).
#pragma clang fp contract(off)

namespace lc {
namespace {

typedef float f32x8 __attribute__((ext_vector_type(8)));

// 8 consecutive elements as fp32 (one 16-byte load for bf16, two for fp32).
template <typename T>
__device__ __forceinline__ f32x8 load8(const T* p);
template <>
__device__ __forceinline__ f32x8 load8<uint16_t>(const uint16_t* p) {
  const uint4 u = *reinterpret_cast<const uint4*>(p);
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
  f32x8 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    r[2 * i] = __uint_as_float(w[i] << 16);
    r[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
  return r;
}
template <>
__device__ __forceinline__ f32x8 load8<float>(const float* p) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  const float4 b = *reinterpret_cast<const float4*>(p + 4);
  return f32x8{a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
}

template <typename T>
__device__ __forceinline__ void store8(T* p, const f32x8& v);
template <>
__device__ __forceinline__ void store8<uint16_t>(uint16_t* p, const f32x8& v) {
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    w[i] = (uint32_t)f32_to_bf16(v[2 * i]) | ((uint32_t)f32_to_bf16(v[2 * i + 1]) << 16);
  *reinterpret_cast<uint4*>(p) = uint4{w[0], w[1], w[2], w[3]};
}
template <>
__device__ __forceinline__ void store8<float>(float* p, const f32x8& v) {
  *reinterpret_cast<float4*>(p) = float4{v[0], v[1], v[2], v[3]};
  *reinterpret_cast<float4*>(p + 4) = float4{v[4], v[5], v[6], v[7]};
}


// Non-temporal forms, for the prefill's streams: read or written once, far
// larger than the caches.  (A decode step's single rows are read right after
// they are written, so they keep the default policy.)
template <typename T>
__device__ __forceinline__ f32x8 load8_nt(const T* p);
template <>
__device__ __forceinline__ f32x8 load8_nt<uint16_t>(const uint16_t* p) {
  typedef uint32_t u4 __attribute__((ext_vector_type(4)));
  const u4 u = __builtin_nontemporal_load(reinterpret_cast<const u4*>(p));
  f32x8 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    r[2 * i] = __uint_as_float(u[i] << 16);
    r[2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
  }
  return r;
}
template <>
__device__ __forceinline__ f32x8 load8_nt<float>(const float* p) {
  typedef float f4 __attribute__((ext_vector_type(4)));
  const f4 a = __builtin_nontemporal_load(reinterpret_cast<const f4*>(p));
  const f4 b = __builtin_nontemporal_load(reinterpret_cast<const f4*>(p + 4));
  return f32x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}
template <typename T>
__device__ __forceinline__ void store8_nt(T* p, const f32x8& v);
template <>
__device__ __forceinline__ void store8_nt<uint16_t>(uint16_t* p, const f32x8& v) {
  typedef uint32_t u4 __attribute__((ext_vector_type(4)));
  u4 w;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    w[i] = (uint32_t)f32_to_bf16(v[2 * i]) | ((uint32_t)f32_to_bf16(v[2 * i + 1]) << 16);
  __builtin_nontemporal_store(w, reinterpret_cast<u4*>(p));
}
template <>
__device__ __forceinline__ void store8_nt<float>(float* p, const f32x8& v) {
  typedef float f4 __attribute__((ext_vector_type(4)));
  __builtin_nontemporal_store(f4{v[0], v[1], v[2], v[3]}, reinterpret_cast<f4*>(p));
  __builtin_nontemporal_store(f4{v[4], v[5], v[6], v[7]}, reinterpret_cast<f4*>(p + 4));
}
template <typename T, bool NT>
__device__ __forceinline__ f32x8 ld8(const T* p) {
  if constexpr (NT) return load8_nt<T>(p);
  else return load8<T>(p);
}
template <typename T, bool NT>
__device__ __forceinline__ void st8(T* p, const f32x8& v) {
  if constexpr (NT) store8_nt<T>(p, v);
  else store8<T>(p, v);
}
// Row counts from which the row kernels stream non-temporally (prefill shapes).
constexpr int64_t kStreamRows = 1024;

// Round to the storage type and back (identity for fp32).
template <typename T>
__device__ __forceinline__ float rnd(float x);
template <>
__device__ __forceinline__ float rnd<float>(float x) {
  return x;
}
template <>
__device__ __forceinline__ float rnd<uint16_t>(float x) {
  return bf16_to_f32(f32_to_bf16(x));
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) x += __shfl_xor(x, off, 64);
  return x;
}

// ---------------------------------------------------------------- RMSNorm --
// WPR waves per row (one for rows of up to 4096 columns, four above); each
// lane keeps its NC 8-element chunks of the row in registers between the sum
// of squares and the scaling.  Chunk i of lane l in wave w of the row is
// chunk (64 w + l) + 64 WPR i of the row.  With at most 8 chunks per lane the
// row, the residual and the weight chunks fit the registers without spilling.
template <typename T, int NC, int WPR, bool NT>
__global__ __launch_bounds__(256) void rmsnorm_kernel(int64_t rows, int cols, float eps,
                                                      const T* __restrict__ x, int64_t xs,
                                                      const T* __restrict__ res, int64_t rs,
                                                      T* __restrict__ res_out, int64_t ros,
                                                      const T* __restrict__ w,
                                                      T* __restrict__ out, int64_t os) {
  static_assert(4 % WPR == 0, "waves per row divide the workgroup");
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wsub = wave % WPR;  // this wave's part of the row
  const int64_t row = (int64_t)blockIdx.x * (4 / WPR) + wave / WPR;
  if (row >= rows) return;  // with WPR > 1 the workgroup holds one row: all or none return
  const int nchunk = cols / 8;
  const int c0 = 64 * wsub + lane;
  // All loads of the row are issued, unconditionally (chunks past the row
  // re-read its last chunk and are zeroed), before the first use, so a row
  // costs one memory latency rather than one per chunk (a decode step
  // normalises single rows, where that latency is the whole cost).
  f32x8 v[NC];
#pragma unroll
  for (int i = 0; i < NC; ++i) v[i] = ld8<T, NT>(x + row * xs + 8 * min(c0 + 64 * WPR * i, nchunk - 1));
  if (res != nullptr) {
    f32x8 r[NC];
#pragma unroll
    for (int i = 0; i < NC; ++i) r[i] = ld8<T, NT>(res + row * rs + 8 * min(c0 + 64 * WPR * i, nchunk - 1));
#pragma unroll
    for (int i = 0; i < NC; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) v[i][j] = rnd<T>(v[i][j] + r[i][j]);  // x + attn(x) in the model dtype
    if (res_out != nullptr) {
#pragma unroll
      for (int i = 0; i < NC; ++i) {
        const int c = c0 + 64 * WPR * i;
        if (c < nchunk) st8<T, NT>(res_out + row * ros + 8 * c, v[i]);
      }
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const bool in = c0 + 64 * WPR * i < nchunk;
#pragma unroll
    for (int j = 0; j < 8; ++j) ss = fmaf(v[i][j], in ? v[i][j] : 0.f, ss);
  }
  ss = wave_sum(ss);
  if constexpr (WPR > 1) {  // the row's waves add their parts in LDS
    __shared__ float part[4];
    if (lane == 0) part[wave] = ss;
    __syncthreads();
    ss = 0.f;
#pragma unroll
    for (int k = 0; k < WPR; ++k) ss += part[k];
  }
  // mean(h^2) + eps, then sqrt and reciprocal as two rounded steps (model.rs:57).
  const float inv = 1.0f / __fsqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)cols), eps));
#pragma unroll
  for (int i = 0; i < NC; ++i) {  // weight chunk i, then v[i] is done with
    const int c = c0 + 64 * WPR * i;
    const f32x8 wt = load8<T>(w + 8 * min(c, nchunk - 1));
#pragma unroll
    for (int j = 0; j < 8; ++j) v[i][j] = rnd<T>(rnd<T>(__fmul_rn(v[i][j], inv)) * wt[j]);
  }
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int c = c0 + 64 * WPR * i;
    if (c < nchunk) st8<T, NT>(out + row * os + 8 * c, v[i]);
  }
}

template <typename T>
hipError_t launch_rmsnorm_t(int64_t rows, int cols, float eps, const void* x, int64_t xs,
                            const void* res, int64_t rs, void* res_out, int64_t ros,
                            const void* w, void* out, int64_t os, hipStream_t s) {
  const int nchunk = cols / 8;
  auto args = [&](auto kernel, int rows_per_block) {
    const dim3 grid((unsigned)((rows + rows_per_block - 1) / rows_per_block)), block(256);
    hipLaunchKernelGGL(kernel, grid, block, 0, s, rows, cols, eps, static_cast<const T*>(x), xs,
                       static_cast<const T*>(res), rs, static_cast<T*>(res_out), ros,
                       static_cast<const T*>(w), static_cast<T*>(out), os);
  };
  const bool nt = rows >= kStreamRows;
  if (nchunk <= 64 * 2)
    nt ? args(rmsnorm_kernel<T, 2, 1, true>, 4) : args(rmsnorm_kernel<T, 2, 1, false>, 4);
  else if (nchunk <= 64 * 8)
    nt ? args(rmsnorm_kernel<T, 8, 1, true>, 4) : args(rmsnorm_kernel<T, 8, 1, false>, 4);
  else  // up to 64 * 4 * 8 chunks = 16384 columns
    nt ? args(rmsnorm_kernel<T, 8, 4, true>, 1) : args(rmsnorm_kernel<T, 8, 4, false>, 1);
  return hipGetLastError();
}

// ------------------------------------------------------------------- RoPE --
struct RopeTableArgs {
  float inv[128];
  float cos_factor;
  float pos_scale;  // 1/factor for the linear profile
  int linear;
  int half;
  int64_t tokens, pos0;
  float* table;
};

// table[t][0][i] = cos(f) * cos_factor, table[t][1][i] = sin(f), f = pos * inv[i]
// with the position converted to fp32 first (rope.rs:101-114).
__global__ __launch_bounds__(256) void rope_table_kernel(RopeTableArgs a) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= a.tokens * a.half) return;
  const int64_t t = idx / a.half;
  const int i = (int)(idx - t * a.half);
  float pos = (float)(a.pos0 + t);
  if (a.linear) pos = __fmul_rn(pos, a.pos_scale);
  const float f = __fmul_rn(pos, a.inv[i]);
  float* row = a.table + t * 2 * a.half;
  row[i] = __fmul_rn(cosf(f), a.cos_factor);
  row[a.half + i] = sinf(f);
}

// One thread per (token, head, 8 rotation pairs): x1 = x[8c..8c+7] and
// x2 = x[half+8c..], out1 = x1*cos - x2*sin, out2 = x2*cos + x1*sin.
template <typename T, bool NT>
__global__ __launch_bounds__(256) void rope_apply_kernel(int64_t tokens, int heads, int half,
                                                         const float* table, const T* src,
                                                         int64_t sts, T* dst) {
  const int cph = half / 8;  // chunks per head
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t total = tokens * heads * cph;
  if (idx >= total) return;
  const int c = (int)(idx % cph);
  const int64_t th = idx / cph;
  const int h = (int)(th % heads);
  const int64_t t = th / heads;
  const T* s = src + t * sts + (int64_t)h * 2 * half + 8 * c;
  T* d = dst + (t * heads + h) * 2 * half + 8 * c;
  const f32x8 x1 = ld8<T, NT>(s);
  const f32x8 x2 = ld8<T, NT>(s + half);
  const float* tr = table + t * 2 * half + 8 * c;
  const f32x8 cs = load8<float>(tr);
  const f32x8 sn = load8<float>(tr + half);
  f32x8 o1, o2;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    o1[j] = x1[j] * cs[j] - x2[j] * sn[j];
    o2[j] = x2[j] * cs[j] + x1[j] * sn[j];
  }
  st8<T, NT>(d, o1);
  st8<T, NT>(d + half, o2);
}

// ----------------------------------------------------------------- SwiGLU --
template <typename T, bool NT>
__global__ __launch_bounds__(256) void swiglu_kernel(int64_t rows, int cols, const T* g,
                                                     int64_t gs, const T* u, int64_t us,
                                                     T* out) {
  const int cpr = cols / 8;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= rows * cpr) return;
  const int64_t r = idx / cpr;
  const int c = (int)(idx - r * cpr);
  const f32x8 gv = ld8<T, NT>(g + r * gs + 8 * c);
  const f32x8 uv = ld8<T, NT>(u + r * us + 8 * c);
  f32x8 o;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float sl = rnd<T>(__fdiv_rn(gv[j], __fadd_rn(1.0f, expf(-gv[j]))));
    o[j] = __fmul_rn(sl, uv[j]);
  }
  st8<T, NT>(out + r * (int64_t)cols + 8 * c, o);
}

unsigned blocks_for(int64_t n) { return (unsigned)((n + 255) / 256); }

}  // namespace

hipError_t launch_rmsnorm(int dtype, int64_t rows, int cols, float eps, const void* x,
                          int64_t xs, const void* res, int64_t rs, void* res_out, int64_t ros,
                          const void* w, void* out, int64_t os, hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  return dtype == 1 ? launch_rmsnorm_t<uint16_t>(rows, cols, eps, x, xs, res, rs, res_out, ros, w,
                                                 out, os, s)
                    : launch_rmsnorm_t<float>(rows, cols, eps, x, xs, res, rs, res_out, ros, w,
                                              out, os, s);
}

hipError_t launch_rope_table(const float* inv, int half, float cos_factor, bool linear,
                             float pos_scale, int64_t tokens, int64_t pos0, float* table,
                             hipStream_t s) {
  if (tokens <= 0) return hipSuccess;
  RopeTableArgs a;
  for (int i = 0; i < half; ++i) a.inv[i] = inv[i];
  a.cos_factor = cos_factor;
  a.pos_scale = pos_scale;
  a.linear = linear ? 1 : 0;
  a.half = half;
  a.tokens = tokens;
  a.pos0 = pos0;
  a.table = table;
  hipLaunchKernelGGL(rope_table_kernel, dim3(blocks_for(tokens * half)), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_rope_apply(int dtype, int64_t tokens, int heads, int head_dim,
                             const float* table, const void* src, int64_t sts, void* dst,
                             hipStream_t s) {
  const int half = head_dim / 2;
  const int64_t n = tokens * heads * (half / 8);
  if (n <= 0) return hipSuccess;
  auto go = [&](auto kernel, auto* src_t, auto* dst_t) {
    hipLaunchKernelGGL(kernel, dim3(blocks_for(n)), dim3(256), 0, s, tokens, heads, half, table,
                       src_t, sts, dst_t);
  };
  const bool nt = tokens >= kStreamRows;
  if (dtype == 1) {
    const uint16_t* sp = static_cast<const uint16_t*>(src);
    uint16_t* dp = static_cast<uint16_t*>(dst);
    nt ? go(rope_apply_kernel<uint16_t, true>, sp, dp) : go(rope_apply_kernel<uint16_t, false>, sp, dp);
  } else {
    const float* sp = static_cast<const float*>(src);
    float* dp = static_cast<float*>(dst);
    nt ? go(rope_apply_kernel<float, true>, sp, dp) : go(rope_apply_kernel<float, false>, sp, dp);
  }
  return hipGetLastError();
}

hipError_t launch_swiglu(int dtype, int64_t rows, int cols, const void* g, int64_t gs,
                         const void* u, int64_t us, void* out, hipStream_t s) {
  const int64_t n = rows * (cols / 8);
  if (n <= 0) return hipSuccess;
  auto go = [&](auto kernel, auto* g_t, auto* u_t, auto* o_t) {
    hipLaunchKernelGGL(kernel, dim3(blocks_for(n)), dim3(256), 0, s, rows, cols, g_t, gs, u_t, us,
                       o_t);
  };
  const bool nt = rows >= kStreamRows;
  if (dtype == 1) {
    const uint16_t* gp = static_cast<const uint16_t*>(g);
    const uint16_t* up = static_cast<const uint16_t*>(u);
    uint16_t* op = static_cast<uint16_t*>(out);
    nt ? go(swiglu_kernel<uint16_t, true>, gp, up, op) : go(swiglu_kernel<uint16_t, false>, gp, up, op);
  } else {
    const float* gp = static_cast<const float*>(g);
    const float* up = static_cast<const float*>(u);
    float* op = static_cast<float*>(out);
    nt ? go(swiglu_kernel<float, true>, gp, up, op) : go(swiglu_kernel<float, false>, gp, up, op);
  }
  return hipGetLastError();
}

}  // namespace lc
