// Device helpers shared by the gfx950 attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lc {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kFltMin = 1.17549435e-38f;  // FLT_MIN, the reference's l clamp (rs:227)

__device__ __forceinline__ float bf16_to_f32(uint16_t x) {
  return __uint_as_float(static_cast<uint32_t>(x) << 16);
}

// Round-to-nearest-even fp32 -> bf16 (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  __bf16 b = static_cast<__bf16>(f);
  return __builtin_bit_cast(uint16_t, b);
}

template <typename T>
__device__ __forceinline__ float load_f32(const T* p);
template <>
__device__ __forceinline__ float load_f32<float>(const float* p) {
  return *p;
}
template <>
__device__ __forceinline__ float load_f32<uint16_t>(const uint16_t* p) {
  return bf16_to_f32(*p);
}

template <typename T>
__device__ __forceinline__ void store_from_f32(T* p, float v);
template <>
__device__ __forceinline__ void store_from_f32<float>(float* p, float v) {
  *p = v;
}
template <>
__device__ __forceinline__ void store_from_f32<uint16_t>(uint16_t* p, float v) {
  *p = f32_to_bf16(v);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ f32x4 mfma16x16x32(const bf16x8& a, const bf16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// 32x32x16 bf16 MFMA.  Operand layouts (lane l, h = l / 32):
//   A (32 x 16): lane l holds A[l % 32][8h .. 8h+7];
//   B (16 x 32): lane l holds B[8h .. 8h+7][l % 32];
//   D (32 x 32): lane l, element v holds D[8(v/4) + 4h + v%4][l % 32].
__device__ __forceinline__ f32x16 mfma32x32x16(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Hides a value from loop-invariant code motion, so offsets derived from it
// by an XOR are formed next to their use instead of occupying registers.
__device__ __forceinline__ int opaque(int x) {
  asm volatile("" : "+v"(x));
  return x;
}

__device__ __forceinline__ bf16x8 pack_bf16x8(const f32x4& lo, const f32x4& hi) {
  bf16x8 r;
  r[0] = static_cast<__bf16>(lo[0]);
  r[1] = static_cast<__bf16>(lo[1]);
  r[2] = static_cast<__bf16>(lo[2]);
  r[3] = static_cast<__bf16>(lo[3]);
  r[4] = static_cast<__bf16>(hi[0]);
  r[5] = static_cast<__bf16>(hi[1]);
  r[6] = static_cast<__bf16>(hi[2]);
  r[7] = static_cast<__bf16>(hi[3]);
  return r;
}

__device__ __forceinline__ bf16x8 concat_bf16x4(const bf16x4& lo, const bf16x4& hi) {
  bf16x8 r;
  r[0] = lo[0];
  r[1] = lo[1];
  r[2] = lo[2];
  r[3] = lo[3];
  r[4] = hi[0];
  r[5] = hi[1];
  r[6] = hi[2];
  r[7] = hi[3];
  return r;
}

// Max / sum over the four 16-lane groups of a wave (lanes l, l^16, l^32, l^48),
// with gfx950's v_permlane32_swap / v_permlane16_swap (no LDS round trip):
// swap(x, x) returns (x with its upper half replaced by the lower, x with its
// lower half replaced by the upper), so combining the pair combines l and
// l ^ 32 (resp. l ^ 16).
__device__ __forceinline__ float xor32_max(float x) {
  const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}
__device__ __forceinline__ float xor16_max(float x) {
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}
__device__ __forceinline__ float xor32_sum(float x) {
  const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}
__device__ __forceinline__ float xor16_sum(float x) {
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}
__device__ __forceinline__ float group4_max(float x) { return xor16_max(xor32_max(x)); }
__device__ __forceinline__ float group4_sum(float x) { return xor16_sum(xor32_sum(x)); }

// Weights of the two partials in the merged output.  With m = max(m_a, m_b):
// l = e^{m_a-m} l_a + e^{m_b-m} l_b and o = (e^{m_a-m} l_a o_a + e^{m_b-m} l_b o_b) / l,
// which equals carrying the reference's unnormalised (m, l, acc) across the
// two partials (rs:36-53 applied blockwise).  No key seen on either side:
// weights 0, l = 0, m = -inf.
struct MergeW {
  float wa, wb, m, l;
};
__device__ __forceinline__ MergeW merge_weights(float ma, float la, float mb, float lb) {
  MergeW w;
  w.m = fmaxf(ma, mb);
  if (w.m == -INFINITY) {
    w.wa = w.wb = w.l = 0.f;
    return w;
  }
  const float ea = expf(ma - w.m) * la;
  const float eb = expf(mb - w.m) * lb;
  w.l = ea + eb;
  const float inv = w.l > 0.f ? 1.f / w.l : 0.f;
  w.wa = ea * inv;
  w.wb = eb * inv;
  return w;
}

// Workgroups are dispatched round-robin over the 8 XCDs (workgroup p runs on
// XCD p % 8).  Give every XCD a contiguous range of logical tile ids so the
// tiles that share K/V (same head) share that XCD's L2.
__device__ __forceinline__ int xcd_remap(int pid, int nwg) {
  constexpr int kXcds = 8;
  const int per = nwg / kXcds;
  const int rem = nwg % kXcds;
  const int xcd = pid % kXcds;
  const int idx = pid / kXcds;
  return xcd * per + (xcd < rem ? xcd : rem) + idx;
}

// Byte-select of two dwords (v_perm_b32): result byte i = sel byte i indexes
// {lo bytes 0-3, hi bytes 4-7}.
__device__ __forceinline__ uint32_t perm_b32(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}
constexpr uint32_t kSelLoHalves = 0x05040100u;  // {lo.h0, hi.h0}
constexpr uint32_t kSelHiHalves = 0x07060302u;  // {lo.h1, hi.h1}

}  // namespace lc
