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
#include <algorithm>
#include <type_traits>

#include "common.h"
#include "kernels.h"

// The folded row operations round every product and sum on their own, as
// layer.hip's stand-alone kernels do: no contraction into fused multiply-adds
// in this file (the build also passes -ffp-contract=off for it).  The _rn
// intrinsics alone do not ensure that: without OCML_BASIC_ROUNDED_OPERATIONS
// they are plain operators, which contraction fuses once inlined (one RoPE
// output in thousands came out an ulp apart).  The dot products use explicit
// fmaf and are unaffected.
#pragma clang fp contract(off)

namespace lc {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kPlainRows = 4;
constexpr int kUnroll = 4;
constexpr int kPlainSplit = 4;  // waves per workgroup, each over 1/kPlainSplit of the row
// The fused forms: four rows per workgroup (their row maps pair rows for
// SwiGLU and RoPE), kSplit waves over each row.
constexpr int kRows = 4;
constexpr int kSplit = 4;
// Each lane sums its chunks in increasing order whatever the rows per
// workgroup and the unroll; the split of a row over waves and the order of the
// wave sums are the rest of the reduction order, so the fused forms equal
// lc_gemv bit for bit only with the same split.
static_assert(kSplit == kPlainSplit, "fused and plain kernels reduce in the same order");

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

__global__ __launch_bounds__(64 * kPlainSplit) void gemv_bf16_kernel(int64_t n, int k,
                                                                 const uint16_t* w, int64_t ws,
                                                                 const uint16_t* x, uint16_t* y) {
  __shared__ float part[kPlainSplit][kPlainRows];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t row0 = (int64_t)blockIdx.x * kPlainRows;
  const int nch = k / 8;  // 16-byte chunks per row
  const int per = (nch + kPlainSplit - 1) / kPlainSplit;
  const int cb = wave * per;
  const int ce = min(nch, cb + per);
  const uint4* xv = reinterpret_cast<const uint4*>(x);
  const uint4* wr[kPlainRows];
#pragma unroll
  for (int r = 0; r < kPlainRows; ++r) {
    const int64_t row = row0 + r < n ? row0 + r : n - 1;  // tail rows re-read the last one
    wr[r] = reinterpret_cast<const uint4*>(w + row * ws);
  }
  float acc[kPlainRows] = {};
  for (int c0 = cb; c0 < ce; c0 += 64 * kUnroll) {
    uint4 xc[kUnroll], wc[kPlainRows][kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int c = c0 + 64 * u + lane;
      const bool in = c < ce;
      xc[u] = in ? xv[c] : uint4{0, 0, 0, 0};
#pragma unroll
      for (int r = 0; r < kPlainRows; ++r) {  // weights stream once per token: non-temporal
        const u32x4 v = in ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(&wr[r][c]))
                           : u32x4{0, 0, 0, 0};
        wc[r][u] = uint4{v[0], v[1], v[2], v[3]};
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
#pragma unroll
      for (int r = 0; r < kPlainRows; ++r) acc[r] = dot8(wc[r][u], xc[u], acc[r]);
  }
#pragma unroll
  for (int r = 0; r < kPlainRows; ++r)
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) acc[r] += __shfl_xor(acc[r], off);
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < kPlainRows; ++r) part[wave][r] = acc[r];
  }
  __syncthreads();
  if (threadIdx.x < kPlainRows && row0 + threadIdx.x < n) {
    float v = 0.f;
#pragma unroll
    for (int i = 0; i < kPlainSplit; ++i) v += part[i][threadIdx.x];
    y[row0 + threadIdx.x] = f32_to_bf16(v);
  }
}

// ---------------------------------------------------------- fused forms --
// The same streaming loop with the row operation before or after the
// projection folded in (one launch in place of two to four in the decode
// step).  Each folded operation repeats the arithmetic of its stand-alone
// kernel step for step, with every product and sum rounded on its own
// (explicit _rn intrinsics), so the results are bit-identical:
//   RMSNorm (layer.hip rmsnorm_kernel, one wave per row of <= 4096 columns):
//     v = bf16(x + residual); ss = lane-sequential fmaf chain over the
//     lane's chunks l + 64 i (i < 2 up to 1024 columns, else i < 8), then a
//     butterfly over offsets 1, 2, .., 32; inv = 1 / sqrt(ss / cols + eps);
//     h = bf16(bf16(v * inv) * weight).  The workgroup stages v in LDS once
//     and every wave runs the chain on it (same order, same sum).
//   cast of the fp32 attention output to bf16: nearest even.
//   SwiGLU (swiglu_kernel): s = bf16(g / (1 + exp(-g))), out = bf16(s * u)
//     of the bf16 gate and up products.
//   RoPE (rope_apply_kernel): x1 cos - x2 sin, x2 cos + x1 sin of the bf16
//     products, each product rounded, then the difference / sum.
// A workgroup owns kRows weight rows: four consecutive rows (plain, and the v
// part of the QKV form), gate rows i, i+1 with up rows I+i, I+i+1 (SwiGLU),
// or rows i, i+1, i+half, i+half+1 of one q or k head (RoPE).

enum { kInBf16 = 0, kInF32 = 1, kInNorm = 2 };
enum { kOutPlain = 0, kOutSwiglu = 1, kOutRope = 2 };
constexpr int kNormMaxChunks = 512;  // 4096 columns
// Workgroups of the folded-norm form, each computing the norm once and
// looping over row blocks: the norm costs a workgroup its row's loads and a
// barrier, so fewer, longer-lived workgroups stream faster (gate/up
// projection, 7168 row blocks: 37.1 us at 1024, 38 at 2048, 41 at 4096,
// 54 with one block per workgroup).
constexpr int64_t kNormMaxGrid = 1024;
// Chunks per row per lane and round: 2 covers a 4096-column row in one round
// (the decode step's projections but the down projection, which takes the
// plain bf16 form and so lc_gemv's kernel).
constexpr int kFusedUnroll = 2;

struct GemvFused {
  int64_t rows;
  int cols;
  const uint16_t* w;
  int64_t ws;
  const void* x;
  uint16_t* y;
  const uint16_t* res;
  uint16_t* res_out;
  const uint16_t* nw;
  float eps;
  int q_heads, kv_heads, head_dim;
  const float* rope;
  uint16_t* k_out;
  uint16_t* v_out;
  int64_t rope_blocks;  // row blocks of q/k rotation pairs (the v rows follow)
  int64_t blocks;       // row blocks in all
};

__device__ __forceinline__ float bf16r(float v) { return bf16_to_f32(f32_to_bf16(v)); }

__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  return (uint32_t)f32_to_bf16(lo) | ((uint32_t)f32_to_bf16(hi) << 16);
}

template <int IN, int OUT>
__global__ __launch_bounds__(64 * kSplit) void gemv_fused_kernel(GemvFused a) {
  __shared__ float part[kSplit][kRows];
  __shared__ uint4 hbuf[IN == kInNorm ? kNormMaxChunks : 1];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nch = a.cols / 8;
  const int per = (nch + kSplit - 1) / kSplit;
  const int cb = wave * per;
  const int ce = min(nch, cb + per);

  // Loads first (the folded norm's row, residual and weight chunks, then the
  // first row block's weights, see below), so that the norm's arithmetic and
  // barrier run while the weights are in flight.
  uint4 xr[kNormMaxChunks / (64 * kSplit)], rr[kNormMaxChunks / (64 * kSplit)];
  uint4 gv[kFusedUnroll];
  if constexpr (IN == kInNorm) {
#pragma unroll
    for (int i = 0; i < kNormMaxChunks / (64 * kSplit); ++i) {
      const int c = threadIdx.x + 64 * kSplit * i;
      xr[i] = rr[i] = uint4{0, 0, 0, 0};
      if (c < nch) {
        xr[i] = reinterpret_cast<const uint4*>(a.x)[c];
        if (a.res != nullptr) rr[i] = reinterpret_cast<const uint4*>(a.res)[c];
      }
    }
#pragma unroll
    for (int u = 0; u < kFusedUnroll; ++u) {
      const int c = cb + 64 * u + lane;
      gv[u] = c < ce ? reinterpret_cast<const uint4*>(a.nw)[c] : uint4{0, 0, 0, 0};
    }
  }
  float inv = 0.f;  // the folded norm's 1/rms
  // The folded RMSNorm's 1/rms, once per workgroup (the grid of this form is
  // capped, each workgroup looping over several row blocks): v = x (+ res) to
  // LDS (and to res_out from workgroup 0), then every wave runs the
  // stand-alone kernel's sum-of-squares chain on it.
  auto norm_scale = [&]() -> float {
#pragma unroll
    for (int i = 0; i < kNormMaxChunks / (64 * kSplit); ++i) {
      const int c = threadIdx.x + 64 * kSplit * i;
      if (c >= nch) continue;
      uint4 v = xr[i];
      if (a.res != nullptr) {
        const uint32_t xw[4] = {v.x, v.y, v.z, v.w}, rw[4] = {rr[i].x, rr[i].y, rr[i].z, rr[i].w};
        uint32_t o[4];
#pragma unroll
        for (int k = 0; k < 4; ++k)
          o[k] = pack2(__fadd_rn(bf16_lo(xw[k]), bf16_lo(rw[k])),
                       __fadd_rn(bf16_hi(xw[k]), bf16_hi(rw[k])));
        v = uint4{o[0], o[1], o[2], o[3]};
        if (a.res_out != nullptr && blockIdx.x == 0) reinterpret_cast<uint4*>(a.res_out)[c] = v;
      }
      hbuf[c] = v;
    }
    __syncthreads();
    const int nc = nch <= 128 ? 2 : 8;
    float ss = 0.f;
    for (int i = 0; i < nc; ++i) {
      const int c = lane + 64 * i;
      const uint4 v = hbuf[min(c, nch - 1)];
      const bool in = c < nch;
      const uint32_t vw[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float lo = bf16_lo(vw[k]), hi = bf16_hi(vw[k]);
        ss = fmaf(lo, in ? lo : 0.f, ss);
        ss = fmaf(hi, in ? hi : 0.f, ss);
      }
    }
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) ss += __shfl_xor(ss, off, 64);
    return 1.0f / __fsqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)a.cols), a.eps));
  };

  // The bf16 chunk c of the multiplied vector (u: its slot among the lane's chunks).
  auto xchunk = [&](int c, int u) -> uint4 {
    if constexpr (IN == kInBf16) {
      return reinterpret_cast<const uint4*>(a.x)[c];
    } else if constexpr (IN == kInF32) {
      const float4* xf = reinterpret_cast<const float4*>(a.x);
      const float4 p = xf[2 * c], q = xf[2 * c + 1];
      return uint4{pack2(p.x, p.y), pack2(p.z, p.w), pack2(q.x, q.y), pack2(q.z, q.w)};
    } else {
      const uint4 v = hbuf[c];
      const uint4 g = gv[u];  // norm weight chunk c, loaded up front
      const uint32_t vw[4] = {v.x, v.y, v.z, v.w}, gw[4] = {g.x, g.y, g.z, g.w};
      uint32_t o[4];
#pragma unroll
      for (int k = 0; k < 4; ++k)
        o[k] = pack2(__fmul_rn(bf16r(__fmul_rn(bf16_lo(vw[k]), inv)), bf16_lo(gw[k])),
                     __fmul_rn(bf16r(__fmul_rn(bf16_hi(vw[k]), inv)), bf16_hi(gw[k])));
      return uint4{o[0], o[1], o[2], o[3]};
    }
  };

  // Weight rows of row block blk.
  auto block_rows = [&](int64_t blk, int64_t (&row)[kRows]) {
    if constexpr (OUT == kOutPlain) {
#pragma unroll
      for (int r = 0; r < kRows; ++r) row[r] = min(blk * kRows + r, a.rows - 1);
    } else if constexpr (OUT == kOutSwiglu) {
      const int64_t inter = a.rows / 2, i0 = 2 * blk;
      row[0] = i0;
      row[1] = i0 + 1;
      row[2] = inter + i0;
      row[3] = inter + i0 + 1;
    } else {
      const int half = a.head_dim / 2;
      if (blk < a.rope_blocks) {
        const int64_t p0 = 2 * blk;  // rotation pairs p0, p0 + 1 of one head (half is even)
        const int64_t head = p0 / half;
        const int64_t base = head * a.head_dim + (p0 - head * half);
        row[0] = base;
        row[1] = base + 1;
        row[2] = base + half;
        row[3] = base + half + 1;
      } else {
        const int64_t v0 = (int64_t)(a.q_heads + a.kv_heads) * a.head_dim +
                           kRows * (blk - a.rope_blocks);
#pragma unroll
        for (int r = 0; r < kRows; ++r) row[r] = v0 + r;
      }
    }
  };
  // This lane's weight chunks c0 + 64 u + lane (u < kFusedUnroll) of the block's rows.
  auto load_w = [&](int64_t blk, int c0, uint4 (&wc)[kRows][kFusedUnroll]) {
    int64_t row[kRows];
    block_rows(blk, row);
#pragma unroll
    for (int u = 0; u < kFusedUnroll; ++u) {
      const int c = c0 + 64 * u + lane;
      const bool in = c < ce;
#pragma unroll
      for (int r = 0; r < kRows; ++r) {
        const u32x4 v = in ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(
                                 a.w + row[r] * a.ws + 8 * (int64_t)c))
                           : u32x4{0, 0, 0, 0};
        wc[r][u] = uint4{v[0], v[1], v[2], v[3]};
      }
    }
  };

  // Row totals of block blk (threads 0..kRows-1) to the output form.
  auto finish = [&](int64_t blk, const float (&acc_in)[kRows]) {
    float acc[kRows];
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
      acc[r] = acc_in[r];
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) acc[r] += __shfl_xor(acc[r], off);
    }
    if (lane == 0) {
#pragma unroll
      for (int r = 0; r < kRows; ++r) part[wave][r] = acc[r];
    }
    __syncthreads();
    if (threadIdx.x < kRows) {
      const int t = threadIdx.x;
      float tot[kRows];  // the row totals, summed over the waves in lc_gemv's order
#pragma unroll
      for (int r = 0; r < kRows; ++r) {
        float v = 0.f;
#pragma unroll
        for (int i = 0; i < kSplit; ++i) v += part[i][r];
        tot[r] = v;
      }
      if constexpr (OUT == kOutPlain) {
        if (blk * kRows + t < a.rows) a.y[blk * kRows + t] = f32_to_bf16(tot[t]);
      } else if constexpr (OUT == kOutSwiglu) {
        if (t < 2) {
          const float g = bf16r(t == 0 ? tot[0] : tot[1]);
          const float u = bf16r(t == 0 ? tot[2] : tot[3]);
          const float sl = bf16r(__fdiv_rn(g, __fadd_rn(1.0f, expf(-g))));
          a.y[2 * blk + t] = f32_to_bf16(__fmul_rn(sl, u));
        }
      } else if (blk >= a.rope_blocks) {
        a.v_out[kRows * (blk - a.rope_blocks) + t] = f32_to_bf16(tot[t]);
      } else if (t < 2) {
        const int half = a.head_dim / 2;
        const int64_t p0 = 2 * blk;
        const int head = (int)(p0 / half);
        const int pi = (int)(p0 - (int64_t)head * half);
        const float x1 = bf16r(t == 0 ? tot[0] : tot[1]);
        const float x2 = bf16r(t == 0 ? tot[2] : tot[3]);
        const float cs = a.rope[pi + t], sn = a.rope[half + pi + t];
        const float o1 = __fsub_rn(__fmul_rn(x1, cs), __fmul_rn(x2, sn));
        const float o2 = __fadd_rn(__fmul_rn(x2, cs), __fmul_rn(x1, sn));
        uint16_t* dst = head < a.q_heads ? a.y + (int64_t)head * a.head_dim
                                         : a.k_out + (int64_t)(head - a.q_heads) * a.head_dim;
        dst[pi + t] = f32_to_bf16(o1);
        dst[pi + half + t] = f32_to_bf16(o2);
      }
    }
    __syncthreads();  // part is rewritten by the next block
  };

  // The choice depends on `per` (the same for every wave), not on the wave's
  // own ce - cb (shorter for the last wave), so all waves of the workgroup
  // take the same loop and reach finish()'s barriers from the same place.
  if (IN == kInNorm || per <= 64 * kFusedUnroll) {  // the norm form has cols <= 4096
    // One round per row (rows of up to 4096 columns, so every folded-norm
    // call): the lane's chunks of the multiplied vector are formed once and
    // kept in registers, and the next block's weight loads are issued before
    // this block's reduction, so loads stay in flight between blocks.
    uint4 wc[kRows][kFusedUnroll];
    int64_t blk = blockIdx.x;
    if (blk < a.blocks) load_w(blk, cb, wc);
    if constexpr (IN == kInNorm) inv = norm_scale();
    uint4 xc[kFusedUnroll];
#pragma unroll
    for (int u = 0; u < kFusedUnroll; ++u) {
      const int c = cb + 64 * u + lane;
      xc[u] = c < ce ? xchunk(c, u) : uint4{0, 0, 0, 0};
    }
    for (; blk < a.blocks; blk += gridDim.x) {
      float acc[kRows] = {};
#pragma unroll
      for (int u = 0; u < kFusedUnroll; ++u)
#pragma unroll
        for (int r = 0; r < kRows; ++r) acc[r] = dot8(wc[r][u], xc[u], acc[r]);
      if (blk + gridDim.x < a.blocks) load_w(blk + gridDim.x, cb, wc);
      finish(blk, acc);
    }
  } else {
    for (int64_t blk = blockIdx.x; blk < a.blocks; blk += gridDim.x) {
      float acc[kRows] = {};
      for (int c0 = cb; c0 < ce; c0 += 64 * kFusedUnroll) {
        uint4 xc[kFusedUnroll], wc[kRows][kFusedUnroll];
#pragma unroll
        for (int u = 0; u < kFusedUnroll; ++u) {  // the vector's chunks first: waits on them leave the weights in flight
          const int c = c0 + 64 * u + lane;
          xc[u] = c < ce ? xchunk(c, u) : uint4{0, 0, 0, 0};
        }
        load_w(blk, c0, wc);
#pragma unroll
        for (int u = 0; u < kFusedUnroll; ++u)
#pragma unroll
          for (int r = 0; r < kRows; ++r) acc[r] = dot8(wc[r][u], xc[u], acc[r]);
      }
      finish(blk, acc);
    }
  }
}

}  // namespace

hipError_t launch_gemv_fused(int in_form, int out_form, int64_t rows, int cols, const void* w,
                             int64_t ws, const void* x, void* y, const void* res, void* res_out,
                             const void* nw, float eps, int q_heads, int kv_heads, int head_dim,
                             const float* rope, void* k_out, void* v_out, hipStream_t s) {
  GemvFused a;
  a.rows = rows;
  a.cols = cols;
  a.w = static_cast<const uint16_t*>(w);
  a.ws = ws;
  a.x = x;
  a.y = static_cast<uint16_t*>(y);
  a.res = static_cast<const uint16_t*>(res);
  a.res_out = static_cast<uint16_t*>(res_out);
  a.nw = static_cast<const uint16_t*>(nw);
  a.eps = eps;
  a.q_heads = q_heads;
  a.kv_heads = kv_heads;
  a.head_dim = head_dim;
  a.rope = rope;
  a.k_out = static_cast<uint16_t*>(k_out);
  a.v_out = static_cast<uint16_t*>(v_out);
  a.rope_blocks = 0;
  int64_t grid;
  if (out_form == kOutPlain) {
    grid = (rows + kRows - 1) / kRows;
  } else if (out_form == kOutSwiglu) {
    grid = rows / 4;  // two outputs per workgroup; rows % 4 == 0
  } else {
    a.rope_blocks = (int64_t)(q_heads + kv_heads) * (head_dim / 2) / 2;
    grid = a.rope_blocks + (int64_t)kv_heads * head_dim / kRows;
  }
  if (grid <= 0) return hipSuccess;
  if (in_form == kInBf16 && out_form == kOutPlain)  // nothing folded: lc_gemv's kernel
    return launch_gemv_bf16(rows, cols, w, ws, x, y, s);
  a.blocks = grid;
  // The folded RMSNorm is computed once per workgroup: cap its grid so that
  // the long projections (the LM head has 32,064 row blocks) do not repeat it
  // for every block; the other forms run one block per workgroup.
  if (in_form == kInNorm) grid = std::min<int64_t>(grid, kNormMaxGrid);
  auto go = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, dim3((unsigned)grid), dim3(64 * kSplit), 0, s, a);
  };
  auto pick_out = [&](auto in_tag) {
    constexpr int I = decltype(in_tag)::value;
    if (out_form == kOutPlain) go(gemv_fused_kernel<I, kOutPlain>);
    else if (out_form == kOutSwiglu) go(gemv_fused_kernel<I, kOutSwiglu>);
    else go(gemv_fused_kernel<I, kOutRope>);
  };
  if (in_form == kInBf16) pick_out(std::integral_constant<int, kInBf16>{});
  else if (in_form == kInF32) pick_out(std::integral_constant<int, kInF32>{});
  else pick_out(std::integral_constant<int, kInNorm>{});
  return hipGetLastError();
}

hipError_t launch_gemv_bf16(int64_t n, int k, const void* w, int64_t ws, const void* x, void* y,
                            hipStream_t s) {
  const int64_t grid = (n + kPlainRows - 1) / kPlainRows;
  hipLaunchKernelGGL(gemv_bf16_kernel, dim3((unsigned)grid), dim3(64 * kPlainSplit), 0, s, n, k,
                     static_cast<const uint16_t*>(w), ws, static_cast<const uint16_t*>(x),
                     static_cast<uint16_t*>(y));
  return hipGetLastError();
}

}  // namespace lc
