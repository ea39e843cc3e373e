// Split-KV decode attention for head_dim 128 on bf16 MFMA (gfx950): a few new
// query tokens against a long KV cache.
//
// Same semantics and outputs as the blockwise forward of one ring hop
// (rust/longctx100m-model/src/ring_attention.rs:15-106 and the finalize of
// :227): normalised o [B, Nq, Hq, D] fp32 and the row statistics m, l.  The
// work split is the decode one: each (batch, KV head) has R = Nq * group
// query rows (group = Hq / Hkv, R <= 16: one MFMA column block), so the
// key range is split over S one-wave workgroups that stream the cache, each
// leaving a partial (o, m, l) in the workspace; decode_merge_kernel combines
// the S partials by log-sum-exp.
//
// Per wave: Q^T of the R rows in VGPRs (B operand, rows >= R are zero);
// 32-key tiles: K straight into VGPRs (the A operand of S^T = K Q^T wants each
// lane's 8 dims of one key, which a 16-byte global load gives), V
// double-buffered in LDS by direct global->LDS loads (tile128.h layout), both
// one tile ahead; S^T = K Q^T, exact online softmax per row in the log2
// domain, O^T += V^T P^T with V^T from transposed LDS reads.
#include "common.h"
#include "kernels.h"
#include "tile128.h"

#include <mutex>
#include <type_traits>

namespace lc {

// Workspace of lc_attn_decode_static: split partials of the decode kernel,
// read back by the merge kernel.  Every partial is written before it is read,
// so nothing here needs clearing between calls.  Each device holds its own
// copy from the library's load until the process ends, and every call on a
// device shares it (calls that overlap on one device race).  Host code never
// passes `scratch` itself to a kernel: its host-side name is not a device
// address; decode_static_scratch() returns the device address.
static __device__ __align__(256) uint8_t scratch[kDecodeStaticScratchBytes];

namespace {

constexpr int D = 128;
constexpr int TK = 32;  // keys per tile
// V tiles in LDS per workgroup: the one in use and one in flight.  With K
// staged in LDS as well, one C4 layer (262,144 keys, 8 KV heads) read the
// cache at 4.72-5.24 TB/s (2-5 stages); K in VGPRs (the LDS round trip costs
// SIMD cycles per byte) and eight one-wave workgroups per CU (the register
// limit of two waves per SIMD) read it at 5.68 TB/s.
constexpr int kStages = 2;
constexpr int KS = D / 32;
constexpr int DB = D / 16;
constexpr int kTileBytes = TK * t128::kRowBytes;

struct DecodeArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  float* o_part;  // [S][B*Nq*Hq][D]
  float* m_part;  // [S][B*Nq*Hq]
  float* l_part;
  int Nq, Nk, Hq, Hkv, group, rows, S, chunk;  // chunk: keys per split (multiple of TK)
  int64_t prows;                               // B * Nq * Hq: rows of one split's partial
  int64_t q_pos0, k_pos0, valid;
  int causal;
  float sl2;  // scale * log2(e)
};

__global__ __launch_bounds__(64) void decode128_kernel(DecodeArgs a) {
  __shared__ __attribute__((aligned(1024))) uint8_t vbuf[kStages][kTileBytes];

  const int lane = threadIdx.x;
  const int c = lane & 15;
  const int g = lane >> 4;
  const int s = blockIdx.x % a.S;
  const int bh = blockIdx.x / a.S;
  const int hk = bh % a.Hkv;
  const int b = bh / a.Hkv;

  const int64_t ks = (int64_t)a.Hkv * D;
  const uint16_t* kbase = a.k + (int64_t)b * a.Nk * ks + (int64_t)hk * D;
  const uint16_t* vbase = a.v + (int64_t)b * a.Nk * ks + (int64_t)hk * D;

  // Keys any row can see, then this split's share of them.
  int64_t kend = a.Nk;
  if (a.causal) kend = min(kend, a.q_pos0 + a.Nq - a.k_pos0);
  kend = min(kend, a.valid - a.k_pos0);
  const int64_t kb0 = (int64_t)s * a.chunk;
  const int64_t kb1 = min(kb0 + a.chunk, kend);
  const int ntiles = kb1 > kb0 ? (int)((kb1 - kb0 + TK - 1) / TK) : 0;

  t128::RowLoader<TK, 1> ld;
  ld.init(ks, 0, lane);
  auto issue = [&](int j) {  // V tile j into stage j % kStages
    const int st = j % kStages;
    ld.load<false, true>(vbase, ks, (int)(kb0 + (int64_t)j * TK), a.Nk,
                         t128::lds_addr(vbuf) + st * kTileBytes, 0, lane);
  };
  // K tile j straight into VGPRs (no LDS round trip): lane (c, g) holds key
  // 16 mb + c of the tile, dims 32 kk + 8 g, the A operand of S^T = K Q^T.
  // The cache is read once per step, so K and V are loaded non-temporally
  // (5.77 -> 6.58 TB/s per layer against the same kernel with default loads).
  auto kload = [&](int j, bf16x8 (&kr)[2][4]) {
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      int64_t row = kb0 + (int64_t)j * TK + 16 * mb + c;
      row = row < a.Nk ? row : a.Nk - 1;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
        kr[mb][kk] = __builtin_nontemporal_load(
            reinterpret_cast<const bf16x8*>(kbase + row * ks + 32 * kk + 8 * g));
    }
  };

  // Row c of this (batch, KV head): query head hk*group + c / Nq, query c % Nq.
  const bool row_ok = c < a.rows;
  const int qi = row_ok ? c % a.Nq : 0;
  const int qh = hk * a.group + (row_ok ? c / a.Nq : 0);
  const int64_t qpos = a.q_pos0 + qi;
  bf16x8 qreg[KS];
  {
    const uint16_t* qrow = a.q + (((int64_t)b * a.Nq + qi) * a.Hq + qh) * D;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      qreg[kk] = *reinterpret_cast<const bf16x8*>(qrow + 32 * kk + 8 * g);
      if (!row_ok) qreg[kk] = bf16x8{};
    }
  }

  // Q is in VGPRs from here on (the compiler, which cannot count the tile
  // loads below, would otherwise wait for every load before each use of Q).
  t128::wait_vmem();
  bf16x8 kra[2][KS], krb[2][KS];
  if (ntiles > 0) {
    issue(0);
    kload(0, kra);
  }

  int voff[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) voff[db] = t128::tr_off(0, 16 * db, lane);

  f32x4 o[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) o[db] = f32x4{0.f, 0.f, 0.f, 0.f};
  float mrow = -INFINITY;  // running max of this lane's row (log2 units)
  float lsum = 0.f;        // lane-partial sum of p

  // Tile j: wait for V(j) in LDS and K(j) in VGPRs (both issued at tile j - 1),
  // issue V(j + 1) into the other stage (read by tile j - 1, done) and
  // K(j + 1) into the other register set, then compute tile j.
  auto tile = [&](int j, bf16x8 (&kc)[2][KS], bf16x8 (&kn)[2][KS]) {
    t128::wait_vmem();
    if (j + 1 < ntiles) {
      issue(j + 1);
      kload(j + 1, kn);
    }
    const uint8_t* vt = vbuf[j % kStages];
    const int64_t key0 = kb0 + (int64_t)j * TK;

    f32x4 sc[2];
    sc[0] = sc[1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) sc[mb] = mfma16x16x32(kc[mb][kk], qreg[kk], sc[mb]);
    }
    // Mask: past the split / cache end, valid_length, causal (per row).
    const int64_t kmax = kb1 - key0;  // keys of this tile inside the split
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int kr = 16 * mb + 4 * g + i;
        const int64_t kp = a.k_pos0 + key0 + kr;
        const bool bad = kr >= kmax || (a.causal && kp > qpos);
        sc[mb][i] = bad ? -INFINITY : sc[mb][i] * a.sl2;
      }
    float mx = fmaxf(fmaxf(fmaxf(sc[0][0], sc[0][1]), fmaxf(sc[0][2], sc[0][3])),
                     fmaxf(fmaxf(sc[1][0], sc[1][1]), fmaxf(sc[1][2], sc[1][3])));
    mx = group4_max(mx);
    if (mx > mrow) {
      const float alpha = fast_exp2(mrow - mx);  // mrow = -inf: 0
      lsum *= alpha;
#pragma unroll
      for (int db = 0; db < DB; ++db) o[db] *= alpha;
      mrow = mx;
    }
    const float muse = mrow == -INFINITY ? 0.f : mrow;  // no key yet: p = 0
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p = fast_exp2(sc[mb][i] - muse);
        lsum += p;
        sc[mb][i] = p;
      }
    const bf16x8 pb = pack_bf16x8(sc[0], sc[1]);
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      const uint8_t* p = vt + voff[db];
      const bf16x8 va = concat_bf16x4(t128::ds_read_tr(p), t128::ds_read_tr(p + 16 * t128::kRowBytes));
      o[db] = mfma16x16x32(va, pb, o[db]);
    }
  };
  for (int j = 0; j < ntiles; j += 2) {
    tile(j, kra, krb);
    if (j + 1 < ntiles) tile(j + 1, krb, kra);
  }

  // Partial of this split: normalised o, m (natural log), l.
  const float lt = group4_sum(lsum);
  if (row_ok) {
    const int64_t row = ((int64_t)b * a.Nq + qi) * a.Hq + qh;
    const int64_t prow = (int64_t)s * a.prows + row;
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    float* orow = a.o_part + prow * D;
#pragma unroll
    for (int db = 0; db < DB; ++db)
      *reinterpret_cast<f32x4*>(orow + 16 * db + 4 * g) = o[db] * inv;
    if (g == 0) {
      a.m_part[prow] = mrow == -INFINITY ? -INFINITY : mrow * kLn2;
      a.l_part[prow] = lt;
    }
  }
}

// Log-sum-exp merge of the S split partials of each row (b, i, h) =
// ((b * Nq) + i) * Hq + h of o.  A decode step has only B * Nq * Hq rows, so
// each row's D dims are split over kMergeParts 1024-thread workgroups (four
// per row: 128 workgroups for the 32 rows of a GQA 32/8 token) and every
// chain is short: one round of statistics loads (each thread holds the (m, l)
// of up to four splits; every workgroup of a row forms all split weights),
// the max M and the sum L of the weights w_s = l_s * exp(m_s - M) reduced by
// wave shuffles and one LDS exchange each, then thread (d, g) of the
// workgroup's D / kMergeParts dims sums w_s * o_s[d] over the splits
// s = g mod kMergeGroups and the group sums meet in LDS.  m and l (written by
// the first workgroup of the row) use the [B, Hq, Nq] layout of the
// statistics.
constexpr int kMergeMaxSplits = 4096;
constexpr int kMergeThreads = 1024;
constexpr int kMergePer = kMergeMaxSplits / kMergeThreads;  // splits per thread
constexpr int kMergeWaves = kMergeThreads / 64;
constexpr int kMergeParts = 4;                        // workgroups per row
constexpr int kMergeDims = D / kMergeParts;           // dims per workgroup
constexpr int kMergeGroups = kMergeThreads / kMergeDims;

__global__ __launch_bounds__(kMergeThreads) void decode_merge_kernel(
    int64_t nrows, int S, int Nq, int Hq, const float* o_part, const float* m_part,
    const float* l_part, float* o, float* m, float* l) {
  __shared__ float w[kMergeMaxSplits];
  __shared__ float wave_max[kMergeWaves];
  __shared__ float wave_sum[kMergeWaves];
  __shared__ float part[kMergeThreads];
  const int t = threadIdx.x;
  const int wave = t >> 6;
  const int64_t row = blockIdx.x / kMergeParts;
  const int d0 = (int)(blockIdx.x % kMergeParts) * kMergeDims;
  float ms[kMergePer], ls[kMergePer];
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < kMergePer; ++i) {
    const int sp = t + i * kMergeThreads;
    ms[i] = sp < S ? m_part[(int64_t)sp * nrows + row] : -INFINITY;
    ls[i] = sp < S ? l_part[(int64_t)sp * nrows + row] : 0.f;
    mx = fmaxf(mx, ms[i]);
  }
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  if ((t & 63) == 0) wave_max[wave] = mx;
  __syncthreads();
  float M = -INFINITY;
#pragma unroll
  for (int i = 0; i < kMergeWaves; ++i) M = fmaxf(M, wave_max[i]);
  float lsum = 0.f;
#pragma unroll
  for (int i = 0; i < kMergePer; ++i) {
    const int sp = t + i * kMergeThreads;
    const float ws = (M == -INFINITY || !(ls[i] > 0.f)) ? 0.f : ls[i] * expf(ms[i] - M);
    if (sp < S) w[sp] = ws;
    lsum += ws;
  }
  for (int off = 32; off > 0; off >>= 1) lsum += __shfl_xor(lsum, off, 64);
  if ((t & 63) == 0) wave_sum[wave] = lsum;
  __syncthreads();  // w[] and the wave sums are complete
  float L = 0.f;
#pragma unroll
  for (int i = 0; i < kMergeWaves; ++i) L += wave_sum[i];
  // weighted sum of the partial outputs: thread (d, g) over splits g, g + kMergeGroups, ...
  const int dd = t % kMergeDims;
  const int d = d0 + dd;
  const int g = t / kMergeDims;
  float acc = 0.f;  // partials of empty splits are zeros with zero weight
  const float* op = o_part + row * D + d;
  const int64_t sstride = (int64_t)nrows * D;
#pragma unroll 4
  for (int sp = g; sp < S; sp += kMergeGroups) acc = fmaf(w[sp], op[(int64_t)sp * sstride], acc);
  part[t] = acc;
  __syncthreads();
  if (g == 0) {
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < kMergeGroups; ++i) sum += part[i * kMergeDims + dd];
    const float inv = L > 0.f ? 1.f / L : 0.f;
    o[row * D + d] = sum * inv;
  }
  if (d0 != 0) return;  // the row's statistics come from its first workgroup
  if (t == 0) {
    const int h = (int)(row % Hq);
    const int64_t bi = row / Hq;
    const int64_t si = (bi / Nq * Hq + h) * Nq + bi % Nq;
    m[si] = L > 0.f ? M : -INFINITY;
    l[si] = L;
  }
}

}  // namespace

// Splits per (batch, KV head): as many one-wave workgroups as fit the CUs'
// LDS (kStages tiles each), at least two tiles per split.
int decode_splits(const Problem& p) {
  constexpr int kLdsPerCu = (160 * 1024) / (kStages * kTileBytes);
  constexpr int kPerCu = kLdsPerCu < 8 ? kLdsPerCu : 8;  // two waves per SIMD (registers)
  const int64_t tiles = ((int64_t)p.Nk + TK - 1) / TK;
  const int64_t want = (kPerCu * 256 + (int64_t)p.B * p.Hkv - 1) / ((int64_t)p.B * p.Hkv);
  int64_t s = want < 1 ? 1 : want;
  const int64_t max_s = tiles / 2 < 1 ? 1 : tiles / 2;
  if (s > max_s) s = max_s;
  if (s > kMergeMaxSplits) s = kMergeMaxSplits;
  return (int)s;
}

bool decode_supported(const Problem& p) {
  return p.dtype == 1 && !p.precise && p.D == D && (int64_t)p.Nq * (p.Hq / p.Hkv) <= 16;
}

size_t decode_workspace_bytes(const Problem& p) {
  const int64_t rows = (int64_t)p.B * p.Nq * p.Hq;
  const int64_t S = decode_splits(p);
  return (size_t)(S * rows * D * 4 + 2 * S * rows * 4);
}

hipError_t decode_static_scratch(hipStream_t st, void** ptr) {
  constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static void* addr[kMaxDevices] = {};
  // The kernels run on the stream's device, so the array must be that
  // device's copy: a null stream means the current device.
  int cur = 0;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess) return e;
  int dev = cur;
  if (st != nullptr) {
    hipDevice_t sd = 0;
    e = hipStreamGetDevice(st, &sd);
    if (e != hipSuccess) return e;
    dev = (int)sd;
  }
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(mu);
  if (addr[dev] == nullptr) {
    // hipGetSymbolAddress resolves the symbol on the current device: make
    // the stream's device current for the lookup, then restore the caller's.
    if (dev != cur && (e = hipSetDevice(dev)) != hipSuccess) return e;
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (dev != cur) {
      const hipError_t r = hipSetDevice(cur);
      if (e == hipSuccess) e = r;
    }
    if (e != hipSuccess) return e;
    addr[dev] = p;
  }
  *ptr = addr[dev];
  return hipSuccess;
}

hipError_t launch_decode128(const Problem& p, const void* q, const void* k, const void* v,
                            float* o, float* m, float* l, void* ws, hipStream_t st) {
  if (!decode_supported(p)) return hipErrorInvalidValue;
  const int S = decode_splits(p);
  const int64_t rows = (int64_t)p.B * p.Nq * p.Hq;
  float* o_part = static_cast<float*>(ws);
  float* m_part = o_part + (int64_t)S * rows * D;
  float* l_part = m_part + (int64_t)S * rows;
  DecodeArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.o_part = o_part;
  a.m_part = m_part;
  a.l_part = l_part;
  a.Nq = p.Nq;
  a.Nk = p.Nk;
  a.Hq = p.Hq;
  a.Hkv = p.Hkv;
  a.group = p.Hq / p.Hkv;
  a.rows = p.Nq * a.group;
  a.S = S;
  a.prows = rows;
  const int64_t per = ((int64_t)p.Nk + S - 1) / S;
  a.chunk = (int)((per + TK - 1) / TK * TK);
  a.q_pos0 = p.q_pos0;
  a.k_pos0 = p.k_pos0;
  a.valid = p.valid;
  a.causal = p.causal ? 1 : 0;
  a.sl2 = p.scale * kLog2e;
  hipLaunchKernelGGL(decode128_kernel, dim3((unsigned)(S * p.Hkv * p.B)), dim3(64), 0, st, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(decode_merge_kernel, dim3((unsigned)(rows * kMergeParts)), dim3(kMergeThreads), 0, st,
                     rows, S, p.Nq, p.Hq, o_part, m_part, l_part, o, m, l);
  return hipGetLastError();
}

}  // namespace lc
