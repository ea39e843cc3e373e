// LDS tiles of bf16 [rows x 128] for the d=128 MFMA kernels (gfx950).
//
// Layout: row-major, 256 bytes per row, no padding; the sixteen 16-byte
// chunks of row r are stored XOR-swizzled, logical chunk L at physical chunk
// L ^ swz(r).  gfx950's LDS has 64 banks of 4 bytes (256 bytes per cycle) and,
// as measured with the SQ_LDS_BANK_CONFLICT counter:
//   * ds_read_b128 serves 16 lanes per cycle, grouped by quads (4 lanes) with
//     the quad index of equal parity: lanes {0-3, 12-15, 20-27} together,
//     {4-11, 16-19, 28-31} together, and likewise in lanes 32-63;
//   * ds_read_b64_tr_b16 serves lanes 0-31 and lanes 32-63 in separate cycles.
// The MFMA reads of this file are: row reads (lane c of group g reads row c,
// logical chunk 4kk + g) and transposed reads (lanes of group g read rows
// 4g..4g+3, 32 bytes each, a chunk pair 2db, 2db+1).  swz maps rows 0-7 to
// chunks 0,2,..,14, rows 8-11 to 9,11,13,15 and rows 12-15 to 1,3,5,7, which
// makes every cycle of both patterns touch 16 distinct chunks (no conflicts).
//
// Tiles are filled with global_load_lds (16 bytes per lane, lane l lands at
// base + 16*l), so one wave instruction writes 4 whole rows and staging needs
// no VGPRs; each lane fetches the logical chunk its physical slot holds.
//
// Transposed operands come from the same tile through ds_read_b64_tr_b16.
// Within a 16-lane group, output lane c slot t receives element (c % 4) of the
// 8 bytes addressed by lane 4*t + c/4.  So if lane 4*t + q addresses row
// (row0 + t), columns (col0 + 4q .. +3), lane c receives
// X[row0 + t][col0 + c] for t = 0..3: the tile's columns are spread over the
// lanes and its rows over the four slots, i.e. the MFMA operand whose M/N
// index is the column and whose K index is the row.
#pragma once

#include "common.h"

namespace lc {
namespace t128 {

constexpr int kRowBytes = 256;

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ int swz(int r) {
  r &= 15;
  return (((r + 4 * (r >> 3)) & 7) << 1) | (r >> 3);
}

// LDS DMA: each lane copies 16 (dma_b128) or 4 (dma_b32) bytes from global
// memory to LDS address lds + 16 * lane (4 * lane); lds must be uniform.
// Issued from inline asm so that the compiler's wait insertion does not track
// it: it cannot tell which LDS buffer a DMA writes, and would put an
// s_waitcnt vmcnt(0) before every later LDS read, i.e. wait for a prefetch of
// the next tile before reading the current one.  Callers wait explicitly
// (wait_vmem, plus a barrier when several waves fill one tile) before reading
// the destination.
// LDS byte address of a pointer into a __shared__ array (pass the array
// itself or a constant offset into it, so that the cast folds to a constant;
// tiles are then addressed as that constant plus an offset).
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(lds_void*)p;
}

// A pointer the caller guarantees to be wave-uniform, as SGPRs (an "s" asm
// operand would otherwise receive a VGPR when uniformity is not provable).
__device__ __forceinline__ const void* uniform_ptr(const void* p) {
  const uint64_t v = (uint64_t)(uintptr_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (const void*)(uintptr_t)(((uint64_t)hi << 32) | lo);
}

// The LDS address (uniform) goes to M0 through the "{m0}" operand, so the
// compiler knows M0's value.  The compiler does not insert wait states for
// the instructions inside an asm statement, so s_nop 4 provides them: 5 for a
// VALU write of an SGPR (v_readfirstlane of the base or of M0) followed by a
// VMEM read of it, which also covers the 1 of an M0 write before an LDS DMA.
__device__ __forceinline__ void dma_b128(const void* g, uint32_t lds) {
  asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(g), "{m0}"(__builtin_amdgcn_readfirstlane(lds))
               : "memory");
}

// Same, from a uniform base plus a per-lane 32-bit byte offset.
__device__ __forceinline__ void dma_b128(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(off), "s"(uniform_ptr(base)), "{m0}"(__builtin_amdgcn_readfirstlane(lds))
               : "memory");
}

// Non-temporal forms (streaming data read once: L2 does not keep it).
__device__ __forceinline__ void dma_b128_nt(const void* g, uint32_t lds) {
  asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, off nt"
               :
               : "v"(g), "{m0}"(__builtin_amdgcn_readfirstlane(lds))
               : "memory");
}

__device__ __forceinline__ void dma_b128_nt(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, %1 nt"
               :
               : "v"(off), "s"(uniform_ptr(base)), "{m0}"(__builtin_amdgcn_readfirstlane(lds))
               : "memory");
}

__device__ __forceinline__ void dma_b32(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_nop 4\n\tglobal_load_lds_dword %0, %1"
               :
               : "v"(off), "s"(uniform_ptr(base)), "{m0}"(__builtin_amdgcn_readfirstlane(lds))
               : "memory");
}

// Direct global->LDS loader for tiles of ROWS rows of a [*, 128] bf16
// matrix (row stride `stride` elements), NW waves, one wave instruction per
// 4 rows.  The per-lane byte offsets inside a tile and the wave's LDS offset
// are computed once; a tile that lies fully inside the matrix is issued from
// a uniform base pointer plus those offsets, the last (partial) tile re-reads
// row nrows - 1 for rows past the end (finite data; callers mask those rows).
template <int ROWS, int NW>
struct RowLoader {
  static_assert(ROWS % (4 * NW) == 0, "4 rows per wave instruction");
  static constexpr int kInst = ROWS / (4 * NW);
  uint32_t off[kInst];  // byte offset of this lane's 16-byte chunk within a tile
  uint32_t wave_lds;    // LDS byte offset of this wave's first 4 rows (uniform)

  __device__ __forceinline__ void init(int64_t stride, int wave, int lane) {
#pragma unroll
    for (int i = 0; i < kInst; ++i) {
      const int r = (i * NW + wave) * 4 + (lane >> 4);
      off[i] = (uint32_t)(r * stride * 2 + 16 * ((lane & 15) ^ swz(r)));
    }
    wave_lds = __builtin_amdgcn_readfirstlane((uint32_t)wave * 4 * kRowBytes);
  }

  // lds: LDS byte address of the tile.  kTracked: issue through the compiler
  // builtin, whose DMA the compiler tracks (it then waits for the DMA before
  // any later LDS read); otherwise through the untracked form above, and the
  // caller waits.  kNt (untracked only): non-temporal loads, for a stream
  // that no other workgroup reads again.
  template <bool kTracked = false, bool kNt = false>
  __device__ __forceinline__ void load(const uint16_t* base, int64_t stride, int row0, int nrows,
                                       uint32_t lds, int wave, int lane) const {
    if (row0 + ROWS <= nrows) {
      const uint8_t* tb = reinterpret_cast<const uint8_t*>(base + (int64_t)row0 * stride);
#pragma unroll
      for (int i = 0; i < kInst; ++i) {
        const uint32_t dst = lds + wave_lds + i * NW * 4 * kRowBytes;
        if constexpr (kTracked)
          __builtin_amdgcn_global_load_lds(tb + off[i], (lds_void*)(uintptr_t)dst, 16, 0, 0);
        else if constexpr (kNt)
          dma_b128_nt(tb, off[i], dst);
        else
          dma_b128(tb, off[i], dst);
      }
    } else {
#pragma unroll
      for (int i = 0; i < kInst; ++i) {
        const int r = (i * NW + wave) * 4 + (lane >> 4);
        const int chunk = (lane & 15) ^ swz(r);
        int grow = row0 + r;
        grow = grow < nrows ? grow : nrows - 1;
        const uint16_t* g = base + (int64_t)grow * stride + chunk * 8;
        const uint32_t dst = lds + wave_lds + i * NW * 4 * kRowBytes;
        if constexpr (kTracked)
          __builtin_amdgcn_global_load_lds(g, (lds_void*)(uintptr_t)dst, 16, 0, 0);
        else if constexpr (kNt)
          dma_b128_nt(g, dst);
        else
          dma_b128(g, dst);
      }
    }
  }
};

// Direct load of 64 consecutive fp32 values (one wave instruction) to LDS
// byte address lds.  Entries at or beyond n re-read entry n - 1.
__device__ __forceinline__ void load_f32x64(const float* base, int i0, int n, uint32_t lds,
                                            int lane) {
  int i = i0 + lane;
  i = i < n ? i : n - 1;
  dma_b32(base, 4u * (uint32_t)i, lds);
}

// s_waitcnt vmcnt(0) through the builtin, so that the compiler's wait
// insertion knows every earlier vector memory load has completed here (it does
// not parse inline asm).  Immediate: vmcnt 0, expcnt 7, lgkmcnt 15.
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// s_waitcnt vmcnt(N): all but the N most recent vector memory operations
// (loads and stores alike; gfx9 reports their completion in issue order).
// vmcnt is 6 bits: 3:0 in bits 3:0 of the immediate, 5:4 in bits 15:14.
template <int N>
__device__ __forceinline__ void wait_vmem_but() {
  static_assert(N >= 0 && N < 64, "vmcnt immediate");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

// Byte offset of logical chunk `chunk` of tile row `r`.
__device__ __forceinline__ int row_chunk_off(int r, int chunk) {
  return r * kRowBytes + 16 * (chunk ^ swz(r));
}

// Per-lane byte offset for a transposed read of columns col0..col0+15 over
// rows row0 + 4g + t (t = slot): lane (4t + q) of group g addresses row
// row0 + 4g + t, columns col0 + 4q .. +3.  row0 must be a multiple of 16.
__device__ __forceinline__ int tr_off(int row0, int col0, int lane) {
  const int g = lane >> 4;
  const int i = lane & 15;
  const int r = row0 + 4 * g + (i >> 2);
  const int q = i & 3;
  const int col = col0 + 4 * q;
  return r * kRowBytes + 16 * ((col >> 3) ^ swz(r)) + 2 * (col & 7);
}

// Byte offset of a transposed read for the 32x32x16 A operand X^T (X a tile
// of this file; k index = tile row, m index = column), column block 0 and
// k-half p: lane l receives X[row(l/32, p, t)][l%32] in slot t, with
// row(h, p, t) = 4h + p + 2(t%2) + 8(t/2).  The four rows read in one cycle
// (lanes 0-31 or 32-63) then have distinct swz(r) / 4, so the 4 rows x 4
// chunks land on 16 distinct chunks (no bank conflict).  Column block dblk is
// offset ^ (64 * dblk) (the block index occupies chunk bits 2-3 alone); rows
// 16u .. 16u+15 are offset + 16u * kRowBytes (swz depends on r % 16).  A B
// operand built from 32x32 accumulators over the same rows must use the same
// order: k-step u, slot 4p + t <- element 8u' + 4(t/2) + 2(t%2) + p of the
// block holding rows 16u .. 16u+15 (u' = u % 2).
__device__ __forceinline__ int tr32_off(int p, int lane) {
  const int G = lane >> 4, i = lane & 15, t = i >> 2;
  const int col = 16 * (G & 1) + 4 * (i & 3);
  const int r = 4 * (G >> 1) + p + 2 * (t & 1) + 8 * (t >> 1);
  return r * kRowBytes + 16 * ((col >> 3) ^ swz(r)) + 2 * (col & 7);
}

__device__ __forceinline__ bf16x4 ds_read_tr(const uint8_t* p) {
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)p);
  return __builtin_bit_cast(bf16x4, v);
}

}  // namespace t128
}  // namespace lc
