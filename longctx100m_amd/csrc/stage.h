// Global -> register -> LDS staging of bf16 [rows x D] tiles for the MFMA
// kernels.  Loads are issued into registers one tile ahead (so HBM latency
// overlaps the current tile's MFMA work) and written to LDS after a barrier.
#pragma once

#include "common.h"

namespace lc {

// Row-major copy: LDS [ROWS][PITCH], 16-byte chunks (8 bf16 of one row).
// Rows at or beyond `nrows` are zero-filled.
template <int ROWS, int D, int PITCH, int NT>
struct RowStager {
  static constexpr int kChunksPerRow = D / 8;
  static constexpr int kChunks = ROWS * kChunksPerRow;
  static constexpr int kPerThread = (kChunks + NT - 1) / NT;
  uint4 r[kPerThread];

  __device__ __forceinline__ void load(const uint16_t* base, int64_t stride, int row0, int nrows,
                                       int tid) {
#pragma unroll
    for (int i = 0; i < kPerThread; ++i) {
      const int idx = i * NT + tid;
      const int row = idx / kChunksPerRow;
      const int ch = idx % kChunksPerRow;
      uint4 val = make_uint4(0u, 0u, 0u, 0u);
      if ((kChunks % NT == 0 || idx < kChunks) && row0 + row < nrows)
        val = *reinterpret_cast<const uint4*>(base + (int64_t)(row0 + row) * stride + ch * 8);
      r[i] = val;
    }
  }

  __device__ __forceinline__ void store(uint16_t* lds, int tid) const {
#pragma unroll
    for (int i = 0; i < kPerThread; ++i) {
      const int idx = i * NT + tid;
      if (kChunks % NT == 0 || idx < kChunks) {
        const int row = idx / kChunksPerRow;
        const int ch = idx % kChunksPerRow;
        *reinterpret_cast<uint4*>(lds + row * PITCH + ch * 8) = r[i];
      }
    }
  }
};

// Transposed copy: LDS [D][PITCH] holding column d of the tile as a row, so a
// lane can read 4 consecutive tile rows of one head-dim index with one 8-byte
// LDS read.  Each thread moves an (8 rows x 4 dims) block: eight 8-byte global
// loads along d, a register transpose with v_perm_b32, four 16-byte LDS stores.
template <int ROWS, int D, int PITCH, int NT>
struct TransStager {
  static constexpr int kDGroups = D / 4;
  static constexpr int kUnits = (ROWS / 8) * kDGroups;
  static_assert(kUnits <= NT, "one (8 x 4) unit per thread");
  uint2 r[8];

  __device__ __forceinline__ void load(const uint16_t* base, int64_t stride, int row0, int nrows,
                                       int tid) {
    if (tid < kUnits) {
      const int dg = tid % kDGroups;
      const int rg = tid / kDGroups;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int row = row0 + rg * 8 + k;
        uint2 val = make_uint2(0u, 0u);
        if (row < nrows) val = *reinterpret_cast<const uint2*>(base + (int64_t)row * stride + dg * 4);
        r[k] = val;
      }
    }
  }

  __device__ __forceinline__ void store(uint16_t* lds, int tid) const {
    if (tid < kUnits) {
      const int dg = tid % kDGroups;
      const int rg = tid / kDGroups;
#pragma unroll
      for (int dd = 0; dd < 4; ++dd) {
        const uint32_t sel = (dd & 1) ? kSelHiHalves : kSelLoHalves;
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t lo = (dd < 2) ? r[2 * i].x : r[2 * i].y;
          const uint32_t hi = (dd < 2) ? r[2 * i + 1].x : r[2 * i + 1].y;
          w[i] = perm_b32(hi, lo, sel);
        }
        *reinterpret_cast<uint4*>(lds + (dg * 4 + dd) * PITCH + rg * 8) =
            make_uint4(w[0], w[1], w[2], w[3]);
      }
    }
  }
};

}  // namespace lc
