// Global -> register -> LDS staging of one operand tile per K stage.
//
// Two source orientations exist:
//  * K-major: every tile row is a source row and K is contiguous inside it
//    (A in NN/NT, B in NT).  Lanes read 16-byte pieces, four or eight lanes
//    per row, so each load instruction covers whole 64/128-byte row segments.
//  * MN-major: every source row is one (packed) K index and the tile rows are
//    contiguous inside it (B in NN/TN, A in TN).  A lane reads an 8x8-byte
//    block with 8-byte loads and transposes it with v_perm_b32 so that every
//    tile row gets 8 K-contiguous bytes: a whole 16-value chunk after int4
//    widening, half a chunk for int8.
//
// Both write the chunk-major swizzled int8 layout described in shk_common.h.
// A stage's K window may be partial (ragged / masked K): `kvalid` counts the
// valid source K units (packed bytes for int4, values for int8) from the start
// of the stage, and `odd_tail` marks that the last valid int4 byte holds only
// its low nibble (the odd-length K of the ragged backward, ragged.py:734-739).
// Tile rows at or past `rows_valid` (per half for split tiles) read as zero.
// A stage is loaded on the vector fast path only when it is entirely in bounds
// and 8/16-byte aligned; otherwise (GUARDED stagers only) every byte is loaded
// with its own bounds check.
#pragma once

#include "shk_common.h"

namespace shk {

__device__ __forceinline__ uint8_t masked_byte(const uint8_t* p, bool valid, bool low_only) {
  uint8_t b = valid ? *p : (uint8_t)0;
  return low_only ? (uint8_t)(b & 0x0F) : b;
}

// Source rows of a (possibly split) tile: rows [0, HALF) come from base0,
// rows [HALF, ROWS) from base1 (the gate half of a fused [up|gate] tile).
struct RowSource {
  const uint8_t* base0;
  const uint8_t* base1;
  long ld;         // bytes between consecutive source rows
  int rows_valid;  // valid tile rows per half
};

template <int BITS, int ROWS, int BK, int NT, int HALF, bool GUARDED>
struct KMajorStager {
  static constexpr int SB = BK * BITS / 8;  // source bytes per row per stage
  static constexpr int PR = SB / 16;        // 16-byte pieces per row
  static constexpr int TOTAL = ROWS * PR;
  static constexpr int PT = (TOTAL + NT - 1) / NT;
  static_assert(SB % 16 == 0, "stage K width must cover whole 16-byte pieces");
  uint4 v[PT];

  // `src.base*` point at source row 0 of each half; `kbyte0` is the stage's
  // byte offset inside a row.
  __device__ __forceinline__ void load(const RowSource& src, long kbyte0, int kvalid,
                                       bool odd_tail, bool fast) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < PT; ++i) {
      const int idx = tid + NT * i;
      if (TOTAL % NT != 0 && idx >= TOTAL) break;
      const int row = idx / PR;
      const int q = idx % PR;
      const int hr = row < HALF ? row : row - HALF;
      const uint8_t* rp = (row < HALF ? src.base0 : src.base1) + (long)hr * src.ld + kbyte0 + 16 * q;
      if (fast) {
        v[i] = *reinterpret_cast<const uint4*>(rp);
      } else if constexpr (GUARDED) {
        const bool row_ok = hr < src.rows_valid;
        uint32_t w[4];
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          uint32_t x = 0;
#pragma unroll
          for (int b = 0; b < 4; ++b) {
            const int kb = 16 * q + 4 * d + b;
            const bool ok = row_ok && kb < kvalid;
            const bool low_only = (BITS == 4) && odd_tail && kb == kvalid - 1;
            x |= (uint32_t)masked_byte(rp + 4 * d + b, ok, low_only) << (8 * b);
          }
          w[d] = x;
        }
        v[i] = make_uint4(w[0], w[1], w[2], w[3]);
      }
    }
  }

  __device__ __forceinline__ void store(uint8_t* lds) const {
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < PT; ++i) {
      const int idx = tid + NT * i;
      if (TOTAL % NT != 0 && idx >= TOTAL) break;
      const int row = idx / PR;
      const int q = idx % PR;
      if constexpr (BITS == 4) {
        *reinterpret_cast<uint4*>(lds + lds_chunk_off<ROWS>(row, 2 * q)) = widen_chunk(v[i].x, v[i].y);
        *reinterpret_cast<uint4*>(lds + lds_chunk_off<ROWS>(row, 2 * q + 1)) = widen_chunk(v[i].z, v[i].w);
      } else {
        *reinterpret_cast<uint4*>(lds + lds_chunk_off<ROWS>(row, q)) = v[i];
      }
    }
  }
};

template <int BITS, int ROWS, int BK, int NT, int HALF, bool GUARDED>
struct MNMajorStager {
  // A unit is 8 source rows x 8 tile rows (64 bytes).  For int4 the 8 packed
  // rows widen to one whole 16-value chunk; for int8 they fill half a chunk.
  static constexpr int KR = 8;
  static constexpr int UPC = (BITS == 4) ? 1 : 2;   // units per chunk
  static constexpr int RG = (BK / 16) * UPC;        // unit rows per stage
  static constexpr int UNITS = RG * (ROWS / 8);
  static constexpr int UPT = (UNITS + NT - 1) / NT;
  static_assert(ROWS % 8 == 0 && HALF % 8 == 0, "tile rows come in groups of 8");
  uint2 v[UPT][KR];

  // `src.base*` point at column 0 of the tile's first source row for each
  // half (the column offset of the tile is already applied); `krow0` is the
  // stage's first source row.
  __device__ __forceinline__ void load(const RowSource& src, long krow0, int kvalid, bool odd_tail,
                                       bool fast) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < UPT; ++i) {
      const int u = tid + NT * i;
      if (UNITS % NT != 0 && u >= UNITS) break;
      const int rg = u % RG;
      const int cg = u / RG;
      const int trow = 8 * cg;
      const int hc = trow < HALF ? trow : trow - HALF;
      const uint8_t* cp = (trow < HALF ? src.base0 : src.base1) + hc;
      const long r0 = krow0 + (long)rg * KR;
      if (fast) {
#pragma unroll
        for (int r = 0; r < KR; ++r) v[i][r] = *reinterpret_cast<const uint2*>(cp + (r0 + r) * src.ld);
      } else if constexpr (GUARDED) {
#pragma unroll
        for (int r = 0; r < KR; ++r) {
          const int kr = rg * KR + r;
          const bool k_ok = kr < kvalid;
          const bool low_only = (BITS == 4) && odd_tail && kr == kvalid - 1;
          const uint8_t* rp = cp + (r0 + r) * src.ld;
          uint32_t w[2];
#pragma unroll
          for (int d = 0; d < 2; ++d) {
            uint32_t x = 0;
#pragma unroll
            for (int b = 0; b < 4; ++b) {
              const int c = 4 * d + b;
              const bool ok = k_ok && (hc + c) < src.rows_valid;
              x |= (uint32_t)masked_byte(rp + c, ok, low_only) << (8 * b);
            }
            w[d] = x;
          }
          v[i][r] = make_uint2(w[0], w[1]);
        }
      }
    }
  }

  __device__ __forceinline__ void store(uint8_t* lds) const {
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < UPT; ++i) {
      const int u = tid + NT * i;
      if (UNITS % NT != 0 && u >= UNITS) break;
      const int rg = u % RG;
      const int cg = u / RG;
      const int chunk = rg / UPC;
      const int half = (rg % UPC) * 8;
#pragma unroll
      for (int d = 0; d < 2; ++d) {
        uint32_t x0[4], x1[4];
        transpose4x4(d ? v[i][0].y : v[i][0].x, d ? v[i][1].y : v[i][1].x, d ? v[i][2].y : v[i][2].x,
                     d ? v[i][3].y : v[i][3].x, x0[0], x0[1], x0[2], x0[3]);
        transpose4x4(d ? v[i][4].y : v[i][4].x, d ? v[i][5].y : v[i][5].x, d ? v[i][6].y : v[i][6].x,
                     d ? v[i][7].y : v[i][7].x, x1[0], x1[1], x1[2], x1[3]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          uint8_t* dst = lds + lds_chunk_off<ROWS>(8 * cg + 4 * d + j, chunk) + half;
          if constexpr (BITS == 4) {
            *reinterpret_cast<uint4*>(dst) = widen_chunk(x0[j], x1[j]);
          } else {
            *reinterpret_cast<uint2*>(dst) = make_uint2(x0[j], x1[j]);
          }
        }
      }
    }
  }
};

// Selects the stager for an operand orientation.
template <int BITS, bool KMAJOR, int ROWS, int BK, int NT, int HALF, bool GUARDED>
struct StagerFor;
template <int BITS, int ROWS, int BK, int NT, int HALF, bool GUARDED>
struct StagerFor<BITS, true, ROWS, BK, NT, HALF, GUARDED> {
  using type = KMajorStager<BITS, ROWS, BK, NT, HALF, GUARDED>;
};
template <int BITS, int ROWS, int BK, int NT, int HALF, bool GUARDED>
struct StagerFor<BITS, false, ROWS, BK, NT, HALF, GUARDED> {
  using type = MNMajorStager<BITS, ROWS, BK, NT, HALF, GUARDED>;
};

}  // namespace shk
