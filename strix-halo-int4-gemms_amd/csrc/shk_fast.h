// Software-pipelined MFMA engine for tile-multiple shapes (the dense GEMMs).
//
// Operands are read with buffer loads: a buffer resource (SGPRs) is built at
// the tile's first byte, every lane keeps the byte offset of its pieces for
// the whole K loop, and the stage's K position travels in the scalar offset,
// so a K stage costs no address arithmetic.  LDS read and write offsets are
// likewise computed once; the two stage buffers are addressed by immediates.
//
// A K stage (S = BK/MK MFMA steps) is one basic block ended by the stage's
// only barrier: each step reads its fragments from the current buffer and
// issues its MFMAs; the first step also issues the widening / transposing LDS
// writes of the prefetched stage k+1 into the other buffer, the last step the
// buffer loads of stage k+2, so the scheduler interleaves both with MFMAs.
#pragma once

#include "shk_gemm.h"


namespace shk {

typedef __amdgpu_buffer_rsrc_t rsrc_t;

// Raw (stride 0) buffer resource over [base, base + bytes); loads past the end
// return zero.
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, unsigned long long bytes) {
  const unsigned n = bytes > 0xFFFFFFFFull ? 0xFFFFFFFFu : (unsigned)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)n, 0x00020000);
}

__device__ __forceinline__ uint4 bload128(rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}
__device__ __forceinline__ uint2 bload64(rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0));
}

// K-major operand: tile row r is source row r (rows of the gate half are
// shifted by `gate_rows` source rows); each lane stages 16-byte pieces.
template <int BITS, int ROWS, int BK, int NT, int HALF>
struct FastKMajor {
  static constexpr int SB = BK * BITS / 8;
  static constexpr int PR = SB / 16;
  static constexpr int TOTAL = ROWS * PR;
  static constexpr int PT = TOTAL >= NT ? TOTAL / NT : 1;
  static constexpr bool PARTIAL = TOTAL < NT;  // some threads stage nothing
  static constexpr int ROWS_PER_I = NT / PR;
  static_assert(PARTIAL ? (TOTAL % 64 == 0) : (TOTAL % NT == 0), "pieces must spread evenly over the waves");
  static_assert(NT % PR == 0 && (PT == 1 || ROWS_PER_I % 8 == 0), "row stride per piece must keep the swizzle");
  uint4 v[PT];
  uint32_t voff[PT];
  uint32_t wbase[2];  // LDS byte offset of this lane's first chunk(s) in a stage buffer

  __device__ __forceinline__ void init(uint32_t ld, uint32_t gate_rows) {
    const int tid = threadIdx.x;
    const int row0 = tid / PR;
    const int q = tid % PR;
#pragma unroll
    for (int i = 0; i < PT; ++i) {
      const int row = row0 + ROWS_PER_I * i;
      const uint32_t src_row = row < HALF ? (uint32_t)row : (uint32_t)(row - HALF) + gate_rows;
      voff[i] = src_row * ld + 16u * q;
    }
    if constexpr (BITS == 4) {
      wbase[0] = lds_chunk_off<ROWS>(row0, 2 * q);
      wbase[1] = lds_chunk_off<ROWS>(row0, 2 * q + 1);
    } else {
      wbase[0] = lds_chunk_off<ROWS>(row0, q);
      wbase[1] = 0;
    }
  }
  __device__ __forceinline__ void load(rsrc_t r, uint32_t soff) {
    if (PARTIAL && (int)threadIdx.x >= TOTAL) return;
#pragma unroll
    for (int i = 0; i < PT; ++i) v[i] = bload128(r, voff[i], soff);
  }
  __device__ __forceinline__ void store(uint8_t* lds) const {
    if (PARTIAL && (int)threadIdx.x >= TOTAL) return;
#pragma unroll
    for (int i = 0; i < PT; ++i) {
      const uint32_t step = 16u * ROWS_PER_I * i;
      if constexpr (BITS == 4) {
        *reinterpret_cast<uint4*>(lds + wbase[0] + step) = widen_chunk(v[i].x, v[i].y);
        *reinterpret_cast<uint4*>(lds + wbase[1] + step) = widen_chunk(v[i].z, v[i].w);
      } else {
        *reinterpret_cast<uint4*>(lds + wbase[0] + step) = v[i];
      }
    }
  }
};

// MN-major operand: source row = K index, tile rows contiguous; units of
// 8 source rows x 8 tile rows, transposed with v_perm_b32.
template <int BITS, int ROWS, int BK, int NT, int HALF>
struct FastMNMajor {
  static constexpr int UPC = (BITS == 4) ? 1 : 2;
  static constexpr int RG = (BK / 16) * UPC;
  static constexpr int UNITS = RG * (ROWS / 8);
  static constexpr int UPT = UNITS >= NT ? UNITS / NT : 1;
  static constexpr bool PARTIAL = UNITS < NT;  // some threads stage nothing
  static constexpr int CG_PER_I = NT / RG;
  static_assert(PARTIAL || UNITS % NT == 0, "units must spread evenly over the threads");
  static_assert(NT % RG == 0, "a thread keeps one unit row");
  uint2 v[UPT][8];
  uint32_t voff[UPT];
  uint32_t wofs[8];  // LDS byte offsets of this lane's 8 tile rows in unit 0
  uint32_t ld;

  __device__ __forceinline__ void init(uint32_t ld_, uint32_t gate_cols) {
    ld = ld_;
    const int tid = threadIdx.x;
    const int rg = tid % RG;
    const int cg0 = tid / RG;
#pragma unroll
    for (int i = 0; i < UPT; ++i) {
      const int trow = 8 * (cg0 + CG_PER_I * i);
      const uint32_t col = trow < HALF ? (uint32_t)trow : (uint32_t)(trow - HALF) + gate_cols;
      voff[i] = (uint32_t)(rg * 8) * ld + col;
    }
    const int chunk = rg / UPC;
    const int half = (rg % UPC) * 8;
#pragma unroll
    for (int p = 0; p < 8; ++p) wofs[p] = lds_chunk_off<ROWS>(8 * cg0 + p, chunk) + half;
  }
  // `krow` is the stage's first source row.
  __device__ __forceinline__ void load(rsrc_t r, uint32_t krow) {
    if (PARTIAL && (int)threadIdx.x >= UNITS) return;
#pragma unroll
    for (int i = 0; i < UPT; ++i)
#pragma unroll
      for (int rr = 0; rr < 8; ++rr) v[i][rr] = bload64(r, voff[i], (krow + rr) * ld);
  }
  __device__ __forceinline__ void store(uint8_t* lds) const {
    if (PARTIAL && (int)threadIdx.x >= UNITS) return;
#pragma unroll
    for (int i = 0; i < UPT; ++i) {
      const uint32_t step = 16u * 8 * CG_PER_I * i;
#pragma unroll
      for (int d = 0; d < 2; ++d) {
        uint32_t x0[4], x1[4];
        transpose4x4(d ? v[i][0].y : v[i][0].x, d ? v[i][1].y : v[i][1].x, d ? v[i][2].y : v[i][2].x,
                     d ? v[i][3].y : v[i][3].x, x0[0], x0[1], x0[2], x0[3]);
        transpose4x4(d ? v[i][4].y : v[i][4].x, d ? v[i][5].y : v[i][5].x, d ? v[i][6].y : v[i][6].x,
                     d ? v[i][7].y : v[i][7].x, x1[0], x1[1], x1[2], x1[3]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          uint8_t* dst = lds + wofs[4 * d + j] + step;
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

template <int BITS, bool KMAJOR, int ROWS, int BK, int NT, int HALF>
struct FastStagerFor;
template <int BITS, int ROWS, int BK, int NT, int HALF>
struct FastStagerFor<BITS, true, ROWS, BK, NT, HALF> {
  using type = FastKMajor<BITS, ROWS, BK, NT, HALF>;
  static constexpr bool KM = true;
};
template <int BITS, int ROWS, int BK, int NT, int HALF>
struct FastStagerFor<BITS, false, ROWS, BK, NT, HALF> {
  using type = FastMNMajor<BITS, ROWS, BK, NT, HALF>;
  static constexpr bool KM = false;
};

// Fragments of one MFMA step.
template <class C>
struct Frags {
  using T = typename std::conditional<C::MK == 64, v4i, v2i>::type;
  T y[C::FM];
  T x[C::FN2];
};

template <class C>
struct FastEngine {
  using AS = typename FastStagerFor<C::BITS, C::A_KMAJOR, C::BM, C::BK, C::NT, C::BM>::type;
  using BS = typename FastStagerFor<C::BITS, C::B_KMAJOR, C::BROWS, C::BK, C::NT, C::BHALF>::type;
  static constexpr int S = C::BK / C::MK;                 // MFMA steps per stage
  static constexpr int NPAT = 128 / C::MK;                // distinct XOR patterns of a step
  static constexpr int CPS = C::MK / 16;                  // chunks per step

  v4i acc[C::FM][C::FN2];
  Frags<C> f;
  AS sa;
  BS sb;
  rsrc_t ra, rb;
  uint32_t ard[NPAT], brd[NPAT];  // fragment read offsets per step pattern
  int lane, wm, wn;

  __device__ __forceinline__ void init_reads() {
    lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    wm = wave % C::WM;
    wn = wave / C::WM;
    const int l15 = lane & 15;
    const int g = lane >> 4;
#pragma unroll
    for (int p = 0; p < NPAT; ++p) {
      // step s with s % NPAT == p reads chunk CPS*s + g' (g' = lane's chunk in the step)
      int chunk, half;
      if (C::MK == 64) {
        chunk = CPS * p + g;
        half = 0;
      } else {
        chunk = CPS * p + (g >> 1);
        half = (g & 1) * 8;
      }
      const int arow = wm * C::TM + l15;
      const int brow = wn * C::TN + l15;
      ard[p] = lds_chunk_off<C::BM>(arow, chunk) + half;
      brd[p] = lds_chunk_off<C::BROWS>(brow, chunk) + half;
    }
#pragma unroll
    for (int i = 0; i < C::FM; ++i)
#pragma unroll
      for (int j = 0; j < C::FN2; ++j) acc[i][j] = v4i{0, 0, 0, 0};
  }

  // Byte offset of step s's chunk plane beyond the pattern's base offset.
  template <int ROWS>
  static constexpr uint32_t step_plane(int s) {
    return (uint32_t)((CPS * (s - s % NPAT)) * ROWS * 16);
  }

  __device__ __forceinline__ void read_frags(const uint8_t* la, const uint8_t* lb, int s, Frags<C>& fr) const {
    using T = typename Frags<C>::T;
    const int p = s % NPAT;
    const uint8_t* pa = la + ard[p] + step_plane<C::BM>(s);
    const uint8_t* pb = lb + brd[p] + step_plane<C::BROWS>(s);
#pragma unroll
    for (int i = 0; i < C::FM; ++i) fr.y[i] = *reinterpret_cast<const T*>(pa + 256 * i);
#pragma unroll
    for (int j = 0; j < C::FN2; ++j) {
      const uint32_t o = j < C::FN ? 256u * j : 16u * C::BHALF + 256u * (j - C::FN);
      fr.x[j] = *reinterpret_cast<const T*>(pb + o);
    }
  }

  // MFMAs of one step over fragment rows [I0, I1).
  template <int I0 = 0, int I1 = C::FM>
  __device__ __forceinline__ void mma(const Frags<C>& fr) {
#pragma unroll
    for (int i = I0; i < I1; ++i)
#pragma unroll
      for (int j = 0; j < C::FN2; ++j) {
        if constexpr (C::MK == 64) acc[i][j] = mfma64(fr.x[j], fr.y[i], acc[i][j]);
        else acc[i][j] = mfma32(fr.x[j], fr.y[i], acc[i][j]);
      }
  }

  __device__ __forceinline__ void zero_acc() {
#pragma unroll
    for (int i = 0; i < C::FM; ++i)
#pragma unroll
      for (int j = 0; j < C::FN2; ++j) acc[i][j] = v4i{0, 0, 0, 0};
  }

  __device__ __forceinline__ int out_row(int i) const { return wm * C::TM + 16 * i + (lane & 15); }
  __device__ __forceinline__ int out_col(int j) const {
    return wn * C::TN + 16 * (j < C::FN ? j : j - C::FN) + 4 * (lane >> 4);
  }
  __device__ __forceinline__ int true_acc(int v) const { return v >> C::ACC_SHIFT; }

  __device__ __forceinline__ void setup(const DenseArgs& p, int m0, int n0, int gate) {
    const unsigned long long kbytes = (unsigned long long)p.K * C::BITS / 8;
    if (C::A_KMAJOR) {  // A [M, kbytes]
      ra = make_rsrc(p.a + (long)m0 * p.lda, (unsigned long long)(p.M - m0) * p.lda);
    } else {            // A [kbytes, M]
      ra = make_rsrc(p.a + m0, kbytes * p.M - m0);
    }
    sa.init((uint32_t)p.lda, 0);
    if (C::B_KMAJOR) {  // B [b_cols, kbytes]
      rb = make_rsrc(p.b + (long)n0 * p.ldb, (unsigned long long)(p.b_cols - n0) * p.ldb);
    } else {            // B [kbytes, b_cols]
      rb = make_rsrc(p.b + n0, kbytes * p.b_cols - n0);
    }
    sb.init((uint32_t)p.ldb, (uint32_t)gate);
  }

  // Stage-source position for the stagers (bytes along K for K-major sources,
  // first source row for MN-major sources; the same number for both).
  static __device__ __forceinline__ uint32_t kpos(int stage) { return (uint32_t)stage * (C::BK * C::BITS / 8); }

  __device__ __forceinline__ void load_stage(int stage) {
    sa.load(ra, kpos(stage));
    sb.load(rb, kpos(stage));
  }
  __device__ __forceinline__ void store_stage(uint8_t* buf) {
    sa.store(buf);
    sb.store(buf + C::A_STAGE);
  }

  // Runs the whole K loop.  on_step(k_end) follows each MFMA step (subchannel
  // flushes); it must not touch LDS.
  // One K stage: the widening / transposing LDS writes of the prefetched
  // stage it+1 are issued with the first step's MFMAs, the buffer loads of
  // stage it+2 with the last step's, and the barrier closes the stage.  The
  // buffer parity is a runtime offset so that the loop has a single body and
  // the accumulators stay in place across iterations.
  template <class OnStep>
  __device__ __forceinline__ void stage_body(uint8_t* smem, int it, int nst, OnStep& on_step) {
    const int cur = it & 1;
    const uint8_t* la = smem + cur * C::STAGE;
    const uint8_t* lb = la + C::A_STAGE;
    uint8_t* nb = smem + (cur ^ 1) * C::STAGE;
    const int nxt = it + 2 < nst ? it + 2 : nst - 1;
#pragma unroll
    for (int s = 0; s < S; ++s) {
      read_frags(la, lb, s, f);
      if (s == 0) store_stage(nb);
      if (s == S - 1) load_stage(nxt);
      mma(f);
      on_step((it * S + s + 1) * C::MK);
    }
    __syncthreads();
  }

  template <class OnStep>
  __device__ __forceinline__ void run(uint8_t* smem, int nst, OnStep on_step) {
    load_stage(0);
    store_stage(smem);
    load_stage(nst > 1 ? 1 : 0);
    __syncthreads();
    for (int it = 0; it < nst; ++it) stage_body(smem, it, nst, on_step);
  }
};

}  // namespace shk
