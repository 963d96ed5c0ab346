// int8 x int8 dense GEMM on the 32x32x32 int8 MFMA, operands read in their
// own layouts (no conversion pass).
//
// The engine follows the fp6 engine (shk_f6.h): four waves in 2 x 2, each
// owning 128 rows x 128 packed B rows as 4 x 4 int32 accumulators of 32 x 32
// (SwiGLU: 64 up columns then the same 64 gate columns), one branch-free
// sequence per stage of inline-asm MFMAs, LDS reads and LDS-DMA loads, and
// the same epilogues.  What differs is the operand path:
//  * A stage is 64 K (64 source bytes per tile row).  LDS-DMA copies it from
//    the operand as stored into a ring of four 32 KiB stages, in the
//    swizzled layouts of the direct-to-LDS engine (shk_dma.h): a K-major
//    stage holds 256 rows x 64 bytes with 16-byte unit q of row r at
//    r*64 + 16*(q ^ ((r >> 1) & 3)); an MN-major stage holds 64 K rows x 256
//    bytes with unit u of K row kp at kp*256 + 16*(u ^ swm(kp)).
//  * The 32x32x32 MFMA takes, per lane l, row (or column) l % 32 and the 16
//    K values 16*(l/32) + [0, 16) of a 32-K step (measured on the box).  A
//    K-major fragment is one ds_read_b128 of unit 2s + l/32; an MN-major one
//    is two ds_read_b64_tr_b8 over K rows 32s + 16*(l/32) + [0, 8) and
//    [8, 16), which hand lane l the bytes of its column.
// Stage k waits for its own DMA of stage k+1, then the barrier; its 32 MFMAs
// (2 steps x 4 x 4) carry the LDS reads of stage k+1 and, on the odd MFMAs
// 1 .. 15, the DMA loads of stage k+P into slot k % P (P = 4 ring slots:
// three stages ahead).
#pragma once

#include "shk_f6.h"

namespace shk {

typedef int v16i __attribute__((ext_vector_type(16)));

template <class C>
struct I8Engine {
  static constexpr bool SWIGLU = C::SWIGLU;
  static constexpr int P = C::PIPE;                     // ring slots: 4 (one workgroup per CU) or 3
  static constexpr int NW = 4;
  static constexpr int MI = C::BM / 64;                // 32-row A fragments per wave: 4 or 2
  static constexpr int WROWS = 32 * MI;                // output rows per wave
  using OA = DmaOperand<8, C::A_KMAJOR, C::BM, NW, C::BM>;
  using OB = DmaOperand<8, C::B_KMAJOR, 256, NW, C::BHALF>;
  static constexpr int A_BYTES = C::BM * 64;           // A's part of a stage: 16 or 8 KiB
  static constexpr int STAGE = A_BYTES + 256 * 64;     // then 16 KiB of B
  static constexpr int LDS_BYTES = P * STAGE;          // 128 or 96 KiB
  static constexpr int DPW = OA::BLK + OB::BLK;        // 8 or 6 DMA loads per wave per stage
  static constexpr int TN = SWIGLU ? 64 : 128;         // output columns per wave
  static constexpr int FN = SWIGLU ? 2 : 4;            // output column fragments per wave
  static constexpr int NA = C::A_KMAJOR ? 1 : 2;       // LDS reads per A fragment and step
  static constexpr int NB = C::B_KMAJOR ? 1 : 2;
  static constexpr int RSTEP = MI * NA + 4 * NB;       // LDS reads per step
  static constexpr int READS = 2 * RSTEP;              // per stage
  static constexpr int TICKS = 2 * MI * 4;             // MFMAs per stage
  static_assert(C::BITS == 8 && (C::BM == 256 || (C::BM == 128 && C::A_KMAJOR)) && C::BROWS == 256 &&
                    C::WM == 2 && C::WN == 2,
                "int8, 256-row tiles (128-row tiles with a K-major A), 2x2 waves");
  static_assert(2 * DPW <= TICKS && READS <= 2 * TICKS && (P == 3 || P == 4), "schedule");

  v16i acc[MI][4];
  v4i fa[2][2][MI];  // [set][step][i]
  v4i fb[2][2][4];   // [set][step][j]
  OA oa;
  OB ob;
  v4i rsa, rsb;
  uint32_t lda, ldb;
  uint32_t lds0;
  int lane, wave, wm, wn;
  // LDS read bases of this lane in the next stage's slot: K-major operands
  // one per step (fragments add 64 bytes per row), MN-major ones one per
  // fragment (step 1 adds 32 K rows, the second half 8 K rows).
  uint32_t ra[C::A_KMAJOR ? 2 : 4];
  uint32_t rb[C::B_KMAJOR ? 2 : 4];

  // first tile row of B fragment j (packed B rows of the tile)
  __device__ __forceinline__ int brow(int j) const {
    return SWIGLU ? (j < 2 ? 64 * wn + 32 * j : 128 + 64 * wn + 32 * (j - 2)) : 128 * wn + 32 * j;
  }
  __device__ __forceinline__ int out_row(int i) const { return wm * WROWS + 32 * i + (lane & 31); }
  __device__ __forceinline__ int out_col(int j, int q) const { return wn * TN + 32 * j + 8 * q + 4 * (lane >> 5); }
  __device__ __forceinline__ float acc_value(int i, int j, int x) const { return (float)acc[i][j][x]; }
  static constexpr float UNSCALE = 1.0f;
  __device__ __forceinline__ float acc_stored(int i, int j, int x) const { return (float)acc[i][j][x]; }
  __device__ __forceinline__ int acc_int(int i, int j, int x) const { return acc[i][j][x]; }

  // K-major read base of step s (fragment rows are a multiple of 32, so the
  // swizzle (r >> 1) & 3 depends on the lane only); `row0` is the wave's
  // first row of the operand within the stage.
  __device__ __forceinline__ uint32_t kmajor_base(int row0, int s) const {
    const uint32_t r = (uint32_t)(lane & 31);
    const uint32_t q = (uint32_t)(2 * s + (lane >> 5));
    return (uint32_t)row0 * 64u + r * 64u + 16u * (q ^ ((r >> 1) & 3u));
  }
  // MN-major read base of the fragment whose first tile column is `col0`:
  // lane i of each 16-lane group addresses K row kp = 16*(l/32) + i/2 at
  // byte 8*(i%2) of its 16-column unit; swm(kp) = (i/2) | 8*(l/32).
  __device__ __forceinline__ uint32_t mnmajor_base(int col0) const {
    const uint32_t i = (uint32_t)(lane & 15), g = (uint32_t)(lane >> 5);
    const uint32_t kp = 16u * g + i / 2;
    const uint32_t u = (uint32_t)col0 / 16u + (uint32_t)((lane & 31) >> 4);
    return kp * 256u + 16u * (u ^ ((i / 2) | (8u * g))) + 8u * (i & 1u);
  }

  __device__ __forceinline__ void setup(uint8_t* smem, const DenseArgs& p, int m0, int n0, int gate) {
    lane = threadIdx.x & 63;
    wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    wm = wave % 2;
    wn = wave / 2;
    lds0 = lds_address(smem);
    const unsigned long long kbytes = (unsigned long long)p.K;
    lda = (uint32_t)p.lda;
    ldb = (uint32_t)p.ldb;
    if (C::A_KMAJOR) rsa = buffer_words(p.a + (long)m0 * p.lda, (unsigned long long)(p.M - m0) * p.lda);
    else rsa = buffer_words(p.a + m0, kbytes * p.M - m0);
    if (C::B_KMAJOR) rsb = buffer_words(p.b + (long)n0 * p.ldb, (unsigned long long)(p.b_cols - n0) * p.ldb);
    else rsb = buffer_words(p.b + n0, kbytes * p.b_cols - n0);
    oa.init(wave, lane, lda, 0);
    ob.init(wave, lane, ldb, (uint32_t)gate);
    // read bases of slot 1 (stage 1 is read during stage 0)
    const uint32_t s1 = lds0 + (uint32_t)STAGE;
    if constexpr (C::A_KMAJOR) {
      ra[0] = s1 + kmajor_base(WROWS * wm, 0);
      ra[1] = s1 + kmajor_base(WROWS * wm, 1);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) ra[i] = s1 + mnmajor_base(128 * wm + 32 * i);
    }
    if constexpr (C::B_KMAJOR) {
      rb[0] = s1 + A_BYTES + kmajor_base(brow(0), 0);
      rb[1] = s1 + A_BYTES + kmajor_base(brow(0), 1);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) rb[j] = s1 + A_BYTES + mnmajor_base(brow(j));
    }
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;
  }

  // Moves the read bases by `d` bytes.
  __device__ __forceinline__ void add_reads(uint32_t d) {
#pragma unroll
    for (auto& x : ra) x += d;
#pragma unroll
    for (auto& x : rb) x += d;
  }

  // Read Q of a stage into set S.  Per step the fragments in the order of
  // their first use: A0, B0..B3, A1..A(MI-1), each in NA / NB parts.
  template <int S, int Q>
  __device__ __forceinline__ void read() {
    constexpr int ST = Q / RSTEP;
    constexpr int W = Q % RSTEP;
    // position W in [A0 | B0 B1 B2 B3 | A1 A2 A3]
    constexpr bool IS_A = W < NA || W >= NA + 4 * NB;
    constexpr int IDX = W < NA ? 0 : (W < NA + 4 * NB ? (W - NA) / NB : 1 + (W - NA - 4 * NB) / NA);
    constexpr int PART = W < NA ? W : (W < NA + 4 * NB ? (W - NA) % NB : (W - NA - 4 * NB) % NA);
    constexpr bool KM = IS_A ? C::A_KMAJOR : C::B_KMAJOR;
    v4i& dst = IS_A ? fa[S][ST][IDX] : fb[S][ST][IDX];
    if constexpr (KM) {
      // K-major: fragment rows 32*IDX (A) or the B fragment's rows, relative
      // to the base of fragment 0; SwiGLU gate fragments are 128 - 64 rows
      // further than the up pattern (64*wn + 32j) continues.
      constexpr int ROWS = IS_A ? 32 * IDX : (SWIGLU ? (IDX < 2 ? 32 * IDX : 128 + 32 * (IDX - 2)) : 32 * IDX);
      const uint32_t base = IS_A ? ra[ST] : rb[ST];
      asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(dst) : "v"(base), "i"(ROWS * 64));
    } else {
      constexpr int OFF = ST * 32 * 256 + PART * 8 * 256;
      const uint32_t base = IS_A ? ra[IDX] : rb[IDX];
      v2i y;
      asm volatile("ds_read_b64_tr_b8 %0, %1 offset:%2" : "=v"(y) : "v"(base), "i"(OFF));
      if constexpr (PART == 0) {
        dst.x = y.x;
        dst.y = y.y;
      } else {
        dst.z = y.x;
        dst.w = y.y;
      }
    }
  }

  // MFMA T (0..TICKS-1) of a stage on set S (step T / (4 MI), A fragment
  // (T % 4 MI) / 4, B fragment T % 4), fused with DMA load T/2 (odd T <
  // 2 DPW: A blocks, then B blocks) of the stage being loaded, followed by
  // LDS reads T and T + TICKS (while below READS) of the next stage.  No
  // branch surrounds an asm MFMA or LDS read (see shk_f6.h).
  template <int S, int T>
  __device__ __forceinline__ void tick(const v4i& rsa_st, const v4i& rsb_st, uint32_t soa, uint32_t sob, uint32_t m0) {
    constexpr int ST = T / (4 * MI), I = (T % (4 * MI)) / 4, J = T % 4;
    if constexpr (T % 2 == 1 && T < 2 * DPW) {
      constexpr int c = T / 2;
      constexpr bool DA = c < OA::BLK;
      const v4i& rs = DA ? rsa_st : rsb_st;
      const uint32_t voff = DA ? oa.voff[c] : ob.voff[c - OA::BLK];
      const uint32_t dst = m0 + (DA ? 1024u * (OA::BLK * wave + c) : A_BYTES + 1024u * (OB::BLK * wave + c - OA::BLK));
      asm volatile(
          "v_mfma_i32_32x32x32_i8 %0, %1, %2, %0\n\t"
          "buffer_load_dwordx4 %3, %4, %5 offen lds"
          : "+a"(acc[I][J])
          : "v"(fb[S][ST][J]), "v"(fa[S][ST][I]), "v"(voff), "s"(rs), "s"(DA ? soa : sob), "{m0}"(dst)
          : "memory");
    } else {
      asm volatile("v_mfma_i32_32x32x32_i8 %0, %1, %2, %0"
                   : "+a"(acc[I][J])
                   : "v"(fb[S][ST][J]), "v"(fa[S][ST][I]));
    }
    if constexpr (T < READS) read<1 - S, T>();
    if constexpr (T + TICKS < READS) read<1 - S, T + TICKS>();
  }
  template <int S, int... T>
  __device__ __forceinline__ void ticks(const v4i& rsa_st, const v4i& rsb_st, uint32_t soa, uint32_t sob,
                                        uint32_t m0, std::integer_sequence<int, T...>) {
    (tick<S, T>(rsa_st, rsb_st, soa, sob, m0), ...);
  }
  template <int S, int... Q>
  __device__ __forceinline__ void reads(std::integer_sequence<int, Q...>) {
    (read<S, Q>(), ...);
  }

  // fence<4> (s_nop 4: 5 wait states) stands between VALU writes of the
  // accumulators (the clear before the loop) and the first asm MFMA that reads
  // them as its C operand: a VALU write followed by an MFMA reading the
  // register needs 2 wait states.  fence<7> (5 x s_nop 7: 40 wait states)
  // stands between the last asm MFMA and any other access to its result: an
  // XDL MFMA of up to 16 passes needs 18 wait states before a VALU, VMEM,
  // LDS or v_accvgpr_read instruction reads its destination or a VALU
  // instruction overwrites it (v_mfma_i32_32x32x32_i8 is a 16-pass form), so 40 covers
  // every MFMA here with margin.  Every accumulator is an operand of the
  // fence, so no compiler access (or register-allocator copy on a merge)
  // crosses it.
  template <int N>
  __device__ __forceinline__ void fence() {
    static_assert(N == 4 || N == 7, "wait states");
#define SHK_I8_ACC(i) "+a"(acc[i][0]), "+a"(acc[i][1]), "+a"(acc[i][2]), "+a"(acc[i][3])
    if constexpr (MI == 4) {
      if constexpr (N == 4)
        asm volatile("s_nop 4" : SHK_I8_ACC(0), SHK_I8_ACC(1), SHK_I8_ACC(2), SHK_I8_ACC(3));
      else
        asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7"
                     : SHK_I8_ACC(0), SHK_I8_ACC(1), SHK_I8_ACC(2), SHK_I8_ACC(3));
    } else {
      if constexpr (N == 4)
        asm volatile("s_nop 4" : SHK_I8_ACC(0), SHK_I8_ACC(1));
      else
        asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" : SHK_I8_ACC(0), SHK_I8_ACC(1));
    }
#undef SHK_I8_ACC
  }

  // Stage k on set S: wait for this wave's DMA of stage k+1 (k+2 .. k+P-1
  // may stay outstanding), then the barrier; MFMAs of stage k, reads of
  // stage k+1, DMA of stage k+P into slot `slot` (k's), through zero-record
  // resources past the last stage.
  // This wave's LDS reads into set S (step ST) have landed.  The reads are
  // asm statements, so the compiler does not know that their registers are
  // written later than the statement: every register of the set is an
  // operand here, so none is copied before the data is in.
  template <int S, int ST>
  __device__ __forceinline__ void frag_fence() {
    if constexpr (MI == 4)
      asm volatile("s_waitcnt lgkmcnt(0)"
                   : "+v"(fa[S][ST][0]), "+v"(fa[S][ST][1]), "+v"(fa[S][ST][2]), "+v"(fa[S][ST][3]),
                     "+v"(fb[S][ST][0]), "+v"(fb[S][ST][1]), "+v"(fb[S][ST][2]), "+v"(fb[S][ST][3])::"memory");
    else
      asm volatile("s_waitcnt lgkmcnt(0)"
                   : "+v"(fa[S][ST][0]), "+v"(fa[S][ST][1]), "+v"(fb[S][ST][0]), "+v"(fb[S][ST][1]),
                     "+v"(fb[S][ST][2]), "+v"(fb[S][ST][3])::"memory");
  }
  template <int S>
  __device__ __forceinline__ void stage(int k, int nst, int slot, const v4i& rsa_end, const v4i& rsb_end) {
    wait_vmcnt<(P - 2) * DPW>();
    frag_fence<S, 0>();
    frag_fence<S, 1>();
    asm volatile("s_barrier" ::: "memory");
    const bool live = k + P < nst;
    const v4i rsa_st = live ? rsa : rsa_end;
    const v4i rsb_st = live ? rsb : rsb_end;
    const uint32_t soa = live ? OA::soff(k + P, lda) : 0u;
    const uint32_t sob = live ? OB::soff(k + P, ldb) : 0u;
    ticks<S>(rsa_st, rsb_st, soa, sob, lds0 + (uint32_t)slot * STAGE, std::make_integer_sequence<int, TICKS>{});
  }
  // Moves the read bases one slot ahead (wrapping after the last) and the
  // stage slot.
  __device__ __forceinline__ void advance(int& slot) {
    add_reads(slot == P - 2 ? (uint32_t)(-(P - 1) * STAGE) : (uint32_t)STAGE);
    slot = slot == P - 1 ? 0 : slot + 1;
  }

  // nst: 64-K stages (at least one; none leaves the sums at zero).
  __device__ __forceinline__ void run(int nst) {
    if (nst <= 0) {
      wait_vmcnt<0>();  // loads issued before the call (the B scales)
      return;
    }
    const v4i rsa_end = v4i{rsa.x, rsa.y, 0, rsa.w};
    const v4i rsb_end = v4i{rsb.x, rsb.y, 0, rsb.w};
    // stages 0..3 (zeros past the last stage), then stage 0 into set 0
#pragma unroll
    for (int st = 0; st < P; ++st) {
      const uint32_t base = lds0 + (uint32_t)st * STAGE;
#pragma unroll
      for (int c = 0; c < OA::BLK; ++c)
        lds_dma16(st < nst ? rsa : rsa_end, oa.voff[c], st < nst ? OA::soff(st, lda) : 0u,
                  base + 1024u * (OA::BLK * wave + c));
#pragma unroll
      for (int c = 0; c < OB::BLK; ++c)
        lds_dma16(st < nst ? rsb : rsb_end, ob.voff[c], st < nst ? OB::soff(st, ldb) : 0u,
                  base + A_BYTES + 1024u * (OB::BLK * wave + c));
    }
    wait_vmcnt<(P - 1) * DPW>();
    asm volatile("s_barrier" ::: "memory");
    // the bases point at slot 1; read stage 0 from slot 0
    add_reads((uint32_t)(-STAGE));
    reads<0>(std::make_integer_sequence<int, READS>{});
    add_reads((uint32_t)STAGE);
    fence<4>();
    int slot = 0;
    int k = 0;
    for (; k + 2 <= nst; k += 2) {
      stage<0>(k, nst, slot, rsa_end, rsb_end);
      advance(slot);
      stage<1>(k + 1, nst, slot, rsa_end, rsb_end);
      advance(slot);
    }
    // the last stage's reads land before the paths merge and before their
    // registers could be reused, and the MFMAs finish (see shk_f6.h)
    frag_fence<0, 0>();
    frag_fence<0, 1>();
    fence<7>();
    if (k < nst) {
      stage<0>(k, nst, slot, rsa_end, rsb_end);
      frag_fence<1, 0>();
      frag_fence<1, 1>();
      fence<7>();
    }
    fence<7>();
    // the loads past the last stage land before the workgroup's LDS is freed
    wait_vmcnt<0>();
  }
};

// One int8 tile at (m0, n0) on the engine of configuration T.
template <class T, int MODE, int EPI>
__device__ __forceinline__ void i8_tile(const DenseArgs& p, uint8_t* smem, int m0, int n0) {
  using E = I8Engine<T>;
  E e;
  e.setup(smem, p, m0, n0, T::SWIGLU ? p.N : 0);
  float sa[4] = {};
#pragma unroll
  for (int i = 0; i < E::MI; ++i) sa[i] = MODE == OUT_I32 ? 0.0f : load_bf16(p.a_scale + m0 + e.out_row(i));
  const OutView o = dense_view<T, MODE>(p);
  mfma32_prefetch_b_scales<T, MODE>(e, o, n0, e.lds0 + E::LDS_BYTES + 256u * e.wave);
  e.run(p.K / 64);
  mfma32_finish<T, MODE, EPI>(e, o, smem, m0, n0, sa);
}

// The 128-row tile of a 256-row int8 configuration (K-major A).
template <class C>
using I8Half = Cfg<8, C::A_KMAJOR, C::B_KMAJOR, 128, C::BN, C::BK, 2, 2, C::SWIGLU, false, C::MK, false, C::PIPE>;

// One kernel per output mode and epilogue (chosen by the host).  One
// workgroup per tile.  With p.split_tn > 0 (256-row tiles, K-major A), the
// column tiles [split_tn, N / BN) run last as twice as many 128-row tiles:
// the host sets it when those columns would otherwise form a partial last
// round of workgroups, which then takes about half as long.
template <class C, int MODE, int EPI>
__global__ __launch_bounds__(256) void i8_gemm_kernel(const DenseArgs p) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[I8Engine<C>::LDS_BYTES + MFMA32_SCALE_BYTES];
  const int tiles_m = p.M / C::BM;
  const int tiles_n = p.N / C::BN;
  const int main_n = p.split_tn > 0 ? p.split_tn : tiles_n;
  const int main_tiles = tiles_m * main_n;
  int tm, tn;
  if constexpr (C::BM == 256 && C::A_KMAJOR) {
    static_assert(I8Engine<I8Half<C>>::LDS_BYTES <= I8Engine<C>::LDS_BYTES, "the half tile fits the LDS");
    if ((int)blockIdx.x >= main_tiles) {
      dense_tile_coords((int)blockIdx.x - main_tiles, 2 * tiles_m, tiles_n - main_n, p.group_m, tm, tn);
      i8_tile<I8Half<C>, MODE, EPI>(p, smem, tm * 128, (main_n + tn) * C::BN);
      return;
    }
  }
  dense_tile_coords(blockIdx.x, tiles_m, main_n, p.group_m, tm, tn);
  i8_tile<C, MODE, EPI>(p, smem, tm * C::BM, tn * C::BN);
}

}  // namespace shk
