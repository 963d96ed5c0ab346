// int4 x int4 dense GEMM on the fp6 MFMA.
//
// gfx950 has no int4 MFMA, and -8..7 does not fit fp4 e2m1.  Every int4 value
// v is, however, exact as v/8 in the 6-bit float e2m3 ("fp6": sign, 2
// exponent bits with bias 1, 3 mantissa bits): |v| <= 7 are the subnormals
// |v|/8 and 8 is 2^0, so the code is simply sign << 5 | |v|.  The f8f6f4 MFMA
// multiplies fp6 operands at twice the int8 MFMA rate.  A product of two such
// operands is an integer / 64 of magnitude <= 1, and the MFMA accumulates in
// fp32, which holds every multiple of 1/64 below 2^18 exactly, so for
// K <= 2^18 every partial sum is exact and 64 * acc is the exact int32 sum
// (|sum| <= 64 * K <= 2^24).  The epilogue therefore sees the same integer as
// the int8 engines and produces the same bits.  e2m3 rather than bf6 (e3m2,
// where -8..7 are exact too) because the same MFMA then draws less power,
// which is the limit on this chip with full-rate MFMAs on random data.  The
// GEMM issues v_mfma_f32_32x32x64_f8f6f4 (cbsz = blgp = 2: both operands
// e2m3).
//
// The path runs in two launches:
//  1. f6_pack_* converts each operand, in whichever layout it arrives, into
//     the "block" format in a caller workspace: a 32-row x 64-K block is
//     1536 bytes, 24 per MFMA lane (lane l: row l % 32, K values
//     32*(l/32) + [0, 32) of the block) split into a 1024-byte part (the
//     lane's first 16 bytes at 16*l) and a 512-byte part (its last 8 bytes at
//     1024 + 8*l).  Blocks are stored panel-major: block (p, kb) of the
//     32-row panel p and 64-K block kb sits at (p * K/64 + kb) * 1536.
//  2. f6_gemm_kernel streams the 256-row x 128-K stages of both operands
//     with LDS-DMA into a three-slot ring (48 KiB per stage) and reads each
//     fragment with one ds_read_b128 and one ds_read_b64 of consecutive lane
//     addresses, which is free of bank conflicts without a swizzle.  The K
//     loop has no VALU work: DMA, LDS reads and MFMAs only.
//
// K order inside a lane's 32 values.  The conversion turns the lane's 16
// packed bytes (byte b holds K values 2b, 2b+1, low nibble first) into f16
// pairs with one mask per nibble position, so field f of the lane holds the
// value at nibble 8*(f/8) + (f%8)/2 + 4*(f%2) of the 32.  A and B go through
// the same conversion, so both operands see the same permutation of K and
// the dot products are unchanged.
#pragma once

#include <utility>

#include "shk_dense.h"
#include "shk_tasks.h"

namespace shk {

typedef int v6i __attribute__((ext_vector_type(6)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 f6_h2 __attribute__((ext_vector_type(2)));
typedef _Float16 f6_h32 __attribute__((ext_vector_type(32)));
typedef __bf16 f6_bf8 __attribute__((ext_vector_type(8)));

constexpr int F6_BLOCK = 1536;     // bytes of a 32-row x 64-K fp6 block
constexpr int F6_MAX_K = 262144;   // 64 * K <= 2^24: fp32 partial sums stay exact
// Largest K of the fp6 entries.  Per-channel calls with K > F6_MAX_K run in
// K slices of F6_MAX_K, each exact, whose int32 sums add into an int32
// workspace (exact while |sum| < 2^31, i.e. K < 2^25); the bound here comes
// from the 32-bit buffer offsets of one tile's 8 panels (8 * 24 * K < 2^32).
constexpr int F6_MAX_K_SLICED = 1 << 24;
constexpr int F6_TILE = 256;       // packed rows per GEMM tile (A rows, B columns)
// Each operand holds v/8, so the accumulator is sum / 64; multiplying by 64
// is exact.
constexpr float F6_UNSCALE = 64.0f;

// Bytes of one operand with `rows` rows (a multiple of 256) and K (a
// multiple of 128) in block format.
__host__ __device__ constexpr unsigned long long f6_operand_bytes(long rows, long k) {
  return (unsigned long long)rows * (unsigned long long)k * 3ull / 4ull;
}

// One operand, or a batch of `groups` operands of the same shape (the
// ragged path's per-expert matrices).  Rows past `rows` convert as zeros up
// to the next 32-row panel.  K values at or past the operand's length
// (min(k_len[g], k_cap), or k_cap without k_len) convert as zeros, and 64-K
// blocks past the last 128-K stage that holds any K of that length are not
// written (no GEMM reads them).  Sources are read in pieces of `vec` bytes
// (16, 8 or 1), the alignment of their base and row pitch (MN-major: the
// pitch is the row count).
struct F6PackArgs {
  const uint8_t* src;
  uint8_t* dst;
  long ld;                      // bytes between consecutive source rows
  int rows;                     // packed rows of one operand
  int kb;                       // 64-K blocks per panel
  int swiglu_n;                 // > 0: SwiGLU B with N output columns (rows interleave up and gate)
  int groups;                   // operands in the batch (1 for a dense call)
  long src_group;               // source bytes between consecutive operands
  unsigned long long dst_group; // block bytes between consecutive operands
  const int32_t* k_len;         // per-operand logical K length, or null
  int k_cap;                    // K length without k_len; the upper clamp of k_len
  int vec;                      // source alignment: 16, 8 or 1
  bool write_through = false;   // the block stores write through the L2 (cache policy SC1)
  int kmajor_blocks = 1;        // K-major: 64-K blocks per wave (1 or 2)
  int k_stage = 128;            // with k_len: the GEMM reads whole stages of this many K (128 or 256)
};

// 32-row panels of an operand with `rows` rows.
__host__ __device__ constexpr int f6_panels(int rows) { return (rows + 31) / 32; }

// Converts one operand into block format (k_f6pack.hip).  mn_major: the
// source is stored K-row by K-row (two K values per byte of every row).
hipError_t launch_f6_pack(const F6PackArgs& a, bool mn_major, hipStream_t s);
// Both operands in one launch; with a job (sizes non-null, at most
// kFusedTaskGroups groups) an extra first workgroup builds a ragged task
// list beside the conversion.  interleave: the two operands' workgroups
// alternate in proportion instead of running A's first (the per-channel
// dense calls).
hipError_t launch_f6_pack2(const F6PackArgs& a, bool a_mn, const F6PackArgs& b, bool b_mn, hipStream_t s,
                           const TaskJob* job = nullptr, bool interleave = false);

// ---------------------------------------------------------------------------
// GEMM engine.  Four waves in 2 x 2, each owning 128 rows x 128 packed B
// rows of the 256 x 256 tile: 4 x 4 accumulators of 32 x 32 (SwiGLU: the
// packed B rows of a wave are 64 up columns then the same 64 gate columns,
// so fragments j = 2, 3 are the gate of j = 0, 1).  The B fragment is the
// MFMA's first operand, so lane l holds output row 32*i + l % 32 and, in
// registers 4q .. 4q+3, the four consecutive columns 32*j + 8q + 4*(l/32).
//
// Schedule of stage k (128 K = two 64-K steps, slot k % 3 of the ring):
//  * top: wait for this wave's DMA of stage k+1 and its own LDS reads of
//    stage k, then the barrier: stage k+1 is complete in LDS and no wave
//    still reads slot k % 3;
//  * 32 MFMAs (2 steps x 4 x 4) on the fragments of stage k (register set
//    k % 2); after each, one LDS read of stage k+1 into the other set; the
//    odd MFMAs 1 .. 23 each carry one DMA load of stage k+3 into slot k % 3.
// The DMA of a stage is thus issued two stages before its data is read.
// A stage in LDS holds, per operand, eight 32-row panels of two blocks.
template <class C>
struct F6Engine {
  static constexpr bool SWIGLU = C::SWIGLU;
  static constexpr int P = 3;
  static constexpr int NW = 4;
  static constexpr int PANEL = 2 * F6_BLOCK;     // 32 rows x 128 K: 3 KiB
  static constexpr int OPB = 8 * PANEL;          // one operand's stage: 24 KiB
  static constexpr int STAGE = 2 * OPB;          // 48 KiB
  static constexpr int LDS_BYTES = P * STAGE;    // 144 KiB
  static constexpr int DPW = STAGE / 1024 / NW;  // 12 DMA loads per wave per stage
  static constexpr int TN = SWIGLU ? 64 : 128;   // output columns per wave
  static constexpr int FN = SWIGLU ? 2 : 4;      // output column fragments per wave
  static constexpr int MI = 4;                   // 32-row fragments per wave
  static constexpr int WROWS = 32 * MI;          // output rows per wave
  static_assert(C::BM == 256 && C::WM == 2 && C::WN == 2 && C::BROWS == 256, "256-row tiles, 2x2 waves");

  v16f acc[4][4];
  v6i fa[2][2][4];  // [set][step][i]
  v6i fb[2][2][4];  // [set][step][j]
  uint32_t voff[DPW];
  v4i rs;         // this wave's DMA operand (waves 0-1: A, 2-3: B)
  uint32_t lds0;  // LDS address of slot 0
  int lane, wave, wm, wn;

  // LDS read addresses of this lane in one slot: 16- and 8-byte parts of
  // the wave's A panel 0 and B panel 0, step 0 (panel f adds PANEL * f,
  // step 1 adds one block).
  struct Reads {
    uint32_t a16, a8, b16, b8;
    __device__ __forceinline__ void add(uint32_t d) {
      a16 += d;
      a8 += d;
      b16 += d;
      b8 += d;
    }
  };

  __device__ __forceinline__ int out_row(int i) const { return wm * 128 + 32 * i + (lane & 31); }
  // first of the four columns of fragment j (< FN), register group q
  __device__ __forceinline__ int out_col(int j, int q) const { return wn * TN + 32 * j + 8 * q + 4 * (lane >> 5); }
  // the exact integer sum of accumulator register x of [i][j], as fp32 / int32
  __device__ __forceinline__ float acc_value(int i, int j, int x) const { return acc[i][j][x] * F6_UNSCALE; }
  // the accumulator as held (the sum / 64) and the power of two restoring it
  static constexpr float UNSCALE = F6_UNSCALE;
  __device__ __forceinline__ float acc_stored(int i, int j, int x) const { return acc[i][j][x]; }
  __device__ __forceinline__ int acc_int(int i, int j, int x) const { return (int)(acc[i][j][x] * F6_UNSCALE); }

  // a6 / b6: block-format operands; the tile's first panels are m0 / 32 and
  // 8 * bt (bt: B tile index).
  // kb0: first 64-K block of the K range this workgroup multiplies (a K
  // slice of a large-K launch; 0 otherwise).
  // FRESH (a persistent kernel's tile loop): the thread index passes through
  // an empty asm statement, so nothing derived from it is computed once
  // before the loop and held, or spilled, across every tile's K loop.
  template <bool FRESH = false>
  __device__ __forceinline__ void setup(uint8_t* smem, const uint8_t* a6, const uint8_t* b6, int m0, int bt, int kb,
                                        unsigned long long a_bytes, unsigned long long b_bytes, int kb0 = 0) {
    int tid = (int)threadIdx.x;
    if constexpr (FRESH) asm volatile("" : "+v"(tid));
    lane = tid & 63;
    wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    wm = wave % 2;
    wn = wave / 2;
    lds0 = lds_address(smem);
    const unsigned long long panel_bytes = (unsigned long long)kb * F6_BLOCK;
    const bool is_a = wave < 2;
    const unsigned long long first =
        (is_a ? (unsigned long long)(m0 / 32) : (unsigned long long)bt * 8) * panel_bytes +
        (unsigned long long)kb0 * F6_BLOCK;
    rs = buffer_words((is_a ? a6 : b6) + first, (is_a ? a_bytes : b_bytes) - first);
    // DMA load c of this wave fills stage bytes [1024 * (DPW*wave + c), +1024):
    // panel o / PANEL of the operand, byte o % PANEL of its two blocks
#pragma unroll
    for (int c = 0; c < DPW; ++c) {
      const uint32_t o = 1024u * (DPW * wave + c) + 16u * lane - (is_a ? 0u : (uint32_t)OPB);
      voff[c] = (o / PANEL) * (uint32_t)panel_bytes + o % PANEL;
    }
  }

  __device__ __forceinline__ Reads reads_of_slot(int slot) const {
    const uint32_t s = lds0 + (uint32_t)slot * STAGE;
    const uint32_t a = s + 4u * wm * PANEL, b = s + OPB + 4u * wn * PANEL;
    return Reads{a + 16u * lane, a + 1024u + 8u * lane, b + 16u * lane, b + 1024u + 8u * lane};
  }

  // LDS read Q (0..31) of a stage into set S: per step, the fragments in the
  // order of their first use (A0, B0..B3, A1..A3), each as its 16-byte then
  // its 8-byte part.
  template <int S, int Q>
  __device__ __forceinline__ void read(const Reads& r) {
    constexpr int ST = Q / 16;
    constexpr int F = (Q % 16) / 2;
    constexpr bool IS_A = F == 0 || F >= 5;
    constexpr int IDX = F == 0 ? 0 : (F >= 5 ? F - 4 : F - 1);
    constexpr int OFF = IDX * PANEL + ST * F6_BLOCK;
    v6i& dst = IS_A ? fa[S][ST][IDX] : fb[S][ST][IDX];
    if constexpr (Q % 2 == 0) {
      v4i x;
      asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(x) : "v"(IS_A ? r.a16 : r.b16), "i"(OFF));
      dst.s0 = x.x;
      dst.s1 = x.y;
      dst.s2 = x.z;
      dst.s3 = x.w;
    } else {
      v2i y;
      asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(y) : "v"(IS_A ? r.a8 : r.b8), "i"(OFF));
      dst.s4 = y.x;
      dst.s5 = y.y;
    }
  }

  // MFMA T (0..31) of a stage on set S (step T/16, A fragment (T%16)/4, B
  // fragment T%4), fused with DMA load (T-1)/2 of the stage for odd T < 24,
  // followed by LDS read T of the next stage.  Every stage runs the same
  // sequence with no branch: a branch around an asm MFMA or LDS read would
  // let the register allocator copy an accumulator or fragment between the
  // asm statements, and the copy would read a value the hardware has not
  // written yet (the compiler cannot see the MFMA or the load in the asm).
  // FIRST (the first stage of a tile): the MFMAs of its first 64-K step take
  // 0 as the C operand and define the accumulators, so no VALU write ever
  // precedes an MFMA's read of them (see run()).
  template <int S, int T, bool FIRST>
  __device__ __forceinline__ void tick(const Reads& r, const v4i& rs_st, uint32_t so, uint32_t m0) {
    constexpr int ST = T / 16, I = (T % 16) / 4, J = T % 4;
    if constexpr (FIRST && T < 16 && T % 2 == 1 && T < 2 * DPW) {
      constexpr int c = T / 2;
      asm volatile(
          "v_mfma_f32_32x32x64_f8f6f4 %0, %1, %2, 0 cbsz:2 blgp:2\n\t"
          "buffer_load_dwordx4 %3, %4, %5 offen lds"
          : "=a"(acc[I][J])
          : "v"(fb[S][ST][J]), "v"(fa[S][ST][I]), "v"(voff[c]), "s"(rs_st), "s"(so), "{m0}"(m0 + 1024u * c)
          : "memory");
    } else if constexpr (FIRST && T < 16) {
      asm volatile("v_mfma_f32_32x32x64_f8f6f4 %0, %1, %2, 0 cbsz:2 blgp:2"
                   : "=a"(acc[I][J])
                   : "v"(fb[S][ST][J]), "v"(fa[S][ST][I]));
    } else if constexpr (T % 2 == 1 && T < 2 * DPW) {
      constexpr int c = T / 2;
      // the compiler writes M0 before the statement; the MFMA is the wait
      // state the LDS-DMA load needs after that write
      asm volatile(
          "v_mfma_f32_32x32x64_f8f6f4 %0, %1, %2, %0 cbsz:2 blgp:2\n\t"
          "buffer_load_dwordx4 %3, %4, %5 offen lds"
          : "+a"(acc[I][J])
          : "v"(fb[S][ST][J]), "v"(fa[S][ST][I]), "v"(voff[c]), "s"(rs_st), "s"(so), "{m0}"(m0 + 1024u * c)
          : "memory");
    } else {
      asm volatile("v_mfma_f32_32x32x64_f8f6f4 %0, %1, %2, %0 cbsz:2 blgp:2"
                   : "+a"(acc[I][J])
                   : "v"(fb[S][ST][J]), "v"(fa[S][ST][I]));
    }
    read<1 - S, T>(r);
  }
  template <int S, bool FIRST, int... T>
  __device__ __forceinline__ void ticks(const Reads& r, const v4i& rs_st, uint32_t so, uint32_t m0,
                                        std::integer_sequence<int, T...>) {
    (tick<S, T, FIRST>(r, rs_st, so, m0), ...);
  }
  template <int S, int... Q>
  __device__ __forceinline__ void reads(const Reads& r, std::integer_sequence<int, Q...>) {
    (read<S, Q>(r), ...);
  }

  // fence<4> (s_nop 4: 5 wait states) stands between VALU writes of the
  // accumulators and an asm MFMA that reads them as its C operand: a VALU
  // write followed by an MFMA reading the register needs 2 wait states (the
  // kernels here no longer make such writes: each tile's first MFMAs take 0
  // as the C operand).  fence<7> (5 x s_nop 7: 40 wait states)
  // stands between the last asm MFMA and any other access to its result: an
  // XDL MFMA of up to 16 passes needs 18 wait states before a VALU, VMEM,
  // LDS or v_accvgpr_read instruction reads its destination or a VALU
  // instruction overwrites it (the 8-pass fp6 forms need 10), so 40 covers
  // every MFMA here with margin.  Every accumulator is an operand of the
  // fence, so no compiler access (or register-allocator copy on a merge)
  // crosses it.
  template <int N>
  __device__ __forceinline__ void fence() {
    static_assert(N == 4 || N == 7, "wait states");
#define SHK_F6_ACC(i) "+a"(acc[i][0]), "+a"(acc[i][1]), "+a"(acc[i][2]), "+a"(acc[i][3])
    if constexpr (N == 4)
      asm volatile("s_nop 4" : SHK_F6_ACC(0), SHK_F6_ACC(1), SHK_F6_ACC(2), SHK_F6_ACC(3));
    else
      asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7"
                   : SHK_F6_ACC(0), SHK_F6_ACC(1), SHK_F6_ACC(2), SHK_F6_ACC(3));
#undef SHK_F6_ACC
  }

  // This wave's LDS reads into set S (step ST) have landed.  The reads are
  // asm statements, so the compiler does not know that their registers are
  // written later than the statement: every register of the set is an
  // operand here, so none is copied before the data is in.
  template <int S, int ST>
  __device__ __forceinline__ void frag_fence() {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(fa[S][ST][0]), "+v"(fa[S][ST][1]), "+v"(fa[S][ST][2]), "+v"(fa[S][ST][3]),
                   "+v"(fb[S][ST][0]), "+v"(fb[S][ST][1]), "+v"(fb[S][ST][2]), "+v"(fb[S][ST][3])::"memory");
  }

  // Stage k on set S.  Top: this wave's DMA of stage k+1 has landed (that
  // of k+2 may be outstanding), its LDS reads are done, then the barrier.
  // Then the MFMAs of stage k, the reads of stage k+1 (slot `r`) and the DMA
  // of stage k+3 into slot `slot` (k's).  Past the last stage, the reads
  // fetch a stale slot into the unused set and the DMA loads go through
  // `rs_end`, a resource of zero records: they return zeros without touching
  // memory, into a slot that holds no live data.
  template <int S, bool FIRST = false>
  __device__ __forceinline__ void stage(const Reads& r, int k, int nst, int slot, const v4i& rs_end) {
    wait_vmcnt<DPW>();
    frag_fence<S, 0>();
    frag_fence<S, 1>();
    asm volatile("s_barrier" ::: "memory");
    const bool live = k + 3 < nst;
    const v4i rs_st = live ? rs : rs_end;
    const uint32_t so = live ? (uint32_t)(k + 3) * PANEL : 0u;
    ticks<S, FIRST>(r, rs_st, so, lds0 + (uint32_t)slot * STAGE + 1024u * DPW * wave,
                    std::make_integer_sequence<int, 32>{});
  }
  // Moves the read slot one ahead (wrapping after slot 2) and the stage slot.
  static __device__ __forceinline__ void advance(Reads& r, int& slot) {
    r.add(slot == 1 ? (uint32_t)(-2 * STAGE) : (uint32_t)STAGE);
    slot = slot == 2 ? 0 : slot + 1;
  }

  // nst: 128-K stages (at least one; none leaves the sums at zero).
  // The first stage runs on its own with FIRST MFMAs, which define the
  // accumulators: a persistent workgroup's accumulators were last written by
  // the previous tile's MFMAs, and an asm MFMA whose C operand a VALU write
  // (a clear) had overwritten after an earlier MFMA of the wave was seen to
  // read stale values.  The remaining stages alternate register sets from
  // set 1.
  __device__ __forceinline__ void run(int nst) {
    if (nst <= 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.0f;  // no MFMA reads them
      wait_vmcnt<0>();  // loads issued before the call (the B scales)
      return;
    }
    const v4i rs_end = v4i{rs.x, rs.y, 0, rs.w};
    // stages 0..2 (zeros past the last stage), then stage 0 into set 0
#pragma unroll
    for (int st = 0; st < 3; ++st)
#pragma unroll
      for (int c = 0; c < DPW; ++c)
        lds_dma16(st < nst ? rs : rs_end, voff[c], st < nst ? (uint32_t)st * PANEL : 0u,
                  lds0 + (uint32_t)st * STAGE + 1024u * (DPW * wave + c));
    wait_vmcnt<2 * DPW>();
    asm volatile("s_barrier" ::: "memory");
    reads<0>(reads_of_slot(0), std::make_integer_sequence<int, 32>{});
    // r: read slot of stage k+1; slot: slot of stage k
    Reads r = reads_of_slot(1);
    int slot = 0;
    stage<0, true>(r, 0, nst, slot, rs_end);
    advance(r, slot);
    int k = 1;
    for (; k + 2 <= nst; k += 2) {
      stage<1>(r, k, nst, slot, rs_end);
      advance(r, slot);
      stage<0>(r, k + 1, nst, slot, rs_end);
      advance(r, slot);
    }
    // The last stage's reads fetch a stale slot into the set that no MFMA
    // uses.  They land before the paths merge and before the set's
    // registers could be reused: the fences name every register of the set
    // (set 1 after the first stage and after the pairs, set 0 after an even
    // last stage).  Wait states after the last MFMA likewise, so that a copy
    // the register allocator places on a merge reads finished accumulators.
    frag_fence<1, 0>();
    frag_fence<1, 1>();
    fence<7>();
    if (k < nst) {
      stage<1>(r, k, nst, slot, rs_end);
      frag_fence<0, 0>();
      frag_fence<0, 1>();
      fence<7>();
    }
    fence<7>();
    // the loads past the last stage land before the workgroup's LDS is freed
    wait_vmcnt<0>();
  }
};

// bf16 pair halves as fp32
__device__ __forceinline__ float f6_bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float f6_bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }
__device__ __forceinline__ float f6_bf16_at(const uint2& w, int t) {
  return t == 0 ? f6_bf16_lo(w.x) : t == 1 ? f6_bf16_hi(w.x) : t == 2 ? f6_bf16_lo(w.y) : f6_bf16_hi(w.y);
}

// Where the epilogue of a 32x32 engine writes.  Element (r, c) of the
// output is at out + r * ld + c (elements); B scale of column c at
// b_scale[c], the SwiGLU gate's at b_scale[n + c].  A dense tile is written
// whole; with MASK (the ragged kernels) only rows [row_lo, row_hi) and
// columns below col_hi are, and B scales of columns at or past col_hi are
// not read.
struct OutView {
  void* out;
  const uint16_t* b_scale;
  int ld;    // elements between output rows
  int rows;  // rows of the output (the range of its stores)
  int n;     // output columns (SwiGLU: the gate's offset)
  int row_lo, row_hi, col_hi;
};

// The view of a dense call: [M, N] (int32 SwiGLU: [M, 2N], up then gate).
template <class C, int MODE>
__device__ __forceinline__ OutView dense_view(const DenseArgs& p) {
  return OutView{p.out, p.b_scale, (MODE == OUT_I32 && C::SWIGLU) ? 2 * p.N : p.N, p.M, p.N, 0, p.M, p.N};
}

// Writes a wave's results: lane l writes output row out_row(i) and, per
// register group q, the four columns out_col(j, q) + [0, 4) (for SwiGLU from
// accumulator j and its gate partner j + 2).
//  * OUT_I32: the exact integers ([M, 2N] for SwiGLU: up, then gate at +N);
//  * otherwise (float(acc) * a_scale) * b_scale, then ReLU^2 or SwiGLU, as
//    fp32 or bf16 (NO_NAN: no value is NaN, so the hardware conversion,
//    which does not canonicalize NaN, may be used).
// sb[j][q]: the four bf16 B scales of those columns (j >= FN: the gate's).
template <class C, int MODE, int EPI, bool NO_NAN, bool MASK, class E>
__device__ __forceinline__ void f6_epilogue(const E& e, const OutView& o, int m0, int n0, const float (&sa)[4],
                                            const uint2 (&sb)[4][4]) {
  constexpr uint32_t ESZ = MODE == OUT_BF16 ? 2 : 4;
  const uint32_t ldo = (uint32_t)o.ld;
  const unsigned long long first = (unsigned long long)m0 * ldo + n0;
  const rsrc_t r = make_rsrc(static_cast<uint8_t*>(o.out) + first * ESZ,
                             ((unsigned long long)o.rows * ldo - first) * ESZ);
  const uint32_t voff = ((uint32_t)e.out_row(0) * ldo + (uint32_t)e.out_col(0, 0)) * ESZ;
  // rows of this lane inside the written range (MASK)
  bool row_in[E::MI];
#pragma unroll
  for (int i = 0; i < E::MI; ++i) {
    const int row = m0 + e.out_row(i);
    row_in[i] = !MASK || (row >= o.row_lo && row < o.row_hi);
  }
  // column group (j, q) outer, rows i inner: each group's four B scales are
  // unpacked once and die after the group
#pragma unroll
  for (int j = 0; j < E::FN; ++j) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t off = voff + (uint32_t)(32 * j + 8 * q) * ESZ;
      const bool col_in = !MASK || n0 + e.out_col(j, q) < o.col_hi;
      float su[4], sg[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        su[t] = f6_bf16_at(sb[j][q], t);
        sg[t] = C::SWIGLU ? f6_bf16_at(sb[j + 2 < 4 ? j + 2 : j][q], t) : 0.0f;
      }
#pragma unroll
      for (int i = 0; i < E::MI; ++i) {
        const uint32_t soff = (uint32_t)(32 * i) * ldo * ESZ;
        const bool in = !MASK || (row_in[i] && col_in);
        if constexpr (MODE == OUT_I32) {
          if (in)
            __builtin_amdgcn_raw_buffer_store_b128(
                v4i{e.acc_int(i, j, 4 * q), e.acc_int(i, j, 4 * q + 1), e.acc_int(i, j, 4 * q + 2),
                    e.acc_int(i, j, 4 * q + 3)},
                r, off, soff, 0);
          if constexpr (C::SWIGLU) {
            __builtin_amdgcn_raw_buffer_store_b128(
                v4i{e.acc_int(i, j + 2, 4 * q), e.acc_int(i, j + 2, 4 * q + 1), e.acc_int(i, j + 2, 4 * q + 2),
                    e.acc_int(i, j + 2, 4 * q + 3)},
                r, off + (uint32_t)o.n * ESZ, soff, 0);
          }
        } else {
          float v[4];
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            float x = e.acc_value(i, j, 4 * q + t) * sa[i];
            x = x * su[t];
            if constexpr (C::SWIGLU) {
              float g = e.acc_value(i, j + 2, 4 * q + t) * sa[i];
              g = g * sg[t];
              x = swiglu(x, g);
            } else if constexpr (EPI == EPI_RELU2) {
              x = apply_epi(x, EPI_RELU2);
            }
            v[t] = x;
          }
          if constexpr (MODE == OUT_BF16) {
            uint32_t lo, hi;
            if constexpr (NO_NAN) {
              lo = pack_bf16x2_nonan(v[0], v[1]);
              hi = pack_bf16x2_nonan(v[2], v[3]);
            } else {
              lo = f32_to_bf16_rne(v[0]) | (f32_to_bf16_rne(v[1]) << 16);
              hi = f32_to_bf16_rne(v[2]) | (f32_to_bf16_rne(v[3]) << 16);
            }
            if (in) __builtin_amdgcn_raw_buffer_store_b64(v2i{(int)lo, (int)hi}, r, off, soff, 0);
          } else {
            if (in)
              __builtin_amdgcn_raw_buffer_store_b128(
                  v4i{__float_as_int(v[0]), __float_as_int(v[1]), __float_as_int(v[2]), __float_as_int(v[3])}, r,
                  off, soff, 0);
          }
        }
      }
      // one column group at a time: keeps accumulator reads and scale
      // unpacking from being hoisted ahead of their use
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

// bf16 epilogue through LDS.  Each wave writes its WROWS-row bf16 results
// into its own region of the (now idle) ring, then reads the region back
// row-contiguously and writes whole row segments with 16-byte stores,
// instead of 32 rows x 16 bytes per store instruction.  16-byte unit u
// (columns 8u .. 8u+7) of row r sits at r * PITCH + 16 * (u ^ swz(r)):
//  * 128 columns (PITCH 256, 16 units): swz(r) = r % 16;
//  * 64 columns, SwiGLU (PITCH 128, 8 units): swz(r) = (r / 2) % 8.
// Both keep the writes (lanes 0-15 hold rows r .. r+15 of one unit) and the
// reads (16 lanes hold one or two whole rows) free of bank conflicts.
template <class C, int EPI, bool NO_NAN, bool MASK, class E>
__device__ __forceinline__ void mfma32_epilogue_lds(const E& e, const OutView& o, uint8_t* smem, int m0, int n0,
                                                    const float (&sa)[4], const uint2 (&sb)[4][4]) {
  constexpr int UNITS = E::TN / 8;
  constexpr int PITCH = 16 * UNITS;
  auto swz = [](int r) { return UNITS == 16 ? (r & 15) : ((r >> 1) & 7); };
  // With bounded scales (NO_NAN) the engine's power-of-two factor folds into
  // the A scale: UNSCALE * sa is exact below 2^48, so stored * (UNSCALE * sa)
  // is the same real product as (stored * UNSCALE) * sa and rounds alike.
  float sx[E::MI];
#pragma unroll
  for (int i = 0; i < E::MI; ++i) sx[i] = NO_NAN ? sa[i] * E::UNSCALE : sa[i];
  auto scaled = [&](int i, int j, int x) {
    return (NO_NAN ? e.acc_stored(i, j, x) : e.acc_value(i, j, x)) * sx[i];
  };
  // every wave has finished reading the ring
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  uint8_t* region = smem + (size_t)e.wave * E::WROWS * PITCH;
  const int lane = e.lane;
  const int half = 8 * (lane >> 5);  // columns +4 .. +7 of a unit
#pragma unroll
  for (int j = 0; j < E::FN; ++j) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float su[4], sg[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        su[t] = f6_bf16_at(sb[j][q], t);
        sg[t] = C::SWIGLU ? f6_bf16_at(sb[j + 2 < 4 ? j + 2 : j][q], t) : 0.0f;
      }
      const int u = 4 * j + q;  // columns 32j + 8q .. +7
      float v[E::MI][4];        // [row i][column t]
      if constexpr (C::SWIGLU) {
        float up[E::MI][4], gt[E::MI][4];
        float gmax = 0.0f;
#pragma unroll
        for (int i = 0; i < E::MI; ++i)
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            up[i][t] = scaled(i, j, 4 * q + t);
            up[i][t] = up[i][t] * su[t];
            gt[i][t] = scaled(i, j + 2, 4 * q + t);
            gt[i][t] = gt[i][t] * sg[t];
            gmax = __builtin_fmaxf(gmax, __builtin_fabsf(gt[i][t]));
          }
        // one wave-uniform choice per 16 outputs: the hardware exp2 /
        // reciprocal path where it is accurate (fmax skips a NaN gate, which
        // gives NaN on either path)
        if (__all(gmax <= SWIGLU_FAST_MAX)) {
#pragma unroll
          for (int i = 0; i < E::MI; ++i)
#pragma unroll
            for (int t = 0; t < 4; ++t) v[i][t] = swiglu_fast(up[i][t], gt[i][t]);
        } else {
#pragma unroll
          for (int i = 0; i < E::MI; ++i)
#pragma unroll
            for (int t = 0; t < 4; ++t) v[i][t] = swiglu(up[i][t], gt[i][t]);
        }
      } else {
#pragma unroll
        for (int i = 0; i < E::MI; ++i)
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            float x = scaled(i, j, 4 * q + t);
            x = x * su[t];
            if constexpr (EPI == EPI_RELU2) x = apply_epi(x, EPI_RELU2);
            v[i][t] = x;
          }
      }
#pragma unroll
      for (int i = 0; i < E::MI; ++i) {
        uint32_t lo, hi;
        if constexpr (NO_NAN) {
          lo = pack_bf16x2_nonan(v[i][0], v[i][1]);
          hi = pack_bf16x2_nonan(v[i][2], v[i][3]);
        } else {
          lo = f32_to_bf16_rne(v[i][0]) | (f32_to_bf16_rne(v[i][1]) << 16);
          hi = f32_to_bf16_rne(v[i][2]) | (f32_to_bf16_rne(v[i][3]) << 16);
        }
        const int r = 32 * i + (lane & 31);
        *reinterpret_cast<uint2*>(region + r * PITCH + 16 * (u ^ swz(r)) + half) = make_uint2(lo, hi);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // read back 64 / UNITS rows per instruction and store whole row segments
  const uint32_t ldo = (uint32_t)o.ld;
  const unsigned long long first = (unsigned long long)m0 * ldo + n0;
  const rsrc_t rs = make_rsrc(static_cast<uint8_t*>(o.out) + first * 2, ((unsigned long long)o.rows * ldo - first) * 2);
  constexpr int ROWS = 64 / UNITS;
  const int rr = lane / UNITS, u = lane % UNITS;
  const uint32_t voff = ((uint32_t)(e.wm * E::WROWS + rr) * ldo + (uint32_t)(e.wn * E::TN + 8 * u)) * 2u;
  const bool col_in = !MASK || n0 + e.wn * E::TN + 8 * u < o.col_hi;
#pragma unroll
  for (int t = 0; t < E::WROWS / ROWS; ++t) {
    const int r = ROWS * t + rr;
    const uint4 x = *reinterpret_cast<const uint4*>(region + r * PITCH + 16 * (u ^ swz(r)));
    const int row = m0 + e.wm * E::WROWS + r;
    if (!MASK || (col_in && row >= o.row_lo && row < o.row_hi))
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4i, x), rs, voff, (uint32_t)(ROWS * t) * ldo * 2u,
                                             0);
  }
}

// B scales of a 32x32-engine tile.  Before the K loop each wave copies its
// window of TN columns (SwiGLU: TN up, then the same TN gate columns, 256
// bytes either way) into its own 256-byte slot past the ring with one
// direct-to-LDS dword load per lane: lane l fetches scales 2l, 2l + 1 (for
// SwiGLU lanes 32.. the gate's).  The loop's final wait for every vector
// load covers the copy, so the epilogue reads the slot after the loop;
// neither holds a register across the loop.  Columns at or past the
// buffer's range (col_hi with MASK) read as zeros.  OUT_I32 reads none.
constexpr int MFMA32_SCALE_BYTES = 4 * 256;

template <class C, int MODE, bool MASK = false, class E>
__device__ __forceinline__ void mfma32_prefetch_b_scales(const E& e, const OutView& o, int n0, uint32_t slot) {
  if constexpr (MODE != OUT_I32) {
    const int c0 = n0 + e.wn * E::TN;  // the window's first column
    const int lane = e.lane;
    const int col = C::SWIGLU ? c0 + 2 * (lane & 31) + (lane >> 5) * o.n : c0 + 2 * lane;
    const unsigned long long cols = MASK ? (unsigned long long)o.col_hi : (C::SWIGLU ? 2ull : 1ull) * o.n;
    lds_dma4(buffer_words(o.b_scale, 2 * cols), 2u * (uint32_t)col, 0u, slot);
  }
}

// sb[j][q]: the four bf16 B scales of fragment j, register group q (j >= FN:
// the gate's), from the wave's slot.
template <class C, class E>
__device__ __forceinline__ void mfma32_read_b_scales(const E& e, const uint8_t* slot, uint2 (&sb)[4][4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int jj = j < E::FN ? j : j - E::FN;
      const int c = e.out_col(jj, q) - e.wn * E::TN;
      sb[j][q] = *reinterpret_cast<const uint2*>(slot + 2 * c + (j < E::FN ? 0 : 2 * E::TN));
    }
}

// Epilogue of the 32x32 engines after the K loop: OUT_I32 and OUT_F32 store
// directly; bf16 goes through LDS, with the hardware conversion when no
// value can be NaN.  That holds when every scale is below 2^48 in
// magnitude: |acc| < 2^31, so each scaled product stays below 2^127 and
// finite, ReLU^2 of a finite value is no NaN, and SwiGLU of finite up and
// gate is finite or +-0 (a large negative gate gives gate / inf = -0) or
// +-inf, never NaN.  Larger or non-finite scales round in software.
// smem: the ring, followed by the scale slots.
template <class C, int MODE, int EPI, bool MASK = false, class E>
__device__ __forceinline__ void mfma32_finish(const E& e, const OutView& o, uint8_t* smem, int m0, int n0,
                                              const float (&sa)[4]) {
  static_assert(!(MASK && C::SWIGLU), "masked tiles are plain");
  if constexpr (MODE == OUT_I32) {
    const uint2 none[4][4] = {};
    f6_epilogue<C, OUT_I32, EPI_NONE, false, MASK>(e, o, m0, n0, sa, none);
    return;
  }
  uint2 sb[4][4];
  mfma32_read_b_scales<C>(e, smem + E::LDS_BYTES + 256 * e.wave, sb);
  if constexpr (MODE == OUT_F32) {
    f6_epilogue<C, OUT_F32, EPI, false, MASK>(e, o, m0, n0, sa, sb);
  } else {
    constexpr uint32_t F32_LIM = (127u + 48u) << 23, BF16_LIM = (127u + 48u) << 7;
    bool bounded = true;
#pragma unroll
    for (int i = 0; i < E::MI; ++i) bounded = bounded && (__float_as_uint(sa[i]) & 0x7F800000u) < F32_LIM;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint2 w = sb[j][q];
        bounded = bounded && (w.x & 0x7F80u) < BF16_LIM && (w.x & 0x7F800000u) < (BF16_LIM << 16) &&
                  (w.y & 0x7F80u) < BF16_LIM && (w.y & 0x7F800000u) < (BF16_LIM << 16);
      }
    if (__all(bounded)) mfma32_epilogue_lds<C, EPI, true, MASK>(e, o, smem, m0, n0, sa, sb);
    else mfma32_epilogue_lds<C, EPI, false, MASK>(e, o, smem, m0, n0, sa, sb);
  }
}

// Adds a wave's exact integer sums into the int32 buffer out ([M, ld],
// SwiGLU: up columns, then the gate's at +n), as a K slice of a large-K
// launch does.  Integer adds commute, so the total is exact and the same in
// every order.
template <class C, class E>
__device__ __forceinline__ void f6_add_i32(const E& e, int32_t* out, int ld, int n, int m0, int n0) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    int32_t* row = out + (long)(m0 + e.out_row(i)) * ld + n0;
#pragma unroll
    for (int j = 0; j < E::FN; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int c = e.out_col(j, q) + t;
          __hip_atomic_fetch_add(row + c, e.acc_int(i, j, 4 * q + t), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          if constexpr (C::SWIGLU)
            __hip_atomic_fetch_add(row + n + c, e.acc_int(i, j + 2, 4 * q + t), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        }
  }
}

// One output tile of the fp6 GEMM: tile index `tile` in the XCD-aware order
// of dense_tile_coords.  OUT_I32_ADD: K slice blockIdx.y of F6_MAX_K values
// (the last one shorter), added into the int32 buffer p.out ([M, b_cols]).
template <class C, int MODE, int EPI, bool PERSIST = false>
__device__ __forceinline__ void f6_gemm_tile(const DenseArgs& p, uint8_t* smem, int tile) {
  using E = F6Engine<C>;
  constexpr bool RAW = MODE == OUT_I32 || MODE == OUT_I32_ADD;
  const int tiles_m = p.M / C::BM;
  const int tiles_n = p.N / C::BN;
  int tm, tn;
  dense_tile_coords(tile, tiles_m, tiles_n, p.group_m, tm, tn);
  const int m0 = tm * C::BM;
  const int n0 = tn * C::BN;
  int k0 = 0, klen = p.K;
  if constexpr (MODE == OUT_I32_ADD) {
    k0 = (int)blockIdx.y * F6_MAX_K;
    klen = min(F6_MAX_K, p.K - k0);
  }
  E e;
  e.template setup<PERSIST>(smem, p.a, p.b, m0, tn, p.K / 64, f6_operand_bytes(p.M, p.K),
                            f6_operand_bytes(p.b_cols, p.K), k0 / 64);
  float sa[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) sa[i] = RAW ? 0.0f : load_bf16(p.a_scale + m0 + e.out_row(i));
  const OutView o = dense_view<C, RAW ? OUT_I32 : MODE>(p);
  if constexpr (!RAW) mfma32_prefetch_b_scales<C, MODE>(e, o, n0, e.lds0 + E::LDS_BYTES + 256u * e.wave);
  e.run(klen / 128);
  if constexpr (MODE == OUT_I32_ADD)
    f6_add_i32<C>(e, static_cast<int32_t*>(p.out), p.b_cols, p.N, m0, n0);
  else
    mfma32_finish<C, MODE, EPI>(e, o, smem, m0, n0, sa);
}

// One kernel per output mode and epilogue (chosen by the host), so that
// each holds a single straight-line epilogue.  One workgroup per tile.
template <class C, int MODE, int EPI>
__global__ __launch_bounds__(256) void f6_gemm_kernel(const DenseArgs p) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[F6Engine<C>::LDS_BYTES + MFMA32_SCALE_BYTES];
  f6_gemm_tile<C, MODE, EPI>(p, smem, blockIdx.x);
}

// Persistent schedule: gridDim.x workgroups (a multiple of 8, at most one
// per resident slot) take tiles blockIdx.x, blockIdx.x + gridDim.x, ...; a
// workgroup therefore stays on one XCD, as in the one-tile-per-workgroup
// order.  Between tiles, every wave has finished reading LDS before the next
// tile's prologue refills it.
template <class C, int MODE, int EPI>
__global__ __launch_bounds__(256) void f6_gemm_persistent(const DenseArgs p) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[F6Engine<C>::LDS_BYTES + MFMA32_SCALE_BYTES];
  const int tiles = (p.M / C::BM) * (p.N / C::BN);
  for (int t = blockIdx.x; t < tiles; t += gridDim.x) {
    f6_gemm_tile<C, MODE, EPI, true>(p, smem, t);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  }
}

}  // namespace shk
