// int4 x int4 subchannel GEMM on the fp6 MFMA.
//
// out = epilogue(sum over K groups g of (float(A_g @ B_g) * a_scale[m, g]) *
// b_scale[g, n]), groups of S = 32, 64, 128 or 256 K values, summed in fp32
// in group order (api.py:299-325).  The operands are the fp6 blocks of
// shk_f6.h.
//
// Each group's partial products must be scaled on their own, so every S K
// values the accumulators are folded into fp32 totals with VALU work; that
// fold, not the MFMA, bounds this kernel.  The design keeps it at two VALU
// operations per value (a multiply by a * b from a rank-1 MFMA, and the add;
// see fold()) and lets other waves' MFMAs run meanwhile:
//  * the MFMA is the scaled form (v_mfma_scale_f32_32x32x64_f8f6f4) with a
//    scale of 2^3 on both v/8 operands, so the accumulators hold the exact
//    integer partial sums (no x64 pass), and the first MFMA of each block in
//    a group takes 0 as its C operand (no clearing pass);
//  * a wave owns 64 x 64 outputs (4 accumulators of 32 x 32 and 64 fp32
//    totals), so a wave stays within 256 registers and two 4-wave
//    workgroups of 128 x 128 share a CU: while one wave folds, the other
//    wave on its SIMD issues MFMAs;
//  * the accumulators are VGPRs (the MFMA reads and writes them there), so
//    the fold reads them directly instead of copying each out of an AGPR;
//  * the scales reach LDS by LDS-DMA in the same stream as the operands,
//    so no load the compiler tracks sits in the K loop.
//
// Two engines fill the same 72 KiB ring: groups of S = 256 run F6SubEngine
// below (three 128-K slots, four scale slots), groups of S = 32, 64 and 128
// run F6SubEngine64 (six 64-K slots, two groups per stage or one or two
// stages per group, eight scale slots; described above it).  The table
// entry's num_stages (3) is that of the 128-K engine; its LDS the largest
// layout, the 64-K engine's for groups of 32.
//
// Pipeline of F6SubEngine (that of shk_f6small.h): 128-K stages (two 32 x 64
// fp6 blocks per 32-row panel; 12 KiB of A and 12 KiB of B) in a ring of three
// slots. Stage k: wait for this wave's DMA of stage k+1 and its LDS reads of
// stage k (with every fragment register of that set as an operand), then the
// barrier; 8 MFMAs on the fragments of stage k (two 64-K steps of 2 x 2
// blocks), each followed by two of the 16 LDS reads of stage k+1 into the
// other register set, the first seven carrying the DMA loads of stage k+3 into
// slot k % 3 (six operand loads and one scale load per wave).  A group is two
// stages (S = 256); after its last stage the wave waits for the reads of the
// next stage (naming their registers, so no compiler copy of a fragment
// precedes its data) and folds.  128-K stages halve the barriers and waits of
// 64-K ones, and give each stage's reads a whole stage of MFMAs to land.
//
// Scales of group g sit in slot g % 4 of a small ring: the a_scale dword
// holding row r's scale (dword-aligned pair (e & ~1, e | 1) of e = row * G +
// g) at 4 r, and the 128 b_scale values at 512.  With groups of 256 the scales
// of a group load with its first stage, three stages before that stage (by the
// previous group's second stage; those of groups 0 and 1 in the prologue).
// The slot a load writes last held the scales of a group every wave has
// folded before the stage's barrier.
#pragma once

#include <type_traits>

#include "shk_f6.h"

namespace shk {

// The fast fold of one group for a wave's 2 x 2 blocks of 32 x 32:
// tot += part * ab, ab[i][j] = a_scale (rows of block i) x b_scale (columns
// of block j) from one two-block rank-1 MFMA per column block j
// (v_mfma_f32_32x32x1_2b_f32: block i takes the second operand from lanes
// 32i .. 32i+31, so lanes 0-31 give the a_scale of block 0's rows and lanes
// 32-63 that of block 1's; both halves give block j's b_scale as the first
// operand).  Its output blocks are laid out as the accumulators (lane l: row
// l % 32 of the block, its 16 columns), and each product of two bf16 values
// is exact in fp32.  sa_bits / sb_bits: the bf16 bits of the lane's scales
// (rows out_row(0), out_row(1); columns 32j + lane % 32).
typedef float f6_v32f __attribute__((ext_vector_type(32)));
__device__ __forceinline__ void f6sub_fold_fast(const v16f (&acc)[2][2], float (&tot)[2][2][16], int lane,
                                                const uint32_t (&sa_bits)[2], const uint32_t (&sb_bits)[2]) {
  const float av = __uint_as_float((lane < 32 ? sa_bits[0] : sa_bits[1]) << 16);
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const f6_v32f ab = __builtin_amdgcn_mfma_f32_32x32x1f32(__uint_as_float(sb_bits[j] << 16), av, f6_v32f{}, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float x = acc[i][j][r] * ab[16 * i + r];
        tot[i][j][r] = tot[i][j][r] + x;
      }
  }
}

template <class C>
struct F6SubEngine {
  static constexpr int P = 3;                       // ring slots
  static constexpr int NW = 4;
  static constexpr int PANEL = 2 * F6_BLOCK;        // 32 rows x 128 K: 3 KiB
  static constexpr int OPB = 4 * PANEL;             // 128 rows x 128 K: 12 KiB
  static constexpr int STAGE = 2 * OPB;             // 24 KiB
  static constexpr int RING = P * STAGE;            // 72 KiB
  static constexpr int SCALE_SLOT = 768;            // 128 a dwords + 128 b halves
  static constexpr int LDS_BYTES = RING + 4 * SCALE_SLOT;
  static constexpr int OPW = STAGE / 1024 / NW;     // 6 operand loads per wave per stage
  static constexpr int DPW = OPW + 1;               // and one scale load
  static constexpr int TN = 64;                     // output columns per wave
  static constexpr int FN = 2;
  static_assert(C::BM == 128 && C::BROWS == 128 && C::WM == 2 && C::WN == 2 && C::SUBCH && !C::SWIGLU,
                "128 x 128 tiles of 2 x 2 waves, subchannel, plain epilogue");
  static constexpr int SPG = 2;                     // stages per group of 256 K

  v16f acc[2][2];
  float tot[2][2][16];
  v6i fa[2][2][2];  // [set][step][i]
  v6i fb[2][2][2];  // [set][step][j]
  uint32_t voff[OPW];
  v4i rs;        // operand DMA resource (waves 0-1: A, 2-3: B)
  v4i rss;       // scale DMA resource (waves 0-1: a_scale, 2-3: b_scale)
  int sbase;     // waves 0-1: element index row * G of the lane's row; 2-3: byte of its b_scale pair
  int groups;    // G = K / S
  int sb_row;    // bytes of one b_scale row (N * 2)
  uint32_t lds0;
  int lane, wave, wm, wn, m0;
  // every group so far took the fast fold: all totals are sums of finite
  // products below 2^110 in magnitude, so none is NaN
  bool all_fast;

  __device__ __forceinline__ int out_row(int i) const { return wm * 64 + 32 * i + (lane & 31); }
  __device__ __forceinline__ int out_col(int j, int q) const { return wn * TN + 32 * j + 8 * q + 4 * (lane >> 5); }

  // a6 / b6: block-format operands; tile rows m0 (A) and n0 (B).
  __device__ __forceinline__ void setup(uint8_t* smem, const uint8_t* a6, const uint8_t* b6, int m0_, int n0,
                                        int kb, unsigned long long a_bytes, unsigned long long b_bytes,
                                        const uint16_t* a_scale, const uint16_t* b_scale, int m_rows, int n_cols,
                                        int g) {
    lane = threadIdx.x & 63;
    wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    wm = wave % 2;
    wn = wave / 2;
    m0 = m0_;
    groups = g;
    lds0 = lds_address(smem);
    const unsigned long long panel_bytes = (unsigned long long)kb * F6_BLOCK;
    const bool is_a = wave < 2;
    const unsigned long long first = (unsigned long long)((is_a ? m0 : n0) / 32) * panel_bytes;
    rs = buffer_words((is_a ? a6 : b6) + first, (is_a ? a_bytes : b_bytes) - first);
    // DMA load c of this wave fills stage bytes [1024 * (OPW*wave + c), +1024):
    // panel o / PANEL of the operand, byte o % PANEL of its two blocks
#pragma unroll
    for (int c = 0; c < OPW; ++c) {
      const uint32_t o = 1024u * (OPW * wave + c) + 16u * lane - (is_a ? 0u : (uint32_t)OPB);
      voff[c] = (o / PANEL) * (uint32_t)panel_bytes + o % PANEL;
    }
    sb_row = 2 * n_cols;
    if (is_a) {
      rss = buffer_words(a_scale, 2ull * (unsigned long long)m_rows * g);
      sbase = (m0 + 64 * wave + lane) * g;
    } else {
      rss = buffer_words(b_scale, 2ull * (unsigned long long)g * n_cols);
      sbase = 2 * (n0 + 2 * lane);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          acc[i][j][r] = 0.0f;
          tot[i][j][r] = 0.0f;
        }
    all_fast = true;
  }

  // byte offset of this lane's scale dword for group g
  __device__ __forceinline__ uint32_t scale_voff(int g) const {
    return wave < 2 ? (uint32_t)(2 * (sbase + g)) & ~3u : (uint32_t)(g * sb_row + sbase);
  }
  // LDS destination of this wave's scale load for group g
  __device__ __forceinline__ uint32_t scale_m0(int g) const {
    return lds0 + (uint32_t)RING + (uint32_t)(g & 3) * SCALE_SLOT + (wave < 2 ? 256u * wave : 512u);
  }

  struct Reads {
    uint32_t a16, a8, b16, b8;
    __device__ __forceinline__ void add(uint32_t d) {
      a16 += d;
      a8 += d;
      b16 += d;
      b8 += d;
    }
  };
  // this lane's read addresses in a slot: the wave's A panel 0 and B panel 0
  // (panel i adds PANEL * i, step 1 adds one block)
  __device__ __forceinline__ Reads reads_of_slot(int slot) const {
    const uint32_t s = lds0 + (uint32_t)slot * STAGE;
    const uint32_t a = s + 2u * wm * PANEL, b = s + OPB + 2u * wn * PANEL;
    return Reads{a + 16u * lane, a + 1024u + 8u * lane, b + 16u * lane, b + 1024u + 8u * lane};
  }

  // LDS read Q (0..15) of a stage into set S: per step (Q / 8), fragments
  // A0, B0, B1, A1 (the order of first use), each as its 16-byte then its
  // 8-byte part.
  template <int S, int Q>
  __device__ __forceinline__ void read(const Reads& r) {
    constexpr int ST = Q / 8;
    constexpr int F = (Q % 8) / 2;
    constexpr bool IS_A = F == 0 || F == 3;
    constexpr int IDX = F == 0 ? 0 : (F == 3 ? 1 : F - 1);
    constexpr int OFF = IDX * PANEL + ST * F6_BLOCK;
    v6i& dst = IS_A ? fa[S][ST][IDX] : fb[S][ST][IDX];
    if constexpr (Q % 2 == 0) {
      v4i x;
      asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(x) : "v"(IS_A ? r.a16 : r.b16), "i"(OFF));
      // a whole new value: the fragment's previous contents are dead here
      dst = __builtin_shufflevector(x, x, 0, 1, 2, 3, -1, -1);
    } else {
      v2i y;
      asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(y) : "v"(IS_A ? r.a8 : r.b8), "i"(OFF));
      dst.s4 = y.x;
      dst.s5 = y.y;
    }
  }
  template <int S, int... Q>
  __device__ __forceinline__ void reads(const Reads& r, std::integer_sequence<int, Q...>) {
    (read<S, Q>(r), ...);
  }

  // MFMA T (0..7) of a stage on set S (step T / 4, A fragment (T % 4) / 2,
  // B fragment T % 2; the step-0 MFMAs of a group's first stage (ZERO) take
  // 0 as their C operand), fused for T < OPW with operand DMA load T and,
  // in a group's second stage, for T = OPW with the scale load of the stage
  // loaded now (which is the first stage of its group: the first stage of a
  // group loads the second stage of a group whose scales are already
  // loaded), then (READ) LDS reads 2T, 2T+1 of the next stage into the
  // other set.  Every stage of a kind runs the same branch-free sequence
  // (see shk_f6.h).
  template <int S, int T, bool ZERO, bool READ>
  __device__ __forceinline__ void tick(const Reads& r, const v4i& rs_st, uint32_t so, uint32_t m0_st,
                                       const v4i& rss_st, uint32_t svo, uint32_t sm0, int s8) {
    constexpr int ST = T / 4, I = (T % 4) / 2, J = T % 2;
    constexpr bool Z = ZERO && ST == 0;
    // the compiler writes M0 before each statement; the MFMA is the wait
    // state the LDS-DMA load needs after that write
    if constexpr (T < OPW) {
      if constexpr (Z)
        asm volatile(
            "v_mfma_scale_f32_32x32x64_f8f6f4 %0, %1, %2, 0, %3, %3 op_sel_hi:[0,0,0] cbsz:2 blgp:2\n\t"
            "buffer_load_dwordx4 %4, %5, %6 offen lds"
            : "+v"(acc[I][J])
            : "v"(fb[S][ST][J]), "v"(fa[S][ST][I]), "v"(s8), "v"(voff[T]), "s"(rs_st), "s"(so),
              "{m0}"(m0_st + 1024u * T)
            : "memory");
      else
        asm volatile(
            "v_mfma_scale_f32_32x32x64_f8f6f4 %0, %1, %2, %0, %3, %3 op_sel_hi:[0,0,0] cbsz:2 blgp:2\n\t"
            "buffer_load_dwordx4 %4, %5, %6 offen lds"
            : "+v"(acc[I][J])
            : "v"(fb[S][ST][J]), "v"(fa[S][ST][I]), "v"(s8), "v"(voff[T]), "s"(rs_st), "s"(so),
              "{m0}"(m0_st + 1024u * T)
            : "memory");
    } else if constexpr (T == OPW && !ZERO) {
      static_assert(!Z, "the scale load rides on a step-1 MFMA");
      asm volatile(
          "v_mfma_scale_f32_32x32x64_f8f6f4 %0, %1, %2, %0, %3, %3 op_sel_hi:[0,0,0] cbsz:2 blgp:2\n\t"
          "buffer_load_dword %4, %5, 0 offen lds"
          : "+v"(acc[I][J])
          : "v"(fb[S][ST][J]), "v"(fa[S][ST][I]), "v"(s8), "v"(svo), "s"(rss_st), "{m0}"(sm0)
          : "memory");
    } else {
      asm volatile("v_mfma_scale_f32_32x32x64_f8f6f4 %0, %1, %2, %0, %3, %3 op_sel_hi:[0,0,0] cbsz:2 blgp:2"
                   : "+v"(acc[I][J])
                   : "v"(fb[S][ST][J]), "v"(fa[S][ST][I]), "v"(s8));
    }
    if constexpr (READ) {
      read<1 - S, 2 * T>(r);
      read<1 - S, 2 * T + 1>(r);
    }
  }
  template <int S, bool ZERO, bool READ, int... T>
  __device__ __forceinline__ void ticks(const Reads& r, const v4i& rs_st, uint32_t so, uint32_t m0_st,
                                        const v4i& rss_st, uint32_t svo, uint32_t sm0, int s8,
                                        std::integer_sequence<int, T...>) {
    (tick<S, T, ZERO, READ>(r, rs_st, so, m0_st, rss_st, svo, sm0, s8), ...);
  }

  // fence<4> (s_nop 4: 5 wait states) stands between VALU writes of the
  // accumulators (the clear before the loop) and the first asm MFMA that
  // writes them: a VALU write followed by an MFMA reading the register
  // needs 2 wait states.  fence<7> (5 x s_nop 7: 40 wait states) stands
  // between the last asm MFMA and any other access to its result: an XDL
  // MFMA of up to 16 passes needs 18 wait states before a VALU, VMEM, LDS or
  // v_accvgpr_read instruction reads its destination or a VALU instruction
  // overwrites it (the 8-pass fp6 forms need 10), so 40 covers every MFMA
  // here with margin.  Every accumulator is an operand of the fence, so no
  // compiler access (or register-allocator copy on a merge) crosses it.
  template <int N>
  __device__ __forceinline__ void fence() {
    static_assert(N == 4 || N == 7, "wait states");
    if constexpr (N == 4)
      asm volatile("s_nop 4" : "+v"(acc[0][0]), "+v"(acc[0][1]), "+v"(acc[1][0]), "+v"(acc[1][1]));
    else
      asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7"
                   : "+v"(acc[0][0]), "+v"(acc[0][1]), "+v"(acc[1][0]), "+v"(acc[1][1]));
  }
  // This wave's LDS reads into set S have landed.  The reads are asm
  // statements, so the compiler does not know that their registers are
  // written later than the statement: every register of the set is an
  // operand here, so none is copied before the data is in.
  template <int S>
  __device__ __forceinline__ void frag_fence() {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(fa[S][0][0]), "+v"(fa[S][0][1]), "+v"(fb[S][0][0]), "+v"(fb[S][0][1]), "+v"(fa[S][1][0]),
                   "+v"(fa[S][1][1]), "+v"(fb[S][1][0]), "+v"(fb[S][1][1])::"memory");
  }

  // Stage k (128 K) on set S (ZERO: the first stage of a group; READ: the
  // next stage's fragments are read here, else after the group's fold, and
  // the group's scales are read at the top).
  // Top: this wave's DMA of stage k+1 has landed (that of k+2, issued by
  // the previous stage: DPW loads after a group's second stage or the
  // prologue, OPW after a first stage, may be outstanding) and its LDS
  // reads of stage k are done, then the barrier:
  // stage k+1 and the scales it loaded are complete in LDS, no wave still
  // reads slot k % 3, and every wave has folded the groups before stage k.
  // Past the last stage the DMA loads go through zero-record resources into
  // a slot that holds no live data, and the reads fetch a stale slot into
  // the set no MFMA uses.
  template <int S, bool ZERO, bool READ>
  __device__ __forceinline__ void stage(const uint8_t* smem, const Reads& r, int k, int nst, int slot,
                                        const v4i& rs_end, const v4i& rss_end, int s8) {
    wait_vmcnt<ZERO ? DPW : OPW>();
    frag_fence<S>();
    asm volatile("s_barrier" ::: "memory");
    if constexpr (!READ) load_scales(smem, k / SPG);
    const int kl = k + P;  // the stage loaded now
    const bool live = kl < nst;
    const v4i rs_st = live ? rs : rs_end;
    const v4i rss_st = live ? rss : rss_end;
    const int gl = kl / SPG;
    const uint32_t so = live ? (uint32_t)kl * PANEL : 0u;
    const uint32_t svo = live ? scale_voff(gl) : 0u;
    const uint32_t m0_st = lds0 + (uint32_t)slot * STAGE + 1024u * OPW * wave;
    ticks<S, ZERO, READ>(r, rs_st, so, m0_st, rss_st, svo, scale_m0(gl), s8,
                         std::make_integer_sequence<int, 8>{});
  }
  static __device__ __forceinline__ void advance(Reads& r, int& slot) {
    r.add(slot == 1 ? (uint32_t)(-2 * STAGE) : (uint32_t)STAGE);
    slot = slot == 2 ? 0 : slot + 1;
  }

  // Folds group g's partial sums into the totals:
  // tot += (float(part) * a_scale[row, g]) * b_scale[g, col].
  //
  // Fast form, two VALU operations per value: tot += part * ab with
  // ab = a_scale * b_scale from rank-1 MFMAs (f6sub_fold_fast).  It
  // gives the same bits as the reference's order whenever every scale of the
  // group is zero or a normal number of magnitude in [2^-60, 2^48): part is
  // an integer of at most 15 significant bits (|part| <= 64 * 256) and a has
  // 8, so part * a is exact, and a * b (16 bits, within the normal range) is
  // exact too; both orders therefore round the same real product part*a*b
  // once.  (A zero product's sign may differ, which changes no sum: the
  // totals start at +0, and x + -0 = x + +0 for every x.)  A wave whose
  // scales fall outside that range folds in the reference's order.
  // The scales of group g this lane folds with: a_scale of its rows
  // out_row(0), out_row(1) and b_scale of columns 32j + lane % 32 of its
  // window.  Read at the top of the group's last stage (after its barrier,
  // so the DMA that loaded them is complete and visible), so that their
  // latency passes under that stage's MFMAs.
  uint32_t sa_bits[2], sb_bits[2];
  __device__ __forceinline__ void load_scales(const uint8_t* smem, int g) {
    const uint8_t* sl = smem + RING + (g & 3) * SCALE_SLOT;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int row = out_row(i);
      const uint32_t w = *reinterpret_cast<const uint32_t*>(sl + 4 * row);
      const int e = (m0 + row) * groups + g;
      sa_bits[i] = (e & 1) ? (w >> 16) : (w & 0xFFFFu);
    }
#pragma unroll
    for (int j = 0; j < 2; ++j)
      sb_bits[j] = *reinterpret_cast<const uint16_t*>(sl + 512 + 2 * (wn * TN + 32 * j + (lane & 31)));
  }

  __device__ __forceinline__ void fold(const uint8_t* smem, int g) {
    const uint8_t* sl = smem + RING + (g & 3) * SCALE_SLOT;
    auto in_range = [](uint32_t b) {
      return (b & 0x7FFFu) == 0u || (((b >> 7) & 0xFFu) - (127u - 60u)) < 108u;
    };
    const bool ok = in_range(sa_bits[0]) && in_range(sa_bits[1]) && in_range(sb_bits[0]) && in_range(sb_bits[1]);
    if (__all(ok)) {
      f6sub_fold_fast(acc, tot, lane, sa_bits, sb_bits);
      return;
    }
    all_fast = false;
    float sa[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) sa[i] = __uint_as_float(sa_bits[i] << 16);
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint2 w = *reinterpret_cast<const uint2*>(sl + 512 + 2 * out_col(j, q));
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            float x = acc[i][j][4 * q + t] * sa[i];
            x = x * f6_bf16_at(w, t);
            tot[i][j][4 * q + t] = tot[i][j][4 * q + t] + x;
          }
      }
  }

  // RAW mode: adds group g's exact integer partial sums into the totals,
  // which then hold int32 bit patterns.
  __device__ __forceinline__ void fold_raw() {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int x = 0; x < 16; ++x)
          tot[i][j][x] = __int_as_float(__float_as_int(tot[i][j][x]) + (int)acc[i][j][x]);
  }

  // After group g's last stage (on set S, which read nothing): the MFMA
  // results land, the group folds, then the next stage's fragments are read
  // into set 1 - S from `r`.  Reading them after the fold rather than during
  // the stage keeps their 48 registers free while the fold needs its own
  // beside the totals and accumulators.
  template <bool RAW, int S>
  __device__ __forceinline__ void end_group(const uint8_t* smem, int g, const Reads& r) {
    fence<7>();
    if constexpr (RAW) fold_raw();
    else fold(smem, g);
    // keeps the reads (and their destination registers) after the fold
    __builtin_amdgcn_sched_barrier(0);
    reads<1 - S>(r, std::make_integer_sequence<int, 16>{});
  }

  // nst: 128-K stages (a multiple of 2).  RAW: the totals receive the exact
  // int32 sum over all K instead of the scaled fp32 sum.  The step-0 MFMAs
  // of every group's first stage take 0 as their C operand in both modes: no
  // MFMA reads accumulators that VALU code wrote (between the tiles of a
  // persistent workgroup, such a read returned stale values).
  template <bool RAW>
  __device__ __forceinline__ void run(const uint8_t* smem, int nst) {
    const v4i rs_end = v4i{rs.x, rs.y, 0, rs.w};
    const v4i rss_end = v4i{rss.x, rss.y, 0, rss.w};
    const int s8 = 130;  // E8M0 2^3: both operands hold v/8
    // stages 0 .. P-1 (zeros past the last stage) with their groups' scales
#pragma unroll
    for (int st = 0; st < P; ++st) {
      const bool live = st < nst;
#pragma unroll
      for (int c = 0; c < OPW; ++c)
        lds_dma16(live ? rs : rs_end, voff[c], live ? (uint32_t)st * PANEL : 0u,
                  lds0 + (uint32_t)st * STAGE + 1024u * (OPW * wave + c));
      // (the nops: the wait states after the M0 write and after a VALU write
      // of the resource's SGPRs, as in lds_dma16)
      asm volatile("s_nop 4\n\tbuffer_load_dword %0, %1, 0 offen lds"
                   :
                   : "v"(live ? scale_voff(st / SPG) : 0u), "s"(live ? rss : rss_end), "{m0}"(scale_m0(st / SPG))
                   : "memory");
    }
    wait_vmcnt<(P - 1) * DPW>();
    asm volatile("s_barrier" ::: "memory");
    reads<0>(reads_of_slot(0), std::make_integer_sequence<int, 16>{});
    fence<4>();
    Reads r = reads_of_slot(1);
    int slot = 0;
    int k = 0;
    // The reads after the last fold fetch a stale slot into the set no MFMA
    // uses (set 0); they land, naming their registers, before the registers
    // could be reused.
    for (; k < nst; k += 2) {
      stage<0, true, true>(smem, r, k, nst, slot, rs_end, rss_end, s8);
      advance(r, slot);
      stage<1, false, false>(smem, r, k + 1, nst, slot, rs_end, rss_end, s8);
      end_group<RAW, 1>(smem, k / 2, r);
      advance(r, slot);
    }
    frag_fence<0>();
    // the loads past the last stage land before the workgroup's LDS is freed
    wait_vmcnt<0>();
    fence<7>();
  }
};

// The 64-K-stage engine, for groups of 32, 64 and 128: one 32 x 64 fp6
// block per 32-row panel per stage (6 KiB of A and 6 KiB of B) in a ring of
// six slots, SPG = 1 or 2 stages per group (SPG = 0: two groups of 32 per
// stage, see half_stage).  Stage k: wait for this wave's DMA
// of stage k+1, then the barrier; 4 MFMAs on the fragments of stage k,
// carrying (the first two) the 8 LDS reads of stage k+1's fragments and the
// 4 DMA loads of stage k+6 into slot k % 6 (3 operand loads and one scale
// load per wave); then a fence that waits for this stage's LDS reads with
// every fragment register of the other set as an operand.  Stage k loads
// the scales of stage k+6's group into slot (group % 8) of the scale ring
// (laid out as for the 128-K engine): with one stage per group, groups k ..
// k+6 are live at stage k (group k folds after it), and every earlier group
// folded before stage k's barrier; with two groups per stage, a slot holds
// both groups' a_scale dwords and b_scale rows.  (The 128-K engine does not
// fit 256 registers with a fold after every stage.)
template <class C, int SPG>
struct F6SubEngine64 {
  static constexpr int P = 6;                       // ring slots
  static constexpr int NW = 4;
  static constexpr int OPB = 4 * F6_BLOCK;          // 128 rows x 64 K: 6 KiB
  static constexpr int STAGE = 2 * OPB;             // 12 KiB
  static constexpr int RING = P * STAGE;            // 72 KiB
  static constexpr bool HALF = SPG == 0;            // groups of 32: two per stage
  static constexpr int SCALE_SLOT = HALF ? 1024 : 768;  // 128 a dwords + 128 b halves (HALF: two b rows)
  static constexpr int SCALE_SLOTS = 8;
  static constexpr int LDS_BYTES = RING + SCALE_SLOTS * SCALE_SLOT;
  static constexpr int OPW = STAGE / 1024 / NW;     // 3 operand loads per wave per stage
  static constexpr int DPW = OPW + 1;               // and one scale load
  static constexpr int TN = 64;                     // output columns per wave
  static constexpr int FN = 2;
  static_assert(C::BM == 128 && C::BROWS == 128 && C::WM == 2 && C::WN == 2 && C::SUBCH && !C::SWIGLU,
                "128 x 128 tiles of 2 x 2 waves, subchannel, plain epilogue");
  static_assert(SPG == 0 || SPG == 1 || SPG == 2 || SPG == 4, "groups of 32, 64, 128 or 256 K");

  v16f acc[2][2];
  float tot[2][2][16];
  v6i fa[2][2];  // [set][i]
  v6i fb[2][2];  // [set][j]
  uint32_t voff[OPW];
  v4i rs;        // operand DMA resource (waves 0-1: A, 2-3: B)
  v4i rss;       // scale DMA resource (waves 0-1: a_scale, 2-3: b_scale)
  int sbase;     // waves 0-1: element index row * G of the lane's row; 2-3: byte of its b_scale pair
                 // (HALF: the byte offset of the lane's scale dword of group 0; wave 3: of group 1)
  int groups;    // G = K / S
  int sb_row;    // bytes of one b_scale row (N * 2)
  uint32_t lds0;
  int lane, wave, wm, wn, m0;
  // every group so far took the fast fold: all totals are sums of finite
  // products below 2^110 in magnitude, so none is NaN
  bool all_fast;
  // HALF: the last group folded; later ones are not (their partial sums
  // are zeros; a caller whose K ends inside a stage sets it, so that no
  // scale past its last group is read into the totals).  The default, the
  // largest int, makes every comparison with it a constant.
  int fold_last;

  __device__ __forceinline__ int out_row(int i) const { return wm * 64 + 32 * i + (lane & 31); }
  __device__ __forceinline__ int out_col(int j, int q) const { return wn * TN + 32 * j + 8 * q + 4 * (lane >> 5); }

  // a6 / b6: block-format operands; tile rows m0 (A) and n0 (B).
  __device__ __forceinline__ void setup(uint8_t* smem, const uint8_t* a6, const uint8_t* b6, int m0_, int n0,
                                        int kb, unsigned long long a_bytes, unsigned long long b_bytes,
                                        const uint16_t* a_scale, const uint16_t* b_scale, int m_rows, int n_cols,
                                        int g) {
    lane = threadIdx.x & 63;
    wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    wm = wave % 2;
    wn = wave / 2;
    m0 = m0_;
    groups = g;
    lds0 = lds_address(smem);
    const unsigned long long panel_bytes = (unsigned long long)kb * F6_BLOCK;
    const bool is_a = wave < 2;
    const unsigned long long first = (unsigned long long)((is_a ? m0 : n0) / 32) * panel_bytes;
    rs = buffer_words((is_a ? a6 : b6) + first, (is_a ? a_bytes : b_bytes) - first);
    // DMA load c of this wave fills stage bytes [1024 * (OPW*wave + c), +1024):
    // panel o / F6_BLOCK of the operand, byte o % F6_BLOCK of its block
#pragma unroll
    for (int c = 0; c < OPW; ++c) {
      const uint32_t o = 1024u * (OPW * wave + c) + 16u * lane - (is_a ? 0u : (uint32_t)OPB);
      voff[c] = (o / F6_BLOCK) * (uint32_t)panel_bytes + o % F6_BLOCK;
    }
    sb_row = 2 * n_cols;
    if (is_a) {
      rss = buffer_words(a_scale, 2ull * (unsigned long long)m_rows * g);
      sbase = (m0 + 64 * wave + lane) * g;
    } else {
      rss = buffer_words(b_scale, 2ull * (unsigned long long)g * n_cols);
      sbase = 2 * (n0 + 2 * lane);
    }
    // (G is a multiple of 4 with groups of 32, so row * G is even)
    if constexpr (HALF) sbase = is_a ? 2 * sbase : sbase + (wave == 3 ? sb_row : 0);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          acc[i][j][r] = 0.0f;
          tot[i][j][r] = 0.0f;
        }
    all_fast = true;
    fold_last = 0x7FFFFFFF;
  }

  // byte offset of this lane's scale dword for stage st: waves 0-1 the
  // a_scale dword of the stage's group (HALF: the dword holding both of its
  // groups, the first one even), waves 2-3 two b_scale columns of it (HALF:
  // wave 3 those of the second group)
  __device__ __forceinline__ uint32_t scale_voff(int st) const {
    if constexpr (HALF) return (uint32_t)(sbase + (wave < 2 ? 4 * st : 2 * st * sb_row));
    const int g = st / (HALF ? 1 : SPG);
    return wave < 2 ? (uint32_t)(2 * (sbase + g)) & ~3u : (uint32_t)(g * sb_row + sbase);
  }
  // LDS destination of this wave's scale load for stage st
  __device__ __forceinline__ uint32_t scale_m0(int st) const {
    const int slot = (HALF ? st : st / (HALF ? 1 : SPG)) & (SCALE_SLOTS - 1);
    return lds0 + (uint32_t)RING + (uint32_t)slot * SCALE_SLOT +
           (wave < 2 ? 256u * wave : (HALF && wave == 3 ? 768u : 512u));
  }

  struct Reads {
    uint32_t a16, a8, b16, b8;
    __device__ __forceinline__ void add(uint32_t d) {
      a16 += d;
      a8 += d;
      b16 += d;
      b8 += d;
    }
  };
  __device__ __forceinline__ Reads reads_of_slot(int slot) const {
    const uint32_t s = lds0 + (uint32_t)slot * STAGE;
    const uint32_t a = s + 2u * wm * F6_BLOCK, b = s + OPB + 2u * wn * F6_BLOCK;
    return Reads{a + 16u * lane, a + 1024u + 8u * lane, b + 16u * lane, b + 1024u + 8u * lane};
  }

  // LDS read Q (0..7) of a stage into set S: fragments A0, B0, B1, A1 (the
  // order of first use), each as its 16-byte then its 8-byte part.
  template <int S, int Q>
  __device__ __forceinline__ void read(const Reads& r) {
    constexpr int F = Q / 2;
    constexpr bool IS_A = F == 0 || F == 3;
    constexpr int IDX = F == 0 ? 0 : (F == 3 ? 1 : F - 1);
    constexpr int OFF = IDX * F6_BLOCK;
    v6i& dst = IS_A ? fa[S][IDX] : fb[S][IDX];
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

  // MFMA T (0..3) of a stage on set S (A fragment T/2, B fragment T%2; ZERO:
  // the group's first, C = 0), fused with DMA load T (T < 3: operands; 3:
  // the scale dword), followed by LDS reads 4T .. 4T+3 of the next stage
  // for T < 2: all reads go out early, so they have landed when the stage's
  // closing fence waits for them.
  // PART 1: the DMA load only, PART 2: the LDS reads only (the two halves
  // of a HALF stage).
  template <int S, int T, bool ZERO, int PART = 0>
  __device__ __forceinline__ void tick(const Reads& r, const v4i& rs_st, uint32_t so, uint32_t m0_st,
                                       const v4i& rss_st, uint32_t svo, uint32_t sm0, int s8) {
    constexpr int I = T / 2, J = T % 2;
    if constexpr (PART == 2) {
      if constexpr (ZERO)
        asm volatile("v_mfma_scale_f32_32x32x64_f8f6f4 %0, %1, %2, 0, %3, %3 op_sel_hi:[0,0,0] cbsz:2 blgp:2"
                     : "+v"(acc[I][J])
                     : "v"(fb[S][J]), "v"(fa[S][I]), "v"(s8)
                     : "memory");
      else
        asm volatile("v_mfma_scale_f32_32x32x64_f8f6f4 %0, %1, %2, %0, %3, %3 op_sel_hi:[0,0,0] cbsz:2 blgp:2"
                     : "+v"(acc[I][J])
                     : "v"(fb[S][J]), "v"(fa[S][I]), "v"(s8)
                     : "memory");
    } else if constexpr (T < OPW) {
      // the compiler writes M0 before the statement; the MFMA is the wait
      // state the LDS-DMA load needs after that write
      if constexpr (ZERO)
        asm volatile(
            "v_mfma_scale_f32_32x32x64_f8f6f4 %0, %1, %2, 0, %3, %3 op_sel_hi:[0,0,0] cbsz:2 blgp:2\n\t"
            "buffer_load_dwordx4 %4, %5, %6 offen lds"
            : "+v"(acc[I][J])
            : "v"(fb[S][J]), "v"(fa[S][I]), "v"(s8), "v"(voff[T]), "s"(rs_st), "s"(so), "{m0}"(m0_st + 1024u * T)
            : "memory");
      else
        asm volatile(
            "v_mfma_scale_f32_32x32x64_f8f6f4 %0, %1, %2, %0, %3, %3 op_sel_hi:[0,0,0] cbsz:2 blgp:2\n\t"
            "buffer_load_dwordx4 %4, %5, %6 offen lds"
            : "+v"(acc[I][J])
            : "v"(fb[S][J]), "v"(fa[S][I]), "v"(s8), "v"(voff[T]), "s"(rs_st), "s"(so), "{m0}"(m0_st + 1024u * T)
            : "memory");
    } else {
      if constexpr (ZERO)
        asm volatile(
            "v_mfma_scale_f32_32x32x64_f8f6f4 %0, %1, %2, 0, %3, %3 op_sel_hi:[0,0,0] cbsz:2 blgp:2\n\t"
            "buffer_load_dword %4, %5, 0 offen lds"
            : "+v"(acc[I][J])
            : "v"(fb[S][J]), "v"(fa[S][I]), "v"(s8), "v"(svo), "s"(rss_st), "{m0}"(sm0)
            : "memory");
      else
        asm volatile(
            "v_mfma_scale_f32_32x32x64_f8f6f4 %0, %1, %2, %0, %3, %3 op_sel_hi:[0,0,0] cbsz:2 blgp:2\n\t"
            "buffer_load_dword %4, %5, 0 offen lds"
            : "+v"(acc[I][J])
            : "v"(fb[S][J]), "v"(fa[S][I]), "v"(s8), "v"(svo), "s"(rss_st), "{m0}"(sm0)
            : "memory");
    }
    if constexpr (T < 2 && PART != 1) {
      read<1 - S, 4 * T>(r);
      read<1 - S, 4 * T + 1>(r);
      read<1 - S, 4 * T + 2>(r);
      read<1 - S, 4 * T + 3>(r);
    }
  }

  // fence<4> (s_nop 4: 5 wait states) stands between VALU writes of the
  // accumulators (the fold's clears) and the first asm MFMA that reads
  // them as its C operand: a VALU write followed by an MFMA reading the
  // register needs 2 wait states.  fence<7> (5 x s_nop 7: 40 wait states)
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
    if constexpr (N == 4)
      asm volatile("s_nop 4" : "+v"(acc[0][0]), "+v"(acc[0][1]), "+v"(acc[1][0]), "+v"(acc[1][1]));
    else
      asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7"
                   : "+v"(acc[0][0]), "+v"(acc[0][1]), "+v"(acc[1][0]), "+v"(acc[1][1]));
  }
  // Every total is an operand: a fold's adds are all done here, so none is
  // moved below the next MFMAs, which write the accumulators it reads (the
  // compiler would give those MFMAs a second accumulator set).
  __device__ __forceinline__ void tot_fence() {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        float* t = tot[i][j];
        asm volatile(""
                     : "+v"(t[0]), "+v"(t[1]), "+v"(t[2]), "+v"(t[3]), "+v"(t[4]), "+v"(t[5]), "+v"(t[6]),
                       "+v"(t[7]), "+v"(t[8]), "+v"(t[9]), "+v"(t[10]), "+v"(t[11]), "+v"(t[12]), "+v"(t[13]),
                       "+v"(t[14]), "+v"(t[15]));
      }
  }
  // This wave's LDS reads into set S have landed; every register of the set
  // is an operand, so no copy of it is placed before this point.
  template <int S>
  __device__ __forceinline__ void frag_fence() {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(fa[S][0]), "+v"(fa[S][1]), "+v"(fb[S][0]), "+v"(fb[S][1])::"memory");
  }

  // Stage k on set S (ZERO: the first stage of a group).  Past the last
  // stage the DMA loads go through zero-record resources.
  template <int S, bool ZERO>
  __device__ __forceinline__ void stage(const Reads& r, int k, int nst, int slot, const v4i& rs_end,
                                        const v4i& rss_end, int s8) {
    wait_vmcnt<(P - 2) * DPW>();
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    const int kl = k + P;  // the stage loaded now
    const bool live = kl < nst;
    const v4i rs_st = live ? rs : rs_end;
    const v4i rss_st = live ? rss : rss_end;
    const uint32_t so = live ? (uint32_t)kl * F6_BLOCK : 0u;
    const uint32_t svo = live ? scale_voff(kl) : 0u;
    const uint32_t m0_st = lds0 + (uint32_t)slot * STAGE + 1024u * OPW * wave;
    const uint32_t sm0 = scale_m0(kl);
    tick<S, 0, ZERO>(r, rs_st, so, m0_st, rss_st, svo, sm0, s8);
    tick<S, 1, ZERO>(r, rs_st, so, m0_st, rss_st, svo, sm0, s8);
    tick<S, 2, ZERO>(r, rs_st, so, m0_st, rss_st, svo, sm0, s8);
    tick<S, 3, ZERO>(r, rs_st, so, m0_st, rss_st, svo, sm0, s8);
    frag_fence<1 - S>();
  }

  // HALF: stage k holds groups 2k (K 0..31 of every block) and 2k+1 (K
  // 32..63); lanes 0-31 of each fragment hold K 0..31 of their row or column
  // and lanes 32-63 K 32..63, and each lane's E8M0 scale applies to its own
  // 32 values.  The four MFMAs of group 2k take scale 2^3 on lanes 0-31 and
  // 2^-127 on lanes 32-63 (s_lo), whose products (at most 2^-249 in
  // magnitude) round away in the fp32 result; they carry the stage's DMA
  // loads.  Then group 2k's fold; the same four MFMAs with the scales swapped
  // (s_hi) take group 2k+1 and carry the reads of stage k+1's fragments; the
  // wait for those reads; group 2k+1's fold.
  template <int S, bool RAW>
  __device__ __forceinline__ void half_stage(const uint8_t* smem, const Reads& r, int k, int nst, int slot,
                                             const v4i& rs_end, const v4i& rss_end, int s_lo, int s_hi) {
    wait_vmcnt<(P - 2) * DPW>();
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    const int kl = k + P;  // the stage loaded now
    const bool live = kl < nst;
    const v4i rs_st = live ? rs : rs_end;
    const v4i rss_st = live ? rss : rss_end;
    const uint32_t so = live ? (uint32_t)kl * F6_BLOCK : 0u;
    const uint32_t svo = live ? scale_voff(kl) : 0u;
    const uint32_t m0_st = lds0 + (uint32_t)slot * STAGE + 1024u * OPW * wave;
    const uint32_t sm0 = scale_m0(kl);
    tick<S, 0, true, 1>(r, rs_st, so, m0_st, rss_st, svo, sm0, s_lo);
    tick<S, 1, true, 1>(r, rs_st, so, m0_st, rss_st, svo, sm0, s_lo);
    tick<S, 2, true, 1>(r, rs_st, so, m0_st, rss_st, svo, sm0, s_lo);
    tick<S, 3, true, 1>(r, rs_st, so, m0_st, rss_st, svo, sm0, s_lo);
    fence<7>();
    if constexpr (RAW) fold_raw();
    else if (2 * k <= fold_last) fold<false>(smem, 2 * k);
    tot_fence();
    tick<S, 0, true, 2>(r, rs_st, so, m0_st, rss_st, svo, sm0, s_hi);
    tick<S, 1, true, 2>(r, rs_st, so, m0_st, rss_st, svo, sm0, s_hi);
    tick<S, 2, true, 2>(r, rs_st, so, m0_st, rss_st, svo, sm0, s_hi);
    tick<S, 3, true, 2>(r, rs_st, so, m0_st, rss_st, svo, sm0, s_hi);
    frag_fence<1 - S>();
    fence<7>();
    if constexpr (RAW) fold_raw();
    else if (2 * k + 1 <= fold_last) fold<false>(smem, 2 * k + 1);
    tot_fence();
  }
  static __device__ __forceinline__ void advance(Reads& r, int& slot) {
    r.add(slot == P - 2 ? (uint32_t)(-(P - 1) * STAGE) : (uint32_t)STAGE);
    slot = slot == P - 1 ? 0 : slot + 1;
  }

  // Folds group g's partial sums into the totals:
  // tot += (float(part) * a_scale[row, g]) * b_scale[g, col].
  //
  // Fast form, two VALU operations per value: tot += part * ab with
  // ab = a_scale * b_scale from rank-1 MFMAs (f6sub_fold_fast).  It
  // gives the same bits as the reference's order whenever every scale of the
  // group is zero or a normal number of magnitude in [2^-60, 2^48): part is
  // an integer of at most 15 significant bits (|part| <= 64 * 256) and a has
  // 8, so part * a is exact, and a * b (16 bits, within the normal range) is
  // exact too; both orders therefore round the same real product part*a*b
  // once.  (A zero product's sign may differ, which changes no sum: the
  // totals start at +0, and x + -0 = x + +0 for every x.)  A wave whose
  // scales fall outside that range folds in the reference's order.
  // FAST false (one stage per group): every wave folds in the reference's
  // order, three VALU operations per value and no rank-1 products, whose
  // two 32-register results do not fit beside the registers of two stages
  // per loop trip; all_fast still records whether the scales were in range.
  template <bool FAST>
  __device__ __forceinline__ void fold(const uint8_t* smem, int g) {
    const uint8_t* sl = smem + RING + ((HALF ? g >> 1 : g) & (SCALE_SLOTS - 1)) * SCALE_SLOT;
    const uint8_t* sbl = sl + 512 + (HALF ? 256 * (g & 1) : 0);  // the group's b_scale row
    uint32_t sa_bits[2], sb_bits[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int row = out_row(i);
      const uint32_t w = *reinterpret_cast<const uint32_t*>(sl + 4 * row);
      const int e = (m0 + row) * groups + g;
      sa_bits[i] = (e & 1) ? (w >> 16) : (w & 0xFFFFu);
    }
#pragma unroll
    for (int j = 0; j < 2; ++j)
      sb_bits[j] = *reinterpret_cast<const uint16_t*>(sbl + 2 * (wn * TN + 32 * j + (lane & 31)));
    auto in_range = [](uint32_t b) {
      return (b & 0x7FFFu) == 0u || (((b >> 7) & 0xFFu) - (127u - 60u)) < 108u;
    };
    const bool ok = in_range(sa_bits[0]) & in_range(sa_bits[1]) & in_range(sb_bits[0]) & in_range(sb_bits[1]);
    if constexpr (FAST) {
      if (__all(ok)) {
        f6sub_fold_fast(acc, tot, lane, sa_bits, sb_bits);
        return;
      }
      all_fast = false;
    } else {
      if (!__all(ok)) all_fast = false;
    }
    float sa[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) sa[i] = __uint_as_float(sa_bits[i] << 16);
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint2 w = *reinterpret_cast<const uint2*>(sbl + 2 * out_col(j, q));
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            float x = acc[i][j][4 * q + t] * sa[i];
            x = x * f6_bf16_at(w, t);
            tot[i][j][4 * q + t] = tot[i][j][4 * q + t] + x;
          }
      }
  }

  // RAW mode: adds group g's exact integer partial sums into the totals,
  // which then hold int32 bit patterns.
  __device__ __forceinline__ void fold_raw() {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int x = 0; x < 16; ++x)
          tot[i][j][x] = __int_as_float(__float_as_int(tot[i][j][x]) + (int)acc[i][j][x]);
  }

  // nst: 64-K stages (a multiple of SPG).  RAW: the totals receive the exact
  // int32 sum over all K instead of the scaled fp32 sum.  Every group's first
  // MFMA takes 0 as its C operand in both modes: no MFMA reads accumulators
  // that VALU code wrote (between the tiles of a persistent workgroup, such a
  // read returned stale values).
  template <bool RAW>
  __device__ __forceinline__ void run(const uint8_t* smem, int nst) {
    const v4i rs_end = v4i{rs.x, rs.y, 0, rs.w};
    const v4i rss_end = v4i{rss.x, rss.y, 0, rss.w};
    const int s8 = 130;  // E8M0 2^3: both operands hold v/8
    // stages 0 .. P-1 (zeros past the last stage) with their groups' scales
#pragma unroll
    for (int st = 0; st < P; ++st) {
      const bool live = st < nst;
#pragma unroll
      for (int c = 0; c < OPW; ++c)
        lds_dma16(live ? rs : rs_end, voff[c], live ? (uint32_t)st * F6_BLOCK : 0u,
                  lds0 + (uint32_t)st * STAGE + 1024u * (OPW * wave + c));
      // (the nops: the wait states after the M0 write and after a VALU write
      // of the resource's SGPRs, as in lds_dma16)
      asm volatile("s_nop 4\n\tbuffer_load_dword %0, %1, 0 offen lds"
                   :
                   : "v"(live ? scale_voff(st) : 0u), "s"(live ? rss : rss_end), "{m0}"(scale_m0(st))
                   : "memory");
    }
    wait_vmcnt<(P - 1) * DPW>();
    asm volatile("s_barrier" ::: "memory");
    Reads r = reads_of_slot(0);
    read<0, 0>(r);
    read<0, 1>(r);
    read<0, 2>(r);
    read<0, 3>(r);
    read<0, 4>(r);
    read<0, 5>(r);
    read<0, 6>(r);
    read<0, 7>(r);
    frag_fence<0>();
    fence<4>();
    r = reads_of_slot(1);
    int slot = 0;
    if constexpr (HALF) {
      const int s_lo = lane < 32 ? s8 : 0, s_hi = lane < 32 ? 0 : s8;
      for (int k = 0; k < nst; k += 2) {
        half_stage<0, RAW>(smem, r, k, nst, slot, rs_end, rss_end, s_lo, s_hi);
        advance(r, slot);
        half_stage<1, RAW>(smem, r, k + 1, nst, slot, rs_end, rss_end, s_lo, s_hi);
        advance(r, slot);
      }
    } else if constexpr (SPG == 1) {
      // one group per stage: two stages (one per register set) per trip,
      // each followed by its fold (nst is even: K is a multiple of 128)
      for (int k = 0; k < nst; k += 2) {
        stage<0, true>(r, k, nst, slot, rs_end, rss_end, s8);
        advance(r, slot);
        fence<7>();
        if constexpr (RAW) fold_raw();
        else fold<false>(smem, k);
        stage<1, true>(r, k + 1, nst, slot, rs_end, rss_end, s8);
        advance(r, slot);
        fence<7>();
        if constexpr (RAW) fold_raw();
        else fold<false>(smem, k + 1);
      }
    } else {
      for (int k = 0; k < nst; k += SPG) {
        // one group: SPG stages, alternating register sets (SPG is even)
        stage<0, true>(r, k, nst, slot, rs_end, rss_end, s8);
        advance(r, slot);
        stage<1, false>(r, k + 1, nst, slot, rs_end, rss_end, s8);
        advance(r, slot);
        if constexpr (SPG == 4) {
          stage<0, false>(r, k + 2, nst, slot, rs_end, rss_end, s8);
          advance(r, slot);
          stage<1, false>(r, k + 3, nst, slot, rs_end, rss_end, s8);
          advance(r, slot);
        }
        fence<7>();
        if constexpr (RAW) fold_raw();
        else fold<true>(smem, k / SPG);
      }
    }
    // the loads past the last stage land before the workgroup's LDS is freed
    wait_vmcnt<0>();
    fence<7>();
  }
};

// Stores a wave's 64 x 64 results v(i, j, x) (accumulator layout) as bf16
// through its own 8 KiB region of the idle ring: unit u = 4j + q (columns
// 8u .. 8u+7) of row r at r * 128 + 16 * (u ^ ((r / 2) % 8)), read back one
// 128-byte row segment per 8 lanes.
// NO_NAN: no value is NaN, so the hardware conversion (round to nearest
// even, which keeps a NaN's payload where torch writes 0x7FC0) gives torch's
// bits.  MASK: only rows [o.row_lo, o.row_hi) and columns below o.col_hi (a
// multiple of 8) are written (the ragged forward's tasks).
template <bool NO_NAN, bool MASK = false, class E, class V>
__device__ __forceinline__ void f6sub_store_bf16(const E& e, const OutView& o, uint8_t* smem, int m0, int n0,
                                                 V v) {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  uint8_t* region = smem + (size_t)e.wave * 64 * 128;
  const int lane = e.lane;
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int u = 4 * j + q;
      const int half = 8 * (lane >> 5);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int x = 4 * q;
        uint32_t lo, hi;
        if constexpr (NO_NAN) {
          lo = pack_bf16x2_nonan(v(i, j, x), v(i, j, x + 1));
          hi = pack_bf16x2_nonan(v(i, j, x + 2), v(i, j, x + 3));
        } else {
          lo = f32_to_bf16_rne(v(i, j, x)) | (f32_to_bf16_rne(v(i, j, x + 1)) << 16);
          hi = f32_to_bf16_rne(v(i, j, x + 2)) | (f32_to_bf16_rne(v(i, j, x + 3)) << 16);
        }
        const int r = 32 * i + (lane & 31);
        *reinterpret_cast<uint2*>(region + r * 128 + 16 * (u ^ ((r >> 1) & 7)) + half) = make_uint2(lo, hi);
      }
    }
  const uint32_t ldo = (uint32_t)o.ld;
  const unsigned long long first = (unsigned long long)m0 * ldo + n0;
  const rsrc_t rs = make_rsrc(static_cast<uint8_t*>(o.out) + first * 2, ((unsigned long long)o.rows * ldo - first) * 2);
  const int rr = lane / 8, u = lane % 8;
  const uint32_t voff = ((uint32_t)(e.wm * 64 + rr) * ldo + (uint32_t)(e.wn * 64 + 8 * u)) * 2u;
  const bool col_ok = !MASK || n0 + e.wn * 64 + 8 * u < o.col_hi;
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const int r = 8 * t + rr;
    const uint4 x = *reinterpret_cast<const uint4*>(region + r * 128 + 16 * (u ^ ((r >> 1) & 7)));
    const int row = m0 + e.wm * 64 + r;
    if (!MASK || (col_ok && row >= o.row_lo && row < o.row_hi))
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4i, x), rs, voff, (uint32_t)(8 * t) * ldo * 2u, 0);
  }
}

// fp32 / int32 results: four consecutive columns per store (MASK as for
// f6sub_store_bf16).
template <bool MASK = false, class E, class V>
__device__ __forceinline__ void f6sub_store_words(const E& e, const OutView& o, int m0, int n0, V v) {
  const uint32_t ldo = (uint32_t)o.ld;
  const unsigned long long first = (unsigned long long)m0 * ldo + n0;
  const rsrc_t r = make_rsrc(static_cast<uint8_t*>(o.out) + first * 4, ((unsigned long long)o.rows * ldo - first) * 4);
  const uint32_t voff = ((uint32_t)e.out_row(0) * ldo + (uint32_t)e.out_col(0, 0)) * 4u;
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int x = 4 * q;
        const int row = m0 + e.out_row(i), col = n0 + e.out_col(j, q);
        if (!MASK || (row >= o.row_lo && row < o.row_hi && col < o.col_hi))
          __builtin_amdgcn_raw_buffer_store_b128(v4i{v(i, j, x), v(i, j, x + 1), v(i, j, x + 2), v(i, j, x + 3)},
                                                 r, voff + (uint32_t)(32 * j + 8 * q) * 4u,
                                                 (uint32_t)(32 * i) * ldo * 4u, 0);
      }
}

// The engine for groups of S = 32 * G32: the 128-K-stage engine for 256,
// the 64-K-stage one for 32, 64 and 128 (G32 / 2 stages per group; 0: two
// groups per stage).
template <class C, int G32>
using F6SubEngineFor = std::conditional_t<G32 == 8, F6SubEngine<C>, F6SubEngine64<C, G32 / 2>>;
// The largest LDS layout of the subchannel kernels (the table entry's).
template <class C>
constexpr int f6_sub_lds_bytes() {
  return F6SubEngine<C>::LDS_BYTES > F6SubEngine64<C, 0>::LDS_BYTES ? F6SubEngine<C>::LDS_BYTES
                                                                       : F6SubEngine64<C, 0>::LDS_BYTES;
}

// One 128 x 128 output tile of the subchannel GEMM over fp6 blocks (p.a /
// p.b point at the converted A and B); G32 = S / 32.
template <class C, int MODE, int EPI, int G32>
__device__ __forceinline__ void f6_sub_tile(const DenseArgs& p, uint8_t* smem, int tile) {
  static_assert(G32 == 1 || G32 == 2 || G32 == 4 || G32 == 8, "groups of 32, 64, 128 or 256");
  using E = F6SubEngineFor<C, G32>;
  const int tiles_m = p.M / C::BM;
  const int tiles_n = p.N / C::BN;
  int tm, tn;
  dense_tile_coords(tile, tiles_m, tiles_n, p.group_m, tm, tn);
  const int m0 = tm * C::BM;
  const int n0 = tn * C::BN;
  E e;
  e.setup(smem, p.a, p.b, m0, n0, p.K / 64, f6_operand_bytes(p.M, p.K), f6_operand_bytes(p.N, p.K), p.a_scale,
          p.b_scale, p.M, p.N, p.K / p.subchannel);
  e.template run<MODE == OUT_I32>(smem, p.K / (G32 == 8 ? 128 : 64));
  const OutView o{p.out, p.b_scale, p.N, p.M, p.N, 0, p.M, p.N};
  if constexpr (MODE == OUT_I32) {
    f6sub_store_words(e, o, m0, n0, [&](int i, int j, int x) { return __float_as_int(e.tot[i][j][x]); });
  } else if constexpr (MODE == OUT_F32) {
    f6sub_store_words(e, o, m0, n0,
                      [&](int i, int j, int x) { return __float_as_int(apply_epi(e.tot[i][j][x], EPI)); });
  } else {
    auto val = [&](int i, int j, int x) { return apply_epi(e.tot[i][j][x], EPI); };
    if (e.all_fast) f6sub_store_bf16<true>(e, o, smem, m0, n0, val);
    else f6sub_store_bf16<false>(e, o, smem, m0, n0, val);
  }
}

// One kernel per output mode, epilogue and group size; one workgroup per
// tile, two workgroups per CU.
template <class C, int MODE, int EPI, int G32>
__global__ __launch_bounds__(256, 2) void f6_sub_kernel(const DenseArgs p) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[F6SubEngineFor<C, G32>::LDS_BYTES];
  f6_sub_tile<C, MODE, EPI, G32>(p, smem, blockIdx.x);
}

// Persistent schedule (as f6_gemm_persistent): gridDim.x workgroups stride
// over the tiles, with every LDS read done before the next tile's prologue.
template <class C, int MODE, int EPI, int G32>
__global__ __launch_bounds__(256, 2) void f6_sub_persistent(const DenseArgs p) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[F6SubEngineFor<C, G32>::LDS_BYTES];
  const int tiles = (p.M / C::BM) * (p.N / C::BN);
  for (int t = blockIdx.x; t < tiles; t += gridDim.x) {
    f6_sub_tile<C, MODE, EPI, G32>(p, smem, t);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  }
}

}  // namespace shk
