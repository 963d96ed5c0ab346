// Direct-to-LDS pipelined MFMA engine for the large dense tiles.
//
// K is consumed in stages of 64 source bytes per tile row: 128 K values for
// int4, 64 for int8.  The operand tiles stay packed in LDS.  The LDS-DMA form
// of the buffer load (`buffer_load_dwordx4 ... lds`) copies each 16-byte
// piece from HBM straight into a ring of P stage buffers, so the copy needs
// no staging registers and no VALU work.  With P = 4, the loads of a stage
// are issued three stages before the stage is consumed, which covers HBM
// latency with one wave per SIMD.
//
// Ring layouts.  A source row is K-contiguous for a "K-major" operand (A of
// NN/NT, B of NT) and tile-contiguous for an "MN-major" one (B of NN/TN, A of
// TN).
//  * A K-major stage holds ROWS x 64 bytes.  16-byte unit q of tile row r
//    sits at r*64 + 16*(q ^ swk(r)), with swk(r) = (r >> 1) & 3.
//  * An MN-major stage holds 64 source rows x 256 bytes (ROWS = 256).  Unit
//    u (tile rows 16u..16u+15) of source row kp sits at kp*256 + 16*(u ^
//    swm(kp)), with swm(kp) = (kp & 7) | ((kp & 16) >> 1).
// The swizzles act on 16-byte units, so each DMA lane still copies one
// contiguous 16-byte source piece; the swizzle is applied by choosing which
// piece a lane fetches.  Both swizzles were chosen by measurement
// (SQ_LDS_BANK_CONFLICT on gfx950): the fragment reads below are free of LDS
// bank conflicts, where the plain layouts conflict two- to sixteen-fold and
// (r >> 2) & 3 conflicts two-fold for ds_read_b128.
//
// Fragment reads.  An MFMA step (64 K values) takes a 16-value chunk per lane
// group g = lane / 16 from each of its 16 rows:
//  * int4: step s of a stage uses K values 32g + 16s + [0, 16).
//    - K-major: one ds_read_b128 of unit g per stage gives both steps'
//      packed bytes.
//    - MN-major: one ds_read_b64_tr_b8 per step.  Lane i of a 16-lane group
//      addresses source row 16g + 8s + i/2 at byte 8*(i%2) of the fragment's
//      unit, and receives the 8 bytes of those 8 rows of column i.
//  * int8: K values 16g + [0, 16).
//    - K-major: one ds_read_b128 of unit g.
//    - MN-major: two ds_read_b64_tr_b8, rows 16g + [0, 8) and 16g + [8, 16).
// Packed int4 bytes p0..p7 of a step are widened after the read to the chunk
// [lo(p0..3), hi(p0..3), lo(p4..7), hi(p4..7)] as 16*v.  Both operands get
// the same order (shk_common.h).
//
// Schedule.  Step t multiplies operand set t%2 while it prepares set
// (t+1)%2.  int4 widens the packed fragments of step t+1, which were read
// earlier, and refills the freed registers: MN-major fragments with step t+2,
// K-major fragments with the whole next stage at the stage's first step.
// int8 reads step t+1.  Stage k opens with its only barrier:
//  * before it, each wave waits for its own DMA of stage k+1, so after it
//    stage k+1 is complete (the reads issued during stage k target it);
//  * every wave has read all of stage k (before the barrier, which waits for
//    outstanding LDS reads), so the loads of stage k+P go into stage k's slot.
#pragma once

#include <utility>

#include "shk_fast.h"

namespace shk {

typedef __attribute__((address_space(3))) uint8_t lds_byte;
typedef __attribute__((address_space(3))) v2i lds_v2i;

// LDS byte address of a pointer into a __shared__ array.
__device__ __forceinline__ uint32_t lds_address(const uint8_t* p) {
  return (uint32_t)(uintptr_t)(const lds_byte*)p;
}

// Raw buffer resource words (stride 0, `bytes` records; reads past the end
// return zero) for use as an SGPR quad operand.
__device__ __forceinline__ v4i buffer_words(const void* base, unsigned long long bytes) {
  const unsigned long long a = (unsigned long long)base;
  const uint32_t n = bytes > 0xFFFFFFFFull ? 0xFFFFFFFFu : (uint32_t)bytes;
  return v4i{(int)(uint32_t)a, (int)((uint32_t)(a >> 32) & 0xFFFFu), (int)n, 0x00020000};
}

// One LDS-DMA load: lane L's 16 bytes at rsrc + voff + soff land at LDS
// address m0 + 16*L.  The compiler does not know about this write, so the
// waits for it are explicit (wait_vmcnt) and the asm clobbers memory.
// The asm opens with the wait states its operands need, which the compiler's
// hazard recognizer cannot insert because it does not see the load: 1 after
// the M0 write, and 5 after a VALU write of an SGPR the load reads (the
// compiler reloads spilled scalars such as the offset with v_readlane_b32,
// possibly right before the asm).  tests/_asm_check.py scans for the latter.
__device__ __forceinline__ void lds_dma16(const v4i& rs, uint32_t voff, uint32_t soff, uint32_t m0) {
  asm volatile(
      "s_nop 4\n\t"
      "buffer_load_dwordx4 %0, %1, %2 offen lds"
      :
      : "v"(voff), "s"(rs), "s"(soff), "{m0}"(m0)
      : "memory");
}

// The same with 4 bytes per lane: lane L's land at m0 + 4*L.
__device__ __forceinline__ void lds_dma4(const v4i& rs, uint32_t voff, uint32_t soff, uint32_t m0) {
  asm volatile(
      "s_nop 4\n\t"
      "buffer_load_dword %0, %1, %2 offen lds"
      :
      : "v"(voff), "s"(rs), "s"(soff), "{m0}"(m0)
      : "memory");
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is six bits");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__device__ __forceinline__ v2i ds_read_tr8(const uint8_t* p) {
  return __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i*)(const lds_byte*)p);
}

// One operand's part of a stage: where this lane's DMA pieces come from.
// HALF: tile rows below HALF come from the operand's first rows (columns);
// the rest, SwiGLU's gate half, are shifted by `gate`.
template <int BITS, bool KMAJOR, int ROWS, int NW, int HALF>
struct DmaOperand {
  static constexpr int BYTES = ROWS * 64;        // one stage
  static constexpr int BLK = BYTES / 1024 / NW;  // 1 KiB DMA blocks per wave per stage
  static_assert(BYTES % (1024 * NW) == 0, "a stage must split into whole 1 KiB blocks per wave");
  static_assert(KMAJOR || ROWS == 256, "the MN-major ring layout has 256-byte rows");
  uint32_t voff[BLK];

  // swk and swm of the ring layouts.
  static __device__ __forceinline__ uint32_t k_swz(uint32_t r) { return (r >> 1) & 3u; }
  static __device__ __forceinline__ uint32_t mn_swz(uint32_t kp) { return (kp & 7u) | ((kp & 16u) >> 1); }

  __device__ __forceinline__ void init(int wave, int lane, uint32_t ld, uint32_t gate) {
#pragma unroll
    for (int c = 0; c < BLK; ++c) {
      const int b = wave * BLK + c;
      if constexpr (KMAJOR) {
        const uint32_t r = 16u * b + lane / 4;
        const uint32_t q = (lane & 3) ^ k_swz(r);
        const uint32_t src = r < (uint32_t)HALF ? r : r - HALF + gate;
        voff[c] = src * ld + 16u * q;
      } else {
        const uint32_t kp = 4u * b + lane / 16;
        const uint32_t col = 16u * ((lane & 15) ^ mn_swz(kp));
        voff[c] = kp * ld + (col < (uint32_t)HALF ? col : col - HALF + gate);
      }
    }
  }

  // Source offset of stage `st`, shared by the wave.
  static __device__ __forceinline__ uint32_t soff(int st, uint32_t ld) {
    return KMAJOR ? 64u * (uint32_t)st : 64u * (uint32_t)st * ld;
  }

  // Issues this wave's blocks of one stage into the region at LDS address `dst`.
  __device__ __forceinline__ void issue(const v4i& rs, uint32_t so, uint32_t dst, int wave) const {
#pragma unroll
    for (int c = 0; c < BLK; ++c) issue_one(rs, so, dst, wave, c);
  }
  __device__ __forceinline__ void issue_one(const v4i& rs, uint32_t so, uint32_t dst, int wave, int c) const {
    lds_dma16(rs, voff[c], so, dst + (uint32_t)(wave * BLK + c) * 1024u);
  }
};

// Wait states between the accumulators' last non-asm access and the asm
// MFMAs (before the loop), and between the last asm MFMA and the first
// accumulator read (after it).  acc_fence<4> (5 wait states) covers the 2
// a VALU or v_accvgpr_write needs before an MFMA reads the register as its
// C operand; acc_fence<7> (3 x s_nop 7: 24 wait states) covers the 10 that
// v_mfma_i32_16x16x64_i8, an 8-pass form, needs before a VALU, memory or
// v_accvgpr_read instruction touches its result (18 for 16 passes).  Every
// accumulator is an operand, so the compiler cannot move an accumulator
// access across the statement.
template <int N>
__device__ __forceinline__ void acc_fence(v4i (&a)[8][8]) {
  static_assert(N == 4 || N == 7, "wait states");
  if constexpr (N == 4) {
    asm volatile("s_nop 4" : "+a"(a[0][0]), "+a"(a[0][1]), "+a"(a[0][2]), "+a"(a[0][3]), "+a"(a[0][4]), "+a"(a[0][5]), "+a"(a[0][6]), "+a"(a[0][7]), "+a"(a[1][0]), "+a"(a[1][1]), "+a"(a[1][2]), "+a"(a[1][3]), "+a"(a[1][4]), "+a"(a[1][5]), "+a"(a[1][6]), "+a"(a[1][7]), "+a"(a[2][0]), "+a"(a[2][1]), "+a"(a[2][2]), "+a"(a[2][3]), "+a"(a[2][4]), "+a"(a[2][5]), "+a"(a[2][6]), "+a"(a[2][7]), "+a"(a[3][0]), "+a"(a[3][1]), "+a"(a[3][2]), "+a"(a[3][3]), "+a"(a[3][4]), "+a"(a[3][5]), "+a"(a[3][6]), "+a"(a[3][7]), "+a"(a[4][0]), "+a"(a[4][1]), "+a"(a[4][2]), "+a"(a[4][3]), "+a"(a[4][4]), "+a"(a[4][5]), "+a"(a[4][6]), "+a"(a[4][7]), "+a"(a[5][0]), "+a"(a[5][1]), "+a"(a[5][2]), "+a"(a[5][3]), "+a"(a[5][4]), "+a"(a[5][5]), "+a"(a[5][6]), "+a"(a[5][7]), "+a"(a[6][0]), "+a"(a[6][1]), "+a"(a[6][2]), "+a"(a[6][3]), "+a"(a[6][4]), "+a"(a[6][5]), "+a"(a[6][6]), "+a"(a[6][7]), "+a"(a[7][0]), "+a"(a[7][1]), "+a"(a[7][2]), "+a"(a[7][3]), "+a"(a[7][4]), "+a"(a[7][5]), "+a"(a[7][6]), "+a"(a[7][7]));
  } else {
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" : "+a"(a[0][0]), "+a"(a[0][1]), "+a"(a[0][2]), "+a"(a[0][3]), "+a"(a[0][4]), "+a"(a[0][5]), "+a"(a[0][6]), "+a"(a[0][7]), "+a"(a[1][0]), "+a"(a[1][1]), "+a"(a[1][2]), "+a"(a[1][3]), "+a"(a[1][4]), "+a"(a[1][5]), "+a"(a[1][6]), "+a"(a[1][7]), "+a"(a[2][0]), "+a"(a[2][1]), "+a"(a[2][2]), "+a"(a[2][3]), "+a"(a[2][4]), "+a"(a[2][5]), "+a"(a[2][6]), "+a"(a[2][7]), "+a"(a[3][0]), "+a"(a[3][1]), "+a"(a[3][2]), "+a"(a[3][3]), "+a"(a[3][4]), "+a"(a[3][5]), "+a"(a[3][6]), "+a"(a[3][7]), "+a"(a[4][0]), "+a"(a[4][1]), "+a"(a[4][2]), "+a"(a[4][3]), "+a"(a[4][4]), "+a"(a[4][5]), "+a"(a[4][6]), "+a"(a[4][7]), "+a"(a[5][0]), "+a"(a[5][1]), "+a"(a[5][2]), "+a"(a[5][3]), "+a"(a[5][4]), "+a"(a[5][5]), "+a"(a[5][6]), "+a"(a[5][7]), "+a"(a[6][0]), "+a"(a[6][1]), "+a"(a[6][2]), "+a"(a[6][3]), "+a"(a[6][4]), "+a"(a[6][5]), "+a"(a[6][6]), "+a"(a[6][7]), "+a"(a[7][0]), "+a"(a[7][1]), "+a"(a[7][2]), "+a"(a[7][3]), "+a"(a[7][4]), "+a"(a[7][5]), "+a"(a[7][6]), "+a"(a[7][7]));
  }
}

template <class C>
struct DmaEngine {
  static constexpr int P = C::PIPE;
  static constexpr int NW = C::NT / 64;
  using OA = DmaOperand<C::BITS, C::A_KMAJOR, C::BM, NW, C::BM>;
  using OB = DmaOperand<C::BITS, C::B_KMAJOR, C::BROWS, NW, C::BHALF>;
  static constexpr int A_BYTES = OA::BYTES;
  static constexpr int STAGE = OA::BYTES + OB::BYTES;
  static constexpr int LDS_BYTES = P * STAGE;
  static constexpr int DPW = OA::BLK + OB::BLK;  // DMA loads per wave per stage
  static constexpr int STEPS = C::BK / 64;       // MFMA steps per stage
  static constexpr bool I4 = C::BITS == 4;
  // Eight waves (two per SIMD): each wave reads and widens a step's
  // fragments right before its MFMAs and the other wave of the SIMD fills
  // the gaps; four waves (one per SIMD) prepare the next step's operands
  // while multiplying the current ones.
  static constexpr bool PING = NW == 8;
  static constexpr int WSETS = PING ? 1 : 2;
  static_assert(C::MK == 64, "the DMA engine issues 16x16x64 MFMAs");
  static_assert(C::BK * C::BITS == 512, "a stage is 64 source bytes per row");
  static_assert(P >= 2 && (P - 2) * DPW < 64 && (P - 1) * DPW < 64, "vmcnt range");
  static_assert(LDS_BYTES <= 160 * 1024, "LDS budget");

  v4i acc[C::FM][C::FN2];
  // MFMA operands of the current and the next step (widened for int4), and
  // for int4 the packed fragments waiting to be widened: a whole stage
  // (ds_read_b128) for a K-major operand, one step for an MN-major one.
  template <bool KMAJOR>
  using Packed = typename std::conditional<!I4, v4i, typename std::conditional<KMAJOR, uint4, uint2>::type>::type;
  v4i wa[WSETS][C::FM];
  v4i wb[WSETS][C::FN2];
  Packed<C::A_KMAJOR> pa[C::FM];
  Packed<C::B_KMAJOR> pb[C::FN2];
  OA oa;
  OB ob;
  v4i rsa, rsb;
  uint32_t lda, ldb;
  // LDS byte offsets of this lane's fragment reads in the current read slot:
  // one for a K-major operand (fragment f adds 1024*f), one per fragment for
  // an MN-major operand (the second step / second half adds 2048).
  uint32_t rda[C::A_KMAJOR ? 1 : C::FM];
  uint32_t rdb[C::B_KMAJOR ? 1 : C::FN2];
  int lane, wave, wm, wn, slot;

  // First B tile row of fragment j relative to the wave's first up row.
  static constexpr int brow_rel(int j) { return j < C::FN ? 16 * j : C::BHALF + 16 * (j - C::FN); }

  __device__ __forceinline__ void init_reads() {
    lane = threadIdx.x & 63;
    wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    wm = wave % C::WM;
    wn = wave / C::WM;
    slot = 0;
    const uint32_t l15 = lane & 15;
    const uint32_t g = lane >> 4;
    const uint32_t kp = 16u * g + l15 / 2;
    const uint32_t half = 8u * (l15 & 1);
    if constexpr (C::A_KMAJOR) {
      rda[0] = (wm * C::TM + l15) * 64u + 16u * (g ^ OA::k_swz(l15));
    } else {
#pragma unroll
      for (int i = 0; i < C::FM; ++i) {
        const uint32_t u = (uint32_t)(wm * C::TM + 16 * i) / 16;
        rda[i] = kp * 256u + 16u * (u ^ OA::mn_swz(kp)) + half;
      }
    }
    if constexpr (C::B_KMAJOR) {
      rdb[0] = A_BYTES + (wn * C::TN + l15) * 64u + 16u * (g ^ OB::k_swz(l15));
    } else {
#pragma unroll
      for (int j = 0; j < C::FN2; ++j) {
        const uint32_t u = (uint32_t)(wn * C::TN + brow_rel(j)) / 16;
        rdb[j] = A_BYTES + kp * 256u + 16u * (u ^ OB::mn_swz(kp)) + half;
      }
    }
    zero_acc();
  }

  __device__ __forceinline__ void setup(const DenseArgs& p, int m0, int n0, int gate) {
    const unsigned long long kbytes = (unsigned long long)p.K * C::BITS / 8;
    lda = (uint32_t)p.lda;
    ldb = (uint32_t)p.ldb;
    if (C::A_KMAJOR) rsa = buffer_words(p.a + (long)m0 * p.lda, (unsigned long long)(p.M - m0) * p.lda);
    else rsa = buffer_words(p.a + m0, kbytes * p.M - m0);
    if (C::B_KMAJOR) rsb = buffer_words(p.b + (long)n0 * p.ldb, (unsigned long long)(p.b_cols - n0) * p.ldb);
    else rsb = buffer_words(p.b + n0, kbytes * p.b_cols - n0);
    oa.init(wave, lane, lda, 0);
    ob.init(wave, lane, ldb, (uint32_t)gate);
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

  __device__ __forceinline__ void dma_stage(uint8_t* smem, int st, int slot_) const {
    const uint32_t base = lds_address(smem) + (uint32_t)slot_ * STAGE;
    oa.issue(rsa, OA::soff(st, lda), base, wave);
    ob.issue(rsb, OB::soff(st, ldb), base + A_BYTES, wave);
  }
  // DMA block b (A blocks first, then B) of stage st into ring slot slot_.
  __device__ __forceinline__ void dma_block(uint8_t* smem, int st, int slot_, int b) const {
    const uint32_t base = lds_address(smem) + (uint32_t)slot_ * STAGE;
    if (b < OA::BLK) oa.issue_one(rsa, OA::soff(st, lda), base, wave, b);
    else ob.issue_one(rsb, OB::soff(st, ldb), base + A_BYTES, wave, b - OA::BLK);
  }

  // Waits until at most n stages of this wave's DMA loads are outstanding
  // (n = 0 .. P-1).
  static __device__ __forceinline__ void wait_stages(int n) {
    static_assert(P <= 5, "wait_stages covers rings of up to five stages");
    if (n <= 0) wait_vmcnt<0>();
    else if (n == 1) wait_vmcnt<DPW>();
    else if (n == 2) wait_vmcnt<(P > 2 ? 2 : 1) * DPW>();
    else if (n == 3) wait_vmcnt<(P > 3 ? 3 : 1) * DPW>();
    else wait_vmcnt<(P > 4 ? 4 : 1) * DPW>();
  }
  static __device__ __forceinline__ int imin(int a, int b) { return a < b ? a : b; }

  // Moves the read offsets to the next ring slot.
  __device__ __forceinline__ void advance_reads() {
    const uint32_t delta = slot == P - 1 ? (uint32_t)(-(P - 1) * STAGE) : (uint32_t)STAGE;
    slot = slot == P - 1 ? 0 : slot + 1;
#pragma unroll
    for (auto& x : rda) x += delta;
#pragma unroll
    for (auto& x : rdb) x += delta;
  }

  // Raw fragment reads from the current read slot.  S: step (int4) or half
  // (int8) for MN-major operands; K-major reads cover the whole stage.
  template <bool KMAJOR, int S>
  static __device__ __forceinline__ Packed<KMAJOR> read_raw(const uint8_t* q) {
    if constexpr (KMAJOR) {
      // volatile keeps this one ds_read_b128: the compiler would otherwise
      // split the int4 stage fragment, whose halves are used one step apart,
      // into 8-byte reads and pair those of neighbouring fragments (1 KiB
      // apart, the same banks) into conflicting ds_read2st64_b64.
      typedef const volatile __attribute__((address_space(3))) v4i lds_cv4i;
      const v4i x = *(lds_cv4i*)(const lds_byte*)q;
      return __builtin_bit_cast(Packed<KMAJOR>, x);
    } else if constexpr (I4) {
      return __builtin_bit_cast(uint2, ds_read_tr8(q + S * 2048));
    } else {
      const v2i lo = ds_read_tr8(q);
      const v2i hi = ds_read_tr8(q + 2048);
      return v4i{lo.x, lo.y, hi.x, hi.y};
    }
  }
  template <int S>
  __device__ __forceinline__ Packed<C::A_KMAJOR> read_a(const uint8_t* smem, int i) const {
    return read_raw<C::A_KMAJOR, S>(smem + (C::A_KMAJOR ? rda[0] + 1024 * i : rda[C::A_KMAJOR ? 0 : i]));
  }
  template <int S>
  __device__ __forceinline__ Packed<C::B_KMAJOR> read_b(const uint8_t* smem, int j) const {
    return read_raw<C::B_KMAJOR, S>(smem + (C::B_KMAJOR ? rdb[0] + 64 * brow_rel(j) : rdb[C::B_KMAJOR ? 0 : j]));
  }

  // MFMA operand of step S from packed int4 bytes (widened) or int8 (as is).
  template <int S>
  static __device__ __forceinline__ v4i operand(const uint4& f) {
    return __builtin_bit_cast(v4i, S == 0 ? widen_chunk(f.x, f.y) : widen_chunk(f.z, f.w));
  }
  template <int S>
  static __device__ __forceinline__ v4i operand(const uint2& f) {
    return __builtin_bit_cast(v4i, widen_chunk(f.x, f.y));
  }
  template <int S>
  static __device__ __forceinline__ v4i operand(const v4i& f) { return f; }

  // Opens stage k: waits for this wave's DMA of stage k+1 (loads are only
  // issued for stages that exist, so near the end fewer are outstanding),
  // then the barrier
  // (stage k+1 complete in LDS; every wave has read all of stage k, whose
  // fragments are in registers), issues the loads of stage k+P into stage
  // k's slot and moves the reads to stage k+1.
  __device__ __forceinline__ void open_stage(uint8_t* smem, int k, int nst) {
    wait_stages(imin(P - 2, nst - 2 - k));
    __syncthreads();
    if (k + P < nst) dma_stage(smem, k + P, slot);
    advance_reads();
  }

  // Prepares operand set W for the next step from the packed registers and
  // refills them.  int4 step S of stage k (reads point at stage k+1): the
  // next step is step 1 of stage k (S = 0) or step 0 of stage k+1 (S = 1);
  // K-major operands hold stage k until S = 0 widens its step 1 and reloads
  // stage k+1, MN-major ones hold the next step and reload step S of k+1.
  template <bool KMAJOR, int S, int NF, class R>
  __device__ __forceinline__ void prepare(v4i (&w)[NF], Packed<KMAJOR> (&pk)[NF], R read) const {
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      if constexpr (!I4) {
        w[f] = read(f);
      } else if constexpr (KMAJOR) {
        w[f] = operand<1 - S>(pk[f]);
        if (S == 0) pk[f] = read(f);
      } else {
        w[f] = operand<0>(pk[f]);
        pk[f] = read(f);
      }
    }
  }

  // MFMA through inline asm: the accumulator is a tied AGPR operand, which
  // keeps all 256 accumulators in place, and volatile asm keeps its issue
  // position.  D = src0 * src1^T with the B fragment as src0 (mfma64).
  static __device__ __forceinline__ void mfma_asm(v4i& acc, const v4i& b, const v4i& a) {
    asm volatile("v_mfma_i32_16x16x64_i8 %0, %1, %2, %0" : "+a"(acc) : "v"(b), "v"(a));
  }
  template <int CUR>
  __device__ __forceinline__ void mfma_x(int x) {
    const int i = x / C::FN2, j = x % C::FN2;
    mfma_asm(acc[i][j], wb[CUR][j], wa[CUR][i]);
  }
  // The int4 step is issued as a fixed sequence of asm statements, each an
  // MFMA followed by at most one LDS or DMA load and two VALU instructions:
  // one wave then co-issues the VALU work with its MFMAs, and a load placed
  // right after an MFMA (before the VALU) costs no MFMA issue slot.  The
  // LDS reads here are invisible to the compiler's wait-count tracking, so
  // each fragment unit waits explicitly (unit_wait) for the read it widens;
  // the loop has no other LGKM traffic (no scalar loads) that could make
  // the in-order count inexact.
  //
  // Widening one packed fragment (dwords x0, x1) takes six VALU in three
  // parts:
  //   part 0: t0 = x0 << 4, t1 = x1 << 4
  //   part 1: hi0 = x0 & 0xF0F0F0F0, hi1 = x1 & 0xF0F0F0F0
  //   part 2: lo0 = t0 & 0xF0F0F0F0, lo1 = t1 & 0xF0F0F0F0
  // No asm statement reads a VGPR written by the one right before it (the
  // compiler would put an s_nop between them), and every output is
  // early-clobber so it never overwrites a source of the same statement.
  // Read kinds: 0 none, 1 ds_read_b64_tr_b8 (2 dwords), 2 ds_read_b128.
  template <int CUR, int PART>
  __device__ __forceinline__ void mfma_widen(int x, uint32_t in0, uint32_t in1, uint32_t& o0, uint32_t& o1) {
    const int i = x / C::FN2, j = x % C::FN2;
    if constexpr (PART == 0) {
      asm volatile("v_mfma_i32_16x16x64_i8 %0, %3, %4, %0\n\t"
                   "v_lshlrev_b32 %1, 4, %5\n\t"
                   "v_lshlrev_b32 %2, 4, %6"
                   : "+a"(acc[i][j]), "=&v"(o0), "=&v"(o1)
                   : "v"(wb[CUR][j]), "v"(wa[CUR][i]), "v"(in0), "v"(in1));
    } else {
      asm volatile("v_mfma_i32_16x16x64_i8 %0, %3, %4, %0\n\t"
                   "v_and_b32 %1, 0xf0f0f0f0, %5\n\t"
                   "v_and_b32 %2, 0xf0f0f0f0, %6"
                   : "+a"(acc[i][j]), "=&v"(o0), "=&v"(o1)
                   : "v"(wb[CUR][j]), "v"(wa[CUR][i]), "v"(in0), "v"(in1));
    }
  }
  template <int CUR, int OFF>
  __device__ __forceinline__ void mfma_widen0_tr(int x, uint32_t in0, uint32_t in1, uint32_t& o0, uint32_t& o1,
                                                 v2i& r, uint32_t addr) {
    const int i = x / C::FN2, j = x % C::FN2;
    asm volatile("v_mfma_i32_16x16x64_i8 %0, %4, %5, %0\n\t"
                 "ds_read_b64_tr_b8 %3, %8 offset:%9\n\t"
                 "v_lshlrev_b32 %1, 4, %6\n\t"
                 "v_lshlrev_b32 %2, 4, %7"
                 : "+a"(acc[i][j]), "=&v"(o0), "=&v"(o1), "=&v"(r)
                 : "v"(wb[CUR][j]), "v"(wa[CUR][i]), "v"(in0), "v"(in1), "v"(addr), "n"(OFF));
  }
  template <int CUR, int OFF>
  __device__ __forceinline__ void mfma_widen0_b128(int x, uint32_t in0, uint32_t in1, uint32_t& o0, uint32_t& o1,
                                                   v4i& r, uint32_t addr) {
    const int i = x / C::FN2, j = x % C::FN2;
    asm volatile("v_mfma_i32_16x16x64_i8 %0, %4, %5, %0\n\t"
                 "ds_read_b128 %3, %8 offset:%9\n\t"
                 "v_lshlrev_b32 %1, 4, %6\n\t"
                 "v_lshlrev_b32 %2, 4, %7"
                 : "+a"(acc[i][j]), "=&v"(o0), "=&v"(o1), "=&v"(r)
                 : "v"(wb[CUR][j]), "v"(wa[CUR][i]), "v"(in0), "v"(in1), "v"(addr), "n"(OFF));
  }
  // Part 1 with one LDS-DMA load after the MFMA (the compiler writes M0
  // before the statement; the MFMA is the wait state the load needs).
  template <int CUR>
  __device__ __forceinline__ void mfma_widen1_dma(int x, uint32_t in0, uint32_t in1, uint32_t& o0, uint32_t& o1,
                                                  const v4i& rs, uint32_t voff, uint32_t soff, uint32_t m0) {
    const int i = x / C::FN2, j = x % C::FN2;
    asm volatile("v_mfma_i32_16x16x64_i8 %0, %3, %4, %0\n\t"
                 "buffer_load_dwordx4 %7, %8, %9 offen lds\n\t"
                 "v_and_b32 %1, 0xf0f0f0f0, %5\n\t"
                 "v_and_b32 %2, 0xf0f0f0f0, %6"
                 : "+a"(acc[i][j]), "=&v"(o0), "=&v"(o1)
                 : "v"(wb[CUR][j]), "v"(wa[CUR][i]), "v"(in0), "v"(in1), "v"(voff), "s"(rs), "s"(soff), "{m0}"(m0)
                 : "memory");
  }
  // A plain MFMA, optionally followed by one LDS read.
  template <int CUR, int KIND, int OFF, class R>
  __device__ __forceinline__ void mfma_read(int x, R& r, uint32_t addr) {
    const int i = x / C::FN2, j = x % C::FN2;
    if constexpr (KIND == 1) {
      asm volatile("v_mfma_i32_16x16x64_i8 %0, %2, %3, %0\n\t"
                   "ds_read_b64_tr_b8 %1, %4 offset:%5"
                   : "+a"(acc[i][j]), "=&v"(r)
                   : "v"(wb[CUR][j]), "v"(wa[CUR][i]), "v"(addr), "n"(OFF));
    } else if constexpr (KIND == 2) {
      asm volatile("v_mfma_i32_16x16x64_i8 %0, %2, %3, %0\n\t"
                   "ds_read_b128 %1, %4 offset:%5"
                   : "+a"(acc[i][j]), "=&v"(r)
                   : "v"(wb[CUR][j]), "v"(wa[CUR][i]), "v"(addr), "n"(OFF));
    } else {
      mfma_asm(acc[i][j], wb[CUR][j], wa[CUR][i]);
    }
  }

  // Refill read of fragment f at sub-step S: kind, LDS address and offset.
  template <int S>
  static constexpr int refill_kind(int f) {
    return f < C::FN2 ? (C::B_KMAJOR ? (S == 0 ? 2 : 0) : 1) : (C::A_KMAJOR ? (S == 0 ? 2 : 0) : 1);
  }
  template <int S>
  static constexpr int refill_off(int f) {
    if (f < C::FN2) return C::B_KMAJOR ? 64 * brow_rel(f) : S * 2048;
    return C::A_KMAJOR ? 1024 * (f - C::FN2) : S * 2048;
  }
  __device__ __forceinline__ uint32_t refill_addr(uint32_t lds0, int f) const {
    if (f < C::FN2) return lds0 + (C::B_KMAJOR ? rdb[0] : rdb[C::B_KMAJOR ? 0 : f]);
    return lds0 + (C::A_KMAJOR ? rda[0] : rda[C::A_KMAJOR ? 0 : f - C::FN2]);
  }
  // Stores a refill read result into fragment f's packed registers.
  __device__ __forceinline__ void put_packed(int f, const v2i& r2, const v4i& r4, int kind) {
    if (f < C::FN2) {
      if constexpr (C::B_KMAJOR) { if (kind == 2) pb[f] = __builtin_bit_cast(Packed<true>, r4); }
      else pb[f] = __builtin_bit_cast(Packed<false>, r2);
    } else {
      if constexpr (C::A_KMAJOR) { if (kind == 2) pa[f - C::FN2] = __builtin_bit_cast(Packed<true>, r4); }
      else pa[f - C::FN2] = __builtin_bit_cast(Packed<false>, r2);
    }
  }

  // Packed dwords of fragment f (B fragments first, then A) for the next
  // step; see prepare().
  template <int S>
  __device__ __forceinline__ uint2 next_packed(int f) const {
    if (f < C::FN2) {
      if constexpr (C::B_KMAJOR) return S == 0 ? make_uint2(pb[f].z, pb[f].w) : make_uint2(pb[f].x, pb[f].y);
      else return pb[f];
    } else {
      if constexpr (C::A_KMAJOR) {
        const int i = f - C::FN2;
        return S == 0 ? make_uint2(pa[i].z, pa[i].w) : make_uint2(pa[i].x, pa[i].y);
      } else {
        return pa[f - C::FN2];
      }
    }
  }
  template <int S>
  __device__ __forceinline__ void refill(const uint8_t* smem, int f) {
    if (f < C::FN2) {
      if (!C::B_KMAJOR || S == 0) pb[f] = read_b<S>(smem, f);
    } else {
      if (!C::A_KMAJOR || S == 0) pa[f - C::FN2] = read_a<S>(smem, f - C::FN2);
    }
  }

  // The refill reads are asm statements, so the compiler does not know that
  // their registers are written later than the statement.  The last step's
  // refills are never widened: without this wait, with each packed register
  // an operand, their registers could be reused while the reads are in
  // flight.
  template <class T>
  static __device__ __forceinline__ void hold_until_landed(T& x) {
    typedef int nv __attribute__((ext_vector_type(sizeof(T) / 4)));
    nv v = __builtin_bit_cast(nv, x);
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(v)::"memory");
    x = __builtin_bit_cast(T, v);
  }
  __device__ __forceinline__ void drain_refills() {
#pragma unroll
    for (int i = 0; i < C::FM; ++i) hold_until_landed(pa[i]);
#pragma unroll
    for (int j = 0; j < C::FN2; ++j) hold_until_landed(pb[j]);
  }

  // Stage and ring slot of the loads issued during the current stage.
  int dma_st, dma_slot;

  // DMA operands of block b of the loads issued during this stage.
  __device__ __forceinline__ void dma_args(uint32_t lds0, int b, const v4i*& rs, uint32_t& voff, uint32_t& soff,
                                           uint32_t& m0) const {
    const uint32_t base = lds0 + (uint32_t)dma_slot * STAGE;
    if (b < OA::BLK) {
      rs = &rsa;
      voff = oa.voff[b];
      soff = OA::soff(dma_st, lda);
      m0 = base + (uint32_t)(wave * OA::BLK + b) * 1024u;
    } else {
      rs = &rsb;
      voff = ob.voff[b - OA::BLK];
      soff = OB::soff(dma_st, ldb);
      m0 = base + A_BYTES + (uint32_t)(wave * OB::BLK + b - OA::BLK) * 1024u;
    }
  }

  // LDS reads issued in step S by units lo..hi (fragments refilled there).
  template <int S>
  static constexpr int reads_in(int lo, int hi) {
    int n = 0;
    for (int f = lo; f <= hi; ++f) n += refill_kind<S>(f) != 0;
    return n;
  }
  // lgkmcnt that unit F of step S waits for before widening fragment F: the
  // LDS reads issued after the one that brought fragment F's packed bytes.
  // Those came one step earlier, except the K-major stage fragments widened
  // at step 0, whose read was two steps earlier.  The refill of fragment f
  // is issued by unit f+1 (the tail for the last fragment).
  template <int S, int F>
  static constexpr int unit_wait() {
    constexpr int NF = C::FN2 + C::FM;
    constexpr bool KM = F < C::FN2 ? C::B_KMAJOR : C::A_KMAJOR;
    const int after = (KM && S == 0) ? reads_in<1 - S>(0, NF - 1) : reads_in<1 - S>(F + 1, NF - 1);
    return after + reads_in<S>(0, F - 2);
  }

  // Fragment unit F of an int4 step: MFMAs 3F..3F+2 widen fragment F of the
  // next operand set; the first also refills fragment F-1's packed
  // registers, the second issues DMA block F at the stage's first step.
  template <int CUR, int S, bool DMA, int F>
  __device__ __forceinline__ void unit(uint32_t lds0) {
    constexpr int NXT = 1 - CUR;
    constexpr int WAIT = unit_wait<S, F>();
    if constexpr (WAIT < 15) asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(WAIT) : "memory");
    const uint2 x = next_packed<S>(F);
    uint32_t t0, t1, lo0, hi0, lo1, hi1;
    constexpr int RK = F > 0 ? refill_kind<S>(F - 1) : 0;
    if constexpr (RK == 1) {
      v2i r;
      mfma_widen0_tr<CUR, refill_off<S>(F - 1)>(3 * F, x.x, x.y, t0, t1, r, refill_addr(lds0, F - 1));
      put_packed(F - 1, r, v4i{}, 1);
    } else if constexpr (RK == 2) {
      v4i r;
      mfma_widen0_b128<CUR, refill_off<S>(F - 1)>(3 * F, x.x, x.y, t0, t1, r, refill_addr(lds0, F - 1));
      put_packed(F - 1, v2i{}, r, 2);
    } else {
      mfma_widen<CUR, 0>(3 * F, x.x, x.y, t0, t1);
    }
    if constexpr (S == 0 && DMA && F < DPW) {
      const v4i* rs;
      uint32_t voff, soff, m0;
      dma_args(lds0, F, rs, voff, soff, m0);
      mfma_widen1_dma<CUR>(3 * F + 1, x.x, x.y, hi0, hi1, *rs, voff, soff, m0);
    } else {
      mfma_widen<CUR, 1>(3 * F + 1, x.x, x.y, hi0, hi1);
    }
    mfma_widen<CUR, 2>(3 * F + 2, t0, t1, lo0, lo1);
    const v4i w = v4i{(int)lo0, (int)hi0, (int)lo1, (int)hi1};
    if constexpr (F < C::FN2) wb[NXT][F] = w;
    else wa[NXT][F - C::FN2] = w;
  }
  template <int CUR, int S, bool DMA, int... F>
  __device__ __forceinline__ void units(uint32_t lds0, std::integer_sequence<int, F...>) {
    (unit<CUR, S, DMA, F>(lds0), ...);
  }
  // MFMAs 3*NF.. of an int4 step; the first refills the last fragment.
  template <int CUR, int S, int... X>
  __device__ __forceinline__ void tail(uint32_t lds0, std::integer_sequence<int, X...>) {
    constexpr int NF = C::FN2 + C::FM;
    constexpr int RK = refill_kind<S>(NF - 1);
    if constexpr (RK == 1) {
      v2i r;
      mfma_read<CUR, 1, refill_off<S>(NF - 1)>(3 * NF, r, refill_addr(lds0, NF - 1));
      put_packed(NF - 1, r, v4i{}, 1);
    } else if constexpr (RK == 2) {
      v4i r;
      mfma_read<CUR, 2, refill_off<S>(NF - 1)>(3 * NF, r, refill_addr(lds0, NF - 1));
      put_packed(NF - 1, v2i{}, r, 2);
    } else {
      mfma_x<CUR>(3 * NF);
    }
    (mfma_x<CUR>(3 * NF + 1 + X), ...);
  }

  // One MFMA step on operand set CUR while set 1-CUR is prepared.  int4
  // steps are the fixed asm sequence above: fragment unit f (MFMAs
  // 3f..3f+2) widens fragment f of the next set, B fragments first; the
  // remaining MFMAs carry no VALU.
  template <int CUR, int S, class OnStep, bool DMA = true>
  __device__ __forceinline__ void step(const uint8_t* smem, int t, OnStep& on_step) {
    constexpr int NXT = 1 - CUR;
    if constexpr (I4) {
      constexpr int NF = C::FN2 + C::FM;
      constexpr int NMF = C::FM * C::FN2;
      static_assert(3 * NF < NMF, "three MFMAs per prepared fragment and one for the last refill");
      static_assert(DPW <= NF, "one load per prepared fragment");
      const uint32_t lds0 = lds_address(smem);
      units<CUR, S, DMA>(lds0, std::make_integer_sequence<int, NF>{});
      tail<CUR, S>(lds0, std::make_integer_sequence<int, NMF - 3 * NF - 1>{});
    } else {
      prepare<C::B_KMAJOR, S>(wb[NXT], pb, [&](int j) { return read_b<S>(smem, j); });
      prepare<C::A_KMAJOR, S>(wa[NXT], pa, [&](int i) { return read_a<S>(smem, i); });
#pragma unroll
      for (int i = 0; i < C::FM; ++i)
#pragma unroll
        for (int j = 0; j < C::FN2; ++j) acc[i][j] = mfma64(wb[CUR][j], wa[CUR][i], acc[i][j]);
    }
    on_step((t + 1) * 64);
  }

  // Two-waves-per-SIMD stage: every step reads its own fragments (K-major
  // int4 fragments once per stage), widens them and multiplies.
  template <class OnStep>
  __device__ __forceinline__ void stage_ping(const uint8_t* smem, int k, OnStep& on_step) {
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
#pragma unroll
      for (int j = 0; j < C::FN2; ++j) {
        if (C::B_KMAJOR && I4 && s == 1) continue;
        pb[j] = s ? read_b<1>(smem, j) : read_b<0>(smem, j);
      }
#pragma unroll
      for (int i = 0; i < C::FM; ++i) {
        if (C::A_KMAJOR && I4 && s == 1) continue;
        pa[i] = s ? read_a<1>(smem, i) : read_a<0>(smem, i);
      }
#pragma unroll
      for (int j = 0; j < C::FN2; ++j) wb[0][j] = s ? operand<1>(pb[j]) : operand<0>(pb[j]);
#pragma unroll
      for (int i = 0; i < C::FM; ++i) {
        const v4i y = s ? operand<1>(pa[i]) : operand<0>(pa[i]);
#pragma unroll
        for (int j = 0; j < C::FN2; ++j) acc[i][j] = mfma64(wb[0][j], y, acc[i][j]);
      }
      on_step((k * STEPS + s + 1) * 64);
    }
  }

  template <class OnStep>
  __device__ __forceinline__ void run(uint8_t* smem, int nst, OnStep on_step) {
#pragma unroll
    for (int q = 0; q < P; ++q)
      if (q < nst) dma_stage(smem, q, q);
    if constexpr (PING) {
      // Stage k is read only during stage k, so the barrier that opens
      // stage k+1 frees stage k's slot: its loads (stage k+P) are issued
      // then, P-1 stages ahead of use.
      wait_stages(imin(P - 1, nst - 1));
      __syncthreads();
      stage_ping(smem, 0, on_step);
      for (int k = 1; k < nst; ++k) {
        wait_stages(imin(P - 2, nst - 1 - k));
        __syncthreads();
        const int prev = k - 1;
        if (prev + P < nst) dma_stage(smem, prev + P, slot);
        advance_reads();
        stage_ping(smem, k, on_step);
      }
      wait_vmcnt<0>();
      return;
    }
    wait_stages(imin(P - 1, nst - 1));
    __syncthreads();
    if constexpr (I4) {
      // operands of step 0; packed registers: step 1 (MN-major) or stage 0
      // (K-major)
#pragma unroll
      for (int j = 0; j < C::FN2; ++j) {
        pb[j] = read_b<0>(smem, j);
        wb[0][j] = operand<0>(pb[j]);
        if (!C::B_KMAJOR) pb[j] = read_b<1>(smem, j);
      }
#pragma unroll
      for (int i = 0; i < C::FM; ++i) {
        pa[i] = read_a<0>(smem, i);
        wa[0][i] = operand<0>(pa[i]);
        if (!C::A_KMAJOR) pa[i] = read_a<1>(smem, i);
      }
      // The asm MFMAs read accumulators the compiler zeroed and the
      // epilogue reads what they wrote; neither dependency is visible to the
      // compiler's hazard recognizer, so the wait states are explicit.
      static_assert(C::FM == 8 && C::FN2 == 8, "the asm step is written for 8x8 accumulator fragments");
      acc_fence<4>(acc);
      static_assert(DPW <= C::FN2 + C::FM, "one load per prepared fragment");
      // Stages open as open_stage() does, with the loads issued by step 0
      // and the asm LDS reads of the last step complete as well.  The last
      // P stages issue no loads (there is no stage k+P).
      int k = 0;
      for (; k + P < nst; ++k) {
        wait_vmcnt<(P - 2) * DPW>();
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __syncthreads();
        dma_st = k + P;
        dma_slot = slot;
        advance_reads();
        step<0, 0>(smem, 2 * k, on_step);
        step<1, 1>(smem, 2 * k + 1, on_step);
      }
      for (; k < nst; ++k) {
        wait_stages(imin(P - 2, nst - 2 - k));
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __syncthreads();
        advance_reads();
        step<0, 0, OnStep, false>(smem, 2 * k, on_step);
        step<1, 1, OnStep, false>(smem, 2 * k + 1, on_step);
      }
      drain_refills();
      acc_fence<7>(acc);
    } else {
#pragma unroll
      for (int j = 0; j < C::FN2; ++j) wb[0][j] = read_b<0>(smem, j);
#pragma unroll
      for (int i = 0; i < C::FM; ++i) wa[0][i] = read_a<0>(smem, i);
      // stage pairs alternate the operand sets; an odd count ends with one
      // more stage on set 0
      int k = 0;
      for (; k + 2 <= nst; k += 2) {
        open_stage(smem, k, nst);
        step<0, 0>(smem, k, on_step);
        open_stage(smem, k + 1, nst);
        step<1, 0>(smem, k + 1, on_step);
      }
      if (k < nst) {
        open_stage(smem, k, nst);
        step<0, 0>(smem, k, on_step);
      }
    }
    wait_vmcnt<0>();
  }
};

}  // namespace shk
