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
// TN).  A K-major stage holds ROWS x 64 bytes.  16-byte unit q of tile row r
// sits at r*64 + 16*(q ^ ((r >> 2) & 3)).  An MN-major stage holds 64 source
// rows x 256 bytes (ROWS = 256).  Unit u (tile rows 16u..16u+15) of source
// row kp sits at kp*256 + 16*(u ^ sw(kp)).  sw is kp & 15 for int4 and
// (kp & 7) | ((kp & 16) >> 1) for int8.  Both swizzles keep every fragment
// read below conflict-free.  They act on 16-byte units, so each DMA lane
// still copies one contiguous 16-byte source piece; the swizzle is applied by
// choosing which piece a lane fetches.
//
// Fragment reads.  MFMA step s (64 K values) of a stage uses 16-value chunk g
// = lane / 16 of each of its 16 rows:
//  * K-major int4: ds_read_b64 of the 8 packed bytes of the chunk.
//  * K-major int8: ds_read_b128 of the 16 bytes.
//  * MN-major: ds_read_b64_tr_b8.  Lane i of a 16-lane group addresses source
//    row kp0 + i/2 at byte 8*(i%2) of the fragment's unit, and receives the
//    8 bytes of rows kp0..kp0+7 of column i.  For int4 those are the 8 packed
//    bytes of the chunk; int8 needs two such reads.
// Packed int4 bytes p0..p7 are widened after the read to the chunk
// [lo(p0..3), hi(p0..3), lo(p4..7), hi(p4..7)] as 16*v.  Both operands get
// the same order (shk_common.h).
//
// Schedule.  Every step multiplies the fragments held in registers (int4
// fragments are widened right before their MFMAs) while it reads the next
// step's fragments.
// The last step of stage k opens with the stage's only barrier:
//  * before it, each wave waits for its own DMA of stage k+1, so after it
//    stage k+1 is complete;
//  * after it, no wave still reads stage k, which was fully read one step
//    earlier, so the loads of stage k+P are issued into stage k's slot.
#pragma once

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
__device__ __forceinline__ void lds_dma16(const v4i& rs, uint32_t voff, uint32_t soff, uint32_t m0) {
  // The compiler sets M0 for the "{m0}" operand; the nop is the wait state
  // an M0 write needs before an LDS-DMA instruction reads it.
  asm volatile(
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %0, %1, %2 offen lds"
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

  static __device__ __forceinline__ uint32_t mn_swz(uint32_t kp) {
    return BITS == 4 ? (kp & 15u) : ((kp & 7u) | ((kp & 16u) >> 1));
  }

  __device__ __forceinline__ void init(int wave, int lane, uint32_t ld, uint32_t gate) {
#pragma unroll
    for (int c = 0; c < BLK; ++c) {
      const int b = wave * BLK + c;
      if constexpr (KMAJOR) {
        const int r = 16 * b + lane / 4;
        const int q = (lane & 3) ^ ((lane >> 4) & 3);
        const uint32_t src = r < HALF ? (uint32_t)r : (uint32_t)(r - HALF) + gate;
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
    for (int c = 0; c < BLK; ++c) lds_dma16(rs, voff[c], so, dst + (uint32_t)(wave * BLK + c) * 1024u);
  }
};

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
  static constexpr int NRA = C::A_KMAJOR ? STEPS : C::FM;   // read-offset registers
  static constexpr int NRB = C::B_KMAJOR ? STEPS : C::FN2;
  static_assert(C::MK == 64, "the DMA engine issues 16x16x64 MFMAs");
  static_assert(C::BK * C::BITS == 512, "a stage is 64 source bytes per row");
  static_assert(P >= 2 && (P - 2) * DPW < 64 && (P - 1) * DPW < 64, "vmcnt range");
  static_assert(LDS_BYTES <= 160 * 1024, "LDS budget");

  v4i acc[C::FM][C::FN2];
  // Fragments: packed int4 (widened right before their MFMAs) or int8 as
  // read.  A fragment i is re-read for the next step as soon as the MFMAs of
  // row i have issued; B fragments are double-buffered (fb: current step,
  // fn: next step) because every row uses all of them.
  using Frag = typename std::conditional<(C::BITS == 4), uint2, v4i>::type;
  Frag fa[C::FM];
  Frag fb[C::FN2];
  Frag fn[C::FN2];
  OA oa;
  OB ob;
  v4i rsa, rsb;
  uint32_t lda, ldb;
  uint32_t rda[NRA], rdb[NRB];
  int lane, wave, wm, wn, slot;

  __device__ __forceinline__ void init_reads() {
    lane = threadIdx.x & 63;
    wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    wm = wave % C::WM;
    wn = wave / C::WM;
    slot = 0;
    const int l15 = lane & 15;
    const int g = lane >> 4;
    const uint32_t kp = I4 ? (uint32_t)(8 * g + l15 / 2) : (uint32_t)(16 * g + l15 / 2);
    const uint32_t half = 8u * (l15 & 1);
    if constexpr (C::A_KMAJOR) {
      const uint32_t r = wm * C::TM + l15;
#pragma unroll
      for (int s = 0; s < NRA; ++s) {
        const int q = I4 ? (2 * s + (g >> 1)) : g;
        rda[s] = r * 64u + 16u * (q ^ ((l15 >> 2) & 3)) + (I4 ? 8u * (g & 1) : 0u);
      }
    } else {
#pragma unroll
      for (int i = 0; i < C::FM; ++i) {
        const uint32_t u = (wm * C::TM + 16 * i) / 16;
        rda[i] = kp * 256u + 16u * (u ^ OA::mn_swz(kp)) + half;
      }
    }
    if constexpr (C::B_KMAJOR) {
      const uint32_t r = wn * C::TN + l15;
#pragma unroll
      for (int s = 0; s < NRB; ++s) {
        const int q = I4 ? (2 * s + (g >> 1)) : g;
        rdb[s] = A_BYTES + r * 64u + 16u * (q ^ ((l15 >> 2) & 3)) + (I4 ? 8u * (g & 1) : 0u);
      }
    } else {
#pragma unroll
      for (int j = 0; j < C::FN2; ++j) {
        const uint32_t u = (uint32_t)brow(j) / 16;
        rdb[j] = A_BYTES + kp * 256u + 16u * (u ^ OB::mn_swz(kp)) + half;
      }
    }
    zero_acc();
  }

  // First B tile row of fragment j relative to the wave's first up row.
  static constexpr int brow_rel(int j) { return j < C::FN ? 16 * j : C::BHALF + 16 * (j - C::FN); }
  __device__ __forceinline__ int brow(int j) const { return wn * C::TN + brow_rel(j); }

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

  // Moves the read offsets to the next ring slot.
  __device__ __forceinline__ void advance_reads() {
    const uint32_t delta = slot == P - 1 ? (uint32_t)(-(P - 1) * STAGE) : (uint32_t)STAGE;
    slot = slot == P - 1 ? 0 : slot + 1;
#pragma unroll
    for (int x = 0; x < NRA; ++x) rda[x] += delta;
#pragma unroll
    for (int x = 0; x < NRB; ++x) rdb[x] += delta;
  }

  // Fragment reads of sub-step S from the current read slot.
  template <int S>
  __device__ __forceinline__ Frag read_a(const uint8_t* smem, int i) const {
    if constexpr (C::A_KMAJOR) {
      return *reinterpret_cast<const Frag*>(smem + rda[I4 ? S : 0] + 1024 * i);
    } else {
      return read_mn<S>(smem + rda[i]);
    }
  }
  template <int S>
  __device__ __forceinline__ Frag read_b(const uint8_t* smem, int j) const {
    if constexpr (C::B_KMAJOR) {
      return *reinterpret_cast<const Frag*>(smem + rdb[I4 ? S : 0] + 64 * brow_rel(j));
    } else {
      return read_mn<S>(smem + rdb[j]);
    }
  }
  template <int S>
  static __device__ __forceinline__ Frag read_mn(const uint8_t* q) {
    if constexpr (I4) {
      return __builtin_bit_cast(uint2, ds_read_tr8(q + S * 32 * 256));
    } else {
      const v2i lo = ds_read_tr8(q);
      const v2i hi = ds_read_tr8(q + 8 * 256);
      return v4i{lo.x, lo.y, hi.x, hi.y};
    }
  }

  static __device__ __forceinline__ v4i operand(const uint2& f) {
    return __builtin_bit_cast(v4i, widen_chunk(f.x, f.y));
  }
  static __device__ __forceinline__ v4i operand(const v4i& f) { return f; }

  // One K stage: STEPS MFMA steps of 64 K values.  Step s multiplies the
  // fragments in registers while it reads those of the next step (sub-step
  // s+1 of this stage, or sub-step 0 of stage k+1 after the barrier).
  template <class OnStep>
  __device__ __forceinline__ void stage_body(uint8_t* smem, int k, int nst, OnStep& on_step) {
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      if (s == STEPS - 1) {
        wait_vmcnt<(P - 2) * DPW>();
        __syncthreads();
        const int ld_stage = k + P < nst ? k + P : nst - 1;
        dma_stage(smem, ld_stage, slot);
        advance_reads();
      }
      const int ns = (s + 1) % STEPS;
#pragma unroll
      for (int j = 0; j < C::FN2; ++j) fn[j] = ns ? read_b<1>(smem, j) : read_b<0>(smem, j);
      v4i xb[C::FN2];
#pragma unroll
      for (int j = 0; j < C::FN2; ++j) xb[j] = operand(fb[j]);
#pragma unroll
      for (int i = 0; i < C::FM; ++i) {
        const v4i ya = operand(fa[i]);
#pragma unroll
        for (int j = 0; j < C::FN2; ++j) acc[i][j] = mfma64(xb[j], ya, acc[i][j]);
        fa[i] = ns ? read_a<1>(smem, i) : read_a<0>(smem, i);
      }
#pragma unroll
      for (int j = 0; j < C::FN2; ++j) fb[j] = fn[j];
      on_step((k * STEPS + s + 1) * 64);
    }
  }

  // Runs the whole K loop.  on_step(k_end) follows each MFMA step
  // (subchannel flushes); it must not touch LDS.
  template <class OnStep>
  __device__ __forceinline__ void run(uint8_t* smem, int nst, OnStep on_step) {
#pragma unroll
    for (int q = 0; q < P; ++q) dma_stage(smem, q < nst ? q : nst - 1, q);
    wait_vmcnt<(P - 1) * DPW>();
    __syncthreads();
#pragma unroll
    for (int i = 0; i < C::FM; ++i) fa[i] = read_a<0>(smem, i);
#pragma unroll
    for (int j = 0; j < C::FN2; ++j) fb[j] = read_b<0>(smem, j);
    for (int k = 0; k < nst; ++k) stage_body(smem, k, nst, on_step);
    wait_vmcnt<0>();
  }
};

}  // namespace shk
