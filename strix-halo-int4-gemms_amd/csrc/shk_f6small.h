// 128 x 128 per-channel tile on the fp6 MFMA, two or three workgroups per CU.
// The ragged kernels (k_f6ragged.hip) run it with two ring slots.
//
// The small-grid counterpart of F6Engine (shk_f6.h) for the ragged calls,
// whose grids hold few 256 x 256 tiles (the C5 forward: ~220 tiles for 256
// CUs, each only 16 K stages deep): a workgroup of 4 waves owns 128 rows x
// 128 columns (64 x 64 per wave, 2 x 2 accumulators of 32 x 32) and uses at
// most 168 registers a lane.  With a ring of P = 3 slots (73 KiB of LDS) two
// workgroups share a CU, with P = 2 (49 KiB) three; one workgroup's
// prologue, epilogue and barriers overlap the others' MFMAs.
//
// Operands are the fp6 blocks of shk_f6.h.  The MFMA is the scaled form
// (v_mfma_scale_f32_32x32x64_f8f6f4) with E8M0 2^3 on both v/8 operands,
// so the accumulators hold the exact integer sums (|sum| <= 64 * K <= 2^24
// for K <= 262144).  The pipeline is F6Engine's at a quarter of the tile:
// 128-K stages (two 32 x 64 blocks per 32-row panel, 12 KiB of A and 12 KiB
// of B) in a ring of P slots.  Stage k: wait for this wave's DMA of stage
// k+1 and its LDS reads of stage k (with every fragment register of that
// set as an operand, so no compiler copy of a fragment precedes its data),
// then the barrier; 8 MFMAs on the fragments of stage k (two K steps of
// 2 x 2 blocks), each followed by two of the 16 LDS reads of stage k+1 into
// the other register set, the first six carrying one DMA load each of stage
// k+P into slot k % P (free: its fragments were read during stage k-1).  A
// stage therefore has 8 MFMAs to hide its reads' latency, where 64-K stages
// of 4 MFMAs waited on them.  The accumulators are cleared by VALU writes
// before the first MFMA of the (one) tile of the workgroup.
#pragma once

#include "shk_f6.h"

namespace shk {

template <class C, int PS = 3>
struct F6SmallEngine {
  static constexpr int P = PS;                      // ring slots
  static_assert(P == 2 || P == 3, "two or three ring slots");
  static constexpr int NW = 4;
  static constexpr int PANEL = 2 * F6_BLOCK;        // 32 rows x 128 K: 3 KiB
  static constexpr int OPB = 4 * PANEL;             // one operand's stage: 12 KiB
  static constexpr int STAGE = 2 * OPB;             // 24 KiB
  static constexpr int RING = P * STAGE;            // 72 or 48 KiB
  static constexpr int LDS_BYTES = RING;            // B scales follow (MFMA32_SCALE_BYTES)
  static constexpr int DPW = STAGE / 1024 / NW;     // 6 DMA loads per wave per stage
  static constexpr int TN = 64;                     // output columns per wave
  static constexpr int FN = 2;
  static constexpr float UNSCALE = 1.0f;            // the accumulators hold the integer sums
  static_assert(C::BM == 128 && C::BROWS == 128 && C::WM == 2 && C::WN == 2 && !C::SUBCH && !C::SWIGLU,
                "128 x 128 tiles of 2 x 2 waves, per-channel, plain epilogue");

  v16f acc[2][2];
  v6i fa[2][2][2];  // [set][step][i]
  v6i fb[2][2][2];  // [set][step][j]
  uint32_t voff[DPW];
  v4i rs;           // this wave's DMA operand (waves 0-1: A, 2-3: B)
  uint32_t lds0;
  int lane, wave, wm, wn;

  __device__ __forceinline__ int out_row(int i) const { return wm * 64 + 32 * i + (lane & 31); }
  __device__ __forceinline__ int out_col(int j, int q) const { return wn * TN + 32 * j + 8 * q + 4 * (lane >> 5); }
  __device__ __forceinline__ float acc_value(int i, int j, int x) const { return acc[i][j][x]; }
  __device__ __forceinline__ int acc_int(int i, int j, int x) const { return (int)acc[i][j][x]; }

  // a6 / b6: block-format operands; the tile's first A row m0 and first B
  // row n0 (multiples of 32); kb: 64-K blocks per panel.
  __device__ __forceinline__ void setup(uint8_t* smem, const uint8_t* a6, const uint8_t* b6, int m0, int n0, int kb,
                                        unsigned long long a_bytes, unsigned long long b_bytes) {
    lane = threadIdx.x & 63;
    wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    wm = wave % 2;
    wn = wave / 2;
    lds0 = lds_address(smem);
    const unsigned long long panel_bytes = (unsigned long long)kb * F6_BLOCK;
    const bool is_a = wave < 2;
    const unsigned long long first = (unsigned long long)((is_a ? m0 : n0) / 32) * panel_bytes;
    rs = buffer_words((is_a ? a6 : b6) + first, (is_a ? a_bytes : b_bytes) - first);
    // DMA load c of this wave fills stage bytes [1024 * (DPW*wave + c), +1024):
    // panel o / PANEL of the operand, byte o % PANEL of its two blocks
#pragma unroll
    for (int c = 0; c < DPW; ++c) {
      const uint32_t o = 1024u * (DPW * wave + c) + 16u * lane - (is_a ? 0u : (uint32_t)OPB);
      voff[c] = (o / PANEL) * (uint32_t)panel_bytes + o % PANEL;
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
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
  template <int S, int... Q>
  __device__ __forceinline__ void reads(const Reads& r, std::integer_sequence<int, Q...>) {
    (read<S, Q>(r), ...);
  }

  // MFMA T (0..7) of a stage on set S (step T / 4, A fragment (T % 4) / 2,
  // B fragment T % 2), fused for T < 6 with DMA load T of the stage loaded
  // now, followed by LDS reads 2T, 2T+1 of the next stage into the other
  // set.  Every stage runs the same branch-free sequence: a branch around
  // an asm MFMA or LDS read would let the register allocator copy an
  // accumulator or fragment between the statements before the hardware has
  // written it (the compiler cannot see the MFMA or the load in the asm).
  template <int S, int T>
  __device__ __forceinline__ void tick(const Reads& r, const v4i& rs_st, uint32_t so, uint32_t m0_st, int s8) {
    constexpr int ST = T / 4, I = (T % 4) / 2, J = T % 2;
    if constexpr (T < DPW) {
      // the compiler writes M0 before the statement; the MFMA is the wait
      // state the LDS-DMA load needs after that write
      asm volatile(
          "v_mfma_scale_f32_32x32x64_f8f6f4 %0, %1, %2, %0, %3, %3 op_sel_hi:[0,0,0] cbsz:2 blgp:2\n\t"
          "buffer_load_dwordx4 %4, %5, %6 offen lds"
          : "+v"(acc[I][J])
          : "v"(fb[S][ST][J]), "v"(fa[S][ST][I]), "v"(s8), "v"(voff[T]), "s"(rs_st), "s"(so),
            "{m0}"(m0_st + 1024u * T)
          : "memory");
    } else {
      asm volatile("v_mfma_scale_f32_32x32x64_f8f6f4 %0, %1, %2, %0, %3, %3 op_sel_hi:[0,0,0] cbsz:2 blgp:2"
                   : "+v"(acc[I][J])
                   : "v"(fb[S][ST][J]), "v"(fa[S][ST][I]), "v"(s8));
    }
    read<1 - S, 2 * T>(r);
    read<1 - S, 2 * T + 1>(r);
  }
  template <int S, int... T>
  __device__ __forceinline__ void ticks(const Reads& r, const v4i& rs_st, uint32_t so, uint32_t m0_st, int s8,
                                        std::integer_sequence<int, T...>) {
    (tick<S, T>(r, rs_st, so, m0_st, s8), ...);
  }

  // fence<4> (s_nop 4: 5 wait states) stands between VALU writes of the
  // accumulators (the prologue's clear) and the first asm MFMA that reads
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

  // Stage k (128 K) on set S.  Top: this wave's DMA of stage k+1 has landed
  // (with three slots that of k+2 may be outstanding) and its LDS reads of
  // stage k are done, then the barrier: stage k+1 is complete in LDS and no
  // wave still reads slot k % P.  Then the 8 MFMAs of stage k, the reads of
  // stage k+1 and the DMA of stage k+P into slot k % P.  Past the last stage
  // the DMA loads go through a resource of zero records into a slot that
  // holds no live data, and the reads fetch a stale slot into the set no
  // MFMA uses.
  template <int S>
  __device__ __forceinline__ void stage(const Reads& r, int k, int nst, int slot, const v4i& rs_end, int s8) {
    wait_vmcnt<(P - 2) * DPW>();
    frag_fence<S>();
    asm volatile("s_barrier" ::: "memory");
    const bool live = k + P < nst;
    const v4i rs_st = live ? rs : rs_end;
    const uint32_t so = live ? (uint32_t)(k + P) * PANEL : 0u;
    ticks<S>(r, rs_st, so, lds0 + (uint32_t)slot * STAGE + 1024u * DPW * wave, s8,
             std::make_integer_sequence<int, 8>{});
  }
  // Moves the read slot (that of stage k+1, one past `slot`) one ahead,
  // wrapping after slot P-1, and the stage slot.
  static __device__ __forceinline__ void advance(Reads& r, int& slot) {
    r.add(slot == P - 2 ? (uint32_t)(-(P - 1) * STAGE) : (uint32_t)STAGE);
    slot = slot == P - 1 ? 0 : slot + 1;
  }

  // nst: 128-K stages (0 leaves the sums at zero).
  __device__ __forceinline__ void run(int nst) {
    if (nst <= 0) {
      wait_vmcnt<0>();  // loads issued before the call (the B scales)
      return;
    }
    const v4i rs_end = v4i{rs.x, rs.y, 0, rs.w};
    const int s8 = 130;  // E8M0 2^3: both operands hold v/8
    // stages 0..P-1 (zeros past the last stage), then stage 0 into set 0
#pragma unroll
    for (int st = 0; st < P; ++st)
#pragma unroll
      for (int c = 0; c < DPW; ++c)
        lds_dma16(st < nst ? rs : rs_end, voff[c], st < nst ? (uint32_t)st * PANEL : 0u,
                  lds0 + (uint32_t)st * STAGE + 1024u * (DPW * wave + c));
    wait_vmcnt<(P - 1) * DPW>();
    asm volatile("s_barrier" ::: "memory");
    reads<0>(reads_of_slot(0), std::make_integer_sequence<int, 16>{});
    fence<4>();
    // r: read slot of stage k+1; slot: slot of stage k
    Reads r = reads_of_slot(1);
    int slot = 0;
    int k = 0;
    for (; k + 2 <= nst; k += 2) {
      stage<0>(r, k, nst, slot, rs_end, s8);
      advance(r, slot);
      stage<1>(r, k + 1, nst, slot, rs_end, s8);
      advance(r, slot);
    }
    // The last stage's reads fetch a stale slot into the set that no MFMA
    // uses.  They land before the paths merge and before the set's
    // registers could be reused: the fences name every register of the set
    // (set 0 after the pairs, set 1 after an odd last stage).  Wait states
    // after the last MFMA likewise, so that a copy the register allocator
    // places on a merge reads finished accumulators.
    frag_fence<0>();
    fence<7>();
    if (k < nst) {
      stage<0>(r, k, nst, slot, rs_end, s8);
      frag_fence<1>();
      fence<7>();
    }
    fence<7>();
    // the loads past the last stage land before the workgroup's LDS is
    // freed or reused
    wait_vmcnt<0>();
  }
};

// B scales of the wave's 64 columns, sb[j][q] = the four bf16 scales of
// output columns out_col(j, q) + [0, 4), from the wave's 256-byte slot
// (filled by mfma32_prefetch_b_scales, 2 scales a lane from column wn*64).
template <class E>
__device__ __forceinline__ void f6s_read_b_scales(const E& e, const uint8_t* slot, uint2 (&sb)[2][4]) {
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int q = 0; q < 4; ++q) sb[j][q] = *reinterpret_cast<const uint2*>(slot + 2 * (e.out_col(j, q) - e.wn * E::TN));
}

// Epilogue of the 128 x 128 per-channel tile.  Values: (float(acc) *
// a_scale) * b_scale (OUT_BF16, OUT_F32) or the raw int32 sums (OUT_I32).
// Every wave stages its 64 x 64 results in its own region of the idle ring
// (4 bytes a value: row r, 16-byte unit u at r * 256 + 16 * (u ^ (r % 16)),
// conflict-free both ways; bf16: 8 KiB, unit u at r * 128 + 16 * (u ^
// ((r / 2) % 8))), then writes whole row segments with 16-byte stores.
// With MASK only rows [row_lo, row_hi) and columns below col_hi are written
// (col_hi a multiple of 8, so a 16-byte unit is in or out whole).
// NO_NAN (bf16): no value is NaN, so the hardware conversion is exact.
// The stores write through the L2 (cache policy SC1, bit 16 of the buffer
// intrinsics on gfx950): a tile's output then leaves no dirty lines for the
// write-back at the end of the kernel, which the last workgroups' outputs
// otherwise wait for (the C5 forward, one box, A/B of four builds: 1.1 us
// faster per call with a three-slot ring, 1.2 us with a two-slot one).
// With two slots the 4-byte outputs (64 KiB for the four waves) stage in
// two passes.
template <int MODE, bool NO_NAN, bool MASK, class E>
__device__ __forceinline__ void f6s_store(const E& e, const OutView& o, uint8_t* smem, int m0, int n0,
                                          const float (&sa)[2], const uint2 (&sb)[2][4]) {
  constexpr int ESZ = MODE == OUT_BF16 ? 2 : 4;
  constexpr int PITCH = 64 * ESZ;  // bytes of a staged row
  constexpr int UNITS = PITCH / 16;
  constexpr int WRITE_THROUGH = 16;
  // All 64 rows of a wave at once when the four waves' rows fit the ring,
  // else (4-byte values in a two-slot ring) one 32-row half i per pass
  // through the same region: a wave's LDS accesses run in order, so a pass's
  // writes follow the previous pass's reads.
  constexpr int PASSES = E::NW * 64 * PITCH <= E::RING ? 1 : 2;
  constexpr int SROWS = 64 / PASSES;
  static_assert(E::NW * SROWS * PITCH <= E::RING, "the staged results fit the ring");
  auto swz = [](int r) { return UNITS == 16 ? (r & 15) : ((r >> 1) & 7); };
  // every wave has finished reading the ring
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  uint8_t* region = smem + (size_t)e.wave * SROWS * PITCH;
  const int lane = e.lane;
  // read back 64 / UNITS rows per instruction and store whole row segments
  const uint32_t ldo = (uint32_t)o.ld;
  const unsigned long long first = (unsigned long long)m0 * ldo + n0;
  const rsrc_t rsc =
      make_rsrc(static_cast<uint8_t*>(o.out) + first * ESZ, ((unsigned long long)o.rows * ldo - first) * ESZ);
  constexpr int ROWS = 64 / UNITS;
  const int rr = lane / UNITS, u = lane % UNITS;
  const int col = e.wn * E::TN + u * (16 / ESZ);  // first column of the unit in the tile
  const uint32_t voff = ((uint32_t)(e.wm * 64 + rr) * ldo + (uint32_t)col) * ESZ;
  const bool col_in = !MASK || n0 + col < o.col_hi;
#pragma unroll
  for (int h = 0; h < PASSES; ++h) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float s4[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) s4[t] = f6_bf16_at(sb[j][q], t);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          if (PASSES == 2 && i != h) continue;
          const int r = (PASSES == 1 ? 32 * i : 0) + (lane & 31);  // staged row
          const int c = 32 * j + 8 * q + 4 * (lane >> 5);  // first of the lane's 4 columns in the wave's 64
          uint32_t w[4];
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            if constexpr (MODE == OUT_I32) {
              w[t] = (uint32_t)e.acc_int(i, j, 4 * q + t);
            } else {
              float x = e.acc_value(i, j, 4 * q + t) * sa[i];
              x = x * s4[t];
              w[t] = __float_as_uint(x);
            }
          }
          if constexpr (MODE == OUT_BF16) {
            uint32_t lo, hi;
            if constexpr (NO_NAN) {
              lo = pack_bf16x2_nonan(__uint_as_float(w[0]), __uint_as_float(w[1]));
              hi = pack_bf16x2_nonan(__uint_as_float(w[2]), __uint_as_float(w[3]));
            } else {
              lo = f32_to_bf16_rne(__uint_as_float(w[0])) | (f32_to_bf16_rne(__uint_as_float(w[1])) << 16);
              hi = f32_to_bf16_rne(__uint_as_float(w[2])) | (f32_to_bf16_rne(__uint_as_float(w[3])) << 16);
            }
            // unit c / 8, half (c / 4) % 2
            *reinterpret_cast<uint2*>(region + r * PITCH + 16 * ((c >> 3) ^ swz(r)) + 8 * ((c >> 2) & 1)) =
                make_uint2(lo, hi);
          } else {
            *reinterpret_cast<uint4*>(region + r * PITCH + 16 * ((c >> 2) ^ swz(r))) =
                make_uint4(w[0], w[1], w[2], w[3]);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
    for (int t = 0; t < SROWS / ROWS; ++t) {
      const int r = ROWS * t + rr;
      const uint4 x = *reinterpret_cast<const uint4*>(region + r * PITCH + 16 * (u ^ swz(r)));
      const int row = m0 + e.wm * 64 + h * SROWS + r;
      if (!MASK || (col_in && row >= o.row_lo && row < o.row_hi))
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4i, x), rsc, voff,
                                               (uint32_t)(h * SROWS + ROWS * t) * ldo * ESZ, WRITE_THROUGH);
    }
  }
}

// Scales and epilogue of a 128 x 128 tile after the K loop: sa of the
// lane's two rows, B scales from the wave's slot past the ring; bf16 with
// the hardware conversion when every scale is below 2^48 in magnitude
// (then |acc| < 2^31 keeps each product finite: no NaN).
template <int MODE, bool MASK, class E>
__device__ __forceinline__ void f6s_finish(const E& e, const OutView& o, uint8_t* smem, int m0, int n0,
                                           const float (&sa)[2]) {
  uint2 sb[2][4];
  if constexpr (MODE == OUT_I32) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) sb[j][q] = make_uint2(0u, 0u);
    f6s_store<OUT_I32, false, MASK>(e, o, smem, m0, n0, sa, sb);
    return;
  }
  f6s_read_b_scales(e, smem + E::LDS_BYTES + 256 * e.wave, sb);
  if constexpr (MODE == OUT_F32) {
    f6s_store<OUT_F32, false, MASK>(e, o, smem, m0, n0, sa, sb);
  } else {
    constexpr uint32_t F32_LIM = (127u + 48u) << 23, BF16_LIM = (127u + 48u) << 7;
    bool bounded = (__float_as_uint(sa[0]) & 0x7F800000u) < F32_LIM && (__float_as_uint(sa[1]) & 0x7F800000u) < F32_LIM;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint2 w = sb[j][q];
        bounded = bounded && (w.x & 0x7F80u) < BF16_LIM && (w.x & 0x7F800000u) < (BF16_LIM << 16) &&
                  (w.y & 0x7F80u) < BF16_LIM && (w.y & 0x7F800000u) < (BF16_LIM << 16);
      }
    if (__all(bounded)) f6s_store<OUT_BF16, true, MASK>(e, o, smem, m0, n0, sa, sb);
    else f6s_store<OUT_BF16, false, MASK>(e, o, smem, m0, n0, sa, sb);
  }
}

}  // namespace shk
