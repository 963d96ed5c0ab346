// Skinny dense GEMM: output tiles of R = 16, 32 or 64 rows by 64 columns and
// K in steps of 32, for the decode-sized M (and the K multiples of 32) that
// the 64-row-and-up tiles cannot take.
//
// With few output rows the GEMM is bound by reading B once from HBM, so the
// packed operands are streamed as they are (no conversion pass) and widened
// in registers: int4 bytes become int8 values 16*v (shk_common.h) and feed
// v_mfma_i32_16x16x64_i8 with int32 accumulation; int8 operands feed it
// directly.
//
// Streaming.  Every wave owns a private ring of D LDS stage slots filled by
// LDS-DMA (`buffer_load_dwordx4 ... lds`), so the K loop has no workgroup
// barrier: a wave waits only for its own loads.  A stage holds 64 source
// bytes per K-major row (128 int4 / 64 int8 K values) or 64 source rows of an
// MN-major operand.  Loads past an operand's end read zeros through the
// buffer range; A fragments whose K lies at or past K are zeroed, so the
// garbage a K-major row read past its end never reaches a product.
//
// Work split.
//  * Per-channel scales, WOUT = 0: the four waves of a workgroup split the
//    64-column tile's K stages round-robin (stage st goes to wave st % 4)
//    and each multiplies the whole tile; their int32 partials add through
//    LDS.  WOUT > 0: each wave multiplies WOUT output columns of a 4 * WOUT
//    column tile over all of the workgroup's K, so the workgroup reads
//    4 * WOUT contiguous bytes of every MN-major B row.  Either way
//    workgroups can split K further (`splits`): each one writes its exact
//    int32 partial to a workspace slot and counts itself in the tile's
//    arrival counter; the last to arrive adds the other slots and writes the
//    output.  Integer sums do not depend on the order, so the result equals
//    the unsplit one bit for bit.  Partials, counters and the last
//    workgroup's reads use device-scope (sc1) accesses, which stay coherent
//    across the XCDs' L2 caches without a cache writeback; each workgroup
//    waits for its partial stores to complete before it counts itself.  The
//    workspace must be zero before the first launch, and every launch
//    leaves all of it that it used zero (the last workgroup clears the
//    tile's slots and counter), since the counters of one shape can lie
//    where the partials of another were.
//  * Subchannel scales: each group's partial must be scaled and folded into
//    the fp32 total in group order.  The four waves share the tile's 16
//    output columns (GSPLIT) and take the groups in turn: in round r wave w
//    multiplies group 4r + w and scales its integer partial; the four scaled
//    partials meet in LDS, and after the round's barrier wave 0 adds them
//    into the totals in group order (sk_unit_sc).  The group scales come
//    into the stage slots by LDS-DMA.
//
// Fragment layout.  v_mfma_i32_16x16x64_i8 takes B as its first operand
// (D rows = output columns) and A as its second (D columns = output rows);
// lane l carries row or column l % 16 and the 16 K values 16*(l/16) + [0, 16)
// of a 64-K step, so its accumulators hold output row l % 16, columns
// 4*(l/16) + [0, 4) of the 16-column tile.
//  * K-major part (rows x 64 bytes): 16-byte unit u of row r sits at
//    r*64 + 16*(u ^ ((r >> 2) & 3)).  An int4 step s reads 8 bytes at bytes
//    32s + 8*(l/16) of the row (ds_read_b64); an int8 stage reads 16 bytes
//    at 16*(l/16) (ds_read_b128).
//  * MN-major part (64 source rows of RB bytes, RB = 16 * U): unit u (16
//    columns) of source row kp sits at kp*RB + 16*(u ^ ((kp / (256/RB)) &
//    (U - 1))).  ds_read_b64_tr_b8 gives lane i of a 16-lane group column i
//    of 8 consecutive rows: int4 step s reads rows 32s + 8*(l/16) + [0, 8),
//    int8 reads rows 16*(l/16) + [0, 8) and + [8, 16).
// Both swizzles keep the fragment reads of 16 rows or 16 lanes on distinct
// LDS banks.  Packed int4 rows p0..p7 of a lane widen to the K order
// [lo(p0..3), hi(p0..3), lo(p4..7), hi(p4..7)] for A and B alike.
#pragma once

#include "../../include/strix_halo_gfx950.h"
#include "shk_dma.h"

namespace shk {

constexpr int SK_NW = 4;        // waves per workgroup of the subchannel and wide per-channel tiles
constexpr int SK_BN = 64;       // output columns per K-split tile
// An int4 wave accumulates 256 * sum(a*b) in int32: |256 * 64 * K| < 2^31
// for K below 131072, i.e. at most 1023 stages of 128 K per wave and split.
constexpr int SK_MAX_WAVE_STAGES_I4 = 1023;

// Ring depth: the deepest of 4, 3, 2 stage slots whose rings fit the LDS
// budget: 78 KiB for four waves (two workgroups share a CU where the tile
// allows), 150 KiB for eight or more (one workgroup per CU).
constexpr int sk_stage_bytes(int r, int wcols, bool subch) {
  return r * 64 + wcols * 64 + (subch ? (r / 16) * 256 + 256 : 0);
}
constexpr int sk_ring_depth(int stage, int nw, int reserved = 0) {
  const int budget = (nw >= 8 ? 153600 : 79872) - reserved;  // reserved: LDS the tile uses beside the rings
  return nw * 4 * stage <= budget ? 4 : (nw * 3 * stage <= budget ? 3 : 2);
}

template <int BITS_, int LAYOUT_, int R_, bool SWIGLU_, bool SUBCH_, int WOUT_ = SUBCH_ ? 16 : 0, int NW_ = SK_NW,
          int BNK_ = SK_BN, int DEPTH_ = 0>
struct SkCfg {
  static constexpr int BITS = BITS_;
  static constexpr int LAYOUT = LAYOUT_;
  static constexpr bool A_KM = LAYOUT_ != SHK_LAYOUT_TN;
  static constexpr bool B_KM = LAYOUT_ == SHK_LAYOUT_NT;
  static constexpr int R = R_;
  static constexpr int RT = R / 16;
  static constexpr bool SWIGLU = SWIGLU_;
  static constexpr bool SUBCH = SUBCH_;
  static constexpr int NW = NW_;
  static constexpr int NT = 64 * NW;
  static constexpr int WOUT = WOUT_;                  // output columns per wave (0: waves split K)
  static constexpr bool KSPLIT = WOUT == 0;
  static constexpr bool GSPLIT = SUBCH;              // the waves share WOUT columns and split the groups
  static constexpr int BN = KSPLIT ? BNK_ : (GSPLIT ? WOUT : NW * WOUT);  // output columns of a tile
  static constexpr int BNB = SWIGLU ? 2 * BN : BN;    // B columns of a tile ([up | gate] for SwiGLU)
  static constexpr int WCOLS = KSPLIT || GSPLIT ? BNB : BNB / NW;  // B columns a wave loads and multiplies
  static constexpr int CT = WCOLS / 16;              // 16-column B tiles of a wave
  static constexpr int FT = KSPLIT ? 1 : WOUT / 16;   // 16-column output tiles a wave writes
  static constexpr int NFIN = KSPLIT ? BN / 16 : NW;  // waves that write output (K-split: one tile each)
  static constexpr int CF = SWIGLU ? 2 : 1;          // up (and gate)
  static constexpr int FC = FT * CF;                 // int32 tiles a wave holds after the K sum
  static constexpr int KS = BITS == 4 ? 128 : 64;    // K per stage
  static constexpr int STEPS = KS / 64;              // MFMA steps per stage
  static constexpr int A_BYTES = R * 64;
  static constexpr int B_BYTES = WCOLS * 64;
  static constexpr int SA_BYTES = SUBCH ? RT * 256 : 0;
  static constexpr int SB_BYTES = SUBCH ? 256 : 0;
  static constexpr int STAGE = sk_stage_bytes(R, WCOLS, SUBCH);
  static constexpr int A_DMA = A_BYTES / 1024;
  static constexpr int B_DMA = B_BYTES / 1024;
  static constexpr int DPS = A_DMA + B_DMA + (SUBCH ? RT + 1 : 0);  // DMA loads per stage
  // GSPLIT: each wave takes CH consecutive groups per round; two rounds'
  // scaled partials, one 16 x 16 tile (1 KiB) per wave, group, row tile and
  // B column tile, follow the rings
  static constexpr int CH = !GSPLIT ? 0 : (RT * CT == 1 ? 4 : (RT * CT == 2 ? 2 : 1));
  static constexpr int CHAIN = GSPLIT ? 2 * NW * CH * RT * CT * 1024 : 0;
  static constexpr int D = DEPTH_ > 0 ? DEPTH_ : sk_ring_depth(STAGE, NW, CHAIN);
  static constexpr int RING = NW * D * STAGE;
  static constexpr int RED = KSPLIT ? NW * CT * 1024 : 0;  // one row tile of the cross-wave sum
  static constexpr int LDS_BYTES = (RING > RED ? RING : RED) + CHAIN;
  static constexpr int SHIFT = BITS == 4 ? 8 : 0;  // int4 accumulators hold 256 * sum
  static_assert(STAGE == A_BYTES + B_BYTES + SA_BYTES + SB_BYTES, "stage layout");
  static_assert(A_BYTES % 1024 == 0 && B_BYTES % 1024 == 0, "whole DMA blocks per stage");
  static_assert((D - 1) * DPS < 64, "vmcnt range");
  static_assert(LDS_BYTES <= 160 * 1024, "LDS budget");
  static_assert(!KSPLIT || NFIN <= NW, "a K-split tile has a wave for each output column tile");
  static_assert(!KSPLIT || BN == 32 || BN == 64, "K-split tiles are 32 or 64 columns wide");
  static_assert(!SUBCH || WOUT == 16 || (WOUT == 32 && !SWIGLU),
                "subchannel tiles: 16 output columns, or 32 without SwiGLU (one 256-byte b_scale load per stage)");
  static_assert(KSPLIT || WOUT % 16 == 0, "whole 16-column tiles per wave");
};

// Typed LDS loads through address-space-3 pointers (ds_read, not flat loads,
// which would also count against vmcnt).
typedef __attribute__((address_space(3))) v2i sk_lds_v2i;
typedef __attribute__((address_space(3))) v4i sk_lds_v4i;
typedef __attribute__((address_space(3))) uint32_t sk_lds_u32;
__device__ __forceinline__ uint2 sk_ld64(const uint8_t* p) {
  const v2i v = *(const sk_lds_v2i*)(const lds_byte*)p;
  return make_uint2((uint32_t)v.x, (uint32_t)v.y);
}
__device__ __forceinline__ v4i sk_ld128(const uint8_t* p) { return *(const sk_lds_v4i*)(const lds_byte*)p; }
__device__ __forceinline__ uint32_t sk_ld32(const uint8_t* p) { return *(const sk_lds_u32*)(const lds_byte*)p; }
__device__ __forceinline__ void sk_st128(uint8_t* p, const v4i& v) { *(sk_lds_v4i*)(lds_byte*)p = v; }

// XCD-aware order: dispatch sends workgroup u to XCD u % 8, so XCD x gets the
// contiguous logical range that starts at x * (units / 8) + min(x, units % 8).
__device__ __forceinline__ int sk_xcd_remap(int u, int units) {
  const int per = units >> 3, rem = units & 7, x = u & 7;
  return x * per + (x < rem ? x : rem) + (u >> 3);
}

// One operand's part of a stage slot, as seen by one wave.
//  KM: K-major (ROWS tile rows x 64 bytes); otherwise MN-major (64 source
//  rows x RB bytes).  NDMA 1 KiB DMA blocks per stage.
template <bool KM, int NBYTES, int RB>
struct SkPart {
  static constexpr int NDMA = NBYTES / 1024;
  static constexpr int U = RB / 16;
  static constexpr int W = RB > 0 ? 256 / RB : 1;
  uint32_t voff[NDMA];

  static __device__ __forceinline__ uint32_t swk(uint32_t r) { return (r >> 2) & 3u; }
  static __device__ __forceinline__ uint32_t swm(uint32_t kp) { return (kp / (uint32_t)W) & (uint32_t)(U - 1); }

  // rowsrc(r): byte offset of tile row r (K-major); colsrc(u): byte offset
  // of the 16-column unit u inside a source row (MN-major).
  template <class RowSrc, class ColSrc>
  __device__ __forceinline__ void init(int lane, uint32_t ld, RowSrc rowsrc, ColSrc colsrc) {
#pragma unroll
    for (int j = 0; j < NDMA; ++j) {
      const uint32_t pos = 1024u * j + 16u * lane;
      if constexpr (KM) {
        const uint32_t r = pos / 64u, u = ((pos / 16u) & 3u) ^ swk(r);
        voff[j] = rowsrc(r) + 16u * u;
      } else {
        const uint32_t kp = pos / (uint32_t)RB, u = ((pos % (uint32_t)RB) / 16u) ^ swm(kp);
        voff[j] = kp * ld + colsrc(u);
      }
    }
  }
  static __device__ __forceinline__ uint32_t soff(int st, uint32_t ld) {
    return KM ? 64u * (uint32_t)st : 64u * (uint32_t)st * ld;
  }
  __device__ __forceinline__ void issue(const v4i& rs, uint32_t so, uint32_t m0) const {
#pragma unroll
    for (int j = 0; j < NDMA; ++j) lds_dma16(rs, voff[j], so, m0 + 1024u * j);
  }

  // Fragment of 16-row (K-major) or 16-column (MN-major) tile `tb` for MFMA
  // step s of the stage at `base`, widened to int8 for int4.
  template <int BITS>
  static __device__ __forceinline__ v4i frag(const uint8_t* base, int tb, int s, int lane) {
    const int g = lane >> 4, i = lane & 15;
    if constexpr (KM) {
      const uint32_t r = 16u * tb + i;
      if constexpr (BITS == 4) {
        const uint32_t q = 2u * s + (g >> 1);
        const uint2 w = sk_ld64(base + r * 64u + 16u * (q ^ swk(r)) + 8u * (g & 1));
        const uint4 x = widen_chunk(w.x, w.y);
        return v4i{(int)x.x, (int)x.y, (int)x.z, (int)x.w};
      } else {
        return sk_ld128(base + r * 64u + 16u * ((uint32_t)g ^ swk(r)));
      }
    } else {
      if constexpr (BITS == 4) {
        const uint32_t kp = 32u * s + 8u * g + (i >> 1);
        const v2i y = ds_read_tr8(base + kp * RB + 16u * ((uint32_t)tb ^ swm(kp)) + 8u * (i & 1));
        const uint4 x = widen_chunk((uint32_t)y.x, (uint32_t)y.y);
        return v4i{(int)x.x, (int)x.y, (int)x.z, (int)x.w};
      } else {
        const uint32_t kp0 = 16u * g + (i >> 1), kp1 = kp0 + 8u;
        const v2i y0 = ds_read_tr8(base + kp0 * RB + 16u * ((uint32_t)tb ^ swm(kp0)) + 8u * (i & 1));
        const v2i y1 = ds_read_tr8(base + kp1 * RB + 16u * ((uint32_t)tb ^ swm(kp1)) + 8u * (i & 1));
        return v4i{y0.x, y0.y, y1.x, y1.y};
      }
    }
  }
};

// Output of one lane: four consecutive columns n..n+3 of row m.
template <class C>
__device__ __forceinline__ void sk_store(const DenseArgs& p, int m, int n, const float (&up)[4],
                                         const float (&gate)[4], const int (&iup)[4], const int (&igate)[4]) {
  if (p.out_mode == OUT_I32) {
    const long cols = C::SWIGLU ? 2L * p.N : (long)p.N;
    int* o = reinterpret_cast<int*>(p.out) + (long)m * cols + n;
    *reinterpret_cast<int4*>(o) = make_int4(iup[0], iup[1], iup[2], iup[3]);
    if constexpr (C::SWIGLU)
      *reinterpret_cast<int4*>(o + p.N) = make_int4(igate[0], igate[1], igate[2], igate[3]);
    return;
  }
  float v[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) v[q] = C::SWIGLU ? swiglu(up[q], gate[q]) : apply_epi(up[q], p.epilogue);
  const long idx = (long)m * p.N + n;
  if (p.out_mode == OUT_F32) {
    *reinterpret_cast<float4*>(reinterpret_cast<float*>(p.out) + idx) = make_float4(v[0], v[1], v[2], v[3]);
  } else {
    const uint32_t lo = f32_to_bf16_rne(v[0]) | (f32_to_bf16_rne(v[1]) << 16);
    const uint32_t hi = f32_to_bf16_rne(v[2]) | (f32_to_bf16_rne(v[3]) << 16);
    *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(p.out) + idx) = make_uint2(lo, hi);
  }
}

__device__ __forceinline__ void sk_bf16x4(uint2 w, float (&o)[4]) {
  o[0] = __uint_as_float(w.x << 16);
  o[1] = __uint_as_float(w.x & 0xFFFF0000u);
  o[2] = __uint_as_float(w.y << 16);
  o[3] = __uint_as_float(w.y & 0xFFFF0000u);
}

template <class C>
struct SkEngine {
  using PA = SkPart<C::A_KM, C::A_BYTES, C::A_KM ? 0 : C::R>;
  using PB = SkPart<C::B_KM, C::B_BYTES, C::B_KM ? 0 : C::WCOLS>;
  static constexpr int SA_OFF = C::A_BYTES + C::B_BYTES;
  static constexpr int SB_OFF = SA_OFF + C::SA_BYTES;

  const DenseArgs& p;
  int lane, wave;
  int m0, n0;
  PA pa;
  PB pb;
  v4i rsa, rsb;
  uint32_t ring;         // LDS address of this wave's slot 0
  const uint8_t* ringp;  // the same as a pointer
  // subchannel scale loads: a_scale through a resource based at its address
  // rounded down to 4 bytes (sa_mis = 0 or 2 bytes past it)
  v4i rss_a, rss_b;
  uint32_t sb_voff, sa_mis;
  int sh;                  // log2 of the group size (a power of two, 32 .. 256)
  uint32_t sa_row[C::RT];  // element index m * G + lane / 16 of the lane's a_scale load, per row tile

  __device__ __forceinline__ SkEngine(const DenseArgs& args, uint8_t* smem, int lane_, int wave_, int m0_, int n0_)
      : p(args), lane(lane_), wave(wave_), m0(m0_), n0(n0_) {
    ringp = smem + wave * C::D * C::STAGE;
    ring = lds_address(ringp);
    const uint32_t lda = (uint32_t)p.lda, ldb = (uint32_t)p.ldb;
    const int rows_a = C::A_KM ? p.M : p.K * C::BITS / 8;
    const int rows_b = C::B_KM ? p.b_cols : p.K * C::BITS / 8;
    rsa = buffer_words(p.a, (unsigned long long)rows_a * lda);
    rsb = buffer_words(p.b, (unsigned long long)rows_b * ldb);
    const int mm0 = m0, nn0 = n0, w = wave, N = p.N;
    pa.init(lane, lda, [=](uint32_t r) { return (uint32_t)(mm0 + (int)r) * lda; },
            [=](uint32_t u) { return (uint32_t)(mm0 + 16 * (int)u); });
    // B column of tile column t: the wave's window (KSPLIT: the whole tile),
    // SwiGLU gate columns N further.
    auto bcol = [=](int t) -> uint32_t {
      if constexpr (C::KSPLIT) {
        if constexpr (C::SWIGLU) return (uint32_t)(t < C::BN ? nn0 + t : N + nn0 + t - C::BN);
        return (uint32_t)(nn0 + t);
      } else {
        constexpr int WO = C::WOUT;
        const int wo = C::GSPLIT ? 0 : WO * w;  // GSPLIT: every wave takes the tile's columns
        if constexpr (C::SWIGLU) return (uint32_t)(t < WO ? nn0 + wo + t : N + nn0 + wo + t - WO);
        return (uint32_t)(nn0 + wo + t);
      }
    };
    pb.init(lane, ldb, [=](uint32_t r) { return bcol((int)r) * ldb; }, [=](uint32_t u) { return bcol(16 * (int)u); });
    if constexpr (C::SUBCH) {
      const unsigned long long ab = (unsigned long long)p.a_scale;
      sa_mis = (uint32_t)(ab & 3u);
      // records rounded up to whole dwords: the last scale's dword may end
      // 2 bytes past the tensor, inside the same aligned dword
      rss_a = buffer_words((const void*)(ab - sa_mis),
                           (sa_mis + 2ull * (unsigned long long)p.M * p.scale_cols + 3ull) & ~3ull);
      rss_b = buffer_words(p.b_scale, 2ull * (unsigned long long)p.scale_cols * p.b_cols);
      // lane = 16 j + e: group slot j, dword e % 8 of piece e / 8 (up, gate)
      const int j = lane >> 4, e = lane & 15;
      const int piece = C::CT == 2 ? (e >> 3) : 0;  // 16-column piece (SwiGLU: up, gate)
      const int col = (int)bcol(16 * piece) + 2 * (e & 7);
      sb_voff = 2u * (uint32_t)(j * p.b_cols + col);
      sh = __builtin_ctz((unsigned)p.subchannel);
#pragma unroll
      for (int rt = 0; rt < C::RT; ++rt)
        sa_row[rt] = (uint32_t)((m0 + 16 * rt + (lane & 15)) * p.scale_cols + (lane >> 4));
    }
  }

  // DMA of stage st into slot `slot`.
  __device__ __forceinline__ void issue(int st, int slot) const {
    const uint32_t base = ring + (uint32_t)(slot * C::STAGE);
    pa.issue(rsa, PA::soff(st, (uint32_t)p.lda), base);
    pb.issue(rsb, PB::soff(st, (uint32_t)p.ldb), base + C::A_BYTES);
    if constexpr (C::SUBCH) {
      const int g0 = (st * C::KS) >> sh;  // the first group of the stage
      // a-scale dword holding element (m, g0 + j) of row m = m0 + 16 rt + lane % 16
#pragma unroll
      for (int rt = 0; rt < C::RT; ++rt)
        lds_dma4(rss_a, (sa_mis + 2u * (sa_row[rt] + (uint32_t)g0)) & ~3u, 0u, base + SA_OFF + 256u * rt);
      lds_dma4(rss_b, sb_voff, 2u * (uint32_t)g0 * (uint32_t)p.b_cols, base + SB_OFF);
    }
  }
};

// Waits for the LDS reads still in flight before a DMA may overwrite their slot.
__device__ __forceinline__ void sk_lds_drain() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// vmcnt wait with a compile-time count, chosen at run time from {N, 0}.
template <int N>
__device__ __forceinline__ void sk_wait(bool full) {
  if (full)
    wait_vmcnt<N>();
  else
    wait_vmcnt<0>();
}

// ---------------------------------------------------------------------------
// Per-channel tile: waves split K (WOUT = 0) or columns, workgroups split K
// `splits` ways.

// Device-scope (sc1) 16-byte accesses of the split partials (cache policy
// bit SC1 = 16 of the buffer intrinsics on gfx950).
constexpr int SK_SC1 = 16;
// Partial slots the last workgroup of a split tile loads at once.
constexpr int SK_BATCH = 4;

// The epilogue scales of a finalizer wave, loaded before its K loop so that
// their latency passes under it: a_scale of its RT rows, b_scale of the
// four columns n..n+3 of each output tile (up, and gate for SwiGLU).
template <class C>
struct SkScales {
  float sa[C::RT];
  float sbu[C::FT][4], sbg[C::FT][4];
  __device__ __forceinline__ void load(const DenseArgs& p, int m0, int n0, int wave, int lane) {
    const int g = lane >> 4;
#pragma unroll
    for (int rt = 0; rt < C::RT; ++rt) sa[rt] = load_bf16(p.a_scale + m0 + 16 * rt + (lane & 15));
#pragma unroll
    for (int f = 0; f < C::FT; ++f) {
      const int n = n0 + (C::KSPLIT ? 16 * wave : C::WOUT * wave + 16 * f) + 4 * g;
      sk_bf16x4(*reinterpret_cast<const uint2*>(p.b_scale + n), sbu[f]);
      if constexpr (C::SWIGLU) {
        sk_bf16x4(*reinterpret_cast<const uint2*>(p.b_scale + p.N + n), sbg[f]);
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) sbg[f][q] = 0.0f;
      }
    }
  }
};

template <class C>
__device__ __forceinline__ void sk_unit_pc(const DenseArgs& p, uint8_t* smem, int* last_flag, int lane, int wave,
                                           int tm, int tn, int split, int splits, int tile) {
  SkEngine<C> e(p, smem, lane, wave, tm * C::R, tn * C::BN);
  const int nst = (p.K + C::KS - 1) / C::KS;
  const int per = (nst + splits - 1) / splits;
  const int lo = split * per, hi = min(nst, lo + per);
  // this wave's stages: lo + first + i * stride for i < mine
  const int first = C::KSPLIT ? wave : 0, stride = C::KSPLIT ? C::NW : 1;
  const int mine = hi - lo - first > 0 ? (hi - lo - first + stride - 1) / stride : 0;

  v4i acc[C::RT][C::CT];
#pragma unroll
  for (int rt = 0; rt < C::RT; ++rt)
#pragma unroll
    for (int c = 0; c < C::CT; ++c) acc[rt][c] = v4i{0, 0, 0, 0};

  const int g = lane >> 4;
  // the first stages' loads go out before anything else waits on memory
#pragma unroll
  for (int i = 0; i < C::D - 1; ++i)
    if (i < mine) e.issue(lo + first + i * stride, i);
  SkScales<C> scl;
  if (p.out_mode != OUT_I32 && wave < C::NFIN) scl.load(p, e.m0, e.n0, wave, lane);
  for (int i = 0; i < mine; ++i) {
    const bool ahead = i + C::D - 1 < mine;
    if (ahead) {
      sk_lds_drain();
      e.issue(lo + first + (i + C::D - 1) * stride, (i + C::D - 1) % C::D);
    }
    sk_wait<(C::D - 1) * C::DPS>(ahead);
    const int st = lo + first + i * stride;
    const uint8_t* slot = e.ringp + (i % C::D) * C::STAGE;
#pragma unroll
    for (int s = 0; s < C::STEPS; ++s) {
      const bool kin = st * C::KS + 64 * s + 16 * g < p.K;
      v4i y[C::RT], x[C::CT];
#pragma unroll
      for (int rt = 0; rt < C::RT; ++rt) {
        const v4i f = SkEngine<C>::PA::template frag<C::BITS>(slot, rt, s, lane);
        y[rt] = kin ? f : v4i{0, 0, 0, 0};
      }
#pragma unroll
      for (int c = 0; c < C::CT; ++c) x[c] = SkEngine<C>::PB::template frag<C::BITS>(slot + C::A_BYTES, c, s, lane);
#pragma unroll
      for (int rt = 0; rt < C::RT; ++rt)
#pragma unroll
        for (int c = 0; c < C::CT; ++c) acc[rt][c] = mfma64(x[c], y[rt], acc[rt][c]);
    }
  }
  wait_vmcnt<0>();

  // fin[rt][fc]: fc = f (up of output tile f) or FT + f (its gate).  K-split
  // waves add their sums through LDS, one row tile at a time, and wave
  // w < NFIN keeps output tile w: B tiles w (up) and C::BN / 16 + w (gate).
  const bool finalizer = wave < C::NFIN;
  v4i fin[C::RT][C::FC];
  if constexpr (C::KSPLIT) {
#pragma unroll
    for (int rt = 0; rt < C::RT; ++rt) {
      __syncthreads();
#pragma unroll
      for (int c = 0; c < C::CT; ++c) {
        v4i v = acc[rt][c];
        if constexpr (C::SHIFT) v = v4i{v.x >> C::SHIFT, v.y >> C::SHIFT, v.z >> C::SHIFT, v.w >> C::SHIFT};
        sk_st128(smem + 16 * ((wave * C::CT + c) * 64 + lane), v);
      }
      __syncthreads();
#pragma unroll
      for (int cf = 0; cf < C::CF; ++cf) {
        const int c = cf * C::NFIN + (finalizer ? wave : 0);
        v4i s = v4i{0, 0, 0, 0};
        if (finalizer) {
#pragma unroll
          for (int w = 0; w < C::NW; ++w) s += sk_ld128(smem + 16 * ((w * C::CT + c) * 64 + lane));
        }
        fin[rt][cf] = s;
      }
    }
  } else {
#pragma unroll
    for (int rt = 0; rt < C::RT; ++rt)
#pragma unroll
      for (int c = 0; c < C::CT; ++c) {
        const v4i v = acc[rt][c];
        fin[rt][c] = C::SHIFT ? v4i{v.x >> C::SHIFT, v.y >> C::SHIFT, v.z >> C::SHIFT, v.w >> C::SHIFT} : v;
      }
  }

  if (splits > 1) {
    // exact int32 partials: slot (tile, split) of the workspace after the
    // counters; finalizer wave w's part is RT x FC tiles of 64 lanes x 16 bytes
    int* counters = reinterpret_cast<int*>(p.work);
    const long counter_bytes = ((long)(p.M / C::R) * (p.N / C::BN) * 4 + 255) & ~255L;
    constexpr long WAVE_BYTES = (long)C::RT * C::FC * 1024;
    constexpr long SLOT_BYTES = C::NFIN * WAVE_BYTES;
    const uint8_t* parts = p.work + counter_bytes;
    const long ws_bytes = counter_bytes + ((long)(p.M / C::R) * (p.N / C::BN)) * splits * SLOT_BYTES;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(parts), 0, (int)(ws_bytes - counter_bytes), 0x00020000);
    const uint32_t mine_off = (uint32_t)(((long)tile * splits + split) * SLOT_BYTES + wave * WAVE_BYTES);
    if (finalizer) {
#pragma unroll
      for (int rt = 0; rt < C::RT; ++rt)
#pragma unroll
        for (int fc = 0; fc < C::FC; ++fc)
          __builtin_amdgcn_raw_buffer_store_b128(fin[rt][fc], rs, mine_off + ((rt * C::FC + fc) * 64 + lane) * 16u, 0,
                                                 SK_SC1);
    }
    wait_vmcnt<0>();  // the partial has reached the device-coherent level
    __syncthreads();
    if (threadIdx.x == 0)
      *last_flag = __hip_atomic_fetch_add(counters + tile, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                   splits - 1;
    __syncthreads();
    if (!*last_flag || !finalizer) return;
    // The other splits' partials, SK_BATCH slots at a time: every load of a
    // batch is issued before the first add, so their round trips overlap
    // (M = 16, N = K = 8192 on 4 splits: 15.4 -> 14.9 us per launch from
    // HBM).  This split's own slot and the slots past the last read through
    // an offset beyond the resource, which returns zeros.
    for (int s0 = 0; s0 < splits; s0 += SK_BATCH) {
      v4i part[SK_BATCH][C::RT][C::FC];
#pragma unroll
      for (int j = 0; j < SK_BATCH; ++j) {
        const int s2 = s0 + j;
        const uint32_t off = (s2 < splits && s2 != split)
                                 ? (uint32_t)(((long)tile * splits + s2) * SLOT_BYTES + wave * WAVE_BYTES)
                                 : 0x80000000u;
#pragma unroll
        for (int rt = 0; rt < C::RT; ++rt)
#pragma unroll
          for (int fc = 0; fc < C::FC; ++fc)
            part[j][rt][fc] = __builtin_amdgcn_raw_buffer_load_b128(
                rs, off + ((rt * C::FC + fc) * 64 + lane) * 16u, 0, SK_SC1);
      }
#pragma unroll
      for (int j = 0; j < SK_BATCH; ++j)
#pragma unroll
        for (int rt = 0; rt < C::RT; ++rt)
#pragma unroll
          for (int fc = 0; fc < C::FC; ++fc) fin[rt][fc] += part[j][rt][fc];
    }
    // Every slot of the tile goes back to zero, and so does its counter: a
    // later launch of another shape may place its counters over this
    // launch's partials, so a launch leaves all the workspace it used zero.
    for (int s2 = 0; s2 < splits; ++s2) {
      const uint32_t off = (uint32_t)(((long)tile * splits + s2) * SLOT_BYTES + wave * WAVE_BYTES);
#pragma unroll
      for (int rt = 0; rt < C::RT; ++rt)
#pragma unroll
        for (int fc = 0; fc < C::FC; ++fc)
          __builtin_amdgcn_raw_buffer_store_b128(v4i{0, 0, 0, 0}, rs, off + ((rt * C::FC + fc) * 64 + lane) * 16u, 0,
                                                 SK_SC1);
    }
    if (threadIdx.x == 0) __hip_atomic_store(counters + tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  if (!finalizer) return;
  // Epilogue: (float(sum) * a_scale[m]) * b_scale[n], then ReLU2 / SwiGLU.
#pragma unroll
  for (int f = 0; f < C::FT; ++f) {
    const int n = e.n0 + (C::KSPLIT ? 16 * wave : C::WOUT * wave + 16 * f) + 4 * g;
    const float(&sbu)[4] = scl.sbu[f];
    const float(&sbg)[4] = scl.sbg[f];
#pragma unroll
    for (int rt = 0; rt < C::RT; ++rt) {
      const int m = e.m0 + 16 * rt + (lane & 15);
      float up[4], gt[4];
      int iu[4], ig[4];
      const float sa = scl.sa[rt];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        iu[q] = fin[rt][f][q];
        ig[q] = fin[rt][C::SWIGLU ? C::FT + f : f][q];
        float v = (float)iu[q];
        v = v * sa;
        up[q] = v * sbu[q];
        if constexpr (C::SWIGLU) {
          float u = (float)ig[q];
          u = u * sa;
          gt[q] = u * sbg[q];
        } else {
          gt[q] = 0.0f;
        }
      }
      sk_store<C>(p, m, n, up, gt, iu, ig);
    }
  }
}

// ---------------------------------------------------------------------------
// Subchannel tile (GSPLIT): the four waves share the tile's 16 output
// columns (and the gate's 16 for SwiGLU) and take its groups in chunks of
// CH consecutive groups: in round r, wave w multiplies chunk 4r + w (its
// stages, or for chunks shorter than a stage its groups' steps of one
// stage, the A fragments of the other lanes zeroed for groups of 32) and
// scales each group's integer partial,
// x = (float(sum_g) * a_scale[m, g]) * b_scale[g, n] (api.py:311-325).  The
// round's 4 CH values of x go through LDS; after the round's barrier wave 0
// adds them into the totals in group order, which is the reference's order
// of the sums (the raw mode adds the integer partials).  Wave 0 stores the
// tile.

// x of one group from its integer partials and the scales in the stage slot
// (j: the group's slot among the stage's scales; odd_a[rt]: whether the
// lane's a_scale element of group 0 is the high half of its dword).
template <class C>
__device__ __forceinline__ void sk_scale_group(const DenseArgs& p, const uint8_t* slot, int j, int g, int lane,
                                               const int (&odd_a)[C::RT], const v4i (&acc)[C::RT][C::CT],
                                               v4i (&x)[C::RT][C::CT]) {
  if (p.out_mode == OUT_I32) {
#pragma unroll
    for (int rt = 0; rt < C::RT; ++rt)
#pragma unroll
      for (int c = 0; c < C::CT; ++c)
#pragma unroll
        for (int q = 0; q < 4; ++q) x[rt][c][q] = acc[rt][c][q] >> C::SHIFT;
    return;
  }
  float sb[C::CT][4];
#pragma unroll
  for (int c = 0; c < C::CT; ++c)
    sk_bf16x4(sk_ld64(slot + SkEngine<C>::SB_OFF + 64 * j + 32 * c + 8 * (lane >> 4)), sb[c]);
#pragma unroll
  for (int rt = 0; rt < C::RT; ++rt) {
    const uint32_t w = sk_ld32(slot + SkEngine<C>::SA_OFF + 256 * rt + 4 * (16 * j + (lane & 15)));
    const float sa = __uint_as_float(((odd_a[rt] + g) & 1) ? (w & 0xFFFF0000u) : (w << 16));
#pragma unroll
    for (int c = 0; c < C::CT; ++c)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float v = (float)(acc[rt][c][q] >> C::SHIFT);
        v = v * sa;
        v = v * sb[c][q];
        x[rt][c][q] = __float_as_int(v);
      }
  }
}

template <class C>
__device__ __forceinline__ void sk_unit_sc(const DenseArgs& p, uint8_t* smem, int lane, int wave, int tm, int tn) {
  static_assert(C::GSPLIT && C::NW == 4, "four waves take the groups in turn");
  SkEngine<C> e(p, smem, lane, wave, tm * C::R, tn * C::BN);
  constexpr int KSH = C::BITS == 4 ? 7 : 6;  // log2(KS)
  static_assert((1 << KSH) == C::KS, "stage K");
  constexpr int CH = C::CH;
  constexpr int CHSH = CH == 4 ? 2 : (CH == 2 ? 1 : 0);
  static_assert((1 << CHSH) == CH, "CH is a power of two");
  const int sh = e.sh;
  const int S = 1 << sh;
  const int G = p.scale_cols;                   // K / S
  const int nch = (G + CH - 1) >> CHSH;         // chunks of CH groups
  const int lsh = sh + CHSH;                    // log2 of a chunk's K
  const int spc_sh = lsh > KSH ? lsh - KSH : 0;
  const int spc = 1 << spc_sh;                  // stages per chunk (a chunk shorter than a stage: 1)
  const int rounds = (nch + 3) >> 2;
  const int my_chunks = wave < nch ? ((nch - 1 - wave) >> 2) + 1 : 0;
  const int n_i = my_chunks << spc_sh;          // this wave's stages
  const int lg = lane >> 4;
  // this wave's stage i: stage i % spc of chunk 4 (i / spc) + wave
  auto stage_of = [&](int i) { return (((4 * (i >> spc_sh) + wave) << lsh) >> KSH) + (i & (spc - 1)); };
  uint8_t* chain = smem + (C::LDS_BYTES - C::CHAIN);
  auto chain_at = [&](int par, int w, int cg, int rt, int c) {
    return chain + ((((par * C::NW + w) * CH + cg) * C::RT + rt) * C::CT + c) * 1024 + 16 * lane;
  };
  int odd_a[C::RT];
#pragma unroll
  for (int rt = 0; rt < C::RT; ++rt) {
    const int m = e.m0 + 16 * rt + (lane & 15);
    odd_a[rt] = ((m & p.scale_cols) + (int)(e.sa_mis >> 1)) & 1;  // parity of m * G + sa_mis / 2
  }
  // one 64-K MFMA step of a stage into a; A fragments zeroed off the lanes `on`
  auto step = [&](const uint8_t* slot, int s, bool on, v4i (&a)[C::RT][C::CT]) {
    v4i y[C::RT], xb[C::CT];
#pragma unroll
    for (int rt = 0; rt < C::RT; ++rt) {
      const v4i f = SkEngine<C>::PA::template frag<C::BITS>(slot, rt, s, lane);
      y[rt] = on ? f : v4i{0, 0, 0, 0};
    }
#pragma unroll
    for (int c = 0; c < C::CT; ++c) xb[c] = SkEngine<C>::PB::template frag<C::BITS>(slot + C::A_BYTES, c, s, lane);
#pragma unroll
    for (int rt = 0; rt < C::RT; ++rt)
#pragma unroll
      for (int c = 0; c < C::CT; ++c) a[rt][c] = mfma64(xb[c], y[rt], a[rt][c]);
  };
  auto clear = [](v4i (&a)[C::RT][C::CT]) {
#pragma unroll
    for (int rt = 0; rt < C::RT; ++rt)
#pragma unroll
      for (int c = 0; c < C::CT; ++c) a[rt][c] = v4i{0, 0, 0, 0};
  };
  // group g's partials, scaled, into its place of the round's chain buffer
  auto put = [&](const uint8_t* slot, int st, int g, int k, int par, const v4i (&a)[C::RT][C::CT]) {
    v4i x[C::RT][C::CT];
    sk_scale_group<C>(p, slot, g - ((st << KSH) >> sh), g, lane, odd_a, a, x);
#pragma unroll
    for (int rt = 0; rt < C::RT; ++rt)
#pragma unroll
      for (int c = 0; c < C::CT; ++c) sk_st128(chain_at(par, wave, g - (k << CHSH), rt, c), x[rt][c]);
  };

  float tot[C::RT][C::CT][4];
#pragma unroll
  for (int rt = 0; rt < C::RT; ++rt)
#pragma unroll
    for (int c = 0; c < C::CT; ++c)
#pragma unroll
      for (int q = 0; q < 4; ++q) tot[rt][c][q] = 0.0f;

#pragma unroll
  for (int d = 0; d < C::D - 1; ++d)
    if (d < n_i) e.issue(stage_of(d), d);
  v4i acc[C::RT][C::CT];
  clear(acc);
  int i = 0;
  for (int r = 0; r < rounds; ++r) {
    const int k = 4 * r + wave;  // this wave's chunk: groups [k CH, (k + 1) CH)
    const int par = r & 1;
    if (k < nch) {
      for (int j = 0; j < spc; ++j, ++i) {
        const bool ahead = i + C::D - 1 < n_i;
        if (ahead) {
          sk_lds_drain();
          e.issue(stage_of(i + C::D - 1), (i + C::D - 1) % C::D);
        }
        sk_wait<(C::D - 1) * C::DPS>(ahead);
        const uint8_t* slot = e.ringp + (i % C::D) * C::STAGE;
        const int st = stage_of(i);
        if (S >= C::KS) {
          // the stage is part of group (st KS) / S, whose last stage folds it
#pragma unroll
          for (int s = 0; s < C::STEPS; ++s) step(slot, s, (st << KSH) + 64 * s + 16 * lg < p.K, acc);
          if ((((st + 1) << KSH) & (S - 1)) == 0) {
            put(slot, st, (st << KSH) >> sh, k, par, acc);
            clear(acc);
          }
        } else {
          // groups q of the stage that belong to the chunk: K [q S, (q + 1) S)
          // of the stage, one step (S = 64) or one half of one (S = 32)
          const int gs = (st << KSH) >> sh;
#pragma unroll
          for (int q = 0; q < C::KS / 32; ++q) {
            const int g = gs + q;
            if ((q << sh) >= C::KS || g < (k << CHSH) || g >= ((k + 1) << CHSH) || g >= G) continue;
            const int s = (q << sh) >> 6;
            const int kb = (st << KSH) + 64 * s;
            const bool on = (S >= 64 || (lg >> 1) == (q & 1)) && kb + 16 * lg < p.K;
            v4i a[C::RT][C::CT];
            clear(a);
            step(slot, s, on, a);
            put(slot, st, g, k, par, a);
          }
        }
      }
    }
    // the round's partials are in LDS (no wait on the wave-private DMA)
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (wave == 0) {
#pragma unroll
      for (int w = 0; w < 4; ++w)
#pragma unroll
        for (int cg = 0; cg < CH; ++cg) {
          if ((((4 * r + w) << CHSH) + cg) >= G) continue;
#pragma unroll
          for (int rt = 0; rt < C::RT; ++rt)
#pragma unroll
            for (int c = 0; c < C::CT; ++c) {
              const v4i v = sk_ld128(chain_at(par, w, cg, rt, c));
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                if (p.out_mode == OUT_I32)
                  tot[rt][c][q] = __int_as_float(__float_as_int(tot[rt][c][q]) + v[q]);
                else
                  tot[rt][c][q] = tot[rt][c][q] + __int_as_float(v[q]);
              }
            }
        }
    }
  }
  wait_vmcnt<0>();
  if (wave != 0) return;

  constexpr int OT = C::SWIGLU ? C::CT / 2 : C::CT;  // 16-column output tiles (SwiGLU: the gate's follow)
#pragma unroll
  for (int rt = 0; rt < C::RT; ++rt)
#pragma unroll
    for (int ot = 0; ot < OT; ++ot) {
      const int m = e.m0 + 16 * rt + (lane & 15);
      const int n = e.n0 + 16 * ot + 4 * lg;
      float up[4], gt[4];
      int iu[4], ig[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        up[q] = tot[rt][ot][q];
        gt[q] = tot[rt][C::SWIGLU ? ot + OT : ot][q];
        iu[q] = __float_as_int(up[q]);
        ig[q] = __float_as_int(gt[q]);
      }
      sk_store<C>(p, m, n, up, gt, iu, ig);
    }
}

// One workgroup per unit (standard schedule) or one per resident slot,
// striding over the units (persistent schedule).  Units are (split, column
// tile, row tile) with the row tile fastest, so the workgroups reading the
// same B columns run together on one XCD.
template <class C>
__global__ __launch_bounds__(C::NT) void sk_gemm_kernel(const DenseArgs p) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[C::LDS_BYTES];
  __shared__ int last_flag;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tiles_m = p.M / C::R, tiles = tiles_m * (p.N / C::BN);
  const int splits = C::SUBCH ? 1 : p.sk_splits;
  const int units = tiles * splits;
  for (int u = blockIdx.x; u < units; u += gridDim.x) {
    const int lu = sk_xcd_remap(u, units);
    const int split = lu / tiles, t = lu - split * tiles;
    const int tn = t / tiles_m, tm = t - tn * tiles_m;
    if constexpr (C::SUBCH)
      sk_unit_sc<C>(p, smem, lane, wave, tm, tn);
    else
      sk_unit_pc<C>(p, smem, &last_flag, lane, wave, tm, tn, split, splits, tn * tiles_m + tm);
    __syncthreads();
  }
}

}  // namespace shk
