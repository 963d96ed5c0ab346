// int4 x int4 dense GEMM on the bf6 (e3m2) MFMA.
//
// gfx950 has no int4 MFMA, but every int4 value -8..7 is exact in the 6-bit
// float format e3m2 ("bf6": sign, 3 exponent bits with bias 3, 2 mantissa
// bits: 1, 2, 3 = 1.5*2, 4, 5 = 1.25*4, 6, 7 = 1.75*4 and 8 are all
// representable), and v_mfma_scale_f32_16x16x128_f8f6f4 multiplies bf6
// operands at twice the int8 MFMA rate.  Products of two such values are
// integers of magnitude <= 64 and the MFMA accumulates in fp32, which holds
// every integer below 2^24 exactly, so for K <= 2^18 every partial sum, and
// the result, is the exact int32 sum (|sum| <= 64 * K <= 2^24).  The epilogue
// therefore sees the same integer as the int8 engines and produces the same
// bits.
//
// The path runs in two launches:
//  1. f6_pack_* converts each operand, in whichever layout it arrives, into
//     the "block" format in a caller workspace: a 16-row x 128-K block is
//     1536 bytes, 24 per MFMA lane (lane l: row l % 16, K values
//     32*(l/16) + [0, 32) of the block) split into a 1024-byte part (the
//     lane's first 16 bytes at 16*l) and a 512-byte part (its last 8 bytes at
//     1024 + 8*l).  Blocks are stored panel-major: block (p, kb) of the
//     16-row panel p and K block kb sits at (p * KB + kb) * 1536.
//  2. f6_gemm_kernel streams 256 x 128 blocks of both operands with LDS-DMA
//     into a three-slot ring (48 KiB per stage) and reads each fragment with
//     one ds_read_b128 and one ds_read_b64 of consecutive lane addresses,
//     which is free of bank conflicts without a swizzle.  The K loop has no
//     VALU work: DMA, LDS reads and MFMAs only.
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

namespace shk {

typedef int v6i __attribute__((ext_vector_type(6)));
typedef _Float16 f6_h2 __attribute__((ext_vector_type(2)));
typedef _Float16 f6_h32 __attribute__((ext_vector_type(32)));

constexpr int F6_BLOCK = 1536;     // bytes of a 16-row x 128-K bf6 block
constexpr int F6_MAX_K = 262144;   // 64 * K <= 2^24: fp32 partial sums stay exact
constexpr int F6_TILE = 256;       // packed rows per GEMM tile (A rows, B columns)

// Bytes of one operand with `rows` rows (a multiple of 256) and K (a
// multiple of 128) in block format.
__host__ __device__ constexpr unsigned long long f6_operand_bytes(long rows, long k) {
  return (unsigned long long)rows * (unsigned long long)k * 3ull / 4ull;
}

struct F6PackArgs {
  const uint8_t* src;
  uint8_t* dst;
  long ld;       // bytes between consecutive source rows
  int rows;      // packed rows (a multiple of 256)
  int kb;        // K / 128
  int swiglu_n;  // > 0: SwiGLU B with N output columns (rows interleave up and gate)
};

// Converts one operand into block format (k_f6pack.hip).  mn_major: the
// source is stored K-row by K-row (two K values per byte of every row).
hipError_t launch_f6_pack(const F6PackArgs& a, bool mn_major, hipStream_t s);

// ---------------------------------------------------------------------------
// GEMM engine.  Four waves in 2 x 2, each owning 128 x 128 of the 256-row
// tile (SwiGLU: 128 rows x 64 output columns, up and gate).  Accumulator
// [i][j] is the 16 x 16 block of A fragment i and B fragment j; the B
// fragment is the MFMA's first operand, so lane l holds row l % 16 and the
// four columns 4*(l/16) + [0, 4) of the block.
//
// Schedule of stage k (one 128-K block, slot k % 3 of the ring):
//  * top: wait for this wave's DMA of stage k+1 and its own LDS reads of
//    stage k, then the barrier: stage k+1 is complete in LDS and no wave
//    still reads slot k % 3;
//  * 64 MFMAs on the fragments of stage k (register set k % 2); after each
//    of the first 32 one LDS read of stage k+1 into the other set, after
//    each odd one of the next 24 one DMA load of stage k+3 into slot k % 3.
// The DMA of a stage is thus issued two stages before its data is read.
template <class C>
struct F6Engine {
  static constexpr int P = 3;
  static constexpr int NW = 4;
  static constexpr int OPB = 16 * F6_BLOCK;      // one operand's stage: 24 KiB
  static constexpr int STAGE = 2 * OPB;          // 48 KiB
  static constexpr int LDS_BYTES = P * STAGE;    // 144 KiB
  static constexpr int DPW = STAGE / 1024 / NW;  // 12 DMA loads per wave per stage
  static_assert(C::BM == 256 && C::WM == 2 && C::WN == 2 && C::FM == 8 && C::FN2 == 8, "256-row tiles, 2x2 waves");
  static_assert(C::BROWS == 256, "256 packed B rows per tile");

  v4i acc[8][8];
  v6i fa[2][8];
  v6i fb[2][8];
  uint32_t voff[DPW];
  v4i rs;        // this wave's DMA operand (waves 0-1: A, 2-3: B)
  uint32_t lds0; // LDS address of slot 0
  int lane, wave, wm, wn;
  int one;       // E8M0 scale 2^0

  // LDS read addresses of this lane in one slot: 16- and 8-byte parts of
  // the wave's A fragment 0 and B fragment 0 (fragment f adds 1536 * f).
  struct Reads {
    uint32_t a16, a8, b16, b8;
    __device__ __forceinline__ void add(uint32_t d) {
      a16 += d;
      a8 += d;
      b16 += d;
      b8 += d;
    }
  };

  __device__ __forceinline__ int out_row(int i) const { return wm * C::TM + 16 * i + (lane & 15); }
  __device__ __forceinline__ int out_col(int j) const {
    return wn * C::TN + 16 * (j < C::FN ? j : j - C::FN) + 4 * (lane >> 4);
  }

  // a6 / b6: block-format operands; the tile's first panels are m0 / 16 and
  // 16 * bt (bt: B tile index).
  __device__ __forceinline__ void setup(uint8_t* smem, const uint8_t* a6, const uint8_t* b6, int m0, int bt, int kb,
                                        unsigned long long a_bytes, unsigned long long b_bytes) {
    lane = threadIdx.x & 63;
    wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    wm = wave % 2;
    wn = wave / 2;
    one = 127;
    lds0 = lds_address(smem);
    const unsigned long long panel_bytes = (unsigned long long)kb * F6_BLOCK;
    const bool is_a = wave < 2;
    const unsigned long long first =
        (is_a ? (unsigned long long)(m0 / 16) : (unsigned long long)bt * 16) * panel_bytes;
    rs = buffer_words((is_a ? a6 : b6) + first, (is_a ? a_bytes : b_bytes) - first);
    // DMA load c of this wave fills stage bytes [1024 * (DPW*wave + c), +1024)
#pragma unroll
    for (int c = 0; c < DPW; ++c) {
      const uint32_t o = 1024u * (DPW * wave + c) + 16u * lane - (is_a ? 0u : (uint32_t)OPB);
      const uint32_t blk = o / F6_BLOCK, r = o % F6_BLOCK;
      voff[c] = blk * (uint32_t)panel_bytes + r;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[i][j] = v4i{0, 0, 0, 0};
  }

  __device__ __forceinline__ Reads reads_of_slot(int slot) const {
    const uint32_t s = lds0 + (uint32_t)slot * STAGE;
    return Reads{s + 8u * wm * F6_BLOCK + 16u * lane, s + 8u * wm * F6_BLOCK + 1024u + 8u * lane,
                 s + OPB + 8u * wn * F6_BLOCK + 16u * lane, s + OPB + 8u * wn * F6_BLOCK + 1024u + 8u * lane};
  }

  __device__ __forceinline__ void dma(int st, int slot, int c) const {
    lds_dma16(rs, voff[c], (uint32_t)st * F6_BLOCK, lds0 + (uint32_t)slot * STAGE + 1024u * (DPW * wave + c));
  }

  // LDS read Q (0..31) of a stage into set S: fragments in the order A0,
  // B0..B7, A1..A7 (the order of their first use), each as its 16-byte then
  // its 8-byte part.
  template <int S, int Q>
  __device__ __forceinline__ void read(const Reads& r) {
    constexpr int F = Q / 2;
    constexpr bool IS_A = F == 0 || F >= 9;
    constexpr int IDX = F == 0 ? 0 : (F >= 9 ? F - 8 : F - 1);
    v6i& dst = IS_A ? fa[S][IDX] : fb[S][IDX];
    if constexpr (Q % 2 == 0) {
      v4i x;
      asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(x) : "v"(IS_A ? r.a16 : r.b16), "i"(IDX * F6_BLOCK));
      dst.s0 = x.x;
      dst.s1 = x.y;
      dst.s2 = x.z;
      dst.s3 = x.w;
    } else {
      v2i y;
      asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(y) : "v"(IS_A ? r.a8 : r.b8), "i"(IDX * F6_BLOCK));
      dst.s4 = y.x;
      dst.s5 = y.y;
    }
  }

  template <int S>
  __device__ __forceinline__ void mfma(int i, int j) {
    asm volatile("v_mfma_scale_f32_16x16x128_f8f6f4 %0, %1, %2, %0, %3, %3 op_sel_hi:[0,0,0] cbsz:3 blgp:3"
                 : "+a"(acc[i][j])
                 : "v"(fb[S][j]), "v"(fa[S][i]), "v"(one));
  }

  // MFMA T (0..63) of a stage on set S, followed by LDS read T of the next
  // stage (T < 32) or DMA load (T - 33) / 2 of the stage `dma_st` (odd T from
  // 33 on).
  template <int S, int T>
  __device__ __forceinline__ void tick(bool rd, const Reads& r, int dma_st, int dma_slot) {
    mfma<S>(T / 8, T % 8);
    if constexpr (T < 32) {
      if (rd) read<1 - S, T>(r);
    } else if constexpr (T % 2 == 1 && (T - 33) / 2 < DPW) {
      if (dma_st >= 0) dma(dma_st, dma_slot, (T - 33) / 2);
    }
  }
  template <int S, int... T>
  __device__ __forceinline__ void ticks(bool rd, const Reads& r, int dma_st, int dma_slot,
                                        std::integer_sequence<int, T...>) {
    (tick<S, T>(rd, r, dma_st, dma_slot), ...);
  }
  template <int S, int... Q>
  __device__ __forceinline__ void reads(const Reads& r, std::integer_sequence<int, Q...>) {
    (read<S, Q>(r), ...);
  }

  // Top of a stage: this wave's DMA of the next stage has landed (the
  // stage after it may stay outstanding), its LDS reads are done, then the
  // barrier.
  static __device__ __forceinline__ void open(bool one_pending) {
    if (one_pending) wait_vmcnt<DPW>();
    else wait_vmcnt<0>();
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  }

  // Stage k on set S: reads stage k+1 through `r` if `rd`, loads stage
  // `dma_st` (k + 3, or -1) into slot `dma_slot` (k's).
  template <int S>
  __device__ __forceinline__ void stage(bool one_pending, bool rd, const Reads& r, int dma_st, int dma_slot) {
    open(one_pending);
    ticks<S>(rd, r, dma_st, dma_slot, std::make_integer_sequence<int, 64>{});
  }

  __device__ __forceinline__ void run(int nst) {
    for (int s = 0; s < 3 && s < nst; ++s)
#pragma unroll
      for (int c = 0; c < DPW; ++c) dma(s, s, c);
    if (nst >= 3) wait_vmcnt<2 * DPW>();
    else if (nst == 2) wait_vmcnt<DPW>();
    else wait_vmcnt<0>();
    asm volatile("s_barrier" ::: "memory");
    reads<0>(reads_of_slot(0), std::make_integer_sequence<int, 32>{});
    acc_fence<4>(acc);
    // r: read slot of stage k+1; slot: slot of stage k
    Reads r = reads_of_slot(1);
    int slot = 0;
    const uint32_t step = (uint32_t)STAGE;
    auto advance = [&]() {
      r.add(slot == 1 ? (uint32_t)(-2 * (int)step) : step);
      slot = slot == 2 ? 0 : slot + 1;
    };
    int k = 0;
    for (; k + 4 < nst; k += 2) {
      stage<0>(true, true, r, k + 3, slot);
      advance();
      stage<1>(true, true, r, k + 4, slot);
      advance();
    }
    // at most four stages remain; stage k uses set 0
    while (k < nst) {
      stage<0>(k + 2 < nst, k + 1 < nst, r, k + 3 < nst ? k + 3 : -1, slot);
      advance();
      if (++k >= nst) break;
      stage<1>(k + 2 < nst, k + 1 < nst, r, k + 3 < nst ? k + 3 : -1, slot);
      advance();
      ++k;
    }
    // wait states between the last MFMA and the first accumulator read
    acc_fence<7>(acc);
    acc_fence<7>(acc);
  }
};

template <class C>
__global__ __launch_bounds__(256) void f6_gemm_kernel(const DenseArgs p) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[F6Engine<C>::LDS_BYTES];
  const int tiles_m = p.M / C::BM;
  const int tiles_n = p.N / C::BN;
  int tm, tn;
  dense_tile_coords(blockIdx.x, tiles_m, tiles_n, p.group_m, tm, tn);
  const int m0 = tm * C::BM;
  const int n0 = tn * C::BN;
  const int kb = p.K / 128;
  F6Engine<C> e;
  e.setup(smem, p.a, p.b, m0, tn, kb, f6_operand_bytes(p.M, p.K), f6_operand_bytes(p.b_cols, p.K));
  float sa[C::FM];
#pragma unroll
  for (int i = 0; i < C::FM; ++i) sa[i] = load_bf16(p.a_scale + m0 + e.out_row(i));
  float sb[C::FN2][4];
  const int gate = C::SWIGLU ? p.N : 0;
#pragma unroll
  for (int j = 0; j < C::FN2; ++j) {
    if (!C::SWIGLU && j >= C::FN) continue;
    load_bf16x4(p.b_scale + (j < C::FN ? 0 : gate) + n0 + e.out_col(j), 4, true, sb[j]);
  }
  e.run(kb);
  // The accumulator is the exact integer sum as an fp32 value.
  auto scaled = [&](int i, int j, int r) {
    float x = __int_as_float(e.acc[i][j][r]) * sa[i];
    return x * sb[j][r];
  };
  bool finite = true;
#pragma unroll
  for (int i = 0; i < C::FM; ++i) finite = finite && (__float_as_uint(sa[i]) & 0x7F800000u) != 0x7F800000u;
#pragma unroll
  for (int j = 0; j < C::FN; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) finite = finite && (__float_as_uint(sb[j][r]) & 0x7F800000u) != 0x7F800000u;
  const bool no_nan = __all(finite);
  auto raw_of = [&](int i, int j, int r) { return (int)__int_as_float(e.acc[i][j][r]); };
  if (C::SWIGLU) {
    dense_store<C>(e, p, m0, n0, [&](int i, int j, int r) { return swiglu(scaled(i, j, r), scaled(i, j + C::FN, r)); },
                   raw_of);
  } else if (p.epilogue == EPI_RELU2) {
    dense_store<C>(e, p, m0, n0, [&](int i, int j, int r) { return apply_epi(scaled(i, j, r), EPI_RELU2); }, raw_of,
                   no_nan);
  } else {
    dense_store<C>(e, p, m0, n0, scaled, raw_of, no_nan);
  }
}

}  // namespace shk
