// Dense GEMM kernel instantiations for one (operand width, layout) pair,
// selected at compile time with -DSHK_BITS={4,8} -DSHK_LAYOUT={0:NN,1:NT,2:TN}
// and -DSHK_DENSE_DMA={1: the large tiles on the direct-to-LDS engine,
// 0: the other tiles}.  The build compiles this file once per combination so
// the instantiations build in parallel; each object contributes its entries
// to the kernel table through append_dense_dma_<bits>_<layout>() or
// append_dense_<bits>_<layout>().
//
// The large tiles keep 256 int32 accumulators per lane in AGPRs.  With the
// default machine scheduler the register allocator rotates them between
// AGPRs through copies every K step; the build compiles the DMA objects with
// the iterative ILP scheduler, which keeps every accumulator in place.
#include "shk_table.h"

#ifndef SHK_BITS
#error "SHK_BITS must be defined"
#endif
#ifndef SHK_LAYOUT
#error "SHK_LAYOUT must be defined"
#endif
#ifndef SHK_DENSE_DMA
#error "SHK_DENSE_DMA must be defined"
#endif

namespace shk {
namespace {

constexpr int kBits = SHK_BITS;
constexpr int kLayout = SHK_LAYOUT;
constexpr bool kAKmajor = kLayout != SHK_LAYOUT_TN;  // NN/NT: A[M, K']
constexpr bool kBKmajor = kLayout == SHK_LAYOUT_NT;  // NT: B[N, K']

template <int BM, int BN, int BK, int WM, int WN, bool SWIGLU, bool SUBCH, int MK, int PIPE = 0>
using C = Cfg<kBits, kAKmajor, kBKmajor, BM, BN, BK, WM, WN, SWIGLU, SUBCH, MK, false, PIPE>;

// Table order inside one (bits, layout) block.  The large tiles come first:
// 256x256 per-channel (one wave per SIMD, 128x128 per wave) and the SwiGLU
// 256x128 output tile, which multiplies 256 B columns [up | gate].  Both run
// on the direct-to-LDS engine with a ring of 4 packed stages (64 source bytes
// per row each: 128 int4 / 64 int8 K values).  The remaining tiles run on
// the register-staged engine: 128x128 and 64x64 per-channel and SwiGLU tiles
// for smaller shapes, and the subchannel tiles, which keep an fp32 sum per
// accumulator in VGPRs and therefore run eight waves of 64x64 (two waves per
// SIMD: one wave's scale flush overlaps the other's MFMAs).  int8 stages are
// 64 deep so the prefetched stage and two fragment sets fit in registers.
constexpr int kBigBK = kBits == 4 ? 128 : 64;

#if SHK_DENSE_DMA
// int8 large tiles run on the 32x32 int8 engine (shk_i8.h), int4 ones on the
// direct-to-LDS engine with widening (the fp6 entries precede them).
void append_all(std::vector<Entry>& t) {
  if constexpr (kBits == 8) {
    t.push_back(i8_entry<C<256, 256, kBigBK, 2, 2, false, false, 64, 4>>(kLayout, 8));
    t.push_back(i8_entry<C<256, 128, kBigBK, 2, 2, true, false, 64, 4>>(kLayout, 8));
  } else {
    t.push_back(dense_entry<C<256, 256, kBigBK, 2, 2, false, false, 64, 4>>(kLayout, 8));
    t.push_back(dense_entry<C<256, 128, kBigBK, 2, 2, true, false, 64, 4>>(kLayout, 8));
  }
}
#else
void append_all(std::vector<Entry>& t) {
  t.push_back(dense_entry<C<128, 128, 64, 2, 2, false, false, 64>>(kLayout, 8));
  t.push_back(dense_entry<C<64, 64, 64, 2, 2, false, false, 64>>(kLayout, 8));
  t.push_back(dense_entry<C<64, 64, 64, 2, 2, true, false, 64>>(kLayout, 8));
  t.push_back(dense_entry<C<256, 128, kBigBK, 4, 2, false, true, 64>>(kLayout, 8));
  t.push_back(dense_entry<C<64, 64, 64, 2, 2, false, true, 64>>(kLayout, 8));
  t.push_back(dense_entry<C<256, 64, kBigBK, 4, 2, true, true, 64>>(kLayout, 8));
  t.push_back(dense_entry<C<64, 64, 64, 2, 2, true, true, 64>>(kLayout, 8));
  t.push_back(dense_entry<C<64, 64, 64, 2, 2, false, true, 32>>(kLayout, 8));
  t.push_back(dense_entry<C<64, 64, 64, 2, 2, true, true, 32>>(kLayout, 8));
}
#endif

#if !SHK_DENSE_DMA
// Persistent schedule: the 64 x 64 subchannel tiles for groups of 64 and up
// and of 32 (int4; the fp6 tiles serve per-channel and groups of 64 to 256).
void append_persistent(std::vector<Entry>& t) {
  if constexpr (kBits == 4) {
    t.push_back(dense_persistent_entry<C<64, 64, 64, 2, 2, false, true, 64>>(kLayout, 8));
    t.push_back(dense_persistent_entry<C<64, 64, 64, 2, 2, false, true, 32>>(kLayout, 8));
  }
}

// Split-K: the 128x128 per-channel tile and the 64x64 subchannel tiles, in
// 2, 4 and 8 K slices.
void append_split(std::vector<Entry>& t) {
  for (int split : {2, 4, 8}) t.push_back(split_entry<C<128, 128, 64, 2, 2, false, false, 64>>(kLayout, 8, split));
  if constexpr (kBits == 4) {
    for (int split : {2, 4, 8}) t.push_back(split_entry<C<64, 64, 64, 2, 2, false, true, 64>>(kLayout, 8, split));
    for (int split : {2, 4, 8}) t.push_back(split_entry<C<64, 64, 64, 2, 2, false, true, 32>>(kLayout, 8, split));
  }
}
#endif

}  // namespace

#define SHK_CAT3(a, b, c) a##b##_##c
#if !SHK_DENSE_DMA
#define SHK_PERSISTENT_NAME(b, l) SHK_CAT3(append_persistent_, b, l)
void SHK_PERSISTENT_NAME(SHK_BITS, SHK_LAYOUT)(std::vector<Entry>& t) { append_persistent(t); }
#define SHK_SPLIT_NAME(b, l) SHK_CAT3(append_split_, b, l)
void SHK_SPLIT_NAME(SHK_BITS, SHK_LAYOUT)(std::vector<Entry>& t) { append_split(t); }
#endif
#if SHK_DENSE_DMA
#define SHK_APPEND_NAME(b, l) SHK_CAT3(append_dense_dma_, b, l)
#else
#define SHK_APPEND_NAME(b, l) SHK_CAT3(append_dense_, b, l)
#endif
void SHK_APPEND_NAME(SHK_BITS, SHK_LAYOUT)(std::vector<Entry>& t) { append_all(t); }

}  // namespace shk
