// Dense GEMM kernel instantiations for one (operand width, layout) pair,
// selected at compile time with -DSHK_BITS={4,8} -DSHK_LAYOUT={0:NN,1:NT,2:TN}.
// The build compiles this file once per pair so the instantiations build in
// parallel; each object contributes its entries to the kernel table through
// append_dense_<bits>_<layout>().
#include "shk_table.h"

#ifndef SHK_BITS
#error "SHK_BITS must be defined"
#endif
#ifndef SHK_LAYOUT
#error "SHK_LAYOUT must be defined"
#endif

namespace shk {
namespace {

constexpr int kBits = SHK_BITS;
constexpr int kLayout = SHK_LAYOUT;
constexpr bool kAKmajor = kLayout != SHK_LAYOUT_TN;  // NN/NT: A[M, K']
constexpr bool kBKmajor = kLayout == SHK_LAYOUT_NT;  // NT: B[N, K']

template <int BM, int BN, int BK, int WM, int WN, bool SWIGLU, bool SUBCH, int MK>
using C = Cfg<kBits, kAKmajor, kBKmajor, BM, BN, BK, WM, WN, SWIGLU, SUBCH, MK, false>;

// Table order inside one (bits, layout) block.  Per-channel plain tiles:
// 256x256 is the large-shape tile (one wave per SIMD, 128x128 per wave);
// 128x128 and 64x64 serve smaller shapes.  SwiGLU tiles stage [up | gate]
// B rows, so a 256x128 output tile multiplies 256 B columns.  Subchannel tiles
// keep an fp32 sum per accumulator in VGPRs, so they run eight waves of 64x64
// (two waves per SIMD: one wave's scale flush overlaps the other's MFMAs).
// int8 stages are 64 deep so the prefetched stage and two fragment sets fit
// in registers.
constexpr int kBigBK = kBits == 4 ? 128 : 64;

void append_all(std::vector<Entry>& t) {
  t.push_back(dense_entry<C<256, 256, kBigBK, 2, 2, false, false, 64>>(kLayout, 8));
  t.push_back(dense_entry<C<128, 128, 64, 2, 2, false, false, 64>>(kLayout, 8));
  t.push_back(dense_entry<C<64, 64, 64, 2, 2, false, false, 64>>(kLayout, 8));
  t.push_back(dense_entry<C<256, 128, kBigBK, 2, 2, true, false, 64>>(kLayout, 8));
  t.push_back(dense_entry<C<64, 64, 64, 2, 2, true, false, 64>>(kLayout, 8));
  t.push_back(dense_entry<C<256, 128, kBigBK, 4, 2, false, true, 64>>(kLayout, 8));
  t.push_back(dense_entry<C<64, 64, 64, 2, 2, false, true, 64>>(kLayout, 8));
  t.push_back(dense_entry<C<256, 64, kBigBK, 4, 2, true, true, 64>>(kLayout, 8));
  t.push_back(dense_entry<C<64, 64, 64, 2, 2, true, true, 64>>(kLayout, 8));
  t.push_back(dense_entry<C<64, 64, 64, 2, 2, false, true, 32>>(kLayout, 8));
  t.push_back(dense_entry<C<64, 64, 64, 2, 2, true, true, 32>>(kLayout, 8));
}

}  // namespace

#define SHK_CAT3(a, b, c) a##b##_##c
#define SHK_APPEND_NAME(b, l) SHK_CAT3(append_dense_, b, l)
void SHK_APPEND_NAME(SHK_BITS, SHK_LAYOUT)(std::vector<Entry>& t) { append_all(t); }

}  // namespace shk
