// Skinny dense kernel instantiations (shk_skinny.h) for one (operand width,
// layout) pair, selected with -DSHK_BITS={4,8} -DSHK_LAYOUT={0:NN,1:NT,2:TN};
// the build compiles this file once per pair and each object appends its
// table entries through append_skinny_<bits>_<layout>().
//
// The entries give every dense family the reference registers with small
// tiles (block_m 16 and 32, registry.py:29, 48-77) a gfx950 counterpart with
// block_m 16, 32 and 64 and block_k 32 (the reference's int4 per-channel and
// SwiGLU tiles take K in multiples of 32, registry.py:112-176): per-channel
// and subchannel, plain and SwiGLU, for int4 the persistent schedule
// (registry.py:230-251, split-K variants included), and split-K 2/4/8
// (SUPPORTED_SPLIT_K).
#include "shk_skinny.h"
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

template <int R, bool SWIGLU, bool SUBCH>
using SC = SkCfg<kBits, kLayout, R, SWIGLU, SUBCH>;

// grid.x = output tiles; per-channel tiles run sk_splits workgroups each.
template <class C>
unsigned sk_units(const DenseArgs& a, dim3 grid) {
  return grid.x * (unsigned)(C::SUBCH ? 1 : (a.sk_splits > 0 ? a.sk_splits : 1));
}
template <class C>
hipError_t launch_sk_t(const DenseArgs& a, dim3 grid, hipStream_t s) {
  hipLaunchKernelGGL(sk_gemm_kernel<C>, dim3(sk_units<C>(a, grid)), dim3(C::NT), 0, s, a);
  return hipGetLastError();
}
template <class C>
hipError_t launch_sk_persistent_t(const DenseArgs& a, dim3 grid, hipStream_t s) {
  return launch_persistent<&sk_gemm_kernel<C>>(a, sk_units<C>(a, grid), C::NT, s);
}

template <class C>
Entry sk_entry(int schedule, int split) {
  shk_kernel_desc d{};
  d.index = -1;
  d.family = SHK_FAMILY_DENSE;
  d.dtype_bits = kBits;
  d.layout = kLayout;
  d.scale_mode = C::SUBCH ? SHK_SCALE_SUBCHANNEL : SHK_SCALE_PER_CHANNEL;
  d.min_subchannel = C::SUBCH ? 32 : 0;
  d.max_subchannel = C::SUBCH ? 256 : 0;
  d.epilogue_kind = C::SWIGLU ? SHK_EPI_KIND_SWIGLU : SHK_EPI_KIND_PLAIN;
  d.block_m = C::R;
  d.block_n = C::BN;
  d.block_k = 32;
  d.num_waves = C::NW;
  d.num_stages = C::D;
  d.lds_bytes = C::LDS_BYTES;
  d.group_size_m = 1;
  d.operand_format = SHK_OPERANDS_STREAM;
  d.schedule = schedule;
  d.split_k = split;
  return Entry{d, schedule == SHK_SCHEDULE_PERSISTENT ? &launch_sk_persistent_t<C> : &launch_sk_t<C>, nullptr,
               nullptr, nullptr};
}

template <int R>
void append_tiles(std::vector<Entry>& t) {
  t.push_back(sk_entry<SC<R, false, false>>(SHK_SCHEDULE_STANDARD, 1));
  t.push_back(sk_entry<SC<R, true, false>>(SHK_SCHEDULE_STANDARD, 1));
  t.push_back(sk_entry<SC<R, false, true>>(SHK_SCHEDULE_STANDARD, 1));
  t.push_back(sk_entry<SC<R, true, true>>(SHK_SCHEDULE_STANDARD, 1));
}

void append_all(std::vector<Entry>& t) {
  append_tiles<16>(t);
  append_tiles<32>(t);
  append_tiles<64>(t);
  if constexpr (kBits == 4) {
    // the reference's persistent int4 tiles are its NONE tiles, split-K
    // variants included (registry.py:230-251)
    for (int split : {1, 2, 4, 8}) {
      t.push_back(sk_entry<SC<16, false, false>>(SHK_SCHEDULE_PERSISTENT, split));
      t.push_back(sk_entry<SC<16, false, true>>(SHK_SCHEDULE_PERSISTENT, split));
      t.push_back(sk_entry<SC<32, false, false>>(SHK_SCHEDULE_PERSISTENT, split));
      t.push_back(sk_entry<SC<32, false, true>>(SHK_SCHEDULE_PERSISTENT, split));
      t.push_back(sk_entry<SC<64, false, false>>(SHK_SCHEDULE_PERSISTENT, split));
      t.push_back(sk_entry<SC<64, false, true>>(SHK_SCHEDULE_PERSISTENT, split));
    }
  }
  for (int split : {2, 4, 8}) {
    t.push_back(sk_entry<SC<16, false, false>>(SHK_SCHEDULE_STANDARD, split));
    t.push_back(sk_entry<SC<16, false, true>>(SHK_SCHEDULE_STANDARD, split));
    t.push_back(sk_entry<SC<32, false, false>>(SHK_SCHEDULE_STANDARD, split));
    t.push_back(sk_entry<SC<32, false, true>>(SHK_SCHEDULE_STANDARD, split));
    t.push_back(sk_entry<SC<64, false, false>>(SHK_SCHEDULE_STANDARD, split));
    t.push_back(sk_entry<SC<64, false, true>>(SHK_SCHEDULE_STANDARD, split));
  }
}

}  // namespace

#define SHK_CAT3(a, b, c) a##b##_##c
#define SHK_APPEND_NAME(b, l) SHK_CAT3(append_skinny_, b, l)
void SHK_APPEND_NAME(SHK_BITS, SHK_LAYOUT)(std::vector<Entry>& t) { append_all(t); }

}  // namespace shk
