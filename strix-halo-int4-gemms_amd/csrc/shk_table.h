// Internal kernel-table plumbing shared by the kernel translation units and
// the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <vector>

#include "../../include/strix_halo_gfx950.h"
#include "shk_i8.h"

namespace shk {

using DenseLaunchFn = hipError_t (*)(const DenseArgs&, dim3, hipStream_t);
using RaggedFwdLaunchFn = hipError_t (*)(const RaggedFwdArgs&, dim3, hipStream_t);
using RaggedBwdLaunchFn = hipError_t (*)(const RaggedBwdArgs&, dim3, hipStream_t);

struct Entry {
  shk_kernel_desc d;
  DenseLaunchFn dense;
  RaggedFwdLaunchFn fwd;
  RaggedBwdLaunchFn bwd;
  DenseLaunchFn converted;  // fp6 entries: the GEMM alone, on converted operands
};

template <class C>
hipError_t launch_dense_t(const DenseArgs& a, dim3 grid, hipStream_t s) {
  hipLaunchKernelGGL(dense_gemm_kernel<C>, grid, dim3(C::NT), 0, s, a);
  return hipGetLastError();
}
// fp6 path.  f6_convert_operand converts A (operand 0) or B (operand 1) of
// a dense call into its part of the workspace (A first, then B); the GEMM
// then reads both parts.
inline F6PackArgs f6_pack_args(const DenseArgs& a, int operand, bool swiglu) {
  const int kb = a.K / 64;
  // dense operands are validated 16-byte aligned
  if (operand == 0) return F6PackArgs{a.a, a.work, a.lda, a.M, kb, 0, 1, 0, 0, nullptr, a.K, 16};
  return F6PackArgs{a.b,    a.work + f6_operand_bytes(a.M, a.K), a.ldb, a.b_cols, kb, swiglu ? a.N : 0, 1, 0, 0,
                    nullptr, a.K, 16};
}
inline bool f6_mn_major(const DenseArgs& a, int operand) {
  return operand == 0 ? a.layout == SHK_LAYOUT_TN : a.layout != SHK_LAYOUT_NT;
}
inline hipError_t f6_convert_operand(const DenseArgs& a, int operand, bool swiglu, hipStream_t s) {
  return launch_f6_pack(f6_pack_args(a, operand, swiglu), f6_mn_major(a, operand), s);
}
// Large-K per-channel fp6 calls (K > F6_MAX_K): the int32 sums of the K
// slices go to the workspace past both converted operands, [M, b_cols]
// int32, which f6_large_k_begin clears and f6_large_k_end turns into the
// output (scales and epilogue, or the raw sums) (k_f6.hip).
inline int32_t* f6_large_k_acc(const DenseArgs& a) {
  return reinterpret_cast<int32_t*>(a.work + f6_operand_bytes(a.M, a.K) + f6_operand_bytes(a.b_cols, a.K));
}
hipError_t f6_large_k_begin(const DenseArgs& a, hipStream_t s);
hipError_t f6_large_k_end(const DenseArgs& a, bool swiglu, hipStream_t s);

template <class C>
hipError_t launch_f6_gemm_t(const DenseArgs& a, dim3 grid, hipStream_t s) {
  DenseArgs g = a;
  g.a = a.work;
  g.b = a.work + f6_operand_bytes(a.M, a.K);
  if (a.K > F6_MAX_K) {
    hipError_t err = f6_large_k_begin(a, s);
    if (err != hipSuccess) return err;
    g.out = f6_large_k_acc(a);
    const unsigned slices = (unsigned)((a.K + F6_MAX_K - 1) / F6_MAX_K);
    hipLaunchKernelGGL((f6_gemm_kernel<C, OUT_I32_ADD, EPI_NONE>), dim3(grid.x, slices), dim3(256), 0, s, g);
    err = hipGetLastError();
    if (err != hipSuccess) return err;
    return f6_large_k_end(a, C::SWIGLU, s);
  }
  if (a.out_mode == OUT_I32) {
    hipLaunchKernelGGL((f6_gemm_kernel<C, OUT_I32, EPI_NONE>), grid, dim3(256), 0, s, g);
  } else if (a.out_mode == OUT_F32) {
    if (!C::SWIGLU && a.epilogue == EPI_RELU2)
      hipLaunchKernelGGL((f6_gemm_kernel<C, OUT_F32, EPI_RELU2>), grid, dim3(256), 0, s, g);
    else
      hipLaunchKernelGGL((f6_gemm_kernel<C, OUT_F32, EPI_NONE>), grid, dim3(256), 0, s, g);
  } else if (!C::SWIGLU && a.epilogue == EPI_RELU2) {
    hipLaunchKernelGGL((f6_gemm_kernel<C, OUT_BF16, EPI_RELU2>), grid, dim3(256), 0, s, g);
  } else {
    hipLaunchKernelGGL((f6_gemm_kernel<C, OUT_BF16, EPI_NONE>), grid, dim3(256), 0, s, g);
  }
  return hipGetLastError();
}
template <class C>
hipError_t launch_f6_t(const DenseArgs& a, dim3 grid, hipStream_t s) {
  hipError_t err = launch_f6_pack2(f6_pack_args(a, 0, C::SWIGLU), f6_mn_major(a, 0), f6_pack_args(a, 1, C::SWIGLU),
                                   f6_mn_major(a, 1), s, nullptr, true);
  if (err == hipSuccess) err = launch_f6_gemm_t<C>(a, grid, s);
  return err;
}
// Workgroups of a persistent launch of `kernel` with `block` threads: its
// resident slots on the current device (occupancy x CUs), rounded down to a
// multiple of 8 so that a workgroup keeps its XCD, and at most `tiles`
// (capi.hip).
hipError_t persistent_grid(const void* kernel, int block, unsigned tiles, unsigned* grid);
template <auto K>
hipError_t launch_persistent(const DenseArgs& g, unsigned tiles, int block, hipStream_t s) {
  unsigned n = 0;
  const hipError_t err = persistent_grid(reinterpret_cast<const void*>(K), block, tiles, &n);
  if (err != hipSuccess) return err;
  void* args[] = {const_cast<DenseArgs*>(&g)};
  return hipLaunchKernel(reinterpret_cast<const void*>(K), dim3(n), dim3(block), args, 0, s);
}
// fp6 GEMM on converted operands, persistent schedule (plain epilogues).
template <class C>
hipError_t launch_f6_gemm_persistent_t(const DenseArgs& a, dim3 grid, hipStream_t s) {
  static_assert(!C::SWIGLU, "persistent entries are plain");
  DenseArgs g = a;
  g.a = a.work;
  g.b = a.work + f6_operand_bytes(a.M, a.K);
  const bool relu2 = a.epilogue == EPI_RELU2;
  if (a.out_mode == OUT_I32) return launch_persistent<&f6_gemm_persistent<C, OUT_I32, EPI_NONE>>(g, grid.x, 256, s);
  if (a.out_mode == OUT_F32)
    return relu2 ? launch_persistent<&f6_gemm_persistent<C, OUT_F32, EPI_RELU2>>(g, grid.x, 256, s)
                 : launch_persistent<&f6_gemm_persistent<C, OUT_F32, EPI_NONE>>(g, grid.x, 256, s);
  return relu2 ? launch_persistent<&f6_gemm_persistent<C, OUT_BF16, EPI_RELU2>>(g, grid.x, 256, s)
               : launch_persistent<&f6_gemm_persistent<C, OUT_BF16, EPI_NONE>>(g, grid.x, 256, s);
}
template <class C>
hipError_t launch_f6_persistent_t(const DenseArgs& a, dim3 grid, hipStream_t s) {
  hipError_t err = launch_f6_pack2(f6_pack_args(a, 0, false), f6_mn_major(a, 0), f6_pack_args(a, 1, false),
                                   f6_mn_major(a, 1), s, nullptr, true);
  if (err == hipSuccess) err = launch_f6_gemm_persistent_t<C>(a, grid, s);
  return err;
}
template <class C>
hipError_t launch_dense_persistent_t(const DenseArgs& a, dim3 grid, hipStream_t s) {
  return launch_persistent<&dense_gemm_persistent<C>>(a, grid.x, C::NT, s);
}
// int8 32x32 engine: one kernel per output mode and epilogue.  A grid of
// 256-row tiles (K-major A) whose last round of workgroups would be partial
// runs the column tiles of that round as 128-row tiles, twice as many and
// half as long, when they fit one round (i8_gemm_kernel).
template <class C, int MODE, int EPI>
hipError_t launch_i8_k(const DenseArgs& a, dim3 grid, hipStream_t s) {
  auto* k = &i8_gemm_kernel<C, MODE, EPI>;
  DenseArgs g = a;
  g.split_tn = 0;
  if constexpr (C::BM == 256 && C::A_KMAJOR) {
    const long tiles_m = a.M / C::BM, tiles_n = a.N / C::BN;
    unsigned slots = 0;
    const hipError_t err = persistent_grid(reinterpret_cast<const void*>(k), 256, 0xFFFFFFFFu, &slots);
    if (err != hipSuccess) return err;
    const long tiles = tiles_m * tiles_n;
    const long rest = slots > 0 ? tiles % slots : 0;
    if (tiles > (long)slots && rest > 0) {
      const long c = (rest + tiles_m - 1) / tiles_m;  // trailing column tiles holding the partial round
      if (2 * tiles_m * c <= (long)slots && c < tiles_n) {
        g.split_tn = (int)(tiles_n - c);
        grid = dim3((unsigned)(tiles_m * (tiles_n - c) + 2 * tiles_m * c));
      }
    }
  }
  hipLaunchKernelGGL(k, grid, dim3(256), 0, s, g);
  return hipGetLastError();
}
template <class C>
hipError_t launch_i8_t(const DenseArgs& a, dim3 grid, hipStream_t s) {
  if (a.out_mode == OUT_I32) return launch_i8_k<C, OUT_I32, EPI_NONE>(a, grid, s);
  if (a.out_mode == OUT_F32) {
    if (!C::SWIGLU && a.epilogue == EPI_RELU2) return launch_i8_k<C, OUT_F32, EPI_RELU2>(a, grid, s);
    return launch_i8_k<C, OUT_F32, EPI_NONE>(a, grid, s);
  }
  if (!C::SWIGLU && a.epilogue == EPI_RELU2) return launch_i8_k<C, OUT_BF16, EPI_RELU2>(a, grid, s);
  return launch_i8_k<C, OUT_BF16, EPI_NONE>(a, grid, s);
}
template <class C>
hipError_t launch_fwd_t(const RaggedFwdArgs& a, dim3 grid, hipStream_t s) {
  hipLaunchKernelGGL(ragged_fwd_kernel<C>, grid, dim3(C::NT), 0, s, a);
  return hipGetLastError();
}
template <class C>
hipError_t launch_bwd_t(const RaggedBwdArgs& a, dim3 grid, hipStream_t s) {
  hipLaunchKernelGGL(ragged_bwd_kernel<C>, grid, dim3(C::NT), 0, s, a);
  return hipGetLastError();
}

template <class C>
constexpr shk_kernel_desc desc_of(int family, int layout, int group_m) {
  return shk_kernel_desc{
      -1,
      family,
      C::BITS,
      layout,
      C::SUBCH ? SHK_SCALE_SUBCHANNEL : SHK_SCALE_PER_CHANNEL,
      C::SUBCH ? (C::MK == 32 ? 32 : 64) : 0,
      C::SUBCH ? (C::MK == 32 ? 32 : 256) : 0,
      C::SWIGLU ? SHK_EPI_KIND_SWIGLU : SHK_EPI_KIND_PLAIN,
      C::BM,
      C::BN,
      C::BK,
      C::NT / 64,
      C::NUM_STAGES,
      C::LDS_BYTES,
      group_m,
      SHK_OPERANDS_PACKED,
      SHK_SCHEDULE_STANDARD,
      1,
  };
}

template <class C>
Entry dense_entry(int layout, int group_m) {
  return Entry{desc_of<C>(SHK_FAMILY_DENSE, layout, group_m), &launch_dense_t<C>, nullptr, nullptr, nullptr};
}
template <class C>
Entry i8_entry(int layout, int group_m) {
  static_assert(C::LDS_BYTES == I8Engine<C>::LDS_BYTES && C::NUM_STAGES == I8Engine<C>::P, "table geometry");
  shk_kernel_desc d = desc_of<C>(SHK_FAMILY_DENSE, layout, group_m);
  d.lds_bytes += MFMA32_SCALE_BYTES;
  return Entry{d, &launch_i8_t<C>, nullptr, nullptr, nullptr};
}
template <class C>
Entry f6_entry(int layout) {
  shk_kernel_desc d = desc_of<C>(SHK_FAMILY_DENSE, layout, 8);
  d.num_stages = F6Engine<C>::P;
  d.lds_bytes = F6Engine<C>::LDS_BYTES + MFMA32_SCALE_BYTES;
  d.operand_format = SHK_OPERANDS_FP6;
  return Entry{d, &launch_f6_t<C>, nullptr, nullptr, &launch_f6_gemm_t<C>};
}
// Persistent-schedule entries of the same kernels.
template <class C>
Entry f6_persistent_entry(int layout) {
  Entry e = f6_entry<C>(layout);
  e.d.schedule = SHK_SCHEDULE_PERSISTENT;
  e.dense = &launch_f6_persistent_t<C>;
  e.converted = &launch_f6_gemm_persistent_t<C>;
  return e;
}
template <class C>
Entry dense_persistent_entry(int layout, int group_m) {
  Entry e = dense_entry<C>(layout, group_m);
  e.d.schedule = SHK_SCHEDULE_PERSISTENT;
  e.dense = &launch_dense_persistent_t<C>;
  return e;
}
// Split-K entries of a dense tile: grid.y = split, each workgroup sums one
// K slice and adds its scaled fp32 partial into the zeroed output.
template <class C>
Entry split_entry(int layout, int group_m, int split) {
  Entry e = dense_entry<C>(layout, group_m);
  e.d.split_k = split;
  return e;
}
template <class C>
Entry fwd_entry(int layout) {
  return Entry{desc_of<C>(SHK_FAMILY_RAGGED_FWD, layout, 1), nullptr, &launch_fwd_t<C>, nullptr, nullptr};
}
template <class C>
Entry bwd_entry(int layout) {
  return Entry{desc_of<C>(SHK_FAMILY_RAGGED_BWD, layout, 1), nullptr, nullptr, &launch_bwd_t<C>, nullptr};
}

// Skinny entries (SHK_OPERANDS_STREAM, shk_skinny.h).  Workgroups that share
// a per-channel tile's K: enough to give about kSkTargetUnits workgroups (one
// per CU of an MI355X; at M = 16, N = K = 8192 two workgroups per tile run
// 8.8 us against 9.9 us for four, each K split adding a tail of device-scope
// round trips) while every wave keeps at least two stages, at most 16;
// and for int4 at least as many as keep each wave's x256 int32 sum within
// 1023 stages of 128 K (up to 64 at K = 2^24).  Without a workspace only
// one, or 0 when K needs more.  Subchannel tiles always use one.
constexpr int kSkTargetUnits = 256;
inline int sk_split_count(const shk_kernel_desc& d, long m, long n, long k, bool with_workspace) {
  if (d.scale_mode == SHK_SCALE_SUBCHANNEL) return 1;
  const long ks = d.dtype_bits == 4 ? 128 : 64;
  const long nst = (k + ks - 1) / ks;
  long need = 1;
  if (d.dtype_bits == 4)
    while (need * 4L * 1023L < nst) need *= 2;
  if (!with_workspace) return need == 1 ? 1 : 0;
  const long tiles = (m / d.block_m) * (n / d.block_n);
  long s = 1;
  while (s * 2 <= 16 && tiles * s * 2 <= kSkTargetUnits && nst >= 16L * s) s *= 2;
  return (int)(s > need ? s : need);
}
// Workspace of a skinny launch with more than one split: the tiles' arrival
// counters, padded to 256 bytes, then an exact int32 partial of every (tile,
// split).  All of it is zero before the first launch and every launch leaves
// what it used zero, whatever the shapes of the launches that share it.
inline unsigned long long sk_workspace_bytes(const shk_kernel_desc& d, long m, long n, long k) {
  const int s = sk_split_count(d, m, n, k, true);
  if (s <= 1) return 0;
  const long tiles = (m / d.block_m) * (n / d.block_n);
  const long cf = d.epilogue_kind == SHK_EPI_KIND_SWIGLU ? 2 : 1;
  // per (tile, split): (block_n / 16) output column tiles x (block_m / 16)
  // row tiles x (up, gate) x 1 KiB
  return (unsigned long long)((tiles * 4 + 255) & ~255L) +
         (unsigned long long)tiles * s * (d.block_n / 16) * (d.block_m / 16) * cf * 1024;
}
inline unsigned long long sk_counter_bytes(const shk_kernel_desc& d, long m, long n) {
  return (unsigned long long)((((m / d.block_m) * (n / d.block_n)) * 4 + 255) & ~255L);
}

// Each kernel translation unit appends its entries in a fixed order
// (append_dense_f6(layout), append_dense_dma_<bits>_<layout>,
// append_dense_<bits>_<layout>, append_ragged_<layout>).
void append_dense_f6(std::vector<Entry>& t, int layout);
void append_dense_dma_4_0(std::vector<Entry>& t);
void append_dense_dma_4_1(std::vector<Entry>& t);
void append_dense_dma_4_2(std::vector<Entry>& t);
void append_dense_dma_8_0(std::vector<Entry>& t);
void append_dense_dma_8_1(std::vector<Entry>& t);
void append_dense_dma_8_2(std::vector<Entry>& t);
void append_dense_4_0(std::vector<Entry>& t);
void append_dense_4_1(std::vector<Entry>& t);
void append_dense_4_2(std::vector<Entry>& t);
void append_dense_8_0(std::vector<Entry>& t);
void append_dense_8_1(std::vector<Entry>& t);
void append_dense_8_2(std::vector<Entry>& t);
// Persistent-schedule int4 entries (plain epilogue kind), appended after
// the ragged families: the fp6 per-channel and subchannel tiles
// (append_persistent_f6(layout)) and the register-staged 64 x 64
// subchannel tiles for groups of 64 and 32 (append_persistent_4_<layout>).
void append_persistent_f6(std::vector<Entry>& t, int layout);
void append_persistent_4_0(std::vector<Entry>& t);
void append_persistent_4_1(std::vector<Entry>& t);
void append_persistent_4_2(std::vector<Entry>& t);
// Split-K 2/4/8 entries of the 128x128 per-channel tile (int4, int8) and of
// the 64x64 subchannel tiles (int4), per layout (append_split_<bits>_<layout>).
void append_split_4_0(std::vector<Entry>& t);
void append_split_4_1(std::vector<Entry>& t);
void append_split_4_2(std::vector<Entry>& t);
void append_split_8_0(std::vector<Entry>& t);
void append_split_8_1(std::vector<Entry>& t);
void append_split_8_2(std::vector<Entry>& t);
// Skinny entries per (bits, layout) (k_skinny.hip): for block_m 16, 32, 64
// the per-channel and subchannel tiles, plain and SwiGLU; for int4 the
// persistent plain tiles, split-K 1/2/4/8; then split-K 2/4/8 plain tiles.
void append_skinny_4_0(std::vector<Entry>& t);
void append_skinny_4_1(std::vector<Entry>& t);
void append_skinny_4_2(std::vector<Entry>& t);
void append_skinny_8_0(std::vector<Entry>& t);
void append_skinny_8_1(std::vector<Entry>& t);
void append_skinny_8_2(std::vector<Entry>& t);
void append_ragged_0(std::vector<Entry>& t);
void append_ragged_1(std::vector<Entry>& t);
void append_ragged_2(std::vector<Entry>& t);
void append_ragged_3(std::vector<Entry>& t);
int max_info_groups();
// fp6 ragged entries of one layout (k_f6ragged.hip): the forward (task
// tile 128) and the K-ragged backward, each per-channel and subchannel.
Entry f6_ragged_fwd_entry(int layout);
Entry f6_ragged_sub_fwd_entry(int layout);
Entry f6_ragged_bwd_entry(int layout);
Entry f6_ragged_sub_bwd_entry(int layout);
// Workspace bytes of the fp6 ragged paths.
unsigned long long f6_ragged_fwd_workspace(int m, int n, int k, int groups, bool subchannel);
unsigned long long f6_ragged_bwd_workspace(int m, int n, int k_cap, int groups, bool subchannel);

// Non-table kernels (ragged.hip).
hipError_t launch_group_info(const int32_t* sizes, int groups, int tile, int align, int capacity,
                             int32_t* tasks, int32_t* num_tasks, int64_t* info, hipStream_t s);
hipError_t launch_bwd_finalize(float* out, const uint16_t* a_scale, const uint16_t* b_scale, int groups,
                               int m, int n, hipStream_t s);

}  // namespace shk
