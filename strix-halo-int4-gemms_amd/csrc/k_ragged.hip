// Ragged forward / backward kernel instantiations for one layout
// (-DSHK_LAYOUT={0:NN,1:NT,2:TN,3:TT}); the file also holds, in the NN build
// only, the device task-list builder (calculate_group_info) and the split-K
// finalize pass of the backward.
#include "shk_table.h"

#ifndef SHK_LAYOUT
#error "SHK_LAYOUT must be defined"
#endif

namespace shk {
namespace {

constexpr int kLayout = SHK_LAYOUT;
// Ragged operands are always packed int4 (ragged.py:1045-1050).
constexpr bool kAKmajor = kLayout == SHK_LAYOUT_NN || kLayout == SHK_LAYOUT_NT;
constexpr bool kBKmajor = kLayout == SHK_LAYOUT_NT || kLayout == SHK_LAYOUT_TT;

template <int BM, int BN, int BK, int WM, int WN, bool SUBCH, int MK>
using C = Cfg<4, kAKmajor, kBKmajor, BM, BN, BK, WM, WN, false, SUBCH, MK>;

template <bool SUBCH, int MK>
void append_fwd(std::vector<Entry>& t) {
  t.push_back(fwd_entry<C<16, 128, 128, 1, 4, SUBCH, MK>>(kLayout));
  t.push_back(fwd_entry<C<32, 128, 128, 2, 2, SUBCH, MK>>(kLayout));
  t.push_back(fwd_entry<C<64, 128, 128, 2, 2, SUBCH, MK>>(kLayout));
  t.push_back(fwd_entry<C<128, 128, 128, 2, 2, SUBCH, MK>>(kLayout));
}

// The fp6 entries (k_f6ragged.hip) lead each family.
void append_all(std::vector<Entry>& t) {
  t.push_back(f6_ragged_fwd_entry(kLayout));
  t.push_back(f6_ragged_sub_fwd_entry(kLayout));
  append_fwd<false, 64>(t);
  append_fwd<true, 64>(t);
  append_fwd<true, 32>(t);
  t.push_back(f6_ragged_bwd_entry(kLayout));
  t.push_back(f6_ragged_sub_bwd_entry(kLayout));
  t.push_back(bwd_entry<C<128, 128, 128, 2, 2, false, 64>>(kLayout));
  t.push_back(bwd_entry<C<128, 128, 128, 2, 2, true, 64>>(kLayout));
  t.push_back(bwd_entry<C<128, 128, 128, 2, 2, true, 32>>(kLayout));
}

}  // namespace

#define SHK_CAT2(a, b) a##b
#define SHK_APPEND_NAME(l) SHK_CAT2(append_ragged_, l)
void SHK_APPEND_NAME(SHK_LAYOUT)(std::vector<Entry>& t) { append_all(t); }

#if SHK_LAYOUT == 0

// ---------------------------------------------------------------------------
// Task list (calculate_group_info, ragged.py:201-323): one workgroup of
// kInfoThreads threads runs build_task_list (shk_tasks.h).

constexpr int kInfoThreads = 1024;
constexpr int kMaxInfoGroups = 16384;

__global__ __launch_bounds__(kInfoThreads) void group_info_kernel(const TaskJob job) {
  __shared__ int starts[kMaxInfoGroups + 1];       // first row of each group
  __shared__ int task_starts[kMaxInfoGroups + 1];  // first task of each group
  __shared__ int scratch[kInfoThreads / 64];
  build_task_list<kInfoThreads>(job, starts, task_starts, scratch);
}

// out[g, m, n] (int32 bits of the exact split-K sum) -> (float(sum) * a_scale[g, m]) * b_scale[g, n].
__global__ __launch_bounds__(256) void bwd_finalize_kernel(float* out, const uint16_t* a_scale,
                                                           const uint16_t* b_scale, int groups, int m,
                                                           int n) {
  const long total = (long)groups * m * n;
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < total; i += (long)gridDim.x * 256) {
    const long g = i / ((long)m * n);
    const long rem = i - g * m * n;
    const int row = (int)(rem / n);
    const int col = (int)(rem - (long)row * n);
    const int acc = __float_as_int(out[i]);
    float x = (float)acc * load_bf16(a_scale + g * m + row);
    x = x * load_bf16(b_scale + g * n + col);
    out[i] = x;
  }
}

}  // namespace shk

namespace shk {

hipError_t launch_group_info(const int32_t* sizes, int groups, int tile, int align, int capacity,
                             int32_t* tasks, int32_t* num_tasks, int64_t* info, hipStream_t s) {
  const TaskJob job{sizes, groups, tile, align, capacity, tasks, num_tasks, info};
  hipLaunchKernelGGL(group_info_kernel, dim3(1), dim3(kInfoThreads), 0, s, job);
  return hipGetLastError();
}

hipError_t launch_bwd_finalize(float* out, const uint16_t* a_scale, const uint16_t* b_scale, int groups,
                               int m, int n, hipStream_t s) {
  const long total = (long)groups * m * n;
  long blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(bwd_finalize_kernel, dim3((unsigned)blocks), dim3(256), 0, s, out, a_scale, b_scale,
                     groups, m, n);
  return hipGetLastError();
}

int max_info_groups() { return kMaxInfoGroups; }

#endif  // SHK_LAYOUT == 0

}  // namespace shk
