// GEMM kernels of the fp6 path: the 256x256 per-channel tile and the
// 256x128 SwiGLU tile (shk_f6.h), and the 128x128 subchannel tile
// (shk_f6sub.h).  They read operands already converted to the block format,
// so one instantiation serves every layout; the table holds one entry per
// layout (NN, NT, TN), which differ in how the operands are converted.
// Compiled with the iterative ILP scheduler, which keeps the accumulators in
// place (k_dense.hip).
#include "shk_f6sub.h"
#include "shk_table.h"

namespace shk {
namespace {

template <int BN, bool SWIGLU>
using C = Cfg<4, true, true, 256, BN, 128, 2, 2, SWIGLU, false, 64, false, 0>;
using CSub = Cfg<4, true, true, 128, 128, 128, 2, 2, false, true, 64, false, 0>;

// Subchannel GEMM on converted operands: one kernel per output mode,
// epilogue and group size (S = 128 or 256: 2 or 4 stages per group).
template <int MODE, int EPI>
void launch_sub(const DenseArgs& g, dim3 grid, hipStream_t s) {
  if (g.subchannel == 128) hipLaunchKernelGGL((f6_sub_kernel<CSub, MODE, EPI, 2>), grid, dim3(256), 0, s, g);
  else hipLaunchKernelGGL((f6_sub_kernel<CSub, MODE, EPI, 4>), grid, dim3(256), 0, s, g);
}
hipError_t launch_f6sub_gemm(const DenseArgs& a, dim3 grid, hipStream_t s) {
  DenseArgs g = a;
  g.a = a.work;
  g.b = a.work + f6_operand_bytes(a.M, a.K);
  const bool relu2 = a.epilogue == EPI_RELU2;
  if (a.out_mode == OUT_I32) launch_sub<OUT_I32, EPI_NONE>(g, grid, s);
  else if (a.out_mode == OUT_F32) relu2 ? launch_sub<OUT_F32, EPI_RELU2>(g, grid, s) : launch_sub<OUT_F32, EPI_NONE>(g, grid, s);
  else relu2 ? launch_sub<OUT_BF16, EPI_RELU2>(g, grid, s) : launch_sub<OUT_BF16, EPI_NONE>(g, grid, s);
  return hipGetLastError();
}
hipError_t launch_f6sub(const DenseArgs& a, dim3 grid, hipStream_t s) {
  hipError_t err = launch_f6_pack2(f6_pack_args(a, 0, false), f6_mn_major(a, 0), f6_pack_args(a, 1, false),
                                   f6_mn_major(a, 1), s);
  if (err == hipSuccess) err = launch_f6sub_gemm(a, grid, s);
  return err;
}
template <int MODE, int EPI>
hipError_t launch_sub_persistent(const DenseArgs& g, unsigned tiles, hipStream_t s) {
  if (g.subchannel == 128) return launch_persistent<&f6_sub_persistent<CSub, MODE, EPI, 2>>(g, tiles, 256, s);
  return launch_persistent<&f6_sub_persistent<CSub, MODE, EPI, 4>>(g, tiles, 256, s);
}
hipError_t launch_f6sub_gemm_persistent(const DenseArgs& a, dim3 grid, hipStream_t s) {
  DenseArgs g = a;
  g.a = a.work;
  g.b = a.work + f6_operand_bytes(a.M, a.K);
  const bool relu2 = a.epilogue == EPI_RELU2;
  if (a.out_mode == OUT_I32) return launch_sub_persistent<OUT_I32, EPI_NONE>(g, grid.x, s);
  if (a.out_mode == OUT_F32)
    return relu2 ? launch_sub_persistent<OUT_F32, EPI_RELU2>(g, grid.x, s)
                 : launch_sub_persistent<OUT_F32, EPI_NONE>(g, grid.x, s);
  return relu2 ? launch_sub_persistent<OUT_BF16, EPI_RELU2>(g, grid.x, s)
               : launch_sub_persistent<OUT_BF16, EPI_NONE>(g, grid.x, s);
}
hipError_t launch_f6sub_persistent(const DenseArgs& a, dim3 grid, hipStream_t s) {
  hipError_t err = launch_f6_pack2(f6_pack_args(a, 0, false), f6_mn_major(a, 0), f6_pack_args(a, 1, false),
                                   f6_mn_major(a, 1), s);
  if (err == hipSuccess) err = launch_f6sub_gemm_persistent(a, grid, s);
  return err;
}
Entry f6sub_entry(int layout) {
  shk_kernel_desc d = desc_of<CSub>(SHK_FAMILY_DENSE, layout, 8);
  d.min_subchannel = 128;
  d.max_subchannel = 256;
  d.num_stages = F6SubEngine<CSub, 4>::P;
  d.lds_bytes = F6SubEngine<CSub, 4>::LDS_BYTES;
  d.operand_format = SHK_OPERANDS_FP6;
  return Entry{d, &launch_f6sub, nullptr, nullptr, &launch_f6sub_gemm};
}

}  // namespace

void append_dense_f6(std::vector<Entry>& t, int layout) {
  t.push_back(f6_entry<C<256, false>>(layout));
  t.push_back(f6_entry<C<128, true>>(layout));
  t.push_back(f6sub_entry(layout));
}

void append_persistent_f6(std::vector<Entry>& t, int layout) {
  t.push_back(f6_persistent_entry<C<256, false>>(layout));
  Entry sub = f6sub_entry(layout);
  sub.d.schedule = SHK_SCHEDULE_PERSISTENT;
  sub.dense = &launch_f6sub_persistent;
  sub.converted = &launch_f6sub_gemm_persistent;
  t.push_back(sub);
}

}  // namespace shk
