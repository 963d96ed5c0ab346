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
// epilogue and group size (S = 32, 64, 128 or 256: S / 32 is the template's
// last argument).
template <int MODE, int EPI>
void launch_sub(const DenseArgs& g, dim3 grid, hipStream_t s) {
  if (g.subchannel == 32) hipLaunchKernelGGL((f6_sub_kernel<CSub, MODE, EPI, 1>), grid, dim3(256), 0, s, g);
  else if (g.subchannel == 64) hipLaunchKernelGGL((f6_sub_kernel<CSub, MODE, EPI, 2>), grid, dim3(256), 0, s, g);
  else if (g.subchannel == 128) hipLaunchKernelGGL((f6_sub_kernel<CSub, MODE, EPI, 4>), grid, dim3(256), 0, s, g);
  else hipLaunchKernelGGL((f6_sub_kernel<CSub, MODE, EPI, 8>), grid, dim3(256), 0, s, g);
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
  if (g.subchannel == 32) return launch_persistent<&f6_sub_persistent<CSub, MODE, EPI, 1>>(g, tiles, 256, s);
  if (g.subchannel == 64) return launch_persistent<&f6_sub_persistent<CSub, MODE, EPI, 2>>(g, tiles, 256, s);
  if (g.subchannel == 128) return launch_persistent<&f6_sub_persistent<CSub, MODE, EPI, 4>>(g, tiles, 256, s);
  return launch_persistent<&f6_sub_persistent<CSub, MODE, EPI, 8>>(g, tiles, 256, s);
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
  d.min_subchannel = 32;
  d.max_subchannel = 256;
  d.num_stages = F6SubEngine<CSub>::P;
  d.lds_bytes = f6_sub_lds_bytes<CSub>();
  d.operand_format = SHK_OPERANDS_FP6;
  return Entry{d, &launch_f6sub, nullptr, nullptr, &launch_f6sub_gemm};
}

// Large-K per-channel calls: clearing the int32 workspace, and the pass
// that turns the exact int32 sums into the output with the reference's op
// order, (float(acc) * a_scale) * b_scale, then ReLU^2 or
// up * (gate / (1 + exp(-gate))), then the bf16 cast (api.py:283-309).
// One thread per 4 consecutive output columns of a row.
__global__ __launch_bounds__(256) void zero_i32_kernel(int4* p, long n4) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i < n4) p[i] = make_int4(0, 0, 0, 0);
}

template <bool SWIGLU, int MODE, int EPI>
__global__ __launch_bounds__(256) void f6_finalize_kernel(const DenseArgs p, const int32_t* acc) {
  const int quads = p.N / 4;
  const long idx = (long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (long)p.M * quads) return;
  const int row = (int)(idx / quads);
  const int c = 4 * (int)(idx - (long)row * quads);
  const int4 up = *reinterpret_cast<const int4*>(acc + (long)row * p.b_cols + c);
  if constexpr (MODE == OUT_I32) {
    // the raw sums, laid out as the one-launch raw output ([M, 2N] for SwiGLU)
    int32_t* o = static_cast<int32_t*>(p.out) + (long)row * p.b_cols + c;
    *reinterpret_cast<int4*>(o) = up;
    if constexpr (SWIGLU) *reinterpret_cast<int4*>(o + p.N) = *reinterpret_cast<const int4*>(acc + (long)row * p.b_cols + p.N + c);
    return;
  } else {
    const int u[4] = {up.x, up.y, up.z, up.w};
    int gt[4] = {0, 0, 0, 0};
    if constexpr (SWIGLU) {
      const int4 g = *reinterpret_cast<const int4*>(acc + (long)row * p.b_cols + p.N + c);
      gt[0] = g.x, gt[1] = g.y, gt[2] = g.z, gt[3] = g.w;
    }
    const float sa = load_bf16(p.a_scale + row);
    float v[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      float x = (float)u[t] * sa;
      x = x * load_bf16(p.b_scale + c + t);
      if constexpr (SWIGLU) {
        float g = (float)gt[t] * sa;
        g = g * load_bf16(p.b_scale + p.N + c + t);
        x = swiglu(x, g);
      } else if constexpr (EPI == EPI_RELU2) {
        x = apply_epi(x, EPI_RELU2);
      }
      v[t] = x;
    }
    if constexpr (MODE == OUT_F32) {
      *reinterpret_cast<float4*>(static_cast<float*>(p.out) + (long)row * p.N + c) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
      const uint32_t lo = f32_to_bf16_rne(v[0]) | (f32_to_bf16_rne(v[1]) << 16);
      const uint32_t hi = f32_to_bf16_rne(v[2]) | (f32_to_bf16_rne(v[3]) << 16);
      *reinterpret_cast<uint2*>(static_cast<uint16_t*>(p.out) + (long)row * p.N + c) = make_uint2(lo, hi);
    }
  }
}

template <bool SWIGLU>
void launch_finalize(const DenseArgs& a, dim3 grid, hipStream_t s) {
  const int32_t* acc = f6_large_k_acc(a);
  if (a.out_mode == OUT_I32) hipLaunchKernelGGL((f6_finalize_kernel<SWIGLU, OUT_I32, EPI_NONE>), grid, dim3(256), 0, s, a, acc);
  else if (a.out_mode == OUT_F32 && !SWIGLU && a.epilogue == EPI_RELU2)
    hipLaunchKernelGGL((f6_finalize_kernel<SWIGLU, OUT_F32, EPI_RELU2>), grid, dim3(256), 0, s, a, acc);
  else if (a.out_mode == OUT_F32)
    hipLaunchKernelGGL((f6_finalize_kernel<SWIGLU, OUT_F32, EPI_NONE>), grid, dim3(256), 0, s, a, acc);
  else if (!SWIGLU && a.epilogue == EPI_RELU2)
    hipLaunchKernelGGL((f6_finalize_kernel<SWIGLU, OUT_BF16, EPI_RELU2>), grid, dim3(256), 0, s, a, acc);
  else
    hipLaunchKernelGGL((f6_finalize_kernel<SWIGLU, OUT_BF16, EPI_NONE>), grid, dim3(256), 0, s, a, acc);
}

}  // namespace

hipError_t f6_large_k_begin(const DenseArgs& a, hipStream_t s) {
  const long n4 = (long)a.M * a.b_cols / 4;  // b_cols is a multiple of 128
  const long blocks = (n4 + 255) / 256;
  if (blocks > 0x7FFFFFFFL) return hipErrorInvalidValue;
  hipLaunchKernelGGL(zero_i32_kernel, dim3((unsigned)blocks), dim3(256), 0, s, reinterpret_cast<int4*>(f6_large_k_acc(a)),
                     n4);
  return hipGetLastError();
}

hipError_t f6_large_k_end(const DenseArgs& a, bool swiglu, hipStream_t s) {
  const long threads = (long)a.M * (a.N / 4);
  const long blocks = (threads + 255) / 256;
  if (blocks > 0x7FFFFFFFL) return hipErrorInvalidValue;
  if (swiglu) launch_finalize<true>(a, dim3((unsigned)blocks), s);
  else launch_finalize<false>(a, dim3((unsigned)blocks), s);
  return hipGetLastError();
}

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
