// Fake quantization and int4 packing on the device (the step before the
// GEMM): the reference's quant.py:14-51 (fake_quant_int, pack_int4_k_major)
// in one pass over HBM instead of a chain of torch element-wise kernels.
//
// A thread writes one 8-byte group of an output row:
//  * CODES: 8 int8 codes of 8 consecutive values of one row;
//  * PACK_COLS: 8 packed bytes of 16 consecutive values of one row;
//  * PACK_ROWS: 8 packed bytes of the same 8 columns of rows 2r and 2r+1.
// Values come in 16-byte loads (8-byte for 8 int8 codes) when the thread's
// values lie inside the row and are so aligned, element by element otherwise; values past the
// row or column count read as 0, whose code is 0 (the zero padding of an odd
// count).  Bytes past the output row are not written.  Bound: HBM, with
// bytes = the source plus the output, each touched once.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../include/strix_halo_gfx950.h"
#include "shk_quant.h"

namespace shk {
namespace {

__device__ __forceinline__ float src_value(const void* x, long i, int src) {
  if (src == SHK_SRC_F32) return static_cast<const float*>(x)[i];
  const uint16_t h = static_cast<const uint16_t*>(x)[i];
  if (src == SHK_SRC_BF16) return __uint_as_float((uint32_t)h << 16);
  return (float)__builtin_bit_cast(_Float16, h);
}

// The code of one value: torch.clamp(torch.round(v * inv), lo, hi).to(int8)
// as torch evaluates it on the GPU (round half to even; NaN converts to 0).
__device__ __forceinline__ int quant_code(float v, float inv, float lo, float hi) {
  const float q = __builtin_rintf(v * inv);
  return q == q ? (int)__builtin_fminf(__builtin_fmaxf(q, lo), hi) : 0;
}

// Codes of the N values of row `r` starting at column `c` (columns at or
// past `cols`, and rows at or past `rows`, give 0).
template <int SRC, int N>
__device__ __forceinline__ void row_codes(const QuantArgs& p, long r, long c, int (&code)[N]) {
  const float lo = -(float)(1 << (p.bits - 1)), hi = (float)((1 << (p.bits - 1)) - 1);
  if (r >= p.rows) {
#pragma unroll
    for (int t = 0; t < N; ++t) code[t] = 0;
    return;
  }
  constexpr int ESZ = SRC == SHK_SRC_F32 ? 4 : (SRC == SHK_SRC_I8 ? 1 : 2);
  const uint8_t* base = static_cast<const uint8_t*>(p.x) + (r * p.ld_x + c) * ESZ;
  // whole-row pieces of 16 bytes (or 8 when the values span 8)
  constexpr int PIECE = N * ESZ >= 16 ? 16 : 8;
  static_assert((N * ESZ) % PIECE == 0, "values fill whole pieces");
  if (c + N <= p.cols && (reinterpret_cast<uintptr_t>(base) & (PIECE - 1)) == 0) {
    uint32_t u[N * ESZ / 4];
#pragma unroll
    for (int i = 0; i < N * ESZ / PIECE; ++i) {
      if constexpr (PIECE == 16) {
        const uint4 w = reinterpret_cast<const uint4*>(base)[i];
        u[4 * i] = w.x, u[4 * i + 1] = w.y, u[4 * i + 2] = w.z, u[4 * i + 3] = w.w;
      } else {
        const uint2 w = reinterpret_cast<const uint2*>(base)[i];
        u[2 * i] = w.x, u[2 * i + 1] = w.y;
      }
    }
#pragma unroll
    for (int t = 0; t < N; ++t) {
      if constexpr (SRC == SHK_SRC_I8) {
        code[t] = (int)((u[t / 4] >> (8 * (t % 4))) & 0xFFu);
      } else {
        float v;
        if constexpr (SRC == SHK_SRC_F32) v = __uint_as_float(u[t]);
        else if constexpr (SRC == SHK_SRC_BF16) v = __uint_as_float((t % 2 ? u[t / 2] >> 16 : u[t / 2]) << 16);
        else v = (float)__builtin_bit_cast(_Float16, (uint16_t)(t % 2 ? u[t / 2] >> 16 : u[t / 2]));
        code[t] = quant_code(v, p.inv, lo, hi);
      }
    }
    return;
  }
#pragma unroll
  for (int t = 0; t < N; ++t) {
    if (c + t >= p.cols) {
      code[t] = 0;
    } else if constexpr (SRC == SHK_SRC_I8) {
      code[t] = (int)static_cast<const uint8_t*>(p.x)[r * p.ld_x + c + t];
    } else {
      code[t] = quant_code(src_value(p.x, r * p.ld_x + c + t, SRC), p.inv, lo, hi);
    }
  }
}

template <int SRC, int MODE>
__global__ __launch_bounds__(256) void quant_kernel(const QuantArgs p) {
  const long groups_per_row = (p.out_cols + 7) / 8;
  const long g = (long)blockIdx.x * 256 + threadIdx.x;
  if (g >= p.out_rows * groups_per_row) return;
  const long r = g / groups_per_row;
  const long ob = (g - r * groups_per_row) * 8;  // first output byte of the group
  uint32_t lo = 0, hi = 0;
  if constexpr (MODE == SHK_QUANT_CODES) {
    int code[8];
    row_codes<SRC, 8>(p, r, ob, code);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      lo |= ((uint32_t)code[t] & 0xFFu) << (8 * t);
      hi |= ((uint32_t)code[t + 4] & 0xFFu) << (8 * t);
    }
  } else if constexpr (MODE == SHK_QUANT_PACK_COLS) {
    int code[16];
    row_codes<SRC, 16>(p, r, 2 * ob, code);
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const uint32_t b = ((uint32_t)code[2 * t] & 0xFu) | (((uint32_t)code[2 * t + 1] & 0xFu) << 4);
      if (t < 4) lo |= b << (8 * t);
      else hi |= b << (8 * (t - 4));
    }
  } else {
    int even[8], odd[8];
    row_codes<SRC, 8>(p, 2 * r, ob, even);
    row_codes<SRC, 8>(p, 2 * r + 1, ob, odd);
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const uint32_t b = ((uint32_t)even[t] & 0xFu) | (((uint32_t)odd[t] & 0xFu) << 4);
      if (t < 4) lo |= b << (8 * t);
      else hi |= b << (8 * (t - 4));
    }
  }
  uint8_t* dst = p.out + r * p.ld_out + ob;
  if (ob + 8 <= p.out_cols && (reinterpret_cast<uintptr_t>(dst) & 7) == 0) {
    *reinterpret_cast<uint2*>(dst) = make_uint2(lo, hi);
  } else {
#pragma unroll
    for (int t = 0; t < 8; ++t)
      if (ob + t < p.out_cols) dst[t] = (uint8_t)((t < 4 ? lo >> (8 * t) : hi >> (8 * (t - 4))) & 0xFFu);
  }
}

template <int SRC>
hipError_t launch_src(const QuantArgs& p, dim3 grid, hipStream_t s) {
  if (p.mode == SHK_QUANT_CODES) hipLaunchKernelGGL((quant_kernel<SRC, SHK_QUANT_CODES>), grid, dim3(256), 0, s, p);
  else if (p.mode == SHK_QUANT_PACK_COLS)
    hipLaunchKernelGGL((quant_kernel<SRC, SHK_QUANT_PACK_COLS>), grid, dim3(256), 0, s, p);
  else hipLaunchKernelGGL((quant_kernel<SRC, SHK_QUANT_PACK_ROWS>), grid, dim3(256), 0, s, p);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_quantize(const QuantArgs& p, hipStream_t s) {
  const long groups = p.out_rows * ((p.out_cols + 7) / 8);
  if (groups <= 0) return hipSuccess;
  const long blocks = (groups + 255) / 256;
  if (blocks > 0x7FFFFFFFL) return hipErrorInvalidValue;
  const dim3 grid((unsigned)blocks);
  switch (p.src) {
    case SHK_SRC_F32: return launch_src<SHK_SRC_F32>(p, grid, s);
    case SHK_SRC_F16: return launch_src<SHK_SRC_F16>(p, grid, s);
    case SHK_SRC_BF16: return launch_src<SHK_SRC_BF16>(p, grid, s);
    default: return launch_src<SHK_SRC_I8>(p, grid, s);
  }
}

}  // namespace shk
