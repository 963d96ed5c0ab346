// Dense GEMM kernel on the pipelined engine (tile-multiple shapes, aligned
// operands; both checked on the host).
#pragma once

#include "shk_dma.h"

namespace shk {

template <class C>
using DenseEngine = typename std::conditional<(C::PIPE > 0), DmaEngine<C>, FastEngine<C>>::type;

// Writes one tile's results.  `value(i, j, r)` gives the scaled, epilogue-
// applied fp32 value, `raw(i, j, r)` the int32 written in verification mode.
// `no_nan` (uniform across the wave) promises that no value is NaN, which
// allows the hardware bf16 conversion.
template <class C, class E, class Value, class Raw>
__device__ __forceinline__ void dense_store(const E& e, const DenseArgs& p, int m0, int n0, Value value, Raw raw,
                                            bool no_nan = false) {
  const bool swiglu_raw = C::SWIGLU && p.out_mode == OUT_I32;
  const long ldo = swiglu_raw ? 2L * p.N : (long)p.N;
  if (p.out_mode == OUT_I32) {
#pragma unroll
    for (int i = 0; i < C::FM; ++i)
#pragma unroll
      for (int j = 0; j < C::FN2; ++j) {
        if (!C::SWIGLU && j >= C::FN) continue;
        const long col = (j < C::FN ? 0 : p.N) + n0 + e.out_col(j);
        int* o = reinterpret_cast<int*>(p.out) + (long)(m0 + e.out_row(i)) * ldo + col;
        *reinterpret_cast<int4*>(o) = make_int4(raw(i, j, 0), raw(i, j, 1), raw(i, j, 2), raw(i, j, 3));
      }
    return;
  }
#pragma unroll
  for (int i = 0; i < C::FM; ++i)
#pragma unroll
    for (int j = 0; j < C::FN; ++j) {
      const long idx = (long)(m0 + e.out_row(i)) * p.N + n0 + e.out_col(j);
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = value(i, j, r);
      if (p.out_mode == OUT_BF16) {
        uint32_t lo, hi;
        if (no_nan) {
          lo = pack_bf16x2_nonan(v[0], v[1]);
          hi = pack_bf16x2_nonan(v[2], v[3]);
        } else {
          lo = f32_to_bf16_rne(v[0]) | (f32_to_bf16_rne(v[1]) << 16);
          hi = f32_to_bf16_rne(v[2]) | (f32_to_bf16_rne(v[3]) << 16);
        }
        *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(p.out) + idx) = make_uint2(lo, hi);
      } else {
        *reinterpret_cast<float4*>(reinterpret_cast<float*>(p.out) + idx) = make_float4(v[0], v[1], v[2], v[3]);
      }
      // one fragment at a time: keeps the accumulator reads from being
      // hoisted ahead of their use, which would need more VGPRs than exist
      __builtin_amdgcn_sched_barrier(0);
    }
}

template <class C>
__global__ __launch_bounds__(C::NT) void dense_gemm_kernel(const DenseArgs p) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[C::LDS_BYTES];
  const int tiles_m = p.M / C::BM;
  const int tiles_n = p.N / C::BN;
  int tm, tn;
  dense_tile_coords(blockIdx.x, tiles_m, tiles_n, p.group_m, tm, tn);
  const int m0 = tm * C::BM;
  const int n0 = tn * C::BN;
  const int gate = C::SWIGLU ? p.N : 0;

  DenseEngine<C> e;
  e.init_reads();
  e.setup(p, m0, n0, gate);
  const int nst = p.K / C::BK;
  const bool raw = p.out_mode == OUT_I32;

  if constexpr (C::SUBCH) {
    SubAcc<C> s;
    s.zero();
    const int S = p.subchannel;
    auto on_step = [&](int ke) {
      if (ke % S == 0) {
        const int g = ke / S - 1;
        float sa[C::FM];
        if (raw) {
#pragma unroll
          for (int i = 0; i < C::FM; ++i)
#pragma unroll
            for (int j = 0; j < C::FN2; ++j)
#pragma unroll
              for (int r = 0; r < 4; ++r)
                s.f[i][j][r] = __int_as_float(__float_as_int(s.f[i][j][r]) + e.true_acc(e.acc[i][j][r]));
        } else {
#pragma unroll
          for (int i = 0; i < C::FM; ++i)
            sa[i] = load_bf16(p.a_scale + (long)(m0 + e.out_row(i)) * p.scale_cols + g);
#pragma unroll
          for (int j = 0; j < C::FN2; ++j) {
            float sb[4];
            const int col = (j < C::FN ? 0 : gate) + n0 + e.out_col(j);
            load_bf16x4(p.b_scale + (long)g * p.b_cols + col, 4, true, sb);
#pragma unroll
            for (int i = 0; i < C::FM; ++i)
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                float t = (float)e.acc[i][j][r] * sa[i];
                t = t * sb[r];
                s.f[i][j][r] = s.f[i][j][r] + t;
              }
          }
        }
        e.zero_acc();
      }
    };
    e.run(smem, nst, on_step);
    auto raw_of = [&](int i, int j, int r) { return __float_as_int(s.f[i][j][r]); };
    if (C::SWIGLU) {
      dense_store<C>(e, p, m0, n0, [&](int i, int j, int r) {
        return swiglu(s.f[i][j][r] * C::ACC_UNSCALE, s.f[i][j + C::FN][r] * C::ACC_UNSCALE);
      }, raw_of);
    } else if (p.epilogue == EPI_RELU2) {
      dense_store<C>(e, p, m0, n0, [&](int i, int j, int r) {
        return apply_epi(s.f[i][j][r] * C::ACC_UNSCALE, EPI_RELU2);
      }, raw_of);
    } else {
      dense_store<C>(e, p, m0, n0, [&](int i, int j, int r) { return s.f[i][j][r] * C::ACC_UNSCALE; }, raw_of);
    }
  } else {
    auto nop = [](int) {};
    e.run(smem, nst, nop);
    float sa[C::FM];
#pragma unroll
    for (int i = 0; i < C::FM; ++i) sa[i] = load_bf16(p.a_scale + m0 + e.out_row(i));
    float sb[C::FN2][4];
#pragma unroll
    for (int j = 0; j < C::FN2; ++j) {
      if (!C::SWIGLU && j >= C::FN) continue;
      load_bf16x4(p.b_scale + (j < C::FN ? 0 : gate) + n0 + e.out_col(j), 4, true, sb[j]);
    }
    // (float(acc) * a_scale) * b_scale on the true accumulator (the shift
    // removes the int4 widening factor exactly).
    auto scaled = [&](int i, int j, int r) {
      float x = (float)e.true_acc(e.acc[i][j][r]) * sa[i];
      return x * sb[j][r];
    };
    // Finite scales times a finite int32 sum give no NaN (at most +-inf),
    // and neither does ReLU^2 of such a value.
    bool finite = true;
#pragma unroll
    for (int i = 0; i < C::FM; ++i) finite = finite && (__float_as_uint(sa[i]) & 0x7F800000u) != 0x7F800000u;
#pragma unroll
    for (int j = 0; j < C::FN; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) finite = finite && (__float_as_uint(sb[j][r]) & 0x7F800000u) != 0x7F800000u;
    const bool no_nan = __all(finite);
    auto raw_of = [&](int i, int j, int r) { return e.true_acc(e.acc[i][j][r]); };
    if (C::SWIGLU) {
      dense_store<C>(e, p, m0, n0, [&](int i, int j, int r) {
        return swiglu(scaled(i, j, r), scaled(i, j + C::FN, r));
      }, raw_of);
    } else if (p.epilogue == EPI_RELU2) {
      dense_store<C>(e, p, m0, n0, [&](int i, int j, int r) { return apply_epi(scaled(i, j, r), EPI_RELU2); },
                     raw_of, no_nan);
    } else {
      dense_store<C>(e, p, m0, n0, scaled, raw_of, no_nan);
    }
  }
}

}  // namespace shk
