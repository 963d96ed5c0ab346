// Dense GEMM kernel on the pipelined engine (tile-multiple shapes, aligned
// operands; both checked on the host).
#pragma once

#include "shk_dma.h"

namespace shk {

template <class C>
using DenseEngine = typename std::conditional<(C::PIPE > 0), DmaEngine<C>, FastEngine<C>>::type;

// Writes the scaled values of one tile: `value(i, j, r)` gives the
// scaled, epilogue-applied fp32 value.  MODE is OUT_BF16 or OUT_F32; NO_NAN
// promises that no value is NaN, which allows the hardware bf16 conversion.
template <class C, int MODE, bool NO_NAN, class E, class Value>
__device__ __forceinline__ void store_values(const E& e, const DenseArgs& p, int m0, int n0, Value value) {
  // Buffer stores: the tile's first element is the resource base, the lane's
  // row and column inside a fragment are its offset, the fragment row block
  // travels in the scalar offset and the fragment column in the immediate,
  // so a store needs no address arithmetic.  The host keeps 256 output rows
  // of fp32 below 4 GiB.
  constexpr uint32_t ESZ = MODE == OUT_BF16 ? 2 : 4;
  const unsigned long long first = (unsigned long long)m0 * p.N + n0;
  const rsrc_t r = make_rsrc(static_cast<uint8_t*>(p.out) + first * ESZ,
                             ((unsigned long long)p.M * p.N - first) * ESZ);
  const uint32_t voff = ((uint32_t)e.out_row(0) * (uint32_t)p.N + (uint32_t)e.out_col(0)) * ESZ;
#pragma unroll
  for (int i = 0; i < C::FM; ++i) {
    const uint32_t soff = (uint32_t)(16 * i) * (uint32_t)p.N * ESZ;
#pragma unroll
    for (int j = 0; j < C::FN; ++j) {
      float v[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] = value(i, j, q);
      const uint32_t off = voff + 16u * j * ESZ;
      if constexpr (MODE == OUT_BF16) {
        uint32_t lo, hi;
        if constexpr (NO_NAN) {
          lo = pack_bf16x2_nonan(v[0], v[1]);
          hi = pack_bf16x2_nonan(v[2], v[3]);
        } else {
          lo = f32_to_bf16_rne(v[0]) | (f32_to_bf16_rne(v[1]) << 16);
          hi = f32_to_bf16_rne(v[2]) | (f32_to_bf16_rne(v[3]) << 16);
        }
        __builtin_amdgcn_raw_buffer_store_b64(v2i{(int)lo, (int)hi}, r, off, soff, 0);
      } else {
        __builtin_amdgcn_raw_buffer_store_b128(v4i{__float_as_int(v[0]), __float_as_int(v[1]), __float_as_int(v[2]),
                                                   __float_as_int(v[3])},
                                               r, off, soff, 0);
      }
      // one fragment at a time: keeps the accumulator reads from being
      // hoisted ahead of their use, which would need more VGPRs than exist
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

// Writes one tile's results.  `value(i, j, r)` gives the scaled, epilogue-
// applied fp32 value, `raw(i, j, r)` the int32 written in verification mode.
// `no_nan` (uniform across the wave) promises that no value is NaN, which
// allows the hardware bf16 conversion.  Each output mode is its own
// straight-line store sequence.
template <class C, class E, class Value, class Raw>
__device__ __forceinline__ void dense_store(const E& e, const DenseArgs& p, int m0, int n0, Value value, Raw raw,
                                            bool no_nan = false) {
  if (p.out_mode == OUT_F32_ADD) {
    float* o = static_cast<float*>(p.out);
#pragma unroll
    for (int i = 0; i < C::FM; ++i)
#pragma unroll
      for (int j = 0; j < C::FN; ++j) {
        float* row = o + (long)(m0 + e.out_row(i)) * p.N + n0 + e.out_col(j);
#pragma unroll
        for (int r = 0; r < 4; ++r) unsafeAtomicAdd(row + r, value(i, j, r));
      }
  } else if (p.out_mode == OUT_I32) {
    const long ldo = C::SWIGLU ? 2L * p.N : (long)p.N;
#pragma unroll
    for (int i = 0; i < C::FM; ++i)
#pragma unroll
      for (int j = 0; j < C::FN2; ++j) {
        if (!C::SWIGLU && j >= C::FN) continue;
        const long col = (j < C::FN ? 0 : p.N) + n0 + e.out_col(j);
        int* o = reinterpret_cast<int*>(p.out) + (long)(m0 + e.out_row(i)) * ldo + col;
        *reinterpret_cast<int4*>(o) = make_int4(raw(i, j, 0), raw(i, j, 1), raw(i, j, 2), raw(i, j, 3));
      }
  } else if (p.out_mode == OUT_F32) {
    store_values<C, OUT_F32, false>(e, p, m0, n0, value);
  } else if (no_nan) {
    store_values<C, OUT_BF16, true>(e, p, m0, n0, value);
  } else {
    store_values<C, OUT_BF16, false>(e, p, m0, n0, value);
  }
}

// The arguments of K slice blockIdx.y of gridDim.y (split-K): the operands
// start at the slice's first K value, subchannel scales at its first group,
// and the tile adds its fp32 result into the output.  The host checks that
// K is a multiple of BK * gridDim.y and, for subchannel scales, that a slice
// holds whole groups.
template <class C>
__device__ __forceinline__ DenseArgs k_slice(DenseArgs p) {
  const int ks = p.K / (int)gridDim.y;
  const long k0 = (long)blockIdx.y * ks * C::BITS / 8;  // bytes into a K row
  p.a += C::A_KMAJOR ? k0 : k0 * p.lda;
  p.b += C::B_KMAJOR ? k0 : k0 * p.ldb;
  if (C::SUBCH) {
    const int g0 = (int)blockIdx.y * (ks / p.subchannel);
    p.a_scale += g0;
    p.b_scale += (long)g0 * p.b_cols;
  }
  p.K = ks;
  p.out_mode = OUT_F32_ADD;
  return p;
}

// One output tile, tile index `tile` in the XCD-aware order.
template <class C>
__device__ __forceinline__ void dense_tile(const DenseArgs& p_all, uint8_t* smem, int tile) {
  const DenseArgs p = gridDim.y > 1 ? k_slice<C>(p_all) : p_all;
  const int tiles_m = p.M / C::BM;
  const int tiles_n = p.N / C::BN;
  int tm, tn;
  dense_tile_coords(tile, tiles_m, tiles_n, p.group_m, tm, tn);
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
    // the scales are loaded before the K loop so their latency is hidden
    float sa[C::FM];
#pragma unroll
    for (int i = 0; i < C::FM; ++i) sa[i] = load_bf16(p.a_scale + m0 + e.out_row(i));
    float sb[C::FN2][4];
#pragma unroll
    for (int j = 0; j < C::FN2; ++j) {
      if (!C::SWIGLU && j >= C::FN) continue;
      load_bf16x4(p.b_scale + (j < C::FN ? 0 : gate) + n0 + e.out_col(j), 4, true, sb[j]);
    }
    auto nop = [](int) {};
    e.run(smem, nst, nop);
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

// One workgroup per tile.
template <class C>
__global__ __launch_bounds__(C::NT) void dense_gemm_kernel(const DenseArgs p) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[C::LDS_BYTES];
  dense_tile<C>(p, smem, blockIdx.x);
}

// Persistent schedule: gridDim.x workgroups (a multiple of 8, at most one
// per resident slot) stride over the tiles, so a workgroup stays on one XCD;
// every LDS read is done before the next tile's stages refill LDS.
template <class C>
__global__ __launch_bounds__(C::NT) void dense_gemm_persistent(const DenseArgs p) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[C::LDS_BYTES];
  const int tiles = (p.M / C::BM) * (p.N / C::BN);
  for (int t = blockIdx.x; t < tiles; t += gridDim.x) {
    dense_tile<C>(p, smem, t);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  }
}

}  // namespace shk
