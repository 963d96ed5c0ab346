// MFMA tile engine and the three kernel families built on it: the dense GEMM
// (mm / fused_swiglu_up_gate / explicit_mm), the grouped ragged forward and the
// K-ragged grouped backward.
//
// A workgroup owns a BM x BN output tile and WM x WN waves; each wave owns a
// (BM/WM) x (BN/WN) sub-tile held as int32 MFMA accumulators (16x16 blocks of
// v_mfma_i32_16x16x64_i8, or 16x16x32 when a subchannel group is 32 wide).
// The B tile is fed as the MFMA's first operand, so a lane's four accumulator
// values are four consecutive output columns of one output row (8-byte bf16 /
// 16-byte fp32 stores).  K is consumed in BK-wide stages through two LDS
// buffers: while the waves multiply stage k out of one buffer, the registers
// prefetched for stage k+1 are widened/transposed into the other and the
// global loads for stage k+2 are in flight; one barrier per stage.
//
// Numerics follow the reference's torch oracle (api.py:299-325,
// ragged.py tests test_ragged_dot.py:19-117): the int32 sum is exact; the
// per-channel result is (float(acc) * a_scale) * b_scale; the subchannel
// result accumulates ((float(acc_g) * a_scale_g) * b_scale_g) in group order
// into an fp32 sum starting at zero; ReLU2 is relu(x)*relu(x); SwiGLU is
// up * (gate / (1 + exp(-gate))).  Every kernel is compiled with
// -ffp-contract=off so none of these products is fused.  int4 operands carry
// the factor 16 per operand (see shk_common.h): float(256*t) == 256*float(t)
// and both scale products are exact scalings by 2^8, so the epilogue works in
// the x256 domain and multiplies by 2^-8 once, which is exact.
#pragma once

#include "shk_tasks.h"
#include "shk_stage.h"

namespace shk {

// OUT_F32_ADD and OUT_I32_ADD are internal: a split-K slice adds its fp32
// partial into out; a K slice of a large-K fp6 launch adds its exact int32
// sums into an int32 workspace.
enum OutMode : int { OUT_BF16 = 0, OUT_F32 = 1, OUT_I32 = 2, OUT_F32_ADD = 3, OUT_I32_ADD = 4 };
enum EpiKind : int { EPI_NONE = 0, EPI_RELU2 = 1 };

template <int BITS_, bool A_KMAJOR_, bool B_KMAJOR_, int BM_, int BN_, int BK_, int WM_, int WN_,
          bool SWIGLU_, bool SUBCH_, int MK_, bool GUARDED_ = true, int PIPE_ = 0>
struct Cfg {
  static constexpr int BITS = BITS_;
  static constexpr bool A_KMAJOR = A_KMAJOR_;
  static constexpr bool B_KMAJOR = B_KMAJOR_;
  static constexpr int BM = BM_;
  static constexpr int BN = BN_;  // output columns of the tile
  static constexpr int BK = BK_;
  static constexpr int WM = WM_;
  static constexpr int WN = WN_;
  static constexpr bool SWIGLU = SWIGLU_;
  static constexpr bool SUBCH = SUBCH_;
  static constexpr int MK = MK_;  // K per MFMA instruction: 64 or 32
  // Guarded kernels carry the per-byte bounds-checked staging path (ragged
  // rows, N tails, masked K); unguarded ones (dense, tile-multiple shapes with
  // aligned operands checked on the host) only have the vector path.
  static constexpr bool GUARDED = GUARDED_;
  // PIPE > 0 selects the direct-to-LDS engine (shk_dma.h) with a ring of PIPE
  // packed stages; 0 the register-staged engine with two widened stages.
  static constexpr int PIPE = PIPE_;
  static constexpr int NT = 64 * WM * WN;
  static constexpr int BROWS = SWIGLU ? 2 * BN : BN;  // B rows staged per stage
  static constexpr int BHALF = BN;
  static constexpr int TM = BM / WM;
  static constexpr int TN = BN / WN;
  static constexpr int FM = TM / 16;
  static constexpr int FN = TN / 16;
  static constexpr int FN2 = SWIGLU ? 2 * FN : FN;
  static constexpr int A_STAGE = BM * BK;
  static constexpr int B_STAGE = BROWS * BK;
  static constexpr int STAGE = A_STAGE + B_STAGE;
  static constexpr int LDS_BYTES = PIPE ? PIPE * (BM + BROWS) * 64 : 2 * STAGE;
  static constexpr int NUM_STAGES = PIPE ? PIPE : 2;
  static constexpr float ACC_UNSCALE = (BITS == 4) ? (1.0f / 256.0f) : 1.0f;
  static constexpr int ACC_SHIFT = (BITS == 4) ? 8 : 0;
  static_assert(TM % 16 == 0 && TN % 16 == 0, "wave tile must be a multiple of 16");
  static_assert(BK % 64 == 0, "stage K must be a multiple of 64");
  static_assert(MK == 64 || MK == 32, "MFMA K is 64 or 32");
  static_assert(LDS_BYTES <= 160 * 1024, "LDS budget");
};

// Per-stage bounds in source units (bytes for int4, values for int8).
template <int BITS>
__device__ __forceinline__ void stage_bounds(int k, int k_limit, int bk, int& kvalid, bool& odd_tail) {
  int valid = k_limit - k;
  valid = valid < 0 ? 0 : (valid > bk ? bk : valid);
  if (BITS == 4) {
    kvalid = (valid + 1) >> 1;
    odd_tail = (valid & 1) != 0;
  } else {
    kvalid = valid;
    odd_tail = false;
  }
}

template <class C>
struct Engine {
  using AStager = typename StagerFor<C::BITS, C::A_KMAJOR, C::BM, C::BK, C::NT, C::BM, C::GUARDED>::type;
  using BStager = typename StagerFor<C::BITS, C::B_KMAJOR, C::BROWS, C::BK, C::NT, C::BHALF, C::GUARDED>::type;

  v4i acc[C::FM][C::FN2];
  int lane, wave, wm, wn;
  int arow0;                // first A tile row of this wave
  int xrow0[2];             // first B tile row of this wave's up / gate fragments

  __device__ __forceinline__ void init() {
    lane = threadIdx.x & 63;
    wave = threadIdx.x >> 6;
    wm = wave % C::WM;
    wn = wave / C::WM;
    arow0 = wm * C::TM;
    xrow0[0] = wn * C::TN;
    xrow0[1] = C::BHALF + wn * C::TN;
#pragma unroll
    for (int i = 0; i < C::FM; ++i)
#pragma unroll
      for (int j = 0; j < C::FN2; ++j) acc[i][j] = v4i{0, 0, 0, 0};
  }

  __device__ __forceinline__ int xrow(int j) const {
    return j < C::FN ? xrow0[0] + 16 * j : xrow0[1] + 16 * (j - C::FN);
  }

  // Output coordinates of accumulator element (i, j, r) relative to the tile.
  __device__ __forceinline__ int out_row(int i) const { return arow0 + 16 * i + (lane & 15); }
  __device__ __forceinline__ int out_col(int j) const {
    return (j < C::FN ? xrow0[0] + 16 * j : xrow0[0] + 16 * (j - C::FN)) + 4 * (lane >> 4);
  }

  // One MFMA K step (MK wide) at step index s inside the stage buffers.
  __device__ __forceinline__ void mma_step(const uint8_t* la, const uint8_t* lb, int s) {
    if (C::MK == 64) {
      const int chunk = 4 * s + (lane >> 4);
      v4i y[C::FM];
      v4i x[C::FN2];
#pragma unroll
      for (int i = 0; i < C::FM; ++i)
        y[i] = *reinterpret_cast<const v4i*>(la + lds_chunk_off<C::BM>(arow0 + 16 * i + (lane & 15), chunk));
#pragma unroll
      for (int j = 0; j < C::FN2; ++j)
        x[j] = *reinterpret_cast<const v4i*>(lb + lds_chunk_off<C::BROWS>(xrow(j) + (lane & 15), chunk));
#pragma unroll
      for (int i = 0; i < C::FM; ++i)
#pragma unroll
        for (int j = 0; j < C::FN2; ++j) acc[i][j] = mfma64(x[j], y[i], acc[i][j]);
    } else {
      const int g = lane >> 4;
      const int chunk = 2 * s + (g >> 1);
      const int half = (g & 1) * 8;
      v2i y[C::FM];
      v2i x[C::FN2];
#pragma unroll
      for (int i = 0; i < C::FM; ++i)
        y[i] = *reinterpret_cast<const v2i*>(la + lds_chunk_off<C::BM>(arow0 + 16 * i + (lane & 15), chunk) + half);
#pragma unroll
      for (int j = 0; j < C::FN2; ++j)
        x[j] = *reinterpret_cast<const v2i*>(lb + lds_chunk_off<C::BROWS>(xrow(j) + (lane & 15), chunk) + half);
#pragma unroll
      for (int i = 0; i < C::FM; ++i)
#pragma unroll
        for (int j = 0; j < C::FN2; ++j) acc[i][j] = mfma32(x[j], y[i], acc[i][j]);
    }
  }

  __device__ __forceinline__ void zero_acc() {
#pragma unroll
    for (int i = 0; i < C::FM; ++i)
#pragma unroll
      for (int j = 0; j < C::FN2; ++j) acc[i][j] = v4i{0, 0, 0, 0};
  }

  // Runs the K loop over `nstages` stages whose logical K starts are given by
  // stage_k(i).  After every MFMA step, on_step(k_step_begin, k_step_end) is
  // called (used for subchannel flushes); steps entirely at or beyond k_limit
  // are skipped.  The stagers' row sources are fixed for the whole loop.
  template <class StageK, class OnStep>
  __device__ __forceinline__ void mainloop(uint8_t* smem, const RowSource& asrc, const RowSource& bsrc,
                                           int nstages, StageK stage_k, int k_limit, bool a_fast_ok,
                                           bool b_fast_ok, OnStep on_step) {
    AStager sa;
    BStager sb;
    if (nstages <= 0) return;
    auto load = [&](int i) {
      const int k = stage_k(i);
      int kv;
      bool odd;
      stage_bounds<C::BITS>(k, k_limit, C::BK, kv, odd);
      const bool full = (k + C::BK) <= k_limit;
      const long koff = (long)k * C::BITS / 8;
      sa.load(asrc, koff, kv, odd, !C::GUARDED || (full && a_fast_ok));
      sb.load(bsrc, koff, kv, odd, !C::GUARDED || (full && b_fast_ok));
    };
    auto store = [&](int buf) {
      uint8_t* base = smem + buf * C::STAGE;
      sa.store(base);
      sb.store(base + C::A_STAGE);
    };
    load(0);
    store(0);
    if (nstages > 1) load(1);
    __syncthreads();
    for (int it = 0; it < nstages; ++it) {
      const int cur = it & 1;
      if (it + 1 < nstages) {
        store(cur ^ 1);
        if (it + 2 < nstages) load(it + 2);
      }
      const uint8_t* la = smem + cur * C::STAGE;
      const uint8_t* lb = la + C::A_STAGE;
      const int k = stage_k(it);
#pragma unroll
      for (int s = 0; s < C::BK / C::MK; ++s) {
        const int kb = k + s * C::MK;
        if (kb < k_limit) {
          mma_step(la, lb, s);
          on_step(kb, kb + C::MK);
        }
      }
      __syncthreads();
    }
  }

  // int32 accumulator as its true integer value.
  __device__ __forceinline__ int true_acc(int v) const { return v >> C::ACC_SHIFT; }
};

// Subchannel fp32 accumulators (one per int32 accumulator element).
template <class C>
struct SubAcc {
  float f[C::FM][C::FN2][4];
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int i = 0; i < C::FM; ++i)
#pragma unroll
      for (int j = 0; j < C::FN2; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) f[i][j][r] = 0.0f;
  }
};

// Loads four consecutive bf16 values that may be unaligned or partially out
// of range (`count` valid).
__device__ __forceinline__ void load_bf16x4(const uint16_t* p, int count, bool vec, float (&o)[4]) {
  if (vec && count >= 4) {
    const uint2 v = *reinterpret_cast<const uint2*>(p);
    o[0] = __uint_as_float(v.x << 16);
    o[1] = __uint_as_float(v.x & 0xFFFF0000u);
    o[2] = __uint_as_float(v.y << 16);
    o[3] = __uint_as_float(v.y & 0xFFFF0000u);
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r) o[r] = r < count ? load_bf16(p + r) : 0.0f;
  }
}

// Folds the current int32 group partials into the fp32 sums:
// f += (float(acc) * a_scale[row, g]) * b_scale[g, col], then clears acc.
// In raw mode the true int32 partial is added to the integer held in f.
// a_scale_row(i) returns a pointer already offset to group g (always in
// bounds); b_scale_col(j) returns the pointer of the fragment's first column
// in group g's scale row, of which `b_count(j)` are valid and `b_vec` says
// whether an aligned 8-byte load may be used.
template <class C, class ARow, class BCol, class BCount>
__device__ __forceinline__ void subchannel_flush(Engine<C>& e, SubAcc<C>& s, ARow a_scale_row,
                                                 BCol b_scale_col, BCount b_count, bool b_vec, bool raw) {
  if (raw) {
#pragma unroll
    for (int i = 0; i < C::FM; ++i)
#pragma unroll
      for (int j = 0; j < C::FN2; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          s.f[i][j][r] = __int_as_float(__float_as_int(s.f[i][j][r]) + e.true_acc(e.acc[i][j][r]));
  } else {
    float sa[C::FM];
#pragma unroll
    for (int i = 0; i < C::FM; ++i) sa[i] = load_bf16(a_scale_row(i));
#pragma unroll
    for (int j = 0; j < C::FN2; ++j) {
      float sb[4];
      load_bf16x4(b_scale_col(j), b_count(j), b_vec, sb);
#pragma unroll
      for (int i = 0; i < C::FM; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float p = (float)e.acc[i][j][r] * sa[i];
          p = p * sb[r];
          s.f[i][j][r] = s.f[i][j][r] + p;
        }
    }
  }
  e.zero_acc();
}

// relu keeps NaN (torch.relu does): only values below zero become zero.
__device__ __forceinline__ float apply_epi(float v, int epi) {
  if (epi == EPI_RELU2) {
    v = v < 0.0f ? 0.0f : v;
    v = v * v;
  }
  return v;
}

__device__ __forceinline__ float swiglu(float up, float gate) {
  return up * (gate / (1.0f + expf(-gate)));
}

// SwiGLU with exp(-g) = 2^(-g * log2(e)) on the hardware exp2 and 1/(1+e) on
// the hardware reciprocal.  For |g| <= SWIGLU_FAST_MAX, e stays in the normal
// range and the result is within a few fp32 ulp of swiglu (the rounding of
// the exponent argument, |g| * log2(e) * 2^-24 relative, dominates), far
// inside the 2-ulp bf16 tolerance of the SwiGLU outputs.
constexpr float SWIGLU_FAST_MAX = 80.0f;
__device__ __forceinline__ float swiglu_fast(float up, float gate) {
  const float e = __builtin_amdgcn_exp2f(gate * -1.4426950408889634f);
  return up * (gate * __builtin_amdgcn_rcpf(1.0f + e));
}

// Writes four consecutive output values of one row (`count` valid).
__device__ __forceinline__ void store_row4(void* out, long idx, const float (&v)[4], const int (&raw)[4],
                                           int count, bool vec, int mode) {
  if (mode == OUT_BF16) {
    uint16_t* o = reinterpret_cast<uint16_t*>(out) + idx;
    if (vec && count >= 4) {
      const uint32_t lo = f32_to_bf16_rne(v[0]) | (f32_to_bf16_rne(v[1]) << 16);
      const uint32_t hi = f32_to_bf16_rne(v[2]) | (f32_to_bf16_rne(v[3]) << 16);
      *reinterpret_cast<uint2*>(o) = make_uint2(lo, hi);
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (r < count) o[r] = (uint16_t)f32_to_bf16_rne(v[r]);
    }
  } else if (mode == OUT_F32) {
    float* o = reinterpret_cast<float*>(out) + idx;
    if (vec && count >= 4) {
      *reinterpret_cast<float4*>(o) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (r < count) o[r] = v[r];
    }
  } else {
    int* o = reinterpret_cast<int*>(out) + idx;
    if (vec && count >= 4) {
      *reinterpret_cast<int4*>(o) = make_int4(raw[0], raw[1], raw[2], raw[3]);
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (r < count) o[r] = raw[r];
    }
  }
}

// ===========================================================================
// Dense GEMM

struct DenseArgs {
  const uint8_t* a;
  const uint8_t* b;
  const uint16_t* a_scale;
  const uint16_t* b_scale;
  void* out;
  int M, N, K;       // logical; N = output columns (D for SwiGLU)
  long lda, ldb;     // bytes between consecutive source rows
  int b_cols;        // columns of the logical B (2*D for SwiGLU): b_scale row length
  int subchannel;    // S, or 0 for per-channel
  int scale_cols;    // ceil(K / S)
  int epilogue;      // EpiKind (SwiGLU is a compile-time property)
  int out_mode;      // OutMode
  int a_aligned;     // operand base/stride alignment allows vector loads
  int b_aligned;
  int group_m;       // tile-row swizzle width
  int layout;        // SHK_LAYOUT_* (read by the fp6 path's operand conversion)
  uint8_t* work;     // fp6 path: caller workspace for the converted operands
  int split_tn;      // int8 256-row tiles: first column tile run as 128-row tiles (0: none)
  int sk_splits;     // skinny per-channel tiles: workgroups sharing a tile's K (1: none)
};

// Tile order: workgroups are dispatched round-robin over the 8 XCDs, so the
// linear id is first remapped to give each XCD a contiguous range, then
// grouped GROUP_M rows at a time so concurrently running tiles on one XCD
// share A rows and B columns in that XCD's L2.
__device__ __forceinline__ void dense_tile_coords(int pid, int tiles_m, int tiles_n, int group_m, int& tm,
                                                  int& tn) {
  const int total = tiles_m * tiles_n;
  if ((total & 7) == 0) pid = (pid & 7) * (total >> 3) + (pid >> 3);
  const int per_group = group_m * tiles_n;
  const int grp = pid / per_group;
  const int first_m = grp * group_m;
  const int gsz = min(tiles_m - first_m, group_m);
  const int in_grp = pid - grp * per_group;
  tm = first_m + in_grp % gsz;
  tn = in_grp / gsz;
}

// dense_gemm_kernel is defined in shk_dense.h on the pipelined engine.

// ===========================================================================
// Ragged forward: out[rows of group g] = lhs[rows] @ rhs[g]

struct RaggedFwdArgs {
  const uint8_t* lhs;
  const uint8_t* rhs;
  const uint16_t* a_scale;
  const uint16_t* b_scale;
  const int* tasks;      // [capacity][4]: group, block_start, actual_start, actual_end
  const int* num_tasks;  // device scalar
  int capacity;          // task slots covered by the grid
  void* out;
  int M, N, K;           // logical rows, output columns, logical K
  int groups;
  long lda, ldb;         // bytes between consecutive source rows of lhs / rhs[g]
  int subchannel, scale_cols;
  int out_mode;
  int a_aligned, b_aligned, out_vec;
  int layout;     // SHK_LAYOUT_* (fp6 entries convert either layout)
  uint8_t* work;  // fp6 entries: operand workspace
  // fp6 entries: a task list to build in the conversion launch, before the
  // GEMM reads it (job.sizes == nullptr: the list is already built)
  TaskJob job;
};

template <class C>
__global__ __launch_bounds__(C::NT) void ragged_fwd_kernel(const RaggedFwdArgs p) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[C::LDS_BYTES];
  const int tiles_n = (p.N + C::BN - 1) / C::BN;
  const int task = blockIdx.x / tiles_n;
  const int tn = blockIdx.x - task * tiles_n;
  const int ntasks = *p.num_tasks;
  // A task list that overflowed its capacity is refused as a whole.
  if (ntasks > p.capacity || task >= ntasks) return;
  const int4 t = *reinterpret_cast<const int4*>(p.tasks + 4 * task);
  const int g = t.x, block_start = t.y, act_start = t.z, act_end = t.w;
  const int n0 = tn * C::BN;
  const long kp = (long)p.K * C::BITS / 8;  // source bytes of K per row

  RowSource asrc, bsrc;
  if (C::A_KMAJOR) {  // lhs [M, Kp]
    asrc.base0 = p.lhs + (long)block_start * p.lda;
  } else {            // lhs [Kp, M]
    asrc.base0 = p.lhs + block_start;
  }
  asrc.base1 = asrc.base0;
  asrc.ld = p.lda;
  asrc.rows_valid = min(C::BM, p.M - block_start);
  const uint8_t* rg = p.rhs + (long)g * kp * p.N;
  if (C::B_KMAJOR) {  // rhs[g] [N, Kp]
    bsrc.base0 = rg + (long)n0 * p.ldb;
  } else {            // rhs[g] [Kp, N]
    bsrc.base0 = rg + n0;
  }
  bsrc.base1 = bsrc.base0;
  bsrc.ld = p.ldb;
  bsrc.rows_valid = min(C::BN, p.N - n0);
  const bool a_fast = p.a_aligned && asrc.rows_valid == C::BM;
  const bool b_fast = p.b_aligned && bsrc.rows_valid == C::BN;

  Engine<C> e;
  e.init();
  const int nst = (p.K + C::BK - 1) / C::BK;
  auto stage_k = [](int i) { return i * C::BK; };
  const bool raw = p.out_mode == OUT_I32;
  const uint16_t* bscale_g = p.b_scale + (long)g * p.scale_cols * p.N;  // per-channel: scale_cols == 1

  float v[C::FM][C::FN][4];
  int rv[C::FM][C::FN][4];
  if (C::SUBCH) {
    SubAcc<C> s;
    s.zero();
    const int S = p.subchannel;
    auto on_step = [&](int kb, int ke) {
      if ((ke % S) == 0 || ke >= p.K) {
        const int gi = kb / S;
        subchannel_flush<C>(
            e, s,
            [&](int i) {
              const int m = min(block_start + e.out_row(i), p.M - 1);
              return p.a_scale + (long)m * p.scale_cols + gi;
            },
            [&](int j) { return bscale_g + (long)gi * p.N + min(n0 + e.out_col(j), p.N); },
            [&](int j) { return p.N - (n0 + e.out_col(j)); }, p.out_vec != 0, raw);
      }
    };
    e.mainloop(smem, asrc, bsrc, nst, stage_k, p.K, a_fast, b_fast, on_step);
#pragma unroll
    for (int i = 0; i < C::FM; ++i)
#pragma unroll
      for (int j = 0; j < C::FN; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          rv[i][j][r] = __float_as_int(s.f[i][j][r]);
          v[i][j][r] = s.f[i][j][r] * C::ACC_UNSCALE;
        }
  } else {
    e.mainloop(smem, asrc, bsrc, nst, stage_k, p.K, a_fast, b_fast, [](int, int) {});
#pragma unroll
    for (int i = 0; i < C::FM; ++i) {
      const int m = min(block_start + e.out_row(i), p.M - 1);
      const float sa = load_bf16(p.a_scale + m);
#pragma unroll
      for (int j = 0; j < C::FN; ++j) {
        const int n = n0 + e.out_col(j);
        float sb[4];
        load_bf16x4(bscale_g + n, p.N - n, p.out_vec, sb);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int a = e.acc[i][j][r];
          rv[i][j][r] = e.true_acc(a);
          float x = (float)a * sa;
          x = x * sb[r];
          v[i][j][r] = x * C::ACC_UNSCALE;
        }
      }
    }
  }
#pragma unroll
  for (int i = 0; i < C::FM; ++i) {
    const int m = block_start + e.out_row(i);
    if (m < act_start || m >= act_end) continue;
#pragma unroll
    for (int j = 0; j < C::FN; ++j) {
      const int n = n0 + e.out_col(j);
      if (n >= p.N) continue;
      store_row4(p.out, (long)m * p.N + n, v[i][j], rv[i][j], p.N - n, p.out_vec, p.out_mode);
    }
  }
}

// ===========================================================================
// Ragged backward: out[g] = op(lhs[g]) @ op(rhs[g]) over K = group_sizes[g]

struct RaggedBwdArgs {
  const uint8_t* lhs;
  const uint8_t* rhs;
  const uint16_t* a_scale;
  const uint16_t* b_scale;
  const int* group_sizes;  // int32 [G]
  void* out;               // fp32 [G, M, N] (int32 partials when split_k > 1 per-channel)
  int M, N, k_cap;         // output rows, output columns, logical K capacity (2 * K_PACKED)
  int groups;
  long lda, ldb;           // bytes between consecutive source rows of lhs[g] / rhs[g]
  int subchannel, scale_cols;
  int split_k;
  int out_mode;            // OUT_F32, or OUT_I32 raw
  int a_aligned, b_aligned, out_vec;
  int layout;              // SHK_LAYOUT_* (fp6 entries convert either layout)
  uint8_t* work;           // fp6 entries: operand workspace
};

template <class C>
__global__ __launch_bounds__(C::NT) void ragged_bwd_kernel(const RaggedBwdArgs p) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[C::LDS_BYTES];
  const int tiles_m = (p.M + C::BM - 1) / C::BM;
  const int tiles_n = (p.N + C::BN - 1) / C::BN;
  const int per_group = tiles_m * tiles_n;
  const int g = blockIdx.x / per_group;
  const int tile = blockIdx.x - g * per_group;
  const int tm = tile / tiles_n;
  const int tn = tile - tm * tiles_n;
  const int split = blockIdx.y;
  const int m0 = tm * C::BM;
  const int n0 = tn * C::BN;
  // Lengths outside [0, k_cap] are clamped so no load leaves the operands.
  const int gk = min(max(p.group_sizes[g], 0), p.k_cap);
  const long kp = (long)p.k_cap * C::BITS / 8;

  RowSource asrc, bsrc;
  const uint8_t* lg = p.lhs + (long)g * kp * p.M;
  if (C::A_KMAJOR) {  // lhs[g] [M, Kp]
    asrc.base0 = lg + (long)m0 * p.lda;
  } else {            // lhs[g] [Kp, M]
    asrc.base0 = lg + m0;
  }
  asrc.base1 = asrc.base0;
  asrc.ld = p.lda;
  asrc.rows_valid = min(C::BM, p.M - m0);
  const uint8_t* rg = p.rhs + (long)g * kp * p.N;
  if (C::B_KMAJOR) {  // rhs[g] [N, Kp]
    bsrc.base0 = rg + (long)n0 * p.ldb;
  } else {            // rhs[g] [Kp, N]
    bsrc.base0 = rg + n0;
  }
  bsrc.base1 = bsrc.base0;
  bsrc.ld = p.ldb;
  bsrc.rows_valid = min(C::BN, p.N - n0);
  const bool a_fast = p.a_aligned && asrc.rows_valid == C::BM;
  const bool b_fast = p.b_aligned && bsrc.rows_valid == C::BN;

  Engine<C> e;
  e.init();
  const bool raw = p.out_mode == OUT_I32;
  const int SK = p.split_k;
  const int total_stages = (gk + C::BK - 1) / C::BK;
  float v[C::FM][C::FN][4];
  int rv[C::FM][C::FN][4];
  const uint16_t* ascale_g = p.a_scale + (long)g * p.M * p.scale_cols;
  const uint16_t* bscale_g = p.b_scale + (long)g * p.scale_cols * p.N;

  if (C::SUBCH) {
    SubAcc<C> s;
    s.zero();
    const int S = p.subchannel;
    auto on_step = [&](int kb, int ke) {
      if ((ke % S) == 0 || ke >= gk) {
        const int gi = kb / S;
        subchannel_flush<C>(
            e, s,
            [&](int i) {
              const int m = min(m0 + e.out_row(i), p.M - 1);
              return ascale_g + (long)m * p.scale_cols + gi;
            },
            [&](int j) { return bscale_g + (long)gi * p.N + min(n0 + e.out_col(j), p.N); },
            [&](int j) { return p.N - (n0 + e.out_col(j)); }, p.out_vec != 0, raw);
      }
    };
    if (S >= C::BK) {
      // Split over whole scale groups: split s owns groups s, s+SK, ...
      const int spg = S / C::BK;
      const int ngroups = (gk + S - 1) / S;
      const int my_groups = ngroups > split ? (ngroups - split + SK - 1) / SK : 0;
      auto stage_k = [=](int i) { return (split + (i / spg) * SK) * S + (i % spg) * C::BK; };
      e.mainloop(smem, asrc, bsrc, my_groups * spg, stage_k, gk, a_fast, b_fast, on_step);
    } else {
      // Each stage holds whole groups: split over stages.
      const int my = total_stages > split ? (total_stages - split + SK - 1) / SK : 0;
      auto stage_k = [=](int i) { return (split + i * SK) * C::BK; };
      e.mainloop(smem, asrc, bsrc, my, stage_k, gk, a_fast, b_fast, on_step);
    }
#pragma unroll
    for (int i = 0; i < C::FM; ++i)
#pragma unroll
      for (int j = 0; j < C::FN; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          rv[i][j][r] = __float_as_int(s.f[i][j][r]);
          v[i][j][r] = s.f[i][j][r] * C::ACC_UNSCALE;
        }
  } else {
    const int my = total_stages > split ? (total_stages - split + SK - 1) / SK : 0;
    auto stage_k = [=](int i) { return (split + i * SK) * C::BK; };
    e.mainloop(smem, asrc, bsrc, my, stage_k, gk, a_fast, b_fast, [](int, int) {});
#pragma unroll
    for (int i = 0; i < C::FM; ++i) {
      const int m = min(m0 + e.out_row(i), p.M - 1);
      const float sa = load_bf16(ascale_g + m);
#pragma unroll
      for (int j = 0; j < C::FN; ++j) {
        const int n = n0 + e.out_col(j);
        float sb[4];
        load_bf16x4(bscale_g + n, p.N - n, p.out_vec, sb);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int a = e.acc[i][j][r];
          rv[i][j][r] = e.true_acc(a);
          float x = (float)a * sa;
          x = x * sb[r];
          v[i][j][r] = x * C::ACC_UNSCALE;
        }
      }
    }
  }

  float* outg = reinterpret_cast<float*>(p.out) + (long)g * p.M * p.N;
#pragma unroll
  for (int i = 0; i < C::FM; ++i) {
    const int m = m0 + e.out_row(i);
    if (m >= p.M) continue;
#pragma unroll
    for (int j = 0; j < C::FN; ++j) {
      const int n = n0 + e.out_col(j);
      if (n >= p.N) continue;
      const int cnt = min(4, p.N - n);
      const long idx = (long)m * p.N + n;
      if (SK == 1) {
        store_row4(outg, idx, v[i][j], rv[i][j], cnt, p.out_vec, raw ? OUT_I32 : OUT_F32);
      } else if (C::SUBCH && !raw) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (r < cnt) atomicAdd(outg + idx + r, v[i][j][r]);
      } else {
        // Exact int32 partials; a finalize pass applies the scales.
        int* o = reinterpret_cast<int*>(outg) + idx;
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (r < cnt) atomicAdd(o + r, rv[i][j][r]);
      }
    }
  }
}

}  // namespace shk
