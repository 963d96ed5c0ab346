// Ragged forward and K-ragged backward on the fp6 MFMA.
//
// Both convert their int4 operands into fp6 blocks in a caller workspace
// first (one f6_pack_two launch for both operands), then run the 128 x 128
// fp6 tile of shk_f6small.h over the converted blocks: the ragged grids are
// small (the MoE forward of G=8, M=8192, N=1408 makes ~750 of these tiles
// against ~220 of 256 x 256), so the finer tile fills the CUs and lets one
// workgroup's prologue and epilogue overlap another's MFMAs.  Both run the
// engine's two-slot ring, three workgroups per CU, so that the 748 tiles of
// that forward start in one round (768 slots) instead of 1.46 rounds of
// 512.  The conversion absorbs the operand layouts, so one GEMM kernel per
// output mode serves every layout.
//
// Forward (ragged.py:1008-1229 semantics): out[rows of group g] =
// lhs[rows] @ rhs[g].  Workgroup (task, tn) takes the task's 128 rows from
// block_start (a multiple of 32: the task list is built with align_tile a
// multiple of 32) against group g's 128-column tile tn, and writes rows
// [actual_start, actual_end) and columns below N.  K is zero-padded to Kw,
// a multiple of 128.  Workspace: A as round32(M) rows x Kw, then per group
// B as round32(N) rows x Kw.
//
// Subchannel forward: the same tasks and converted operands on the 128 x 128
// subchannel tile of shk_f6sub.h (groups of 32 to 256 added into fp32 in
// group order, api.py:311-325 as ragged.py applies it), two workgroups per
// CU, its stores masked to the task's rows and the columns below N.  Its
// workspace pads K to 256 and the conversion writes whole 256-K stages for
// groups of 256, so the ceil(K / S) groups (the last one ending at K, whose
// values past K the conversion zeroes) run whole stages of the tile.
//
// Backward (ragged.py:1232-1402 semantics): out[g] = lhs[g] @ rhs[g] over
// the first group_sizes[g] K values.  The conversion zeroes K at and past
// that length, so group g runs ceil(len / 128) whole 128-K stages.
// Workspace: per group A (round32(M) rows x Kw), then per group B
// (round32(N) rows x Kw), Kw = K capacity rounded up to 128.
#include "shk_f6small.h"
#include "shk_f6sub.h"
#include "shk_table.h"

namespace shk {
namespace {

// 128 A rows x 128 B rows, 2 x 2 waves, plain epilogue.
using F6R = Cfg<4, true, true, 128, 128, 128, 2, 2, false, false, 64, false, 0>;
// ring slots of both kernels (see above)
constexpr int kSlots = 2;
using F6RE = F6SmallEngine<F6R, kSlots>;
constexpr int kTile = 128;

__host__ __device__ inline int round32(int x) { return (x + 31) & ~31; }
__host__ __device__ inline int round128(int x) { return (x + 127) & ~127; }
__host__ __device__ inline int round256(int x) { return (x + 255) & ~255; }

// Workgroups are dispatched round-robin over the 8 XCDs (workgroup w on XCD
// w % 8), each with its own L2.  Maps the first `total` workgroup ids onto
// [0, total) so that XCD x runs one contiguous range, x * q + min(x, r) +
// [0, q + (x < r)) for total = 8q + r.
__device__ __forceinline__ int xcd_contiguous(int w, int total) {
  const int x = w & 7, i = w >> 3, q = total >> 3, r = total & 7;
  return x * q + (x < r ? x : r) + i;
}

template <int MODE>
__global__ __launch_bounds__(256, 3) void f6_ragged_fwd_kernel(const RaggedFwdArgs p) {
  using E = F6RE;
  __shared__ __attribute__((aligned(16))) uint8_t smem[E::LDS_BYTES + MFMA32_SCALE_BYTES];
  const int tiles_n = (p.N + kTile - 1) / kTile;
  const int ntasks = *p.num_tasks;
  // A task list that overflowed its capacity is refused as a whole.
  const int live = ntasks * tiles_n;
  if (ntasks > p.capacity || (int)blockIdx.x >= live) return;
  // each XCD takes consecutive tasks with all their column tiles: A tiles
  // are shared by the column tiles and B tiles by the tasks of a group
  const int w = xcd_contiguous(blockIdx.x, live);
  const int task = w / tiles_n;
  const int tn = w - task * tiles_n;
  const int4 t = *reinterpret_cast<const int4*>(p.tasks + 4 * task);
  const int g = t.x, m0 = t.y;
  const int kw = round128(p.K);
  const unsigned long long a_bytes = f6_operand_bytes(round32(p.M), kw);
  const unsigned long long b_bytes = f6_operand_bytes(round32(p.N), kw);
  E e;
  e.setup(smem, p.work, p.work + a_bytes + (unsigned long long)g * b_bytes, m0, tn * kTile, kw / 64, a_bytes,
          b_bytes);
  float sa[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int m = m0 + e.out_row(i);
    sa[i] = MODE == OUT_I32 ? 0.0f : load_bf16(p.a_scale + (m < p.M ? m : p.M - 1));
  }
  const OutView o{p.out, p.b_scale + (long)g * p.N, p.N, p.M, p.N, t.z, t.w, p.N};
  mfma32_prefetch_b_scales<F6R, MODE, true>(e, o, tn * kTile, e.lds0 + E::LDS_BYTES + 256u * e.wave);
  e.run(kw / 128);
  f6s_finish<MODE, true>(e, o, smem, m0, tn * kTile, sa);
}

// The subchannel tile (128 A rows x 128 B rows, 2 x 2 waves).
using F6RS = Cfg<4, true, true, 128, 128, 128, 2, 2, false, true, 64, false, 0>;

// Stages of the subchannel tile for ng groups of 32 * G32: 128-K stages,
// two per group of 256; else 64-K stages, G32 / 2 per group, or one per two
// groups of 32.  A count that the engine's loop does not divide ends with
// stages past the last one, whose operands and scales load as zeros.
// LIMIT, with groups of 32 and ng possibly odd: fold_last stops the folds at
// group ng - 1 (the second half of the last stage starts past the length,
// where the reference reads no scale).  Without it the limit stays the
// engine's constant default, and the folds carry no test.
template <int G32, bool LIMIT, class E>
__device__ __forceinline__ int sub_stages(E& e, int ng) {
  if constexpr (G32 == 1 && LIMIT) e.fold_last = ng - 1;
  return G32 == 8 ? 2 * ng : (G32 == 1 ? (ng + 1) / 2 : ng * (G32 / 2));
}

template <int MODE, int G32>
__global__ __launch_bounds__(256, 2) void f6_ragged_sub_fwd_kernel(const RaggedFwdArgs p) {
  using E = F6SubEngineFor<F6RS, G32>;
  __shared__ __attribute__((aligned(16))) uint8_t smem[E::LDS_BYTES];
  const int tiles_n = (p.N + kTile - 1) / kTile;
  const int ntasks = *p.num_tasks;
  const int live = ntasks * tiles_n;
  if (ntasks > p.capacity || (int)blockIdx.x >= live) return;
  const int w = xcd_contiguous(blockIdx.x, live);
  const int task = w / tiles_n;
  const int tn = w - task * tiles_n;
  const int4 t = *reinterpret_cast<const int4*>(p.tasks + 4 * task);
  const int g = t.x, m0 = t.y, n0 = tn * kTile;
  const int kw = round256(p.K);
  const unsigned long long a_bytes = f6_operand_bytes(round32(p.M), kw);
  const unsigned long long b_bytes = f6_operand_bytes(round32(p.N), kw);
  E e;
  e.setup(smem, p.work, p.work + a_bytes + (unsigned long long)g * b_bytes, m0, n0, kw / 64, a_bytes, b_bytes,
          p.a_scale, p.b_scale + (long)g * p.scale_cols * p.N, p.M, p.N, p.scale_cols);
  // (ceil(K/32) is even for groups of 32: every stage holds two live groups)
  e.template run<MODE == OUT_I32>(smem, sub_stages<G32, false>(e, p.scale_cols));
  const OutView o{p.out, nullptr, p.N, p.M, p.N, t.z, t.w, p.N};
  if constexpr (MODE == OUT_I32 || MODE == OUT_F32) {
    f6sub_store_words<true>(e, o, m0, n0, [&](int i, int j, int x) { return __float_as_int(e.tot[i][j][x]); });
  } else {
    auto val = [&](int i, int j, int x) { return e.tot[i][j][x]; };
    if (e.all_fast) f6sub_store_bf16<true, true>(e, o, smem, m0, n0, val);
    else f6sub_store_bf16<false, true>(e, o, smem, m0, n0, val);
  }
}

// Regions of the backward's per-group tile grid: sm x sn = 8, one per XCD;
// 0 x 0 where none fits.  Rows split evenly; columns may split unevenly.
__host__ __device__ inline void bwd_regions(int tiles_m, int tiles_n, int& sm, int& sn) {
  sm = sn = 0;
  if (tiles_m % 4 == 0 && tiles_n >= 2) sm = 4, sn = 2;
  else if (tiles_m % 2 == 0 && tiles_n % 4 == 0) sm = 2, sn = 4;
  else if (tiles_m % 8 == 0) sm = 8, sn = 1;
  else if (tiles_n % 8 == 0) sm = 1, sn = 8;
}

// The backward tile of this workgroup: group g, tile row tm, tile column tn;
// false for the spare workgroups of the narrower column regions.  Each
// group's tiles_m x tiles_n grid splits into 8 regions, sm along M and sn
// along N, one per XCD, so an XCD reads each of its A tiles for the column
// tiles of its region and each B tile for its row tiles from its own L2,
// and holds tiles of every group, whatever their lengths.  Rows split
// evenly, columns into floor or ceil(tiles_n / sn) (C5's 11 column tiles: 5
// and 6, so a B tile is read by 4 XCDs instead of all 8 with 8 x 1
// regions: the C5 backward 42.4 -> 41.8 us per call, A/B on one box).
// Grids that split no such way run in order.
__device__ __forceinline__ bool bwd_tile(const RaggedBwdArgs& p, int& g, int& tm, int& tn) {
  const int tiles_m = (p.M + kTile - 1) / kTile;
  const int tiles_n = (p.N + kTile - 1) / kTile;
  int sm = 0, sn = 0;  // region counts along M and N (sm * sn = 8)
  bwd_regions(tiles_m, tiles_n, sm, sn);
  if (sm) {
    const int x = blockIdx.x & 7, i = blockIdx.x >> 3;
    // rows: bm per region; columns: regions of floor or ceil(tiles_n / sn),
    // each XCD's workgroups laid out for the widest (the rest return)
    const int bm = tiles_m / sm, bn = (tiles_n + sn - 1) / sn;
    g = i / (bm * bn);
    const int local = i - g * (bm * bn);
    const int xn = x % sn;
    const int c0 = tiles_n * xn / sn, width = tiles_n * (xn + 1) / sn - c0;
    if (local % bn >= width) return false;
    tm = (x / sn) * bm + local / bn;
    tn = c0 + local % bn;
  } else {
    g = blockIdx.x / (tiles_m * tiles_n);
    const int t = blockIdx.x - g * (tiles_m * tiles_n);
    tm = t / tiles_n;
    tn = t - tm * tiles_n;
  }
  return true;
}

template <int MODE>
__global__ __launch_bounds__(256, 3) void f6_ragged_bwd_kernel(const RaggedBwdArgs p) {
  using E = F6RE;
  __shared__ __attribute__((aligned(16))) uint8_t smem[E::LDS_BYTES + MFMA32_SCALE_BYTES];
  int g, tm, tn;
  if (!bwd_tile(p, g, tm, tn)) return;
  const int m0 = tm * kTile;
  const int kw = round128(p.k_cap);
  int len = p.group_sizes[g];
  len = len < 0 ? 0 : (len > p.k_cap ? p.k_cap : len);
  const unsigned long long a_bytes = f6_operand_bytes(round32(p.M), kw);
  const unsigned long long b_bytes = f6_operand_bytes(round32(p.N), kw);
  const uint8_t* a6 = p.work + (unsigned long long)g * a_bytes;
  const uint8_t* b6 = p.work + (unsigned long long)p.groups * a_bytes + (unsigned long long)g * b_bytes;
  E e;
  e.setup(smem, a6, b6, m0, tn * kTile, kw / 64, a_bytes, b_bytes);
  const uint16_t* sa_g = p.a_scale + (long)g * p.M;
  float sa[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int m = m0 + e.out_row(i);
    sa[i] = MODE == OUT_I32 ? 0.0f : load_bf16(sa_g + (m < p.M ? m : p.M - 1));
  }
  const OutView o{static_cast<float*>(p.out) + (long)g * p.M * p.N, p.b_scale + (long)g * p.N, p.N, p.M, p.N, 0,
                  p.M, p.N};
  mfma32_prefetch_b_scales<F6R, MODE, true>(e, o, tn * kTile, e.lds0 + E::LDS_BYTES + 256u * e.wave);
  // whole 128-K stages: the conversion writes no block past the last one
  e.run((len + 127) / 128);
  f6s_finish<MODE, true>(e, o, smem, m0, tn * kTile, sa);
}

// The subchannel backward: group g's tile over the scale groups that start
// below its length, ceil(len / S) of them, each folded into fp32 in group
// order (the conversion zeroes K past len and writes the blocks up to whole
// groups of 256 for S = 256, so the last group's partial sums cover exactly
// its first len - S * (ceil(len / S) - 1) values).  K is padded to 256, so
// those groups' stages never pass the converted blocks.
// With one 64-K stage per group (S = 64), or two groups per stage (S = 32),
// an odd stage count ends with a stage past the last one, whose operands
// and scales load as zeros.  With groups of 32 the last stage may hold one
// group past the length: the engine stops folding after group ng - 1, so
// its scales are never read into the totals.
template <int MODE, int G32>
__global__ __launch_bounds__(256, 2) void f6_ragged_sub_bwd_kernel(const RaggedBwdArgs p) {
  static_assert(G32 == 1 || G32 == 2 || G32 == 4 || G32 == 8, "groups of 32, 64, 128 or 256");
  using E = F6SubEngineFor<F6RS, G32>;
  __shared__ __attribute__((aligned(16))) uint8_t smem[E::LDS_BYTES];
  int g, tm, tn;
  if (!bwd_tile(p, g, tm, tn)) return;
  const int m0 = tm * kTile, n0 = tn * kTile;
  const int kw = round256(p.k_cap);
  int len = p.group_sizes[g];
  len = len < 0 ? 0 : (len > p.k_cap ? p.k_cap : len);
  const unsigned long long a_bytes = f6_operand_bytes(round32(p.M), kw);
  const unsigned long long b_bytes = f6_operand_bytes(round32(p.N), kw);
  const uint8_t* a6 = p.work + (unsigned long long)g * a_bytes;
  const uint8_t* b6 = p.work + (unsigned long long)p.groups * a_bytes + (unsigned long long)g * b_bytes;
  E e;
  e.setup(smem, a6, b6, m0, n0, kw / 64, a_bytes, b_bytes, p.a_scale + (long)g * p.M * p.scale_cols,
          p.b_scale + (long)g * p.scale_cols * p.N, p.M, p.N, p.scale_cols);
  e.template run<MODE == OUT_I32>(smem, sub_stages<G32, true>(e, (len + 32 * G32 - 1) / (32 * G32)));
  const OutView o{static_cast<float*>(p.out) + (long)g * p.M * p.N, nullptr, p.N, p.M, p.N, 0, p.M, p.N};
  f6sub_store_words<true>(e, o, m0, n0, [&](int i, int j, int x) { return __float_as_int(e.tot[i][j][x]); });
}

bool lhs_mn_major(int layout) { return layout == SHK_LAYOUT_TN || layout == SHK_LAYOUT_TT; }
bool rhs_mn_major(int layout) { return layout == SHK_LAYOUT_NN || layout == SHK_LAYOUT_TN; }
// Source piece size of the conversion: the alignment (16, 8 or 1) of the
// base and the row pitch (the pitch of an MN-major source is its row
// count); each operand of a batch starts K/2 * rows bytes after the
// previous one, a multiple of the pitch.
int piece_bytes(const uint8_t* src, long ld) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(src) | (uintptr_t)ld;
  return (a & 15) == 0 ? 16 : ((a & 7) == 0 ? 8 : 1);
}

hipError_t launch_f6_ragged_fwd(const RaggedFwdArgs& a, dim3 grid, hipStream_t s) {
  const int kw = round128(a.K);
  const unsigned long long a_bytes = f6_operand_bytes(round32(a.M), kw);
  const F6PackArgs pa{a.lhs, a.work, a.lda, a.M, kw / 64, 0, 1, 0, 0, nullptr, a.K, piece_bytes(a.lhs, a.lda),
                      false, 2};
  const F6PackArgs pb{a.rhs,   a.work + a_bytes, a.ldb, a.N, kw / 64, 0, a.groups, (long)(a.K / 2) * a.N,
                      f6_operand_bytes(round32(a.N), kw), nullptr, a.K, piece_bytes(a.rhs, a.ldb), false, 2};
  hipError_t err = launch_f6_pack2(pa, lhs_mn_major(a.layout), pb, rhs_mn_major(a.layout), s,
                                   a.job.sizes != nullptr ? &a.job : nullptr);
  if (err != hipSuccess) return err;
  if (a.out_mode == OUT_I32) hipLaunchKernelGGL(f6_ragged_fwd_kernel<OUT_I32>, grid, dim3(256), 0, s, a);
  else if (a.out_mode == OUT_F32) hipLaunchKernelGGL(f6_ragged_fwd_kernel<OUT_F32>, grid, dim3(256), 0, s, a);
  else hipLaunchKernelGGL(f6_ragged_fwd_kernel<OUT_BF16>, grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

template <int MODE>
void launch_ragged_sub(const RaggedFwdArgs& a, dim3 grid, hipStream_t s) {
  if (a.subchannel == 32) hipLaunchKernelGGL((f6_ragged_sub_fwd_kernel<MODE, 1>), grid, dim3(256), 0, s, a);
  else if (a.subchannel == 64) hipLaunchKernelGGL((f6_ragged_sub_fwd_kernel<MODE, 2>), grid, dim3(256), 0, s, a);
  else if (a.subchannel == 128) hipLaunchKernelGGL((f6_ragged_sub_fwd_kernel<MODE, 4>), grid, dim3(256), 0, s, a);
  else hipLaunchKernelGGL((f6_ragged_sub_fwd_kernel<MODE, 8>), grid, dim3(256), 0, s, a);
}
hipError_t launch_f6_ragged_sub_fwd(const RaggedFwdArgs& a, dim3 grid, hipStream_t s) {
  const int kw = round256(a.K);
  const unsigned long long a_bytes = f6_operand_bytes(round32(a.M), kw);
  F6PackArgs pa{a.lhs, a.work, a.lda, a.M, kw / 64, 0, 1, 0, 0, nullptr, a.K, piece_bytes(a.lhs, a.lda),
                false, 2};
  F6PackArgs pb{a.rhs,   a.work + a_bytes, a.ldb, a.N, kw / 64, 0, a.groups, (long)(a.K / 2) * a.N,
                f6_operand_bytes(round32(a.N), kw), nullptr, a.K, piece_bytes(a.rhs, a.ldb), false, 2};
  // groups of 256 run two 128-K stages each
  pa.k_stage = pb.k_stage = a.subchannel > 128 ? 256 : 128;
  hipError_t err = launch_f6_pack2(pa, lhs_mn_major(a.layout), pb, rhs_mn_major(a.layout), s,
                                   a.job.sizes != nullptr ? &a.job : nullptr);
  if (err != hipSuccess) return err;
  if (a.out_mode == OUT_I32) launch_ragged_sub<OUT_I32>(a, grid, s);
  else if (a.out_mode == OUT_F32) launch_ragged_sub<OUT_F32>(a, grid, s);
  else launch_ragged_sub<OUT_BF16>(a, grid, s);
  return hipGetLastError();
}

// The backward's grid (with XCD regions, every XCD's workgroups cover its
// widest region) and its conversion of both operands, K padded to kw, each
// group's blocks written up to whole k_stage-K stages past its length.
hipError_t bwd_grid(const RaggedBwdArgs& a, dim3& grid) {
  const int tiles_m = (a.M + kTile - 1) / kTile, tiles_n = (a.N + kTile - 1) / kTile;
  int sm, sn;
  bwd_regions(tiles_m, tiles_n, sm, sn);
  if (sm) {
    const long long n = 8LL * a.groups * (tiles_m / sm) * ((tiles_n + sn - 1) / sn);
    if (n > 0x7FFFFFFFLL) return hipErrorInvalidValue;
    grid.x = (unsigned)n;
  }
  return hipSuccess;
}
hipError_t bwd_convert(const RaggedBwdArgs& a, int kw, int k_stage, hipStream_t s) {
  const unsigned long long a_group = f6_operand_bytes(round32(a.M), kw);
  const long kp = a.k_cap / 2;
  F6PackArgs pa{a.lhs,     a.work,  a.lda,         a.M,    kw / 64, 0, a.groups, kp * a.M, a_group,
                      a.group_sizes, a.k_cap, piece_bytes(a.lhs, a.lda), true, 2};
  F6PackArgs pb{a.rhs,
                      a.work + (unsigned long long)a.groups * a_group,
                      a.ldb,
                      a.N,
                      kw / 64,
                      0,
                      a.groups,
                      kp * a.N,
                      f6_operand_bytes(round32(a.N), kw),
                      a.group_sizes,
                      a.k_cap,
                      piece_bytes(a.rhs, a.ldb),
                      true,
                      2};
  pa.k_stage = pb.k_stage = k_stage;
  return launch_f6_pack2(pa, lhs_mn_major(a.layout), pb, rhs_mn_major(a.layout), s);
}

hipError_t launch_f6_ragged_bwd(const RaggedBwdArgs& a, dim3 grid, hipStream_t s) {
  hipError_t err = bwd_grid(a, grid);
  if (err == hipSuccess) err = bwd_convert(a, round128(a.k_cap), 128, s);
  if (err != hipSuccess) return err;
  if (a.out_mode == OUT_I32) hipLaunchKernelGGL(f6_ragged_bwd_kernel<OUT_I32>, grid, dim3(256), 0, s, a);
  else hipLaunchKernelGGL(f6_ragged_bwd_kernel<OUT_F32>, grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

template <int MODE>
void launch_ragged_sub_bwd(const RaggedBwdArgs& a, dim3 grid, hipStream_t s) {
  if (a.subchannel == 32) hipLaunchKernelGGL((f6_ragged_sub_bwd_kernel<MODE, 1>), grid, dim3(256), 0, s, a);
  else if (a.subchannel == 64) hipLaunchKernelGGL((f6_ragged_sub_bwd_kernel<MODE, 2>), grid, dim3(256), 0, s, a);
  else if (a.subchannel == 128) hipLaunchKernelGGL((f6_ragged_sub_bwd_kernel<MODE, 4>), grid, dim3(256), 0, s, a);
  else hipLaunchKernelGGL((f6_ragged_sub_bwd_kernel<MODE, 8>), grid, dim3(256), 0, s, a);
}
hipError_t launch_f6_ragged_sub_bwd(const RaggedBwdArgs& a, dim3 grid, hipStream_t s) {
  hipError_t err = bwd_grid(a, grid);
  // groups of 256 run two 128-K stages each
  if (err == hipSuccess) err = bwd_convert(a, round256(a.k_cap), a.subchannel > 128 ? 256 : 128, s);
  if (err != hipSuccess) return err;
  if (a.out_mode == OUT_I32) launch_ragged_sub_bwd<OUT_I32>(a, grid, s);
  else launch_ragged_sub_bwd<OUT_F32>(a, grid, s);
  return hipGetLastError();
}

shk_kernel_desc f6_ragged_desc(int family, int layout) {
  shk_kernel_desc d = desc_of<F6R>(family, layout, 1);
  d.num_stages = F6RE::P;
  d.lds_bytes = F6RE::LDS_BYTES + MFMA32_SCALE_BYTES;
  d.operand_format = SHK_OPERANDS_FP6;
  return d;
}

}  // namespace

Entry f6_ragged_fwd_entry(int layout) {
  return Entry{f6_ragged_desc(SHK_FAMILY_RAGGED_FWD, layout), nullptr, &launch_f6_ragged_fwd, nullptr, nullptr};
}
Entry f6_ragged_sub_fwd_entry(int layout) {
  shk_kernel_desc d = desc_of<F6RS>(SHK_FAMILY_RAGGED_FWD, layout, 1);
  d.min_subchannel = 32;
  d.max_subchannel = 256;
  d.num_stages = F6SubEngine<F6RS>::P;
  d.lds_bytes = f6_sub_lds_bytes<F6RS>();
  d.operand_format = SHK_OPERANDS_FP6;
  return Entry{d, nullptr, &launch_f6_ragged_sub_fwd, nullptr, nullptr};
}
Entry f6_ragged_sub_bwd_entry(int layout) {
  shk_kernel_desc d = desc_of<F6RS>(SHK_FAMILY_RAGGED_BWD, layout, 1);
  d.min_subchannel = 32;
  d.max_subchannel = 256;
  d.num_stages = F6SubEngine<F6RS>::P;
  d.lds_bytes = f6_sub_lds_bytes<F6RS>();
  d.operand_format = SHK_OPERANDS_FP6;
  return Entry{d, nullptr, nullptr, &launch_f6_ragged_sub_bwd, nullptr};
}
Entry f6_ragged_bwd_entry(int layout) {
  return Entry{f6_ragged_desc(SHK_FAMILY_RAGGED_BWD, layout), nullptr, nullptr, &launch_f6_ragged_bwd, nullptr};
}

unsigned long long f6_ragged_fwd_workspace(int m, int n, int k, int groups, bool subchannel) {
  const int kw = subchannel ? round256(k) : round128(k);
  return f6_operand_bytes(round32(m), kw) + (unsigned long long)groups * f6_operand_bytes(round32(n), kw);
}
unsigned long long f6_ragged_bwd_workspace(int m, int n, int k_cap, int groups, bool subchannel) {
  const int kw = subchannel ? round256(k_cap) : round128(k_cap);
  return (unsigned long long)groups * (f6_operand_bytes(round32(m), kw) + f6_operand_bytes(round32(n), kw));
}

}  // namespace shk
