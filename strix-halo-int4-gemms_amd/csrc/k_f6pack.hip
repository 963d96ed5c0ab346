// Operand conversion of the fp6 GEMM path: packed int4 (either layout) to
// the block format of shk_f6.h.  Compiled apart from the GEMM, with the
// default scheduler.
#include "shk_table.h"

namespace shk {
namespace {

// 16 packed int4 bytes -> the lane's 24 fp6 bytes.  x ^ 0x8 per nibble is
// the offset-binary value v + 8; 0x6400 | (v + 8) is the f16 1024 + v + 8;
// subtracting 1032 and scaling by 1/8 gives v/8 exactly (f16 holds both
// steps exactly), and v/8 is exact in e2m3.
__device__ __forceinline__ v6i f6_convert(const uint4& x) {
  f6_h32 h;
  const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint32_t u = w[q] ^ 0x88888888u;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t d = ((u >> (4 * j)) & 0x000F000Fu) | 0x64006400u;
      f6_h2 v = __builtin_bit_cast(f6_h2, d) - f6_h2{(_Float16)1032.0f, (_Float16)1032.0f};
      v = v * f6_h2{(_Float16)0.125f, (_Float16)0.125f};
      h[8 * q + 2 * j] = v.x;
      h[8 * q + 2 * j + 1] = v.y;
    }
  }
  return __builtin_bit_cast(v6i, __builtin_amdgcn_cvt_scalef32_pk32_fp6_f16(h, 1.0f));
}

// write_through (uniform): the stores carry SC1, so the block's lines go to
// memory as they are written instead of at the end of the kernel.
__device__ __forceinline__ void f6_store_lane(uint8_t* block, int lane, const v6i& y, bool write_through) {
  if (write_through) {
    const v4i lo = v4i{y[0], y[1], y[2], y[3]};
    const v2i hi = v2i{y[4], y[5]};
    asm volatile("global_store_dwordx4 %0, %1, off sc1" : : "v"(block + 16 * lane), "v"(lo) : "memory");
    asm volatile("global_store_dwordx2 %0, %1, off sc1" : : "v"(block + 1024 + 8 * lane), "v"(hi) : "memory");
    return;
  }
  *reinterpret_cast<uint4*>(block + 16 * lane) = make_uint4(y[0], y[1], y[2], y[3]);
  *reinterpret_cast<uint2*>(block + 1024 + 8 * lane) = make_uint2(y[4], y[5]);
}

// Source row of packed row r.  For SwiGLU B the packed rows of each 256-row
// tile (output columns 128t .. 128t+127) are, per 128-row half h (one wave
// column of the GEMM tile), 64 up columns followed by the same 64 gate
// columns: 128t + 64h + q (q < 64) and N + 128t + 64h + q - 64.
__device__ __forceinline__ int f6_src_row(int r, int swiglu_n) {
  if (swiglu_n == 0) return r;
  const int t = r >> 8, h = (r >> 7) & 1, q = r & 127;
  return 128 * t + 64 * h + (q & 63) + (q >= 64 ? swiglu_n : 0);
}

// Logical K length of operand g.
__device__ __forceinline__ int f6_k_len(const F6PackArgs& p, int g) {
  if (p.k_len == nullptr) return p.k_cap;
  const int l = p.k_len[g];
  return l < 0 ? 0 : (l > p.k_cap ? p.k_cap : l);
}
// 16 source bytes of which the first `valid` (>= 1) exist, in pieces of
// `unit` bytes (16, 8 or 1: the alignment of the source): 16-byte pieces
// are whole by construction, the second 8-byte half exists when more than
// 8 bytes do, and single bytes past `valid` are not read.
__device__ __forceinline__ uint4 f6_load(const uint8_t* q, int unit, int valid) {
  if (unit == 16) return *reinterpret_cast<const uint4*>(q);
  if (unit == 8) {
    const uint2 lo = *reinterpret_cast<const uint2*>(q);
    const uint2 hi = valid > 8 ? *reinterpret_cast<const uint2*>(q + 8) : make_uint2(0u, 0u);
    return make_uint4(lo.x, lo.y, hi.x, hi.y);
  }
  uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int b = 0; b < 16; ++b)
    if (b < valid) w[b / 4] |= (uint32_t)q[b] << (8 * (b % 4));
  return make_uint4(w[0], w[1], w[2], w[3]);
}
// 64-K blocks that the GEMM reads for K length `len`: whole stages of
// p.k_stage K (128, or 256 for the subchannel tile's groups of 256).
__device__ __forceinline__ int f6_blocks_read(const F6PackArgs& p, int len) {
  return p.k_stage == 256 ? 4 * ((len + 255) / 256) : 2 * ((len + 127) / 128);
}
// bytes of one MN-major source tile in LDS: 32 K rows x 256 packed rows
constexpr int F6_KTILE = 32 * 256;

// Blocks per wave (K-major: F6PackArgs::kmajor_blocks, 1 or 2) and 64-K
// blocks per workgroup (MN-major), with every load of a wave issued before
// its first conversion.  Measured on the C2 operands (8192 x 8192): one
// block per K-major wave runs at the speed of a device copy of the same
// bytes (two per wave: the C2 call 0.6% slower, four: 3%), while two 64-K
// blocks per MN-major workgroup are 19% faster than one when the source is
// cache-resident and equal from HBM.  The ragged calls' conversions take two
// blocks per K-major wave: the C5 forward call 34.3 -> 33.1 us (A/B, one
// box), with a third fewer workgroups to dispatch.
constexpr int kKW = 2;

// K-major source (row r holds its K values contiguously, two per byte): a
// wave converts NB consecutive blocks (panel-major order, so mostly the
// same panel's next 64-K blocks); a lane loads its 16 source bytes of each
// directly.  Nibble j of a little-endian source word is K value 8w + j of
// its 32, so K values at or past the operand's length are cleared word by
// word.
template <int NB>
__device__ __forceinline__ void pack_kmajor_nb(const F6PackArgs& p, int wg) {
  constexpr int kNB = NB;
  const int lane = threadIdx.x & 63;
  const long blocks = (long)f6_panels(p.rows) * p.kb;
  const long per_group = (blocks + 4 * kNB - 1) / (4 * kNB);
  const int g = (int)(wg / per_group);
  const long first = ((wg - (long)g * per_group) * 4 + (threadIdx.x >> 6)) * kNB;
  if (first >= blocks) return;
  const int len = f6_k_len(p, g);
  const int nread = f6_blocks_read(p, len);
  const uint8_t* src = p.src + g * p.src_group;
  int panel = (int)(first / p.kb);
  int kb = (int)(first - (long)panel * p.kb);
  uint4 x[kNB];
  bool live[kNB];
#pragma unroll
  for (int b = 0; b < kNB; ++b) {
    live[b] = first + b < blocks && kb < nread;
    x[b] = make_uint4(0u, 0u, 0u, 0u);
    const int r = 32 * panel + (lane & 31);
    const int k0 = 64 * kb + 32 * (lane >> 5);
    if (live[b] && r < p.rows && k0 < len) {
      const uint8_t* q = src + (long)f6_src_row(r, p.swiglu_n) * p.ld + 32L * kb + 16 * (lane >> 5);
      const int keep = len - k0;  // K values of the 32 to keep
      // bytes holding any of them (the source row ends within the length)
      x[b] = f6_load(q, p.vec, (keep + 1) / 2);
      if (keep < 32) {
        uint32_t w[4] = {x[b].x, x[b].y, x[b].z, x[b].w};
#pragma unroll
        for (int wq = 0; wq < 4; ++wq) {
          const int c = keep - 8 * wq;
          w[wq] &= c >= 8 ? 0xFFFFFFFFu : (c <= 0 ? 0u : (1u << (4 * c)) - 1u);
        }
        x[b] = make_uint4(w[0], w[1], w[2], w[3]);
      }
    }
    if (++kb == p.kb) kb = 0, ++panel;
  }
  uint8_t* dst = p.dst + g * p.dst_group + first * F6_BLOCK;
#pragma unroll
  for (int b = 0; b < kNB; ++b)
    if (live[b]) f6_store_lane(dst + b * F6_BLOCK, lane, f6_convert(x[b]), p.write_through);
}

__device__ __forceinline__ void pack_kmajor(const F6PackArgs& p, int wg) {
  if (p.kmajor_blocks == 2) pack_kmajor_nb<2>(p, wg);
  else pack_kmajor_nb<1>(p, wg);
}

// MN-major source (K row kp holds two K values of every packed row, one per
// nibble, the even one low): a workgroup converts the blocks of one 256-row
// tile and kKW consecutive 64-K blocks.  Each 32 x 256-byte source tile goes
// through LDS in the MN-major ring layout of the DMA engine, whose
// transposing reads hand each lane its row's bytes in K order: within a
// 16-lane group, lane i addresses source row kp + i/2 at byte 8*(i%2) of a
// 16-row unit and receives the 8 bytes of those 8 rows in column i.  Units
// past the rows and K rows past the length load as zeros; panels past the
// rows and 64-K blocks the GEMM does not read are not stored.
__device__ __forceinline__ void pack_mnmajor(const F6PackArgs& p, int wg, uint8_t* tile) {
  const int tiles = (p.rows + F6_TILE - 1) / F6_TILE;
  const int kgroups = (p.kb + kKW - 1) / kKW;
  const int per_group = tiles * kgroups;
  const int g = wg / per_group;
  const int local = wg - g * per_group;
  const int t = local / kgroups;
  const int kb0 = (local - t * kgroups) * kKW;
  const int len = f6_k_len(p, g);
  const int nread = min(f6_blocks_read(p, len), p.kb);
  if (kb0 >= nread) return;  // uniform over the workgroup
  const int tid = threadIdx.x;
  const int u = tid & 15;  // 16-row unit of the tile
  const int r0 = F6_TILE * t + 16 * u;
  const long col = f6_src_row(r0, p.swiglu_n);
  const uint8_t* src = p.src + g * p.src_group;
  uint4 x[kKW][2];
#pragma unroll
  for (int w = 0; w < kKW; ++w)
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int kb = kb0 + w;
      const int kp = 16 * q + (tid >> 4);
      const int k = 2 * (32 * kb + kp);  // K of the low nibbles
      x[w][q] = make_uint4(0u, 0u, 0u, 0u);
      if (kb < nread && r0 < p.rows && k < len) {
        x[w][q] = f6_load(src + (32L * kb + kp) * p.ld + col, p.vec, p.rows - r0);
        if (k + 1 >= len)
          x[w][q] = make_uint4(x[w][q].x & 0x0F0F0F0Fu, x[w][q].y & 0x0F0F0F0Fu, x[w][q].z & 0x0F0F0F0Fu,
                               x[w][q].w & 0x0F0F0F0Fu);
      }
    }
#pragma unroll
  for (int w = 0; w < kKW; ++w)
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int kp = 16 * q + (tid >> 4);
      const int swz = (kp & 7) | ((kp & 16) >> 1);
      *reinterpret_cast<uint4*>(tile + w * F6_KTILE + kp * 256 + 16 * (u ^ swz)) = x[w][q];
    }
  __syncthreads();
  // lane l of a block: packed row 32b + l % 32 (unit 2b + (l/16) % 2, column
  // l % 16 of it), K rows 16*(l/32) + [0, 16)
  const int lane = tid & 63;
  const int i = lane & 15;
  const int kp = 16 * (lane >> 5) + i / 2;
  const int swz = (kp & 7) | ((kp & 16) >> 1);
  const int panels = f6_panels(p.rows);
  uint8_t* dst = p.dst + g * p.dst_group;
#pragma unroll
  for (int w = 0; w < kKW; ++w) {
    const int kb = kb0 + w;
    if (kb >= nread) break;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int b = 2 * (tid >> 6) + c;
      if (8 * t + b >= panels) continue;
      const int unit = 2 * b + ((lane >> 4) & 1);
      const uint8_t* q = tile + w * F6_KTILE + kp * 256 + 16 * (unit ^ swz) + 8 * (i & 1);
      const v2i lo = ds_read_tr8(q);
      const v2i hi = ds_read_tr8(q + 2048);
      const uint4 y = make_uint4(lo.x, lo.y, hi.x, hi.y);
      const long blk = (long)(8 * t + b) * p.kb + kb;
      f6_store_lane(dst + blk * F6_BLOCK, lane, f6_convert(y), p.write_through);
    }
  }
}

// Workgroups of one operand batch: per operand, one per 256-row tile and kKW
// 64-K blocks (MN-major) or per 4 * NB blocks (K-major: NB per wave).
long pack_groups(const F6PackArgs& a, bool mn_major) {
  const int nb = a.kmajor_blocks == 2 ? 2 : 1;
  const long per = mn_major ? (long)((a.rows + F6_TILE - 1) / F6_TILE) * ((a.kb + kKW - 1) / kKW)
                            : ((long)f6_panels(a.rows) * a.kb + 4 * nb - 1) / (4 * nb);
  return per * a.groups;
}

__global__ __launch_bounds__(256) void f6_pack_one(const F6PackArgs p, int mn_major) {
  __shared__ __attribute__((aligned(16))) uint8_t tile[kKW * F6_KTILE];
  if (mn_major) pack_mnmajor(p, blockIdx.x, tile);
  else pack_kmajor(p, blockIdx.x);
}

// Both operands of a call in one launch: workgroups [0, a_groups) convert
// A, the rest B, or with `interleave` the two alternate in proportion
// (workgroup w converts B when floor((w + 1) gb / T) passes floor(w gb / T),
// T = ga + gb), so that both operands' streams share the memory system over
// the whole launch.  On C2 (8192 A blocks of 4 waves, then 2048 MN-major B
// tiles) A-then-B took 35 us of workgroup span, the B tiles ~22 us of it at
// ~3.6 TB/s; interleaved, 29 us (the C2 call 2% faster).  The subchannel
// and ragged calls keep A then B: interleaved, the C3 call was 0.5-0.8%
// slower, the C5 forward 3 us and the C5 backward ~1.4 us.  With a task job, workgroup
// 0 (dispatched first) builds the task list in the tile's LDS and the
// conversion shifts up by one.
__global__ __launch_bounds__(256) void f6_pack_two(const F6PackArgs a, const F6PackArgs b, int a_mn, int b_mn,
                                                   int a_groups, const TaskJob job, int interleave) {
  __shared__ __attribute__((aligned(16))) uint8_t tile[kKW * F6_KTILE];
  static_assert(sizeof(int) * (2 * (kFusedTaskGroups + 1) + 4) <= sizeof(tile), "task arrays fit the tile");
  int wg = blockIdx.x;
  if (job.sizes != nullptr) {
    if (wg == 0) {
      int* starts = reinterpret_cast<int*>(tile);
      build_task_list<256>(job, starts, starts + kFusedTaskGroups + 1, starts + 2 * (kFusedTaskGroups + 1));
      return;
    }
    --wg;
  }
  const long long total = (long long)gridDim.x - (job.sizes != nullptr ? 1 : 0);
  const long long gb = total - a_groups;
  // B workgroups before this one
  const long long before = interleave ? (long long)wg * gb / total : (wg < a_groups ? 0 : wg - a_groups);
  if (interleave ? (long long)(wg + 1) * gb / total > before : wg >= a_groups) {
    if (b_mn) pack_mnmajor(b, (int)before, tile);
    else pack_kmajor(b, (int)before);
  } else {
    if (a_mn) pack_mnmajor(a, wg - (int)before, tile);
    else pack_kmajor(a, wg - (int)before);
  }
}

}  // namespace

hipError_t launch_f6_pack(const F6PackArgs& a, bool mn_major, hipStream_t s) {
  const long n = pack_groups(a, mn_major);
  if (n <= 0) return hipSuccess;
  if (n > 0x7FFFFFFFL) return hipErrorInvalidValue;
  hipLaunchKernelGGL(f6_pack_one, dim3((unsigned)n), dim3(256), 0, s, a, (int)mn_major);
  return hipGetLastError();
}

hipError_t launch_f6_pack2(const F6PackArgs& a, bool a_mn, const F6PackArgs& b, bool b_mn, hipStream_t s,
                           const TaskJob* job, bool interleave) {
  const long ga = pack_groups(a, a_mn), gb = pack_groups(b, b_mn);
  const bool with_job = job != nullptr && job->sizes != nullptr;
  if (with_job && (job->groups > kFusedTaskGroups || job->groups < 0)) return hipErrorInvalidValue;
  const long total = ga + gb + (with_job ? 1 : 0);
  if (total <= 0) return hipSuccess;
  if (total > 0x7FFFFFFFL) return hipErrorInvalidValue;
  const TaskJob none{nullptr, 0, 1, 1, 0, nullptr, nullptr, nullptr};
  hipLaunchKernelGGL(f6_pack_two, dim3((unsigned)total), dim3(256), 0, s, a, b, (int)a_mn, (int)b_mn, (int)ga,
                     with_job ? *job : none, (int)interleave);
  return hipGetLastError();
}

}  // namespace shk
