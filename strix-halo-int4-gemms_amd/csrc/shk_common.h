// Shared device helpers for the gfx950 quantized GEMM kernels.
//
// Operand tiles live in LDS as int8, "chunk-major": a stage buffer for an
// operand of ROWS rows and BK logical K values holds BK/16 chunk planes; plane c
// holds, for every row r, the 16 int8 values of K range [16c, 16c+16) of that
// row.  Inside a plane the row index is XOR-swizzled with (c & 7) so that the
// 16 lanes of an MFMA fragment read (16 consecutive rows, one chunk) and the
// transposing stager's writes (8 chunks x 2 row groups) both land on distinct
// 16-byte bank groups.
//
// Packed int4 (two's-complement nibbles, low nibble = even K, high nibble = odd
// K, as produced by the reference's quant.pack_int4_k_major, quant.py:32-38) is
// widened to int8 as 16*v: (byte << 4) & 0xF0 for the even element and
// byte & 0xF0 for the odd one.  Both operands carry the factor 16, so the int32
// MFMA accumulator holds 256 * sum(a*b); the epilogue divides it out exactly.
// Inside one 16-value chunk built from packed bytes p0..p7 the K order is
// [lo(p0..p3), hi(p0..p3), lo(p4..p7), hi(p4..p7)]; both operands use the same
// order, so every chunk still contracts exactly its 16 logical K values.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace shk {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// Byte shuffles

__device__ __forceinline__ uint32_t perm_b32(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

// 4x4 byte transpose: r[i].byte[j] -> x[j].byte[i].
__device__ __forceinline__ void transpose4x4(uint32_t r0, uint32_t r1, uint32_t r2, uint32_t r3,
                                             uint32_t& x0, uint32_t& x1, uint32_t& x2,
                                             uint32_t& x3) {
  const uint32_t t0 = perm_b32(r1, r0, 0x05010400u);  // r0.b0 r1.b0 r0.b1 r1.b1
  const uint32_t t1 = perm_b32(r1, r0, 0x07030602u);  // r0.b2 r1.b2 r0.b3 r1.b3
  const uint32_t t2 = perm_b32(r3, r2, 0x05010400u);  // r2.b0 r3.b0 r2.b1 r3.b1
  const uint32_t t3 = perm_b32(r3, r2, 0x07030602u);  // r2.b2 r3.b2 r2.b3 r3.b3
  x0 = perm_b32(t2, t0, 0x05040100u);
  x1 = perm_b32(t2, t0, 0x07060302u);
  x2 = perm_b32(t3, t1, 0x05040100u);
  x3 = perm_b32(t3, t1, 0x07060302u);
}

// Packed int4 dword (4 bytes = 8 K values) -> two int8x4 dwords holding 16*v.
__device__ __forceinline__ uint32_t nib_lo16(uint32_t w) { return (w << 4) & 0xF0F0F0F0u; }
__device__ __forceinline__ uint32_t nib_hi16(uint32_t w) { return w & 0xF0F0F0F0u; }

// 8 packed bytes (w0 = p0..p3, w1 = p4..p7) -> one 16-value int8 chunk.
__device__ __forceinline__ uint4 widen_chunk(uint32_t w0, uint32_t w1) {
  return make_uint4(nib_lo16(w0), nib_hi16(w0), nib_lo16(w1), nib_hi16(w1));
}

// ---------------------------------------------------------------------------
// LDS addressing (byte offsets inside one operand stage buffer)

template <int ROWS>
__device__ __forceinline__ uint32_t lds_chunk_off(int row, int chunk) {
  return (uint32_t)((chunk * ROWS + (row ^ (chunk & 7))) * 16);
}

// ---------------------------------------------------------------------------
// bf16

// fp32 -> bf16 round-to-nearest-even (the conversion torch's .to(bfloat16)
// performs); NaN maps to the canonical quiet NaN 0x7FC0.
__device__ __forceinline__ uint32_t f32_to_bf16_rne(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

// Two fp32 values -> packed bf16 pair with v_cvt_pk_bf16_f32 (round to
// nearest even, subnormals kept).  Only for values that are not NaN: the
// instruction keeps a NaN's payload where torch writes 0x7FC0.
typedef float shk_f2 __attribute__((ext_vector_type(2)));
typedef __bf16 shk_bf2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2_nonan(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(shk_f2{a, b}, shk_bf2));
}

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
  return __uint_as_float(((uint32_t)b) << 16);
}

__device__ __forceinline__ float load_bf16(const uint16_t* p) { return bf16_bits_to_f32(*p); }

// ---------------------------------------------------------------------------
// MFMA

// D = X * Y^T over 64 int8 K values: X rows -> D rows (4 per lane group),
// Y rows -> D columns (lane % 16).
__device__ __forceinline__ v4i mfma64(const v4i& x, const v4i& y, const v4i& acc) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(x, y, acc, 0, 0, 0);
}

// Same with 32 K values per instruction (used when a subchannel group is 32 wide).
__device__ __forceinline__ v4i mfma32(const v2i& x, const v2i& y, const v4i& acc) {
  long xl = __builtin_bit_cast(long, x);
  long yl = __builtin_bit_cast(long, y);
  return __builtin_amdgcn_mfma_i32_16x16x32_i8(xl, yl, acc, 0, 0, 0);
}

__device__ __forceinline__ int ceil_div(int a, int b) { return (a + b - 1) / b; }

}  // namespace shk
