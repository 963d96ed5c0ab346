/*
 * CPU oracle (test infrastructure only): plain-C restatement of the
 * reference's torch numerical path for the dense quantized GEMM.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this
 * library; the product never does.
 *
 *   oracle_matmul_i8   exact int32 C = A @ B of int8 matrices
 *                      (torch.matmul on int32 operands, api.py:304 / :319).
 *   oracle_dense_int4_nn
 *                      the whole per-channel or subchannel path of
 *                      reference_mm (api.py:257-325) for packed int4 NN
 *                      operands: unpack (quant.py:41-51) -> int32 matmul ->
 *                      (float(acc) * a_scale) * b_scale (per-channel,
 *                      api.py:304-309) or the ordered per-group
 *                      scale-accumulate (api.py:311-325) -> ReLU2 / none
 *                      (api.py:290-291) -> bf16 round-to-nearest-even
 *                      (api.py:292-293).
 * Built with -ffp-contract=off so no multiply is fused with an add.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

static void set_threads(int threads) {
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#else
  (void)threads;
#endif
}

/* Sign-extends the nibbles of a packed K-major row: byte j holds element 2j
 * in its low nibble and 2j+1 in its high nibble (quant.py:32-38). */
static void unpack_row(const uint8_t* src, int kbytes, int8_t* dst) {
  for (int j = 0; j < kbytes; ++j) {
    const int lo = src[j] & 0xF;
    const int hi = (src[j] >> 4) & 0xF;
    dst[2 * j] = (int8_t)(lo >= 8 ? lo - 16 : lo);
    dst[2 * j + 1] = (int8_t)(hi >= 8 ? hi - 16 : hi);
  }
}

static inline int32_t dot_i8(const int8_t* a, const int8_t* b, int k) {
  int32_t s = 0;
  for (int i = 0; i < k; ++i) s += (int32_t)a[i] * (int32_t)b[i];
  return s;
}

static inline float bf16_to_f32(uint16_t h) {
  uint32_t u = ((uint32_t)h) << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static inline uint16_t f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

/* c[M,N] = a[M,K] @ b[K,N], int8 operands row-major, exact int32. */
void oracle_matmul_i8(const int8_t* a, const int8_t* b, int32_t* c, int m, int n, int k, int threads) {
  set_threads(threads);
  int8_t* bt = (int8_t*)malloc((size_t)n * (size_t)k);
  for (int kk = 0; kk < k; ++kk)
    for (int j = 0; j < n; ++j) bt[(size_t)j * k + kk] = b[(size_t)kk * n + j];
#pragma omp parallel for schedule(static)
  for (int i = 0; i < m; ++i)
    for (int j = 0; j < n; ++j) c[(size_t)i * n + j] = dot_i8(a + (size_t)i * k, bt + (size_t)j * k, k);
  free(bt);
}

/*
 * Full dense path for packed int4 NN operands: a[M, K/2], b[K/2, N] (uint8),
 * bf16 scales (per-channel a_scale[M], b_scale[N]; subchannel S > 0:
 * a_scale[M, ceil(K/S)], b_scale[ceil(K/S), N]), epilogue 0 = none,
 * 1 = relu2.  Writes bf16 bits to out[M, N].  Rows [row0, row0 + rows) only,
 * so callers can time a bounded slice.
 */
void oracle_dense_int4_nn(const uint8_t* a, const uint8_t* b, const uint16_t* a_scale, const uint16_t* b_scale,
                          uint16_t* out, int m, int n, int k, int subchannel, int epilogue, int row0, int rows,
                          int threads) {
  set_threads(threads);
  const int kb = k / 2;
  int8_t* bt = (int8_t*)malloc((size_t)n * (size_t)k);
  /* unpack B column-wise into K-contiguous rows */
  {
    int8_t* col = (int8_t*)malloc((size_t)k);
    uint8_t* packed = (uint8_t*)malloc((size_t)kb);
    for (int j = 0; j < n; ++j) {
      for (int p = 0; p < kb; ++p) packed[p] = b[(size_t)p * n + j];
      unpack_row(packed, kb, col);
      memcpy(bt + (size_t)j * k, col, (size_t)k);
    }
    free(col);
    free(packed);
  }
  const int scale_cols = subchannel > 0 ? (k + subchannel - 1) / subchannel : 1;
  if (row0 < 0) row0 = 0;
  if (row0 + rows > m) rows = m - row0;
#pragma omp parallel
  {
    int8_t* arow = (int8_t*)malloc((size_t)k);
#pragma omp for schedule(static)
    for (int i = row0; i < row0 + rows; ++i) {
      unpack_row(a + (size_t)i * kb, kb, arow);
      for (int j = 0; j < n; ++j) {
        const int8_t* bj = bt + (size_t)j * k;
        float v;
        if (subchannel <= 0) {
          v = (float)dot_i8(arow, bj, k);
          v = v * bf16_to_f32(a_scale[i]);
          v = v * bf16_to_f32(b_scale[j]);
        } else {
          v = 0.0f;
          for (int g = 0; g < scale_cols; ++g) {
            const int k0 = g * subchannel;
            const int k1 = k0 + subchannel < k ? k0 + subchannel : k;
            float p = (float)dot_i8(arow + k0, bj + k0, k1 - k0);
            p = p * bf16_to_f32(a_scale[(size_t)i * scale_cols + g]);
            p = p * bf16_to_f32(b_scale[(size_t)g * n + j]);
            v = v + p;
          }
        }
        if (epilogue == 1) {
          v = v > 0.0f ? v : 0.0f;
          v = v * v;
        }
        out[(size_t)i * n + j] = f32_to_bf16(v);
      }
    }
    free(arow);
  }
  free(bt);
}

int oracle_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
