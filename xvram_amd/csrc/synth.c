/*
 * synth.c — seeded synthetic operands for the benchmark (libxvram_synth.so).
 *
 * Element e of a matrix with seed s is U[-1,1) = 2*(x>>40)*2^-24 - 1 with
 * x = splitmix64(splitmix64(s) ^ e), e = the element's column-major storage
 * index; N(0, sigma^2) uses Box-Muller on draws 2e and 2e+1 in FP64. Values
 * are exactly representable in FP32. The checker keeps an independent copy of
 * this definition; tests assert both produce identical bits.
 */
#include <math.h>
#include <stdint.h>

static inline uint64_t mix(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

static inline float uniform_at(uint64_t key, uint64_t e) {
  const uint64_t x = mix(key ^ e);
  return (float)(2.0 * (double)(x >> 40) * 0x1p-24 - 1.0);
}

/* out[i] = U(first + i), i < count. */
void synth_fill_uniform(float* out, uint64_t count, uint64_t seed, uint64_t first) {
  const uint64_t key = mix(seed);
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < (int64_t)count; ++i) out[i] = uniform_at(key, first + (uint64_t)i);
}

/* out[r + c*rows] = U(first + r*row_stride + c*col_stride): a strided sample
 * (e.g. a block of rows of a column-major matrix). */
void synth_fill_uniform_strided(float* out, uint64_t rows, uint64_t cols, uint64_t seed,
                                uint64_t first, uint64_t row_stride, uint64_t col_stride) {
  const uint64_t key = mix(seed);
#pragma omp parallel for schedule(static)
  for (int64_t c = 0; c < (int64_t)cols; ++c)
    for (uint64_t r = 0; r < rows; ++r)
      out[r + (uint64_t)c * rows] = uniform_at(key, first + r * row_stride + (uint64_t)c * col_stride);
}

void synth_fill_normal(float* out, uint64_t count, uint64_t seed, uint64_t first, double sigma) {
  const uint64_t key = mix(seed);
  const double two_pi = 6.283185307179586476925286766559;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < (int64_t)count; ++i) {
    const uint64_t e = first + (uint64_t)i;
    const uint64_t x1 = mix(key ^ (2u * e));
    const uint64_t x2 = mix(key ^ (2u * e + 1u));
    const double u1 = ((double)(x1 >> 11) + 1.0) * 0x1p-53;
    const double u2 = (double)(x2 >> 11) * 0x1p-53;
    out[i] = (float)(sigma * sqrt(-2.0 * log(u1)) * cos(two_pi * u2));
  }
}

/* The analytic integer pattern of the reference's GEMM benchmark
 * (src/gemm_bench/pattern.cpp:207-237): A(i,k) = 1 + i%3 + k%2 and
 * B(k,j) = 1 + j%5 + k%3, whose product is exact in FP32 while 28*K < 2^24.
 * These fill columns [col0, col0 + cols) of the operand as stored column-major
 * with `rows` rows (out[x + c*rows] is stored element (x, col0 + c)); a
 * transposed operand is stored as its transpose (op T). */
void synth_fill_pattern_a(float* out, uint64_t rows, uint64_t cols, uint64_t col0, int transposed) {
#pragma omp parallel for schedule(static)
  for (int64_t c = 0; c < (int64_t)cols; ++c) {
    const uint64_t y = col0 + (uint64_t)c;
    float* col = out + (uint64_t)c * rows;
    for (uint64_t x = 0; x < rows; ++x)
      col[x] = transposed ? (float)(1 + y % 3 + x % 2) : (float)(1 + x % 3 + y % 2);
  }
}

void synth_fill_pattern_b(float* out, uint64_t rows, uint64_t cols, uint64_t col0, int transposed) {
#pragma omp parallel for schedule(static)
  for (int64_t c = 0; c < (int64_t)cols; ++c) {
    const uint64_t y = col0 + (uint64_t)c;
    float* col = out + (uint64_t)c * rows;
    for (uint64_t x = 0; x < rows; ++x)
      col[x] = transposed ? (float)(1 + x % 5 + y % 3) : (float)(1 + y % 5 + x % 3);
  }
}
