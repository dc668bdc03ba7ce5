/*
 * vbsr_oracle.c -- CPU restatement of the reference VBSR algorithms.
 *
 * TEST INFRASTRUCTURE ONLY (see vbsr_oracle.h): the checker for the product
 * library, never part of it.
 *
 * Compiled with -ffp-contract=off so that no multiply-add below is fused
 * unless it is written as fmaf().
 *
 * Parity pins per function (tests/ hold the checks):
 *   orc_mt64_* / orc_mt32_*   C++ standard known answers ([rand.predef]) and
 *                             libstdc++'s std::mt19937(_64) streams.
 *   orc_uniform_pm1_*         libstdc++ generate_canonical<float,24> +
 *                             uniform_real_distribution<float>::operator()
 *                             (bits/random.tcc, bits/random.h of GCC 11), the
 *                             library routine the reference's generator calls.
 *   orc_generate              reference CSV fingerprints (sum of h*w per
 *                             instance) for 4 distributions x 2 localities x
 *                             4 degrees x 6 (rows, seed) pairs.
 *   orc_validate              reference negative tests + rule-by-rule cases.
 *   orc_cpu_reference         brute force on dense expansions, closed forms
 *                             (identity blocks, unit-vector B, linearity,
 *                             degree-1 batched GEMM).
 *   orc_cpu_reference_threads bit-identical to orc_cpu_reference (each
 *                             row's arithmetic is unchanged; rows run in
 *                             parallel).
 *   orc_abs_product_sum(_threads)  the dense product of |A| and |B|
 *                             (brute force); the threaded form bit-identical
 *                             to the serial one.
 *   orc_fmaf_order            same checks as orc_cpu_reference within fp32
 *                             tolerance, plus closed forms whose bits differ
 *                             with k order, block order and fusion (one row
 *                             summing 2^24, 1, -2^24 gives 0 only in order;
 *                             -(1+2^-11) + (1+2^-12)^2 gives 2^-24 only
 *                             fused and in order); bit-exact emulation pins
 *                             the GPU order-preserving kernel.
 *   orc_make_random_input     C++ standard known answer for mt19937 and
 *                             libstdc++'s stream.
 */
#include "vbsr_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---- mt19937_64 ([rand.predef]: w=64 n=312 m=156 r=31) ------------------ */

#define MT64_N 312
#define MT64_M 156
#define MT64_UPPER 0xFFFFFFFF80000000ULL
#define MT64_LOWER 0x000000007FFFFFFFULL

void orc_mt64_seed(orc_mt64* e, uint64_t seed) {
  e->state[0] = seed;
  for (int i = 1; i < MT64_N; ++i) {
    const uint64_t prev = e->state[i - 1];
    e->state[i] = 6364136223846793005ULL * (prev ^ (prev >> 62)) + (uint64_t)i;
  }
  e->index = MT64_N;
}

static void mt64_twist(orc_mt64* e) {
  for (int i = 0; i < MT64_N; ++i) {
    const uint64_t y = (e->state[i] & MT64_UPPER) | (e->state[(i + 1) % MT64_N] & MT64_LOWER);
    uint64_t next = e->state[(i + MT64_M) % MT64_N] ^ (y >> 1);
    if (y & 1ULL) next ^= 0xB5026F5AA96619E9ULL;
    e->state[i] = next;
  }
  e->index = 0;
}

uint64_t orc_mt64_next(orc_mt64* e) {
  if (e->index >= MT64_N) mt64_twist(e);
  uint64_t z = e->state[e->index++];
  z ^= (z >> 29) & 0x5555555555555555ULL;
  z ^= (z << 17) & 0x71D67FFFEDA60000ULL;
  z ^= (z << 37) & 0xFFF7EEE000000000ULL;
  z ^= z >> 43;
  return z;
}

/* ---- mt19937 ([rand.predef]: w=32 n=624 m=397 r=31) --------------------- */

#define MT32_N 624
#define MT32_M 397

void orc_mt32_seed(orc_mt32* e, uint32_t seed) {
  e->state[0] = seed;
  for (int i = 1; i < MT32_N; ++i) {
    const uint32_t prev = e->state[i - 1];
    e->state[i] = 1812433253U * (prev ^ (prev >> 30)) + (uint32_t)i;
  }
  e->index = MT32_N;
}

static void mt32_twist(orc_mt32* e) {
  for (int i = 0; i < MT32_N; ++i) {
    const uint32_t y = (e->state[i] & 0x80000000U) | (e->state[(i + 1) % MT32_N] & 0x7FFFFFFFU);
    uint32_t next = e->state[(i + MT32_M) % MT32_N] ^ (y >> 1);
    if (y & 1U) next ^= 0x9908B0DFU;
    e->state[i] = next;
  }
  e->index = 0;
}

uint32_t orc_mt32_next(orc_mt32* e) {
  if (e->index >= MT32_N) mt32_twist(e);
  uint32_t z = e->state[e->index++];
  z ^= z >> 11;
  z ^= (z << 7) & 0x9D2C5680U;
  z ^= (z << 15) & 0xEFC60000U;
  z ^= z >> 18;
  return z;
}

/* ---- uniform_real_distribution<float>(-1, 1) ----------------------------
 * libstdc++'s generate_canonical<float, 24> takes ceil(24 / log2(range))
 * = 1 engine output for both engines, converts it to float (round to
 * nearest), divides by float(range) (a power of two, exact) and maps a
 * result of 1 to nextafter(1, 0).  uniform_real_distribution then returns
 * u * (b - a) + a in float, i.e. u * 2 - 1. */

static float canonical_to_pm1(float u) {
  if (u >= 1.0f) u = nextafterf(1.0f, 0.0f);
  return u * 2.0f + -1.0f;
}

float orc_uniform_pm1_from_u64(uint64_t x) {
  const float sum = (float)x;
  const float range = 18446744073709551616.0f; /* 2^64 */
  return canonical_to_pm1(sum / range);
}

float orc_uniform_pm1_from_u32(uint32_t x) {
  const float sum = (float)x;
  const float range = 4294967296.0f; /* 2^32 */
  return canonical_to_pm1(sum / range);
}

/* ---- generator (src/format/generator.cpp:7-88) -------------------------- */

static int draw_block_size(orc_mt64* e, int32_t distribution) {
  static const int all_sizes[] = {8, 16, 24, 32, 40, 48, 56, 64};
  static const int low_sizes[] = {24, 32, 40};
  static const int bimodal_sizes[] = {8, 16, 48, 64};
  static const int two_sizes[] = {8, 64};
  switch (distribution) {
  case ORC_DIST_UNIFORM: return 32; /* generator.cpp:20-21: no draw */
  case ORC_DIST_LOW: return low_sizes[orc_mt64_next(e) % 3];
  case ORC_DIST_HIGH:
  case ORC_DIST_TIED_8_64: return all_sizes[orc_mt64_next(e) % 8];
  case ORC_DIST_BIMODAL: return bimodal_sizes[orc_mt64_next(e) % 4];
  case ORC_DIST_BIMODAL_8_64: return two_sizes[orc_mt64_next(e) % 2];
  default: return -1;
  }
}

void orc_matrix_free(orc_matrix* m) {
  if (!m) return;
  free(m->row_ptr);
  free(m->block_col);
  free(m->row_size);
  free(m->col_size);
  free(m->row_scalar_off);
  free(m->col_scalar_off);
  free(m->value_off);
  free(m->values);
  memset(m, 0, sizeof(*m));
}

static int cmp_int(const void* a, const void* b) {
  const int x = *(const int*)a, y = *(const int*)b;
  return (x > y) - (x < y);
}

static int generate_impl(int32_t R, int32_t C, int32_t degree, int32_t distribution,
                         int32_t locality, uint64_t seed, int store_values, orc_matrix* out) {
  memset(out, 0, sizeof(*out));
  /* generator.cpp:8-11 */
  if (degree < 1 || degree > 16 || R < 1 || C < 1 || degree > C) return ORC_INVALID;
  if (distribution < ORC_DIST_UNIFORM || distribution > ORC_DIST_TIED_8_64) return ORC_INVALID;
  if (locality < ORC_LOCALITY_RANDOM || locality > ORC_LOCALITY_CLAMPED) return ORC_INVALID;

  orc_mt64 e;
  orc_mt64_seed(&e, seed); /* generator.cpp:13 */

  const int64_t nnzb = (int64_t)R * degree;
  out->block_rows = R;
  out->block_cols = C;
  out->nnzb = nnzb;
  out->row_size = (int32_t*)malloc(sizeof(int32_t) * (size_t)R);
  out->col_size = (int32_t*)malloc(sizeof(int32_t) * (size_t)C);
  out->row_scalar_off = (int64_t*)malloc(sizeof(int64_t) * ((size_t)R + 1));
  out->col_scalar_off = (int64_t*)malloc(sizeof(int64_t) * ((size_t)C + 1));
  out->row_ptr = (int32_t*)malloc(sizeof(int32_t) * ((size_t)R + 1));
  out->block_col = (int32_t*)malloc(sizeof(int32_t) * (size_t)nnzb);
  out->value_off = (int64_t*)malloc(sizeof(int64_t) * ((size_t)nnzb + 1));
  if (!out->row_size || !out->col_size || !out->row_scalar_off || !out->col_scalar_off ||
      !out->row_ptr || !out->block_col || !out->value_off) {
    orc_matrix_free(out);
    return ORC_NOMEM;
  }

  /* Sizes: all rows first, then all columns (generator.cpp:37-42). */
  for (int32_t i = 0; i < R; ++i) out->row_size[i] = draw_block_size(&e, distribution);
  for (int32_t j = 0; j < C; ++j) {
    if (distribution == ORC_DIST_TIED_8_64 && j < R)
      out->col_size[j] = out->row_size[j];
    else
      out->col_size[j] = draw_block_size(&e, distribution);
  }

  /* Prefix sums (generator.cpp:44-52). */
  out->row_scalar_off[0] = 0;
  for (int32_t i = 0; i < R; ++i) out->row_scalar_off[i + 1] = out->row_scalar_off[i] + out->row_size[i];
  out->col_scalar_off[0] = 0;
  for (int32_t j = 0; j < C; ++j) out->col_scalar_off[j + 1] = out->col_scalar_off[j] + out->col_size[j];

  /* Growable value buffer: counts are known only once columns are drawn. */
  int64_t capacity = 1 << 16, count = 0;
  float* values = store_values ? (float*)malloc(sizeof(float) * (size_t)capacity) : NULL;
  if (store_values && !values) {
    orc_matrix_free(out);
    return ORC_NOMEM;
  }

  out->row_ptr[0] = 0;
  out->value_off[0] = 0;
  int64_t block = 0;
  for (int32_t i = 0; i < R; ++i) {
    int selected[16];
    int n = 0;
    /* Rejection sampling of distinct columns (generator.cpp:60-71). */
    while (n < degree) {
      int column;
      const uint64_t x = orc_mt64_next(&e);
      if (locality == ORC_LOCALITY_RANDOM) {
        column = (int)(x % (uint64_t)C);
      } else if (locality == ORC_LOCALITY_CYCLIC) {
        column = (i + (int)(x % (uint64_t)(2 * degree + 1)) - degree + C) % C;
      } else {
        /* The window's centre is the diagonal, held inside [0, C) so that a
         * window always holds at least `degree` distinct columns. */
        const int centre = i < C ? i : C - 1;
        column = centre + (int)(x % (uint64_t)(2 * degree + 1)) - degree;
        if (column < 0) column = 0;
        if (column > C - 1) column = C - 1;
      }
      int seen = 0;
      for (int s = 0; s < n; ++s) seen |= (selected[s] == column);
      if (!seen) selected[n++] = column;
    }
    qsort(selected, (size_t)n, sizeof(int), cmp_int); /* generator.cpp:72 */

    /* Values per block in sorted column order (generator.cpp:74-82). */
    for (int s = 0; s < n; ++s) {
      const int column = selected[s];
      out->block_col[block] = column;
      const int64_t value_count = (int64_t)out->row_size[i] * out->col_size[column];
      if (!store_values) {
        /* Consume the engine exactly as the value draws do. */
        for (int64_t v = 0; v < value_count; ++v) (void)orc_mt64_next(&e);
        count += value_count;
      } else if (count + value_count > capacity) {
        while (count + value_count > capacity) capacity *= 2;
        float* grown = (float*)realloc(values, sizeof(float) * (size_t)capacity);
        if (!grown) {
          free(values);
          orc_matrix_free(out);
          return ORC_NOMEM;
        }
        values = grown;
      }
      if (store_values)
        for (int64_t v = 0; v < value_count; ++v) values[count++] = orc_uniform_pm1_from_u64(orc_mt64_next(&e));
      out->value_off[block + 1] = out->value_off[block] + value_count;
      ++block;
    }
    out->row_ptr[i + 1] = (int32_t)block;
  }
  out->values = values;
  out->value_count = count;
  return ORC_OK;
}

int orc_generate(int32_t R, int32_t C, int32_t degree, int32_t distribution, int32_t locality,
                 uint64_t seed, orc_matrix* out) {
  return generate_impl(R, C, degree, distribution, locality, seed, 1, out);
}

int orc_generate_structure(int32_t R, int32_t C, int32_t degree, int32_t distribution,
                           int32_t locality, uint64_t seed, orc_matrix* out) {
  return generate_impl(R, C, degree, distribution, locality, seed, 0, out);
}

/* ---- validation (src/format/vbsr.cpp:29-82) ----------------------------- */
/* Rule codes: 1 block dims (:32-34), 2 metadata sizes (:35-38),
 * 3 scalar offset sizes (:39-42), 4 row_ptr ends (:43-45),
 * 5 value offsets (:46-49), 6 block row (:51-57), 7 block column (:58-64),
 * 8 block column index (:73-76), 9 block payload (:77-80). */

int orc_validate(const orc_view* v, int* rule) {
  int dummy;
  if (!rule) rule = &dummy;
  *rule = 0;
  const int64_t R = v->block_rows, C = v->block_cols;
  if (R <= 0 || C <= 0) { *rule = 1; return ORC_INVALID; }
  if (v->row_ptr_len != R + 1 || v->row_size_len != R || v->col_size_len != C) { *rule = 2; return ORC_INVALID; }
  if (v->row_scalar_off_len != R + 1 || v->col_scalar_off_len != C + 1) { *rule = 3; return ORC_INVALID; }
  if (v->row_ptr[0] != 0 || v->row_ptr[R] < 0 || (int64_t)v->row_ptr[R] != v->block_col_len) { *rule = 4; return ORC_INVALID; }
  if (v->value_off_len != v->block_col_len + 1 || v->value_off[0] != 0 ||
      v->value_off[v->value_off_len - 1] != v->values_len) { *rule = 5; return ORC_INVALID; }
  for (int64_t i = 0; i < R; ++i) {
    const int32_t h = v->row_size[i];
    if (v->row_ptr[i] > v->row_ptr[i + 1] || h < 8 || h > 64 || h % 8 != 0 ||
        v->row_scalar_off[i + 1] - v->row_scalar_off[i] != h) { *rule = 6; return ORC_INVALID; }
  }
  for (int64_t j = 0; j < C; ++j) {
    const int32_t w = v->col_size[j];
    if (w < 8 || w > 64 || w % 8 != 0 || v->col_scalar_off[j + 1] - v->col_scalar_off[j] != w) { *rule = 7; return ORC_INVALID; }
  }
  int64_t row = 0;
  for (int64_t b = 0; b < v->block_col_len; ++b) {
    while (v->row_ptr[row + 1] <= b) ++row;
    const int32_t column = v->block_col[b];
    if (column < 0 || column >= C) { *rule = 8; return ORC_INVALID; }
    const int64_t expected = (int64_t)v->row_size[row] * v->col_size[column];
    if (v->value_off[b + 1] - v->value_off[b] != expected) { *rule = 9; return ORC_INVALID; }
  }
  return ORC_OK;
}

/* ---- products ------------------------------------------------------------ */

static int64_t scalar_rows(const orc_view* a) { return a->row_scalar_off[a->block_rows]; }
static int64_t scalar_cols(const orc_view* a) { return a->col_scalar_off[a->block_cols]; }

/* src/format/vbsr.cpp:167-201 */
/* One block row of cpu_reference (vbsr.cpp:176-199): C's rows of block row i
 * are written by this call only. */
static void reference_row(const orc_view* a, const float* b, int32_t rhs, int64_t M, int64_t K, int32_t i,
                          float* c) {
  const int32_t h = a->row_size[i];
  for (int32_t blk = a->row_ptr[i]; blk < a->row_ptr[i + 1]; ++blk) {
    const int32_t col = a->block_col[blk];
    const int32_t w = a->col_size[col];
    const float* A = a->values + a->value_off[blk];
    for (int32_t r = 0; r < h; ++r) {
      for (int32_t n = 0; n < rhs; ++n) {
        const float* Bn = b + a->col_scalar_off[col] + (int64_t)n * K;
        double sum = 0.0;
        for (int32_t k = 0; k < w; ++k) sum += (double)A[r + (int64_t)k * h] * (double)Bn[k];
        c[a->row_scalar_off[i] + r + (int64_t)n * M] += (float)sum;
      }
    }
  }
}

int orc_cpu_reference(const orc_view* a, const float* b, int64_t b_len, int32_t rhs, float* c) {
  const int64_t M = scalar_rows(a), K = scalar_cols(a);
  if (b_len != K * rhs) return ORC_INVALID; /* :169-171 */
  memset(c, 0, sizeof(float) * (size_t)(M * rhs)); /* :175 */
  for (int32_t i = 0; i < a->block_rows; ++i) reference_row(a, b, rhs, M, K, i, c);
  return ORC_OK;
}

int orc_cpu_reference_threads(const orc_view* a, const float* b, int64_t b_len, int32_t rhs, int32_t threads,
                              float* c) {
  const int64_t M = scalar_rows(a), K = scalar_cols(a);
  if (b_len != K * rhs || threads < 1) return ORC_INVALID;
  memset(c, 0, sizeof(float) * (size_t)(M * rhs));
  const int32_t rows = a->block_rows;
#pragma omp parallel for schedule(dynamic, 16) num_threads(threads)
  for (int32_t i = 0; i < rows; ++i) reference_row(a, b, rhs, M, K, i, c);
  return ORC_OK;
}

/* Sum |a||b| of one block row's outputs (the elementwise error scale). */
static void abs_product_row(const orc_view* a, const float* b, int32_t rhs, int64_t M, int64_t K, int32_t i,
                            double* bound) {
  const int32_t h = a->row_size[i];
  for (int32_t blk = a->row_ptr[i]; blk < a->row_ptr[i + 1]; ++blk) {
    const int32_t col = a->block_col[blk];
    const int32_t w = a->col_size[col];
    const float* A = a->values + a->value_off[blk];
    for (int32_t r = 0; r < h; ++r) {
      for (int32_t n = 0; n < rhs; ++n) {
        const float* Bn = b + a->col_scalar_off[col] + (int64_t)n * K;
        double sum = 0.0;
        for (int32_t k = 0; k < w; ++k) sum += fabs((double)A[r + (int64_t)k * h]) * fabs((double)Bn[k]);
        bound[a->row_scalar_off[i] + r + (int64_t)n * M] += sum;
      }
    }
  }
}

int orc_abs_product_sum(const orc_view* a, const float* b, int64_t b_len, int32_t rhs, double* bound) {
  return orc_abs_product_sum_threads(a, b, b_len, rhs, 1, bound);
}

int orc_abs_product_sum_threads(const orc_view* a, const float* b, int64_t b_len, int32_t rhs, int32_t threads,
                                double* bound) {
  const int64_t M = scalar_rows(a), K = scalar_cols(a);
  if (b_len != K * rhs || threads < 1) return ORC_INVALID;
  memset(bound, 0, sizeof(double) * (size_t)(M * rhs));
  const int32_t rows = a->block_rows;
#pragma omp parallel for schedule(dynamic, 16) num_threads(threads)
  for (int32_t i = 0; i < rows; ++i) abs_product_row(a, b, rhs, M, K, i, bound);
  return ORC_OK;
}

/* src/kernels/row_owned.cu:24-43 (the order shared by every reference kernel) */
int orc_fmaf_order(const orc_view* a, const float* b, int64_t b_len, int32_t rhs, float* c) {
  const int64_t M = scalar_rows(a), K = scalar_cols(a);
  if (b_len != K * rhs) return ORC_INVALID;
  for (int32_t i = 0; i < a->block_rows; ++i) {
    const int32_t h = a->row_size[i];
    for (int32_t r = 0; r < h; ++r) {
      for (int32_t n = 0; n < rhs; ++n) {
        float acc = 0.0f;
        for (int32_t blk = a->row_ptr[i]; blk < a->row_ptr[i + 1]; ++blk) {
          const int32_t col = a->block_col[blk];
          const int32_t w = a->col_size[col];
          const float* A = a->values + a->value_off[blk] + r;
          const float* Bn = b + a->col_scalar_off[col] + (int64_t)n * K;
          for (int32_t k = 0; k < w; ++k) acc = fmaf(A[(int64_t)k * h], Bn[k], acc);
        }
        c[a->row_scalar_off[i] + r + (int64_t)n * M] = acc;
      }
    }
  }
  return ORC_OK;
}

/* tests/test_main.cpp:42-51 */
void orc_make_random_input(int64_t count, uint64_t seed, float* out) {
  orc_mt32 e;
  orc_mt32_seed(&e, (uint32_t)seed);
  for (int64_t i = 0; i < count; ++i) out[i] = orc_uniform_pm1_from_u32(orc_mt32_next(&e));
}

/* bench/benchmark.cpp:197-207 */
double orc_useful_flops(const orc_view* a, int32_t rhs) {
  double flops = 0.0;
  for (int32_t i = 0; i < a->block_rows; ++i)
    for (int32_t blk = a->row_ptr[i]; blk < a->row_ptr[i + 1]; ++blk)
      flops += 2.0 * a->row_size[i] * a->col_size[a->block_col[blk]] * rhs;
  return flops;
}
