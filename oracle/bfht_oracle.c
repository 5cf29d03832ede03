/*
 * CPU oracle for the BlockFHT path, in C — TEST INFRASTRUCTURE, NOT PRODUCT.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * this library, and only as the checker.  It restates, in float64 with plain
 * loops, the reference semantics:
 *
 *   lowbias32 / sign_word_for    latent_weight_lab/block_fht.py:36-52
 *                                (device twin csrc/block_fht_ext_cuda.cu:27-43)
 *   sign of position p           block_fht.py:55-81 (bit p&31 of word p>>5)
 *   normalized FHT               block_fht.py:18-33 (pairs (a, a+step), /sqrt(B))
 *   slice forward                block_fht.py:84-109
 *   slice backward (adjoint)     block_fht_ext_cuda.cu:185-223, block_fht.py:180-196
 *
 * It is pinned against the reference's golden vectors and the numpy oracle by
 * tests/test_oracle.py.  Blocks are independent, so the forward and the
 * per-block backward run in parallel with OpenMP; the backward sums the
 * per-block partials in block order, so the result does not depend on the
 * thread count.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static uint32_t lowbias32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352dU;
  x ^= x >> 15;
  x *= 0x846ca68bU;
  x ^= x >> 16;
  return x;
}

uint32_t oracle_sign_word(int64_t seed, int64_t block, int64_t layer, int64_t word) {
  uint64_t s = (uint64_t)seed;
  uint32_t x = (uint32_t)s ^ (uint32_t)(s >> 32);
  x ^= 0x9e3779b9U * (uint32_t)(uint64_t)(block + 1);
  x ^= 0x85ebca6bU * (uint32_t)(uint64_t)(layer + 1);
  x ^= 0xc2b2ae35U * (uint32_t)(uint64_t)(word + 1);
  return lowbias32(x);
}

void oracle_sign_words(int64_t seed, int64_t block, int64_t layer, int64_t first_word,
                       int64_t nwords, uint32_t* out) {
  for (int64_t i = 0; i < nwords; ++i) out[i] = oracle_sign_word(seed, block, layer, first_word + i);
}

static int64_t next_pow2(int64_t v) {
  int64_t b = 1;
  while (b < v) b <<= 1;
  return b;
}

static void apply_signs(double* v, int64_t B, int64_t seed, int64_t block, int64_t layer) {
  for (int64_t w = 0; w * 32 < B; ++w) {
    uint32_t bits = oracle_sign_word(seed, block, layer, w);
    for (int64_t b = 0; b < 32 && w * 32 + b < B; ++b)
      if (!((bits >> b) & 1u)) v[w * 32 + b] = -v[w * 32 + b];
  }
}

static void fht(double* v, int64_t B) {
  for (int64_t step = 1; step < B; step <<= 1)
    for (int64_t g = 0; g < B; g += 2 * step)
      for (int64_t i = g; i < g + step; ++i) {
        double a = v[i], b = v[i + step];
        v[i] = a + b;
        v[i + step] = a - b;
      }
  double s = 1.0 / sqrt((double)B);
  for (int64_t i = 0; i < B; ++i) v[i] *= s;
}

static int check_args(int64_t n, int64_t size, int layers, int64_t start, int64_t stop) {
  if (n <= 0 || size <= 0 || layers < 0) return -1;
  if (start < 0 || stop < start || stop > size) return -1;
  return 0;
}

/* out[g - start] = T_{g/B}(pad(latent))[g % B] for g in [start, stop). */
int oracle_forward(const double* latent, int64_t n, int64_t size, int layers, int64_t seed,
                   int64_t start, int64_t stop, double* out) {
  if (check_args(n, size, layers, start, stop)) return -1;
  int64_t B = next_pow2(n);
  int64_t first = start / B, last = (stop + B - 1) / B;
  int err = 0;
#pragma omp parallel
  {
    double* v = (double*)malloc((size_t)B * sizeof(double));
    if (!v) {
#pragma omp atomic write
      err = -2;
    }
#pragma omp for schedule(dynamic)
    for (int64_t block = first; block < last; ++block) {
      if (!v) continue;
      memset(v, 0, (size_t)B * sizeof(double));
      memcpy(v, latent, (size_t)n * sizeof(double));
      apply_signs(v, B, seed, block, 0);
      for (int l = 0; l < layers; ++l) {
        fht(v, B);
        apply_signs(v, B, seed, block, l + 1);
      }
      int64_t lo = start - block * B > 0 ? start - block * B : 0;
      int64_t hi = stop - block * B < B ? stop - block * B : B;
      memcpy(out + (block * B + lo - start), v + lo, (size_t)(hi - lo) * sizeof(double));
    }
    free(v);
  }
  return err;
}

/* grad_latent[p] = sum_b [D_0 H D_1 ... H D_L scatter_b(grad_out)][p], p < n. */
int oracle_backward(const double* grad_out, int64_t n, int64_t size, int layers, int64_t seed,
                    int64_t start, int64_t stop, double* grad_latent) {
  if (check_args(n, size, layers, start, stop)) return -1;
  int64_t B = next_pow2(n);
  int64_t first = start / B, last = (stop + B - 1) / B;
  int64_t nb = last - first;
  memset(grad_latent, 0, (size_t)n * sizeof(double));
  if (nb <= 0) return 0;
  double* part = (double*)malloc((size_t)nb * (size_t)n * sizeof(double));
  if (!part) return -2;
  int err = 0;
#pragma omp parallel
  {
    double* v = (double*)malloc((size_t)B * sizeof(double));
    if (!v) {
#pragma omp atomic write
      err = -2;
    }
#pragma omp for schedule(dynamic)
    for (int64_t block = first; block < last; ++block) {
      if (!v) continue;
      memset(v, 0, (size_t)B * sizeof(double));
      int64_t lo = start - block * B > 0 ? start - block * B : 0;
      int64_t hi = stop - block * B < B ? stop - block * B : B;
      memcpy(v + lo, grad_out + (block * B + lo - start), (size_t)(hi - lo) * sizeof(double));
      for (int l = layers - 1; l >= 0; --l) {
        apply_signs(v, B, seed, block, l + 1);
        fht(v, B);
      }
      apply_signs(v, B, seed, block, 0);
      memcpy(part + (block - first) * n, v, (size_t)n * sizeof(double));
    }
    free(v);
  }
  if (!err)
    for (int64_t b = 0; b < nb; ++b)
      for (int64_t p = 0; p < n; ++p) grad_latent[p] += part[b * n + p];
  free(part);
  return err;
}
