/*
 * CPU oracle of the exact k-NN search path. TEST INFRASTRUCTURE ONLY: tests/, the smoke check of
 * __graft_entry__ and the cpu_baseline leg of bench.py use it to check and to time the GPU path;
 * the library never calls it.
 *
 * It restates the reference's exhaustive fp64 search, certex.verify (certex/index.py:487-548),
 * with the exact score definitions of that function and of warp_score
 * (cpp/src/neighbors/certex/detail/certex_kernels.cuh:247-273):
 *   l2      score = sum_j (q_j - x_j)^2                       (smaller is better)
 *   inner   score = -sum_j q_j x_j                            (index.py:532, -(rows * Qs).sum)
 *   cosine  score = -sum_j q_j x_j / sqrt(sum q^2 * sum x^2)  (index.py:527-532 normalises both)
 * evaluated in fp64 in a fixed order that a 64-lane wave reproduces bit for bit: coordinate j goes
 * to partial sum j mod 64, each partial accumulates its coordinates in increasing order with fused
 * multiply-adds, and the 64 partials are combined by a butterfly (for off = 32, 16, ..., 1:
 * p[i] = p[i] + p[i ^ off]). The reference sums per warp lane and combines by shuffles the same
 * way (warp_score, 32 lanes). Results are ranked
 * by the total order (score, id): ties go to the lower id, as in the only tie-break of the
 * reference (certex_shards.cu:154-157). Filters follow the reference semantics: a bitset over ids,
 * a bitmap of one row of bits per query (certex.h:176-182), or equal labels (certex.hpp:702-705);
 * removed ids never appear (tests/test_exact.py:83-84). Missing entries get id -1 and score +inf
 * (ann_certex.cuh:76-141 pads with -1).
 *
 * The searches use type-specialised scorers (below) that give the same bits as oracle_score;
 * tests/test_oracle.py checks them against it.
 *
 * Pinned by tests/test_oracle.py: brute-force numpy on small inputs (integer data exactly), the
 * closed form for duplicates and ties, the reference's own known answers (verify = 2/3 after
 * corrupting 100 of 300 queries, test_exact.py:440-452) and the filter semantics.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

enum { DT_F32 = 0, DT_F16 = 1, DT_I8 = 2, DT_U8 = 3 };
enum { M_L2 = 0, M_INNER = 1, M_COSINE = 2 };

static double half_to_double(uint16_t h)
{
  const int s = h >> 15, e = (h >> 10) & 31, m = h & 1023;
  double v;
  if (e == 0) {
    v = ldexp((double)m, -24);
  } else if (e == 31) {
    v = m ? NAN : INFINITY;
  } else {
    v = ldexp((double)(m | 1024), e - 25);
  }
  return s ? -v : v;
}

static double coord(const void* p, int dt, int64_t i)
{
  switch (dt) {
    case DT_F32: return (double)((const float*)p)[i];
    case DT_F16: return half_to_double(((const uint16_t*)p)[i]);
    case DT_I8: return (double)((const int8_t*)p)[i];
    default: return (double)((const uint8_t*)p)[i];
  }
}

enum { LANES = 64 };

/** Butterfly combination of 64 partial sums (every lane of a wave ends with this value). */
static double combine(double* p)
{
  for (int off = LANES / 2; off; off >>= 1) {
    for (int i = 0; i < LANES; ++i) {
      if (!(i & off)) {
        const double v = p[i] + p[i | off];
        p[i]           = v;
        p[i | off]     = v;
      }
    }
  }
  return p[0];
}

/** The exact score of query row q against stored row x (see the header). */
double oracle_score(const void* q, const void* x, int dt, int64_t d, int metric)
{
  double acc[LANES] = {0}, qq[LANES] = {0}, xx[LANES] = {0};
  for (int64_t j = 0; j < d; ++j) {
    const double a = coord(q, dt, j), b = coord(x, dt, j);
    const int l    = (int)(j % LANES);
    if (metric == M_L2) {
      const double t = a - b;
      acc[l]         = fma(t, t, acc[l]);
    } else {
      acc[l] = fma(a, b, acc[l]);
      if (metric == M_COSINE) {
        qq[l] = fma(a, a, qq[l]);
        xx[l] = fma(b, b, xx[l]);
      }
    }
  }
  const double s = combine(acc);
  if (metric == M_L2) { return s; }
  if (metric == M_INNER) { return -s; }
  return -s / sqrt(combine(qq) * combine(xx));
}

static int elem_size(int dt) { return dt == DT_F32 ? 4 : (dt == DT_F16 ? 2 : 1); }

/*
 * Type-specialised scorers: the same scores, bit for bit, without the per-coordinate type switch
 * (they are what bench.py times as the CPU baseline). 8-bit data: every product and partial sum
 * of the canonical order is an exact integer below 2^53, so an exact int32 sum converted to
 * double equals it (d <= 32768 keeps |sum| below 2^31). Float data: the canonical order itself,
 * with the 64 partial sums of one block of coordinates updated together so that the compiler
 * vectorises across them; each partial still accumulates its coordinates in increasing order with
 * one fused multiply-add each. target_clones picks AVX-512, AVX2 or the baseline at load time.
 */
#define CLONES __attribute__((target_clones("avx512f", "avx2", "default")))
enum { MAX_FAST_INT_DIM = 32768 };

CLONES static double score_u8(const void* qv, const void* xv, int64_t d, int metric)
{
  const uint8_t *q = (const uint8_t*)qv, *x = (const uint8_t*)xv;
  int32_t acc = 0;
  if (metric == M_L2) {
    for (int64_t j = 0; j < d; ++j) {
      const int32_t t = (int32_t)q[j] - (int32_t)x[j];
      acc += t * t;
    }
    return (double)acc;
  }
  for (int64_t j = 0; j < d; ++j) { acc += (int32_t)q[j] * (int32_t)x[j]; }
  return -(double)acc;
}

CLONES static double score_i8(const void* qv, const void* xv, int64_t d, int metric)
{
  const int8_t *q = (const int8_t*)qv, *x = (const int8_t*)xv;
  int32_t acc = 0;
  if (metric == M_L2) {
    for (int64_t j = 0; j < d; ++j) {
      const int32_t t = (int32_t)q[j] - (int32_t)x[j];
      acc += t * t;
    }
    return (double)acc;
  }
  for (int64_t j = 0; j < d; ++j) { acc += (int32_t)q[j] * (int32_t)x[j]; }
  return -(double)acc;
}

/* one float type: blocks of 64 coordinates, partial l takes coordinate 64 b + l */
#define FLOAT_SCORER(name, T, load)                                                         \
  CLONES static double name(const void* qv, const void* xv, int64_t d, int metric)          \
  {                                                                                        \
    const T *q = (const T*)qv, *x = (const T*)xv;                                          \
    double acc[LANES], qq[LANES], xx[LANES];                                               \
    for (int l = 0; l < LANES; ++l) { acc[l] = qq[l] = xx[l] = 0.0; }                      \
    for (int64_t b = 0; b < d; b += LANES) {                                               \
      const int m = d - b < LANES ? (int)(d - b) : LANES;                                  \
      if (metric == M_L2) {                                                                \
        for (int l = 0; l < m; ++l) {                                                      \
          const double t = load(q[b + l]) - load(x[b + l]);                                \
          acc[l]         = fma(t, t, acc[l]);                                              \
        }                                                                                  \
      } else {                                                                             \
        for (int l = 0; l < m; ++l) {                                                      \
          const double a = load(q[b + l]), c = load(x[b + l]);                             \
          acc[l]         = fma(a, c, acc[l]);                                              \
          if (metric == M_COSINE) {                                                        \
            qq[l] = fma(a, a, qq[l]);                                                      \
            xx[l] = fma(c, c, xx[l]);                                                      \
          }                                                                                \
        }                                                                                  \
      }                                                                                    \
    }                                                                                      \
    const double s = combine(acc);                                                         \
    if (metric == M_L2) { return s; }                                                      \
    if (metric == M_INNER) { return -s; }                                                  \
    return -s / sqrt(combine(qq) * combine(xx));                                           \
  }

#define LOAD_F32(v) ((double)(v))
#define LOAD_F16(v) half_to_double(v)
FLOAT_SCORER(score_f32, float, LOAD_F32)
FLOAT_SCORER(score_f16, uint16_t, LOAD_F16)

typedef double (*scorer_fn)(const void*, const void*, int64_t, int);

static int g_generic = 0; /* tests: 1 = every score through oracle_score */

/** Use the generic scorer (1) or the type-specialised ones (0); returns the previous setting. */
int oracle_set_generic(int on)
{
  const int was = g_generic;
  g_generic     = on;
  return was;
}

static double generic_f32(const void* q, const void* x, int64_t d, int m) { return oracle_score(q, x, DT_F32, d, m); }
static double generic_f16(const void* q, const void* x, int64_t d, int m) { return oracle_score(q, x, DT_F16, d, m); }
static double generic_i8(const void* q, const void* x, int64_t d, int m) { return oracle_score(q, x, DT_I8, d, m); }
static double generic_u8(const void* q, const void* x, int64_t d, int m) { return oracle_score(q, x, DT_U8, d, m); }

/** The scorer of a type and metric: the generic one for cosine on 8-bit data and huge dims. */
static scorer_fn scorer_of(int dt, int64_t d, int metric)
{
  const int integer = dt == DT_I8 || dt == DT_U8;
  if (g_generic || (integer && (metric == M_COSINE || d > MAX_FAST_INT_DIM))) {
    switch (dt) {
      case DT_F32: return generic_f32;
      case DT_F16: return generic_f16;
      case DT_I8: return generic_i8;
      default: return generic_u8;
    }
  }
  switch (dt) {
    case DT_F32: return score_f32;
    case DT_F16: return score_f16;
    case DT_I8: return score_i8;
    default: return score_u8;
  }
}

static int worse(double sa, int64_t ia, double sb, int64_t ib)
{
  return sa > sb || (sa == sb && ia > ib);
}

/* max-heap of the k best (root = the worst kept entry) */
static void sift_down(double* s, int64_t* id, int n, int i)
{
  for (;;) {
    int l = 2 * i + 1, r = l + 1, w = i;
    if (l < n && worse(s[l], id[l], s[w], id[w])) { w = l; }
    if (r < n && worse(s[r], id[r], s[w], id[w])) { w = r; }
    if (w == i) { return; }
    double ts = s[i];
    s[i]      = s[w];
    s[w]      = ts;
    int64_t ti = id[i];
    id[i]      = id[w];
    id[w]      = ti;
    i          = w;
  }
}

static void sift_up(double* s, int64_t* id, int i)
{
  while (i > 0) {
    int p = (i - 1) / 2;
    if (!worse(s[i], id[i], s[p], id[p])) { return; }
    double ts = s[i];
    s[i]      = s[p];
    s[p]      = ts;
    int64_t ti = id[i];
    id[i]      = id[p];
    id[p]      = ti;
    i          = p;
  }
}

/**
 * Exhaustive search: out_score / out_id [nq, k] in increasing (score, id); -1 / +inf where fewer
 * than k stored rows pass the filter. Optional (NULL to skip): removed [n] flags, bitset words over
 * ids, bitmap words of nq rows of n bits, row / query labels.
 */
void oracle_knn(const void* base, int dt, int64_t n, int64_t d, const void* queries, int64_t nq,
                int metric, int k, const uint8_t* removed, const uint32_t* bitset,
                const uint32_t* bitmap, const int32_t* row_labels, const int32_t* query_labels,
                double* out_score, int64_t* out_id)
{
  const int es         = elem_size(dt);
  const scorer_fn score = scorer_of(dt, d, metric);
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t qi = 0; qi < nq; ++qi) {
    double* s   = (double*)malloc(sizeof(double) * (size_t)k);
    int64_t* id = (int64_t*)malloc(sizeof(int64_t) * (size_t)k);
    int have    = 0;
    const char* q = (const char*)queries + qi * d * es;
    for (int64_t i = 0; i < n; ++i) {
      if (removed && removed[i]) { continue; }
      if (bitset && !((bitset[i >> 5] >> (i & 31)) & 1u)) { continue; }
      if (bitmap) {
        const int64_t bit = qi * n + i;
        if (!((bitmap[bit >> 5] >> (bit & 31)) & 1u)) { continue; }
      }
      if (row_labels && query_labels && row_labels[i] != query_labels[qi]) { continue; }
      const double sc = score(q, (const char*)base + i * d * es, d, metric);
      if (have < k) {
        s[have]  = sc;
        id[have] = i;
        sift_up(s, id, have);
        ++have;
      } else if (worse(s[0], id[0], sc, i)) {
        s[0]  = sc;
        id[0] = i;
        sift_down(s, id, have, 0);
      }
    }
    /* heap sort: repeatedly move the worst to the end */
    for (int m = have; m > 1; --m) {
      double ts = s[0];
      s[0]      = s[m - 1];
      s[m - 1]  = ts;
      int64_t ti = id[0];
      id[0]      = id[m - 1];
      id[m - 1]  = ti;
      sift_down(s, id, m - 1, 0);
    }
    for (int j = 0; j < k; ++j) {
      out_score[qi * k + j] = j < have ? s[j] : INFINITY;
      out_id[qi * k + j]    = j < have ? id[j] : -1;
    }
    free(s);
    free(id);
  }
}

/** Scores of given ids (-1: +inf), for checking results the way certex.verify does. */
void oracle_scores_of(const void* base, int dt, int64_t n, int64_t d, const void* queries,
                      int64_t nq, int metric, int k, const int64_t* ids, double* out)
{
  const int es         = elem_size(dt);
  const scorer_fn score = scorer_of(dt, d, metric);
#pragma omp parallel for schedule(static)
  for (int64_t qi = 0; qi < nq; ++qi) {
    const char* q = (const char*)queries + qi * d * es;
    for (int j = 0; j < k; ++j) {
      const int64_t i     = ids[qi * k + j];
      out[qi * k + j] = (i < 0 || i >= n)
                          ? INFINITY
                          : score(q, (const char*)base + i * d * es, d, metric);
    }
  }
}

int oracle_threads(void)
{
#ifdef _OPENMP
  extern int omp_get_max_threads(void);
  return omp_get_max_threads();
#else
  return 1;
#endif
}
