/* The C API driven from C (compiled as C99), as the reference's c/tests/neighbors/run_certex_c.c
 * and certex_c.cu (cases Plain, Lists, Bitset, SaveLoad) do: build an index of uint8 vectors,
 * search with and without a bitset filter, remove ids; build one with k-means lists and search it
 * with the list probe; save it, load it into a new handle and search again. Every returned id and
 * distance is checked against a brute force in this file. Exit status 0 = pass. */
#define __HIP_PLATFORM_AMD__ 1
#define _XOPEN_SOURCE 700 /* mkstemp, close, unlink */
#include <cuvs/neighbors/certex.h>
#include <hip/hip_runtime_api.h>

#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#define CHECK(call)                                                            \
  do {                                                                         \
    if ((call) != CUVS_SUCCESS) {                                              \
      fprintf(stderr, "FAIL %s: %s\n", #call, cuvsGetLastErrorText());         \
      return 1;                                                                \
    }                                                                          \
  } while (0)
#define HCHECK(call)                                                           \
  do {                                                                         \
    if ((call) != hipSuccess) {                                                \
      fprintf(stderr, "FAIL %s\n", #call);                                     \
      return 1;                                                                \
    }                                                                          \
  } while (0)

static void tensor(DLManagedTensor* t, void* data, int ndim, int64_t* shape, uint8_t code,
                   uint8_t bits, int device)
{
  memset(t, 0, sizeof(*t));
  t->dl_tensor.data               = data;
  t->dl_tensor.device.device_type = device ? kDLROCM : kDLCPU;
  t->dl_tensor.ndim               = ndim;
  t->dl_tensor.dtype.code         = code;
  t->dl_tensor.dtype.bits         = bits;
  t->dl_tensor.dtype.lanes        = 1;
  t->dl_tensor.shape              = shape;
}

static uint64_t rng = 88172645463325252ull;
static uint8_t next_byte(void)
{
  rng ^= rng << 13;
  rng ^= rng >> 7;
  rng ^= rng << 17;
  return (uint8_t)(rng >> 56) & 0x1f; /* 32 levels: many exact ties */
}

/* k best of query qi by (squared distance, id) among rows with keep[i] != 0 */
static void brute(const uint8_t* x, const uint8_t* q, int64_t n, int64_t d, int64_t k,
                  const uint8_t* keep, int64_t* ids, double* dist)
{
  for (int64_t j = 0; j < k; ++j) {
    ids[j]  = -1;
    dist[j] = 1e300;
  }
  for (int64_t i = 0; i < n; ++i) {
    if (!keep[i]) continue;
    double s = 0;
    for (int64_t c = 0; c < d; ++c) {
      const double t = (double)q[c] - (double)x[i * d + c];
      s += t * t;
    }
    int64_t pos = k;
    while (pos > 0 && (dist[pos - 1] > s || (dist[pos - 1] == s && ids[pos - 1] > i))) --pos;
    if (pos == k) continue;
    for (int64_t j = k - 1; j > pos; --j) {
      ids[j]  = ids[j - 1];
      dist[j] = dist[j - 1];
    }
    ids[pos]  = i;
    dist[pos] = s;
  }
}

static int compare(const uint8_t* x, const uint8_t* q, int64_t n, int64_t d, int64_t nq,
                   int64_t k, const uint8_t* keep, const int64_t* got_ids, const float* got_d)
{
  int64_t* ids = malloc(sizeof(int64_t) * k);
  double* dist = malloc(sizeof(double) * k);
  int bad      = 0;
  for (int64_t qi = 0; qi < nq && !bad; ++qi) {
    brute(x, q + qi * d, n, d, k, keep, ids, dist);
    for (int64_t j = 0; j < k; ++j) {
      const float want = ids[j] < 0 ? (float)1e300 : (float)dist[j];
      if (got_ids[qi * k + j] != ids[j] || (ids[j] >= 0 && got_d[qi * k + j] != want)) {
        fprintf(stderr, "query %lld slot %lld: got %lld (%g) want %lld (%g)\n", (long long)qi,
                (long long)j, (long long)got_ids[qi * k + j], got_d[qi * k + j],
                (long long)ids[j], dist[j]);
        bad = 1;
        break;
      }
    }
  }
  free(ids);
  free(dist);
  return bad;
}

int main(void)
{
  const int64_t n = 30000, nq = 300, d = 48, k = 10;
  uint8_t* x    = malloc((size_t)(n * d));
  uint8_t* q    = malloc((size_t)(nq * d));
  uint8_t* keep = malloc((size_t)n);
  for (int64_t i = 0; i < n * d; ++i) x[i] = next_byte();
  for (int64_t i = 0; i < nq * d; ++i) q[i] = next_byte();

  void *dq, *dn, *dd, *dw, *dr;
  HCHECK(hipMalloc(&dq, (size_t)(nq * d)));
  HCHECK(hipMalloc(&dn, sizeof(int64_t) * nq * k));
  HCHECK(hipMalloc(&dd, sizeof(float) * nq * k));
  HCHECK(hipMemcpy(dq, q, (size_t)(nq * d), hipMemcpyHostToDevice));

  int64_t x_shape[2] = {n, d}, q_shape[2] = {nq, d}, o_shape[2] = {nq, k};
  DLManagedTensor X, Q, NB, DS;
  tensor(&X, x, 2, x_shape, kDLUInt, 8, 0); /* a host dataset, streamed to the GPU */
  tensor(&Q, dq, 2, q_shape, kDLUInt, 8, 1);
  tensor(&NB, dn, 2, o_shape, kDLInt, 64, 1);
  tensor(&DS, dd, 2, o_shape, kDLFloat, 32, 1);

  cuvsResources_t res;
  CHECK(cuvsResourcesCreate(&res));
  cuvsCertexIndexParams_t params;
  CHECK(cuvsCertexIndexParamsCreate(&params));
  cuvsCertexIndex_t index;
  CHECK(cuvsCertexIndexCreate(&index));
  CHECK(cuvsCertexBuild(res, params, &X, index));
  if (cuvsCertexBuild(res, params, &X, index) != CUVS_ERROR) { /* refuses a non-empty handle */
    fprintf(stderr, "FAIL: second build accepted\n");
    return 1;
  }
  int64_t size = 0, dim = 0;
  CHECK(cuvsCertexIndexGetSize(index, &size));
  CHECK(cuvsCertexIndexGetDim(index, &dim));
  if (size != n || dim != d) {
    fprintf(stderr, "FAIL: size %lld dim %lld\n", (long long)size, (long long)dim);
    return 1;
  }

  cuvsCertexSearchParams_t sp;
  CHECK(cuvsCertexSearchParamsCreate(&sp));
  cuvsFilter none = {0, NO_FILTER};
  int64_t* got_ids = malloc(sizeof(int64_t) * nq * k);
  float* got_d     = malloc(sizeof(float) * nq * k);
  for (int64_t i = 0; i < n; ++i) keep[i] = 1;
  CHECK(cuvsCertexSearch(res, sp, index, &Q, &NB, &DS, none));
  CHECK(cuvsStreamSync(res));
  HCHECK(hipMemcpy(got_ids, dn, sizeof(int64_t) * nq * k, hipMemcpyDeviceToHost));
  HCHECK(hipMemcpy(got_d, dd, sizeof(float) * nq * k, hipMemcpyDeviceToHost));
  if (compare(x, q, n, d, nq, k, keep, got_ids, got_d)) return 1;

  /* bitset filter keeping every third id */
  const int64_t n_words = (n + 31) / 32;
  uint32_t* words       = calloc((size_t)n_words, sizeof(uint32_t));
  for (int64_t i = 0; i < n; ++i) {
    keep[i] = (uint8_t)(i % 3 == 0);
    if (keep[i]) words[i >> 5] |= 1u << (i & 31);
  }
  HCHECK(hipMalloc(&dw, sizeof(uint32_t) * n_words));
  HCHECK(hipMemcpy(dw, words, sizeof(uint32_t) * n_words, hipMemcpyHostToDevice));
  int64_t w_shape[1] = {n_words};
  DLManagedTensor W;
  tensor(&W, dw, 1, w_shape, kDLUInt, 32, 1);
  cuvsFilter bits = {(uintptr_t)&W, BITSET};
  CHECK(cuvsCertexSearch(res, sp, index, &Q, &NB, &DS, bits));
  CHECK(cuvsStreamSync(res));
  HCHECK(hipMemcpy(got_ids, dn, sizeof(int64_t) * nq * k, hipMemcpyDeviceToHost));
  HCHECK(hipMemcpy(got_d, dd, sizeof(float) * nq * k, hipMemcpyDeviceToHost));
  if (compare(x, q, n, d, nq, k, keep, got_ids, got_d)) return 1;

  /* remove the first 5000 ids */
  int64_t* rem = malloc(sizeof(int64_t) * 5000);
  for (int64_t i = 0; i < 5000; ++i) rem[i] = i;
  HCHECK(hipMalloc(&dr, sizeof(int64_t) * 5000));
  HCHECK(hipMemcpy(dr, rem, sizeof(int64_t) * 5000, hipMemcpyHostToDevice));
  int64_t r_shape[1] = {5000};
  DLManagedTensor R;
  tensor(&R, dr, 1, r_shape, kDLInt, 64, 1);
  CHECK(cuvsCertexRemove(res, &R, index));
  for (int64_t i = 0; i < n; ++i) keep[i] = (uint8_t)(i >= 5000);
  CHECK(cuvsCertexSearch(res, sp, index, &Q, &NB, &DS, none));
  CHECK(cuvsStreamSync(res));
  HCHECK(hipMemcpy(got_ids, dn, sizeof(int64_t) * nq * k, hipMemcpyDeviceToHost));
  HCHECK(hipMemcpy(got_d, dd, sizeof(float) * nq * k, hipMemcpyDeviceToHost));
  if (compare(x, q, n, d, nq, k, keep, got_ids, got_d)) return 1;

  /* Lists: 32 k-means lists, two probed per query (reference certex_c.cu:135), with the
   * removals applied to this index too, then a bitset */
  cuvsCertexIndex_t listed;
  CHECK(cuvsCertexIndexCreate(&listed));
  params->n_lists = 32;
  CHECK(cuvsCertexBuild(res, params, &X, listed));
  CHECK(cuvsCertexRemove(res, &R, listed));
  sp->probe_lists = 2;
  CHECK(cuvsCertexSearch(res, sp, listed, &Q, &NB, &DS, none));
  CHECK(cuvsStreamSync(res));
  HCHECK(hipMemcpy(got_ids, dn, sizeof(int64_t) * nq * k, hipMemcpyDeviceToHost));
  HCHECK(hipMemcpy(got_d, dd, sizeof(float) * nq * k, hipMemcpyDeviceToHost));
  if (compare(x, q, n, d, nq, k, keep, got_ids, got_d)) return 1;
  for (int64_t i = 0; i < n; ++i) keep[i] = (uint8_t)(i >= 5000 && i % 3 == 0);
  CHECK(cuvsCertexSearch(res, sp, listed, &Q, &NB, &DS, bits));
  CHECK(cuvsStreamSync(res));
  HCHECK(hipMemcpy(got_ids, dn, sizeof(int64_t) * nq * k, hipMemcpyDeviceToHost));
  HCHECK(hipMemcpy(got_d, dd, sizeof(float) * nq * k, hipMemcpyDeviceToHost));
  if (compare(x, q, n, d, nq, k, keep, got_ids, got_d)) return 1;

  /* SaveLoad (reference certex_c.cu:139): the index with lists and removals, into a new handle */
  char path[] = "/tmp/run_certex_c_XXXXXX";
  const int fd = mkstemp(path);
  if (fd < 0) {
    fprintf(stderr, "FAIL: no temporary file\n");
    return 1;
  }
  close(fd);
  CHECK(cuvsCertexSerialize(res, path, listed));
  CHECK(cuvsCertexIndexDestroy(listed));
  cuvsCertexIndex_t loaded;
  CHECK(cuvsCertexIndexCreate(&loaded));
  CHECK(cuvsCertexDeserialize(res, path, loaded));
  if (cuvsCertexDeserialize(res, path, loaded) != CUVS_ERROR) { /* refuses a non-empty handle */
    fprintf(stderr, "FAIL: deserialize into a non-empty handle accepted\n");
    return 1;
  }
  unlink(path);
  CHECK(cuvsCertexIndexGetSize(loaded, &size));
  if (size != n) {
    fprintf(stderr, "FAIL: loaded size %lld\n", (long long)size);
    return 1;
  }
  CHECK(cuvsCertexSearch(res, sp, loaded, &Q, &NB, &DS, bits));
  CHECK(cuvsStreamSync(res));
  HCHECK(hipMemcpy(got_ids, dn, sizeof(int64_t) * nq * k, hipMemcpyDeviceToHost));
  HCHECK(hipMemcpy(got_d, dd, sizeof(float) * nq * k, hipMemcpyDeviceToHost));
  if (compare(x, q, n, d, nq, k, keep, got_ids, got_d)) return 1;
  for (int64_t i = 0; i < n; ++i) keep[i] = (uint8_t)(i >= 5000);
  CHECK(cuvsCertexSearch(res, sp, loaded, &Q, &NB, &DS, none));
  CHECK(cuvsStreamSync(res));
  HCHECK(hipMemcpy(got_ids, dn, sizeof(int64_t) * nq * k, hipMemcpyDeviceToHost));
  HCHECK(hipMemcpy(got_d, dd, sizeof(float) * nq * k, hipMemcpyDeviceToHost));
  if (compare(x, q, n, d, nq, k, keep, got_ids, got_d)) return 1;
  CHECK(cuvsCertexIndexDestroy(loaded));

  /* queries of another vector type are rejected */
  DLManagedTensor QF;
  tensor(&QF, dq, 2, q_shape, kDLFloat, 32, 1);
  if (cuvsCertexSearch(res, sp, index, &QF, &NB, &DS, none) != CUVS_ERROR) {
    fprintf(stderr, "FAIL: float queries accepted by a uint8 index\n");
    return 1;
  }

  CHECK(cuvsCertexSearchParamsDestroy(sp));
  CHECK(cuvsCertexIndexDestroy(index));
  CHECK(cuvsCertexIndexParamsDestroy(params));
  CHECK(cuvsResourcesDestroy(res));
  hipFree(dq); hipFree(dn); hipFree(dd); hipFree(dw); hipFree(dr);
  printf("run_certex_c: ok\n");
  return 0;
}
