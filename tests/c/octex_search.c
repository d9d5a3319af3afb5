/* A C caller of the cuvsOctex* ABI (include/cuvs/neighbors/octex.h), as a program of the reference's C users
 * (examples/c/search.c, c/tests) would be: build an index directory from a host dataset, load it, search host
 * queries.  Usage: octex_search_c DIR N D M K DATA.f32 QUERIES.f32 OUT (raw row-major float32 inputs; writes
 * OUT.i64 and OUT.f32, the neighbors and distances [M, K]). */
#include <cuvs/core/c_api.h>
#include <cuvs/neighbors/octex.h>

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define CHECK(call)                                                                  \
  do {                                                                               \
    if ((call) != CUVS_SUCCESS) {                                                    \
      fprintf(stderr, "%s failed: %s\n", #call, cuvsGetLastErrorText());             \
      return 1;                                                                      \
    }                                                                                \
  } while (0)

static void host_matrix(DLManagedTensor* t, void* data, int64_t* shape, uint8_t code, uint8_t bits)
{
  memset(t, 0, sizeof(*t));
  t->dl_tensor.data               = data;
  t->dl_tensor.device.device_type = kDLCPU;
  t->dl_tensor.ndim               = 2;
  t->dl_tensor.dtype.code         = code;
  t->dl_tensor.dtype.bits         = bits;
  t->dl_tensor.dtype.lanes        = 1;
  t->dl_tensor.shape              = shape;
}

static void* read_all(const char* path, size_t bytes)
{
  FILE* f = fopen(path, "rb");
  void* p = malloc(bytes);
  if (f == NULL || p == NULL || fread(p, 1, bytes, f) != bytes) {
    fprintf(stderr, "cannot read %zu bytes of %s\n", bytes, path);
    exit(1);
  }
  fclose(f);
  return p;
}

static int write_all(const char* path, const char* ext, const void* p, size_t bytes)
{
  char name[4096];
  snprintf(name, sizeof(name), "%s%s", path, ext);
  FILE* f = fopen(name, "wb");
  if (f == NULL || fwrite(p, 1, bytes, f) != bytes) return 1;
  return fclose(f) != 0;
}

int main(int argc, char** argv)
{
  if (argc != 9) {
    fprintf(stderr, "usage: %s DIR N D M K DATA.f32 QUERIES.f32 OUT\n", argv[0]);
    return 2;
  }
  const char* dir = argv[1];
  int64_t n = atoll(argv[2]), d = atoll(argv[3]), m = atoll(argv[4]), k = atoll(argv[5]);
  float* x = (float*)read_all(argv[6], (size_t)(n * d) * sizeof(float));
  float* q = (float*)read_all(argv[7], (size_t)(m * d) * sizeof(float));
  int64_t* nb = (int64_t*)malloc((size_t)(m * k) * sizeof(int64_t));
  float* dist = (float*)malloc((size_t)(m * k) * sizeof(float));

  cuvsResources_t res;
  CHECK(cuvsResourcesCreate(&res));

  cuvsOctexIndexParams_t ip;
  CHECK(cuvsOctexIndexParamsCreate(&ip));
  ip->copies      = 16;
  ip->list_len    = 32;
  ip->table_len   = 32;
  ip->log_buckets = 12;
  ip->seed        = 1;
  int64_t xs[2] = {n, d};
  DLManagedTensor dataset;
  host_matrix(&dataset, x, xs, kDLFloat, 32);
  CHECK(cuvsOctexBuild(res, ip, &dataset, dir));
  CHECK(cuvsOctexIndexParamsDestroy(ip));

  cuvsOctexIndex_t index;
  CHECK(cuvsOctexIndexCreate(&index));
  CHECK(cuvsOctexLoad(res, dir, NULL, index));
  int64_t size = 0, dim = 0;
  CHECK(cuvsOctexIndexGetSize(index, &size));
  CHECK(cuvsOctexIndexGetDim(index, &dim));
  if (size != n || dim != d) {
    fprintf(stderr, "index holds %lld x %lld, built from %lld x %lld\n", (long long)size, (long long)dim,
            (long long)n, (long long)d);
    return 1;
  }

  cuvsOctexSearchParams_t sp;
  CHECK(cuvsOctexSearchParamsCreate(&sp));
  sp->read   = 16;
  sp->starts = 64;
  sp->waves  = 2;
  int64_t qs[2] = {m, d}, os[2] = {m, k};
  DLManagedTensor queries, neighbors, distances;
  host_matrix(&queries, q, qs, kDLFloat, 32);
  host_matrix(&neighbors, nb, os, kDLInt, 64);
  host_matrix(&distances, dist, os, kDLFloat, 32);
  CHECK(cuvsOctexSearch(res, sp, index, &queries, &neighbors, &distances));
  CHECK(cuvsOctexSearchParamsDestroy(sp));
  CHECK(cuvsOctexIndexDestroy(index));
  CHECK(cuvsResourcesDestroy(res));

  if (write_all(argv[8], ".i64", nb, (size_t)(m * k) * sizeof(int64_t)) ||
      write_all(argv[8], ".f32", dist, (size_t)(m * k) * sizeof(float))) {
    fprintf(stderr, "cannot write %s.*\n", argv[8]);
    return 1;
  }
  printf("c caller: %lld queries, first ids %lld %lld %lld\n", (long long)m, (long long)nb[0], (long long)nb[1],
         (long long)nb[2]);
  free(x);
  free(q);
  free(nb);
  free(dist);
  return 0;
}
