// Row and query encoding for the int8 MFMA screen, tombstones and small fills (gfx950).
//
// Reference contracts: encode_int8_rows / encode_int8_queries (detail/int8.cuh:30-136) and
// remove_rows / remove_int8_rows (certex_kernels.cuh:391-415, detail/int8.cuh:139-147). For 8-bit
// integer vectors the code is the vector itself shifted into int8 (no projection, no scale), so
// the screen is exact; the row term folds the norm (l2) or the shift correction (inner product).

#include "../kernels.hpp"

namespace certex_amd {
namespace {

__global__ void encode_rows_kernel(const uint8_t* x, int64_t n, int64_t dim, int row_bytes,
                                   uint8_t flip, metric_kind metric, int8_t* codes, int32_t* rowc)
{
  const int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x;
  if (i >= n) { return; }
  const uint8_t* src = x + i * dim;
  int8_t* dst        = codes + i * row_bytes;
  int norm = 0, sum = 0;
  for (int64_t j = 0; j < dim; ++j) {
    const int c = int(int8_t(src[j] ^ flip));
    dst[j]      = int8_t(c);
    norm += c * c;
    sum += c;
  }
  for (int64_t j = dim; j < row_bytes; ++j) { dst[j] = 0; }
  if (metric == metric_kind::l2) {
    rowc[i] = -(norm >> 1);
  } else {
    rowc[i] = flip ? 128 * sum : 0;
  }
}

__global__ void encode_queries_kernel(const uint8_t* q, int64_t nq, int64_t nq_pad, int64_t dim,
                                      int row_bytes, uint8_t flip, int8_t* qcodes)
{
  const int64_t t = blockIdx.x * int64_t(blockDim.x) + threadIdx.x;
  if (t >= nq_pad * row_bytes) { return; }
  const int64_t i = t / row_bytes, j = t % row_bytes;
  qcodes[t]       = (i < nq && j < dim) ? int8_t(q[i * dim + j] ^ flip) : int8_t(0);
}

__global__ void remove_kernel(const int64_t* ids, int64_t n, int64_t size, int32_t* rowc,
                              unsigned long long* newly)
{
  const int64_t t = blockIdx.x * int64_t(blockDim.x) + threadIdx.x;
  if (t >= n) { return; }
  const int64_t id = ids[t];
  if (id < 0 || id >= size) { return; }
  if (atomicExch(rowc + id, kDeadRow) != kDeadRow) { atomicAdd(newly, 1ull); }
}

template <typename T>
__global__ void fill_kernel(T* p, int64_t n, T v)
{
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < n;
       i += int64_t(gridDim.x) * blockDim.x) {
    p[i] = v;
  }
}

inline unsigned blocks_for(int64_t n, int block = 256)
{
  return unsigned((n + block - 1) / block);
}

}  // namespace

void encode_rows_i8(const uint8_t* x, int64_t n, int64_t dim, int row_bytes, uint8_t flip,
                    metric_kind metric, int8_t* codes, int32_t* rowc, hipStream_t stream)
{
  if (n == 0) { return; }
  encode_rows_kernel<<<blocks_for(n), 256, 0, stream>>>(x, n, dim, row_bytes, flip, metric, codes,
                                                        rowc);
}

void encode_queries_i8(const uint8_t* q, int64_t nq, int64_t nq_pad, int64_t dim, int row_bytes,
                       uint8_t flip, int8_t* qcodes, hipStream_t stream)
{
  const int64_t n = nq_pad * row_bytes;
  if (n == 0) { return; }
  encode_queries_kernel<<<blocks_for(n), 256, 0, stream>>>(q, nq, nq_pad, dim, row_bytes, flip,
                                                           qcodes);
}

void remove_rows_i8(const int64_t* ids, int64_t n, int64_t size, int32_t* rowc,
                    unsigned long long* newly_removed, hipStream_t stream)
{
  if (n == 0) { return; }
  remove_kernel<<<blocks_for(n), 256, 0, stream>>>(ids, n, size, rowc, newly_removed);
}

void fill_u32(uint32_t* p, int64_t n, uint32_t v, hipStream_t stream)
{
  if (n == 0) { return; }
  const unsigned b = blocks_for(n) < 4096 ? blocks_for(n) : 4096;
  fill_kernel<uint32_t><<<b, 256, 0, stream>>>(p, n, v);
}

void fill_i32(int32_t* p, int64_t n, int32_t v, hipStream_t stream)
{
  if (n == 0) { return; }
  const unsigned b = blocks_for(n) < 4096 ? blocks_for(n) : 4096;
  fill_kernel<int32_t><<<b, 256, 0, stream>>>(p, n, v);
}

}  // namespace certex_amd
