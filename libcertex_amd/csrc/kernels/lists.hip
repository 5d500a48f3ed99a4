// k-means lists of the screening rows and the nearest lists of every query (gfx950).
//
// Reference contract: fit_lists and the probe's nearest_lists (detail/lists.cuh:137-210,
// 218-264): the lists are k-means clusters of the vectors trained on an evenly strided sample,
// every vector joins its nearest center, and a search first screens the p nearest lists of each
// query so that exact scores of their rows bound its threshold. Here the clusters live in
// screening coordinates (int8 codes or fp16 rows, squared L2). Center distances run on the MFMA
// units against centers quantized to the rows' type (int8 centers are rounded means, exact int32
// dot products; fp16 centers accumulate in fp32): the lists only order the rows and pick which of
// them a query meets first, so any rounding changes speed, never results.

#include "../kernels.hpp"

#include <cfloat>

namespace certex_amd {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

inline unsigned blocks_for(int64_t n, int block = 256) { return unsigned((n + block - 1) / block); }

/** Row tiles (16 rows) of a distance workgroup: its rows stay in LDS, at most 64 KB. */
inline int rows_tiles(int row_bytes) { return row_bytes <= 512 ? 4 : (row_bytes <= 1024 ? 2 : 1); }

/**
 * dot products of 16 centers x 16 rows over the row length: operand A = centers (lane l: center
 * c0 + l % 16), operand B = rows from LDS; lane l gets <center 4 (l / 16) + r, row l % 16>.
 */
template <bool F16>
__device__ inline v4f tile_dots(const int8_t* centers, int64_t c0, const int8_t* lrow, int ks_n,
                                int lane)
{
  const int8_t* ca = centers + (c0 + (lane & 15)) * int64_t(ks_n) * 64 + (lane >> 4) * 16;
  const int8_t* rb = lrow + (lane & 15) * ks_n * 64 + (lane >> 4) * 16;
  if constexpr (F16) {
    v4f acc = {0, 0, 0, 0};
    for (int ks = 0; ks < ks_n; ++ks) {
      const v8h a = *reinterpret_cast<const v8h*>(ca + 64 * ks);
      const v8h b = *reinterpret_cast<const v8h*>(rb + 64 * ks);
      acc         = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc, 0, 0, 0);
    }
    return acc;
  } else {
    v4i acc = {0, 0, 0, 0};
    for (int ks = 0; ks < ks_n; ++ks) {
      const v4i a = *reinterpret_cast<const v4i*>(ca + 64 * ks);
      const v4i b = *reinterpret_cast<const v4i*>(rb + 64 * ks);
      acc         = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, acc, 0, 0, 0);
    }
    return v4f{float(acc[0]), float(acc[1]), float(acc[2]), float(acc[3])};
  }
}

/**
 * Center distances of 16 * RT rows per workgroup: dist(row, c) = cterm[c] - <row, center c>
 * (cterm = |center|^2 / 2, so the order is that of |row - center|^2). The rows sit in LDS; wave w
 * takes the center tiles w, w + 4, ... (n_centers is a multiple of 64; padding centers carry
 * cterm = +inf). ARGMIN: out[row] = the nearest center (ties to the lower center); otherwise
 * dist[row, :] is written (row stride n_centers).
 */
template <bool F16, bool ARGMIN>
__global__ __launch_bounds__(256) void center_dist_kernel(const int8_t* rows, int64_t n,
                                                          int row_bytes, int rt,
                                                          const int8_t* centers,
                                                          const float* cterm, int n_centers,
                                                          int32_t* out, float* dist)
{
  extern __shared__ __attribute__((aligned(16))) int8_t lrows[];  // [16 rt, row_bytes]
  __shared__ float wbest[4][64];
  __shared__ int wbi[4][64];
  const int tid     = threadIdx.x;
  const int lane    = tid & 63;
  const int wave    = tid >> 6;
  const int ks_n    = row_bytes / 64;
  const int64_t r0  = int64_t(blockIdx.x) * 16 * rt;
  const int units   = 16 * rt * row_bytes / 16;
  for (int u = tid; u < units; u += 256) {
    const int64_t r = r0 + (u * 16) / row_bytes;
    v4i v           = {0, 0, 0, 0};
    if (r < n) { v = reinterpret_cast<const v4i*>(rows + r0 * row_bytes)[u]; }
    reinterpret_cast<v4i*>(lrows)[u] = v;
  }
  __syncthreads();

  float best[4];
  int bi[4];
  for (int t = 0; t < 4; ++t) {
    best[t] = INFINITY;
    bi[t]   = INT32_MAX;
  }
  for (int ct = wave; ct * 16 < n_centers; ct += 4) {
    const int64_t c0 = int64_t(ct) * 16;
    const v4f ch     = *reinterpret_cast<const v4f*>(cterm + c0 + (lane >> 4) * 4);
    for (int t = 0; t < rt; ++t) {
      const v4f d = tile_dots<F16>(centers, c0, lrows + t * 16 * row_bytes, ks_n, lane);
      v4f s;
      for (int r = 0; r < 4; ++r) { s[r] = ch[r] - d[r]; }
      if constexpr (ARGMIN) {
        for (int r = 0; r < 4; ++r) {  // centers ascend within a lane: strict keeps the lower
          if (s[r] < best[t]) {
            best[t] = s[r];
            bi[t]   = int(c0) + (lane >> 4) * 4 + r;
          }
        }
      } else {
        const int64_t row = r0 + t * 16 + (lane & 15);
        if (row < n) {
          *reinterpret_cast<v4f*>(dist + row * n_centers + c0 + (lane >> 4) * 4) = s;
        }
      }
    }
  }
  if constexpr (ARGMIN) {
    for (int t = 0; t < rt; ++t) {
      // the four lanes of one row (lane % 16) hold different centers
      float v = best[t];
      int i   = bi[t];
      for (int off = 16; off <= 32; off <<= 1) {
        const float ov = __shfl_xor(v, off);
        const int oi   = __shfl_xor(i, off);
        if (ov < v || (ov == v && oi < i)) {
          v = ov;
          i = oi;
        }
      }
      if (lane < 16) {
        wbest[wave][t * 16 + lane] = v;
        wbi[wave][t * 16 + lane]   = i;
      }
    }
    __syncthreads();
    if (tid < 16 * rt) {
      float v = wbest[0][tid];
      int i   = wbi[0][tid];
      for (int w = 1; w < 4; ++w) {
        const float ov = wbest[w][tid];
        const int oi   = wbi[w][tid];
        if (ov < v || (ov == v && oi < i)) {
          v = ov;
          i = oi;
        }
      }
      if (r0 + tid < n) { out[r0 + tid] = i < n_centers ? i : 0; }
    }
  }
}

/**
 * lists[q, 0 .. p) = the p smallest of dist[q, 0 .. n_lists) in ascending order, ties to the lower
 * list. One wave per query: every lane keeps its own p best, then p rounds of a wave argmin pop
 * the heads.
 */
__global__ __launch_bounds__(256) void top_lists_kernel(const float* dist, int64_t nq,
                                                        int n_lists, int ld, int p, int32_t* lists)
{
  const int64_t q = (blockIdx.x * int64_t(blockDim.x) + threadIdx.x) >> 6;
  const int lane  = threadIdx.x & 63;
  if (q >= nq) { return; }
  float bv[kMaxProbe];
  int bi[kMaxProbe];
#pragma unroll
  for (int j = 0; j < kMaxProbe; ++j) {
    bv[j] = INFINITY;
    bi[j] = INT32_MAX;
  }
  for (int c = lane; c < n_lists; c += 64) {
    const float v = dist[q * ld + c];
    if (!(v < bv[kMaxProbe - 1])) { continue; }
    // insertion after the entries <= v (lists ascend per lane, so equal values keep list order)
#pragma unroll
    for (int j = kMaxProbe - 1; j > 0; --j) {
      const bool up   = v < bv[j - 1];  // v goes above j: slot j takes slot j - 1's entry
      const bool here = !up && v < bv[j];
      const float nv  = up ? bv[j - 1] : (here ? v : bv[j]);
      const int ni    = up ? bi[j - 1] : (here ? c : bi[j]);
      bv[j]           = nv;
      bi[j]           = ni;
    }
    if (v < bv[0]) {
      bv[0] = v;
      bi[0] = c;
    }
  }
  for (int r = 0; r < p; ++r) {
    float v = bv[0];
    int i   = bi[0];
    for (int off = 32; off > 0; off >>= 1) {
      const float ov = __shfl_xor(v, off);
      const int oi   = __shfl_xor(i, off);
      if (ov < v || (ov == v && oi < i)) {
        v = ov;
        i = oi;
      }
    }
    if (lane == 0) { lists[q * p + r] = i < n_lists ? i : -1; }
    if (bi[0] == i) {  // the winner's lane pops its head
#pragma unroll
      for (int j = 0; j + 1 < kMaxProbe; ++j) {
        bv[j] = bv[j + 1];
        bi[j] = bi[j + 1];
      }
      bv[kMaxProbe - 1] = INFINITY;
      bi[kMaxProbe - 1] = INT32_MAX;
    }
  }
}

__device__ inline float element(const int8_t* rows, bool f16, int64_t i)
{
  return f16 ? float(reinterpret_cast<const _Float16*>(rows)[i]) : float(rows[i]);
}

/** sums[assign[i], :] += row i, counts[assign[i]] += 1 (width elements per row). */
__global__ void center_sums_kernel(const int8_t* rows, bool f16, int64_t n, int width,
                                   const int32_t* assign, int n_centers, float* sums,
                                   unsigned int* counts)
{
  const int64_t t = blockIdx.x * int64_t(blockDim.x) + threadIdx.x;
  if (t >= n * width) { return; }
  const int64_t i = t / width;
  const int j     = int(t % width);
  const int c     = assign[i];
  if (c < 0 || c >= n_centers) { return; }
  atomicAdd(sums + int64_t(c) * width + j, element(rows, f16, t));
  if (j == 0) { atomicAdd(counts + c, 1u); }
}

/**
 * Center c (one workgroup): the mean of its rows (a center without rows keeps its place), its copy
 * in the rows' type (int8 rounded and clamped to [-127, 127], or fp16) and cterm = |copy|^2 / 2.
 * Centers c >= n_centers up to the padded count get zero rows and cterm = +inf.
 */
__global__ __launch_bounds__(256) void finish_centers_kernel(const float* sums,
                                                             const unsigned int* counts,
                                                             int n_centers, int width, bool f16,
                                                             float* centers, int8_t* centers_q,
                                                             float* cterm)
{
  const int c = blockIdx.x;
  __shared__ float part[256];
  float nn = 0;
  for (int j = threadIdx.x; j < width; j += blockDim.x) {
    float v = 0;
    if (c < n_centers) {
      v = centers[int64_t(c) * width + j];
      if (counts != nullptr && counts[c] > 0) { v = sums[int64_t(c) * width + j] / float(counts[c]); }
      centers[int64_t(c) * width + j] = v;
    }
    float qv;
    if (f16) {
      const _Float16 h = _Float16(v);
      reinterpret_cast<_Float16*>(centers_q)[int64_t(c) * width + j] = h;
      qv = float(h);
    } else {
      const float r = fminf(fmaxf(rintf(v), -127.0f), 127.0f);
      centers_q[int64_t(c) * width + j] = int8_t(r);
      qv = r;
    }
    nn = fmaf(qv, qv, nn);
  }
  part[threadIdx.x] = nn;
  __syncthreads();
  for (int s = blockDim.x / 2; s > 0; s >>= 1) {
    if (threadIdx.x < s) { part[threadIdx.x] += part[threadIdx.x + s]; }
    __syncthreads();
  }
  if (threadIdx.x == 0) { cterm[c] = c < n_centers ? part[0] / 2 : INFINITY; }
}

/** centers[c, :] = row ids[c] as floats. */
__global__ void rows_to_centers_kernel(const int8_t* rows, bool f16, const int32_t* ids,
                                       int n_centers, int width, float* centers)
{
  const int64_t t = blockIdx.x * int64_t(blockDim.x) + threadIdx.x;
  if (t >= int64_t(n_centers) * width) { return; }
  const int64_t c = t / width;
  const int j     = int(t % width);
  centers[t]      = element(rows, f16, int64_t(ids[c]) * width + j);
}

template <bool ARGMIN>
void launch_dist(const void* rows, bool f16, int64_t n, int row_bytes, const void* centers_q,
                 const float* cterm, int n_centers_pad, int32_t* out, float* dist,
                 hipStream_t stream)
{
  if (n == 0) { return; }
  const int rt        = rows_tiles(row_bytes);
  const unsigned grid = unsigned((n + 16 * rt - 1) / (16 * rt));
  const size_t lds    = size_t(16) * rt * row_bytes;
  const auto* r       = static_cast<const int8_t*>(rows);
  const auto* c       = static_cast<const int8_t*>(centers_q);
  auto go             = [&](auto kernel) {
    if (lds > 32768) {  // the widest fp16 rows: 64 KB of rows per workgroup
      (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
    }
    kernel<<<grid, 256, lds, stream>>>(r, n, row_bytes, rt, c, cterm, n_centers_pad, out, dist);
  };
  if (f16) {
    go(center_dist_kernel<true, ARGMIN>);
  } else {
    go(center_dist_kernel<false, ARGMIN>);
  }
}

}  // namespace

void nearest_centers(const void* rows, bool f16, int64_t n, int row_bytes, const void* centers_q,
                     const float* cterm, int n_centers_pad, int32_t* out, hipStream_t stream)
{
  launch_dist<true>(rows, f16, n, row_bytes, centers_q, cterm, n_centers_pad, out, nullptr,
                    stream);
}

void center_distances(const void* rows, bool f16, int64_t n, int row_bytes,
                      const void* centers_q, const float* cterm, int n_centers_pad, float* dist,
                      hipStream_t stream)
{
  launch_dist<false>(rows, f16, n, row_bytes, centers_q, cterm, n_centers_pad, nullptr, dist,
                     stream);
}

void nearest_lists(const float* dist, int64_t nq, int n_lists, int ld, int p, int32_t* lists,
                   hipStream_t stream)
{
  if (nq == 0) { return; }
  top_lists_kernel<<<blocks_for(nq * 64), 256, 0, stream>>>(dist, nq, n_lists, ld, p, lists);
}

void center_sums(const void* rows, bool f16, int64_t n, int width, const int32_t* assign,
                 int n_centers, float* sums, unsigned int* counts, hipStream_t stream)
{
  if (n == 0) { return; }
  center_sums_kernel<<<blocks_for(n * width), 256, 0, stream>>>(
    static_cast<const int8_t*>(rows), f16, n, width, assign, n_centers, sums, counts);
}

void finish_centers(const float* sums, const unsigned int* counts, int n_centers,
                    int n_centers_pad, int width, bool f16, float* centers, void* centers_q,
                    float* cterm, hipStream_t stream)
{
  if (n_centers_pad == 0) { return; }
  finish_centers_kernel<<<unsigned(n_centers_pad), 256, 0, stream>>>(
    sums, counts, n_centers, width, f16, centers, static_cast<int8_t*>(centers_q), cterm);
}

void rows_to_centers(const void* rows, bool f16, const int32_t* ids, int n_centers, int width,
                     float* centers, hipStream_t stream)
{
  if (n_centers == 0) { return; }
  rows_to_centers_kernel<<<blocks_for(int64_t(n_centers) * width), 256, 0, stream>>>(
    static_cast<const int8_t*>(rows), f16, ids, n_centers, width, centers);
}

}  // namespace certex_amd
