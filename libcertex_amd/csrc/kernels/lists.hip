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

#include <algorithm>
#include <cfloat>
#include <stdexcept>

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

/**
 * The 8 nearest lists of 64 queries per workgroup (int8 codes of 64 KS bytes): center distances
 * cterm[c] - <q', center c> on the MFMA (operand A the centers, B the 4 query tiles held in
 * registers, so that a center tile is read once for 64 queries). A lane sees the values (query
 * 16 qt + lane % 16, center 4 (lane / 16) + r) of every W-th center tile, a fixed 32nd of the
 * centers, and keeps the best two of them; the 64 candidates of a query (two from each of its 4
 * lanes in each of the 8 waves) meet in LDS (candidate-major, so that the queries' threads read
 * consecutive words), where one thread per query keeps its 8 best (ties to the lower list) and
 * counts the query into counts[list] (the pairs per list of list_anchor_groups). These are the 8
 * nearest lists unless three of them share a 32nd (the lists choose anchors near the query, so a
 * near list in place of a nearer one changes speed, never results; keeping one list per 32nd
 * measured 4% more survivors at config 2, with a tail past the small re-rank's buckets). No distance matrix is
 * written. Centers of cterm +inf (padding, lists left out) are never picked.
 */
template <int KS>
__global__ __launch_bounds__(512) void nearest_lists_i8_kernel(const int8_t* qcodes, int64_t nq,
                                                               const int8_t* centers,
                                                               const float* cterm, int n_centers,
                                                               int32_t* lists, int32_t* counts)
{
  constexpr int ROWB = 64 * KS;
  constexpr int P    = kMaxProbe;
  constexpr int W    = 8;           // waves: each takes every W-th center tile
  constexpr int QT   = 4;           // query tiles of the workgroup
  constexpr int NC   = 4 * W * 2;   // candidates of a query: two per lane group
  __shared__ float cv[NC][16 * QT];
  __shared__ int ci[NC][16 * QT];
  const int lane   = threadIdx.x & 63;
  const int wave   = threadIdx.x >> 6;
  const int64_t q0 = int64_t(blockIdx.x) * 16 * QT;
  v4i qb[QT][KS];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int64_t q  = q0 + 16 * qt + (lane & 15);
    const int64_t qr = q < nq ? q : nq - 1;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      qb[qt][ks] = *reinterpret_cast<const v4i*>(qcodes + qr * ROWB + 64 * ks + 16 * (lane >> 4));
    }
  }
  // per query tile, the lane's two best, b0 <= b1 (centers grow along a lane: strict < keeps the
  // lower center on ties)
  float b0[QT], b1[QT];
  int i0[QT], i1[QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    b0[qt] = b1[qt] = INFINITY;
    i0[qt] = i1[qt] = INT32_MAX;
  }
  constexpr int U = 4;  // tiles whose loads are in flight together
  for (int ct0 = wave * 16; ct0 < n_centers; ct0 += 16 * W * U) {
    v4i a[U][KS];
    v4f ch[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c0 = ct0 + 16 * W * u < n_centers ? ct0 + 16 * W * u : ct0;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        a[u][ks] = *reinterpret_cast<const v4i*>(centers + int64_t(c0 + (lane & 15)) * ROWB +
                                                 64 * ks + 16 * (lane >> 4));
      }
      ch[u] = *reinterpret_cast<const v4f*>(cterm + c0 + 4 * (lane >> 4));
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (ct0 + 16 * W * u >= n_centers) { break; }
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        v4i acc = {0, 0, 0, 0};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[u][ks], qb[qt][ks], acc, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float v  = ch[u][r] - float(acc[r]);
          const int c    = ct0 + 16 * W * u + 4 * (lane >> 4) + r;
          const bool lt0 = v < b0[qt], lt1 = v < b1[qt];
          b1[qt]         = lt0 ? b0[qt] : (lt1 ? v : b1[qt]);
          i1[qt]         = lt0 ? i0[qt] : (lt1 ? c : i1[qt]);
          b0[qt]         = lt0 ? v : b0[qt];
          i0[qt]         = lt0 ? c : i0[qt];
        }
      }
    }
  }
  const int grp = wave * 4 + (lane >> 4);
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int ql        = 16 * qt + (lane & 15);
    cv[2 * grp][ql]     = b0[qt];
    ci[2 * grp][ql]     = i0[qt];
    cv[2 * grp + 1][ql] = b1[qt];
    ci[2 * grp + 1][ql] = i1[qt];
  }
  __syncthreads();
  const int ql    = threadIdx.x;
  const int64_t q = q0 + ql;
  if (ql >= 16 * QT || q >= nq) { return; }
  float bv[P];
  int bi[P];
#pragma unroll
  for (int r = 0; r < P; ++r) {
    bv[r] = INFINITY;
    bi[r] = INT32_MAX;
  }
  for (int c = 0; c < NC; ++c) {
    const float v = cv[c][ql];
    const int i   = ci[c][ql];
    // insertion by (value, list): the candidates do not arrive in list order
    if (!(v < bv[P - 1] || (v == bv[P - 1] && i < bi[P - 1]))) { continue; }
    int at = P - 1;
    while (at > 0 && (v < bv[at - 1] || (v == bv[at - 1] && i < bi[at - 1]))) {
      bv[at] = bv[at - 1];
      bi[at] = bi[at - 1];
      --at;
    }
    bv[at] = v;
    bi[at] = i;
  }
#pragma unroll
  for (int r = 0; r < P; ++r) {
    const int i = bi[r] < n_centers && bv[r] < INFINITY ? bi[r] : -1;
    lists[q * P + r] = i;
    if (i >= 0) { atomicAdd(counts + i, 1); }
  }
}

/** Pairs of a list per workgroup of list_anchor_groups_kernel. */
constexpr int kSlicePairs = 32;

/**
 * start[j] = the exclusive prefix sum of counts[0, L) (start[L] = the total), cursor = start, and
 * slice[j] = the exclusive prefix sum of ceil(counts[j] / kSlicePairs) (slice[L] = the total): the
 * first workgroup of list j in list_anchor_groups_kernel, and slices[b] = {list, first pair, end
 * pair, 0} of its workgroup b. One workgroup of 1,024 threads, each over a run of consecutive
 * lists.
 */
__global__ __launch_bounds__(1024) void list_pair_scan_kernel(const int32_t* counts, int L,
                                                              int32_t* start, int32_t* cursor,
                                                              int32_t* slice, int4* slices)
{
  __shared__ int part[1024], spart[1024];
  const int t   = threadIdx.x;
  const int per = (L + 1023) / 1024;
  const int b   = t * per;
  const int e   = b + per < L ? b + per : L;
  int sum = 0, ssum = 0;
  for (int j = b; j < e; ++j) {
    sum += counts[j];
    ssum += (counts[j] + kSlicePairs - 1) / kSlicePairs;
  }
  part[t]  = sum;
  spart[t] = ssum;
  __syncthreads();
  for (int off = 1; off < 1024; off <<= 1) {
    const int v  = t >= off ? part[t - off] : 0;
    const int sv = t >= off ? spart[t - off] : 0;
    __syncthreads();
    part[t] += v;
    spart[t] += sv;
    __syncthreads();
  }
  int run = part[t] - sum, srun = spart[t] - ssum;
  for (int j = b; j < e; ++j) {
    start[j]     = run;
    cursor[j]    = run;
    slice[j]     = srun;
    const int ns = (counts[j] + kSlicePairs - 1) / kSlicePairs;
    for (int x = 0; x < ns; ++x) {
      const int b0     = run + kSlicePairs * x;
      const int b1     = b0 + kSlicePairs < run + counts[j] ? b0 + kSlicePairs : run + counts[j];
      slices[srun + x] = int4{j, b0, b1, 0};
    }
    run += counts[j];
    srun += ns;
  }
  if (t == 1023) {
    start[L] = part[t];
    slice[L] = spart[t];
  }
}

/** pairs[cursor[j]++] = e for every pair e of lists[0, n) naming list j (the order within a list
 *  is that of the atomics; each pair writes its own columns, so it does not matter). A pair
 *  without a list (-1) gets its 64 columns of gmax (64 p per query) at the lowest value here. */
__global__ void list_pair_fill_kernel(const int32_t* lists, int64_t n, int p, int32_t* cursor,
                                      int32_t* pairs, int32_t* gmax)
{
  for (int64_t e = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; e < n;
       e += int64_t(gridDim.x) * blockDim.x) {
    const int32_t j = lists[e];
    if (j >= 0) {
      pairs[atomicAdd(cursor + j, 1)] = int32_t(e);
    } else {
      int32_t* col = gmax + (e / p) * 64 * int64_t(p) + (e % p) * 64;
      for (int g = 0; g < 64; ++g) { col[g] = INT32_MIN; }
    }
  }
}

/**
 * Group table of the list anchors (int8 rows of ROWB = 128 or 256 bytes). Workgroup b serves list j
 * (slice[j] <= b < slice[j + 1]) and its pairs (query q, slot t) [start[j] + kSlicePairs s, + 32),
 * s = b - slice[j]. The anchors of j, its stored rows offsets[j] + i stride (i < ceil(rows of j /
 * stride)), go into LDS in chunks of AC; anchor i joins group i % 64 of the pair's 64 columns
 * gmax[q, 64 t, +64), so the groups hold distinct rows. The scores run on the int8 MFMA: operand A
 * 16 anchors (from LDS; chunk c of anchor u in slot c ^ (u % 8) of its row), B 16 pairs' queries
 * (registers, straight from the query codes), C the anchors' row terms, so lane l gets anchor 16 T +
 * 4 (l / 16) + r of pair l % 16, in group 16 (T % 4) + 4 (l / 16) + r. Wave w takes the pairs'
 * tile w % 2 and the anchor tiles T = w / 2, w / 2 + 2, ...: the two waves of a pair tile keep
 * disjoint groups (T % 4 even or odd), 8 maxima per lane. A later chunk of a long list merges into
 * the columns the earlier wrote (the same lanes own them).
 */
template <int ROWB>
__global__ __launch_bounds__(256) void list_anchor_groups_kernel(
  const int8_t* codes, const int32_t* rowc, const int8_t* qcodes, int p, const int64_t* offsets,
  int n_lists, int64_t stride, const int32_t* slice, const int4* slices, const int32_t* pairs,
  int32_t* gmax)
{
  constexpr int KS  = ROWB / 64;      // 64-byte k-slices of a row
  constexpr int NCH = ROWB / 16;      // 16-byte chunks of a row
  // anchors per LDS chunk, a multiple of 64: 24 KB of 128-byte rows (a list of 10M rows in 4,096
  // lists holds about 150 anchors at stride 16), 32 KB of 256-byte rows
  constexpr int AC  = ROWB == 128 ? 192 : 128;
  static_assert(kSlicePairs == 32, "two pair tiles per workgroup");
  __shared__ v4i la[AC * NCH];
  __shared__ __attribute__((aligned(16))) int32_t lc[AC];
  const int b = blockIdx.x;
  if (b >= slice[n_lists]) { return; }
  const int4 sl  = slices[b];
  const int j    = sl.x;
  const int b0   = sl.y;
  const int b1   = sl.z;
  const int tid  = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int pt   = wave & 1;   // pair tile
  const int par  = wave >> 1;  // anchor tiles of this parity
  const int64_t r0 = offsets[j];
  const int64_t na = (offsets[j + 1] - r0 + stride - 1) / stride;
  const int64_t ng = 64 * int64_t(p);
  const int pl   = 16 * pt + (lane & 15);  // the lane's pair in the slice
  const bool own = b0 + pl < b1;
  // the pair's query fragments (operand B), loaded while the anchors are copied
  const int e0    = pairs[own ? b0 + pl : b0];
  v4i qv[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    qv[ks] = *reinterpret_cast<const v4i*>(qcodes + int64_t(e0 / p) * ROWB + 64 * ks + 16 * (lane >> 4));
  }
  for (int64_t a0 = 0; a0 < na; a0 += AC) {
    const int nc = int(na - a0 < AC ? na - a0 : AC);
    if (a0 > 0) { __syncthreads(); }  // the previous chunk's reads are done
#pragma unroll 4
    for (int u = tid; u < nc * NCH; u += 256) {
      const int i = u / NCH, c = u % NCH;
      la[i * NCH + (c ^ (i & 7))] =
        *reinterpret_cast<const v4i*>(codes + (r0 + (a0 + i) * stride) * ROWB + 16 * c);
    }
    for (int i = tid; i < nc; i += 256) { lc[i] = rowc[r0 + (a0 + i) * stride]; }
    __syncthreads();
    if (b0 + 16 * pt >= b1) { continue; }  // no pair in this wave's tile
    int32_t run[2][4];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int r = 0; r < 4; ++r) { run[h][r] = INT32_MIN; }
    }
    const int nt = (nc + 15) / 16;
    for (int T = par; T < nt; T += 2) {
      const int ua = 16 * T + (lane & 15);  // the anchor of the lane's A operand
      v4i acc = *reinterpret_cast<const v4i*>(lc + 16 * T + 4 * (lane >> 4));
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const v4i a = la[ua * NCH + ((4 * ks + (lane >> 4)) ^ (ua & 7))];
        acc         = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, qv[ks], acc, 0, 0, 0);
      }
      const int h = (T >> 1) & 1;  // T % 4 = par + 2 h
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const bool live = 16 * T + 4 * (lane >> 4) + r < nc;
        if (live && acc[r] > run[h][r]) { run[h][r] = acc[r]; }
      }
    }
    if (own) {
      int32_t* row = gmax + int64_t(e0 / p) * ng + (e0 % p) * 64;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          // anchor a0 + 16 T + 4 (l / 16) + r, a0 a multiple of 64: group 16 (T % 4) + 4 (l / 16) + r
          int32_t* col = row + 16 * (par + 2 * h) + 4 * (lane >> 4) + r;
          if (a0 == 0) {
            *col = run[h][r];
          } else if (run[h][r] > *col) {
            *col = run[h][r];
          }
        }
      }
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

void nearest_lists_i8(const int8_t* qcodes, int row_bytes, int64_t nq, const void* centers_q,
                      const float* cterm, int n_centers_pad, int n_lists, int32_t* lists,
                      void* temp, hipStream_t stream)
{
  if (nq == 0) { return; }
  auto* counts = static_cast<int32_t*>(temp);  // the pairs per list (list_anchor_groups' temp)
  fill_u32(reinterpret_cast<uint32_t*>(counts), n_lists, 0, stream);
  const unsigned grid = unsigned((nq + 63) / 64);
  const auto* c       = static_cast<const int8_t*>(centers_q);
  if (row_bytes == 128) {
    nearest_lists_i8_kernel<2><<<grid, 512, 0, stream>>>(qcodes, nq, c, cterm, n_centers_pad,
                                                         lists, counts);
  } else if (row_bytes == 256) {
    nearest_lists_i8_kernel<4><<<grid, 512, 0, stream>>>(qcodes, nq, c, cterm, n_centers_pad,
                                                         lists, counts);
  } else {
    throw std::logic_error("certex: the nearest lists of int8 queries take rows of 128 or 256 bytes");
  }
}

size_t list_anchor_temp_bytes(int64_t nq, int n_lists)
{
  const int64_t n = nq * kMaxProbe;
  return size_t(4 * (int64_t(n_lists) + 1) + (n + 3) / 4 * 4) * 4 +
         size_t(n_lists + (n + kSlicePairs - 1) / kSlicePairs) * sizeof(int4);
}

void list_anchor_groups(const int8_t* codes, const int32_t* rowc, int row_bytes,
                        const int8_t* qcodes, int64_t nq, const int32_t* lists,
                        const int64_t* offsets, int n_lists, int64_t stride, void* temp,
                        int32_t* gmax, hipStream_t stream)
{
  if (nq == 0 || n_lists == 0) { return; }
  if (row_bytes != 128 && row_bytes != 256) {
    throw std::logic_error("certex: list anchors take rows of 128 or 256 bytes");
  }
  if (stride < 1) { throw std::logic_error("certex: bad list anchor stride"); }
  const int64_t n = nq * kMaxProbe;
  auto* counts    = static_cast<int32_t*>(temp);
  auto* start     = counts + (n_lists + 1);
  auto* cursor    = start + (n_lists + 1);
  auto* slice     = cursor + (n_lists + 1);
  auto* pairs      = slice + (n_lists + 1);
  auto* slices     = reinterpret_cast<int4*>(pairs + (n + 3) / 4 * 4);
  const unsigned g = unsigned(std::min<int64_t>((n + 255) / 256, 1024));
  list_pair_scan_kernel<<<1, 1024, 0, stream>>>(counts, n_lists, start, cursor, slice, slices);
  list_pair_fill_kernel<<<g, 256, 0, stream>>>(lists, n, kMaxProbe, cursor, pairs, gmax);
  // at most one partial slice per list: n_lists + n / kSlicePairs workgroups cover every slice
  const unsigned wg = unsigned(n_lists + (n + kSlicePairs - 1) / kSlicePairs);
  if (row_bytes == 128) {
    list_anchor_groups_kernel<128><<<wg, 256, 0, stream>>>(codes, rowc, qcodes, kMaxProbe, offsets,
                                                           n_lists, stride, slice, slices,
                                                           pairs, gmax);
  } else {
    list_anchor_groups_kernel<256><<<wg, 256, 0, stream>>>(codes, rowc, qcodes, kMaxProbe, offsets,
                                                           n_lists, stride, slice, slices,
                                                           pairs, gmax);
  }
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
