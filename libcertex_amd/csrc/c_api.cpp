// C API over the C++ API (reference c/src/neighbors/certex.cpp:1-371, c/src/core/exceptions.hpp
// and c/src/core/interop.hpp). Every entry point turns C++ exceptions into CUVS_ERROR and the
// last-error text of the calling thread; a successful call clears that text.

#include <cuvs/neighbors/certex.h>

#include "certex_state.hpp"

#include <cstring>
#include <exception>
#include <fstream>
#include <map>
#include <mutex>
#include <string>

namespace {

namespace certex = cuvs::neighbors::certex;

thread_local std::string t_last_error;
thread_local bool t_has_error = false;

template <typename Fn>
cuvsError_t translate(Fn fn)
{
  try {
    fn();
    t_has_error = false;
    t_last_error.clear();
    return CUVS_SUCCESS;
  } catch (std::exception const& e) {
    t_last_error = e.what();
    t_has_error  = true;
  } catch (...) {
    t_last_error = "unknown exception";
    t_has_error  = true;
  }
  return CUVS_ERROR;
}

auto is_device(DLTensor const& t) -> bool
{
  return t.device.device_type == kDLROCM || t.device.device_type == kDLCUDA ||
         t.device.device_type == kDLCUDAManaged;
}

auto is_host(DLTensor const& t) -> bool
{
  return t.device.device_type == kDLCPU || t.device.device_type == kDLCUDAHost ||
         t.device.device_type == kDLROCMHost;
}

template <typename T>
auto code_of() -> uint8_t
{
  if constexpr (std::is_same_v<T, float> || std::is_same_v<T, certex::half_t>) {
    return kDLFloat;
  } else if constexpr (std::is_same_v<T, certex::bfloat16_t>) {
    return kDLBfloat;
  } else if constexpr (std::is_signed_v<T>) {
    return kDLInt;
  } else {
    return kDLUInt;
  }
}

/** Checks of reference interop.hpp:52-66: rank, data type, dense row-major layout. */
template <typename T>
void check_tensor(DLManagedTensor* m, int ndim, const char* what)
{
  certex::expects(m != nullptr, "certex: a tensor argument is NULL");
  DLTensor const& t = m->dl_tensor;
  if (t.ndim != ndim) {
    throw std::invalid_argument(std::string("certex: ") + what +
                                " has the wrong number of dimensions");
  }
  if (!(t.dtype.code == code_of<T>() && t.dtype.bits == 8 * sizeof(T) && t.dtype.lanes == 1)) {
    throw std::invalid_argument(std::string("certex: ") + what + " has the wrong data type");
  }
  if (t.strides != nullptr) {
    int64_t expect = 1;
    for (int i = ndim - 1; i >= 0; --i) {
      certex::expects(t.shape[i] == 1 || t.strides[i] == expect,
                      "certex: the DLPack tensor must be dense and row major");
      expect *= t.shape[i];
    }
  }
}

template <typename T>
auto data_of(DLTensor const& t) -> T*
{
  return reinterpret_cast<T*>(static_cast<char*>(t.data) + t.byte_offset);
}

template <typename T>
auto matrix_of(DLManagedTensor* m, const char* what) -> certex::matrix_view<const T>
{
  check_tensor<T>(m, 2, what);
  DLTensor const& t = m->dl_tensor;
  certex::expects(is_device(t) || is_host(t), "certex: unsupported DLPack device");
  certex::matrix_view<const T> v;
  v.data      = data_of<const T>(t);
  v.rows      = t.shape[0];
  v.cols      = t.shape[1];
  v.on_device = is_device(t);
  return v;
}

template <typename T>
auto device_data(DLManagedTensor* m, int ndim, const char* what) -> T*
{
  check_tensor<T>(m, ndim, what);
  certex::expects(is_device(m->dl_tensor), "certex: expected a tensor in device memory");
  return data_of<T>(m->dl_tensor);
}

auto res_of(cuvsResources_t res) -> cuvs::resources&
{
  certex::expects(res != 0, "certex: the resources handle is NULL");
  return *reinterpret_cast<cuvs::resources*>(res);
}

/** Call f with a value of the vector type of a DLPack data type (reference certex.cpp:62-76). */
template <typename F>
void dispatch(DLDataType dtype, F&& f)
{
  if (dtype.code == kDLFloat && dtype.bits == 32) {
    f(float{});
  } else if (dtype.code == kDLFloat && dtype.bits == 16) {
    f(certex::half_t{});
  } else if (dtype.code == kDLBfloat && dtype.bits == 16) {
    f(certex::bfloat16_t{});
  } else if (dtype.code == kDLInt && dtype.bits == 8) {
    f(int8_t{});
  } else if (dtype.code == kDLUInt && dtype.bits == 8) {
    f(uint8_t{});
  } else {
    throw std::invalid_argument("certex: vectors must be float32, float16, bfloat16, int8, or uint8");
  }
}

template <typename T>
auto as_index(cuvsCertexIndex const& index) -> certex::index<T>*
{
  certex::expects(index.addr != 0, "certex: the index is empty (build or deserialize it first)");
  return reinterpret_cast<certex::index<T>*>(index.addr);
}

auto to_cpp(cuvsCertexIndexParams const& p) -> certex::index_params
{
  certex::index_params out;
  out.metric            = static_cast<cuvs::distance::DistanceType>(int(p.metric));
  out.width             = p.width;
  out.variance          = p.variance;
  out.anchor_stride     = p.anchor_stride;
  out.pca_sample        = p.pca_sample;
  out.host_vectors      = p.host_vectors;
  out.n_lists           = p.n_lists;
  out.local_projections = p.local_projections;
  out.int8_rows         = p.int8_rows;
  return out;
}

auto to_cpp(cuvsCertexSearchParams const& p) -> certex::search_params
{
  certex::search_params out;
  out.anchors     = p.anchors;
  out.batch_size  = p.batch_size;
  out.probe_lists = p.probe_lists;
  return out;
}

}  // namespace

extern "C" {

cuvsError_t cuvsResourcesCreate(cuvsResources_t* res)
{
  return translate([=] { *res = reinterpret_cast<cuvsResources_t>(new cuvs::resources()); });
}

cuvsError_t cuvsResourcesDestroy(cuvsResources_t res)
{
  return translate([=] { delete reinterpret_cast<cuvs::resources*>(res); });
}

cuvsError_t cuvsStreamSet(cuvsResources_t res, void* stream)
{
  return translate([=] { res_of(res).set_stream(stream); });
}

cuvsError_t cuvsStreamGet(cuvsResources_t res, void** stream)
{
  return translate([=] { *stream = res_of(res).stream(); });
}

cuvsError_t cuvsStreamSync(cuvsResources_t res)
{
  return translate([=] { res_of(res).sync(); });
}

const char* cuvsGetLastErrorText(void) { return t_has_error ? t_last_error.c_str() : nullptr; }

void cuvsSetLastErrorText(const char* error)
{
  t_has_error  = error != nullptr;
  t_last_error = error != nullptr ? error : "";
}

cuvsError_t cuvsCertexIndexParamsCreate(cuvsCertexIndexParams_t* params)
{
  return translate([=] {
    certex::index_params d;
    *params = new cuvsCertexIndexParams{static_cast<cuvsDistanceType>(int(d.metric)),
                                        d.width,
                                        d.variance,
                                        d.anchor_stride,
                                        d.pca_sample,
                                        d.host_vectors,
                                        d.n_lists,
                                        d.local_projections,
                                        d.int8_rows};
  });
}

cuvsError_t cuvsCertexIndexParamsDestroy(cuvsCertexIndexParams_t params)
{
  return translate([=] { delete params; });
}

cuvsError_t cuvsCertexSearchParamsCreate(cuvsCertexSearchParams_t* params)
{
  return translate([=] {
    certex::search_params d;
    *params = new cuvsCertexSearchParams{d.anchors, d.batch_size, d.probe_lists};
  });
}

cuvsError_t cuvsCertexSearchParamsDestroy(cuvsCertexSearchParams_t params)
{
  return translate([=] { delete params; });
}

cuvsError_t cuvsCertexIndexCreate(cuvsCertexIndex_t* index)
{
  return translate([=] { *index = new cuvsCertexIndex{}; });
}

namespace {
// capacities reserved on handles that hold no index yet: the next build allocates them
std::mutex g_pending_mutex;
std::map<cuvsCertexIndex_t, int64_t> g_pending_capacity;

auto take_pending_capacity(cuvsCertexIndex_t index) -> int64_t
{
  std::lock_guard lk(g_pending_mutex);
  auto it = g_pending_capacity.find(index);
  if (it == g_pending_capacity.end()) { return 0; }
  const int64_t c = it->second;
  g_pending_capacity.erase(it);
  return c;
}
}  // namespace

cuvsError_t cuvsCertexIndexDestroy(cuvsCertexIndex_t index)
{
  return translate([=] {
    if (index == nullptr) { return; }
    (void)take_pending_capacity(index);
    if (index->addr != 0) {
      dispatch(index->dtype, [&](auto tag) {
        delete reinterpret_cast<certex::index<decltype(tag)>*>(index->addr);
      });
    }
    delete index;
  });
}

cuvsError_t cuvsCertexIndexGetSize(cuvsCertexIndex_t index, int64_t* size)
{
  return translate([=] {
    dispatch(index->dtype, [&](auto tag) { *size = as_index<decltype(tag)>(*index)->size(); });
  });
}

cuvsError_t cuvsCertexIndexGetDim(cuvsCertexIndex_t index, int64_t* dim)
{
  return translate([=] {
    dispatch(index->dtype, [&](auto tag) { *dim = as_index<decltype(tag)>(*index)->dim(); });
  });
}

cuvsError_t cuvsCertexBuild(cuvsResources_t res,
                            cuvsCertexIndexParams_t params,
                            DLManagedTensor* dataset,
                            cuvsCertexIndex_t index)
{
  return translate([=] {
    certex::expects(index != nullptr && params != nullptr && dataset != nullptr,
                    "certex: NULL argument");
    certex::expects(index->addr == 0, "certex: the index handle already holds an index");
    auto& r    = res_of(res);
    auto p     = to_cpp(*params);
    p.capacity = take_pending_capacity(index);
    dispatch(dataset->dl_tensor.dtype, [&](auto tag) {
      using T = decltype(tag);
      auto* out =
        new certex::index<T>(certex::build<T>(r, p, matrix_of<T>(dataset, "the dataset")));
      index->dtype = dataset->dl_tensor.dtype;
      index->addr  = reinterpret_cast<uintptr_t>(out);
    });
  });
}

cuvsError_t cuvsCertexExtend(cuvsResources_t res,
                             DLManagedTensor* new_vectors,
                             cuvsCertexIndex_t index)
{
  return translate([=] {
    auto& r = res_of(res);
    dispatch(index->dtype, [&](auto tag) {
      using T = decltype(tag);
      certex::extend<T>(r, matrix_of<T>(new_vectors, "the new vectors"), as_index<T>(*index));
    });
  });
}

cuvsError_t cuvsCertexRemove(cuvsResources_t res, DLManagedTensor* ids, cuvsCertexIndex_t index)
{
  return translate([=] {
    auto& r        = res_of(res);
    const auto* p  = device_data<int64_t>(ids, 1, "the ids");
    const int64_t n = ids->dl_tensor.shape[0];
    dispatch(index->dtype,
             [&](auto tag) { certex::remove<decltype(tag)>(r, p, n, as_index<decltype(tag)>(*index)); });
  });
}

cuvsError_t cuvsCertexSetLabels(cuvsResources_t res,
                                DLManagedTensor* labels,
                                int64_t first,
                                cuvsCertexIndex_t index)
{
  return translate([=] {
    auto& r         = res_of(res);
    const auto* p   = device_data<int32_t>(labels, 1, "the labels");
    const int64_t n = labels->dl_tensor.shape[0];
    dispatch(index->dtype, [&](auto tag) {
      certex::set_labels<decltype(tag)>(r, p, n, as_index<decltype(tag)>(*index), first);
    });
  });
}

cuvsError_t cuvsCertexPartitionByLabels(cuvsResources_t res, cuvsCertexIndex_t index)
{
  return translate([=] {
    auto& r = res_of(res);
    dispatch(index->dtype, [&](auto tag) {
      certex::partition_by_labels<decltype(tag)>(r, as_index<decltype(tag)>(*index));
    });
  });
}

}  // extern "C"

namespace {

/** cuvsCertexSearch and cuvsCertexSearchNoAlloc: checks of the tensors and the filter, then the
 *  search (reference certex.cpp:113-143, 292-311). */
cuvsError_t search_c(cuvsResources_t res,
                     cuvsCertexSearchParams_t params,
                     cuvsCertexIndex_t index,
                     DLManagedTensor* queries,
                     DLManagedTensor* neighbors,
                     DLManagedTensor* distances,
                     cuvsFilter filter,
                     bool no_alloc)
{
  return translate([=] {
    auto& r      = res_of(res);
    const auto p = to_cpp(*params);
    certex::expects(queries->dl_tensor.dtype.code == index->dtype.code &&
                      queries->dl_tensor.dtype.bits == index->dtype.bits,
                    "certex: the queries must have the vector type of the index");
    dispatch(index->dtype, [&](auto tag) {
      using T   = decltype(tag);
      auto& idx = *as_index<T>(*index);
      auto q    = matrix_of<T>(queries, "the queries");
      certex::expects(q.on_device, "certex: expected a tensor in device memory");
      auto* nb = device_data<int64_t>(neighbors, 2, "the neighbors");
      auto* ds = device_data<float>(distances, 2, "the distances");
      const int64_t k = neighbors->dl_tensor.shape[1];
      certex::expects(neighbors->dl_tensor.shape[0] == q.rows &&
                        distances->dl_tensor.shape[0] == q.rows &&
                        distances->dl_tensor.shape[1] == k,
                      "output shapes do not match the queries");
      certex::filter f;
      if (filter.type == BITSET || filter.type == BITMAP) {
        auto* m = reinterpret_cast<DLManagedTensor*>(filter.addr);
        check_tensor<uint32_t>(m, 1, "the filter words");
        certex::expects(is_device(m->dl_tensor), "certex: the filter words must be on the device");
        const int64_t bits = filter.type == BITSET ? idx.size() : q.rows * idx.size();
        certex::expects(m->dl_tensor.shape[0] * 32 >= bits, "certex: too few filter words");
        f.type  = filter.type == BITSET ? certex::filter::kind::bitset : certex::filter::kind::bitmap;
        f.words = data_of<const uint32_t>(m->dl_tensor);
      } else {
        certex::expects(filter.type == NO_FILTER, "certex: unsupported filter type");
      }
      if (no_alloc) {
        certex::search_without_allocation<T>(r, p, idx, q, nb, ds, k, f);
      } else {
        certex::search<T>(r, p, idx, q, nb, ds, k, f);
      }
    });
  });
}

}  // namespace

extern "C" {

cuvsError_t cuvsCertexSearch(cuvsResources_t res,
                             cuvsCertexSearchParams_t params,
                             cuvsCertexIndex_t index,
                             DLManagedTensor* queries,
                             DLManagedTensor* neighbors,
                             DLManagedTensor* distances,
                             cuvsFilter filter)
{
  return search_c(res, params, index, queries, neighbors, distances, filter, false);
}

cuvsError_t cuvsCertexSearchNoAlloc(cuvsResources_t res,
                                    cuvsCertexSearchParams_t params,
                                    cuvsCertexIndex_t index,
                                    DLManagedTensor* queries,
                                    DLManagedTensor* neighbors,
                                    DLManagedTensor* distances,
                                    cuvsFilter filter)
{
  return search_c(res, params, index, queries, neighbors, distances, filter, true);
}

cuvsError_t cuvsCertexSearchWithLabels(cuvsResources_t res,
                                       cuvsCertexSearchParams_t params,
                                       cuvsCertexIndex_t index,
                                       DLManagedTensor* queries,
                                       DLManagedTensor* query_labels,
                                       DLManagedTensor* neighbors,
                                       DLManagedTensor* distances)
{
  return translate([=] {
    auto& r      = res_of(res);
    const auto p = to_cpp(*params);
    dispatch(index->dtype, [&](auto tag) {
      using T   = decltype(tag);
      auto& idx = *as_index<T>(*index);
      auto q    = matrix_of<T>(queries, "the queries");
      certex::expects(q.on_device, "certex: expected a tensor in device memory");
      // query labels in device or host memory (host labels spare the routed search a read-back)
      check_tensor<int32_t>(query_labels, 1, "the query labels");
      const DLTensor& lt = query_labels->dl_tensor;
      certex::expects(is_device(lt) || is_host(lt), "certex: unsupported DLPack device");
      const auto* ql = data_of<const int32_t>(lt);
      certex::expects(lt.shape[0] == q.rows, "one label per query");
      auto* nb        = device_data<int64_t>(neighbors, 2, "the neighbors");
      auto* ds        = device_data<float>(distances, 2, "the distances");
      const int64_t k = neighbors->dl_tensor.shape[1];
      certex::expects(neighbors->dl_tensor.shape[0] == q.rows &&
                        distances->dl_tensor.shape[0] == q.rows &&
                        distances->dl_tensor.shape[1] == k,
                      "output shapes do not match the queries");
      certex::search<T>(r, p, idx, q, ql, nb, ds, k, is_host(lt));
    });
  });
}

cuvsError_t cuvsCertexSerialize(cuvsResources_t res, const char* filename, cuvsCertexIndex_t index)
{
  return translate([=] {
    auto& r = res_of(res);
    certex::expects(filename != nullptr, "certex: NULL file name");
    dispatch(index->dtype, [&](auto tag) {
      certex::serialize<decltype(tag)>(r, std::string(filename), *as_index<decltype(tag)>(*index));
    });
  });
}

/** The vector type of a saved index from its leading NumPy descriptor (certex.cpp:146-158). */
static DLDataType dtype_of_file(const char* filename)
{
  std::ifstream is(filename, std::ios::binary);
  certex::expects(is.good(), "certex: cannot open the index file");
  char prefix[4] = {};
  is.read(prefix, 4);
  const std::string d(prefix + 1, 2);
  if (d == "f4") { return {kDLFloat, 32, 1}; }
  if (d == "f2") { return {kDLFloat, 16, 1}; }
  if (d == "b2") { return {kDLBfloat, 16, 1}; }
  if (d == "i1") { return {kDLInt, 8, 1}; }
  if (d == "u1") { return {kDLUInt, 8, 1}; }
  throw std::invalid_argument("certex: not a CertEx index file");
}

cuvsError_t cuvsCertexDeserialize(cuvsResources_t res,
                                  const char* filename,
                                  cuvsCertexIndex_t index)
{
  return translate([=] {
    auto& r = res_of(res);
    certex::expects(filename != nullptr, "certex: NULL file name");
    certex::expects(index->addr == 0, "certex: the index handle already holds an index");
    const DLDataType dtype = dtype_of_file(filename);
    dispatch(dtype, [&](auto tag) {
      using T = decltype(tag);
      auto* p = new certex::index<T>(r);
      try {
        certex::deserialize<T>(r, std::string(filename), p);
      } catch (...) {
        delete p;
        throw;
      }
      index->dtype = dtype;
      index->addr  = reinterpret_cast<uintptr_t>(p);
    });
  });
}

cuvsError_t cuvsCertexIndexGetRemoved(cuvsCertexIndex_t index, int64_t* n_removed)
{
  return translate([=] {
    dispatch(index->dtype,
             [&](auto tag) { *n_removed = as_index<decltype(tag)>(*index)->n_removed(); });
  });
}

cuvsError_t cuvsCertexIndexGetCapacity(cuvsCertexIndex_t index, int64_t* capacity)
{
  return translate([=] {
    dispatch(index->dtype,
             [&](auto tag) { *capacity = as_index<decltype(tag)>(*index)->capacity(); });
  });
}

cuvsError_t cuvsCertexIndexGetWidth(cuvsCertexIndex_t index, int32_t* width)
{
  return translate([=] {
    dispatch(index->dtype, [&](auto tag) { *width = as_index<decltype(tag)>(*index)->width(); });
  });
}

cuvsError_t cuvsCertexIndexGetMetric(cuvsCertexIndex_t index, cuvsDistanceType* metric)
{
  return translate([=] {
    dispatch(index->dtype, [&](auto tag) {
      *metric = static_cast<cuvsDistanceType>(int(as_index<decltype(tag)>(*index)->metric()));
    });
  });
}

cuvsError_t cuvsCertexIndexGetAnchorStride(cuvsCertexIndex_t index, int32_t* stride)
{
  return translate([=] {
    dispatch(index->dtype,
             [&](auto tag) { *stride = as_index<decltype(tag)>(*index)->anchor_stride(); });
  });
}

cuvsError_t cuvsCertexIndexHasLabels(cuvsCertexIndex_t index, bool* has_labels)
{
  return translate([=] {
    dispatch(index->dtype,
             [&](auto tag) { *has_labels = as_index<decltype(tag)>(*index)->has_labels(); });
  });
}

cuvsError_t cuvsCertexIndexGetHostVectors(cuvsCertexIndex_t index, bool* host_vectors)
{
  return translate([=] {
    dispatch(index->dtype,
             [&](auto tag) { *host_vectors = as_index<decltype(tag)>(*index)->host_vectors(); });
  });
}

cuvsError_t cuvsCertexIndexGetPartitioned(cuvsCertexIndex_t index, int64_t* n_partitioned)
{
  return translate([=] {
    dispatch(index->dtype, [&](auto tag) {
      *n_partitioned = as_index<decltype(tag)>(*index)->n_partitioned();
    });
  });
}

cuvsError_t cuvsCertexIndexGetLists(cuvsCertexIndex_t index, int32_t* n_lists, int64_t* n_listed)
{
  return translate([=] {
    dispatch(index->dtype, [&](auto tag) {
      auto const* idx = as_index<decltype(tag)>(*index);
      *n_lists        = idx->n_lists();
      *n_listed       = idx->n_lists() > 0 ? idx->list_offsets().back() : 0;
    });
  });
}

cuvsError_t cuvsCertexReserve(cuvsResources_t res, int64_t capacity, cuvsCertexIndex_t index)
{
  return translate([=] {
    certex::expects(index != nullptr, "certex: NULL argument");
    if (index->addr == 0) {  // no index yet: the next build allocates the capacity
      std::lock_guard lk(g_pending_mutex);
      g_pending_capacity[index] = capacity;
      return;
    }
    auto& r = res_of(res);
    dispatch(index->dtype, [&](auto tag) {
      certex::reserve<decltype(tag)>(r, capacity, as_index<decltype(tag)>(*index));
    });
  });
}

cuvsError_t cuvsCertexIndexListOrder(cuvsResources_t res,
                                     cuvsCertexIndex_t index,
                                     DLManagedTensor* order)
{
  return translate([=] {
    auto& r = res_of(res);
    dispatch(index->dtype, [&](auto tag) {
      using T         = decltype(tag);
      auto const& idx = *as_index<T>(*index);
      auto* out       = device_data<int32_t>(order, 1, "the list order");
      certex::expects(order->dl_tensor.shape[0] == idx.size(),
                      "certex: list_order needs an int32 device vector of one entry per vector");
      certex::list_order<T>(r, idx, out);
    });
  });
}

cuvsError_t cuvsCertexStatsBegin(void)
{
  return translate([] { certex::stats_begin(); });
}

cuvsError_t cuvsCertexStatsEnd(int64_t* queries, int64_t* survivors, int64_t* verified)
{
  return translate([=] {
    const auto s = certex::stats_end();
    *queries     = s.queries;
    *survivors   = s.survivors;
    *verified    = s.verified;
  });
}

cuvsError_t cuvsCertexTestCaptureBegin(void)
{
  return translate([] { certex::capture_begin(); });
}

cuvsError_t cuvsCertexTestCaptureGet(const char* name, void* host, int64_t* bytes)
{
  return translate([=] {
    certex::expects(name != nullptr && bytes != nullptr, "certex: NULL argument");
    *bytes = certex::capture_get(std::string(name), host);
  });
}

cuvsError_t cuvsCertexTimingShaderClock(double* mhz)
{
  return translate([=] {
    certex::expects(mhz != nullptr, "certex: NULL output");
    *mhz = certex::timing_shader_clock_mhz();
  });
}

cuvsError_t cuvsCertexTrimPool(cuvsResources_t res)
{
  return translate([=] { res_of(res).trim(); });
}

cuvsError_t cuvsCertexTestScratchCap(cuvsResources_t res, int64_t bytes)
{
  return translate([=] {
    certex::expects(bytes >= 0, "certex: the scratch cap must not be negative");
    res_of(res).set_scratch_cap(size_t(bytes));
  });
}

cuvsError_t cuvsCertexTimingBegin(void)
{
  return translate([] { certex::timing_begin(); });
}

cuvsError_t cuvsCertexTimingEnd(double* ms, int64_t* launches)
{
  return translate([=] {
    const auto t = certex::timing_end();
    for (int i = 0; i < CERTEX_N_PHASES; ++i) {
      ms[i]       = t.ms[i];
      launches[i] = t.launches[i];
    }
  });
}

}  // extern "C"
