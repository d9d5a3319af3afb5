// The cuvsOctex* C ABI (the reference: c/src/neighbors/octex.cpp:31-333) and the subset of the cuVS
// core C API it needs (resources, stream, last error text; c/src/core/exceptions.hpp:17-33), on
// DLPack tensors in HIP device memory (kDLROCM) or host memory (kDLCPU, kDLROCMHost).

#include "build.hpp"
#include "common.hpp"
#include "directory.hpp"
#include "kernels.hpp"
#include "index_impl.hpp"
#include "search.hpp"

#include <cuvs/core/c_api.h>
#include <cuvs/neighbors/octex.h>
#include <cuvs/neighbors/octex.hpp>
#include <octex_amd/octex_amd.h>

#include <hip/hip_runtime.h>

#include <cstring>
#include <exception>
#include <string>
#include <type_traits>
#include <vector>

namespace {

namespace octex = cuvs::neighbors::octex;

thread_local std::string g_last_error;

template <typename Fn>
auto translate_exceptions(Fn func) -> cuvsError_t
{
  try {
    func();
    cuvsSetLastErrorText(nullptr);
    return CUVS_SUCCESS;
  } catch (std::exception const& e) {
    cuvsSetLastErrorText(e.what());
  } catch (...) {
    cuvsSetLastErrorText("unknown exception");
  }
  return CUVS_ERROR;
}

auto as_res(cuvsResources_t res) -> raft::resources*
{
  OCTEX_EXPECTS(res != 0, "octex: the resources handle is NULL");
  return reinterpret_cast<raft::resources*>(res);
}

auto to_cpp(cuvsOctexIndexParams const& p) -> octex::index_params
{
  octex::index_params out;
  out.copies   = p.copies;
  out.blocks   = p.blocks;
  out.pca_dims = p.pca_dims;
  if (p.spacings != nullptr && p.n_spacings > 0) out.spacings.assign(p.spacings, p.spacings + p.n_spacings);
  out.list_len           = p.list_len;
  out.min_cell           = p.min_cell;
  out.log_buckets        = p.log_buckets;
  out.sketch_width       = p.sketch_width;
  out.table_len          = p.table_len;
  out.reverse_edges      = p.reverse_edges;
  out.exact_lists        = p.exact_lists;
  out.list_probes        = p.list_probes;
  out.member_lists       = p.member_lists;
  out.exact_table_max    = p.exact_table_max;
  out.table_passes       = p.table_passes;
  out.table_sketch_order = p.table_sketch_order;
  out.write_behind       = p.write_behind;
  out.seed               = p.seed;
  if (p.devices != nullptr && p.n_devices > 0) out.devices.assign(p.devices, p.devices + p.n_devices);
  return out;
}

// A C caller can store any int in an enum field; reading it as the C++ enum type is undefined for values outside
// the enumeration, so the fields are read as the ints they are
template <typename E>
auto enum_value(E const& field) -> int
{
  static_assert(sizeof(E) == sizeof(int), "C enums are int-sized");
  int v = 0;
  std::memcpy(&v, &field, sizeof v);
  return v;
}

auto to_cpp(cuvsOctexLoadParams const& p) -> octex::load_params
{
  const int placement = enum_value(p.placement), sketch = enum_value(p.sketch);
  OCTEX_EXPECTS(placement == OCTEX_PLACEMENT_REPLICATE || placement == OCTEX_PLACEMENT_SHARD,
                "octex: unknown placement");
  OCTEX_EXPECTS(sketch == OCTEX_SKETCH_REPLICATE || sketch == OCTEX_SKETCH_SHARD || sketch == OCTEX_SKETCH_HOST,
                "octex: unknown sketch placement");
  octex::load_params out;
  if (p.devices != nullptr && p.n_devices > 0) out.devices.assign(p.devices, p.devices + p.n_devices);
  out.mode            = static_cast<octex::placement>(placement);
  out.vectors_on_host = p.vectors_on_host;
  out.shard_vectors   = p.shard_vectors;
  out.table_on_host   = p.table_on_host;
  out.sketch          = static_cast<octex::sketch_placement>(sketch);
  out.parts           = p.parts;
  out.copies_per_part = p.copies_per_part;
  out.copies_limit    = p.copies_limit;
  out.list_limit      = p.list_limit;
  return out;
}

auto to_cpp(cuvsOctexSearchParams const& p) -> octex::search_params
{
  octex::search_params out;
  out.read            = p.read;
  out.starts          = p.starts;
  out.waves           = p.waves;
  out.rerank          = p.rerank;
  out.wave_rerank     = p.wave_rerank;
  out.batch           = p.batch;
  out.sketch_rank     = p.sketch_rank;
  out.final_rerank    = p.final_rerank;
  out.balanced_gather = p.balanced_gather;
  out.fused_merge     = p.fused_merge;
  out.use_graph       = p.use_graph;
  return out;
}

auto as_index(cuvsOctexIndex const& index) -> octex::index*
{
  OCTEX_EXPECTS(index.addr != 0, "octex: the index is empty (load it first)");
  return reinterpret_cast<octex::index*>(index.addr);
}

// ---- DLPack tensors (the reference: c/src/core/interop.hpp:25-97)

auto host_compatible(DLTensor const& t) -> bool
{
  return t.device.device_type == kDLCPU || t.device.device_type == kDLROCMHost;
}
auto device_compatible(DLTensor const& t) -> bool
{
  return t.device.device_type == kDLROCM || t.device.device_type == kDLROCMHost;
}

template <typename T>
auto dl_code() -> uint8_t
{
  if constexpr (std::is_floating_point_v<T> || std::is_same_v<T, __half>) return kDLFloat;
  if constexpr (std::is_signed_v<T>) return kDLInt;
  return kDLUInt;
}

template <typename T>
auto dl_matrix(DLManagedTensor* m, bool device) -> T*
{
  OCTEX_EXPECTS(m != nullptr, "octex: a DLPack tensor is NULL");
  DLTensor const& t = m->dl_tensor;
  if (device)
    OCTEX_EXPECTS(device_compatible(t), "octex: expected a tensor in device memory");
  else
    OCTEX_EXPECTS(host_compatible(t), "octex: expected a tensor in host memory");
  OCTEX_EXPECTS(t.ndim == 2, "octex: the DLPack tensor has the wrong number of dimensions");
  OCTEX_EXPECTS(t.dtype.code == dl_code<T>() && t.dtype.bits == 8 * sizeof(T) && t.dtype.lanes == 1,
                "octex: the DLPack tensor has the wrong data type");
  if (t.strides != nullptr) {
    int64_t expect = 1;
    for (int i = t.ndim - 1; i >= 0; --i) {
      OCTEX_EXPECTS(t.shape[i] == 1 || t.strides[i] == expect, "octex: the DLPack tensor must be dense and row major");
      expect *= t.shape[i];
    }
  }
  return reinterpret_cast<T*>(static_cast<char*>(t.data) + t.byte_offset);
}

/** The dataset of a build, where it lies: float32 or float16, host or device. */
auto dataset_of(DLManagedTensor* m) -> octex::detail::dataset_view
{
  OCTEX_EXPECTS(m != nullptr, "octex: a DLPack tensor is NULL");
  auto const& t  = m->dl_tensor;
  const bool dev = t.device.device_type == kDLROCM;  // pinned host memory is read as host memory
  octex::detail::dataset_view v;
  if (t.dtype.code == kDLFloat && t.dtype.bits == 32) {
    v.data = dl_matrix<float>(m, dev);
    v.f32  = true;
  } else if (t.dtype.code == kDLFloat && t.dtype.bits == 16) {
    v.data = dl_matrix<__half>(m, dev);
  } else {
    octex::detail::fail("octex: the dataset must be float32 or float16");
  }
  v.n = t.shape[0], v.d = t.shape[1], v.device = dev;
  return v;
}

}  // namespace

// ==================================================================== cuVS core

extern "C" cuvsError_t cuvsResourcesCreate(cuvsResources_t* res)
{
  return translate_exceptions([=] {
    OCTEX_EXPECTS(res != nullptr, "octex: NULL output pointer");
    *res = reinterpret_cast<cuvsResources_t>(new raft::resources());
  });
}

extern "C" cuvsError_t cuvsResourcesDestroy(cuvsResources_t res)
{
  return translate_exceptions([=] { delete reinterpret_cast<raft::resources*>(res); });
}

extern "C" cuvsError_t cuvsStreamSet(cuvsResources_t res, void* stream)
{
  return translate_exceptions([=] { as_res(res)->set_stream(static_cast<hipStream_t>(stream)); });
}

extern "C" cuvsError_t cuvsStreamGet(cuvsResources_t res, void** stream)
{
  return translate_exceptions([=] { *stream = static_cast<void*>(as_res(res)->get_stream()); });
}

extern "C" cuvsError_t cuvsStreamSync(cuvsResources_t res)
{
  return translate_exceptions([=] { OCTEX_HIP(hipStreamSynchronize(as_res(res)->get_stream())); });
}

extern "C" const char* cuvsGetLastErrorText(void) { return g_last_error.c_str(); }

extern "C" void cuvsSetLastErrorText(const char* error) { g_last_error = error != nullptr ? error : ""; }

// ==================================================================== cuvsOctex*

extern "C" cuvsError_t cuvsOctexIndexParamsCreate(cuvsOctexIndexParams_t* params)
{
  return translate_exceptions([=] {
    octex::index_params d;
    *params = new cuvsOctexIndexParams{d.copies,        d.blocks,          d.pca_dims,     nullptr,
                                       0,               d.list_len,        d.min_cell,     d.log_buckets,
                                       d.sketch_width,  d.table_len,       d.reverse_edges, d.exact_lists,
                                       d.list_probes,   d.member_lists,    d.exact_table_max,
                                       d.table_passes,  d.table_sketch_order, d.write_behind, d.seed,
                                       nullptr,         0};
  });
}

extern "C" cuvsError_t cuvsOctexIndexParamsDestroy(cuvsOctexIndexParams_t params)
{
  return translate_exceptions([=] { delete params; });
}

extern "C" cuvsError_t cuvsOctexLoadParamsCreate(cuvsOctexLoadParams_t* params)
{
  return translate_exceptions([=] {
    octex::load_params d;
    *params = new cuvsOctexLoadParams{nullptr,
                                      0,
                                      static_cast<cuvsOctexPlacement>(static_cast<int>(d.mode)),
                                      d.vectors_on_host,
                                      d.shard_vectors,
                                      d.table_on_host,
                                      static_cast<cuvsOctexSketchPlacement>(static_cast<int>(d.sketch)),
                                      d.parts,
                                      d.copies_per_part,
                                      d.copies_limit,
                                      d.list_limit};
  });
}

extern "C" cuvsError_t cuvsOctexLoadParamsDestroy(cuvsOctexLoadParams_t params)
{
  return translate_exceptions([=] { delete params; });
}

extern "C" cuvsError_t cuvsOctexSearchParamsCreate(cuvsOctexSearchParams_t* params)
{
  return translate_exceptions([=] {
    octex::search_params d;
    *params = new cuvsOctexSearchParams{d.read,        d.starts,       d.waves,           d.rerank,
                                        d.wave_rerank, d.batch,        d.sketch_rank,     d.final_rerank,
                                        d.balanced_gather, d.fused_merge, d.use_graph};
  });
}

extern "C" cuvsError_t cuvsOctexSearchParamsDestroy(cuvsOctexSearchParams_t params)
{
  return translate_exceptions([=] { delete params; });
}

extern "C" cuvsError_t cuvsOctexIndexCreate(cuvsOctexIndex_t* index)
{
  return translate_exceptions([=] { *index = new cuvsOctexIndex{}; });
}

extern "C" cuvsError_t cuvsOctexIndexDestroy(cuvsOctexIndex_t index)
{
  return translate_exceptions([=] {
    if (index == nullptr) return;
    if (index->addr != 0) delete reinterpret_cast<octex::index*>(index->addr);
    delete index;
  });
}

extern "C" cuvsError_t cuvsOctexIndexGetSize(cuvsOctexIndex_t index, int64_t* size)
{
  return translate_exceptions([=] { *size = as_index(*index)->size(); });
}

extern "C" cuvsError_t cuvsOctexIndexGetDim(cuvsOctexIndex_t index, int64_t* dim)
{
  return translate_exceptions([=] { *dim = as_index(*index)->dim(); });
}

extern "C" cuvsError_t cuvsOctexIndexGetCopies(cuvsOctexIndex_t index, int32_t* copies)
{
  return translate_exceptions([=] { *copies = as_index(*index)->copies(); });
}

extern "C" cuvsError_t cuvsOctexIndexGetNumDevices(cuvsOctexIndex_t index, int32_t* n_devices)
{
  return translate_exceptions(
    [=] { *n_devices = static_cast<int32_t>(as_index(*index)->devices().size()); });
}

extern "C" cuvsError_t cuvsOctexIndexGetDevices(cuvsOctexIndex_t index, int32_t* devices)
{
  return translate_exceptions([=] {
    auto const& d = as_index(*index)->devices();
    for (size_t i = 0; i < d.size(); ++i)
      devices[i] = d[i];
  });
}

extern "C" cuvsError_t cuvsOctexIndexGetDeviceBytes(cuvsOctexIndex_t index, int64_t* bytes)
{
  return translate_exceptions([=] {
    auto b = as_index(*index)->device_bytes();
    for (size_t i = 0; i < b.size(); ++i)
      bytes[i] = b[i];
  });
}

extern "C" cuvsError_t cuvsOctexBuild(cuvsResources_t res, cuvsOctexIndexParams_t params,
                                      DLManagedTensor* dataset, const char* path)
{
  return translate_exceptions([=] {
    OCTEX_EXPECTS(path != nullptr, "octex: the index directory is NULL");
    OCTEX_EXPECTS(params != nullptr && dataset != nullptr, "octex: NULL parameters or dataset");
    (void)as_res(res);
    const auto p = to_cpp(*params);
    octex::detail::build_record rec;
    octex::detail::build_to_directory(p, dataset_of(dataset), std::string(path), rec);
  });
}

extern "C" cuvsError_t cuvsOctexLoad(cuvsResources_t res, const char* path, cuvsOctexLoadParams_t params,
                                     cuvsOctexIndex_t index)
{
  return translate_exceptions([=] {
    OCTEX_EXPECTS(index != nullptr, "octex: the index handle is NULL");
    OCTEX_EXPECTS(index->addr == 0, "octex: the index handle already holds an index");
    OCTEX_EXPECTS(path != nullptr, "octex: the index directory is NULL");
    auto* r      = as_res(res);
    const auto p = params != nullptr ? to_cpp(*params) : octex::load_params{};
    index->addr  = reinterpret_cast<uintptr_t>(new octex::index(octex::load(*r, std::string(path), p)));
  });
}

extern "C" cuvsError_t cuvsOctexSearch(cuvsResources_t res, cuvsOctexSearchParams_t params,
                                       cuvsOctexIndex_t index, DLManagedTensor* queries,
                                       DLManagedTensor* neighbors, DLManagedTensor* distances)
{
  return translate_exceptions([=] {
    auto* r        = as_res(res);
    OCTEX_EXPECTS(params != nullptr, "octex: the search parameters are NULL");
    const auto p   = to_cpp(*params);
    auto const& ix = *as_index(*index);
    OCTEX_EXPECTS(queries != nullptr && neighbors != nullptr && distances != nullptr, "octex: NULL tensor");
    const bool dev = queries->dl_tensor.device.device_type == kDLROCM;
    auto* q        = dl_matrix<float>(queries, dev);
    auto* nb       = dl_matrix<int64_t>(neighbors, dev);
    auto* ds       = dl_matrix<float>(distances, dev);
    const auto& qt = queries->dl_tensor;
    const auto& nt = neighbors->dl_tensor;
    const auto& dt = distances->dl_tensor;
    OCTEX_EXPECTS(nt.shape[0] == qt.shape[0] && dt.shape[0] == qt.shape[0] && dt.shape[1] == nt.shape[1],
                  "octex: output shapes");
    octex::detail::search_impl(*r, p, ix, q, qt.shape[0], qt.shape[1], nb, ds, nt.shape[1], !dev, false);
  });
}

// ==================================================================== octex_amd.h

extern "C" cuvsError_t octexSearchNoAlloc(cuvsOctexSearchParams_t params, cuvsOctexIndex_t index, const float* queries,
                                          int64_t nq, int64_t dim, int64_t k, int64_t* neighbors, float* distances,
                                          void* stream)
{
  return translate_exceptions([=] {
    OCTEX_EXPECTS(params != nullptr && index != nullptr, "octex: NULL parameters or index");
    octex::detail::search_no_alloc(to_cpp(*params), *as_index(*index), queries, nq, dim, k, neighbors, distances,
                                   static_cast<hipStream_t>(stream));
  });
}

// ==================================================================== introspection (octex_amd.h)

extern "C" cuvsError_t octexIndexCheckDirectory(const char* path, cuvsOctexLoadParams_t params, int64_t* info)
{
  return translate_exceptions([=] {
    OCTEX_EXPECTS(path != nullptr, "octex: the index directory is NULL");
    const auto p = params != nullptr ? to_cpp(*params) : octex::load_params{};
    auto dir     = octex::detail::open_directory(std::string(path), p);
    if (info != nullptr) {
      const int64_t v[10] = {dir.n,      dir.dim,         static_cast<int64_t>(dir.copy_list.size()),
                             dir.all_copies, dir.blocks, static_cast<int64_t>(dir.spacings.size()),
                             dir.list_len, dir.log_buckets, dir.sketch_width, dir.table_len};
      std::memcpy(info, v, sizeof(v));
    }
  });
}

extern "C" cuvsError_t octexIndexCopyPlanBuffer(cuvsOctexIndex_t index, const char* name, void* dst,
                                                int64_t bytes, int64_t* size)
{
  return translate_exceptions([=] {
    auto& ix = as_index(*index)->impl();
    std::lock_guard<std::mutex> run(ix.stream_mu);
    std::shared_ptr<octex::detail::plan> pl;
    {
      std::lock_guard<std::mutex> lock(ix.mu);
      OCTEX_EXPECTS(!ix.plans.empty(), "octex: no search ran on this index yet");
      pl = ix.plans.begin()->second;
    }
    auto [src, sz] = octex::detail::named_buffer(ix, pl->shape, pl->buf, std::string(name != nullptr ? name : ""));
    if (size != nullptr) *size = static_cast<int64_t>(sz);
    if (dst != nullptr && bytes > 0 && src != nullptr) {
      OCTEX_HIP(hipSetDevice(ix.device));
      OCTEX_HIP(hipStreamSynchronize(ix.stream));
      OCTEX_HIP(hipMemcpy(dst, src, std::min<size_t>(sz, static_cast<size_t>(bytes)), hipMemcpyDefault));
    }
  });
}

extern "C" cuvsError_t octexIndexPlanInfo(cuvsOctexIndex_t index, int32_t* info)
{
  return translate_exceptions([=] {
    auto& ix = as_index(*index)->impl();
    std::lock_guard<std::mutex> lock(ix.mu);
    OCTEX_EXPECTS(!ix.plans.empty(), "octex: no search ran on this index yet");
    auto const& pl = *ix.plans.begin()->second;
    auto const& sh = pl.shape;
    int32_t v[] = {sh.m, sh.k, sh.KO, sh.lr, sh.W, sh.W2, sh.R1, sh.R2, sh.FR, pl.graph != nullptr ? 1 : 0};
    std::memcpy(info, v, sizeof(v));
  });
}

extern "C" cuvsError_t octexBuildInMemory(cuvsResources_t res, cuvsOctexIndexParams_t params, DLManagedTensor* dataset,
                                          const char* path, cuvsOctexIndex_t index, double* seconds)
{
  return translate_exceptions([=] {
    (void)as_res(res);
    OCTEX_EXPECTS(params != nullptr && dataset != nullptr && index != nullptr, "octex: NULL argument");
    OCTEX_EXPECTS(index->addr == 0, "octex: the index handle already holds an index");
    const auto p = to_cpp(*params);
    octex::detail::build_record rec;
    auto impl = path != nullptr ? octex::detail::build_to_directory(p, dataset_of(dataset), std::string(path), rec)
                                : octex::detail::build_in_memory(p, dataset_of(dataset), rec);
    if (seconds != nullptr) *seconds = rec.phases.empty() ? 0.0 : rec.phases.back().second;
    index->addr = reinterpret_cast<uintptr_t>(new octex::index(impl));
  });
}

extern "C" cuvsError_t octexIndexProfileBatch(cuvsOctexIndex_t index, cuvsOctexSearchParams_t params,
                                              DLManagedTensor* queries, int64_t k, int32_t reps, char* names,
                                              double* ms, int32_t* nstages, int64_t* counters)
{
  return translate_exceptions([=] {
    OCTEX_EXPECTS(params != nullptr && queries != nullptr && names != nullptr && ms != nullptr, "octex: NULL argument");
    auto& idx      = *as_index(*index);
    auto& ix       = idx.impl();
    auto const p   = to_cpp(*params);
    const bool dev = queries->dl_tensor.device.device_type == kDLROCM;
    auto* q        = dl_matrix<float>(queries, dev);
    const int64_t nq = queries->dl_tensor.shape[0];
    OCTEX_EXPECTS(nq <= std::max(p.batch, 1), "octex: the profiled queries must fit one batch");
    OCTEX_EXPECTS(p.waves <= 16, "octex: at most 16 waves are profiled");
    std::vector<int64_t> nb(nq * k);
    std::vector<float> nd(nq * k);
    raft::resources r;
    std::vector<float> hq;
    const float* qh = q;
    if (dev) {
      hq.resize(static_cast<size_t>(nq * ix.dim));
      OCTEX_HIP(hipMemcpy(hq.data(), q, hq.size() * sizeof(float), hipMemcpyDeviceToHost));
      qh = hq.data();
    }
    // a normal search first: the plan, and the queries in its buffer
    octex::detail::search_impl(r, p, idx, qh, nq, ix.dim, nb.data(), nd.data(), k, true, false);
    std::lock_guard<std::mutex> run(ix.stream_mu);
    std::shared_ptr<octex::detail::plan> pl;
    {  // the plan of this call's parameters: another thread's search may have replaced it since
      std::lock_guard<std::mutex> lock(ix.mu);
      const int m = static_cast<int>(std::min<int64_t>(std::max(p.batch, 1), nq));
      auto it     = ix.plans.find(octex::detail::plan_key(p, m, static_cast<int>(k)));
      OCTEX_EXPECTS(it != ix.plans.end(), "octex: the profiled plan was evicted by another search");
      pl = it->second;
    }
    OCTEX_HIP(hipSetDevice(ix.device));
    std::vector<std::string> nm;
    std::vector<double> t;
    octex::detail::profile_counters cnt;
    octex::detail::profile_batch(ix, *pl, std::max(reps, 1), nm, t, cnt);
    OCTEX_EXPECTS(nm.size() <= 64, "octex: too many stages");
    for (size_t i = 0; i < nm.size(); i++) {
      std::memset(names + 32 * i, 0, 32);
      std::strncpy(names + 32 * i, nm[i].c_str(), 31);
      ms[i] = t[i];
    }
    *nstages = static_cast<int32_t>(nm.size());
    if (counters != nullptr) {
      int64_t v[4 + 48 + 8 + 48] = {cnt.seg_hits, cnt.entries1, cnt.distinct1, cnt.reranked1};
      for (int w = 0; w < 16; w++) {
        v[4 + w]       = cnt.starts2[w];
        v[4 + 16 + w]  = cnt.distinct2[w];
        v[4 + 32 + w]  = cnt.reranked2[w];
        v[60 + w]      = cnt.skipped2[w];
        v[60 + 16 + w] = cnt.known2[w];
        v[60 + 32 + w] = cnt.oldread2[w];
      }
      for (int j = 0; j < 8; j++)
        v[52 + j] = cnt.hit_level[j];
      std::memcpy(counters, v, sizeof(v));
    }
  });
}

extern "C" cuvsError_t octexIndexPlaceOnHost(cuvsOctexIndex_t index, int32_t vectors, int32_t table, int32_t sketch)
{
  return translate_exceptions([=] {
    auto& ix = as_index(*index)->impl();
    std::lock_guard<std::mutex> run(ix.stream_mu);
    OCTEX_HIP(hipSetDevice(ix.device));
    OCTEX_HIP(hipStreamSynchronize(ix.stream));
    {
      std::lock_guard<std::mutex> lock(ix.mu);
      ix.plans.clear();  // cached plans and their graphs hold the arrays' device addresses
    }
    auto move = [&](octex::detail::dbuf& d, octex::detail::hbuf& h) {
      if (d.ptr == nullptr) return;  // on the host already, or absent
      octex::detail::hbuf to(d.size);
      OCTEX_HIP(hipMemcpy(to.ptr, d.ptr, d.size, hipMemcpyDeviceToHost));
      ix.bytes -= static_cast<int64_t>(d.size);
      d = octex::detail::dbuf();
      h = std::move(to);
    };
    if (vectors != 0) move(ix.vectors, ix.host_vectors);
    if (table != 0) move(ix.table, ix.host_table);
    if (sketch != 0) move(ix.sketch, ix.host_sketch);
  });
}

namespace {

/** The device (or pinned host) bytes of an index array by name: lists of one copy, or a whole array. */
auto index_array(octex::detail::index_impl& ix, std::string const& n, int32_t copy) -> std::pair<const void*, size_t>
{
  auto of = [](octex::detail::dbuf const& b) { return std::pair<const void*, size_t>(b.ptr, b.size); };
  if (n == "lists") {
    OCTEX_EXPECTS(copy >= 0 && copy < ix.copies, "octex: no copy %d", copy);
    if (!ix.copy_lists.empty())
      return {ix.copy_lists[copy].ptr, static_cast<size_t>(ix.list_rows[copy]) * ix.list_len * sizeof(int32_t)};
    return {ix.lists.as<int32_t>() + copy * ix.stride, static_cast<size_t>(ix.stride) * sizeof(int32_t)};
  }
  if (n == "keys") return of(ix.keys);
  if (n == "offsets") return of(ix.offsets);
  if (n == "base") return of(ix.base);
  if (n == "ucatT") return of(ix.ucatT);
  if (n == "shift") return of(ix.shift);
  if (n == "inv_f") return of(ix.inv_f);
  if (n == "mean") return of(ix.mean);
  if (n == "basis") return of(ix.basis);
  if (n == "scale") return of(ix.scale);
  if (n == "sketch") return {ix.code(), static_cast<size_t>(ix.n) * ix.sketch_pitch};
  if (n == "vectors") return {ix.vecs(), static_cast<size_t>(ix.n) * ix.dim * sizeof(__half)};
  if (n == "table") return {ix.rows(), static_cast<size_t>(ix.n) * ix.table_len * sizeof(int32_t)};
  octex::detail::fail("octex: unknown index array %s", n.c_str());
}

}  // namespace

extern "C" cuvsError_t octexIndexCopyArray(cuvsOctexIndex_t index, const char* name, int32_t copy, void* dst,
                                           int64_t bytes, int64_t* size)
{
  return translate_exceptions([=] {
    auto& ix = as_index(*index)->impl();
    std::string n(name != nullptr ? name : "");
    if (n == "meta") {  // n, dim, copies, blocks, levels, list_len, log_buckets, sketch_width, table_len, mmax, T1,
                        // sketch_pitch
      int64_t m[12] = {ix.n,           ix.dim,       ix.copies,    ix.blocks, ix.levels(), ix.list_len,
                       ix.log_buckets, ix.sketch_width, ix.table_len, ix.mmax, ix.T1,     ix.sketch_pitch};
      if (size != nullptr) *size = sizeof(m);
      if (dst != nullptr) std::memcpy(dst, m, std::min<size_t>(sizeof(m), static_cast<size_t>(bytes)));
      return;
    }
    if (n == "spacings") {
      if (size != nullptr) *size = static_cast<int64_t>(ix.spacings.size() * sizeof(float));
      if (dst != nullptr)
        std::memcpy(dst, ix.spacings.data(), std::min<size_t>(ix.spacings.size() * sizeof(float), bytes));
      return;
    }
    auto [src, sz] = index_array(ix, n, copy);
    if (size != nullptr) *size = static_cast<int64_t>(sz);
    if (dst != nullptr && bytes > 0 && src != nullptr) {
      OCTEX_HIP(hipSetDevice(ix.device));
      OCTEX_HIP(hipStreamSynchronize(ix.stream));  // the index's own stream may still write it
      OCTEX_HIP(hipMemcpy(dst, src, std::min<size_t>(sz, static_cast<size_t>(bytes)), hipMemcpyDefault));
    }
  });
}

extern "C" cuvsError_t octexIndexCopyArrayRanges(cuvsOctexIndex_t index, const char* name, int32_t copy,
                                                 const int64_t* offsets, int64_t count, int64_t bytes, void* dst)
{
  return translate_exceptions([=] {
    OCTEX_EXPECTS(count >= 0 && bytes >= 0 && (count == 0 || (offsets != nullptr && dst != nullptr)),
                  "octex: NULL offsets or destination");
    if (count == 0 || bytes == 0) return;
    auto& ix       = as_index(*index)->impl();
    auto [src, sz] = index_array(ix, std::string(name != nullptr ? name : ""), copy);
    OCTEX_EXPECTS(bytes % 4 == 0, "octex: ranges are whole 32-bit words");
    std::vector<int64_t> words(static_cast<size_t>(count));
    for (int64_t r = 0; r < count; r++) {
      OCTEX_EXPECTS(offsets[r] >= 0 && offsets[r] % 4 == 0 && static_cast<size_t>(offsets[r] + bytes) <= sz,
                    "octex: range %lld (bytes [%lld, %lld)) is outside the array (%zu bytes) or unaligned",
                    static_cast<long long>(r), static_cast<long long>(offsets[r]),
                    static_cast<long long>(offsets[r] + bytes), sz);
      words[r] = offsets[r] / 4;
    }
    OCTEX_HIP(hipSetDevice(ix.device));
    octex::detail::dbuf doff(words.size() * sizeof(int64_t)), dout(static_cast<size_t>(count * bytes));
    octex::detail::upload(doff.ptr, words.data(), doff.size, ix.stream);
    octex::detail::launch_copy_ranges(static_cast<const uint32_t*>(src), doff.as<int64_t>(), count,
                                      static_cast<int>(bytes / 4), dout.as<uint32_t>(), ix.stream);
    OCTEX_HIP(hipStreamSynchronize(ix.stream));
    OCTEX_HIP(hipMemcpy(dst, dout.ptr, dout.size, hipMemcpyDefault));
  });
}

extern "C" cuvsError_t octexIndexCopyArrayRange(cuvsOctexIndex_t index, const char* name, int32_t copy,
                                                int64_t offset, void* dst, int64_t bytes)
{
  return translate_exceptions([=] {
    OCTEX_EXPECTS(dst != nullptr || bytes == 0, "octex: NULL destination");
    auto& ix       = as_index(*index)->impl();
    auto [src, sz] = index_array(ix, std::string(name != nullptr ? name : ""), copy);
    OCTEX_EXPECTS(offset >= 0 && bytes >= 0 && static_cast<size_t>(offset + bytes) <= sz,
                  "octex: bytes [%lld, %lld) are outside the array (%zu bytes)", static_cast<long long>(offset),
                  static_cast<long long>(offset + bytes), sz);
    if (bytes == 0) return;
    OCTEX_HIP(hipSetDevice(ix.device));
    OCTEX_HIP(hipStreamSynchronize(ix.stream));
    OCTEX_HIP(hipMemcpy(dst, static_cast<const char*>(src) + offset, static_cast<size_t>(bytes), hipMemcpyDefault));
  });
}
