// octex::load for one MI355X: an index directory (format 1) into HBM (the reference: load.cu:206-494,
// single device).  Every array is memory mapped and copied once; the projections become fp16 ucatT
// [C * 8b, D] and the shifts fp16, inv_f = float(1 / spacing) from the JSON value (load.cu:385-402).

#include "common.hpp"
#include "directory.hpp"
#include "index_impl.hpp"
#include "kernels.hpp"
#include "meta.hpp"
#include "npy.hpp"

#include <hip/hip_fp16.h>

#include <algorithm>
#include <cmath>
#include <fstream>
#include <sstream>
#include <thread>

namespace cuvs::neighbors::octex {

namespace {

using detail::dbuf;
using detail::hbuf;
using detail::index_impl;
using detail::npy_file;

auto read_text(std::string const& path) -> std::string
{
  std::ifstream f(path);
  OCTEX_EXPECTS(f.good(), "octex: cannot open %s", path.c_str());
  std::stringstream ss;
  ss << f.rdbuf();
  return ss.str();
}

/** bytes from host memory (mapped file pages) to device memory, in chunks through pinned staging. */
void upload_to(void* dst, const void* src, size_t bytes, hipStream_t s)
{
  constexpr size_t kChunk = size_t{64} << 20;
  if (bytes == 0) return;
  if (bytes <= kChunk) {
    detail::upload(dst, src, bytes, s);
    return;
  }
  hbuf stage[2] = {hbuf(kChunk), hbuf(kChunk)};
  hipEvent_t ev[2];
  for (auto& e : ev) {
    OCTEX_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    OCTEX_HIP(hipEventRecord(e, s));
  }
  int next = 0;
  for (size_t o = 0; o < bytes; o += kChunk) {
    size_t len = std::min(kChunk, bytes - o);
    OCTEX_HIP(hipEventSynchronize(ev[next]));
    std::memcpy(stage[next].ptr, static_cast<const char*>(src) + o, len);
    OCTEX_HIP(hipMemcpyAsync(static_cast<char*>(dst) + o, stage[next].ptr, len, hipMemcpyHostToDevice, s));
    OCTEX_HIP(hipEventRecord(ev[next], s));
    next ^= 1;
  }
  OCTEX_HIP(hipStreamSynchronize(s));
  for (auto& e : ev)
    (void)hipEventDestroy(e);
}

auto upload(index_impl& ix, const void* src, size_t bytes) -> dbuf
{
  dbuf b(bytes);
  upload_to(b.ptr, src, bytes, ix.stream);
  ix.bytes += static_cast<int64_t>(bytes);
  return b;
}

/** A file's data in pinned host memory, read in place by the kernels. */
auto to_pinned(npy_file const& f, size_t bytes) -> hbuf
{
  hbuf h(bytes);
  std::memcpy(h.ptr, f.data, bytes);
  return h;
}

}  // namespace

namespace detail {

void make_bucket_lines(index_impl& ix, size_t keep_free)
{
  if (const char* e = std::getenv("OCTEX_PROBE_LINES"); e != nullptr && std::string(e) == "0") return;
  const int64_t CL = static_cast<int64_t>(ix.offsets.size / sizeof(int32_t)) / std::max<int64_t>(ix.T1, 1);
  if (CL == 0 || ix.T1 < 2 || ix.keys.ptr == nullptr) return;
  const size_t bytes = static_cast<size_t>(CL) * static_cast<size_t>(ix.T1 - 1) * sizeof(bucket_line);
  size_t fr = 0, tot = 0;
  OCTEX_HIP(hipMemGetInfo(&fr, &tot));
  if (fr < bytes + keep_free) return;  // the probe reads the offsets
  ix.lines = dbuf(bytes);
  ix.bytes += static_cast<int64_t>(bytes);
  launch_bucket_lines(ix.offsets.as<int32_t>(), ix.T1, ix.keys.as<long long>(), ix.mmax, CL,
                      ix.lines.as<bucket_line>(), ix.stream);
  OCTEX_HIP(hipStreamSynchronize(ix.stream));
}

auto open_directory(std::string const& path, load_params const& params) -> directory
{
  return open_directory(path, params, read_text(path + "/meta.json"));
}

auto open_directory(std::string const& path, load_params const& params, std::string const& text) -> directory
{
  directory dir;
  dir.path  = path;
  auto meta = json_parser(text).parse();
  OCTEX_EXPECTS(static_cast<int>(meta.number("format", 1)) == 1, "octex: unknown index format");
  auto count = [&](const char* key, double dflt) {
    const double v = meta.number(key, dflt);
    OCTEX_EXPECTS(v >= 0 && v == std::floor(v) && v < 9.2e18, "octex: meta.json: %s must be a non-negative integer",
                  key);
    return static_cast<int64_t>(v);
  };
  dir.n            = count("n", 0);
  dir.dim          = count("dim", 0);
  dir.all_copies   = static_cast<int>(count("copies", 0));
  dir.blocks       = static_cast<int>(count("blocks", 4));
  dir.list_len     = static_cast<int>(count("list_len", 0));
  dir.log_buckets  = static_cast<int>(count("log_buckets", 20));
  dir.sketch_width = static_cast<int>(count("sketch_width", 0));
  dir.table_len    = static_cast<int>(count("table_len", 0));
  if (auto sp = meta.get("spacings"); sp != nullptr && sp->kind == json_value::array_v)
    for (auto const& v : sp->a) {
      OCTEX_EXPECTS(v.kind == json_value::number_v && v.d > 0, "octex: meta.json: spacings must be positive numbers");
      dir.spacings.push_back(v.d);
    }
  if (auto fm = meta.get("files"); fm != nullptr && fm->kind == json_value::object_v)
    for (auto const& [name, where] : fm->o) {
      OCTEX_EXPECTS(where.kind == json_value::string_v && !where.s.empty(),
                    "octex: meta.json: files.%s must be a path", name.c_str());
      dir.files[name] = where.s;
    }
  OCTEX_EXPECTS(dir.dim % 2 == 0, "octex: the dimension must be even");
  OCTEX_EXPECTS(dir.sketch_width % 16 == 0 && dir.sketch_width <= 512 && dir.sketch_width > 0,
                "octex: sketch width: a multiple of 16, <= 512");
  OCTEX_EXPECTS(dir.blocks >= 1 && dir.blocks <= 8 && dir.blocks != 7, "octex: blocks must be 1-6 or 8");
  OCTEX_EXPECTS(!dir.spacings.empty(), "octex: at least one spacing");
  OCTEX_EXPECTS(dir.list_len >= 1 && dir.log_buckets >= 1 && dir.log_buckets <= 30 && dir.n >= 1 && dir.n < (int64_t{1} << 31),
                "octex: meta.json: list_len, log_buckets or n out of range");

  // copies: the saved parts (equal consecutive ranges) cut to copies_per_part, or the first copies_limit
  // copies of a single part (load.cu:252-263); one GPU holds them all
  const int nparts = std::max(1, params.parts);
  for (int q = 0; q < nparts; q++) {
    const int lo = static_cast<int>(int64_t{dir.all_copies} * q / nparts);
    int hi       = static_cast<int>(int64_t{dir.all_copies} * (q + 1) / nparts);
    if (params.copies_per_part > 0) hi = std::min(hi, lo + params.copies_per_part);
    if (nparts == 1 && params.copies_limit > 0) hi = std::min(hi, lo + params.copies_limit);
    for (int c = lo; c < hi; c++)
      dir.copy_list.push_back(c);
  }
  OCTEX_EXPECTS(!dir.copy_list.empty(), "octex: a device holds no copies (fewer copies or parts than devices)");

  auto file = [&](std::string const& name) {
    auto it = dir.files.find(name);
    if (it == dir.files.end()) return path + "/" + name + ".npy";
    return it->second[0] == '/' ? it->second : path + "/" + it->second;
  };
  const int64_t C = dir.all_copies, L = static_cast<int64_t>(dir.spacings.size()), w = 8 * dir.blocks;
  const int64_t D = dir.dim, N = dir.n, S = dir.sketch_width, T1 = (int64_t{1} << dir.log_buckets) + 1;
  // every array with its dtype and full shape against meta.json, before anything is read from it
  auto open = [&](std::string const& name, const char* descr, std::vector<int64_t> const& shape) {
    npy_file f(file(name));
    OCTEX_EXPECTS(f.hdr.descr == descr, "octex: %s has dtype %s, expected %s", f.path().c_str(), f.hdr.descr.c_str(),
                  descr);
    bool same = f.shape().size() == shape.size();
    for (size_t i = 0; same && i < shape.size(); i++)
      same = shape[i] < 0 ? f.shape()[i] >= 0 : f.shape()[i] == shape[i];
    std::string want, got;
    for (auto v : shape)
      want += (want.empty() ? "" : ", ") + (v < 0 ? std::string("*") : std::to_string(v));
    for (auto v : f.shape())
      got += (got.empty() ? "" : ", ") + std::to_string(v);
    OCTEX_EXPECTS(same, "octex: %s has shape (%s), meta.json needs (%s)", f.path().c_str(), got.c_str(), want.c_str());
    return f;
  };
  dir.lists   = open("lists", "<i4", {C, -1});
  dir.keys    = open("keys", "<i8", {C, L, -1});
  dir.offsets = open("offsets", "<i4", {C, L, T1});
  dir.base    = open("base", "<i4", {C, L});
  dir.proj    = open("proj", "<f4", {C, D, w});
  dir.shift   = open("shift", "<f4", {C, w});
  dir.mean    = open("mean", "<f4", {D});
  dir.basis   = open("sketch_basis", "<f4", {D, S});
  dir.scale   = open("sketch_scale", "<f4", {S});
  dir.sketch  = open("sketch", "|i1", {N, S});
  dir.vectors = open("vectors", "<f2", {N, D});
  if (dir.table_len > 0) dir.table = open("table", "<i4", {N, dir.table_len});
  OCTEX_EXPECTS(dir.lists.dim(1) % dir.list_len == 0, "octex: lists rows hold %lld entries, not a multiple of list_len %d",
                static_cast<long long>(dir.lists.dim(1)), dir.list_len);
  // the cell tables stay inside their arrays: every bucket run [o[i], o[i + 1]) inside keys (0 = o[0] <= o[1] <= ...
  // <= o[T1 - 1] <= mmax: the probe reads keys o[i] .. o[i + 1] - 1 of any bucket), every level's rows inside lists.
  // Every entry of every selected copy and level is checked, the copies spread over host threads.
  const int64_t mmax = dir.keys.dim(2), rows = dir.lists.dim(1) / dir.list_len;
  const int32_t* off = dir.offsets.as<int32_t>();
  const int32_t* bs  = dir.base.as<int32_t>();
  std::vector<int> const& sel = dir.copy_list;
  std::vector<int64_t> bad(sel.size(), -1);  // per selected copy: the first bad level, or -1
  auto check_copy = [&](size_t s) {
    const int c = sel[s];
    for (int64_t j = 0; j < L && bad[s] < 0; j++) {
      const int32_t* o = off + (c * L + j) * T1;
      bool ok          = o[0] == 0 && o[T1 - 1] <= mmax && bs[c * L + j] >= 0 && bs[c * L + j] + o[T1 - 1] <= rows;
      bool down        = false;
      for (int64_t i = 0; i + 1 < T1; i++)
        down |= o[i + 1] < o[i];
      if (!ok || down) bad[s] = j;
    }
  };
  const int nth = static_cast<int>(std::min<size_t>(sel.size(), std::max(1u, std::min(16u, std::thread::hardware_concurrency()))));
  std::vector<std::thread> th;
  for (int t = 0; t < nth; t++)
    th.emplace_back([&, t] {
      for (size_t s = t; s < sel.size(); s += nth)
        check_copy(s);
    });
  for (auto& t : th)
    t.join();
  for (size_t s = 0; s < sel.size(); s++)
    OCTEX_EXPECTS(bad[s] < 0,
                  "octex: copy %d level %lld: its cells run past keys (%lld) or lists (%lld rows), or its bucket "
                  "offsets decrease",
                  sel[s], static_cast<long long>(bad[s]), static_cast<long long>(mmax), static_cast<long long>(rows));
  return dir;
}

}  // namespace detail

auto load(raft::resources const& res, std::string const& path, load_params const& params) -> index
{
  (void)res;
  detail::directory dir = detail::open_directory(path, params);  // every check, no device call
  return index(detail::load_directory(dir, path, params));
}

namespace {

auto load_opened(detail::directory const& dir, std::string const& path, load_params const& params)
  -> std::shared_ptr<index_impl>
{
  int cur = 0;
  OCTEX_HIP(hipGetDevice(&cur));
  auto impl = std::make_shared<index_impl>();
  auto& ix  = *impl;
  ix.path   = path;
  ix.params = params;
  ix.n            = dir.n;
  ix.dim          = dir.dim;
  ix.blocks       = dir.blocks;
  ix.list_len     = dir.list_len;
  ix.log_buckets  = dir.log_buckets;
  ix.sketch_width = dir.sketch_width;
  ix.table_len    = dir.table_len;
  for (double f : dir.spacings)
    ix.spacings.push_back(static_cast<float>(f));
  const int all_c = dir.all_copies;
  const int ll    = params.list_limit > 0 ? std::min(params.list_limit, ix.list_len) : ix.list_len;
  ix.device  = params.devices.empty() ? cur : params.devices.front();
  ix.devices = {ix.device};
  std::vector<int> const& cl = dir.copy_list;
  ix.copies = static_cast<int>(cl.size());
  npy_file const &lists = dir.lists, &keys = dir.keys, &offsets = dir.offsets, &base = dir.base;
  npy_file const &proj = dir.proj, &shift = dir.shift, &mean = dir.mean, &basis = dir.basis, &scale = dir.scale;
  npy_file const &sketch = dir.sketch, &vectors = dir.vectors;
  npy_file const* table = ix.table_len > 0 ? &dir.table : nullptr;
  std::vector<double> const& spacings = dir.spacings;
  const int L     = ix.levels();
  const int width = 8 * ix.blocks;
  const int64_t D = ix.dim, N = ix.n, S = ix.sketch_width;
  ix.T1 = offsets.dim(2);
  (void)all_c;

  OCTEX_HIP(hipSetDevice(ix.device));
  OCTEX_HIP(hipStreamCreateWithFlags(&ix.stream, hipStreamNonBlocking));
  const int Cg = ix.copies;
  // runs of consecutive copies of per_copy bytes each, in list order
  auto put = [&](const char* src, size_t per_copy) {
    dbuf dst(per_copy * Cg);
    ix.bytes += static_cast<int64_t>(dst.size);
    for (int i = 0; i < Cg;) {
      int j = i + 1;
      while (j < Cg && cl[j] == cl[j - 1] + 1)
        j++;
      upload_to(dst.as<char>() + per_copy * i, src + per_copy * cl[i], per_copy * (j - i), ix.stream);
      i = j;
    }
    return dst;
  };

  // lists: the first ll entries of every cell row (load.cu:361-379)
  const int64_t stride0 = lists.dim(1);
  const int32_t* lsrc   = lists.as<int32_t>();
  if (ll == ix.list_len) {
    ix.stride = stride0;
    ix.lists  = put(reinterpret_cast<const char*>(lsrc), stride0 * sizeof(int32_t));
  } else {
    const int64_t rows = stride0 / ix.list_len;
    ix.stride          = rows * ll;
    ix.lists           = dbuf(static_cast<size_t>(Cg * ix.stride) * sizeof(int32_t));
    ix.bytes += static_cast<int64_t>(ix.lists.size);
    std::vector<int32_t> tmp(ix.stride);
    for (int c = 0; c < Cg; c++) {
      const int32_t* src = lsrc + cl[c] * stride0;
      for (int64_t r = 0; r < rows; r++)
        std::memcpy(tmp.data() + r * ll, src + r * ix.list_len, ll * sizeof(int32_t));
      upload_to(ix.lists.as<int32_t>() + c * ix.stride, tmp.data(), ix.stride * sizeof(int32_t), ix.stream);
    }
  }
  {
    std::vector<long long> hp(Cg);
    for (int c = 0; c < Cg; c++)
      hp[c] = reinterpret_cast<long long>(ix.lists.as<int32_t>() + c * ix.stride);
    ix.list_ptr = upload(ix, hp.data(), hp.size() * sizeof(long long));
  }
  ix.mmax    = keys.dim(2);
  ix.keys    = put(reinterpret_cast<const char*>(keys.as<int64_t>()), L * ix.mmax * sizeof(int64_t));
  ix.offsets = put(reinterpret_cast<const char*>(offsets.as<int32_t>()), L * ix.T1 * sizeof(int32_t));
  ix.base    = put(reinterpret_cast<const char*>(base.as<int32_t>()), L * sizeof(int32_t));

  // projections as fp16 rows of ucatT [Cg * 8b, D], shifts fp16 (load.cu:385-396)
  {
    std::vector<__half> uc(static_cast<size_t>(Cg) * width * D), sh(static_cast<size_t>(Cg) * width);
    const float* pr = proj.as<float>();
    const float* sp = shift.as<float>();
    for (int c = 0; c < Cg; c++) {
      for (int s = 0; s < width; s++) {
        for (int64_t d = 0; d < D; d++)
          uc[(static_cast<size_t>(c) * width + s) * D + d] =
            __float2half(pr[(int64_t{cl[c]} * D + d) * width + s]);
        sh[static_cast<size_t>(c) * width + s] = __float2half(sp[int64_t{cl[c]} * width + s]);
      }
    }
    std::vector<float> inv(L);
    for (int j = 0; j < L; j++)
      inv[j] = static_cast<float>(1.0 / spacings[j]);
    ix.ucatT = upload(ix, uc.data(), uc.size() * sizeof(__half));
    ix.shift = upload(ix, sh.data(), sh.size() * sizeof(__half));
    ix.inv_f = upload(ix, inv.data(), inv.size() * sizeof(float));
  }
  ix.mean  = upload(ix, mean.as<float>(), D * sizeof(float));
  ix.basis = upload(ix, basis.as<float>(), D * S * sizeof(float));
  ix.scale = upload(ix, scale.as<float>(), S * sizeof(float));
  ix.sketch_pitch = detail::sketch_pitch_for(S, N, detail::device_memory_bytes());
  if (ix.sketch_pitch == S) {
    const size_t code_bytes = static_cast<size_t>(N * S);
    if (params.sketch == sketch_placement::host) {
      sketch.as<int8_t>();
      ix.host_sketch = to_pinned(sketch, code_bytes);
    } else {
      ix.sketch = upload(ix, sketch.as<int8_t>(), code_bytes);
    }
  } else {  // rows of S codes spread to the padded pitch, a chunk of rows at a time
    const int64_t P = ix.sketch_pitch;
    const char* src = reinterpret_cast<const char*>(sketch.as<int8_t>());
    const bool host = params.sketch == sketch_placement::host;
    if (host)
      ix.host_sketch = hbuf(static_cast<size_t>(N * P));
    else {
      ix.sketch = dbuf(static_cast<size_t>(N * P));
      ix.bytes += static_cast<int64_t>(ix.sketch.size);
    }
    const int64_t chunk = std::max<int64_t>(1, (int64_t{64} << 20) / P);
    std::vector<char> tmp(host ? 0 : static_cast<size_t>(std::min(chunk, N) * P), 0);
    for (int64_t r0 = 0; r0 < N; r0 += chunk) {
      const int64_t m = std::min(chunk, N - r0);
      char* dst       = host ? static_cast<char*>(ix.host_sketch.ptr) + r0 * P : tmp.data();
      for (int64_t r = 0; r < m; r++) {
        std::memcpy(dst + r * P, src + (r0 + r) * S, S);
        std::memset(dst + r * P + S, 0, P - S);
      }
      if (!host) upload_to(ix.sketch.as<char>() + r0 * P, tmp.data(), static_cast<size_t>(m * P), ix.stream);
    }
  }
  const size_t vec_bytes = static_cast<size_t>(N * D) * sizeof(__half);
  if (params.vectors_on_host) {
    vectors.as<__half>();
    ix.host_vectors = to_pinned(vectors, vec_bytes);
  } else {
    ix.vectors = upload(ix, vectors.as<__half>(), vec_bytes);
  }
  if (table) {
    const size_t tb = static_cast<size_t>(N * ix.table_len) * sizeof(int32_t);
    table->as<int32_t>();
    if (params.table_on_host)
      ix.host_table = to_pinned(*table, tb);
    else
      ix.table = upload(ix, table->as<int32_t>(), tb);
  }
  OCTEX_HIP(hipStreamSynchronize(ix.stream));
  detail::make_bucket_lines(ix, detail::kSearchReserve);
  ix.list_len = ll;
  OCTEX_HIP(hipSetDevice(cur));
  return impl;
}

}  // namespace

auto detail::load_directory(directory const& dir, std::string const& path, load_params const& params)
  -> std::shared_ptr<index_impl>
{
  return load_opened(dir, path, params);
}

}  // namespace cuvs::neighbors::octex
