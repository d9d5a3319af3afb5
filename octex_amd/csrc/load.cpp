// octex::load for one MI355X: an index directory (format 1) into HBM (the reference: load.cu:206-494,
// single device).  Every array is memory mapped and copied once; the projections become fp16 ucatT
// [C * 8b, D] and the shifts fp16, inv_f = float(1 / spacing) from the JSON value (load.cu:385-402).

#include "common.hpp"
#include "index_impl.hpp"
#include "meta.hpp"
#include "npy.hpp"

#include <hip/hip_fp16.h>

#include <algorithm>
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

auto load(raft::resources const& res, std::string const& path, load_params const& params) -> index
{
  (void)res;
  int cur = 0;
  OCTEX_HIP(hipGetDevice(&cur));
  auto impl = std::make_shared<index_impl>();
  auto& ix  = *impl;
  ix.path   = path;
  ix.params = params;
  const std::string text = read_text(path + "/meta.json");
  auto meta              = detail::json_parser(text).parse();
  OCTEX_EXPECTS(static_cast<int>(meta.number("format", 1)) == 1, "octex: unknown index format");
  ix.n             = static_cast<int64_t>(meta.number("n", 0));
  ix.dim           = static_cast<int64_t>(meta.number("dim", 0));
  const int all_c  = static_cast<int>(meta.number("copies", 0));
  ix.blocks        = static_cast<int>(meta.number("blocks", 4));
  ix.list_len      = static_cast<int>(meta.number("list_len", 0));
  ix.log_buckets   = static_cast<int>(meta.number("log_buckets", 20));
  ix.sketch_width  = static_cast<int>(meta.number("sketch_width", 0));
  ix.table_len     = static_cast<int>(meta.number("table_len", 0));
  std::vector<double> spacings;
  if (auto sp = meta.get("spacings"); sp != nullptr && sp->kind == detail::json_value::array_v)
    for (auto const& v : sp->a)
      spacings.push_back(v.d);
  for (double f : spacings)
    ix.spacings.push_back(static_cast<float>(f));
  std::map<std::string, std::string> files;
  if (auto fm = meta.get("files"); fm != nullptr && fm->kind == detail::json_value::object_v)
    for (auto const& kv : fm->o)
      files[kv.first] = kv.second.s;
  auto file = [&](std::string const& name) {
    auto it = files.find(name);
    if (it == files.end()) return path + "/" + name + ".npy";
    return it->second[0] == '/' ? it->second : path + "/" + it->second;
  };
  OCTEX_EXPECTS(ix.dim % 2 == 0, "octex: the dimension must be even");
  OCTEX_EXPECTS(ix.sketch_width % 16 == 0 && ix.sketch_width <= 512 && ix.sketch_width > 0,
                "octex: sketch width: a multiple of 16, <= 512");
  OCTEX_EXPECTS(ix.blocks >= 1 && ix.blocks <= 8 && ix.blocks != 7, "octex: blocks must be 1-6 or 8");
  const int ll = params.list_limit > 0 ? std::min(params.list_limit, ix.list_len) : ix.list_len;

  // one GPU holds the whole index: the first listed device, or the current one
  ix.device  = params.devices.empty() ? cur : params.devices.front();
  ix.devices = {ix.device};
  // copies: the saved parts (equal consecutive ranges) cut to copies_per_part, or the first
  // copies_limit copies of a single part (load.cu:252-263)
  const int nparts = std::max(1, params.parts);
  std::vector<int> cl;
  for (int q = 0; q < nparts; q++) {
    int lo = static_cast<int>(int64_t{all_c} * q / nparts);
    int hi = static_cast<int>(int64_t{all_c} * (q + 1) / nparts);
    if (params.copies_per_part > 0) hi = std::min(hi, lo + params.copies_per_part);
    if (nparts == 1 && params.copies_limit > 0) hi = std::min(hi, lo + params.copies_limit);
    for (int c = lo; c < hi; c++)
      cl.push_back(c);
  }
  OCTEX_EXPECTS(!cl.empty(), "octex: a device holds no copies (fewer copies or parts than devices)");
  ix.copies = static_cast<int>(cl.size());

  npy_file lists(file("lists")), keys(file("keys")), offsets(file("offsets")), base(file("base"));
  npy_file proj(file("proj")), shift(file("shift")), mean(file("mean"));
  npy_file basis(file("sketch_basis")), scale(file("sketch_scale"));
  npy_file sketch(file("sketch")), vectors(file("vectors"));
  std::unique_ptr<npy_file> table;
  if (ix.table_len > 0) table = std::make_unique<npy_file>(file("table"));

  const int L     = ix.levels();
  const int width = 8 * ix.blocks;
  const int64_t D = ix.dim, N = ix.n, S = ix.sketch_width;
  OCTEX_EXPECTS(L >= 1, "octex: at least one spacing");
  OCTEX_EXPECTS(lists.dim(0) == all_c && keys.dim(1) == L && proj.dim(2) == width &&
                  offsets.dim(1) == L && base.dim(1) == L && proj.dim(1) == D,
                "octex: bad shapes");
  OCTEX_EXPECTS(vectors.shape().size() >= 2 && vectors.dim(0) == N && vectors.dim(1) == D,
                "octex: vectors shape");
  OCTEX_EXPECTS(sketch.dim(0) == N && sketch.dim(1) == S, "octex: sketch shape");
  OCTEX_EXPECTS(!table || (table->dim(0) == N && table->dim(1) == ix.table_len), "octex: table shape");
  ix.T1 = offsets.dim(2);
  OCTEX_EXPECTS(ix.T1 == (int64_t{1} << ix.log_buckets) + 1,
                "octex: offsets hold %lld buckets, log_buckets %d", static_cast<long long>(ix.T1 - 1),
                ix.log_buckets);

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
  ix.sketch_pitch = detail::sketch_pitch_for(S);
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
  ix.list_len = ll;
  OCTEX_HIP(hipSetDevice(cur));
  return index(impl);
}

}  // namespace cuvs::neighbors::octex
