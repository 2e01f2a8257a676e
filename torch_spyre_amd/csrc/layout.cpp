// Host side of the stick layout: the SpyreTensorLayout descriptor and the
// DMA loop nests that move a tensor between host order and device order.
//
// Device order: a layout is (device_size, stride_map).  Device memory is
// row-major over device_size; the last device dim is the 128-byte stick.
// Stepping +1 along device dim j advances stride_map[j] elements in host
// memory (-1: synthetic / padded dim with no host counterpart), so
// host_offset = dot(device_coords, stride_map)
// (docs/source/user_guide/tensors_and_layouts.md:165-221).
//
// The algorithms follow torch_spyre/csrc/spyre_tensor_impl.cpp:46-179 (default
// tiling) and torch_spyre/csrc/spyre_mem.cpp:60-354 (DMA description), so
// that the loop nests, including their remainder splitting, are the ones the
// reference hands to its DMA engine.

#include <algorithm>
#include <cstring>
#include <map>
#include <vector>

#include "spyre_common.h"

namespace spyre_hip {

namespace {

thread_local std::string g_last_error;

}  // namespace

void set_error(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
}

void clear_error() { g_last_error.clear(); }

const char* last_error() { return g_last_error.c_str(); }

}  // namespace spyre_hip

namespace {

using I64 = std::vector<int64_t>;
constexpr int64_t kBytesInStick = 128;  // torch_spyre/csrc/spyre_tensor_impl.cpp:31

int64_t stick_elems(int fmt) {
  switch (fmt) {
    case SPYRE_FMT_SEN169_FP16: return kBytesInStick / 2;
    case SPYRE_FMT_IEEE_FP32: return kBytesInStick / 4;
    case SPYRE_FMT_IEEE_INT32: return kBytesInStick / 4;
    default: return -1;
  }
}

// Host element type -> device format (torch_spyre/csrc/types_mapping.h:71-92).
int format_of(int scalar_type) {
  switch (scalar_type) {
    case SPYRE_DT_FLOAT16:
    case SPYRE_DT_BFLOAT16:
    case SPYRE_DT_BOOL: return SPYRE_FMT_SEN169_FP16;
    case SPYRE_DT_FLOAT32: return SPYRE_FMT_IEEE_FP32;
    case SPYRE_DT_INT32:
    case SPYRE_DT_INT64: return SPYRE_FMT_IEEE_INT32;
    default: return SPYRE_FMT_INVALID;
  }
}

// Default tiling of a dim order o (ranks 1..6): every non-stick dim once, in
// order o1..o_{r-1}, then o0, then the stick dim o_{r-1} again as the
// innermost 64-element stick.  The entry at position r-1 (the first
// occurrence of o_{r-1}) is the stick's tile index.
std::vector<int32_t> tiling_of(const std::vector<int32_t>& o) {
  const int r = static_cast<int>(o.size());
  std::vector<int32_t> m;
  m.reserve(r + 1);
  for (int i = 1; i < r; ++i) m.push_back(o[i]);
  m.push_back(o[0]);
  m.push_back(o[r - 1]);
  return m;
}

// stride_map from a dim map: walking from the innermost device dim outwards,
// the first device dim of a host dim takes that host dim's stride and each
// further one the stride reached after the previous one's extent.
I64 strides_of_tiling(const std::vector<int32_t>& dim_map, const I64& host_size,
                      const I64& host_stride, const I64& device_size) {
  const int n = static_cast<int>(dim_map.size());
  I64 sm(n, -1);
  I64 next(host_size.size(), -1);
  for (int j = n - 1; j >= 0; --j) {
    const int32_t d = dim_map[j];
    if (d < 0 || host_size[d] == 1) continue;
    sm[j] = next[d] == -1 ? host_stride[d] : next[d];
    next[d] = sm[j] * device_size[j];
  }
  return sm;
}

// ---- DMA description --------------------------------------------------

// Host dim that owns each device dim: the host dim with the largest stride
// not above stride_map[j]; the stick's tile slot follows the stick itself
// (spyre_mem.cpp:60-96).
std::vector<int> owners(const I64& sizes, const I64& strides, const I64& dsize, const I64& smap) {
  const int hr = static_cast<int>(strides.size());
  const int dr = static_cast<int>(smap.size());
  const int tile_slot = dr > 2 ? dr - 3 : 0;
  std::vector<int> own(dr, -1);
  I64 best(dr, 0);
  for (int h = 0; h < hr; ++h) {
    if (sizes[h] == 1 || strides[h] == 0) continue;
    for (int j = 0; j < dr; ++j) {
      if (dsize[j] == 1) continue;
      if (strides[h] > best[j] && strides[h] <= smap[j]) {
        best[j] = strides[h];
        own[j] = h;
      }
    }
  }
  if (own[tile_slot] != -1) own[tile_slot] = own[dr - 1];
  return own;
}

// Per host dim, its device dims ordered by stride_map (stick keyed -1); on
// equal keys the outermost-inserted entry (highest j) is kept
// (spyre_mem.cpp:107-162).
std::vector<std::vector<int>> tiles_per_host_dim(const I64& sizes, const I64& strides,
                                                 const I64& dsize, const I64& smap) {
  const std::vector<int> own = owners(sizes, strides, dsize, smap);
  const int hr = static_cast<int>(strides.size());
  const int dr = static_cast<int>(smap.size());
  std::vector<std::map<int64_t, int>> keyed(hr);
  if (own[dr - 1] != -1) keyed[own[dr - 1]].emplace(-1, dr - 1);
  for (int j = dr - 2; j >= 0; --j)
    if (own[j] != -1) keyed[own[j]].emplace(smap[j], j);
  std::vector<std::vector<int>> out(hr);
  for (int h = 0; h < hr; ++h)
    for (const auto& kv : keyed[h]) out[h].push_back(kv.second);
  return out;
}

int plan_dma(const I64& sizes, const I64& dma_strides, const I64& cpu_strides,
             int64_t storage_offset, const I64& dsize, const I64& smap, bool h2d,
             std::vector<spyre_stride_info>& out) {
  const int hr = static_cast<int>(cpu_strides.size());
  const int dr = static_cast<int>(smap.size());
  const auto tiles = tiles_per_host_dim(sizes, dma_strides, dsize, smap);

  I64 hstr(dr, 1), cpu(dr, 1), dstr(dr, 1), extent(dr, 1);
  int64_t run = 1;
  for (int j = dr - 1; j >= 0; --j) {
    if (smap[j] == 0) extent[j] = dsize[j];  // broadcast dim: written for every coordinate
    dstr[j] = run;
    run *= dsize[j];
    if (smap[j] != -1) hstr[j] = cpu[j] = smap[j];
  }
  // Device dims whose stride equals a host dim's dma stride take that host
  // dim's actual (cpu) stride.
  for (int j = 0; j < dr; ++j) {
    if (smap[j] <= 0) continue;
    for (int h = 0; h < hr; ++h)
      if (dma_strides[h] == smap[j]) {
        cpu[j] = cpu_strides[h];
        break;
      }
  }

  struct Rem {
    I64 ext;
    int64_t host_off, dev_off;
  };
  std::vector<Rem> rems;
  for (int h = hr - 1; h >= 0; --h) {
    const auto& t = tiles[h];
    if (t.empty()) continue;
    const int64_t hs = dma_strides[h];
    int64_t span = sizes[h];
    for (int o = h - 1; o >= 0 && tiles[o].empty(); --o)  // fold unowned outer dims
      if (dma_strides[o] != 0) span *= sizes[o];
    int64_t covered = 1;
    for (int k = static_cast<int>(t.size()) - 1; k >= 0; --k) {
      const int j = t[k];
      if (dsize[j] == 1) continue;
      const int64_t step = hstr[j] / hs;
      SPYRE_REQUIRE(span % covered == 0, SPYRE_EINVAL,
                    "Invalid device sizes and stride map for host sizes and strides");
      const int64_t left = span / covered;
      const int64_t whole = left / step;
      SPYRE_REQUIRE(whole > 0, SPYRE_EINVAL,
                    "Invalid device sizes and stride map for host sizes and strides");
      if (left % step == 0) {
        extent[j] = std::min(whole, dsize[j]);
        covered *= extent[j];
        continue;
      }
      // Partial tile: this dim gets `whole` full steps and the next inner
      // dim (which must exist) gets a tail of `inner % dsize[i]` elements.
      SPYRE_REQUIRE(k != 0, SPYRE_EINVAL, "Invalid tiling for dimension");
      const int i = t[--k];
      const int64_t inner = left / (hstr[i] / hs);
      extent[j] = whole;
      extent[i] = dsize[i];
      covered *= inner;
      Rem r{I64(dr, 0), whole * hstr[j], whole * dstr[j]};
      r.ext[j] = 1;
      r.ext[i] = inner % dsize[i];
      rems.push_back(r);
    }
  }

  auto fill = [&](spyre_stride_info& s, const I64& ext, int64_t osrc, int64_t odst) {
    std::memset(&s, 0, sizeof(s));
    s.rank = dr;
    for (int q = 0; q < dr; ++q) {  // innermost first
      const int j = dr - 1 - q;
      s.size[q] = ext[j];
      s.stride_src[q] = h2d ? cpu[j] : dstr[j];
      s.stride_dst[q] = h2d ? dstr[j] : cpu[j];
    }
    s.offset_src = osrc;
    s.offset_dst = odst;
  };
  out.clear();
  out.emplace_back();
  fill(out.back(), extent, h2d ? storage_offset : 0, h2d ? 0 : storage_offset);
  for (const Rem& r : rems) {
    const size_t n = out.size();
    for (size_t k = 0; k < n; ++k) {
      spyre_stride_info s = out[k];
      for (int q = 0; q < dr; ++q) {
        const int64_t e = r.ext[dr - 1 - q];
        if (e != 0) s.size[q] = e;
      }
      s.offset_src += h2d ? r.host_off : r.dev_off;
      s.offset_dst += h2d ? r.dev_off : r.host_off;
      out.push_back(s);
      SPYRE_REQUIRE(out.size() <= SPYRE_MAX_INFOS, SPYRE_EUNSUPPORTED,
                    "DMA description needs more than %d loop nests", SPYRE_MAX_INFOS);
    }
  }
  return SPYRE_OK;
}

bool valid_layout_args(const int64_t* a, const int64_t* b, int rank) {
  return a != nullptr && b != nullptr && rank >= 1 && rank <= SPYRE_MAX_RANK;
}

// One layout's view of a dense host tensor as digits of a mixed radix:
// (host stride, extent, device stride), sorted by host stride.
struct Digit {
  int64_t hs, ext, ds;
};

int digits_of(const I64& host_size, const I64& dsize, const I64& smap, std::vector<Digit>& dig) {
  I64 hst(host_size.size());
  int64_t run = 1;
  for (int h = static_cast<int>(host_size.size()) - 1; h >= 0; --h) {
    hst[h] = run;
    run *= host_size[h];
  }
  const int64_t numel = run;
  std::vector<spyre_stride_info> infos;
  int rc = plan_dma(host_size, hst, hst, 0, dsize, smap, true, infos);
  if (rc != SPYRE_OK) return rc;
  SPYRE_REQUIRE(infos.size() == 1, SPYRE_EUNSUPPORTED,
                "restickify: layout has partial tiles (padding); no single-pass plan");
  const spyre_stride_info& s = infos[0];
  dig.clear();
  for (int q = 0; q < s.rank; ++q) {
    if (s.size[q] == 1) continue;
    SPYRE_REQUIRE(s.stride_src[q] > 0, SPYRE_EUNSUPPORTED,
                  "restickify: broadcast layouts have no single-pass plan");
    dig.push_back({s.stride_src[q], s.size[q], s.stride_dst[q]});
  }
  std::sort(dig.begin(), dig.end(), [](const Digit& a, const Digit& b) { return a.hs < b.hs; });
  int64_t expect = 1;
  for (const Digit& d : dig) {
    SPYRE_REQUIRE(d.hs == expect, SPYRE_EUNSUPPORTED,
                  "restickify: layout does not tile the host tensor exactly");
    expect = d.hs * d.ext;
  }
  SPYRE_REQUIRE(expect == numel, SPYRE_EUNSUPPORTED,
                "restickify: layout covers %lld of %lld elements", (long long)expect,
                (long long)numel);
  return SPYRE_OK;
}

// Splits every digit at the given host-stride cut points.
int refine(std::vector<Digit>& dig, const std::vector<int64_t>& cuts) {
  std::vector<Digit> out;
  for (const Digit& d : dig) {
    int64_t lo = d.hs, ds = d.ds;
    const int64_t hi = d.hs * d.ext;
    for (int64_t c : cuts) {
      if (c <= lo || c >= hi) continue;
      SPYRE_REQUIRE(c % lo == 0 && hi % c == 0, SPYRE_EUNSUPPORTED,
                    "restickify: tilings do not nest");
      out.push_back({lo, c / lo, ds});
      ds *= c / lo;
      lo = c;
    }
    out.push_back({lo, hi / lo, ds});
  }
  dig.swap(out);
  return SPYRE_OK;
}

}  // namespace

extern "C" {

int spyre_abi_version(void) { return SPYRE_ABI_VERSION; }

const char* spyre_last_error(void) { return spyre_hip::last_error(); }

int spyre_device_format(int scalar_type) { return format_of(scalar_type); }

int64_t spyre_elems_per_stick(int data_format) { return stick_elems(data_format); }

int spyre_stl_init(const int64_t* host_size, int host_rank, const int64_t* host_strides,
                   int scalar_type, const int32_t* dim_order, int dim_order_len,
                   int64_t* device_size, int64_t* stride_map, int* device_rank,
                   int* data_format) {
  spyre_hip::clear_error();
  SPYRE_REQUIRE(host_rank >= 0 && host_rank <= 6, SPYRE_EINVAL, "Unsupported tensor rank: %d",
                host_rank);
  SPYRE_REQUIRE(device_size && stride_map && device_rank && data_format, SPYRE_EINVAL,
                "null output pointer");
  SPYRE_REQUIRE(host_rank == 0 || host_size, SPYRE_EINVAL, "null host_size");
  const int fmt = format_of(scalar_type);
  SPYRE_REQUIRE(fmt != SPYRE_FMT_INVALID, SPYRE_EINVAL, "unsupported dtype code %d", scalar_type);
  const int64_t eps = stick_elems(fmt);
  *data_format = fmt;

  I64 hsize(host_size, host_size + host_rank);
  I64 hstride(host_rank);
  if (host_strides) {
    hstride.assign(host_strides, host_strides + host_rank);
  } else {
    int64_t run = 1;
    for (int i = host_rank - 1; i >= 0; --i) {
      hstride[i] = run;
      run *= hsize[i];
    }
  }
  std::vector<int32_t> order;
  if (dim_order) {
    order.assign(dim_order, dim_order + dim_order_len);
  } else {
    for (int i = 0; i < host_rank; ++i) order.push_back(i);
  }
  const bool sparse = !order.empty() && order.back() == -1;
  SPYRE_REQUIRE(order.size() == hsize.size() || (sparse && order.size() == hsize.size() + 1),
                SPYRE_EINVAL, "Incompatible host_size and dim_order");
  for (int32_t d : order)
    SPYRE_REQUIRE(d >= -1 && d < host_rank, SPYRE_EINVAL, "dim_order entry %d out of range", d);

  if (host_rank == 0) {  // scalar: one stick, nothing mapped
    device_size[0] = 1;
    device_size[1] = eps;
    stride_map[0] = stride_map[1] = -1;
    *device_rank = 2;
    return SPYRE_OK;
  }
  SPYRE_REQUIRE(order.size() <= 6, SPYRE_EINVAL, "Unsupported tensor rank: %d",
                static_cast<int>(order.size()));
  const std::vector<int32_t> dim_map = tiling_of(order);
  const int dr = static_cast<int>(dim_map.size());
  const int32_t stick = dim_map.back();
  I64 dsize(dr);
  dsize[dr - 1] = eps;
  for (int i = 0; i < dr - 1; ++i) {
    const int32_t d = dim_map[i];
    if (d == stick)
      dsize[i] = sparse ? 1 : (hsize[stick] + eps - 1) / eps;
    else
      dsize[i] = hsize[d];
  }
  const I64 smap = strides_of_tiling(dim_map, hsize, hstride, dsize);
  for (int i = 0; i < dr; ++i) {
    device_size[i] = dsize[i];
    stride_map[i] = smap[i];
  }
  *device_rank = dr;
  return SPYRE_OK;
}

uint64_t spyre_device_size_in_bytes(const int64_t* device_size, int device_rank) {
  if (!device_size || device_rank < 1) return 0;
  uint64_t n = kBytesInStick;
  for (int i = 0; i < device_rank - 1; ++i) n *= static_cast<uint64_t>(device_size[i]);
  return n;
}

int spyre_dma_plan(const int64_t* sizes, const int64_t* dma_strides, const int64_t* cpu_strides,
                   int host_rank, int64_t storage_offset, const int64_t* device_size,
                   const int64_t* stride_map, int device_rank, int host2device,
                   spyre_stride_info* infos, int max_infos, int* n_infos) {
  spyre_hip::clear_error();
  SPYRE_REQUIRE(host_rank >= 1 && host_rank <= SPYRE_MAX_RANK && sizes && dma_strides &&
                    cpu_strides,
                SPYRE_EINVAL, "bad host shape arguments");
  SPYRE_REQUIRE(valid_layout_args(device_size, stride_map, device_rank), SPYRE_EINVAL,
                "bad layout arguments");
  SPYRE_REQUIRE(infos && n_infos && max_infos > 0, SPYRE_EINVAL, "bad output arguments");
  std::vector<spyre_stride_info> out;
  const int rc = plan_dma(I64(sizes, sizes + host_rank), I64(dma_strides, dma_strides + host_rank),
                          I64(cpu_strides, cpu_strides + host_rank), storage_offset,
                          I64(device_size, device_size + device_rank),
                          I64(stride_map, stride_map + device_rank), host2device != 0, out);
  if (rc != SPYRE_OK) return rc;
  SPYRE_REQUIRE(static_cast<int>(out.size()) <= max_infos, SPYRE_ENOSPC,
                "need %d stride infos, capacity %d", static_cast<int>(out.size()), max_infos);
  std::copy(out.begin(), out.end(), infos);
  *n_infos = static_cast<int>(out.size());
  return SPYRE_OK;
}

int spyre_restick_plan(const int64_t* host_size, int host_rank,
                       const int64_t* src_device_size, const int64_t* src_stride_map, int src_rank,
                       const int64_t* dst_device_size, const int64_t* dst_stride_map, int dst_rank,
                       spyre_stride_info* info) {
  spyre_hip::clear_error();
  SPYRE_REQUIRE(host_size && host_rank >= 1 && host_rank <= 6 && info, SPYRE_EINVAL,
                "bad arguments");
  SPYRE_REQUIRE(valid_layout_args(src_device_size, src_stride_map, src_rank) &&
                    valid_layout_args(dst_device_size, dst_stride_map, dst_rank),
                SPYRE_EINVAL, "bad layout arguments");
  const I64 hs(host_size, host_size + host_rank);
  std::vector<Digit> a, b;
  int rc = digits_of(hs, I64(src_device_size, src_device_size + src_rank),
                     I64(src_stride_map, src_stride_map + src_rank), a);
  if (rc != SPYRE_OK) return rc;
  rc = digits_of(hs, I64(dst_device_size, dst_device_size + dst_rank),
                 I64(dst_stride_map, dst_stride_map + dst_rank), b);
  if (rc != SPYRE_OK) return rc;
  std::vector<int64_t> cuts;
  for (const Digit& d : a) cuts.push_back(d.hs);
  for (const Digit& d : b) cuts.push_back(d.hs);
  std::sort(cuts.begin(), cuts.end());
  if ((rc = refine(a, cuts)) != SPYRE_OK) return rc;
  if ((rc = refine(b, cuts)) != SPYRE_OK) return rc;
  SPYRE_REQUIRE(a.size() == b.size(), SPYRE_EUNSUPPORTED, "restickify: tilings do not nest");
  SPYRE_REQUIRE(a.size() <= SPYRE_MAX_RANK, SPYRE_EUNSUPPORTED, "restickify: too many loops");
  std::memset(info, 0, sizeof(*info));
  info->rank = static_cast<int32_t>(a.size());
  for (size_t q = 0; q < a.size(); ++q) {
    SPYRE_REQUIRE(a[q].hs == b[q].hs && a[q].ext == b[q].ext, SPYRE_EUNSUPPORTED,
                  "restickify: tilings do not nest");
    info->size[q] = a[q].ext;
    info->stride_src[q] = a[q].ds;
    info->stride_dst[q] = b[q].ds;
  }
  if (info->rank == 0) {  // single element
    info->rank = 1;
    info->size[0] = 1;
    info->stride_src[0] = info->stride_dst[0] = 1;
  }
  return SPYRE_OK;
}

}  // extern "C"
