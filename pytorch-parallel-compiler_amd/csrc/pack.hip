// Byte-movement kernels of the wide path: pack (pointer-table gather), the
// N-first <-> channel-packed boundary transpose, and the embedding row gather.
//
// All three are "segment copies": the destination is a sequence of equally
// sized segments and each segment is read from an address that the map
// computes.  One kernel template serves them; a thread moves UNROLL vectors of
// V bytes (V = the widest power of two <= 16 that every address and size
// allows), issuing all loads before any store so that each wave keeps several
// HBM requests in flight.  Chunk indices are 32-bit; larger copies are split
// into several launches.
#include "wc_common.h"

namespace wc {
namespace {

constexpr int kBlock = 256;
constexpr int kUnroll = 4;
constexpr uint32_t kMaxChunksPerLaunch = 1u << 30;

template <int V> struct VecT;
template <> struct VecT<16> { typedef uint4 type; };
template <> struct VecT<8> { typedef uint2 type; };
template <> struct VecT<4> { typedef uint32_t type; };
template <> struct VecT<2> { typedef uint16_t type; };
template <> struct VecT<1> { typedef uint8_t type; };

template <typename VT> __device__ __forceinline__ VT vzero();
template <> __device__ __forceinline__ uint4 vzero<uint4>() { return make_uint4(0, 0, 0, 0); }
template <> __device__ __forceinline__ uint2 vzero<uint2>() { return make_uint2(0, 0); }
template <> __device__ __forceinline__ uint32_t vzero<uint32_t>() { return 0u; }
template <> __device__ __forceinline__ uint16_t vzero<uint16_t>() { return 0; }
template <> __device__ __forceinline__ uint8_t vzero<uint8_t>() { return 0; }

template <int V, class Map>
__global__ __launch_bounds__(kBlock) void seg_copy_kernel(Map map, uint32_t seg_base,
                                                          uint32_t total_chunks, FastDiv cps) {
  typedef typename VecT<V>::type VT;
  const uint32_t base = blockIdx.x * (kBlock * kUnroll) + threadIdx.x;
  VT vals[kUnroll];
  uint32_t segs[kUnroll], offs[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const uint32_t k = base + u * kBlock;
    if (k < total_chunks) {
      const uint32_t seg = fdiv(k, cps);
      const uint32_t c = k - seg * cps.d;
      segs[u] = seg + seg_base;
      offs[u] = c;
      const char* src = map.src(segs[u]);
      vals[u] = src ? *reinterpret_cast<const VT*>(src + static_cast<uint64_t>(c) * V) : vzero<VT>();
    }
  }
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const uint32_t k = base + u * kBlock;
    if (k < total_chunks)
      *reinterpret_cast<VT*>(map.dst(segs[u]) + static_cast<uint64_t>(offs[u]) * V) = vals[u];
  }
}

// Launches seg_copy over segments [0, nseg) of seg_bytes each, splitting into
// launches of at most kMaxChunksPerLaunch chunks.
template <class Map>
int32_t launch_seg_copy(const Map& map, int vbytes, uint64_t nseg, uint64_t seg_bytes,
                        hipStream_t stream, const char* what) {
  if (nseg == 0 || seg_bytes == 0) return WC_OK;
  const uint64_t cps = seg_bytes / static_cast<uint64_t>(vbytes);
  if (cps >= kMaxChunksPerLaunch)
    return set_error(WC_ERR_LIMIT, "%s: segment of %llu bytes is too large", what,
                     static_cast<unsigned long long>(seg_bytes));
  const uint64_t segs_per_launch = kMaxChunksPerLaunch / cps;
  const FastDiv fd = make_fastdiv(static_cast<uint32_t>(cps));
  for (uint64_t s0 = 0; s0 < nseg; s0 += segs_per_launch) {
    const uint64_t ns = (nseg - s0 < segs_per_launch) ? (nseg - s0) : segs_per_launch;
    if (s0 + ns > 0x7fffffffull)
      return set_error(WC_ERR_LIMIT, "%s: too many segments (%llu)", what,
                       static_cast<unsigned long long>(nseg));
    const uint32_t total = static_cast<uint32_t>(ns * cps);
    const dim3 grid(static_cast<uint32_t>(cdiv(total, kBlock * kUnroll)));
    switch (vbytes) {
      case 16: seg_copy_kernel<16, Map><<<grid, kBlock, 0, stream>>>(map, (uint32_t)s0, total, fd); break;
      case 8: seg_copy_kernel<8, Map><<<grid, kBlock, 0, stream>>>(map, (uint32_t)s0, total, fd); break;
      case 4: seg_copy_kernel<4, Map><<<grid, kBlock, 0, stream>>>(map, (uint32_t)s0, total, fd); break;
      case 2: seg_copy_kernel<2, Map><<<grid, kBlock, 0, stream>>>(map, (uint32_t)s0, total, fd); break;
      default: seg_copy_kernel<1, Map><<<grid, kBlock, 0, stream>>>(map, (uint32_t)s0, total, fd); break;
    }
    int32_t rc = check_launch(what);
    if (rc) return rc;
  }
  return WC_OK;
}

// ---------------------------------------------------------------------------
// pack: dst[r, i0 + i, :] = src_i[r, :]
// ---------------------------------------------------------------------------
constexpr int kPackMaxSrc = 120;

struct PackMap {
  const char* srcp[kPackMaxSrc];
  int64_t src_stride[kPackMaxSrc];
  char* dstp;           // already offset to column block i0
  int64_t dst_row;      // bytes between dst rows (n_total * row_bytes)
  int64_t row_bytes;
  FastDiv nsrc;         // sources in this launch
  __device__ __forceinline__ const char* src(uint32_t seg) const {
    const uint32_t r = fdiv(seg, nsrc);
    const uint32_t i = seg - r * nsrc.d;
    return srcp[i] + static_cast<int64_t>(r) * src_stride[i];
  }
  __device__ __forceinline__ char* dst(uint32_t seg) const {
    const uint32_t r = fdiv(seg, nsrc);
    const uint32_t i = seg - r * nsrc.d;
    return dstp + static_cast<int64_t>(r) * dst_row + static_cast<int64_t>(i) * row_bytes;
  }
};

// ---------------------------------------------------------------------------
// swap01: dst[j, i, :] = src[i, j, :]  (dst contiguous [d1, d0, inner])
// ---------------------------------------------------------------------------
struct SwapMap {
  const char* srcp;
  char* dstp;
  int64_t s0, s1, inner;
  FastDiv d0;
  __device__ __forceinline__ const char* src(uint32_t seg) const {
    const uint32_t j = fdiv(seg, d0);
    const uint32_t i = seg - j * d0.d;
    return srcp + static_cast<int64_t>(i) * s0 + static_cast<int64_t>(j) * s1;
  }
  __device__ __forceinline__ char* dst(uint32_t seg) const {
    return dstp + static_cast<int64_t>(seg) * inner;
  }
};

// ---------------------------------------------------------------------------
// embedding gather: out[i, r, :] = W[i, ids[(i,) r], :]
// ---------------------------------------------------------------------------
struct GatherMap {
  const char* w;
  const int64_t* ids;
  char* out;
  int64_t vocab, row_bytes;
  int32_t* err;
  int32_t shared;
  FastDiv rows;
  __device__ __forceinline__ const char* src(uint32_t seg) const {
    const uint32_t i = fdiv(seg, rows);
    const uint32_t r = seg - i * rows.d;
    const int64_t id = shared ? ids[r] : ids[seg];
    if (id < 0 || id >= vocab) {
      if (err) *err = 1;
      return nullptr;
    }
    return w + (static_cast<int64_t>(i) * vocab + id) * row_bytes;
  }
  __device__ __forceinline__ char* dst(uint32_t seg) const {
    return out + static_cast<int64_t>(seg) * row_bytes;
  }
};

}  // namespace
}  // namespace wc

using namespace wc;

extern "C" int32_t wc_pack_rows(const void* const* srcs, const int64_t* src_row_stride_bytes,
                                int64_t n, int64_t rows, int64_t row_bytes, void* dst,
                                void* stream) {
  clear_error();
  WC_REQUIRE(n >= 0 && rows >= 0 && row_bytes >= 0, WC_ERR_SHAPE,
             "wc_pack_rows: negative size (n=%lld rows=%lld row_bytes=%lld)", (long long)n,
             (long long)rows, (long long)row_bytes);
  if (n == 0 || rows == 0 || row_bytes == 0) return WC_OK;
  WC_REQUIRE(srcs && src_row_stride_bytes && dst, WC_ERR_NULL, "wc_pack_rows: null pointer");
  uint64_t g = reinterpret_cast<uintptr_t>(dst) | static_cast<uint64_t>(row_bytes);
  for (int64_t i = 0; i < n; ++i) {
    WC_REQUIRE(srcs[i] != nullptr, WC_ERR_NULL, "wc_pack_rows: source %lld is null", (long long)i);
    g |= reinterpret_cast<uintptr_t>(srcs[i]) | static_cast<uint64_t>(src_row_stride_bytes[i]);
  }
  const int vb = common_vec_bytes({g});
  for (int64_t i0 = 0; i0 < n; i0 += kPackMaxSrc) {
    const int64_t nc = (n - i0 < kPackMaxSrc) ? (n - i0) : kPackMaxSrc;
    PackMap m;
    for (int64_t i = 0; i < nc; ++i) {
      m.srcp[i] = static_cast<const char*>(srcs[i0 + i]);
      m.src_stride[i] = src_row_stride_bytes[i0 + i];
    }
    m.dstp = static_cast<char*>(dst) + i0 * row_bytes;
    m.dst_row = n * row_bytes;
    m.row_bytes = row_bytes;
    m.nsrc = make_fastdiv(static_cast<uint32_t>(nc));
    int32_t rc = launch_seg_copy(m, vb, static_cast<uint64_t>(rows * nc),
                                 static_cast<uint64_t>(row_bytes), as_stream(stream), "wc_pack_rows");
    if (rc) return rc;
  }
  return WC_OK;
}

extern "C" int32_t wc_swap01(const void* src, int64_t d0, int64_t d1, int64_t src_stride0_bytes,
                             int64_t src_stride1_bytes, int64_t inner_bytes, void* dst,
                             void* stream) {
  clear_error();
  WC_REQUIRE(d0 >= 0 && d1 >= 0 && inner_bytes >= 0, WC_ERR_SHAPE, "wc_swap01: negative size");
  if (d0 == 0 || d1 == 0 || inner_bytes == 0) return WC_OK;
  WC_REQUIRE(src && dst, WC_ERR_NULL, "wc_swap01: null pointer");
  WC_REQUIRE(d0 < 0x7fffffffll && d1 < 0x7fffffffll, WC_ERR_LIMIT, "wc_swap01: dims too large");
  const int vb = common_vec_bytes({reinterpret_cast<uintptr_t>(src), reinterpret_cast<uintptr_t>(dst),
                                   static_cast<uint64_t>(src_stride0_bytes),
                                   static_cast<uint64_t>(src_stride1_bytes),
                                   static_cast<uint64_t>(inner_bytes)});
  SwapMap m;
  m.srcp = static_cast<const char*>(src);
  m.dstp = static_cast<char*>(dst);
  m.s0 = src_stride0_bytes;
  m.s1 = src_stride1_bytes;
  m.inner = inner_bytes;
  m.d0 = make_fastdiv(static_cast<uint32_t>(d0));
  return launch_seg_copy(m, vb, static_cast<uint64_t>(d0 * d1), static_cast<uint64_t>(inner_bytes),
                         as_stream(stream), "wc_swap01");
}

extern "C" int32_t wc_embedding_gather(const void* weight, int64_t n, int64_t vocab, int64_t dim,
                                       int32_t dtype, const int64_t* ids, int64_t rows,
                                       int32_t ids_shared, void* out, int32_t* err_flag,
                                       void* stream) {
  clear_error();
  const int es = dtype_size(dtype);
  WC_REQUIRE(es > 0, WC_ERR_DTYPE, "wc_embedding_gather: unsupported dtype %d", dtype);
  WC_REQUIRE(n >= 0 && vocab >= 0 && dim >= 0 && rows >= 0, WC_ERR_SHAPE,
             "wc_embedding_gather: negative size");
  if (n == 0 || rows == 0 || dim == 0) return WC_OK;
  WC_REQUIRE(weight && ids && out, WC_ERR_NULL, "wc_embedding_gather: null pointer");
  WC_REQUIRE(rows < 0x7fffffffll && mul_sat({n, rows}) < 0x7fffffffll && dim < (int64_t{1} << 40),
             WC_ERR_LIMIT, "wc_embedding_gather: too many rows");
  const int64_t row_bytes = dim * es;
  const int vb = common_vec_bytes({reinterpret_cast<uintptr_t>(weight),
                                   reinterpret_cast<uintptr_t>(out),
                                   static_cast<uint64_t>(row_bytes)});
  GatherMap m;
  m.w = static_cast<const char*>(weight);
  m.ids = ids;
  m.out = static_cast<char*>(out);
  m.vocab = vocab;
  m.row_bytes = row_bytes;
  m.err = err_flag;
  m.shared = ids_shared;
  m.rows = make_fastdiv(static_cast<uint32_t>(rows));
  return launch_seg_copy(m, vb, static_cast<uint64_t>(n * rows), static_cast<uint64_t>(row_bytes),
                         as_stream(stream), "wc_embedding_gather");
}
