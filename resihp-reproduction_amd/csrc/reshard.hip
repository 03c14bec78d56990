// Bit-exact TP re-slicing on the device: concatenation (pack) and chunking
// (unpack) of row-major shards along dim 0 or dim 1, as batched strided byte
// copies.  A dim-0 shard is one contiguous block; a dim-1 shard is `rows`
// strided runs.  Each launch moves up to kMaxSeg runs-of-rows with the widest
// access (16/8/4/2/1 bytes) that every address, stride and run length allows.
#include "common.hpp"

namespace {

constexpr int kMaxSeg = 32;

struct CopySeg {
  const uint8_t* src;
  uint8_t* dst;
  int64_t src_ld;  // bytes
  int64_t dst_ld;  // bytes
  int64_t rows;
  int64_t row_bytes;
};

struct CopyBatch {
  CopySeg seg[kMaxSeg];
};

template <int W>
struct Vec;
template <> struct Vec<16> { typedef uint32_t __attribute__((ext_vector_type(4))) type; };
template <> struct Vec<8> { typedef uint32_t __attribute__((ext_vector_type(2))) type; };
template <> struct Vec<4> { typedef uint32_t type; };
template <> struct Vec<2> { typedef uint16_t type; };
template <> struct Vec<1> { typedef uint8_t type; };

template <int W>
__global__ __launch_bounds__(256) void copy_kernel(CopyBatch b) {
  typedef typename Vec<W>::type V;
  const CopySeg s = b.seg[blockIdx.y];
  const int64_t per_row = s.row_bytes / W;
  const int64_t total = s.rows * per_row;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t r = i / per_row, c = i - r * per_row;
    *reinterpret_cast<V*>(s.dst + r * s.dst_ld + c * W) = *reinterpret_cast<const V*>(s.src + r * s.src_ld + c * W);
  }
}

int width_for(const CopySeg* segs, int n) {
  uintptr_t acc = 0;
  for (int i = 0; i < n; ++i) {
    acc |= reinterpret_cast<uintptr_t>(segs[i].src) | reinterpret_cast<uintptr_t>(segs[i].dst);
    acc |= (uintptr_t)segs[i].src_ld | (uintptr_t)segs[i].dst_ld | (uintptr_t)segs[i].row_bytes;
  }
  for (int w = 16; w > 1; w >>= 1)
    if (acc % (uintptr_t)w == 0) return w;
  return 1;
}

int run_batch(const CopySeg* segs, int n, hipStream_t st) {
  int64_t most = 0;
  for (int i = 0; i < n; ++i) most = std::max<int64_t>(most, segs[i].rows * segs[i].row_bytes);
  if (n == 0 || most == 0) return RH_OK;
  CopyBatch b{};
  for (int i = 0; i < n; ++i) b.seg[i] = segs[i];
  const int w = width_for(segs, n);
  int64_t blocks = rh_cdiv(most / w, 256);
  if (blocks > 2048) blocks = 2048;
  dim3 grid((unsigned)std::max<int64_t>(blocks, 1), (unsigned)n);
  switch (w) {
    case 16: hipLaunchKernelGGL(copy_kernel<16>, grid, dim3(256), 0, st, b); break;
    case 8: hipLaunchKernelGGL(copy_kernel<8>, grid, dim3(256), 0, st, b); break;
    case 4: hipLaunchKernelGGL(copy_kernel<4>, grid, dim3(256), 0, st, b); break;
    case 2: hipLaunchKernelGGL(copy_kernel<2>, grid, dim3(256), 0, st, b); break;
    default: hipLaunchKernelGGL(copy_kernel<1>, grid, dim3(256), 0, st, b); break;
  }
  return rh_check_launch("rh_reshard copy");
}

int run_all(const CopySeg* segs, int n, hipStream_t st) {
  for (int i = 0; i < n; i += kMaxSeg) {
    int rc = run_batch(segs + i, std::min(kMaxSeg, n - i), st);
    if (rc) return rc;
  }
  return RH_OK;
}

int check_pack(int n, int64_t rows, int64_t cols, int dim, int64_t eb, const int64_t* extent) {
  RH_REQUIRE(n >= 1 && n <= 4096, "rh_reshard: shard count %d out of range", n);
  RH_REQUIRE(dim == 0 || dim == 1, "rh_reshard: shard_dim must be 0 or 1 (got %d)", dim);
  RH_REQUIRE(eb >= 1 && eb <= 16, "rh_reshard: element size %lld", (long long)eb);
  RH_REQUIRE(rows >= 0 && cols >= 0, "rh_reshard: negative extent");
  RH_REQUIRE(extent != nullptr, "rh_reshard: null extents");
  for (int i = 0; i < n; ++i) RH_REQUIRE(extent[i] >= 0, "rh_reshard: negative extent for shard %d", i);
  return RH_OK;
}

}  // namespace

extern "C" int rh_reshard_pack(const void* const* src, const int64_t* extent, int n_src, int64_t rows, int64_t cols,
                               int shard_dim, int64_t elem_bytes, void* dst, void* stream) {
  int rc = check_pack(n_src, rows, cols, shard_dim, elem_bytes, extent);
  if (rc) return rc;
  RH_REQUIRE(src != nullptr, "rh_reshard_pack: null source list");
  int64_t total = 0;
  for (int i = 0; i < n_src; ++i) total += extent[i];
  const int64_t dst_bytes = shard_dim == 0 ? total * cols * elem_bytes : rows * total * elem_bytes;
  if (dst_bytes == 0) return RH_OK;
  RH_REQUIRE(dst != nullptr, "rh_reshard_pack: null destination");
  CopySeg* segs = new CopySeg[n_src];
  int n = 0;
  int64_t off = 0;
  for (int i = 0; i < n_src; ++i) {
    const int64_t e = extent[i];
    if (e > 0) {
      if (!src[i]) {
        delete[] segs;
        return rh_set_error(RH_ERR_INVALID, "rh_reshard_pack: null source %d", i);
      }
      CopySeg s;
      s.src = static_cast<const uint8_t*>(src[i]);
      if (shard_dim == 0) {
        s.dst = static_cast<uint8_t*>(dst) + off * cols * elem_bytes;
        s.rows = 1;
        s.row_bytes = e * cols * elem_bytes;
        s.src_ld = s.dst_ld = s.row_bytes;
      } else {
        s.dst = static_cast<uint8_t*>(dst) + off * elem_bytes;
        s.rows = rows;
        s.row_bytes = e * elem_bytes;
        s.src_ld = e * elem_bytes;
        s.dst_ld = total * elem_bytes;
      }
      if (s.rows * s.row_bytes > 0) segs[n++] = s;
    }
    off += e;
  }
  rc = run_all(segs, n, static_cast<hipStream_t>(stream));
  delete[] segs;
  return rc;
}

extern "C" int rh_reshard_unpack(const void* src, int64_t rows, int64_t cols, int shard_dim, int64_t elem_bytes,
                                 int n_dst, void* const* dst, const int64_t* extent, void* stream) {
  int rc = check_pack(n_dst, rows, cols, shard_dim, elem_bytes, extent);
  if (rc) return rc;
  RH_REQUIRE(dst != nullptr, "rh_reshard_unpack: null destination list");
  int64_t total = 0;
  for (int i = 0; i < n_dst; ++i) total += extent[i];
  const int64_t full = shard_dim == 0 ? rows : cols;
  RH_REQUIRE(total <= full, "rh_reshard_unpack: extents (%lld) exceed the source extent (%lld)", (long long)total,
             (long long)full);
  CopySeg* segs = new CopySeg[n_dst];
  int n = 0;
  int64_t off = 0;
  for (int i = 0; i < n_dst; ++i) {
    const int64_t e = extent[i];
    if (e > 0) {
      if (!dst[i]) {  // skipped extent
        off += e;
        continue;
      }
      if (!src) {
        delete[] segs;
        return rh_set_error(RH_ERR_INVALID, "rh_reshard_unpack: null source");
      }
      CopySeg s;
      s.dst = static_cast<uint8_t*>(dst[i]);
      if (shard_dim == 0) {
        s.src = static_cast<const uint8_t*>(src) + off * cols * elem_bytes;
        s.rows = 1;
        s.row_bytes = e * cols * elem_bytes;
        s.src_ld = s.dst_ld = s.row_bytes;
      } else {
        s.src = static_cast<const uint8_t*>(src) + off * elem_bytes;
        s.rows = rows;
        s.row_bytes = e * elem_bytes;
        s.src_ld = cols * elem_bytes;
        s.dst_ld = e * elem_bytes;
      }
      if (s.rows * s.row_bytes > 0) segs[n++] = s;
    }
    off += e;
  }
  rc = run_all(segs, n, static_cast<hipStream_t>(stream));
  delete[] segs;
  return rc;
}

extern "C" int rh_copy2d_batch(const rh_copy2d* segs, int n, void* stream) {
  RH_REQUIRE(n >= 0 && (n == 0 || segs), "rh_copy2d_batch: bad segment list");
  CopySeg* cs = new CopySeg[n > 0 ? n : 1];
  int m = 0;
  for (int i = 0; i < n; ++i) {
    const rh_copy2d& s = segs[i];
    if (s.rows < 0 || s.row_bytes < 0 || (s.rows > 1 && (s.src_ld_bytes < s.row_bytes || s.dst_ld_bytes < s.row_bytes))) {
      delete[] cs;
      return rh_set_error(RH_ERR_INVALID, "rh_copy2d_batch: segment %d has bad extents", i);
    }
    if (s.rows == 0 || s.row_bytes == 0) continue;
    if (!s.src || !s.dst) {
      delete[] cs;
      return rh_set_error(RH_ERR_INVALID, "rh_copy2d_batch: segment %d has a null pointer", i);
    }
    CopySeg c;
    c.src = static_cast<const uint8_t*>(s.src);
    c.dst = static_cast<uint8_t*>(s.dst);
    c.src_ld = s.rows > 1 ? s.src_ld_bytes : s.row_bytes;
    c.dst_ld = s.rows > 1 ? s.dst_ld_bytes : s.row_bytes;
    c.rows = s.rows;
    c.row_bytes = s.row_bytes;
    cs[m++] = c;
  }
  const int rc = run_all(cs, m, static_cast<hipStream_t>(stream));
  delete[] cs;
  return rc;
}
