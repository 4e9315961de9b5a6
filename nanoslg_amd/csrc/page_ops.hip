// Byte-moving kernels of the KV pool: append (scatter of new token rows),
// zero-pages, copy-pages (copy-on-write) and gather (paged -> contiguous).
//
// All four are HBM-bound row copies. A "row" is one token's Hkv*D elements
// (2 KiB at Hkv=8, D=128, fp16). Rows are moved with the widest vector access
// the pointers and strides allow (16 B on the normal path), one workgroup per
// row or per page, consecutive lanes on consecutive 16 B words so each wave
// issues fully coalesced 1 KiB requests.
#include "nslg_common.h"

namespace nslg {
namespace {

template <typename V>
__global__ void __launch_bounds__(256)
append_rows_kernel(const char* __restrict__ k_src, const char* __restrict__ v_src,
                   int64_t k_src_stride, int64_t v_src_stride,  // bytes
                   const int32_t* __restrict__ slot_mapping,
                   char* __restrict__ k_pool, char* __restrict__ v_pool,
                   int64_t pool_slots, int32_t row_bytes) {
  const int t = blockIdx.x;
  const int32_t slot = slot_mapping[t];
  if (slot < 0 || (int64_t)slot >= pool_slots) return;
  const bool is_v = blockIdx.y != 0;
  const V* src = reinterpret_cast<const V*>((is_v ? v_src : k_src) +
                                            (int64_t)t * (is_v ? v_src_stride : k_src_stride));
  V* dst = reinterpret_cast<V*>((is_v ? v_pool : k_pool) + (int64_t)slot * row_bytes);
  const int nvec = row_bytes / (int)sizeof(V);
  for (int i = threadIdx.x; i < nvec; i += blockDim.x) stream_store(dst + i, src[i]);
}

// Flat grid over (page list entry, 16-byte word of the page) for one layer
// (blockIdx.y) and one of K|V (blockIdx.z): each thread moves one word, so even
// a handful of pages spreads over many workgroups.
template <typename V>
__global__ void __launch_bounds__(256)
zero_pages_kernel(char* __restrict__ k_pool, char* __restrict__ v_pool, int64_t num_pages,
                  int64_t page_bytes, const int32_t* __restrict__ ids, int32_t n) {
  const int64_t nvec = page_bytes / (int64_t)sizeof(V);
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= nvec * n) return;
  const int i = (int)(idx / nvec);
  const int64_t w = idx - (int64_t)i * nvec;
  const int32_t pid = ids[i];
  if (pid < 0 || (int64_t)pid >= num_pages) return;
  char* base = (blockIdx.z ? v_pool : k_pool) + ((int64_t)blockIdx.y * num_pages + pid) * page_bytes;
  V z;
  __builtin_memset(&z, 0, sizeof(V));
  stream_store(reinterpret_cast<V*>(base) + w, z);
}

template <typename V>
__global__ void __launch_bounds__(256)
copy_pages_kernel(char* __restrict__ k_pool, char* __restrict__ v_pool, int64_t num_pages,
                  int64_t page_bytes, const int32_t* __restrict__ src_ids,
                  const int32_t* __restrict__ dst_ids, int32_t n) {
  const int64_t nvec = page_bytes / (int64_t)sizeof(V);
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= nvec * n) return;
  const int i = (int)(idx / nvec);
  const int64_t w = idx - (int64_t)i * nvec;
  const int32_t s = src_ids[i];
  const int32_t d = dst_ids[i];
  if (s < 0 || (int64_t)s >= num_pages || d < 0 || (int64_t)d >= num_pages) return;
  char* pool = blockIdx.z ? v_pool : k_pool;
  const int64_t layer_off = (int64_t)blockIdx.y * num_pages;
  const V* src = reinterpret_cast<const V*>(pool + (layer_off + s) * page_bytes);
  V* dst = reinterpret_cast<V*>(pool + (layer_off + d) * page_bytes);
  stream_store(dst + w, src[w]);
}

// grid (max_len, batch, 2): row t of sequence b, K or V.
template <typename V>
__global__ void __launch_bounds__(256)
gather_rows_kernel(const char* __restrict__ k_pool, const char* __restrict__ v_pool,
                   int64_t num_pages, int32_t page_size, const int32_t* __restrict__ indptr,
                   const int32_t* __restrict__ indices, const int32_t* __restrict__ last_len,
                   int32_t max_len, int32_t row_bytes, char* __restrict__ k_out,
                   char* __restrict__ v_out) {
  const int t = blockIdx.x;
  const int b = blockIdx.y;
  const bool is_v = blockIdx.z != 0;
  const int32_t p0 = indptr[b];
  const int32_t np = indptr[b + 1] - p0;
  int32_t lpl = last_len[b];
  lpl = lpl < 1 ? 1 : (lpl > page_size ? page_size : lpl);
  const int64_t len = np > 0 ? (int64_t)(np - 1) * page_size + lpl : 0;
  V* dst = reinterpret_cast<V*>((is_v ? v_out : k_out) + ((int64_t)b * max_len + t) * row_bytes);
  const int nvec = row_bytes / (int)sizeof(V);
  if (t < len) {
    int32_t pid = indices[p0 + t / page_size];
    if (pid < 0 || (int64_t)pid >= num_pages) pid = 0;
    const int64_t slot = (int64_t)pid * page_size + t % page_size;
    const V* src = reinterpret_cast<const V*>((is_v ? v_pool : k_pool) + slot * row_bytes);
    for (int i = threadIdx.x; i < nvec; i += blockDim.x) dst[i] = src[i];
  } else {
    V z;
    __builtin_memset(&z, 0, sizeof(V));
    for (int i = threadIdx.x; i < nvec; i += blockDim.x) dst[i] = z;
  }
}

// Widest access (16, 8, 4 or 2 bytes) that divides every byte quantity given.
inline int pick_vec(std::initializer_list<int64_t> quantities) {
  int w = 16;
  for (int64_t q : quantities) {
    while (w > 2 && (q % w) != 0) w >>= 1;
  }
  return w;
}

inline int threads_for(int64_t nvec) {
  int64_t t = ((nvec + 63) / 64) * 64;
  if (t > 256) t = 256;
  if (t < 64) t = 64;
  return (int)t;
}

}  // namespace
}  // namespace nslg

using namespace nslg;

extern "C" int nslg_append_kv(const void* k_src, const void* v_src, int64_t k_src_stride,
                              int64_t v_src_stride, const int32_t* slot_mapping,
                              int32_t num_tokens, void* k_pool, void* v_pool,
                              int64_t pool_slots, int32_t num_kv_heads, int32_t head_dim,
                              int32_t dtype, nslg_stream_t stream) {
  const int eb = elem_bytes(dtype);
  if (!eb) return fail(NSLG_EINVAL, "append_kv: bad dtype %d", dtype);
  if (num_tokens < 0 || num_kv_heads <= 0 || head_dim <= 0 || pool_slots <= 0)
    return fail(NSLG_EINVAL, "append_kv: bad sizes T=%d Hkv=%d D=%d slots=%lld", num_tokens,
                num_kv_heads, head_dim, (long long)pool_slots);
  if (num_tokens == 0) return NSLG_OK;
  if (!k_src || !v_src || !slot_mapping || !k_pool || !v_pool)
    return fail(NSLG_EINVAL, "append_kv: null pointer");
  if (num_tokens > 0x7fffffff / 2) return fail(NSLG_EINVAL, "append_kv: too many tokens");
  const int64_t row_bytes = (int64_t)num_kv_heads * head_dim * eb;
  if (row_bytes > (1 << 30)) return fail(NSLG_EINVAL, "append_kv: row too large");
  const int64_t ks = k_src_stride * eb, vs = v_src_stride * eb;
  if (k_src_stride < (int64_t)num_kv_heads * head_dim && num_tokens > 1)
    return fail(NSLG_EINVAL, "append_kv: k source rows overlap (stride %lld)", (long long)k_src_stride);
  if (v_src_stride < (int64_t)num_kv_heads * head_dim && num_tokens > 1)
    return fail(NSLG_EINVAL, "append_kv: v source rows overlap (stride %lld)", (long long)v_src_stride);
  const int w = pick_vec({row_bytes, ks, vs, (int64_t)(uintptr_t)k_src, (int64_t)(uintptr_t)v_src,
                          (int64_t)(uintptr_t)k_pool, (int64_t)(uintptr_t)v_pool});
  const int threads = threads_for(row_bytes / w);
  dim3 grid(num_tokens, 2);
  hipStream_t s = as_stream(stream);
  const char* ksrc = (const char*)k_src;
  const char* vsrc = (const char*)v_src;
  char* kp = (char*)k_pool;
  char* vp = (char*)v_pool;
  switch (w) {
    case 16: append_rows_kernel<u32x4><<<grid, threads, 0, s>>>(ksrc, vsrc, ks, vs, slot_mapping, kp, vp, pool_slots, (int)row_bytes); break;
    case 8: append_rows_kernel<u32x2><<<grid, threads, 0, s>>>(ksrc, vsrc, ks, vs, slot_mapping, kp, vp, pool_slots, (int)row_bytes); break;
    case 4: append_rows_kernel<uint32_t><<<grid, threads, 0, s>>>(ksrc, vsrc, ks, vs, slot_mapping, kp, vp, pool_slots, (int)row_bytes); break;
    default: append_rows_kernel<uint16_t><<<grid, threads, 0, s>>>(ksrc, vsrc, ks, vs, slot_mapping, kp, vp, pool_slots, (int)row_bytes); break;
  }
  return check_launch("append_kv");
}

static int page_geometry(int32_t num_layers, int64_t num_pages, int32_t page_size,
                         int32_t num_kv_heads, int32_t head_dim, int32_t dtype,
                         int64_t* page_bytes, const char* what) {
  const int eb = elem_bytes(dtype);
  if (!eb) return fail(NSLG_EINVAL, "%s: bad dtype %d", what, dtype);
  if (num_layers <= 0 || num_layers > 65535 || num_pages <= 0 || page_size <= 0 ||
      num_kv_heads <= 0 || head_dim <= 0)
    return fail(NSLG_EINVAL, "%s: bad geometry L=%d P=%lld ps=%d Hkv=%d D=%d", what, num_layers,
                (long long)num_pages, page_size, num_kv_heads, head_dim);
  *page_bytes = (int64_t)page_size * num_kv_heads * head_dim * eb;
  return NSLG_OK;
}

extern "C" int nslg_zero_pages(void* k_pool, void* v_pool, int32_t num_layers, int64_t num_pages,
                               int32_t page_size, int32_t num_kv_heads, int32_t head_dim,
                               int32_t dtype, const int32_t* page_ids, int32_t n,
                               nslg_stream_t stream) {
  int64_t pb = 0;
  int rc = page_geometry(num_layers, num_pages, page_size, num_kv_heads, head_dim, dtype, &pb,
                         "zero_pages");
  if (rc) return rc;
  if (n < 0) return fail(NSLG_EINVAL, "zero_pages: n=%d", n);
  if (n == 0) return NSLG_OK;
  if (!k_pool || !v_pool || !page_ids) return fail(NSLG_EINVAL, "zero_pages: null pointer");
  const int w = pick_vec({pb, (int64_t)(uintptr_t)k_pool, (int64_t)(uintptr_t)v_pool});
  const int64_t blocks = ((pb / w) * n + 255) / 256;
  if (blocks > 0x7fffffff) return fail(NSLG_EINVAL, "zero_pages: too many pages in one call");
  dim3 grid((unsigned)blocks, num_layers, 2);
  hipStream_t s = as_stream(stream);
  char* kp = (char*)k_pool;
  char* vp = (char*)v_pool;
  switch (w) {
    case 16: zero_pages_kernel<u32x4><<<grid, 256, 0, s>>>(kp, vp, num_pages, pb, page_ids, n); break;
    case 8: zero_pages_kernel<u32x2><<<grid, 256, 0, s>>>(kp, vp, num_pages, pb, page_ids, n); break;
    case 4: zero_pages_kernel<uint32_t><<<grid, 256, 0, s>>>(kp, vp, num_pages, pb, page_ids, n); break;
    default: zero_pages_kernel<uint16_t><<<grid, 256, 0, s>>>(kp, vp, num_pages, pb, page_ids, n); break;
  }
  return check_launch("zero_pages");
}

extern "C" int nslg_copy_pages(void* k_pool, void* v_pool, int32_t num_layers, int64_t num_pages,
                               int32_t page_size, int32_t num_kv_heads, int32_t head_dim,
                               int32_t dtype, const int32_t* src_ids, const int32_t* dst_ids,
                               int32_t n, nslg_stream_t stream) {
  int64_t pb = 0;
  int rc = page_geometry(num_layers, num_pages, page_size, num_kv_heads, head_dim, dtype, &pb,
                         "copy_pages");
  if (rc) return rc;
  if (n < 0) return fail(NSLG_EINVAL, "copy_pages: n=%d", n);
  if (n == 0) return NSLG_OK;
  if (!k_pool || !v_pool || !src_ids || !dst_ids) return fail(NSLG_EINVAL, "copy_pages: null pointer");
  const int w = pick_vec({pb, (int64_t)(uintptr_t)k_pool, (int64_t)(uintptr_t)v_pool});
  const int64_t blocks = ((pb / w) * n + 255) / 256;
  if (blocks > 0x7fffffff) return fail(NSLG_EINVAL, "copy_pages: too many pages in one call");
  dim3 grid((unsigned)blocks, num_layers, 2);
  hipStream_t s = as_stream(stream);
  char* kp = (char*)k_pool;
  char* vp = (char*)v_pool;
  switch (w) {
    case 16: copy_pages_kernel<u32x4><<<grid, 256, 0, s>>>(kp, vp, num_pages, pb, src_ids, dst_ids, n); break;
    case 8: copy_pages_kernel<u32x2><<<grid, 256, 0, s>>>(kp, vp, num_pages, pb, src_ids, dst_ids, n); break;
    case 4: copy_pages_kernel<uint32_t><<<grid, 256, 0, s>>>(kp, vp, num_pages, pb, src_ids, dst_ids, n); break;
    default: copy_pages_kernel<uint16_t><<<grid, 256, 0, s>>>(kp, vp, num_pages, pb, src_ids, dst_ids, n); break;
  }
  return check_launch("copy_pages");
}

extern "C" int nslg_gather_kv(const void* k_pool, const void* v_pool, int64_t num_pages,
                              int32_t page_size, const int32_t* kv_indptr,
                              const int32_t* kv_indices, const int32_t* kv_last_page_len,
                              int32_t batch, int32_t max_len, int32_t num_kv_heads,
                              int32_t head_dim, int32_t dtype, void* k_out, void* v_out,
                              nslg_stream_t stream) {
  const int eb = elem_bytes(dtype);
  if (!eb) return fail(NSLG_EINVAL, "gather_kv: bad dtype %d", dtype);
  if (num_pages <= 0 || page_size <= 0 || batch < 0 || batch > 65535 || max_len < 0 ||
      num_kv_heads <= 0 || head_dim <= 0)
    return fail(NSLG_EINVAL, "gather_kv: bad sizes");
  if (batch == 0 || max_len == 0) return NSLG_OK;
  if (!k_pool || !v_pool || !kv_indptr || !kv_indices || !kv_last_page_len || !k_out || !v_out)
    return fail(NSLG_EINVAL, "gather_kv: null pointer");
  const int64_t row_bytes = (int64_t)num_kv_heads * head_dim * eb;
  if (row_bytes > (1 << 30)) return fail(NSLG_EINVAL, "gather_kv: row too large");
  const int w = pick_vec({row_bytes, (int64_t)(uintptr_t)k_pool, (int64_t)(uintptr_t)v_pool,
                          (int64_t)(uintptr_t)k_out, (int64_t)(uintptr_t)v_out});
  const int threads = threads_for(row_bytes / w);
  dim3 grid(max_len, batch, 2);
  hipStream_t s = as_stream(stream);
  const char* kp = (const char*)k_pool;
  const char* vp = (const char*)v_pool;
  char* ko = (char*)k_out;
  char* vo = (char*)v_out;
  switch (w) {
    case 16: gather_rows_kernel<u32x4><<<grid, threads, 0, s>>>(kp, vp, num_pages, page_size, kv_indptr, kv_indices, kv_last_page_len, max_len, (int)row_bytes, ko, vo); break;
    case 8: gather_rows_kernel<u32x2><<<grid, threads, 0, s>>>(kp, vp, num_pages, page_size, kv_indptr, kv_indices, kv_last_page_len, max_len, (int)row_bytes, ko, vo); break;
    case 4: gather_rows_kernel<uint32_t><<<grid, threads, 0, s>>>(kp, vp, num_pages, page_size, kv_indptr, kv_indices, kv_last_page_len, max_len, (int)row_bytes, ko, vo); break;
    default: gather_rows_kernel<uint16_t><<<grid, threads, 0, s>>>(kp, vp, num_pages, page_size, kv_indptr, kv_indices, kv_last_page_len, max_len, (int)row_bytes, ko, vo); break;
  }
  return check_launch("gather_kv");
}
