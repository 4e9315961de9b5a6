// Device-side plan of one decode step: the CSR block table, slot mapping and
// positions of step i+1 from those of step i, for a batch in which every sequence
// gains exactly one token.
//
// The host only says which sequences opened a page this step and which page it
// got (a few entries per step at batch 64, passed in the kernel arguments), so a
// steady decode step moves no plan bytes over PCIe and the compute stream never
// waits on a copy. Workgroup b rebuilds sequence b's segment: its offset is the
// prefix sum of the new page counts (recomputed per workgroup from kv_indptr,
// which is a few hundred bytes), its page ids are copied and the new page, if
// any, is appended; lane 0 writes the sequence's last-page length, the slot of the
// new token and its position, and the id of the new page into the list of pages
// to zero. When the pool is given, further workgroups zero the opened pages in
// every layer (the zero-on-alloc), 16 KiB each, so the step needs no separate
// zeroing launch.
#include "nslg_common.h"

namespace nslg {
namespace {

constexpr int kMaxPlanBatch = 512;
// Batches up to this size launch with a 64-entry list in the arguments (256 bytes
// instead of 2 KiB: measured 2.4 vs 3.2 us of host time per launch).
constexpr int kSmallPlanBatch = 64;
constexpr int kZeroBytes = 16 << 10;  // bytes zeroed per workgroup

template <int N>
struct PlanStepArgs {
  const int32_t* indptr_in;
  const int32_t* indices_in;
  const int32_t* last_len_in;
  int32_t* indptr_out;
  int32_t* indices_out;
  int32_t* last_len_out;
  int32_t* slot_out;
  int32_t* pos_out;
  int32_t* new_pages_out;
  int32_t batch;
  int32_t page_size;
  // zero-on-alloc of the opened pages (k_pool == nullptr: none)
  char* k_pool;
  char* v_pool;
  int64_t num_pages;
  int64_t page_bytes;  // bytes of one page in one layer (a multiple of 16)
  int32_t num_layers;
  int32_t zero_parts;  // ceil(page_bytes / kZeroBytes)
  const int32_t* new_page_dev;  // nullptr: the list below; else the same list in device memory
  int32_t new_page[N];  // page opened by sequence b this step, or -1
};

template <int N>
__device__ inline int opened_page(const PlanStepArgs<N>& a, int b) {
  return a.new_page_dev ? a.new_page_dev[b] : a.new_page[b];
}

// Workgroup z of the zeroing part: (page, layer, K or V, 16 KiB part), where the
// page is the j-th opened one of the list in the kernel arguments, or, with the
// list in memory, the one sequence j opened (if any: one read of the list each).
template <int N>
__device__ void zero_part(const PlanStepArgs<N>& a, int z) {
  const int part = z % a.zero_parts;
  z /= a.zero_parts;
  const int kv = z & 1;
  z >>= 1;
  const int layer = z % a.num_layers;
  const int j = z / a.num_layers;
  int page = -1;
  if (a.new_page_dev) {
    page = j < a.batch ? a.new_page_dev[j] : -1;
  } else {
    int seen = 0;
    for (int b = 0; b < a.batch; ++b) {  // the j-th opened page
      if (a.new_page[b] >= 0) {
        if (seen == j) {
          page = a.new_page[b];
          break;
        }
        ++seen;
      }
    }
  }
  if (page < 0 || (int64_t)page >= a.num_pages) return;
  char* base = (kv ? a.v_pool : a.k_pool) + ((int64_t)layer * a.num_pages + page) * a.page_bytes;
  const int64_t off0 = (int64_t)part * kZeroBytes;
  const int64_t end = min(off0 + (int64_t)kZeroBytes, a.page_bytes);
  const u32x4 zero = {0u, 0u, 0u, 0u};
  for (int64_t off = off0 + 16 * (int64_t)threadIdx.x; off < end; off += 16 * (int64_t)blockDim.x)
    stream_store(reinterpret_cast<u32x4*>(base + off), zero);
}

// Pages of sequence s before the step, and whether this step opens one.
template <int N>
__device__ inline void seq_step(const PlanStepArgs<N>& a, int s, int& np_in, int& lpl_in, bool& opens) {
  // all three loads issued at once (the length is read whether or not it is used)
  const int ip0 = a.indptr_in[s], ip1 = a.indptr_in[s + 1], lpl = a.last_len_in[s];
  np_in = ip1 - ip0;
  lpl_in = np_in > 0 ? lpl : a.page_size;
  lpl_in = lpl_in < 1 ? 1 : (lpl_in > a.page_size ? a.page_size : lpl_in);
  opens = lpl_in == a.page_size;
}

template <int N>
__global__ void __launch_bounds__(256) decode_plan_step_kernel(PlanStepArgs<N> a) {
  if ((int)blockIdx.x >= a.batch) {
    zero_part(a, blockIdx.x - a.batch);
    return;
  }
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // offset of sequence b's segment in the new table, and the number of new pages
  // opened by sequences before b (its index in the zero list); the first wave
  // computes both, the other waves only copy
  __shared__ int seg_out_sh, new_before_sh;
  // this sequence's own numbers first: their loads overlap the prefix's below
  int np_in, lpl_in;
  bool opens;
  seq_step(a, b, np_in, lpl_in, opens);
  const int seg_in = a.indptr_in[b];
  if (tid < 64) {
    int pages = 0, opened = 0;
    for (int s = lane; s < b; s += 64) {
      int np_s, lpl_s;
      bool opens_s;
      seq_step(a, s, np_s, lpl_s, opens_s);
      pages += np_s + (opens_s ? 1 : 0);
      opened += opens_s ? 1 : 0;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      pages += __shfl_xor(pages, off, 64);
      opened += __shfl_xor(opened, off, 64);
    }
    if (tid == 0) {
      seg_out_sh = pages;
      new_before_sh = opened;
    }
  }
  __syncthreads();
  const int seg_out = seg_out_sh;
  for (int i = tid; i < np_in; i += blockDim.x) a.indices_out[seg_out + i] = a.indices_in[seg_in + i];
  if (tid == 0) {
    int page;  // the page the new token goes to
    int lpl;
    if (opens) {
      page = opened_page(a, b);
      if (page < 0) page = 0;  // no page given: the null page (the sink of writes past a table)
      a.indices_out[seg_out + np_in] = page;
      a.new_pages_out[new_before_sh] = page;
      lpl = 1;
    } else {
      page = a.indices_in[seg_in + np_in - 1];
      lpl = lpl_in + 1;
    }
    const int np_out = np_in + (opens ? 1 : 0);
    a.last_len_out[b] = lpl;
    a.indptr_out[b + 1] = seg_out + np_out;
    if (b == 0) a.indptr_out[0] = 0;
    a.slot_out[b] = page * a.page_size + (lpl - 1);
    a.pos_out[b] = (np_out - 1) * a.page_size + (lpl - 1);
  }
}

}  // namespace
}  // namespace nslg

using namespace nslg;

namespace {

// Shared set-up of both entry points; new_page_host xor new_page_dev is given. With
// the list in memory the number of opened pages is not known here: the zeroing grid
// has a slot per sequence and the slots of sequences that open no page exit.
int plan_step_impl(const int32_t* kv_indptr, const int32_t* kv_indices, const int32_t* kv_last_page_len,
                   int32_t batch, int32_t page_size, const int32_t* new_page_host, const int32_t* new_page_dev,
                   int32_t* kv_indptr_out, int32_t* kv_indices_out,
                   int32_t* kv_last_page_len_out, int32_t* slot_mapping_out, int32_t* positions_out,
                   int32_t* new_pages_out, void* k_pool, void* v_pool, int32_t num_layers, int64_t num_pages,
                   int32_t num_kv_heads, int32_t head_dim, int32_t dtype, nslg_stream_t stream) {
  if (batch < 0 || page_size <= 0) return fail(NSLG_EINVAL, "decode_plan_step: bad sizes");
  if (batch == 0) return NSLG_OK;
  if (batch > kMaxPlanBatch)
    return fail(NSLG_EUNSUPPORTED, "decode_plan_step: batch %d > %d", batch, kMaxPlanBatch);
  if (!kv_indptr || !kv_indices || !kv_last_page_len || !(new_page_host || new_page_dev) || !kv_indptr_out ||
      !kv_indices_out || !kv_last_page_len_out || !slot_mapping_out || !positions_out || !new_pages_out)
    return fail(NSLG_EINVAL, "decode_plan_step: null pointer");
  if (kv_indices_out == kv_indices || kv_indptr_out == kv_indptr || kv_last_page_len_out == kv_last_page_len)
    return fail(NSLG_EINVAL, "decode_plan_step: output tables must not alias the input ones");
  // the same arguments at either list size
  auto run = [&](auto& a) -> int {
    a.indptr_in = kv_indptr;
    a.indices_in = kv_indices;
    a.last_len_in = kv_last_page_len;
    a.indptr_out = kv_indptr_out;
    a.indices_out = kv_indices_out;
    a.last_len_out = kv_last_page_len_out;
    a.slot_out = slot_mapping_out;
    a.pos_out = positions_out;
    a.new_pages_out = new_pages_out;
    a.batch = batch;
    a.page_size = page_size;
    a.new_page_dev = new_page_dev;
    int opened = 0;
    if (new_page_host) {
      for (int b = 0; b < batch; ++b) {
        a.new_page[b] = new_page_host[b];
        opened += new_page_host[b] >= 0 ? 1 : 0;
      }
    } else {
      opened = batch;  // one zeroing slot per sequence: sequence j's page, if it opens one
    }
    a.k_pool = (char*)k_pool;
    a.v_pool = (char*)v_pool;
    a.num_layers = 0;
    a.num_pages = 0;
    a.page_bytes = 0;
    a.zero_parts = 1;
    int64_t zero_groups = 0;
    if (k_pool || v_pool) {
      if (!k_pool || !v_pool || num_layers <= 0 || num_pages <= 0 || num_kv_heads <= 0 || head_dim <= 0)
        return fail(NSLG_EINVAL, "decode_plan_step: bad pool for zeroing");
      const int eb = elem_bytes(dtype);
      if (!eb) return fail(NSLG_EINVAL, "decode_plan_step: dtype %d", dtype);
      const int64_t pb = (int64_t)page_size * num_kv_heads * head_dim * eb;
      if (pb % 16 || ((uintptr_t)k_pool | (uintptr_t)v_pool) & 15)
        return fail(NSLG_EINVAL, "decode_plan_step: pool pages must be 16-byte aligned");
      a.num_layers = num_layers;
      a.num_pages = num_pages;
      a.page_bytes = pb;
      a.zero_parts = (int32_t)((pb + kZeroBytes - 1) / kZeroBytes);
      zero_groups = (int64_t)opened * num_layers * 2 * a.zero_parts;
      if (batch + zero_groups > 0x7fffffff) return fail(NSLG_EINVAL, "decode_plan_step: too much to zero");
    }
    decode_plan_step_kernel<<<(unsigned)(batch + zero_groups), 256, 0, as_stream(stream)>>>(a);
    return check_launch("decode_plan_step");
  };
  if (batch <= kSmallPlanBatch) {
    PlanStepArgs<kSmallPlanBatch> a;
    return run(a);
  }
  PlanStepArgs<kMaxPlanBatch> a;
  return run(a);
}

}  // namespace

extern "C" int nslg_decode_plan_step(const int32_t* kv_indptr, const int32_t* kv_indices,
                                     const int32_t* kv_last_page_len, int32_t batch, int32_t page_size,
                                     const int32_t* new_page, int32_t* kv_indptr_out, int32_t* kv_indices_out,
                                     int32_t* kv_last_page_len_out, int32_t* slot_mapping_out,
                                     int32_t* positions_out, int32_t* new_pages_out, void* k_pool,
                                     void* v_pool, int32_t num_layers, int64_t num_pages,
                                     int32_t num_kv_heads, int32_t head_dim, int32_t dtype,
                                     nslg_stream_t stream) {
  return plan_step_impl(kv_indptr, kv_indices, kv_last_page_len, batch, page_size, new_page, nullptr,
                        kv_indptr_out, kv_indices_out, kv_last_page_len_out, slot_mapping_out, positions_out,
                        new_pages_out, k_pool, v_pool, num_layers, num_pages, num_kv_heads, head_dim, dtype,
                        stream);
}

extern "C" int nslg_decode_plan_step_device(const int32_t* kv_indptr, const int32_t* kv_indices,
                                            const int32_t* kv_last_page_len, int32_t batch, int32_t page_size,
                                            const int32_t* new_page, int32_t* kv_indptr_out,
                                            int32_t* kv_indices_out, int32_t* kv_last_page_len_out,
                                            int32_t* slot_mapping_out, int32_t* positions_out,
                                            int32_t* new_pages_out, void* k_pool, void* v_pool,
                                            int32_t num_layers, int64_t num_pages, int32_t num_kv_heads,
                                            int32_t head_dim, int32_t dtype, nslg_stream_t stream) {
  if (!new_page) return fail(NSLG_EINVAL, "decode_plan_step_device: null pointer");
  // pinned host memory is read through its device mapping
  hipPointerAttribute_t attr;
  if (hipPointerGetAttributes(&attr, new_page) == hipSuccess && attr.type == hipMemoryTypeHost) {
    void* dptr = nullptr;
    if (hipHostGetDevicePointer(&dptr, const_cast<int32_t*>(new_page), 0) != hipSuccess || !dptr) {
      (void)hipGetLastError();
      return fail(NSLG_EINVAL, "decode_plan_step_device: host list is not pinned, mapped memory");
    }
    new_page = static_cast<const int32_t*>(dptr);
  }
  (void)hipGetLastError();
  return plan_step_impl(kv_indptr, kv_indices, kv_last_page_len, batch, page_size, nullptr, new_page,
                        kv_indptr_out, kv_indices_out, kv_last_page_len_out, slot_mapping_out, positions_out,
                        new_pages_out, k_pool, v_pool, num_layers, num_pages, num_kv_heads, head_dim, dtype,
                        stream);
}
