// Device-side write plan of a multi-token forward (prefill chunks, ragged
// batches): each new token's slot in the pool and position, and the ragged row
// layout, from the forward's CSR block table and per-sequence counts.
//
// The host builds the small per-sequence tables (the CSR after copy-on-write,
// each sequence's start position, new token count, input offset and allocated
// page count) and uploads them; this kernel expands them to per-token arrays
// (slot_mapping and positions over the [B, iw] input grid, the grid row of each
// ragged row, qo_indptr), which for a 8 x 512 chunk are 4096-entry arrays the host
// would otherwise compute and upload every forward. One workgroup per sequence:
// its first wave sums the new token counts of the sequences before it (the
// sequence's first ragged row), then the workgroup fills the sequence's grid
// rows. The rule is the cache's: token t of sequence b is at position
// start_b + t, in page (start_b + t) / page_size of its table and slot
// (start_b + t) % page_size; a page past the allocated ones is the null page,
// slot 0 (kv_cache.py:575-594, 583-584); grid rows without a token get slot -1
// and position 0 (kv_cache.py:267-278).
#include "block_table.h"

namespace nslg {
namespace {

struct ForwardPlanArgs {
  const int32_t* indptr;  // [B+1] CSR of this forward
  const int32_t* indices;
  const int32_t* start;   // [B] tokens cached before the forward
  const int32_t* ntok;    // [B] new tokens
  const int32_t* offs;    // [B] input offsets (first grid column of the new tokens)
  const int32_t* have;    // [B] pages allocated to the sequence
  int32_t* slot_out;      // [B * iw]
  int32_t* pos_out;       // [B * iw]
  int32_t* rows_out;      // [T] grid row of ragged row
  int32_t* qo_out;        // [B + 1]
  int32_t batch;
  int32_t iw;
  int32_t page_size;
};

// Sequence b's rows of the plan, by the workgroup's threads; page(pi) is entry pi of
// the sequence's table (pi < its allocated pages and its CSR segment).
template <typename PageOf>
__device__ inline void plan_segment(const ForwardPlanArgs& a, int b, PageOf page) {
  const int tid = threadIdx.x;
  __shared__ int qo_sh;
  if (tid < 64) {
    int before = 0;
    for (int s = tid; s < b; s += 64) before += max(a.ntok[s], 0);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) before += __shfl_xor(before, off, 64);
    if (tid == 0) qo_sh = before;
  }
  __syncthreads();
  const int qo = qo_sh;
  const int n = max(a.ntok[b], 0);
  const int st = a.start[b];
  const int off = a.offs[b];
  const int have = a.have[b];
  const int np_seg = a.indptr[b + 1] - a.indptr[b];
  const int ps = a.page_size;
  if (tid == 0) {
    a.qo_out[b + 1] = qo + n;
    if (b == 0) a.qo_out[0] = 0;
  }
  const int64_t row0 = (int64_t)b * a.iw;
  for (int r = tid; r < a.iw; r += blockDim.x) {
    const int t = r - off;
    int slot = -1, pos = 0;
    if (t >= 0 && t < n) {
      const int ap = st + t;
      const int pi = ap / ps;
      pos = ap;
      slot = pi < have && pi < np_seg ? page(pi) * ps + (ap - pi * ps) : 0;
      a.rows_out[qo + t] = (int32_t)(row0 + r);
    }
    a.slot_out[row0 + r] = slot;
    a.pos_out[row0 + r] = pos;
  }
}

__global__ void __launch_bounds__(256) forward_plan_kernel(ForwardPlanArgs a) {
  const int b = blockIdx.x;
  const int seg = a.indptr[b];
  plan_segment(a, b, [&](int pi) { return a.indices[seg + pi]; });
}

// Both launches of a device-planned forward in one: workgroup b builds sequence b's
// CSR segment from the arena and the upload, and its plan rows, which take each
// page id from the same sources (not from the CSR being written, so no workgroup
// waits for another).
__global__ void __launch_bounds__(256) forward_plan_csr_kernel(TableCsrArgs t, ForwardPlanArgs a) {
  const int b = blockIdx.x;
  csr_segment(t, b);
  plan_segment(a, b, [&](int pi) { return table_entry(t, b, pi); });
}

}  // namespace
}  // namespace nslg

using namespace nslg;

extern "C" int nslg_forward_plan(const int32_t* kv_indptr, const int32_t* kv_indices, const int32_t* start,
                                 const int32_t* new_tokens, const int32_t* input_offsets,
                                 const int32_t* pages_allocated, int32_t batch, int32_t input_width,
                                 int32_t page_size, int32_t* slot_mapping_out, int32_t* positions_out,
                                 int32_t* ragged_rows_out, int32_t* qo_indptr_out, nslg_stream_t stream) {
  if (batch < 0 || input_width < 0 || page_size <= 0) return fail(NSLG_EINVAL, "forward_plan: bad sizes");
  if (batch == 0) return NSLG_OK;
  if ((int64_t)batch * input_width > 0x7fffffff) return fail(NSLG_EINVAL, "forward_plan: grid too large");
  if (!kv_indptr || !kv_indices || !start || !new_tokens || !input_offsets || !pages_allocated ||
      !slot_mapping_out || !positions_out || !ragged_rows_out || !qo_indptr_out)
    return fail(NSLG_EINVAL, "forward_plan: null pointer");
  ForwardPlanArgs a;
  a.indptr = kv_indptr;
  a.indices = kv_indices;
  a.start = start;
  a.ntok = new_tokens;
  a.offs = input_offsets;
  a.have = pages_allocated;
  a.slot_out = slot_mapping_out;
  a.pos_out = positions_out;
  a.rows_out = ragged_rows_out;
  a.qo_out = qo_indptr_out;
  a.batch = batch;
  a.iw = input_width;
  a.page_size = page_size;
  forward_plan_kernel<<<batch, 256, 0, as_stream(stream)>>>(a);
  return check_launch("forward_plan");
}

extern "C" int nslg_forward_plan_csr(int32_t* tables, int64_t table_capacity, const int32_t* row_offset,
                                     const int32_t* pages_have, const int32_t* synced,
                                     const int32_t* patch_indptr, const int32_t* patch, int64_t patch_total,
                                     const int32_t* kv_indptr, int32_t* kv_indices, int64_t total_pages,
                                     const int32_t* start, const int32_t* new_tokens,
                                     const int32_t* input_offsets, int32_t batch, int32_t input_width,
                                     int32_t page_size, int32_t* slot_mapping_out, int32_t* positions_out,
                                     int32_t* ragged_rows_out, int32_t* qo_indptr_out, nslg_stream_t stream) {
  if (batch < 0 || input_width < 0 || page_size <= 0 || table_capacity < 0 || patch_total < 0 || total_pages < 0)
    return fail(NSLG_EINVAL, "forward_plan_csr: bad sizes");
  if (batch == 0) return NSLG_OK;
  if ((int64_t)batch * input_width > 0x7fffffff) return fail(NSLG_EINVAL, "forward_plan_csr: grid too large");
  if (!tables || !row_offset || !pages_have || !synced || !patch_indptr || !kv_indptr || !kv_indices ||
      (patch_total > 0 && !patch) || !start || !new_tokens || !input_offsets || !slot_mapping_out ||
      !positions_out || !ragged_rows_out || !qo_indptr_out)
    return fail(NSLG_EINVAL, "forward_plan_csr: null pointer");
  TableCsrArgs t;
  t.tables = tables;
  t.table_capacity = table_capacity;
  t.row_offset = row_offset;
  t.pages_have = pages_have;
  t.synced = synced;
  t.patch_indptr = patch_indptr;
  t.patch = patch;
  t.patch_total = patch_total;
  t.kv_indptr = kv_indptr;
  t.kv_indices = kv_indices;
  t.total_pages = total_pages;
  t.batch = batch;
  ForwardPlanArgs a;
  a.indptr = kv_indptr;
  a.indices = kv_indices;
  a.start = start;
  a.ntok = new_tokens;
  a.offs = input_offsets;
  a.have = pages_have;
  a.slot_out = slot_mapping_out;
  a.pos_out = positions_out;
  a.rows_out = ragged_rows_out;
  a.qo_out = qo_indptr_out;
  a.batch = batch;
  a.iw = input_width;
  a.page_size = page_size;
  forward_plan_csr_kernel<<<batch, 256, 0, as_stream(stream)>>>(t, a);
  return check_launch("forward_plan_csr");
}
