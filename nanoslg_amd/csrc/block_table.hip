// CSR block table of a forward from the cache's device-resident block tables.
//
// The cache keeps every live sequence's block table in a persistent int32 arena
// on the device, one row per sequence (the page ids of its logical pages 0, 1,
// ...). The host mirrors the tables and knows, per row, how many leading entries
// the device already holds; a forward uploads only the rest (the pages allocated
// since the row was last used, copy-on-write replacements) and this kernel
// builds the forward's CSR from the rows, so planning a forward moves O(batch +
// changed pages) over PCIe instead of every page of every sequence.
//
// Workgroup b serves sequence b: entry i < npg_b of its CSR segment is row entry
// i (from the arena below the synced mark, from the upload above it) or the null
// page 0 past the entries the sequence has (the sink of writes past a block
// table, kv_cache.py:583-584, 606-607); the uploaded entries are also written
// into the row for later forwards. Reads and writes stay inside the arena, the
// upload and the CSR (every index is checked against the sizes passed in).
#include "nslg_common.h"

namespace nslg {
namespace {

struct TableCsrArgs {
  int32_t* tables;            // arena
  int64_t table_capacity;     // entries of the arena
  const int32_t* row_offset;  // [B] first arena entry of sequence b's row
  const int32_t* pages_have;  // [B] valid entries of the row
  const int32_t* synced;      // [B] entries [0, synced) are current in the arena
  const int32_t* patch_indptr;  // [B+1] uploaded entries [synced_b, pages_have_b) of row b
  const int32_t* patch;
  int64_t patch_total;
  const int32_t* kv_indptr;   // [B+1] CSR pointers of the forward
  int32_t* kv_indices;        // [kv_indptr[B]] out
  int64_t total_pages;
  int32_t batch;
};

__global__ void __launch_bounds__(256) block_table_csr_kernel(TableCsrArgs a) {
  const int b = blockIdx.x;
  const int64_t row = a.row_offset[b];
  const int have = a.pages_have[b];
  const int syn = a.synced[b];
  const int64_t p0 = a.patch_indptr[b];
  const int64_t seg = a.kv_indptr[b];
  const int npg = a.kv_indptr[b + 1] - a.kv_indptr[b];
  for (int i = threadIdx.x; i < npg || i < have; i += blockDim.x) {
    int pid = 0;
    if (i < have) {
      const int64_t at = row + i;
      const bool in_table = row >= 0 && at < a.table_capacity;
      if (i >= syn) {
        const int64_t pk = p0 + (i - syn);
        pid = pk >= 0 && pk < a.patch_total ? a.patch[pk] : 0;
        if (in_table) a.tables[at] = pid;
      } else if (in_table) {
        pid = a.tables[at];
      }
    }
    if (i < npg && seg + i < a.total_pages) a.kv_indices[seg + i] = pid;
  }
}

}  // namespace
}  // namespace nslg

using namespace nslg;

extern "C" int nslg_block_table_csr(int32_t* tables, int64_t table_capacity, const int32_t* row_offset,
                                    const int32_t* pages_have, const int32_t* synced,
                                    const int32_t* patch_indptr, const int32_t* patch, int64_t patch_total,
                                    const int32_t* kv_indptr, int32_t* kv_indices, int64_t total_pages,
                                    int32_t batch, nslg_stream_t stream) {
  if (batch < 0 || table_capacity < 0 || patch_total < 0 || total_pages < 0)
    return fail(NSLG_EINVAL, "block_table_csr: bad sizes");
  if (batch == 0) return NSLG_OK;
  if (!tables || !row_offset || !pages_have || !synced || !patch_indptr || !kv_indptr || !kv_indices ||
      (patch_total > 0 && !patch))
    return fail(NSLG_EINVAL, "block_table_csr: null pointer");
  TableCsrArgs a;
  a.tables = tables;
  a.table_capacity = table_capacity;
  a.row_offset = row_offset;
  a.pages_have = pages_have;
  a.synced = synced;
  a.patch_indptr = patch_indptr;
  a.patch = patch;
  a.patch_total = patch_total;
  a.kv_indptr = kv_indptr;
  a.kv_indices = kv_indices;
  a.total_pages = total_pages;
  a.batch = batch;
  block_table_csr_kernel<<<batch, 256, 0, as_stream(stream)>>>(a);
  return check_launch("block_table_csr");
}
