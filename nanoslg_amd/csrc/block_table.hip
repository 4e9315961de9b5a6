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
#include "block_table.h"

namespace nslg {
namespace {

__global__ void __launch_bounds__(256) block_table_csr_kernel(TableCsrArgs a) { csr_segment(a, blockIdx.x); }

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
