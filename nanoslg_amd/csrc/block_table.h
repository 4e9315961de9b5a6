// The CSR segment of one sequence built from the cache's device-resident block
// tables (shared by nslg_block_table_csr and nslg_forward_plan_csr).
#pragma once
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

// Entry i (< pages_have_b) of sequence b's table: from the upload at and above the
// synced mark, from the arena below it; 0 where an index falls outside either.
__device__ inline int table_entry(const TableCsrArgs& a, int b, int i) {
  const int64_t row = a.row_offset[b];
  const int syn = a.synced[b];
  if (i >= syn) {
    const int64_t pk = (int64_t)a.patch_indptr[b] + (i - syn);
    return pk >= 0 && pk < a.patch_total ? a.patch[pk] : 0;
  }
  const int64_t at = row + i;
  return row >= 0 && at < a.table_capacity ? a.tables[at] : 0;
}

// Sequence b's CSR segment (entry i < npg_b: table entry i, or the null page 0 past
// the entries the sequence has), by the workgroup's threads; the uploaded entries are
// also written into the sequence's arena row.
__device__ inline void csr_segment(const TableCsrArgs& a, int b) {
  const int64_t row = a.row_offset[b];
  const int have = a.pages_have[b];
  const int syn = a.synced[b];
  const int64_t seg = a.kv_indptr[b];
  const int npg = a.kv_indptr[b + 1] - a.kv_indptr[b];
  for (int i = threadIdx.x; i < npg || i < have; i += blockDim.x) {
    int pid = 0;
    if (i < have) {
      pid = table_entry(a, b, i);
      const int64_t at = row + i;
      if (i >= syn && row >= 0 && at < a.table_capacity) a.tables[at] = pid;
    }
    if (i < npg && seg + i < a.total_pages) a.kv_indices[seg + i] = pid;
  }
}

}  // namespace
}  // namespace nslg
