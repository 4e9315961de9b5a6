/*
 * nslg_kv.h — C ABI of the MI355X (gfx950) KV-cache hot path.
 *
 * Every entry point:
 *   - takes raw device pointers, element counts and an explicit hipStream_t
 *     (pass torch.cuda.current_stream().cuda_stream from Python);
 *   - is asynchronous on that stream and never synchronises the host;
 *   - never allocates device memory: scratch space is caller-owned
 *     ("workspace") and sized by the matching *_workspace_size() call;
 *   - returns 0 on success and a negative NSLG_E* code on a bad argument,
 *     an unsupported shape or a launch failure (nslg_last_error() gives text).
 *
 * KV pool layout (one layer): a flat array of token rows
 *     pool[P * page_size][num_kv_heads][head_dim]
 * i.e. [P, page_size, Hkv, D] with D fastest, token "slot id" = page * page_size + slot.
 * The reference PagePool stores [L, P, ps, Hkv, D] per K and V
 * (nanoslg/kv_cache.py:389-392); the layer-l slice of it is exactly this layout.
 * The contiguous backend's [L, Bmax, Smax, Hkv, D] pool (kv_cache.py:229-232) is the
 * same layout with P = Bmax, page_size = Smax and an identity block table.
 *
 * Block tables are CSR, as the reference builds them for FlashInfer
 * (kv_cache.py:598-615): kv_indptr[B+1], kv_indices[kv_indptr[B]],
 * kv_last_page_len[B] in [1, page_size].
 */
#ifndef NSLG_KV_H
#define NSLG_KV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* nslg_stream_t; /* a hipStream_t; NULL = the null stream */

enum nslg_dtype { NSLG_F16 = 0, NSLG_BF16 = 1, NSLG_F32 = 2 };

enum nslg_status {
  NSLG_OK = 0,
  NSLG_EINVAL = -1,      /* bad pointer / size / stride */
  NSLG_EUNSUPPORTED = -2,/* shape or dtype this build has no kernel for */
  NSLG_ELAUNCH = -3,     /* the HIP launch itself failed */
  NSLG_EWORKSPACE = -4,  /* workspace too small */
  NSLG_ECAPTURE = -5     /* the call's first use of a kernel variant on a device would
                            query the device while its stream is being captured into a
                            graph: make one call (or a workspace-size query) outside
                            the capture first */
};

/* Library version (major*10000 + minor*100 + patch). */
int nslg_version(void);

/* Human-readable text of the last error seen on the calling thread. */
const char* nslg_last_error(void);

/*
 * K/V append (scatter of the new tokens' rows into the pool).
 * Replaces the per-run slice copies of FlashInferCacheContext._write_kv
 * (nanoslg/kv_cache.py:661-674) and the decode index-put of
 * ContiguousCacheContext.attend (kv_cache.py:301-303, 305-310).
 *
 *   k_src, v_src      [num_tokens] rows of Hkv*D elements; row i starts at
 *                     element i*k_src_stride (resp. v_src_stride); D contiguous,
 *                     heads at stride D inside a row.
 *   slot_mapping      int32[num_tokens]: destination slot id (page*page_size+slot);
 *                     a negative entry skips that row (padding), an entry
 *                     >= pool_slots is rejected on the device (row skipped).
 *   k_pool, v_pool    layer base pointers, pool_slots rows of Hkv*D elements.
 * Bit-exact copy.
 */
int nslg_append_kv(const void* k_src, const void* v_src,
                   int64_t k_src_stride, int64_t v_src_stride,
                   const int32_t* slot_mapping, int32_t num_tokens,
                   void* k_pool, void* v_pool, int64_t pool_slots,
                   int32_t num_kv_heads, int32_t head_dim, int32_t dtype,
                   nslg_stream_t stream);

/*
 * Zero whole pages across all layers (the zero-on-alloc of PagePool.alloc,
 * nanoslg/kv_cache.py:411, and of ContiguousKVCache.allocate_sequence, :340),
 * batched into one launch.
 *   k_pool, v_pool    base of the [L, P, page_size, Hkv, D] pools
 *   page_ids          int32[n] device array; ids outside [0, P) are skipped
 */
int nslg_zero_pages(void* k_pool, void* v_pool, int32_t num_layers,
                    int64_t num_pages, int32_t page_size, int32_t num_kv_heads,
                    int32_t head_dim, int32_t dtype,
                    const int32_t* page_ids, int32_t n, nslg_stream_t stream);

/*
 * Copy whole pages across all layers and all page slots: dst <- src for K and V
 * (the copy-on-write of PagePool.cow, nanoslg/kv_cache.py:429-436), batched.
 *   src_ids, dst_ids  int32[n] device arrays; a pair with an id outside [0, P)
 *                     is skipped. dst ids must be distinct from every src id.
 */
int nslg_copy_pages(void* k_pool, void* v_pool, int32_t num_layers,
                    int64_t num_pages, int32_t page_size, int32_t num_kv_heads,
                    int32_t head_dim, int32_t dtype,
                    const int32_t* src_ids, const int32_t* dst_ids, int32_t n,
                    nslg_stream_t stream);

/*
 * Gather paged K/V into a contiguous [B, max_len, Hkv, D] buffer per K and V
 * (the slice read of ContiguousCacheContext.attend, nanoslg/kv_cache.py:312-314,
 * without the transpose). Rows past a sequence's length are written as zeros.
 * Bit-exact.
 */
int nslg_gather_kv(const void* k_pool, const void* v_pool, int64_t num_pages,
                   int32_t page_size, const int32_t* kv_indptr,
                   const int32_t* kv_indices, const int32_t* kv_last_page_len,
                   int32_t batch, int32_t max_len, int32_t num_kv_heads,
                   int32_t head_dim, int32_t dtype, void* k_out, void* v_out,
                   nslg_stream_t stream);

/*
 * Paged GQA decode attention, one query token per sequence.
 * Replaces FlashInfer BatchDecodeWithPagedKVCacheWrapper.plan/run
 * (nanoslg/kv_cache.py:617-621, 650) and, with an identity block table, the
 * contiguous decode SDPA (kv_cache.py:312-321).
 *
 * The sequences' tokens are cut into equal chunks (about 1024 over the batch);
 * one wave per (chunk, KV head) streams its pages through MFMA tiles and a
 * second launch merges the chunks of each sequence in fp32 (log-sum-exp).
 *
 *   q        [batch] rows of Hq*D elements at element stride q_stride
 *   out      [batch] rows of Hq*D elements at element stride out_stride (q's dtype)
 *   k_pool, v_pool, num_pages, page_size: one layer of the pool (see above)
 *   kv_indptr/kv_indices/kv_last_page_len: CSR block table (device)
 *   total_pages       host copy of kv_indptr[batch] (sizes the launch)
 *   sm_scale          softmax scale (1/sqrt(D) for the reference)
 *   workspace         caller-owned device scratch of at least
 *                     nslg_paged_decode_workspace_size(...) bytes, 256-byte aligned;
 *                     one call at a time per workspace
 *   layout            0: the call cuts its sequences into chunks from their lengths
 *                     (every wave reads the lengths and searches the chunk length);
 *                     t > 0: the same, and the chunks' work is recorded in the
 *                     workspace under tag t; -t: a later call of the same forward
 *                     (another layer: same batch, block table, lengths, sizes and
 *                     workspace) reads the record instead, when the workspace still
 *                     holds tag t (else it cuts the chunks itself). Results are
 *                     bit-identical in all three modes; a tag must not be reused for
 *                     another forward (a wrong record gives wrong results, though
 *                     every access stays inside the block table and the pool).
 * Query head h reads KV head h / (Hq/Hkv). Supported: f16, bf16 (MFMA, split-K as
 * above) and f32 (a VALU kernel, one workgroup per 16 query rows of a sequence and
 * KV head and key split, then an fp32 merge, for caches kept in fp32 such as the
 * contiguous backend of an fp32 model, kv_cache.py:227-322); D in {64, 128, 256};
 * 1 <= Hq/Hkv <= 16. A sequence with no tokens gets zeros.
 * The first f16/bf16 call of a (dtype, head_dim, page_size) variant on a device
 * (or the first workspace-size query for it) queries the device's occupancy
 * once; a decode call that would do so while its stream is being captured into
 * a graph returns NSLG_ECAPTURE and launches nothing.
 */
size_t nslg_paged_decode_workspace_size(int32_t batch, int32_t num_qo_heads,
                                        int32_t num_kv_heads, int32_t head_dim,
                                        int64_t total_pages, int32_t page_size,
                                        int32_t dtype);

int nslg_paged_decode(const void* q, int64_t q_stride,
                      const void* k_pool, const void* v_pool, int64_t num_pages,
                      int32_t page_size, const int32_t* kv_indptr,
                      const int32_t* kv_indices, const int32_t* kv_last_page_len,
                      int64_t total_pages, int32_t batch, int32_t num_qo_heads,
                      int32_t num_kv_heads, int32_t head_dim, float sm_scale,
                      int32_t dtype, void* out, int64_t out_stride,
                      void* workspace, size_t workspace_bytes,
                      int64_t layout, nslg_stream_t stream);

/*
 * The decode step of one layer: each sequence's new token written into the pool,
 * then decode attention over its tokens including that one. Replaces the write of
 * FlashInferCacheContext.attend (_write_kv, nanoslg/kv_cache.py:661-674; the slot
 * mapping of :575-594) together with the decode run (:650), which the reference
 * issues back to back for one decode forward (:639-655). Same result as
 * nslg_append_kv of the rows followed by nslg_paged_decode (bit-identical).
 *
 *   k_new, v_new   [batch] rows of Hkv*D elements at element strides k_new_stride,
 *                  v_new_stride (device, the pool's dtype; f16/bf16: 16-byte aligned
 *                  rows, f32: 4-byte)
 *   other arguments as nslg_paged_decode (layout included)
 * Row b is sequence b's token L_b - 1 (the last token its block table covers, the
 * reference's slot for the decode write): the slot is found through the block
 * table, so no slot mapping is passed. The chunk that reads that token writes it
 * first, in the same kernel (f32 pools: one launch ahead of the attention kernel).
 * Precondition, which the reference's copy-on-write rule gives (kv_cache.py:575-594):
 * no other sequence of the call reads a row being written (a written page is not
 * shared). A row whose page id is out of the pool is not written.
 */
int nslg_paged_decode_append(const void* q, int64_t q_stride,
                             const void* k_new, int64_t k_new_stride,
                             const void* v_new, int64_t v_new_stride,
                             void* k_pool, void* v_pool, int64_t num_pages,
                             int32_t page_size, const int32_t* kv_indptr,
                             const int32_t* kv_indices, const int32_t* kv_last_page_len,
                             int64_t total_pages, int32_t batch, int32_t num_qo_heads,
                             int32_t num_kv_heads, int32_t head_dim, float sm_scale,
                             int32_t dtype, void* out, int64_t out_stride,
                             void* workspace, size_t workspace_bytes,
                             int64_t layout, nslg_stream_t stream);

/*
 * nslg_paged_decode without a caller workspace: the split-K partials live in a
 * static device array of NSLG_NOALLOC_SCRATCH_BYTES (16 MiB) that the library
 * holds on every GPU it runs on until the process ends. No counterpart in the
 * reference: this entry point is for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). It allocates nothing and calls no allocating routine.
 *
 * Arguments and results as nslg_paged_decode (same kernels, bit-identical output),
 * without workspace / workspace_bytes. The call's device is the current device
 * (hipSetDevice), which must be the stream's. A call that would need more scratch
 * than the static array (nslg_paged_decode_workspace_size(...) >
 * NSLG_NOALLOC_SCRATCH_BYTES: e.g. batches of several hundred long sequences)
 * returns NSLG_EWORKSPACE without launching. All calls on one GPU share the one
 * array: calls that overlap on a GPU (different streams, or host threads, without
 * ordering between them) race and give wrong results.
 */
#define NSLG_NOALLOC_SCRATCH_BYTES (16u << 20)

int nslg_paged_decode_noalloc(const void* q, int64_t q_stride,
                              const void* k_pool, const void* v_pool, int64_t num_pages,
                              int32_t page_size, const int32_t* kv_indptr,
                              const int32_t* kv_indices, const int32_t* kv_last_page_len,
                              int64_t total_pages, int32_t batch, int32_t num_qo_heads,
                              int32_t num_kv_heads, int32_t head_dim, float sm_scale,
                              int32_t dtype, void* out, int64_t out_stride,
                              nslg_stream_t stream);

/*
 * Paged decode for a batch in which groups of sequences share their first pages
 * (a radix prefix: the same page ids, kv_cache.py:459-472, 707-716). Same result
 * as nslg_paged_decode (within the attention tolerance: the split differs); the
 * shared K/V of a group is read once for all its members instead of once per
 * member: the group's prefix is one more work unit whose MFMA tiles carry the
 * query heads of all members (G = Hq/Hkv columns each, 16 columns in all).
 * Replaces the same FlashInfer decode run (kv_cache.py:617-621, 650).
 *
 *   seq_group_slot      int32[batch] (device): 16 * g + m when sequence b is member
 *                       m of group g, else -1; must agree with group_members
 *   num_groups          1..32
 *   group_prefix_pages  HOST int32[num_groups]: pages shared by the group's members,
 *                       >= 1; every member's first group_prefix_pages[g] page ids
 *                       are the same and its length is at least that many pages
 *   group_members       HOST int32[num_groups * 16]: member sequences of group g at
 *                       [16 g, 16 g + n_g), -1 after them; 1 <= n_g <= 16 / G;
 *                       a sequence is in at most one group
 * The workspace holds 16 / G partial slots per chunk:
 * nslg_paged_decode_grouped_workspace_size(...) bytes. layout as nslg_paged_decode. f16/bf16 only (the size
 * query returns 0 for f32; decode f32 batches with nslg_paged_decode).
 */
size_t nslg_paged_decode_grouped_workspace_size(int32_t batch, int32_t num_qo_heads,
                                                int32_t num_kv_heads, int32_t head_dim,
                                                int64_t total_pages, int32_t page_size,
                                                int32_t dtype, int32_t num_groups);

int nslg_paged_decode_grouped(const void* q, int64_t q_stride,
                              const void* k_pool, const void* v_pool, int64_t num_pages,
                              int32_t page_size, const int32_t* kv_indptr,
                              const int32_t* kv_indices, const int32_t* kv_last_page_len,
                              int64_t total_pages, int32_t batch, int32_t num_qo_heads,
                              int32_t num_kv_heads, int32_t head_dim, float sm_scale,
                              int32_t dtype, const int32_t* seq_group_slot, int32_t num_groups,
                              const int32_t* group_prefix_pages, const int32_t* group_members,
                              void* out, int64_t out_stride,
                              void* workspace, size_t workspace_bytes,
                              int64_t layout, nslg_stream_t stream);

/*
 * nslg_paged_decode_grouped with each sequence's new token written first, as
 * nslg_paged_decode_append does for nslg_paged_decode (the same replacement of
 * kv_cache.py:661-674 + 650). Group prefixes must lie below every member's last
 * page (the page the new row goes to), as a shared page is never written.
 */
int nslg_paged_decode_grouped_append(const void* q, int64_t q_stride,
                                     const void* k_new, int64_t k_new_stride,
                                     const void* v_new, int64_t v_new_stride,
                                     void* k_pool, void* v_pool, int64_t num_pages,
                                     int32_t page_size, const int32_t* kv_indptr,
                                     const int32_t* kv_indices, const int32_t* kv_last_page_len,
                                     int64_t total_pages, int32_t batch, int32_t num_qo_heads,
                                     int32_t num_kv_heads, int32_t head_dim, float sm_scale,
                                     int32_t dtype, const int32_t* seq_group_slot,
                                     int32_t num_groups, const int32_t* group_prefix_pages,
                                     const int32_t* group_members, void* out, int64_t out_stride,
                                     void* workspace, size_t workspace_bytes,
                                     int64_t layout, nslg_stream_t stream);

/*
 * nslg_paged_decode_append with the rotary position embedding of the step folded in:
 * a model's decode layer (the position gather and the two apply_rotary_emb calls of
 * _attention_forward, nanoslg/models.py:96-103 and :69-83, then attend's write and
 * decode run, kv_cache.py:661-674 + 650) in one decode launch and its merge. Each
 * wave rotates its query heads' q at their sequence's position as it loads them, and
 * the chunk that writes sequence b's new row writes k_new rotated; v_new is written
 * as given. The rotation is nslg_rope_append's, element for element:
 *   positions       int32[batch] (device): sequence b's new token's position,
 *                   clamped into the tables
 *   cos_table, sin_table   fp32 [table_rows] rows of >= head_dim floats at
 *                   table_stride, rows 16-byte aligned (the model's tables)
 * The other arguments are nslg_paged_decode_append's. Outputs and pool bytes are
 * bit-identical with nslg_rope_append (q rotated into a buffer, the rotated K and V
 * rows written) followed by nslg_paged_decode on the rotated q. f16/bf16 pools
 * (f32: NSLG_EUNSUPPORTED; use nslg_rope_append, then nslg_paged_decode).
 */
int nslg_paged_decode_rope_append(const void* q, int64_t q_stride, const void* k_new,
                                  int64_t k_new_stride, const void* v_new, int64_t v_new_stride,
                                  const int32_t* positions, const float* cos_table,
                                  const float* sin_table, int64_t table_stride, int64_t table_rows,
                                  void* k_pool, void* v_pool, int64_t num_pages, int32_t page_size,
                                  const int32_t* kv_indptr, const int32_t* kv_indices,
                                  const int32_t* kv_last_page_len, int64_t total_pages,
                                  int32_t batch, int32_t num_qo_heads, int32_t num_kv_heads,
                                  int32_t head_dim, float sm_scale, int32_t dtype, void* out,
                                  int64_t out_stride, void* workspace, size_t workspace_bytes,
                                  int64_t layout, nslg_stream_t stream);

/*
 * The same for a batch with radix-shared prefixes (nslg_paged_decode_grouped_append
 * with the rotation folded in): each member's query heads are rotated at that
 * member's position.
 */
int nslg_paged_decode_grouped_rope_append(
    const void* q, int64_t q_stride, const void* k_new, int64_t k_new_stride, const void* v_new,
    int64_t v_new_stride, const int32_t* positions, const float* cos_table, const float* sin_table,
    int64_t table_stride, int64_t table_rows, void* k_pool, void* v_pool, int64_t num_pages,
    int32_t page_size, const int32_t* kv_indptr, const int32_t* kv_indices,
    const int32_t* kv_last_page_len, int64_t total_pages, int32_t batch, int32_t num_qo_heads,
    int32_t num_kv_heads, int32_t head_dim, float sm_scale, int32_t dtype,
    const int32_t* seq_group_slot, int32_t num_groups, const int32_t* group_prefix_pages,
    const int32_t* group_members, void* out, int64_t out_stride, void* workspace,
    size_t workspace_bytes, int64_t layout, nslg_stream_t stream);

/*
 * Paged causal prefill attention over a ragged batch of new tokens whose K/V
 * are already appended to the pool (chunked prefill).
 * Replaces FlashInfer BatchPrefillWithPagedKVCacheWrapper.plan/run with
 * causal=True (nanoslg/kv_cache.py:622-632, 654) and the contiguous
 * masked/causal SDPA (kv_cache.py:317-321).
 *
 *   q           [T = qo_indptr[batch]] rows of Hq*D elements at stride q_stride
 *   qo_indptr   int32[batch+1] (device): new tokens of sequence b are rows
 *               [qo_indptr[b], qo_indptr[b+1]) and sit at the LAST positions of
 *               that sequence's L_b tokens (bottom-right causal alignment):
 *               row t of b attends to keys j <= L_b - n_b + t.
 *   total_q     host copy of qo_indptr[batch]; max_q: host max of n_b (sizes the
 *               longest-first tile order of near-uniform batches; a value below
 *               the true max only costs that order, never correctness)
 *   out         [T] rows of Hq*D elements at stride out_stride
 *   sm_scale    positive and finite (EINVAL otherwise)
 * Supported: f16, bf16 with D in {64, 128, 256} (MFMA); f32 with D in {64, 128,
 * 256} (the VALU kernel of nslg_paged_decode's f32 path); 1 <= Hq/Hkv <= 16.
 */
size_t nslg_paged_prefill_workspace_size(int32_t batch, int32_t num_qo_heads,
                                         int32_t head_dim, int64_t total_q,
                                         int32_t max_q);

int nslg_paged_prefill(const void* q, int64_t q_stride, const int32_t* qo_indptr,
                       int64_t total_q, int32_t max_q,
                       const void* k_pool, const void* v_pool, int64_t num_pages,
                       int32_t page_size, const int32_t* kv_indptr,
                       const int32_t* kv_indices, const int32_t* kv_last_page_len,
                       int32_t batch, int32_t num_qo_heads, int32_t num_kv_heads,
                       int32_t head_dim, float sm_scale, int32_t dtype,
                       void* out, int64_t out_stride,
                       void* workspace, size_t workspace_bytes,
                       nslg_stream_t stream);

/*
 * nslg_paged_prefill on the forward's padded input grid: q and out hold
 * batch x grid_width rows (the [B, S, Hq, D] grid of a padded forward, S =
 * grid_width), sequence b's block being rows b * grid_width .. + grid_width - 1.
 * Its n_b new tokens are rows q_rows[qo_indptr[b]] .. + n_b - 1 of the grid,
 * contiguous inside that block (the rows the forward's input offsets give,
 * kv_cache.py:567-573); every other row of the block is written as zeros.
 * Replaces the pack of the forward's rows into the ragged layout FlashInfer runs
 * on and the unpack of its output into the padded grid (kv_cache.py:676-691):
 * the kernel reads and writes the grid rows directly. q_rows: int32[total_q]
 * (device); a row outside the grid is neither read nor written. Other arguments
 * as nslg_paged_prefill (workspace unused).
 */
int nslg_paged_prefill_grid(const void* q, int64_t q_stride, const int32_t* qo_indptr,
                            const int32_t* q_rows, int32_t grid_width, int64_t total_q,
                            int32_t max_q, const void* k_pool, const void* v_pool,
                            int64_t num_pages, int32_t page_size, const int32_t* kv_indptr,
                            const int32_t* kv_indices, const int32_t* kv_last_page_len,
                            int32_t batch, int32_t num_qo_heads, int32_t num_kv_heads,
                            int32_t head_dim, float sm_scale, int32_t dtype,
                            void* out, int64_t out_stride,
                            void* workspace, size_t workspace_bytes,
                            nslg_stream_t stream);

/*
 * The multi-token forward of one layer (prefill chunks, ragged batches): the new
 * tokens' K/V rows written into the pool, then causal attention of their queries,
 * in one launch. Replaces the write of FlashInferCacheContext.attend (_write_kv,
 * nanoslg/kv_cache.py:661-674, slots of :575-594) together with the prefill run
 * (:657-659), which the reference issues back to back for one forward (:639-659).
 * Same result as nslg_append_kv of the rows followed by nslg_paged_prefill (q_rows
 * null) or nslg_paged_prefill_grid (q_rows set), bit for bit.
 *
 *   k_new, v_new   rows of Hkv*D elements at element strides k_new_stride,
 *                  v_new_stride (device, the pool's dtype, 16-byte aligned rows),
 *                  laid out as q's rows: token t of sequence b is row
 *                  qo_indptr[b] + t (q_rows null) or q_rows[qo_indptr[b]] + t of
 *                  the batch x grid_width grid
 *   other arguments as nslg_paged_prefill_grid (q_rows may be null: ragged rows)
 * Token t of sequence b is position L_b - n_b + t; its K/V rows go to that
 * position's page slot through the block table (a position past the table: slot 0
 * of page 0, the null page of the reference's slot mapping), so no slot mapping is
 * passed. Keys at the new positions are read from k_new / v_new, so no workgroup
 * waits for another's writes. Precondition, which the reference's copy-on-write
 * rule gives: no other sequence of the call reads a row being written. A row whose
 * page id is out of the pool is not written. f16 and bf16 pools (EUNSUPPORTED for
 * f32: append, then nslg_paged_prefill); k_new / v_new spanning >= 4 GiB:
 * EUNSUPPORTED.
 */
int nslg_paged_prefill_append(const void* q, int64_t q_stride, const int32_t* qo_indptr,
                              const int32_t* q_rows, int32_t grid_width, int64_t total_q,
                              int32_t max_q, const void* k_new, int64_t k_new_stride,
                              const void* v_new, int64_t v_new_stride,
                              void* k_pool, void* v_pool, int64_t num_pages,
                              int32_t page_size, const int32_t* kv_indptr,
                              const int32_t* kv_indices, const int32_t* kv_last_page_len,
                              int32_t batch, int32_t num_qo_heads, int32_t num_kv_heads,
                              int32_t head_dim, float sm_scale, int32_t dtype,
                              void* out, int64_t out_stride,
                              void* workspace, size_t workspace_bytes,
                              nslg_stream_t stream);

/*
 * Device-side plan of one decode step in which every sequence gains one token:
 * the CSR block table, slot mapping and positions of the next step from those of
 * this one. Replaces, for a steady decode batch, the per-step rebuild of the CSR
 * in FlashInferCacheContext._plan_flashinfer (nanoslg/kv_cache.py:598-615) and the
 * write plan of FlashInferCacheContext.__init__ (kv_cache.py:575-594) when no page
 * is shared (copy-on-write still goes through the host plan).
 *
 *   kv_indptr/kv_indices/kv_last_page_len   this step's CSR (device), batch rows
 *   new_page        HOST int32[batch]: the page sequence b opens this step (when its
 *                   last page is full or it has none), else -1; a sequence that
 *                   needs a page and gets -1 writes to the null page 0, slot 0
 *   *_out           the next step's CSR (device; indices capacity kv_indptr[batch]
 *                   + the pages opened), must not alias the inputs
 *   slot_mapping_out[b]  page * page_size + slot of sequence b's new token
 *   positions_out[b]     its position (the sequence's length minus one)
 *   new_pages_out   the pages opened, in batch order
 *   k_pool, v_pool  NULL, or the [L, P, page_size, Hkv, D] pools: then the opened
 *                   pages are also zeroed in every layer, K and V, in the same launch
 *                   (the zero-on-alloc of PagePool.alloc, kv_cache.py:411)
 * batch <= 512. Bit-exact with the host plan.
 */
int nslg_decode_plan_step(const int32_t* kv_indptr, const int32_t* kv_indices,
                          const int32_t* kv_last_page_len, int32_t batch, int32_t page_size,
                          const int32_t* new_page, int32_t* kv_indptr_out, int32_t* kv_indices_out,
                          int32_t* kv_last_page_len_out, int32_t* slot_mapping_out,
                          int32_t* positions_out, int32_t* new_pages_out, void* k_pool, void* v_pool,
                          int32_t num_layers, int64_t num_pages, int32_t num_kv_heads,
                          int32_t head_dim, int32_t dtype, nslg_stream_t stream);

/*
 * nslg_decode_plan_step with the opened-page list read from memory at run time
 * (int32[batch], same meaning as new_page above): device memory or pinned host
 * memory (hipHostMalloc; read through its device mapping). For a step captured in
 * a HIP graph: the launch's arguments stay the same from step to step and the host
 * writes the list before each replay. The zeroing grid has a slot per sequence;
 * slots of sequences that open no page exit. new_pages_out needs batch entries.
 */
int nslg_decode_plan_step_device(const int32_t* kv_indptr, const int32_t* kv_indices,
                                 const int32_t* kv_last_page_len, int32_t batch, int32_t page_size,
                                 const int32_t* new_page, int32_t* kv_indptr_out,
                                 int32_t* kv_indices_out, int32_t* kv_last_page_len_out,
                                 int32_t* slot_mapping_out, int32_t* positions_out, int32_t* new_pages_out,
                                 void* k_pool, void* v_pool, int32_t num_layers, int64_t num_pages,
                                 int32_t num_kv_heads, int32_t head_dim, int32_t dtype,
                                 nslg_stream_t stream);

/*
 * CSR block table of a forward from device-resident block tables. Replaces the
 * O(sum of pages) loop of FlashInferCacheContext._plan_flashinfer
 * (nanoslg/kv_cache.py:598-615, missing entries -> page 0 at :606-607) that
 * rebuilt the CSR from the Python block tables on every forward, and its upload
 * (:611-615).
 *
 *   tables          int32 arena (device) of table_capacity entries holding one row
 *                   per sequence: entry i of a row = page id of logical page i
 *   row_offset      int32[batch]: first arena entry of sequence b's row (rows of
 *                   the batch must not overlap)
 *   pages_have      int32[batch]: entries of row b that are valid (pages allocated)
 *   synced          int32[batch]: entries [0, synced_b) are already in the arena
 *   patch_indptr    int32[batch+1], patch int32[patch_total]: the values of entries
 *                   [synced_b, pages_have_b) of row b are patch[patch_indptr[b] ..];
 *                   they are also written into the arena (rows stay current)
 *   kv_indptr       int32[batch+1]: CSR pointers of the forward (npg_b pages of b)
 *   kv_indices      int32[total_pages] out: entry i < npg_b of segment b = row entry
 *                   i for i < pages_have_b, else 0 (the null page)
 * All arrays are device memory. Indices outside the arena, the patch or the CSR
 * are skipped (read as page 0). Bit-exact with the host CSR.
 */
int nslg_block_table_csr(int32_t* tables, int64_t table_capacity, const int32_t* row_offset,
                         const int32_t* pages_have, const int32_t* synced,
                         const int32_t* patch_indptr, const int32_t* patch, int64_t patch_total,
                         const int32_t* kv_indptr, int32_t* kv_indices, int64_t total_pages,
                         int32_t batch, nslg_stream_t stream);

/*
 * Device-side write plan of a multi-token forward: expands the forward's
 * per-sequence tables into the per-token arrays the append and the prefill take.
 * Replaces the per-token loop of FlashInferCacheContext.__init__ (slot of every new
 * token, nanoslg/kv_cache.py:575-594, writes past the table to the null page's slot
 * 0, :583-584), the positions of get_position_ids (:567-573, 635-637) and the ragged
 * layout of _pack_q / qo_indptr (:622-632, 676-691).
 *
 *   kv_indptr/kv_indices   this forward's CSR block table (device; after copy-on-write)
 *   start, new_tokens, input_offsets, pages_allocated   int32[batch] (device)
 *   input_width            iw = max(input_offsets[b] + new_tokens[b])
 *   slot_mapping_out, positions_out   int32[batch * iw]: grid row b*iw + off_b + t
 *                          gets page*page_size+slot and start_b + t; other rows -1
 *                          and 0
 *   ragged_rows_out        int32[sum(new_tokens)]: grid row of ragged row qo_b + t
 *   qo_indptr_out          int32[batch + 1]
 * Bit-exact with the host plan.
 */
int nslg_forward_plan(const int32_t* kv_indptr, const int32_t* kv_indices, const int32_t* start,
                      const int32_t* new_tokens, const int32_t* input_offsets,
                      const int32_t* pages_allocated, int32_t batch, int32_t input_width,
                      int32_t page_size, int32_t* slot_mapping_out, int32_t* positions_out,
                      int32_t* ragged_rows_out, int32_t* qo_indptr_out, nslg_stream_t stream);

/*
 * nslg_block_table_csr and nslg_forward_plan in one launch (the two device steps of
 * a forward planned on the device, kv_cache.py:575-615): the arguments of
 * nslg_block_table_csr, then those of nslg_forward_plan that it lacks, with
 * pages_have standing for pages_allocated. kv_indices, the arena rows and every
 * output are bit-identical with the two calls made in order; the plan takes each
 * page id from the arena and the patch, as the CSR does, so no part waits for
 * another.
 */
int nslg_forward_plan_csr(int32_t* tables, int64_t table_capacity, const int32_t* row_offset,
                          const int32_t* pages_have, const int32_t* synced, const int32_t* patch_indptr,
                          const int32_t* patch, int64_t patch_total, const int32_t* kv_indptr,
                          int32_t* kv_indices, int64_t total_pages, const int32_t* start,
                          const int32_t* new_tokens, const int32_t* input_offsets, int32_t batch,
                          int32_t input_width, int32_t page_size, int32_t* slot_mapping_out,
                          int32_t* positions_out, int32_t* ragged_rows_out, int32_t* qo_indptr_out,
                          nslg_stream_t stream);

/*
 * Fused rotary position embedding + K/V append. Replaces, per layer, the position
 * gather and the two apply_rotary_emb calls of _attention_forward
 * (nanoslg/models.py:96-103, apply_rotary_emb :69-83) together with the cache write
 * of attend (kv_cache.py:661-674 paged, :301-310 contiguous); the positions are the
 * forward's (get_position_ids, kv_cache.py:567-573, 635-637).
 *
 *   q               [num_rows] rows of Hq*D elements at stride q_stride
 *   q_out           rotated q, rows at stride q_out_stride; may be q itself (in
 *                   place), must not overlap it otherwise
 *   k_new, v_new    [num_rows] rows of Hkv*D elements at k_stride / v_stride
 *   positions       int32[num_rows] (device): the row's position; clamped into the
 *                   table (callers check the range, as indexing the table would)
 *   slot_mapping    int32[num_rows] (device): page*page_size+slot of the row's K/V;
 *                   negative (padding) or >= pool_slots: the row's K/V are not written
 *   cos_table, sin_table   fp32 [table_rows] rows of >= D floats at table_stride
 *                   (the model's precomputed tables, models.py:37-66)
 *   k_pool, v_pool  one layer, pool_slots rows of Hkv*D elements
 * q_out and the pool's K rows = rnd(rnd(x*c) + rnd(rot(x)*s)) in the storage type
 * with c, s the table values rounded to it, rot(x) = cat(-x[D/2:], x[:D/2]):
 * bit-exact with the eager expression. V rows are copied. f16/bf16/f32,
 * D in {64,128,256}.
 */
int nslg_rope_append(const void* q, int64_t q_stride, void* q_out, int64_t q_out_stride,
                     const void* k_new, int64_t k_stride, const void* v_new, int64_t v_stride,
                     const int32_t* positions, const int32_t* slot_mapping, int64_t num_rows,
                     const float* cos_table, const float* sin_table, int64_t table_stride,
                     int64_t table_rows, int32_t num_qo_heads, int32_t num_kv_heads,
                     int32_t head_dim, void* k_pool, void* v_pool, int64_t pool_slots,
                     int32_t dtype, nslg_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* NSLG_KV_H */
