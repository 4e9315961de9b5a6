// Split-K paged GQA decode attention for gfx950 (CDNA4), plus the fp32
// log-sum-exp merge of the splits.
//
// Work decomposition
//   Each sequence's tokens are cut into ceil(L / chunk_tokens) chunks of equal
//   length (boundaries on 16-token tiles). Workgroup (x, y) of the grid is
//   (chunk, group of KV heads); each wave owns one (chunk, KV head) and works
//   alone: no LDS, no barriers. The chunk length is the smallest one whose chunk
//   count fits the device's resident workgroup slots (the host passes that
//   budget; every wave finds the same length by a binary search over the
//   sequence lengths), so every wave starts at launch and streams one long chunk
//   and no second, partly filled round of workgroups trails the first. A wave
//   finds its sequence by a wave-wide prefix sum over the per-sequence chunk
//   counts (kv_indptr is a few hundred bytes and L2-resident), so no separate
//   planning launch is needed.
//
// Per 16-token tile (one page at page_size 16), for the G query heads of the
// wave's KV head (G = Hq/Hkv <= 16):
//   S[16 tok x 16 col] = K[16 tok x D] * Q^T[D x 16 col]   (v_mfma 16x16x32, D/32 steps)
//     A = K rows straight from HBM (lane l: token l%16, 16 B at d = 32s + 8(l/16)),
//     B = Q^T held in registers for the whole chunk; columns >= G are zero.
//   online softmax in fp32 on the accumulator layout (lane l holds tokens
//     4(l/16)+j of head l%16); max over the 16 tokens = 3 in-lane max + 2 xor-shuffles.
//   O^T[D x 16 col] += V^T[D x 16 tok] * P^T[16 tok x 16 col]  (v_mfma 16x16x16, D/16 tiles)
//     B = P^T is exactly the S accumulator layout, converted to 16 bit;
//     A = V^T: lane l loads tokens 4(l/16)+j (j=0..3), 16 B at d = (D/16)*(l%16), so each
//     load instruction reads 4 whole 256 B rows; output tile n then holds
//     d = (D/16)*row + n, a permutation undone when the result is stored.
// K and V of the next tile are loaded before the current tile is computed.
//
// HBM traffic per (token, kv head): 2*D*2 bytes (K and V, read once).
#include "nslg_common.h"

#include <math.h>

#include <atomic>
#include <mutex>
#include <type_traits>

namespace nslg {
namespace {

constexpr int kMaxWaves = 4;  // waves (KV heads) per workgroup

struct DecodeParams {
  const uint16_t* q;
  int64_t q_stride;  // elements between batch rows
  const uint16_t* k_pool;
  const uint16_t* v_pool;
  int64_t num_pages;
  int32_t page_size;
  const int32_t* indptr;
  const int32_t* indices;
  const int32_t* last_len;
  int32_t batch;
  int32_t num_qo_heads;
  int32_t num_kv_heads;
  int32_t group;  // Hq / Hkv
  float scale_log2;
  int32_t chunk_tokens;  // an upper bound that fits chunk_budget, or the length to use
  int32_t chunk_budget;  // > 0: search the smallest length with <= this many chunks
  int32_t max_chunks;
  int32_t head_groups;   // workgroups per chunk (grid y)
  int2* meta;            // per sequence: first chunk, chunk count (for the merge launch)
  // Layout of the call's chunks, kept in the workspace for the other layers of a
  // forward (same batch and plan): layout_mode 0: found from the lengths; > 0: found,
  // and recorded under layout_tag; < 0: read from the record when *layout_tag_ptr is
  // layout_tag, found otherwise. Two int4 per chunk (see the kernel).
  int32_t layout_mode;
  int64_t total_pages;  // entries of indices (kv_indptr[batch])
  uint64_t layout_tag;
  uint64_t* layout_tag_ptr;
  int4* layout_map;
  uint16_t* out;
  int64_t out_stride;
  float* part_o;   // [max_chunks, slot_members, Hq, D]
  float* part_ml;  // [max_chunks, slot_members, Hq, 2]
  int32_t slot_members;  // partial slots per (chunk, query head): 1, or the members of a group
  int32_t stream;        // 1: the call's K/V exceed the caches: stream them (non-temporal loads)
  // New rows (null: none). Sequence b's row of k_new / v_new is its token L_b - 1:
  // the chunk holding that token writes it into the pool before reading it.
  const uint16_t* k_new;
  const uint16_t* v_new;
  int64_t k_new_stride;  // elements between batch rows
  int64_t v_new_stride;
  // Rotary embedding (rope_cos null: none): q and the new K rows are rotated at
  // sequence b's position rope_pos[b] (clamped into the tables) before use, with the
  // arithmetic of nslg_rope_append; tables fp32 [rope_rows] rows at rope_stride.
  const int32_t* rope_pos;
  const float* rope_cos;
  const float* rope_sin;
  int64_t rope_stride;
  int64_t rope_rows;
};

// Table rows of sequence b's position (rope_pos[b], clamped into the tables).
__device__ inline void rope_rows_of(const DecodeParams& p, int b, const float*& crow, const float*& srow) {
  int64_t pos = p.rope_pos[b];
  pos = pos < 0 ? 0 : (pos >= p.rope_rows ? p.rope_rows - 1 : pos);
  crow = p.rope_cos + pos * p.rope_stride;
  srow = p.rope_sin + pos * p.rope_stride;
}

// Prefix groups of a grouped decode call: sequences whose first pages are the same
// pages (a shared radix prefix). The prefix of a group is one more work unit whose
// chunks serve all its members at once: member m's query heads take MFMA columns
// G*m .. G*m + G-1, so the shared K/V is read once per group instead of once per
// member. Passed as kernel arguments; the host checks them.
constexpr int kMaxGroups = 32;
constexpr int kGroupCols = 16;  // MFMA columns

template <bool kGrouped>
struct GroupArgs {};

template <>
struct GroupArgs<true> {
  const int32_t* seq_group_slot;  // [batch]: 16 * group + member, or -1
  int2* group_meta;               // [num_groups]: first chunk and chunk count of the prefix
  int32_t num_groups;
  int32_t prefix_pages[kMaxGroups];
  int16_t member_seq[kMaxGroups * kGroupCols];  // sequence of member m of group g, or -1
};

__device__ inline int seq_len_of(const int32_t* indptr, const int32_t* last_len, int s,
                                 int page_size) {
  const int np = indptr[s + 1] - indptr[s];
  if (np <= 0) return 0;
  int lpl = last_len[s];
  lpl = lpl < 1 ? 1 : (lpl > page_size ? page_size : lpl);
  return (np - 1) * page_size + lpl;
}

__device__ inline int wave_sum_i32(int x) {
  x += __builtin_amdgcn_mov_dpp(x, 0x128, 0xf, 0xf, false);  // row_ror:8
  x += __builtin_amdgcn_mov_dpp(x, 0x124, 0xf, 0xf, false);  // row_ror:4
  x += __builtin_amdgcn_mov_dpp(x, 0x122, 0xf, 0xf, false);  // row_ror:2
  x += __builtin_amdgcn_mov_dpp(x, 0x121, 0xf, 0xf, false);  // row_ror:1
  const auto a = __builtin_amdgcn_permlane16_swap((unsigned)x, (unsigned)x, false, false);
  x = (int)(a[0] + a[1]);
  const auto c = __builtin_amdgcn_permlane32_swap((unsigned)x, (unsigned)x, false, false);
  return (int)(c[0] + c[1]);
}

// Tokens of the prefix of group g (its first member's length bounds it, so the
// prefix never reads past that member's block table).
__device__ inline int group_prefix_tokens(const DecodeParams& p, const GroupArgs<true>& ga, int g) {
  const int m0 = ga.member_seq[g * kGroupCols];
  const int L0 = m0 >= 0 && m0 < p.batch ? seq_len_of(p.indptr, p.last_len, m0, p.page_size) : 0;
  return min(ga.prefix_pages[g] * p.page_size, L0);
}

// Tokens of sequence b read through its group's prefix (0 outside a group).
__device__ inline int seq_prefix_tokens(const DecodeParams& p, const GroupArgs<true>& ga, int b, int len) {
  const int gs = ga.seq_group_slot[b];
  const int g = gs >> 4;
  if (gs < 0 || g >= ga.num_groups) return 0;
  return min(ga.prefix_pages[g] * p.page_size, len);
}

// Work units of a call: sequence u's own tokens for u < batch (all of them, or those
// after its group's prefix), then the prefix of group u - batch.
template <bool kGrouped>
__device__ inline int unit_len(const DecodeParams& p, const GroupArgs<kGrouped>& ga, int u) {
  if (u < p.batch) {
    int len = seq_len_of(p.indptr, p.last_len, u, p.page_size);
    if constexpr (kGrouped) len -= seq_prefix_tokens(p, ga, u, len);
    return len;
  }
  if constexpr (kGrouped) {
    const int g = u - p.batch;
    if (g < ga.num_groups) return group_prefix_tokens(p, ga, g);
  }
  return 0;
}

// Unit lengths as the lanes see them: lane l holds unit 64 i + l in v[i] for the
// first 256 units (loaded once, so the searches below do not go back to memory);
// later ones are read on demand.
template <bool kGrouped>
struct LaneLens {
  static constexpr int kRegs = 4;
  int v[kRegs];
  int units;

  __device__ LaneLens(const DecodeParams& p, const GroupArgs<kGrouped>& ga, int n) : units(n) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < kRegs; ++i) {
      const int s = 64 * i + lane;
      v[i] = s < units ? unit_len<kGrouped>(p, ga, s) : 0;
    }
  }
  // length of unit 64 i + lane (0 past the units)
  __device__ int at(const DecodeParams& p, const GroupArgs<kGrouped>& ga, int i) const {
    if (i < kRegs) {
      int r = v[0];
#pragma unroll
      for (int j = 1; j < kRegs; ++j) r = i == j ? v[j] : r;
      return r;
    }
    const int s = 64 * i + (threadIdx.x & 63);
    return s < units ? unit_len<kGrouped>(p, ga, s) : 0;
  }
};

// Smallest chunk length in [lo, hi] (multiples of 16) for which the units' chunk
// count sum_u ceil(L_u / len) is at most `budget`; `hi` is known to fit. The
// count does not grow with the length, so a binary search finds it; all waves
// compute the same value from the same lengths.
template <bool kGrouped>
__device__ inline int fit_chunk_tokens(const DecodeParams& p, const GroupArgs<kGrouped>& ga,
                                       const LaneLens<kGrouped>& lens, int lo, int hi, int budget) {
  int a = lo >> 4, z = hi >> 4;
  const int groups = (lens.units + 63) >> 6;
  while (a < z) {
    const int mid = (a + z) >> 1;
    const int ct = mid << 4;
    int cnt = 0;
    for (int i = 0; i < groups; ++i) cnt += (lens.at(p, ga, i) + ct - 1) / ct;
    cnt = __builtin_amdgcn_readfirstlane(wave_sum_i32(cnt));
    if (cnt <= budget)
      z = mid;
    else
      a = mid + 1;
  }
  return a << 4;
}

// Wave-wide search for the unit owning global chunk `g`.
template <bool kGrouped>
__device__ inline bool locate_chunk(const DecodeParams& p, const GroupArgs<kGrouped>& ga,
                                    const LaneLens<kGrouped>& lens, int chunk_tokens, int g, int& b,
                                    int& cstart, int& nchunks) {
  const int lane = threadIdx.x & 63;
  int base = 0;
  const int groups = (lens.units + 63) >> 6;
  for (int i = 0; i < groups; ++i) {
    const int len = lens.at(p, ga, i);
    const int nc = (len + chunk_tokens - 1) / chunk_tokens;
    int incl = nc;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int y = __shfl_up(incl, off, 64);
      if (lane >= off) incl += y;
    }
    const int excl = incl - nc;
    const bool hit = nc > 0 && g >= base + excl && g < base + incl;
    const unsigned long long m = __ballot(hit);
    if (m) {
      const int src = __ffsll((long long)m) - 1;
      b = 64 * i + src;
      cstart = base + __shfl(excl, src, 64);
      nchunks = __shfl(nc, src, 64);
      return true;
    }
    base += __shfl(incl, 63, 64);
  }
  return false;
}

template <int N>
struct RowVec {
  typedef unsigned short type __attribute__((ext_vector_type(N)));
};

template <int D>
struct Tile {
  static constexpr int kSteps = D / 32;  // QK k-steps of 32
  static constexpr int kNT = D / 16;     // PV output tiles; V elements per lane per token
  u16x8 k[kSteps];
  typename RowVec<kNT>::type v[4];
};

// Address of token `tok` (clamped into [0, len)) for kv head h (any page size).
__device__ inline const uint16_t* token_row(const uint16_t* pool, const int32_t* idx, int64_t num_pages,
                                            int page_size, int64_t row_elems, int head_off, int tok) {
  int32_t pid = idx[tok / page_size];
  if (pid < 0 || (int64_t)pid >= num_pages) pid = 0;
  return pool + ((int64_t)pid * page_size + (tok % page_size)) * row_elems + head_off;
}

// K/V rows are read once per decode call. When a call's K/V are larger than the
// memory-side cache can hold (kStreamBytes), the loads carry the non-temporal hint
// (`nt`) and stream from HBM: measured on the KV-pressure page pattern (pure loads,
// 3 GB) 6.15 TB/s plain, 6.95 TB/s non-temporal; the batch-64 decode call 494 ->
// 456 us. A smaller call's K/V stay in the caches from one decode step to the next,
// which only ordinary loads keep using (4 sequences of 1-4k tokens: 13.7 us plain,
// 15.9 us streamed). A group's shared prefix, which every group sharing it reads, is
// always loaded normally so the later reads can hit in the caches.
template <typename V, bool kStream>
__device__ inline V kv_load(const char* p) {
  if constexpr (kStream)
    return __builtin_nontemporal_load(reinterpret_cast<const V*>(p));
  else
    return *reinterpret_cast<const V*>(p);
}

// Loads of one tile whose 16 token rows are consecutive in one page. kbase/vbase:
// wave-uniform byte address of the tile's first row (head offset included); rows
// past `last` repeat row `last`.
//   K, D <= 128: load s, lane l reads row (64 / (D/8)) s + l / (D/8), 16 B at
//                d = 8 (l % (D/8)): whole rows, turned into MFMA operands through
//                the wave's LDS stage (k_operands_from_rows)
//   K, D = 256:  lane l reads row l%16, 16 B at d = 32 s + 8 (l/16), the operand
//                itself (the stage's operand registers would cost the kernel its
//                second wave per SIMD at this head dim)
//   V: lane l reads rows 4 (l/16) + j, D/16 elements at d = (D/16) (l%16)
template <int D>
constexpr bool kKRows = D <= 128;

template <int D, bool kStream>
__device__ inline void load_tile_rows(const char* kbase, const char* vbase, int row_bytes, int last,
                                      Tile<D>& t) {
  const int lane = threadIdx.x & 63;
  const int r = lane & 15;
  const int gq = lane >> 4;
  constexpr int NT = D / 16;
  typedef typename RowVec<NT>::type VT;
  if constexpr (kKRows<D>) {
    // K as whole rows: load s takes tokens kTokPerLoad*s .. +kTokPerLoad-1, D/8 lanes
    // per token, 16 bytes each (as the V loads below, each instruction reads whole
    // 2D-byte rows; 16 tokens x 64 bytes per instruction streamed 3.5 % slower at
    // batch 64). The MFMA operand layout comes from the wave's stage in LDS.
    constexpr int kLanesPerTok = D / 8;
    constexpr int kTokPerLoad = 64 / kLanesPerTok;
    const int k_tok = lane / kLanesPerTok;
    const int k_ch = lane % kLanesPerTok;
#pragma unroll
    for (int s = 0; s < Tile<D>::kSteps; ++s) {
      const int kr = kTokPerLoad * s + k_tok;
      t.k[s] = kv_load<u16x8, kStream>(kbase + (kr < last ? kr : last) * row_bytes + 16 * k_ch);
    }
  } else {  // the MFMA operand layout straight from memory
    const char* kp = kbase + (r < last ? r : last) * row_bytes + 16 * gq;
#pragma unroll
    for (int s = 0; s < Tile<D>::kSteps; ++s) t.k[s] = kv_load<u16x8, kStream>(kp + 64 * s);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int vr = 4 * gq + j;
    t.v[j] = kv_load<VT, kStream>(vbase + (vr < last ? vr : last) * row_bytes + 2 * NT * r);
  }
}

// Per-wave LDS stage of one K tile (16 tokens x D, rows padded by 8 elements: the
// 16-byte operand reads of 8 consecutive tokens hit distinct bank groups). The rows
// arrive from load_tile_rows one token per D/8 lanes; the QK MFMA wants lane
// r + 16 gq to hold token r, elements 32 ks + 8 gq .. +7.
template <int D>
struct KStage {
  static constexpr int kPitch = D + 8;
  uint16_t e[16 * kPitch];
};

template <int D>
__device__ inline void k_operands_from_rows(KStage<D>& st, const Tile<D>& t, u16x8 (&ka)[Tile<D>::kSteps]) {
  constexpr int kLanesPerTok = D / 8;
  constexpr int kTokPerLoad = 64 / kLanesPerTok;
  constexpr int kPitch = KStage<D>::kPitch;
  const int lane = threadIdx.x & 63;
  const int k_tok = lane / kLanesPerTok;
  const int k_ch = lane % kLanesPerTok;
  const int r = lane & 15;
  const int gq = lane >> 4;
  // the wave's previous reads of the stage come before these writes, and the writes
  // before the reads below: one wave's LDS operations complete in order, and the
  // fences keep the compiler from moving a lane's access across another lane's
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
#pragma unroll
  for (int s = 0; s < Tile<D>::kSteps; ++s)
    *reinterpret_cast<u16x8*>(&st.e[(kTokPerLoad * s + k_tok) * kPitch + 8 * k_ch]) = t.k[s];
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
#pragma unroll
  for (int ks = 0; ks < Tile<D>::kSteps; ++ks)
    ka[ks] = *reinterpret_cast<const u16x8*>(&st.e[r * kPitch + 32 * ks + 8 * gq]);
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The MFMA operand positions (K as for D = 256 above, V as above), each lane
// resolving its own token's page (page sizes that are not a multiple of 16, where a
// tile can straddle pages).
template <int D, bool kStream>
__device__ inline void load_tile_any(const DecodeParams& p, const int32_t* idx, int head_off, int t0,
                                     int t_last, Tile<D>& t) {
  const int lane = threadIdx.x & 63;
  const int r = lane & 15;
  const int gq = lane >> 4;
  const int64_t row_elems = (int64_t)p.num_kv_heads * D;
  constexpr int NT = D / 16;
  typedef typename RowVec<NT>::type VT;
  int tk = t0 + r;
  tk = tk > t_last ? t_last : tk;
  const uint16_t* krow = token_row(p.k_pool, idx, p.num_pages, p.page_size, row_elems, head_off, tk);
#pragma unroll
  for (int s = 0; s < Tile<D>::kSteps; ++s)
    t.k[s] = kv_load<u16x8, kStream>(reinterpret_cast<const char*>(krow + 32 * s + 8 * gq));
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    int tv = t0 + 4 * gq + j;
    tv = tv > t_last ? t_last : tv;
    const uint16_t* vrow = token_row(p.v_pool, idx, p.num_pages, p.page_size, row_elems, head_off, tv);
    t.v[j] = kv_load<VT, kStream>(reinterpret_cast<const char*>(vrow + NT * r));
  }
}

// Running-max rescale threshold (log2 units): the accumulators are rescaled only
// when a tile's max exceeds the running max by more than this, so probabilities
// stay <= 2^8 and most tiles never touch the accumulators. Exact: O and l are
// always relative to the same m.
constexpr float kRescaleSlack = 8.0f;

template <typename T, int D, bool kTileInPage, int kDepth, bool kGrouped>
__global__ void __launch_bounds__(64 * kMaxWaves)
paged_decode_kernel(DecodeParams p, GroupArgs<kGrouped> ga) {
  constexpr int kSteps = D / 32;
  constexpr int NT = D / 16;
  constexpr bool kSplitP = T::kDtype == NSLG_BF16;  // P = hi + lo for bf16's 8-bit mantissa
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int chunk = blockIdx.x;
  const int h = blockIdx.y * (blockDim.x >> 6) + wave;
  if (h >= p.num_kv_heads) return;

  // The chunk's work: unit u (sequence b's own tokens, or group g's prefix read
  // through member b's table), its chunk range [cstart, cstart + nchunks), the
  // chunk's tokens [t_begin, t_end), b's block-table offset and page count, and
  // whether b's result also takes its group's prefix. Either read from the layout
  // an earlier call of the same forward recorded in the workspace (layout < 0, when
  // the workspace holds its tag), or found from the lengths.
  int u = 0, cstart = 0, nchunks = 0, b = 0, g = -1, t_begin = 0, t_end = 0, idx_off = 0, np_seq = 0;
  bool merged = false;
  bool mapped = false;
  if (p.layout_mode < 0 && *p.layout_tag_ptr == p.layout_tag) {
    const int4 e0 = p.layout_map[2 * chunk];
    const int4 e1 = p.layout_map[2 * chunk + 1];
    u = __builtin_amdgcn_readfirstlane(e0.x);
    if (u < 0) return;  // no unit: past the forward's chunks
    cstart = __builtin_amdgcn_readfirstlane(e0.y);
    nchunks = __builtin_amdgcn_readfirstlane(e0.z);
    idx_off = __builtin_amdgcn_readfirstlane(e0.w);
    b = __builtin_amdgcn_readfirstlane(e1.x);
    t_begin = __builtin_amdgcn_readfirstlane(e1.y);
    t_end = __builtin_amdgcn_readfirstlane(e1.z);
    const int w1 = __builtin_amdgcn_readfirstlane(e1.w);
    np_seq = w1 & 0x3fffffff;
    merged = (w1 >> 30) & 1;
    if constexpr (kGrouped) g = u >= p.batch ? u - p.batch : -1;
    // a record of another batch (a caller's mistake) must not send a wave outside
    // the block table: such an entry is found from the lengths instead
    int units = p.batch;
    if constexpr (kGrouped) units += ga.num_groups;
    mapped = u < units && b >= 0 && b < p.batch && nchunks > 0 && cstart >= 0 && cstart <= chunk &&
             chunk < cstart + nchunks && idx_off >= 0 && (int64_t)idx_off + np_seq <= p.total_pages &&
             t_begin >= 0 && t_begin < t_end && (int64_t)t_end <= (int64_t)np_seq * p.page_size;
  }
  const bool record = p.layout_mode > 0 && blockIdx.y == 0 && threadIdx.x == 0;
  if (!mapped) {
    g = -1;
    merged = false;
    if (record && chunk == 0) *p.layout_tag_ptr = p.layout_tag;
    int units = p.batch;
    if constexpr (kGrouped) units += ga.num_groups;
    const LaneLens<kGrouped> lens(p, ga, units);
    int ct = p.chunk_tokens;
    if (p.chunk_budget > 0) {
      // An upper bound that fits, from the lengths themselves: with T tokens over U
      // units, length ceil(T / (budget - U)) gives at most T / len + U <= budget
      // chunks. (It is at most the host's bound, which came from an upper bound of T,
      // so the search finds the same length; and a launch captured once stays right
      // while the lengths grow.)
      int tot = 0;
      const int groups = (lens.units + 63) >> 6;
      for (int i = 0; i < groups; ++i) tot += lens.at(p, ga, i);
      const int64_t t_all = (int64_t)__builtin_amdgcn_readfirstlane(wave_sum_i32(tot));
      const int64_t usable = (int64_t)p.chunk_budget - lens.units;
      int64_t hi = (t_all + usable - 1) / usable;
      hi = ((hi + 15) / 16) * 16;
      // Shortest chunk: a chunk costs a fixed set-up and a partial to merge, so small
      // batches (where the slots are not the limit) take fewer, longer chunks: about
      // t_all / 96 tokens, between 64 and 256 (measured best at 4 sequences of 1k-4k
      // tokens and at 16-64 sequences of 1k-2k; large batches are bounded by `hi`).
      // Grouped calls merge each member's own partials with its group prefix's, so
      // longer chunks pay there sooner: t_all / 64 (16 requests on a 2040-token
      // prefix: 25.0 -> 22.4 us per call; t_all / 48 the same as / 64).
      constexpr int64_t kLoDiv = kGrouped ? 64 : 96;
      int64_t lo = ((t_all / kLoDiv + 15) / 16) * 16;
      lo = lo < 64 ? 64 : (lo > 256 ? 256 : lo);
      hi = hi < lo ? lo : (hi > ((int64_t)1 << 30) ? ((int64_t)1 << 30) : hi);
      ct = fit_chunk_tokens<kGrouped>(p, ga, lens, (int)lo, (int)hi, p.chunk_budget);
    }
    if (!locate_chunk<kGrouped>(p, ga, lens, ct, chunk, u, cstart, nchunks)) {
      if (record) p.layout_map[2 * chunk] = make_int4(-1, 0, 0, 0);
      return;
    }
    u = __builtin_amdgcn_readfirstlane(u);
    cstart = __builtin_amdgcn_readfirstlane(cstart);
    nchunks = __builtin_amdgcn_readfirstlane(nchunks);
    // sequence b's tokens [base, base + len) (all of them, or those after its group's
    // prefix), or group g's prefix [0, len), read through member 0's table
    b = u;
    int base = 0, len = 0;
    if constexpr (kGrouped) {
      if (u >= p.batch) {
        g = u - p.batch;
        b = ga.member_seq[g * kGroupCols];
        len = group_prefix_tokens(p, ga, g);
      } else {
        const int L = seq_len_of(p.indptr, p.last_len, b, p.page_size);
        base = seq_prefix_tokens(p, ga, b, L);
        len = L - base;
        merged = ga.seq_group_slot[b] >= 0 && (ga.seq_group_slot[b] >> 4) < ga.num_groups;
      }
      b = __builtin_amdgcn_readfirstlane(b);
      g = __builtin_amdgcn_readfirstlane(g);
      base = __builtin_amdgcn_readfirstlane(base);
      len = __builtin_amdgcn_readfirstlane(len);
    } else {
      len = seq_len_of(p.indptr, p.last_len, b, p.page_size);
    }
    // chunk c of the unit's nchunks covers tiles [c*ntiles/nchunks, (c+1)*ntiles/nchunks)
    const int ntiles_seq = (len + 15) >> 4;
    const int c_local = chunk - cstart;
    t_begin = base + 16 * (int)((int64_t)c_local * ntiles_seq / nchunks);
    t_end = base + min(16 * (int)((int64_t)(c_local + 1) * ntiles_seq / nchunks), len);
    idx_off = p.indptr[b];
    np_seq = p.indptr[b + 1] - idx_off;
    if (record) {
      p.layout_map[2 * chunk] = make_int4(u, cstart, nchunks, idx_off);
      p.layout_map[2 * chunk + 1] = make_int4(b, t_begin, t_end, np_seq | (merged ? 1 << 30 : 0));
    }
  }
  // the chunk ranges of the merge (written by every call: a call between two calls
  // of one forward may have used the workspace)
  if (chunk == cstart && blockIdx.y == 0 && threadIdx.x == 0) {
    if constexpr (kGrouped) {
      if (g >= 0)
        ga.group_meta[g] = make_int2(cstart, nchunks);
      else
        p.meta[b] = make_int2(cstart, nchunks);
    } else {
      p.meta[b] = make_int2(cstart, nchunks);
    }
  }
  const int c_local = chunk - cstart;
  const int t_last = t_end - 1;
  const int32_t* idx = p.indices + idx_off;

  // The new row of sequence b (its last token, in its last page) is written by its
  // last chunk, this wave for its own KV head, before any of the chunk's loads: the
  // loads of one wave after its store to the same address return the stored data,
  // and no other chunk (nor, by the copy-on-write rule, any other sequence) reads
  // that row. 16-byte vectors: lanes [0, D/8) carry K, [D/8, D/4) V.
  if (p.k_new != nullptr && u < p.batch && c_local == nchunks - 1 && t_end > t_begin) {
    const int tok = t_end - 1;
    const int pid = idx[tok / p.page_size];
    if (pid >= 0 && (int64_t)pid < p.num_pages) {
      constexpr int kVecs = D / 8;
      const int64_t row = ((int64_t)pid * p.page_size + tok % p.page_size) * p.num_kv_heads * D + (int64_t)h * D;
      if (lane < 2 * kVecs) {
        const bool is_v = lane >= kVecs;
        const int e = 8 * (is_v ? lane - kVecs : lane);
        const uint16_t* src = (is_v ? p.v_new + (int64_t)b * p.v_new_stride : p.k_new + (int64_t)b * p.k_new_stride) +
                              (int64_t)h * D + e;
        uint16_t* dst = const_cast<uint16_t*>(is_v ? p.v_pool : p.k_pool) + row + e;
        u16x8 val = *reinterpret_cast<const u16x8*>(src);
        if (!is_v && p.rope_cos != nullptr) {  // the K row rotated at the token's position
          const bool lo = e < D / 2;
          const u16x8 partner = *reinterpret_cast<const u16x8*>(src + (lo ? D / 2 : -D / 2));
          const float *crow, *srow;
          rope_rows_of(p, b, crow, srow);
          val = rope8<T>(val, partner, crow, srow, e, lo);
        }
        *reinterpret_cast<u16x8*>(dst) = val;
      }
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);  // keep the compiler from moving loads above the store
  }

  // Column r of the MFMA tiles (lane l: r = l % 16) is query head h*G + r of sequence
  // b; in a group's prefix it is head h*G + r%G of member r/G.
  const int r = lane & 15;
  const int gq = lane >> 4;
  int hq = h * p.group + r;
  bool head_ok = r < p.group;
  int col_seq = b;
  int member = 0;
  if constexpr (kGrouped) {
    if (g >= 0) {
      member = r / p.group;
      hq = h * p.group + r % p.group;
      col_seq = ga.member_seq[g * kGroupCols + member];
      head_ok = col_seq >= 0 && col_seq < p.batch;
    }
  }

  // Q^T operand: lane l holds Q[column l%16][32s + 8(l/16) .. +8]; zero for padding columns.
  u16x8 qb[kSteps];
  if (head_ok) {
    const uint16_t* qrow = p.q + (int64_t)col_seq * p.q_stride + (int64_t)hq * D;
#pragma unroll
    for (int s = 0; s < kSteps; ++s) qb[s] = *reinterpret_cast<const u16x8*>(qrow + 32 * s + 8 * gq);
    if (p.rope_cos != nullptr) {
      // rotated at the column's sequence's position: element d = 32s + 8gq + e of
      // qb[s] (s < kSteps / 2) pairs with d + D/2 in qb[s + kSteps / 2], the same lane
      const float *crow, *srow;
      rope_rows_of(p, col_seq, crow, srow);
#pragma unroll
      for (int s = 0; s < kSteps / 2; ++s) {
        const u16x8 lo = qb[s], hi = qb[s + kSteps / 2];
        qb[s] = rope8<T>(lo, hi, crow, srow, 32 * s + 8 * gq, true);
        qb[s + kSteps / 2] = rope8<T>(hi, lo, crow, srow, 32 * s + 8 * gq + D / 2, false);
      }
    }
  } else {
#pragma unroll
    for (int s = 0; s < kSteps; ++s) qb[s] = u16x8{0, 0, 0, 0, 0, 0, 0, 0};
  }

  float m_run = -INFINITY;
  float l_run = 0.f;
  f32x4 o[NT];
#pragma unroll
  for (int n = 0; n < NT; ++n) o[n] = f32x4{0.f, 0.f, 0.f, 0.f};

  // K tiles of the page-aligned path arrive as rows (head dims up to 128) and are
  // turned into operands in LDS
  __shared__ KStage<D> k_stage[kTileInPage && kKRows<D> ? kMaxWaves : 1];
  auto process = [&](const Tile<D>& cur, int t0) {
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
    if constexpr (kTileInPage && kKRows<D>) {
      u16x8 ka[kSteps];
      k_operands_from_rows<D>(k_stage[wave], cur, ka);
#pragma unroll
      for (int ks = 0; ks < kSteps; ++ks) s = T::mma_k32(ka[ks], qb[ks], s);
    } else {
#pragma unroll
      for (int ks = 0; ks < kSteps; ++ks) s = T::mma_k32(cur.k[ks], qb[ks], s);
    }
    float sv[4];
    if (t0 + 16 <= t_end) {
#pragma unroll
      for (int j = 0; j < 4; ++j) sv[j] = s[j] * p.scale_log2;
    } else {  // the chunk's partial last tile
#pragma unroll
      for (int j = 0; j < 4; ++j) sv[j] = (t0 + 4 * gq + j < t_end) ? s[j] * p.scale_log2 : -INFINITY;
    }
    float mx = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
    mx = rows_max(mx);
    if (__ballot(mx > m_run + kRescaleSlack)) {
      const float m_new = fmaxf(m_run, mx);
      const float alpha = fast_exp2(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int n = 0; n < NT; ++n) o[n] *= alpha;
      m_run = m_new;
    }
    float pj[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) pj[j] = fast_exp2(sv[j] - m_run);
    l_run += (pj[0] + pj[1]) + (pj[2] + pj[3]);
    u16x4 pb;
#pragma unroll
    for (int j = 0; j < 4; ++j) pb[j] = T::from_f32(pj[j]);
    u16x4 pb_lo;
    if constexpr (kSplitP) {
#pragma unroll
      for (int j = 0; j < 4; ++j) pb_lo[j] = T::from_f32(pj[j] - T::to_f32(pb[j]));
    }
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      u16x4 a = {cur.v[0][n], cur.v[1][n], cur.v[2][n], cur.v[3][n]};
      o[n] = T::mma_k16(a, pb, o[n]);
      if constexpr (kSplitP) o[n] = T::mma_k16(a, pb_lo, o[n]);
    }
  };

  // Software pipeline over the chunk's 16-token tiles: tile i+kDepth-1 is loaded
  // while tile i is computed. Loads are issued unconditionally (past the end the
  // last tile is issued again, an L2 hit) so the compiler's wait counts stay exact
  // and no wait drains the prefetched tiles.
  const int n_tiles = (t_end - t_begin + 15) >> 4;
  auto pipeline = [&](auto stream_tag) {
    constexpr bool kStream = decltype(stream_tag)::value;
    Tile<D> buf[kDepth];
    if constexpr (kTileInPage) {
      // Every tile lies inside one page. The ids of a window of 128 pages sit one per
      // lane in two registers and each tile's id is broadcast to a scalar register
      // (readlane), so page lookups never wait behind the K/V loads in flight; a chunk
      // longer than the window refills it once per 128 pages.
      const int ps = p.page_size;
      const int row_bytes = p.num_kv_heads * D * 2;
      const char* kpool = reinterpret_cast<const char*>(p.k_pool) + h * D * 2;
      const char* vpool = reinterpret_cast<const char*>(p.v_pool) + h * D * 2;
      const int first_page = t_begin / ps;
      int win_lo = 0, win_hi = 0;  // window = pages [first_page + win_base, +128)
      int win_base = 0;
      auto load_window = [&]() {
        const int pg0 = first_page + win_base + lane;
        int a = pg0 < np_seq ? idx[pg0] : 0;
        int c = pg0 + 64 < np_seq ? idx[pg0 + 64] : 0;
        win_lo = (a < 0 || (int64_t)a >= p.num_pages) ? 0 : a;
        win_hi = (c < 0 || (int64_t)c >= p.num_pages) ? 0 : c;
      };
      load_window();
      int ld_tile = 0;
      int page_ld = 0;  // page of the next tile, relative to first_page
      int slot_ld = t_begin - first_page * ps;
      const char* kb = kpool;
      const char* vb = vpool;
      int last = 0;
      auto issue = [&](Tile<D>& dst) {
        if (ld_tile < n_tiles) {
          if (page_ld - win_base == 128) {
            win_base += 128;
            load_window();
          }
          const int j = page_ld - win_base;
          const int pid = j < 64 ? __builtin_amdgcn_readlane(win_lo, j) : __builtin_amdgcn_readlane(win_hi, j - 64);
          const int64_t row0 = (int64_t)pid * ps + slot_ld;
          kb = kpool + row0 * row_bytes;
          vb = vpool + row0 * row_bytes;
          last = min(15, t_last - (t_begin + 16 * ld_tile));
          slot_ld += 16;
          if (slot_ld == ps) {
            slot_ld = 0;
            ++page_ld;
          }
          ++ld_tile;
        } else {
          // past the chunk's end: the issue only keeps the wait counts exact and its
          // tile is never computed, so every lane reads the last tile's first row
          // (512 B per wave, not the whole 8 KB tile again)
          last = 0;
        }
        load_tile_rows<D, kStream>(kb, vb, row_bytes, last, dst);
      };
  #pragma unroll
      for (int j = 0; j < kDepth - 1; ++j) issue(buf[j]);
      for (int i = 0; i < n_tiles; i += kDepth) {
  #pragma unroll
        for (int j = 0; j < kDepth; ++j) {
          if (i + j >= n_tiles) break;
          issue(buf[(j + kDepth - 1) % kDepth]);
          // keep the prefetch ahead of this tile's math (the scheduler would otherwise
          // sink the loads below the first MFMAs)
          __builtin_amdgcn_sched_barrier(0);
          process(buf[j], t_begin + 16 * (i + j));
        }
      }
    } else {
      const int head_off = h * D;
      auto issue_any = [&](int tile, Tile<D>& dst) {
        load_tile_any<D, kStream>(p, idx, head_off, t_begin + 16 * min(tile, n_tiles - 1), t_last, dst);
      };
  #pragma unroll
      for (int j = 0; j < kDepth - 1; ++j) issue_any(j, buf[j]);
      for (int i = 0; i < n_tiles; i += kDepth) {
  #pragma unroll
        for (int j = 0; j < kDepth; ++j) {
          if (i + j >= n_tiles) break;
          issue_any(i + j + kDepth - 1, buf[(j + kDepth - 1) % kDepth]);
          __builtin_amdgcn_sched_barrier(0);
          process(buf[j], t_begin + 16 * (i + j));
        }
      }
    }
  };
  bool stream = p.stream != 0;
  if constexpr (kGrouped) stream = stream && g < 0;  // a group's prefix: read by every group sharing it
  if (stream)
    pipeline(std::true_type{});
  else
    pipeline(std::false_type{});

  const float l_tot = rows_sum(l_run);
  if (!head_ok) return;

  // Lane l holds O[column r][d = NT*(4*gq + i) + n] in o[n][i].
  if (nchunks == 1 && g < 0 && !merged) {
    const float inv = 1.f / l_tot;
    uint16_t* orow = p.out + (int64_t)b * p.out_stride + (int64_t)hq * D;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      typename RowVec<NT>::type w;
#pragma unroll
      for (int n = 0; n < NT; ++n) w[n] = T::from_f32(o[n][i] * inv);
      *reinterpret_cast<typename RowVec<NT>::type*>(orow + NT * (4 * gq + i)) = w;
    }
  } else {
    const int64_t slot = ((int64_t)chunk * p.slot_members + member) * p.num_qo_heads + hq;
    float* prow = p.part_o + slot * D;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int n4 = 0; n4 < NT; n4 += 4) {
        f32x4 w = {o[n4][i], o[n4 + 1][i], o[n4 + 2][i], o[n4 + 3][i]};
        *reinterpret_cast<f32x4*>(prow + NT * (4 * gq + i) + n4) = w;
      }
    }
    if (gq == 0) {
      float2 ml = make_float2(m_run, l_tot);
      *reinterpret_cast<float2*>(p.part_ml + slot * 2) = ml;
    }
  }
}

struct MergeParams {
  const int32_t* indptr;
  const int32_t* last_len;
  int32_t batch;
  int32_t page_size;
  int32_t num_qo_heads;
  const int2* meta;  // per sequence: first chunk, chunk count, from the decode launch
  int32_t max_chunks;
  int32_t slot_members;
  const float* part_o;
  const float* part_ml;
  uint16_t* out;
  int64_t out_stride;
};

// Merge of the split-K partials: one wave per (sequence, query head), or, when the
// sequences average more than kSplitMergeChunks partials, one workgroup of 4 waves
// per (sequence, query head), each wave over a quarter of the partials. Sequences with several partials
// (chunks of their own tokens, and of their group's prefix) are merged; empty
// sequences get zero rows; sequences with a single chunk and no group were finished
// by the decode kernel. A wave reads the sequence's chunk range (one round of
// loads), then its partials' (m, l) with lanes over partials and the first rows of
// O with lanes over (partial, d) in one more round: O row c is D floats, D/4 lanes
// read it as float4s, 64/(D/4) rows per load. The four waves' (m, l, O), each
// relative to its own max, are combined through LDS by the first wave. Splitting a
// sequence's partials over 4 waves shortens the chain of dependent load rounds for
// sequences with many chunks (small batches: ~100 chunks each; measured 6.5 -> 4.2
// us at 4 sequences), and costs more than it saves at a few chunks each (5.3 ->
// 8.8 us at 64 sequences of ~6 chunks).
constexpr int kSplitMergeChunks = 32;
template <typename T, int D, bool kGrouped, bool kSplit>
__global__ void __launch_bounds__(256) decode_merge_kernel(MergeParams p, GroupArgs<kGrouped> ga) {
  constexpr int LPC = D / 4;     // lanes per O row
  constexpr int CPI = 64 / LPC;  // O rows per load instruction
  constexpr int kBatch = 8;      // load instructions per lane in flight
  constexpr int kParts = 4;      // kSplit: waves per (sequence, query head), a quarter of the chunks each
  __shared__ float s_m[kParts], s_l[kParts];
  __shared__ __attribute__((aligned(16))) float s_o[kParts][D];
  const int b = blockIdx.x;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  // kSplit: the workgroup's 4 waves share one query head; else each wave has its own
  const int hq = kSplit ? blockIdx.y : blockIdx.y * 4 + wave;
  if (!kSplit && hq >= p.num_qo_heads) return;
  const int len = seq_len_of(p.indptr, p.last_len, b, p.page_size);
  const int2 mt = p.meta[b];
  const int sub = lane / LPC;
  const int d0 = 4 * (lane % LPC);
  uint16_t* orow = p.out + (int64_t)b * p.out_stride + (int64_t)hq * D + d0;
  if (len == 0) {
    // A sequence with no tokens attends to nothing: its output rows are zero.
    if ((!kSplit || wave == 0) && sub == 0) *reinterpret_cast<u16x4*>(orow) = u16x4{0, 0, 0, 0};
    return;
  }
  // own chunks [cstart, cstart + nown) at member slot 0; the group prefix's chunks
  // [gstart, gstart + ngrp) at the sequence's member slot
  int own = len, member = 0, gstart = 0, ngrp = 0;
  if constexpr (kGrouped) {
    const int gs = ga.seq_group_slot[b];
    const int g = gs >> 4;
    if (gs >= 0 && g < ga.num_groups && (gs & 15) < p.slot_members) {
      own = len - min(ga.prefix_pages[g] * p.page_size, len);
      const int2 gm = ga.group_meta[g];
      member = gs & 15;
      gstart = gm.x;
      ngrp = gm.y;
      if (gstart < 0 || gstart >= p.max_chunks || ngrp < 0) ngrp = 0;
      if (gstart + ngrp > p.max_chunks) ngrp = p.max_chunks - gstart;
    }
  }
  const int cstart = mt.x;
  int nown = own > 0 ? mt.y : 0;
  if (nown > 0 && (cstart < 0 || cstart >= p.max_chunks)) nown = 0;
  if (cstart + nown > p.max_chunks) nown = p.max_chunks - cstart;
  if (ngrp == 0 && nown <= 1) return;  // uniform over the workgroup
  const int nchunks = nown + ngrp;

  // partial k of the sequence -> its slot
  auto slot_of = [&](int k) -> int64_t {
    const int64_t ck = k < nown ? (int64_t)(cstart + k) * p.slot_members
                                : (int64_t)(gstart + k - nown) * p.slot_members + member;
    return ck * p.num_qo_heads + hq;
  };
  // this wave's chunks [k0, k0 + cnt)
  const int per = kSplit ? (nchunks + kParts - 1) / kParts : nchunks;
  const int k0 = kSplit ? wave * per : 0;
  const int cnt = min(nchunks, k0 + per) - k0;

  float mmax = -INFINITY, lsum = 0.f;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  if (cnt > 0) {
    f32x4 oc[kBatch];
    float mc[kBatch];
    auto load_rows = [&](int c0) {
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        const int64_t sl = slot_of(k0 + min(c0 + CPI * k + sub, cnt - 1));
        oc[k] = *reinterpret_cast<const f32x4*>(p.part_o + sl * D + d0);
        mc[k] = p.part_ml[sl * 2];
      }
    };
    load_rows(0);  // in flight with the (m, l) pass below

    // the running max M and the denominator sum_c 2^(m_c - M) l_c, lanes over chunks
    for (int c = lane; c < cnt; c += 64) {
      const float2 v = *reinterpret_cast<const float2*>(p.part_ml + slot_of(k0 + c) * 2);
      const float m_new = fmaxf(mmax, v.x);
      lsum = lsum * fast_exp2(mmax - m_new) + v.y * fast_exp2(v.x - m_new);
      mmax = m_new;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      const float om = __shfl_xor(mmax, off, 64);
      const float ol = __shfl_xor(lsum, off, 64);
      const float m_new = fmaxf(mmax, om);
      lsum = (mmax == -INFINITY ? 0.f : lsum * fast_exp2(mmax - m_new)) +
             (om == -INFINITY ? 0.f : ol * fast_exp2(om - m_new));
      mmax = m_new;
    }

    // sum_c 2^(m_c - M) O_c over the lane's rows, then over the CPI rows of a load
    for (int c0 = 0; c0 < cnt; c0 += CPI * kBatch) {
      if (c0 > 0) load_rows(c0);
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        const float w = c0 + CPI * k + sub < cnt ? fast_exp2(mc[k] - mmax) : 0.f;
        acc += w * oc[k];
      }
    }
#pragma unroll
    for (int off = LPC; off < 64; off <<= 1) {
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[j] += __shfl_xor(acc[j], off, 64);
    }
  }
  if constexpr (!kSplit) {
    if (sub == 0) {
      const float inv = 1.f / lsum;
      u16x4 w16;
#pragma unroll
      for (int j = 0; j < 4; ++j) w16[j] = T::from_f32(acc[j] * inv);
      *reinterpret_cast<u16x4*>(orow) = w16;
    }
    return;
  }
  if (lane == 0) {
    s_m[wave] = mmax;
    s_l[wave] = lsum;
  }
  if (sub == 0) *reinterpret_cast<f32x4*>(&s_o[wave][d0]) = acc;
  __syncthreads();
  if (wave == 0 && sub == 0) {
    // the waves' parts, each relative to its own max: rescale to the common one
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kParts; ++w) M = fmaxf(M, s_m[w]);
    float L = 0.f;
    f32x4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < kParts; ++w) {
      if (s_m[w] == -INFINITY) continue;
      const float f = fast_exp2(s_m[w] - M);
      L += f * s_l[w];
      o += f * *reinterpret_cast<const f32x4*>(&s_o[w][d0]);
    }
    const float inv = 1.f / L;
    u16x4 w16;
#pragma unroll
    for (int j = 0; j < 4; ++j) w16[j] = T::from_f32(o[j] * inv);
    *reinterpret_cast<u16x4*>(orow) = w16;
  }
}

// Resident workgroup slots of the decode kernel on the current device (CUs x
// workgroups per CU at its register footprint), cached per device and variant.
// Without a device (a host-only process sizing a workspace) the MI355X figure
// is used: 256 CUs x 3 workgroups of 4 waves.
constexpr int kMaxDevices = 64;
constexpr int kDefaultSlots = 768;

// Whether a call may be inside a stream capture (a launch on `stream`), and the stream.
struct CaptureCheck {
  bool check = false;
  hipStream_t stream = nullptr;
};

inline bool stream_capturing(hipStream_t s) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &st) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  return st != hipStreamCaptureStatusNone;
}

// Calls whose K/V (both, all KV heads) exceed this stream them with non-temporal
// loads; smaller ones are left in the caches (MI355X: 256 MB of memory-side cache).
constexpr int64_t kStreamBytes = (int64_t)128 << 20;

// The first call of a variant on a device queries the device (attribute and
// occupancy); a call whose stream is being captured into a graph must not make
// those queries, so it returns 0 (refused) when the figure is not cached yet.
template <typename T, int D, bool kTileInPage, bool kGrouped>
int decode_wg_slots(int waves, const CaptureCheck& cc) {
  static std::atomic<int> cache[kMaxDevices][kMaxWaves + 1];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    (void)hipGetLastError();
    return kDefaultSlots;
  }
  int v = cache[dev][waves].load(std::memory_order_relaxed);
  if (v > 0) return v;
  if (cc.check && stream_capturing(cc.stream)) return 0;
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, paged_decode_kernel<T, D, kTileInPage, 2, kGrouped>,
                                                   64 * waves, 0) != hipSuccess ||
      cus <= 0 || per_cu <= 0) {
    (void)hipGetLastError();
    return kDefaultSlots;
  }
  v = cus * per_cu;
  cache[dev][waves].store(v, std::memory_order_relaxed);
  return v;
}

struct DecodeShape {
  bool refused = false;  // the variant's first use happened inside a stream capture
  int waves;         // waves (KV heads) per workgroup
  int head_groups;   // workgroups per chunk
  int chunk_tokens;  // upper bound passed to the kernel
  int chunk_budget;  // 0: no device-side search
  int64_t max_chunks;
};

// Chunk length for `total_tokens` (an upper bound of the units' tokens) over
// `units` work units (sequences, plus group prefixes). Unit u gets
// ceil(L_u / len) chunks, at most total / len + units in all, so
// len = total / (capacity - units) keeps every chunk of the grid resident at
// once; the kernel then lowers it to the smallest length that still fits
// `capacity` chunks for the actual lengths. Too many units for that
// (capacity <= 2 * units) get about `capacity` chunks per round at the host's
// length. Lengths are multiples of 16 (tiles never straddle a chunk) and at
// least 64.
template <typename T, int D, bool kGrouped>
DecodeShape decode_shape(int32_t units, int32_t num_kv_heads, int64_t total_tokens, int page_size,
                         const CaptureCheck& cc) {
  DecodeShape sh;
  sh.waves = num_kv_heads < kMaxWaves ? num_kv_heads : kMaxWaves;
  sh.head_groups = (num_kv_heads + sh.waves - 1) / sh.waves;
  const int slots = page_size % 16 == 0 ? decode_wg_slots<T, D, true, kGrouped>(sh.waves, cc)
                                        : decode_wg_slots<T, D, false, kGrouped>(sh.waves, cc);
  if (slots <= 0) {  // refused: first use of the variant inside a stream capture
    sh.refused = true;
    return sh;
  }
  int64_t capacity = slots / sh.head_groups;
  if (capacity < 1) capacity = 1;
  const bool fit = capacity > 2 * (int64_t)units;
  const int64_t usable = fit ? capacity - units : capacity;
  int64_t c = (total_tokens + usable - 1) / usable;
  c = ((c + 15) / 16) * 16;
  if (c < 64) c = 64;
  if (c > ((int64_t)1 << 30)) c = (int64_t)1 << 30;
  sh.chunk_tokens = (int)c;
  sh.chunk_budget = fit ? (int)capacity : 0;
  sh.max_chunks = fit ? capacity : (total_tokens + c - 1) / c + units;
  return sh;
}

template <typename T, bool kGrouped>
DecodeShape decode_shape_for(int32_t head_dim, int32_t units, int32_t num_kv_heads, int64_t total_tokens,
                             int page_size, const CaptureCheck& cc) {
  switch (head_dim) {
    case 64: return decode_shape<T, 64, kGrouped>(units, num_kv_heads, total_tokens, page_size, cc);
    case 128: return decode_shape<T, 128, kGrouped>(units, num_kv_heads, total_tokens, page_size, cc);
    default: return decode_shape<T, 256, kGrouped>(units, num_kv_heads, total_tokens, page_size, cc);
  }
}

template <bool kGrouped>
DecodeShape shape_of(int32_t dtype, int32_t head_dim, int32_t units, int32_t num_kv_heads, int64_t total_tokens,
                     int page_size, const CaptureCheck& cc = CaptureCheck{}) {
  return dtype == NSLG_BF16
             ? decode_shape_for<BF16, kGrouped>(head_dim, units, num_kv_heads, total_tokens, page_size, cc)
             : decode_shape_for<F16, kGrouped>(head_dim, units, num_kv_heads, total_tokens, page_size, cc);
}

template <typename T, int D, bool kGrouped>
int launch_decode(const DecodeParams& p, const MergeParams& mp, const GroupArgs<kGrouped>& ga, int waves,
                  hipStream_t s) {
  const dim3 grid((unsigned)p.max_chunks, (unsigned)p.head_groups);
  if (p.page_size % 16 == 0)
    paged_decode_kernel<T, D, true, 2, kGrouped><<<grid, 64 * waves, 0, s>>>(p, ga);
  else
    paged_decode_kernel<T, D, false, 2, kGrouped><<<grid, 64 * waves, 0, s>>>(p, ga);
  int rc = check_launch("paged_decode");
  if (rc) return rc;
  // sequences of many chunks (small batches) split their partials over 4 waves
  if (p.max_chunks > kSplitMergeChunks * p.batch)
    decode_merge_kernel<T, D, kGrouped, true><<<dim3(p.batch, p.num_qo_heads), 256, 0, s>>>(mp, ga);
  else
    decode_merge_kernel<T, D, kGrouped, false><<<dim3(p.batch, (p.num_qo_heads + 3) / 4), 256, 0, s>>>(mp, ga);
  return check_launch("paged_decode_merge");
}

// New rows of an fp32 decode call (whose attention kernel has no folded write):
// grid (batch, 2), workgroup b writes sequence b's K (y = 0) or V (y = 1) row as
// its token L_b - 1, the slot found through its block table. 4-byte words.
__global__ void __launch_bounds__(256)
write_last_rows_kernel(const uint32_t* __restrict__ k_new, const uint32_t* __restrict__ v_new,
                       int64_t k_stride_words, int64_t v_stride_words, const int32_t* __restrict__ indptr,
                       const int32_t* __restrict__ indices, const int32_t* __restrict__ last_len,
                       int32_t page_size, int64_t num_pages, int32_t row_words, uint32_t* __restrict__ k_pool,
                       uint32_t* __restrict__ v_pool) {
  const int b = blockIdx.x;
  const int len = seq_len_of(indptr, last_len, b, page_size);
  if (len <= 0) return;
  const int tok = len - 1;
  const int pid = indices[indptr[b] + tok / page_size];
  if (pid < 0 || (int64_t)pid >= num_pages) return;
  const bool is_v = blockIdx.y != 0;
  const uint32_t* src = is_v ? v_new + (int64_t)b * v_stride_words : k_new + (int64_t)b * k_stride_words;
  uint32_t* dst = (is_v ? v_pool : k_pool) + ((int64_t)pid * page_size + tok % page_size) * row_words;
  for (int i = threadIdx.x; i < row_words; i += blockDim.x) dst[i] = src[i];
}

inline size_t round256(size_t x) { return (x + 255) & ~(size_t)255; }

// Workspace: partials [max_chunks, slot_members, Hq, D] and [..., 2] fp32, then each
// sequence's chunk range, then each group prefix's chunk range (int32 pairs), then
// the recorded chunk layout (a 16-byte tag, then two int4 per chunk), each region
// rounded up to 256 bytes.
size_t workspace_bytes_for(const DecodeShape& sh, int32_t batch, int32_t num_qo_heads, int32_t head_dim,
                           int32_t slot_members, int32_t num_groups) {
  return (size_t)(sh.max_chunks * slot_members * num_qo_heads * (head_dim + 2) * (int64_t)sizeof(float)) +
         round256((size_t)batch * 8) + (num_groups > 0 ? round256((size_t)num_groups * 8) : 0) +
         round256(16 + (size_t)sh.max_chunks * 32);
}

bool shape_ok(int32_t batch, int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim, int64_t total_pages,
              int32_t page_size) {
  return batch > 0 && num_qo_heads > 0 && num_kv_heads > 0 && total_pages >= 0 && page_size > 0 &&
         num_qo_heads % num_kv_heads == 0 && (head_dim == 64 || head_dim == 128 || head_dim == 256);
}

// The new rows of an append-and-decode call (k = v = null: a decode call alone).
struct NewRows {
  const void* k = nullptr;
  const void* v = nullptr;
  int64_t k_stride = 0;  // elements between batch rows
  int64_t v_stride = 0;
  // rotary embedding of q and the new K rows (cos null: none)
  const int32_t* pos = nullptr;
  const float* cos = nullptr;
  const float* sin = nullptr;
  int64_t table_stride = 0;  // floats between table rows
  int64_t table_rows = 0;
};

template <bool kGrouped>
int decode_impl(const void* q, int64_t q_stride, const void* k_pool, const void* v_pool, int64_t num_pages,
                int32_t page_size, const int32_t* kv_indptr, const int32_t* kv_indices,
                const int32_t* kv_last_page_len, int64_t total_pages, int32_t batch, int32_t num_qo_heads,
                int32_t num_kv_heads, int32_t head_dim, float sm_scale, int32_t dtype, void* out,
                int64_t out_stride, GroupArgs<kGrouped>& ga, int32_t num_groups, int32_t slot_members,
                void* workspace, size_t workspace_bytes, nslg_stream_t stream, const NewRows& nr = NewRows{},
                int64_t layout = 0) {
  if (batch < 0 || num_qo_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || page_size <= 0 ||
      num_pages <= 0 || total_pages < 0)
    return fail(NSLG_EINVAL, "paged_decode: bad sizes");
  if (batch == 0) return NSLG_OK;
  if (!q || !k_pool || !v_pool || !kv_indptr || !kv_indices || !kv_last_page_len || !out)
    return fail(NSLG_EINVAL, "paged_decode: null pointer");
  if (num_qo_heads % num_kv_heads != 0)
    return fail(NSLG_EINVAL, "paged_decode: Hq=%d not a multiple of Hkv=%d", num_qo_heads, num_kv_heads);
  if (nr.k || nr.v) {
    const int eb = dtype == NSLG_F32 ? 4 : 2;
    const int64_t row = (int64_t)num_kv_heads * head_dim;
    if (!nr.k || !nr.v) return fail(NSLG_EINVAL, "paged_decode_append: null k_new or v_new");
    if (batch > 1 && (nr.k_stride < row || nr.v_stride < row))
      return fail(NSLG_EINVAL, "paged_decode_append: new rows overlap (strides %lld, %lld < Hkv*D = %lld)",
                  (long long)nr.k_stride, (long long)nr.v_stride, (long long)row);
    const int64_t align = dtype == NSLG_F32 ? 4 : 16;
    if ((int64_t)((uintptr_t)nr.k % align) || (int64_t)((uintptr_t)nr.v % align) || (nr.k_stride * eb) % align ||
        (nr.v_stride * eb) % align)
      return fail(NSLG_EINVAL, "paged_decode_append: new rows must be %lld-byte aligned", (long long)align);
  }
  if (nr.cos) {
    if (!nr.k || !nr.sin || !nr.pos) return fail(NSLG_EINVAL, "paged_decode_rope_append: null table, positions or rows");
    if (dtype == NSLG_F32)
      return fail(NSLG_EUNSUPPORTED, "paged_decode_rope_append: f16/bf16 pools (f32: nslg_rope_append, then decode)");
    if (nr.table_rows <= 0 || nr.table_stride < head_dim)
      return fail(NSLG_EINVAL, "paged_decode_rope_append: tables of %lld rows at stride %lld for head_dim %d",
                  (long long)nr.table_rows, (long long)nr.table_stride, head_dim);
    if (((uintptr_t)nr.cos | (uintptr_t)nr.sin) & 15 || (nr.table_stride * 4) % 16)
      return fail(NSLG_EINVAL, "paged_decode_rope_append: table rows must be 16-byte aligned");
  }
  const int group = num_qo_heads / num_kv_heads;
  if (group > 16) return fail(NSLG_EUNSUPPORTED, "paged_decode: GQA group %d > 16", group);
  if (num_qo_heads > 65535) return fail(NSLG_EUNSUPPORTED, "paged_decode: %d query heads", num_qo_heads);
  if (dtype == NSLG_F32) {
    // fp32 pools: one query row per sequence through the fp32 attention kernel
    if constexpr (kGrouped) {
      return fail(NSLG_EUNSUPPORTED, "paged_decode_grouped: f16/bf16 only");
    } else {
      if (head_dim != 64 && head_dim != 128 && head_dim != 256)
        return fail(NSLG_EUNSUPPORTED, "paged_decode: head_dim %d", head_dim);
      if (q_stride < (int64_t)num_qo_heads * head_dim || out_stride < (int64_t)num_qo_heads * head_dim)
        return fail(NSLG_EINVAL, "paged_decode: row stride smaller than Hq*D");
      AttnF32Args a;
      a.q = (const float*)q;
      a.q_stride = q_stride;
      a.qo_indptr = nullptr;
      a.k_pool = (const float*)k_pool;
      a.v_pool = (const float*)v_pool;
      a.num_pages = num_pages;
      a.page_size = page_size;
      a.indptr = kv_indptr;
      a.indices = kv_indices;
      a.last_len = kv_last_page_len;
      a.batch = batch;
      a.num_qo_heads = num_qo_heads;
      a.num_kv_heads = num_kv_heads;
      a.group = group;
      a.scale = sm_scale;
      a.out = (float*)out;
      a.out_stride = out_stride;
      a.row_tiles = 0;
      // long sequences are split over keys; the partials go to the workspace
      a.splits = attention_f32_splits(batch, total_pages * (int64_t)page_size);
      a.part_o = nullptr;
      a.part_ml = nullptr;
      if (a.splits > 1) {
        const size_t need = attention_f32_workspace(batch, num_qo_heads, head_dim, a.splits);
        if (!workspace || workspace_bytes < need)
          return fail(NSLG_EWORKSPACE, "paged_decode: workspace %zu < %zu bytes", workspace_bytes, need);
        if (((uintptr_t)workspace) & 255) return fail(NSLG_EINVAL, "paged_decode: workspace must be 256-byte aligned");
        a.part_o = (float*)workspace;
        a.part_ml = a.part_o + (int64_t)batch * num_qo_heads * a.splits * head_dim;
      }
      if (nr.k) {
        const int row_words = num_kv_heads * head_dim;
        write_last_rows_kernel<<<dim3(batch, 2), row_words < 256 ? 64 : 256, 0, as_stream(stream)>>>(
            (const uint32_t*)nr.k, (const uint32_t*)nr.v, nr.k_stride, nr.v_stride, kv_indptr, kv_indices,
            kv_last_page_len, page_size, num_pages, row_words, (uint32_t*)k_pool, (uint32_t*)v_pool);
        const int rc = check_launch("paged_decode_append (rows)");
        if (rc) return rc;
      }
      return attention_f32(a, batch, head_dim, as_stream(stream));
    }
  }
  if (dtype != NSLG_F16 && dtype != NSLG_BF16)
    return fail(NSLG_EUNSUPPORTED, "paged_decode: dtype %d", dtype);
  if (head_dim != 64 && head_dim != 128 && head_dim != 256)
    return fail(NSLG_EUNSUPPORTED, "paged_decode: head_dim %d", head_dim);
  if (q_stride < (int64_t)num_qo_heads * head_dim || out_stride < (int64_t)num_qo_heads * head_dim)
    return fail(NSLG_EINVAL, "paged_decode: row stride smaller than Hq*D");
  if (((uintptr_t)q | (uintptr_t)k_pool | (uintptr_t)v_pool | (uintptr_t)out) & 15 ||
      (q_stride * 2) % 16 || (out_stride * 2) % 16)
    return fail(NSLG_EINVAL, "paged_decode: q/pool/out must be 16-byte aligned");
  const int64_t total_tokens = total_pages * page_size;
  if (total_tokens >= (int64_t)1 << 31) return fail(NSLG_EUNSUPPORTED, "paged_decode: >2^31 tokens");
  CaptureCheck cc;
  cc.check = true;
  cc.stream = as_stream(stream);
  const DecodeShape sh =
      shape_of<kGrouped>(dtype, head_dim, batch + num_groups, num_kv_heads, total_tokens, page_size, cc);
  if (sh.refused)
    return fail(NSLG_ECAPTURE,
                "paged_decode: first call of this variant (dtype %d, head_dim %d, page_size %d) is inside a "
                "stream capture; make one call, or a workspace-size query, outside the capture first",
                dtype, head_dim, page_size);
  const int64_t mc = sh.max_chunks;
  const size_t need = workspace_bytes_for(sh, batch, num_qo_heads, head_dim, slot_members, num_groups);
  if (!workspace || workspace_bytes < need)
    return fail(NSLG_EWORKSPACE, "paged_decode: workspace %zu < %zu bytes", workspace_bytes, need);
  if (((uintptr_t)workspace) & 255) return fail(NSLG_EINVAL, "paged_decode: workspace must be 256-byte aligned");

  DecodeParams p;
  p.q = (const uint16_t*)q;
  p.q_stride = q_stride;
  p.k_pool = (const uint16_t*)k_pool;
  p.v_pool = (const uint16_t*)v_pool;
  p.num_pages = num_pages;
  p.page_size = page_size;
  p.indptr = kv_indptr;
  p.indices = kv_indices;
  p.last_len = kv_last_page_len;
  p.batch = batch;
  p.num_qo_heads = num_qo_heads;
  p.num_kv_heads = num_kv_heads;
  p.group = group;
  p.scale_log2 = sm_scale * 1.4426950408889634f;
  p.chunk_tokens = sh.chunk_tokens;
  p.chunk_budget = sh.chunk_budget;
  p.max_chunks = (int32_t)mc;
  p.head_groups = sh.head_groups;
  p.out = (uint16_t*)out;
  p.out_stride = out_stride;
  p.slot_members = slot_members;
  // distinct K/V tokens of the call: the members' own tokens and, since the groups of
  // a batch usually share one cached prompt, the longest group prefix once
  int64_t distinct_tokens = total_tokens;
  if constexpr (kGrouped) {
    int64_t longest = 0;
    for (int g = 0; g < num_groups; ++g) {
      int members = 0;
      for (int m = 0; m < kGroupCols; ++m) members += ga.member_seq[g * kGroupCols + m] >= 0 ? 1 : 0;
      const int64_t prefix = (int64_t)ga.prefix_pages[g] * page_size;
      distinct_tokens -= members * prefix;
      longest = prefix > longest ? prefix : longest;
    }
    distinct_tokens += longest;
  }
  p.stream = distinct_tokens * num_kv_heads * head_dim * 2 * 2 > kStreamBytes ? 1 : 0;
  p.k_new = (const uint16_t*)nr.k;
  p.v_new = (const uint16_t*)nr.v;
  p.k_new_stride = nr.k_stride;
  p.v_new_stride = nr.v_stride;
  p.rope_pos = nr.pos;
  p.rope_cos = nr.cos;
  p.rope_sin = nr.sin;
  p.rope_stride = nr.table_stride;
  p.rope_rows = nr.table_rows;
  char* ws = (char*)workspace;
  p.part_o = (float*)ws;
  p.part_ml = p.part_o + mc * slot_members * num_qo_heads * head_dim;
  char* meta = ws + (size_t)(mc * slot_members * num_qo_heads * (head_dim + 2) * (int64_t)sizeof(float));
  p.meta = reinterpret_cast<int2*>(meta);
  if constexpr (kGrouped) ga.group_meta = reinterpret_cast<int2*>(meta + round256((size_t)batch * 8));
  char* lay = meta + round256((size_t)batch * 8) + (num_groups > 0 ? round256((size_t)num_groups * 8) : 0);
  p.layout_mode = layout > 0 ? 1 : (layout < 0 ? -1 : 0);
  p.layout_tag = (uint64_t)(layout > 0 ? layout : -layout);
  p.layout_tag_ptr = reinterpret_cast<uint64_t*>(lay);
  p.layout_map = reinterpret_cast<int4*>(lay + 16);
  p.total_pages = total_pages;

  MergeParams mp;
  mp.indptr = kv_indptr;
  mp.last_len = kv_last_page_len;
  mp.batch = batch;
  mp.page_size = page_size;
  mp.num_qo_heads = num_qo_heads;
  mp.meta = p.meta;
  mp.max_chunks = (int32_t)mc;
  mp.slot_members = slot_members;
  mp.part_o = p.part_o;
  mp.part_ml = p.part_ml;
  mp.out = p.out;
  mp.out_stride = out_stride;

  hipStream_t s = as_stream(stream);
  if (dtype == NSLG_F16) {
    switch (head_dim) {
      case 64: return launch_decode<F16, 64, kGrouped>(p, mp, ga, sh.waves, s);
      case 128: return launch_decode<F16, 128, kGrouped>(p, mp, ga, sh.waves, s);
      default: return launch_decode<F16, 256, kGrouped>(p, mp, ga, sh.waves, s);
    }
  }
  switch (head_dim) {
    case 64: return launch_decode<BF16, 64, kGrouped>(p, mp, ga, sh.waves, s);
    case 128: return launch_decode<BF16, 128, kGrouped>(p, mp, ga, sh.waves, s);
    default: return launch_decode<BF16, 256, kGrouped>(p, mp, ga, sh.waves, s);
  }
}

}  // namespace
}  // namespace nslg

using namespace nslg;

extern "C" size_t nslg_paged_decode_workspace_size(int32_t batch, int32_t num_qo_heads,
                                                   int32_t num_kv_heads, int32_t head_dim,
                                                   int64_t total_pages, int32_t page_size,
                                                   int32_t dtype) {
  if (!shape_ok(batch, num_qo_heads, num_kv_heads, head_dim, total_pages, page_size)) return 0;
  if (dtype == NSLG_F32)  // partials of the key splits of the fp32 path
    return attention_f32_workspace(batch, num_qo_heads, head_dim,
                                   attention_f32_splits(batch, total_pages * (int64_t)page_size));
  const DecodeShape sh = shape_of<false>(dtype, head_dim, batch, num_kv_heads, total_pages * page_size, page_size);
  return workspace_bytes_for(sh, batch, num_qo_heads, head_dim, 1, 0);
}

extern "C" size_t nslg_paged_decode_grouped_workspace_size(int32_t batch, int32_t num_qo_heads,
                                                           int32_t num_kv_heads, int32_t head_dim,
                                                           int64_t total_pages, int32_t page_size,
                                                           int32_t dtype, int32_t num_groups) {
  if (!shape_ok(batch, num_qo_heads, num_kv_heads, head_dim, total_pages, page_size)) return 0;
  if (num_groups < 1 || num_groups > kMaxGroups) return 0;
  if (dtype == NSLG_F32) return 0;  // grouped decode runs on the 16-bit MFMA path only
  const int group = num_qo_heads / num_kv_heads;
  if (group > kGroupCols) return 0;
  const DecodeShape sh =
      shape_of<true>(dtype, head_dim, batch + num_groups, num_kv_heads, total_pages * page_size, page_size);
  return workspace_bytes_for(sh, batch, num_qo_heads, head_dim, kGroupCols / group, num_groups);
}

extern "C" int nslg_paged_decode(const void* q, int64_t q_stride, const void* k_pool,
                                 const void* v_pool, int64_t num_pages, int32_t page_size,
                                 const int32_t* kv_indptr, const int32_t* kv_indices,
                                 const int32_t* kv_last_page_len, int64_t total_pages,
                                 int32_t batch, int32_t num_qo_heads, int32_t num_kv_heads,
                                 int32_t head_dim, float sm_scale, int32_t dtype, void* out,
                                 int64_t out_stride, void* workspace, size_t workspace_bytes,
                                 int64_t layout, nslg_stream_t stream) {
  GroupArgs<false> ga;
  return decode_impl<false>(q, q_stride, k_pool, v_pool, num_pages, page_size, kv_indptr, kv_indices,
                            kv_last_page_len, total_pages, batch, num_qo_heads, num_kv_heads, head_dim, sm_scale,
                            dtype, out, out_stride, ga, 0, 1, workspace, workspace_bytes, stream, NewRows{},
                            layout);
}

// ---- decode without a caller workspace ---------------------------------------------
// The split-K partials and chunk ranges of nslg_paged_decode_noalloc live in this
// fixed device array instead of a caller's workspace. Every GPU the library runs on
// holds its own copy at its own address until the process ends. Host code never
// passes the array's name to a kernel: its device address is looked up once per
// device (hipGetSymbolAddress, with that device current) and used from then on.
static __device__ __align__(256) unsigned char scratch[NSLG_NOALLOC_SCRATCH_BYTES];

namespace {

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device (looked up on the first call
// made with that device current).
int scratch_of_current_device(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    (void)hipGetLastError();
    return fail(NSLG_EINVAL, "paged_decode_noalloc: no current device (or device %d >= %d)", dev, kMaxDevices);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      (void)hipGetLastError();
      return fail(NSLG_ELAUNCH, "paged_decode_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                  hipGetErrorString(e));
    }
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return NSLG_OK;
}

}  // namespace

extern "C" int nslg_paged_decode_noalloc(const void* q, int64_t q_stride, const void* k_pool,
                                         const void* v_pool, int64_t num_pages, int32_t page_size,
                                         const int32_t* kv_indptr, const int32_t* kv_indices,
                                         const int32_t* kv_last_page_len, int64_t total_pages,
                                         int32_t batch, int32_t num_qo_heads, int32_t num_kv_heads,
                                         int32_t head_dim, float sm_scale, int32_t dtype, void* out,
                                         int64_t out_stride, nslg_stream_t stream) {
  // Same scratch layout and size as nslg_paged_decode's workspace; nothing in it has
  // to start at zero (every chunk range and partial is written before it is read).
  const size_t need = nslg_paged_decode_workspace_size(batch, num_qo_heads, num_kv_heads, head_dim, total_pages,
                                                       page_size, dtype);
  if (need > (size_t)NSLG_NOALLOC_SCRATCH_BYTES)
    return fail(NSLG_EWORKSPACE,
                "paged_decode_noalloc: this call needs %zu bytes of scratch, more than the %zu-byte static "
                "scratch; call nslg_paged_decode with a workspace",
                need, (size_t)NSLG_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  const int rc = scratch_of_current_device(&ws);
  if (rc) return rc;
  GroupArgs<false> ga;
  return decode_impl<false>(q, q_stride, k_pool, v_pool, num_pages, page_size, kv_indptr, kv_indices,
                            kv_last_page_len, total_pages, batch, num_qo_heads, num_kv_heads, head_dim, sm_scale,
                            dtype, out, out_stride, ga, 0, 1, ws, (size_t)NSLG_NOALLOC_SCRATCH_BYTES, stream);
}

extern "C" int nslg_paged_decode_append(const void* q, int64_t q_stride, const void* k_new,
                                        int64_t k_new_stride, const void* v_new, int64_t v_new_stride,
                                        void* k_pool, void* v_pool, int64_t num_pages, int32_t page_size,
                                        const int32_t* kv_indptr, const int32_t* kv_indices,
                                        const int32_t* kv_last_page_len, int64_t total_pages,
                                        int32_t batch, int32_t num_qo_heads, int32_t num_kv_heads,
                                        int32_t head_dim, float sm_scale, int32_t dtype, void* out,
                                        int64_t out_stride, void* workspace, size_t workspace_bytes,
                                        int64_t layout, nslg_stream_t stream) {
  if (batch > 0 && (!k_new || !v_new)) return fail(NSLG_EINVAL, "paged_decode_append: null k_new or v_new");
  NewRows nr;
  nr.k = k_new;
  nr.v = v_new;
  nr.k_stride = k_new_stride;
  nr.v_stride = v_new_stride;
  GroupArgs<false> ga;
  return decode_impl<false>(q, q_stride, k_pool, v_pool, num_pages, page_size, kv_indptr, kv_indices,
                            kv_last_page_len, total_pages, batch, num_qo_heads, num_kv_heads, head_dim, sm_scale,
                            dtype, out, out_stride, ga, 0, 1, workspace, workspace_bytes, stream, nr, layout);
}

extern "C" int nslg_paged_decode_rope_append(
    const void* q, int64_t q_stride, const void* k_new, int64_t k_new_stride, const void* v_new,
    int64_t v_new_stride, const int32_t* positions, const float* cos_table, const float* sin_table,
    int64_t table_stride, int64_t table_rows, void* k_pool, void* v_pool, int64_t num_pages, int32_t page_size,
    const int32_t* kv_indptr, const int32_t* kv_indices, const int32_t* kv_last_page_len, int64_t total_pages,
    int32_t batch, int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim, float sm_scale, int32_t dtype,
    void* out, int64_t out_stride, void* workspace, size_t workspace_bytes, int64_t layout, nslg_stream_t stream) {
  if (batch > 0 && (!k_new || !v_new || !cos_table))
    return fail(NSLG_EINVAL, "paged_decode_rope_append: null k_new, v_new or tables");
  NewRows nr;
  nr.k = k_new;
  nr.v = v_new;
  nr.k_stride = k_new_stride;
  nr.v_stride = v_new_stride;
  nr.pos = positions;
  nr.cos = cos_table;
  nr.sin = sin_table;
  nr.table_stride = table_stride;
  nr.table_rows = table_rows;
  GroupArgs<false> ga;
  return decode_impl<false>(q, q_stride, k_pool, v_pool, num_pages, page_size, kv_indptr, kv_indices,
                            kv_last_page_len, total_pages, batch, num_qo_heads, num_kv_heads, head_dim, sm_scale,
                            dtype, out, out_stride, ga, 0, 1, workspace, workspace_bytes, stream, nr, layout);
}

namespace {

int grouped_impl(const void* q, int64_t q_stride, const void* k_pool, const void* v_pool, int64_t num_pages,
                 int32_t page_size, const int32_t* kv_indptr, const int32_t* kv_indices,
                 const int32_t* kv_last_page_len, int64_t total_pages, int32_t batch, int32_t num_qo_heads,
                 int32_t num_kv_heads, int32_t head_dim, float sm_scale, int32_t dtype,
                 const int32_t* seq_group_slot, int32_t num_groups, const int32_t* group_prefix_pages,
                 const int32_t* group_members, void* out, int64_t out_stride, void* workspace,
                 size_t workspace_bytes, nslg_stream_t stream, const NewRows& nr, int64_t layout) {
  if (num_groups < 1 || num_groups > kMaxGroups)
    return fail(NSLG_EUNSUPPORTED, "paged_decode_grouped: %d groups (1..%d)", num_groups, kMaxGroups);
  if (!seq_group_slot || !group_prefix_pages || !group_members)
    return fail(NSLG_EINVAL, "paged_decode_grouped: null group table");
  if (num_kv_heads <= 0 || num_qo_heads <= 0 || num_qo_heads % num_kv_heads)
    return fail(NSLG_EINVAL, "paged_decode_grouped: bad head counts");
  const int group = num_qo_heads / num_kv_heads;
  if (group > kGroupCols) return fail(NSLG_EUNSUPPORTED, "paged_decode_grouped: GQA group %d > 16", group);
  const int max_members = kGroupCols / group;
  GroupArgs<true> ga;
  ga.seq_group_slot = seq_group_slot;
  ga.group_meta = nullptr;
  ga.num_groups = num_groups;
  // host check of the group table: members are distinct sequences of the batch,
  // at least one and at most 16 / G per group, listed first; prefixes are >= 1 page
  for (int g = 0; g < kMaxGroups; ++g) {
    ga.prefix_pages[g] = 0;
    for (int m = 0; m < kGroupCols; ++m) ga.member_seq[g * kGroupCols + m] = -1;
  }
  for (int g = 0; g < num_groups; ++g) {
    if (group_prefix_pages[g] < 1 || (int64_t)group_prefix_pages[g] * page_size >= ((int64_t)1 << 31))
      return fail(NSLG_EINVAL, "paged_decode_grouped: group %d prefix of %d pages", g, group_prefix_pages[g]);
    ga.prefix_pages[g] = group_prefix_pages[g];
    bool ended = false;
    int count = 0;
    for (int m = 0; m < kGroupCols; ++m) {
      const int sq = group_members[g * kGroupCols + m];
      if (sq < 0) {
        ended = true;
        continue;
      }
      if (ended || sq >= batch || m >= max_members)
        return fail(NSLG_EINVAL, "paged_decode_grouped: group %d member %d (sequence %d) invalid", g, m, sq);
      for (int g2 = 0; g2 <= g; ++g2)
        for (int m2 = 0; m2 < (g2 == g ? m : kGroupCols); ++m2)
          if (group_members[g2 * kGroupCols + m2] == sq)
            return fail(NSLG_EINVAL, "paged_decode_grouped: sequence %d in two group slots", sq);
      ga.member_seq[g * kGroupCols + m] = (int16_t)sq;
      ++count;
    }
    if (count == 0) return fail(NSLG_EINVAL, "paged_decode_grouped: group %d has no member", g);
  }
  if (batch > 32767) return fail(NSLG_EUNSUPPORTED, "paged_decode_grouped: batch %d > 32767", batch);
  return decode_impl<true>(q, q_stride, k_pool, v_pool, num_pages, page_size, kv_indptr, kv_indices,
                           kv_last_page_len, total_pages, batch, num_qo_heads, num_kv_heads, head_dim, sm_scale,
                           dtype, out, out_stride, ga, num_groups, max_members, workspace, workspace_bytes, stream,
                           nr, layout);
}

}  // namespace

extern "C" int nslg_paged_decode_grouped(const void* q, int64_t q_stride, const void* k_pool,
                                         const void* v_pool, int64_t num_pages, int32_t page_size,
                                         const int32_t* kv_indptr, const int32_t* kv_indices,
                                         const int32_t* kv_last_page_len, int64_t total_pages,
                                         int32_t batch, int32_t num_qo_heads, int32_t num_kv_heads,
                                         int32_t head_dim, float sm_scale, int32_t dtype,
                                         const int32_t* seq_group_slot, int32_t num_groups,
                                         const int32_t* group_prefix_pages, const int32_t* group_members,
                                         void* out, int64_t out_stride, void* workspace,
                                         size_t workspace_bytes, int64_t layout, nslg_stream_t stream) {
  return grouped_impl(q, q_stride, k_pool, v_pool, num_pages, page_size, kv_indptr, kv_indices, kv_last_page_len,
                      total_pages, batch, num_qo_heads, num_kv_heads, head_dim, sm_scale, dtype, seq_group_slot,
                      num_groups, group_prefix_pages, group_members, out, out_stride, workspace, workspace_bytes,
                      stream, NewRows{}, layout);
}

extern "C" int nslg_paged_decode_grouped_append(
    const void* q, int64_t q_stride, const void* k_new, int64_t k_new_stride, const void* v_new,
    int64_t v_new_stride, void* k_pool, void* v_pool, int64_t num_pages, int32_t page_size,
    const int32_t* kv_indptr, const int32_t* kv_indices, const int32_t* kv_last_page_len, int64_t total_pages,
    int32_t batch, int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim, float sm_scale, int32_t dtype,
    const int32_t* seq_group_slot, int32_t num_groups, const int32_t* group_prefix_pages,
    const int32_t* group_members, void* out, int64_t out_stride, void* workspace, size_t workspace_bytes,
    int64_t layout, nslg_stream_t stream) {
  if (batch > 0 && (!k_new || !v_new)) return fail(NSLG_EINVAL, "paged_decode_grouped_append: null k_new or v_new");
  NewRows nr;
  nr.k = k_new;
  nr.v = v_new;
  nr.k_stride = k_new_stride;
  nr.v_stride = v_new_stride;
  return grouped_impl(q, q_stride, k_pool, v_pool, num_pages, page_size, kv_indptr, kv_indices, kv_last_page_len,
                      total_pages, batch, num_qo_heads, num_kv_heads, head_dim, sm_scale, dtype, seq_group_slot,
                      num_groups, group_prefix_pages, group_members, out, out_stride, workspace, workspace_bytes,
                      stream, nr, layout);
}

extern "C" int nslg_paged_decode_grouped_rope_append(
    const void* q, int64_t q_stride, const void* k_new, int64_t k_new_stride, const void* v_new,
    int64_t v_new_stride, const int32_t* positions, const float* cos_table, const float* sin_table,
    int64_t table_stride, int64_t table_rows, void* k_pool, void* v_pool, int64_t num_pages, int32_t page_size,
    const int32_t* kv_indptr, const int32_t* kv_indices, const int32_t* kv_last_page_len, int64_t total_pages,
    int32_t batch, int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim, float sm_scale, int32_t dtype,
    const int32_t* seq_group_slot, int32_t num_groups, const int32_t* group_prefix_pages,
    const int32_t* group_members, void* out, int64_t out_stride, void* workspace, size_t workspace_bytes,
    int64_t layout, nslg_stream_t stream) {
  if (batch > 0 && (!k_new || !v_new || !cos_table))
    return fail(NSLG_EINVAL, "paged_decode_grouped_rope_append: null k_new, v_new or tables");
  NewRows nr;
  nr.k = k_new;
  nr.v = v_new;
  nr.k_stride = k_new_stride;
  nr.v_stride = v_new_stride;
  nr.pos = positions;
  nr.cos = cos_table;
  nr.sin = sin_table;
  nr.table_stride = table_stride;
  nr.table_rows = table_rows;
  return grouped_impl(q, q_stride, k_pool, v_pool, num_pages, page_size, kv_indptr, kv_indices, kv_last_page_len,
                      total_pages, batch, num_qo_heads, num_kv_heads, head_dim, sm_scale, dtype, seq_group_slot,
                      num_groups, group_prefix_pages, group_members, out, out_stride, workspace, workspace_bytes,
                      stream, nr, layout);
}
