// Paged causal (chunked) prefill attention for gfx950 (CDNA4), MFMA fp16/bf16
// with fp32 accumulation.
//
// Query rows are packed GQA-style: for KV head h of sequence b the row space is
// the b's n_b new tokens x the G query heads of h, row = token*G + g. A
// workgroup (8 waves, 2 per SIMD) owns 256 consecutive rows of one (sequence, KV
// head); each wave owns 32 rows as two 16-row column blocks of the MFMA.
//
// Keys are staged in LDS in 128-key tiles (double buffered, shared by the 8 waves)
// and consumed in 32-key blocks. Per block:
//   S^T[16 key x 16 row] = K[16 key x D] * Q^T[D x 16 row]   v_mfma 16x16x32, D/32 steps
//   online softmax per row (column) in fp32, running max raised lazily
//   O^T[D x 16 row] += V^T[D x 32 key] * P^T[32 key x 16 row]  v_mfma 16x16x32,
//     V^T operands read from the row-major V tile with transposing LDS reads
//   the row sums of P come from one more MFMA with an all-ones A operand
// (P.V runs over 32-key blocks so it uses the full-rate 16x16x32 instruction; the
// 16x16x16 one issues at half the rate on gfx950). Within a tile the blocks are
// software pipelined: the scores of block i+1 are computed before the
// probabilities of block i, and the K operands of block i+2 are read from LDS
// during P.V of block i. The next tile is fetched from HBM and stashed into the
// other LDS stage in two 64-key halves at two points of the current tile, so
// only one half's staging registers are live at a time.
//
// Causality is bottom-right aligned: sequence b holds L_b tokens of which the
// last n_b are the new ones, so row token t sees keys j <= L_b - n_b + t.
// The sequence's page ids for the workgroup's key range sit in LDS (windows of
// 2048 pages), so tile loads never wait on index loads.
//
// Built with -fno-honor-nans (nanoslg_amd/_build.py): the running maxima are
// taken with plain v_max/v_max3 instead of NaN-quieting ones.
#include "nslg_common.h"

#include <math.h>

namespace nslg {
namespace {

constexpr int kPageWin = 2048;                     // page ids per LDS window
constexpr float kRescaleSlack = 8.0f;

// Tile shape per head dim: column blocks of 16 query rows per wave, keys per LDS
// tile, waves per workgroup. D = 64, 128: two column blocks per wave and 128-key
// tiles (256 rows per workgroup, two 128-key stages of K and V in LDS). D = 256:
// one column block per wave (its Q, O, K and V operands fill the 256 registers of
// 2 waves per SIMD) and 64-key tiles (two stages of 256-wide rows fit the LDS);
// 128 rows per workgroup.
template <int D>
struct PrefillTile {
  static constexpr int kCB = D == 256 ? 1 : 2;
  static constexpr int kKeys = D == 256 ? 64 : 128;
  static constexpr int kWaves = 8;
  static constexpr int kRowsPerWG = 16 * kCB * kWaves;
};

inline int rows_per_wg(int head_dim) {
  return head_dim == 256 ? PrefillTile<256>::kRowsPerWG : PrefillTile<128>::kRowsPerWG;
}

struct PrefillParams {
  const uint16_t* q;
  int64_t q_stride;
  const int32_t* qo_indptr;
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
  int32_t group;
  float scale_log2;
  uint16_t* out;
  int64_t out_stride;
  int32_t row_tiles;  // row-tile slots per KV head (an upper bound over the batch)
  int32_t num_work;   // row_tiles * num_kv_heads
  int32_t per_xcd;    // ceil((num_work + pad_work) / 8)
  // Grid rows (null: q and out are the ragged rows themselves): ragged row t is row
  // q_rows[t] of q and out, [batch x grid_width] rows, sequence b's block being rows
  // b * grid_width .. + grid_width - 1; pad_work workgroups zero the rows of each
  // block that hold no new token.
  const int32_t* q_rows;
  int32_t grid_width;
  int32_t pad_work;
  int32_t by_round;   // > 0: longest-first rounds of this many tiles per sequence (see below)
  int32_t rows_wg;    // query rows per workgroup (the kernel's tile shape)
  // The forward's new K/V rows (k_new null: already in the pool). Token t of sequence
  // b is row r_b + t of k_new / v_new, r_b the row of its first token (q's row map);
  // keys at positions >= start_b are read from these rows, and the workgroup holding
  // a token's first query row writes its K/V rows of the workgroup's KV head into the
  // token's page slot (slot 0 of page 0 past the table), as nslg_append_kv would.
  const uint16_t* k_new;
  const uint16_t* v_new;
  int64_t k_new_stride;  // elements between rows
  int64_t v_new_stride;
  uint32_t k_new_bytes;  // bytes of k_new's rows (the grid's or total_q), < 4 GiB
  uint32_t v_new_bytes;
};

// Word 3 of a raw (untyped, unswizzled) buffer resource on CDNA: 32-bit data format,
// no index stride; num_records (word 2) bounds the byte offset of each load.
constexpr int kBufferWord3 = 0x00020000;

template <typename V>
__device__ inline u32x4 u32x4_of(V v) {
  return __builtin_bit_cast(u32x4, v);
}

template <int N>
struct Vec {
  typedef unsigned short type __attribute__((ext_vector_type(N)));
};

// Row of q / out holding ragged row t (-1 for a grid row out of range: not read or written).
__device__ inline int64_t grid_row(const PrefillParams& p, int t) {
  if (!p.q_rows) return t;
  const int64_t r = p.q_rows[t];
  return r >= 0 && r < (int64_t)p.batch * p.grid_width ? r : -1;
}

__device__ inline int kv_len_of(const PrefillParams& p, int s) {
  const int np = p.indptr[s + 1] - p.indptr[s];
  if (np <= 0) return 0;
  int lpl = p.last_len[s];
  lpl = lpl < 1 ? 1 : (lpl > p.page_size ? p.page_size : lpl);
  return (np - 1) * p.page_size + lpl;
}

// Longest first: slot g is round r = g / batch of sequence g % batch, and round r
// takes each sequence's r-th tile from the end. A later row tile sees more keys
// (causal), so the first slots dispatched carry the most work and the short tiles
// fill in behind them. Slots past a sequence's tiles are empty.
__device__ inline bool locate_tile_by_round(const PrefillParams& p, int g, int& b, int& tile) {
  b = g % p.batch;
  const int r = g / p.batch;
  const int n = p.qo_indptr[b + 1] - p.qo_indptr[b];
  const int nt = n > 0 ? (n * p.group + p.rows_wg - 1) / p.rows_wg : 0;
  if (r >= nt) return false;
  tile = nt - 1 - r;
  return true;
}

// Most row tiles of any sequence of the batch (wave-wide, uniform).
__device__ inline int most_tiles(const PrefillParams& p) {
  const int lane = threadIdx.x & 63;
  int most = 0;
  for (int s0 = 0; s0 < p.batch; s0 += 64) {
    const int s = s0 + lane;
    int nt = 0;
    if (s < p.batch) {
      const int n = p.qo_indptr[s + 1] - p.qo_indptr[s];
      nt = n > 0 ? (n * p.group + p.rows_wg - 1) / p.rows_wg : 0;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) nt = max(nt, __shfl_xor(nt, off, 64));
    most = max(most, nt);
  }
  return __builtin_amdgcn_readfirstlane(most);
}

// Wave-wide search for the (sequence, row tile) of workgroup x.
__device__ inline bool locate_tile(const PrefillParams& p, int g, int& b, int& tile) {
  const int lane = threadIdx.x & 63;
  int base = 0;
  for (int s0 = 0; s0 < p.batch; s0 += 64) {
    const int s = s0 + lane;
    int nt = 0;
    if (s < p.batch) {
      const int n = p.qo_indptr[s + 1] - p.qo_indptr[s];
      nt = n > 0 ? (n * p.group + p.rows_wg - 1) / p.rows_wg : 0;
    }
    int incl = nt;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int y = __shfl_up(incl, off, 64);
      if (lane >= off) incl += y;
    }
    const int excl = incl - nt;
    const unsigned long long m = __ballot(nt > 0 && g >= base + excl && g < base + incl);
    if (m) {
      const int src = __ffsll((long long)m) - 1;
      b = s0 + src;
      tile = g - base - __shfl(excl, src, 64);
      return true;
    }
    base += __shfl(incl, 63, 64);
  }
  return false;
}

template <typename T, int D>
__global__ void __launch_bounds__(64 * PrefillTile<D>::kWaves) paged_prefill_kernel(PrefillParams p) {
  constexpr int kCB = PrefillTile<D>::kCB;
  constexpr int kKeys = PrefillTile<D>::kKeys;
  constexpr int kWaves = PrefillTile<D>::kWaves;
  constexpr int kRowsPerWG = PrefillTile<D>::kRowsPerWG;
  constexpr int kRowsPerWave = 16 * kCB;  // kCB column blocks of 16 rows
  constexpr int kBlocks = kKeys / 32;     // 32-key blocks per tile
  constexpr int kThreads = 64 * kWaves;
  constexpr int kSteps = D / 32;
  constexpr int NT = D / 16;
  // Tile row pitches in elements. K: D + 16, not D + 8: at D + 8 the 16-byte operand
  // reads stalled on bank conflicts for 28 % of the LDS's busy cycles (counters); at
  // D + 16 none, and the long-context chunk runs 3 % faster. V: D + 16, conflict-free
  // for the transposing 8-byte reads of 8 rows x 4 lanes.
  constexpr int kPitch = D + 16;
  constexpr int kVPitch = D + 16;
  constexpr bool kSplitP = T::kDtype == NSLG_BF16;
  constexpr bool kLean = D == 256;

  __shared__ __attribute__((aligned(16))) uint16_t k_lds[2][kKeys * kPitch];
  __shared__ __attribute__((aligned(16))) uint16_t v_lds[2][kKeys * kVPitch];
  __shared__ int32_t page_lds[kPageWin];
  __shared__ uint8_t page_st[kPageWin];  // per window entry: 0 a page of the pool, 1 past the table, 2 bad id

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  // XCD-aware order: workgroup i runs on XCD i % 8, so work item
  // w = (i % 8) * per_xcd + i / 8 gives each XCD a contiguous run of row tiles of
  // one KV head, which read the same K/V and so share that XCD's L2.
  const int w = (blockIdx.x & 7) * p.per_xcd + (blockIdx.x >> 3);
  if (w >= p.num_work) {
    if (w < p.num_work + p.pad_work)
      zero_pad_rows(p.qo_indptr, p.q_rows, p.grid_width, w - p.num_work, p.out, p.out_stride,
                    (int64_t)p.num_qo_heads * D, (int64_t)p.batch * p.grid_width);
    return;
  }
  const int h = w / p.row_tiles;
  int b = 0, tile = 0;
  const int g = w - h * p.row_tiles;
  // longest-first rounds when the host's round count covers every sequence (it came
  // from the caller's max_q); otherwise the packed order, which the grid also fits
  const bool rounds = p.by_round > 0 && most_tiles(p) <= p.by_round;
  if (!(rounds ? locate_tile_by_round(p, g, b, tile) : locate_tile(p, g, b, tile)))
    return;  // uniform across the workgroup
  b = __builtin_amdgcn_readfirstlane(b);
  tile = __builtin_amdgcn_readfirstlane(tile);

  const int q0 = p.qo_indptr[b];
  const int n_new = p.qo_indptr[b + 1] - q0;
  const int L = kv_len_of(p, b);
  const int start = L - n_new > 0 ? L - n_new : 0;  // position of the first new token
  const int G = p.group;
  const int nrows = n_new * G;
  const int row0_wg = tile * kRowsPerWG;
  // keys this workgroup needs: up to the last row's position (inclusive)
  const int last_row = min(row0_wg + kRowsPerWG, nrows) - 1;
  const int kv_end = min(L, start + last_row / G + 1);
  const int n_kt = (kv_end + kKeys - 1) / kKeys;
  const int32_t* idx = p.indices + p.indptr[b];
  const int np_seq = p.indptr[b + 1] - p.indptr[b];
  const int ps = p.page_size;
  const int row_bytes = p.num_kv_heads * D * 2;
  const char* kpool = reinterpret_cast<const char*>(p.k_pool) + h * D * 2;
  const char* vpool = reinterpret_cast<const char*>(p.v_pool) + h * D * 2;
  // keys from new_from on are this forward's rows of k_new / v_new (none: no fused append)
  const int new_from = p.k_new != nullptr ? start : 0x7fffffff;
  // row of k_new / v_new holding the sequence's first new token (its rows are
  // contiguous; a row map outside the grid reads zeros: the loads are range-checked)
  int new_row0 = q0;
  if (p.k_new != nullptr && p.q_rows && n_new > 0) new_row0 = __builtin_amdgcn_readfirstlane(p.q_rows[q0]);
  // keys of this workgroup's own tokens (those whose first query row is in its row
  // tile: each token has one such workgroup per KV head), [own_lo, own_hi), are
  // written into the pool as they are staged
  int own_lo = 0x7fffffff, own_hi = 0;
  if (p.k_new != nullptr) {
    own_lo = start + (row0_wg + G - 1) / G;
    own_hi = start + min((row0_wg + kRowsPerWG + G - 1) / G, n_new);
  }
  // k_new / v_new through buffer resources: the new-row loads take one 32-bit offset
  // register (the pool's take a 64-bit address) and are range-checked by the hardware
  // (based at the workgroup's head: the offsets are those of the pool's loads within a row)
  const __amdgpu_buffer_rsrc_t knew_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(p.k_new) + h * D, (short)0, (int)(p.k_new_bytes - h * D * 2), kBufferWord3);
  const __amdgpu_buffer_rsrc_t vnew_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(p.v_new) + h * D, (short)0, (int)(p.v_new_bytes - h * D * 2), kBufferWord3);
  const uint32_t knew_row_bytes = (uint32_t)p.k_new_stride * 2u;
  const uint32_t vnew_row_bytes = (uint32_t)p.v_new_stride * 2u;
  const int r = lane & 15;
  const int gq = lane >> 4;

  // ---- per-wave rows: two 16-row column blocks --------------------------------------
  u16x8 qb[kCB][kSteps];
  int row_tok[kCB];
  bool row_ok[kCB];
#pragma unroll
  for (int cb = 0; cb < kCB; ++cb) {
    const int row = row0_wg + wave * kRowsPerWave + cb * 16 + r;
    row_ok[cb] = row < nrows;
    const int t = row_ok[cb] ? row / G : 0;
    row_tok[cb] = start + t;  // absolute position of this row's token
    const int64_t qr = row_ok[cb] ? grid_row(p, q0 + t) : -1;
    if (qr >= 0) {
      const uint16_t* qrow = p.q + qr * p.q_stride + (int64_t)(h * G + row % G) * D;
#pragma unroll
      for (int s = 0; s < kSteps; ++s) qb[cb][s] = *reinterpret_cast<const u16x8*>(qrow + 32 * s + 8 * gq);
    } else {
#pragma unroll
      for (int s = 0; s < kSteps; ++s) qb[cb][s] = u16x8{0, 0, 0, 0, 0, 0, 0, 0};
    }
  }
  // highest key any row of this wave may see (rows are token-major, so the wave's last row)
  const int wave_last_row = min(row0_wg + wave * kRowsPerWave + kRowsPerWave, nrows) - 1;
  const int wave_kv_end = __builtin_amdgcn_readfirstlane(
      wave_last_row >= row0_wg + wave * kRowsPerWave ? start + wave_last_row / G + 1 : 0);
  // lowest position among the wave's rows: keys below start + first_tok + 1 are visible to all
  const int wave_first_tok = __builtin_amdgcn_readfirstlane(start + (row0_wg + wave * kRowsPerWave) / G);

  float m_run[kCB];
  // row sums of P on the MFMA: an all-ones A operand makes every row of the 16x16
  // output tile the column's sum over the block's keys
  f32x4 lsum[kCB];
  const unsigned short one16 = T::from_f32(1.f);
  const u16x8 ones = u16x8{one16, one16, one16, one16, one16, one16, one16, one16};
  // per column block: raw-score threshold above which the running max must be raised,
  // and the exponent offset -m (0 while m = -inf); both change only with m
  float thr[kCB];
  float neg_m[kCB];
  const float inv_scale_log2 = 1.f / p.scale_log2;
  f32x4 o[kCB][NT];
#pragma unroll
  for (int cb = 0; cb < kCB; ++cb) {
    m_run[cb] = -INFINITY;
    thr[cb] = -INFINITY;
    neg_m[cb] = 0.f;
    lsum[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int n = 0; n < NT; ++n) o[cb][n] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // ---- cooperative tile loads: kKeys keys x D for K and V in two halves ------------
  // Each half (kKeys / 2 keys) is fetched into registers and stashed into the next LDS
  // stage at its own point of the current tile, so only one half's staging registers
  // are live at a time.
  constexpr int kChunks = D / 8;                             // 16 B chunks per row
  constexpr int kHalf = kKeys / 2;
  constexpr int kPerThreadH = kHalf * kChunks / kThreads;    // D=128: 2 (8 waves) or 4 (4 waves)
  u32x4 kreg[kPerThreadH], vreg[kPerThreadH];
  int win_base = -1;

  auto load_pages = [&](int first_key) {
    // page ids for keys [first_key, first_key + kPageWin*ps), one window
    const int pg0 = first_key / ps;
    for (int i = tid; i < kPageWin; i += kThreads) {
      int v = 0, st = 1;
      if (pg0 + i < np_seq) {
        v = idx[pg0 + i];
        st = 0;
        if (v < 0 || (int64_t)v >= p.num_pages) v = 0, st = 2;
      }
      page_lds[i] = v;
      page_st[i] = (uint8_t)st;
    }
    win_base = pg0;
  };
  // thread tid moves 16-byte chunk tid % kChunks of keys tid / kChunks + (kThreads / kChunks) i
  const int f_ch16 = (tid % kChunks) * 16;
  const int f_key = tid / kChunks;
  const bool ps_pow2 = (ps & (ps - 1)) == 0;
  const int ps_shift = __builtin_ctz((unsigned)ps);
  const uint32_t page_bytes = (uint32_t)ps * (uint32_t)row_bytes;  // < 2^32 (checked by the host)
  // key kabs from the pool, through the page-id window
  auto fetch_pool = [&](int i, int kabs) {
      int pg, slot;
      if (ps_pow2) {
        pg = kabs >> ps_shift;
        slot = kabs & (ps - 1);
      } else {
        pg = kabs / ps;
        slot = kabs - pg * ps;
      }
      // page ids in the window are checked (>= 0): one 32 x 32 -> 64-bit multiply-add
      const uint32_t pid = (uint32_t)page_lds[pg - win_base];
      const uint64_t off = (uint64_t)pid * page_bytes + (uint32_t)(slot * row_bytes + f_ch16);
      kreg[i] = *reinterpret_cast<const u32x4*>(kpool + off);
      vreg[i] = *reinterpret_cast<const u32x4*>(vpool + off);
  };
  auto fetch_half = [&](int kt, int half) {
    const int key0 = kt * kKeys + half * kHalf;
    if (key0 + kHalf <= new_from) {  // uniform: every key of this half is in the pool
#pragma unroll
      for (int i = 0; i < kPerThreadH; ++i) {
        const int kabs = key0 + f_key + (kThreads / kChunks) * i;
        fetch_pool(i, kabs < kv_end ? kabs : kv_end - 1);
      }
      return;
    }
    // a half with keys of this forward: those from k_new / v_new (32-bit offsets from
    // uniform bases: the rows span < 4 GiB, checked by the host), the rest from the pool
#pragma unroll
    for (int i = 0; i < kPerThreadH; ++i) {
      int kabs = key0 + f_key + (kThreads / kChunks) * i;
      kabs = kabs < kv_end ? kabs : kv_end - 1;
      if (kabs >= new_from) {
        const uint32_t nr = (uint32_t)(new_row0 + (kabs - start));
        kreg[i] = u32x4_of(__builtin_amdgcn_raw_buffer_load_b128(knew_rsrc, (int)(nr * knew_row_bytes + f_ch16), 0, 0));
        vreg[i] = u32x4_of(__builtin_amdgcn_raw_buffer_load_b128(vnew_rsrc, (int)(nr * vnew_row_bytes + f_ch16), 0, 0));
      } else {
        fetch_pool(i, kabs);
      }
    }
  };
  auto stash_half = [&](int stage, int half) {
#pragma unroll
    for (int i = 0; i < kPerThreadH; ++i) {
      const int key = half * kHalf + f_key + (kThreads / kChunks) * i;
      *reinterpret_cast<u32x4*>(&k_lds[stage][key * kPitch + f_ch16 / 2]) = kreg[i];
      *reinterpret_cast<u32x4*>(&v_lds[stage][key * kVPitch + f_ch16 / 2]) = vreg[i];
    }
  };
  // The keys of this workgroup's own tokens in tile kt (staged in LDS stage `stage`,
  // the page-id window covering the tile) into their page slots: slot 0 of page 0 past
  // the table, not at all for an id outside the pool. Taken from LDS at the end of the
  // tile's iteration, where the block pipeline holds no registers, so the forward's
  // K/V rows are written with no load of their own.
  auto write_own = [&](int stage, int kt) {
    // the thread's key and chunk through an empty asm: the compiler cannot hoist the
    // addresses below out of the tile loop (registers held across the loop spill)
    int fk = f_key, fc = f_ch16;
    asm volatile("" : "+v"(fk), "+v"(fc));
#pragma unroll
    for (int i = 0; i < 2 * kPerThreadH; ++i) {
      const int key = fk + (kThreads / kChunks) * i;
      const int kabs = kt * kKeys + key;
      if (kabs < own_lo || kabs >= own_hi) continue;
      const int pg = kabs / ps;
      const int st = page_st[pg - win_base];
      if (st == 2) continue;
      const uint64_t off = st == 0 ? (uint64_t)(uint32_t)page_lds[pg - win_base] * page_bytes +
                                         (uint32_t)((kabs - pg * ps) * row_bytes + fc)
                                   : (uint64_t)fc;
      stream_store(reinterpret_cast<u32x4*>(const_cast<char*>(kpool) + off),
                   *reinterpret_cast<const u32x4*>(&k_lds[stage][key * kPitch + fc / 2]));
      stream_store(reinterpret_cast<u32x4*>(const_cast<char*>(vpool) + off),
                   *reinterpret_cast<const u32x4*>(&v_lds[stage][key * kVPitch + fc / 2]));
    }
  };
  // first key of the window holding tile kt must cover the whole tile
  auto window_ok = [&](int kt) {
    const int k_first = kt * kKeys;
    const int k_last = min(k_first + kKeys, kv_end) - 1;
    return win_base >= 0 && k_first / ps >= win_base && k_last / ps < win_base + kPageWin;
  };

  // ---- per-block pieces ------------------------------------------------------------
  // K operands of a 32-key block: keys kbase + 16t + r, columns 32s + 8gq .. +7
  // The lane's (r, gq) for the LDS operand addresses. bf16 (two MFMAs per P tile, 8
  // more registers) recomputes them per block from the lane id through an empty asm,
  // so they are not held across the loop: held, they spilled, and each reload's wait
  // on the vector memory counter also waited for the next tile's loads.
  auto lane_rg = [&](int& rr, int& gg) {
    int ln = lane;
    if constexpr (kSplitP) asm volatile("" : "+v"(ln));
    rr = ln & 15;
    gg = ln >> 4;
  };
  auto load_k = [&](int stage, int kb, u16x8 (&ka)[2][kSteps]) {
    int r, gq;
    lane_rg(r, gq);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const uint16_t* krow = &k_lds[stage][(32 * kb + 16 * t + r) * kPitch + 8 * gq];
#pragma unroll
      for (int s = 0; s < kSteps; ++s) ka[t][s] = *reinterpret_cast<const u16x8*>(krow + 32 * s);
    }
  };
  // S^T of both column blocks: keys kbase + 16t + 4gq + j in lane (r, gq), element j
  auto qk = [&](const u16x8 (&ka)[2][kSteps], f32x4 (&sacc)[kCB][2]) {

#pragma unroll
    for (int cb = 0; cb < kCB; ++cb)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        sacc[cb][t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < kSteps; ++s) sacc[cb][t] = T::mma_k32(ka[t][s], qb[cb][s], sacc[cb][t]);
      }

  };
  // A operand of output tile n, V^T[d = 16n + r][keys of k = 8gq + j], read from the
  // row-major tile with gfx950's transposing LDS read: in each 16-lane group, lane
  // i = 4a + c receives element c of the 8-byte blocks addressed by lanes a, 4 + a,
  // 8 + a and 12 + a. Lane r addresses keys kbase + 4gq + r/4 (then + 16), columns
  // 16n + 4(r%4) .. +3, so it receives keys kbase + 4gq + 0..3 (+ 16) at d = 16n + r.
  auto load_v = [&](int stage, int kb, u16x8 (&va)[NT]) {
    int r, gq;
    lane_rg(r, gq);
    const uint16_t* vsrc = &v_lds[stage][(32 * kb + 4 * gq + (r >> 2)) * kVPitch + 4 * (r & 3)];
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      typedef short i16x4 __attribute__((ext_vector_type(4)));
      typedef __attribute__((address_space(3))) i16x4* lds_i16x4;
      const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4)(vsrc + 16 * n));
      const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4)(vsrc + 16 * n + 16 * kVPitch));
      va[n] = __builtin_bit_cast(u16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
    }
  };
  // masking (blocks touching the causal diagonal or the end of the keys) and the lazy
  // rescale: the row's running max m is raised only when some score of the block
  // exceeds it by more than the slack, which each lane checks on its own 8 scores;
  // the cross-lane row max is needed only then
  auto mask_and_rescale = [&](int kbase, f32x4 (&sacc)[kCB][2]) {
    const bool full = kbase + 32 <= wave_first_tok + 1 && kbase + 32 <= kv_end;
#pragma unroll
    for (int cb = 0; cb < kCB; ++cb) {
      if (!full) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int key = kbase + 16 * (j >> 2) + 4 * gq + (j & 3);
          if (!(key < kv_end && key <= row_tok[cb])) sacc[cb][j >> 2][j & 3] = -INFINITY;
        }
      }
      const f32x4 a = sacc[cb][0], b = sacc[cb][1];
      const float lmax = fmaxf(fmaxf(fmaxf(a[0], a[1]), fmaxf(a[2], a[3])),
                               fmaxf(fmaxf(b[0], b[1]), fmaxf(b[2], b[3])));
      if (__ballot(lmax > thr[cb])) {
        const float m_new = fmaxf(m_run[cb], rows_max(lmax * p.scale_log2));
        const float alpha = m_new == -INFINITY ? 1.f : fast_exp2(m_run[cb] - m_new);
        lsum[cb] *= alpha;
#pragma unroll
        for (int n = 0; n < NT; ++n) o[cb][n] *= alpha;
        m_run[cb] = m_new;
        thr[cb] = (m_new + kRescaleSlack) * inv_scale_log2;
        neg_m[cb] = m_new == -INFINITY ? 0.f : -m_new;
      }
    }
  };
  // probabilities of both column blocks as 16-bit MFMA B operands (k index 8gq + j
  // stands for the lane's keys: j < 4 the first 16-key tile, j >= 4 the second)
  auto probs = [&](const f32x4 (&sacc)[kCB][2], u16x8 (&pb)[kCB], u16x8 (&pb_lo)[kCB]) {
#pragma unroll
    for (int cb = 0; cb < kCB; ++cb)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float pj = fast_exp2(fmaf(sacc[cb][j >> 2][j & 3], p.scale_log2, neg_m[cb]));
        pb[cb][j] = T::from_f32(pj);
        if constexpr (kSplitP) pb_lo[cb][j] = T::from_f32(pj - T::to_f32(pb[cb][j]));
      }
  };
  auto pv = [&](const u16x8 (&va)[NT], const u16x8 (&pb)[kCB], const u16x8 (&pb_lo)[kCB]) {

#pragma unroll
    for (int cb = 0; cb < kCB; ++cb) {
#pragma unroll
      for (int n = 0; n < NT; ++n) {
        o[cb][n] = T::mma_k32(va[n], pb[cb], o[cb][n]);
        if constexpr (kSplitP) o[cb][n] = T::mma_k32(va[n], pb_lo[cb], o[cb][n]);
      }
      lsum[cb] = T::mma_k32(ones, pb[cb], lsum[cb]);
      if constexpr (kSplitP) lsum[cb] = T::mma_k32(ones, pb_lo[cb], lsum[cb]);
    }

  };

  // D = 256 (lean): scores of one 16-key half at a time, P.V over half the output
  // tiles at a time, each with its operands read from LDS just before
  auto qk_lean = [&](int stage, int kb, f32x4 (&sacc)[kCB][2]) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      u16x8 kh[kSteps];
      const uint16_t* krow = &k_lds[stage][(32 * kb + 16 * t + r) * kPitch + 8 * gq];
#pragma unroll
      for (int s = 0; s < kSteps; ++s) kh[s] = *reinterpret_cast<const u16x8*>(krow + 32 * s);
#pragma unroll
      for (int cb = 0; cb < kCB; ++cb) {
        sacc[cb][t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < kSteps; ++s) sacc[cb][t] = T::mma_k32(kh[s], qb[cb][s], sacc[cb][t]);
      }
    }
  };
  auto pv_lean = [&](int stage, int kb, const u16x8 (&pb)[kCB], const u16x8 (&pb_lo)[kCB]) {
    const uint16_t* vsrc = &v_lds[stage][(32 * kb + 4 * gq + (r >> 2)) * kVPitch + 4 * (r & 3)];
    constexpr int kHalfNT = NT / 2;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      u16x8 va[kHalfNT];
#pragma unroll
      for (int n = 0; n < kHalfNT; ++n) {
        typedef short i16x4 __attribute__((ext_vector_type(4)));
        typedef __attribute__((address_space(3))) i16x4* lds_i16x4;
        const uint16_t* vp = vsrc + 16 * (hh * kHalfNT + n);
        const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4)vp);
        const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4)(vp + 16 * kVPitch));
        va[n] = __builtin_bit_cast(u16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
      }
#pragma unroll
      for (int cb = 0; cb < kCB; ++cb)
#pragma unroll
        for (int n = 0; n < kHalfNT; ++n) {
          o[cb][hh * kHalfNT + n] = T::mma_k32(va[n], pb[cb], o[cb][hh * kHalfNT + n]);
          if constexpr (kSplitP) o[cb][hh * kHalfNT + n] = T::mma_k32(va[n], pb_lo[cb], o[cb][hh * kHalfNT + n]);
        }
    }
#pragma unroll
    for (int cb = 0; cb < kCB; ++cb) {
      lsum[cb] = T::mma_k32(ones, pb[cb], lsum[cb]);
      if constexpr (kSplitP) lsum[cb] = T::mma_k32(ones, pb_lo[cb], lsum[cb]);
    }
  };

  if (n_kt > 0) {
    load_pages(0);
    __syncthreads();
    fetch_half(0, 0);
    stash_half(0, 0);
    fetch_half(0, 1);
    stash_half(0, 1);
  }
  __syncthreads();

  for (int kt = 0; kt < n_kt; ++kt) {
    const int stage = kt & 1;
    const bool more = kt + 1 < n_kt;
    const bool staged = more && window_ok(kt + 1);  // next tile fetched in halves during this one
    if (staged) fetch_half(kt + 1, 0);
    const int key0 = kt * kKeys;
    // 32-key blocks of this tile that the wave's rows can see (wave-uniform)
    int nb = (min(wave_kv_end, key0 + kKeys) - key0 + 31) / 32;
    nb = nb < 0 ? 0 : (nb > kBlocks ? kBlocks : nb);
    bool half1_done = false;
    if constexpr (kLean) {
      // D = 256: the same order without holding a whole block's K or V operands at
      // once (64 registers each): the K operands of each 16-key half and the V
      // operands of each half of the output tiles are read from LDS right before
      // their MFMAs.
      if (nb > 0) {
        f32x4 sacc[2][kCB][2];
        qk_lean(stage, 0, sacc[0]);
#pragma unroll
        for (int kb = 0; kb < kBlocks; ++kb) {
          if (kb >= nb) break;
          const int cur = kb & 1;
          mask_and_rescale(key0 + 32 * kb, sacc[cur]);
          u16x8 pb[kCB], pb_lo[kCB];
          if (kb + 1 < nb) qk_lean(stage, kb + 1, sacc[cur ^ 1]);
          probs(sacc[cur], pb, pb_lo);
          pv_lean(stage, kb, pb, pb_lo);
          if (kb == 1 && staged) {
            stash_half(stage ^ 1, 0);
            fetch_half(kt + 1, 1);
            half1_done = true;
          }
        }
      }
    } else if (nb > 0) {
      // Software pipeline over the tile's blocks: the scores of block kb + 1 are
      // computed (MFMA) while the probabilities of block kb are (VALU), and P.V of
      // block kb runs while the K operands of block kb + 2 are read from LDS.
      u16x8 ka[2][kSteps];
      f32x4 sacc[2][kCB][2];
      load_k(stage, 0, ka);
      qk(ka, sacc[0]);
      if (nb > 1) load_k(stage, 1, ka);
#pragma unroll
      for (int kb = 0; kb < kBlocks; ++kb) {
        if (kb >= nb) break;
        const int cur = kb & 1;
        const int kbase = key0 + 32 * kb;
        mask_and_rescale(kbase, sacc[cur]);
        u16x8 va[NT];
        u16x8 pb[kCB], pb_lo[kCB];
        load_v(stage, kb, va);
        if (kb + 1 < nb) qk(ka, sacc[cur ^ 1]);
        probs(sacc[cur], pb, pb_lo);
        if (kb + 2 < nb) load_k(stage, kb + 2, ka);
        pv(va, pb, pb_lo);
        if (kb == 1 && staged) {
          stash_half(stage ^ 1, 0);
          fetch_half(kt + 1, 1);
          half1_done = true;
        }
      }
    }
    // this tile's own keys go out after the next tile's loads have been waited for (the
    // wait counter covers stores too), under the page-id window of this tile
    const bool own_tile = kt * kKeys + kKeys > own_lo && kt * kKeys < own_hi;  // uniform
    if (staged) {
      if (!half1_done) {
        stash_half(stage ^ 1, 0);
        fetch_half(kt + 1, 1);
      }
      stash_half(stage ^ 1, 1);
      if (own_tile) write_own(stage, kt);
    } else if (more) {
      if (own_tile) write_own(stage, kt);
      // the next tile crosses the page-id window: reload it (every thread is done
      // reading page ids of the current window once all reach the barrier)
      __syncthreads();
      load_pages((kt + 1) * kKeys);
      __syncthreads();
      fetch_half(kt + 1, 0);
      stash_half(stage ^ 1, 0);
      fetch_half(kt + 1, 1);
      stash_half(stage ^ 1, 1);
    } else if (own_tile) {
      write_own(stage, kt);  // the last tile
    }
    __syncthreads();
  }
  // ---- epilogue: normalise and store rows ----------------------------------------
  // The rows' output addresses are found again here (the lane index through an empty
  // asm, so the compiler cannot keep the prologue's values alive across the tile loop)
  int er = r;
  asm volatile("" : "+v"(er));
#pragma unroll
  for (int cb = 0; cb < kCB; ++cb) {
    const float l_tot = lsum[cb][0];
    const int row = row0_wg + wave * kRowsPerWave + cb * 16 + er;
    if (row >= nrows) continue;
    const int t = row / G;
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    const int64_t orr = grid_row(p, q0 + t);
    if (orr < 0) continue;
    uint16_t* orow = p.out + orr * p.out_stride + (int64_t)(h * G + row % G) * D;
    // lane holds O[row][16n + 4gq + i] in o[cb][n][i]
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      u16x4 w;
#pragma unroll
      for (int i = 0; i < 4; ++i) w[i] = T::from_f32(o[cb][n][i] * inv);
      *reinterpret_cast<u16x4*>(orow + 16 * n + 4 * gq) = w;
    }
  }
}

// Rows of every sequence with no key to attend (n_new > 0 but L = 0 cannot occur
// with a consistent plan; sequences with n_new = 0 have no rows) need no pass.

inline int64_t grid_tiles(int64_t total_q, int32_t batch, int group, int rows_wg) {
  return (total_q * group + rows_wg - 1) / rows_wg + batch;
}

template <typename T, int D>
int launch_prefill(const PrefillParams& p, hipStream_t s) {
  // D = 64, 128: two column blocks (32 rows) per wave, 8 waves: measured faster than
  // four per wave at one wave per SIMD (chunk 3584..4095 of 8 x 4096: 276 vs 338 us)
  paged_prefill_kernel<T, D><<<dim3((unsigned)(8 * p.per_xcd)), 64 * PrefillTile<D>::kWaves, 0, s>>>(p);
  return check_launch("paged_prefill");
}

}  // namespace
}  // namespace nslg

using namespace nslg;

extern "C" size_t nslg_paged_prefill_workspace_size(int32_t batch, int32_t num_qo_heads,
                                                    int32_t head_dim, int64_t total_q,
                                                    int32_t max_q) {
  (void)batch;
  (void)num_qo_heads;
  (void)head_dim;
  (void)total_q;
  (void)max_q;
  return 256;  // the prefill kernel keeps all state on chip
}

namespace {

int prefill_impl(const void* q, int64_t q_stride, const int32_t* qo_indptr, const int32_t* q_rows,
                 int32_t grid_width, int64_t total_q, int32_t max_q, const void* k_pool, const void* v_pool,
                 int64_t num_pages, int32_t page_size, const int32_t* kv_indptr, const int32_t* kv_indices,
                 const int32_t* kv_last_page_len, int32_t batch, int32_t num_qo_heads, int32_t num_kv_heads,
                 int32_t head_dim, float sm_scale, int32_t dtype, void* out, int64_t out_stride,
                 nslg_stream_t stream, const void* k_new = nullptr, int64_t k_new_stride = 0,
                 const void* v_new = nullptr, int64_t v_new_stride = 0) {
  if (batch < 0 || num_qo_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || page_size <= 0 ||
      num_pages <= 0 || total_q < 0)
    return fail(NSLG_EINVAL, "paged_prefill: bad sizes");
  if (q_rows && (grid_width < 1 || (int64_t)batch * grid_width > 0x7fffffff || total_q > (int64_t)batch * grid_width))
    return fail(NSLG_EINVAL, "paged_prefill_grid: grid of %d x %d rows for %lld tokens", batch, grid_width,
                (long long)total_q);
  if (!(sm_scale > 0.f) || !(sm_scale < INFINITY))
    return fail(NSLG_EINVAL, "paged_prefill: sm_scale must be positive and finite");
  if (batch == 0) return NSLG_OK;
  if (total_q == 0 && !q_rows) return NSLG_OK;  // (a grid without tokens still has its pad rows zeroed)
  if (!q || !qo_indptr || !k_pool || !v_pool || !kv_indptr || !kv_indices || !kv_last_page_len || !out)
    return fail(NSLG_EINVAL, "paged_prefill: null pointer");
  if (num_qo_heads % num_kv_heads != 0)
    return fail(NSLG_EINVAL, "paged_prefill: Hq=%d not a multiple of Hkv=%d", num_qo_heads, num_kv_heads);
  const int group = num_qo_heads / num_kv_heads;
  if (group > 16) return fail(NSLG_EUNSUPPORTED, "paged_prefill: GQA group %d > 16", group);
  if (k_new && dtype != NSLG_F16 && dtype != NSLG_BF16)
    return fail(NSLG_EUNSUPPORTED, "paged_prefill_append: dtype %d (f16 or bf16 pools)", dtype);
  if (dtype == NSLG_F32) {
    // fp32 pools: the VALU attention kernel, ragged rows, bottom-right causal
    if (q_stride < (int64_t)num_qo_heads * head_dim || out_stride < (int64_t)num_qo_heads * head_dim)
      return fail(NSLG_EINVAL, "paged_prefill: row stride smaller than Hq*D");
    AttnF32Args a;
    a.dtype = dtype;
    a.q = (const float*)q;
    a.q_stride = q_stride;
    a.qo_indptr = qo_indptr;
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
    a.q_rows = q_rows;
    a.grid_width = grid_width;
    a.splits = 1;  // the query rows fill the GPU
    a.part_o = nullptr;
    a.part_ml = nullptr;
    return attention_f32(a, total_q, head_dim, as_stream(stream));
  }
  if (dtype != NSLG_F16 && dtype != NSLG_BF16)
    return fail(NSLG_EUNSUPPORTED, "paged_prefill: dtype %d", dtype);
  if (head_dim != 64 && head_dim != 128 && head_dim != 256)
    return fail(NSLG_EUNSUPPORTED, "paged_prefill: head_dim %d (64, 128 or 256)", head_dim);
  if (num_kv_heads > 65535) return fail(NSLG_EUNSUPPORTED, "paged_prefill: too many KV heads");
  if (q_stride < (int64_t)num_qo_heads * head_dim || out_stride < (int64_t)num_qo_heads * head_dim)
    return fail(NSLG_EINVAL, "paged_prefill: row stride smaller than Hq*D");
  if (((uintptr_t)q | (uintptr_t)k_pool | (uintptr_t)v_pool | (uintptr_t)out) & 15 ||
      (q_stride * 2) % 16 || (out_stride * 2) % 16)
    return fail(NSLG_EINVAL, "paged_prefill: q/pool/out must be 16-byte aligned");
  if (k_new) {
    if (!v_new) return fail(NSLG_EINVAL, "paged_prefill_append: null v_new");
    if (k_new_stride < (int64_t)num_kv_heads * head_dim || v_new_stride < (int64_t)num_kv_heads * head_dim)
      return fail(NSLG_EINVAL, "paged_prefill_append: k/v row stride smaller than Hkv*D");
    if (((uintptr_t)k_new | (uintptr_t)v_new) & 15 || (k_new_stride * 2) % 16 || (v_new_stride * 2) % 16)
      return fail(NSLG_EINVAL, "paged_prefill_append: k_new/v_new rows must be 16-byte aligned");
    // the kernel addresses k_new / v_new rows with 32-bit byte offsets
    const int64_t rows = q_rows ? (int64_t)batch * grid_width : total_q;
    if (rows * (k_new_stride > v_new_stride ? k_new_stride : v_new_stride) * 2 > (int64_t)0xffffffff)
      return fail(NSLG_EUNSUPPORTED, "paged_prefill_append: k_new/v_new rows span >= 4 GiB");
  }
  if (num_pages * (int64_t)page_size >= ((int64_t)1 << 31))
    return fail(NSLG_EUNSUPPORTED, "paged_prefill: pool has >= 2^31 token slots");
  if ((int64_t)page_size * num_kv_heads * head_dim * 2 > (int64_t)0xffffffff)
    return fail(NSLG_EUNSUPPORTED, "paged_prefill: pages of >= 4 GiB");
  const int rows_wg = rows_per_wg(head_dim);
  const int64_t tiles = grid_tiles(total_q, batch, group, rows_wg);
  if (tiles > 0x7fffffff) return fail(NSLG_EUNSUPPORTED, "paged_prefill: too many rows");

  PrefillParams p;
  p.q = (const uint16_t*)q;
  p.q_stride = q_stride;
  p.qo_indptr = qo_indptr;
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
  p.out = (uint16_t*)out;
  p.out_stride = out_stride;
  if (tiles * num_kv_heads > 0x7fffffff) return fail(NSLG_EUNSUPPORTED, "paged_prefill: too many rows");
  // Longest-first rounds need batch x (most tiles of a sequence) slots; taken when
  // that is at most 5/4 of the slots of the packed order (near-uniform batches,
  // such as the chunks of a batch of prompts), so few slots are empty.
  // The grid fits both orders; the kernel checks the rounds against the batch.
  const int64_t most = max_q > 0 ? ((int64_t)max_q * group + rows_wg - 1) / rows_wg : 0;
  const int64_t round_slots = (int64_t)batch * most;
  const bool by_round = most > 0 && most <= 0x7fffffff && 4 * round_slots <= 5 * tiles;
  p.by_round = by_round ? (int32_t)most : 0;
  p.rows_wg = rows_wg;
  const int64_t slots = by_round && round_slots > tiles ? round_slots : tiles;
  if (slots * num_kv_heads > 0x7fffffff) return fail(NSLG_EUNSUPPORTED, "paged_prefill: too many rows");
  p.row_tiles = (int32_t)slots;
  p.num_work = (int32_t)(slots * num_kv_heads);
  p.q_rows = q_rows;
  p.grid_width = grid_width;
  p.pad_work = q_rows ? batch : 0;
  if ((int64_t)p.num_work + p.pad_work > 0x7fffffff - 8) return fail(NSLG_EUNSUPPORTED, "paged_prefill: too many rows");
  p.per_xcd = (p.num_work + p.pad_work + 7) / 8;
  p.k_new = (const uint16_t*)k_new;
  p.v_new = (const uint16_t*)v_new;
  p.k_new_stride = k_new_stride;
  p.v_new_stride = v_new_stride;
  p.k_new_bytes = p.v_new_bytes = 0;
  if (k_new) {
    const int64_t rows = q_rows ? (int64_t)batch * grid_width : total_q;
    p.k_new_bytes = (uint32_t)(rows * k_new_stride * 2);
    p.v_new_bytes = (uint32_t)(rows * v_new_stride * 2);
  }
  hipStream_t s = as_stream(stream);
  if (dtype == NSLG_F16) {
    switch (head_dim) {
      case 64: return launch_prefill<F16, 64>(p, s);
      case 128: return launch_prefill<F16, 128>(p, s);
      default: return launch_prefill<F16, 256>(p, s);
    }
  }
  switch (head_dim) {
    case 64: return launch_prefill<BF16, 64>(p, s);
    case 128: return launch_prefill<BF16, 128>(p, s);
    default: return launch_prefill<BF16, 256>(p, s);
  }
}

}  // namespace

extern "C" int nslg_paged_prefill(const void* q, int64_t q_stride, const int32_t* qo_indptr,
                                  int64_t total_q, int32_t max_q, const void* k_pool,
                                  const void* v_pool, int64_t num_pages, int32_t page_size,
                                  const int32_t* kv_indptr, const int32_t* kv_indices,
                                  const int32_t* kv_last_page_len, int32_t batch,
                                  int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                                  float sm_scale, int32_t dtype, void* out, int64_t out_stride,
                                  void* workspace, size_t workspace_bytes, nslg_stream_t stream) {
  (void)workspace;
  (void)workspace_bytes;
  return prefill_impl(q, q_stride, qo_indptr, nullptr, 0, total_q, max_q, k_pool, v_pool, num_pages, page_size,
                      kv_indptr, kv_indices, kv_last_page_len, batch, num_qo_heads, num_kv_heads, head_dim, sm_scale,
                      dtype, out, out_stride, stream);
}

extern "C" int nslg_paged_prefill_grid(const void* q, int64_t q_stride, const int32_t* qo_indptr,
                                       const int32_t* q_rows, int32_t grid_width, int64_t total_q,
                                       int32_t max_q, const void* k_pool, const void* v_pool,
                                       int64_t num_pages, int32_t page_size, const int32_t* kv_indptr,
                                       const int32_t* kv_indices, const int32_t* kv_last_page_len,
                                       int32_t batch, int32_t num_qo_heads, int32_t num_kv_heads,
                                       int32_t head_dim, float sm_scale, int32_t dtype, void* out,
                                       int64_t out_stride, void* workspace, size_t workspace_bytes,
                                       nslg_stream_t stream) {
  (void)workspace;
  (void)workspace_bytes;
  if (batch > 0 && !q_rows) return fail(NSLG_EINVAL, "paged_prefill_grid: null q_rows");
  return prefill_impl(q, q_stride, qo_indptr, q_rows, grid_width, total_q, max_q, k_pool, v_pool, num_pages,
                      page_size, kv_indptr, kv_indices, kv_last_page_len, batch, num_qo_heads, num_kv_heads,
                      head_dim, sm_scale, dtype, out, out_stride, stream);
}

extern "C" int nslg_paged_prefill_append(const void* q, int64_t q_stride, const int32_t* qo_indptr,
                                         const int32_t* q_rows, int32_t grid_width, int64_t total_q,
                                         int32_t max_q, const void* k_new, int64_t k_new_stride,
                                         const void* v_new, int64_t v_new_stride, void* k_pool, void* v_pool,
                                         int64_t num_pages, int32_t page_size, const int32_t* kv_indptr,
                                         const int32_t* kv_indices, const int32_t* kv_last_page_len,
                                         int32_t batch, int32_t num_qo_heads, int32_t num_kv_heads,
                                         int32_t head_dim, float sm_scale, int32_t dtype, void* out,
                                         int64_t out_stride, void* workspace, size_t workspace_bytes,
                                         nslg_stream_t stream) {
  (void)workspace;
  (void)workspace_bytes;
  if (batch > 0 && total_q > 0 && (!k_new || !v_new)) return fail(NSLG_EINVAL, "paged_prefill_append: null k_new/v_new");
  return prefill_impl(q, q_stride, qo_indptr, q_rows, grid_width, total_q, max_q, k_pool, v_pool, num_pages,
                      page_size, kv_indptr, kv_indices, kv_last_page_len, batch, num_qo_heads, num_kv_heads,
                      head_dim, sm_scale, dtype, out, out_stride, stream, k_new, k_new_stride, v_new, v_new_stride);
}
