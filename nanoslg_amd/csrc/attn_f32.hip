// Paged attention on the VALU (decode and causal chunked prefill alike), for gfx950.
// The 16-bit paths run on MFMA; this one serves caches kept in fp32 (the contiguous
// backend of an fp32 model, kv_cache.py:227-322, whose attention is torch SDPA in the
// model's dtype). It computes in fp32 with its operands staged in LDS.
//
// A workgroup (256 threads) owns 16 query rows of one (sequence, KV head); rows are
// packed GQA-style, row = token * G + g, so one K/V tile serves all G query heads of
// the KV head. Keys are taken 32 per tile. Per tile:
//   K, V rows gathered through the block table into LDS (16 B per thread access)
//   scores: thread (row i = tid / 16, lane j = tid % 16) computes keys j and j + 16
//   online softmax per row over its 16-lane group (xor shuffles), natural exponent
//   O: thread (row i, d-slice tid % 16) accumulates D/16 output columns
// Causality is bottom-right aligned: token t of a sequence with L keys and n new
// tokens sees keys j <= L - n + t (FlashInfer's causal prefill with a KV prefix,
// kv_cache.py:627-632, and the contiguous path's mask, kv_cache.py:218-220).
#include "nslg_common.h"

#include <math.h>

namespace nslg {
namespace {

constexpr int kRowsF = 16;
constexpr int kKeysF = 32;
constexpr int kThreadsF = 256;

// Four consecutive elements of a pool, q or out row (fp32, 16-byte accesses).
template <typename T>
struct Vec4;
template <>
struct Vec4<float> {
  using E = float;
  __device__ static inline f32x4 load(const E* p) { return *reinterpret_cast<const f32x4*>(p); }
  __device__ static inline void store(E* p, f32x4 v) { *reinterpret_cast<f32x4*>(p) = v; }
};

// Row of q / out holding new token t (-1: a grid row out of range, not read or written).
__device__ inline int64_t f32_grid_row(const AttnF32Args& p, int t) {
  if (!p.q_rows) return t;
  const int64_t r = p.q_rows[t];
  return r >= 0 && r < (int64_t)p.batch * p.grid_width ? r : -1;
}

__device__ inline int kv_len_f32(const AttnF32Args& p, int s) {
  const int np = p.indptr[s + 1] - p.indptr[s];
  if (np <= 0) return 0;
  int lpl = p.last_len[s];
  lpl = lpl < 1 ? 1 : (lpl > p.page_size ? p.page_size : lpl);
  return (np - 1) * p.page_size + lpl;
}

__device__ inline int new_tokens_f32(const AttnF32Args& p, int s) {
  return p.qo_indptr ? p.qo_indptr[s + 1] - p.qo_indptr[s] : 1;
}

// Wave-wide search for the (sequence, 16-row tile) of tile slot g.
__device__ inline bool locate_f32(const AttnF32Args& p, int g, int& b, int& tile) {
  const int lane = threadIdx.x & 63;
  int base = 0;
  for (int s0 = 0; s0 < p.batch; s0 += 64) {
    const int s = s0 + lane;
    int nt = 0;
    if (s < p.batch) {
      const int n = new_tokens_f32(p, s);
      nt = n > 0 ? (n * p.group + kRowsF - 1) / kRowsF : 0;
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
__global__ void __launch_bounds__(kThreadsF) attention_f32_kernel(AttnF32Args p) {
  using VE = Vec4<T>;
  using E = typename VE::E;
  const E* q_src = reinterpret_cast<const E*>(p.q);
  const E* k_src = reinterpret_cast<const E*>(p.k_pool);
  const E* v_src = reinterpret_cast<const E*>(p.v_pool);
  E* out = reinterpret_cast<E*>(p.out);
  constexpr int kPitch = D + 4;     // floats; 16 B row padding against bank conflicts
  constexpr int kCols = D / 16;     // output columns per thread
  __shared__ __attribute__((aligned(16))) float q_lds[kRowsF * kPitch];
  __shared__ __attribute__((aligned(16))) float k_lds[kKeysF * kPitch];
  __shared__ __attribute__((aligned(16))) float v_lds[kKeysF * kPitch];
  __shared__ float p_lds[kRowsF][kKeysF + 1];

  const int tid = threadIdx.x;
  const int64_t work = (int64_t)p.row_tiles * p.num_kv_heads;
  if ((int64_t)blockIdx.x >= work) {  // a padded grid's pad rows: one workgroup per sequence
    if (p.q_rows && blockIdx.y == 0)
      zero_pad_rows(p.qo_indptr, p.q_rows, p.grid_width, (int)(blockIdx.x - work), out, p.out_stride,
                    (int64_t)p.num_qo_heads * D, (int64_t)p.batch * p.grid_width);
    return;
  }
  const int h = blockIdx.x / p.row_tiles;
  int b = 0, tile = 0;
  if (!locate_f32(p, blockIdx.x - h * p.row_tiles, b, tile)) return;  // uniform over the workgroup
  b = __builtin_amdgcn_readfirstlane(b);
  tile = __builtin_amdgcn_readfirstlane(tile);

  const int G = p.group;
  const int n_new = new_tokens_f32(p, b);
  const int q0 = p.qo_indptr ? p.qo_indptr[b] : b;
  const int L = kv_len_f32(p, b);
  const int start = L - n_new > 0 ? L - n_new : 0;
  const int nrows = n_new * G;
  const int row0 = tile * kRowsF;
  const int last_row = min(row0 + kRowsF, nrows) - 1;
  const int kv_all = min(L, start + last_row / G + 1);
  // split y of p.splits takes keys [kv_begin, kv_end) (32-key aligned pieces)
  const int split = blockIdx.y;
  const int piece = ((kv_all + p.splits - 1) / p.splits + kKeysF - 1) / kKeysF * kKeysF;
  const int kv_begin = min(kv_all, split * piece);
  const int kv_end = min(kv_all, kv_begin + piece);
  const int32_t* idx = p.indices + p.indptr[b];
  const int ps = p.page_size;
  const int64_t row_elems = (int64_t)p.num_kv_heads * D;

  // query rows of the tile into LDS (zeros for rows past the sequence's)
  for (int e = tid; e < kRowsF * (D / 4); e += kThreadsF) {
    const int i = e / (D / 4), c = e % (D / 4);
    const int row = row0 + i;
    f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
    if (row < nrows) {
      const int t = row / G, g = row % G;
      const int64_t qr = f32_grid_row(p, q0 + t);
      if (qr >= 0) v = VE::load(q_src + qr * p.q_stride + (int64_t)(h * G + g) * D + 4 * c);
    }
    *reinterpret_cast<f32x4*>(&q_lds[i * kPitch + 4 * c]) = v;
  }

  // thread roles
  const int ri = tid / 16;            // row of the tile
  const int rj = tid % 16;            // key lane (scores) / column slice (output)
  const int my_row = row0 + ri;
  const bool row_ok = my_row < nrows;
  const int my_pos = row_ok ? start + my_row / G : -1;  // absolute position of the row's token
  float m_run = -INFINITY, l_run = 0.f;
  float o[kCols];
#pragma unroll
  for (int c = 0; c < kCols; ++c) o[c] = 0.f;

  for (int key0 = kv_begin; key0 < kv_end; key0 += kKeysF) {
    __syncthreads();  // previous tile's K/V/P reads are done (and q_lds is written)
    for (int e = tid; e < kKeysF * (D / 4); e += kThreadsF) {
      const int j = e / (D / 4), c = e % (D / 4);
      int key = key0 + j;
      key = key < kv_end ? key : kv_end - 1;
      int pid = idx[key / ps];
      pid = (pid < 0 || (int64_t)pid >= p.num_pages) ? 0 : pid;
      const int64_t off = ((int64_t)pid * ps + key % ps) * row_elems + (int64_t)h * D + 4 * c;
      *reinterpret_cast<f32x4*>(&k_lds[j * kPitch + 4 * c]) = VE::load(k_src + off);
      *reinterpret_cast<f32x4*>(&v_lds[j * kPitch + 4 * c]) = VE::load(v_src + off);
    }
    __syncthreads();
    // scores of keys key0 + rj and key0 + rj + 16 for row ri
    float s0 = 0.f, s1 = 0.f;
    const float* qr = &q_lds[ri * kPitch];
    const float* k0 = &k_lds[rj * kPitch];
    const float* k1 = &k_lds[(rj + 16) * kPitch];
#pragma unroll 8
    for (int d = 0; d < D; d += 4) {
      const f32x4 a = *reinterpret_cast<const f32x4*>(qr + d);
      const f32x4 x = *reinterpret_cast<const f32x4*>(k0 + d);
      const f32x4 y = *reinterpret_cast<const f32x4*>(k1 + d);
      s0 = fmaf(a[0], x[0], fmaf(a[1], x[1], fmaf(a[2], x[2], fmaf(a[3], x[3], s0))));
      s1 = fmaf(a[0], y[0], fmaf(a[1], y[1], fmaf(a[2], y[2], fmaf(a[3], y[3], s1))));
    }
    const int ka = key0 + rj, kb = key0 + rj + 16;
    s0 = (row_ok && ka < kv_end && ka <= my_pos) ? s0 * p.scale : -INFINITY;
    s1 = (row_ok && kb < kv_end && kb <= my_pos) ? s1 * p.scale : -INFINITY;
    // online softmax over the row's 16 lanes
    float tmax = fmaxf(s0, s1);
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) tmax = fmaxf(tmax, __shfl_xor(tmax, off, 64));
    const float m_new = fmaxf(m_run, tmax);
    const float alpha = m_new == -INFINITY ? 1.f : expf(m_run - m_new);
    const float p0 = s0 == -INFINITY ? 0.f : expf(s0 - m_new);
    const float p1 = s1 == -INFINITY ? 0.f : expf(s1 - m_new);
    float psum = p0 + p1;
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) psum += __shfl_xor(psum, off, 64);
    l_run = l_run * alpha + psum;
    m_run = m_new;
    p_lds[ri][rj] = p0;
    p_lds[ri][rj + 16] = p1;
    __syncthreads();
    // O[row ri][cols rj*kCols ...] = alpha * O + P[ri, :] V[:, cols]
#pragma unroll
    for (int c = 0; c < kCols; ++c) o[c] *= alpha;
    const int nk = min(kKeysF, kv_end - key0);
    for (int j = 0; j < nk; ++j) {
      const float pj = p_lds[ri][j];
      const float* vr = &v_lds[j * kPitch + rj * kCols];
#pragma unroll
      for (int c = 0; c < kCols; c += 4) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(vr + c);
        o[c] = fmaf(pj, v[0], o[c]);
        o[c + 1] = fmaf(pj, v[1], o[c + 1]);
        o[c + 2] = fmaf(pj, v[2], o[c + 2]);
        o[c + 3] = fmaf(pj, v[3], o[c + 3]);
      }
    }
  }

  if (!row_ok) return;
  const int t = my_row / G, g = my_row % G;
  if (p.splits > 1) {
    // partial of this split: unnormalised O, running max and sum (merged later)
    const int64_t slot = ((int64_t)(q0 + t) * p.num_qo_heads + h * G + g) * p.splits + split;
    float* po = p.part_o + slot * D + rj * kCols;
#pragma unroll
    for (int c = 0; c < kCols; c += 4) *reinterpret_cast<f32x4*>(po + c) = f32x4{o[c], o[c + 1], o[c + 2], o[c + 3]};
    if (rj == 0) {
      p.part_ml[slot * 2] = m_run;
      p.part_ml[slot * 2 + 1] = l_run;
    }
    return;
  }
  const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
  const int64_t orr = f32_grid_row(p, q0 + t);
  if (orr < 0) return;
  E* orow = out + orr * p.out_stride + (int64_t)(h * G + g) * D + rj * kCols;
#pragma unroll
  for (int c = 0; c < kCols; c += 4) VE::store(orow + c, f32x4{o[c] * inv, o[c + 1] * inv, o[c + 2] * inv, o[c + 3] * inv});
}

// Merge of the splits of one (query token, query head) row: one wave, lanes over D.
template <int D>
__global__ void __launch_bounds__(64) attention_f32_merge_kernel(AttnF32Args p, int64_t rows) {
  const int64_t row = blockIdx.x;  // (token, head) in [0, total_q * Hq)
  if (row >= rows) return;
  const int lane = threadIdx.x;
  const float* ml = p.part_ml + row * p.splits * 2;
  float M = -INFINITY;
  for (int s = 0; s < p.splits; ++s) M = fmaxf(M, ml[2 * s]);
  float lsum = 0.f;
  float acc[D / 64];
#pragma unroll
  for (int c = 0; c < D / 64; ++c) acc[c] = 0.f;
  for (int s = 0; s < p.splits; ++s) {
    const float m = ml[2 * s];
    if (m == -INFINITY) continue;
    const float f = expf(m - M);
    lsum += f * ml[2 * s + 1];
    const float* po = p.part_o + (row * p.splits + s) * D;
#pragma unroll
    for (int c = 0; c < D / 64; ++c) acc[c] = fmaf(f, po[c * 64 + lane], acc[c]);
  }
  const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
  const int64_t t = row / p.num_qo_heads, hq = row % p.num_qo_heads;
  float* orow = p.out + t * p.out_stride + hq * D;
#pragma unroll
  for (int c = 0; c < D / 64; ++c) orow[c * 64 + lane] = acc[c] * inv;
}

}  // namespace

int attention_f32_splits(int64_t batch, int64_t total_tokens) {
  // a split per ~512 keys of the average sequence, up to 64, for one query token
  // per sequence (decode); the prefill rows fill the GPU on their own
  if (batch <= 0) return 1;
  const int64_t per_seq = total_tokens / batch;
  int64_t sp = per_seq / 512;
  const int64_t cap = 4096 / batch;  // keep splits x sequences near a few thousand workgroups
  sp = sp > cap ? cap : sp;
  return (int)(sp < 1 ? 1 : (sp > 64 ? 64 : sp));
}

size_t attention_f32_workspace(int64_t total_q, int32_t num_qo_heads, int32_t head_dim, int splits) {
  if (splits <= 1) return 256;
  return (size_t)total_q * num_qo_heads * splits * (head_dim + 2) * sizeof(float) + 256;
}

int attention_f32(const AttnF32Args& a, int64_t total_q, int32_t head_dim, hipStream_t s) {
  if (a.group > kRowsF * 64) return fail(NSLG_EUNSUPPORTED, "attention_f32: GQA group %d", a.group);
  if (a.dtype != NSLG_F32)
    return fail(NSLG_EUNSUPPORTED, "attention_f32: dtype %d (16-bit pools run on the MFMA kernels)", a.dtype);
  // 16-byte rows: the kernel's vector accesses and the pad-row zeroing (16-byte stores)
  if (((uintptr_t)a.q | (uintptr_t)a.k_pool | (uintptr_t)a.v_pool | (uintptr_t)a.out) & 15 ||
      (a.q_stride * 4) % 16 || (a.out_stride * 4) % 16)
    return fail(NSLG_EINVAL, "attention_f32: q/pool/out must be 16-byte aligned with row strides of 16 bytes");
  if (a.num_pages * (int64_t)a.page_size >= ((int64_t)1 << 31))
    return fail(NSLG_EUNSUPPORTED, "attention_f32: pool has >= 2^31 token slots");
  // row-tile slots per KV head: an upper bound over the batch (every sequence may
  // end in a partial tile)
  const int64_t tiles = (total_q * a.group + kRowsF - 1) / kRowsF + a.batch;
  if (tiles * a.num_kv_heads > 0x7fffffff) return fail(NSLG_EUNSUPPORTED, "attention_f32: too many rows");
  if (head_dim != 64 && head_dim != 128 && head_dim != 256)
    return fail(NSLG_EUNSUPPORTED, "attention_f32: head_dim %d (64, 128 or 256)", head_dim);
  if (a.splits < 1 || a.splits > 64) return fail(NSLG_EINVAL, "attention_f32: %d splits", a.splits);
  if (a.splits > 1 && (!a.part_o || !a.part_ml)) return fail(NSLG_EWORKSPACE, "attention_f32: no workspace");
  if (a.q_rows && (a.splits != 1 || !a.qo_indptr || a.grid_width < 1))
    return fail(NSLG_EINVAL, "attention_f32: a padded grid needs ragged rows, a width and one split");
  AttnF32Args p = a;
  p.row_tiles = (int32_t)tiles;
  const int64_t pad_wgs = a.q_rows ? a.batch : 0;
  if (tiles * a.num_kv_heads + pad_wgs > 0x7fffffff) return fail(NSLG_EUNSUPPORTED, "attention_f32: too many rows");
  const dim3 grid((unsigned)(tiles * a.num_kv_heads + pad_wgs), (unsigned)a.splits);
  switch (head_dim) {
    case 64: attention_f32_kernel<float, 64><<<grid, kThreadsF, 0, s>>>(p); break;
    case 128: attention_f32_kernel<float, 128><<<grid, kThreadsF, 0, s>>>(p); break;
    default: attention_f32_kernel<float, 256><<<grid, kThreadsF, 0, s>>>(p); break;
  }
  int rc = check_launch("attention_f32");
  if (rc || a.splits == 1) return rc;
  const int64_t rows = total_q * a.num_qo_heads;
  if (rows > 0x7fffffff) return fail(NSLG_EUNSUPPORTED, "attention_f32: too many rows");
  switch (head_dim) {
    case 64: attention_f32_merge_kernel<64><<<dim3((unsigned)rows), 64, 0, s>>>(p, rows); break;
    case 128: attention_f32_merge_kernel<128><<<dim3((unsigned)rows), 64, 0, s>>>(p, rows); break;
    default: attention_f32_merge_kernel<256><<<dim3((unsigned)rows), 64, 0, s>>>(p, rows); break;
  }
  return check_launch("attention_f32_merge");
}

}  // namespace nslg
