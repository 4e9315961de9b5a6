// Fused rotary position embedding + K/V append for gfx950.
//
// One launch per layer and forward does what the model's attention forward and
// the cache's write do in separate steps: gather cos/sin at each token's position,
// rotate q and k_new, and scatter the rotated k and the unrotated v into the pool
// slots of the forward's write plan. q is written rotated to q_out (in place when
// q_out == q); k_new and v_new are only read.
//
// Arithmetic is that of the eager tensor expression it replaces, element by
// element in the storage type (each product and the sum rounded to it; fp16, bf16
// or fp32):
//   c = rnd(cos[pos][d]), s = rnd(sin[pos][d])
//   out[d] = rnd(rnd(x[d] * c) + rnd(rot[d] * s)),  rot = cat(-x[H:], x[:H])
// A 16-bit times 16-bit product is exact in fp32 and the sum is done in fp32, as
// the eager ops do, so results match them bit for bit.
//
// Work decomposition: one workgroup per token row. An item is 8 consecutive
// elements (16 B) of the lower half of a head together with the matching 8 of
// the upper half, so each thread holds both operands of its rotation and every
// access is a 16 B vector load or store; v rows are copied in 16 B items.
// HBM bytes per row: q read + write, k read + write, v read + write, and 2*D
// floats of the cos/sin tables (L2-resident for nearby positions).
#include "nslg_common.h"

namespace nslg {
namespace {

struct RopeArgs {
  const uint16_t* q;
  int64_t q_stride;  // elements between rows
  uint16_t* q_out;
  int64_t q_out_stride;
  const uint16_t* k;
  int64_t k_stride;
  const uint16_t* v;
  int64_t v_stride;
  const int32_t* positions;
  const int32_t* slots;
  const float* cos;
  const float* sin;
  int64_t table_stride;  // floats between table rows
  int64_t table_rows;
  uint16_t* k_pool;
  uint16_t* v_pool;
  int64_t pool_slots;
  int32_t num_qo_heads;
  int32_t num_kv_heads;
};

template <typename T, int D>
__global__ void __launch_bounds__(256) rope_append_kernel(RopeArgs a) {
  constexpr int H = D / 2;
  constexpr int W = 8;
  constexpr int kRotPerHead = H / W;
  constexpr int kCopyPerHead = D / W;
  const int64_t t = blockIdx.x;
  int pos = a.positions[t];
  pos = pos < 0 ? 0 : (pos >= a.table_rows ? (int)(a.table_rows - 1) : pos);
  const int32_t slot = a.slots[t];
  const bool write = slot >= 0 && (int64_t)slot < a.pool_slots;
  const int64_t row_elems = (int64_t)a.num_kv_heads * D;
  const float* crow = a.cos + (int64_t)pos * a.table_stride;
  const float* srow = a.sin + (int64_t)pos * a.table_stride;
  const int rot_items = (a.num_qo_heads + (write ? a.num_kv_heads : 0)) * kRotPerHead;
  const int items = rot_items + (write ? a.num_kv_heads * kCopyPerHead : 0);
  for (int i = threadIdx.x; i < items; i += blockDim.x) {
    if (i < rot_items) {
      const int head = i / kRotPerHead;
      const int j = (i % kRotPerHead) * W;
      const uint16_t* src;
      uint16_t* dst;
      if (head < a.num_qo_heads) {
        src = a.q + t * a.q_stride + (int64_t)head * D;
        dst = a.q_out + t * a.q_out_stride + (int64_t)head * D;
      } else {
        const int kh = head - a.num_qo_heads;
        src = a.k + t * a.k_stride + (int64_t)kh * D;
        dst = a.k_pool + (int64_t)slot * row_elems + (int64_t)kh * D;
      }
      const u16x8 lo = *reinterpret_cast<const u16x8*>(src + j);
      const u16x8 hi = *reinterpret_cast<const u16x8*>(src + H + j);
      float c_lo[8], c_hi[8], s_lo[8], s_hi[8];
      load8f(crow + j, c_lo);
      load8f(crow + H + j, c_hi);
      load8f(srow + j, s_lo);
      load8f(srow + H + j, s_hi);
      u16x8 o_lo, o_hi;
#pragma unroll
      for (int e = 0; e < W; ++e) {
        const float x1 = T::to_f32(lo[e]);
        const float x2 = T::to_f32(hi[e]);
        const float cl = T::to_f32(T::from_f32(c_lo[e]));
        const float ch = T::to_f32(T::from_f32(c_hi[e]));
        const float sl = T::to_f32(T::from_f32(s_lo[e]));
        const float sh = T::to_f32(T::from_f32(s_hi[e]));
        o_lo[e] = rope_elem<T>(x1, cl, -x2, sl);  // d < H: rot = -x[d + H]
        o_hi[e] = rope_elem<T>(x2, ch, x1, sh);   // d >= H: rot = x[d - H]
      }
      if (head < a.num_qo_heads) {  // q: read again right away by the attention kernel
        *reinterpret_cast<u16x8*>(dst + j) = o_lo;
        *reinterpret_cast<u16x8*>(dst + H + j) = o_hi;
      } else {  // pool rows: streamed out (non-temporal)
        stream_store(reinterpret_cast<u16x8*>(dst + j), o_lo);
        stream_store(reinterpret_cast<u16x8*>(dst + H + j), o_hi);
      }
    } else {
      const int k = i - rot_items;
      const int vh = k / kCopyPerHead;
      const int j = (k % kCopyPerHead) * W;
      stream_store(reinterpret_cast<u16x8*>(a.v_pool + (int64_t)slot * row_elems + (int64_t)vh * D + j),
                   *reinterpret_cast<const u16x8*>(a.v + t * a.v_stride + (int64_t)vh * D + j));
    }
  }
}

// fp32 storage: the same items, 8 floats (two 16 B vectors) per half; the products
// are kept apart from the add so each is rounded on its own, as in the eager ops.
__device__ inline float rope_elem_f32(float x, float c, float r, float s) {
  float a = x * c;
  float b = r * s;
  asm volatile("" : "+v"(a), "+v"(b));
  return a + b;
}

template <int D>
__global__ void __launch_bounds__(256) rope_append_f32_kernel(RopeArgs a) {
  constexpr int H = D / 2;
  constexpr int W = 8;
  constexpr int kRotPerHead = H / W;
  constexpr int kCopyPerHead = D / W;
  const int64_t t = blockIdx.x;
  int pos = a.positions[t];
  pos = pos < 0 ? 0 : (pos >= a.table_rows ? (int)(a.table_rows - 1) : pos);
  const int32_t slot = a.slots[t];
  const bool write = slot >= 0 && (int64_t)slot < a.pool_slots;
  const int64_t row_elems = (int64_t)a.num_kv_heads * D;
  const float* crow = a.cos + (int64_t)pos * a.table_stride;
  const float* srow = a.sin + (int64_t)pos * a.table_stride;
  const float* q = reinterpret_cast<const float*>(a.q);
  float* q_out = reinterpret_cast<float*>(a.q_out);
  const float* k = reinterpret_cast<const float*>(a.k);
  const float* v = reinterpret_cast<const float*>(a.v);
  float* k_pool = reinterpret_cast<float*>(a.k_pool);
  float* v_pool = reinterpret_cast<float*>(a.v_pool);
  const int rot_items = (a.num_qo_heads + (write ? a.num_kv_heads : 0)) * kRotPerHead;
  const int items = rot_items + (write ? a.num_kv_heads * kCopyPerHead : 0);
  for (int i = threadIdx.x; i < items; i += blockDim.x) {
    if (i < rot_items) {
      const int head = i / kRotPerHead;
      const int j = (i % kRotPerHead) * W;
      const float* src;
      float* dst;
      if (head < a.num_qo_heads) {
        src = q + t * a.q_stride + (int64_t)head * D;
        dst = q_out + t * a.q_out_stride + (int64_t)head * D;
      } else {
        const int kh = head - a.num_qo_heads;
        src = k + t * a.k_stride + (int64_t)kh * D;
        dst = k_pool + (int64_t)slot * row_elems + (int64_t)kh * D;
      }
      float lo[8], hi[8], c_lo[8], c_hi[8], s_lo[8], s_hi[8];
      load8f(src + j, lo);
      load8f(src + H + j, hi);
      load8f(crow + j, c_lo);
      load8f(crow + H + j, c_hi);
      load8f(srow + j, s_lo);
      load8f(srow + H + j, s_hi);
      float o_lo[8], o_hi[8];
#pragma unroll
      for (int e = 0; e < W; ++e) {
        o_lo[e] = rope_elem_f32(lo[e], c_lo[e], -hi[e], s_lo[e]);  // d < H: rot = -x[d + H]
        o_hi[e] = rope_elem_f32(hi[e], c_hi[e], lo[e], s_hi[e]);   // d >= H: rot = x[d - H]
      }
      const f32x4 w[4] = {f32x4{o_lo[0], o_lo[1], o_lo[2], o_lo[3]}, f32x4{o_lo[4], o_lo[5], o_lo[6], o_lo[7]},
                          f32x4{o_hi[0], o_hi[1], o_hi[2], o_hi[3]}, f32x4{o_hi[4], o_hi[5], o_hi[6], o_hi[7]}};
      f32x4* d4[4] = {reinterpret_cast<f32x4*>(dst + j), reinterpret_cast<f32x4*>(dst + j + 4),
                      reinterpret_cast<f32x4*>(dst + H + j), reinterpret_cast<f32x4*>(dst + H + j + 4)};
      if (head < a.num_qo_heads) {  // q: read again right away by the attention kernel
#pragma unroll
        for (int e = 0; e < 4; ++e) *d4[e] = w[e];
      } else {  // pool rows: streamed out (non-temporal)
#pragma unroll
        for (int e = 0; e < 4; ++e) stream_store(d4[e], w[e]);
      }
    } else {
      const int kk = i - rot_items;
      const int vh = kk / kCopyPerHead;
      const int j = (kk % kCopyPerHead) * W;
      const float* vs = v + t * a.v_stride + (int64_t)vh * D + j;
      float* vd = v_pool + (int64_t)slot * row_elems + (int64_t)vh * D + j;
      stream_store(reinterpret_cast<f32x4*>(vd), *reinterpret_cast<const f32x4*>(vs));
      stream_store(reinterpret_cast<f32x4*>(vd + 4), *reinterpret_cast<const f32x4*>(vs + 4));
    }
  }
}

int launch_rope_f32(const RopeArgs& a, int64_t rows, int head_dim, hipStream_t s) {
  const dim3 grid((unsigned)rows);
  switch (head_dim) {
    case 64: rope_append_f32_kernel<64><<<grid, 256, 0, s>>>(a); break;
    case 128: rope_append_f32_kernel<128><<<grid, 256, 0, s>>>(a); break;
    default: rope_append_f32_kernel<256><<<grid, 256, 0, s>>>(a); break;
  }
  return check_launch("rope_append");
}

template <typename T>
int launch_rope(const RopeArgs& a, int64_t rows, int head_dim, hipStream_t s) {
  const dim3 grid((unsigned)rows);
  switch (head_dim) {
    case 64: rope_append_kernel<T, 64><<<grid, 256, 0, s>>>(a); break;
    case 128: rope_append_kernel<T, 128><<<grid, 256, 0, s>>>(a); break;
    default: rope_append_kernel<T, 256><<<grid, 256, 0, s>>>(a); break;
  }
  return check_launch("rope_append");
}

bool overlaps(const void* a, int64_t a_bytes, const void* b, int64_t b_bytes) {
  const uintptr_t x = (uintptr_t)a, y = (uintptr_t)b;
  return x < y + (uintptr_t)b_bytes && y < x + (uintptr_t)a_bytes;
}

}  // namespace
}  // namespace nslg

using namespace nslg;

extern "C" int nslg_rope_append(const void* q, int64_t q_stride, void* q_out, int64_t q_out_stride,
                                const void* k_new, int64_t k_stride, const void* v_new, int64_t v_stride,
                                const int32_t* positions, const int32_t* slot_mapping, int64_t num_rows,
                                const float* cos_table, const float* sin_table, int64_t table_stride,
                                int64_t table_rows, int32_t num_qo_heads, int32_t num_kv_heads,
                                int32_t head_dim, void* k_pool, void* v_pool, int64_t pool_slots,
                                int32_t dtype, nslg_stream_t stream) {
  if (num_rows < 0 || num_qo_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || pool_slots <= 0 ||
      table_rows <= 0 || table_stride < head_dim)
    return fail(NSLG_EINVAL, "rope_append: bad sizes");
  if (num_rows == 0) return NSLG_OK;
  if (num_rows > 0x7fffffff) return fail(NSLG_EINVAL, "rope_append: too many rows");
  if (!q || !q_out || !k_new || !v_new || !positions || !slot_mapping || !cos_table || !sin_table || !k_pool ||
      !v_pool)
    return fail(NSLG_EINVAL, "rope_append: null pointer");
  if (dtype != NSLG_F16 && dtype != NSLG_BF16 && dtype != NSLG_F32)
    return fail(NSLG_EUNSUPPORTED, "rope_append: dtype %d", dtype);
  const int64_t es = elem_bytes(dtype);
  if (head_dim != 64 && head_dim != 128 && head_dim != 256)
    return fail(NSLG_EUNSUPPORTED, "rope_append: head_dim %d", head_dim);
  const int64_t q_row = (int64_t)num_qo_heads * head_dim;
  const int64_t kv_row = (int64_t)num_kv_heads * head_dim;
  if ((num_rows > 1 && (q_stride < q_row || q_out_stride < q_row || k_stride < kv_row || v_stride < kv_row)) ||
      q_stride < 0 || q_out_stride < 0 || k_stride < 0 || v_stride < 0)
    return fail(NSLG_EINVAL, "rope_append: row stride smaller than the row");
  if (((uintptr_t)q | (uintptr_t)q_out | (uintptr_t)k_new | (uintptr_t)v_new | (uintptr_t)k_pool |
       (uintptr_t)v_pool | (uintptr_t)cos_table | (uintptr_t)sin_table) & 15 ||
      ((q_stride | q_out_stride | k_stride | v_stride) * es) % 16 || table_stride % 4)
    return fail(NSLG_EINVAL, "rope_append: pointers and row strides must be 16-byte aligned");
  const int64_t q_bytes = ((num_rows - 1) * q_stride + q_row) * es;
  const int64_t qo_bytes = ((num_rows - 1) * q_out_stride + q_row) * es;
  if (q_out != q || q_out_stride != q_stride) {
    if (overlaps(q, q_bytes, q_out, qo_bytes))
      return fail(NSLG_EINVAL, "rope_append: q_out overlaps q without being q itself");
  }
  RopeArgs a;
  a.q = (const uint16_t*)q;
  a.q_stride = q_stride;
  a.q_out = (uint16_t*)q_out;
  a.q_out_stride = q_out_stride;
  a.k = (const uint16_t*)k_new;
  a.k_stride = k_stride;
  a.v = (const uint16_t*)v_new;
  a.v_stride = v_stride;
  a.positions = positions;
  a.slots = slot_mapping;
  a.cos = cos_table;
  a.sin = sin_table;
  a.table_stride = table_stride;
  a.table_rows = table_rows;
  a.k_pool = (uint16_t*)k_pool;
  a.v_pool = (uint16_t*)v_pool;
  a.pool_slots = pool_slots;
  a.num_qo_heads = num_qo_heads;
  a.num_kv_heads = num_kv_heads;
  hipStream_t s = as_stream(stream);
  if (dtype == NSLG_F32) return launch_rope_f32(a, num_rows, head_dim, s);
  return dtype == NSLG_F16 ? launch_rope<F16>(a, num_rows, head_dim, s) : launch_rope<BF16>(a, num_rows, head_dim, s);
}
