// Internal helpers shared by the gfx950 KV-cache kernels: error reporting,
// dtype traits, 16-bit vector types for the MFMA builtins, wave primitives.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "../../include/nslg_kv.h"

namespace nslg {

// ---- error reporting (thread-local text, integer status) -------------------
void set_error(const char* fmt, ...);
int fail(int code, const char* fmt, ...);
int check_launch(const char* what);

inline int elem_bytes(int dtype) {
  switch (dtype) {
    case NSLG_F16: return 2;
    case NSLG_BF16: return 2;
    case NSLG_F32: return 4;
    default: return 0;
  }
}

inline hipStream_t as_stream(nslg_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// ---- vector types -------------------------------------------------------------
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef unsigned short u16x4 __attribute__((ext_vector_type(4)));
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

// 16-bit element tags. Kernels move raw 16-bit words and only reinterpret them
// at the MFMA / conversion boundary.
struct F16 {
  static constexpr int kDtype = NSLG_F16;
  __device__ static inline float to_f32(unsigned short u) {
    return (float)__builtin_bit_cast(_Float16, u);
  }
  __device__ static inline unsigned short from_f32(float x) {
    return __builtin_bit_cast(unsigned short, (_Float16)x);
  }
  // D[16x16] += A[16x32] * B[32x16]   (8 elements per lane per operand)
  __device__ static inline f32x4 mma_k32(u16x8 a, u16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  // D[16x16] += A[16x16] * B[16x16]   (4 elements per lane per operand)
  __device__ static inline f32x4 mma_k16(u16x4 a, u16x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a),
                                                 __builtin_bit_cast(f16x4, b), c, 0, 0, 0);
  }
};

struct BF16 {
  static constexpr int kDtype = NSLG_BF16;
  __device__ static inline float to_f32(unsigned short u) {
    return __builtin_bit_cast(float, (unsigned int)u << 16);
  }
  __device__ static inline unsigned short from_f32(float x) {
    return __builtin_bit_cast(unsigned short, (__bf16)x);
  }
  __device__ static inline f32x4 mma_k32(u16x8 a, u16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  __device__ static inline f32x4 mma_k16(u16x4 a, u16x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4, a),
                                                     __builtin_bit_cast(i16x4, b), c, 0, 0, 0);
  }
};

// ---- wave helpers ---------------------------------------------------------------
__device__ inline float wave_xor_max(float x, int mask) {
  return fmaxf(x, __shfl_xor(x, mask, 64));
}
__device__ inline float wave_xor_sum(float x, int mask) {
  return x + __shfl_xor(x, mask, 64);
}

// Reductions over the four 16-lane rows of a wave (lanes l, l^16, l^32, l^48) with
// gfx950's row-swap permutes: v_permlane16_swap(x, x) leaves rows {0,0,2,2} in one
// result and {1,1,3,3} in the other, v_permlane32_swap(x, x) rows {0,1,0,1} and
// {2,3,2,3}. VALU only: no LDS instruction, no wait on the LDS counter.
__device__ inline float rows_max(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ inline float rows_sum(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ---- rotary embedding, the eager expression's arithmetic -------------------------
// out[d] = rnd(rnd(x[d] * c) + rnd(rot[d] * s)) in the storage type T, with c and s
// the table values rounded to T and rot = cat(-x[D/2:], x[:D/2]). A 16-bit times
// 16-bit product is exact in fp32 and the sum is done in fp32, as the eager ops do,
// so results match them bit for bit.
template <typename T>
__device__ inline unsigned short rope_elem(float x, float c, float r, float s) {
  float a = T::to_f32(T::from_f32(x * c));
  float b = T::to_f32(T::from_f32(r * s));
  // Both products stay rounded on their own: without this the compiler narrows the
  // ops to 16 bits and fuses one product into the add (v_fma_f16 / v_fma_mix),
  // which rounds once where the eager ops round twice.
  asm volatile("" : "+v"(a), "+v"(b));
  return T::from_f32(a + b);
}

__device__ inline void load8f(const float* p, float (&f)[8]) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(p);
  const f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    f[e] = a[e];
    f[4 + e] = b[e];
  }
}

// Rotates the 8 elements at d0 .. d0 + 7 of one head (lo: d0 < D/2, whose partners
// are at d0 + D/2; else partners at d0 - D/2) at table rows crow / srow: x holds the
// elements, y their partners.
template <typename T, typename V8>
__device__ inline V8 rope8(V8 x, V8 y, const float* crow, const float* srow, int d0, bool lo) {
  float c[8], sn[8];
  load8f(crow + d0, c);
  load8f(srow + d0, sn);
  V8 o;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float xe = T::to_f32(x[e]);
    const float ye = T::to_f32(y[e]);
    const float ce = T::to_f32(T::from_f32(c[e]));
    const float se = T::to_f32(T::from_f32(sn[e]));
    o[e] = lo ? rope_elem<T>(xe, ce, -ye, se) : rope_elem<T>(xe, ce, ye, se);
  }
  return o;
}

// ---- streaming (non-temporal) vector accesses -----------------------------------
// Pool pages written by the append / zero / copy kernels are not read again by the
// writing kernel: stored with the non-temporal hint they go out to HBM instead of
// lingering as dirty lines in the memory-side cache, where the next decode, which
// streams the whole pool, would pay for writing them back (measured: a decode right
// after ~300 MB of ordinary stores into the pool, 590 us instead of 470 us).
template <typename V>
__device__ inline void stream_store(V* p, V v) {
  __builtin_nontemporal_store(v, p);
}

// ---- padded output grids of the prefill entries ----------------------------------
// One workgroup's share of a padded grid of batch x width rows (row_elems elements
// each, rows 16-byte aligned): the rows of sequence b's block (rows b * width ..
// b * width + width - 1) that hold none of its new tokens are set to zero. The
// sequence's n_b = qo[b + 1] - qo[b] tokens sit at rows q_rows[qo[b]] .. + n_b - 1,
// contiguous and inside the block (the forward's padded layout).
template <typename E>
__device__ inline void zero_pad_rows(const int32_t* qo, const int32_t* q_rows, int width, int b, E* out,
                                     int64_t out_stride, int64_t row_elems, int64_t grid_rows) {
  const int q0 = qo[b];
  const int n = qo[b + 1] - q0;
  int64_t first = n > 0 ? (int64_t)q_rows[q0] - (int64_t)b * width : 0;
  first = first < 0 ? 0 : (first > width ? width : first);
  int64_t last = first + (n > 0 ? n : 0);
  last = last > width ? width : last;
  const int64_t vecs = row_elems * (int64_t)sizeof(E) / 16;
  const int64_t pads = width - (last - first);
  const u32x4 z = {0u, 0u, 0u, 0u};
  for (int64_t i = threadIdx.x; i < pads * vecs; i += blockDim.x) {
    const int64_t pr = i / vecs;
    const int64_t r = (int64_t)b * width + (pr < first ? pr : pr + (last - first));
    if (r >= grid_rows) continue;
    *reinterpret_cast<u32x4*>(reinterpret_cast<char*>(out + r * out_stride) + 16 * (i - pr * vecs)) = z;
  }
}

// ---- fp32 attention (attn_f32.hip), shared by the decode and prefill entries ----
struct AttnF32Args {
  int32_t dtype = NSLG_F32;    // element type of q, the pools and out (fp32 only)
  const float* q;
  int64_t q_stride;            // elements between query tokens
  const int32_t* qo_indptr;    // [B+1] new-token offsets; null: one token per sequence
  const int32_t* q_rows = nullptr;  // null, or row of q / out of each new token (a padded grid)
  int32_t grid_width = 0;           // rows per sequence of that grid (q_rows set)
  const float* k_pool;         // one layer, [P, ps, Hkv, D]
  const float* v_pool;
  int64_t num_pages;
  int32_t page_size;
  const int32_t* indptr;
  const int32_t* indices;
  const int32_t* last_len;
  int32_t batch;
  int32_t num_qo_heads;
  int32_t num_kv_heads;
  int32_t group;
  float scale;                 // softmax scale, natural-exponent units
  float* out;
  int64_t out_stride;
  int32_t row_tiles;           // set by attention_f32
  int32_t splits;              // key ranges per row tile (1: no partials)
  float* part_o;               // splits > 1: [total_q, Hq, splits, D] partial outputs
  float* part_ml;              // splits > 1: [total_q, Hq, splits, 2] running max and sum
};
// Launch on stream s; total_q = number of query tokens (B for decode).
int attention_f32(const AttnF32Args& a, int64_t total_q, int32_t head_dim, hipStream_t s);
// Key splits for a decode batch, and the workspace they need.
int attention_f32_splits(int64_t batch, int64_t total_tokens);
size_t attention_f32_workspace(int64_t total_q, int32_t num_qo_heads, int32_t head_dim, int splits);

}  // namespace nslg
