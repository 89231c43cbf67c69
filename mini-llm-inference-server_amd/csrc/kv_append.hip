// KV append: scatter the step's new K and V rows into the paged pool at slot_mapping
// (reference src/minillm/attention/paged_torch_ref.py:23-28, index_copy_ into the flat pool view).
//
// Fast path (same dtype, 16-byte aligned rows): every thread moves one 16-byte chunk, so a token's
// [Hkv, Dh] row (2 KB for 8 x 128 bf16) is written by a run of consecutive threads into one contiguous
// pool row.  K and V are the two halves of one launch (blockIdx.y).  General path: one element per
// thread with a round-to-nearest-even conversion, for mixed dtypes or unaligned strides.
//
// fp8 pool (mllm_kv_append_fp8, mllm_rope_kv_append_fp8): each element is stored as
// e4m3fn(float(x) * (1 / scale)), the reciprocal taken in fp32 on the host, one per-tensor scale for K
// and one for V; a thread quantizes 16 elements into one 16-byte pool chunk.
#include <type_traits>

#include "common.h"

namespace mllm {
namespace {

template <typename T>
__device__ __forceinline__ float to_f32(uint16_t b) {
  if constexpr (std::is_same<T, BF16>::value)
    return bf16_bits_to_f32(b);
  else
    return f16_bits_to_f32(b);
}
template <typename T>
__device__ __forceinline__ uint16_t from_f32(float f) {
  if constexpr (std::is_same<T, BF16>::value)
    return f32_to_bf16_bits(f);
  else
    return f32_to_f16_bits(f);
}

// Four 16-bit values (two dwords) -> four e4m3fn bytes of x * inv.
template <typename T>
__device__ __forceinline__ uint32_t quant4(uint32_t w0, uint32_t w1, float inv) {
  return f32_to_e4m3fn_bits(to_f32<T>((uint16_t)w0) * inv) |
         (f32_to_e4m3fn_bits(to_f32<T>((uint16_t)(w0 >> 16)) * inv) << 8) |
         (f32_to_e4m3fn_bits(to_f32<T>((uint16_t)w1) * inv) << 16) |
         (f32_to_e4m3fn_bits(to_f32<T>((uint16_t)(w1 >> 16)) * inv) << 24);
}
// Eight 16-bit values (16 bytes) -> eight e4m3fn bytes.
template <typename T>
__device__ __forceinline__ u32x2 quant8(u32x4 x, float inv) {
  return u32x2{quant4<T>(x[0], x[1], inv), quant4<T>(x[2], x[3], inv)};
}

__global__ __launch_bounds__(256) void kv_append_vec_kernel(const char* __restrict__ k, int64_t k_st, int64_t k_sh,
                                                           const char* __restrict__ v, int64_t v_st, int64_t v_sh,
                                                           char* __restrict__ k_cache, char* __restrict__ v_cache,
                                                           int64_t num_slots, int32_t hkv, int32_t chunks_per_head,
                                                           const int64_t* __restrict__ slots, int64_t num_tokens) {
  // strides here are in bytes
  const int64_t per_tok = (int64_t)hkv * chunks_per_head;
  const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= num_tokens * per_tok) return;
  const int64_t t = c / per_tok;
  const int64_t rem = c - t * per_tok;
  const int h = (int)(rem / chunks_per_head);
  const int ch = (int)(rem - (int64_t)h * chunks_per_head);
  const int64_t slot = slots[t];
  if (slot < 0 || slot >= num_slots) return;
  const bool is_v = blockIdx.y != 0;
  const char* src = is_v ? v + t * v_st + h * v_sh : k + t * k_st + h * k_sh;
  char* dst = (is_v ? v_cache : k_cache) + (slot * per_tok + rem) * 16;
  st16(dst, ld16(src + (int64_t)ch * 16));
}

// fp8 pool: one thread per 16 elements of a (token, head) row: 32 source bytes -> one 16-byte chunk.
template <typename T>
__global__ __launch_bounds__(256) void kv_append_fp8_kernel(const char* __restrict__ k, int64_t k_st, int64_t k_sh,
                                                           const char* __restrict__ v, int64_t v_st, int64_t v_sh,
                                                           char* __restrict__ k_cache, char* __restrict__ v_cache,
                                                           int64_t num_slots, int32_t hkv, int32_t chunks_per_head,
                                                           const int64_t* __restrict__ slots, int64_t num_tokens,
                                                           float k_inv, float v_inv) {
  // source strides in bytes
  const int64_t per_tok = (int64_t)hkv * chunks_per_head;
  const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= num_tokens * per_tok) return;
  const int64_t t = c / per_tok;
  const int64_t rem = c - t * per_tok;
  const int h = (int)(rem / chunks_per_head);
  const int ch = (int)(rem - (int64_t)h * chunks_per_head);
  const int64_t slot = slots[t];
  if (slot < 0 || slot >= num_slots) return;
  const bool is_v = blockIdx.y != 0;
  const char* src = (is_v ? v + t * v_st + h * v_sh : k + t * k_st + h * k_sh) + (int64_t)ch * 32;
  const float inv = is_v ? v_inv : k_inv;
  const u32x2 lo = quant8<T>(ld16(src), inv), hi = quant8<T>(ld16(src + 16), inv);
  st16((is_v ? v_cache : k_cache) + (slot * per_tok + rem) * 16, u32x4{lo[0], lo[1], hi[0], hi[1]});
}

template <int SRC, int DST>
__device__ __forceinline__ void move_elem(const char* src, char* dst) {
  if constexpr (SRC == DST) {
    if constexpr (SRC == MLLM_DTYPE_F32)
      *reinterpret_cast<uint32_t*>(dst) = *reinterpret_cast<const uint32_t*>(src);
    else
      *reinterpret_cast<uint16_t*>(dst) = *reinterpret_cast<const uint16_t*>(src);
  } else {
    float f;
    if constexpr (SRC == MLLM_DTYPE_F32)
      f = *reinterpret_cast<const float*>(src);
    else if constexpr (SRC == MLLM_DTYPE_BF16)
      f = bf16_bits_to_f32(*reinterpret_cast<const uint16_t*>(src));
    else
      f = f16_bits_to_f32(*reinterpret_cast<const uint16_t*>(src));
    if constexpr (DST == MLLM_DTYPE_F32)
      *reinterpret_cast<float*>(dst) = f;
    else if constexpr (DST == MLLM_DTYPE_BF16)
      *reinterpret_cast<uint16_t*>(dst) = f32_to_bf16_bits(f);
    else
      *reinterpret_cast<uint16_t*>(dst) = f32_to_f16_bits(f);
  }
}

template <int SRC, int DST>
__global__ __launch_bounds__(256) void kv_append_elem_kernel(const char* __restrict__ k, int64_t k_st, int64_t k_sh,
                                                            const char* __restrict__ v, int64_t v_st, int64_t v_sh,
                                                            char* __restrict__ k_cache, char* __restrict__ v_cache,
                                                            int64_t num_slots, int32_t hkv, int32_t dh,
                                                            const int64_t* __restrict__ slots, int64_t num_tokens) {
  constexpr int ses = SRC == MLLM_DTYPE_F32 ? 4 : 2;
  constexpr int des = DST == MLLM_DTYPE_F32 ? 4 : 2;
  const int64_t per_tok = (int64_t)hkv * dh;
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= num_tokens * per_tok) return;
  const int64_t t = e / per_tok;
  const int64_t rem = e - t * per_tok;
  const int h = (int)(rem / dh);
  const int d = (int)(rem - (int64_t)h * dh);
  const int64_t slot = slots[t];
  if (slot < 0 || slot >= num_slots) return;
  const bool is_v = blockIdx.y != 0;
  const char* src = is_v ? v + (t * v_st + h * v_sh + d) * ses : k + (t * k_st + h * k_sh + d) * ses;
  char* dst = (is_v ? v_cache : k_cache) + (slot * per_tok + rem) * des;
  move_elem<SRC, DST>(src, dst);
}

template <int SRC, int DST>
void launch_elem(dim3 grid, hipStream_t st, const void* k, int64_t k_st, int64_t k_sh, const void* v, int64_t v_st,
                 int64_t v_sh, void* kc, void* vc, int64_t num_slots, int hkv, int dh, const int64_t* slots,
                 int64_t n) {
  kv_append_elem_kernel<SRC, DST><<<grid, 256, 0, st>>>((const char*)k, k_st, k_sh, (const char*)v, v_st, v_sh,
                                                         (char*)kc, (char*)vc, num_slots, hkv, dh, slots, n);
}

int esize(int dtype) { return dtype == MLLM_DTYPE_F32 ? 4 : 2; }

}  // namespace
}  // namespace mllm

extern "C" int mllm_kv_append(const void* k, int64_t k_stride_tok, int64_t k_stride_head, const void* v,
                              int64_t v_stride_tok, int64_t v_stride_head, int32_t src_dtype, void* k_cache,
                              void* v_cache, int32_t cache_dtype, int64_t num_slots, int32_t num_kv_heads,
                              int32_t head_dim, const int64_t* slot_mapping, int64_t num_tokens, void* stream) {
  using namespace mllm;
  MLLM_REQUIRE(src_dtype >= 0 && src_dtype <= 2 && cache_dtype >= 0 && cache_dtype <= 2, MLLM_ERR_UNSUPPORTED,
               "mllm_kv_append: dtype must be float32, float16 or bfloat16");
  MLLM_REQUIRE(num_tokens >= 0 && num_slots >= 0 && num_kv_heads > 0 && head_dim > 0, MLLM_ERR_INVALID,
               "mllm_kv_append: bad sizes");
  if (num_tokens == 0) return MLLM_OK;
  MLLM_REQUIRE(k && v && k_cache && v_cache && slot_mapping, MLLM_ERR_INVALID, "mllm_kv_append: null pointer");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int es = esize(src_dtype);
  const int row_bytes = head_dim * es;
  const bool aligned = src_dtype == cache_dtype && row_bytes % 16 == 0 && ((uintptr_t)k % 16 == 0) &&
                       ((uintptr_t)v % 16 == 0) && ((uintptr_t)k_cache % 16 == 0) && ((uintptr_t)v_cache % 16 == 0) &&
                       (k_stride_tok * es) % 16 == 0 && (k_stride_head * es) % 16 == 0 &&
                       (v_stride_tok * es) % 16 == 0 && (v_stride_head * es) % 16 == 0;
  if (aligned) {
    const int cph = row_bytes / 16;
    const int64_t total = num_tokens * num_kv_heads * cph;
    dim3 grid((unsigned)((total + 255) / 256), 2);
    kv_append_vec_kernel<<<grid, 256, 0, st>>>((const char*)k, k_stride_tok * es, k_stride_head * es,
                                               (const char*)v, v_stride_tok * es, v_stride_head * es,
                                               (char*)k_cache, (char*)v_cache, num_slots, num_kv_heads, cph,
                                               slot_mapping, num_tokens);
    return check_launch("mllm_kv_append");
  }
  const int64_t total = num_tokens * num_kv_heads * head_dim;
  dim3 grid((unsigned)((total + 255) / 256), 2);
#define MLLM_APPEND_CASE(S, D)                                                                                   \
  if (src_dtype == S && cache_dtype == D) {                                                                      \
    launch_elem<S, D>(grid, st, k, k_stride_tok, k_stride_head, v, v_stride_tok, v_stride_head, k_cache, v_cache, \
                      num_slots, num_kv_heads, head_dim, slot_mapping, num_tokens);                              \
    return check_launch("mllm_kv_append");                                                                       \
  }
  MLLM_APPEND_CASE(0, 0)
  MLLM_APPEND_CASE(0, 1)
  MLLM_APPEND_CASE(0, 2)
  MLLM_APPEND_CASE(1, 0)
  MLLM_APPEND_CASE(1, 1)
  MLLM_APPEND_CASE(1, 2)
  MLLM_APPEND_CASE(2, 0)
  MLLM_APPEND_CASE(2, 1)
  MLLM_APPEND_CASE(2, 2)
#undef MLLM_APPEND_CASE
  return fail(MLLM_ERR_UNSUPPORTED, "mllm_kv_append: dtype pair");
}

extern "C" int mllm_kv_append_fp8(const void* k, int64_t k_stride_tok, int64_t k_stride_head, const void* v,
                                  int64_t v_stride_tok, int64_t v_stride_head, int32_t src_dtype, void* k_cache,
                                  void* v_cache, int64_t num_slots, int32_t num_kv_heads, int32_t head_dim,
                                  const int64_t* slot_mapping, int64_t num_tokens, float k_scale, float v_scale,
                                  void* stream) {
  using namespace mllm;
  MLLM_REQUIRE(src_dtype == MLLM_DTYPE_BF16 || src_dtype == MLLM_DTYPE_F16, MLLM_ERR_UNSUPPORTED,
               "mllm_kv_append_fp8: k and v must be bfloat16 or float16");
  MLLM_REQUIRE(num_tokens >= 0 && num_slots >= 0 && num_kv_heads > 0 && head_dim > 0, MLLM_ERR_INVALID,
               "mllm_kv_append_fp8: bad sizes");
  MLLM_REQUIRE(head_dim % 16 == 0, MLLM_ERR_UNSUPPORTED, "mllm_kv_append_fp8: head_dim must be a multiple of 16");
  MLLM_REQUIRE(k_scale > 0.f && v_scale > 0.f && k_scale < INFINITY && v_scale < INFINITY, MLLM_ERR_INVALID,
               "mllm_kv_append_fp8: scales must be positive and finite");
  if (num_tokens == 0) return MLLM_OK;
  MLLM_REQUIRE(k && v && k_cache && v_cache && slot_mapping, MLLM_ERR_INVALID, "mllm_kv_append_fp8: null pointer");
  const bool aligned = ((uintptr_t)k | (uintptr_t)v | (uintptr_t)k_cache | (uintptr_t)v_cache) % 16 == 0 &&
                       (k_stride_tok * 2) % 16 == 0 && (k_stride_head * 2) % 16 == 0 &&
                       (v_stride_tok * 2) % 16 == 0 && (v_stride_head * 2) % 16 == 0;
  MLLM_REQUIRE(aligned, MLLM_ERR_UNSUPPORTED, "mllm_kv_append_fp8: rows must be 16-byte aligned");
  const int cph = head_dim / 16;
  const int64_t total = num_tokens * num_kv_heads * cph;
  MLLM_REQUIRE(total < (1ll << 40), MLLM_ERR_UNSUPPORTED, "mllm_kv_append_fp8: too many tokens");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  dim3 grid((unsigned)((total + 255) / 256), 2);
  const float k_inv = 1.f / k_scale, v_inv = 1.f / v_scale;
  if (src_dtype == MLLM_DTYPE_BF16)
    kv_append_fp8_kernel<BF16><<<grid, 256, 0, st>>>((const char*)k, k_stride_tok * 2, k_stride_head * 2,
                                                     (const char*)v, v_stride_tok * 2, v_stride_head * 2,
                                                     (char*)k_cache, (char*)v_cache, num_slots, num_kv_heads, cph,
                                                     slot_mapping, num_tokens, k_inv, v_inv);
  else
    kv_append_fp8_kernel<F16><<<grid, 256, 0, st>>>((const char*)k, k_stride_tok * 2, k_stride_head * 2,
                                                    (const char*)v, v_stride_tok * 2, v_stride_head * 2,
                                                    (char*)k_cache, (char*)v_cache, num_slots, num_kv_heads, cph,
                                                    slot_mapping, num_tokens, k_inv, v_inv);
  return check_launch("mllm_kv_append_fp8");
}

// ---------------------------------------------------------------- rotary embedding fused with the append
// out[d] = x[d] * cos[d] + rotate_half(x)[d] * sin[d], rotate_half(x) = cat(-x[half:], x[:half])
// (reference src/minillm/model/llama.py:58-72), evaluated the way torch evaluates that expression on
// 16-bit tensors: each product in fp32 (exact for 16-bit operands) rounded to the tensor dtype, then the
// sum in fp32 rounded again.  One thread owns dims [8c, 8c + 8) of both halves of one (token, head)
// row, so each rotation pair stays in the thread; rows are the H query heads (to q_out), then the Hkv
// key heads (rotated, to the pool at the token's slot), then the Hkv value heads (copied to the pool).

namespace mllm {
namespace {

// round(round(x c) + round(r s)) in the 16-bit type.  The rounded products pass through an empty asm:
// for fp16 the compiler narrows these float ops to native half arithmetic and would otherwise fuse the
// first product into the sum's fma, skipping that product's own rounding.
template <typename T>
__device__ __forceinline__ uint16_t rot1(uint16_t x, uint16_t c, float r, uint16_t s) {
  float a = to_f32<T>(from_f32<T>(to_f32<T>(x) * to_f32<T>(c)));
  float b = to_f32<T>(from_f32<T>(r * to_f32<T>(s)));
  asm volatile("" : "+v"(a), "+v"(b));
  return from_f32<T>(a + b);
}

union Chunk {
  u32x4 v;
  uint16_t e[8];
};

// Q8: the pool is e4m3fn: the rotated k (rounded to T, as the unfused sequence stores it before the
// append) and v are quantized with k_inv / v_inv, 8 bytes per half row instead of 16.
template <typename T, bool Q8>
__global__ __launch_bounds__(256) void rope_append_kernel(
    const char* __restrict__ q, int64_t q_st, int64_t q_sh, const char* __restrict__ k, int64_t k_st, int64_t k_sh,
    const char* __restrict__ v, int64_t v_st, int64_t v_sh, const char* __restrict__ cosp,
    const char* __restrict__ sinp, int64_t cs_st, char* __restrict__ q_out, int64_t qo_st, int64_t qo_sh,
    char* __restrict__ k_cache, char* __restrict__ v_cache, int64_t num_slots, int32_t H, int32_t Hkv,
    int32_t half_bytes, int32_t chunks, const int64_t* __restrict__ slots, int64_t num_tokens, float k_inv,
    float v_inv) {
  // strides in bytes; one thread = one 16-byte chunk of the first half and its partner in the second
  const int rows = H + 2 * Hkv;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= num_tokens * rows * chunks) return;
  const int64_t t = i / ((int64_t)rows * chunks);
  const int rem = (int)(i - t * rows * chunks);
  const int row = rem / chunks;
  const int64_t lo = (int64_t)(rem - row * chunks) * 16;  // byte offset of the chunk in the first half
  const int64_t row_bytes = 2 * (int64_t)half_bytes;
  const int64_t pool_row = Q8 ? row_bytes / 2 : row_bytes;  // bytes of one (slot, head) row of the pool
  const char* src;
  char* dst;
  bool rotate = true, to_pool = false;
  float inv = 1.f;
  if (row < H) {
    src = q + t * q_st + row * q_sh;
    dst = q_out + t * qo_st + row * qo_sh;
  } else {
    const int64_t slot = slots[t];
    if (slot < 0 || slot >= num_slots) return;
    const int kh = row - H;
    to_pool = true;
    if (kh < Hkv) {
      src = k + t * k_st + kh * k_sh;
      dst = k_cache + (slot * Hkv + kh) * pool_row;
      inv = k_inv;
    } else {
      src = v + t * v_st + (kh - Hkv) * v_sh;
      dst = v_cache + (slot * Hkv + kh - Hkv) * pool_row;
      rotate = false;
      inv = v_inv;
    }
  }
  Chunk x1, x2;
  x1.v = ld16(src + lo);
  x2.v = ld16(src + half_bytes + lo);
  if (rotate) {
    Chunk c1, c2, s1, s2, o1, o2;
    const char* cr = cosp + t * cs_st;
    const char* sr = sinp + t * cs_st;
    c1.v = ld16(cr + lo);
    c2.v = ld16(cr + half_bytes + lo);
    s1.v = ld16(sr + lo);
    s2.v = ld16(sr + half_bytes + lo);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      o1.e[e] = rot1<T>(x1.e[e], c1.e[e], -to_f32<T>(x2.e[e]), s1.e[e]);  // d < half: rotate_half = -x[d + half]
      o2.e[e] = rot1<T>(x2.e[e], c2.e[e], to_f32<T>(x1.e[e]), s2.e[e]);   // d >= half: rotate_half = x[d - half]
    }
    x1 = o1;
    x2 = o2;
  }
  if (Q8 && to_pool) {
    st8(dst + lo / 2, quant8<T>(x1.v, inv));
    st8(dst + half_bytes / 2 + lo / 2, quant8<T>(x2.v, inv));
    return;
  }
  st16(dst + lo, x1.v);
  st16(dst + half_bytes + lo, x2.v);
}

}  // namespace
}  // namespace mllm

namespace {

int rope_kv_append(const void* q, int64_t q_stride_tok, int64_t q_stride_head, const void* k, int64_t k_stride_tok,
                   int64_t k_stride_head, const void* v, int64_t v_stride_tok, int64_t v_stride_head, const void* cos,
                   const void* sin, int64_t cs_stride_tok, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                   int32_t dtype, void* q_out, int64_t q_out_stride_tok, int64_t q_out_stride_head, void* k_cache,
                   void* v_cache, int64_t num_slots, const int64_t* slot_mapping, int64_t num_tokens, bool fp8,
                   float k_scale, float v_scale, void* stream) {
  using namespace mllm;
  const std::string fn = fp8 ? "mllm_rope_kv_append_fp8" : "mllm_rope_kv_append";
  MLLM_REQUIRE(dtype == MLLM_DTYPE_BF16 || dtype == MLLM_DTYPE_F16, MLLM_ERR_UNSUPPORTED,
               fn + ": dtype must be bfloat16 or float16");
  MLLM_REQUIRE(num_tokens >= 0 && num_slots >= 0 && num_heads > 0 && num_kv_heads > 0 && head_dim > 0,
               MLLM_ERR_INVALID, fn + ": bad sizes");
  MLLM_REQUIRE(head_dim % 16 == 0, MLLM_ERR_UNSUPPORTED, fn + ": head_dim must be a multiple of 16");
  MLLM_REQUIRE(k_scale > 0.f && v_scale > 0.f && k_scale < INFINITY && v_scale < INFINITY, MLLM_ERR_INVALID,
               fn + ": scales must be positive and finite");
  if (num_tokens == 0) return MLLM_OK;
  MLLM_REQUIRE(q && k && v && cos && sin && q_out && k_cache && v_cache && slot_mapping, MLLM_ERR_INVALID,
               fn + ": null pointer");
  const int64_t strides[] = {q_stride_tok, q_stride_head, k_stride_tok, k_stride_head, v_stride_tok,
                             v_stride_head, cs_stride_tok, q_out_stride_tok, q_out_stride_head};
  bool aligned = ((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)cos | (uintptr_t)sin | (uintptr_t)q_out |
                  (uintptr_t)k_cache | (uintptr_t)v_cache) % 16 == 0;
  for (int64_t s : strides) aligned = aligned && (s * 2) % 16 == 0;
  MLLM_REQUIRE(aligned, MLLM_ERR_UNSUPPORTED, fn + ": rows must be 16-byte aligned");
  const int chunks = head_dim / 16;  // 16-byte chunks per half row
  const int64_t total = num_tokens * (num_heads + 2 * num_kv_heads) * chunks;
  MLLM_REQUIRE(total < (1ll << 40), MLLM_ERR_UNSUPPORTED, fn + ": too many tokens");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const unsigned grid = (unsigned)((total + 255) / 256);
  const float k_inv = 1.f / k_scale, v_inv = 1.f / v_scale;
  auto launch = [&](auto tag, auto q8) {
    using T = decltype(tag);
    rope_append_kernel<T, decltype(q8)::value><<<grid, 256, 0, st>>>(
        (const char*)q, q_stride_tok * 2, q_stride_head * 2, (const char*)k, k_stride_tok * 2, k_stride_head * 2,
        (const char*)v, v_stride_tok * 2, v_stride_head * 2, (const char*)cos, (const char*)sin, cs_stride_tok * 2,
        (char*)q_out, q_out_stride_tok * 2, q_out_stride_head * 2, (char*)k_cache, (char*)v_cache, num_slots,
        num_heads, num_kv_heads, head_dim, chunks, slot_mapping, num_tokens, k_inv, v_inv);
  };
  if (dtype == MLLM_DTYPE_BF16) {
    if (fp8)
      launch(BF16{}, std::true_type{});
    else
      launch(BF16{}, std::false_type{});
  } else {
    if (fp8)
      launch(F16{}, std::true_type{});
    else
      launch(F16{}, std::false_type{});
  }
  return check_launch(fn.c_str());
}

}  // namespace

extern "C" int mllm_rope_kv_append(const void* q, int64_t q_stride_tok, int64_t q_stride_head, const void* k,
                                   int64_t k_stride_tok, int64_t k_stride_head, const void* v, int64_t v_stride_tok,
                                   int64_t v_stride_head, const void* cos, const void* sin, int64_t cs_stride_tok,
                                   int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t dtype,
                                   void* q_out, int64_t q_out_stride_tok, int64_t q_out_stride_head, void* k_cache,
                                   void* v_cache, int64_t num_slots, const int64_t* slot_mapping, int64_t num_tokens,
                                   void* stream) {
  return rope_kv_append(q, q_stride_tok, q_stride_head, k, k_stride_tok, k_stride_head, v, v_stride_tok,
                        v_stride_head, cos, sin, cs_stride_tok, num_heads, num_kv_heads, head_dim, dtype, q_out,
                        q_out_stride_tok, q_out_stride_head, k_cache, v_cache, num_slots, slot_mapping, num_tokens,
                        false, 1.f, 1.f, stream);
}

extern "C" int mllm_rope_kv_append_fp8(const void* q, int64_t q_stride_tok, int64_t q_stride_head, const void* k,
                                       int64_t k_stride_tok, int64_t k_stride_head, const void* v,
                                       int64_t v_stride_tok, int64_t v_stride_head, const void* cos, const void* sin,
                                       int64_t cs_stride_tok, int32_t num_heads, int32_t num_kv_heads,
                                       int32_t head_dim, int32_t dtype, void* q_out, int64_t q_out_stride_tok,
                                       int64_t q_out_stride_head, void* k_cache, void* v_cache, int64_t num_slots,
                                       const int64_t* slot_mapping, int64_t num_tokens, float k_scale, float v_scale,
                                       void* stream) {
  return rope_kv_append(q, q_stride_tok, q_stride_head, k, k_stride_tok, k_stride_head, v, v_stride_tok,
                        v_stride_head, cos, sin, cs_stride_tok, num_heads, num_kv_heads, head_dim, dtype, q_out,
                        q_out_stride_tok, q_out_stride_head, k_cache, v_cache, num_slots, slot_mapping, num_tokens,
                        true, k_scale, v_scale, stream);
}
