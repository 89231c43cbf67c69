// KV append: scatter the step's new K and V rows into the paged pool at slot_mapping
// (reference src/minillm/attention/paged_torch_ref.py:23-28, index_copy_ into the flat pool view).
//
// Fast path (same dtype, 16-byte aligned rows): every thread moves one 16-byte chunk, so a token's
// [Hkv, Dh] row (2 KB for 8 x 128 bf16) is written by a run of consecutive threads into one contiguous
// pool row.  K and V are the two halves of one launch (blockIdx.y).  General path: one element per
// thread with a round-to-nearest-even conversion, for mixed dtypes or unaligned strides.
#include "common.h"

namespace mllm {
namespace {

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
