// Contiguous (non-paged) causal attention: the backend's `prefill` method
// (reference src/minillm/attention/torch_ref.py:20-44, base.py:19-33).
//
// q [B, H, Tq, Dh], k/v [B, Hkv, Tk, Dh] with arbitrary element strides; query i sits at position
// Tk - Tq + i and sees keys 0 .. Tk - Tq + i; with key_valid [B, Tk] it sees only real keys among them,
// and a query that has none sees its own position.  This path serves batch-1 generation and
// correctness checks, not the paged engine step, so it favours generality (fp32/fp16/bf16, any Dh up
// to 256, any strides) over speed: one workgroup per query row, keys in chunks of 256 with an fp32
// online softmax.
#include <math.h>

#include "common.h"

namespace mllm {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxDh = 256;

struct DenseArgs {
  const char* q;
  const char* k;
  const char* v;
  const uint8_t* key_valid;
  char* out;
  int64_t q_sb, q_sh, q_st;
  int64_t k_sb, k_sh, k_st;
  int64_t v_sb, v_sh, v_st;
  int64_t o_sb, o_sh, o_st;
  int64_t kv_sb, kv_st;
  int B, H, Hkv, Tq, Tk, Dh;
  float scale;
};

template <int DT>
__device__ __forceinline__ float ld_elem(const char* base, int64_t idx) {
  if constexpr (DT == MLLM_DTYPE_F32)
    return reinterpret_cast<const float*>(base)[idx];
  else if constexpr (DT == MLLM_DTYPE_BF16)
    return bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(base)[idx]);
  else
    return f16_bits_to_f32(reinterpret_cast<const uint16_t*>(base)[idx]);
}

template <int DT>
__device__ __forceinline__ void st_elem(char* base, int64_t idx, float f) {
  if constexpr (DT == MLLM_DTYPE_F32)
    reinterpret_cast<float*>(base)[idx] = f;
  else if constexpr (DT == MLLM_DTYPE_BF16)
    reinterpret_cast<uint16_t*>(base)[idx] = f32_to_bf16_bits(f);
  else
    reinterpret_cast<uint16_t*>(base)[idx] = f32_to_f16_bits(f);
}

__device__ __forceinline__ float block_max(float v, float* red) {
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  const int wave = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  float r = red[0];
  for (int i = 1; i < kThreads / 64; ++i) r = fmaxf(r, red[i]);
  return r;
}

__device__ __forceinline__ float block_sum(float v, float* red) {
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  const int wave = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  float r = 0.f;
  for (int i = 0; i < kThreads / 64; ++i) r += red[i];
  return r;
}

template <int DT>
__global__ __launch_bounds__(kThreads) void dense_kernel(const DenseArgs a) {
  __shared__ float qs[kMaxDh];
  __shared__ float ps[kThreads];
  __shared__ float red[kThreads / 64];
  const int i = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x;
  const int kvh = h / (a.H / a.Hkv);
  const int qpos = a.Tk - a.Tq + i;
  const char* kb = a.k;
  const int64_t k_row0 = (int64_t)b * a.k_sb + (int64_t)kvh * a.k_sh;
  const int64_t v_row0 = (int64_t)b * a.v_sb + (int64_t)kvh * a.v_sh;
  const int64_t q_row = (int64_t)b * a.q_sb + (int64_t)h * a.q_sh + (int64_t)i * a.q_st;
  for (int d = tid; d < a.Dh; d += kThreads) qs[d] = ld_elem<DT>(a.q, q_row + d);

  // a query with no real key among 0 .. qpos sees only its own position
  bool own_only = false;
  if (a.key_valid) {
    int any = 0;
    for (int j = tid; j <= qpos; j += kThreads) any |= a.key_valid[(int64_t)b * a.kv_sb + (int64_t)j * a.kv_st] != 0;
    own_only = block_sum((float)any, red) == 0.f;
  }
  __syncthreads();

  float m_run = -INFINITY, l_run = 0.f, acc = 0.f;
  for (int j0 = 0; j0 <= qpos; j0 += kThreads) {
    const int j = j0 + tid;
    float s = -INFINITY;
    bool allowed = j <= qpos;
    if (allowed && a.key_valid)
      allowed = own_only ? (j == qpos) : (a.key_valid[(int64_t)b * a.kv_sb + (int64_t)j * a.kv_st] != 0);
    if (allowed) {
      float dot = 0.f;
      const int64_t kr = k_row0 + (int64_t)j * a.k_st;
      for (int d = 0; d < a.Dh; ++d) dot += qs[d] * ld_elem<DT>(kb, kr + d);
      s = dot * a.scale;
    }
    const float cm = block_max(s, red);
    const float m_new = fmaxf(m_run, cm);
    const float p = (s == -INFINITY) ? 0.f : expf(s - m_new);
    ps[tid] = p;
    const float cs = block_sum(p, red);
    const float alpha = (m_run == -INFINITY) ? 0.f : expf(m_run - m_new);
    l_run = l_run * alpha + cs;
    m_run = m_new;
    if (tid < a.Dh) {
      float part = 0.f;
      const int jn = min(kThreads, qpos + 1 - j0);
      for (int jj = 0; jj < jn; ++jj) {
        const float pj = ps[jj];
        if (pj != 0.f) part += pj * ld_elem<DT>(a.v, v_row0 + (int64_t)(j0 + jj) * a.v_st + tid);
      }
      acc = acc * alpha + part;
    }
    __syncthreads();
  }
  if (tid < a.Dh)
    st_elem<DT>(a.out, (int64_t)b * a.o_sb + (int64_t)h * a.o_sh + (int64_t)i * a.o_st + tid, acc / l_run);
}

}  // namespace
}  // namespace mllm

extern "C" int mllm_dense_attention(const void* q, int64_t q_sb, int64_t q_sh, int64_t q_st, const void* k, int64_t k_sb,
                                    int64_t k_sh, int64_t k_st, const void* v, int64_t v_sb, int64_t v_sh, int64_t v_st,
                                    const uint8_t* key_valid, int64_t kv_sb, int64_t kv_st, int32_t batch,
                                    int32_t num_heads, int32_t num_kv_heads, int32_t q_len, int32_t kv_len,
                                    int32_t head_dim, float softmax_scale, int32_t dtype, void* out, int64_t o_sb,
                                    int64_t o_sh, int64_t o_st, void* stream) {
  using namespace mllm;
  MLLM_REQUIRE(dtype >= 0 && dtype <= 2, MLLM_ERR_UNSUPPORTED, "mllm_dense_attention: unsupported dtype");
  MLLM_REQUIRE(batch >= 0 && q_len >= 0 && kv_len >= q_len, MLLM_ERR_INVALID,
               "mllm_dense_attention: need kv_len >= q_len >= 0");
  MLLM_REQUIRE(head_dim > 0 && head_dim <= kMaxDh, MLLM_ERR_UNSUPPORTED, "mllm_dense_attention: head_dim must be in [1, 256]");
  MLLM_REQUIRE(num_kv_heads > 0 && num_heads % num_kv_heads == 0, MLLM_ERR_INVALID,
               "mllm_dense_attention: num_heads must be a multiple of num_kv_heads");
  MLLM_REQUIRE(num_heads <= 65535 && batch <= 65535, MLLM_ERR_UNSUPPORTED, "mllm_dense_attention: grid too large");
  if (batch == 0 || q_len == 0 || num_heads == 0) return MLLM_OK;
  MLLM_REQUIRE(q && k && v && out, MLLM_ERR_INVALID, "mllm_dense_attention: null pointer");
  DenseArgs a{(const char*)q, (const char*)k, (const char*)v, key_valid, (char*)out, q_sb, q_sh, q_st, k_sb, k_sh,
              k_st, v_sb, v_sh, v_st, o_sb, o_sh, o_st, kv_sb, kv_st, batch, num_heads, num_kv_heads, q_len,
              kv_len, head_dim, softmax_scale};
  dim3 grid(q_len, num_heads, batch);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (dtype == MLLM_DTYPE_F32)
    dense_kernel<MLLM_DTYPE_F32><<<grid, kThreads, 0, st>>>(a);
  else if (dtype == MLLM_DTYPE_F16)
    dense_kernel<MLLM_DTYPE_F16><<<grid, kThreads, 0, st>>>(a);
  else
    dense_kernel<MLLM_DTYPE_BF16><<<grid, kThreads, 0, st>>>(a);
  return check_launch("mllm_dense_attention");
}
