// Ragged metadata build on the GPU (reference src/minillm/attention/metadata.py:70-103).
//
// Launch 1 (one workgroup): exclusive scans over the S sequences -> qo_indptr (scan of num_new),
//   kv_indptr (scan of ceil(len / bs)), plus the per-sequence fields seq_lens, kv_last_page_len and
//   logits_index.
// Launch 2 (one workgroup per sequence): the per-token fields (positions, slot_mapping), the padded
//   block-table row (int64 and int32) and the sequence's page list (kv_indices), all written with
//   coalesced stores from the CSR copy of the block manager's tables.
#include "common.h"

namespace mllm {
namespace {

constexpr int kScanThreads = 1024;

// Inclusive scan of one value per thread over the workgroup; returns the thread's inclusive prefix and
// the workgroup total in *total.
__device__ __forceinline__ int block_inclusive_scan(int v, int* lds_wave_sums, int* total) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nwaves = blockDim.x >> 6;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    int t = __shfl_up(v, off, 64);
    if (lane >= off) v += t;
  }
  if (lane == 63) lds_wave_sums[wave] = v;
  __syncthreads();
  if (wave == 0) {
    int w = lane < nwaves ? lds_wave_sums[lane] : 0;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      int t = __shfl_up(w, off, 64);
      if (lane >= off) w += t;
    }
    if (lane < nwaves) lds_wave_sums[lane] = w;  // inclusive scan of wave sums
  }
  __syncthreads();
  int prefix = wave > 0 ? lds_wave_sums[wave - 1] : 0;
  *total = lds_wave_sums[nwaves - 1];
  __syncthreads();
  return v + prefix;
}

__global__ __launch_bounds__(kScanThreads) void metadata_scan_kernel(
    const int32_t* __restrict__ num_cached, const int32_t* __restrict__ num_new, int32_t num_seqs, int32_t block_size,
    int32_t* __restrict__ qo_indptr, int32_t* __restrict__ kv_indptr, int32_t* __restrict__ seq_lens,
    int32_t* __restrict__ kv_last_page_len, int64_t* __restrict__ logits_index) {
  __shared__ int wave_sums[kScanThreads / 64];
  int carry_q = 0, carry_k = 0;
  if (threadIdx.x == 0) {
    qo_indptr[0] = 0;
    kv_indptr[0] = 0;
  }
  for (int base = 0; base < num_seqs; base += kScanThreads) {
    const int s = base + threadIdx.x;
    int nn = 0, len = 0, pages = 0;
    if (s < num_seqs) {
      nn = num_new[s];
      len = num_cached[s] + nn;
      pages = (len + block_size - 1) / block_size;
    }
    int tq, tk;
    const int iq = block_inclusive_scan(nn, wave_sums, &tq);
    const int ik = block_inclusive_scan(pages, wave_sums, &tk);
    if (s < num_seqs) {
      qo_indptr[s + 1] = carry_q + iq;
      kv_indptr[s + 1] = carry_k + ik;
      if (seq_lens) seq_lens[s] = len;
      if (kv_last_page_len) kv_last_page_len[s] = len - (pages - 1) * block_size;
      if (logits_index) logits_index[s] = (int64_t)(carry_q + iq) - 1;
    }
    carry_q += tq;
    carry_k += tk;
  }
}

__global__ __launch_bounds__(256) void metadata_fill_kernel(
    const int32_t* __restrict__ num_cached, const int32_t* __restrict__ num_new,
    const int32_t* __restrict__ table_indptr, const int32_t* __restrict__ table_ids, int32_t block_size,
    int32_t table_width, const int32_t* __restrict__ qo_indptr, const int32_t* __restrict__ kv_indptr,
    int64_t* __restrict__ positions, int64_t* __restrict__ slot_mapping, int64_t* __restrict__ block_tables,
    int32_t* __restrict__ block_tables_i32, int32_t* __restrict__ kv_indices) {
  const int s = blockIdx.x;
  const int nc = num_cached[s];
  const int nn = num_new[s];
  const int tb = table_indptr[s];
  const int nb = table_indptr[s + 1] - tb;
  const int qs = qo_indptr[s];
  const int ks = kv_indptr[s];
  const int np = kv_indptr[s + 1] - ks;
  const int32_t* ids = table_ids + tb;

  for (int j = threadIdx.x; j < nn; j += blockDim.x) {
    const int p = nc + j;
    if (positions) positions[qs + j] = p;
    if (slot_mapping) slot_mapping[qs + j] = (int64_t)ids[p / block_size] * block_size + p % block_size;
  }
  const int64_t row = (int64_t)s * table_width;
  for (int j = threadIdx.x; j < table_width; j += blockDim.x) {
    const int32_t b = j < nb ? ids[j] : 0;
    if (block_tables) block_tables[row + j] = b;
    if (block_tables_i32) block_tables_i32[row + j] = b;
  }
  if (kv_indices) {
    for (int j = threadIdx.x; j < np; j += blockDim.x) kv_indices[ks + j] = ids[j];
  }
}

}  // namespace
}  // namespace mllm

extern "C" int mllm_build_metadata(const int32_t* num_cached, const int32_t* num_new, const int32_t* table_indptr,
                                   const int32_t* table_ids, int32_t num_seqs, int32_t block_size,
                                   int32_t table_width, int64_t* positions, int64_t* slot_mapping,
                                   int64_t* block_tables, int64_t* logits_index, int32_t* qo_indptr, int32_t* seq_lens,
                                   int32_t* block_tables_i32, int32_t* kv_indptr, int32_t* kv_indices,
                                   int32_t* kv_last_page_len, void* stream) {
  using namespace mllm;
  MLLM_REQUIRE(num_seqs >= 0, MLLM_ERR_INVALID, "mllm_build_metadata: num_seqs < 0");
  MLLM_REQUIRE(block_size > 0, MLLM_ERR_INVALID, "mllm_build_metadata: block_size must be positive");
  MLLM_REQUIRE(table_width >= 0, MLLM_ERR_INVALID, "mllm_build_metadata: table_width < 0");
  MLLM_REQUIRE(qo_indptr && kv_indptr, MLLM_ERR_INVALID, "mllm_build_metadata: qo_indptr and kv_indptr are required");
  if (num_seqs > 0) {
    MLLM_REQUIRE(num_cached && num_new && table_indptr && table_ids, MLLM_ERR_INVALID,
                 "mllm_build_metadata: null input pointer");
  }
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  metadata_scan_kernel<<<1, kScanThreads, 0, st>>>(num_cached, num_new, num_seqs, block_size, qo_indptr, kv_indptr,
                                                   seq_lens, kv_last_page_len, logits_index);
  int rc = check_launch("mllm_build_metadata(scan)");
  if (rc) return rc;
  if (num_seqs == 0) return MLLM_OK;
  metadata_fill_kernel<<<num_seqs, 256, 0, st>>>(num_cached, num_new, table_indptr, table_ids, block_size,
                                                  table_width, qo_indptr, kv_indptr, positions, slot_mapping,
                                                  block_tables, block_tables_i32, kv_indices);
  return check_launch("mllm_build_metadata(fill)");
}
