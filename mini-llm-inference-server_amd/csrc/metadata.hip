// Ragged metadata build on the GPU (reference src/minillm/attention/metadata.py:70-103).
//
// Launch 1 (one workgroup): exclusive scans over the S sequences -> qo_indptr (scan of num_new),
//   kv_indptr (scan of ceil(len / bs)), plus the per-sequence fields seq_lens, kv_last_page_len and
//   logits_index.
// Launch 2 (one workgroup per sequence): the per-token fields (positions, slot_mapping), the padded
//   block-table row (int64 and int32) and the sequence's page list (kv_indices), all written with
//   coalesced stores from the block manager's tables: either a CSR copy uploaded with the step
//   (mllm_build_metadata) or a device-resident mirror with one row per request, read through the step's
//   row ids (mllm_build_metadata_rows), which the caller keeps current with mllm_update_block_tables.
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

// Tables: CSR (table_indptr[S+1] into table_ids) when seq_rows is null; otherwise sequence s reads row
// seq_rows[s] of the resident mirror table_ids[rows x table_stride], of which its first seq_nblk[s] entries
// are its table.
__global__ __launch_bounds__(256) void metadata_fill_kernel(
    const int32_t* __restrict__ num_cached, const int32_t* __restrict__ num_new,
    const int32_t* __restrict__ table_indptr, const int32_t* __restrict__ table_ids,
    const int32_t* __restrict__ seq_rows, const int32_t* __restrict__ seq_nblk, int32_t table_stride,
    int32_t block_size, int32_t table_width, const int32_t* __restrict__ qo_indptr,
    const int32_t* __restrict__ kv_indptr, int64_t* __restrict__ positions, int64_t* __restrict__ slot_mapping,
    int64_t* __restrict__ block_tables, int32_t* __restrict__ block_tables_i32, int32_t* __restrict__ kv_indices) {
  const int s = blockIdx.x;
  const int nc = num_cached[s];
  const int nn = num_new[s];
  int nb;
  const int32_t* ids;
  if (seq_rows) {
    nb = seq_nblk[s];
    ids = table_ids + (int64_t)seq_rows[s] * table_stride;
  } else {
    const int tb = table_indptr[s];
    nb = table_indptr[s + 1] - tb;
    ids = table_ids + tb;
  }
  const int qs = qo_indptr[s];
  const int ks = kv_indptr[s];
  const int np = kv_indptr[s + 1] - ks;

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

// Resident-mirror updates: entry updates[2 i] of the flat table gets block id updates[2 i + 1].
__global__ __launch_bounds__(256) void table_update_kernel(int32_t* __restrict__ tables, int64_t table_size,
                                                           const int32_t* __restrict__ updates, int32_t n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int32_t at = updates[2 * i];
  if (at >= 0 && at < table_size) tables[at] = updates[2 * i + 1];
}

int build(const int32_t* num_cached, const int32_t* num_new, const int32_t* table_indptr, const int32_t* table_ids,
          const int32_t* seq_rows, const int32_t* seq_nblk, int32_t table_stride, int32_t num_seqs,
          int32_t block_size, int32_t table_width, int64_t* positions, int64_t* slot_mapping, int64_t* block_tables,
          int64_t* logits_index, int32_t* qo_indptr, int32_t* seq_lens, int32_t* block_tables_i32,
          int32_t* kv_indptr, int32_t* kv_indices, int32_t* kv_last_page_len, void* stream, const char* fn) {
  const std::string f = fn;
  MLLM_REQUIRE(num_seqs >= 0, MLLM_ERR_INVALID, f + ": num_seqs < 0");
  MLLM_REQUIRE(block_size > 0, MLLM_ERR_INVALID, f + ": block_size must be positive");
  MLLM_REQUIRE(table_width >= 0, MLLM_ERR_INVALID, f + ": table_width < 0");
  MLLM_REQUIRE(qo_indptr && kv_indptr, MLLM_ERR_INVALID, f + ": qo_indptr and kv_indptr are required");
  if (num_seqs > 0) {
    MLLM_REQUIRE(num_cached && num_new && table_ids && (seq_rows ? seq_nblk != nullptr : table_indptr != nullptr),
                 MLLM_ERR_INVALID, f + ": null input pointer");
  }
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  metadata_scan_kernel<<<1, kScanThreads, 0, st>>>(num_cached, num_new, num_seqs, block_size, qo_indptr, kv_indptr,
                                                   seq_lens, kv_last_page_len, logits_index);
  int rc = check_launch((f + "(scan)").c_str());
  if (rc) return rc;
  if (num_seqs == 0) return MLLM_OK;
  metadata_fill_kernel<<<num_seqs, 256, 0, st>>>(num_cached, num_new, table_indptr, table_ids, seq_rows, seq_nblk,
                                                  table_stride, block_size, table_width, qo_indptr, kv_indptr,
                                                  positions, slot_mapping, block_tables, block_tables_i32, kv_indices);
  return check_launch((f + "(fill)").c_str());
}

}  // namespace
}  // namespace mllm

extern "C" int mllm_update_block_tables(int32_t* tables, int64_t table_size, const int32_t* updates,
                                        int32_t num_updates, void* stream) {
  using namespace mllm;
  MLLM_REQUIRE(num_updates >= 0 && table_size >= 0, MLLM_ERR_INVALID, "mllm_update_block_tables: bad sizes");
  if (num_updates == 0) return MLLM_OK;
  MLLM_REQUIRE(tables && updates, MLLM_ERR_INVALID, "mllm_update_block_tables: null pointer");
  table_update_kernel<<<(num_updates + 255) / 256, 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      tables, table_size, updates, num_updates);
  return check_launch("mllm_update_block_tables");
}

extern "C" int mllm_build_metadata_rows(const int32_t* num_cached, const int32_t* num_new, const int32_t* seq_rows,
                                        const int32_t* seq_num_blocks, const int32_t* tables, int32_t table_stride,
                                        int32_t num_seqs, int32_t block_size, int32_t table_width,
                                        int64_t* positions, int64_t* slot_mapping, int64_t* block_tables,
                                        int64_t* logits_index, int32_t* qo_indptr, int32_t* seq_lens,
                                        int32_t* block_tables_i32, int32_t* kv_indptr, int32_t* kv_indices,
                                        int32_t* kv_last_page_len, void* stream) {
  using namespace mllm;
  MLLM_REQUIRE(table_stride > 0, MLLM_ERR_INVALID, "mllm_build_metadata_rows: table_stride must be positive");
  MLLM_REQUIRE(num_seqs == 0 || seq_rows, MLLM_ERR_INVALID, "mllm_build_metadata_rows: null seq_rows");
  return build(num_cached, num_new, nullptr, tables, seq_rows, seq_num_blocks, table_stride, num_seqs, block_size,
               table_width, positions, slot_mapping, block_tables, logits_index, qo_indptr, seq_lens,
               block_tables_i32, kv_indptr, kv_indices, kv_last_page_len, stream, "mllm_build_metadata_rows");
}

extern "C" int mllm_build_metadata(const int32_t* num_cached, const int32_t* num_new, const int32_t* table_indptr,
                                   const int32_t* table_ids, int32_t num_seqs, int32_t block_size,
                                   int32_t table_width, int64_t* positions, int64_t* slot_mapping,
                                   int64_t* block_tables, int64_t* logits_index, int32_t* qo_indptr, int32_t* seq_lens,
                                   int32_t* block_tables_i32, int32_t* kv_indptr, int32_t* kv_indices,
                                   int32_t* kv_last_page_len, void* stream) {
  return mllm::build(num_cached, num_new, table_indptr, table_ids, nullptr, nullptr, 0, num_seqs, block_size,
                     table_width, positions, slot_mapping, block_tables, logits_index, qo_indptr, seq_lens,
                     block_tables_i32, kv_indptr, kv_indices, kv_last_page_len, stream, "mllm_build_metadata");
}
