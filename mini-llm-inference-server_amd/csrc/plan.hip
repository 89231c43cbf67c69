// Per-step work plan, built on the GPU once per step and reused by every layer (the role of
// FlashInfer's plan(), reference src/minillm/attention/flashinfer_backend.py:44-64).
//
// One workgroup scans the S sequences.
// Decode rows (one new token): their pages, in sequence order, form one stream of T pages, cut into
// nb = ceil(T / C) bins of floor or ceil(T / nb) pages (stream-K).  One decode workgroup streams one bin,
// so every wavefront of the launch gets the same number of pages and the launch is one round of equal
// work, whatever the rows' lengths.  A row's part inside a bin is a segment; a row cut into several
// segments writes fp32 partials, one slot per segment, that the merge combines.
// Rows with several new tokens: ceil(new / q_tile) prefill items, launched longest first (a counting
// sort on the 64-key tiles each item's causal context spans), so the short items fill the tail.
#include "common.h"

namespace mllm {
namespace {

constexpr int kPlanThreads = 1024;
constexpr int kMaxSplitPages = 192;  // pages a decode segment's page-id registers hold
constexpr int kPrefillKeyTile = 64;               // keys per tile of the prefill kernel (its cost unit)
constexpr int kPrefillClasses = kPlanThreads;     // prefill size classes: 1 .. 1023 tiles, the last one open

__device__ __forceinline__ int wg_exclusive_scan(int v, int* sums, int* total) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nwaves = blockDim.x >> 6;
  int x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    int t = __shfl_up(x, off, 64);
    if (lane >= off) x += t;
  }
  if (lane == 63) sums[wave] = x;
  __syncthreads();
  if (wave == 0) {
    int w = lane < nwaves ? sums[lane] : 0;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      int t = __shfl_up(w, off, 64);
      if (lane >= off) w += t;
    }
    if (lane < nwaves) sums[lane] = w;
  }
  __syncthreads();
  const int prefix = wave > 0 ? sums[wave - 1] : 0;
  *total = sums[nwaves - 1];
  __syncthreads();
  return prefix + x - v;
}

// Size class of the prefill item of the row (cached, nn new tokens) whose tokens start at t0: the number of
// key tiles its last token's causal context spans, capped at the last class.
__device__ __forceinline__ int prefill_class(int cached, int t0, int nn, int q_tile) {
  const int kv_end = cached + min(t0 + q_tile, nn);
  return min(max((kv_end + kPrefillKeyTile - 1) / kPrefillKeyTile, 0), kPrefillClasses - 1);
}

// Bin of page p of the step's decode page stream: B(b) <= p < B(b + 1), B(b) = floor(b T / nb).  The
// quotient floor(p nb / T) is that bin or the one before it (every bin holds at least one page: nb <= T).
__device__ __forceinline__ int64_t bin_start(int64_t b, int64_t total, int64_t nb) { return b * total / nb; }
__device__ __forceinline__ int bin_of(int64_t p, int64_t total, int nb) {
  int b = (int)(p * nb / total);
  if (b + 1 < nb && bin_start(b + 1, total, nb) <= p) ++b;
  return b;
}

// split_dev: when not null, the split size is read from device memory (clamped to [pages_per_split, 192]:
// the capacities were sized for pages_per_split, so no item is ever dropped).
__global__ __launch_bounds__(kPlanThreads) void plan_kernel(const int32_t* __restrict__ qo_indptr,
                                                            const int32_t* __restrict__ kv_indptr,
                                                            const int32_t* __restrict__ seq_lens, int32_t num_seqs,
                                                            int32_t pages_per_split_arg,
                                                            const int32_t* __restrict__ split_dev, int32_t q_tile,
                                                            int4* __restrict__ decode_work, int32_t cap_decode,
                                                            int4* __restrict__ merge_work, int32_t cap_merge,
                                                            int4* __restrict__ prefill_work, int32_t cap_prefill) {
  __shared__ int sums[kPlanThreads / 64];
  __shared__ int phist[kPrefillClasses];  // prefill items per size class (tiles, capped)
  __shared__ unsigned long long s_pages;  // decode pages of the step
  const int pages_per_split =
      split_dev ? min(max(*split_dev, pages_per_split_arg), kMaxSplitPages) : pages_per_split_arg;
  for (int i = threadIdx.x; i < kPrefillClasses; i += blockDim.x) phist[i] = 0;
  if (threadIdx.x == 0) s_pages = 0;
  __syncthreads();
  // pass 1: the step's decode pages T, and the prefill items per size class
  for (int base = 0; base < num_seqs; base += kPlanThreads) {
    const int s = base + threadIdx.x;
    const int nn = s < num_seqs ? qo_indptr[s + 1] - qo_indptr[s] : 0;
    if (nn == 1) {
      atomicAdd(&s_pages, (unsigned long long)max(kv_indptr[s + 1] - kv_indptr[s], 0));
    } else if (nn > 1) {
      const int cached = seq_lens[s] - nn;
      for (int t0 = 0; t0 < nn; t0 += q_tile) atomicAdd(&phist[prefill_class(cached, t0, nn, q_tile)], 1);
    }
  }
  __syncthreads();  // every count is in before the scan reads them
  {  // prefill classes in descending order: thread t scans class kPrefillClasses - 1 - t
    const int cls = kPrefillClasses - 1 - (int)threadIdx.x;
    int total;
    const int off = wg_exclusive_scan(phist[cls], sums, &total);
    phist[cls] = off;  // from here on: the next free position of the class
  }
  __syncthreads();
  const int64_t total = (int64_t)s_pages;
  const int nb = total ? (int)((total + pages_per_split - 1) / pages_per_split) : 0;

  // Decode rows' pages, in sequence order, form one stream of T pages cut into nb bins of floor / ceil
  // (T / nb) pages; a row's segment in a bin is the part of the row that bin holds.  Passes 2 and 3 walk
  // the rows with the same scans: pass 2 counts segments, partial slots and merges to check the
  // capacities, pass 3 writes them.
  int n_seg = 0, n_slot = 0, n_merge = 0;
  bool fits = false;
  for (int pass = 2; pass <= 3; ++pass) {
    int64_t base_p = 0;
    int base_g = 0, base_sl = 0, base_m = 0;
    for (int base = 0; base < num_seqs; base += kPlanThreads) {
      const int s = base + threadIdx.x;
      const int nn = s < num_seqs ? qo_indptr[s + 1] - qo_indptr[s] : 0;
      const int pages = nn == 1 ? max(kv_indptr[s + 1] - kv_indptr[s], 0) : 0;
      int tp;
      const int64_t off = base_p + wg_exclusive_scan(pages, sums, &tp);
      int first = 0, nseg = 0;
      if (pages > 0) {
        first = bin_of(off, total, nb);
        nseg = bin_of(off + pages - 1, total, nb) - first + 1;
      }
      const bool cut = nseg > 1;
      int tg, tsl, tm;
      const int g0 = base_g + wg_exclusive_scan(nseg, sums, &tg);
      const int sl0 = base_sl + wg_exclusive_scan(cut ? nseg : 0, sums, &tsl);
      const int m0 = base_m + wg_exclusive_scan(cut ? 1 : 0, sums, &tm);
      if (pass == 3 && fits && nseg > 0) {
        // segment records: {first page in kv_indices, pages, first page within the row, row length},
        // {q row, partial slot (-1: the row's only segment writes the output), sequence, 0}
        int4* segs = decode_work + 1 + nb;
        const int kv0 = kv_indptr[s], len = seq_lens[s], qrow = qo_indptr[s];
        for (int j = 0; j < nseg; ++j) {
          const int b = first + j;
          const int64_t bs0 = bin_start(b, total, nb), bs1 = bin_start(b + 1, total, nb);
          const int lo = (int)(max(off, bs0) - off), hi = (int)(min(off + pages, bs1) - off);
          const int g = g0 + j;
          segs[2 * g] = make_int4(kv0 + lo, hi - lo, lo, len);
          segs[2 * g + 1] = make_int4(qrow, cut ? sl0 + j : -1, s, 0);
          if (j > 0 || bs0 == off) {  // bin b starts in this row
            decode_work[1 + b].x = g;
            decode_work[1 + b].z = 1 + nb;  // the record index of segment 0
          }
          if (bs1 <= off + pages) decode_work[1 + b].y = g + 1;   // and ends in it
        }
        if (cut) merge_work[m0] = make_int4(s, sl0, nseg, 0);
      }
      base_p += tp;
      base_g += tg;
      base_sl += tsl;
      base_m += tm;
    }
    if (pass == 2) {
      n_seg = base_g;
      n_slot = base_sl;
      n_merge = base_m;
      // a step larger than the capacities gets no decode work at all, so the decode and merge kernels
      // never index past a workspace sized for cap_decode partial slots
      fits = nb > 0 && 1 + (int64_t)nb + 2 * (int64_t)n_seg <= cap_decode && n_merge <= cap_merge &&
             n_slot <= (cap_decode - 1) / 2;  // the workspace holds (records - 1) / 2 partial slots
    }
  }
  // header: {nb, segments, partial slots, 0}; a step with decode pages that does not fit reports what it
  // needed instead, {0, records, merges, -1}, and gets no decode work; a step without decode pages {0, 0, 0, 0}
  if (threadIdx.x == 0 && cap_decode > 0) {
    if (fits)
      decode_work[0] = make_int4(nb, n_seg, n_slot, 0);
    else if (nb > 0)
      decode_work[0] = make_int4(0, 1 + nb + 2 * n_seg, n_merge, -1);
    else
      decode_work[0] = make_int4(0, 0, 0, 0);
  }

  // prefill items, longest first
  for (int base = 0; base < num_seqs; base += kPlanThreads) {
    const int s = base + threadIdx.x;
    if (s >= num_seqs) continue;
    const int qs = qo_indptr[s], nn = qo_indptr[s + 1] - qs;
    if (nn <= 1) continue;
    // {seq, t0, qs, nn, cached, kv_start, kv_end, ntiles}: what the prefill kernel reads per item
    const int cached = seq_lens[s] - nn, kv0 = kv_indptr[s];
    for (int t0 = 0; t0 < nn; t0 += q_tile) {
      const int pos = atomicAdd(&phist[prefill_class(cached, t0, nn, q_tile)], 1);
      const int kv_end = cached + min(t0 + q_tile, nn);
      if (pos < cap_prefill) {
        prefill_work[2 * pos] = make_int4(s, t0, qs, nn);
        prefill_work[2 * pos + 1] = make_int4(cached, kv0, kv_end, (kv_end + kPrefillKeyTile - 1) / kPrefillKeyTile);
      }
    }
  }
}

}  // namespace
}  // namespace mllm

namespace {

int plan(const int32_t* qo_indptr, const int32_t* kv_indptr, const int32_t* seq_lens, int32_t num_seqs,
         int32_t pages_per_split,
         const int32_t* split_dev, int32_t q_tile_tokens, int32_t* decode_work, int32_t num_decode_work,
         int32_t* merge_work, int32_t num_merge_work, int32_t* prefill_work, int32_t num_prefill_work, void* stream,
         const char* fn) {
  using namespace mllm;
  const std::string f = fn;
  MLLM_REQUIRE(num_seqs >= 0, MLLM_ERR_INVALID, f + ": num_seqs < 0");
  MLLM_REQUIRE(pages_per_split >= 1 && pages_per_split <= kMaxSplitPages, MLLM_ERR_INVALID,
               f + ": pages_per_split must be in [1, 192]");
  MLLM_REQUIRE(q_tile_tokens >= 1, MLLM_ERR_INVALID, f + ": q_tile_tokens must be positive");
  MLLM_REQUIRE(num_decode_work >= 0 && num_merge_work >= 0 && num_prefill_work >= 0, MLLM_ERR_INVALID,
               f + ": negative capacity");
  MLLM_REQUIRE((num_decode_work == 0 || decode_work) && (num_merge_work == 0 || merge_work) &&
                   (num_prefill_work == 0 || prefill_work),
               MLLM_ERR_INVALID, f + ": null work buffer");
  if (num_seqs == 0) return MLLM_OK;
  MLLM_REQUIRE(qo_indptr && kv_indptr && seq_lens, MLLM_ERR_INVALID, f + ": null indptr or seq_lens");
  plan_kernel<<<1, kPlanThreads, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      qo_indptr, kv_indptr, seq_lens, num_seqs, pages_per_split, split_dev, q_tile_tokens,
      reinterpret_cast<int4*>(decode_work), num_decode_work, reinterpret_cast<int4*>(merge_work), num_merge_work,
      reinterpret_cast<int4*>(prefill_work), num_prefill_work);
  return check_launch(fn);
}

}  // namespace

extern "C" int mllm_plan(const int32_t* qo_indptr, const int32_t* kv_indptr, const int32_t* seq_lens,
                         int32_t num_seqs, int32_t pages_per_split, int32_t q_tile_tokens, int32_t* decode_work,
                         int32_t num_decode_work, int32_t* merge_work, int32_t num_merge_work, int32_t* prefill_work,
                         int32_t num_prefill_work, void* stream) {
  return plan(qo_indptr, kv_indptr, seq_lens, num_seqs, pages_per_split, nullptr, q_tile_tokens, decode_work,
              num_decode_work, merge_work, num_merge_work, prefill_work, num_prefill_work, stream, "mllm_plan");
}

extern "C" int mllm_plan_dev(const int32_t* qo_indptr, const int32_t* kv_indptr, const int32_t* seq_lens,
                             int32_t num_seqs, const int32_t* pages_per_split, int32_t min_pages_per_split,
                             int32_t q_tile_tokens,
                             int32_t* decode_work, int32_t num_decode_work, int32_t* merge_work,
                             int32_t num_merge_work, int32_t* prefill_work, int32_t num_prefill_work, void* stream) {
  using namespace mllm;
  MLLM_REQUIRE(pages_per_split, MLLM_ERR_INVALID, "mllm_plan_dev: null pages_per_split");
  return plan(qo_indptr, kv_indptr, seq_lens, num_seqs, min_pages_per_split, pages_per_split, q_tile_tokens,
              decode_work, num_decode_work, merge_work, num_merge_work, prefill_work, num_prefill_work, stream,
              "mllm_plan_dev");
}
