// Per-step work plan, built on the GPU once per step and reused by every layer (the role of
// FlashInfer's plan(), reference src/minillm/attention/flashinfer_backend.py:44-64).
//
// One workgroup scans the S sequences: a decode row (one new token) of P pages becomes ns = ceil(P / C)
// split-KV items of P / ns pages each (balanced); a row with several new tokens becomes ceil(new / q_tile)
// prefill items.  Both lists are launched longest first (counting sorts: decode items on their size in
// pages, prefill items on the 64-key tiles their causal context spans), so the short items fill the tail
// of each launch.  An exclusive scan gives each decoded row its canonical partial slots.
#include "common.h"

namespace mllm {
namespace {

constexpr int kPlanThreads = 1024;
constexpr int kMaxSplitPages = 128;
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

// split_dev: when not null, the split size is read from device memory (clamped to [pages_per_split, 128]:
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
  __shared__ int hist[kMaxSplitPages + 1];  // decode items per size in pages
  __shared__ int offs[kMaxSplitPages + 1];  // next free position of each size class
  __shared__ int phist[kPrefillClasses];    // prefill items per size class (tiles, capped)
  const int pages_per_split =
      split_dev ? min(max(*split_dev, pages_per_split_arg), kMaxSplitPages) : pages_per_split_arg;
  for (int i = threadIdx.x; i <= kMaxSplitPages; i += blockDim.x) hist[i] = 0;
  for (int i = threadIdx.x; i < kPrefillClasses; i += blockDim.x) phist[i] = 0;
  __syncthreads();
  // pass 1: sizes of the items.  A decode row of P pages gets ns = ceil(P / C) splits of P / ns pages
  // (the first P % ns of them one page more), so every split of a long row holds C/2 .. C pages.  A
  // prefill row gets one item per q_tile new tokens, sized by prefill_class.
  for (int base = 0; base < num_seqs; base += kPlanThreads) {
    const int s = base + threadIdx.x;
    const int nn = s < num_seqs ? qo_indptr[s + 1] - qo_indptr[s] : 0;
    if (nn == 1) {
      const int pages = kv_indptr[s + 1] - kv_indptr[s];
      const int ns = (pages + pages_per_split - 1) / pages_per_split;
      const int q = pages / ns, rem = pages - q * ns;
      atomicAdd(&hist[q], ns - rem);
      if (rem) atomicAdd(&hist[q + 1], rem);
    } else if (nn > 1) {
      const int cached = seq_lens[s] - nn;
      for (int t0 = 0; t0 < nn; t0 += q_tile) atomicAdd(&phist[prefill_class(cached, t0, nn, q_tile)], 1);
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) {  // largest items first: the short ones fill the tail of the launch
    int run = 0;
    for (int sz = kMaxSplitPages; sz >= 1; --sz) {
      offs[sz] = run;
      run += hist[sz];
    }
  }
  {  // prefill classes in descending order: thread t scans class kPrefillClasses - 1 - t
    const int cls = kPrefillClasses - 1 - (int)threadIdx.x;
    int total;
    const int off = wg_exclusive_scan(phist[cls], sums, &total);
    phist[cls] = off;  // from here on: the next free position of the class
  }
  __syncthreads();
  // pass 2: emit.  A decode item carries its row's canonical partial slot (row-major order), which is
  // where the merge looks for it whatever its position in the launch.
  int base_d = 0, base_m = 0;
  for (int base = 0; base < num_seqs; base += kPlanThreads) {
    const int s = base + threadIdx.x;
    int nd = 0, nm = 0, pages = 0;
    bool pf = false;
    if (s < num_seqs) {
      const int nn = qo_indptr[s + 1] - qo_indptr[s];
      pages = kv_indptr[s + 1] - kv_indptr[s];
      if (nn == 1) {
        nd = (pages + pages_per_split - 1) / pages_per_split;
        nm = nd > 1 ? 1 : 0;
      } else {
        pf = nn > 1;
      }
    }
    int td, tm;
    const int od = base_d + wg_exclusive_scan(nd, sums, &td);
    const int om = base_m + wg_exclusive_scan(nm, sums, &tm);
    // An item is emitted only when its position and its partial slot are inside the capacities, and a
    // merge item only when every slot of its row is: a step larger than the caller sized for loses
    // those rows' items instead of writing or reading partials past the workspace.
    for (int j = 0; j < nd; ++j) {
      const int sz = (int)(((int64_t)(j + 1) * pages) / nd - ((int64_t)j * pages) / nd);
      const int pos = atomicAdd(&offs[sz], 1);
      if (pos < cap_decode && od + j < cap_decode) decode_work[pos] = make_int4(s, j, nd, od + j);
    }
    if (nm && om < cap_merge && od + nd <= cap_decode) merge_work[om] = make_int4(s, od, nd, 0);
    if (pf) {  // {seq, t0, qs, nn, cached, kv_start, kv_end, ntiles}: what the prefill kernel reads per item
      const int qs = qo_indptr[s], nn = qo_indptr[s + 1] - qs, cached = seq_lens[s] - nn, kv0 = kv_indptr[s];
      for (int t0 = 0; t0 < nn; t0 += q_tile) {
        const int pos = atomicAdd(&phist[prefill_class(cached, t0, nn, q_tile)], 1);
        const int kv_end = cached + min(t0 + q_tile, nn);
        if (pos < cap_prefill) {
          prefill_work[2 * pos] = make_int4(s, t0, qs, nn);
          prefill_work[2 * pos + 1] = make_int4(cached, kv0, kv_end, (kv_end + kPrefillKeyTile - 1) / kPrefillKeyTile);
        }
      }
    }
    base_d += td;
    base_m += tm;
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
  MLLM_REQUIRE(pages_per_split >= 1 && pages_per_split <= 128, MLLM_ERR_INVALID,
               f + ": pages_per_split must be in [1, 128]");
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
