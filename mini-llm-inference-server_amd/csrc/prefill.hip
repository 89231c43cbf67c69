// Ragged prefill / mixed attention on gfx950 MFMA (reference src/minillm/attention/paged_torch_ref.py:61-73:
// rows with several new tokens, causal within the new chunk and aligned bottom-right over the cached
// prefix; query i of a row with n new tokens and `len` keys sees keys 0 .. len - n + i).
//
// One workgroup (4 wavefronts) per (q tile, KV head).  A q tile is 128 / G new tokens of one row,
// times the G query heads that share the KV head: 128 MFMA rows, 32 per wavefront (rows are
// token-major: row = token * G + head).  K/V are streamed in tiles of 64 keys gathered through
// kv_indices into LDS (double-buffered; the next tile's global loads are in flight while the current
// tile is consumed):
//   K  as Ks[key][dim]  (row stride 136 elements)
//   V  as Vt[dim][key'] (row stride  72 elements), key' a permutation inside each 16-key group
//      (bits 2 and 3 of the key swapped) so that the PV operand of every lane is one 16-byte read.
// Per wavefront and K/V tile:
//   S^T[64 keys x 32 rows] = K . Q^T     2 x 8 v_mfma_f32_32x32x16 (Q^T held in VGPRs for the whole row)
//   O^T[128 x 32 rows]    += V^T . P^T   4 x 4 v_mfma_f32_32x32x16
// S^T and P^T share a lane layout (lane l: row l % 32), so the online softmax (fp32, exp2 domain)
// reduces each row's max and sum inside the lane plus one exchange with lane l ^ 32, and P^T feeds
// the PV product without leaving its lanes.  Tiles entirely above a wavefront's causal diagonal are
// skipped; keys past the tile's causal limit are stored to LDS as zeros.  The grid is 1-D with
// the KV head fastest, so with 8 KV heads each XCD (workgroups are dealt round-robin to the 8 XCDs)
// serves one KV head and keeps that head's shared-prefix pages in its own L2.
#include <math.h>

#include "common.h"

namespace mllm {
namespace {

constexpr int kHeadDim = 128;
constexpr int kBN = 64;          // keys per K/V tile
constexpr int kKs = 136;         // Ks row stride (elements)
constexpr int kVt = 72;          // Vt row stride (elements)
constexpr int kKsElems = kBN * kKs;
constexpr int kVtElems = kHeadDim * kVt;
constexpr int kBufElems = kKsElems + kVtElems;

struct PrefillArgs {
  const uint16_t* q;
  int64_t q_st, q_sh;
  const uint16_t* kc;
  const uint16_t* vc;
  int64_t num_blocks;
  int bs, bs_shift, H, Hkv, G;
  const int32_t* qo_indptr;
  const int32_t* kv_indptr;
  const int32_t* kv_indices;
  const int32_t* seq_lens;
  const int2* work;
  int QT;
  float scale_log2;
  uint16_t* out;
  int64_t o_st, o_sh;
};

// Key position -> position inside the permuted Vt row: within each 16-key group swap bits 2 and 3.
__device__ __forceinline__ int vt_pos(int key) {
  return (key & ~12) | ((key & 4) << 1) | ((key & 8) >> 1);
}

// Page ids of this thread's keys in one K/V tile.  Loaded without branches (a key past the tile's causal
// limit reads the id of the limit's page instead), so the compiler never has to wait on them before
// the tile is needed; validity is applied when the tile is stored to LDS.
struct TileIds {
  int k[4];  // block of each of this thread's 4 K keys
  int v;     // block of this thread's 4 V keys
};

__device__ __forceinline__ TileIds load_ids(const PrefillArgs& a, int pg0, int kv0, int kv_end, int tid) {
  TileIds ids;
  const int last = kv_end - 1;
#pragma unroll
  for (int j = 0; j < 4; ++j) ids.k[j] = a.kv_indices[pg0 + (min(kv0 + tid / 16 + 16 * j, last) >> a.bs_shift)];
  ids.v = a.kv_indices[pg0 + (min(kv0 + 4 * (tid & 15), last) >> a.bs_shift)];
  return ids;
}

struct TileRegs {
  u32x4 k[4];
  u32x4 v[4];
};

__device__ __forceinline__ int64_t pool_row(const PrefillArgs& a, int blk, int key) {
  blk = ((unsigned)blk < (unsigned)a.num_blocks) ? blk : 0;  // never taken with valid metadata
  return ((int64_t)blk << a.bs_shift) + (key & (a.bs - 1));
}

// Issues the tile's global loads (unconditionally: rows past the causal limit are read from a valid
// slot of the same pool and zeroed in store_tile).
__device__ __forceinline__ TileRegs load_data(const PrefillArgs& a, const TileIds& ids, int kv0, int kvh, int tid) {
  TileRegs r;
  const int64_t tok_stride = (int64_t)a.Hkv * kHeadDim;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t row = pool_row(a, ids.k[j], kv0 + tid / 16 + 16 * j);
    r.k[j] = ld16(a.kc + row * tok_stride + kvh * kHeadDim + 8 * (tid & 15));
  }
  const int key0 = kv0 + 4 * (tid & 15);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t row = pool_row(a, ids.v, key0 + i);
    r.v[i] = ld16(a.vc + row * tok_stride + kvh * kHeadDim + 8 * (tid >> 4));
  }
  return r;
}

__device__ __forceinline__ void store_tile(uint16_t* buf, const TileRegs& r, int kv0, int kv_end, int tid) {
  uint16_t* ks = buf;
  uint16_t* vt = buf + kKsElems;
  const u32x4 zero = u32x4{0, 0, 0, 0};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const bool ok = kv0 + tid / 16 + 16 * j < kv_end;
    st16(ks + (tid / 16 + 16 * j) * kKs + 8 * (tid & 15), ok ? r.k[j] : zero);
  }
  // V: this thread holds keys 4kg .. 4kg+3 at dims 8dc .. 8dc+7; write, per dim, the 4 keys as 8 bytes.
  const int kg = tid & 15, dc = tid >> 4;
  const int pos = vt_pos(4 * kg);
  u32x4 v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = kv0 + 4 * kg + i < kv_end ? r.v[i] : zero;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int dw = e >> 1, hf = e & 1;
    u32x2 pk = u32x2{pick_halves(v[0][dw], hf, v[1][dw], hf), pick_halves(v[2][dw], hf, v[3][dw], hf)};
    st8(vt + (8 * dc + e) * kVt + pos, pk);
  }
}

template <typename T>
__global__ __launch_bounds__(256) void prefill_kernel(const PrefillArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * kBufElems];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int kvh = blockIdx.x % a.Hkv;
  const int2 w = a.work[blockIdx.x / a.Hkv];
  const int seq = w.x, t0 = w.y;
  if (seq < 0) return;  // unfilled plan slot (the host pre-fills the plan with -1)
  const int qs = a.qo_indptr[seq];
  const int nn = a.qo_indptr[seq + 1] - qs;
  const int len = a.seq_lens[seq];
  const int cached = len - nn;
  const int pg0 = a.kv_indptr[seq];
  const int tpw = 32 / a.G;  // tokens per wavefront
  const int qt_valid = min(a.QT, nn - t0);
  // keys any row of this workgroup may see
  const int kv_end = min(len, cached + t0 + qt_valid);
  const int ntiles = (kv_end + kBN - 1) / kBN;

  // this lane's row
  const int n = lane & 31, h = lane >> 5;
  const int tok = t0 + wave * tpw + n / a.G;  // new-token index within the row
  const bool row_valid = tok < nn;
  const int qp = row_valid ? cached + tok : len - 1;  // context position of the row's token
  const int wave_tok_hi = min(t0 + wave * tpw + tpw, nn) - 1;
  const int wave_qp_hi = wave_tok_hi >= t0 + wave * tpw ? cached + wave_tok_hi : -1;  // -1: no valid row
  const int wave_qp_lo = cached + t0 + wave * tpw;  // position of the wavefront's first row

  // Q^T operand: lane (n, h) holds row n at dims 16 kk + 8 h .. +7.
  u32x4 qf[8];
  {
    const int head = kvh * a.G + (n % a.G);
    const uint16_t* qp_row = a.q + (int64_t)(qs + (row_valid ? tok : 0)) * a.q_st + (int64_t)head * a.q_sh;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      u32x4 v = ld16(qp_row + 16 * kk + 8 * h);
      qf[kk] = row_valid ? v : u32x4{0, 0, 0, 0};
    }
  }

  f32x16 oacc[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[dt][r] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  TileIds ids_next = load_ids(a, pg0, 0, kv_end, tid);
  TileRegs regs = load_data(a, ids_next, 0, kvh, tid);
  if (ntiles > 1) ids_next = load_ids(a, pg0, kBN, kv_end, tid);
  store_tile(lds, regs, 0, kv_end, tid);
  __syncthreads();

  for (int it = 0; it < ntiles; ++it) {
    const int kv0 = it * kBN;
    if (it + 1 < ntiles) {
      regs = load_data(a, ids_next, kv0 + kBN, kvh, tid);
      if (it + 2 < ntiles) ids_next = load_ids(a, pg0, kv0 + 2 * kBN, kv_end, tid);
    }
    const uint16_t* ks = lds + (it & 1) * kBufElems;
    const uint16_t* vt = ks + kKsElems;

    if (kv0 <= wave_qp_hi) {  // some key of this tile is visible to some row of this wavefront
      f32x16 sacc[2];
#pragma unroll
      for (int b = 0; b < 2; ++b) {
#pragma unroll
        for (int r = 0; r < 16; ++r) sacc[b][r] = 0.f;
        const uint16_t* krow = ks + (32 * b + n) * kKs + 8 * h;
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) sacc[b] = Mfma<T>::m32x32x16(ld16(krow + 16 * kk), qf[kk], sacc[b]);
      }
      // sacc[b][r]: raw score of key kv0 + 32 b + 8 (r / 4) + 4 h + r % 4 for row n.  Only tiles that
      // reach past the wavefront's first row need the causal mask (a wave-uniform test).
      if (kv0 + kBN - 1 > wave_qp_lo) {
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = kv0 + 32 * b + 8 * (r >> 2) + 4 * h + (r & 3);
            sacc[b][r] = key > qp ? -INFINITY : sacc[b][r];
          }
      }
      float mx = -INFINITY;
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int r = 0; r < 16; r += 2) mx = fmaxf(mx, fmaxf(sacc[b][r], sacc[b][r + 1]));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      // Lazy rescale: the running max only moves (and O, l are rescaled) when some row's max grew by
      // more than 2^8 in the exp2 domain; otherwise p = 2^((s - m) c) stays below 256, which fp32
      // accumulation and the bf16 P operand hold exactly as well as values below 1.
      if (__any((mx - m_run) * a.scale_log2 > 8.f)) {
        const float m_new = fmaxf(m_run, mx);
        const float alpha = fast_exp2((m_run - m_new) * a.scale_log2);
        l_run *= alpha;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) oacc[dt] *= alpha;
        m_run = m_new;
      }
      const float mc = m_run * a.scale_log2;
      float ps = 0.f;
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float p = fast_exp2(__builtin_fmaf(sacc[b][r], a.scale_log2, -mc));
          sacc[b][r] = p;
          ps += p;
        }
      ps += __shfl_xor(ps, 32, 64);
      l_run += ps;

#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int r0 = 8 * u;
          const u32x4 pfrag = u32x4{pack2<T>(sacc[b][r0 + 0], sacc[b][r0 + 1]), pack2<T>(sacc[b][r0 + 2], sacc[b][r0 + 3]),
                                    pack2<T>(sacc[b][r0 + 4], sacc[b][r0 + 5]), pack2<T>(sacc[b][r0 + 6], sacc[b][r0 + 7])};
          const uint16_t* vrow = vt + n * kVt + (2 * b + u) * 16 + 8 * h;
#pragma unroll
          for (int dt = 0; dt < 4; ++dt) oacc[dt] = Mfma<T>::m32x32x16(ld16(vrow + 32 * dt * kVt), pfrag, oacc[dt]);
        }
    }

    if (it + 1 < ntiles) store_tile(lds + ((it + 1) & 1) * kBufElems, regs, kv0 + kBN, kv_end, tid);
    __syncthreads();
  }

  if (!row_valid) return;
  const float inv = 1.f / l_run;
  const int head = kvh * a.G + (n % a.G);
  uint16_t* orow = a.out + (int64_t)(qs + tok) * a.o_st + (int64_t)head * a.o_sh;
  // oacc[dt][r]: dim 32 dt + 8 (r / 4) + 4 h + r % 4
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const int r = 4 * g4;
      u32x2 pk = u32x2{pack2<T>(oacc[dt][r] * inv, oacc[dt][r + 1] * inv),
                       pack2<T>(oacc[dt][r + 2] * inv, oacc[dt][r + 3] * inv)};
      st8(orow + 32 * dt + 8 * g4 + 4 * h, pk);
    }
}

}  // namespace
}  // namespace mllm

extern "C" int mllm_paged_prefill(const void* q, int64_t q_stride_tok, int64_t q_stride_head, const void* k_cache,
                                  const void* v_cache, int64_t num_blocks, int32_t block_size, int32_t num_heads,
                                  int32_t num_kv_heads, int32_t head_dim, const int32_t* qo_indptr,
                                  const int32_t* kv_indptr, const int32_t* kv_indices, const int32_t* seq_lens,
                                  const int32_t* prefill_work, int32_t num_prefill_work, int32_t q_tile_tokens,
                                  float softmax_scale, int32_t dtype, void* out, int64_t out_stride_tok,
                                  int64_t out_stride_head, void* stream) {
  using namespace mllm;
  MLLM_REQUIRE(dtype == MLLM_DTYPE_BF16 || dtype == MLLM_DTYPE_F16, MLLM_ERR_UNSUPPORTED,
               "mllm_paged_prefill: dtype must be bfloat16 or float16");
  MLLM_REQUIRE(head_dim == kHeadDim, MLLM_ERR_UNSUPPORTED, "mllm_paged_prefill: head_dim must be 128");
  MLLM_REQUIRE(block_size >= 16 && (block_size & (block_size - 1)) == 0, MLLM_ERR_UNSUPPORTED,
               "mllm_paged_prefill: block_size must be a power of two >= 16");
  MLLM_REQUIRE(num_kv_heads > 0 && num_heads > 0 && num_heads % num_kv_heads == 0, MLLM_ERR_INVALID,
               "mllm_paged_prefill: num_heads must be a multiple of num_kv_heads");
  const int G = num_heads / num_kv_heads;
  MLLM_REQUIRE(32 % G == 0, MLLM_ERR_UNSUPPORTED, "mllm_paged_prefill: H / Hkv must divide 32");
  MLLM_REQUIRE(q_tile_tokens == 128 / G, MLLM_ERR_INVALID, "mllm_paged_prefill: q_tile_tokens must be 128 / (H / Hkv)");
  MLLM_REQUIRE(num_prefill_work >= 0, MLLM_ERR_INVALID, "mllm_paged_prefill: negative count");
  if (num_prefill_work == 0) return MLLM_OK;
  MLLM_REQUIRE(q && k_cache && v_cache && out && qo_indptr && kv_indptr && kv_indices && seq_lens && prefill_work,
               MLLM_ERR_INVALID, "mllm_paged_prefill: null pointer");
  const bool aligned = ((uintptr_t)q % 16 == 0) && ((uintptr_t)out % 8 == 0) && ((uintptr_t)k_cache % 16 == 0) &&
                       ((uintptr_t)v_cache % 16 == 0) && (q_stride_tok * 2) % 16 == 0 &&
                       (q_stride_head * 2) % 16 == 0 && (out_stride_tok * 2) % 8 == 0 && (out_stride_head * 2) % 8 == 0;
  MLLM_REQUIRE(aligned, MLLM_ERR_UNSUPPORTED, "mllm_paged_prefill: q, out and pools need aligned rows");
  MLLM_REQUIRE((int64_t)num_prefill_work * num_kv_heads < (1ll << 31), MLLM_ERR_UNSUPPORTED,
               "mllm_paged_prefill: too many work items");
  PrefillArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.q_st = q_stride_tok;
  a.q_sh = q_stride_head;
  a.kc = static_cast<const uint16_t*>(k_cache);
  a.vc = static_cast<const uint16_t*>(v_cache);
  a.num_blocks = num_blocks;
  a.bs = block_size;
  a.bs_shift = __builtin_ctz((unsigned)block_size);
  a.H = num_heads;
  a.Hkv = num_kv_heads;
  a.G = G;
  a.qo_indptr = qo_indptr;
  a.kv_indptr = kv_indptr;
  a.kv_indices = kv_indices;
  a.seq_lens = seq_lens;
  a.work = reinterpret_cast<const int2*>(prefill_work);
  a.QT = q_tile_tokens;
  a.scale_log2 = softmax_scale * kLog2e;
  a.out = static_cast<uint16_t*>(out);
  a.o_st = out_stride_tok;
  a.o_sh = out_stride_head;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const unsigned grid = (unsigned)num_prefill_work * (unsigned)num_kv_heads;
  if (dtype == MLLM_DTYPE_BF16)
    prefill_kernel<BF16><<<grid, 256, 0, st>>>(a);
  else
    prefill_kernel<F16><<<grid, 256, 0, st>>>(a);
  return check_launch("mllm_paged_prefill");
}
