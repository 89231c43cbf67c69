// Ragged prefill / mixed attention on gfx950 MFMA (reference src/minillm/attention/paged_torch_ref.py:61-73:
// rows with several new tokens, causal within the new chunk and aligned bottom-right over the cached
// prefix; query i of a row with n new tokens and `len` keys sees keys 0 .. len - n + i).
//
// One workgroup (8 wavefronts) per (q tile, KV head).  A q tile is 256 / G new tokens of one row,
// times the G query heads that share the KV head: 256 MFMA rows, 32 per wavefront (rows are
// token-major: row = token * G + head).  K/V are streamed in tiles of 64 keys gathered through
// kv_indices into LDS (two buffers each):
//   K  as Ks[key][dim]  (row stride 136 elements)
//   V  as Vt[dim][key'] (row stride  72 elements), key' a permutation inside each 16-key group
//      (bits 2 and 3 of the key swapped) so that the PV operand of every lane is one 16-byte read.
// Per wavefront and K/V tile:
//   S^T[64 keys x 32 rows] = K . Q^T     2 x 8 v_mfma_f32_32x32x16 (Q^T held in VGPRs for the whole row)
//   O^T[128 x 32 rows]    += V^T . P^T   4 x 4 v_mfma_f32_32x32x16
// S^T and P^T share a lane layout (lane l: row l % 32), so the online softmax (fp32, exp2 domain)
// reduces each row's max and sum inside the lane plus one exchange with lane l ^ 32, and P^T feeds
// the PV product without leaving its lanes.
//
// The two halves of the workgroup run phase-shifted (see prefill_kernel): one half's matrix phase
// coincides with the other half's softmax, so every SIMD has an MFMA stream and a vector stream at
// once.  Tiles entirely above a wavefront's causal diagonal are skipped; keys past the tile's causal
// limit are stored to LDS as zeros.  The grid is 1-D with the KV head fastest, so with 8 KV heads
// each XCD (workgroups are dealt round-robin to the 8 XCDs) serves one KV head and keeps that head's
// shared-prefix pages in its own L2.
#include <math.h>

#include "common.h"

namespace mllm {
namespace {

constexpr int kHeadDim = 128;
constexpr int kBN = 64;   // keys per K/V tile
constexpr int kKs = 136;  // Ks row stride (elements)
constexpr int kVt = 72;   // Vt row stride (elements)
constexpr int kKsElems = kBN * kKs;
constexpr int kVtElems = kHeadDim * kVt;
constexpr int kQTileRows = 256;  // query rows (token x head of the group) per workgroup: 8 waves x 32

struct PrefillArgs {
  const uint16_t* q;
  int64_t q_st, q_sh;
  const uint16_t* kc;
  const uint16_t* vc;
  int64_t num_blocks;
  unsigned page_bytes;  // bytes of one block of one pool: bs * Hkv * Dh * 2 (< 2^32)
  int row_bytes;        // bytes of one token row: Hkv * Dh * 2 (< 2^24)
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
__device__ __forceinline__ int vt_pos(int key) { return (key & ~12) | ((key & 4) << 1) | ((key & 8) >> 1); }

// Page ids are loaded without branches (a key past the causal limit reads the id of the limit's
// page), so the compiler never waits on them early; validity is applied when a tile is stored.
// Thread tid handles K keys tid / 16 + 16 j (j < 4), dims 8 (tid % 16) .. +7, and V keys
// 4 (tid % 16) .. +3, dims 8 (tid / 16) .. +7.
struct KIds {
  int b[4];
};

__device__ __forceinline__ KIds k_ids(const PrefillArgs& a, const int32_t* pages, int kv0, int last, int tid) {
  KIds ids;
#pragma unroll
  for (int j = 0; j < 4; ++j) ids.b[j] = pages[(unsigned)min(kv0 + tid / 16 + 16 * j, last) >> a.bs_shift];
  return ids;
}

__device__ __forceinline__ int v_id(const PrefillArgs& a, const int32_t* pages, int kv0, int last, int tid) {
  return pages[(unsigned)min(kv0 + 4 * (tid & 15), last) >> a.bs_shift];
}

// pool + block * page_bytes + slot * row_bytes + col_bytes (slot < block_size and row_bytes < 2^24, so
// the in-page product is a 24-bit multiply).
__device__ __forceinline__ const char* row_ptr(const char* pool, const PrefillArgs& a, int blk, int slot,
                                               int col_bytes) {
  const unsigned b = ((unsigned)blk < (unsigned)a.num_blocks) ? (unsigned)blk : 0u;  // else-branch never taken
  const unsigned in_page = __umul24((unsigned)slot, (unsigned)a.row_bytes) + (unsigned)col_bytes;
  return pool + ((uint64_t)b * a.page_bytes + in_page);
}

struct Regs4 {
  u32x4 x[4];
};

// Global loads of one tile (issued unconditionally; rows past the causal limit come from a valid slot
// and are zeroed when stored).
__device__ __forceinline__ Regs4 load_k(const PrefillArgs& a, const KIds& ids, int kv0, int kvh, int tid) {
  Regs4 r;
  const char* kc = reinterpret_cast<const char*>(a.kc);
  const int col = kvh * kHeadDim * 2 + 16 * (tid & 15);
#pragma unroll
  for (int j = 0; j < 4; ++j) r.x[j] = ld16(row_ptr(kc, a, ids.b[j], (kv0 + tid / 16 + 16 * j) & (a.bs - 1), col));
  return r;
}

__device__ __forceinline__ Regs4 load_v(const PrefillArgs& a, int id, int kv0, int kvh, int tid) {
  Regs4 r;
  const char* vp = row_ptr(reinterpret_cast<const char*>(a.vc), a, id, (kv0 + 4 * (tid & 15)) & (a.bs - 1),
                           kvh * kHeadDim * 2 + 16 * (tid >> 4));
#pragma unroll
  for (int i = 0; i < 4; ++i) r.x[i] = ld16(vp + i * a.row_bytes);
  return r;
}

// LDS stores of one tile; keys at or past kv_end become zeros (only a row's last tile has any).
__device__ __forceinline__ void store_k(uint16_t* ks, Regs4 r, int kv0, int kv_end, int tid) {
  if (kv0 + kBN > kv_end) {
#pragma unroll
    for (int j = 0; j < 4; ++j) r.x[j] = kv0 + tid / 16 + 16 * j < kv_end ? r.x[j] : u32x4{0, 0, 0, 0};
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) st16(ks + (tid / 16 + 16 * j) * kKs + 8 * (tid & 15), r.x[j]);
}

__device__ __forceinline__ void store_v(uint16_t* vt, Regs4 r, int kv0, int kv_end, int tid) {
  const int kg = tid & 15, dc = tid >> 4;
  if (kv0 + kBN > kv_end) {
#pragma unroll
    for (int i = 0; i < 4; ++i) r.x[i] = kv0 + 4 * kg + i < kv_end ? r.x[i] : u32x4{0, 0, 0, 0};
  }
  // this thread holds keys 4kg .. 4kg+3 at dims 8dc .. 8dc+7; write, per dim, the 4 keys as 8 bytes
  const int pos = vt_pos(4 * kg);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int dw = e >> 1, hf = e & 1;
    const u32x2 pk =
        u32x2{pick_halves(r.x[0][dw], hf, r.x[1][dw], hf), pick_halves(r.x[2][dw], hf, r.x[3][dw], hf)};
    st8(vt + (8 * dc + e) * kVt + pos, pk);
  }
}

struct STile {
  f32x16 s[2];  // s[b][r]: key 32 b + 8 (r / 4) + 4 h + r % 4 of the tile, row n
};

// The two 32-key halves are independent accumulation chains; alternating them keeps two MFMAs in
// flight instead of waiting on each accumulator in turn.
template <typename T>
__device__ __forceinline__ STile scores(const uint16_t* ks, const u32x4 (&qf)[8], int n, int h) {
  STile t;
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) t.s[b][r] = 0.f;
  const uint16_t* krow = ks + n * kKs + 8 * h;
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) {
    const u32x4 k0 = ld16(krow + 16 * kk);
    const u32x4 k1 = ld16(krow + 32 * kKs + 16 * kk);
    t.s[0] = Mfma<T>::m32x32x16(k0, qf[kk], t.s[0]);
    t.s[1] = Mfma<T>::m32x32x16(k1, qf[kk], t.s[1]);
  }
  return t;
}

// Softmax of one score tile (online, exp2 domain) -> the bf16/fp16 P^T operands of its PV product.
// Masks keys past each row's position when the tile reaches past the wavefront's first row; rescales
// O and l lazily: only when some row's max grew by more than 2^8, otherwise p = 2^((s - m) c) stays
// below 256, which the fp32 accumulation and the P operand hold as exactly as values below 1.
template <typename T>
__device__ __forceinline__ void softmax_tile(STile& st, u32x4 (&pf)[2][2], f32x16 (&oacc)[4], float& m_run,
                                             float& l_run, int kv0, int qp, int wave_qp_lo, int h, float c) {
  if (kv0 + kBN - 1 > wave_qp_lo) {
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kv0 + 32 * b + 8 * (r >> 2) + 4 * h + (r & 3);
        st.s[b][r] = key > qp ? -INFINITY : st.s[b][r];
      }
  }
  float mx = -INFINITY;
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int r = 0; r < 16; r += 2) mx = __builtin_fmaxf(__builtin_fmaxf(mx, st.s[b][r]), st.s[b][r + 1]);
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
  if (__any((mx - m_run) * c > 8.f)) {
    const float m_new = fmaxf(m_run, mx);
    const float alpha = fast_exp2((m_run - m_new) * c);
    l_run *= alpha;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) oacc[dt] *= alpha;
    m_run = m_new;
  }
  const float mc = m_run * c;
  float ps = 0.f;
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float p = fast_exp2(__builtin_fmaf(st.s[b][r], c, -mc));
      st.s[b][r] = p;
      ps += p;
    }
  ps += __shfl_xor(ps, 32, 64);
  l_run += ps;
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int r0 = 8 * u;
      pf[b][u] = u32x4{pack2<T>(st.s[b][r0 + 0], st.s[b][r0 + 1]), pack2<T>(st.s[b][r0 + 2], st.s[b][r0 + 3]),
                       pack2<T>(st.s[b][r0 + 4], st.s[b][r0 + 5]), pack2<T>(st.s[b][r0 + 6], st.s[b][r0 + 7])};
    }
}

// O^T += V^T . P^T for one tile: 16 MFMAs, the four 32-dim output tiles as independent chains.
template <typename T>
__device__ __forceinline__ void pv_tile(const uint16_t* vt, const u32x4 (&pf)[2][2], f32x16 (&oacc)[4], int n,
                                        int h) {
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const uint16_t* vrow = vt + n * kVt + (2 * b + u) * 16 + 8 * h;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) oacc[dt] = Mfma<T>::m32x32x16(ld16(vrow + 32 * dt * kVt), pf[b][u], oacc[dt]);
    }
}

// Two wavefront groups of one workgroup, phase-shifted by half an iteration: while group A (waves
// 0-3) runs its matrix phase, group B (waves 4-7) runs its vector phase, and the next barrier swaps
// them, so each SIMD (one wave of each group) keeps its matrix pipe and its vector ALU busy together.
//   matrix phase i : O += V(i) P(i)  and  S(i+1) = K(i+1) Q^T
//   vector phase   : P(i+1) = softmax(S(i+1)) (group B's vector phase runs half an iteration earlier)
// Group A also stages K (K(i+2) into the buffer of K(i), then issues the loads of K(i+3)); group B
// stages V (V(i+1) over V(i-1), loads of V(i+2)), each in its vector phase.  Every buffer is rewritten
// only after both groups' last read of it, one barrier earlier.
template <typename T>
__global__ __launch_bounds__(512) void prefill_kernel(const PrefillArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * kKsElems + 2 * kVtElems];
  uint16_t* const kbuf0 = lds;
  uint16_t* const vbuf0 = lds + 2 * kKsElems;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int grp = wave >> 2;  // 0: matrix phase first, stages K; 1: vector phase first, stages V
  const int gtid = tid & 255;
  const int kvh = blockIdx.x % a.Hkv;
  const int2 w = a.work[blockIdx.x / a.Hkv];
  const int seq = w.x, t0 = w.y;
  if (seq < 0) return;  // unfilled plan slot (the host pre-fills the plan with -1)
  const int qs = a.qo_indptr[seq];
  const int nn = a.qo_indptr[seq + 1] - qs;
  const int len = a.seq_lens[seq];
  const int cached = len - nn;
  const int32_t* pages = a.kv_indices + a.kv_indptr[seq];
  const int tpw = 32 / a.G;  // tokens per wavefront
  const int qt_valid = min(a.QT, nn - t0);
  const int kv_end = min(len, cached + t0 + qt_valid);  // keys any row of this workgroup may see
  const int last = kv_end - 1;
  const int ntiles = (kv_end + kBN - 1) / kBN;

  const int n = lane & 31, h = lane >> 5;
  const int tok = t0 + wave * tpw + n / a.G;  // new-token index within the row
  const bool row_valid = tok < nn;
  const int qp = row_valid ? cached + tok : len - 1;  // context position of the row's token
  const int wave_tok_hi = min(t0 + wave * tpw + tpw, nn) - 1;
  const int wave_qp_hi = wave_tok_hi >= t0 + wave * tpw ? cached + wave_tok_hi : -1;  // -1: no valid row
  const int wave_qp_lo = cached + t0 + wave * tpw;  // position of the wavefront's first row
  const float c = a.scale_log2;

  u32x4 qf[8];  // Q^T operand: lane (n, h) holds row n at dims 16 kk + 8 h .. +7
  {
    const int head = kvh * a.G + (n % a.G);
    const uint16_t* qrow = a.q + (int64_t)(qs + (row_valid ? tok : 0)) * a.q_st + (int64_t)head * a.q_sh;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      const u32x4 v = ld16(qrow + 16 * kk + 8 * h);
      qf[kk] = row_valid ? v : u32x4{0, 0, 0, 0};
    }
  }
  f32x16 oacc[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[dt][r] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  // prologue: group A stages K(0), K(1) and loads K(2); group B stages V(0) and loads V(1)
  Regs4 kr, vr;
  KIds kid_next;
  int vid_next = 0;
  if (grp == 0) {
    store_k(kbuf0, load_k(a, k_ids(a, pages, 0, last, gtid), 0, kvh, gtid), 0, kv_end, gtid);
    if (ntiles > 1)
      store_k(kbuf0 + kKsElems, load_k(a, k_ids(a, pages, kBN, last, gtid), kBN, kvh, gtid), kBN, kv_end, gtid);
    if (ntiles > 2) kr = load_k(a, k_ids(a, pages, 2 * kBN, last, gtid), 2 * kBN, kvh, gtid);
    kid_next = k_ids(a, pages, 3 * kBN, last, gtid);
  } else {
    store_v(vbuf0, load_v(a, v_id(a, pages, 0, last, gtid), 0, kvh, gtid), 0, kv_end, gtid);
    if (ntiles > 1) vr = load_v(a, v_id(a, pages, kBN, last, gtid), kBN, kvh, gtid);
    vid_next = v_id(a, pages, 2 * kBN, last, gtid);
  }
  __syncthreads();
  STile st;
  u32x4 pf[2][2];
  if (0 <= wave_qp_hi) {
    st = scores<T>(kbuf0, qf, n, h);
    if (grp == 0) softmax_tile<T>(st, pf, oacc, m_run, l_run, 0, qp, wave_qp_lo, h, c);
  }

  for (int p = 0; p < 2 * ntiles; ++p) {
    if ((p & 1) == grp) {  // matrix phase i
      const int i = p >> 1;
      if (i * kBN <= wave_qp_hi) pv_tile<T>(vbuf0 + (i & 1) * kVtElems, pf, oacc, n, h);
      if (i + 1 < ntiles && (i + 1) * kBN <= wave_qp_hi) st = scores<T>(kbuf0 + ((i + 1) & 1) * kKsElems, qf, n, h);
    } else {  // vector phase: softmax of S(j), then this group's staging duty
      const int j = (p + 1) >> 1;
      if (j < ntiles && j * kBN <= wave_qp_hi) softmax_tile<T>(st, pf, oacc, m_run, l_run, j * kBN, qp, wave_qp_lo, h, c);
      const int i = p >> 1;
      if (grp == 0) {
        if (i + 2 < ntiles) store_k(kbuf0 + (i & 1) * kKsElems, kr, (i + 2) * kBN, kv_end, gtid);
        if (i + 3 < ntiles) kr = load_k(a, kid_next, (i + 3) * kBN, kvh, gtid);
        if (i + 4 < ntiles) kid_next = k_ids(a, pages, (i + 4) * kBN, last, gtid);
      } else {
        if (i + 1 < ntiles) store_v(vbuf0 + ((i + 1) & 1) * kVtElems, vr, (i + 1) * kBN, kv_end, gtid);
        if (i + 2 < ntiles) vr = load_v(a, vid_next, (i + 2) * kBN, kvh, gtid);
        if (i + 3 < ntiles) vid_next = v_id(a, pages, (i + 3) * kBN, last, gtid);
      }
    }
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
      const u32x2 pk = u32x2{pack2<T>(oacc[dt][r] * inv, oacc[dt][r + 1] * inv),
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
  MLLM_REQUIRE(q_tile_tokens == kQTileRows / G, MLLM_ERR_INVALID,
               "mllm_paged_prefill: q_tile_tokens must be 256 / (H / Hkv)");
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
  MLLM_REQUIRE(num_kv_heads * head_dim * 2 < (1 << 24) && (int64_t)block_size * num_kv_heads * head_dim * 2 < (1ll << 32),
               MLLM_ERR_UNSUPPORTED, "mllm_paged_prefill: KV block too large");
  PrefillArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.q_st = q_stride_tok;
  a.q_sh = q_stride_head;
  a.kc = static_cast<const uint16_t*>(k_cache);
  a.vc = static_cast<const uint16_t*>(v_cache);
  a.num_blocks = num_blocks;
  a.row_bytes = num_kv_heads * head_dim * 2;
  a.page_bytes = (unsigned)((int64_t)block_size * a.row_bytes);
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
    prefill_kernel<BF16><<<grid, 512, 0, st>>>(a);
  else
    prefill_kernel<F16><<<grid, 512, 0, st>>>(a);
  return check_launch("mllm_paged_prefill");
}
