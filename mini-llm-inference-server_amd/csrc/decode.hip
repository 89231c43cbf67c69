// Split-KV paged decode attention on gfx950 MFMA (reference src/minillm/attention/paged_torch_ref.py:47-59:
// one new token per row, softmax(q K^T / sqrt(Dh)) V over the row's whole context).
//
// Work: one wavefront per (bin, KV head).  The plan (mllm_plan) cuts the step's decode pages, rows in
// sequence order, into equal bins of at most C pages; a bin holds one or more row segments.  The
// wavefront streams its bin's pages 16 tokens at a time straight from HBM into VGPRs, across segment
// boundaries without a pause:
//   S^T[16 tok x 16] = K[16 tok x 128] . Q^T[128 x 16]      4 x v_mfma_f32_16x16x32 (bf16/f16)
//   O^T[128 x 16]   += V^T[128 x 16 tok] . P^T[16 tok x 16]  8 x v_mfma_f32_16x16x16
// The 16 MFMA columns hold the G = H / Hkv query heads that share the KV head (4 for Llama-3.1-8B);
// the other columns are zero.  Because S^T and the B operand of the PV product share one lane layout
// (lane l: column l % 16, k-rows 4 (l / 16) .. +3), P^T never leaves its lanes; the online-softmax
// max and sum of a head are reduced across the four lanes l, l^16, l^32, l^48 that hold its column.
// Each lane loads K row (l % 16) in four 16-byte pieces and V rows 4 (l / 16) .. +3 at dims
// 8 (l % 16) .. +7, so every wave-wide V load reads four whole 256-byte rows; the V^T operand is then
// assembled with v_perm_b32.  The next 16-token tile is loaded before the current one is consumed.
// A row that lies in one bin gets its normalised output from that segment; a row cut across bins gets
// fp32 (m, l, acc) partials, one per segment, that a second kernel merges with a log-sum-exp.
//
// fp8 (e4m3fn) pools with an even number of KV heads and at most 8 query heads per KV head run
// decode_pair_kernel (below): two KV heads per wavefront, loaded with the 16-bit kernel's shapes.  Other
// fp8 pools run this kernel with one head per wavefront, where a tile is half the bytes.  Each lane
// loads K row (l % 16) as two 16-byte pieces, dims 64 h + 16 (l / 16) .. +15 for h = 0, 1, so S^T's
// k-dimension runs through the dims in that order (the Q^T operand is loaded in the same order; a dot
// product does not depend on it), and V rows 4 (l / 16) .. +3 at dims 8 (l % 16) .. +7 as four 8-byte
// pieces.  The tile is widened to bf16/fp16 in registers (v_cvt_scalef32_pk_*_fp8 with scale 1: exact)
// right before it is consumed, so the MFMA stream is the 16-bit one; k_scale is folded into the softmax
// scale and v_scale into the output.
#include <math.h>

#include <mutex>
#include <string>

#include "common.h"

namespace mllm {
namespace {

constexpr int kHeadDim = 128;
constexpr int kWaves = 4;  // KV heads per workgroup of the decode kernel on small steps
// Whole-page decode (16-bit pools): one workgroup of 8 wavefronts reads all 8 KV heads of a bin's pages,
// each 16-token page of the pool one contiguous 32 KB run, at 2 wavefronts per SIMD: one workgroup per CU.
// The library launches it when the KV heads are a multiple of 8 and the split size is at least
// kWholePageMinSplit pages; the host then sizes the bins so the step is one round of workgroups (at most
// one bin per CU).  Same box, against 4-wavefront workgroups at 3 per SIMD: decode_256 341.7 against
// 349.6 us (255 bins of 134 pages against 383 of 89), mixed_128's decode 322.8 against 329.4 us, 128 rows
// of 960 tokens 81.4 against 82.8 us; on small steps it is slower (4 rows: 16.0 against 11.5 us; 32 rows of
// 960 tokens at 8 pages a bin: 27.8 against 26.7 us), hence the threshold.
constexpr int kWavesWhole = 8;
constexpr int kOccupancyWhole = 2;
constexpr int kWholePageMinSplit = 24;
__host__ __device__ constexpr bool whole_page(bool fp8, int num_kv_heads, int pages_per_split) {
  return !fp8 && num_kv_heads % kWavesWhole == 0 && pages_per_split >= kWholePageMinSplit;
}
#ifndef MLLM_DECODE_LAZY_RESCALE
#define MLLM_DECODE_LAZY_RESCALE 1
#endif
constexpr bool kLazyRescale = MLLM_DECODE_LAZY_RESCALE;
#ifndef MLLM_DECODE_K_NT
#define MLLM_DECODE_K_NT 1
#endif
constexpr bool kKNonTemporal = MLLM_DECODE_K_NT;  // K loads of 16-bit pools with the non-temporal hint

struct DecodeArgs {
  const uint16_t* q;
  int64_t q_st, q_sh;
  const char* kc;  // pools, addressed in bytes
  const char* vc;
  int64_t num_blocks;
  int bs, H, Hkv, G, HG;
  const int32_t* qo_indptr;
  const int32_t* kv_indptr;
  const int32_t* kv_indices;
  const int32_t* seq_lens;
  const int4* work;  // the plan's decode bins and segments
  float scale_log2;  // softmax scale x k_scale x log2(e)
  float v_scale;     // output scale of an fp8 pool
  uint16_t* out;
  int64_t o_st, o_sh;
  float* part_o;
  float2* part_ml;
};

template <bool NT>
__device__ __forceinline__ u32x4 ldkv(const char* p) {
  if constexpr (NT)
    return ld16_nt(p);
  else
    return ld16(p);
}
template <bool NT>
__device__ __forceinline__ u32x2 ldkv8(const char* p) {
  if constexpr (NT)
    return __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
  else
    return ld8(p);
}

// The registers of one loaded 16-token tile, as the pool stores it.
template <bool F8>
struct TileRegs {  // 16-bit pool: K row c at dims 32 kk + 8 g .. +7; V rows 4 g + i at dims 8 c .. 8 c + 7
  u32x4 k[4];
  u32x4 v[4];
};
template <>
struct TileRegs<true> {  // fp8 pool: K row c at dims 64 h + 16 g .. +15; V rows 4 g + i at dims 8 c .. 8 c + 7
  u32x4 k[2];
  u32x2 v[4];
};

// Dims of the Q^T operand (and of the K operand) that lane group g holds at k-step kk of S^T = K Q^T.
template <bool F8>
__device__ __forceinline__ int qk_dim0(int kk, int g) {
  return F8 ? 64 * (kk >> 1) + 16 * g + 8 * (kk & 1) : 32 * kk + 8 * g;
}

// The next 16-token tile to load: its page within the segment and its 16-token slice of that page (tiles
// are loaded in order, once each, so a counter replaces a division by the tiles per page).
struct LoadCursor {
  int page = 0, sub = 0;
  __device__ __forceinline__ void advance(int tpp) {
    if (++sub == tpp) {
      sub = 0;
      ++page;
    }
  }
};

// A segment's page ids, one per lane in three registers: pages 0-63, 64-127 and 128-191 of the segment
// (a bin holds at most kMaxSplitPages pages).
constexpr int kMaxSplitPages = 192;
struct PageIds {
  int r[3];
};
__device__ __forceinline__ PageIds load_page_ids(const int32_t* kv_indices, const int4& r0, int lane) {
  PageIds p;
#pragma unroll
  for (int i = 0; i < 3; ++i) p.r[i] = lane + 64 * i < r0.y ? kv_indices[r0.x + 64 * i + lane] : 0;
  return p;
}
// Page `page` (wave-uniform) of the segment.
__device__ __forceinline__ int page_id(const PageIds& p, int page) {
  return __builtin_amdgcn_readlane(page < 64 ? p.r[0] : (page < 128 ? p.r[1] : p.r[2]), page & 63);
}

// Loads the 16-token tile at `at` of this wave's page range (lane (c, g); kbase/vbase: this head's bytes
// of the pools, strides in bytes).
template <bool F8, bool NT>
__device__ __forceinline__ void load_tile(const DecodeArgs& a, const char* kbase, const char* vbase, int64_t tok_stride,
                                          int64_t blk_stride, const PageIds& pages, LoadCursor at, int c, int g,
                                          TileRegs<F8>& r) {
  const int page = at.page, sub = at.sub;
  int blk = page_id(pages, page);
  if ((unsigned)blk >= (unsigned)a.num_blocks) blk = 0;  // never taken with valid metadata; keeps reads in the pool
  const int64_t off = (int64_t)blk * blk_stride + (int64_t)(sub * 16) * tok_stride;
  const char* kp = kbase + off + c * tok_stride;
  const char* vp = vbase + off + (4 * g) * tok_stride;
  if constexpr (F8) {
#pragma unroll
    for (int h = 0; h < 2; ++h) r.k[h] = ldkv<NT>(kp + 64 * h + 16 * g);
#pragma unroll
    for (int i = 0; i < 4; ++i) r.v[i] = ldkv8<NT>(vp + (int64_t)i * tok_stride + 8 * c);
  } else {
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) r.k[kk] = ldkv<NT && kKNonTemporal>(kp + 2 * qk_dim0<false>(kk, g));
#pragma unroll
    for (int i = 0; i < 4; ++i) r.v[i] = ldkv<NT>(vp + (int64_t)i * tok_stride + 16 * c);
  }
}

// A loaded fp8 tile as 16-bit MFMA operands: K in the A layout of S^T (k-step kk) and V rows 4 g + i.
template <typename T>
__device__ __forceinline__ void widen(const TileRegs<true>& r, u32x4 (&ka)[4], u32x4 (&va)[4]) {
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) ka[kk] = fp8x8_to<T>(r.k[kk >> 1][2 * (kk & 1)], r.k[kk >> 1][2 * (kk & 1) + 1]);
#pragma unroll
  for (int i = 0; i < 4; ++i) va[i] = fp8x8_to<T>(r.v[i][0], r.v[i][1]);
}

// One 16-token tile: scores, online-softmax update, PV accumulation.
template <typename T>
__device__ __forceinline__ void consume_tile(const u32x4 (&ka)[4], u32x4 (&va)[4], const u32x4 (&qf)[4],
                                             float scale_log2, int tpos0, int len, int g, float& m_run, float& l_run,
                                             f32x4 (&o)[8]) {
  f32x4 sc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) sc = Mfma<T>::m16x16x32(ka[kk], qf[kk], sc);
  float s[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) s[i] = sc[i] * scale_log2;
  if (tpos0 + 16 > len) {  // the row's last, partly filled tile: mask the keys past its end, zero their V
    const int tpos = tpos0 + 4 * g;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (tpos + i >= len) {
        s[i] = -INFINITY;
        va[i] = u32x4{0, 0, 0, 0};
      }
    }
  }
  // the column's max over its four lanes l, l^16, l^32, l^48: two VALU swaps, no LDS round trip
  const float mx = maximum_xor32(maximum_xor16(maximum(maximum(s[0], s[1]), maximum(s[2], s[3]))));
  if constexpr (kLazyRescale) {
    // the running max moves only when some column's tile max exceeds it by more than 2^8 (exp2 domain):
    // p then stays <= 256, which P and the fp32 accumulators hold as well as values below 1, and most
    // tiles skip rescaling O and l
    if (__any(mx > m_run + 8.f)) {
      const float m_new = fmaxf(m_run, mx);
      const float alpha = fast_exp2(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int m = 0; m < 8; ++m) o[m] *= alpha;
      m_run = m_new;
    }
  } else {
    const float m_new = fmaxf(m_run, mx);
    const float alpha = fast_exp2(m_run - m_new);
    l_run *= alpha;
#pragma unroll
    for (int m = 0; m < 8; ++m) o[m] *= alpha;
    m_run = m_new;
  }
  float p[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) p[i] = fast_exp2(s[i] - m_run);
  l_run += sum_xor32(sum_xor16((p[0] + p[1]) + (p[2] + p[3])));
  const u32x2 pfrag = u32x2{pack2<T>(p[0], p[1]), pack2<T>(p[2], p[3])};
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    const int dw = m >> 1, hf = m & 1;
    const u32x2 vfrag = u32x2{pick_halves(va[0][dw], hf, va[1][dw], hf), pick_halves(va[2][dw], hf, va[3][dw], hf)};
    o[m] = Mfma<T>::m16x16x16(vfrag, pfrag, o[m]);
  }
}

// The records of one segment of a bin (the plan's layout): r0 = {first page in kv_indices, pages, first
// page within the row, row length}, r1 = {q row, partial slot or -1, sequence, 0}.
struct SegRec {
  int4 r0, r1;
};
// The plan is read through the constant address space: it does not change during the launch, so its
// uniform records become scalar loads, which the wave waits for with lgkmcnt apart from the vector
// loads of K, V and q (read as global memory, a record would be a vector load, and waiting for it would
// wait for every vector load issued before it).
typedef const __attribute__((address_space(4))) int PlanInt;
__device__ __forceinline__ int4 plan_rec(const int4* work, int i) {
  const PlanInt* p = (const PlanInt*)(work + i);
  return make_int4(p[0], p[1], p[2], p[3]);
}
__device__ __forceinline__ SegRec seg_rec(const int4* segs, int g) {
  return SegRec{plan_rec(segs, 2 * g), plan_rec(segs, 2 * g + 1)};
}

// One wavefront per (bin, KV head) streams the bin's segments back to back, one 16-token tile ahead.
// While a segment streams, the wavefront already holds the next segment's records (read one segment
// earlier), loads its page ids and q, and reads the records of the segment after it; the lookahead
// load of a segment's last tile fetches the next segment's first tile.  So the stream does not stop at
// a row boundary: a new segment costs its finalisation (output or partial stores) and a fresh
// online-softmax state.
template <typename T, bool F8, bool NT, int OCC, int WAVES>
__global__ __launch_bounds__(64 * WAVES) __attribute__((amdgpu_waves_per_eu(OCC, OCC))) void decode_kernel(
    const DecodeArgs a) {
  const int lane = threadIdx.x & 63;
  // the KV-head group varies fastest, so the workgroups of one bin (adjacent heads of the same pages)
  // run side by side
  const int hg = blockIdx.x % a.HG;
  const int bin = blockIdx.x / a.HG;
  const int kvh = hg * WAVES + (threadIdx.x >> 6);
  if (kvh >= a.Hkv) return;  // wave-uniform
  // the header and the bin's record load together (the record carries the segments' base): the
  // grid covers the plan's capacity, and workgroups past the step's nbins bins exit
  const int nbins = plan_rec(a.work, 0).x;
  const int4 bw = plan_rec(a.work, 1 + bin);
  if (bin >= nbins) return;
  const int4* segs = a.work + bw.z;
  const int tpp = a.bs >> 4;
  const int c = lane & 15;
  const int g = lane >> 4;
  const bool qvalid = c < a.G;  // lane column c is query head c of the group
  constexpr int kElem = F8 ? 1 : 2;  // pool bytes per element
  const int64_t tok_stride = (int64_t)a.Hkv * kHeadDim * kElem;
  const int64_t blk_stride = (int64_t)a.bs * tok_stride;
  const char* kbase = a.kc + kvh * kHeadDim * kElem;
  const char* vbase = a.vc + kvh * kHeadDim * kElem;
  const int qhead = kvh * a.G + (qvalid ? c : 0);

  // B operand of S^T = K Q^T: lane (c, g) holds q head c of the group at the dims qk_dim0 gives
  auto load_q = [&](int qrow, u32x4 (&qf)[4]) {
    const char* qp = reinterpret_cast<const char*>(a.q + (int64_t)qrow * a.q_st + (int64_t)qhead * a.q_sh);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const u32x4 v = ld16(qp + 2 * qk_dim0<F8>(kk, g));
      qf[kk] = qvalid ? v : u32x4{0, 0, 0, 0};
    }
  };

  // The next segment's records, page ids and q are loaded whether or not there is a next segment (the
  // last one's again, unused), so no loaded value meets a branch join: a join would make the wave wait
  // there for every load in flight, the tile loaded ahead included.
  const int glast = bw.y - 1;
  int gi = bw.x;
  SegRec cur = seg_rec(segs, gi);
  SegRec nxt = seg_rec(segs, min(gi + 1, glast));
  PageIds pages = load_page_ids(a.kv_indices, cur.r0, lane);
  u32x4 qf[4];
  load_q(cur.r1.x, qf);
  TileRegs<F8> tile, ahead;  // the tile being consumed, the one loaded ahead of it
  LoadCursor at;
  load_tile<F8, NT>(a, kbase, vbase, tok_stride, blk_stride, pages, at, c, g, tile);
  at.advance(tpp);

  while (true) {
    gi = __builtin_amdgcn_readfirstlane(gi);  // uniform: the records below are scalar loads
    const bool has_next = gi < glast;
    const int tok0 = cur.r0.z * a.bs, len = cur.r0.w;
    // pages past the row's last token (a block table may hold pages ahead) have no tiles: a segment of
    // only such pages has none
    const int ntiles = max(min(len, tok0 + cur.r0.y * a.bs) - tok0 + 15, 0) >> 4;
    const PageIds next_pages = load_page_ids(a.kv_indices, nxt.r0, lane);
    u32x4 next_q[4];
    load_q(nxt.r1.x, next_q);
    const SegRec after = seg_rec(segs, min(gi + 2, glast));
    float m_run = -INFINITY, l_run = 0.f;
    f32x4 o[8];
#pragma unroll
    for (int m = 0; m < 8; ++m) o[m] = f32x4{0.f, 0.f, 0.f, 0.f};
    bool next_loaded = false;  // the next segment's first tile is on its way into `tile`
    for (int t = 0; t < ntiles; ++t) {
      if (t + 1 < ntiles) {
        load_tile<F8, NT>(a, kbase, vbase, tok_stride, blk_stride, pages, at, c, g, ahead);
        at.advance(tpp);
      } else if (has_next) {
        load_tile<F8, NT>(a, kbase, vbase, tok_stride, blk_stride, next_pages, LoadCursor{}, c, g, ahead);
        next_loaded = true;
      }
      if constexpr (F8) {
        u32x4 ka[4], va[4];
        widen<T>(tile, ka, va);
        consume_tile<T>(ka, va, qf, a.scale_log2, tok0 + t * 16, len, g, m_run, l_run, o);
      } else {
        consume_tile<T>(tile.k, tile.v, qf, a.scale_log2, tok0 + t * 16, len, g, m_run, l_run, o);
      }
      tile = ahead;
    }

    if (qvalid) {
      const int head = kvh * a.G + c;
      const int slot = cur.r1.y;
      // lane (c, g) owns dims 32 g + 8 i + m of head c: o[m][i]
      if (slot < 0) {  // the row's only segment: the normalised output
        const float inv = F8 ? a.v_scale / l_run : 1.f / l_run;
        char* op = reinterpret_cast<char*>(a.out + (int64_t)cur.r1.x * a.o_st + (int64_t)head * a.o_sh + 32 * g);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          u32x4 pk = u32x4{pack2<T>(o[0][i] * inv, o[1][i] * inv), pack2<T>(o[2][i] * inv, o[3][i] * inv),
                           pack2<T>(o[4][i] * inv, o[5][i] * inv), pack2<T>(o[6][i] * inv, o[7][i] * inv)};
          st16(op + 16 * i, pk);
        }
      } else {
        const int64_t row = (int64_t)slot * a.H + head;
        float* po = a.part_o + row * kHeadDim + 32 * g;
        if constexpr (F8) {
#pragma unroll
          for (int m = 0; m < 8; ++m) o[m] *= a.v_scale;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          *reinterpret_cast<f32x4*>(po + 8 * i) = f32x4{o[0][i], o[1][i], o[2][i], o[3][i]};
          *reinterpret_cast<f32x4*>(po + 8 * i + 4) = f32x4{o[4][i], o[5][i], o[6][i], o[7][i]};
        }
        if (g == 0) a.part_ml[row] = make_float2(m_run, l_run);
      }
    }
    if (!has_next) break;
    ++gi;
    cur = nxt;
    nxt = after;
    pages = next_pages;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) qf[kk] = next_q[kk];
    at = LoadCursor{};
    if (!next_loaded)  // this segment had no tile to load it behind
      load_tile<F8, NT>(a, kbase, vbase, tok_stride, blk_stride, pages, at, c, g, tile);
    at.advance(tpp);  // the new segment's first tile is in `tile`
  }
}

// fp8 pools, two adjacent KV heads per wavefront (heads 2j and 2j + 1).  Their 128-byte rows of one
// token are one 256-byte row of the pool, so the pair is loaded exactly as the 16-bit kernel loads one
// head: K row c as four 16-byte pieces (bytes 64 p + 16 g .. +15, p = 0..3; pieces 0-1 are head A's,
// 2-3 head B's) and V rows 4 g + i as one 16-byte piece each (bytes 16 c .. +15: lanes c < 8 hold head
// A's dims 16 c .., lanes c >= 8 head B's dims 16 (c - 8) ..).  A 16-token tile is 8 KB, as in the
// 16-bit kernel.
//   S^T[16 tok x 16] = [K_A | K_B] . [Q_A^T ; Q_B^T]   8 x v_mfma_f32_16x16x32 over k = 256
// Columns 0 .. G-1 are head A's query heads, G .. 2G-1 head B's; a column's Q^T operand is zero on the
// other head's k-steps, so one product gives both heads' scores and the softmax runs once for the pair.
//   O^T[16 x 16]_m += V^T_m[16 x 16 tok] . P^T[16 tok x 16], m = 0..15   16 x v_mfma_f32_16x16x16
// Row r of product m is element m of V lane r's 16 dims: head A dim 16 r + m for r < 8, head B dim
// 16 (r - 8) + m for r >= 8.  Only head A's columns of rows 0-7 and head B's columns of rows 8-15 are
// kept, so lane (c, g) ends holding dims 64 (g & 1) + 16 i + m of query head 2j G + c when
// c < G and g < 2 or G <= c < 2G and g >= 2.  Same MFMA count per head as the one-head kernel, half the
// softmax and load instructions per head.
struct PairTile {
  u32x4 k[4];
  u32x4 v[4];
};

template <bool NT>
__device__ __forceinline__ void load_pair(const DecodeArgs& a, const char* kbase, const char* vbase, int64_t tok_stride,
                                          int64_t blk_stride, const PageIds& pages, LoadCursor at, int c, int g,
                                          PairTile& r) {
  int blk = page_id(pages, at.page);
  if ((unsigned)blk >= (unsigned)a.num_blocks) blk = 0;  // never taken with valid metadata; keeps reads in the pool
  const int64_t off = (int64_t)blk * blk_stride + (int64_t)(at.sub * 16) * tok_stride;
  const char* kp = kbase + off + c * tok_stride;
  const char* vp = vbase + off + (4 * g) * tok_stride;
#pragma unroll
  for (int p = 0; p < 4; ++p) r.k[p] = ldkv<NT>(kp + 64 * p + 16 * g);
#pragma unroll
  for (int i = 0; i < 4; ++i) r.v[i] = ldkv<NT>(vp + (int64_t)i * tok_stride + 16 * c);
}

// One 16-token tile of a head pair.  qa / qb: the Q^T operands of head A's and head B's k-steps (zero in
// the other head's columns).
template <typename T>
__device__ __forceinline__ void consume_pair(PairTile& r, const u32x4 (&qa)[4], const u32x4 (&qb)[4], float scale_log2,
                                             int tpos0, int len, int g, float& m_run, float& l_run, f32x4 (&o)[16]) {
  f32x4 sc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const u32x4 (&qh)[4] = p < 2 ? qa : qb;
    sc = Mfma<T>::m16x16x32(fp8x8_to<T>(r.k[p][0], r.k[p][1]), qh[2 * (p & 1)], sc);
    sc = Mfma<T>::m16x16x32(fp8x8_to<T>(r.k[p][2], r.k[p][3]), qh[2 * (p & 1) + 1], sc);
  }
  float s[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) s[i] = sc[i] * scale_log2;
  if (tpos0 + 16 > len) {  // the row's last, partly filled tile: mask the keys past its end, zero their V
    const int tpos = tpos0 + 4 * g;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (tpos + i >= len) {
        s[i] = -INFINITY;
        r.v[i] = u32x4{0, 0, 0, 0};
      }
    }
  }
  const float mx = maximum_xor32(maximum_xor16(maximum(maximum(s[0], s[1]), maximum(s[2], s[3]))));
  if (__any(mx > m_run + 8.f)) {  // lazy rescale, as in the one-head kernel
    const float m_new = fmaxf(m_run, mx);
    const float alpha = fast_exp2(m_run - m_new);
    l_run *= alpha;
#pragma unroll
    for (int m = 0; m < 16; ++m) o[m] *= alpha;
    m_run = m_new;
  }
  float p[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) p[i] = fast_exp2(s[i] - m_run);
  l_run += sum_xor32(sum_xor16((p[0] + p[1]) + (p[2] + p[3])));
  const u32x2 pfrag = u32x2{pack2<T>(p[0], p[1]), pack2<T>(p[2], p[3])};
#pragma unroll
  for (int b = 0; b < 4; ++b) {  // elements 4 b .. 4 b + 3 of the four V rows, widened just in time
    u32x2 w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = fp8x4_to<T>(r.v[i][b]);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int dw = e >> 1, hf = e & 1;
      const u32x2 vfrag = u32x2{pick_halves(w[0][dw], hf, w[1][dw], hf), pick_halves(w[2][dw], hf, w[3][dw], hf)};
      o[4 * b + e] = Mfma<T>::m16x16x16(vfrag, pfrag, o[4 * b + e]);
    }
  }
}

template <typename T, int W, bool NT, int OCC>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(OCC, OCC))) void decode_pair_kernel(
    const DecodeArgs a) {
  const int lane = threadIdx.x & 63;
  // a workgroup of W wavefronts covers 2 W KV heads of one bin; HG = ceil(Hkv / (2 W)) groups per bin
  const int hg = blockIdx.x % a.HG;
  const int bin = blockIdx.x / a.HG;
  const int kvh0 = 2 * (hg * W + (threadIdx.x >> 6));
  if (kvh0 >= a.Hkv) return;  // wave-uniform
  const int nbins = plan_rec(a.work, 0).x;
  const int4 bw = plan_rec(a.work, 1 + bin);
  if (bin >= nbins) return;
  const int4* segs = a.work + bw.z;
  const int tpp = a.bs >> 4;
  const int c = lane & 15;
  const int g = lane >> 4;

  // column c: query head 2j G + c (head A's for c < G, head B's for G <= c < 2G); k-step t of a head
  // covers its dims 64 (t >> 1) + 16 g + 8 (t & 1) .. +7
  const bool qvalid = c < 2 * a.G;
  const bool in_b = c >= a.G;
  const int qhead = kvh0 * a.G + (qvalid ? c : 0);
  auto load_q = [&](int qrow, u32x4 (&qv)[4]) {
    const char* qp = reinterpret_cast<const char*>(a.q + (int64_t)qrow * a.q_st + (int64_t)qhead * a.q_sh);
#pragma unroll
    for (int t = 0; t < 4; ++t) qv[t] = ld16(qp + 2 * (64 * (t >> 1) + 16 * g + 8 * (t & 1)));
  };
  auto split_q = [&](const u32x4 (&qv)[4], u32x4 (&qa)[4], u32x4 (&qb)[4]) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const u32x4 z = u32x4{0, 0, 0, 0};
      qa[t] = qvalid && !in_b ? qv[t] : z;
      qb[t] = qvalid && in_b ? qv[t] : z;
    }
  };

  const int64_t tok_stride = (int64_t)a.Hkv * kHeadDim;  // one byte per element
  const int64_t blk_stride = (int64_t)a.bs * tok_stride;
  const char* kbase = a.kc + kvh0 * kHeadDim;
  const char* vbase = a.vc + kvh0 * kHeadDim;

  const int glast = bw.y - 1;  // next-segment loads as in decode_kernel: unconditional
  int gi = bw.x;
  SegRec cur = seg_rec(segs, gi);
  SegRec nxt = seg_rec(segs, min(gi + 1, glast));
  PageIds pages = load_page_ids(a.kv_indices, cur.r0, lane);
  u32x4 qa[4], qb[4];
  {
    u32x4 qv[4];
    load_q(cur.r1.x, qv);
    split_q(qv, qa, qb);
  }
  PairTile tile, ahead;
  LoadCursor at;
  load_pair<NT>(a, kbase, vbase, tok_stride, blk_stride, pages, at, c, g, tile);
  at.advance(tpp);

  while (true) {
    gi = __builtin_amdgcn_readfirstlane(gi);
    const bool has_next = gi < glast;
    const int tok0 = cur.r0.z * a.bs, len = cur.r0.w;
    // pages past the row's last token (a block table may hold pages ahead) have no tiles: a segment of
    // only such pages has none
    const int ntiles = max(min(len, tok0 + cur.r0.y * a.bs) - tok0 + 15, 0) >> 4;
    const PageIds next_pages = load_page_ids(a.kv_indices, nxt.r0, lane);
    u32x4 next_q[4];
    load_q(nxt.r1.x, next_q);
    const SegRec after = seg_rec(segs, min(gi + 2, glast));
    float m_run = -INFINITY, l_run = 0.f;
    f32x4 o[16];
#pragma unroll
    for (int m = 0; m < 16; ++m) o[m] = f32x4{0.f, 0.f, 0.f, 0.f};
    bool next_loaded = false;  // the next segment's first tile is on its way into `tile`
    for (int t = 0; t < ntiles; ++t) {
      if (t + 1 < ntiles) {
        load_pair<NT>(a, kbase, vbase, tok_stride, blk_stride, pages, at, c, g, ahead);
        at.advance(tpp);
      } else if (has_next) {
        load_pair<NT>(a, kbase, vbase, tok_stride, blk_stride, next_pages, LoadCursor{}, c, g, ahead);
        next_loaded = true;
      }
      consume_pair<T>(tile, qa, qb, a.scale_log2, tok0 + t * 16, len, g, m_run, l_run, o);
      tile = ahead;
    }

    // lanes that hold kept rows: head A's columns in lane groups 0-1, head B's in 2-3
    if (qvalid && in_b == (g >= 2)) {
      const int head = kvh0 * a.G + c;
      const int d0 = 64 * (g & 1);  // o[m][i] is dim d0 + 16 i + m
      const int slot = cur.r1.y;
      if (slot < 0) {
        const float inv = a.v_scale / l_run;
        char* op = reinterpret_cast<char*>(a.out + (int64_t)cur.r1.x * a.o_st + (int64_t)head * a.o_sh + d0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int m = 8 * h;
            const u32x4 pk =
                u32x4{pack2<T>(o[m][i] * inv, o[m + 1][i] * inv), pack2<T>(o[m + 2][i] * inv, o[m + 3][i] * inv),
                      pack2<T>(o[m + 4][i] * inv, o[m + 5][i] * inv), pack2<T>(o[m + 6][i] * inv, o[m + 7][i] * inv)};
            st16(op + 2 * (16 * i + m), pk);
          }
        }
      } else {
        const int64_t row = (int64_t)slot * a.H + head;
        float* po = a.part_o + row * kHeadDim + d0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4) {
            const int m = 4 * q4;
            *reinterpret_cast<f32x4*>(po + 16 * i + m) =
                f32x4{o[m][i] * a.v_scale, o[m + 1][i] * a.v_scale, o[m + 2][i] * a.v_scale, o[m + 3][i] * a.v_scale};
          }
        }
        if ((g & 1) == 0) a.part_ml[row] = make_float2(m_run, l_run);
      }
    }
    if (!has_next) break;
    ++gi;
    cur = nxt;
    nxt = after;
    pages = next_pages;
    split_q(next_q, qa, qb);
    at = LoadCursor{};
    if (!next_loaded)  // this segment had no tile to load it behind
      load_pair<NT>(a, kbase, vbase, tok_stride, blk_stride, pages, at, c, g, tile);
    at.advance(tpp);
  }
}

// Log-sum-exp merge of a cut row's partials (one per segment).  One workgroup of 256 threads per (row, 8
// heads): 32 threads per head, 4 dims per thread, so a row's partials of 8 heads arrive as 16-byte loads
// in one round trip and a 256-row step launches 4 workgroups per cut row instead of 32.  Each output
// element goes through the same operations, in the same order, as with one thread per (head, dim).
constexpr int kMergeThreads = 256;
constexpr int kMergeHeads = kMergeThreads / (kHeadDim / 4);  // heads per workgroup: 8
template <typename T>
__global__ __launch_bounds__(kMergeThreads) void merge_kernel(const int4* __restrict__ merge,
                                                             const float* __restrict__ part_o,
                                                             const float2* __restrict__ part_ml, int H,
                                                             const int32_t* __restrict__ qo_indptr,
                                                             uint16_t* __restrict__ out, int64_t o_st, int64_t o_sh) {
  const int4 mw = merge[blockIdx.x];
  const int seq = mw.x, first = mw.y, n = mw.z;
  if (seq < 0) return;
  const int head = blockIdx.y * kMergeHeads + (int)(threadIdx.x >> 5);
  if (head >= H) return;
  const int d0 = 4 * (threadIdx.x & 31);
  // one online pass over the partials, four at a time so that their loads are in flight together (a row
  // has a few: one round trip instead of two per partial); slots past n re-read partial 0 of the
  // group and weigh it 2^-inf = 0
  constexpr int kGroup = 4;
  float m = -INFINITY, lsum = 0.f, acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int j0 = 0; j0 < n; j0 += kGroup) {
    float2 ml[kGroup];
    f32x4 o[kGroup];
#pragma unroll
    for (int u = 0; u < kGroup; ++u) {
      const int64_t row = (int64_t)(first + (j0 + u < n ? j0 + u : j0)) * H + head;
      ml[u] = part_ml[row];
      o[u] = *reinterpret_cast<const f32x4*>(part_o + row * kHeadDim + d0);
    }
    float mc = m;
#pragma unroll
    for (int u = 0; u < kGroup; ++u) {
      if (j0 + u >= n) ml[u].x = -INFINITY;
      mc = fmaxf(mc, ml[u].x);
    }
    const float sc = fast_exp2(m - mc);  // 0 for the first group (m = -inf, lsum = acc = 0)
    lsum *= sc;
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] *= sc;
#pragma unroll
    for (int u = 0; u < kGroup; ++u) {
      const float wgt = fast_exp2(ml[u].x - mc);
      lsum += wgt * ml[u].y;
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] += wgt * o[u][e];
    }
    m = mc;
  }
  const int qtok = qo_indptr[seq];
  uint16_t* op = out + (int64_t)qtok * o_st + (int64_t)head * o_sh + d0;
#pragma unroll
  for (int e = 0; e < 4; ++e) op[e] = cvt1<T>(acc[e] / lsum);
}

// Occupancy, tuned on MI355X (decode_256): every kernel loads one 16-token tile ahead of the one it
// consumes.  The 16-bit kernel runs 3 wavefronts per SIMD (163 VGPRs, no spills) in workgroups of 4, or 2 per SIMD in
// whole-page workgroups of 8.  With per-row splits, one tile
// of lookahead at 3 per SIMD streamed as fast as two at 2 per SIMD, and the fp8 pair kernel ran the same
// with one tile ahead as with two (192-195 us); the fp8 one-head kernel then ran 198 us with four tiles
// ahead at 2 per SIMD against 205 us with one at 4.
#ifndef MLLM_DECODE_OCC
#define MLLM_DECODE_OCC 3
#endif
constexpr bool kNonTemporal = true;
constexpr int kOccupancy = MLLM_DECODE_OCC;
#ifndef MLLM_DECODE_FP8_OCC
#define MLLM_DECODE_FP8_OCC 2
#endif
constexpr int kOccupancyFp8 = MLLM_DECODE_FP8_OCC;

// The pair kernel (fp8, two KV heads per wavefront): W wavefronts per workgroup at OCC wavefronts per
// SIMD.  With per-row splits on decode_256: 4 per workgroup 192-195 us, 2 per workgroup 199-204 us and 1
// per workgroup 212-214 us (a workgroup on all 8 KV heads reads whole pages).
#ifndef MLLM_DECODE_PAIR_WAVES
#define MLLM_DECODE_PAIR_WAVES 4
#endif
constexpr int kWavesPair = MLLM_DECODE_PAIR_WAVES;
#ifndef MLLM_DECODE_PAIR_OCC
#define MLLM_DECODE_PAIR_OCC 2
#endif
constexpr int kOccupancyPair = MLLM_DECODE_PAIR_OCC;

// fp8 pools run the pair kernel when the KV heads pair up and a pair's query heads fit 16 columns.
__host__ __device__ constexpr bool pair_heads(int num_kv_heads, int group) {
  return num_kv_heads % 2 == 0 && 2 * group <= 16;
}

// Bins a plan of n_work records can hold: a header, then per bin one record and at least one segment
// of two records.  The grid covers that many bins; the workgroups past the step's own exit at once.
constexpr int max_bins(int n_work) { return n_work >= 4 ? (n_work - 1) / 3 : 0; }
// Partial slots a plan of n_work records can use: a cut row takes one slot per segment, and the segments
// take two records each after the header, so slots <= segments <= (n_work - 1) / 2.  The workspace holds
// that many slots: acc[slot][head][Dh], then (m, l)[slot][head].
constexpr int partial_slots(int n_work) { return n_work >= 1 ? (n_work - 1) / 2 : 0; }

template <typename T, bool F8>
int launch(const DecodeArgs& a, int n_work, int pages_per_split, hipStream_t st) {
  const unsigned bins = (unsigned)max_bins(n_work);
  if (bins == 0) return MLLM_OK;
  if constexpr (!F8) {
    if (whole_page(false, a.Hkv, pages_per_split)) {
      DecodeArgs b = a;
      b.HG = a.Hkv / kWavesWhole;
      decode_kernel<T, false, kNonTemporal, kOccupancyWhole, kWavesWhole>
          <<<bins * (unsigned)b.HG, 64 * kWavesWhole, 0, st>>>(b);
      return check_launch("mllm_paged_decode");
    }
  }
  if constexpr (F8) {
    if (pair_heads(a.Hkv, a.G)) {
      DecodeArgs b = a;
      b.HG = (a.Hkv + 2 * kWavesPair - 1) / (2 * kWavesPair);
      decode_pair_kernel<T, kWavesPair, kNonTemporal, kOccupancyPair><<<bins * (unsigned)b.HG, 64 * kWavesPair, 0, st>>>(b);
      return check_launch("mllm_paged_decode_fp8");
    }
  }
  decode_kernel<T, F8, kNonTemporal, F8 ? kOccupancyFp8 : kOccupancy, kWaves><<<bins * (unsigned)a.HG, 64 * kWaves, 0, st>>>(a);
  return check_launch(F8 ? "mllm_paged_decode_fp8" : "mllm_paged_decode");
}

}  // namespace
}  // namespace mllm

extern "C" int64_t mllm_decode_workspace_bytes(int32_t num_decode_work, int32_t num_heads, int32_t head_dim) {
  if (num_decode_work <= 0 || num_heads <= 0 || head_dim <= 0) return 0;
  return (int64_t)mllm::partial_slots(num_decode_work) * num_heads * ((int64_t)head_dim * 4 + 8);
}

namespace {

int paged_decode(const void* q, int64_t q_stride_tok, int64_t q_stride_head, const void* k_cache,
                                 const void* v_cache, int64_t num_blocks, int32_t block_size, int32_t num_heads,
                                 int32_t num_kv_heads, int32_t head_dim, const int32_t* qo_indptr,
                                 const int32_t* kv_indptr, const int32_t* kv_indices, const int32_t* seq_lens,
                                 const int32_t* decode_work, int32_t num_decode_work, const int32_t* merge_work,
                                 int32_t num_merge_work, int32_t pages_per_split, float softmax_scale, int32_t dtype,
                                 void* out, int64_t out_stride_tok, int64_t out_stride_head, void* workspace,
                                 int64_t workspace_bytes, bool fp8, float k_scale, float v_scale, void* stream) {
  using namespace mllm;
  const std::string fn = fp8 ? "mllm_paged_decode_fp8" : "mllm_paged_decode";
  MLLM_REQUIRE(dtype == MLLM_DTYPE_BF16 || dtype == MLLM_DTYPE_F16, MLLM_ERR_UNSUPPORTED,
               fn + ": dtype must be bfloat16 or float16");
  MLLM_REQUIRE(head_dim == kHeadDim, MLLM_ERR_UNSUPPORTED, fn + ": head_dim must be 128");
  MLLM_REQUIRE(k_scale > 0.f && v_scale > 0.f && k_scale < INFINITY && v_scale < INFINITY, MLLM_ERR_INVALID,
               fn + ": scales must be positive and finite");
  MLLM_REQUIRE(block_size > 0 && block_size % 16 == 0, MLLM_ERR_UNSUPPORTED,
               fn + ": block_size must be a multiple of 16");
  MLLM_REQUIRE(num_kv_heads > 0 && num_heads > 0 && num_heads % num_kv_heads == 0, MLLM_ERR_INVALID,
               fn + ": num_heads must be a multiple of num_kv_heads");
  MLLM_REQUIRE(num_heads / num_kv_heads <= 16, MLLM_ERR_UNSUPPORTED,
               fn + ": at most 16 query heads per KV head");
  MLLM_REQUIRE(pages_per_split >= 1 && pages_per_split <= kMaxSplitPages, MLLM_ERR_INVALID,
               fn + ": pages_per_split must be in [1, 192]");
  MLLM_REQUIRE(num_decode_work >= 0 && num_merge_work >= 0, MLLM_ERR_INVALID, fn + ": negative count");
  if (num_decode_work == 0) return MLLM_OK;
  MLLM_REQUIRE(q && k_cache && v_cache && out && qo_indptr && kv_indptr && kv_indices && seq_lens && decode_work,
               MLLM_ERR_INVALID, fn + ": null pointer");
  const int64_t need = num_merge_work ? mllm_decode_workspace_bytes(num_decode_work, num_heads, head_dim) : 0;
  MLLM_REQUIRE(workspace_bytes >= need && (need == 0 || workspace), MLLM_ERR_INVALID,
               fn + ": workspace too small");
  const bool aligned = ((uintptr_t)q % 16 == 0) && ((uintptr_t)out % 16 == 0) && ((uintptr_t)k_cache % 16 == 0) &&
                       ((uintptr_t)v_cache % 16 == 0) && (q_stride_tok * 2) % 16 == 0 &&
                       (q_stride_head * 2) % 16 == 0 && (out_stride_tok * 2) % 16 == 0 &&
                       (out_stride_head * 2) % 16 == 0;
  MLLM_REQUIRE(aligned, MLLM_ERR_UNSUPPORTED, fn + ": q, out and pools need 16-byte aligned rows");

  DecodeArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.q_st = q_stride_tok;
  a.q_sh = q_stride_head;
  a.kc = static_cast<const char*>(k_cache);
  a.vc = static_cast<const char*>(v_cache);
  a.num_blocks = num_blocks;
  a.bs = block_size;
  a.H = num_heads;
  a.Hkv = num_kv_heads;
  a.G = num_heads / num_kv_heads;
  a.HG = (num_kv_heads + kWaves - 1) / kWaves;
  a.qo_indptr = qo_indptr;
  a.kv_indptr = kv_indptr;
  a.kv_indices = kv_indices;
  a.seq_lens = seq_lens;
  a.work = reinterpret_cast<const int4*>(decode_work);
  a.scale_log2 = softmax_scale * k_scale * kLog2e;
  a.v_scale = v_scale;
  a.out = static_cast<uint16_t*>(out);
  a.o_st = out_stride_tok;
  a.o_sh = out_stride_head;
  a.part_o = static_cast<float*>(workspace);
  a.part_ml = reinterpret_cast<float2*>(static_cast<char*>(workspace) +
                                        (int64_t)partial_slots(num_decode_work) * num_heads * head_dim * 4);
  (void)merge_work;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (dtype == MLLM_DTYPE_BF16)
    return fp8 ? launch<BF16, true>(a, num_decode_work, pages_per_split, st)
               : launch<BF16, false>(a, num_decode_work, pages_per_split, st);
  return fp8 ? launch<F16, true>(a, num_decode_work, pages_per_split, st)
             : launch<F16, false>(a, num_decode_work, pages_per_split, st);
}

}  // namespace

extern "C" int mllm_paged_decode(const void* q, int64_t q_stride_tok, int64_t q_stride_head, const void* k_cache,
                                 const void* v_cache, int64_t num_blocks, int32_t block_size, int32_t num_heads,
                                 int32_t num_kv_heads, int32_t head_dim, const int32_t* qo_indptr,
                                 const int32_t* kv_indptr, const int32_t* kv_indices, const int32_t* seq_lens,
                                 const int32_t* decode_work, int32_t num_decode_work, const int32_t* merge_work,
                                 int32_t num_merge_work, int32_t pages_per_split, float softmax_scale, int32_t dtype,
                                 void* out, int64_t out_stride_tok, int64_t out_stride_head, void* workspace,
                                 int64_t workspace_bytes, void* stream) {
  return paged_decode(q, q_stride_tok, q_stride_head, k_cache, v_cache, num_blocks, block_size, num_heads,
                      num_kv_heads, head_dim, qo_indptr, kv_indptr, kv_indices, seq_lens, decode_work, num_decode_work,
                      merge_work, num_merge_work, pages_per_split, softmax_scale, dtype, out, out_stride_tok,
                      out_stride_head, workspace, workspace_bytes, false, 1.f, 1.f, stream);
}

extern "C" int mllm_paged_decode_fp8(const void* q, int64_t q_stride_tok, int64_t q_stride_head, const void* k_cache,
                                     const void* v_cache, int64_t num_blocks, int32_t block_size, int32_t num_heads,
                                     int32_t num_kv_heads, int32_t head_dim, const int32_t* qo_indptr,
                                     const int32_t* kv_indptr, const int32_t* kv_indices, const int32_t* seq_lens,
                                     const int32_t* decode_work, int32_t num_decode_work, const int32_t* merge_work,
                                     int32_t num_merge_work, int32_t pages_per_split, float softmax_scale,
                                     int32_t dtype, float k_scale, float v_scale, void* out, int64_t out_stride_tok,
                                     int64_t out_stride_head, void* workspace, int64_t workspace_bytes, void* stream) {
  return paged_decode(q, q_stride_tok, q_stride_head, k_cache, v_cache, num_blocks, block_size, num_heads,
                      num_kv_heads, head_dim, qo_indptr, kv_indptr, kv_indices, seq_lens, decode_work, num_decode_work,
                      merge_work, num_merge_work, pages_per_split, softmax_scale, dtype, out, out_stride_tok,
                      out_stride_head, workspace, workspace_bytes, true, k_scale, v_scale, stream);
}

namespace {

int launch_merge(const int32_t* merge_work, int32_t num_merge_work, int32_t num_decode_work, int32_t num_heads,
                 const int32_t* qo_indptr, int32_t dtype, void* out, int64_t out_stride_tok, int64_t out_stride_head,
                 const void* workspace, hipStream_t st) {
  using namespace mllm;
  const float* part_o = static_cast<const float*>(workspace);
  const float2* part_ml = reinterpret_cast<const float2*>(static_cast<const char*>(workspace) +
                                                          (int64_t)partial_slots(num_decode_work) * num_heads * kHeadDim * 4);
  dim3 grid(num_merge_work, (num_heads + kMergeHeads - 1) / kMergeHeads);
  const int4* merge = reinterpret_cast<const int4*>(merge_work);
  if (dtype == MLLM_DTYPE_BF16)
    merge_kernel<BF16><<<grid, kMergeThreads, 0, st>>>(merge, part_o, part_ml, num_heads, qo_indptr,
                                                       static_cast<uint16_t*>(out), out_stride_tok, out_stride_head);
  else
    merge_kernel<F16><<<grid, kMergeThreads, 0, st>>>(merge, part_o, part_ml, num_heads, qo_indptr,
                                                      static_cast<uint16_t*>(out), out_stride_tok, out_stride_head);
  return check_launch("mllm_merge_splits");
}

}  // namespace

extern "C" int mllm_merge_splits(const int32_t* merge_work, int32_t num_merge_work, int32_t num_decode_work,
                                 int32_t num_heads, int32_t head_dim, const int32_t* qo_indptr, int32_t dtype,
                                 void* out, int64_t out_stride_tok, int64_t out_stride_head, const void* workspace,
                                 int64_t workspace_bytes, void* stream) {
  using namespace mllm;
  MLLM_REQUIRE(dtype == MLLM_DTYPE_BF16 || dtype == MLLM_DTYPE_F16, MLLM_ERR_UNSUPPORTED,
               "mllm_merge_splits: dtype must be bfloat16 or float16");
  MLLM_REQUIRE(head_dim == kHeadDim, MLLM_ERR_UNSUPPORTED, "mllm_merge_splits: head_dim must be 128");
  MLLM_REQUIRE(num_merge_work >= 0 && num_decode_work >= 0 && num_heads > 0, MLLM_ERR_INVALID,
               "mllm_merge_splits: bad sizes");
  if (num_merge_work == 0) return MLLM_OK;
  MLLM_REQUIRE(merge_work && qo_indptr && out && workspace, MLLM_ERR_INVALID, "mllm_merge_splits: null pointer");
  MLLM_REQUIRE(workspace_bytes >= mllm_decode_workspace_bytes(num_decode_work, num_heads, head_dim), MLLM_ERR_INVALID,
               "mllm_merge_splits: workspace too small");
  MLLM_REQUIRE(num_heads <= 65535, MLLM_ERR_UNSUPPORTED, "mllm_merge_splits: too many heads");
  return launch_merge(merge_work, num_merge_work, num_decode_work, num_heads, qo_indptr, dtype, out, out_stride_tok,
                      out_stride_head, workspace, reinterpret_cast<hipStream_t>(stream));
}

// ---------------------------------------------------------------- decode + merge without allocation
//
// The split-KV partials live in `scratch`, a fixed device array of this library, instead of a workspace
// the caller allocates.  Each GPU holds its own copy for the life of the process; its device address is
// looked up once per device (hipGetSymbolAddress, with that device current) and kept in g_scratch_ptr.
// Nothing in it needs to start at zero: every partial the merge reads is written by the decode launch
// of the same call.  Calls that overlap on one GPU (two streams, two threads) share the array and race.

namespace {

constexpr int64_t kScratchBytes = 64ll << 20;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) char scratch[kScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's address of `scratch` (looked up on the first call on that device).
int scratch_ptr(void** out) {
  using namespace mllm;
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(MLLM_ERR_HIP, std::string("mllm_paged_decode_noalloc: hipGetDevice: ") +
                                                     hipGetErrorString(e));
  MLLM_REQUIRE(dev >= 0 && dev < kMaxDevices, MLLM_ERR_UNSUPPORTED, "mllm_paged_decode_noalloc: device index too large");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(MLLM_ERR_HIP, std::string("mllm_paged_decode_noalloc: hipGetSymbolAddress(scratch): ") +
                                    hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return MLLM_OK;
}

// The most plan records whose partial slots fit in the scratch (two records per slot, plus the header).
int64_t noalloc_max_work(int32_t num_heads, int32_t head_dim) {
  const int64_t per_slot = mllm_decode_workspace_bytes(3, num_heads, head_dim);  // 3 records: one slot
  return per_slot > 0 ? 2 * (kScratchBytes / per_slot) + 2 : 0;
}

}  // namespace

extern "C" int mllm_paged_decode_noalloc(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                                         const void* k_cache, const void* v_cache, int64_t num_blocks,
                                         int32_t block_size, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                         const int32_t* qo_indptr, const int32_t* kv_indptr,
                                         const int32_t* kv_indices, const int32_t* seq_lens,
                                         const int32_t* decode_work, int32_t num_decode_work,
                                         const int32_t* merge_work, int32_t num_merge_work, int32_t pages_per_split,
                                         float softmax_scale, int32_t dtype, void* out, int64_t out_stride_tok,
                                         int64_t out_stride_head, void* stream) {
  using namespace mllm;
  MLLM_REQUIRE(num_decode_work >= 0 && num_merge_work >= 0, MLLM_ERR_INVALID,
               "mllm_paged_decode_noalloc: negative count");
  const int64_t need = num_merge_work ? mllm_decode_workspace_bytes(num_decode_work, num_heads, head_dim) : 0;
  MLLM_REQUIRE(need <= kScratchBytes, MLLM_ERR_INVALID,
               "mllm_paged_decode_noalloc: the step's split partials need " + std::to_string(need) +
                   " bytes, more than the " + std::to_string(kScratchBytes) + "-byte scratch (at most " +
                   std::to_string(noalloc_max_work(num_heads, head_dim)) +
                   " plan records when rows are cut); use mllm_paged_decode with a workspace");
  MLLM_REQUIRE(num_merge_work == 0 || merge_work, MLLM_ERR_INVALID, "mllm_paged_decode_noalloc: null merge_work");
  if (num_decode_work == 0) return MLLM_OK;
  void* ws = nullptr;
  if (need) {
    const int rc = scratch_ptr(&ws);
    if (rc != MLLM_OK) return rc;
  }
  int rc = paged_decode(q, q_stride_tok, q_stride_head, k_cache, v_cache, num_blocks, block_size, num_heads,
                        num_kv_heads, head_dim, qo_indptr, kv_indptr, kv_indices, seq_lens, decode_work,
                        num_decode_work, merge_work, num_merge_work, pages_per_split, softmax_scale, dtype, out,
                        out_stride_tok, out_stride_head, ws, need, false, 1.f, 1.f, stream);
  if (rc != MLLM_OK || num_merge_work == 0) return rc;
  MLLM_REQUIRE(num_heads <= 65535, MLLM_ERR_UNSUPPORTED, "mllm_paged_decode_noalloc: too many heads");
  return launch_merge(merge_work, num_merge_work, num_decode_work, num_heads, qo_indptr, dtype, out, out_stride_tok,
                      out_stride_head, ws, reinterpret_cast<hipStream_t>(stream));
}
