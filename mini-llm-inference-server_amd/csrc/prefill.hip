// Ragged prefill / mixed attention on gfx950 MFMA (reference src/minillm/attention/paged_torch_ref.py:61-73:
// rows with several new tokens, causal within the new chunk and aligned bottom-right over the cached
// prefix; query i of a row with n new tokens and `len` keys sees keys 0 .. len - n + i).
//
// One workgroup (8 wavefronts) per (q tile, KV head).  A q tile is 256 / G new tokens of one row,
// times the G query heads that share the KV head: 256 MFMA rows, 32 per wavefront (rows are
// token-major: row = token * G + head).  K and V stream through LDS in tiles of 64 keys, gathered
// through kv_indices by direct global->LDS loads (global_load_lds_dwordx4: no VGPR staging) into two
// rings of four tiles each (128 KB), so each tile's loads are issued two 128-key phases before its
// first use.  A tile in LDS is its 64 key rows of the head, 256 bytes each, with the 16-byte chunks of row r
// XOR-swizzled (K: chunk ^ (r % 16); V: chunk ^ 4 (r % 4)) so that the MFMA operand reads below hit
// distinct banks.
// Per wavefront and K/V tile:
//   S^T[64 keys x 32 rows] = K . Q^T     2 x 8 v_mfma_f32_32x32x16 (K rows by ds_read_b128; Q^T in VGPRs)
//   O^T[128 x 32 rows]    += V^T . P^T   4 x 4 v_mfma_f32_32x32x16 (V^T by ds_read_b64_tr_b16, the LDS
//                                         transpose read: 4 consecutive keys of one dim per lane)
// S^T and P^T share a lane layout (lane l: row l % 32), so the online softmax (fp32, exp2 domain)
// reduces each row's max and sum inside the lane plus one exchange with lane l ^ 32, and P^T feeds
// the PV product without leaving its lanes.  P^T's 16-key k-order is keys {4h..4h+3, 8+4h..8+4h+3}
// (lane half h); the V^T reads pick their keys in the same order.
//
// The two halves of the workgroup run phase-shifted (prefill128_kernel): one half's matrix phase
// coincides with the other half's softmax, so every SIMD has an MFMA stream and a vector stream at
// once.  A phase covers two tiles (128 keys, one softmax over both score tiles).  Tiles entirely above
// a wavefront's causal diagonal are skipped.  Keys past the workgroup's last visible key are loaded as
// copies of that key's row (their scores are masked, so P is exactly 0 and pool slots past a row's
// length are never read).  The grid is 1-D with the KV head fastest,
// so with 8 KV heads each XCD (workgroups are dealt round-robin to the 8 XCDs) serves one KV head and
// keeps that head's shared-prefix pages in its own L2.
//
// fp8 (e4m3fn) pools: the DMA cannot widen, so tiles go through VGPRs instead.  Each lane loads 16 pool
// bytes of its wavefront's 8 tile rows, widens them to bf16/fp16 (exact) and writes them with
// ds_write_b128 into the same swizzled LDS layout, before the barrier that publishes them (the phase
// of each kernel's loads is stated there).  Everything downstream of LDS is the 16-bit path; k_scale
// is folded into the softmax scale and v_scale into the output.
#include <math.h>

#include "common.h"

namespace mllm {
namespace {

constexpr int kHeadDim = 128;
constexpr int kBN = 64;                      // keys per K/V tile
constexpr int kRowBytes = kHeadDim * 2;      // one key row of the head in LDS
constexpr int kTileBytes = kBN * kRowBytes;  // 16 KB
constexpr int kQTileRows = 256;  // query rows (token x head of the group) per workgroup: 8 waves x 32

struct PrefillArgs {
  const uint16_t* q;
  int64_t q_st, q_sh;
  const uint16_t* kc;
  const uint16_t* vc;
  int64_t num_blocks;
  unsigned page_bytes;  // bytes of one block of one pool: bs * Hkv * Dh * 2 (< 2^32)
  int row_bytes;        // bytes of one token row: Hkv * Dh * 2 (< 2^24)
  int bs, bs_shift, Hkv, G;
  const int32_t* kv_indices;
  const int4* work;  // the plan's prefill records, two int4 each (see the kernel)
  float scale_log2;  // softmax scale x k_scale x log2(e)
  float v_scale;     // output scale of an fp8 pool
  uint16_t* out;
  int64_t o_st, o_sh;
};

// ---------------------------------------------------------------- K/V tile loads
// A 64-key tile is four 16-key groups; a block size is a power of two >= 16, so each group lies in
// one block.  Wavefront w loads tile rows 8 w .. 8 w + 7 (group w / 2) with two DMA instructions of 4
// rows each: lane l writes LDS bytes 16 l .. 16 l + 15 of its instruction's 1 KB, i.e. row
// 8 w + 4 a + l / 16, physical chunk l % 16, and so fetches the logical chunk that the swizzle puts
// there.  The group's block id is wave-uniform (a scalar load); for a full tile the address is a
// 64-bit scalar base plus a per-lane offset that never changes.

// Pool address of slot key0 % bs of block `id` for this head's rows (uniform).
__device__ __forceinline__ const char* group_base(const char* pool, const PrefillArgs& a, int id, int key0) {
  const unsigned b = ((unsigned)id < (unsigned)a.num_blocks) ? (unsigned)id : 0u;  // else-branch never taken
  return pool + ((uint64_t)b * a.page_bytes + (unsigned)(key0 & (a.bs - 1)) * (unsigned)a.row_bytes);
}

// Logical chunk fetched by lane l for tile row r (the inverse of the LDS swizzle; XOR is its own inverse).
__device__ __forceinline__ int k_chunk(int r, int lane) { return (lane & 15) ^ (r & 15); }
__device__ __forceinline__ int v_chunk(int r, int lane) { return (lane & 15) ^ (4 * (r & 3)); }


// This wavefront's share (rows 8 w .. 8 w + 7) of the K or V tile starting at key kv0 into `slot`.
// off0 / off1: the lanes' offsets from the group base for full tiles; IS_V selects the swizzle.
template <bool IS_V>
__device__ __forceinline__ void dma_tile(const char* pool, const PrefillArgs& a, int blk, int kv0, int last,
                                         int kv_end, int w, unsigned off0, unsigned off1, unsigned head_bytes,
                                         int lane, char* slot) {
  const unsigned dst = lds_offset(slot) + 8 * w * kRowBytes;
  if (kv0 + kBN <= kv_end) {
    const char* base = group_base(pool, a, blk, kv0 + 16 * (w >> 1));
    dma16(base, off0, dst);
    dma16(base, off1, dst + 4 * kRowBytes);
  } else {  // a row's last tile: keys past `last` load the row of `last` (same block, P = 0)
    const char* base = group_base(pool, a, blk, 0);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int r = 8 * w + 4 * i + (lane >> 4);
      const int c = IS_V ? v_chunk(r, lane) : k_chunk(r, lane);
      const unsigned slot_bytes = (unsigned)(min(kv0 + r, last) & (a.bs - 1)) * (unsigned)a.row_bytes;
      dma16(base, slot_bytes + head_bytes + 16u * c, dst + 4 * i * kRowBytes);
    }
  }
}

// fp8 pools: this wavefront's share of a tile (rows 8 w .. 8 w + 7, 128 bytes each) is one 16-byte load
// per lane: row 8 w + l / 8, dims 16 (l % 8) .. +15.  off: the lane's offset from the group base for a
// full tile.  Keys past `last` load the row of `last`, as in dma_tile.
__device__ __forceinline__ u32x4 stage_load(const char* pool, const PrefillArgs& a, int blk, int kv0, int last,
                                            int kv_end, int w, unsigned off, unsigned head_bytes, int lane) {
  if (kv0 + kBN <= kv_end) return ld16(group_base(pool, a, blk, kv0 + 16 * (w >> 1)) + off);
  const int r = 8 * w + (lane >> 3);
  const unsigned slot_bytes = (unsigned)(min(kv0 + r, last) & (a.bs - 1)) * (unsigned)a.row_bytes;
  return ld16(group_base(pool, a, blk, 0) + (slot_bytes + head_bytes + 16u * (lane & 7)));
}

// Widens a lane's 16 fp8 values to two 16-byte chunks of 16-bit values (logical chunks 2 (l % 8) and
// 2 (l % 8) + 1 of row 8 w + l / 8) and writes them at their swizzled places in the LDS tile.
template <typename T, bool IS_V>
__device__ __forceinline__ void stage_store(u32x4 x, int w, int lane, char* slot) {
  const int r = 8 * w + (lane >> 3);
  const int c0 = 2 * (lane & 7);
  const int sw = IS_V ? 4 * (r & 3) : (r & 15);
  char* row = slot + r * kRowBytes;
  *reinterpret_cast<u32x4*>(row + 16 * (c0 ^ sw)) = fp8x8_to<T>(x[0], x[1]);
  *reinterpret_cast<u32x4*>(row + 16 * ((c0 + 1) ^ sw)) = fp8x8_to<T>(x[2], x[3]);
}

// ---------------------------------------------------------------- MFMA operands from LDS

__device__ __forceinline__ u32x2 ld_tr(const char* p) {
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)p));
}

struct STile {
  f32x16 s[2];  // s[b][r]: key 32 b + 8 (r / 4) + 4 h + r % 4 of the tile, row n
};

// kb: this lane's byte offset, in the LDS array, of row n at dims 0-15 step (kk = 0) of the K tile:
// row 32 b + n adds 8192 b, and dims step kk moves to logical chunk 2 kk + h, which the swizzle turns
// into a flip of bits 5-7 (kb ^ 32 kk).  The two 32-key halves are independent accumulation chains.
template <typename T>
__device__ __forceinline__ STile scores(const char* lds, unsigned kb, const u32x4 (&qf)[8]) {
  STile t;
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) t.s[b][r] = 0.f;
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) {
    const char* p = lds + (kb ^ (32u * kk));
    t.s[0] = Mfma<T>::m32x32x16(ld16(p), qf[kk], t.s[0]);
    t.s[1] = Mfma<T>::m32x32x16(ld16(p + 32 * kRowBytes), qf[kk], t.s[1]);
  }
  return t;
}

// O^T += V^T . P^T for one tile: 16 MFMAs, the four 32-dim output tiles as independent chains.
// vb: this lane's byte offset, in the LDS array, of its first V^T read (16-key group 0, dims tile 0,
// keys 4h .. 4h+3); dims tile dt flips bits 6-7 (vb ^ 64 dt), 16-key group u adds 4096 u and the
// keys 8+4h .. 8+4h+3 add 2048.  Two transpose reads make one operand: 8 keys of one dim per lane.
template <typename T>
__device__ __forceinline__ void pv_tile(const char* lds, unsigned vb, const u32x4 (&pf)[2][2], f32x16 (&oacc)[4]) {
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        const char* p = lds + (vb ^ (64u * dt)) + 4096 * (2 * b + u);
        const u32x2 lo = ld_tr(p), hi = ld_tr(p + 2048);
        oacc[dt] = Mfma<T>::m32x32x16(u32x4{lo[0], lo[1], hi[0], hi[1]}, pf[b][u], oacc[dt]);
      }
}

// One matrix phase with both products (the common case): O += V(i) P(i), then S(i+1) = K(i+1) Q^T, as
// one sequence of 32 MFMAs whose LDS operands are read kLookahead steps ahead (the wavefront's SIMD
// partner is in its softmax, so nothing else hides the LDS latency).  Step f < 16: PV with 16-key group
// f / 4, dims tile f % 4 (two transpose reads); step f >= 16: S with dims step (f - 16) / 2, key half
// (f - 16) % 2.  sched_barrier keeps the compiler from regrouping the reads next to their MFMAs.
constexpr int kLookahead = 4;

__device__ __forceinline__ u32x4 matrix_operand(const char* lds, unsigned vb, unsigned kb, int f) {
  if (f < 16) {
    const char* p = lds + (vb ^ (64u * (f & 3))) + 4096 * (f >> 2);
    const u32x2 lo = ld_tr(p), hi = ld_tr(p + 2048);
    return u32x4{lo[0], lo[1], hi[0], hi[1]};
  }
  const int g = f - 16;
  return ld16(lds + (kb ^ (32u * (g >> 1))) + 32 * kRowBytes * (g & 1));
}

template <typename T>
__device__ __forceinline__ void matrix_phase(const char* lds, unsigned vb, unsigned kb, const u32x4 (&pf)[2][2],
                                             f32x16 (&oacc)[4], STile& st, const u32x4 (&qf)[8]) {
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) st.s[b][r] = 0.f;
  u32x4 ring[kLookahead + 1];
#pragma unroll
  for (int f = 0; f < kLookahead; ++f) ring[f] = matrix_operand(lds, vb, kb, f);
#pragma unroll
  for (int f = 0; f < 32; ++f) {
    if (f + kLookahead < 32) ring[(f + kLookahead) % (kLookahead + 1)] = matrix_operand(lds, vb, kb, f + kLookahead);
    const u32x4 op = ring[f % (kLookahead + 1)];
    if (f < 16) {
      const int u = f >> 2;
      oacc[f & 3] = Mfma<T>::m32x32x16(op, pf[u >> 1][u & 1], oacc[f & 3]);
    } else {
      const int g = f - 16;
      st.s[g & 1] = Mfma<T>::m32x32x16(op, qf[g >> 1], st.s[g & 1]);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}


// Both matrix phases of a pair as one sequence of 64 MFMAs (PV(a), S(a+2), PV(a+1), S(a+3)), one operand
// ring across it, so the second half's first operands are read while the first half's last MFMAs run.
template <typename T>
__device__ __forceinline__ void matrix_phase_pair(const char* lds, unsigned vb0, unsigned kb0, unsigned vb1,
                                                  unsigned kb1, const u32x4 (&pf0)[2][2], const u32x4 (&pf1)[2][2],
                                                  f32x16 (&oacc)[4], STile& st0, STile& st1, const u32x4 (&qf)[8]) {
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) st0.s[b][r] = st1.s[b][r] = 0.f;
  auto operand = [&](int f) { return (f < 32) ? matrix_operand(lds, vb0, kb0, f) : matrix_operand(lds, vb1, kb1, f - 32); };
  u32x4 ring[kLookahead + 1];
#pragma unroll
  for (int f = 0; f < kLookahead; ++f) ring[f] = operand(f);
#pragma unroll
  for (int f = 0; f < 64; ++f) {
    if (f + kLookahead < 64) ring[(f + kLookahead) % (kLookahead + 1)] = operand(f + kLookahead);
    const u32x4 op = ring[f % (kLookahead + 1)];
    const int g = f & 31;
    const u32x4 (&pf)[2][2] = f < 32 ? pf0 : pf1;
    STile& st = f < 32 ? st0 : st1;
    if (g < 16) {
      const int u = g >> 2;
      oacc[g & 3] = Mfma<T>::m32x32x16(op, pf[u >> 1][u & 1], oacc[g & 3]);
    } else {
      const int e = g - 16;
      st.s[e & 1] = Mfma<T>::m32x32x16(op, qf[e >> 1], st.s[e & 1]);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

// ---------------------------------------------------------------- the kernel: 128-key phases
// Two wavefront groups of one workgroup, phase-shifted by half an iteration: while group A (waves
// 0-3) runs its matrix phase, group B (waves 4-7) runs its vector phase, and the next barrier swaps
// them, so each SIMD (one wave of each group) keeps its matrix pipe and its vector ALU busy together.
// Every phase covers two 64-key tiles (a pair): the matrix phase of pair j runs PV of tiles 2j and
// 2j+1 and S of tiles 2j+2 and 2j+3 (64 MFMAs), and the vector phase runs one softmax over both score
// tiles (one max and one rescale test per 128 keys).  Against phases of one tile (a design measured
// and replaced), half the phases means half the barriers and per-phase bookkeeping per key:
// prefix_64 674 us against 702-716 us, mixed_128 76 against 78-80 us (same box).
// When all four products of a pair run, they are one 64-MFMA sequence with one operand ring
// (matrix_phase_pair), so the second tile's first operands are read under the first tile's last
// MFMAs: another 1.3% on prefix_64 (649 against 657-659 us), bit-identical.
// Rings: K and V four tiles each (128 KB).  Even phase 2j loads V(2j+2), V(2j+3) into the slots of
// V(2j-2), V(2j-1) and K(2j+4), K(2j+5) into those of K(2j), K(2j+1), all freed by the barrier that
// ended phase 2j-1; the barrier ending phase 2j+1 waits for all of them (the next phase reads them).
// A pair's second tile past the row (odd tile counts) or past a wavefront's last row is skipped in the
// matrix phase and fully masked in the softmax, so its P is 0.
// fp8 pools: V(2j+2), V(2j+3) are loaded into VGPRs at the start of phase 2j and K(2j+4), K(2j+5) at
// the start of phase 2j+1, each pair widened into LDS at the end of its phase (the slots are free
// since the barrier that ended phase 2j-1).  The eight staging VGPRs leave no room for the pair's
// single operand ring, so fp8 pools run the two tiles' products one after the other.  Against phases
// of one tile on fp8 pools: prefix_64 725 against 756 us, mixed_128 82 against 87 us (same box).
constexpr int kRingK = 4, kRingV = 4;  // K and V tiles in LDS
constexpr int kVBase = kRingK * kTileBytes;
constexpr int kIdBase = (kRingK + kRingV) * kTileBytes;
constexpr int kLdsBytes = kIdBase + 8 * 2 * 64 * 4;

// Online softmax (exp2 domain) of a pair of score tiles (keys kv0 .. kv0 + 127) -> the bf16/fp16 P^T
// operands of both PV products.  Masks keys past each row's position when the pair reaches past the
// wavefront's first row; rescales O and l lazily: only when some row's max grew by more than 2^8,
// otherwise p = 2^((s - m) c) stays below 256, which the fp32 accumulation and the P operand hold as
// exactly as values below 1.  Row max and row sum run as four chains each (v_max3, plain adds), then
// the other half of the row comes from lane l ^ 32.  The sum is taken over the unrounded p with plain
// adds, because the packed bf16 dot instructions do not run beside MFMAs (each stalls the SIMD
// partner's matrix phase); it differs from the sum of the rounded P operand by unbiased rounding noise.
template <typename T>
__device__ __forceinline__ void softmax_two(STile& s0, STile& s1, u32x4 (&pf0)[2][2], u32x4 (&pf1)[2][2],
                                            f32x16 (&oacc)[4], float& m_run, float& l_run, int kv0, int qp,
                                            int wave_qp_lo, int h, float c) {
  if (kv0 + 2 * kBN - 1 > wave_qp_lo) {  // some key of the pair lies past the wavefront's first row
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kv0 + 32 * b + 8 * (r >> 2) + 4 * h + (r & 3);
        s0.s[b][r] = key > qp ? -INFINITY : s0.s[b][r];
        s1.s[b][r] = key + kBN > qp ? -INFINITY : s1.s[b][r];
      }
  }
  float m4[4] = {s0.s[0][0], s0.s[0][1], s0.s[0][2], s0.s[0][3]};
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      if (b > 0 || r >= 4) m4[r & 3] = __builtin_fmaxf(m4[r & 3], s0.s[b][r]);
      m4[r & 3] = __builtin_fmaxf(m4[r & 3], s1.s[b][r]);
    }
  const float mx = max_xor32(__builtin_fmaxf(__builtin_fmaxf(m4[0], m4[1]), __builtin_fmaxf(m4[2], m4[3])));
  if (__any((mx - m_run) * c > 8.f)) {
    const float m_new = fmaxf(m_run, mx);
    const float alpha = fast_exp2((m_run - m_new) * c);
    l_run *= alpha;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) oacc[dt] *= alpha;
    m_run = m_new;
  }
  const float mc = m_run * c;
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      s0.s[b][r] = fast_exp2(__builtin_fmaf(s0.s[b][r], c, -mc));
      s1.s[b][r] = fast_exp2(__builtin_fmaf(s1.s[b][r], c, -mc));
    }
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int r0 = 8 * u;
      pf0[b][u] = u32x4{pack2<T>(s0.s[b][r0 + 0], s0.s[b][r0 + 1]), pack2<T>(s0.s[b][r0 + 2], s0.s[b][r0 + 3]),
                        pack2<T>(s0.s[b][r0 + 4], s0.s[b][r0 + 5]), pack2<T>(s0.s[b][r0 + 6], s0.s[b][r0 + 7])};
      pf1[b][u] = u32x4{pack2<T>(s1.s[b][r0 + 0], s1.s[b][r0 + 1]), pack2<T>(s1.s[b][r0 + 2], s1.s[b][r0 + 3]),
                        pack2<T>(s1.s[b][r0 + 4], s1.s[b][r0 + 5]), pack2<T>(s1.s[b][r0 + 6], s1.s[b][r0 + 7])};
    }
  float s4[4] = {s0.s[0][0], s0.s[0][1], s0.s[0][2], s0.s[0][3]};
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      if (b > 0 || r >= 4) s4[r & 3] += s0.s[b][r];
      s4[r & 3] += s1.s[b][r];
    }
  l_run += sum_xor32((s4[0] + s4[1]) + (s4[2] + s4[3]));
}

template <typename T, bool F8>
__global__ __launch_bounds__(512) void prefill128_kernel(const PrefillArgs a) {
  __shared__ __attribute__((aligned(1024))) char lds[kLdsBytes];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int grp = wave >> 2;
  const int wu = __builtin_amdgcn_readfirstlane(wave);
  const int kvh = blockIdx.x % a.Hkv;
  const int4 w0 = a.work[2 * (blockIdx.x / a.Hkv)], w1 = a.work[2 * (blockIdx.x / a.Hkv) + 1];
  const int seq = w0.x, t0 = w0.y, qs = w0.z, nn = w0.w, cached = w1.x;
  if (seq < 0 || w1.z <= 0) return;
  const int len = cached + nn;
  const int32_t* pages = a.kv_indices + w1.y;
  const int tpw = 32 / a.G;
  const int kv_end = w1.z;
  const int last = kv_end - 1;
  const int ntiles = w1.w;
  const int npairs = (ntiles + 1) >> 1;

  const int n = lane & 31, h = lane >> 5;
  const int tok = t0 + wave * tpw + n / a.G;
  const bool row_valid = tok < nn;
  const int qp = row_valid ? cached + tok : len - 1;
  const int wave_tok_hi = min(t0 + wave * tpw + tpw, nn) - 1;
  const int wave_qp_hi = wave_tok_hi >= t0 + wave * tpw ? cached + wave_tok_hi : -1;
  const int wave_qp_lo = cached + t0 + wave * tpw;
  const float c = a.scale_log2;

  const unsigned head_bytes = (unsigned)(kvh * kHeadDim * (F8 ? 1 : 2));
  const int r0 = 8 * wave + (lane >> 4), r1 = r0 + 4;
  const unsigned rb = (unsigned)a.row_bytes;
  const unsigned koff0 = (unsigned)(r0 & 15) * rb + head_bytes + 16u * k_chunk(r0, lane);
  const unsigned koff1 = (unsigned)(r1 & 15) * rb + head_bytes + 16u * k_chunk(r1, lane);
  const unsigned voff0 = (unsigned)(r0 & 15) * rb + head_bytes + 16u * v_chunk(r0, lane);
  const unsigned voff1 = (unsigned)(r1 & 15) * rb + head_bytes + 16u * v_chunk(r1, lane);
  const unsigned soff = (unsigned)(8 * (wave & 1) + (lane >> 3)) * rb + head_bytes + 16u * (lane & 7);  // fp8
  const unsigned kread = (unsigned)(n * kRowBytes + 16 * (h ^ (n & 1)) + 32 * ((n & 15) >> 1));
  const unsigned vread = (unsigned)(kVBase + 1024 * h + 320 * ((lane >> 2) & 3) + 32 * ((lane >> 4) & 1) + 8 * (lane & 3));

  const char* kc = reinterpret_cast<const char*>(a.kc);
  const char* vc = reinterpret_cast<const char*>(a.vc);
  const int g16 = 16 * (wu >> 1);
  auto k_slot = [&](int t) { return lds + (t & (kRingK - 1)) * kTileBytes; };
  auto v_slot = [&](int t) { return lds + kVBase + (t & (kRingV - 1)) * kTileBytes; };

  const int* idwin = reinterpret_cast<const int*>(lds + kIdBase) + wu * 128;
  auto load_ids = [&](int base, int sel) {
    dma4(reinterpret_cast<const char*>(pages), 4u * (unsigned)(min((base + lane) * kBN + g16, last) >> a.bs_shift),
         lds_offset(idwin + 64 * sel));
  };
  int wbase = 0, wsel = 0;
  auto blk_of = [&](int t) { return __builtin_amdgcn_readfirstlane(idwin[64 * wsel + t - wbase]); };
  load_ids(0, 0);
  auto blk_direct = [&](int t) { return pages[min(t * kBN + g16, last) >> a.bs_shift]; };

  f32x16 oacc[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[dt][r] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  // prologue: K(0..3), V(0..1), then Q; all of them have landed after the first barrier (fp8 pools: all
  // six tiles loaded into registers first, then widened into LDS)
  if constexpr (F8) {
    u32x4 kx[4], vx[2];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      if (t < ntiles) {
        const int b = blk_direct(t);
        kx[t] = stage_load(kc, a, b, t * kBN, last, kv_end, wu, soff, head_bytes, lane);
        if (t < 2) vx[t] = stage_load(vc, a, b, t * kBN, last, kv_end, wu, soff, head_bytes, lane);
      }
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      if (t < ntiles) {
        stage_store<T, false>(kx[t], wu, lane, k_slot(t));
        if (t < 2) stage_store<T, true>(vx[t], wu, lane, v_slot(t));
      }
    }
  } else {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      if (t < ntiles) {
        const int b = blk_direct(t);
        dma_tile<false>(kc, a, b, t * kBN, last, kv_end, wu, koff0, koff1, head_bytes, lane, k_slot(t));
        if (t < 2) dma_tile<true>(vc, a, b, t * kBN, last, kv_end, wu, voff0, voff1, head_bytes, lane, v_slot(t));
      }
    }
  }
  u32x4 qf[8];
  {
    const int head = kvh * a.G + (n % a.G);
    const uint16_t* qrow = a.q + (int64_t)(qs + (row_valid ? tok : 0)) * a.q_st + (int64_t)head * a.q_sh;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      const u32x4 v = ld16(qrow + 16 * kk + 8 * h);
      qf[kk] = row_valid ? v : u32x4{0, 0, 0, 0};
    }
  }
  asm volatile("" ::"v"(qf[0]), "v"(qf[1]), "v"(qf[2]), "v"(qf[3]), "v"(qf[4]), "v"(qf[5]), "v"(qf[6]), "v"(qf[7])
               : "memory");
  barrier_vm<0>();

  STile st0, st1;
  u32x4 pf0[2][2], pf1[2][2];
  if (0 <= wave_qp_hi) {
    st0 = scores<T>(lds, kread, qf);
    if (1 < ntiles && kBN <= wave_qp_hi) st1 = scores<T>(lds, kread + kTileBytes, qf);
    if (grp == 0) softmax_two<T>(st0, st1, pf0, pf1, oacc, m_run, l_run, 0, qp, wave_qp_lo, h, c);
  }
  barrier_lds();  // K(0), K(1) have been read: phase 0 loads K(4), K(5) into their slots

  // fp8 pools: V(2j+2), V(2j+3) pass through registers during the even phase and K(2j+4), K(2j+5) during
  // the odd one, each widened into LDS at the end of its phase
  u32x4 st_a = {0, 0, 0, 0}, st_b = {0, 0, 0, 0};
  int k0b = 0, k1b = 0;
  for (int p = 0; p < 2 * npairs; ++p) {
    const int j = p >> 1;
    const int ta = 2 * j;  // the pair's first tile
    if ((p & 1) == 0) {
      const int v0b = blk_of(ta + 2), v1b = blk_of(ta + 3);
      k0b = blk_of(ta + 4);
      k1b = blk_of(ta + 5);
      if (ta + 7 >= wbase + 64) {  // the next even phase reads ids of tiles ta + 4 .. ta + 7
        wsel ^= 1;
        wbase = ta + 4;
        load_ids(wbase, wsel);
      }
      if constexpr (F8) {
        if (ta + 2 < ntiles) st_a = stage_load(vc, a, v0b, (ta + 2) * kBN, last, kv_end, wu, soff, head_bytes, lane);
        if (ta + 3 < ntiles) st_b = stage_load(vc, a, v1b, (ta + 3) * kBN, last, kv_end, wu, soff, head_bytes, lane);
      } else {
        if (ta + 2 < ntiles)
          dma_tile<true>(vc, a, v0b, (ta + 2) * kBN, last, kv_end, wu, voff0, voff1, head_bytes, lane, v_slot(ta + 2));
        if (ta + 3 < ntiles)
          dma_tile<true>(vc, a, v1b, (ta + 3) * kBN, last, kv_end, wu, voff0, voff1, head_bytes, lane, v_slot(ta + 3));
        if (ta + 4 < ntiles)
          dma_tile<false>(kc, a, k0b, (ta + 4) * kBN, last, kv_end, wu, koff0, koff1, head_bytes, lane, k_slot(ta + 4));
        if (ta + 5 < ntiles)
          dma_tile<false>(kc, a, k1b, (ta + 5) * kBN, last, kv_end, wu, koff0, koff1, head_bytes, lane, k_slot(ta + 5));
      }
    } else if constexpr (F8) {
      if (ta + 4 < ntiles) st_a = stage_load(kc, a, k0b, (ta + 4) * kBN, last, kv_end, wu, soff, head_bytes, lane);
      if (ta + 5 < ntiles) st_b = stage_load(kc, a, k1b, (ta + 5) * kBN, last, kv_end, wu, soff, head_bytes, lane);
    }
    if ((p & 1) == grp) {  // matrix phase of pair j
      __builtin_amdgcn_s_setprio(1);
      // all four products of the pair (fp8 pools keep two tiles of staging registers: no single ring)
      const bool full = !F8 && ta + 3 < ntiles && (ta + 3) * kBN <= wave_qp_hi;
      if (full) {
        matrix_phase_pair<T>(lds, vread + (ta & (kRingV - 1)) * kTileBytes, kread + ((ta + 2) & (kRingK - 1)) * kTileBytes,
                             vread + ((ta + 1) & (kRingV - 1)) * kTileBytes, kread + ((ta + 3) & (kRingK - 1)) * kTileBytes,
                             pf0, pf1, oacc, st0, st1, qf);
      } else
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int tv = ta + u, tk = ta + 2 + u;
        const unsigned vb = vread + (tv & (kRingV - 1)) * kTileBytes, kb = kread + (tk & (kRingK - 1)) * kTileBytes;
        const bool do_pv = tv < ntiles && tv * kBN <= wave_qp_hi, do_s = tk < ntiles && tk * kBN <= wave_qp_hi;
        STile& st = u ? st1 : st0;
        const u32x4 (&pf)[2][2] = u ? pf1 : pf0;
        if (do_pv && do_s) {
          matrix_phase<T>(lds, vb, kb, pf, oacc, st, qf);
        } else {
          if (do_pv) pv_tile<T>(lds, vb, pf, oacc);
          if (do_s) st = scores<T>(lds, kb, qf);
        }
      }
      __builtin_amdgcn_s_setprio(0);
    } else {  // vector phase: softmax of the pair starting at tile 2 ((p + 1) >> 1)
      const int tn = 2 * ((p + 1) >> 1);
      if (tn < ntiles && tn * kBN <= wave_qp_hi)
        softmax_two<T>(st0, st1, pf0, pf1, oacc, m_run, l_run, tn * kBN, qp, wave_qp_lo, h, c);
    }
    if constexpr (F8) {  // the staged tiles' slots were freed by the barrier that ended phase 2j-1
      if ((p & 1) == 0) {
        if (ta + 2 < ntiles) stage_store<T, true>(st_a, wu, lane, v_slot(ta + 2));
        if (ta + 3 < ntiles) stage_store<T, true>(st_b, wu, lane, v_slot(ta + 3));
      } else {
        if (ta + 4 < ntiles) stage_store<T, false>(st_a, wu, lane, k_slot(ta + 4));
        if (ta + 5 < ntiles) stage_store<T, false>(st_b, wu, lane, k_slot(ta + 5));
      }
      if (p & 1)
        barrier_vm<0>();  // also the id window loaded in the even phase
      else
        barrier_lds();
    } else {
      if (p & 1)
        barrier_vm<0>();
      else
        barrier_lds();
    }
  }

  const float inv = (F8 ? a.v_scale : 1.f) / l_run;
  char* ost = lds + wave * (32 * kRowBytes);
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const int r = 4 * g4;
      const u32x2 pk = u32x2{pack2<T>(oacc[dt][r] * inv, oacc[dt][r + 1] * inv),
                             pack2<T>(oacc[dt][r + 2] * inv, oacc[dt][r + 3] * inv)};
      *reinterpret_cast<u32x2*>(ost + n * kRowBytes + 16 * ((4 * dt + g4) ^ (n & 15)) + 8 * h) = pk;
    }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int row = 4 * i + (lane >> 4), chunk = lane & 15;
    const u32x4 v = *reinterpret_cast<const u32x4*>(ost + row * kRowBytes + 16 * (chunk ^ (row & 15)));
    const int rtok = t0 + wave * tpw + row / a.G;
    if (rtok < nn) {
      uint16_t* o = a.out + (int64_t)(qs + rtok) * a.o_st + (int64_t)(kvh * a.G + row % a.G) * a.o_sh;
      *reinterpret_cast<u32x4*>(o + 8 * chunk) = v;
    }
  }
}

// ---------------------------------------------------------------- the kernel: 4 wavefronts, two per CU
// prefill4w_kernel: one workgroup of 4 wavefronts per (q tile of 128 rows, KV head), 32 rows per
// wavefront as above, one 64-key tile per step.  Its LDS is 80 KB (a K ring of three tiles and a V ring
// of two), and its wavefronts stay within 256 registers, so two workgroups share a CU: while one runs its
// prologue (record, block ids, first tiles, first scores) or drains its output stores, the other's
// matrix and vector work keeps the SIMDs busy.  The two wavefronts on a SIMD come from different
// workgroups and are not phase-locked; the matrix phase runs at raised priority.
// Step j: the matrix phase runs PV(j) and S(j+1) as one 32-MFMA sequence, then the vector phase the
// softmax of tile j+1.  At the start of step j the wavefront issues V(j+1) into the V slot of V(j-1) and
// K(j+3) into the K slot of K(j), both last read in step j-1; the barrier ending step j waits for every
// load but K(j+3), so step j+1 finds V(j+1) and K(j+2) in LDS.  Block ids are read with scalar loads
// one step ahead of their loads.
// fp8 pools: the same two tiles are loaded into VGPRs at the start of step j (two 16-byte loads per lane
// each: the wavefront's 16 rows of 128 bytes) and widened into their LDS slots at its end, before the
// barrier; the slots were last read in step j-1.
constexpr int kQTileRows4 = 128;  // query rows per workgroup: 4 waves x 32
constexpr int kRingK4 = 3, kRingV4 = 2;
constexpr int kVBase4 = kRingK4 * kTileBytes;
constexpr int kLdsBytes4 = (kRingK4 + kRingV4) * kTileBytes;  // 80 KB: two workgroups fill 160 KB

// This wavefront's share (rows 16 w .. 16 w + 15, the tile's 16-key group w) of the K or V tile at kv0,
// four DMA instructions of 4 rows.  off[i]: lane offsets from the group base for a full tile.
template <bool IS_V>
__device__ __forceinline__ void dma_tile4(const char* pool, const PrefillArgs& a, int blk, int kv0, int last,
                                          int kv_end, int w, const unsigned (&off)[4], unsigned head_bytes,
                                          int lane, char* slot) {
  const unsigned dst = lds_offset(slot) + 16 * w * kRowBytes;
  if (kv0 + kBN <= kv_end) {
    const char* base = group_base(pool, a, blk, kv0 + 16 * w);
#pragma unroll
    for (int i = 0; i < 4; ++i) dma16(base, off[i], dst + 4 * i * kRowBytes);
  } else {  // a row's last tile: keys past `last` load the row of `last` (same block, P = 0)
    const char* base = group_base(pool, a, blk, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 16 * w + 4 * i + (lane >> 4);
      const int c = IS_V ? v_chunk(r, lane) : k_chunk(r, lane);
      const unsigned slot_bytes = (unsigned)(min(kv0 + r, last) & (a.bs - 1)) * (unsigned)a.row_bytes;
      dma16(base, slot_bytes + head_bytes + 16u * c, dst + 4 * i * kRowBytes);
    }
  }
}

// Online softmax (exp2 domain) of one score tile (keys kv0 .. kv0 + 63) -> the P^T operand of its PV
// product; the rules of softmax_two (masking, lazy rescale past 2^8, sums over unrounded p) on one tile.
template <typename T>
__device__ __forceinline__ void softmax_one(STile& s, u32x4 (&pf)[2][2], f32x16 (&oacc)[4], float& m_run,
                                            float& l_run, int kv0, int qp, int wave_qp_lo, int h, float c) {
  if (kv0 + kBN - 1 > wave_qp_lo) {
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kv0 + 32 * b + 8 * (r >> 2) + 4 * h + (r & 3);
        s.s[b][r] = key > qp ? -INFINITY : s.s[b][r];
      }
  }
  float m4[4] = {s.s[0][0], s.s[0][1], s.s[0][2], s.s[0][3]};
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r)
      if (b > 0 || r >= 4) m4[r & 3] = __builtin_fmaxf(m4[r & 3], s.s[b][r]);
  const float mx = max_xor32(__builtin_fmaxf(__builtin_fmaxf(m4[0], m4[1]), __builtin_fmaxf(m4[2], m4[3])));
  if (__any((mx - m_run) * c > 8.f)) {
    const float m_new = fmaxf(m_run, mx);
    const float alpha = fast_exp2((m_run - m_new) * c);
    l_run *= alpha;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) oacc[dt] *= alpha;
    m_run = m_new;
  }
  const float mc = m_run * c;
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) s.s[b][r] = fast_exp2(__builtin_fmaf(s.s[b][r], c, -mc));
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int r0 = 8 * u;
      pf[b][u] = u32x4{pack2<T>(s.s[b][r0 + 0], s.s[b][r0 + 1]), pack2<T>(s.s[b][r0 + 2], s.s[b][r0 + 3]),
                       pack2<T>(s.s[b][r0 + 4], s.s[b][r0 + 5]), pack2<T>(s.s[b][r0 + 6], s.s[b][r0 + 7])};
    }
  float s4[4] = {s.s[0][0], s.s[0][1], s.s[0][2], s.s[0][3]};
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r)
      if (b > 0 || r >= 4) s4[r & 3] += s.s[b][r];
  l_run += sum_xor32((s4[0] + s4[1]) + (s4[2] + s4[3]));
}

typedef const __attribute__((address_space(4))) int32_t ConstI32;

template <typename T, bool F8>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void prefill4w_kernel(
    const PrefillArgs a) {
  __shared__ __attribute__((aligned(1024))) char lds[kLdsBytes4];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wu = __builtin_amdgcn_readfirstlane(wave);
  const int kvh = blockIdx.x % a.Hkv;
  const int4 w0 = a.work[2 * (blockIdx.x / a.Hkv)], w1 = a.work[2 * (blockIdx.x / a.Hkv) + 1];
  const int seq = w0.x, t0 = w0.y, qs = w0.z, nn = w0.w, cached = w1.x;
  if (seq < 0 || w1.z <= 0) return;
  const int len = cached + nn;
  ConstI32* pages = (ConstI32*)(a.kv_indices + w1.y);
  const int tpw = 32 / a.G;
  const int kv_end = w1.z;
  const int last = kv_end - 1;
  const int ntiles = w1.w;

  const int n = lane & 31, h = lane >> 5;
  const int tok = t0 + wave * tpw + n / a.G;
  const bool row_valid = tok < nn;
  const int qp = row_valid ? cached + tok : len - 1;
  const int wave_tok_hi = min(t0 + wave * tpw + tpw, nn) - 1;
  const int wave_qp_hi = wave_tok_hi >= t0 + wave * tpw ? cached + wave_tok_hi : -1;
  const int wave_qp_lo = cached + t0 + wave * tpw;
  const float c = a.scale_log2;

  const unsigned head_bytes = (unsigned)(kvh * kHeadDim * (F8 ? 1 : 2));
  const unsigned rb = (unsigned)a.row_bytes;
  unsigned koff[4], voff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 4 * i + (lane >> 4);  // the tile row modulo 16
    koff[i] = (unsigned)r * rb + head_bytes + 16u * k_chunk(r, lane);
    voff[i] = (unsigned)r * rb + head_bytes + 16u * v_chunk(r, lane);
  }
  // fp8: this wavefront's rows as two 8-row shares (those of wavefront 2 w + i of the 8-wavefront layout)
  const unsigned soff0 = (unsigned)(lane >> 3) * rb + head_bytes + 16u * (lane & 7), soff1 = soff0 + 8 * rb;
  auto stage2 = [&](const char* pool, int b, int t, u32x4 (&x)[2]) {
    x[0] = stage_load(pool, a, b, t * kBN, last, kv_end, 2 * wu, soff0, head_bytes, lane);
    x[1] = stage_load(pool, a, b, t * kBN, last, kv_end, 2 * wu + 1, soff1, head_bytes, lane);
  };
  auto store2 = [&](bool is_v, const u32x4 (&x)[2], char* slot) {
    if (is_v) {
      stage_store<T, true>(x[0], 2 * wu, lane, slot);
      stage_store<T, true>(x[1], 2 * wu + 1, lane, slot);
    } else {
      stage_store<T, false>(x[0], 2 * wu, lane, slot);
      stage_store<T, false>(x[1], 2 * wu + 1, lane, slot);
    }
  };
  const unsigned kread = (unsigned)(n * kRowBytes + 16 * (h ^ (n & 1)) + 32 * ((n & 15) >> 1));
  const unsigned vread = (unsigned)(kVBase4 + 1024 * h + 320 * ((lane >> 2) & 3) + 32 * ((lane >> 4) & 1) + 8 * (lane & 3));

  const char* kc = reinterpret_cast<const char*>(a.kc);
  const char* vc = reinterpret_cast<const char*>(a.vc);
  auto k_slot = [&](int t) { return lds + (t % kRingK4) * kTileBytes; };
  auto v_slot = [&](int t) { return lds + kVBase4 + (t & (kRingV4 - 1)) * kTileBytes; };
  // block id of this wavefront's 16-key group of tile t (clamped into the row: always a valid entry)
  auto blk = [&](int t) { return __builtin_amdgcn_readfirstlane(pages[min(t * kBN + 16 * wu, last) >> a.bs_shift]); };

  f32x16 oacc[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[dt][r] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  // prologue: K(0..2), V(0), then Q; all landed after the first barrier
  int i1 = blk(1), i2 = blk(2), i3 = blk(3);  // ids of tiles j + 1 .. j + 3 at step j = 0
  if constexpr (F8) {
    const int b0 = blk(0);
    u32x4 k0[2], v0[2], k1[2], k2[2];
    stage2(kc, b0, 0, k0);
    stage2(vc, b0, 0, v0);
    if (1 < ntiles) stage2(kc, i1, 1, k1);
    if (2 < ntiles) stage2(kc, i2, 2, k2);
    store2(false, k0, k_slot(0));
    store2(true, v0, v_slot(0));
    if (1 < ntiles) store2(false, k1, k_slot(1));
    if (2 < ntiles) store2(false, k2, k_slot(2));
  } else {
    const int b0 = blk(0);
    dma_tile4<false>(kc, a, b0, 0, last, kv_end, wu, koff, head_bytes, lane, k_slot(0));
    dma_tile4<true>(vc, a, b0, 0, last, kv_end, wu, voff, head_bytes, lane, v_slot(0));
    if (1 < ntiles) dma_tile4<false>(kc, a, i1, kBN, last, kv_end, wu, koff, head_bytes, lane, k_slot(1));
    if (2 < ntiles) dma_tile4<false>(kc, a, i2, 2 * kBN, last, kv_end, wu, koff, head_bytes, lane, k_slot(2));
  }
  u32x4 qf[8];
  {
    const int head = kvh * a.G + (n % a.G);
    const uint16_t* qrow = a.q + (int64_t)(qs + (row_valid ? tok : 0)) * a.q_st + (int64_t)head * a.q_sh;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      const u32x4 v = ld16(qrow + 16 * kk + 8 * h);
      qf[kk] = row_valid ? v : u32x4{0, 0, 0, 0};
    }
  }
  asm volatile("" ::"v"(qf[0]), "v"(qf[1]), "v"(qf[2]), "v"(qf[3]), "v"(qf[4]), "v"(qf[5]), "v"(qf[6]), "v"(qf[7])
               : "memory");
  barrier_vm<0>();

  STile st;
  u32x4 pf[2][2];
  if (0 <= wave_qp_hi) {
    st = scores<T>(lds, kread, qf);
    softmax_one<T>(st, pf, oacc, m_run, l_run, 0, qp, wave_qp_lo, h, c);
  }
  barrier_lds();  // K(0) has been read: step 0 loads K(3) into its slot

  u32x4 sv[2] = {}, sk[2] = {};  // fp8: V(j+1) and K(j+3) on their way through registers
  for (int j = 0; j < ntiles; ++j) {
    const bool v_ahead = j + 1 < ntiles, k_ahead = j + 3 < ntiles;
    if constexpr (F8) {
      if (v_ahead) stage2(vc, i1, j + 1, sv);
      if (k_ahead) stage2(kc, i3, j + 3, sk);
    } else {
      if (v_ahead)
        dma_tile4<true>(vc, a, i1, (j + 1) * kBN, last, kv_end, wu, voff, head_bytes, lane, v_slot(j + 1));
      if (k_ahead)
        dma_tile4<false>(kc, a, i3, (j + 3) * kBN, last, kv_end, wu, koff, head_bytes, lane, k_slot(j + 3));
    }
    const int i4 = blk(j + 4);
    i1 = i2;
    i2 = i3;
    i3 = i4;
    const bool do_pv = j * kBN <= wave_qp_hi, do_s = j + 1 < ntiles && (j + 1) * kBN <= wave_qp_hi;
    const unsigned vb = vread + (j & (kRingV4 - 1)) * kTileBytes, kb = kread + ((j + 1) % kRingK4) * kTileBytes;
    __builtin_amdgcn_s_setprio(1);
    if (do_pv && do_s) {
      matrix_phase<T>(lds, vb, kb, pf, oacc, st, qf);
    } else {
      if (do_pv) pv_tile<T>(lds, vb, pf, oacc);
      if (do_s) st = scores<T>(lds, kb, qf);
    }
    __builtin_amdgcn_s_setprio(0);
    if (do_s) softmax_one<T>(st, pf, oacc, m_run, l_run, (j + 1) * kBN, qp, wave_qp_lo, h, c);
    if constexpr (F8) {  // widened into the slots of V(j-1) and K(j), both last read in step j-1
      if (v_ahead) store2(true, sv, v_slot(j + 1));
      if (k_ahead) store2(false, sk, k_slot(j + 3));
      barrier_lds();
    } else if (k_ahead) {  // every load but K(j+3) has landed, and every wavefront is done with V(j), K(j+1)
      barrier_vm<4>();
    } else {
      barrier_vm<0>();
    }
  }

  // output: each wavefront's 32 x 128 block transposed through its 8 KB of the K ring (no DMA is in flight
  // and every wavefront is past its last read of the rings), then whole 16-byte chunks per row
  const float inv = (F8 ? a.v_scale : 1.f) / l_run;
  char* ost = lds + wave * (32 * kRowBytes);
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const int r = 4 * g4;
      const u32x2 pk = u32x2{pack2<T>(oacc[dt][r] * inv, oacc[dt][r + 1] * inv),
                             pack2<T>(oacc[dt][r + 2] * inv, oacc[dt][r + 3] * inv)};
      *reinterpret_cast<u32x2*>(ost + n * kRowBytes + 16 * ((4 * dt + g4) ^ (n & 15)) + 8 * h) = pk;
    }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int row = 4 * i + (lane >> 4), chunk = lane & 15;
    const u32x4 v = *reinterpret_cast<const u32x4*>(ost + row * kRowBytes + 16 * (chunk ^ (row & 15)));
    const int rtok = t0 + wave * tpw + row / a.G;
    if (rtok < nn) {
      uint16_t* o = a.out + (int64_t)(qs + rtok) * a.o_st + (int64_t)(kvh * a.G + row % a.G) * a.o_sh;
      *reinterpret_cast<u32x4*>(o + 8 * chunk) = v;
    }
  }
}
}  // namespace
}  // namespace mllm

namespace {

int paged_prefill(const void* q, int64_t q_stride_tok, int64_t q_stride_head, const void* k_cache,
                                  const void* v_cache, int64_t num_blocks, int32_t block_size, int32_t num_heads,
                                  int32_t num_kv_heads, int32_t head_dim, const int32_t* qo_indptr,
                                  const int32_t* kv_indptr, const int32_t* kv_indices, const int32_t* seq_lens,
                                  const int32_t* prefill_work, int32_t num_prefill_work, int32_t q_tile_tokens,
                                  float softmax_scale, int32_t dtype, void* out, int64_t out_stride_tok,
                                  int64_t out_stride_head, bool fp8, float k_scale, float v_scale, void* stream) {
  using namespace mllm;
  const std::string fn = fp8 ? "mllm_paged_prefill_fp8" : "mllm_paged_prefill";
  MLLM_REQUIRE(dtype == MLLM_DTYPE_BF16 || dtype == MLLM_DTYPE_F16, MLLM_ERR_UNSUPPORTED,
               fn + ": dtype must be bfloat16 or float16");
  MLLM_REQUIRE(head_dim == kHeadDim, MLLM_ERR_UNSUPPORTED, fn + ": head_dim must be 128");
  MLLM_REQUIRE(k_scale > 0.f && v_scale > 0.f && k_scale < INFINITY && v_scale < INFINITY, MLLM_ERR_INVALID,
               fn + ": scales must be positive and finite");
  MLLM_REQUIRE(block_size >= 16 && (block_size & (block_size - 1)) == 0, MLLM_ERR_UNSUPPORTED,
               fn + ": block_size must be a power of two >= 16");
  MLLM_REQUIRE(num_kv_heads > 0 && num_heads > 0 && num_heads % num_kv_heads == 0, MLLM_ERR_INVALID,
               fn + ": num_heads must be a multiple of num_kv_heads");
  const int G = num_heads / num_kv_heads;
  MLLM_REQUIRE(32 % G == 0, MLLM_ERR_UNSUPPORTED, fn + ": H / Hkv must divide 32");
  const bool four_waves = q_tile_tokens == kQTileRows4 / G;
  MLLM_REQUIRE(q_tile_tokens == kQTileRows / G || four_waves, MLLM_ERR_INVALID,
               fn + ": q_tile_tokens must be 256 / (H / Hkv) or 128 / (H / Hkv)");
  MLLM_REQUIRE(num_prefill_work >= 0, MLLM_ERR_INVALID, fn + ": negative count");
  if (num_prefill_work == 0) return MLLM_OK;
  MLLM_REQUIRE(q && k_cache && v_cache && out && qo_indptr && kv_indptr && kv_indices && seq_lens && prefill_work,
               MLLM_ERR_INVALID, fn + ": null pointer");
  const bool aligned = ((uintptr_t)q % 16 == 0) && ((uintptr_t)out % 16 == 0) && ((uintptr_t)k_cache % 16 == 0) &&
                       ((uintptr_t)v_cache % 16 == 0) && (q_stride_tok * 2) % 16 == 0 &&
                       (q_stride_head * 2) % 16 == 0 && (out_stride_tok * 2) % 16 == 0 && (out_stride_head * 2) % 16 == 0;
  MLLM_REQUIRE(aligned, MLLM_ERR_UNSUPPORTED, fn + ": q, out and pools need aligned rows");
  MLLM_REQUIRE((int64_t)num_prefill_work * num_kv_heads < (1ll << 31), MLLM_ERR_UNSUPPORTED,
               fn + ": too many work items");
  MLLM_REQUIRE(num_kv_heads * head_dim * 2 < (1 << 24) && (int64_t)block_size * num_kv_heads * head_dim * 2 < (1ll << 32),
               MLLM_ERR_UNSUPPORTED, fn + ": KV block too large");
  PrefillArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.q_st = q_stride_tok;
  a.q_sh = q_stride_head;
  a.kc = static_cast<const uint16_t*>(k_cache);
  a.vc = static_cast<const uint16_t*>(v_cache);
  a.num_blocks = num_blocks;
  a.row_bytes = num_kv_heads * head_dim * (fp8 ? 1 : 2);
  a.page_bytes = (unsigned)((int64_t)block_size * a.row_bytes);
  a.bs = block_size;
  a.bs_shift = __builtin_ctz((unsigned)block_size);
  a.Hkv = num_kv_heads;
  a.G = G;
  a.kv_indices = kv_indices;  // qo_indptr, kv_indptr and seq_lens are folded into the plan's records
  a.work = reinterpret_cast<const int4*>(prefill_work);
  a.scale_log2 = softmax_scale * k_scale * kLog2e;
  a.v_scale = v_scale;
  a.out = static_cast<uint16_t*>(out);
  a.o_st = out_stride_tok;
  a.o_sh = out_stride_head;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const unsigned grid = (unsigned)num_prefill_work * (unsigned)num_kv_heads;
  if (four_waves) {  // 128-row items: 4-wavefront workgroups, two per CU
    if (dtype == MLLM_DTYPE_BF16) {
      if (fp8)
        prefill4w_kernel<BF16, true><<<grid, 256, 0, st>>>(a);
      else
        prefill4w_kernel<BF16, false><<<grid, 256, 0, st>>>(a);
    } else {
      if (fp8)
        prefill4w_kernel<F16, true><<<grid, 256, 0, st>>>(a);
      else
        prefill4w_kernel<F16, false><<<grid, 256, 0, st>>>(a);
    }
  } else if (dtype == MLLM_DTYPE_BF16) {
    if (fp8)
      prefill128_kernel<BF16, true><<<grid, 512, 0, st>>>(a);
    else
      prefill128_kernel<BF16, false><<<grid, 512, 0, st>>>(a);
  } else {
    if (fp8)
      prefill128_kernel<F16, true><<<grid, 512, 0, st>>>(a);
    else
      prefill128_kernel<F16, false><<<grid, 512, 0, st>>>(a);
  }
  return check_launch(fn.c_str());
}

}  // namespace

extern "C" int mllm_paged_prefill(const void* q, int64_t q_stride_tok, int64_t q_stride_head, const void* k_cache,
                                  const void* v_cache, int64_t num_blocks, int32_t block_size, int32_t num_heads,
                                  int32_t num_kv_heads, int32_t head_dim, const int32_t* qo_indptr,
                                  const int32_t* kv_indptr, const int32_t* kv_indices, const int32_t* seq_lens,
                                  const int32_t* prefill_work, int32_t num_prefill_work, int32_t q_tile_tokens,
                                  float softmax_scale, int32_t dtype, void* out, int64_t out_stride_tok,
                                  int64_t out_stride_head, void* stream) {
  return paged_prefill(q, q_stride_tok, q_stride_head, k_cache, v_cache, num_blocks, block_size, num_heads,
                       num_kv_heads, head_dim, qo_indptr, kv_indptr, kv_indices, seq_lens, prefill_work,
                       num_prefill_work, q_tile_tokens, softmax_scale, dtype, out, out_stride_tok, out_stride_head,
                       false, 1.f, 1.f, stream);
}

extern "C" int mllm_paged_prefill_fp8(const void* q, int64_t q_stride_tok, int64_t q_stride_head, const void* k_cache,
                                      const void* v_cache, int64_t num_blocks, int32_t block_size, int32_t num_heads,
                                      int32_t num_kv_heads, int32_t head_dim, const int32_t* qo_indptr,
                                      const int32_t* kv_indptr, const int32_t* kv_indices, const int32_t* seq_lens,
                                      const int32_t* prefill_work, int32_t num_prefill_work, int32_t q_tile_tokens,
                                      float softmax_scale, int32_t dtype, float k_scale, float v_scale, void* out,
                                      int64_t out_stride_tok, int64_t out_stride_head, void* stream) {
  return paged_prefill(q, q_stride_tok, q_stride_head, k_cache, v_cache, num_blocks, block_size, num_heads,
                       num_kv_heads, head_dim, qo_indptr, kv_indptr, kv_indices, seq_lens, prefill_work,
                       num_prefill_work, q_tile_tokens, softmax_scale, dtype, out, out_stride_tok, out_stride_head,
                       true, k_scale, v_scale, stream);
}
