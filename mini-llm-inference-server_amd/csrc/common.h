// Shared helpers of the gfx950 paged-attention library: error reporting, vector types, 16-byte
// loads/stores, bf16/fp16 conversions and the MFMA wrappers the kernels use.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "minillm_hip.h"

namespace mllm {

// ---------------------------------------------------------------- errors

void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
// Turns the last launch error (or a HIP status) into MLLM_ERR_HIP with its text.
int check_launch(const char* what);

#define MLLM_REQUIRE(cond, code, msg)        \
  do {                                       \
    if (!(cond)) return ::mllm::fail((code), (msg)); \
  } while (0)

// ---------------------------------------------------------------- types

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Storage tags: 16-bit element types are moved around as raw uint16_t bits.
struct BF16 {};
struct F16 {};

// ---------------------------------------------------------------- conversions

// float -> bf16 bits, round to nearest even; NaN -> 0x7FC0 (what torch's .to(torch.bfloat16) gives).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  uint32_t bias = 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)((u + bias) >> 16);
}

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) { return __uint_as_float(((uint32_t)b) << 16); }

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  _Float16 h = (_Float16)f;  // v_cvt_f16_f32: round to nearest even
  return __builtin_bit_cast(uint16_t, h);
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t b) { return (float)__builtin_bit_cast(_Float16, b); }

// ---------------------------------------------------------------- fp8 KV pool (OCP e4m3fn)
// 1 sign, 4 exponent (bias 7) and 3 mantissa bits; no infinities, S.1111.111 is NaN; the largest finite
// magnitude is 448 and the smallest subnormal 2^-9.

struct FP8 {};  // pool storage tag

// float -> e4m3fn bits, round to nearest even on the e4m3 grid (subnormals included).  A magnitude that
// rounds past 448 (anything above 464), infinity and NaN give NaN with the input's sign: the result of
// torch's .to(torch.float8_e4m3fn).
__device__ __forceinline__ uint32_t f32_to_e4m3fn_bits(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7fffffffu;
  if (a >= 0x43f00000u) return sign | 0x7fu;  // |f| >= 480, infinity, NaN
  if (a < 0x3c800000u)                        // |f| < 2^-6: the subnormal grid, steps of 2^-9
    return sign | (uint32_t)__builtin_rintf(__uint_as_float(a) * 512.f);
  const uint32_t r = a + 0x7ffffu + ((a >> 20) & 1u);  // keep 3 mantissa bits, ties to even
  return sign | ((r - (120u << 23)) >> 20);            // exponent bias 127 -> 7
}

// Four e4m3fn values (bytes 0-3 of w) -> four bf16 / fp16 values, two per dword, in byte order.  Exact:
// every e4m3fn value, subnormals and NaN included, is representable in both 16-bit formats.
template <typename T>
__device__ __forceinline__ u32x2 fp8x4_to(uint32_t w);
template <>
__device__ __forceinline__ u32x2 fp8x4_to<BF16>(uint32_t w) {
  return u32x2{__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.f, false)),
               __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.f, true))};
}
template <>
__device__ __forceinline__ u32x2 fp8x4_to<F16>(uint32_t w) {
  return u32x2{__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.f, false)),
               __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.f, true))};
}
// Eight e4m3fn values (two dwords) -> eight 16-bit values (16 bytes).
template <typename T>
__device__ __forceinline__ u32x4 fp8x8_to(uint32_t w0, uint32_t w1) {
  const u32x2 lo = fp8x4_to<T>(w0), hi = fp8x4_to<T>(w1);
  return u32x4{lo[0], lo[1], hi[0], hi[1]};
}

// Packs two floats into one dword of 16-bit values (lo in bits 0-15), rounding to nearest even with
// the hardware conversion (v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32 on gfx950).  For the attention
// kernels' P tiles and outputs; KV append keeps the bit-level conversion above, whose NaN encoding
// is torch's.
template <typename T>
__device__ __forceinline__ uint32_t pack2(float lo, float hi);
template <>
__device__ __forceinline__ uint32_t pack2<BF16>(float lo, float hi) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}
template <>
__device__ __forceinline__ uint32_t pack2<F16>(float lo, float hi) {
  typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
  const f16x2_t v = {(_Float16)lo, (_Float16)hi};
  return __builtin_bit_cast(uint32_t, v);
}
template <typename T>
__device__ __forceinline__ uint16_t cvt1(float f) {
  return (uint16_t)(pack2<T>(f, 0.f) & 0xffffu);
}

// ---------------------------------------------------------------- memory

__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
// Streaming load (non-temporal hint: the data is read once and should not displace reused lines).
__device__ __forceinline__ u32x4 ld16_nt(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ void st16(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }
__device__ __forceinline__ u32x2 ld8(const void* p) { return *reinterpret_cast<const u32x2*>(p); }
__device__ __forceinline__ void st8(void* p, u32x2 v) { *reinterpret_cast<u32x2*>(p) = v; }

// Selects 16-bit halves of two dwords: returns (half `ia` of a) | (half `ib` of b) << 16.
__device__ __forceinline__ uint32_t pick_halves(uint32_t a, int ia, uint32_t b, int ib) {
  // v_perm_b32 selector bytes index {b: bytes 0-3, a: bytes 4-7} of the (a:b) 64-bit pair.
  uint32_t sel_lo = ia ? 0x0706u : 0x0504u;  // half of a -> result bytes 0-1
  uint32_t sel_hi = ib ? 0x0302u : 0x0100u;  // half of b -> result bytes 2-3
  return __builtin_amdgcn_perm(a, b, sel_lo | (sel_hi << 16));
}

// ---------------------------------------------------------------- global -> LDS DMA and its waits

__device__ __forceinline__ unsigned lds_offset(const void* p) {
  return (unsigned)(uintptr_t)(__attribute__((address_space(3))) const void*)p;
}

// One DMA instruction (global_load_lds_dword{x4}): lane l's 16 (4) bytes at base + voff land at LDS
// byte lds + 16 l (4 l).  base and lds are wave-uniform.  Issued from asm, so the compiler neither
// counts these loads nor waits for them: every wait on them is an explicit vmcnt (barrier_vm).  The
// LDS address goes in as an "{m0}" operand: the compiler itself loads m0 right before the instruction
// and knows the register is read there, so no value it keeps in m0 is lost.
__device__ __forceinline__ void dma16(const char* base, unsigned voff, unsigned lds) {
  asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "{m0}"(lds));
}
__device__ __forceinline__ void dma4(const char* base, unsigned voff, unsigned lds) {
  asm volatile("global_load_lds_dword %0, %1" ::"v"(voff), "s"(base), "{m0}"(lds));
}

// Workgroup barrier that first waits for this wavefront's LDS reads and for all but its N most recent
// DMA loads (vmcnt retires loads in issue order).  One asm statement: the compiler moves no LDS access
// across it and does not add the vmcnt(0) drain that __syncthreads' fence would (outstanding DMA
// loads count as LDS writes to that fence).
template <int N>
__device__ __forceinline__ void barrier_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}
__device__ __forceinline__ void barrier_lds() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// ---------------------------------------------------------------- MFMA wrappers (gfx950)

template <typename T>
struct Mfma;

template <>
struct Mfma<BF16> {
  // D(16x16) += A(16x32) B(32x16); lane l holds A[l%16][k-group l/16], B[k-group l/16][l%16].
  static __device__ __forceinline__ f32x4 m16x16x32(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  }
  // D(16x16) += A(16x16) B(16x16), 4 k-values per lane.
  static __device__ __forceinline__ f32x4 m16x16x16(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4, a), __builtin_bit_cast(i16x4, b), c,
                                                     0, 0, 0);
  }
  // D(32x32) += A(32x16) B(16x32), 8 k-values per lane.
  static __device__ __forceinline__ f32x16 m32x32x16(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  }
};

template <>
struct Mfma<F16> {
  static __device__ __forceinline__ f32x4 m16x16x32(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
  }
  static __device__ __forceinline__ f32x4 m16x16x16(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a), __builtin_bit_cast(f16x4, b), c, 0, 0,
                                                 0);
  }
  static __device__ __forceinline__ f32x16 m32x32x16(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
  }
};

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Reductions of lane l with lane l ^ 32 (v_permlane32_swap: the two halves of the wavefront exchange
// values in the VALU, no LDS round trip) or with lane l ^ 16 (v_permlane16_swap: 16-lane rows 0 <-> 1
// and 2 <-> 3).  Each swap returns the lane's own value and its partner's, in an order that depends on
// the lane; max and + are commutative, so both lanes of a pair get the same bits.
__device__ __forceinline__ float max_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __builtin_fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// NaN-propagating maxima (IEEE 754-2019 maximum: v_maximum3_f32, which needs no canonicalising moves on
// values the compiler cannot prove quiet, unlike fmaxf's v_max_f32)
__device__ __forceinline__ float maximum(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ float maximum_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return maximum(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float maximum_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return maximum(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

constexpr float kLog2e = 1.4426950408889634f;

}  // namespace mllm
