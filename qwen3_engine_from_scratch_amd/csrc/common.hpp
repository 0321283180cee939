// Shared helpers of the gfx950 attention kernels: error reporting, bf16
// register types and the MFMA / cross-lane primitives the kernels are built on.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qwen3_attn.h"
#include "qwen3_model_ops.h"

namespace q3 {

// ---- error reporting (thread-local message, C-ABI return codes) ----------
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();
// Converts the launch status of the kernel just enqueued into a return code.
int launch_status(const char* what);

// ---- register types ------------------------------------------------------
typedef __bf16 bf16x8 __attribute__((__vector_size__(8 * sizeof(__bf16))));
typedef __bf16 bf16x4 __attribute__((__vector_size__(4 * sizeof(__bf16))));
typedef float f32x4 __attribute__((__vector_size__(4 * sizeof(float))));
typedef float f32x16 __attribute__((__vector_size__(16 * sizeof(float))));
typedef uint32_t u32x4 __attribute__((__vector_size__(4 * sizeof(uint32_t))));
typedef uint32_t u32x2 __attribute__((__vector_size__(2 * sizeof(uint32_t))));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_inff();

// 16-byte global load / store (dwordx4).  `p` must be 16-byte aligned.
__device__ __forceinline__ u32x4 ld16(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}
// Non-temporal 16-byte load: streamed data that is read once.
__device__ __forceinline__ u32x4 ld16_nt(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ void st16(void* p, u32x4 v) {
  *reinterpret_cast<u32x4*>(p) = v;
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) {
  return __builtin_bit_cast(bf16x8, v);
}
__device__ __forceinline__ bf16x4 as_bf16x4(u32x2 v) {
  return __builtin_bit_cast(bf16x4, v);
}

// Round-to-nearest-even fp32 -> bf16 of two values packed into one dword
// (element 0 in the low half).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef __bf16 bf16x2 __attribute__((__vector_size__(2 * sizeof(__bf16))));
  bf16x2 v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ uint16_t bf16_bits(float x) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(x));
}

__device__ __forceinline__ float bf16_lo(uint32_t w) {
  return __builtin_bit_cast(float, w << 16);
}
__device__ __forceinline__ float bf16_hi(uint32_t w) {
  return __builtin_bit_cast(float, w & 0xffff0000u);
}

__device__ __forceinline__ float fast_exp2(float x) {
  return __builtin_amdgcn_exp2f(x);
}

// Byte permute: result byte k = byte sel[k] of the 8-byte value {hi:lo}.
__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}
// Packs the low (h == 0) or high (h == 1) bf16 halves of two dwords into one
// dword: element 0 from `a`, element 1 from `b`.
__device__ __forceinline__ uint32_t pick_halves(uint32_t a, uint32_t b, int h) {
  return perm(b, a, h ? 0x07060302u : 0x05040100u);
}

// D = A(16x32) * B(32x16) + C, bf16 in, fp32 accumulate.
// A: lane l holds row l%16, one 8-element k-group per l/16.
// B: lane l holds col l%16, the same k-group per l/16.
// C/D: lane l holds col l%16, rows 4*(l/16) + [0..3].
__device__ __forceinline__ f32x4 mfma16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
// D = A(16x16) * B(16x16) + C with 4-element k-groups per l/16.
__device__ __forceinline__ f32x4 mfma16x16x16(bf16x4 a, bf16x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}
// D = A(32x16) * B(16x32) + C.  A: lane l holds row l%32, k-group l/32 (8
// elements); B: col l%32, k-group l/32; D: lane l holds col l%32, rows
// 8*(r/4) + 4*(l/32) + r%4 for register r.
__device__ __forceinline__ f32x16 mfma32x32x16(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float shfl_xor(float v, int mask) {
  return __shfl_xor(v, mask, 64);
}

__host__ __device__ __forceinline__ int64_t cdiv(int64_t a, int64_t b) {
  return (a + b - 1) / b;
}

inline bool aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

// Lane moves inside a 16-lane DPP row: one full-rate VALU instruction
// each, where __shfl_xor compiles to an LDS permute (ds_bpermute) and its
// round trip.  Controls: quad_perm [1,0,3,2] (lane ^ 1), [2,3,0,1]
// (lane ^ 2), row_half_mirror (lane i <-> 7 - i within eight), row_mirror
// (lane i <-> 15 - i), row_ror:8 (lane ^ 8 within sixteen).
enum : int {
  kDppXor1 = 0xB1,
  kDppXor2 = 0x4E,
  kDppHalfMirror = 0x141,
  kDppMirror = 0x140,
  kDppRor8 = 0x128,
};
template <int kCtrl>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_mov_dpp(static_cast<int>(v), kCtrl, 0xF, 0xF, false));
}
template <int kCtrl>
__device__ __forceinline__ float dpp_f32(float v) {
  return __uint_as_float(dpp_u32<kCtrl>(__float_as_uint(v)));
}
// Sum over the 16 lanes of a row.  After the two quad steps every lane of
// a quad holds the quad's sum, so the mirrors pair the same values as a xor
// butterfly over 4 and 8: the result has the butterfly's bits.
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_f32<kDppXor1>(v);
  v += dpp_f32<kDppXor2>(v);
  v += dpp_f32<kDppHalfMirror>(v);
  v += dpp_f32<kDppMirror>(v);
  return v;
}

// x and the value lane l ^ 16 (l ^ 32) holds, on every lane: v_permlane16_swap
// (v_permlane32_swap) of x with itself leaves the value of the pair's lower
// row (half) in r[0] and of its upper one in r[1].  No LDS permute.
__device__ __forceinline__ float max_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

}  // namespace q3
