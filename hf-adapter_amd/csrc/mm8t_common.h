// Blocked-layout MM8 helpers shared by the GEMV (mm8t.hip) and the many-row
// GEMM (mm8g.hip): problem record, raw buffer loads and 8-element decoders.
#pragma once
#include <algorithm>

#include "common.h"

namespace rwkv7mi {

constexpr int MM8T_COLS = 16;
constexpr int MM8T_MAXPROB = 4;
struct Mm8tProb {
  const void* x;
  const void* mix;  // LN-mix prologue only: this problem's token-shift mix [I]
  const uint8_t* w;
  const void* mx;
  const void* rx;
  const void* my;
  const void* ry;
  const void* bias;
  const void* residual;
  void* y;
  int epilogue;
};

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Raw buffer loads: an offset at or beyond the descriptor's byte count returns
// zeros without touching memory, so every load below is unconditional.
constexpr uint32_t MM8T_OOB = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t mm8t_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ u32x4 mm8t_ld16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}

// 8 consecutive elements of type T starting at element e, raw (zeros when
// !valid); loads are issued here and converted later so a batch of them is in
// flight together.
template <typename T>
struct Raw8 {
  u32x4 v[sizeof(T) == 4 ? 2 : 1];
};

template <typename T>
__device__ __forceinline__ Raw8<T> mm8t_ld8(__amdgpu_buffer_rsrc_t r, uint32_t e, bool valid) {
  Raw8<T> o;
  const uint32_t off = valid ? e * (uint32_t)sizeof(T) : MM8T_OOB;
  o.v[0] = mm8t_ld16(r, off);
  if constexpr (sizeof(T) == 4) o.v[1] = mm8t_ld16(r, valid ? off + 16u : MM8T_OOB);
  return o;
}

__device__ __forceinline__ void mm8t_cvt8(const Raw8<float>& a, float (&o)[8]) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    o[q] = __uint_as_float(a.v[0][q]);
    o[4 + q] = __uint_as_float(a.v[1][q]);
  }
}
__device__ __forceinline__ void mm8t_cvt8(const Raw8<__half>& a, float (&o)[8]) {
  const f16x8 v = __builtin_bit_cast(f16x8, a.v[0]);
#pragma unroll
  for (int q = 0; q < 8; ++q) o[q] = (float)v[q];
}
__device__ __forceinline__ void mm8t_cvt8(const Raw8<__hip_bfloat16>& a, float (&o)[8]) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    o[2 * q] = __uint_as_float(a.v[0][q] << 16);
    o[2 * q + 1] = __uint_as_float(a.v[0][q] & 0xffff0000u);
  }
}

// (a & mask) | bits in one v_and_or_b32 (the compiler otherwise emits a
// separate and + or).  A VOP3 encoding on gfx950 takes no literal and reads
// at most one SGPR: the mask comes from an SGPR, the bits from a VGPR (both
// loop-invariant, materialised once).
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t mask, uint32_t bits) {
  uint32_t r;
  __asm__("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(mask), "v"(bits));
  return r;
}

// Compute units of the current device (cached per device).
int64_t mm8t_cus();

}  // namespace rwkv7mi
