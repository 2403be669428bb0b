// Shared device/host helpers for the rwkv7mi gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <hip/hip_bf16.h>
#include <stdint.h>
#include <atomic>
#include <string>

#include "../../include/rwkv7mi.h"

namespace rwkv7mi {

// ------------------------------------------------------------------ errors
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
// Checks the last launch / call; returns RWKV7MI_OK or RWKV7MI_ELAUNCH.
int check_launch(const char* what);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Raises a kernel's dynamic LDS limit on the current device once.  `done` is the
// caller's per-kernel bitmask of devices already raised (bit = device index);
// racing threads may both set the attribute, which is harmless.  Returns
// RWKV7MI_OK or RWKV7MI_ELAUNCH.
int raise_dynamic_lds(const void* kernel, int bytes, std::atomic<uint64_t>& done, const char* who);

inline bool valid_dtype(int d) { return d == RWKV7MI_F32 || d == RWKV7MI_F16 || d == RWKV7MI_BF16; }

// ------------------------------------------------------- scalar conversions
__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(__half x) { return __half2float(x); }
__device__ __forceinline__ float to_f32(__hip_bfloat16 x) { return __bfloat162float(x); }

template <typename T> __device__ __forceinline__ T from_f32(float x);
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <> __device__ __forceinline__ __half from_f32<__half>(float x) { return __float2half_rn(x); }
template <> __device__ __forceinline__ __hip_bfloat16 from_f32<__hip_bfloat16>(float x) {
  return __float2bfloat16(x);
}

// ------------------------------------------------------- lane exchange
// x from lane (i + N) mod 16 of this lane's 16-lane row (DPP row_ror:N)
template <int N>
__device__ __forceinline__ float dpp_row_ror(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x120 + N, 0xF, 0xF, false));
}

template <typename T>
__device__ __forceinline__ float ld(const T* p, int64_t i) { return to_f32(p[i]); }

// -------------------------------------------------------- wave reductions
// (the wave must be fully active: DPP and readlane read every lane)
template <int CTRL>
__device__ __forceinline__ float dpp_quad(float x) {  // quad_perm: lane i of each quad gets lane sel_i
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float lane_f(float x, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), l));
}
// The wave's total, the same in every lane: DPP rotations inside the 16-lane
// rows, then the four row totals read out in a fixed order (no LDS round trips).
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_row_ror<8>(v);
  v += dpp_row_ror<4>(v);
  v += dpp_row_ror<2>(v);
  v += dpp_row_ror<1>(v);
  return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
}

// Sum over aligned groups of G consecutive lanes (G power of two <= 64); every
// lane of a group gets the same bits (pairwise butterfly).
template <int G>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (G >= 2) v += dpp_quad<0xB1>(v);  // lane i ^ 1
  if constexpr (G >= 4) v += dpp_quad<0x4E>(v);  // lane i ^ 2
#pragma unroll
  for (int o = G / 2; o >= 4; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Dispatch a runtime dtype code to a C++ type.  F is a generic lambda taking
// a value of the selected type (only the type is used).
template <typename F>
inline int dispatch_dtype(int code, F&& f) {
  switch (code) {
    case RWKV7MI_F32: return f(float{});
    case RWKV7MI_F16: return f(__half{});
    case RWKV7MI_BF16: return f(__hip_bfloat16{});
    default: return fail(RWKV7MI_EINVAL, "unsupported dtype code " + std::to_string(code));
  }
}

// ------------------------------------------------- 8-element vector I/O
// p must be 16-byte aligned (32-byte for float); values convert to/from fp32.
__device__ __forceinline__ void ld8(const float* p, float (&o)[8]) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  const float4 b = *reinterpret_cast<const float4*>(p + 4);
  o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
  o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
}
// two packed fp16 -> fp32.  (Decoded from a plain uint32_t: hipcc has been seen
// to read element 0 for __builtin_bit_cast applied to a vector subscript.)
__device__ __forceinline__ void f16x2_to_f32(uint32_t w, float& lo, float& hi) {
  lo = __half2float(__ushort_as_half((unsigned short)(w & 0xffffu)));
  hi = __half2float(__ushort_as_half((unsigned short)(w >> 16)));
}

__device__ __forceinline__ void ld8(const __half* p, float (&o)[8]) {
  const uint4 u = *reinterpret_cast<const uint4*>(p);
  const uint32_t d[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) f16x2_to_f32(d[q], o[2 * q], o[2 * q + 1]);
}
__device__ __forceinline__ void ld8(const __hip_bfloat16* p, float (&o)[8]) {
  const uint4 u = *reinterpret_cast<const uint4*>(p);
  const uint32_t d[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    o[2 * q] = __uint_as_float(d[q] << 16);
    o[2 * q + 1] = __uint_as_float(d[q] & 0xffff0000u);
  }
}
__device__ __forceinline__ void st8(float* p, const float (&v)[8]) {
  *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
  *reinterpret_cast<float4*>(p + 4) = make_float4(v[4], v[5], v[6], v[7]);
}
template <typename T>
__device__ __forceinline__ void st8(T* p, const float (&v)[8]) {
  uint32_t d[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const T lo = from_f32<T>(v[2 * q]), hi = from_f32<T>(v[2 * q + 1]);
    d[q] = (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
  }
  *reinterpret_cast<uint4*>(p) = make_uint4(d[0], d[1], d[2], d[3]);
}
// ------------------------------------------------------ raw buffer loads
// An offset at or beyond the descriptor's byte count returns zeros without a
// memory access, so bounds checks become offset selects and loads stay
// unconditional: a straight run of loads is issued back to back and waited on
// once, instead of one branch and one full wait per load.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr uint32_t BUF_OOB = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ u32x4 buf_ld16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}

__device__ __forceinline__ float buf_ldf(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0));
}

// one T element at index e (zero when !valid or past the descriptor) -> fp32
template <typename T>
__device__ __forceinline__ float buf_ld1(__amdgpu_buffer_rsrc_t r, uint32_t e, bool valid) {
  const int off = (int)(valid ? e * (uint32_t)sizeof(T) : BUF_OOB);
  if constexpr (sizeof(T) == 4) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
  } else {
    const unsigned short u = __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
    return to_f32(__builtin_bit_cast(T, u));
  }
}

// 8 consecutive T elements from element index e (zeros when !valid) -> fp32
__device__ __forceinline__ void buf_ld8(__amdgpu_buffer_rsrc_t r, uint32_t e, bool valid, const float*,
                                        float (&o)[8]) {
  const u32x4 a = buf_ld16(r, valid ? e * 4u : BUF_OOB);
  const u32x4 b = buf_ld16(r, valid ? e * 4u + 16u : BUF_OOB);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    o[q] = __uint_as_float(a[q]);
    o[4 + q] = __uint_as_float(b[q]);
  }
}
__device__ __forceinline__ void buf_ld8(__amdgpu_buffer_rsrc_t r, uint32_t e, bool valid, const __half*,
                                        float (&o)[8]) {
  const u32x4 a = buf_ld16(r, valid ? e * 2u : BUF_OOB);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint32_t w = a[q];
    f16x2_to_f32(w, o[2 * q], o[2 * q + 1]);
  }
}
__device__ __forceinline__ void buf_ld8(__amdgpu_buffer_rsrc_t r, uint32_t e, bool valid, const __hip_bfloat16*,
                                        float (&o)[8]) {
  const u32x4 a = buf_ld16(r, valid ? e * 2u : BUF_OOB);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    o[2 * q] = __uint_as_float(a[q] << 16);
    o[2 * q + 1] = __uint_as_float(a[q] & 0xffff0000u);
  }
}

// round each value to T and back (the value a T tensor would hold)
template <typename T>
__device__ __forceinline__ void round8(float (&v)[8]) {
#pragma unroll
  for (int q = 0; q < 8; ++q) v[q] = to_f32(from_f32<T>(v[q]));
}

}  // namespace rwkv7mi

namespace rwkv7mi {
// ------------------------------------------------------ LoRA partial layout
// The LoRA down projections split K = D into `ks` ranges; partial sums are
// stored fp32 [problem][ks][rows][rank] (problems packed back to back).  The
// up projection (lora.hip) and the fused decode (wkv7_decode.hip) both read
// this layout.
constexpr int LORA_ROWS = 64;  // rows per launch pair
inline int64_t lora_tiles(int64_t nprob, const int64_t* ranks) {
  int64_t t = 0;
  for (int64_t i = 0; i < nprob; ++i) t += (ranks[i] + 15) / 16;
  return t;
}
inline int lora_splits(int64_t tiles, int64_t D) {
  // aim for 256-512 down workgroups, each split covering at least 128 inputs
  int64_t ks = 1;
  while (tiles * ks * 2 <= 512 && D / (ks * 2) >= 128) ks *= 2;
  return (int)ks;
}
}  // namespace rwkv7mi

namespace rwkv7mi {
// ------------------------------------------------------------ MFMA types
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// v_mfma_f32_16x16x32_f16 lane layout (gfx950):
//   A (16 x 32): lane l holds row (l % 16), k = 8*(l/16) .. +7
//   B (32 x 16): lane l holds col (l % 16), k = 8*(l/16) .. +7
//   C (16 x 16): lane l holds col (l % 16), rows 4*(l/16) .. +3
__device__ __forceinline__ f32x4 mfma16x16x32(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
}  // namespace rwkv7mi
