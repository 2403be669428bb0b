// Shared device/host helpers for the rwkv7mi gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <hip/hip_bf16.h>
#include <stdint.h>
#include <string>

#include "../../include/rwkv7mi.h"

namespace rwkv7mi {

// ------------------------------------------------------------------ errors
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
// Checks the last launch / call; returns RWKV7MI_OK or RWKV7MI_ELAUNCH.
int check_launch(const char* what);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

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

template <typename T>
__device__ __forceinline__ float ld(const T* p, int64_t i) { return to_f32(p[i]); }

// -------------------------------------------------------- wave reductions
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Sum over aligned groups of G consecutive lanes (G power of two <= 64).
template <int G>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int o = G / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
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
