// Greedy token selection: the argmax of each logits row, as the reference's
// greedy decode loop takes it with torch (`logits[:, -1:].argmax(dim=-1)`,
// bench/bench_native_quant_e2e_decode.py:424-437), so the captured decode
// graph can end with the next tokens and feed them to its own next replay.
//
// One 1024-lane workgroup per row.  A lane scans 8-element runs (16-byte raw
// buffer loads, eight in flight), keeping the best (value, index); the lanes
// then reduce in a fixed order (xor shuffles inside the wave, LDS across the
// 16 waves).  Ties go to the smaller index and NaN beats every number
// (the first NaN wins), which is torch's argmax on CUDA/ROCm.
#include "common.h"

namespace rwkv7mi {

constexpr int AM_THREADS = 1024;
constexpr int AM_RUNS = 8;  // 8-element runs per lane in flight

// (va, ia) better than (vb, ib)
__device__ __forceinline__ bool am_better(float va, int64_t ia, float vb, int64_t ib) {
  const bool na = va != va, nb = vb != vb;
  if (na || nb) return na && (!nb || ia < ib);
  return va > vb || (va == vb && ia < ib);
}

__device__ __forceinline__ bool am_better(float va, int ia, float vb, int ib) {
  const bool na = va != va, nb = vb != vb;
  if (na || nb) return na && (!nb || ia < ib);
  return va > vb || (va == vb && ia < ib);
}

template <typename T>
__device__ __forceinline__ void am_run(uint32_t (&w)[4], int64_t base, int64_t n, float& bv, int64_t& bi) {
  if constexpr (sizeof(T) == 2) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int64_t i = base + 2 * q + h;
        const uint32_t bits = h ? (w[q] >> 16) : (w[q] & 0xffffu);
        float v;
        if constexpr (std::is_same<T, __half>::value)
          v = __half2float(__ushort_as_half((unsigned short)bits));
        else
          v = __uint_as_float(bits << 16);
        if (i < n && am_better(v, i, bv, bi)) {
          bv = v;
          bi = i;
        }
      }
    }
  }
}

template <typename T>
__global__ __launch_bounds__(AM_THREADS) void argmax_rows_kernel(const T* __restrict__ x, int64_t n, int64_t ld,
                                                                 int64_t* out, int64_t* out2) {
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  const T* xr = x + row * ld;
  float bv = -__builtin_inff();
  int64_t bi = INT64_MAX;
  if constexpr (sizeof(T) == 4) {
    const __amdgpu_buffer_rsrc_t r = make_rsrc(xr, (uint32_t)(n * 4));
    for (int64_t i0 = 4 * (int64_t)tid; i0 < n; i0 += 4LL * AM_THREADS * AM_RUNS) {
      uint32_t w[AM_RUNS][4];
#pragma unroll
      for (int u = 0; u < AM_RUNS; ++u) {
        const int64_t i = i0 + 4LL * AM_THREADS * u;
        const u32x4 v = buf_ld16(r, i < n ? (uint32_t)(i * 4) : BUF_OOB);
        w[u][0] = v[0], w[u][1] = v[1], w[u][2] = v[2], w[u][3] = v[3];
      }
#pragma unroll
      for (int u = 0; u < AM_RUNS; ++u)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int64_t i = i0 + 4LL * AM_THREADS * u + q;
          const float v = __uint_as_float(w[u][q]);
          if (i < n && am_better(v, i, bv, bi)) {
            bv = v;
            bi = i;
          }
        }
    }
  } else {
    const __amdgpu_buffer_rsrc_t r = make_rsrc(xr, (uint32_t)(n * 2));
    for (int64_t i0 = 8 * (int64_t)tid; i0 < n; i0 += 8LL * AM_THREADS * AM_RUNS) {
      uint32_t w[AM_RUNS][4];
#pragma unroll
      for (int u = 0; u < AM_RUNS; ++u) {
        const int64_t i = i0 + 8LL * AM_THREADS * u;
        const u32x4 v = buf_ld16(r, i < n ? (uint32_t)(i * 2) : BUF_OOB);
        w[u][0] = v[0], w[u][1] = v[1], w[u][2] = v[2], w[u][3] = v[3];
      }
#pragma unroll
      for (int u = 0; u < AM_RUNS; ++u) am_run<T>(w[u], i0 + 8LL * AM_THREADS * u, n, bv, bi);
    }
  }
  // wave reduction (xor butterfly: every lane ends with the wave's best)
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o, 64);
    const int64_t oi = __shfl_xor(bi, o, 64);
    if (am_better(ov, oi, bv, bi)) {
      bv = ov;
      bi = oi;
    }
  }
  __shared__ float sv[AM_THREADS / 64];
  __shared__ int64_t si[AM_THREADS / 64];
  if ((tid & 63) == 0) {
    sv[tid >> 6] = bv;
    si[tid >> 6] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    float v = sv[0];
    int64_t i = si[0];
    for (int q = 1; q < AM_THREADS / 64; ++q)
      if (am_better(sv[q], si[q], v, i)) {
        v = sv[q];
        i = si[q];
      }
    if (i == INT64_MAX) i = 0;  // n == 0 is refused by the host; keeps the output defined
    out[row] = i;
    if (out2) out2[row] = i;
  }
}

// Two-pass form for long rows: argmax_part_kernel gives each 256-lane
// workgroup AP_CHUNK elements of one row (every lane two 16-byte runs) and
// writes the slice's best (value, index) to the workspace; argmax_final_kernel
// (one wave per row) picks the best of the slices with the same rule.  Many
// workgroups share a row, so a 65536-entry row takes two short launches
// instead of one workgroup's long serial scan.
constexpr int AP_THREADS = 256;
constexpr int AP_LOADS = 2;  // 16-byte runs per lane
template <typename T>
constexpr int ap_chunk() { return AP_THREADS * AP_LOADS * (16 / (int)sizeof(T)); }

__device__ __forceinline__ void am_wave_best(float& bv, int& bi) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o, 64);
    const int oi = __shfl_xor(bi, o, 64);
    if (am_better(ov, oi, bv, bi)) {
      bv = ov;
      bi = oi;
    }
  }
}

template <typename T>
__global__ __launch_bounds__(AP_THREADS) void argmax_part_kernel(const T* __restrict__ x, int n, int64_t ld,
                                                                 float* __restrict__ pv, int* __restrict__ pi) {
  constexpr int E = 16 / (int)sizeof(T);  // elements per run
  const int64_t row = blockIdx.y;
  const int nb = (int)gridDim.x;
  const int tid = threadIdx.x;
  const int c0 = (int)blockIdx.x * ap_chunk<T>();
  const __amdgpu_buffer_rsrc_t r = make_rsrc(x + row * ld, (uint32_t)n * (uint32_t)sizeof(T));
  u32x4 w[AP_LOADS];
#pragma unroll
  for (int u = 0; u < AP_LOADS; ++u) {
    const int i = c0 + (u * AP_THREADS + tid) * E;
    w[u] = buf_ld16(r, i < n ? (uint32_t)i * (uint32_t)sizeof(T) : BUF_OOB);
  }
  float bv = -__builtin_inff();
  int bi = INT32_MAX;
#pragma unroll
  for (int u = 0; u < AP_LOADS; ++u) {
    const int i0 = c0 + (u * AP_THREADS + tid) * E;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int i = i0 + e;
      float v;
      if constexpr (sizeof(T) == 4) {
        v = __uint_as_float(w[u][e]);
      } else {
        const uint32_t bits = (e & 1) ? (w[u][e >> 1] >> 16) : (w[u][e >> 1] & 0xffffu);
        if constexpr (std::is_same<T, __half>::value)
          v = __half2float(__ushort_as_half((unsigned short)bits));
        else
          v = __uint_as_float(bits << 16);
      }
      if (i < n && am_better(v, i, bv, bi)) {
        bv = v;
        bi = i;
      }
    }
  }
  am_wave_best(bv, bi);
  __shared__ float sv[AP_THREADS / 64];
  __shared__ int si[AP_THREADS / 64];
  if ((tid & 63) == 0) {
    sv[tid >> 6] = bv;
    si[tid >> 6] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    float v = sv[0];
    int i = si[0];
#pragma unroll
    for (int q = 1; q < AP_THREADS / 64; ++q)
      if (am_better(sv[q], si[q], v, i)) {
        v = sv[q];
        i = si[q];
      }
    pv[row * nb + blockIdx.x] = v;
    pi[row * nb + blockIdx.x] = i;
  }
}

__global__ __launch_bounds__(64) void argmax_final_kernel(const float* __restrict__ pv, const int* __restrict__ pi,
                                                          int nb, int64_t* out, int64_t* out2) {
  const int64_t row = blockIdx.x;
  float bv = -__builtin_inff();
  int bi = INT32_MAX;
  for (int j = threadIdx.x; j < nb; j += 64) {
    const float v = pv[row * nb + j];
    const int i = pi[row * nb + j];
    if (am_better(v, i, bv, bi)) {
      bv = v;
      bi = i;
    }
  }
  am_wave_best(bv, bi);
  if (threadIdx.x == 0) {
    const int64_t i = bi == INT32_MAX ? 0 : bi;
    out[row] = i;
    if (out2) out2[row] = i;
  }
}

}  // namespace rwkv7mi

using namespace rwkv7mi;

extern "C" int rwkv7mi_argmax_rows(const void* x, int64_t rows, int64_t n, int64_t ld, int dtype, int64_t* out,
                                   int64_t* out2, void* stream) {
  if (rows < 0 || n <= 0 || ld < n) return fail(RWKV7MI_EINVAL, "argmax_rows: bad shape");
  if (rows == 0) return RWKV7MI_OK;
  if (!x || !out) return fail(RWKV7MI_EINVAL, "argmax_rows: null pointer");
  if (!valid_dtype(dtype)) return fail(RWKV7MI_EINVAL, "argmax_rows: bad dtype");
  const int64_t es = dtype == RWKV7MI_F32 ? 4 : 2;
  if (n * es > INT32_MAX || rows > INT32_MAX) return fail(RWKV7MI_EINVAL, "argmax_rows: too large");
  if ((reinterpret_cast<uintptr_t>(x) & 15) || (ld * es) % 16)
    return fail(RWKV7MI_EINVAL, "argmax_rows: rows must start 16-byte aligned");
  return dispatch_dtype(dtype, [&](auto t) {
    using T = decltype(t);
    hipLaunchKernelGGL((argmax_rows_kernel<T>), dim3((unsigned)rows), dim3(AM_THREADS), 0, as_stream(stream),
                       (const T*)x, n, ld, out, out2);
    return check_launch("argmax_rows_kernel");
  });
}

// slices per row and workspace bytes of the two-pass form
static int64_t argmax_slices(int64_t n, int dtype) {
  const int64_t ch = dtype == RWKV7MI_F32 ? ap_chunk<float>() : ap_chunk<__half>();
  return (n + ch - 1) / ch;
}

extern "C" size_t rwkv7mi_argmax_workspace_bytes(int64_t rows, int64_t n, int dtype) {
  if (rows <= 0 || n <= 0 || !valid_dtype(dtype)) return 0;
  return (size_t)(rows * argmax_slices(n, dtype)) * 8u;
}

extern "C" int rwkv7mi_argmax_rows_ws(const void* x, int64_t rows, int64_t n, int64_t ld, int dtype, int64_t* out,
                                      int64_t* out2, void* workspace, size_t workspace_bytes, void* stream) {
  if (rows < 0 || n <= 0 || ld < n) return fail(RWKV7MI_EINVAL, "argmax_rows_ws: bad shape");
  if (rows == 0) return RWKV7MI_OK;
  if (!x || !out) return fail(RWKV7MI_EINVAL, "argmax_rows_ws: null pointer");
  if (!valid_dtype(dtype)) return fail(RWKV7MI_EINVAL, "argmax_rows_ws: bad dtype");
  const int64_t es = dtype == RWKV7MI_F32 ? 4 : 2;
  if (n * es > INT32_MAX || rows > 65535) return fail(RWKV7MI_EINVAL, "argmax_rows_ws: too large");
  if ((reinterpret_cast<uintptr_t>(x) & 15) || (ld * es) % 16)
    return fail(RWKV7MI_EINVAL, "argmax_rows_ws: rows must start 16-byte aligned");
  const int64_t nb = argmax_slices(n, dtype);
  if (!workspace || workspace_bytes < (size_t)(rows * nb) * 8u || (reinterpret_cast<uintptr_t>(workspace) & 7))
    return fail(RWKV7MI_ESIZE, "argmax_rows_ws: workspace missing, unaligned or smaller than "
                               "rwkv7mi_argmax_workspace_bytes");
  float* pv = reinterpret_cast<float*>(workspace);
  int* pi = reinterpret_cast<int*>(pv + rows * nb);
  return dispatch_dtype(dtype, [&](auto t) {
    using T = decltype(t);
    hipLaunchKernelGGL((argmax_part_kernel<T>), dim3((unsigned)nb, (unsigned)rows), dim3(AP_THREADS), 0,
                       as_stream(stream), (const T*)x, (int)n, ld, pv, pi);
    if (int rc = check_launch("argmax_part_kernel")) return rc;
    hipLaunchKernelGGL(argmax_final_kernel, dim3((unsigned)rows), dim3(64), 0, as_stream(stream), (const float*)pv,
                       (const int*)pi, (int)nb, out, out2);
    return check_launch("argmax_final_kernel");
  });
}
