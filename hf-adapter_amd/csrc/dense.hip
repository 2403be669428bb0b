// Grouped dense GEMV / small GEMM with fused bias + activation (gfx950), used
// for the RWKV-7 W/A/G/V LoRA projections (rwkv7_hf/fused_lora.py:706-886,
// torch form :795-803) and other small fp16 linears on the decode path.
//
//   y[r, n] = act( sum_k x[r, k] * W[n, k] + bias[n] )    (W in nn.Linear layout [N, K])
//
// Up to four independent problems share one launch (e.g. the four LoRA down
// projections).  v_mfma_f32_16x16x32_f16: rows are M (16 per tile), 16 output
// features are N, K runs along the contiguous dimension of both x and W, so
// every lane loads 16 contiguous bytes of each operand.  A workgroup owns one
// 16-feature tile; its 4 waves take interleaved 32-wide k-steps and are
// reduced through LDS.  fp16 operands are used as-is; fp32 / bf16 operands are
// split into fp16 hi + lo (three MFMAs) so accuracy stays fp32-class.
// One to four rows take a GEMV form instead (dense_gemv_kernel below).
#include "common.h"

namespace rwkv7mi {

enum { ACT_NONE = 0, ACT_TANH = 1, ACT_SIGMOID = 2, ACT_RELU2 = 3 };

struct DenseProb {
  const void* x;
  const void* W;
  const void* bias;
  void* y;
  int N, K, act, tile0;
};
struct DenseBatch {
  DenseProb p[4];
  int nprob;
};

template <typename T>
__device__ __forceinline__ void load8_split(const T* src, bool ok, f16x8& hi, f16x8& lo) {
  if constexpr (std::is_same<T, __half>::value) {
    if (ok) {
      const uint4 raw = *reinterpret_cast<const uint4*>(src);
      hi = __builtin_bit_cast(f16x8, raw);
    } else {
      hi = (f16x8){0, 0, 0, 0, 0, 0, 0, 0};
    }
    lo = (f16x8){0, 0, 0, 0, 0, 0, 0, 0};
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float f = ok ? to_f32(src[e]) : 0.f;
      const _Float16 h = (_Float16)f;
      hi[e] = h;
      lo[e] = (_Float16)(f - (float)h);
    }
  }
}

__device__ __forceinline__ float apply_act(float v, int act) {
  if (act == ACT_TANH) return tanhf(v);
  if (act == ACT_SIGMOID) return 1.0f / (1.0f + expf(-v));
  if (act == ACT_RELU2) {
    v = fmaxf(v, 0.f);
    return v * v;
  }
  return v;
}

template <int MT, typename TA>
__global__ __launch_bounds__(256) void dense_kernel(DenseBatch batch, int rows) {
  constexpr bool SPLIT = !std::is_same<TA, __half>::value;
  __shared__ float s_red[16 * MT][16];
  int pi = 0;
#pragma unroll
  for (int q = 1; q < 4; ++q)
    if (q < batch.nprob && (int)blockIdx.x >= batch.p[q].tile0) pi = q;
  const DenseProb P = batch.p[pi];
  const TA* x = reinterpret_cast<const TA*>(P.x);
  const TA* W = reinterpret_cast<const TA*>(P.W);
  const int n0 = ((int)blockIdx.x - P.tile0) * 16;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int l16 = lane & 15, kg = lane >> 4;
  const int n = n0 + l16;
  const int K = P.K;

  f32x4 acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = (f32x4){0.f, 0.f, 0.f, 0.f};
  for (int ks = wave * 32; ks < K; ks += 128) {
    const int kk = ks + 8 * kg;
    const bool kok = kk < K;  // K % 8 == 0
    f16x8 bh, bl;
    load8_split(W + (int64_t)n * K + kk, kok && n < P.N, bh, bl);
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int r = 16 * t + l16;
      f16x8 ah, al;
      load8_split(x + (int64_t)r * K + kk, kok && r < rows, ah, al);
      acc[t] = mfma16x16x32(ah, bh, acc[t]);
      if constexpr (SPLIT) {
        acc[t] = mfma16x16x32(ah, bl, acc[t]);
        acc[t] = mfma16x16x32(al, bh, acc[t]);
      }
    }
  }
  for (int wv = 0; wv < 4; ++wv) {
    if (wave == wv) {
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float* dst = &s_red[16 * t + 4 * kg + e][l16];
          *dst = (wv == 0) ? acc[t][e] : *dst + acc[t][e];
        }
    }
    __syncthreads();
  }
  TA* y = reinterpret_cast<TA*>(P.y);
  const TA* bias = reinterpret_cast<const TA*>(P.bias);
  for (int idx = tid; idx < rows * 16; idx += 256) {
    const int r = idx >> 4, nn = idx & 15;
    const int o = n0 + nn;
    if (o >= P.N) continue;
    float v = s_red[r][nn];
    if (bias) v += to_f32(bias[o]);
    y[(int64_t)r * P.N + o] = from_f32<TA>(apply_act(v, P.act));
  }
}

// ---------------------------------------------------------------- 1..4 rows
// GEMV form: one wave per output feature n, a workgroup owns four features
// of one problem (a problem's features start at a multiple of four tiles).
// Lanes split K in 16-byte runs of W's row n and of the x rows at the same k;
// a pass is GV_U runs per lane, and the next pass's runs load while this one
// multiplies.  Plain fp32 FMAs, then a fixed-order wave reduction per row:
// every output is an fp32 dot product whatever the dtype.
constexpr int GV_U = 4;  // 16-byte runs per lane per pass

// 16 raw bytes -> the run's VE elements as fp32
template <typename TA>
__device__ __forceinline__ void gv_cvt(const u32x4& a, float (&o)[16 / sizeof(TA)]) {
  if constexpr (sizeof(TA) == 4) {
#pragma unroll
    for (int q = 0; q < 4; ++q) o[q] = __uint_as_float(a[q]);
  } else if constexpr (std::is_same<TA, __half>::value) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t w = a[q];
      f16x2_to_f32(w, o[2 * q], o[2 * q + 1]);
    }
  } else {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      o[2 * q] = __uint_as_float(a[q] << 16);
      o[2 * q + 1] = __uint_as_float(a[q] & 0xffff0000u);
    }
  }
}

template <typename TA, int R>
__global__ __launch_bounds__(256) void dense_gemv_kernel(DenseBatch batch, int rows) {
  constexpr int VE = 16 / (int)sizeof(TA);  // elements per run
  int pi = 0;
#pragma unroll
  for (int q = 1; q < 4; ++q)
    if (q < batch.nprob && (int)blockIdx.x >= batch.p[q].tile0) pi = q;
  const DenseProb P = batch.p[pi];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int n = ((int)blockIdx.x - P.tile0) * 4 + wave;
  if (n >= P.N) return;  // wave-uniform; no barrier follows
  const int K = P.K;
  const __amdgpu_buffer_rsrc_t rw =
      make_rsrc(reinterpret_cast<const TA*>(P.W) + (int64_t)n * K, (uint32_t)K * (uint32_t)sizeof(TA));
  const __amdgpu_buffer_rsrc_t rx =
      make_rsrc(P.x, (uint32_t)rows * (uint32_t)K * (uint32_t)sizeof(TA));
  const int PASS = 64 * GV_U * VE;  // elements of K per pass
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.f;
  // two register sets of raw runs in turn (named, so every index is static);
  // runs convert to fp32 as they are multiplied
  u32x4 wa[GV_U], xa[R][GV_U], wb[GV_U], xb[R][GV_U];
  auto issue = [&](u32x4 (&w)[GV_U], u32x4 (&x)[R][GV_U], int k0) {
#pragma unroll
    for (int u = 0; u < GV_U; ++u) {
      const int k = k0 + (u * 64 + lane) * VE;
      const bool ok = k < K;  // K % 8 == 0: a run is all in or all out
      w[u] = buf_ld16(rw, ok ? (uint32_t)k * (uint32_t)sizeof(TA) : BUF_OOB);
#pragma unroll
      for (int r = 0; r < R; ++r)
        x[r][u] = buf_ld16(rx, ok && r < rows ? (uint32_t)(r * K + k) * (uint32_t)sizeof(TA) : BUF_OOB);
    }
  };
  auto fma_pass = [&](const u32x4 (&w)[GV_U], const u32x4 (&x)[R][GV_U]) {
#pragma unroll
    for (int u = 0; u < GV_U; ++u) {
      float wf[VE];
      gv_cvt<TA>(w[u], wf);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float xf[VE];
        gv_cvt<TA>(x[r][u], xf);
#pragma unroll
        for (int e = 0; e < VE; ++e) acc[r] = __builtin_fmaf(xf[e], wf[e], acc[r]);
      }
    }
  };
  issue(wa, xa, 0);
  for (int k0 = 0; k0 < K; k0 += 2 * PASS) {
    if (k0 + PASS < K) issue(wb, xb, k0 + PASS);
    fma_pass(wa, xa);
    if (k0 + PASS >= K) break;
    if (k0 + 2 * PASS < K) issue(wa, xa, k0 + 2 * PASS);
    fma_pass(wb, xb);
  }
  const TA* bias = reinterpret_cast<const TA*>(P.bias);
  const float b = bias ? to_f32(bias[n]) : 0.f;
  TA* y = reinterpret_cast<TA*>(P.y);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const float v = wave_sum(acc[r]);
    if (lane == r && r < rows) y[(int64_t)r * P.N + n] = from_f32<TA>(apply_act(v + b, P.act));
  }
}

}  // namespace rwkv7mi

using namespace rwkv7mi;

// x_i [rows, K_i], W_i [N_i, K_i], bias_i [N_i] or NULL, y_i [rows, N_i];
// act_i in {0 none, 1 tanh, 2 sigmoid, 3 relu^2}.  All tensors share act_dtype.
extern "C" int rwkv7mi_dense_multi(const void* const* xs, const void* const* Ws, const void* const* biases,
                                   void* const* ys, const int64_t* Ns, const int64_t* Ks, const int* acts,
                                   int64_t nprob, int64_t rows, int act_dtype, void* stream) {
  if (nprob < 1 || nprob > 4) return fail(RWKV7MI_EINVAL, "dense_multi: 1..4 problems");
  if (rows < 0) return fail(RWKV7MI_EINVAL, "dense_multi: bad rows");
  if (rows == 0) return RWKV7MI_OK;
  DenseBatch batch{};
  int tiles = 0;
  for (int i = 0; i < nprob; ++i) {
    if (!xs[i] || !Ws[i] || !ys[i]) return fail(RWKV7MI_EINVAL, "dense_multi: null pointer");
    if (Ns[i] <= 0 || Ks[i] <= 0 || Ks[i] % 8 || Ns[i] > INT32_MAX || Ks[i] > INT32_MAX)
      return fail(RWKV7MI_EINVAL, "dense_multi: N > 0 and K a positive multiple of 8 required");
    if (acts[i] < 0 || acts[i] > 3) return fail(RWKV7MI_EINVAL, "dense_multi: bad activation");
    if ((reinterpret_cast<uintptr_t>(xs[i]) | reinterpret_cast<uintptr_t>(Ws[i])) & 15)
      return fail(RWKV7MI_EINVAL, "dense_multi: x and W must be 16-byte aligned");
    batch.p[i] = DenseProb{xs[i], Ws[i], biases[i], ys[i], (int)Ns[i], (int)Ks[i], acts[i], tiles};
    tiles += (int)((Ns[i] + 15) / 16);
  }
  batch.nprob = (int)nprob;
  const size_t esz = act_dtype == RWKV7MI_F32 ? 4 : 2;
  if (rows <= 4) {  // the GEMV form: tiles of four features, one wave each
    DenseBatch gb = batch;
    int gt = 0;
    for (int i = 0; i < nprob; ++i) {
      gb.p[i].tile0 = gt;
      gt += (int)((Ns[i] + 3) / 4);
    }
    for (int i = 0; i < nprob; ++i)
      if ((int64_t)rows * Ks[i] * (int64_t)esz > INT32_MAX || Ks[i] * (int64_t)esz > INT32_MAX)
        return fail(RWKV7MI_EINVAL, "dense_multi: too large for 32-bit offsets");
    return dispatch_dtype(act_dtype, [&](auto ta) {
      using TA = decltype(ta);
      if (rows == 1)
        hipLaunchKernelGGL((dense_gemv_kernel<TA, 1>), dim3(gt), dim3(256), 0, as_stream(stream), gb, (int)rows);
      else if (rows == 2)
        hipLaunchKernelGGL((dense_gemv_kernel<TA, 2>), dim3(gt), dim3(256), 0, as_stream(stream), gb, (int)rows);
      else
        hipLaunchKernelGGL((dense_gemv_kernel<TA, 4>), dim3(gt), dim3(256), 0, as_stream(stream), gb, (int)rows);
      return check_launch("dense_gemv_kernel");
    });
  }
  for (int64_t r0 = 0; r0 < rows; r0 += 64) {
    const int64_t nr = rows - r0 > 64 ? 64 : rows - r0;
    DenseBatch bb = batch;
    for (int i = 0; i < nprob; ++i) {
      bb.p[i].x = reinterpret_cast<const char*>(batch.p[i].x) + r0 * Ks[i] * esz;
      bb.p[i].y = reinterpret_cast<char*>(batch.p[i].y) + r0 * Ns[i] * esz;
    }
    const int mt = nr <= 16 ? 1 : nr <= 32 ? 2 : 4;
    int rc = dispatch_dtype(act_dtype, [&](auto ta) {
      using TA = decltype(ta);
      if (mt == 1) hipLaunchKernelGGL((dense_kernel<1, TA>), dim3(tiles), dim3(256), 0, as_stream(stream), bb, (int)nr);
      else if (mt == 2) hipLaunchKernelGGL((dense_kernel<2, TA>), dim3(tiles), dim3(256), 0, as_stream(stream), bb, (int)nr);
      else hipLaunchKernelGGL((dense_kernel<4, TA>), dim3(tiles), dim3(256), 0, as_stream(stream), bb, (int)nr);
      return check_launch("dense_kernel");
    });
    if (rc) return rc;
  }
  return RWKV7MI_OK;
}
