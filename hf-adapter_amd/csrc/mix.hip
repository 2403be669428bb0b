// LayerNorm + token-shift mixes (decode and sequence forms) for gfx950.
//
// Decode (one token per row; one 256-lane workgroup per row, D <= 8192):
//   attn:  [x = LN_pre(x), written back]   h = LN(x);  out_i = h + (prev - h) * mix_i
//          for the six mixes r,w,k,v,a,g;  prev <- h
//          (rwkv7_hf/fused_decode_norm_mix.py:161-293, torch form :203-241)
//   ffn:   x = residual (+ attn_out);  h = LN(x);  out = h + (prev - h) * mix;  prev <- h
//          (rwkv7_hf/fused_decode_norm_mix.py:296-348)
// Sequence ([B,T,D]; one workgroup per (b,t), which also normalises token t-1
// so no intermediate buffer is needed; the carried previous row is read from
// prev_in and token T-1's LN is written to prev_out):
//   (rwkv7_hf/fused_time_mix.py:413-515, torch form native_jit_prefill.py:533-540, :955-961)
// All statistics in fp32 (two-pass variance), biased variance as F.layer_norm.
#include "common.h"

namespace rwkv7mi {

constexpr int MIX_THREADS = 256;
constexpr int MIX_MAXV = 32;  // elements per thread (D <= 8192)

__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int wave = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  return red[0] + red[1] + red[2] + red[3];
}

// Normalise the D values held by this thread (strided by 256) in place.
template <typename TP>
__device__ __forceinline__ void layer_norm_regs(float (&v)[MIX_MAXV], int D, const TP* w, const TP* b,
                                                float eps, float* red) {
  float s = 0.f;
#pragma unroll
  for (int q = 0; q < MIX_MAXV; ++q) {
    const int d = threadIdx.x + q * MIX_THREADS;
    if (d < D) s += v[q];
  }
  const float mean = block_sum(s, red) / (float)D;
  float s2 = 0.f;
#pragma unroll
  for (int q = 0; q < MIX_MAXV; ++q) {
    const int d = threadIdx.x + q * MIX_THREADS;
    if (d < D) {
      const float c = v[q] - mean;
      s2 += c * c;
    }
  }
  const float var = block_sum(s2, red) / (float)D;
  const float inv = rsqrtf(var + eps);
#pragma unroll
  for (int q = 0; q < MIX_MAXV; ++q) {
    const int d = threadIdx.x + q * MIX_THREADS;
    if (d < D) v[q] = (v[q] - mean) * inv * to_f32(w[d]) + to_f32(b[d]);
  }
}

struct Mix6 {
  const void* mix[6];
  void* out[6];
};

template <typename TA, typename TP>
__global__ __launch_bounds__(MIX_THREADS) void attn_norm_mix6_kernel(
    TA* x, TA* prev, const TP* __restrict__ ln_w, const TP* __restrict__ ln_b, const TP* pre_w,
    const TP* pre_b, Mix6 m, int D, int nmix, float eps) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  TA* xr = x + row * D;
  TA* pr = prev + row * D;
  float v[MIX_MAXV];
#pragma unroll
  for (int q = 0; q < MIX_MAXV; ++q) {
    const int d = threadIdx.x + q * MIX_THREADS;
    v[q] = d < D ? to_f32(xr[d]) : 0.f;
  }
  if (pre_w) {
    layer_norm_regs(v, D, pre_w, pre_b, eps, red);
#pragma unroll
    for (int q = 0; q < MIX_MAXV; ++q) {
      const int d = threadIdx.x + q * MIX_THREADS;
      if (d < D) {
        const TA t = from_f32<TA>(v[q]);
        xr[d] = t;
        v[q] = to_f32(t);  // the residual stream continues in the activation dtype
      }
    }
  }
  layer_norm_regs(v, D, ln_w, ln_b, eps, red);
#pragma unroll
  for (int q = 0; q < MIX_MAXV; ++q) {
    const int d = threadIdx.x + q * MIX_THREADS;
    if (d < D) {
      // the reference keeps h in the activation dtype before mixing
      const TA hq = from_f32<TA>(v[q]);
      const float h = to_f32(hq);
      const float dlt = to_f32(pr[d]) - h;
      for (int i = 0; i < nmix; ++i)
        reinterpret_cast<TA*>(m.out[i])[row * D + d] =
            from_f32<TA>(h + dlt * to_f32(reinterpret_cast<const TP*>(m.mix[i])[d]));
      pr[d] = hq;
    }
  }
}

template <typename TA, typename TP>
__global__ __launch_bounds__(MIX_THREADS) void ffn_add_norm_mix_kernel(
    const TA* residual, const TA* attn_out, TA* prev, const TP* __restrict__ ln_w,
    const TP* __restrict__ ln_b, const TP* __restrict__ mix, TA* residual_out, TA* mixed, int D,
    float eps) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  float v[MIX_MAXV];
#pragma unroll
  for (int q = 0; q < MIX_MAXV; ++q) {
    const int d = threadIdx.x + q * MIX_THREADS;
    float xv = 0.f;
    if (d < D) {
      xv = to_f32(residual[row * D + d]);
      if (attn_out) {
        const TA s = from_f32<TA>(xv + to_f32(attn_out[row * D + d]));
        xv = to_f32(s);
        residual_out[row * D + d] = s;
      }
    }
    v[q] = xv;
  }
  layer_norm_regs(v, D, ln_w, ln_b, eps, red);
#pragma unroll
  for (int q = 0; q < MIX_MAXV; ++q) {
    const int d = threadIdx.x + q * MIX_THREADS;
    if (d < D) {
      const TA hq = from_f32<TA>(v[q]);
      const float h = to_f32(hq);
      const float p = to_f32(prev[row * D + d]);
      mixed[row * D + d] = from_f32<TA>(h + (p - h) * to_f32(mix[d]));
      prev[row * D + d] = hq;
    }
  }
}

// Sequence form: workgroup (b, t) normalises x[b,t] and x[b,t-1] (or takes prev_in[b]).
template <typename TA, typename TP>
__global__ __launch_bounds__(MIX_THREADS) void seq_norm_mix_kernel(
    const TA* __restrict__ x, const TA* __restrict__ prev_in, TA* __restrict__ prev_out,
    const TP* __restrict__ ln_w, const TP* __restrict__ ln_b, Mix6 m, int T, int D, int nmix,
    float eps) {
  __shared__ float red[4];
  const int b = blockIdx.x / T;
  const int t = blockIdx.x % T;
  const int64_t row = (int64_t)b * T + t;
  float v[MIX_MAXV], pv[MIX_MAXV];
#pragma unroll
  for (int q = 0; q < MIX_MAXV; ++q) {
    const int d = threadIdx.x + q * MIX_THREADS;
    v[q] = d < D ? to_f32(x[row * D + d]) : 0.f;
    pv[q] = (d < D && t > 0) ? to_f32(x[(row - 1) * D + d]) : 0.f;
  }
  layer_norm_regs(v, D, ln_w, ln_b, eps, red);
  if (t > 0) {
    layer_norm_regs(pv, D, ln_w, ln_b, eps, red);
  } else {
#pragma unroll
    for (int q = 0; q < MIX_MAXV; ++q) {
      const int d = threadIdx.x + q * MIX_THREADS;
      pv[q] = d < D ? to_f32(prev_in[(int64_t)b * D + d]) : 0.f;
    }
  }
#pragma unroll
  for (int q = 0; q < MIX_MAXV; ++q) {
    const int d = threadIdx.x + q * MIX_THREADS;
    if (d < D) {
      // the reference keeps h in the activation dtype before mixing
      const float h = to_f32(from_f32<TA>(v[q]));
      const float p = t > 0 ? to_f32(from_f32<TA>(pv[q])) : pv[q];
      const float dlt = p - h;
      for (int i = 0; i < nmix; ++i)
        reinterpret_cast<TA*>(m.out[i])[row * D + d] =
            from_f32<TA>(h + dlt * to_f32(reinterpret_cast<const TP*>(m.mix[i])[d]));
      if (t == T - 1) prev_out[(int64_t)b * D + d] = from_f32<TA>(v[q]);
    }
  }
}

}  // namespace rwkv7mi

using namespace rwkv7mi;

extern "C" int rwkv7mi_attn_norm_mix6(void* x, void* prev, const void* ln_w, const void* ln_b,
                                      const void* pre_w, const void* pre_b, const void* const* mixes,
                                      void* const* outs, int64_t nmix, int64_t rows, int64_t D, float eps,
                                      int act_dtype, int param_dtype, void* stream) {
  if (rows < 0 || D <= 0 || D > MIX_THREADS * MIX_MAXV) return fail(RWKV7MI_EINVAL, "attn_norm_mix6: bad shape");
  if (nmix < 1 || nmix > 6) return fail(RWKV7MI_EINVAL, "attn_norm_mix6: nmix must be 1..6");
  if (rows == 0) return RWKV7MI_OK;
  if (!x || !prev || !ln_w || !ln_b || !mixes || !outs || (!pre_w) != (!pre_b))
    return fail(RWKV7MI_EINVAL, "attn_norm_mix6: null pointer");
  if (x == prev) return fail(RWKV7MI_EINVAL, "attn_norm_mix6: x and previous must not alias");
  Mix6 m;
  for (int i = 0; i < 6; ++i) {
    m.mix[i] = i < nmix ? mixes[i] : nullptr;
    m.out[i] = i < nmix ? outs[i] : nullptr;
    if (i < nmix && (!m.mix[i] || !m.out[i])) return fail(RWKV7MI_EINVAL, "attn_norm_mix6: null mix/out");
  }
  return dispatch_dtype(act_dtype, [&](auto ta) {
    using TA = decltype(ta);
    return dispatch_dtype(param_dtype, [&](auto tp) {
      using TP = decltype(tp);
      hipLaunchKernelGGL((attn_norm_mix6_kernel<TA, TP>), dim3((unsigned)rows), dim3(MIX_THREADS), 0,
                         as_stream(stream), (TA*)x, (TA*)prev, (const TP*)ln_w, (const TP*)ln_b,
                         (const TP*)pre_w, (const TP*)pre_b, m, (int)D, (int)nmix, eps);
      return check_launch("attn_norm_mix6_kernel");
    });
  });
}

extern "C" int rwkv7mi_ffn_add_norm_mix(const void* residual, const void* attn_out, void* prev,
                                        const void* ln_w, const void* ln_b, const void* mix,
                                        void* residual_out, void* mixed, int64_t rows, int64_t D, float eps,
                                        int act_dtype, int param_dtype, void* stream) {
  if (rows < 0 || D <= 0 || D > MIX_THREADS * MIX_MAXV) return fail(RWKV7MI_EINVAL, "ffn_add_norm_mix: bad shape");
  if (rows == 0) return RWKV7MI_OK;
  if (!residual || !prev || !ln_w || !ln_b || !mix || !mixed || (attn_out && !residual_out))
    return fail(RWKV7MI_EINVAL, "ffn_add_norm_mix: null pointer");
  return dispatch_dtype(act_dtype, [&](auto ta) {
    using TA = decltype(ta);
    return dispatch_dtype(param_dtype, [&](auto tp) {
      using TP = decltype(tp);
      hipLaunchKernelGGL((ffn_add_norm_mix_kernel<TA, TP>), dim3((unsigned)rows), dim3(MIX_THREADS), 0,
                         as_stream(stream), (const TA*)residual, (const TA*)attn_out, (TA*)prev,
                         (const TP*)ln_w, (const TP*)ln_b, (const TP*)mix, (TA*)residual_out, (TA*)mixed,
                         (int)D, eps);
      return check_launch("ffn_add_norm_mix_kernel");
    });
  });
}

extern "C" int rwkv7mi_seq_norm_mix(const void* x, const void* prev_in, void* prev_out, const void* ln_w,
                                    const void* ln_b, const void* const* mixes, void* const* outs, int64_t nmix,
                                    int64_t B, int64_t T, int64_t D, float eps, int act_dtype, int param_dtype,
                                    void* stream) {
  if (B < 0 || T < 0 || D <= 0 || D > MIX_THREADS * MIX_MAXV) return fail(RWKV7MI_EINVAL, "seq_norm_mix: bad shape");
  if (nmix < 1 || nmix > 6) return fail(RWKV7MI_EINVAL, "seq_norm_mix: nmix must be 1..6");
  if (B == 0 || T == 0) return RWKV7MI_OK;
  if (!x || !prev_in || !prev_out || !ln_w || !ln_b || !mixes || !outs)
    return fail(RWKV7MI_EINVAL, "seq_norm_mix: null pointer");
  if (prev_in == prev_out) return fail(RWKV7MI_EINVAL, "seq_norm_mix: prev_in and prev_out must differ");
  if (B * T > INT32_MAX) return fail(RWKV7MI_EINVAL, "seq_norm_mix: too many rows");
  Mix6 m;
  for (int i = 0; i < 6; ++i) {
    m.mix[i] = i < nmix ? mixes[i] : nullptr;
    m.out[i] = i < nmix ? outs[i] : nullptr;
    if (i < nmix && (!m.mix[i] || !m.out[i])) return fail(RWKV7MI_EINVAL, "seq_norm_mix: null mix/out");
  }
  return dispatch_dtype(act_dtype, [&](auto ta) {
    using TA = decltype(ta);
    return dispatch_dtype(param_dtype, [&](auto tp) {
      using TP = decltype(tp);
      hipLaunchKernelGGL((seq_norm_mix_kernel<TA, TP>), dim3((unsigned)(B * T)), dim3(MIX_THREADS), 0,
                         as_stream(stream), (const TA*)x, (const TA*)prev_in, (TA*)prev_out, (const TP*)ln_w,
                         (const TP*)ln_b, m, (int)T, (int)D, (int)nmix, eps);
      return check_launch("seq_norm_mix_kernel");
    });
  });
}

namespace rwkv7mi {
template <typename TA, typename TP>
__global__ __launch_bounds__(MIX_THREADS) void layer_norm_kernel(const TA* x, TA* y, const TP* __restrict__ w,
                                                                 const TP* __restrict__ b, int D, float eps) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  float v[MIX_MAXV];
#pragma unroll
  for (int q = 0; q < MIX_MAXV; ++q) {
    const int d = threadIdx.x + q * MIX_THREADS;
    v[q] = d < D ? to_f32(x[row * D + d]) : 0.f;
  }
  layer_norm_regs(v, D, w, b, eps, red);
#pragma unroll
  for (int q = 0; q < MIX_MAXV; ++q) {
    const int d = threadIdx.x + q * MIX_THREADS;
    if (d < D) y[row * D + d] = from_f32<TA>(v[q]);
  }
}
}  // namespace rwkv7mi

extern "C" int rwkv7mi_layer_norm(const void* x, void* y, const void* w, const void* b, int64_t rows, int64_t D,
                                  float eps, int act_dtype, int param_dtype, void* stream) {
  if (rows < 0 || D <= 0 || D > MIX_THREADS * MIX_MAXV) return fail(RWKV7MI_EINVAL, "layer_norm: bad shape");
  if (rows == 0) return RWKV7MI_OK;
  if (!x || !y || !w || !b) return fail(RWKV7MI_EINVAL, "layer_norm: null pointer");
  if (rows > INT32_MAX) return fail(RWKV7MI_EINVAL, "layer_norm: too many rows");
  return dispatch_dtype(act_dtype, [&](auto ta) {
    using TA = decltype(ta);
    return dispatch_dtype(param_dtype, [&](auto tp) {
      using TP = decltype(tp);
      hipLaunchKernelGGL((layer_norm_kernel<TA, TP>), dim3((unsigned)rows), dim3(MIX_THREADS), 0, as_stream(stream),
                         (const TA*)x, (TA*)y, (const TP*)w, (const TP*)b, (int)D, eps);
      return check_launch("layer_norm_kernel");
    });
  });
}
