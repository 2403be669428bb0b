// LayerNorm + token-shift mixes (decode and sequence forms) for gfx950.
//
// Decode (one token per row; one 256-lane workgroup per row, D <= 8192 and a
// multiple of 8; each thread owns contiguous runs of 8 elements):
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
constexpr int MIX_VEC = 8;                               // contiguous elements per thread per slot
constexpr int MIX_SLOTS = 4;                             // D <= 256 * 8 * 4 = 8192
constexpr int MIX_MAXD = MIX_THREADS * MIX_VEC * MIX_SLOTS;

// Thread t owns elements [8 (t + 256 s), +8) for slot s; every global access is
// a 16-byte vector and all loads of a kernel are issued before its reductions.
__device__ __forceinline__ int mix_base(int s) { return MIX_VEC * ((int)threadIdx.x + MIX_THREADS * s); }

__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int wave = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

// Slots past D, and every slot when !active, read as zeros (unconditional
// buffer loads, so all of a kernel's loads are in flight together).
template <typename T>
__device__ __forceinline__ void ld_slots(const T* row, int D, float (&v)[MIX_SLOTS][MIX_VEC], bool active = true) {
  const __amdgpu_buffer_rsrc_t r = make_rsrc(row, active ? (uint32_t)(D * sizeof(T)) : 0u);
#pragma unroll
  for (int s = 0; s < MIX_SLOTS; ++s)
    buf_ld8(r, (uint32_t)mix_base(s), active && mix_base(s) < D, (const T*)nullptr, v[s]);
}

template <typename T>
__device__ __forceinline__ void st_slots(T* row, int D, const float (&v)[MIX_SLOTS][MIX_VEC]) {
#pragma unroll
  for (int s = 0; s < MIX_SLOTS; ++s)
    if (mix_base(s) < D) st8(row + mix_base(s), v[s]);
}

// In-place LayerNorm of the slots (two-pass fp32 statistics, biased variance);
// w/b are the already loaded weight and bias slots.
__device__ __forceinline__ void ln_slots(float (&v)[MIX_SLOTS][MIX_VEC], int D, const float (&w)[MIX_SLOTS][MIX_VEC],
                                         const float (&b)[MIX_SLOTS][MIX_VEC], float eps, float* red) {
  float s1 = 0.f;
#pragma unroll
  for (int s = 0; s < MIX_SLOTS; ++s)
#pragma unroll
    for (int e = 0; e < MIX_VEC; ++e) s1 += v[s][e];  // padding slots hold zeros
  const float mean = block_sum(s1, red) / (float)D;
  float s2 = 0.f;
#pragma unroll
  for (int s = 0; s < MIX_SLOTS; ++s)
    if (mix_base(s) < D)
#pragma unroll
      for (int e = 0; e < MIX_VEC; ++e) {
        const float c = v[s][e] - mean;
        s2 += c * c;
      }
  const float inv = rsqrtf(block_sum(s2, red) / (float)D + eps);
#pragma unroll
  for (int s = 0; s < MIX_SLOTS; ++s)
#pragma unroll
    for (int e = 0; e < MIX_VEC; ++e) v[s][e] = (v[s][e] - mean) * inv * w[s][e] + b[s][e];
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
  float v[MIX_SLOTS][MIX_VEC], pv[MIX_SLOTS][MIX_VEC], w[MIX_SLOTS][MIX_VEC], b[MIX_SLOTS][MIX_VEC];
  float mx[6][MIX_SLOTS][MIX_VEC];
  ld_slots(xr, D, v);
  ld_slots(pr, D, pv);
  ld_slots(ln_w, D, w);
  ld_slots(ln_b, D, b);
#pragma unroll
  for (int i = 0; i < 6; ++i) ld_slots(reinterpret_cast<const TP*>(m.mix[i]), D, mx[i], i < nmix);
  if (pre_w) {
    float pw[MIX_SLOTS][MIX_VEC], pb[MIX_SLOTS][MIX_VEC];
    ld_slots(pre_w, D, pw);
    ld_slots(pre_b, D, pb);
    ln_slots(v, D, pw, pb, eps, red);
#pragma unroll
    for (int s = 0; s < MIX_SLOTS; ++s) round8<TA>(v[s]);  // the residual stream stays in TA
    st_slots(xr, D, v);
  }
  ln_slots(v, D, w, b, eps, red);
#pragma unroll
  for (int s = 0; s < MIX_SLOTS; ++s) round8<TA>(v[s]);  // the reference keeps h in TA before mixing
#pragma unroll
  for (int i = 0; i < 6; ++i) {
    if (i < nmix) {
      float o[MIX_SLOTS][MIX_VEC];
#pragma unroll
      for (int s = 0; s < MIX_SLOTS; ++s)
#pragma unroll
        for (int e = 0; e < MIX_VEC; ++e) o[s][e] = v[s][e] + (pv[s][e] - v[s][e]) * mx[i][s][e];
      st_slots(reinterpret_cast<TA*>(m.out[i]) + row * D, D, o);
    }
  }
  st_slots(pr, D, v);
}

template <typename TA, typename TP>
__global__ __launch_bounds__(MIX_THREADS) void ffn_add_norm_mix_kernel(
    const TA* residual, const TA* attn_out, TA* prev, const TP* __restrict__ ln_w,
    const TP* __restrict__ ln_b, const TP* __restrict__ mix, TA* residual_out, TA* mixed, int D,
    float eps) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  float v[MIX_SLOTS][MIX_VEC], pv[MIX_SLOTS][MIX_VEC], w[MIX_SLOTS][MIX_VEC], b[MIX_SLOTS][MIX_VEC];
  float mk[MIX_SLOTS][MIX_VEC];
  ld_slots(residual + row * D, D, v);
  ld_slots(prev + row * D, D, pv);
  ld_slots(ln_w, D, w);
  ld_slots(ln_b, D, b);
  ld_slots(mix, D, mk);
  if (attn_out) {
    float a[MIX_SLOTS][MIX_VEC];
    ld_slots(attn_out + row * D, D, a);
#pragma unroll
    for (int s = 0; s < MIX_SLOTS; ++s) {
#pragma unroll
      for (int e = 0; e < MIX_VEC; ++e) v[s][e] += a[s][e];
      round8<TA>(v[s]);
    }
    st_slots(residual_out + row * D, D, v);
  }
  ln_slots(v, D, w, b, eps, red);
#pragma unroll
  for (int s = 0; s < MIX_SLOTS; ++s) round8<TA>(v[s]);
  float o[MIX_SLOTS][MIX_VEC];
#pragma unroll
  for (int s = 0; s < MIX_SLOTS; ++s)
#pragma unroll
    for (int e = 0; e < MIX_VEC; ++e) o[s][e] = v[s][e] + (pv[s][e] - v[s][e]) * mk[s][e];
  st_slots(mixed + row * D, D, o);
  st_slots(prev + row * D, D, v);
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
  float v[MIX_SLOTS][MIX_VEC], pv[MIX_SLOTS][MIX_VEC], w[MIX_SLOTS][MIX_VEC], bb[MIX_SLOTS][MIX_VEC];
  float mx[6][MIX_SLOTS][MIX_VEC];
  // ln_w == null: x is already normalised (the reference's calling convention,
  // rwkv7_hf/fused_time_mix.py:413-515) and is mixed as given
  const bool norm = ln_w != nullptr;
  ld_slots(x + row * D, D, v);
  ld_slots(t > 0 ? x + (row - 1) * D : prev_in + (int64_t)b * D, D, pv);
  if (norm) {
    ld_slots(ln_w, D, w);
    ld_slots(ln_b, D, bb);
  }
#pragma unroll
  for (int i = 0; i < 6; ++i) ld_slots(reinterpret_cast<const TP*>(m.mix[i]), D, mx[i], i < nmix);
  if (norm) {
    ln_slots(v, D, w, bb, eps, red);
    if (t > 0) {
      ln_slots(pv, D, w, bb, eps, red);
#pragma unroll
      for (int s = 0; s < MIX_SLOTS; ++s) round8<TA>(pv[s]);
    }
  }
  if (t == T - 1) st_slots(prev_out + (int64_t)b * D, D, v);
#pragma unroll
  for (int s = 0; s < MIX_SLOTS; ++s) round8<TA>(v[s]);  // the reference keeps h in TA before mixing
#pragma unroll
  for (int i = 0; i < 6; ++i) {
    if (i < nmix) {
      float o[MIX_SLOTS][MIX_VEC];
#pragma unroll
      for (int s = 0; s < MIX_SLOTS; ++s)
#pragma unroll
        for (int e = 0; e < MIX_VEC; ++e) o[s][e] = v[s][e] + (pv[s][e] - v[s][e]) * mx[i][s][e];
      st_slots(reinterpret_cast<TA*>(m.out[i]) + row * D, D, o);
    }
  }
}

static bool mix_aligned(std::initializer_list<const void*> ps) {
  for (const void* p : ps)
    if (reinterpret_cast<uintptr_t>(p) & 15) return false;
  return true;
}

}  // namespace rwkv7mi

using namespace rwkv7mi;

extern "C" int rwkv7mi_attn_norm_mix6(void* x, void* prev, const void* ln_w, const void* ln_b,
                                      const void* pre_w, const void* pre_b, const void* const* mixes,
                                      void* const* outs, int64_t nmix, int64_t rows, int64_t D, float eps,
                                      int act_dtype, int param_dtype, void* stream) {
  if (rows < 0 || D <= 0 || D > MIX_MAXD || D % 8)
    return fail(RWKV7MI_EINVAL, "attn_norm_mix6: D must be a multiple of 8 and at most 8192");
  if (nmix < 1 || nmix > 6) return fail(RWKV7MI_EINVAL, "attn_norm_mix6: nmix must be 1..6");
  if (rows == 0) return RWKV7MI_OK;
  if (!x || !prev || !ln_w || !ln_b || !mixes || !outs || (!pre_w) != (!pre_b))
    return fail(RWKV7MI_EINVAL, "attn_norm_mix6: null pointer");
  if (x == prev) return fail(RWKV7MI_EINVAL, "attn_norm_mix6: x and previous must not alias");
  if (!mix_aligned({x, prev, ln_w, ln_b, pre_w, pre_b})) return fail(RWKV7MI_EINVAL, "attn_norm_mix6: pointers must be 16-byte aligned");
  Mix6 m;
  for (int i = 0; i < 6; ++i) {
    m.mix[i] = i < nmix ? mixes[i] : nullptr;
    m.out[i] = i < nmix ? outs[i] : nullptr;
    if (i < nmix && (!m.mix[i] || !m.out[i])) return fail(RWKV7MI_EINVAL, "attn_norm_mix6: null mix/out");
    if (i < nmix && !mix_aligned({m.mix[i], m.out[i]})) return fail(RWKV7MI_EINVAL, "attn_norm_mix6: pointers must be 16-byte aligned");
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
  if (rows < 0 || D <= 0 || D > MIX_MAXD || D % 8)
    return fail(RWKV7MI_EINVAL, "ffn_add_norm_mix: D must be a multiple of 8 and at most 8192");
  if (rows == 0) return RWKV7MI_OK;
  if (!residual || !prev || !ln_w || !ln_b || !mix || !mixed || (attn_out && !residual_out))
    return fail(RWKV7MI_EINVAL, "ffn_add_norm_mix: null pointer");
  if (!mix_aligned({residual, attn_out, prev, ln_w, ln_b, mix, residual_out, mixed}))
    return fail(RWKV7MI_EINVAL, "ffn_add_norm_mix: pointers must be 16-byte aligned");
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
  if (B < 0 || T < 0 || D <= 0 || D > MIX_MAXD || D % 8)
    return fail(RWKV7MI_EINVAL, "seq_norm_mix: D must be a multiple of 8 and at most 8192");
  if (nmix < 1 || nmix > 6) return fail(RWKV7MI_EINVAL, "seq_norm_mix: nmix must be 1..6");
  if (B == 0 || T == 0) return RWKV7MI_OK;
  if (!x || !prev_in || !prev_out || !mixes || !outs || (!ln_w) != (!ln_b))
    return fail(RWKV7MI_EINVAL, "seq_norm_mix: null pointer (ln_w and ln_b are both given or both null)");
  if (prev_in == prev_out) return fail(RWKV7MI_EINVAL, "seq_norm_mix: prev_in and prev_out must differ");
  if (!mix_aligned({x, prev_in, prev_out, ln_w, ln_b})) return fail(RWKV7MI_EINVAL, "seq_norm_mix: pointers must be 16-byte aligned");
  if (B * T > INT32_MAX) return fail(RWKV7MI_EINVAL, "seq_norm_mix: too many rows");
  Mix6 m;
  for (int i = 0; i < 6; ++i) {
    m.mix[i] = i < nmix ? mixes[i] : nullptr;
    m.out[i] = i < nmix ? outs[i] : nullptr;
    if (i < nmix && (!m.mix[i] || !m.out[i])) return fail(RWKV7MI_EINVAL, "seq_norm_mix: null mix/out");
    if (i < nmix && !mix_aligned({m.mix[i], m.out[i]})) return fail(RWKV7MI_EINVAL, "seq_norm_mix: pointers must be 16-byte aligned");
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
  float v[MIX_SLOTS][MIX_VEC], ww[MIX_SLOTS][MIX_VEC], bb[MIX_SLOTS][MIX_VEC];
  ld_slots(x + row * D, D, v);
  ld_slots(w, D, ww);
  ld_slots(b, D, bb);
  ln_slots(v, D, ww, bb, eps, red);
  st_slots(y + row * D, D, v);
}
}  // namespace rwkv7mi

extern "C" int rwkv7mi_layer_norm(const void* x, void* y, const void* w, const void* b, int64_t rows, int64_t D,
                                  float eps, int act_dtype, int param_dtype, void* stream) {
  if (rows < 0 || D <= 0 || D > MIX_MAXD || D % 8)
    return fail(RWKV7MI_EINVAL, "layer_norm: D must be a multiple of 8 and at most 8192");
  if (rows == 0) return RWKV7MI_OK;
  if (!x || !y || !w || !b) return fail(RWKV7MI_EINVAL, "layer_norm: null pointer");
  if (!mix_aligned({x, y, w, b})) return fail(RWKV7MI_EINVAL, "layer_norm: pointers must be 16-byte aligned");
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
