// Sequence-form elementwise preparation around the wkv7 scan (gfx950).
//
// state prep (rwkv7_hf/fused_prefill.py:43-150, torch form native_jit_prefill.py:779-790):
//   kk = normalize(k_raw * k_k) per head,  k = k_raw * (1 + (a - 1) * k_a),
//   v: mode 1 -> v_first = v;  mode 2 -> v = v + (v_first - v) * v_gate,
//   log_w = -0.606531 * sigmoid(w_raw)  (natural log of the decay) or the decay
//   exp(log_w), in fp32 or the activation dtype;  optionally a = sigmoid(a_raw)
//   and v_gate = sigmoid(v_gate_raw) first (rounded to the activation dtype)
// output prep (rwkv7_hf/fused_output.py:39-84, torch form native_jit_decode.py:862-866):
//   out = (GroupNorm_H(y) + (sum_head r * k * r_k) * v) * g
// Scalar forms: one 64-lane wave per (row, head), lane = channel.  Vector
// forms (taken when every pointer is 16-byte aligned): 8 lanes per (row,
// head), 8 channels per lane.
#include <initializer_list>

#include "common.h"

namespace rwkv7mi {

constexpr int PHD = 64;

template <typename TA, typename TP, typename TW>
__global__ __launch_bounds__(256) void state_prep_kernel(const TA* __restrict__ k_raw, const TA* __restrict__ a,
                                                         const TA* __restrict__ w_raw, const TA* v_raw, TA* v_out,
                                                         TA* v_first, const TA* __restrict__ v_gate,
                                                         const TP* __restrict__ k_k, const TP* __restrict__ k_a,
                                                         TA* __restrict__ kk_out, TA* __restrict__ k_out,
                                                         TW* __restrict__ w_out, int64_t rows, int H, int v_mode,
                                                         int flags) {
  const int64_t unit = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (unit >= rows * H) return;
  const int h = (int)(unit % H);
  const int c = threadIdx.x & 63;
  const int64_t off = unit * PHD + c;
  const int pc = h * PHD + c;
  const float kr = to_f32(k_raw[off]);
  float av = to_f32(a[off]);
  if (flags & RWKV7MI_PREP_A_RAW) av = to_f32(from_f32<TA>(1.0f / (1.0f + expf(-av))));  // sigmoid in the act dtype
  const float ku = kr * to_f32(k_k[pc]);
  const float nrm = sqrtf(wave_sum(ku * ku));
  kk_out[off] = from_f32<TA>(ku / fmaxf(nrm, 1.0e-12f));
  k_out[off] = from_f32<TA>(kr * (1.0f + (av - 1.0f) * to_f32(k_a[pc])));
  const float wr = to_f32(w_raw[off]);
  const float lw = -0.606531f / (1.0f + expf(-wr));
  w_out[off] = from_f32<TW>((flags & RWKV7MI_PREP_W_DECAY) ? expf(lw) : lw);
  // v_out may alias v_raw: each element is read, then written, by one lane
  const TA vr = v_raw[off];
  if (v_mode == 1) {
    v_first[off] = vr;
    v_out[off] = vr;
  } else if (v_mode == 2) {
    const float vv = to_f32(vr);
    float gv = to_f32(v_gate[off]);
    if (flags & RWKV7MI_PREP_VGATE_RAW) gv = to_f32(from_f32<TA>(1.0f / (1.0f + expf(-gv))));
    v_out[off] = from_f32<TA>(vv + (to_f32(v_first[off]) - vv) * gv);
  } else {
    v_out[off] = vr;
  }
}

template <typename TA, typename TP>
__global__ __launch_bounds__(256) void output_prep_kernel(const TA* __restrict__ y, const TA* __restrict__ r,
                                                          const TA* __restrict__ k, const TA* __restrict__ v,
                                                          const TA* __restrict__ g, const TP* __restrict__ r_k,
                                                          const TP* __restrict__ gn_w, const TP* __restrict__ gn_b,
                                                          TA* __restrict__ out, int64_t rows, int H, float eps) {
  const int64_t unit = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (unit >= rows * H) return;
  const int h = (int)(unit % H);
  const int c = threadIdx.x & 63;
  const int64_t off = unit * PHD + c;
  const int pc = h * PHD + c;
  const float yv = to_f32(y[off]);
  const float mean = wave_sum(yv) * (1.0f / PHD);
  const float cen = yv - mean;
  const float var = wave_sum(cen * cen) * (1.0f / PHD);
  const float vv = to_f32(v[off]);
  const float corr = wave_sum(to_f32(r[off]) * to_f32(k[off]) * to_f32(r_k[pc]));
  const float o = (cen * rsqrtf(var + eps) * to_f32(gn_w[pc]) + to_f32(gn_b[pc]) + corr * vv) * to_f32(g[off]);
  out[off] = from_f32<TA>(o);
}

// Vector forms: lane = 8 consecutive channels of one (row, head), 8 lanes per
// head, 16-byte accesses (32-byte for fp32).  Element arithmetic as above;
// the per-head sums run over each lane's 8 values in order, then across the
// head's 8 lanes (xor 1, 2, 4).  Every pointer 16-byte aligned.
__device__ __forceinline__ float group8_sum(float v) {
  v += __shfl_xor(v, 1, 64);
  v += __shfl_xor(v, 2, 64);
  v += __shfl_xor(v, 4, 64);
  return v;
}

template <typename TA, typename TP, typename TW>
__global__ __launch_bounds__(256) void state_prep_vec_kernel(const TA* __restrict__ k_raw, const TA* __restrict__ a,
                                                             const TA* __restrict__ w_raw, const TA* v_raw,
                                                             TA* v_out, TA* v_first, const TA* __restrict__ v_gate,
                                                             const TP* __restrict__ k_k, const TP* __restrict__ k_a,
                                                             TA* __restrict__ kk_out, TA* __restrict__ k_out,
                                                             TW* __restrict__ w_out, int64_t rows, int H, int v_mode,
                                                             int flags) {
  const int64_t unit = (int64_t)blockIdx.x * 32 + (threadIdx.x >> 3);
  if (unit >= rows * H) return;  // whole 8-lane groups leave together
  const int h = (int)(unit % H);
  const int c0 = 8 * (threadIdx.x & 7);
  const int64_t off = unit * PHD + c0;
  const int pc = h * PHD + c0;
  float kr[8], av[8], wr[8], kkw[8], kaw[8];
  ld8(k_raw + off, kr);
  ld8(a + off, av);
  ld8(w_raw + off, wr);
  ld8(k_k + pc, kkw);
  ld8(k_a + pc, kaw);
  float vr[8], vf[8], gv[8];
  ld8(v_raw + off, vr);
  if (v_mode == 2) {
    ld8(v_first + off, vf);
    ld8(v_gate + off, gv);
  }
  float ku[8], ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    if (flags & RWKV7MI_PREP_A_RAW) av[e] = to_f32(from_f32<TA>(1.0f / (1.0f + expf(-av[e]))));
    ku[e] = kr[e] * kkw[e];
    ss += ku[e] * ku[e];
  }
  const float nrm = fmaxf(sqrtf(group8_sum(ss)), 1.0e-12f);
  float kk[8], kv[8], wv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    kk[e] = ku[e] / nrm;
    kv[e] = kr[e] * (1.0f + (av[e] - 1.0f) * kaw[e]);
    const float lw = -0.606531f / (1.0f + expf(-wr[e]));
    wv[e] = (flags & RWKV7MI_PREP_W_DECAY) ? expf(lw) : lw;
  }
  st8(kk_out + off, kk);
  st8(k_out + off, kv);
  st8(w_out + off, wv);
  if (v_mode == 1) {
    st8(v_first + off, vr);
    st8(v_out + off, vr);
  } else if (v_mode == 2) {
    float vo[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float g = gv[e];
      if (flags & RWKV7MI_PREP_VGATE_RAW) g = to_f32(from_f32<TA>(1.0f / (1.0f + expf(-g))));
      vo[e] = vr[e] + (vf[e] - vr[e]) * g;
    }
    st8(v_out + off, vo);
  } else {
    st8(v_out + off, vr);
  }
}

template <typename TA, typename TP>
__global__ __launch_bounds__(256) void output_prep_vec_kernel(const TA* __restrict__ y, const TA* __restrict__ r,
                                                              const TA* __restrict__ k, const TA* __restrict__ v,
                                                              const TA* __restrict__ g, const TP* __restrict__ r_k,
                                                              const TP* __restrict__ gn_w,
                                                              const TP* __restrict__ gn_b, TA* __restrict__ out,
                                                              int64_t rows, int H, float eps) {
  const int64_t unit = (int64_t)blockIdx.x * 32 + (threadIdx.x >> 3);
  if (unit >= rows * H) return;
  const int h = (int)(unit % H);
  const int c0 = 8 * (threadIdx.x & 7);
  const int64_t off = unit * PHD + c0;
  const int pc = h * PHD + c0;
  float yv[8], rv[8], kv[8], vv[8], gv[8], rkw[8], gw[8], gb[8];
  ld8(y + off, yv);
  ld8(r + off, rv);
  ld8(k + off, kv);
  ld8(v + off, vv);
  ld8(g + off, gv);
  ld8(r_k + pc, rkw);
  ld8(gn_w + pc, gw);
  ld8(gn_b + pc, gb);
  float s1 = 0.f, sc = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    s1 += yv[e];
    sc += rv[e] * kv[e] * rkw[e];
  }
  const float mean = group8_sum(s1) * (1.0f / PHD);
  const float corr = group8_sum(sc);
  float s2 = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float c = yv[e] - mean;
    s2 += c * c;
  }
  const float rs = rsqrtf(group8_sum(s2) * (1.0f / PHD) + eps);
  float o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = ((yv[e] - mean) * rs * gw[e] + gb[e] + corr * vv[e]) * gv[e];
  st8(out + off, o);
}

}  // namespace rwkv7mi

using namespace rwkv7mi;

namespace {
bool aligned16(std::initializer_list<const void*> ps) {
  for (const void* p : ps)
    if (reinterpret_cast<uintptr_t>(p) & 15) return false;
  return true;
}
}  // namespace

extern "C" int rwkv7mi_state_prep(const void* k_raw, const void* a, const void* w_raw, const void* v_raw,
                                  void* v_out, void* v_first, const void* v_gate, const void* k_k, const void* k_a,
                                  void* kk_out, void* k_out, void* w_out, int64_t rows, int64_t H, int64_t N,
                                  int v_mode, int flags, int act_dtype, int param_dtype, int w_dtype, void* stream) {
  if (N != PHD) return fail(RWKV7MI_EINVAL, "state_prep: head size must be 64");
  if (rows < 0 || H <= 0) return fail(RWKV7MI_EINVAL, "state_prep: bad shape");
  if (v_mode < 0 || v_mode > 2) return fail(RWKV7MI_EINVAL, "state_prep: bad v_mode");
  if (flags & ~(RWKV7MI_PREP_A_RAW | RWKV7MI_PREP_VGATE_RAW | RWKV7MI_PREP_W_DECAY))
    return fail(RWKV7MI_EINVAL, "state_prep: unknown flags");
  if (w_dtype != RWKV7MI_F32 && w_dtype != act_dtype)
    return fail(RWKV7MI_EINVAL, "state_prep: w_out is fp32 or the activation dtype");
  if (rows == 0) return RWKV7MI_OK;
  if (!k_raw || !a || !w_raw || !v_raw || !v_out || !k_k || !k_a || !kk_out || !k_out || !w_out)
    return fail(RWKV7MI_EINVAL, "state_prep: null pointer");
  if (v_mode && !v_first) return fail(RWKV7MI_EINVAL, "state_prep: v_mode needs v_first");
  if (v_mode == 2 && !v_gate) return fail(RWKV7MI_EINVAL, "state_prep: v_mode 2 needs v_gate");
  const int64_t units = rows * H;
  if ((units + 3) / 4 > INT32_MAX) return fail(RWKV7MI_EINVAL, "state_prep: too large");
  // 16-byte vector form when every tensor allows it (v_out may alias v_raw:
  // each 8-element run is read, then written, by one lane)
  const bool vec = aligned16({k_raw, a, w_raw, v_raw, v_out, v_first, v_gate, k_k, k_a, kk_out, k_out, w_out});
  return dispatch_dtype(act_dtype, [&](auto ta) {
    using TA = decltype(ta);
    return dispatch_dtype(param_dtype, [&](auto tp) {
      using TP = decltype(tp);
      auto go = [&](auto tw) {
        using TW = decltype(tw);
        if (vec) {
          hipLaunchKernelGGL((state_prep_vec_kernel<TA, TP, TW>), dim3((unsigned)((units + 31) / 32)), dim3(256), 0,
                             as_stream(stream), (const TA*)k_raw, (const TA*)a, (const TA*)w_raw, (const TA*)v_raw,
                             (TA*)v_out, (TA*)v_first, (const TA*)v_gate, (const TP*)k_k, (const TP*)k_a,
                             (TA*)kk_out, (TA*)k_out, (TW*)w_out, rows, (int)H, v_mode, flags);
          return check_launch("state_prep_vec_kernel");
        }
        hipLaunchKernelGGL((state_prep_kernel<TA, TP, TW>), dim3((unsigned)((units + 3) / 4)), dim3(256), 0,
                           as_stream(stream), (const TA*)k_raw, (const TA*)a, (const TA*)w_raw, (const TA*)v_raw,
                           (TA*)v_out, (TA*)v_first, (const TA*)v_gate, (const TP*)k_k, (const TP*)k_a,
                           (TA*)kk_out, (TA*)k_out, (TW*)w_out, rows, (int)H, v_mode, flags);
        return check_launch("state_prep_kernel");
      };
      return w_dtype == RWKV7MI_F32 ? go(float{}) : go(TA{});
    });
  });
}

extern "C" int rwkv7mi_output_prepare(const void* y, const void* r, const void* k, const void* v, const void* g,
                                      const void* r_k, const void* gn_w, const void* gn_b, void* out, int64_t rows,
                                      int64_t H, int64_t N, float eps, int act_dtype, int param_dtype,
                                      void* stream) {
  if (N != PHD) return fail(RWKV7MI_EINVAL, "output_prepare: head size must be 64");
  if (rows < 0 || H <= 0) return fail(RWKV7MI_EINVAL, "output_prepare: bad shape");
  if (rows == 0) return RWKV7MI_OK;
  if (!y || !r || !k || !v || !g || !r_k || !gn_w || !gn_b || !out)
    return fail(RWKV7MI_EINVAL, "output_prepare: null pointer");
  const int64_t units = rows * H;
  if ((units + 3) / 4 > INT32_MAX) return fail(RWKV7MI_EINVAL, "output_prepare: too large");
  const bool vec = aligned16({y, r, k, v, g, r_k, gn_w, gn_b, out});
  return dispatch_dtype(act_dtype, [&](auto ta) {
    using TA = decltype(ta);
    return dispatch_dtype(param_dtype, [&](auto tp) {
      using TP = decltype(tp);
      if (vec) {
        hipLaunchKernelGGL((output_prep_vec_kernel<TA, TP>), dim3((unsigned)((units + 31) / 32)), dim3(256), 0,
                           as_stream(stream), (const TA*)y, (const TA*)r, (const TA*)k, (const TA*)v, (const TA*)g,
                           (const TP*)r_k, (const TP*)gn_w, (const TP*)gn_b, (TA*)out, rows, (int)H, eps);
        return check_launch("output_prep_vec_kernel");
      }
      hipLaunchKernelGGL((output_prep_kernel<TA, TP>), dim3((unsigned)((units + 3) / 4)), dim3(256), 0,
                         as_stream(stream), (const TA*)y, (const TA*)r, (const TA*)k, (const TA*)v, (const TA*)g,
                         (const TP*)r_k, (const TP*)gn_w, (const TP*)gn_b, (TA*)out, rows, (int)H, eps);
      return check_launch("output_prep_kernel");
    });
  });
}
