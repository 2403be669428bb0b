// wkv7 single-token decode kernels (gfx950).
//
// One 256-lane workgroup per (batch, head).  The 64x64 fp32 state of the head
// is spread over the workgroup: lane t owns row i = t/4 (a value channel) and
// the 16 key columns [16*(t%4), 16*(t%4)+16), so a state row is four adjacent
// lanes and every lane moves 64 contiguous bytes (4 x 16-byte loads).  The
// per-token vectors are staged once in LDS.  Row dots (S.kk and S'.r) are
// 16 in-lane FMAs plus a 4-lane xor-shuffle reduction; the per-head GroupNorm
// of the output-prep variants reduces over the 4 waves through LDS.
//
// Math (native V x K orientation, rwkv7_hf/fused_recurrent_update.py:757-783):
//   S'[i,j] = S[i,j] * w[j] - (S[i,:] . kk) * kk[j] * a[j] + v[i] * k[j]
//   y[i]    = S'[i,:] . r
#include "common.h"
#include "decode_lora.h"

namespace rwkv7mi {

enum { MODE_UPDATE = 0, MODE_PREP = 1, MODE_RAW = 2 };

constexpr int HEAD = 64;

// After staging: the state row update, y = S' r, and (output-prep modes) the
// per-head GroupNorm, bonus and gate.  Lane t owns row i = t/4, key columns
// j0 .. j0+15 of the head; s[] holds them on entry.
template <bool PREP, typename TA>
__device__ __forceinline__ void decode_core(float (&s)[16], const float* s_r, const float* s_w, const float* s_k,
                                            const float* s_kk, const float* s_ka, const float* s_v, float corr,
                                            float* s_red, float g_i, float gnw_i, float gnb_i, float eps,
                                            float* state_out, int64_t soff, TA* out, int64_t vec) {
  const int tid = threadIdx.x;
  const int i = tid >> 2;
  const int j0 = (tid & 3) * 16;
  float dot = 0.f;
#pragma unroll
  for (int j = 0; j < 16; ++j) dot += s[j] * s_kk[j0 + j];
  dot = group_sum<4>(dot);
  const float vi = s_v[i];
  float y = 0.f;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    float ns = s[j] * s_w[j0 + j] - dot * s_ka[j0 + j] + vi * s_k[j0 + j];
    s[j] = ns;
    y += ns * s_r[j0 + j];
  }
  y = group_sum<4>(y);
  {
    float4* dst = reinterpret_cast<float4*>(state_out + soff);
#pragma unroll
    for (int q = 0; q < 4; ++q) dst[q] = make_float4(s[4 * q], s[4 * q + 1], s[4 * q + 2], s[4 * q + 3]);
  }

  if constexpr (!PREP) {
    if ((tid & 3) == 0) out[vec + i] = from_f32<TA>(y);
  } else {
    // GroupNorm over the head's 64 outputs (each row is replicated in 4 lanes).
    const int wave = tid >> 6;
    float ws = wave_sum(y) * 0.25f;
    if ((tid & 63) == 0) s_red[wave] = ws;
    __syncthreads();
    const float mean = (s_red[0] + s_red[1] + s_red[2] + s_red[3]) * (1.0f / HEAD);
    const float cen = y - mean;
    float wv2 = wave_sum(cen * cen) * 0.25f;
    if ((tid & 63) == 0) s_red[4 + wave] = wv2;
    __syncthreads();
    const float var = (s_red[4] + s_red[5] + s_red[6] + s_red[7]) * (1.0f / HEAD);
    if ((tid & 3) == 0) {
      float normed = cen * rsqrtf(var + eps);
      float o = (normed * gnw_i + gnb_i + corr * vi) * g_i;
      out[vec + i] = from_f32<TA>(o);
    }
  }
}

// kk = normalize(k_raw * k_k), k = k_raw * (1 + (a - 1) * k_a),
// w = exp(-0.606531 * sigmoid(w_raw))  (rwkv7_hf/fused_recurrent_update.py:198-204);
// v_mode 1 stores v as v_first, 2 mixes v toward v_first by v_gate.  Called by
// the first wave (lane = channel c).
template <typename TA>
__device__ __forceinline__ void stage_raw(int c, float rv, float wr, float kraw, float vv, float av, float kkw,
                                          float kaw, float rkw, int v_mode, TA* v_first, float vgate,
                                          int64_t vec, float* s_r, float* s_w, float* s_k, float* s_kk,
                                          float* s_ka, float* s_v, float* s_corr, bool vf_given = false,
                                          float vf_in = 0.f) {
  float kku = kraw * kkw;
  float nrm = sqrtf(wave_sum(kku * kku));
  const float kkv = kku / fmaxf(nrm, 1.0e-12f);
  const float kv = kraw * (1.0f + (av - 1.0f) * kaw);
  const float wv = expf(-0.606531f * (1.0f / (1.0f + expf(-wr))));
  if (v_mode == 1) {
    v_first[vec + c] = from_f32<TA>(vv);
  } else if (v_mode == 2) {
    const float vf = vf_given ? vf_in : to_f32(v_first[vec + c]);
    vv = vv + (vf - vv) * vgate;
  }
  s_r[c] = rv;
  s_w[c] = wv;
  s_k[c] = kv;
  s_kk[c] = kkv;
  s_ka[c] = kkv * av;
  s_v[c] = vv;
  // bonus scale sum_c r*k*r_k (rwkv7_hf/fused_recurrent_update.py:911)
  float corr = wave_sum(rv * kv * rkw);
  if (c == 0) *s_corr = corr;
}

template <int MODE, typename TA, typename TW, typename TP>
__global__ __launch_bounds__(256) void wkv7_decode_kernel(
    const TA* __restrict__ r, const TW* __restrict__ w, const TA* __restrict__ k,
    const TA* __restrict__ v, const TA* __restrict__ kk, const TA* __restrict__ a,
    const float* state_in, float* state_out, const TA* __restrict__ g,
    const TP* __restrict__ k_k, const TP* __restrict__ k_a, const TP* __restrict__ r_k,
    const TP* __restrict__ gn_w, const TP* __restrict__ gn_b, TA* __restrict__ out,
    TA* v_first, const TA* __restrict__ v_gate, int v_mode, int H, float eps) {
  __shared__ float s_r[HEAD], s_w[HEAD], s_k[HEAD], s_kk[HEAD], s_ka[HEAD], s_v[HEAD];
  __shared__ float s_red[8];
  __shared__ float s_corr;

  const int bh = blockIdx.x;
  const int h = bh % H;
  const int tid = threadIdx.x;
  const int64_t vec = (int64_t)bh * HEAD;

  // Issue the state rows (the bulk of the bytes) and the per-row output
  // parameters first, so they are in flight while the vectors are staged.
  const int i = tid >> 2;
  const int j0 = (tid & 3) * 16;
  const int64_t soff = ((int64_t)bh * HEAD + i) * HEAD + j0;
  float s[16];
  {
    const float4* src = reinterpret_cast<const float4*>(state_in + soff);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float4 t4 = src[q];
      s[4 * q + 0] = t4.x; s[4 * q + 1] = t4.y; s[4 * q + 2] = t4.z; s[4 * q + 3] = t4.w;
    }
  }
  float g_i = 0.f, gnw_i = 0.f, gnb_i = 0.f;
  if constexpr (MODE != MODE_UPDATE) {
    const int64_t pi = (int64_t)h * HEAD + i;
    g_i = ld(g, vec + i);
    gnw_i = ld(gn_w, pi);
    gnb_i = ld(gn_b, pi);
  }

  if (tid < HEAD) {
    const int c = tid;
    float rv = ld(r, vec + c);
    float av = ld(a, vec + c);
    float vv = ld(v, vec + c);
    if constexpr (MODE == MODE_RAW) {
      const int64_t pc = (int64_t)h * HEAD + c;
      stage_raw<TA>(c, rv, ld(w, vec + c), ld(k, vec + c), vv, av, ld(k_k, pc), ld(k_a, pc), ld(r_k, pc), v_mode,
                    v_first, v_mode == 2 ? ld(v_gate, vec + c) : 0.f, vec, s_r, s_w, s_k, s_kk, s_ka, s_v, &s_corr);
    } else {
      float kv, kkv, wv;
      kv = ld(k, vec + c);
      kkv = ld(kk, vec + c);
      wv = ld(w, vec + c);
      s_r[c] = rv;
      s_w[c] = wv;
      s_k[c] = kv;
      s_kk[c] = kkv;
      s_ka[c] = kkv * av;
      s_v[c] = vv;
      if constexpr (MODE != MODE_UPDATE) {
        // bonus scale sum_c r*k*r_k (rwkv7_hf/fused_recurrent_update.py:911)
        float corr = wave_sum(rv * kv * ld(r_k, (int64_t)h * HEAD + c));
        if (c == 0) s_corr = corr;
      }
    }
  }
  __syncthreads();
  decode_core<MODE != MODE_UPDATE, TA>(s, s_r, s_w, s_k, s_kk, s_ka, s_v, MODE != MODE_UPDATE ? s_corr : 0.f, s_red,
                                       g_i, gnw_i, gnb_i, eps, state_out, soff, out, vec);
}

// ---------------------------------------------------------------------------
// Decode with the W/A/G/V LoRA up projections fused in (rwkv7_hf/fused_lora.py
// :706 fused_wavg_lora, then fused_recurrent_output_prepare_raw): the four
// waves compute the head's channels of the up projections (dl_up,
// decode_lora.h), then the state update and output prep as in MODE_RAW.
template <typename TA, typename TP, int ZB>
__global__ __launch_bounds__(256) void wkv7_decode_lora_kernel(
    const TA* __restrict__ r, const TA* __restrict__ k, const TA* __restrict__ v, const DecLora LA,
    const float* state_in, float* state_out, const TP* __restrict__ k_k, const TP* __restrict__ k_a,
    const TP* __restrict__ r_k, const TP* __restrict__ gn_w, const TP* __restrict__ gn_b, TA* __restrict__ out,
    TA* v_first, int v_mode, int H, float eps) {
  __shared__ float s_r[HEAD], s_w[HEAD], s_k[HEAD], s_kk[HEAD], s_ka[HEAD], s_v[HEAD];
  __shared__ float s_red[8];
  __shared__ float s_corr;
  __shared__ __align__(16) float s_mid[4][DL_MAXR];
  __shared__ float s_lo[4][HEAD];

  const int bh = blockIdx.x;
  const int b = bh / H;
  const int h = bh % H;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int64_t vec = (int64_t)bh * HEAD;
  const int i = tid >> 2;
  const int j0 = (tid & 3) * 16;
  const int64_t soff = ((int64_t)bh * HEAD + i) * HEAD + j0;

  // state rows, per-row output parameters and channel `lane` of this head's
  // vectors (every wave loads them; only the first uses them) — no branches,
  // so all of these loads are in flight together with the LoRA loads; v_first
  // (v_mode 2) is issued with them rather than where it is used (it would add
  // a memory round trip there)
  float s[16];
  float gnw_i, gnb_i, rv, kraw, vv, kkw, kaw, rkw, vf_pre;
  dl_up<TA, ZB>(LA, b, h, H, wave, lane, s_mid, s_lo, [&] {
    const float4* src = reinterpret_cast<const float4*>(state_in + soff);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float4 t4 = src[q];
      s[4 * q + 0] = t4.x; s[4 * q + 1] = t4.y; s[4 * q + 2] = t4.z; s[4 * q + 3] = t4.w;
    }
    const int64_t pi = (int64_t)h * HEAD + i;
    gnw_i = ld(gn_w, pi);
    gnb_i = ld(gn_b, pi);
    const int64_t pc = (int64_t)h * HEAD + lane;
    rv = ld(r, vec + lane);
    kraw = ld(k, vec + lane);
    vv = ld(v, vec + lane);
    kkw = ld(k_k, pc);
    kaw = ld(k_a, pc);
    rkw = ld(r_k, pc);
    vf_pre = buf_ld1<TA>(make_rsrc(v_first ? v_first + vec : nullptr, v_first ? HEAD * (uint32_t)sizeof(TA) : 0u),
                         (uint32_t)lane, v_mode == 2);
  });
  __syncthreads();

  if (tid < HEAD)
    stage_raw<TA>(tid, rv, s_lo[0][tid], kraw, vv, s_lo[1][tid], kkw, kaw, rkw, v_mode, v_first,
                  v_mode == 2 ? s_lo[3][tid] : 0.f, vec, s_r, s_w, s_k, s_kk, s_ka, s_v, &s_corr, true, vf_pre);
  __syncthreads();
  decode_core<true, TA>(s, s_r, s_w, s_k, s_kk, s_ka, s_v, s_corr, s_red, s_lo[2][i], gnw_i, gnb_i, eps,
                        state_out, soff, out, vec);
}

template <int MODE>
static int launch_decode(const void* r, const void* w, const void* k, const void* v,
                         const void* kk, const void* a, const float* state_in, float* state_out,
                         const void* g, const void* r_k_, const void* k_k_, const void* k_a_,
                         const void* gn_w, const void* gn_b, void* out, void* v_first,
                         const void* v_gate, int v_mode, int64_t B, int64_t H, int64_t N,
                         float eps, int act_dtype, int w_dtype, int param_dtype, void* stream) {
  if (N != HEAD) return fail(RWKV7MI_EINVAL, "wkv7 decode: head size must be 64");
  if (B < 0 || H <= 0) return fail(RWKV7MI_EINVAL, "wkv7 decode: bad B/H");
  if (B == 0) return RWKV7MI_OK;
  if (!r || !w || !k || !v || !a || !state_in || !state_out || !out)
    return fail(RWKV7MI_EINVAL, "wkv7 decode: null pointer");
  if (MODE != MODE_RAW && !kk) return fail(RWKV7MI_EINVAL, "wkv7 decode: null kk");
  if (MODE != MODE_UPDATE && (!g || !r_k_ || !gn_w || !gn_b))
    return fail(RWKV7MI_EINVAL, "wkv7 decode: null output-prep parameter");
  if (MODE == MODE_RAW && (!k_k_ || !k_a_)) return fail(RWKV7MI_EINVAL, "wkv7 decode: null k_k/k_a");
  if (MODE == MODE_RAW && v_mode != 0 && !v_first)
    return fail(RWKV7MI_EINVAL, "wkv7 decode: v_mode needs v_first");
  if (MODE == MODE_RAW && v_mode == 2 && !v_gate)
    return fail(RWKV7MI_EINVAL, "wkv7 decode: v_mode 2 needs v_gate");
  if (v_mode < 0 || v_mode > 2) return fail(RWKV7MI_EINVAL, "wkv7 decode: bad v_mode");
  if ((reinterpret_cast<uintptr_t>(state_in) | reinterpret_cast<uintptr_t>(state_out)) & 15)
    return fail(RWKV7MI_EINVAL, "wkv7 decode: state must be 16-byte aligned");
  if (B * H > INT32_MAX) return fail(RWKV7MI_EINVAL, "wkv7 decode: B*H too large");
  if (MODE == MODE_UPDATE) param_dtype = act_dtype;
  int rc = RWKV7MI_OK;
  auto go = [&](auto ta) {
    using TA = decltype(ta);
    return dispatch_dtype(w_dtype, [&](auto tw) {
      using TW = decltype(tw);
      return dispatch_dtype(param_dtype, [&](auto tp) {
        using TP = decltype(tp);
        hipLaunchKernelGGL((wkv7_decode_kernel<MODE, TA, TW, TP>), dim3((unsigned)(B * H)), dim3(256), 0,
                           as_stream(stream), (const TA*)r, (const TW*)w, (const TA*)k, (const TA*)v,
                           (const TA*)kk, (const TA*)a, state_in, state_out, (const TA*)g,
                           (const TP*)k_k_, (const TP*)k_a_, (const TP*)r_k_, (const TP*)gn_w,
                           (const TP*)gn_b, (TA*)out, (TA*)v_first, (const TA*)v_gate, v_mode, (int)H,
                           eps);
        return check_launch("wkv7_decode_kernel");
      });
    });
  };
  rc = dispatch_dtype(act_dtype, go);
  return rc;
}

}  // namespace rwkv7mi

using namespace rwkv7mi;

extern "C" int rwkv7mi_wkv7_decode_update(const void* r, const void* w, const void* k, const void* v,
                                          const void* kk, const void* a, const float* state_in,
                                          float* state_out, void* y, int64_t B, int64_t H, int64_t N,
                                          int act_dtype, int w_dtype, void* stream) {
  return launch_decode<MODE_UPDATE>(r, w, k, v, kk, a, state_in, state_out, nullptr, nullptr, nullptr,
                                    nullptr, nullptr, nullptr, y, nullptr, nullptr, 0, B, H, N, 0.f,
                                    act_dtype, w_dtype, act_dtype, stream);
}

extern "C" int rwkv7mi_wkv7_decode_output_prepare(const void* r, const void* w, const void* k,
                                                  const void* v, const void* kk, const void* a,
                                                  const float* state_in, float* state_out,
                                                  const void* g, const void* r_k, const void* gn_w,
                                                  const void* gn_b, void* out, int64_t B, int64_t H,
                                                  int64_t N, float eps, int act_dtype, int w_dtype,
                                                  int param_dtype, void* stream) {
  return launch_decode<MODE_PREP>(r, w, k, v, kk, a, state_in, state_out, g, r_k, nullptr, nullptr,
                                  gn_w, gn_b, out, nullptr, nullptr, 0, B, H, N, eps, act_dtype,
                                  w_dtype, param_dtype, stream);
}

extern "C" int rwkv7mi_wkv7_decode_output_prepare_raw(
    const void* r, const void* w_raw, const void* k_raw, const void* v, const void* a,
    const float* state_in, float* state_out, const void* g, const void* k_k, const void* k_a,
    const void* r_k, const void* gn_w, const void* gn_b, void* out, void* v_first,
    const void* v_gate, int v_mode, int64_t B, int64_t H, int64_t N, float eps, int act_dtype,
    int param_dtype, void* stream) {
  return launch_decode<MODE_RAW>(r, w_raw, k_raw, v, nullptr, a, state_in, state_out, g, r_k, k_k,
                                 k_a, gn_w, gn_b, out, v_first, v_gate, v_mode, B, H, N, eps,
                                 act_dtype, act_dtype, param_dtype, stream);
}

extern "C" int rwkv7mi_wkv7_decode_lora_output_prepare(
    const void* r, const void* k_raw, const void* v, const float* lora_part, int64_t nprob,
    const int64_t* ranks, const void* const* w_up, const void* const* b_up, const int* act_down,
    const int* act_up, int64_t D, int64_t lora_splits, const float* state_in, float* state_out, const void* k_k,
    const void* k_a,
    const void* r_k, const void* gn_w, const void* gn_b, void* out, void* v_first, int v_mode, int64_t B,
    int64_t H, int64_t N, float eps, int act_dtype, int param_dtype, void* stream) {
  if (N != HEAD) return fail(RWKV7MI_EINVAL, "wkv7 decode lora: head size must be 64");
  if (B < 0 || H <= 0 || D <= 0) return fail(RWKV7MI_EINVAL, "wkv7 decode lora: bad B/H/D");
  if (B == 0) return RWKV7MI_OK;
  if (B > LORA_ROWS) return fail(RWKV7MI_EINVAL, "wkv7 decode lora: at most 64 rows");
  if (!r || !k_raw || !v || !state_in || !state_out || !k_k || !k_a || !r_k || !gn_w || !gn_b || !out)
    return fail(RWKV7MI_EINVAL, "wkv7 decode lora: null pointer");
  if (v_mode < 0 || v_mode > 2) return fail(RWKV7MI_EINVAL, "wkv7 decode lora: bad v_mode");
  if (v_mode == 2 && nprob != 4) return fail(RWKV7MI_EINVAL, "wkv7 decode lora: v_mode 2 needs the v LoRA");
  if (v_mode != 0 && !v_first) return fail(RWKV7MI_EINVAL, "wkv7 decode lora: v_mode needs v_first");
  if ((reinterpret_cast<uintptr_t>(state_in) | reinterpret_cast<uintptr_t>(state_out)) & 15)
    return fail(RWKV7MI_EINVAL, "wkv7 decode lora: state must be 16-byte aligned");
  if (B * H > INT32_MAX) return fail(RWKV7MI_EINVAL, "wkv7 decode lora: B*H too large");
  DecLora la;
  if (int rc = dl_build(la, "wkv7 decode lora", lora_part, nprob, ranks, w_up, b_up, act_down, act_up, D,
                        lora_splits, B))
    return rc;
  return dispatch_dtype(act_dtype, [&](auto ta) {
    using TA = decltype(ta);
    return dispatch_dtype(param_dtype, [&](auto tp) {
      using TP = decltype(tp);
      // sums that arrive whole (one split) need one partial load per lane, not a batch
      if (la.ks == 1)
        hipLaunchKernelGGL((wkv7_decode_lora_kernel<TA, TP, 1>), dim3((unsigned)(B * H)), dim3(256), 0,
                           as_stream(stream), (const TA*)r, (const TA*)k_raw, (const TA*)v, la, state_in, state_out,
                           (const TP*)k_k, (const TP*)k_a, (const TP*)r_k, (const TP*)gn_w, (const TP*)gn_b,
                           (TA*)out, (TA*)v_first, v_mode, (int)H, eps);
      else
        hipLaunchKernelGGL((wkv7_decode_lora_kernel<TA, TP, DL_ZB>), dim3((unsigned)(B * H)), dim3(256), 0,
                           as_stream(stream), (const TA*)r, (const TA*)k_raw, (const TA*)v, la, state_in, state_out,
                           (const TP*)k_k, (const TP*)k_a, (const TP*)r_k, (const TP*)gn_w, (const TP*)gn_b,
                           (TA*)out, (TA*)v_first, v_mode, (int)H, eps);
      return check_launch("wkv7_decode_lora_kernel");
    });
  });
}
