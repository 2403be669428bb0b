// LayerNorm + token-shift mixes (decode and sequence forms) for gfx950.
//
// Decode (one token per row; one 256-lane workgroup per row, D <= 8192 and a
// multiple of 8; each thread owns contiguous runs of 8 elements):
//   attn:  [x = LN_pre(x), written back]   h = LN(x);  out_i = h + (prev - h) * mix_i
//          for the six mixes r,w,k,v,a,g;  prev <- h
//          (rwkv7_hf/fused_decode_norm_mix.py:161-293, torch form :203-241)
//   ffn:   x = residual (+ attn_out);  h = LN(x);  out = h + (prev - h) * mix;  prev <- h
//          (rwkv7_hf/fused_decode_norm_mix.py:296-348)
// Sequence ([B,T,D]; one workgroup per run of consecutive tokens, each
// normalised once, the first run's shift input read from prev_in and token
// T-1's LN written to prev_out; no intermediate buffer):
//   (rwkv7_hf/fused_time_mix.py:413-515, torch form native_jit_prefill.py:533-540, :955-961)
// All statistics in fp32 (two-pass variance), biased variance as F.layer_norm.
#include <algorithm>
#include <string>
#include <type_traits>

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
// w/b are the already loaded weight and bias slots.  The fused multiply-adds
// are written out, so every kernel that normalises a row gets the same bits.
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
        s2 = fmaf(c, c, s2);
      }
  const float inv = rsqrtf(block_sum(s2, red) / (float)D + eps);
#pragma unroll
  for (int s = 0; s < MIX_SLOTS; ++s)
#pragma unroll
    for (int e = 0; e < MIX_VEC; ++e) v[s][e] = fmaf((v[s][e] - mean) * inv, w[s][e], b[s][e]);
}

struct Mix6 {
  const void* mix[6];
  void* out[6];
};

// Split-K partials of the product that feeds this row's residual add (the
// previous layer's FFN value at 3..16 rows): x <- round(sum_s part[s] + x),
// the sums in split order, exactly as mm8t_split_reduce_kernel would write x.
struct MixParts {
  const float* part;  // part[s * stride + row * D + i], or null
  int64_t stride;     // floats between splits
  int S;
};
constexpr int MIX_MAXS = 4;

template <typename TA, typename TP>
__global__ __launch_bounds__(MIX_THREADS) void attn_norm_mix6_kernel(
    TA* x, TA* prev, const TP* __restrict__ ln_w, const TP* __restrict__ ln_b, const TP* pre_w,
    const TP* pre_b, Mix6 m, int D, int nmix, float eps, MixParts ps) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  TA* xr = x + row * D;
  TA* pr = prev + row * D;
  float v[MIX_SLOTS][MIX_VEC], pv[MIX_SLOTS][MIX_VEC], w[MIX_SLOTS][MIX_VEC], b[MIX_SLOTS][MIX_VEC];
  float mx[6][MIX_SLOTS][MIX_VEC];
  float ps_acc[MIX_SLOTS][MIX_VEC];
  if (ps.part) {  // uniform: every split's row first, so they are in flight with the rest
#pragma unroll
    for (int s = 0; s < MIX_SLOTS; ++s)
#pragma unroll
      for (int e = 0; e < MIX_VEC; ++e) ps_acc[s][e] = 0.f;
#pragma unroll
    for (int sp = 0; sp < MIX_MAXS; ++sp) {
      float t[MIX_SLOTS][MIX_VEC];
      ld_slots(ps.part + sp * ps.stride + row * D, D, t, sp < ps.S);
#pragma unroll
      for (int s = 0; s < MIX_SLOTS; ++s)
#pragma unroll
        for (int e = 0; e < MIX_VEC; ++e) ps_acc[s][e] += t[s][e];  // split order; past-the-end terms are +0
    }
  }
  ld_slots(xr, D, v);
  ld_slots(pr, D, pv);
  ld_slots(ln_w, D, w);
  ld_slots(ln_b, D, b);
#pragma unroll
  for (int i = 0; i < 6; ++i) ld_slots(reinterpret_cast<const TP*>(m.mix[i]), D, mx[i], i < nmix);
  if (ps.part) {
#pragma unroll
    for (int s = 0; s < MIX_SLOTS; ++s) {
#pragma unroll
      for (int e = 0; e < MIX_VEC; ++e) v[s][e] = ps_acc[s][e] + v[s][e];
      round8<TA>(v[s]);  // the residual stream stays in TA
    }
    st_slots(xr, D, v);
  }
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

// Decode attention-side entry for 1..8 rows, LN + token-shift mixes fused
// with the LoRA down projections (rwkv7_hf/fused_decode_norm_mix.py:161-293 and
// the down half of fused_wavg_lora, fused_lora.py:706):
//   x' = LN_pre(x) (layer 0 only, rounded to TA, -> x_out) or x;
//   h = LN(x') rounded to TA (-> h_out);  the r / k / v mixed rows
//   h + (prev - h) mix_i (-> outs);
//   part[q][c][row][j] = sum over K-chunk c of m_q . Wd_q[j], with
//   m_q = h + (prev - h) mix_lmix[q] rounded to TA (the reference's tensor).
// Weight-stationary: workgroup (g, c) owns 16 outputs of one LoRA problem and
// K-chunk c, for every row.  Thread t holds elements 8 (t + 256 s) .. +7
// (s = 0, 1) of every row of x in registers (packed TA) and the row
// statistics come from one batched block reduction per pass (two passes; a
// second pair for the pre-norm).  The threads whose elements fall in chunk c
// (each holds at most one such group) write m_q of every row into LDS; the four
// waves then split the chunk's 32-wide MFMA steps (A = the m rows from LDS, B =
// the 16 weight rows, loaded before anything else).  Rows are padded to 16 in
// the MFMA; pad rows of A are never read back.  Workgroup id w also writes the
// rows b = w (mod #workgroups): x_out, h_out and the r, k, v rows.  The
// per-chunk sums are the fused wkv decode kernel's lora_splits = #chunks.
constexpr int AML_MAXD = 4096;                 // D <= 2 groups of 8 per thread
constexpr int AML_MAXKC = 1024;                // K-chunk (elements)
constexpr int AML_AS = AML_MAXKC + 8;          // LDS row stride of the m rows (elements)
constexpr int AML_MAXROWS = 8;                 // rows live in registers (8 x 16 elements per thread)
struct MixLora {
  const void* mix[6];
  void* out[3];      // mixed rows r, k, v
  const void* lw[4];
  int lrank[4];
  int lmix[4];       // which mix feeds LoRA problem q
  int64_t loff[4];   // part offset of problem q (floats)
  int gbase[5];      // first output-group workgroup of problem q (gbase[nlora] = total)
  int nlora;
};

template <typename TA>
__device__ __forceinline__ auto aml_frag(u32x4 u) {
  if constexpr (std::is_same<TA, __half>::value) return __builtin_bit_cast(f16x8, u);
  else return __builtin_bit_cast(bf16x8, u);
}

// packed 8 x TA <-> fp32
template <typename TA>
__device__ __forceinline__ void aml_unpack(u32x4 u, float (&o)[8]) {
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    if constexpr (std::is_same<TA, __half>::value) {
      f16x2_to_f32(u[h], o[2 * h], o[2 * h + 1]);
    } else {
      o[2 * h] = __uint_as_float(u[h] << 16);
      o[2 * h + 1] = __uint_as_float(u[h] & 0xffff0000u);
    }
  }
}
template <typename TA>
__device__ __forceinline__ u32x4 aml_pack(const float (&v)[8]) {
  u32x4 d;
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    const TA lo = from_f32<TA>(v[2 * h]), hi = from_f32<TA>(v[2 * h + 1]);
    d[h] = (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
  }
  return d;
}

// Per-row block sums of v[b] (b < RM) in a fixed order, the same in every thread.
template <int RM>
__device__ __forceinline__ void aml_row_sums(float (&v)[RM], float (*buf)[4]) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
  for (int b = 0; b < RM; ++b) {
    const float t = wave_sum(v[b]);
    if (lane == 0) buf[b][wave] = t;
  }
  __syncthreads();
#pragma unroll
  for (int b = 0; b < RM; ++b) v[b] = (buf[b][0] + buf[b][1]) + (buf[b][2] + buf[b][3]);
}

// 8 raw elements of T (one or two 16-byte loads; zeros when !valid) and their fp32 values
template <typename T>
struct Raw8 {
  u32x4 u[sizeof(T) == 4 ? 2 : 1];
};
template <typename T>
__device__ __forceinline__ Raw8<T> raw8(__amdgpu_buffer_rsrc_t r, int e, bool valid) {
  Raw8<T> o;
  if constexpr (sizeof(T) == 4) {
    o.u[0] = buf_ld16(r, valid ? (uint32_t)e * 4u : BUF_OOB);
    o.u[1] = buf_ld16(r, valid ? (uint32_t)e * 4u + 16u : BUF_OOB);
  } else {
    o.u[0] = buf_ld16(r, valid ? (uint32_t)e * 2u : BUF_OOB);
  }
  return o;
}
template <typename T>
__device__ __forceinline__ void unraw8(const Raw8<T>& a, float (&o)[8]) {
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = __uint_as_float(a.u[i >> 2][i & 3]);
  } else {
    aml_unpack<T>(a.u[0], o);
  }
}

template <typename TA, typename TP, int RM>
__global__ __launch_bounds__(256) void attn_mix_lora_kernel(
    const TA* __restrict__ x, TA* __restrict__ x_out, const TA* __restrict__ prev, TA* __restrict__ h_out,
    const TP* __restrict__ ln_w, const TP* __restrict__ ln_b, const TP* __restrict__ pre_w,
    const TP* __restrict__ pre_b, const MixLora M, float* __restrict__ part, int rows, int D, int KC, float eps) {
  __shared__ __attribute__((aligned(16))) uint16_t am[16 * AML_AS];
  __shared__ float red[4][16][17];
  __shared__ float rbuf[4][RM][4];  // one buffer per reduction pass (no reuse hazards)
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int g = blockIdx.x, c = blockIdx.y, nch = gridDim.y;
  const int wg = g * nch + c, nwg = gridDim.x * nch;
  int q = 0;
  while (q < M.nlora - 1 && g >= M.gbase[q + 1]) ++q;
  const int r = M.lrank[q];
  const int j0 = (g - M.gbase[q]) * 16;  // first output of this workgroup within problem q
  const int k0 = c * KC;
  const int nsteps = KC / 128;            // 32-wide MFMA steps per wave
  const int e0[2] = {8 * tid, 8 * (tid + 256)};
  const bool in[2] = {e0[0] < D, e0[1] < D};
  // the thread's one group inside [k0, k0 + KC), if any
  const int sc = (e0[0] >= k0 && e0[0] < k0 + KC) ? 0 : 1;
  const bool own = in[sc] && e0[sc] >= k0 && e0[sc] < k0 + KC;
  const int ec = e0[sc];
  const bool writer = wg < rows;  // writes row wg (rows past nwg are taken in a second loop)
  const uint32_t DA = (uint32_t)(D * sizeof(TA)), DP = (uint32_t)(D * sizeof(TP));
  // ---- every load that depends on nothing, issued before the first wait
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(M.lw[q], (uint32_t)((int64_t)r * D * sizeof(TA)));
  const int jo = j0 + (lane & 15);
  u32x4 wreg[AML_MAXKC / 128];
#pragma unroll
  for (int i = 0; i < AML_MAXKC / 128; ++i) {
    const int k = k0 + 32 * (wave + 4 * i) + 8 * (lane >> 4);
    const bool ok = i < nsteps && jo < r;
    wreg[i] = buf_ld16(wr, ok ? (uint32_t)(((int64_t)jo * D + k) * sizeof(TA)) : BUF_OOB);
  }
  u32x4 xv[RM][2];
#pragma unroll
  for (int b = 0; b < RM; ++b) {
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(x + (int64_t)b * D, b < rows ? DA : 0u);
#pragma unroll
    for (int s = 0; s < 2; ++s) xv[b][s] = buf_ld16(xr, in[s] ? (uint32_t)(e0[s] * sizeof(TA)) : BUF_OOB);
  }
  Raw8<TP> lw[2], lb[2], pw[2], pb[2], wm[3][2], mqr;
  Raw8<TA> wp[2], pp[RM];
  {
    const __amdgpu_buffer_rsrc_t a = make_rsrc(ln_w, DP), bq = make_rsrc(ln_b, DP);
    const __amdgpu_buffer_rsrc_t pa = make_rsrc(pre_w, pre_w ? DP : 0u), pbq = make_rsrc(pre_b, pre_w ? DP : 0u);
    const __amdgpu_buffer_rsrc_t pr = make_rsrc(prev + (int64_t)(writer ? wg : 0) * D, writer ? DA : 0u);
    const int rk[3] = {0, 2, 3};  // r, k, v among the mixes r, w, k, v, a, g
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      lw[s] = raw8<TP>(a, e0[s], in[s]);
      lb[s] = raw8<TP>(bq, e0[s], in[s]);
      pw[s] = raw8<TP>(pa, e0[s], in[s]);
      pb[s] = raw8<TP>(pbq, e0[s], in[s]);
      wp[s] = raw8<TA>(pr, e0[s], in[s]);
#pragma unroll
      for (int i = 0; i < 3; ++i)
        wm[i][s] = raw8<TP>(make_rsrc(M.mix[rk[i]], writer ? DP : 0u), e0[s], in[s]);
    }
    mqr = raw8<TP>(make_rsrc(M.mix[M.lmix[q]], DP), ec, own);
#pragma unroll
    for (int b = 0; b < RM; ++b) pp[b] = raw8<TA>(make_rsrc(prev + (int64_t)b * D, b < rows ? DA : 0u), ec, own);
  }
  // ---- row statistics (two-pass); elements past D and rows past `rows` are zeros
  auto stats = [&](int pass, float (&mean)[RM], float (&rstd)[RM]) {
#pragma unroll
    for (int b = 0; b < RM; ++b) {
      float t = 0.f;
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        float v[8];
        aml_unpack<TA>(xv[b][s], v);
#pragma unroll
        for (int e = 0; e < 8; ++e) t += v[e];
      }
      mean[b] = t;
    }
    aml_row_sums<RM>(mean, rbuf[2 * pass]);
#pragma unroll
    for (int b = 0; b < RM; ++b) {
      mean[b] /= (float)D;
      float t = 0.f;
#pragma unroll
      for (int s = 0; s < 2; ++s)
        if (in[s]) {
          float v[8];
          aml_unpack<TA>(xv[b][s], v);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float d = v[e] - mean[b];
            t += d * d;
          }
        }
      rstd[b] = t;
    }
    aml_row_sums<RM>(rstd, rbuf[2 * pass + 1]);
#pragma unroll
    for (int b = 0; b < RM; ++b) rstd[b] = rsqrtf(rstd[b] / (float)D + eps);
  };
  float mean[RM], rstd[RM];
  if (pre_w) {
    stats(0, mean, rstd);
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      float w8[8], b8[8];
      unraw8<TP>(pw[s], w8);
      unraw8<TP>(pb[s], b8);
#pragma unroll
      for (int b = 0; b < RM; ++b) {
        float v[8];
        aml_unpack<TA>(xv[b][s], v);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = b < rows ? (v[e] - mean[b]) * rstd[b] * w8[e] + b8[e] : 0.f;  // 0 past D
        xv[b][s] = aml_pack<TA>(v);
      }
    }
  }
  stats(1, mean, rstd);
  // ---- this workgroup's rows: x_out, h_out and the r / k / v rows
  for (int b = wg; b < rows; b += nwg) {
    Raw8<TA> p8[2];
    Raw8<TP> m8[3][2];
    if (b == wg) {
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        p8[s] = wp[s];
#pragma unroll
        for (int i = 0; i < 3; ++i) m8[i][s] = wm[i][s];
      }
    } else {  // more rows than workgroups (small widths): load this row's operands now
      const int rk[3] = {0, 2, 3};
      const __amdgpu_buffer_rsrc_t pr = make_rsrc(prev + (int64_t)b * D, DA);
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        p8[s] = raw8<TA>(pr, e0[s], in[s]);
#pragma unroll
        for (int i = 0; i < 3; ++i) m8[i][s] = raw8<TP>(make_rsrc(M.mix[rk[i]], DP), e0[s], in[s]);
      }
    }
    // the row's registers are picked by a uniform loop over RM (no dynamic indexing)
    u32x4 u[2] = {xv[0][0], xv[0][1]};
    float mb = mean[0], rb = rstd[0];
#pragma unroll
    for (int bb = 1; bb < RM; ++bb)
      if (bb == b) {
        u[0] = xv[bb][0];
        u[1] = xv[bb][1];
        mb = mean[bb];
        rb = rstd[bb];
      }
#pragma unroll
    for (int s = 0; s < 2; ++s)
      if (in[s]) {
        float xb[8], w8[8], b8[8], p[8], h[8];
        aml_unpack<TA>(u[s], xb);
        if (pre_w) st8(x_out + (int64_t)b * D + e0[s], xb);
        unraw8<TP>(lw[s], w8);
        unraw8<TP>(lb[s], b8);
        unraw8<TA>(p8[s], p);
#pragma unroll
        for (int e = 0; e < 8; ++e) h[e] = (xb[e] - mb) * rb * w8[e] + b8[e];
        round8<TA>(h);
        st8(h_out + (int64_t)b * D + e0[s], h);
#pragma unroll
        for (int i = 0; i < 3; ++i) {
          float mk[8], o[8];
          unraw8<TP>(m8[i][s], mk);
#pragma unroll
          for (int e = 0; e < 8; ++e) o[e] = h[e] + (p[e] - h[e]) * mk[e];
          st8(reinterpret_cast<TA*>(M.out[i]) + (int64_t)b * D + e0[s], o);
        }
      }
  }
  // ---- m_q of the chunk into LDS
  if (own) {
    float mq[8], w8[8], b8[8];
    unraw8<TP>(mqr, mq);
    unraw8<TP>(sc ? lw[1] : lw[0], w8);
    unraw8<TP>(sc ? lb[1] : lb[0], b8);
#pragma unroll
    for (int b = 0; b < RM; ++b) {
      if (b < rows) {
        float h[8], p[8];
        aml_unpack<TA>(sc ? xv[b][1] : xv[b][0], h);
#pragma unroll
        for (int e = 0; e < 8; ++e) h[e] = (h[e] - mean[b]) * rstd[b] * w8[e] + b8[e];
        round8<TA>(h);
        unraw8<TA>(pp[b], p);
#pragma unroll
        for (int e = 0; e < 8; ++e) h[e] = h[e] + (p[e] - h[e]) * mq[e];
        const u32x4 d = aml_pack<TA>(h);
        *reinterpret_cast<uint4*>(&am[b * AML_AS + (ec - k0)]) = make_uint4(d[0], d[1], d[2], d[3]);
      }
    }
  }
  __syncthreads();
  // ---- MFMA over the chunk: wave w takes steps w, w + 4, ...
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  const int arow = lane & 15, akb = 8 * (lane >> 4);
#pragma unroll
  for (int i = 0; i < AML_MAXKC / 128; ++i) {
    if (i < nsteps) {
      const uint4 a = *reinterpret_cast<const uint4*>(&am[arow * AML_AS + 32 * (wave + 4 * i) + akb]);
      const u32x4 au = {a.x, a.y, a.z, a.w};
      acc = mfma16x16x32(aml_frag<TA>(au), aml_frag<TA>(wreg[i]), acc);
    }
  }
  // C: lane holds output column lane%16, rows 4 (lane/16) + e
#pragma unroll
  for (int e = 0; e < 4; ++e) red[wave][4 * (lane >> 4) + e][lane & 15] = acc[e];
  __syncthreads();
  {
    const int row = tid >> 4, col = tid & 15;
    const int j = j0 + col;
    if (row < rows && j < r) {
      const float sum = (red[0][row][col] + red[1][row][col]) + (red[2][row][col] + red[3][row][col]);
      part[M.loff[q] + ((int64_t)c * rows + row) * r + j] = sum;
    }
  }
}

// Sequence norm-mix: one workgroup per run of `run` consecutive tokens of one
// sequence (1..16, chosen so that long prompts get 16 and short ones still
// fill the GPU).  The LayerNorm and mixing parameters are loaded once per run;
// each token is normalised once by the loop below and its normalised row
// carried in registers as the next token's shift input; a run after the first
// starts one token early (its lead-in is normalised by the same loop code, so
// every run length gives the same bits); the next row's loads are in flight
// while a row is reduced.  NS = slots in use (D <= 2048 NS).
constexpr int SEQ_ROWS = 16;

template <int NS, typename T>
__device__ __forceinline__ void ld_ns(const T* row, int D, float (&v)[NS][MIX_VEC], bool active = true) {
  const __amdgpu_buffer_rsrc_t r = make_rsrc(row, active ? (uint32_t)(D * sizeof(T)) : 0u);
#pragma unroll
  for (int s = 0; s < NS; ++s) buf_ld8(r, (uint32_t)mix_base(s), active && mix_base(s) < D, (const T*)nullptr, v[s]);
}

template <int NS>
__device__ __forceinline__ void ln_ns(float (&v)[NS][MIX_VEC], int D, const float (&w)[NS][MIX_VEC],
                                      const float (&b)[NS][MIX_VEC], float eps, float* red) {
  float s1 = 0.f;
#pragma unroll
  for (int s = 0; s < NS; ++s)
#pragma unroll
    for (int e = 0; e < MIX_VEC; ++e) s1 += v[s][e];
  const float mean = block_sum(s1, red) / (float)D;
  float s2 = 0.f;
#pragma unroll
  for (int s = 0; s < NS; ++s)
    if (mix_base(s) < D)
#pragma unroll
      for (int e = 0; e < MIX_VEC; ++e) {
        const float c = v[s][e] - mean;
        s2 = fmaf(c, c, s2);
      }
  const float inv = rsqrtf(block_sum(s2, red) / (float)D + eps);
#pragma unroll
  for (int s = 0; s < NS; ++s)
#pragma unroll
    for (int e = 0; e < MIX_VEC; ++e) v[s][e] = fmaf((v[s][e] - mean) * inv, w[s][e], b[s][e]);
}

template <typename TA, typename TP, int NS>
__global__ __launch_bounds__(MIX_THREADS) void seq_norm_mix_rows_kernel(
    const TA* __restrict__ x, const TA* __restrict__ prev_in, TA* __restrict__ prev_out,
    const TP* __restrict__ ln_w, const TP* __restrict__ ln_b, Mix6 m, int T, int D, int nmix, int run, float eps) {
  __shared__ float red[4];
  const int runs = (T + run - 1) / run;
  const int b = blockIdx.x / runs;
  const int t0 = (blockIdx.x % runs) * run;
  const int t1 = min(T, t0 + run);
  const bool norm = ln_w != nullptr;
  float w[NS][MIX_VEC], bb[NS][MIX_VEC], v[NS][MIX_VEC], pv[NS][MIX_VEC];
  Raw8<TP> mx[6][NS];  // the mixes as loaded (two per register for 16-bit types)
  const int64_t rb = (int64_t)b * T;
  // a run after the first starts one token early: that token is normalised by
  // the same loop code as every other row (and as the run before it did) and
  // only becomes the shift input of the run's first token
  int t = t0 > 0 ? t0 - 1 : t0;
  ld_ns<NS>(prev_in + (int64_t)b * D, D, pv, t0 == 0);
  ld_ns<NS>(x + (rb + t) * D, D, v);
  if (norm) {
    ld_ns<NS>(ln_w, D, w);
    ld_ns<NS>(ln_b, D, bb);
  }
#pragma unroll
  for (int i = 0; i < 6; ++i) {
    const __amdgpu_buffer_rsrc_t r = make_rsrc(m.mix[i], i < nmix ? (uint32_t)(D * sizeof(TP)) : 0u);
#pragma unroll
    for (int s = 0; s < NS; ++s) mx[i][s] = raw8<TP>(r, mix_base(s), i < nmix && mix_base(s) < D);
  }
  for (; t < t1; ++t) {
    float nx[NS][MIX_VEC];
    ld_ns<NS>(x + (rb + t + 1) * D, D, nx, t + 1 < t1);  // the next row, in flight during this one
    if (norm) ln_ns<NS>(v, D, w, bb, eps, red);
#pragma unroll
    for (int s = 0; s < NS; ++s) round8<TA>(v[s]);  // the reference keeps h in TA before mixing
    if (t >= t0) {  // the lead-in token of a run writes nothing
      if (t == T - 1)
#pragma unroll
        for (int s = 0; s < NS; ++s)
          if (mix_base(s) < D) st8(prev_out + (int64_t)b * D + mix_base(s), v[s]);
#pragma unroll
      for (int i = 0; i < 6; ++i) {
        if (i < nmix) {
          TA* orow = reinterpret_cast<TA*>(m.out[i]) + (rb + t) * D;
#pragma unroll
          for (int s = 0; s < NS; ++s) {
            if (mix_base(s) < D) {
              float mf[MIX_VEC], o[MIX_VEC];
              // converted per row (kept packed across the loop, not hoisted)
              asm volatile("" : "+v"(mx[i][s].u[0]));
              unraw8<TP>(mx[i][s], mf);
#pragma unroll
              for (int e = 0; e < MIX_VEC; ++e) o[e] = fmaf(pv[s][e] - v[s][e], mf[e], v[s][e]);
              st8(orow + mix_base(s), o);
            }
          }
        }
      }
    }
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
      for (int e = 0; e < MIX_VEC; ++e) {
        pv[s][e] = v[s][e];
        v[s][e] = nx[s][e];
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

static int attn_norm_mix6_launch(void* x, void* prev, const void* ln_w, const void* ln_b, const void* pre_w,
                                 const void* pre_b, const void* const* mixes, void* const* outs, int64_t nmix,
                                 int64_t rows, int64_t D, float eps, int act_dtype, int param_dtype, MixParts ps,
                                 void* stream) {
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
                         (const TP*)pre_w, (const TP*)pre_b, m, (int)D, (int)nmix, eps, ps);
      return check_launch("attn_norm_mix6_kernel");
    });
  });
}

extern "C" int rwkv7mi_attn_norm_mix6(void* x, void* prev, const void* ln_w, const void* ln_b,
                                      const void* pre_w, const void* pre_b, const void* const* mixes,
                                      void* const* outs, int64_t nmix, int64_t rows, int64_t D, float eps,
                                      int act_dtype, int param_dtype, void* stream) {
  return attn_norm_mix6_launch(x, prev, ln_w, ln_b, pre_w, pre_b, mixes, outs, nmix, rows, D, eps, act_dtype,
                               param_dtype, MixParts{nullptr, 0, 0}, stream);
}

extern "C" int rwkv7mi_attn_norm_mix6_parts(void* x, void* prev, const void* ln_w, const void* ln_b,
                                            const void* const* mixes, void* const* outs, int64_t nmix,
                                            const float* part, int64_t splits, int64_t part_stride, int64_t rows,
                                            int64_t D, float eps, int act_dtype, int param_dtype, void* stream) {
  if (!part || splits < 1 || splits > MIX_MAXS || part_stride < rows * D || (reinterpret_cast<uintptr_t>(part) & 15) ||
      part_stride % 4)
    return fail(RWKV7MI_EINVAL, "attn_norm_mix6_parts: 1..4 splits of 16-byte aligned [rows, D] fp32 partials");
  return attn_norm_mix6_launch(x, prev, ln_w, ln_b, nullptr, nullptr, mixes, outs, nmix, rows, D, eps, act_dtype,
                               param_dtype, MixParts{part, part_stride, (int)splits}, stream);
}

// K-chunks of the fused attention-side launch for width D (0: not supported):
// four 1024-or-smaller chunks when they split into 128-wide wave steps, else two
// or one.
static int aml_chunks(int64_t D) {
  for (int ks : {4, 2, 1})
    if (D % (128 * ks) == 0 && D / ks <= AML_MAXKC) return ks;
  return 0;
}

extern "C" int rwkv7mi_attn_mix_lora_chunks(int64_t D) {
  return D > 0 && D <= AML_MAXD ? aml_chunks(D) : 0;
}

extern "C" int rwkv7mi_attn_mix_lora(const void* x, void* x_out, const void* prev, void* h_out, const void* ln_w,
                                     const void* ln_b, const void* pre_w, const void* pre_b,
                                     const void* const* mixes, void* const* outs, int64_t nlora,
                                     const void* const* lora_w, const int64_t* ranks, const int* lora_mix,
                                     float* part, int64_t rows, int64_t D, float eps, int act_dtype,
                                     int param_dtype, void* stream) {
  const std::string w("attn_mix_lora");
  const int KS = rwkv7mi_attn_mix_lora_chunks(D);
  if (!KS) return fail(RWKV7MI_EINVAL, w + ": D must be a multiple of 128 and at most 4096");
  if (rows < 0 || rows > AML_MAXROWS) return fail(RWKV7MI_EINVAL, w + ": 0..8 rows");
  if (rows == 0) return RWKV7MI_OK;
  if (act_dtype != RWKV7MI_F16 && act_dtype != RWKV7MI_BF16)
    return fail(RWKV7MI_EINVAL, w + ": fp16 or bf16 activations (the down projections run on MFMA)");
  if (!x || !prev || !h_out || !ln_w || !ln_b || !mixes || !outs || (!pre_w) != (!pre_b) || (pre_w && !x_out) ||
      nlora < 1 || nlora > 4 || !lora_w || !ranks || !lora_mix || !part)
    return fail(RWKV7MI_EINVAL, w + ": null pointer or bad count");
  const void* ins[] = {x, prev};
  const void* outs_[] = {x_out, h_out, outs[0], outs[1], outs[2], part};
  for (const void* o : outs_)
    for (const void* i : ins)
      if (o && o == i) return fail(RWKV7MI_EINVAL, w + ": outputs must not alias x or prev");
  if (!mix_aligned({x, x_out, prev, h_out, ln_w, ln_b, pre_w, pre_b, outs[0], outs[1], outs[2]}))
    return fail(RWKV7MI_EINVAL, w + ": pointers must be 16-byte aligned");
  MixLora m{};
  for (int i = 0; i < 6; ++i) {
    if (!mixes[i] || !mix_aligned({mixes[i]})) return fail(RWKV7MI_EINVAL, w + ": six aligned mixes needed");
    m.mix[i] = mixes[i];
  }
  for (int i = 0; i < 3; ++i) {
    if (!outs[i]) return fail(RWKV7MI_EINVAL, w + ": three outputs needed");
    m.out[i] = outs[i];
  }
  int64_t off = 0;
  int groups = 0;
  for (int q = 0; q < nlora; ++q) {
    if (!lora_w[q] || !mix_aligned({lora_w[q]}) || ranks[q] < 1 || ranks[q] > 1024 || lora_mix[q] < 0 ||
        lora_mix[q] > 5)
      return fail(RWKV7MI_EINVAL, w + ": bad LoRA weight, rank or mix index");
    m.lw[q] = lora_w[q];
    m.lrank[q] = (int)ranks[q];
    m.lmix[q] = lora_mix[q];
    m.loff[q] = off;
    m.gbase[q] = groups;
    off += (int64_t)KS * rows * ranks[q];
    groups += (int)((ranks[q] + 15) / 16);
  }
  m.gbase[nlora] = groups;
  m.nlora = (int)nlora;
  return dispatch_dtype(act_dtype, [&](auto ta) {
    using TA = decltype(ta);
    if constexpr (std::is_same<TA, float>::value) {
      return fail(RWKV7MI_EINVAL, w + ": fp16 or bf16 activations");
    } else {
      return dispatch_dtype(param_dtype, [&](auto tp) {
        using TP = decltype(tp);
        hipLaunchKernelGGL((attn_mix_lora_kernel<TA, TP, AML_MAXROWS>), dim3((unsigned)groups, (unsigned)KS),
                           dim3(256), 0, as_stream(stream), (const TA*)x, (TA*)x_out, (const TA*)prev, (TA*)h_out,
                           (const TP*)ln_w, (const TP*)ln_b, (const TP*)pre_w, (const TP*)pre_b, m, part,
                           (int)rows, (int)D, (int)(D / KS), eps);
        return check_launch("attn_mix_lora_kernel");
      });
    }
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
      // tokens per workgroup: 16 from 16k tokens, fewer below (at least ~1k workgroups)
      const int run = (int)std::min<int64_t>(SEQ_ROWS, std::max<int64_t>(1, B * T / 1024));
      const unsigned grid = (unsigned)(B * ((T + run - 1) / run));
      auto go = [&](auto ns) {
        constexpr int NS = decltype(ns)::value;
        hipLaunchKernelGGL((seq_norm_mix_rows_kernel<TA, TP, NS>), dim3(grid), dim3(MIX_THREADS), 0,
                           as_stream(stream), (const TA*)x, (const TA*)prev_in, (TA*)prev_out, (const TP*)ln_w,
                           (const TP*)ln_b, m, (int)T, (int)D, (int)nmix, run, eps);
        return check_launch("seq_norm_mix_rows_kernel");
      };
      const int64_t ns = (D + MIX_THREADS * MIX_VEC - 1) / (MIX_THREADS * MIX_VEC);
      if (ns == 1) return go(std::integral_constant<int, 1>{});
      if (ns == 2) return go(std::integral_constant<int, 2>{});
      if (ns == 3) return go(std::integral_constant<int, 3>{});
      return go(std::integral_constant<int, 4>{});
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
