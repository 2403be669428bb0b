// wkv7 recurrence with an fp16 state (gfx950): the optional fp16-state lane.
//
// The state S [B, H, 64, 64] is fp16, row = value channel, column = key
// channel, and every state operation is a packed fp16 FMA (v_pk_fma_f16,
// one rounding each) in a fixed order, so the result is defined to the bit by
// that order (rwkv7_hf/native_wkv_fp16.py:279-300, :390-410):
//   sa     = fp16 sum over key pairs:  sa2 = fma(-kk[2j..], S[i,2j..], sa2),
//            j = 0..31 in turn, then sa = sa2.lo + sa2.hi
//   S[i,j] = fma(S[i,j], wd[j], fma(k[j], v[i], fma(sa, b[j], S[i,j])))
//   y[i]   = fp16 sum over pairs: y2 = fma(S'[i,2j..], r[2j..], y2), then lo + hi
// where wd = exp(-e^-1/2 * sigmoid(w)) - 1 + dither(phase), computed in fp32
// and rounded once to fp16, and b = kk * a.  The dither is the multiplicative
// hash of the phase (Knuth, golden-ratio constant 0x9E3779B9) as a signed
// 32-bit integer times 2^-41 (|dither| <= 2^-10); phase = elapsed[b] + 64 h + i
// (+ the token index in a sequence).
//
// The fixed FMA order makes one lane own one state row: the two 32-long
// chains (sa and y) run inside the lane.  One 64-lane wave per (batch, head),
// lane i = state row i = channel i.  The head's 8 KB of state moves through
// LDS so that global loads and stores stay coalesced (16 bytes per lane,
// consecutive lanes on consecutive addresses); the per-token key-side vectors
// are staged in LDS and read back as broadcasts.
#include "common.h"
#include "decode_lora.h"

// No implicit fusing in this file: every fp32 expression that ends in an fp16
// value (decay delta, k, kk*a, the V interpolation) is rounded to fp32 first
// and then to fp16, as the reference computes it; a multiply-add fused into a
// mixed-precision FMA with an fp16 result would round once instead.  The
// state's FMAs are explicit.
#pragma clang fp contract(off)

namespace rwkv7mi {

constexpr int F16_N = 64;
constexpr int F16_RS = 72;       // LDS state row stride in halves (144 B: 16 lanes' 16-byte reads hit 64 banks)
constexpr int F16_SLAB = 8;      // tokens staged per LDS fill in the sequence kernel
constexpr float F16_LOG2E = 1.4426950408889634f;
constexpr float F16_DECAY_LOG2 = 0.8750387749145276f;  // e^-1/2 * log2(e)

typedef _Float16 h2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ h2 pk_fma(h2 a, h2 b, h2 c) { return __builtin_elementwise_fma(a, b, c); }

__device__ __forceinline__ h2 h2_bits(uint32_t u) { return __builtin_bit_cast(h2, u); }
__device__ __forceinline__ uint32_t h2_u32(h2 x) { return __builtin_bit_cast(uint32_t, x); }
__device__ __forceinline__ _Float16 h_bits(unsigned short u) { return __builtin_bit_cast(_Float16, u); }

// fp32 -> fp16, round to nearest even, of the fp32 value itself: the empty asm
// pins x as an fp32 register so that the conversion is not folded into the
// instruction producing x (a mixed-precision FMA with an fp16 result would
// round the exact value once instead of the fp32 value)
__device__ __forceinline__ _Float16 f16_rn(float x) {
  asm volatile("" : "+v"(x));
  return (_Float16)x;
}

// 2^-41 * int32(0x9E3779B9 * phase)
__device__ __forceinline__ float f16_dither(uint32_t phase) {
  return 0x1p-41f * (float)(int32_t)(0x9E3779B9u * phase);
}

// exp(-e^-1/2 sigmoid(wv)) - 1 + dither, in fp32, rounded to fp16
// (hardware 2^x and 1/x, each within about an ulp of fp32)
__device__ __forceinline__ _Float16 f16_decay_delta(float wv, uint32_t phase) {
  const float t = __builtin_amdgcn_exp2f(-F16_LOG2E * wv);
  const float e = __builtin_amdgcn_exp2f(-F16_DECAY_LOG2 * __builtin_amdgcn_rcpf(1.0f + t));
  return f16_rn(e - 1.0f + f16_dither(phase));
}

// 16-byte LDS row read -> 4 half pairs
__device__ __forceinline__ void lds_h2x4(const _Float16* p, h2 (&o)[4]) {
  const uint4 u = *reinterpret_cast<const uint4*>(p);
  o[0] = h2_bits(u.x); o[1] = h2_bits(u.y); o[2] = h2_bits(u.z); o[3] = h2_bits(u.w);
}

// Head state [64][64] fp16 at g <-> s_st (row stride F16_RS) with coalesced
// 16-byte accesses by NT threads: thread t, pass q moves the 8 halves of 16-byte
// chunk c = q NT + t, row c/8, column 8(c%8).
template <int NT = 64>
__device__ __forceinline__ void f16_state_in(const _Float16* g, _Float16* s_st, int t) {
  uint4 v[512 / NT];
#pragma unroll
  for (int q = 0; q < 512 / NT; ++q) v[q] = reinterpret_cast<const uint4*>(g)[q * NT + t];
#pragma unroll
  for (int q = 0; q < 512 / NT; ++q) {
    const int c = q * NT + t;
    *reinterpret_cast<uint4*>(s_st + (c >> 3) * F16_RS + (c & 7) * 8) = v[q];
  }
}
template <int NT = 64>
__device__ __forceinline__ void f16_state_out(_Float16* g, const _Float16* s_st, int t) {
  uint4 v[512 / NT];
#pragma unroll
  for (int q = 0; q < 512 / NT; ++q) {
    const int c = q * NT + t;
    v[q] = *reinterpret_cast<const uint4*>(s_st + (c >> 3) * F16_RS + (c & 7) * 8);
  }
#pragma unroll
  for (int q = 0; q < 512 / NT; ++q) reinterpret_cast<uint4*>(g)[q * NT + t] = v[q];
}
// the lane's own row (row `lane`) <-> 32 half pairs
__device__ __forceinline__ void f16_row_get(const _Float16* s_st, int lane, h2 (&s)[32]) {
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    h2 q[4];
    lds_h2x4(s_st + lane * F16_RS + m * 8, q);
    s[4 * m] = q[0]; s[4 * m + 1] = q[1]; s[4 * m + 2] = q[2]; s[4 * m + 3] = q[3];
  }
}
__device__ __forceinline__ void f16_row_put(_Float16* s_st, int lane, const h2 (&s)[32]) {
#pragma unroll
  for (int m = 0; m < 8; ++m)
    *reinterpret_cast<uint4*>(s_st + lane * F16_RS + m * 8) =
        make_uint4(h2_u32(s[4 * m]), h2_u32(s[4 * m + 1]), h2_u32(s[4 * m + 2]), h2_u32(s[4 * m + 3]));
}

// 64 halves of a token vector in LDS -> 32 half pairs
__device__ __forceinline__ void lds_h2x32(const _Float16* p, h2 (&o)[32]) {
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    h2 q[4];
    lds_h2x4(p + 8 * m, q);
    o[4 * m] = q[0]; o[4 * m + 1] = q[1]; o[4 * m + 2] = q[2]; o[4 * m + 3] = q[3];
  }
}

// sa = S[row,:] . (-kk): even and odd key columns in two fp16 chains, then added
__device__ __forceinline__ _Float16 f16_row_sa(const h2 (&s)[32], const h2 (&n)[32]) {
  h2 sa2 = {(_Float16)0.0f, (_Float16)0.0f};
#pragma unroll
  for (int j = 0; j < 32; ++j) sa2 = pk_fma(n[j], s[j], sa2);
  return sa2.x + sa2.y;
}

// The row update and readout given sa, on the token's r, wd, k, kk*a as half
// pairs; vi = v[row].  Returns y[row].
__device__ __forceinline__ _Float16 f16_row_update(h2 (&s)[32], _Float16 sa, const h2 (&r2)[32],
                                                   const h2 (&w2)[32], const h2 (&k2)[32], const h2 (&b2)[32],
                                                   _Float16 vi) {
  const h2 sab = {sa, sa};
  const h2 vv = {vi, vi};
  h2 y2 = {(_Float16)0.0f, (_Float16)0.0f};
#pragma unroll
  for (int j = 0; j < 32; ++j) {
    h2 x = s[j];
    x = pk_fma(x, w2[j], pk_fma(k2[j], vv, pk_fma(sab, b2[j], x)));
    s[j] = x;
    y2 = pk_fma(x, r2[j], y2);
  }
  return y2.x + y2.y;
}

// Pairs 4m .. 4m+3 of a token vector in LDS -> the same pairs of o (m is a
// constant once the callers' loops are unrolled)
__device__ __forceinline__ void lds_group(const _Float16* p, int m, h2 (&o)[32]) {
  h2 q[4];
  lds_h2x4(p + 8 * m, q);
  o[4 * m] = q[0]; o[4 * m + 1] = q[1]; o[4 * m + 2] = q[2]; o[4 * m + 3] = q[3];
}
template <int M0, int M1>
__device__ __forceinline__ void lds_pairs(const _Float16* p, h2 (&o)[32]) {
#pragma unroll
  for (int m = M0; m < M1; ++m) lds_group(p, m, o);
}
// The update operands b, k, wd of pairs 4*M0 .. 4*M1-1, group by group in the
// order the update consumes them.  vec: a token's r; vector q at vec + q*stride.
template <int M0, int M1>
__device__ __forceinline__ void lds_bkw(const _Float16* vec, int stride, h2 (&b2)[32], h2 (&k2)[32],
                                        h2 (&w2)[32]) {
#pragma unroll
  for (int m = M0; m < M1; ++m) {
    lds_group(vec + 4 * stride, m, b2);
    lds_group(vec + 2 * stride, m, k2);
    lds_group(vec + 1 * stride, m, w2);
  }
}
// pairs J0 .. J1-1 of the state update (no readout), written four pairs at a
// stage so that no FMA directly follows the one it depends on
template <int J0, int J1>
__device__ __forceinline__ void f16_update_pairs(h2 (&s)[32], h2 sab, h2 vv, const h2 (&w2)[32],
                                                 const h2 (&k2)[32], const h2 (&b2)[32]) {
#pragma unroll
  for (int j = J0; j < J1; j += 4) {
    h2 u[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) u[q] = pk_fma(sab, b2[j + q], s[j + q]);
#pragma unroll
    for (int q = 0; q < 4; ++q) u[q] = pk_fma(k2[j + q], vv, u[q]);
#pragma unroll
    for (int q = 0; q < 4; ++q) s[j + q] = pk_fma(s[j + q], w2[j + q], u[q]);
  }
}
// Two independent fp16 chains over the updated row: this token's readout
// y = S'.r and the next token's sa = S'.(-kk), interleaved step by step.
__device__ __forceinline__ void f16_row_y_sa(const h2 (&s)[32], const h2 (&r2)[32], const h2 (&n)[32],
                                             _Float16& y, _Float16& sa) {
  h2 y2 = {(_Float16)0.0f, (_Float16)0.0f};
  h2 sa2 = {(_Float16)0.0f, (_Float16)0.0f};
#pragma unroll
  for (int j = 0; j < 32; ++j) {
    y2 = pk_fma(s[j], r2[j], y2);
    sa2 = pk_fma(n[j], s[j], sa2);
  }
  y = y2.x + y2.y;
  sa = sa2.x + sa2.y;
}
// s_waitcnt lgkmcnt(0) (vmcnt and expcnt left at their maxima)
__device__ __forceinline__ void wait_lds_all() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// ---------------------------------------------------------------- decode
// One token from raw projections, then the per-head GroupNorm, bonus and gate
// in fp32 (rwkv7_hf/native_wkv_fp16.py:200-336):
//   kk = fp16(normalize(k_raw * k_k)),  k = fp16(k_raw * (1 + (a - 1) k_a)),
//   b = fp16(kk * a),  out = (GN(y) * gn_w + gn_b + (sum r k r_k) v) * g.
// v_mode (an extension of this build): 1 copies v into v_first (layer 0);
// 2 first forms v + (v_first - v) * v_gate with an fp16 rounding after each
// operation, the values the reference's fp16 torch form gives
// (rwkv7_hf/native_jit_decode.py:762-766).
__device__ __forceinline__ _Float16 f16_v_mix(_Float16 vh, _Float16* v_first, int64_t e, float v_gate, int v_mode) {
  if (v_mode == 1) {
    v_first[e] = vh;
  } else if (v_mode == 2) {
    // three roundings, as three fp16 tensor operations give
    const _Float16 d = f16_rn((float)v_first[e] - (float)vh);
    const _Float16 m = f16_rn((float)d * v_gate);
    vh = f16_rn((float)vh + (float)m);
  }
  return vh;
}

// The head's update by one wave: lane i = channel i = state row i, whose row
// is in s_st (written by this wave, or by the workgroup before a barrier);
// leaves the updated row in s_st and returns out[i].  vh is v after the
// interpolation; the other inputs are the lane's channel values.
__device__ __forceinline__ _Float16 f16_decode_head(int i, _Float16 rh, float wr, float kr, _Float16 vh, float af,
                                                    float gf, float kkw, float kaw, float rkw, float gw, float gb,
                                                    uint32_t phase, float eps, _Float16* s_st,
                                                    _Float16 (&s_vec)[5][F16_N]) {
  const float kku = kr * kkw;
  const float kkv = kku / fmaxf(sqrtf(wave_sum(kku * kku)), 1.0e-12f);
  const _Float16 kh = f16_rn(kr * fmaf(af, kaw, 1.0f - kaw));
  const _Float16 kkh = f16_rn(kkv);
  s_vec[0][i] = rh;
  s_vec[1][i] = f16_decay_delta(wr, phase);
  s_vec[2][i] = kh;
  s_vec[3][i] = -kkh;
  s_vec[4][i] = f16_rn((float)kkh * af);
  // every lane's LDS writes (the vectors, and the state rows when this wave
  // staged them) are complete before any lane reads another's
  wait_lds_all();
  __builtin_amdgcn_wave_barrier();

  h2 s[32], n[32], r2[32], w2[32], k2[32], b2[32];
  f16_row_get(s_st, i, s);
  lds_h2x32(s_vec[3], n);
  lds_h2x32(s_vec[0], r2);
  lds_h2x32(s_vec[1], w2);
  lds_h2x32(s_vec[2], k2);
  lds_h2x32(s_vec[4], b2);
  const _Float16 yh = f16_row_update(s, f16_row_sa(s, n), r2, w2, k2, b2, vh);
  f16_row_put(s_st, i, s);

  const float y = (float)yh;
  const float mean = wave_sum(y) * (1.0f / F16_N);
  const float cen = y - mean;
  const float var = wave_sum(cen * cen) * (1.0f / F16_N);
  const float corr = wave_sum((float)rh * (float)kh * rkw);
  return f16_rn((cen * rsqrtf(var + eps) * gw + gb + corr * (float)vh) * gf);
}

__global__ __launch_bounds__(64) void wkv7_f16_decode_kernel(
    const _Float16* __restrict__ r, const _Float16* __restrict__ w_raw, const _Float16* __restrict__ k_raw,
    const _Float16* __restrict__ v, const _Float16* __restrict__ a, _Float16* __restrict__ state,
    const _Float16* __restrict__ g, const _Float16* __restrict__ k_k, const _Float16* __restrict__ k_a,
    const _Float16* __restrict__ r_k, const _Float16* __restrict__ gn_w, const _Float16* __restrict__ gn_b,
    const int* __restrict__ elapsed, _Float16* __restrict__ out, _Float16* __restrict__ v_first,
    const _Float16* __restrict__ v_gate, int v_mode, int H, float eps) {
  __shared__ __align__(16) _Float16 s_st[F16_N * F16_RS];
  __shared__ __align__(16) _Float16 s_vec[5][F16_N];  // r, wd, k, -kk, kk*a

  const int bh = blockIdx.x;
  const int b = bh / H;
  const int h = bh - b * H;
  const int i = threadIdx.x;
  const int64_t e = (int64_t)bh * F16_N + i;
  const int pc = h * F16_N + i;
  _Float16* sg = state + (int64_t)bh * F16_N * F16_N;

  f16_state_in(sg, s_st, i);
  const _Float16 vh = f16_v_mix(v[e], v_first, e, v_mode == 2 ? (float)v_gate[e] : 0.f, v_mode);
  out[e] = f16_decode_head(i, r[e], (float)w_raw[e], (float)k_raw[e], vh, (float)a[e], (float)g[e], (float)k_k[pc],
                           (float)k_a[pc], (float)r_k[pc], (float)gn_w[pc], (float)gn_b[pc],
                           (uint32_t)elapsed[b] + (uint32_t)pc, eps, s_st, s_vec);
  __syncthreads();
  f16_state_out(sg, s_st, i);
}

// The same update with the W/A/G/V LoRA up projections inside (the second
// half of fused_wavg_lora, rwkv7_hf/fused_lora.py:706): four waves compute the
// head's 64 channels of w_raw, a, g and v_gate (dl_up, decode_lora.h) while the
// fp16 state and the channel inputs load, then wave 0 updates the head.
template <int ZB>
__global__ __launch_bounds__(256) void wkv7_f16_decode_lora_kernel(
    const _Float16* __restrict__ r, const _Float16* __restrict__ k_raw, const _Float16* __restrict__ v,
    const DecLora LA, _Float16* __restrict__ state, const _Float16* __restrict__ k_k,
    const _Float16* __restrict__ k_a, const _Float16* __restrict__ r_k, const _Float16* __restrict__ gn_w,
    const _Float16* __restrict__ gn_b, const int* __restrict__ elapsed, _Float16* __restrict__ out,
    _Float16* __restrict__ v_first, int v_mode, int H, float eps) {
  __shared__ __align__(16) _Float16 s_st[F16_N * F16_RS];
  __shared__ __align__(16) _Float16 s_vec[5][F16_N];
  __shared__ __align__(16) float s_mid[4][DL_MAXR];
  __shared__ float s_lo[4][DL_HEAD];

  const int bh = blockIdx.x;
  const int b = bh / H;
  const int h = bh - b * H;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int64_t e = (int64_t)bh * F16_N + lane;
  const int pc = h * F16_N + lane;
  _Float16* sg = state + (int64_t)bh * F16_N * F16_N;

  // The state and channel loads are issued behind the first LoRA partials and
  // land in registers, so the up weights' loads follow without a wait; the
  // state goes to LDS once dl_up is done.
  uint4 sv0, sv1;
  _Float16 rh, kh, vh, vfh;
  float kkw, kaw, rkw, gw, gb;
  uint32_t phase;
  dl_up<__half, ZB>(LA, b, h, H, wave, lane, s_mid, s_lo, [&] {
    sv0 = reinterpret_cast<const uint4*>(sg)[tid];
    sv1 = reinterpret_cast<const uint4*>(sg)[256 + tid];
    // channel `lane` of this head (every wave loads; wave 0 uses them)
    rh = r[e];
    kh = k_raw[e];
    vh = v[e];
    vfh = v_mode == 2 ? v_first[e] : (_Float16)0.0f;
    kkw = (float)k_k[pc];
    kaw = (float)k_a[pc];
    rkw = (float)r_k[pc];
    gw = (float)gn_w[pc];
    gb = (float)gn_b[pc];
    phase = (uint32_t)elapsed[b] + (uint32_t)pc;
  });
  *reinterpret_cast<uint4*>(s_st + (tid >> 3) * F16_RS + (tid & 7) * 8) = sv0;
  *reinterpret_cast<uint4*>(s_st + ((256 + tid) >> 3) * F16_RS + (tid & 7) * 8) = sv1;
  __syncthreads();  // the state rows and the four up projections are in LDS
  if (wave == 0) {
    _Float16 vm = vh;
    if (v_mode == 1) {
      v_first[e] = vh;
    } else if (v_mode == 2) {
      const _Float16 d = f16_rn((float)vfh - (float)vh);
      const _Float16 m = f16_rn((float)d * s_lo[3][lane]);
      vm = f16_rn((float)vh + (float)m);
    }
    out[e] = f16_decode_head(lane, rh, s_lo[0][lane], (float)kh, vm, s_lo[1][lane], s_lo[2][lane], kkw, kaw, rkw,
                             gw, gb, phase, eps, s_st, s_vec);
  }
  __syncthreads();
  f16_state_out<256>(sg, s_st, tid);
}

__global__ __launch_bounds__(64) void wkv7_f16_advance_kernel(int* __restrict__ elapsed, int B) {
  const int b = blockIdx.x * 64 + threadIdx.x;
  if (b < B) elapsed[b] += 1;
}

// -------------------------------------------------------------- sequence
// T tokens of prepared vectors [B, T, H, 64] (w raw, + w0 when given; -kk and
// kk*a precomputed) with the state resident in registers
// (rwkv7_hf/native_wkv_fp16.py:338-436).  Slabs of F16_SLAB tokens are loaded
// two slabs ahead into registers (lane l: vector q, token l/8, channels
// 8(l%8)..+7 — one 16-byte load per vector) and staged in LDS one slab ahead,
// the slab's decay deltas are computed at staging, and each token's output
// row is stored as it is produced.
template <bool ADD_W0>
__global__ __launch_bounds__(64) void wkv7_f16_sequence_kernel(
    const _Float16* __restrict__ r, const _Float16* __restrict__ w, const _Float16* __restrict__ w0,
    const _Float16* __restrict__ k, const _Float16* __restrict__ v, const _Float16* __restrict__ nkk,
    const _Float16* __restrict__ kka, _Float16* __restrict__ state, _Float16* __restrict__ out,
    const int* __restrict__ elapsed, int T, int H) {
  __shared__ __align__(16) _Float16 s_st[F16_N * F16_RS];
  // [buffer][vector: r, wd, k, -kk, kk*a, v][token][channel]
  __shared__ __align__(16) _Float16 s_slab[2][6][F16_SLAB][F16_N];

  const int bh = blockIdx.x;
  const int b = bh / H;
  const int h = bh - b * H;
  const int lane = threadIdx.x;
  _Float16* sg = state + (int64_t)bh * F16_N * F16_N;

  // per-(b, h) descriptors over tokens 0..T-1 of this head
  const int64_t first = ((int64_t)b * T * H + h) * F16_N;
  const uint32_t tok_bytes = (uint32_t)H * F16_N * 2u;
  const uint32_t span = (uint32_t)(T - 1) * tok_bytes + F16_N * 2u;
  const __amdgpu_buffer_rsrc_t rs[6] = {make_rsrc(r + first, span),   make_rsrc(w + first, span),
                                        make_rsrc(k + first, span),   make_rsrc(nkk + first, span),
                                        make_rsrc(kka + first, span), make_rsrc(v + first, span)};
  const int lt = lane >> 3;       // token within the slab this lane loads
  const int lc = (lane & 7) * 8;  // first channel this lane loads
  float w0v[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) w0v[u] = ADD_W0 ? (float)w0[h * F16_N + lc + u] : 0.0f;
  const uint32_t phase0 = (uint32_t)elapsed[b] + (uint32_t)(h * F16_N + lc);

  u32x4 L[6];
  auto load_slab = [&](int t0) {
    const int t = t0 + lt;
    const uint32_t off = t < T ? (uint32_t)t * tok_bytes + (uint32_t)lc * 2u : BUF_OOB;
#pragma unroll
    for (int q = 0; q < 6; ++q) L[q] = buf_ld16(rs[q], off);
  };
  auto stage_slab = [&](int buf, int t0) {
#pragma unroll
    for (int q = 0; q < 6; ++q) {
      if (q == 1) {
        uint32_t d[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const h2 x = h2_bits(L[1][u]);
          const uint32_t ph = phase0 + (uint32_t)(t0 + lt) + 2u * u;
          const h2 o = {f16_decay_delta((float)x.x + w0v[2 * u], ph),
                        f16_decay_delta((float)x.y + w0v[2 * u + 1], ph + 1u)};
          d[u] = h2_u32(o);
        }
        *reinterpret_cast<uint4*>(&s_slab[buf][1][lt][lc]) = make_uint4(d[0], d[1], d[2], d[3]);
      } else {
        *reinterpret_cast<u32x4*>(&s_slab[buf][q][lt][lc]) = L[q];
      }
    }
  };

  f16_state_in(sg, s_st, lane);
  load_slab(0);
  __syncthreads();
  h2 s[32];
  f16_row_get(s_st, lane, s);
  stage_slab(0, 0);
  if (F16_SLAB < T) {
    load_slab(F16_SLAB);
    stage_slab(1, F16_SLAB);
    if (2 * F16_SLAB < T) load_slab(2 * F16_SLAB);
  }
  __syncthreads();

  // Token t lives in buffer (t / F16_SLAB) & 1, row t % F16_SLAB.  While slab
  // S is processed, slab S + 1 is staged in the other buffer (and slab S + 2
  // is in flight in registers).
  //
  // Per token the readout chain y(t) = S'(t).r(t) runs interleaved with the
  // next token's chain sa(t+1) = S'(t).(-kk(t+1)): two independent chains
  // keep the packed FMA pipeline busy where one would stall on every step.
  // LDS reads are issued at fixed points (scheduling barriers) so that each
  // consumer waits on at most 15 younger reads (the LDS wait counter's range):
  //   [b,k,wd pairs 0-15 of t in registers]  read b,k,wd pairs 16-31
  //   update pairs 0-15   | read r(t), -kk(t+1)
  //   update pairs 16-31  | read b,k,wd pairs 0-15 and v of t+1
  //   y(t) / sa(t+1) chains; store y(t)
  constexpr int VSTRIDE = F16_SLAB * F16_N;  // halves between vectors of one buffer
  h2 n[32], r2[32], w2[32], k2[32], b2[32];
  _Float16 sa, vi;
  lds_h2x32(s_slab[0][3][0], n);
  wait_lds_all();
  {
    h2 sa2 = {(_Float16)0.0f, (_Float16)0.0f};
#pragma unroll
    for (int j = 0; j < 32; ++j) sa2 = pk_fma(n[j], s[j], sa2);
    sa = sa2.x + sa2.y;
  }
  lds_bkw<0, 4>(&s_slab[0][0][0][0], VSTRIDE, b2, k2, w2);
  vi = s_slab[0][5][0][lane];
  _Float16* orow = out + first + lane;
  for (int t = 0; t < T; ++t) {
    const int buf = (t / F16_SLAB) & 1;
    const int tt = t % F16_SLAB;
    if (tt == 0 && t > 0) {
      if (t + F16_SLAB < T) {
        stage_slab(buf ^ 1, t + F16_SLAB);
        if (t + 2 * F16_SLAB < T) load_slab(t + 2 * F16_SLAB);
      }
      __syncthreads();
    }
    const _Float16* vec = &s_slab[buf][0][tt][0];
    const int tn = min(t + 1, T - 1);
    const _Float16* vnext = &s_slab[(tn / F16_SLAB) & 1][0][tn % F16_SLAB][0];
    lds_bkw<4, 8>(vec, VSTRIDE, b2, k2, w2);
    __builtin_amdgcn_sched_barrier(0);
    const h2 sab = {sa, sa};
    const h2 vv = {vi, vi};
    f16_update_pairs<0, 16>(s, sab, vv, w2, k2, b2);
    __builtin_amdgcn_sched_barrier(0);
    lds_pairs<0, 8>(vec, r2);
    lds_pairs<0, 8>(vnext + 3 * VSTRIDE, n);
    __builtin_amdgcn_sched_barrier(0);
    f16_update_pairs<16, 32>(s, sab, vv, w2, k2, b2);
    __builtin_amdgcn_sched_barrier(0);
    lds_bkw<0, 4>(vnext, VSTRIDE, b2, k2, w2);
    vi = vnext[5 * VSTRIDE + lane];
    __builtin_amdgcn_sched_barrier(0);
    _Float16 y;
    f16_row_y_sa(s, r2, n, y, sa);
    orow[(int64_t)t * H * F16_N] = y;
  }

  f16_row_put(s_st, lane, s);
  __syncthreads();
  f16_state_out(sg, s_st, lane);
}

}  // namespace rwkv7mi

using namespace rwkv7mi;

namespace {
bool f16_aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }
}  // namespace

extern "C" int rwkv7mi_wkv7_fp16_decode_output_prepare_raw(
    const void* r, const void* w_raw, const void* k_raw, const void* v, const void* a, void* state,
    const void* g, const void* k_k, const void* k_a, const void* r_k, const void* gn_w, const void* gn_b,
    int32_t* elapsed, int advance_elapsed, void* out, void* v_first, const void* v_gate, int v_mode, int64_t B,
    int64_t H, int64_t N, float eps, void* stream) {
  if (N != F16_N) return fail(RWKV7MI_EINVAL, "wkv7 fp16 decode: head size must be 64");
  if (B < 0 || H <= 0) return fail(RWKV7MI_EINVAL, "wkv7 fp16 decode: bad B/H");
  if (B == 0) return RWKV7MI_OK;
  if (B * H > INT32_MAX) return fail(RWKV7MI_EINVAL, "wkv7 fp16 decode: too many heads");
  if (!r || !w_raw || !k_raw || !v || !a || !state || !g || !k_k || !k_a || !r_k || !gn_w || !gn_b ||
      !elapsed || !out)
    return fail(RWKV7MI_EINVAL, "wkv7 fp16 decode: null pointer");
  if (!f16_aligned16(state)) return fail(RWKV7MI_EINVAL, "wkv7 fp16 decode: state must be 16-byte aligned");
  if (v_mode < 0 || v_mode > 2) return fail(RWKV7MI_EINVAL, "wkv7 fp16 decode: v_mode must be 0, 1 or 2");
  if ((v_mode >= 1 && !v_first) || (v_mode == 2 && !v_gate))
    return fail(RWKV7MI_EINVAL, "wkv7 fp16 decode: v_mode 1 needs v_first, 2 needs v_first and v_gate");
  hipStream_t st = as_stream(stream);
  hipLaunchKernelGGL(wkv7_f16_decode_kernel, dim3((unsigned)(B * H)), dim3(64), 0, st, (const _Float16*)r,
                     (const _Float16*)w_raw, (const _Float16*)k_raw, (const _Float16*)v, (const _Float16*)a,
                     (_Float16*)state, (const _Float16*)g, (const _Float16*)k_k, (const _Float16*)k_a,
                     (const _Float16*)r_k, (const _Float16*)gn_w, (const _Float16*)gn_b, (const int*)elapsed,
                     (_Float16*)out, (_Float16*)v_first, (const _Float16*)v_gate, v_mode, (int)H, eps);
  int rc = check_launch("wkv7_f16_decode_kernel");
  if (rc != RWKV7MI_OK || !advance_elapsed) return rc;
  // Every head of the step reads elapsed[b] before it moves: the increment is
  // a second launch on the same stream.
  hipLaunchKernelGGL(wkv7_f16_advance_kernel, dim3((unsigned)((B + 63) / 64)), dim3(64), 0, st, (int*)elapsed,
                     (int)B);
  return check_launch("wkv7_f16_advance_kernel");
}

extern "C" int rwkv7mi_wkv7_fp16_decode_lora_output_prepare(
    const void* r, const void* k_raw, const void* v, const float* lora_part, int64_t nprob, const int64_t* ranks,
    const void* const* w_up, const void* const* b_up, const int* act_down, const int* act_up, int64_t D,
    int64_t lora_splits, void* state, const void* k_k, const void* k_a, const void* r_k, const void* gn_w,
    const void* gn_b, int32_t* elapsed, int advance_elapsed, void* out, void* v_first, int v_mode, int64_t B,
    int64_t H, int64_t N, float eps, void* stream) {
  if (N != F16_N) return fail(RWKV7MI_EINVAL, "wkv7 fp16 decode lora: head size must be 64");
  if (B < 0 || H <= 0 || D <= 0) return fail(RWKV7MI_EINVAL, "wkv7 fp16 decode lora: bad B/H/D");
  if (B == 0) return RWKV7MI_OK;
  if (B > LORA_ROWS) return fail(RWKV7MI_EINVAL, "wkv7 fp16 decode lora: at most 64 rows");
  if (!r || !k_raw || !v || !state || !k_k || !k_a || !r_k || !gn_w || !gn_b || !elapsed || !out)
    return fail(RWKV7MI_EINVAL, "wkv7 fp16 decode lora: null pointer");
  if (!f16_aligned16(state)) return fail(RWKV7MI_EINVAL, "wkv7 fp16 decode lora: state must be 16-byte aligned");
  if (v_mode < 0 || v_mode > 2) return fail(RWKV7MI_EINVAL, "wkv7 fp16 decode lora: v_mode must be 0, 1 or 2");
  if (v_mode == 2 && nprob != 4) return fail(RWKV7MI_EINVAL, "wkv7 fp16 decode lora: v_mode 2 needs the v LoRA");
  if (v_mode != 0 && !v_first) return fail(RWKV7MI_EINVAL, "wkv7 fp16 decode lora: v_mode needs v_first");
  DecLora la;
  if (int rc = dl_build(la, "wkv7 fp16 decode lora", lora_part, nprob, ranks, w_up, b_up, act_down, act_up, D,
                        lora_splits, B))
    return rc;
  hipStream_t st = as_stream(stream);
  // sums that arrive whole (one split) need one partial load per lane, not a batch
  if (la.ks == 1)
    hipLaunchKernelGGL((wkv7_f16_decode_lora_kernel<1>), dim3((unsigned)(B * H)), dim3(256), 0, st,
                       (const _Float16*)r, (const _Float16*)k_raw, (const _Float16*)v, la, (_Float16*)state,
                       (const _Float16*)k_k, (const _Float16*)k_a, (const _Float16*)r_k, (const _Float16*)gn_w,
                       (const _Float16*)gn_b, (const int*)elapsed, (_Float16*)out, (_Float16*)v_first, v_mode,
                       (int)H, eps);
  else
    hipLaunchKernelGGL((wkv7_f16_decode_lora_kernel<DL_ZB>), dim3((unsigned)(B * H)), dim3(256), 0, st,
                       (const _Float16*)r, (const _Float16*)k_raw, (const _Float16*)v, la, (_Float16*)state,
                       (const _Float16*)k_k, (const _Float16*)k_a, (const _Float16*)r_k, (const _Float16*)gn_w,
                       (const _Float16*)gn_b, (const int*)elapsed, (_Float16*)out, (_Float16*)v_first, v_mode,
                       (int)H, eps);
  int rc = check_launch("wkv7_f16_decode_lora_kernel");
  if (rc != RWKV7MI_OK || !advance_elapsed) return rc;
  hipLaunchKernelGGL(wkv7_f16_advance_kernel, dim3((unsigned)((B + 63) / 64)), dim3(64), 0, st, (int*)elapsed,
                     (int)B);
  return check_launch("wkv7_f16_advance_kernel");
}

extern "C" int rwkv7mi_wkv7_fp16_sequence(const void* r, const void* w, const void* w0, const void* k,
                                          const void* v, const void* neg_kk, const void* kka, void* state,
                                          const int32_t* elapsed, void* out, int64_t B, int64_t T, int64_t H,
                                          int64_t N, void* stream) {
  if (N != F16_N) return fail(RWKV7MI_EINVAL, "wkv7 fp16 sequence: head size must be 64");
  if (B < 0 || T <= 0 || H <= 0) return fail(RWKV7MI_EINVAL, "wkv7 fp16 sequence: bad B/T/H (T must be >= 1)");
  if (B == 0) return RWKV7MI_OK;
  if (B * H > INT32_MAX) return fail(RWKV7MI_EINVAL, "wkv7 fp16 sequence: too many heads");
  // one head's token span is addressed by a 32-bit buffer offset
  if ((T - 1) * H * F16_N * 2 + F16_N * 2 >= (int64_t)BUF_OOB)
    return fail(RWKV7MI_EINVAL, "wkv7 fp16 sequence: T*H too large (one head's span must stay under 2 GiB)");
  if (!r || !w || !k || !v || !neg_kk || !kka || !state || !elapsed || !out)
    return fail(RWKV7MI_EINVAL, "wkv7 fp16 sequence: null pointer");
  for (const void* p : {r, w, k, v, neg_kk, kka, (const void*)state})
    if (!f16_aligned16(p)) return fail(RWKV7MI_EINVAL, "wkv7 fp16 sequence: inputs and state must be 16-byte aligned");
  hipStream_t st = as_stream(stream);
  if (w0) {
    hipLaunchKernelGGL((wkv7_f16_sequence_kernel<true>), dim3((unsigned)(B * H)), dim3(64), 0, st,
                       (const _Float16*)r, (const _Float16*)w, (const _Float16*)w0, (const _Float16*)k,
                       (const _Float16*)v, (const _Float16*)neg_kk, (const _Float16*)kka, (_Float16*)state,
                       (_Float16*)out, (const int*)elapsed, (int)T, (int)H);
  } else {
    hipLaunchKernelGGL((wkv7_f16_sequence_kernel<false>), dim3((unsigned)(B * H)), dim3(64), 0, st,
                       (const _Float16*)r, (const _Float16*)w, nullptr, (const _Float16*)k, (const _Float16*)v,
                       (const _Float16*)neg_kk, (const _Float16*)kka, (_Float16*)state, (_Float16*)out,
                       (const int*)elapsed, (int)T, (int)H);
  }
  return check_launch("wkv7_f16_sequence_kernel");
}
