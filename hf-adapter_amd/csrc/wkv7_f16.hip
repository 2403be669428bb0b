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

// 2^-41 * int32(0x9E3779B9 * phase)
__device__ __forceinline__ float f16_dither(uint32_t phase) {
  return 0x1p-41f * (float)(int32_t)(0x9E3779B9u * phase);
}

// exp(-e^-1/2 sigmoid(wv)) - 1 + dither, in fp32, rounded to fp16
__device__ __forceinline__ _Float16 f16_decay_delta(float wv, uint32_t phase) {
  const float t = exp2f(-F16_LOG2E * wv);
  const float d = exp2f(-F16_DECAY_LOG2 / (1.0f + t)) - 1.0f + f16_dither(phase);
  return (_Float16)d;
}

// 16-byte LDS row read -> 4 half pairs
__device__ __forceinline__ void lds_h2x4(const _Float16* p, h2 (&o)[4]) {
  const uint4 u = *reinterpret_cast<const uint4*>(p);
  o[0] = h2_bits(u.x); o[1] = h2_bits(u.y); o[2] = h2_bits(u.z); o[3] = h2_bits(u.w);
}

// Head state [64][64] fp16 at g -> s_st (row stride F16_RS) with coalesced
// 16-byte loads: lane l, pass q moves 8 halves of row 8q + l/8 at column 8(l%8).
__device__ __forceinline__ void f16_state_in(const _Float16* g, _Float16* s_st, int lane) {
  uint4 t[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) t[q] = reinterpret_cast<const uint4*>(g)[q * 64 + lane];
#pragma unroll
  for (int q = 0; q < 8; ++q)
    *reinterpret_cast<uint4*>(s_st + (q * 8 + (lane >> 3)) * F16_RS + (lane & 7) * 8) = t[q];
}
__device__ __forceinline__ void f16_state_out(_Float16* g, const _Float16* s_st, int lane) {
  uint4 t[8];
#pragma unroll
  for (int q = 0; q < 8; ++q)
    t[q] = *reinterpret_cast<const uint4*>(s_st + (q * 8 + (lane >> 3)) * F16_RS + (lane & 7) * 8);
#pragma unroll
  for (int q = 0; q < 8; ++q) reinterpret_cast<uint4*>(g)[q * 64 + lane] = t[q];
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

// One token on the lane's row.  rv/wv/kv/nv/bv: the token's r, wd, k, -kk,
// kk*a (64 halves each, LDS, read as broadcasts); vi = v[row].  Returns y[row].
__device__ __forceinline__ _Float16 f16_row_step(h2 (&s)[32], const _Float16* rv, const _Float16* wv,
                                                 const _Float16* kv, const _Float16* nv, const _Float16* bv,
                                                 _Float16 vi) {
  h2 sa2 = {(_Float16)0.0f, (_Float16)0.0f};
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    h2 n[4];
    lds_h2x4(nv + 8 * m, n);
#pragma unroll
    for (int u = 0; u < 4; ++u) sa2 = pk_fma(n[u], s[4 * m + u], sa2);
  }
  const _Float16 sa = sa2.x + sa2.y;
  const h2 sab = {sa, sa};
  const h2 vv = {vi, vi};
  h2 y2 = {(_Float16)0.0f, (_Float16)0.0f};
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    h2 w4[4], k4[4], b4[4], r4[4];
    lds_h2x4(wv + 8 * m, w4);
    lds_h2x4(kv + 8 * m, k4);
    lds_h2x4(bv + 8 * m, b4);
    lds_h2x4(rv + 8 * m, r4);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      h2 x = s[4 * m + u];
      x = pk_fma(x, w4[u], pk_fma(k4[u], vv, pk_fma(sab, b4[u], x)));
      s[4 * m + u] = x;
      y2 = pk_fma(x, r4[u], y2);
    }
  }
  return y2.x + y2.y;
}

// ---------------------------------------------------------------- decode
// One token from raw projections, then the per-head GroupNorm, bonus and gate
// in fp32 (rwkv7_hf/native_wkv_fp16.py:200-336):
//   kk = fp16(normalize(k_raw * k_k)),  k = fp16(k_raw * (1 + (a - 1) k_a)),
//   b = fp16(kk * a),  out = (GN(y) * gn_w + gn_b + (sum r k r_k) v) * g.
__global__ __launch_bounds__(64) void wkv7_f16_decode_kernel(
    const _Float16* __restrict__ r, const _Float16* __restrict__ w_raw, const _Float16* __restrict__ k_raw,
    const _Float16* __restrict__ v, const _Float16* __restrict__ a, _Float16* __restrict__ state,
    const _Float16* __restrict__ g, const _Float16* __restrict__ k_k, const _Float16* __restrict__ k_a,
    const _Float16* __restrict__ r_k, const _Float16* __restrict__ gn_w, const _Float16* __restrict__ gn_b,
    const int* __restrict__ elapsed, _Float16* __restrict__ out, int H, float eps) {
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
  const _Float16 rh = r[e], vh = v[e];
  const float kr = (float)k_raw[e], af = (float)a[e], wr = (float)w_raw[e], gf = (float)g[e];
  const float kkw = (float)k_k[pc], kaw = (float)k_a[pc], rkw = (float)r_k[pc];
  const float gw = (float)gn_w[pc], gb = (float)gn_b[pc];
  const uint32_t phase = (uint32_t)elapsed[b] + (uint32_t)pc;

  const float kku = kr * kkw;
  const float kkv = kku / fmaxf(sqrtf(wave_sum(kku * kku)), 1.0e-12f);
  const _Float16 kh = (_Float16)(kr * fmaf(af, kaw, 1.0f - kaw));
  const _Float16 kkh = (_Float16)kkv;
  s_vec[0][i] = rh;
  s_vec[1][i] = f16_decay_delta(wr, phase);
  s_vec[2][i] = kh;
  s_vec[3][i] = -kkh;
  s_vec[4][i] = (_Float16)((float)kkh * af);
  __syncthreads();

  h2 s[32];
  f16_row_get(s_st, i, s);
  const _Float16 yh = f16_row_step(s, s_vec[0], s_vec[1], s_vec[2], s_vec[3], s_vec[4], vh);
  f16_row_put(s_st, i, s);

  const float y = (float)yh;
  const float mean = wave_sum(y) * (1.0f / F16_N);
  const float cen = y - mean;
  const float var = wave_sum(cen * cen) * (1.0f / F16_N);
  const float corr = wave_sum((float)rh * (float)kh * rkw);
  out[e] = (_Float16)((cen * rsqrtf(var + eps) * gw + gb + corr * (float)vh) * gf);

  __syncthreads();
  f16_state_out(sg, s_st, i);
}

__global__ __launch_bounds__(64) void wkv7_f16_advance_kernel(int* __restrict__ elapsed, int B) {
  const int b = blockIdx.x * 64 + threadIdx.x;
  if (b < B) elapsed[b] += 1;
}

// -------------------------------------------------------------- sequence
// T tokens of prepared vectors [B, T, H, 64] (w raw, + w0 when given; -kk and
// kk*a precomputed) with the state resident in registers
// (rwkv7_hf/native_wkv_fp16.py:338-436).  Slabs of F16_SLAB tokens are loaded
// one slab ahead (lane l: vector q, token l/8, channels 8(l%8)..+7 — one
// 16-byte load per vector), the slab's decay deltas are computed at staging,
// and each token's output row is stored as it is produced.
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
  if (F16_SLAB < T) load_slab(F16_SLAB);

  _Float16* orow = out + first + lane;
  for (int t0 = 0, buf = 0; t0 < T; t0 += F16_SLAB, buf ^= 1) {
    __syncthreads();  // slab t0 staged; slab t0 - F16_SLAB's buffer is free
    if (t0 + F16_SLAB < T) {
      stage_slab(buf ^ 1, t0 + F16_SLAB);
      if (t0 + 2 * F16_SLAB < T) load_slab(t0 + 2 * F16_SLAB);
    }
    const int nt = min(F16_SLAB, T - t0);
    for (int tt = 0; tt < nt; ++tt) {
      const _Float16 yh = f16_row_step(s, s_slab[buf][0][tt], s_slab[buf][1][tt], s_slab[buf][2][tt],
                                       s_slab[buf][3][tt], s_slab[buf][4][tt], s_slab[buf][5][tt][lane]);
      orow[(int64_t)(t0 + tt) * H * F16_N] = yh;
    }
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
    int32_t* elapsed, int advance_elapsed, void* out, int64_t B, int64_t H, int64_t N, float eps,
    void* stream) {
  if (N != F16_N) return fail(RWKV7MI_EINVAL, "wkv7 fp16 decode: head size must be 64");
  if (B < 0 || H <= 0) return fail(RWKV7MI_EINVAL, "wkv7 fp16 decode: bad B/H");
  if (B == 0) return RWKV7MI_OK;
  if (B * H > INT32_MAX) return fail(RWKV7MI_EINVAL, "wkv7 fp16 decode: too many heads");
  if (!r || !w_raw || !k_raw || !v || !a || !state || !g || !k_k || !k_a || !r_k || !gn_w || !gn_b ||
      !elapsed || !out)
    return fail(RWKV7MI_EINVAL, "wkv7 fp16 decode: null pointer");
  if (!f16_aligned16(state)) return fail(RWKV7MI_EINVAL, "wkv7 fp16 decode: state must be 16-byte aligned");
  hipStream_t st = as_stream(stream);
  hipLaunchKernelGGL(wkv7_f16_decode_kernel, dim3((unsigned)(B * H)), dim3(64), 0, st, (const _Float16*)r,
                     (const _Float16*)w_raw, (const _Float16*)k_raw, (const _Float16*)v, (const _Float16*)a,
                     (_Float16*)state, (const _Float16*)g, (const _Float16*)k_k, (const _Float16*)k_a,
                     (const _Float16*)r_k, (const _Float16*)gn_w, (const _Float16*)gn_b, (const int*)elapsed,
                     (_Float16*)out, (int)H, eps);
  int rc = check_launch("wkv7_f16_decode_kernel");
  if (rc != RWKV7MI_OK || !advance_elapsed) return rc;
  // Every head of the step reads elapsed[b] before it moves: the increment is
  // a second launch on the same stream.
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
