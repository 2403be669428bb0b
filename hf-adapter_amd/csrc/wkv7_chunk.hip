// wkv7 chunked DPLR prefill (gfx950), chunk C = 16, head size 64.
//
// Recurrence (native V x K state, rwkv7_hf/fused_recurrent_update.py:757-783):
//   S_t = S_{t-1} (diag(w_t) + alpha_t beta_t^T) + v_t k_t^T,  y_t = S_t r_t,
//   alpha = -kk, beta = kk * a.
// Per chunk, with g_t = sum_{s<=t} log2 w_s (per key channel j, 0 at the chunk
// start), centre c = g_8, p_t = 2^{g_t - c}, q_t = 1/p_t and the gated rows
//   rc_t = r_t p_t, ac_t = alpha_t p_{t-1}, kc_t = k_t q_t, bc_t = beta_t q_t,
// the 16x16 causal matrices are
//   A_qk = tril(rc kc^T), A_qb = tril(rc bc^T), A_ak = tril(ac kc^T, -1), A_ab = tril(ac bc^T, -1)
// (entry [t,s] = sum_j x_t y_s 2^{g_t - g_s}, every factor kept within 2^+-120),
// and with S' = S0 diag(2^c), T = (I - A_ab)^{-1}:
//   U   = (T ac) S'^T + (T A_ak) V              (u_t = S_{t-1} alpha_t)
//   Y   = rc S'^T + A_qb U + A_qk V
//   S_C = S0 diag(2^{g_C}) + diag(2^{g_C - c}) (bc^T U + kc^T V)   (as S^T)
// — the WY form of the reference's chunk algebra (rwkv7_hf/self_chunk_rwkv7.py:85-134,
// rwkv7_hf/dplr_prefill.py:221-311) arranged so that one set of gated rows
// serves every product and the per-channel scales fold into the state.
//
// Mapping: one 256-lane workgroup per (batch, head).  Wave q owns value rows
// [16q, 16q+16) of the state, held transposed in MFMA accumulator layout
// (4 key tiles x f32x4 per lane); the state never leaves registers.  Products
// run on v_mfma_f32_16x16x{32,16}_bf16 with operands split into bf16 hi + lo
// (hi*hi + hi*lo + lo*hi, ~1e-5 relative) and fp32 accumulation; K = 16
// products are paired into one K = 32 MFMA ([U ; V] as a single operand).
// Per chunk: (A) derive inputs, stage log-decay and V; (B) per-channel gate
// cumsum and the gated rows (+ transposed copies); (C) the four causal
// matrices, one per wave; (D) T by forward substitution on 16 lanes;
// (E) per wave: T ac and T A_ak by MFMA straight into operand layout, then
// U -> Y -> S.  The next chunk's raw inputs are in flight during (C)-(E).
// Limitation: contributions below 2^-120 of a chunk's gate range are dropped.
#include "common.h"

namespace rwkv7mi {

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

constexpr int CH = 16;      // chunk length
constexpr int HD = 64;      // head size
constexpr int PR = HD + 8;  // padded bf16 row [t][j]
constexpr int PT = CH + 4;  // padded bf16 row [j][t]

struct ChunkLDS {
  float lw[CH][HD];                      // log2 decay
  __bf16 vh[CH][PR], vl[CH][PR];         // V [s][i]
  __bf16 rch[CH][PR], rcl[CH][PR];       // rc [t][j]
  __bf16 ach[CH][PR], acl[CH][PR];       // ac [t][j]
  __bf16 kch[CH][PR], kcl[CH][PR];       // kc [t][j]
  __bf16 bch[CH][PR], bcl[CH][PR];       // bc [t][j]
  __bf16 acth[HD][PT], actl[HD][PT];     // ac^T [j][t]
  __bf16 kcth[HD][PT], kctl[HD][PT];     // kc^T
  __bf16 bcth[HD][PT], bctl[HD][PT];     // bc^T
  float amat[4][CH][CH];                 // [0] A_qk [t][s], [1] A_qb [t][s], [2] A_ak^T [s][t], [3] A_ab [t][s]
  float tmat[CH][CH];                    // T [t][s]
  float ecen[HD], pc[HD], ec[HD];        // 2^c, 2^{g_C - c}, 2^{g_C}
};

// x = hi + lo with hi = x truncated to bf16 (exact) and lo = bf16(x - hi);
// |x - hi - lo| <= 2^-17 |x|.
__device__ __forceinline__ float trunc_bf16(float x) {
  return __uint_as_float(__float_as_uint(x) & 0xffff0000u);
}
__device__ __forceinline__ __bf16 hi_bits(float x) {
  return __builtin_bit_cast(__bf16, (unsigned short)(__float_as_uint(x) >> 16));
}
__device__ __forceinline__ void split2(float x, __bf16& hi, __bf16& lo) {
  hi = hi_bits(x);
  lo = (__bf16)(x - trunc_bf16(x));
}
__device__ __forceinline__ void split4(const float (&x)[4], bf16x4& hi, bf16x4& lo) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    hi[e] = hi_bits(x[e]);
    lo[e] = (__bf16)(x[e] - trunc_bf16(x[e]));
  }
}
__device__ __forceinline__ void split_f4(const f32x4& x, bf16x4& hi, bf16x4& lo) {
  const float a[4] = {x[0], x[1], x[2], x[3]};
  split4(a, hi, lo);
}
__device__ __forceinline__ void split_pair(float x0, float x1, bf16x2& hi, bf16x2& lo) {
  hi = (bf16x2){hi_bits(x0), hi_bits(x1)};
  lo = (bf16x2){(__bf16)(x0 - trunc_bf16(x0)), (__bf16)(x1 - trunc_bf16(x1))};
}

__device__ __forceinline__ f32x4 mma16(bf16x4 a, bf16x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a),
                                                   __builtin_bit_cast(s16x4, b), c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mma3_16(bf16x4 ah, bf16x4 al, bf16x4 bh, bf16x4 bl, f32x4 c) {
  c = mma16(ah, bh, c);
  c = mma16(ah, bl, c);
  return mma16(al, bh, c);
}
__device__ __forceinline__ f32x4 mma3_32(bf16x8 ah, bf16x8 al, bf16x8 bh, bf16x8 bl, f32x4 c) {
  c = mfma16x16x32(ah, bh, c);
  c = mfma16x16x32(ah, bl, c);
  return mfma16x16x32(al, bh, c);
}
// Split-term accumulators: the three products of a bf16x3 GEMM kept in
// independent MFMA chains (summed once at the end) to shorten dependencies.
struct Acc3 {
  f32x4 hh, hl, lh;
  __device__ __forceinline__ void zero() {
    hh = hl = lh = (f32x4){0.f, 0.f, 0.f, 0.f};
  }
  __device__ __forceinline__ void add32(bf16x8 ah, bf16x8 al, bf16x8 bh, bf16x8 bl) {
    hh = mfma16x16x32(ah, bh, hh);
    hl = mfma16x16x32(ah, bl, hl);
    lh = mfma16x16x32(al, bh, lh);
  }
  __device__ __forceinline__ void add16(bf16x4 ah, bf16x4 al, bf16x4 bh, bf16x4 bl) {
    hh = mma16(ah, bh, hh);
    hl = mma16(ah, bl, hl);
    lh = mma16(al, bh, lh);
  }
  __device__ __forceinline__ f32x4 sum() const { return hh + (hl + lh); }
};
__device__ __forceinline__ bf16x8 cat(bf16x4 a, bf16x4 b) {
  return (bf16x8){a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}
__device__ __forceinline__ bf16x4 ld4(const __bf16* p) { return *reinterpret_cast<const bf16x4*>(p); }
__device__ __forceinline__ bf16x8 ld8(const __bf16* p) { return *reinterpret_cast<const bf16x8*>(p); }
__device__ __forceinline__ f32x4 ldf4(const float* p) {
  const float4 q = *reinterpret_cast<const float4*>(p);
  return (f32x4){q.x, q.y, q.z, q.w};
}

__device__ __forceinline__ float clamp_exp(float e) { return fminf(fmaxf(e, -120.f), 120.f); }

template <typename TA, typename TW, bool WLOG>
__global__ __launch_bounds__(256, 2) void wkv7_chunk_kernel(
    const TA* __restrict__ r, const TW* __restrict__ w, const TA* __restrict__ k,
    const TA* __restrict__ v, const TA* __restrict__ kk, const TA* __restrict__ a,
    const float* state_in, float* state_out, TA* __restrict__ y, int T, int H) {
  __shared__ ChunkLDS L;
  const int bh = blockIdx.x;
  const int b = bh / H;
  const int h = bh % H;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int l16 = lane & 15;
  const int kg = lane >> 4;
  const int64_t tok = (int64_t)H * HD;
  const int64_t base = ((int64_t)b * T * H + h) * HD;

  // state S[i][j], i = 16*wave + l16, j = 16*jt + 4*kg + e  (= S^T tile jt, D layout)
  f32x4 S[4];
  const int irow = 16 * wave + l16;
  {
    const float* src = state_in + ((int64_t)bh * HD + irow) * HD + 4 * kg;
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) S[jt] = ldf4(src + 16 * jt);
  }

  // raw inputs of this thread (channel j = lane, tokens 4*wave + tt), kept in
  // their storage type until phase (A) so the prefetch never stalls on them
  const int j = lane;
  TA rr_[4], rk_[4], rv_[4], rkk_[4], ra_[4];
  TW rw_[4];
  auto load_raw = [&](int t0) {
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      const int tg = min(t0 + 4 * wave + tt, T - 1);  // clamped; masked in (A)
      const int64_t off = base + (int64_t)tg * tok + j;
      rr_[tt] = r[off];
      rk_[tt] = k[off];
      rv_[tt] = v[off];
      rkk_[tt] = kk[off];
      ra_[tt] = a[off];
      rw_[tt] = w[off];
    }
  };
  float xr[4], xk[4], xal[4], xbe[4];

  const int nchunks = (T + CH - 1) / CH;
  if (nchunks > 0) load_raw(0);
  for (int c = 0; c < nchunks; ++c) {
    const int t0 = c * CH;
    // ---------------- (A) derive inputs, stage log-decay and v
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      const int t = 4 * wave + tt;
      const bool ok = t0 + t < T;  // padding tokens: zero vectors, decay 1
      const float kkv = to_f32(rkk_[tt]);
      xr[tt] = ok ? to_f32(rr_[tt]) : 0.f;
      xk[tt] = ok ? to_f32(rk_[tt]) : 0.f;
      xal[tt] = ok ? -kkv : 0.f;
      xbe[tt] = ok ? kkv * to_f32(ra_[tt]) : 0.f;
      const float wv = to_f32(rw_[tt]);
      const float lw = WLOG ? wv * 1.4426950408889634f : log2f(wv);
      L.lw[t][j] = ok ? fmaxf(lw, -126.f) : 0.f;
      split2(ok ? to_f32(rv_[tt]) : 0.f, L.vh[t][j], L.vl[t][j]);
    }
    __syncthreads();
    // ---------------- (B) gates and gated rows
    {
      float g[CH];
      float acc = 0.f;
#pragma unroll
      for (int t = 0; t < CH; ++t) {
        acc += L.lw[t][j];
        g[t] = acc;
      }
      const float gC = g[CH - 1];
      const float cen = g[CH / 2 - 1];
      // g[4*wave - 1 .. 4*wave + 3] via a wave-uniform branch (compile-time indices)
      float gprev = 0.f;
      float gt4[4];
      switch (wave) {
        case 0: gt4[0] = g[0]; gt4[1] = g[1]; gt4[2] = g[2]; gt4[3] = g[3]; break;
        case 1: gprev = g[3]; gt4[0] = g[4]; gt4[1] = g[5]; gt4[2] = g[6]; gt4[3] = g[7]; break;
        case 2: gprev = g[7]; gt4[0] = g[8]; gt4[1] = g[9]; gt4[2] = g[10]; gt4[3] = g[11]; break;
        default: gprev = g[11]; gt4[0] = g[12]; gt4[1] = g[13]; gt4[2] = g[14]; gt4[3] = g[15]; break;
      }
      float p[5], q[4];
      p[0] = exp2f(clamp_exp(gprev - cen));
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        p[tt + 1] = exp2f(clamp_exp(gt4[tt] - cen));
        q[tt] = exp2f(clamp_exp(cen - gt4[tt]));
      }
#pragma unroll
      for (int pp = 0; pp < 2; ++pp) {
        const int t = 4 * wave + 2 * pp;
        const int a0 = 2 * pp, a1 = 2 * pp + 1;
        bf16x2 hi, lo;
        split_pair(xr[a0] * p[a0 + 1], xr[a1] * p[a1 + 1], hi, lo);
        L.rch[t][j] = hi[0]; L.rch[t + 1][j] = hi[1]; L.rcl[t][j] = lo[0]; L.rcl[t + 1][j] = lo[1];
        split_pair(xal[a0] * p[a0], xal[a1] * p[a1], hi, lo);
        L.ach[t][j] = hi[0]; L.ach[t + 1][j] = hi[1]; L.acl[t][j] = lo[0]; L.acl[t + 1][j] = lo[1];
        *reinterpret_cast<bf16x2*>(&L.acth[j][t]) = hi;
        *reinterpret_cast<bf16x2*>(&L.actl[j][t]) = lo;
        split_pair(xk[a0] * q[a0], xk[a1] * q[a1], hi, lo);
        L.kch[t][j] = hi[0]; L.kch[t + 1][j] = hi[1]; L.kcl[t][j] = lo[0]; L.kcl[t + 1][j] = lo[1];
        *reinterpret_cast<bf16x2*>(&L.kcth[j][t]) = hi;
        *reinterpret_cast<bf16x2*>(&L.kctl[j][t]) = lo;
        split_pair(xbe[a0] * q[a0], xbe[a1] * q[a1], hi, lo);
        L.bch[t][j] = hi[0]; L.bch[t + 1][j] = hi[1]; L.bcl[t][j] = lo[0]; L.bcl[t + 1][j] = lo[1];
        *reinterpret_cast<bf16x2*>(&L.bcth[j][t]) = hi;
        *reinterpret_cast<bf16x2*>(&L.bctl[j][t]) = lo;
      }
      if (wave == 0) {
        L.ecen[j] = exp2f(cen);
        L.pc[j] = exp2f(clamp_exp(gC - cen));
        L.ec[j] = exp2f(gC);
      }
    }
    if (c + 1 < nchunks) load_raw(t0 + CH);  // in flight during (C)-(E)
    __syncthreads();
    // ---------------- (C) causal matrices: wave 0 A_qk, 1 A_qb, 2 A_ak, 3 A_ab
    {
      const bool use_k = (wave == 0 || wave == 2);
      const bool use_r = (wave < 2);
      const __bf16(*Xh)[PR] = use_k ? L.kch : L.bch;
      const __bf16(*Xl)[PR] = use_k ? L.kcl : L.bcl;
      const __bf16(*Yh)[PR] = use_r ? L.rch : L.ach;
      const __bf16(*Yl)[PR] = use_r ? L.rcl : L.acl;
      f32x4 acc = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int cc = 0; cc < 2; ++cc) {
        const int jo = 32 * cc + 8 * kg;
        acc = mma3_32(ld8(&Xh[l16][jo]), ld8(&Xl[l16][jo]), ld8(&Yh[l16][jo]), ld8(&Yl[l16][jo]), acc);
      }
      // D[m = s][n = t]: lane holds s = 4kg + e, t = l16
      float o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int s = 4 * kg + e;
        const bool keep = use_r ? (s <= l16) : (s < l16);
        o[e] = keep ? acc[e] : 0.f;
      }
      if (wave == 2) {
#pragma unroll
        for (int e = 0; e < 4; ++e) L.amat[2][4 * kg + e][l16] = o[e];  // A_ak^T [s][t]
      } else {
        *reinterpret_cast<float4*>(&L.amat[wave][l16][4 * kg]) = make_float4(o[0], o[1], o[2], o[3]);
      }
    }
    __syncthreads();
    // ---------------- (D) T = (I - A_ab)^{-1}: column s = lane, forward substitution
    if (wave == 0 && lane < CH) {
      float Lm[CH][CH];
#pragma unroll
      for (int t = 1; t < CH; ++t)
#pragma unroll
        for (int qq = 0; qq < (t + 3) / 4; ++qq) {
          const float4 v4 = *reinterpret_cast<const float4*>(&L.amat[3][t][4 * qq]);
          Lm[t][4 * qq] = v4.x; Lm[t][4 * qq + 1] = v4.y; Lm[t][4 * qq + 2] = v4.z; Lm[t][4 * qq + 3] = v4.w;
        }
      float x[CH];
#pragma unroll
      for (int t = 0; t < CH; ++t) {
        float accx = (t == lane) ? 1.f : 0.f;
#pragma unroll
        for (int u = 0; u < t; ++u) accx += Lm[t][u] * x[u];
        x[t] = accx;
        L.tmat[t][lane] = accx;
      }
    }
    __syncthreads();
    // ---------------- (E) state chain for value rows [16*wave, 16*wave + 16)
    {
      // T as B operand (K = s = 4kg + e, N = t = l16): T[t][s]
      bf16x4 TBh, TBl;
      split_f4(ldf4(&L.tmat[l16][4 * kg]), TBh, TBl);
      // W' = T ac, in A layout: (T ac)^T = ac^T T^T, D lane (j = 16jt + 4kg + e, t = l16)
      bf16x4 WAh[4], WAl[4];
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) {
        const int jr = 16 * jt + l16;
        f32x4 wt = mma3_16(ld4(&L.acth[jr][4 * kg]), ld4(&L.actl[jr][4 * kg]), TBh, TBl,
                           (f32x4){0.f, 0.f, 0.f, 0.f});
        split_f4(wt, WAh[jt], WAl[jt]);
      }
      // M = T A_ak, in A layout: (T A_ak)^T = A_ak^T T^T, D lane (s = 4kg + e, t = l16)
      bf16x4 MAh, MAl;
      {
        bf16x4 AkH, AkL;
        split_f4(ldf4(&L.amat[2][l16][4 * kg]), AkH, AkL);
        f32x4 mt = mma3_16(AkH, AkL, TBh, TBl, (f32x4){0.f, 0.f, 0.f, 0.f});
        split_f4(mt, MAh, MAl);
      }
      // S' = S diag(2^c)
      bf16x4 SH[4], SL[4];
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) {
        const f32x4 sc = ldf4(&L.ecen[16 * jt + 4 * kg]);
        split_f4(S[jt] * sc, SH[jt], SL[jt]);
      }
      bf16x4 VH, VL;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        VH[e] = L.vh[4 * kg + e][16 * wave + l16];
        VL[e] = L.vl[4 * kg + e][16 * wave + l16];
      }
      // U = W' S'^T + M V
      Acc3 accU;
      accU.zero();
#pragma unroll
      for (int cc = 0; cc < 2; ++cc)
        accU.add32(cat(WAh[2 * cc], WAh[2 * cc + 1]), cat(WAl[2 * cc], WAl[2 * cc + 1]),
                   cat(SH[2 * cc], SH[2 * cc + 1]), cat(SL[2 * cc], SL[2 * cc + 1]));
      accU.add16(MAh, MAl, VH, VL);
      const f32x4 U = accU.sum();
      bf16x4 UH, UL;
      split_f4(U, UH, UL);
      // [U ; V] as one K = 32 B operand: slots 0-3 = U[s][i], slots 4-7 = V[s][i], s = 4kg + e
      const bf16x8 UVh = cat(UH, VH);
      const bf16x8 UVl = cat(UL, VL);
      // Y = rc S'^T + [A_qb | A_qk] [U ; V]
      Acc3 accY;
      accY.zero();
#pragma unroll
      for (int cc = 0; cc < 2; ++cc) {
        const int jo = 32 * cc + 4 * kg;
        accY.add32(cat(ld4(&L.rch[l16][jo]), ld4(&L.rch[l16][jo + 16])),
                   cat(ld4(&L.rcl[l16][jo]), ld4(&L.rcl[l16][jo + 16])),
                   cat(SH[2 * cc], SH[2 * cc + 1]), cat(SL[2 * cc], SL[2 * cc + 1]));
      }
      {
        bf16x4 QBH, QBL, QKH, QKL;
        split_f4(ldf4(&L.amat[1][l16][4 * kg]), QBH, QBL);
        split_f4(ldf4(&L.amat[0][l16][4 * kg]), QKH, QKL);
        accY.add32(cat(QBH, QKH), cat(QBL, QKL), UVh, UVl);
      }
      const f32x4 Yv = accY.sum();
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int tg = t0 + 4 * kg + e;
        if (tg < T) y[base + (int64_t)tg * tok + 16 * wave + l16] = from_f32<TA>(Yv[e]);
      }
      // S^T = diag(2^{g_C}) S^T + diag(2^{g_C - c}) [bc^T | kc^T] [U ; V]
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) {
        const int jr = 16 * jt + l16;
        const f32x4 X = mma3_32(cat(ld4(&L.bcth[jr][4 * kg]), ld4(&L.kcth[jr][4 * kg])),
                                cat(ld4(&L.bctl[jr][4 * kg]), ld4(&L.kctl[jr][4 * kg])), UVh, UVl,
                                (f32x4){0.f, 0.f, 0.f, 0.f});
        S[jt] = S[jt] * ldf4(&L.ec[16 * jt + 4 * kg]) + X * ldf4(&L.pc[16 * jt + 4 * kg]);
      }
    }
    __syncthreads();
  }

  {
    float* dst = state_out + ((int64_t)bh * HD + irow) * HD + 4 * kg;
#pragma unroll
    for (int jt = 0; jt < 4; ++jt)
      *reinterpret_cast<float4*>(dst + 16 * jt) = make_float4(S[jt][0], S[jt][1], S[jt][2], S[jt][3]);
  }
}

}  // namespace rwkv7mi

using namespace rwkv7mi;

extern "C" int rwkv7mi_wkv7_chunk_prefill(const void* r, const void* w, const void* k, const void* v,
                                          const void* kk, const void* a, const float* state_in,
                                          float* state_out, void* y, int64_t B, int64_t T, int64_t H,
                                          int64_t N, int64_t chunk, int w_is_log, int act_dtype,
                                          int w_dtype, void* stream) {
  if (N != HD) return fail(RWKV7MI_EINVAL, "wkv7 chunk: head size must be 64");
  if (chunk != 16 && chunk != 32 && chunk != 64)
    return fail(RWKV7MI_EINVAL, "wkv7 chunk: chunk must be 16, 32 or 64");
  if (B < 0 || T < 0 || H <= 0) return fail(RWKV7MI_EINVAL, "wkv7 chunk: bad B/T/H");
  if (B == 0) return RWKV7MI_OK;
  if (!state_in || !state_out) return fail(RWKV7MI_EINVAL, "wkv7 chunk: null state");
  if (T > 0 && (!r || !w || !k || !v || !kk || !a || !y)) return fail(RWKV7MI_EINVAL, "wkv7 chunk: null input");
  if ((reinterpret_cast<uintptr_t>(state_in) | reinterpret_cast<uintptr_t>(state_out)) & 15)
    return fail(RWKV7MI_EINVAL, "wkv7 chunk: state must be 16-byte aligned");
  if (B * H > INT32_MAX || T > INT32_MAX) return fail(RWKV7MI_EINVAL, "wkv7 chunk: too large");
  return dispatch_dtype(act_dtype, [&](auto ta) {
    using TA = decltype(ta);
    return dispatch_dtype(w_dtype, [&](auto tw) {
      using TW = decltype(tw);
      if (w_is_log)
        hipLaunchKernelGGL((wkv7_chunk_kernel<TA, TW, true>), dim3((unsigned)(B * H)), dim3(256), 0,
                           as_stream(stream), (const TA*)r, (const TW*)w, (const TA*)k, (const TA*)v,
                           (const TA*)kk, (const TA*)a, state_in, state_out, (TA*)y, (int)T, (int)H);
      else
        hipLaunchKernelGGL((wkv7_chunk_kernel<TA, TW, false>), dim3((unsigned)(B * H)), dim3(256), 0,
                           as_stream(stream), (const TA*)r, (const TW*)w, (const TA*)k, (const TA*)v,
                           (const TA*)kk, (const TA*)a, state_in, state_out, (TA*)y, (int)T, (int)H);
      return check_launch("wkv7_chunk_kernel");
    });
  });
}
