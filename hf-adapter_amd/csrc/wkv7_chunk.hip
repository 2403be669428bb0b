// wkv7 chunked DPLR prefill (gfx950), chunk C = 16, head size 64.
//
// Recurrence (native V x K state, rwkv7_hf/fused_recurrent_update.py:757-783):
//   S_t = S_{t-1} (diag(w_t) + alpha_t beta_t^T) + v_t k_t^T,  y_t = S_t r_t,
//   alpha = -kk, beta = kk * a.
// Per chunk, with g_t = sum_{s<=t} log2 w_s per key channel (g_{-1} = 0, gC = g_15)
// and the causal 16 x 16 matrices
//   A_qk[t,s] = sum_j r_t k_s 2^{g_t - g_s}   (s <= t)     A_qb: beta_s in place of k_s
//   A_ak[t,s] = sum_j alpha_t k_s 2^{g_{t-1} - g_s} (s < t) A_ab: beta_s in place of k_s
// and T = (I - A_ab)^{-1}, the chunk is affine in its start state S:
//   U   = Wa S'^T + M V,   Wa = T ac,  M = T A_ak,          (u_t = S_{t-1} alpha_t)
//   Y   = Rq S'^T + Qm V,  Rq = rc + A_qb Wa,  Qm = A_qb M + A_qk
//   S^T <- diag(2^gC) S^T + diag(2^{gC-c}) (Bc^T U + Kc^T V),   S' = S diag(2^c)
// with the rows centred on c = round(gC / 2) (per key channel):
//   rc = r 2^{g-c}, kc = k 2^{c-g}, ac = alpha 2^{g_{t-1}-c}, bc = beta 2^{c-g}
// — the WY form of the reference's chunk algebra (rwkv7_hf/self_chunk_rwkv7.py:85-134,
// rwkv7_hf/dplr_prefill.py:221-311) with everything that does not depend on S
// moved off the state's critical path, and one set of gated rows serving every
// product (the per-channel scales fold into the state).  Exact while a chunk's
// log2-decay span -gC stays within 252 (per-token w >= 2^-15.75 on average);
// beyond that the factors clamp at 2^+-126 and the call's status word records
// it (WKV7_STATUS_CLAMPED, read by rwkv7mi_wkv7_chunk_status).
//
// The decay w arrives as the decay itself (WMODE 0), its natural log (1) or
// the raw pre-activation of the reference's clampw scan (2):
// w = exp(-0.606531 sigmoid(w_raw)), so log2 w = -0.606531 log2(e) sigmoid(w_raw).
//
// Mapping: one workgroup of 8 waves per (batch, head), specialised:
// * waves 0-3 ("chain") hold the fp32 state — wave q owns 16 value rows, as
//   S^T tiles in MFMA accumulator layout — and per chunk run the products
//   of U, Y and the state update (30 bf16x3 MFMAs per wave);
// * waves 4-7 ("producers") each build whole chunks (chunks p, p+4, ...):
//   loads, gate cumsum (DPP row scan), gated rows, the four A matrices, T by
//   forward substitution, and Wa, Rq, M, Qm and the transposed Bd, Kd, V
//   operands, all by MFMA, written into one of four LDS slots in exactly the
//   per-lane register layout the chain waves consume.
// Slots hand over through LDS flags (producer: ready = chunk id; chain waves:
// done = chunk id); with five slots for four producers a producer never
// waits for a slot in steady state, and no workgroup barrier sits in the
// chunk loop.  All waits are bounded: a wait that gives up (the kernel then
// goes on with whatever the slot holds) sets WKV7_STATUS_TIMEOUT in the
// device's status word, so the host can tell that the call's output is void.
//
// Products run on v_mfma_f32_16x16x{32,16}_bf16 with operands split into bf16
// hi + lo (hi*hi + hi*lo + lo*hi, ~1e-5 relative) and fp32 accumulation.
// Layout changes (transposes) are MFMAs against the identity, which move
// bf16 values exactly.
//
// Key channels are held in a permuted order sigma = 16 jt + 4 kg + e ->
// channel 32 (jt >> 1) + 8 kg + 4 (jt & 1) + e, so that one lane's 16
// channels of a token are two 16-byte runs; value rows use the same map.
#include "common.h"

namespace rwkv7mi {

typedef short s16x4 __attribute__((ext_vector_type(4)));

constexpr int CH = 16;   // chunk length
constexpr int HD = 64;   // head size
constexpr int NSLOT = 6; // LDS slots: more than producer waves, so a producer
                          // rarely waits for the chain to free one
constexpr int WAIT_SPINS = 1 << 20;

// Sticky per-device status bits of the chunk kernel (this file's copy on each
// GPU), read and cleared by rwkv7mi_wkv7_chunk_status.
constexpr int WKV7_STATUS_TIMEOUT = 1;  // a bounded LDS-flag wait gave up
constexpr int WKV7_STATUS_CLAMPED = 2;  // a chunk's gate span exceeded the exact range
__device__ int wkv7_chunk_status_word;

// one chunk's operands for the chain waves, each array indexed [..][lane]
struct ChunkSlot {
  bf16x8 wa[2][2][64];  // [hi/lo][k-half cc] A(Wa): lane (t, kg)
  bf16x8 rq[2][2][64];  // A(Rq)
  bf16x8 bk[2][4][64];  // [hi/lo][jt] A([Bd^T | Kd^T]) rows of key tile jt
  bf16x4 vt[2][4][64];  // [hi/lo][value tile] B(V)
  bf16x4 am[2][64];     // [hi/lo] A(M)
  bf16x4 aq[2][64];     // [hi/lo] A(Qm)
  f32x4 pc[4][4];       // [jt][kg] 2^{gC - c} of channels 16jt + 4kg + e
  f32x4 cen[4][4];      // [jt][kg] 2^c
};

struct ChunkShared {
  ChunkSlot slot[NSLOT];
  float nmat[4][CH][CH];  // per producer: A_ab [t][s]
  float tcol[4][CH][CH];  // per producer: T column-major [s][t]
  int ready[NSLOT];
  int done[4][NSLOT];
};

__device__ __forceinline__ float trunc_bf16(float x) {
  return __uint_as_float(__float_as_uint(x) & 0xffff0000u);
}
__device__ __forceinline__ __bf16 hi_bits(float x) {
  return __builtin_bit_cast(__bf16, (unsigned short)(__float_as_uint(x) >> 16));
}
// x = hi + lo, hi = x truncated to bf16, lo = bf16(x - hi); |x - hi - lo| <= 2^-16 |x|
__device__ __forceinline__ void split_f4(const f32x4& x, bf16x4& hi, bf16x4& lo) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    hi[e] = hi_bits(x[e]);
    lo[e] = (__bf16)(x[e] - trunc_bf16(x[e]));
  }
}
// f32x4 holding bf16 values -> bf16x4 (exact)
__device__ __forceinline__ bf16x4 pack_exact(const f32x4& x) {
  return (bf16x4){hi_bits(x[0]), hi_bits(x[1]), hi_bits(x[2]), hi_bits(x[3])};
}
__device__ __forceinline__ bf16x8 cat(bf16x4 a, bf16x4 b) {
  return (bf16x8){a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

__device__ __forceinline__ f32x4 mma16(bf16x4 a, bf16x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a),
                                                   __builtin_bit_cast(s16x4, b), c, 0, 0, 0);
}
constexpr f32x4 ZERO4 = {0.f, 0.f, 0.f, 0.f};

// bf16x3 products (hi*hi + hi*lo + lo*hi) accumulated onto c in one chain:
// each MFMA takes the previous one's result (same shape) as its C operand
__device__ __forceinline__ f32x4 mma3_16(bf16x4 ah, bf16x4 al, bf16x4 bh, bf16x4 bl) {
  return mma16(al, bh, mma16(ah, bl, mma16(ah, bh, ZERO4)));
}
__device__ __forceinline__ f32x4 mma3_32(bf16x8 ah, bf16x8 al, bf16x8 bh, bf16x8 bl, f32x4 c) {
  return mfma16x16x32(al, bh, mfma16x16x32(ah, bl, mfma16x16x32(ah, bh, c)));
}

// ---- cross-lane helpers on 16-lane rows (lane = token within the chunk)
template <int N>
__device__ __forceinline__ float row_shr(float x) {  // lane t gets lane t-N (0 below the row)
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x110 + N, 0xF, 0xF, true));
}
__device__ __forceinline__ float row_scan(float x) {  // inclusive prefix sum over the row
  x += row_shr<1>(x);
  x += row_shr<2>(x);
  x += row_shr<4>(x);
  x += row_shr<8>(x);
  return x;
}
// lane t gets lane t-1; lane 0 of the row keeps `old` (DPP without bound control)
__device__ __forceinline__ float row_shr1_or(float x, float old) {
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(x), 0x111, 0xF, 0xF, false));
}
__device__ __forceinline__ float row_last(float x) {  // lane 15 of the row in every lane (DPP row_newbcast)
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x15F, 0xF, 0xF, false));
}

// ---- LDS flags (workgroup scope)
// true once *f >= v; false when the wait gives up after WAIT_SPINS polls
__device__ __forceinline__ bool wait_geq(int* f, int v) {
  for (int it = 0; it < WAIT_SPINS; ++it) {
    if (__hip_atomic_load(f, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) >= v) return true;
    __builtin_amdgcn_s_sleep(1);
  }
  return false;
}
// ORs this wave's status bits into the device's status word (one vector atomic
// from lane 0; nothing when the bits are clear)
__device__ __forceinline__ void post_status(int bits) {
  bits = __builtin_amdgcn_readfirstlane(bits);
  if (bits && (threadIdx.x & 63) == 0)
    __hip_atomic_fetch_or(&wkv7_chunk_status_word, bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void set_flag(int* f, int v) {
  __hip_atomic_store(f, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// ---- one token's 16 channels of this lane: channels 8kg..8kg+7 and 32+8kg..32+8kg+7
template <typename T>
struct RawRow {
  u32x4 v[sizeof(T) == 4 ? 4 : 2];
};
template <typename T>
__device__ __forceinline__ void load_row(RawRow<T>& o, __amdgpu_buffer_rsrc_t rs, uint32_t off) {
  if constexpr (sizeof(T) == 4) {
    o.v[0] = buf_ld16(rs, off);
    o.v[1] = buf_ld16(rs, off + 16u);
    o.v[2] = buf_ld16(rs, off + 128u);
    o.v[3] = buf_ld16(rs, off + 144u);
  } else {
    o.v[0] = buf_ld16(rs, off);
    o.v[1] = buf_ld16(rs, off + 64u);
  }
}
// value of slot (jt, e): half jt >> 1, element 4 (jt & 1) + e of that half
// one element of y; an offset past the descriptor (a token beyond T) is dropped
template <typename T>
__device__ __forceinline__ void store_y(__amdgpu_buffer_rsrc_t rs, uint32_t off, float v) {
  if constexpr (sizeof(T) == 4) {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), rs, (int)off, 0, 0);
  } else {
    __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, from_f32<T>(v)), rs, (int)off, 0, 0);
  }
}

template <typename T>
__device__ __forceinline__ float row_val(const RawRow<T>& o, int jt, int e) {
  const int h = jt >> 1, idx = 4 * (jt & 1) + e;
  if constexpr (sizeof(T) == 4) {
    return __uint_as_float(o.v[2 * h + (idx >> 2)][idx & 3]);
  } else {
    const uint32_t w = o.v[h][idx >> 1];
    if constexpr (std::is_same<T, __half>::value) {
      float lo, hi;
      f16x2_to_f32(w, lo, hi);
      return (idx & 1) ? hi : lo;
    } else {
      return __uint_as_float((idx & 1) ? (w & 0xffff0000u) : (w << 16));
    }
  }
}

__device__ __forceinline__ float clamp126(float x) { return fminf(fmaxf(x, -126.f), 126.f); }

template <typename TA, typename TW, int WMODE>
__global__ __launch_bounds__(512, 1) void wkv7_chunk_kernel(
    const TA* __restrict__ r, const TW* __restrict__ w, const TA* __restrict__ k,
    const TA* __restrict__ v, const TA* __restrict__ kk, const TA* __restrict__ a,
    const float* state_in, float* state_out, TA* __restrict__ y, int T, int H) {
  extern __shared__ __align__(16) char smem_raw[];
  ChunkShared& L = *reinterpret_cast<ChunkShared*>(smem_raw);
  const int bh = blockIdx.x;
  const int b = bh / H;
  const int h = bh % H;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int l16 = lane & 15;
  const int kg = lane >> 4;
  const int nchunks = (T + CH - 1) / CH;
  const int64_t tok = (int64_t)H * HD;  // elements per token

  if (tid < NSLOT) L.ready[tid] = -1;
  if (tid < 4 * NSLOT) L.done[tid / NSLOT][tid % NSLOT] = -1;
  __syncthreads();

  if (wave < 4) {
    // ===================== chain wave q: value rows i = phi(16q + l16)
    const int q = wave;
    const int ich = 32 * (q >> 1) + 8 * (l16 >> 2) + 4 * (q & 1) + (l16 & 3);
    // S[jt] lane (l16, kg): S[ich][j], j = 32 (jt >> 1) + 8 kg + 4 (jt & 1) + e
    f32x4 S[4];
    {
      const float* src = state_in + ((int64_t)bh * HD + ich) * HD + 8 * kg;
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) {
        const float4 t4 = *reinterpret_cast<const float4*>(src + 32 * (jt >> 1) + 4 * (jt & 1));
        S[jt] = (f32x4){t4.x, t4.y, t4.z, t4.w};
      }
    }
    // byte offsets of this lane's y elements (tokens 4kg + e, value row ich) within a chunk
    uint32_t yoff[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) yoff[e] = (uint32_t)(((4 * kg + e) * tok + ich) * (int64_t)sizeof(TA));
    int status = 0;
    for (int x = 0; x < nchunks; ++x) {
      const int s = x % NSLOT;
      const ChunkSlot& Z = L.slot[s];
      if (!wait_geq(&L.ready[s], x)) status |= WKV7_STATUS_TIMEOUT;
      bf16x8 waH[2], waL[2], rqH[2], rqL[2], bkH[4], bkL[4];
#pragma unroll
      for (int cc = 0; cc < 2; ++cc) {
        waH[cc] = Z.wa[0][cc][lane];
        waL[cc] = Z.wa[1][cc][lane];
        rqH[cc] = Z.rq[0][cc][lane];
        rqL[cc] = Z.rq[1][cc][lane];
      }
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) {
        bkH[jt] = Z.bk[0][jt][lane];
        bkL[jt] = Z.bk[1][jt][lane];
      }
      const bf16x4 vH = Z.vt[0][q][lane], vL = Z.vt[1][q][lane];
      const bf16x4 amH = Z.am[0][lane], amL = Z.am[1][lane], aqH = Z.aq[0][lane], aqL = Z.aq[1][lane];
      f32x4 pc[4], cen[4];
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) {
        pc[jt] = Z.pc[jt][kg];
        cen[jt] = Z.cen[jt][kg];
      }
      set_flag(&L.done[q][s], x);  // the operands are in registers

      // S' = S diag(2^c): the bf16x3 operand of U and Y, and the seed of the
      // update's product chain, so that S <- 2^{gC-c} (S' + Bc^T U + Kc^T V)
      f32x4 Sp[4];
      bf16x4 SH[4], SL[4];
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) {
        Sp[jt] = S[jt] * cen[jt];
        split_f4(Sp[jt], SH[jt], SL[jt]);
      }
      f32x4 U = ZERO4, Yv = ZERO4;
#pragma unroll
      for (int cc = 0; cc < 2; ++cc) {
        const bf16x8 sh = cat(SH[2 * cc], SH[2 * cc + 1]), sl = cat(SL[2 * cc], SL[2 * cc + 1]);
        U = mma3_32(waH[cc], waL[cc], sh, sl, U);
        Yv = mma3_32(rqH[cc], rqL[cc], sh, sl, Yv);
      }
      // + M V and, below, + Qm V, on 16x16x32 like the rest of each chain
      // (A and B pair positionally: [mH | mH] x [vH | vL] gives hi*hi + hi*lo,
      // [mL | 0] x [vH | 0] gives lo*hi).  A 16x16x16 MFMA that takes a
      // 16x16x32 result as its C operand straight after it read a stale
      // accumulator here, so the shapes are not mixed within a chain.
      const bf16x8 vHL = cat(vH, vL), vH0 = cat(vH, (bf16x4){});
      U = mfma16x16x32(cat(amH, amH), vHL, U);
      U = mfma16x16x32(cat(amL, (bf16x4){}), vH0, U);
      bf16x4 UH, UL;
      split_f4(U, UH, UL);
      const bf16x8 uvH = cat(UH, vH), uvL = cat(UL, vL);
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) S[jt] = pc[jt] * mma3_32(bkH[jt], bkL[jt], uvH, uvL, Sp[jt]);
      Yv = mfma16x16x32(cat(aqH, aqH), vHL, Yv);
      Yv = mfma16x16x32(cat(aqL, (bf16x4){}), vH0, Yv);
      const int t0 = x * CH;
      const __amdgpu_buffer_rsrc_t ys =
          make_rsrc(y + (((int64_t)b * T + t0) * H + h) * HD, (uint32_t)(min(CH, T - t0) * tok * (int64_t)sizeof(TA)));
#pragma unroll
      for (int e = 0; e < 4; ++e) store_y<TA>(ys, yoff[e], Yv[e]);
    }
    float* dst = state_out + ((int64_t)bh * HD + ich) * HD + 8 * kg;
#pragma unroll
    for (int jt = 0; jt < 4; ++jt)
      *reinterpret_cast<float4*>(dst + 32 * (jt >> 1) + 4 * (jt & 1)) = make_float4(S[jt][0], S[jt][1], S[jt][2], S[jt][3]);
    post_status(status);
    return;
  }

  // ===================== producer wave p: chunks p, p+4, ...; lane = (token t = l16, kg)
  const int p = wave - 4;
  // The producers bound the chunk rate (the chain waves wait for a ready slot
  // about half of the time), so where a producer and a chain wave can both
  // issue on a SIMD, the producer goes first.
  __builtin_amdgcn_s_setprio(1);
  const int t = l16;
  // identity as a B operand: lane (n = l16, k = 4kg + e)
  bf16x4 Ib;
#pragma unroll
  for (int e = 0; e < 4; ++e) Ib[e] = (__bf16)((4 * kg + e == l16) ? 1.f : 0.f);
  float(&N)[CH][CH] = L.nmat[p];
  float(&Tc)[CH][CH] = L.tcol[p];

  RawRow<TA> rr, rk, rv, rkk, ra;
  RawRow<TW> rw;
  auto issue = [&](int x) {
    const int t0 = x * CH;
    const int valid = min(CH, T - t0);
    const int64_t base = (((int64_t)b * T + t0) * H + h) * HD;
    const uint32_t nbA = (uint32_t)(valid * tok * (int64_t)sizeof(TA));
    const uint32_t nbW = (uint32_t)(valid * tok * (int64_t)sizeof(TW));
    const uint32_t offA = (uint32_t)(t * tok * (int64_t)sizeof(TA)) + 8u * kg * (uint32_t)sizeof(TA);
    const uint32_t offW = (uint32_t)(t * tok * (int64_t)sizeof(TW)) + 8u * kg * (uint32_t)sizeof(TW);
    load_row<TA>(rr, make_rsrc(r + base, nbA), offA);
    load_row<TA>(rk, make_rsrc(k + base, nbA), offA);
    load_row<TA>(rv, make_rsrc(v + base, nbA), offA);
    load_row<TA>(rkk, make_rsrc(kk + base, nbA), offA);
    load_row<TA>(ra, make_rsrc(a + base, nbA), offA);
    load_row<TW>(rw, make_rsrc(w + base, nbW), offW);
  };
  if (p < nchunks) issue(p);

  bool waited_out = false;
  float gmin = 0.f, gmax = 0.f;  // extremes of the chunk totals gC this lane saw
  for (int x = p; x < nchunks; x += 4) {
    // A token past T loads w = 0 (log2 -> -inf, or 0 as a log) and must add
    // nothing to the gate sums: its floor is 0 instead of -126.
    const float lwlo = x * CH + t < T ? -126.f : 0.f;
    // Wait until the chain waves have taken chunk x - NSLOT out of this slot;
    // every result below is then stored as soon as it exists (D(ac) and rc are
    // parked in the Wa / Rq areas until Wa and Rq replace them).
    const int s = x % NSLOT;
    for (int qq = 0; qq < 4; ++qq) waited_out |= !wait_geq(&L.done[qq][s], x - NSLOT);
    ChunkSlot& Z = L.slot[s];

    // ---- per K half cc (channel tiles 2cc, 2cc+1): gates, gated rows, their
    // A-matrix products, and the transposed operands (identity MFMAs:
    // D(x) tile jt = lane (sigma = 16jt + l16, t = 4kg + e))
    f32x4 AqbA = ZERO4, AqkA = ZERO4, AakD = ZERO4, AabA = ZERO4;
#pragma unroll
    for (int cc = 0; cc < 2; ++cc) {
      bf16x4 rcH[2], rcL[2], kcH[2], kcL[2], acH[2], acL[2], bcH[2], bcL[2];
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const int jt = 2 * cc + jj;
        // gate prefix sums of the four channels of slot (jt, .), the four
        // scans stepped together so no DPP read waits on its own producer
        float g[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float wv = row_val<TW>(rw, jt, e);
          float l2;
          if constexpr (WMODE == 1) {
            l2 = wv * 1.4426950408889634f;
          } else if constexpr (WMODE == 2) {
            l2 = -0.87503927f / (1.0f + __expf(-wv));  // -0.606531 log2(e) sigmoid(w_raw)
          } else {
            l2 = __builtin_amdgcn_logf(wv);
          }
          g[e] = fmaxf(l2, lwlo);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) g[e] += row_shr<1>(g[e]);
#pragma unroll
        for (int e = 0; e < 4; ++e) g[e] += row_shr<2>(g[e]);
#pragma unroll
        for (int e = 0; e < 4; ++e) g[e] += row_shr<4>(g[e]);
#pragma unroll
        for (int e = 0; e < 4; ++e) g[e] += row_shr<8>(g[e]);
        f32x4 rc, kc, ac, bc, xv, gcv;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          // inputs of token t, channel slot (jt, e), read from the raw rows here
          const float xr = row_val<TA>(rr, jt, e), xk = row_val<TA>(rk, jt, e);
          const float xkk = row_val<TA>(rkk, jt, e), xa = row_val<TA>(ra, jt, e);
          xv[e] = row_val<TA>(rv, jt, e);
          const float gC = row_last(g[e]);  // the scan's last token: the chunk total
          gcv[e] = gC;
          gmin = fminf(gmin, gC);
          gmax = fmaxf(gmax, gC);
          const float cf = rintf(0.5f * gC);
          const int ci = (int)cf;
          const float xd = clamp126(g[e] - cf);
          const float pv = __builtin_amdgcn_exp2f(xd);
          const float qv = __builtin_amdgcn_exp2f(-xd);
          const float pp = row_shr1_or(pv, __builtin_amdgcn_ldexpf(1.f, -ci));  // 2^{g_{t-1} - c}, g_{-1} = 0
          rc[e] = xr * pv;
          kc[e] = xk * qv;
          ac[e] = -xkk * pp;
          bc[e] = xkk * xa * qv;
        }
        // the row's last token parks the four chunk totals for the per-channel factors below
        if (t == CH - 1) *reinterpret_cast<f32x4*>(&N[kg][4 * jt]) = gcv;
        split_f4(rc, rcH[jj], rcL[jj]);
        split_f4(kc, kcH[jj], kcL[jj]);
        split_f4(ac, acH[jj], acL[jj]);
        split_f4(bc, bcH[jj], bcL[jj]);
        // transposed operands: D(ac) (parked in the Wa area), [D(bc) | D(kc)], D(v)
        reinterpret_cast<bf16x4*>(&Z.wa[0][cc][lane])[jj] = pack_exact(mma16(acH[jj], Ib, ZERO4));
        reinterpret_cast<bf16x4*>(&Z.wa[1][cc][lane])[jj] = pack_exact(mma16(acL[jj], Ib, ZERO4));
        Z.bk[0][jt][lane] = cat(pack_exact(mma16(bcH[jj], Ib, ZERO4)), pack_exact(mma16(kcH[jj], Ib, ZERO4)));
        Z.bk[1][jt][lane] = cat(pack_exact(mma16(bcL[jj], Ib, ZERO4)), pack_exact(mma16(kcL[jj], Ib, ZERO4)));
        bf16x4 hi, lo;
        split_f4(xv, hi, lo);
        Z.vt[0][jt][lane] = pack_exact(mma16(hi, Ib, ZERO4));
        Z.vt[1][jt][lane] = pack_exact(mma16(lo, Ib, ZERO4));
        *reinterpret_cast<f32x4*>(&Z.rq[jj][cc][lane]) = rc;  // rc, until Rq
      }
      const bf16x8 rH = cat(rcH[0], rcH[1]), rL = cat(rcL[0], rcL[1]);
      const bf16x8 kH = cat(kcH[0], kcH[1]), kL = cat(kcL[0], kcL[1]);
      const bf16x8 aH = cat(acH[0], acH[1]), aL = cat(acL[0], acL[1]);
      const bf16x8 bH = cat(bcH[0], bcH[1]), bL = cat(bcL[0], bcL[1]);
      // A(A_qb), A(A_qk): lane (t = l16, s = 4kg + e); D(A_ak): lane (s = l16, t = 4kg + e); A(A_ab)
      AqbA = mfma16x16x32(bH, rH, AqbA);
      AqkA = mfma16x16x32(kH, rH, AqkA);
      AakD = mfma16x16x32(aH, kH, AakD);
      AabA = mfma16x16x32(bH, aH, AabA);
      AqbA = mfma16x16x32(bH, rL, AqbA);
      AqkA = mfma16x16x32(kH, rL, AqkA);
      AakD = mfma16x16x32(aH, kL, AakD);
      AabA = mfma16x16x32(bH, aL, AabA);
      AqbA = mfma16x16x32(bL, rH, AqbA);
      AqkA = mfma16x16x32(kL, rH, AqkA);
      AakD = mfma16x16x32(aL, kH, AakD);
      AabA = mfma16x16x32(bL, aH, AabA);
    }
    {
      // per channel (one per lane, slot (l16 / 4, l16 % 4) of row kg): 2^{gC - c}
      // and 2^c for the chain's state update, from the totals parked in N
      // (LDS accesses of one wave complete in order; A_ab overwrites N below)
      const float myGC = N[kg][l16];
      const float myCF = rintf(0.5f * myGC);
      const int ci = (int)myCF;
      const int jt = l16 >> 2, e = l16 & 3;
      reinterpret_cast<float*>(&Z.pc[jt][kg])[e] = __builtin_amdgcn_exp2f(clamp126(myGC - myCF));
      reinterpret_cast<float*>(&Z.cen[jt][kg])[e] = __builtin_amdgcn_ldexpf(1.f, ci);
    }
    if (x + 4 < nchunks) issue(x + 4);  // the raw rows are consumed; the next ones land meanwhile
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int s4 = 4 * kg + e;
      AqbA[e] = s4 <= l16 ? AqbA[e] : 0.f;
      AqkA[e] = s4 <= l16 ? AqkA[e] : 0.f;
      AakD[e] = s4 > l16 ? AakD[e] : 0.f;
      AabA[e] = s4 < l16 ? AabA[e] : 0.f;
    }
    // ---- T = (I - A_ab)^{-1} in 8 x 8 blocks, T = [[T11, 0], [T21, T22]]:
    // T11 = (I - N11)^-1 and T22 = (I - N22)^-1 by forward substitution (lane
    // o + c, o in {0, 8}, solves column c of the block at rows/columns o..o+7),
    // then T21 = T22 (N21 T11) on all 64 lanes.  Scratch in N once its blocks
    // are consumed: R = T22 row-major in N[0..7][8..15], X^T = (N21 T11)^T in
    // N[8..15][8..15].  (LDS accesses of one wave complete in order.)
    *reinterpret_cast<float4*>(&N[l16][4 * kg]) = make_float4(AabA[0], AabA[1], AabA[2], AabA[3]);
    if (lane < CH) {
      const int o = lane & 8, c = lane & 7;
      float xc[8];
#pragma unroll
      for (int tt = 0; tt < 8; ++tt) {
        float acc = (tt == c) ? 1.f : 0.f;
#pragma unroll
        for (int u4 = 0; u4 < (tt + 3) / 4; ++u4) {
          const float4 n4 = *reinterpret_cast<const float4*>(&N[o + tt][o + 4 * u4]);
          if (4 * u4 + 0 < tt) acc += n4.x * xc[4 * u4 + 0];
          if (4 * u4 + 1 < tt) acc += n4.y * xc[4 * u4 + 1];
          if (4 * u4 + 2 < tt) acc += n4.z * xc[4 * u4 + 2];
          if (4 * u4 + 3 < tt) acc += n4.w * xc[4 * u4 + 3];
        }
        xc[tt] = acc;
      }
      *reinterpret_cast<float4*>(&Tc[o + c][o]) = make_float4(xc[0], xc[1], xc[2], xc[3]);
      *reinterpret_cast<float4*>(&Tc[o + c][o + 4]) = make_float4(xc[4], xc[5], xc[6], xc[7]);
      // the upper block is zero (for lanes 0-7 this is T21's place, written below)
      *reinterpret_cast<float4*>(&Tc[o + c][8 - o]) = make_float4(0.f, 0.f, 0.f, 0.f);
      *reinterpret_cast<float4*>(&Tc[o + c][12 - o]) = make_float4(0.f, 0.f, 0.f, 0.f);
      if (o) {
#pragma unroll
        for (int tt = 0; tt < 8; ++tt) N[tt][8 + c] = xc[tt];  // R[tt][c] = T22[tt][c]
      }
    }
    {
      const int i = lane >> 3, j = lane & 7;
      // X[i][j] = sum_k N21[i][k] T11[k][j]  (T11[k][j] = Tc[j][k])
      const float4 a0 = *reinterpret_cast<const float4*>(&N[8 + i][0]);
      const float4 a1 = *reinterpret_cast<const float4*>(&N[8 + i][4]);
      const float4 b0 = *reinterpret_cast<const float4*>(&Tc[j][0]);
      const float4 b1 = *reinterpret_cast<const float4*>(&Tc[j][4]);
      const float xij = a0.x * b0.x + a0.y * b0.y + a0.z * b0.z + a0.w * b0.w +
                        a1.x * b1.x + a1.y * b1.y + a1.z * b1.z + a1.w * b1.w;
      N[8 + j][8 + i] = xij;  // X^T
      // T21[i][j] = sum_k T22[i][k] X[k][j] = sum_k R[i][k] X^T[j][k]
      const float4 r0 = *reinterpret_cast<const float4*>(&N[i][8]);
      const float4 r1 = *reinterpret_cast<const float4*>(&N[i][12]);
      const float4 x0 = *reinterpret_cast<const float4*>(&N[8 + j][8]);
      const float4 x1 = *reinterpret_cast<const float4*>(&N[8 + j][12]);
      Tc[j][8 + i] = r0.x * x0.x + r0.y * x0.y + r0.z * x0.z + r0.w * x0.w +
                     r1.x * x1.x + r1.y * x1.y + r1.z * x1.z + r1.w * x1.w;
    }
    // D(T): lane (s = l16, t = 4kg + e); A(T): lane (t = l16, s = 4kg + e)
    f32x4 Dt, At;
    {
      const float4 d4 = *reinterpret_cast<const float4*>(&Tc[l16][4 * kg]);
      Dt = (f32x4){d4.x, d4.y, d4.z, d4.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) At[e] = Tc[4 * kg + e][l16];
    }
    bf16x4 AtH, AtL, DtH, DtL, AakH, AakL, AqbH, AqbL;
    split_f4(At, AtH, AtL);
    split_f4(Dt, DtH, DtL);
    split_f4(AakD, AakH, AakL);
    split_f4(AqbA, AqbH, AqbL);
    // A(M), M = T A_ak;  A(Pm), Pm = A_qb T
    bf16x4 AmH, AmL, ApH, ApL;
    split_f4(mma3_16(AakH, AakL, AtH, AtL), AmH, AmL);
    split_f4(mma3_16(DtH, DtL, AqbH, AqbL), ApH, ApL);

    // ---- Wa = T ac and Rq = rc + Pm ac (lane (t, sigma) layout) replace D(ac) and rc
#pragma unroll
    for (int cc = 0; cc < 2; ++cc) {
      const bf16x8 dH = Z.wa[0][cc][lane], dL = Z.wa[1][cc][lane];
      const f32x4 rc0 = *reinterpret_cast<const f32x4*>(&Z.rq[0][cc][lane]);
      const f32x4 rc1 = *reinterpret_cast<const f32x4*>(&Z.rq[1][cc][lane]);
      bf16x4 waH[2], waL[2], rqH[2], rqL[2];
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const bf16x4 daH = {dH[4 * jj], dH[4 * jj + 1], dH[4 * jj + 2], dH[4 * jj + 3]};
        const bf16x4 daL = {dL[4 * jj], dL[4 * jj + 1], dL[4 * jj + 2], dL[4 * jj + 3]};
        split_f4(mma3_16(daH, daL, AtH, AtL), waH[jj], waL[jj]);
        split_f4((jj ? rc1 : rc0) + mma3_16(daH, daL, ApH, ApL), rqH[jj], rqL[jj]);
      }
      Z.wa[0][cc][lane] = cat(waH[0], waH[1]);
      Z.wa[1][cc][lane] = cat(waL[0], waL[1]);
      Z.rq[0][cc][lane] = cat(rqH[0], rqH[1]);
      Z.rq[1][cc][lane] = cat(rqL[0], rqL[1]);
    }
    // ---- M and Qm = A_qb M + A_qk for the chain's M V and Qm V
    {
      bf16x4 DmH, DmL;
      split_f4(mma3_16(AtH, AtL, AakH, AakL), DmH, DmL);  // D(M) = A(T) x D(A_ak)
      bf16x4 qH, qL;
      split_f4(AqkA + mma3_16(DmH, DmL, AqbH, AqbL), qH, qL);  // A(A_qb M) = D(M) x A(A_qb)
      Z.am[0][lane] = AmH;
      Z.am[1][lane] = AmL;
      Z.aq[0][lane] = qH;
      Z.aq[1][lane] = qL;
    }
    set_flag(&L.ready[s], x);
  }
  // |gC| <= 252 keeps every centred exponent (at most |gC| / 2 + 1/2) within +-126
  const bool clamped = __builtin_amdgcn_ballot_w64(gmin < -252.f || gmax > 252.f) != 0;
  post_status((waited_out ? WKV7_STATUS_TIMEOUT : 0) | (clamped ? WKV7_STATUS_CLAMPED : 0));
}

}  // namespace rwkv7mi

using namespace rwkv7mi;

template <typename TA, typename TW, int WMODE>
static int chunk_go(int64_t B, int64_t T, int64_t H, void* stream, const void* r, const void* w, const void* k,
                    const void* v, const void* kk, const void* a, const float* state_in, float* state_out,
                    void* y) {
  static std::atomic<uint64_t> lds_raised{0};  // devices whose dynamic LDS limit is raised for this instance
  const size_t lds = sizeof(ChunkShared);
  if (int rc = raise_dynamic_lds(reinterpret_cast<const void*>(&wkv7_chunk_kernel<TA, TW, WMODE>), (int)lds,
                                 lds_raised, "wkv7_chunk_kernel"))
    return rc;
  hipLaunchKernelGGL((wkv7_chunk_kernel<TA, TW, WMODE>), dim3((unsigned)(B * H)), dim3(512), lds, as_stream(stream),
                     (const TA*)r, (const TW*)w, (const TA*)k, (const TA*)v, (const TA*)kk, (const TA*)a, state_in,
                     state_out, (TA*)y, (int)T, (int)H);
  return check_launch("wkv7_chunk_kernel");
}

extern "C" int rwkv7mi_wkv7_chunk_prefill(const void* r, const void* w, const void* k, const void* v,
                                          const void* kk, const void* a, const float* state_in,
                                          float* state_out, void* y, int64_t B, int64_t T, int64_t H,
                                          int64_t N, int64_t chunk, int w_is_log, int act_dtype,
                                          int w_dtype, void* stream) {
  if (N != HD) return fail(RWKV7MI_EINVAL, "wkv7 chunk: head size must be 64");
  if (w_is_log < 0 || w_is_log > 2) return fail(RWKV7MI_EINVAL, "wkv7 chunk: w mode must be 0, 1 or 2");
  if (chunk != 16 && chunk != 32 && chunk != 64)
    return fail(RWKV7MI_EINVAL, "wkv7 chunk: chunk must be 16, 32 or 64");
  if (B < 0 || T < 0 || H <= 0) return fail(RWKV7MI_EINVAL, "wkv7 chunk: bad B/T/H");
  if (B == 0) return RWKV7MI_OK;
  if (!state_in || !state_out) return fail(RWKV7MI_EINVAL, "wkv7 chunk: null state");
  if (T > 0 && (!r || !w || !k || !v || !kk || !a || !y)) return fail(RWKV7MI_EINVAL, "wkv7 chunk: null input");
  if ((reinterpret_cast<uintptr_t>(state_in) | reinterpret_cast<uintptr_t>(state_out)) & 15)
    return fail(RWKV7MI_EINVAL, "wkv7 chunk: state must be 16-byte aligned");
  if (B * H > INT32_MAX || T > INT32_MAX) return fail(RWKV7MI_EINVAL, "wkv7 chunk: too large");
  // per-chunk buffer descriptors span 16 tokens of the [B, T, H, 64] inputs
  if (16 * H * HD * 4 > (int64_t)UINT32_MAX) return fail(RWKV7MI_EINVAL, "wkv7 chunk: too many heads");
  return dispatch_dtype(act_dtype, [&](auto ta) {
    using TA = decltype(ta);
    // 16-byte channel runs: every input row must start 16-byte aligned
    const uintptr_t al = reinterpret_cast<uintptr_t>(r) | reinterpret_cast<uintptr_t>(k) |
                         reinterpret_cast<uintptr_t>(v) | reinterpret_cast<uintptr_t>(kk) |
                         reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(w);
    if (al & 15) return fail(RWKV7MI_EINVAL, "wkv7 chunk: inputs must be 16-byte aligned");
    return dispatch_dtype(w_dtype, [&](auto tw) {
      using TW = decltype(tw);
      if (w_is_log == 1) return chunk_go<TA, TW, 1>(B, T, H, stream, r, w, k, v, kk, a, state_in, state_out, y);
      if (w_is_log == 2) return chunk_go<TA, TW, 2>(B, T, H, stream, r, w, k, v, kk, a, state_in, state_out, y);
      return chunk_go<TA, TW, 0>(B, T, H, stream, r, w, k, v, kk, a, state_in, state_out, y);
    });
  });
}

extern "C" int rwkv7mi_wkv7_chunk_status(int clear, int* status) {
  if (!status) return fail(RWKV7MI_EINVAL, "wkv7 chunk status: null output");
  // every kernel issued so far on the device, on any stream, posts first
  if (hipDeviceSynchronize() != hipSuccess) return fail(RWKV7MI_ELAUNCH, "wkv7 chunk status: device error");
  if (hipMemcpyFromSymbol(status, HIP_SYMBOL(wkv7_chunk_status_word), sizeof(int), 0, hipMemcpyDeviceToHost) !=
      hipSuccess)
    return fail(RWKV7MI_ELAUNCH, "wkv7 chunk status: cannot read the status word");
  if (clear) {
    const int zero = 0;
    if (hipMemcpyToSymbol(HIP_SYMBOL(wkv7_chunk_status_word), &zero, sizeof(int), 0, hipMemcpyHostToDevice) !=
        hipSuccess)
      return fail(RWKV7MI_ELAUNCH, "wkv7 chunk status: cannot clear the status word");
  }
  return RWKV7MI_OK;
}
