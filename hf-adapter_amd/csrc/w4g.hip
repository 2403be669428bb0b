// Symmetric group-wise W4 (group 128 / 256) dequant GEMV/GEMM and device packer
// for gfx950.
//
// Format (rwkv7_hf/sm70_quant.py:502-519): weight [O, I] -> packed [O, I/2]
// (byte j of row o = q[o,2j] | q[o,2j+1] << 4, q in [1, 15]) and
// scales [O, I/group];  W[o,i] = (q[o,i] - 8) * scales[o, i/group].
//
// Kernel: v_mfma_f32_16x16x32_f16 with batch rows as M, 16 outputs as N and
// inputs as K.  A workgroup owns 16 output rows; its 4 waves take interleaved
// 128-input blocks (one group-128, or half a group-256).  Lane (n = l%16,
// kg = l/16) loads 16 contiguous bytes of row o0+n, so a wave reads 64
// contiguous bytes per row per block.  Dword s of that load (8 nibbles) is the
// B operand of MFMA step s: nibbles are widened by and/or into fp16
// (1024 + q) pairs in the order [0,4,1,5,2,6,3,7], and a packed add of -1032
// makes the exact value q - 8.  The matching A operand (activations, fp16;
// fp32/bf16 inputs are split hi + lo) is loaded in the same permuted order.
// Each block's 4 MFMAs accumulate from zero, then the lane's per-(o, group)
// scale is applied in fp32.  The 4 waves are reduced through LDS.
//
// Asymmetric (min/max affine) variant, AFF = true: q in [0, 15] with a scale
// and a bias (the group minimum) per (o, group), W[o,i] = q s + b; stored in
// the same packed layout.  With the kernel's centred nibbles (q - 8):
//   sum_i W x = s sum (q - 8) x + (8 s + b) sum_i x,
// and the group sums of x come from one more MFMA per step against a B
// operand of ones, which lands them in the accumulator layout directly.
#include "mm8t_common.h"

namespace rwkv7mi {

template <typename TA>
__device__ __forceinline__ void w4_load_a(const TA* __restrict__ xrow, bool ok, f16x8& hi, f16x8& lo) {
  // returns x[0,4,1,5,2,6,3,7] of the 8 inputs at xrow
  float v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = 0.f;
  if (ok) {
    if constexpr (sizeof(TA) == 2) {
      const uint4 raw = *reinterpret_cast<const uint4*>(xrow);
      const TA* t = reinterpret_cast<const TA*>(&raw);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = to_f32(t[e]);
    } else {
      const float4 p = reinterpret_cast<const float4*>(xrow)[0];
      const float4 q = reinterpret_cast<const float4*>(xrow)[1];
      v[0] = p.x; v[1] = p.y; v[2] = p.z; v[3] = p.w; v[4] = q.x; v[5] = q.y; v[6] = q.z; v[7] = q.w;
    }
  }
  constexpr int perm[8] = {0, 4, 1, 5, 2, 6, 3, 7};
#pragma unroll
  for (int p = 0; p < 8; ++p) {
    const float f = v[perm[p]];
    const _Float16 h = (_Float16)f;
    hi[p] = h;
    lo[p] = (_Float16)(f - (float)h);
  }
}

__device__ __forceinline__ f16x8 w4_nibbles_to_f16(uint32_t d) {
  // d = 8 nibbles n0..n7 (n_{2j} low nibble of byte j); out = [n0,n4,n1,n5,n2,n6,n3,n7] - 8.
  // fp16 pairs with exponent 0x64 hold 1024 + n (nibble in bits 0-3) or
  // 1024 + 16 n (bits 4-7): one packed add of -1032 or one packed fma by
  // 1/16 with -72 gives n - 8 exactly.  9 VALU ops per dword.
  const uint32_t d8 = d >> 8;
  const f16x2 a = __builtin_bit_cast(f16x2, and_or(d, 0x000F000Fu, 0x64006400u));
  const f16x2 b = __builtin_bit_cast(f16x2, and_or(d, 0x00F000F0u, 0x64006400u));
  const f16x2 c = __builtin_bit_cast(f16x2, and_or(d8, 0x000F000Fu, 0x64006400u));
  const f16x2 e = __builtin_bit_cast(f16x2, and_or(d8, 0x00F000F0u, 0x64006400u));
  const f16x2 off = {(_Float16)-1032.0f, (_Float16)-1032.0f};
  const f16x2 sixteenth = {(_Float16)0.0625f, (_Float16)0.0625f};
  const f16x2 off16 = {(_Float16)-72.0f, (_Float16)-72.0f};
  const f16x2 p0 = a + off, p2 = c + off;
  const f16x2 p1 = __builtin_elementwise_fma(b, sixteenth, off16);
  const f16x2 p3 = __builtin_elementwise_fma(e, sixteenth, off16);
  return (f16x8){p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

template <int MT, typename TA, typename TS, bool AFF>
__global__ __launch_bounds__(256) void w4g_kernel(const TA* __restrict__ x, const uint8_t* __restrict__ packed,
                                                  const TS* __restrict__ scales, const TS* __restrict__ gbias,
                                                  const TS* __restrict__ bias, const TA* residual, TA* y, int rows,
                                                  int O, int I, int group, int epilogue) {
  constexpr bool SPLIT = sizeof(TA) != 2 || !std::is_same<TA, __half>::value;
  __shared__ float s_red[16 * MT][16];
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int n = lane & 15;
  const int kg = lane >> 4;
  const int o0 = blockIdx.x * 16;
  const int o = o0 + n;
  const bool ook = o < O;
  const int nblk = I / 128;          // 128-input blocks
  const int ngroups = I / group;
  const int64_t rowbytes = I / 2;

  f32x4 acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = (f32x4){0.f, 0.f, 0.f, 0.f};

  f16x8 ones;
#pragma unroll
  for (int e = 0; e < 8; ++e) ones[e] = (_Float16)1.0f;
  for (int blk = wave; blk < nblk; blk += 4) {
    uint4 wq = make_uint4(0u, 0u, 0u, 0u);
    if (ook) wq = *reinterpret_cast<const uint4*>(packed + (int64_t)o * rowbytes + blk * 64 + 16 * kg);
    const int64_t gi = (int64_t)o * ngroups + (blk * 128) / group;
    const float sc = ook ? ld(scales, gi) : 0.f;
    const float zc = AFF && ook ? 8.f * sc + ld(gbias, gi) : 0.f;  // weight of the group sum of x
    const uint32_t dw[4] = {wq.x, wq.y, wq.z, wq.w};
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int b = 16 * t + n;  // A row of this lane
      f32x4 g = (f32x4){0.f, 0.f, 0.f, 0.f};
      f32x4 gs = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        f16x8 ah, al;
        w4_load_a(x + (int64_t)b * I + blk * 128 + 32 * kg + 8 * s, b < rows, ah, al);
        const f16x8 bv = w4_nibbles_to_f16(dw[s]);
        g = mfma16x16x32(ah, bv, g);
        if constexpr (SPLIT) g = mfma16x16x32(al, bv, g);
        if constexpr (AFF) {
          gs = mfma16x16x32(ah, ones, gs);
          if constexpr (SPLIT) gs = mfma16x16x32(al, ones, gs);
        }
      }
      acc[t] += sc * g;
      if constexpr (AFF) acc[t] += zc * gs;
    }
  }

  // reduce the 4 waves: lane holds C[rows 4kg..4kg+3][col n]
  for (int wv = 0; wv < 4; ++wv) {
    if (wave == wv) {
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float* dst = &s_red[16 * t + 4 * kg + e][n];
          *dst = (wv == 0) ? acc[t][e] : *dst + acc[t][e];
        }
    }
    __syncthreads();
  }
  for (int idx = tid; idx < rows * 16; idx += 256) {
    const int b = idx >> 4, nn = idx & 15;
    const int oo = o0 + nn;
    if (oo >= O) continue;
    float v = s_red[b][nn];
    if (bias) v += ld(bias, oo);
    if (epilogue == RWKV7MI_EPI_RELU2) {
      v = fmaxf(v, 0.f);
      v = v * v;
    } else if (epilogue == RWKV7MI_EPI_RESIDUAL) {
      v += ld(residual, (int64_t)b * O + oo);
    }
    y[(int64_t)b * O + oo] = from_f32<TA>(v);
  }
}

// ---------------------------------------------------------------------------
// Streaming GEMV for 1..16 rows (decode): the weights are read once, in long
// coalesced runs with a load ring in flight, and x is staged in LDS once per
// workgroup instead of re-read from L2 per MFMA.
//
// A workgroup (NW waves) owns 16 output columns at a time and loops over
// column groups g = blockIdx.x, + gridDim.x, ... (persistent).  K is walked in
// 256-input steps (128 bytes of each column): in each chunk wave w takes the
// CSW consecutive steps w CSW .. w CSW + CSW - 1, so its scale (and bias)
// entries are one short run per column, loaded once per (group, chunk) in
// 16-byte loads (the next group's while this one runs) rather than per step;
// lane (n = l%16, kg = l/16) loads bytes 16kg.. and 64 + 16kg.. of
// column n's step, two 16-byte loads whose dwords are the B operands of 8
// MFMAs (nibbles widened to fp16 q - 8, exact).  Each 128-input half of a
// step lies in one scale group (group 128: its own; group 256: half of one),
// so a half's 4 MFMAs accumulate from zero and are scaled once:
//   acc += s[o, grp] * sum_half (q - 8) x          (symmetric)
//       +  (8 s + b)[o, grp] * sum_half x          (affine, the half's x sum
//                                                   from the staging, in LDS)
// x is staged as fp16 in the nibble order [0,4,1,5,2,6,3,7] of each 8-group,
// split hi + lo for fp32 / bf16 activations (two MFMAs per product).  When
// one chunk of KC inputs covers I, x stays staged for all of the workgroup's
// column groups; otherwise each group re-stages its chunks.  Raw buffer loads
// with out-of-range offsets make every load unconditional (tails read zeros).
struct W4tArgs {
  const void* x;        // [rows, I]
  const uint8_t* w;     // [O, I/2]
  const void* scales;   // [O, G]
  const void* gbias;    // [O, G] (affine) or null
  const void* bias;     // [O] or null
  const void* residual; // [rows, O] or null
  void* y;              // [rows, O]
  int rows, I, O, G, gshift, epilogue;  // gshift: log2(group / 128)
  int svec;  // every wave's scale run starts on a 16-byte boundary
};

template <typename TS>
__device__ __forceinline__ uint32_t w4t_ld_raw(__amdgpu_buffer_rsrc_t r, uint32_t e, bool valid) {
  const int off = valid ? (int)(e * (uint32_t)sizeof(TS)) : (int)BUF_OOB;
  if constexpr (sizeof(TS) == 4)
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
  else
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}
template <typename TS>
__device__ __forceinline__ float w4t_raw_f32(uint32_t v) {
  if constexpr (sizeof(TS) == 4)
    return __uint_as_float(v);
  else if constexpr (std::is_same<TS, __half>::value)
    return __half2float(__ushort_as_half((unsigned short)v));
  else
    return __uint_as_float(v << 16);
}

// A wave's scale (and bias) entries of one (column group, chunk): its CSW
// steps are consecutive (steps wave*CSW .. +CSW-1 of the chunk), so their
// 2*CSW 128-input blocks fall in 2*CSW (group 128) or CSW (group 256)
// consecutive groups of the lane's column: raw 16-byte loads of that row of
// the scale matrix, packed TS values.
template <typename TS, int CSW>
struct W4tScales {
  static constexpr int NV = 2 * CSW;                                   // values loaded
  static constexpr int NQ = (NV * (int)sizeof(TS) + 15) / 16;          // 16-byte loads
  u32x4 q[NQ];
  // vec: the run starts on a 16-byte boundary (host-checked for the whole
  // launch); otherwise the values load one by one into the same packing
  __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t r, uint32_t e0, bool ok, bool vec) {
    if (vec) {
#pragma unroll
      for (int i = 0; i < NQ; ++i) q[i] = buf_ld16(r, ok ? e0 * (uint32_t)sizeof(TS) + 16u * i : BUF_OOB);
    } else {
#pragma unroll
      for (int i = 0; i < NQ; ++i) q[i] = (u32x4){0u, 0u, 0u, 0u};
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        const uint32_t x = w4t_ld_raw<TS>(r, e0 + (uint32_t)v, ok);
        if constexpr (sizeof(TS) == 4) q[v >> 2][v & 3] = x;
        else q[v >> 3][(v >> 1) & 3] |= x << (16 * (v & 1));
      }
    }
  }
  // value of 128-input block bi (0 .. 2*CSW-1) of the wave's range
  __device__ __forceinline__ float get(int bi, int gshift) const {
    const int v0 = bi, v1 = bi >> 1;  // both compile-time under unrolling
    const uint32_t a = raw(v0), b = raw(v1);
    return w4t_raw_f32<TS>(gshift ? b : a);
  }
  __device__ __forceinline__ uint32_t raw(int v) const {
    if constexpr (sizeof(TS) == 4) {
      return q[v >> 2][v & 3];
    } else {
      const uint32_t d = q[v >> 3][(v >> 1) & 3];
      return (v & 1) ? d >> 16 : d & 0xffffu;
    }
  }
};

template <typename TA, typename TS, int NW, int CSW, bool AFF>
__global__ __launch_bounds__(64 * NW, 8 / NW) void w4t_kernel(const W4tArgs A) {
  constexpr int NT = 64 * NW;
  constexpr int DEPTH = 2;              // ring steps per wave (2 KB each)
  constexpr int KC = 256 * NW * CSW;    // inputs per staged chunk
  constexpr int XS = KC + 8;            // LDS row stride (halfs)
  constexpr bool HL = !std::is_same<TA, __half>::value;
  static_assert(CSW % DEPTH == 0, "the ring turns whole per chunk");
  const int I = A.I, O = A.O, G = A.G, gshift = A.gshift;
  const int nrows = A.rows;  // 1..16 (checked by the host)
  const int bcol = I / 2;    // bytes per column
  const int ngroups = (O + 15) / 16;
  const int nchunks = (I + KC - 1) / KC;
  const int J = nchunks * CSW;  // steps per wave per column group
  extern __shared__ __align__(16) char smem[];
  _Float16* xh = reinterpret_cast<_Float16*>(smem);
  _Float16* xl = xh + nrows * XS;
  float* gsum = reinterpret_cast<float*>(xh + (HL ? 2 : 1) * nrows * XS);  // [KC / 128][16]
  __shared__ float red[NW][16][17];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int n = lane & 15, kg = lane >> 4;
  const uint32_t lane_off = (uint32_t)n * (uint32_t)bcol + 16u * (uint32_t)kg;

  struct Res {
    __amdgpu_buffer_rsrc_t w, s, b;
  };
  auto group_res = [&](int g) {
    const int nc = g < ngroups ? min(16, O - 16 * g) : 0;
    const int g0 = g < ngroups ? g : 0;
    Res r;
    r.w = make_rsrc(A.w + (int64_t)g0 * 16 * bcol, (uint32_t)nc * (uint32_t)bcol);
    r.s = make_rsrc(reinterpret_cast<const TS*>(A.scales) + (int64_t)g0 * 16 * G, (uint32_t)(nc * G * sizeof(TS)));
    r.b = make_rsrc(AFF ? reinterpret_cast<const TS*>(A.gbias) + (int64_t)g0 * 16 * G : nullptr,
                    AFF ? (uint32_t)(nc * G * sizeof(TS)) : 0u);
    return r;
  };
  // global step of local step jl of chunk c for this wave
  auto gstep = [&](int c, int jl) { return c * (NW * CSW) + wave * CSW + jl; };
  // ring slot: the step's weights
  u32x4 buf[DEPTH][2];
  auto load_step = [&](const Res& r, int j, int d) {
    const int gs = gstep(j / CSW, j % CSW);
    const int b0 = 128 * gs + 16 * kg;
    buf[d][0] = buf_ld16(r.w, b0 < bcol ? lane_off + 128u * (uint32_t)gs : BUF_OOB);
    buf[d][1] = buf_ld16(r.w, b0 + 64 < bcol ? lane_off + 128u * (uint32_t)gs + 64u : BUF_OOB);
  };
  // the wave's scale / bias entries of chunk c of the group behind r
  W4tScales<TS, CSW> sc_cur, sc_next, bi_cur, bi_next;
  auto load_scales = [&](const Res& r, int c, W4tScales<TS, CSW>& sv, W4tScales<TS, CSW>& bv) {
    const int grp0 = (2 * gstep(c, 0)) >> gshift;
    const bool ok = 2 * gstep(c, 0) * 128 < I;
    sv.load(r.s, (uint32_t)(n * G + grp0), ok, A.svec != 0);
    if constexpr (AFF) bv.load(r.b, (uint32_t)(n * G + grp0), ok, A.svec != 0);
  };

  // staging of chunk c: 8-input items (row r, q), 64 consecutive items per
  // wave and pass, so a 16-lane row of a wave covers one 128-input block of
  // one row (its x sum for the affine form is a 16-lane reduction)
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(A.x, (uint32_t)(nrows * I * sizeof(TA)));
  auto stage = [&](int c) {
    constexpr int QPR = KC / 8;  // items per row
    constexpr int SB = 2;        // passes whose loads are in flight together
    const int nitems = nrows * QPR;
    for (int it0 = tid; it0 < nitems; it0 += SB * NT) {
      Raw8<TA> rv[SB];
#pragma unroll
      for (int u = 0; u < SB; ++u) {
        const int it = it0 + u * NT;
        const int r = it / QPR, q = it % QPR;
        const int k = c * KC + 8 * q;
        rv[u] = mm8t_ld8<TA>(xr, (uint32_t)(r * I + k), it < nitems && k < I);
      }
#pragma unroll
      for (int u = 0; u < SB; ++u) {
        const int it = it0 + u * NT;  // wave-uniform validity: nitems is a multiple of 64
        if (it < nitems) {
          const int r = it / QPR, q = it % QPR;
          float v[8];
          mm8t_cvt8(rv[u], v);
          f16x8 hi, lo;
          float sum = 0.f;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float f = v[(e >> 1) + 4 * (e & 1)];
            const _Float16 h = (_Float16)f;
            hi[e] = h;
            lo[e] = (_Float16)(f - (float)h);
            sum += v[e];
          }
          *reinterpret_cast<f16x8*>(xh + r * XS + 8 * q) = hi;
          if constexpr (HL) *reinterpret_cast<f16x8*>(xl + r * XS + 8 * q) = lo;
          if constexpr (AFF) {
            sum = group_sum<16>(sum);
            if ((lane & 15) == 0) gsum[(q >> 4) * 16 + r] = sum;
          }
        }
      }
    }
  };

  const int arow = n < nrows ? n : nrows - 1;
  const _Float16* ah = xh + arow * XS + 32 * kg;
  const _Float16* al = xl + arow * XS + 32 * kg;

  int g = blockIdx.x;
  Res wr = group_res(g), wn = group_res(g + gridDim.x);
#pragma unroll
  for (int d = 0; d < DEPTH; ++d) load_step(wr, d, d);  // DEPTH <= CSW <= J
  load_scales(wr, 0, sc_cur, bi_cur);
  if (nchunks == 1) {
    stage(0);
    __syncthreads();
  }
  const TS* bias = reinterpret_cast<const TS*>(A.bias);
  for (; g < ngroups; g += gridDim.x) {
    f32x4 acc = (f32x4){0.f, 0.f, 0.f, 0.f};
    // the next column group's entries (one chunk), in flight during this group
    if (nchunks == 1) load_scales(wn, 0, sc_next, bi_next);
    for (int c = 0; c < nchunks; ++c) {
      if (nchunks > 1) {
        __syncthreads();  // the previous chunk's (or group's) LDS reads are done
        if (c > 0) load_scales(wr, c, sc_cur, bi_cur);
        stage(c);
        __syncthreads();
      }
      const bool last_chunk = c == nchunks - 1;
#pragma unroll
      for (int jl = 0; jl < CSW; ++jl) {
        const int d = jl % DEPTH;
        f16x8 bv[8];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          bv[q] = w4_nibbles_to_f16(buf[d][0][q]);
          bv[4 + q] = w4_nibbles_to_f16(buf[d][1][q]);
        }
        // refill the slot (from the next column group past the last step)
        const int t = c * CSW + jl + DEPTH;
        if (!last_chunk || jl + DEPTH < CSW)
          load_step(wr, t, d);
        else
          load_step(wn, t - J, d);
        __builtin_amdgcn_sched_barrier(0);
        const int kl = 256 * (wave * CSW + jl);  // chunk-local first input of the step
        f32x4 gh[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          gh[h] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int off = kl + 128 * h + 8 * q;
            gh[h] = mfma16x16x32(*reinterpret_cast<const f16x8*>(ah + off), bv[4 * h + q], gh[h]);
            if constexpr (HL) gh[h] = mfma16x16x32(*reinterpret_cast<const f16x8*>(al + off), bv[4 * h + q], gh[h]);
          }
        }
        const float sc0 = sc_cur.get(2 * jl, gshift), sc1 = sc_cur.get(2 * jl + 1, gshift);
        acc += sc0 * gh[0];
        acc += sc1 * gh[1];
        if constexpr (AFF) {
          const int blk = kl / 128;  // chunk-local 128-input block of half 0
          const f32x4 x0 = *reinterpret_cast<const f32x4*>(gsum + blk * 16 + 4 * kg);
          const f32x4 x1 = *reinterpret_cast<const f32x4*>(gsum + (blk + 1) * 16 + 4 * kg);
          acc += (8.f * sc0 + bi_cur.get(2 * jl, gshift)) * x0;
          acc += (8.f * sc1 + bi_cur.get(2 * jl + 1, gshift)) * x1;
        }
      }
    }
    // ---- waves' partial tiles (lane: column n, rows 4kg..4kg+3), then one
    // thread per (row, column) adds them in wave order and finishes
    __syncthreads();
#pragma unroll
    for (int e = 0; e < 4; ++e) red[wave][4 * kg + e][n] = acc[e];
    __syncthreads();
    if (tid < nrows * 16) {
      const int m = tid >> 4, cn = tid & 15;
      const int o = 16 * g + cn;
      if (o < O) {
        float v = red[0][m][cn];
#pragma unroll
        for (int q = 1; q < NW; ++q) v += red[q][m][cn];
        if (bias) v += ld(bias, o);
        const int64_t oi = (int64_t)m * O + o;
        if (A.epilogue == RWKV7MI_EPI_RELU2) {
          v = fmaxf(v, 0.f);
          v = v * v;
        } else if (A.epilogue == RWKV7MI_EPI_RESIDUAL) {
          v += ld(reinterpret_cast<const TA*>(A.residual), oi);
        }
        reinterpret_cast<TA*>(A.y)[oi] = from_f32<TA>(v);
      }
    }
    wr = wn;
    wn = group_res(g + 2 * gridDim.x);
    if (nchunks == 1) {
      sc_cur = sc_next;
      if constexpr (AFF) bi_cur = bi_next;
    } else {
      load_scales(wr, 0, sc_cur, bi_cur);
    }
  }
}

// Exact restatement of quantize_w4_groupwise (rwkv7_hf/sm70_quant.py:502-519):
// s = max(amax|w| / 7, 1e-6); q = clamp(rint(w / s), -7, 7) + 8 (fp32, RNE).
template <typename TW>
__global__ __launch_bounds__(64) void w4g_pack_kernel(const TW* __restrict__ wt, int O, int I, int group,
                                                      uint8_t* __restrict__ packed, TW* __restrict__ scales) {
  const int ngroups = I / group;
  const int og = blockIdx.x;  // (o, g)
  const int o = og / ngroups, g = og % ngroups;
  const int lane = threadIdx.x;
  const TW* src = wt + (int64_t)o * I + (int64_t)g * group;
  float m = 0.f;
  for (int e = lane; e < group; e += 64) m = fmaxf(m, fabsf(to_f32(src[e])));
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  const float s = fmaxf(__fdiv_rn(m, 7.0f), 1.0e-6f);
  uint8_t* dst = packed + (int64_t)o * (I / 2) + (int64_t)g * (group / 2);
  for (int j = lane; j < group / 2; j += 64) {
    float q0 = rintf(__fdiv_rn(to_f32(src[2 * j]), s));
    float q1 = rintf(__fdiv_rn(to_f32(src[2 * j + 1]), s));
    q0 = fminf(fmaxf(q0, -7.f), 7.f) + 8.f;
    q1 = fminf(fmaxf(q1, -7.f), 7.f) + 8.f;
    dst[j] = (uint8_t)((int)q0 | ((int)q1 << 4));
  }
  if (lane == 0) scales[(int64_t)o * ngroups + g] = from_f32<TW>(s);
}

// Asymmetric group-wise W4 packer (min/max affine, fp32 ops):
// s = max((max - min) / 15, 1e-8) (correctly rounded), b = min,
// q = clamp(rint((w - b) / s), 0, 15); scales and biases stored in the weight
// dtype (round to nearest even).  The group's minimum maps to 0, its maximum to 15.
template <typename TW>
__global__ __launch_bounds__(64) void w4a_pack_kernel(const TW* __restrict__ wt, int O, int I, int group,
                                                      uint8_t* __restrict__ packed, TW* __restrict__ scales,
                                                      TW* __restrict__ biases) {
  const int ngroups = I / group;
  const int og = blockIdx.x;
  const int o = og / ngroups, g = og % ngroups;
  const int lane = threadIdx.x;
  const TW* src = wt + (int64_t)o * I + (int64_t)g * group;
  float mn = INFINITY, mxv = -INFINITY;
  for (int e = lane; e < group; e += 64) {
    const float v = to_f32(src[e]);
    mn = fminf(mn, v);
    mxv = fmaxf(mxv, v);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    mn = fminf(mn, __shfl_xor(mn, off, 64));
    mxv = fmaxf(mxv, __shfl_xor(mxv, off, 64));
  }
  const float s = fmaxf(__fdiv_rn(mxv - mn, 15.0f), 1.0e-8f);
  uint8_t* dst = packed + (int64_t)o * (I / 2) + (int64_t)g * (group / 2);
  for (int j = lane; j < group / 2; j += 64) {
    float q0 = rintf(__fdiv_rn(to_f32(src[2 * j]) - mn, s));
    float q1 = rintf(__fdiv_rn(to_f32(src[2 * j + 1]) - mn, s));
    q0 = fminf(fmaxf(q0, 0.f), 15.f);
    q1 = fminf(fmaxf(q1, 0.f), 15.f);
    dst[j] = (uint8_t)((int)q0 | ((int)q1 << 4));
  }
  if (lane == 0) {
    scales[(int64_t)o * ngroups + g] = from_f32<TW>(s);
    biases[(int64_t)o * ngroups + g] = from_f32<TW>(mn);
  }
}

}  // namespace rwkv7mi

using namespace rwkv7mi;

extern "C" int rwkv7mi_w4a_pack(const void* weight, int64_t O, int64_t I, int64_t group, int w_dtype,
                                uint8_t* packed, void* scales, void* biases, void* stream) {
  if (group != 128 && group != 256) return fail(RWKV7MI_EINVAL, "w4a_pack: group must be 128 or 256");
  if (O <= 0 || I <= 0 || I % group) return fail(RWKV7MI_EINVAL, "w4a_pack: I must be a positive multiple of group");
  if (O * (I / group) > INT32_MAX || I > INT32_MAX) return fail(RWKV7MI_EINVAL, "w4a_pack: too large");
  if (!weight || !packed || !scales || !biases) return fail(RWKV7MI_EINVAL, "w4a_pack: null pointer");
  return dispatch_dtype(w_dtype, [&](auto tw) {
    using TW = decltype(tw);
    hipLaunchKernelGGL((w4a_pack_kernel<TW>), dim3((unsigned)(O * (I / group))), dim3(64), 0, as_stream(stream),
                       (const TW*)weight, (int)O, (int)I, (int)group, packed, (TW*)scales, (TW*)biases);
    return check_launch("w4a_pack_kernel");
  });
}

extern "C" int rwkv7mi_w4g_pack(const void* weight, int64_t O, int64_t I, int64_t group, int w_dtype,
                                uint8_t* packed, void* scales, void* stream) {
  if (group != 128 && group != 256) return fail(RWKV7MI_EINVAL, "w4g_pack: group must be 128 or 256");
  if (O <= 0 || I <= 0 || I % group) return fail(RWKV7MI_EINVAL, "w4g_pack: I must be a positive multiple of group");
  if (O * (I / group) > INT32_MAX || I > INT32_MAX) return fail(RWKV7MI_EINVAL, "w4g_pack: too large");
  if (!weight || !packed || !scales) return fail(RWKV7MI_EINVAL, "w4g_pack: null pointer");
  return dispatch_dtype(w_dtype, [&](auto tw) {
    using TW = decltype(tw);
    hipLaunchKernelGGL((w4g_pack_kernel<TW>), dim3((unsigned)(O * (I / group))), dim3(64), 0, as_stream(stream),
                       (const TW*)weight, (int)O, (int)I, (int)group, packed, (TW*)scales);
    return check_launch("w4g_pack_kernel");
  });
}

// Streaming GEMV plan (rows <= 16): waves per workgroup and steps per wave per
// chunk.  Eight-wave workgroups (one per CU) when the column groups do not
// fill two four-wave workgroups per CU; the smallest chunk that holds all of
// I when its LDS fits (x then stays staged for every column group), else the
// largest that fits (re-staged per group).  Returns the LDS bytes (0: none fits).
static size_t w4t_lds(int64_t rows, int kc, bool hl, bool aff) {
  return (size_t)rows * (size_t)(kc + 8) * 2u * (hl ? 2u : 1u) + (aff ? (size_t)(kc / 128) * 16u * 4u : 0u);
}
static size_t w4t_plan(int64_t rows, int64_t I, int64_t O, bool hl, bool aff, int* nw, int* csw) {
  constexpr size_t TWO = 64 * 1024, ONE = 144 * 1024;  // per workgroup: two per CU / one per CU
  struct C { int nw, csw; };
  static const C cands[] = {{4, 2}, {4, 4}, {8, 2}, {4, 16}, {8, 8}};  // chunks 2K, 4K, 4K, 16K, 16K inputs
  const int64_t ngroups = (O + 15) / 16;
  const int want = ngroups <= mm8t_cus() ? 8 : 4;
  for (int pass = 0; pass < 2; ++pass) {  // whole-I chunks: the preferred width, then the other
    const int wnw = pass == 0 ? want : 12 - want;
    for (const C& c : cands) {
      const int kc = 256 * c.nw * c.csw;
      const size_t lds = w4t_lds(rows, kc, hl, aff);
      if (aff && c.nw == 4 && c.csw == 16) continue;  // (that instance runs out of registers)
      if (c.nw == wnw && kc >= I && lds <= (c.nw == 4 ? TWO : ONE)) {
        *nw = c.nw, *csw = c.csw;
        return lds;
      }
    }
  }
  for (int i = 4; i >= 0; --i) {  // several chunks: the longest that fits one workgroup per CU
    if (aff && cands[i].nw == 4 && cands[i].csw == 16) continue;
    const int kc = 256 * cands[i].nw * cands[i].csw;
    const size_t lds = w4t_lds(rows, kc, hl, aff);
    if (kc < I && lds <= ONE) {
      *nw = cands[i].nw, *csw = cands[i].csw;
      return lds;
    }
  }
  return 0;
}

template <typename TA, typename TS, int NW, int CSW, bool AFF>
static int w4t_launch(dim3 grid, size_t lds, void* stream, const W4tArgs& a) {
  static std::atomic<uint64_t> raised{0};  // devices whose dynamic LDS limit is raised for this instance
  if (int rc = raise_dynamic_lds(reinterpret_cast<const void*>(&w4t_kernel<TA, TS, NW, CSW, AFF>), 144 * 1024 + 1024,
                                 raised, "w4t_kernel"))
    return rc;
  hipLaunchKernelGGL((w4t_kernel<TA, TS, NW, CSW, AFF>), grid, dim3(64 * NW), lds, as_stream(stream), a);
  return check_launch("w4t_kernel");
}

template <typename TA, typename TS, bool AFF>
static int w4t_go(int nw, int csw, dim3 grid, size_t lds, void* stream, const W4tArgs& a) {
  if (nw == 4) {
    if (csw == 2) return w4t_launch<TA, TS, 4, 2, AFF>(grid, lds, stream, a);
    if (csw == 4) return w4t_launch<TA, TS, 4, 4, AFF>(grid, lds, stream, a);
    if constexpr (!AFF) return w4t_launch<TA, TS, 4, 16, AFF>(grid, lds, stream, a);
    return fail(RWKV7MI_EINVAL, "w4t_kernel: no affine instance with that chunk");
  }
  if (csw == 2) return w4t_launch<TA, TS, 8, 2, AFF>(grid, lds, stream, a);
  return w4t_launch<TA, TS, 8, 8, AFF>(grid, lds, stream, a);
}

static int w4_matmul(const char* who, const void* x, const uint8_t* packed, const void* scales, const void* gbias,
                     const void* bias, const void* residual, void* y, int64_t rows, int64_t O, int64_t I,
                     int64_t group, int epilogue, int act_dtype, int scale_dtype, void* stream) {
  const std::string w(who);
  if (group != 128 && group != 256) return fail(RWKV7MI_EINVAL, w + ": group must be 128 or 256");
  if (rows < 0 || O <= 0 || I <= 0 || I % group) return fail(RWKV7MI_EINVAL, w + ": bad shape");
  if (rows == 0) return RWKV7MI_OK;
  if (O > INT32_MAX || I > INT32_MAX) return fail(RWKV7MI_EINVAL, w + ": too large");
  if (!x || !packed || !scales || !y) return fail(RWKV7MI_EINVAL, w + ": null pointer");
  if (epilogue < 0 || epilogue > 2) return fail(RWKV7MI_EINVAL, w + ": bad epilogue");
  if (epilogue == RWKV7MI_EPI_RESIDUAL && !residual) return fail(RWKV7MI_EINVAL, w + ": residual missing");
  if ((reinterpret_cast<uintptr_t>(packed) | reinterpret_cast<uintptr_t>(x)) & 15)
    return fail(RWKV7MI_EINVAL, w + ": x and packed must be 16-byte aligned");
  if (!valid_dtype(act_dtype) || !valid_dtype(scale_dtype)) return fail(RWKV7MI_EINVAL, w + ": bad dtype");
  const size_t esz = act_dtype == RWKV7MI_F32 ? 4 : 2;
  if (rows <= 16 && I <= (1 << 22) && (int64_t)rows * I * (int64_t)esz <= INT32_MAX &&
      16 * (I / 2) <= INT32_MAX) {
    int nw = 4, csw = 4;
    const bool hl = act_dtype != RWKV7MI_F16, aff = gbias != nullptr;
    const size_t lds = w4t_plan(rows, I, O, hl, aff, &nw, &csw);
    if (lds) {
      const int G = (int)(I / group), gsh = group == 256 ? 1 : 0;
      const size_t ssz = scale_dtype == RWKV7MI_F32 ? 4 : 2;
      // a wave's run starts at n G + (2 CSW (c NW + w) >> gshift) entries
      const bool svec = (G * ssz) % 16 == 0 && (((size_t)(2 * csw) >> gsh) * ssz) % 16 == 0 &&
                        (reinterpret_cast<uintptr_t>(scales) & 15) == 0 &&
                        (!gbias || (reinterpret_cast<uintptr_t>(gbias) & 15) == 0);
      W4tArgs a{x, packed, scales, gbias, bias, residual, y, (int)rows, (int)I, (int)O, G, gsh, epilogue,
                svec ? 1 : 0};
      const int64_t ngroups = (O + 15) / 16;
      const int64_t per_cu = nw == 4 && lds <= 64 * 1024 ? 2 : 1;
      const int64_t gx = std::min<int64_t>(ngroups, mm8t_cus() * per_cu);
      const dim3 grid((unsigned)gx);
      return dispatch_dtype(act_dtype, [&](auto ta) {
        using TA = decltype(ta);
        return dispatch_dtype(scale_dtype, [&](auto ts) {
          using TS = decltype(ts);
          return aff ? w4t_go<TA, TS, true>(nw, csw, grid, lds, stream, a)
                     : w4t_go<TA, TS, false>(nw, csw, grid, lds, stream, a);
        });
      });
    }
  }
  for (int64_t r0 = 0; r0 < rows; r0 += 64) {
    const int64_t nr = rows - r0 > 64 ? 64 : rows - r0;
    const int mt = nr <= 16 ? 1 : nr <= 32 ? 2 : 4;
    const char* xr = reinterpret_cast<const char*>(x) + r0 * I * esz;
    char* yr = reinterpret_cast<char*>(y) + r0 * O * esz;
    const char* rr = residual ? reinterpret_cast<const char*>(residual) + r0 * O * esz : nullptr;
    int rc = dispatch_dtype(act_dtype, [&](auto ta) {
      using TA = decltype(ta);
      return dispatch_dtype(scale_dtype, [&](auto ts) {
        using TS = decltype(ts);
        dim3 grid((unsigned)((O + 15) / 16));
#define W4_LAUNCH(MT_, AFF_)                                                                              \
  hipLaunchKernelGGL((w4g_kernel<MT_, TA, TS, AFF_>), grid, dim3(256), 0, as_stream(stream), (const TA*)xr, \
                     packed, (const TS*)scales, (const TS*)gbias, (const TS*)bias, (const TA*)rr, (TA*)yr,   \
                     (int)nr, (int)O, (int)I, (int)group, epilogue)
        if (gbias) {
          if (mt == 1) W4_LAUNCH(1, true);
          else if (mt == 2) W4_LAUNCH(2, true);
          else W4_LAUNCH(4, true);
        } else {
          if (mt == 1) W4_LAUNCH(1, false);
          else if (mt == 2) W4_LAUNCH(2, false);
          else W4_LAUNCH(4, false);
        }
#undef W4_LAUNCH
        return check_launch("w4g_kernel");
      });
    });
    if (rc) return rc;
  }
  return RWKV7MI_OK;
}

extern "C" int rwkv7mi_w4g_matmul(const void* x, const uint8_t* packed, const void* scales, const void* bias,
                                  const void* residual, void* y, int64_t rows, int64_t O, int64_t I,
                                  int64_t group, int epilogue, int act_dtype, int scale_dtype, void* stream) {
  return w4_matmul("w4g_matmul", x, packed, scales, nullptr, bias, residual, y, rows, O, I, group, epilogue,
                   act_dtype, scale_dtype, stream);
}

extern "C" int rwkv7mi_w4a_matmul(const void* x, const uint8_t* packed, const void* scales, const void* biases,
                                  const void* bias, const void* residual, void* y, int64_t rows, int64_t O,
                                  int64_t I, int64_t group, int epilogue, int act_dtype, int scale_dtype,
                                  void* stream) {
  if (!biases) return fail(RWKV7MI_EINVAL, "w4a_matmul: null group biases");
  return w4_matmul("w4a_matmul", x, packed, scales, biases, bias, residual, y, rows, O, I, group, epilogue,
                   act_dtype, scale_dtype, stream);
}
