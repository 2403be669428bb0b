// MM8 (uint8 affine, per-row + per-column scale/offset) dequant GEMV/GEMM and
// the device packer, for gfx950.
//
// Format (rwkv7_hf/native_quant_mm8.py:62-126): W = weight.T is [I, O],
//   W_hat[i,o] = (w_u8[i,o] + 0.5) * ry[i] * rx[o] + my[i] + mx[o]
// so  y[b,o] = rx[o] * sum_i x'[b,i] (w_u8[i,o] + 0.5) + sum_i x[b,i] my[i]
//            + mx[o] * sum_i x[b,i],         x' = x * ry.
//
// Kernel: the big term runs on v_mfma_f32_16x16x32_f16.  Batch rows are the
// MFMA M dimension (16 per tile), the 32-row k-step is K, and 16 output
// columns are N.  A workgroup owns a 128-column strip of W (one 128-byte line
// per row) and a K-range; its four waves take interleaved 32-row k-steps.
// Lane (n = l%16, kg = l/16) loads 8 bytes (8 columns) from each of 8 rows,
// i.e. every row segment a wave touches is 128 contiguous bytes.  For byte
// position c of those 8 columns, two v_perm_b32 per row pair gather the 8
// rows' bytes into fp16 (1024 + w), and one packed add of -1023.5 makes the
// exact fp16 value w + 0.5 — the MFMA B operand for output column 8n + c.
// x' is staged once per workgroup in LDS as fp16 hi + lo (x' = hi + lo to
// ~22 bits), so the product uses two MFMAs and keeps fp32-class accuracy.
// The two per-row sums are plain fp32 reductions during staging.
//
// Split-K: workgroups of one strip write fp32 partials to the workspace; the
// last one to finish (per-strip counter) reduces them in fixed order, applies
// the affine terms and the epilogue, and resets the counter to zero.
#include "common.h"

namespace rwkv7mi {

constexpr int MM8_STRIP = 128;
constexpr int MM8_COUNTERS = 16384;               // counter slots (max strips)
constexpr size_t MM8_COUNTER_BYTES = MM8_COUNTERS * 4;
constexpr int MM8_PSTRIDE = MM8_STRIP + 2;        // partial row: 128 cols + sx + sxmy

__device__ __forceinline__ f16x8 mm8_bytes_to_f16(const uint32_t (&d)[8], int c) {
  // d[i] = dword (c/4) of row i; returns [w(r0,c)+0.5, ..., w(r7,c)+0.5]
  const uint32_t q = c & 3;
  const uint32_t sel_pair = q | ((q + 4) << 8) | (q << 16) | ((q + 4) << 24);
  f16x8 out;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    uint32_t p = __builtin_amdgcn_perm(d[2 * j + 1], d[2 * j], sel_pair);  // [r2j, r2j+1, ..]
    uint32_t hv = __builtin_amdgcn_perm(0x64646464u, p, 0x04010400u);      // [b0,64,b1,64]
    f16x2 h = __builtin_bit_cast(f16x2, hv);
    h = h + (f16x2){(_Float16)-1023.5f, (_Float16)-1023.5f};
    out[2 * j] = h[0];
    out[2 * j + 1] = h[1];
  }
  return out;
}

template <int MT, bool SPLIT, typename TA, typename TM>
__global__ __launch_bounds__(256) void mm8_kernel(
    const TA* __restrict__ x, const uint8_t* __restrict__ w, const TM* __restrict__ mx,
    const TM* __restrict__ rx, const TM* __restrict__ my, const TM* __restrict__ ry,
    const TM* __restrict__ bias, const TA* residual, TA* y, int rows,
    int I, int O, int KR, int ksplit, int epilogue, float* part, unsigned* cnt) {
  constexpr int R = 16 * MT;
  extern __shared__ __align__(16) char smem[];
  const int XS = KR + 8;  // padded LDS row stride (halfs)
  _Float16* xh = reinterpret_cast<_Float16*>(smem);
  _Float16* xl = xh + R * XS;
  float* s_sum = reinterpret_cast<float*>(xl + (SPLIT ? R * XS : 0));  // [R][2]
  float* s_red = s_sum + 2 * R;                                         // [R][128]
  __shared__ int s_last;

  const int strip = blockIdx.x;
  const int z = blockIdx.y;
  const int nstrips = gridDim.x;
  const int c0 = strip * MM8_STRIP;
  const int k0 = z * KR;
  const int kn = min(KR, I - k0);
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;

  // ---- stage x' = x * ry as fp16 hi/lo, and the per-row sums over this K-range
  for (int b = wave; b < R; b += 4) {
    float sx = 0.f, sxmy = 0.f;
    for (int kk = lane; kk < KR; kk += 64) {
      float xp = 0.f;
      if (b < rows && kk < kn) {
        const float xv = ld(x, (int64_t)b * I + k0 + kk);
        xp = xv * ld(ry, k0 + kk);
        sx += xv;
        sxmy += xv * ld(my, k0 + kk);
      }
      const _Float16 hi = (_Float16)xp;
      xh[b * XS + kk] = hi;
      if constexpr (SPLIT) xl[b * XS + kk] = (_Float16)(xp - (float)hi);
    }
    sx = wave_sum(sx);
    sxmy = wave_sum(sxmy);
    if (lane == 0) {
      s_sum[2 * b] = sx;
      s_sum[2 * b + 1] = sxmy;
    }
  }
  __syncthreads();

  // ---- main loop
  const int n = lane & 15;
  const int kg = lane >> 4;
  const int col = c0 + 8 * n;
  const bool colok = col < O;
  f32x4 acc[MT][8];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[t][c] = (f32x4){0.f, 0.f, 0.f, 0.f};

  for (int ks = wave * 32; ks < kn; ks += 128) {
    uint32_t lo[8], hi[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int row = k0 + ks + 8 * kg + i;
      if (colok && row < I) {
        const uint2 v2 = *reinterpret_cast<const uint2*>(w + (int64_t)row * O + col);
        lo[i] = v2.x;
        hi[i] = v2.y;
      } else {
        lo[i] = 0u;
        hi[i] = 0u;
      }
    }
    f16x8 ah[MT], al[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int off = (16 * t + n) * XS + ks + 8 * kg;
      ah[t] = *reinterpret_cast<const f16x8*>(xh + off);
      if constexpr (SPLIT) al[t] = *reinterpret_cast<const f16x8*>(xl + off);
    }
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const f16x8 bv = (c < 4) ? mm8_bytes_to_f16(lo, c) : mm8_bytes_to_f16(hi, c);
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        acc[t][c] = mfma16x16x32(ah[t], bv, acc[t][c]);
        if constexpr (SPLIT) acc[t][c] = mfma16x16x32(al[t], bv, acc[t][c]);
      }
    }
  }

  // ---- reduce the 4 waves: s_red[b][cc], b = 16t + 4kg + e, cc = 8n + c
  for (int wv = 0; wv < 4; ++wv) {
    if (wave == wv) {
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int c = 0; c < 8; ++c)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int b = 16 * t + 4 * kg + e;
            float* dst = s_red + b * MM8_STRIP + 8 * n + c;
            *dst = (wv == 0) ? acc[t][c][e] : *dst + acc[t][c][e];
          }
    }
    __syncthreads();
  }

  const int ncols = min(MM8_STRIP, O - c0);
  if (ksplit > 1) {
    float* mine = part + ((int64_t)z * nstrips + strip) * R * MM8_PSTRIDE;
    for (int idx = tid; idx < rows * MM8_STRIP; idx += 256) {
      const int b = idx / MM8_STRIP, cc = idx % MM8_STRIP;
      mine[b * MM8_PSTRIDE + cc] = s_red[b * MM8_STRIP + cc];
    }
    for (int b = tid; b < rows; b += 256) {
      mine[b * MM8_PSTRIDE + MM8_STRIP] = s_sum[2 * b];
      mine[b * MM8_PSTRIDE + MM8_STRIP + 1] = s_sum[2 * b + 1];
    }
    __threadfence();
    __syncthreads();
    if (tid == 0) s_last = (atomicAdd(&cnt[strip], 1u) == (unsigned)(ksplit - 1));
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    // fixed-order reduction of all K-ranges of this strip into LDS
    for (int idx = tid; idx < rows * MM8_PSTRIDE; idx += 256) {
      const int b = idx / MM8_PSTRIDE, cc = idx % MM8_PSTRIDE;
      float s = 0.f;
      for (int zz = 0; zz < ksplit; ++zz)
        s += __builtin_nontemporal_load(part + ((int64_t)zz * nstrips + strip) * R * MM8_PSTRIDE +
                                        b * MM8_PSTRIDE + cc);
      if (cc < MM8_STRIP) s_red[b * MM8_STRIP + cc] = s;
      else s_sum[2 * b + (cc - MM8_STRIP)] = s;
    }
    __syncthreads();
    if (tid == 0) atomicExch(&cnt[strip], 0u);
  }

  // ---- epilogue
  for (int idx = tid; idx < rows * MM8_STRIP; idx += 256) {
    const int b = idx / MM8_STRIP, cc = idx % MM8_STRIP;
    if (cc >= ncols) continue;
    const int o = c0 + cc;
    float v = ld(rx, o) * s_red[b * MM8_STRIP + cc] + s_sum[2 * b + 1] + ld(mx, o) * s_sum[2 * b];
    if (bias) v += ld(bias, o);
    if (epilogue == RWKV7MI_EPI_RELU2) {
      v = fmaxf(v, 0.f);
      v = v * v;
    } else if (epilogue == RWKV7MI_EPI_RESIDUAL) {
      v += ld(residual, (int64_t)b * O + o);
    }
    y[(int64_t)b * O + o] = from_f32<TA>(v);
  }
}

struct Mm8Plan {
  int mt, KR, ksplit, nstrips;
  size_t lds;
};

static Mm8Plan mm8_plan(int64_t rows, int64_t I, int64_t O) {
  Mm8Plan p;
  p.mt = rows <= 16 ? 1 : rows <= 32 ? 2 : 4;
  const int R = 16 * p.mt;
  const bool split = p.mt == 1;
  p.nstrips = (int)((O + MM8_STRIP - 1) / MM8_STRIP);
  const int64_t ksteps = (I + 127) / 128;
  int64_t want = (512 + p.nstrips - 1) / p.nstrips;
  if (want < 1) want = 1;
  if (want > ksteps) want = ksteps;
  int64_t KR = ((I + want - 1) / want + 127) / 128 * 128;
  // dynamic LDS (x' staging + reduction tile) stays below 64 KB
  const int64_t kr_cap = p.mt == 4 ? 128 : 512;
  if (KR > kr_cap) KR = kr_cap;
  if (KR < 128) KR = 128;
  p.KR = (int)KR;
  p.ksplit = (int)((I + KR - 1) / KR);
  p.lds = (size_t)R * (KR + 8) * 2 * (split ? 2 : 1) + (size_t)2 * R * 4 + (size_t)R * MM8_STRIP * 4;
  return p;
}

// ------------------------------------------------------------------ packer
// Exact restatement of quantize_mm8 (rwkv7_hf/native_quant_mm8.py:62-97) as a
// sequence of IEEE fp32 ops; every reduction is a min/max (order-independent),
// every division is correctly rounded, so the result is bit-exact.
//
// Element (i, j) of the [I, O] matrix W = weight.T lives at i*O + j (row-major,
// OM = false) or at j*I + i (out-major, OM = true: nn.Linear.weight itself).
// Per-out statistics (mx, rx) reduce over i, per-in ones (my, ry) over j.
// Or real output columns are stored; columns Or.. of a padded matrix read as 0
// (the zero pad column rwkv7_hf/native_quant_mm4.py:89-92 appends).
template <typename TW, bool OM>
__device__ __forceinline__ float mm8_w(const TW* w, int i, int j, int I, int Or) {
  if (j >= Or) return 0.f;
  return to_f32(OM ? w[(int64_t)j * I + i] : w[(int64_t)i * Or + j]);
}

// One reduction term.  phase 0: min w; 1: min (w - other offset);
// 2: max of the offset-removed value (per-in: divided by rx[j]).
template <bool PER_OUT>
__device__ __forceinline__ float mm8_term(float v, int i, int j, int phase, bool rows_first, const float* my,
                                          const float* mx, const float* rx) {
  if (phase == 0) return v;
  if (phase == 1) return PER_OUT ? v - my[i] : v - mx[j];
  const float w2 = rows_first ? (v - my[i]) - mx[j] : (v - mx[j]) - my[i];
  return PER_OUT ? w2 : __fdiv_rn(w2, rx[j]);
}

template <bool PER_OUT>
__device__ __forceinline__ void mm8_stat_store(float m, int line, int phase, float* ws, int I, int O) {
  float* dst = PER_OUT ? (phase == 2 ? ws + I + O : ws + I) : (phase == 2 ? ws + I + 2 * O : ws);
  dst[line] = phase == 2 ? fmaxf(m, 1.0e-8f) : m;
}

// One workgroup per line; coalesced when the line is contiguous (PER_OUT == OM).
template <typename TW, bool OM, bool PER_OUT>
__global__ __launch_bounds__(256) void mm8_stat_line(const TW* __restrict__ w, int I, int O, int Or, int phase,
                                                    float* ws) {
  const float* my = ws;
  const float* mx = ws + I;
  const float* rx = ws + I + O;
  __shared__ float red[4];
  const int line = blockIdx.x;
  const int len = PER_OUT ? I : O;
  const bool rows_first = I > O;
  float m = phase == 2 ? -INFINITY : INFINITY;
  for (int t = threadIdx.x; t < len; t += 256) {
    const int i = PER_OUT ? t : line, j = PER_OUT ? line : t;
    const float v = mm8_term<PER_OUT>(mm8_w<TW, OM>(w, i, j, I, Or), i, j, phase, rows_first, my, mx, rx);
    m = phase == 2 ? fmaxf(m, v) : fminf(m, v);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float t = __shfl_xor(m, o, 64);
    m = phase == 2 ? fmaxf(m, t) : fminf(m, t);
  }
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    float r = red[0];
    for (int q = 1; q < 4; ++q) r = phase == 2 ? fmaxf(r, red[q]) : fminf(r, red[q]);
    mm8_stat_store<PER_OUT>(r, line, phase, ws, I, O);
  }
}

// One thread per line; coalesced across threads when the line is strided (PER_OUT != OM).
template <typename TW, bool OM, bool PER_OUT>
__global__ __launch_bounds__(256) void mm8_stat_thread(const TW* __restrict__ w, int I, int O, int Or, int phase,
                                                       float* ws) {
  const float* my = ws;
  const float* mx = ws + I;
  const float* rx = ws + I + O;
  const int line = blockIdx.x * 256 + threadIdx.x;
  const int nlines = PER_OUT ? O : I;
  if (line >= nlines) return;
  const int len = PER_OUT ? I : O;
  const bool rows_first = I > O;
  float m = phase == 2 ? -INFINITY : INFINITY;
  for (int t = 0; t < len; ++t) {
    const int i = PER_OUT ? t : line, j = PER_OUT ? line : t;
    const float v = mm8_term<PER_OUT>(mm8_w<TW, OM>(w, i, j, I, Or), i, j, phase, rows_first, my, mx, rx);
    m = phase == 2 ? fmaxf(m, v) : fminf(m, v);
  }
  mm8_stat_store<PER_OUT>(m, line, phase, ws, I, O);
}

template <typename TW, bool OM>
__global__ void mm8_quantize(const TW* __restrict__ wt, int I, int O, const float* ws,
                             uint8_t* __restrict__ wu8, TW* mx_o, TW* rx_o, TW* my_o, TW* ry_o) {
  const float* my = ws;
  const float* mx = ws + I;
  const float* rx = ws + I + O;
  const float* ry = ws + I + 2 * O;
  const bool rows_first = I > O;
  const int64_t total = (int64_t)I * O;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int i = OM ? (int)(e % I) : (int)(e / O);
    const int j = OM ? (int)(e / I) : (int)(e % O);
    float v = to_f32(wt[e]);
    float w2 = rows_first ? (v - my[i]) - mx[j] : (v - mx[j]) - my[i];
    float w4 = __fdiv_rn(__fdiv_rn(w2, rx[j]), ry[i]);
    float q = floorf(w4 * 256.0f);
    q = fminf(fmaxf(q, 0.0f), 255.0f);
    wu8[e] = (uint8_t)q;
    if (i == 0) {
      mx_o[j] = from_f32<TW>(mx[j]);
      rx_o[j] = from_f32<TW>(rx[j] / 16.0f);
    }
    if (j == 0) {
      my_o[i] = from_f32<TW>(my[i]);
      ry_o[i] = from_f32<TW>(ry[i] / 16.0f);
    }
  }
}

template <typename TW, bool OM, bool PER_OUT>
static void mm8_stat(const TW* w, int I, int O, int Or, int phase, float* ws, hipStream_t s) {
  const int nlines = PER_OUT ? O : I;
  if (PER_OUT == OM)
    hipLaunchKernelGGL((mm8_stat_line<TW, OM, PER_OUT>), dim3((unsigned)nlines), dim3(256), 0, s, w, I, O, Or, phase,
                       ws);
  else
    hipLaunchKernelGGL((mm8_stat_thread<TW, OM, PER_OUT>), dim3((unsigned)((nlines + 255) / 256)), dim3(256), 0, s,
                       w, I, O, Or, phase, ws);
}

// the statistics passes of the reference (rwkv7_hf/native_quant_mm8.py:66-80,
// rwkv7_hf/native_quant_mm4.py:93-100) over O logical columns, Or of them stored
template <typename TW, bool OM>
static void mm8_stats(const TW* w, int I, int O, int Or, float* ws, hipStream_t s) {
  if (I > O) {  // rows first
    mm8_stat<TW, OM, false>(w, I, O, Or, 0, ws, s);
    mm8_stat<TW, OM, true>(w, I, O, Or, 1, ws, s);
  } else {
    mm8_stat<TW, OM, true>(w, I, O, Or, 0, ws, s);
    mm8_stat<TW, OM, false>(w, I, O, Or, 1, ws, s);
  }
  mm8_stat<TW, OM, true>(w, I, O, Or, 2, ws, s);
  mm8_stat<TW, OM, false>(w, I, O, Or, 2, ws, s);
}

template <typename TW, bool OM>
static int mm8_pack_run(const TW* w, int I, int O, uint8_t* w_u8, void* mx, void* rx, void* my, void* ry,
                        float* ws, hipStream_t s) {
  mm8_stats<TW, OM>(w, I, O, O, ws, s);
  hipLaunchKernelGGL((mm8_quantize<TW, OM>), dim3(4096), dim3(256), 0, s, w, I, O, ws, w_u8, (TW*)mx, (TW*)rx,
                     (TW*)my, (TW*)ry);
  return check_launch("mm8_pack");
}

// MM4 affine (rwkv7_hf/native_quant_mm4.py:77-105): 16 levels over the O = Mp
// (even) logical columns.  OM = false: packed [I, O/2], byte (i, b) =
// q(i, 2b) | q(i, 2b+1) << 4 (the reference layout); OM = true: packed
// [O, I/2], byte (j, a) = q(2a, j) | q(2a+1, j) << 4 (pairs along the inputs,
// the fused GEMV's layout; the pad column's nibbles are kept as a last row).
template <typename TW, bool OM>
__device__ __forceinline__ uint32_t mm4_q(const TW* w, int i, int j, int I, int Or, bool rows_first,
                                          const float* my, const float* mx, const float* rx, const float* ry) {
  const float v = mm8_w<TW, OM>(w, i, j, I, Or);
  const float w2 = rows_first ? (v - my[i]) - mx[j] : (v - mx[j]) - my[i];
  const float w4 = __fdiv_rn(__fdiv_rn(w2, rx[j]), ry[i]);
  float q = floorf(w4 * 16.0f);
  q = fminf(fmaxf(q, 0.0f), 15.0f);
  return (uint32_t)q;
}

template <typename TW, bool OM>
__global__ void mm4_quantize(const TW* __restrict__ w, int I, int O, int Or, const float* ws,
                             uint8_t* __restrict__ packed) {
  const float* my = ws;
  const float* mx = ws + I;
  const float* rx = ws + I + O;
  const float* ry = ws + I + 2 * O;
  const bool rows_first = I > O;
  const int64_t total = OM ? (int64_t)O * (I / 2) : (int64_t)I * (O / 2);
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    uint32_t lo, hi;
    if (OM) {
      const int j = (int)(e / (I / 2)), a = (int)(e % (I / 2));
      lo = mm4_q<TW, OM>(w, 2 * a, j, I, Or, rows_first, my, mx, rx, ry);
      hi = mm4_q<TW, OM>(w, 2 * a + 1, j, I, Or, rows_first, my, mx, rx, ry);
    } else {
      const int i = (int)(e / (O / 2)), b = (int)(e % (O / 2));
      lo = mm4_q<TW, OM>(w, i, 2 * b, I, Or, rows_first, my, mx, rx, ry);
      hi = mm4_q<TW, OM>(w, i, 2 * b + 1, I, Or, rows_first, my, mx, rx, ry);
    }
    packed[e] = (uint8_t)(lo | (hi << 4));
  }
}

// mx, rx/4 over the O padded columns; my, ry/4 over the I rows
template <typename TW>
__global__ void mm4_meta(int I, int O, const float* ws, TW* mx_o, TW* rx_o, TW* my_o, TW* ry_o) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t < O) {
    mx_o[t] = from_f32<TW>(ws[I + t]);
    rx_o[t] = from_f32<TW>(ws[I + O + t] / 4.0f);
  }
  if (t < I) {
    my_o[t] = from_f32<TW>(ws[t]);
    ry_o[t] = from_f32<TW>(ws[I + 2 * O + t] / 4.0f);
  }
}

template <typename TW, bool OM>
static int mm4_pack_run(const TW* w, int I, int Or, uint8_t* packed, void* mx, void* rx, void* my, void* ry,
                        float* ws, hipStream_t s) {
  const int Mp = Or + (Or & 1);
  mm8_stats<TW, OM>(w, I, Mp, Or, ws, s);
  hipLaunchKernelGGL((mm4_quantize<TW, OM>), dim3(4096), dim3(256), 0, s, w, I, Mp, Or, ws, packed);
  const int n = I > Mp ? I : Mp;
  hipLaunchKernelGGL((mm4_meta<TW>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, I, Mp, ws, (TW*)mx, (TW*)rx,
                     (TW*)my, (TW*)ry);
  return check_launch("mm4_pack");
}

}  // namespace rwkv7mi

using namespace rwkv7mi;

extern "C" size_t rwkv7mi_mm8_workspace_bytes(int64_t rows, int64_t I, int64_t O) {
  if (rows <= 0 || I <= 0 || O <= 0) return MM8_COUNTER_BYTES;
  // Any chunk of <= 64 rows may be used, so take the largest of the three plans.
  size_t best = 0;
  for (int64_t r : {(int64_t)16, (int64_t)32, (int64_t)64}) {
    Mm8Plan p = mm8_plan(r, I, O);
    const size_t b = (size_t)p.ksplit * p.nstrips * 16 * p.mt * MM8_PSTRIDE * 4;
    if (b > best) best = b;
  }
  return MM8_COUNTER_BYTES + best;
}

extern "C" int rwkv7mi_mm8_matmul(const void* x, const uint8_t* w_u8, const void* mx, const void* rx,
                                  const void* my, const void* ry, const void* bias,
                                  const void* residual, void* y, int64_t rows, int64_t I, int64_t O,
                                  int epilogue, int act_dtype, int meta_dtype, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  if (rows < 0 || I <= 0 || O <= 0) return fail(RWKV7MI_EINVAL, "mm8_matmul: bad shape");
  if (rows == 0) return RWKV7MI_OK;
  if (O % 8) return fail(RWKV7MI_EINVAL, "mm8_matmul: out_features must be a multiple of 8");
  if (I > INT32_MAX || O > INT32_MAX) return fail(RWKV7MI_EINVAL, "mm8_matmul: too large");
  if (!x || !w_u8 || !mx || !rx || !my || !ry || !y) return fail(RWKV7MI_EINVAL, "mm8_matmul: null pointer");
  if (reinterpret_cast<uintptr_t>(w_u8) & 7) return fail(RWKV7MI_EINVAL, "mm8_matmul: w_u8 must be 8-byte aligned");
  if (epilogue < 0 || epilogue > 2) return fail(RWKV7MI_EINVAL, "mm8_matmul: bad epilogue");
  if (epilogue == RWKV7MI_EPI_RESIDUAL && !residual) return fail(RWKV7MI_EINVAL, "mm8_matmul: residual missing");
  if ((O + MM8_STRIP - 1) / MM8_STRIP > MM8_COUNTERS) return fail(RWKV7MI_EINVAL, "mm8_matmul: too many columns");
  if (!workspace || workspace_bytes < rwkv7mi_mm8_workspace_bytes(rows, I, O))
    return fail(RWKV7MI_ESIZE, "mm8_matmul: workspace too small");
  if (!valid_dtype(act_dtype) || !valid_dtype(meta_dtype)) return fail(RWKV7MI_EINVAL, "mm8_matmul: bad dtype");
  unsigned* cnt = reinterpret_cast<unsigned*>(workspace);
  float* part = reinterpret_cast<float*>(reinterpret_cast<char*>(workspace) + MM8_COUNTER_BYTES);
  const size_t esz_a = act_dtype == RWKV7MI_F32 ? 4 : 2;
  for (int64_t r0 = 0; r0 < rows; r0 += 64) {
    const int64_t nr = rows - r0 > 64 ? 64 : rows - r0;
    Mm8Plan p = mm8_plan(nr, I, O);
    const char* xr = reinterpret_cast<const char*>(x) + r0 * I * esz_a;
    char* yr = reinterpret_cast<char*>(y) + r0 * O * esz_a;
    const char* rr = residual ? reinterpret_cast<const char*>(residual) + r0 * O * esz_a : nullptr;
    int rc = dispatch_dtype(act_dtype, [&](auto ta) {
      using TA = decltype(ta);
      return dispatch_dtype(meta_dtype, [&](auto tm) {
        using TM = decltype(tm);
        dim3 grid(p.nstrips, p.ksplit);
#define MM8_LAUNCH(MT_, SPLIT_)                                                                      \
  hipLaunchKernelGGL((mm8_kernel<MT_, SPLIT_, TA, TM>), grid, dim3(256), p.lds, as_stream(stream),  \
                     (const TA*)xr, w_u8, (const TM*)mx, (const TM*)rx, (const TM*)my, (const TM*)ry, \
                     (const TM*)bias, (const TA*)rr, (TA*)yr, (int)nr, (int)I, (int)O, p.KR,       \
                     p.ksplit, epilogue, part, cnt)
        if (p.mt == 1) MM8_LAUNCH(1, true);
        else if (p.mt == 2) MM8_LAUNCH(2, false);
        else MM8_LAUNCH(4, false);
#undef MM8_LAUNCH
        return check_launch("mm8_kernel");
      });
    });
    if (rc) return rc;
  }
  return RWKV7MI_OK;
}

static int mm8_pack_entry(const void* weight, int64_t I, int64_t O, int w_dtype, uint8_t* w_u8, void* mx,
                          void* rx, void* my, void* ry, float* workspace, void* stream, bool out_major) {
  if (I <= 0 || O <= 0 || I > INT32_MAX || O > INT32_MAX) return fail(RWKV7MI_EINVAL, "mm8_pack: bad shape");
  if (!weight || !w_u8 || !mx || !rx || !my || !ry || !workspace)
    return fail(RWKV7MI_EINVAL, "mm8_pack: null pointer");
  hipStream_t s = as_stream(stream);
  return dispatch_dtype(w_dtype, [&](auto tw) {
    using TW = decltype(tw);
    const TW* w = (const TW*)weight;
    return out_major ? mm8_pack_run<TW, true>(w, (int)I, (int)O, w_u8, mx, rx, my, ry, workspace, s)
                     : mm8_pack_run<TW, false>(w, (int)I, (int)O, w_u8, mx, rx, my, ry, workspace, s);
  });
}

extern "C" int rwkv7mi_mm8_pack(const void* weight, int64_t I, int64_t O, int w_dtype, uint8_t* w_u8,
                                void* mx, void* rx, void* my, void* ry, float* workspace, void* stream) {
  return mm8_pack_entry(weight, I, O, w_dtype, w_u8, mx, rx, my, ry, workspace, stream, false);
}

extern "C" int rwkv7mi_mm8_pack_t(const void* weight, int64_t I, int64_t O, int w_dtype, uint8_t* w_t,
                                  void* mx, void* rx, void* my, void* ry, float* workspace, void* stream) {
  return mm8_pack_entry(weight, I, O, w_dtype, w_t, mx, rx, my, ry, workspace, stream, true);
}

static int mm4_pack_entry(const void* weight, int64_t I, int64_t O, int w_dtype, uint8_t* packed, void* mx,
                          void* rx, void* my, void* ry, float* workspace, void* stream, bool out_major) {
  if (I <= 0 || O <= 0 || I > INT32_MAX / 2 || O > INT32_MAX / 2) return fail(RWKV7MI_EINVAL, "mm4_pack: bad shape");
  if (out_major && (I & 1)) return fail(RWKV7MI_EINVAL, "mm4_pack_t: in_features must be even");
  if (!weight || !packed || !mx || !rx || !my || !ry || !workspace)
    return fail(RWKV7MI_EINVAL, "mm4_pack: null pointer");
  hipStream_t s = as_stream(stream);
  return dispatch_dtype(w_dtype, [&](auto tw) {
    using TW = decltype(tw);
    const TW* w = (const TW*)weight;
    return out_major ? mm4_pack_run<TW, true>(w, (int)I, (int)O, packed, mx, rx, my, ry, workspace, s)
                     : mm4_pack_run<TW, false>(w, (int)I, (int)O, packed, mx, rx, my, ry, workspace, s);
  });
}

extern "C" int rwkv7mi_mm4_pack(const void* weight, int64_t I, int64_t O, int w_dtype, uint8_t* packed, void* mx,
                                void* rx_s, void* my, void* ry_s, float* workspace, void* stream) {
  return mm4_pack_entry(weight, I, O, w_dtype, packed, mx, rx_s, my, ry_s, workspace, stream, false);
}

extern "C" int rwkv7mi_mm4_pack_t(const void* weight, int64_t I, int64_t O, int w_dtype, uint8_t* packed_t,
                                  void* mx, void* rx_s, void* my, void* ry_s, float* workspace, void* stream) {
  return mm4_pack_entry(weight, I, O, w_dtype, packed_t, mx, rx_s, my, ry_s, workspace, stream, true);
}

namespace rwkv7mi {
// out[i, o] = (u4[i, o] + 0.5) * ry[i] * rx[o] + my[i] + mx[o] from the reference
// layout [I, Mp/2], fp32 math, one rounding
template <typename TM, typename TO>
__global__ __launch_bounds__(256) void mm4_dequant_kernel(const uint8_t* __restrict__ p, const TM* __restrict__ mx,
                                                          const TM* __restrict__ rx, const TM* __restrict__ my,
                                                          const TM* __restrict__ ry, TO* __restrict__ out, int I,
                                                          int O) {
  const int Mh = (O + 1) / 2;
  for (int i = blockIdx.y; i < I; i += gridDim.y) {
    const float ryi = to_f32(ry[i]), myi = to_f32(my[i]);
    for (int o = blockIdx.x * 256 + threadIdx.x; o < O; o += gridDim.x * 256) {
      const uint32_t b = p[(int64_t)i * Mh + o / 2];
      const float u = (float)((o & 1) ? (b >> 4) : (b & 15u)) + 0.5f;
      out[(int64_t)i * O + o] = from_f32<TO>(u * ryi * to_f32(rx[o]) + myi + to_f32(mx[o]));
    }
  }
}
}  // namespace rwkv7mi

extern "C" int rwkv7mi_mm4_dequant(const uint8_t* packed, const void* mx, const void* rx_s, const void* my,
                                   const void* ry_s, void* out, int64_t I, int64_t O, int meta_dtype, int out_dtype,
                                   void* stream) {
  if (I <= 0 || O <= 0 || I > INT32_MAX || O > INT32_MAX) return fail(RWKV7MI_EINVAL, "mm4_dequant: bad shape");
  if (!packed || !mx || !rx_s || !my || !ry_s || !out) return fail(RWKV7MI_EINVAL, "mm4_dequant: null pointer");
  return dispatch_dtype(meta_dtype, [&](auto tm) {
    using TM = decltype(tm);
    return dispatch_dtype(out_dtype, [&](auto to) {
      using TO = decltype(to);
      const int gx = (int)std::min<int64_t>((O + 255) / 256, 64);
      hipLaunchKernelGGL((mm4_dequant_kernel<TM, TO>), dim3(gx, (unsigned)std::min<int64_t>(I, 32768)), dim3(256), 0,
                         as_stream(stream), packed, (const TM*)mx, (const TM*)rx_s, (const TM*)my, (const TM*)ry_s,
                         (TO*)out, (int)I, (int)O);
      return check_launch("mm4_dequant_kernel");
    });
  });
}

namespace rwkv7mi {
// out[i, o] = (w_u8[i, o] + 0.5) * ry[i] * rx[o] + my[i] + mx[o], fp32 math, one rounding.
template <typename TM, typename TO>
__global__ __launch_bounds__(256) void mm8_dequant_kernel(const uint8_t* __restrict__ w, const TM* __restrict__ mx,
                                                          const TM* __restrict__ rx, const TM* __restrict__ my,
                                                          const TM* __restrict__ ry, TO* __restrict__ out, int I,
                                                          int O) {
  const int i = blockIdx.y;
  const float ryi = to_f32(ry[i]), myi = to_f32(my[i]);
  for (int o = (blockIdx.x * 256 + threadIdx.x) * 4; o < O; o += gridDim.x * 256 * 4) {
    const uint32_t q = *reinterpret_cast<const uint32_t*>(w + (int64_t)i * O + o);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float wq = (float)((q >> (8 * e)) & 0xffu) + 0.5f;
      out[(int64_t)i * O + o + e] = from_f32<TO>(wq * ryi * to_f32(rx[o + e]) + myi + to_f32(mx[o + e]));
    }
  }
}
}  // namespace rwkv7mi

extern "C" int rwkv7mi_mm8_dequant(const uint8_t* w_u8, const void* mx, const void* rx, const void* my,
                                   const void* ry, void* out, int64_t I, int64_t O, int meta_dtype, int out_dtype,
                                   void* stream) {
  if (I <= 0 || O <= 0 || O % 4 || I > 65535 || O > INT32_MAX) return fail(RWKV7MI_EINVAL, "mm8_dequant: bad shape");
  if (!w_u8 || !mx || !rx || !my || !ry || !out) return fail(RWKV7MI_EINVAL, "mm8_dequant: null pointer");
  if (reinterpret_cast<uintptr_t>(w_u8) & 3) return fail(RWKV7MI_EINVAL, "mm8_dequant: w_u8 must be 4-byte aligned");
  return dispatch_dtype(meta_dtype, [&](auto tm) {
    using TM = decltype(tm);
    return dispatch_dtype(out_dtype, [&](auto to) {
      using TO = decltype(to);
      const int gx = (int)std::min<int64_t>((O / 4 + 255) / 256, 64);
      hipLaunchKernelGGL((mm8_dequant_kernel<TM, TO>), dim3(gx, (unsigned)I), dim3(256), 0, as_stream(stream),
                         w_u8, (const TM*)mx, (const TM*)rx, (const TM*)my, (const TM*)ry, (TO*)out, (int)I, (int)O);
      return check_launch("mm8_dequant_kernel");
    });
  });
}
