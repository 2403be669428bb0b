// MM4 affine dequant GEMV/GEMM over the reference's packed layout, gfx950.
//
// Format (rwkv7_hf/native_quant_mm4.py:77-135): packed [I, Mp/2] uint8, byte
// (i, c) = u[i, 2c] | u[i, 2c+1] << 4 (pairs along the OUTPUTS), 16 levels,
//   W_hat[i,o] = (u[i,o] + 0.5) * ry_s[i] * rx_s[o] + my[i] + mx[o]
// so  y[b,o] = rx_s[o] * sum_i x'[b,i] (u[i,o] + 0.5) + sum_i x[b,i] my[i]
//            + mx[o] sum_i x[b,i],       x' = x * ry_s.
// This is the fused form of the reference's mm4_gemv_triton /
// mm4_matmul_triton (native_quant_mm4.py:158-288, 545-578) for callers that
// hold the reference layout; MM4Linear keeps its own pairs-along-inputs layout
// for the decode GEMV (mm8t.hip, BITS = 4).
//
// Kernel: v_mfma_f32_16x16x32_f16 with batch rows as M (16 per tile), a
// 32-row k-step as K and 16 output columns as N.  A workgroup owns a strip of
// 256 output columns (128 bytes per row) and a K range; its four waves take
// interleaved k-steps.  Lane (n = l % 16, kg = l / 16) loads 8 bytes (16
// columns) from each of 8 rows.  For byte position p of those bytes, two
// v_perm_b32 gather that byte from 4 rows, the low and high nibbles are
// masked apart (columns 2p and 2p + 1), and v_perm with 0x64 as the high byte
// turns each nibble into the exact fp16 1024 + u; one packed add of -1023.5
// gives u + 0.5, the B operand of one column.  x' is staged per workgroup in
// LDS as fp16 hi + lo, so each product is two MFMAs with fp32 accumulation.
// Each K range writes fp32 partials (columns and the two row sums); a reduce
// launch adds the ranges in order and applies the affine terms and epilogue
// (deterministic, no atomics).
#include "common.h"

namespace rwkv7mi {

constexpr int MM4R_STRIP = 256;  // output columns per workgroup
constexpr int MM4R_PSTRIDE = MM4R_STRIP + 2;

// byte p of dwords a (row r) and b (row r + 1) -> [a.p, b.p, a.p, b.p]
__device__ __forceinline__ uint32_t mm4r_pair(uint32_t a, uint32_t b, uint32_t p) {
  return __builtin_amdgcn_perm(b, a, p | ((p + 4) << 8) | (p << 16) | ((p + 4) << 24));
}

// fp16 (u + 0.5) of the 8 rows' nibbles at byte p (hi = false: low nibbles,
// column 2p; true: high nibbles, column 2p + 1) of dwords d[0..7]
__device__ __forceinline__ f16x8 mm4r_operand(const uint32_t (&d)[8], uint32_t p, bool hi) {
  f16x8 out;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t t01 = mm4r_pair(d[4 * h], d[4 * h + 1], p);
    const uint32_t t23 = mm4r_pair(d[4 * h + 2], d[4 * h + 3], p);
    const uint32_t g = __builtin_amdgcn_perm(t23, t01, 0x05040100u);  // [r0.p, r1.p, r2.p, r3.p]
    const uint32_t u = (hi ? g >> 4 : g) & 0x0F0F0F0Fu;
    f16x2 a = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u));
    f16x2 b = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u));
    const f16x2 off = {(_Float16)-1023.5f, (_Float16)-1023.5f};
    a = a + off;
    b = b + off;
    out[4 * h] = a[0];
    out[4 * h + 1] = a[1];
    out[4 * h + 2] = b[0];
    out[4 * h + 3] = b[1];
  }
  return out;
}

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// The 8 bytes (16 columns) lane byte0 reads from each of 8 rows of a k-step,
// row lrow0 + i of the workgroup's K range (descriptor r starts at the range's
// first row).  Rows past the range and columns past the packed width read 0.
// The loads are unconditional buffer loads (an invalid one gets an offset
// past the descriptor), so the 8 (or 64) of them issue back to back.
template <bool AL8>
__device__ __forceinline__ void mm4r_load(__amdgpu_buffer_rsrc_t r, int lrow0, int kn, int bpr, int byte0,
                                          uint32_t (&lo)[8], uint32_t (&hi)[8]) {
  const bool colok = byte0 < bpr;  // with AL8 a lane's 8 bytes are all in or all out
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int row = lrow0 + i;
    const bool ok = colok && row < kn;
    const uint32_t base = (uint32_t)row * (uint32_t)bpr + (uint32_t)byte0;
    if constexpr (AL8) {
      const u32x2 v = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, (int)(ok ? base : BUF_OOB),
                                                                                     0, 0));
      lo[i] = v[0];
      hi[i] = v[1];
    } else {
      uint32_t a = 0u, b = 0u;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const bool okj = ok && byte0 + j < bpr;
        const uint32_t v = __builtin_amdgcn_raw_buffer_load_b8(r, (int)(okj ? base + j : BUF_OOB), 0, 0);
        if (j < 4) a |= v << (8 * j);
        else b |= v << (8 * (j - 4));
      }
      lo[i] = a;
      hi[i] = b;
    }
  }
}

// One 32-row k-step: A = x' (hi and lo) of batch row n at k = 8kg .. 8kg+7
// (LDS offset `off`), B = the lane's 16 columns from the 8 rows' bytes.
__device__ __forceinline__ void mm4r_step(const _Float16* xh, const _Float16* xl, int off, const uint32_t (&lo)[8],
                                          const uint32_t (&hi)[8], f32x4 (&acc)[16]) {
  const f16x8 ah = *reinterpret_cast<const f16x8*>(xh + off);
  const f16x8 al = *reinterpret_cast<const f16x8*>(xl + off);
#pragma unroll
  for (int c = 0; c < 16; ++c) {
    // column c of the lane's 16: byte c / 2 of the 8 (dword c / 8), nibble c % 2
    const f16x8 bv = mm4r_operand(c < 8 ? lo : hi, (uint32_t)((c >> 1) & 3), (c & 1) != 0);
    acc[c] = mfma16x16x32(ah, bv, acc[c]);
    acc[c] = mfma16x16x32(al, bv, acc[c]);
  }
}

// LDS reduction tile: column (n, c) of batch row b at b * MM4R_RSTRIDE + 17n + c
// (17-float lane stride: the 16 lanes of one c hit 16 different banks)
constexpr int MM4R_RSTRIDE = 16 * 17 + 4;

// grid (strips, K ranges); rows <= 16 per launch (one MFMA M tile).  A K
// range is KR = 128 NS rows: NS k-steps per wave (wave w takes rows
// 32w .. 32w+31 of every 128).  AL8: rows start on 8-byte boundaries
// (Mp % 16 == 0, aligned base), so a lane's 8 bytes of a row are one dwordx2
// load; otherwise they are loaded bytewise.  Every k-step's bytes are
// requested before x' is staged (up to 32 loads a lane in flight), then the
// steps convert and multiply in order as their bytes arrive.
template <int NS, bool AL8, typename TA, typename TM>
__global__ __launch_bounds__(256) void mm4r_kernel(const TA* __restrict__ x, const uint8_t* __restrict__ w,
                                                   const TM* __restrict__ my, const TM* __restrict__ ry, int rows,
                                                   int I, int Mp, float* __restrict__ part) {
  constexpr int R = 16, KR = 128 * NS, XS = KR + 8;  // XS: padded LDS row stride (halfs)
  constexpr int KJ = KR / 64;                         // k positions per lane when staging x'
  __shared__ __align__(16) _Float16 xh[R * XS], xl[R * XS];
  __shared__ float s_sum[2 * R];
  __shared__ float s_red[R * MM4R_RSTRIDE];

  const int strip = blockIdx.x, z = blockIdx.y, nstrips = gridDim.x;
  const int c0 = strip * MM4R_STRIP;  // first output column
  const int k0 = z * KR;
  const int kn = min(KR, I - k0);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int bpr = Mp / 2;  // bytes per row

  // lane (n, kg) covers columns c0 + 16n .. +15, rows 8kg .. 8kg+7 of each k-step
  const int n = lane & 15, kg = lane >> 4;
  const int byte0 = c0 / 2 + 8 * n;
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(w + (int64_t)k0 * bpr, (uint32_t)kn * (uint32_t)bpr);
  uint32_t lo[NS][8], hi[NS][8];
#pragma unroll
  for (int st = 0; st < NS; ++st) mm4r_load<AL8>(rw, 128 * st + 32 * wave + 8 * kg, kn, bpr, byte0, lo[st], hi[st]);

  // ---- x' = x * ry as fp16 hi + lo, and the per-row sums over this K range;
  // lane covers k = lane + 64j of the range, wave w batch rows w, w+4, ...
  {
    const __amdgpu_buffer_rsrc_t rx_ = make_rsrc(x, (uint32_t)(rows * I) * (uint32_t)sizeof(TA));
    const __amdgpu_buffer_rsrc_t rry = make_rsrc(ry + k0, (uint32_t)kn * (uint32_t)sizeof(TM));
    const __amdgpu_buffer_rsrc_t rmy = make_rsrc(my + k0, (uint32_t)kn * (uint32_t)sizeof(TM));
    float ryv[KJ], myv[KJ];
#pragma unroll
    for (int j = 0; j < KJ; ++j) {
      const int kk = lane + 64 * j;
      ryv[j] = buf_ld1<TM>(rry, kk, kk < kn);
      myv[j] = buf_ld1<TM>(rmy, kk, kk < kn);
    }
    for (int b = wave; b < R; b += 4) {
      if (b >= rows) {  // unused MFMA rows: zeros (their results are never stored)
#pragma unroll
        for (int j = 0; j < KJ; ++j) {
          xh[b * XS + lane + 64 * j] = (_Float16)0.f;
          xl[b * XS + lane + 64 * j] = (_Float16)0.f;
        }
        continue;
      }
      float xv[KJ];
#pragma unroll
      for (int j = 0; j < KJ; ++j) {
        const int kk = lane + 64 * j;
        xv[j] = buf_ld1<TA>(rx_, (uint32_t)(b * I + k0 + kk), kk < kn);
      }
      float sx = 0.f, sxmy = 0.f;
#pragma unroll
      for (int j = 0; j < KJ; ++j) {
        const int kk = lane + 64 * j;
        const float xp = xv[j] * ryv[j];
        sx += xv[j];
        sxmy += xv[j] * myv[j];
        const _Float16 h = (_Float16)xp;
        xh[b * XS + kk] = h;
        xl[b * XS + kk] = (_Float16)(xp - (float)h);
      }
      sx = wave_sum(sx);
      sxmy = wave_sum(sxmy);
      if (lane == 0) {
        s_sum[2 * b] = sx;
        s_sum[2 * b + 1] = sxmy;
      }
    }
  }
  __syncthreads();

  // ---- products (steps past the range hold zero bytes against zero x')
  f32x4 acc[16];
#pragma unroll
  for (int c = 0; c < 16; ++c) acc[c] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int st = 0; st < NS; ++st) mm4r_step(xh, xl, n * XS + 128 * st + 32 * wave + 8 * kg, lo[st], hi[st], acc);

  // ---- the four waves' tiles into LDS in wave order (D lane: column n, batch rows 4kg .. 4kg+3)
  for (int wv = 0; wv < 4; ++wv) {
    if (wave == wv) {
#pragma unroll
      for (int c = 0; c < 16; ++c)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float* dst = s_red + (4 * kg + e) * MM4R_RSTRIDE + 17 * n + c;
          *dst = wv == 0 ? acc[c][e] : *dst + acc[c][e];
        }
    }
    __syncthreads();
  }
  float* mine = part + ((int64_t)z * nstrips + strip) * R * MM4R_PSTRIDE;
  for (int idx = tid; idx < rows * MM4R_PSTRIDE; idx += 256) {
    const int b = idx / MM4R_PSTRIDE, cc = idx % MM4R_PSTRIDE;
    mine[idx] = cc < MM4R_STRIP ? s_red[b * MM4R_RSTRIDE + 17 * (cc >> 4) + (cc & 15)]
                                : s_sum[2 * b + (cc - MM4R_STRIP)];
  }
}

// y[b, o] from the K ranges' partials, added in range order 0..ksplit-1
template <typename TA, typename TM>
__global__ __launch_bounds__(256) void mm4r_reduce_kernel(const float* __restrict__ part, const TM* __restrict__ mx,
                                                          const TM* __restrict__ rx, const TM* __restrict__ bias,
                                                          const TA* residual, TA* y, int rows, int O, int nstrips,
                                                          int ksplit, int epilogue) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)rows * O) return;
  const int b = (int)(idx / O), o = (int)(idx % O);
  const int strip = o / MM4R_STRIP, cc = o % MM4R_STRIP;
  float s = 0.f, sx = 0.f, sxmy = 0.f;
  for (int z = 0; z < ksplit; ++z) {
    const float* pz = part + ((int64_t)z * nstrips + strip) * 16 * MM4R_PSTRIDE + (int64_t)b * MM4R_PSTRIDE;
    s += pz[cc];
    sx += pz[MM4R_STRIP];
    sxmy += pz[MM4R_STRIP + 1];
  }
  float v = ld(rx, o) * s + sxmy + ld(mx, o) * sx;
  if (bias) v += ld(bias, o);
  if (epilogue == RWKV7MI_EPI_RELU2) {
    v = fmaxf(v, 0.f);
    v = v * v;
  } else if (epilogue == RWKV7MI_EPI_RESIDUAL) {
    v += ld(residual, idx);
  }
  y[idx] = from_f32<TA>(v);
}

struct Mm4rPlan {
  int NS, KR, ksplit, nstrips;
};

// K ranges of 128, 256 or 512 rows (1, 2 or 4 k-steps a wave): the longest
// that I fills.  Longer ranges measured faster at every shape tried (fewer
// partials, every load of a wave issued at once): 4096 x 65536 at one row,
// 57.6 / 49.7 / 47.5 us for 1 / 2 / 4 steps.
static Mm4rPlan mm4r_plan(int64_t I, int64_t Mp) {
  Mm4rPlan p;
  p.nstrips = (int)((Mp + MM4R_STRIP - 1) / MM4R_STRIP);
  p.NS = 1;
  while (p.NS < 4 && 128 * p.NS < I) p.NS *= 2;
  p.KR = 128 * p.NS;
  p.ksplit = (int)((I + p.KR - 1) / p.KR);
  return p;
}

}  // namespace rwkv7mi

using namespace rwkv7mi;

extern "C" size_t rwkv7mi_mm4_matmul_workspace_bytes(int64_t I, int64_t Mp) {
  if (I <= 0 || Mp <= 0) return 0;
  const Mm4rPlan p = mm4r_plan(I, Mp);
  return (size_t)p.ksplit * p.nstrips * 16 * MM4R_PSTRIDE * 4;
}

extern "C" int rwkv7mi_mm4_matmul(const void* x, const uint8_t* packed, const void* mx, const void* rx_s,
                                  const void* my, const void* ry_s, const void* bias, const void* residual, void* y,
                                  int64_t rows, int64_t I, int64_t O, int64_t Mp, int epilogue, int act_dtype,
                                  int meta_dtype, void* workspace, size_t workspace_bytes, void* stream) {
  if (rows < 0 || I <= 0 || O <= 0 || Mp < O || Mp % 2) return fail(RWKV7MI_EINVAL, "mm4_matmul: bad shape");
  if (rows == 0) return RWKV7MI_OK;
  // 32-bit buffer offsets: a K range of the packed bytes (<= 512 rows) and
  // 16 rows of x
  if (Mp / 2 * 512 >= INT32_MAX || I * 16 * 4 >= INT32_MAX) return fail(RWKV7MI_EINVAL, "mm4_matmul: too large");
  if (!x || !packed || !mx || !rx_s || !my || !ry_s || !y) return fail(RWKV7MI_EINVAL, "mm4_matmul: null pointer");
  if (epilogue < 0 || epilogue > 2) return fail(RWKV7MI_EINVAL, "mm4_matmul: bad epilogue");
  if (epilogue == RWKV7MI_EPI_RESIDUAL && !residual) return fail(RWKV7MI_EINVAL, "mm4_matmul: residual missing");
  if (!valid_dtype(act_dtype) || !valid_dtype(meta_dtype)) return fail(RWKV7MI_EINVAL, "mm4_matmul: bad dtype");
  const Mm4rPlan p = mm4r_plan(I, Mp);
  if (!workspace || workspace_bytes < rwkv7mi_mm4_matmul_workspace_bytes(I, Mp) ||
      (reinterpret_cast<uintptr_t>(workspace) & 15))
    return fail(RWKV7MI_ESIZE, "mm4_matmul: workspace missing, unaligned or smaller than "
                               "rwkv7mi_mm4_matmul_workspace_bytes");
  float* part = static_cast<float*>(workspace);
  const bool al8 = (Mp / 2) % 8 == 0 && (reinterpret_cast<uintptr_t>(packed) & 7) == 0;
  const size_t esz = act_dtype == RWKV7MI_F32 ? 4 : 2;
  for (int64_t r0 = 0; r0 < rows; r0 += 16) {
    const int nr = (int)std::min<int64_t>(16, rows - r0);
    const char* xr = static_cast<const char*>(x) + r0 * I * esz;
    char* yr = static_cast<char*>(y) + r0 * O * esz;
    const char* rr = residual ? static_cast<const char*>(residual) + r0 * O * esz : nullptr;
    int rc = dispatch_dtype(act_dtype, [&](auto ta) {
      using TA = decltype(ta);
      return dispatch_dtype(meta_dtype, [&](auto tm) {
        using TM = decltype(tm);
        const dim3 grid(p.nstrips, p.ksplit);
        auto go = [&](auto ns, auto al) {
          hipLaunchKernelGGL((mm4r_kernel<decltype(ns)::value, decltype(al)::value, TA, TM>), grid, dim3(256), 0,
                             as_stream(stream), (const TA*)xr, packed, (const TM*)my, (const TM*)ry_s, nr, (int)I,
                             (int)Mp, part);
        };
        using T1 = std::integral_constant<int, 1>;
        using T2 = std::integral_constant<int, 2>;
        using T4 = std::integral_constant<int, 4>;
        using A1 = std::true_type;
        using A0 = std::false_type;
        if (p.NS == 1) al8 ? go(T1{}, A1{}) : go(T1{}, A0{});
        else if (p.NS == 2) al8 ? go(T2{}, A1{}) : go(T2{}, A0{});
        else al8 ? go(T4{}, A1{}) : go(T4{}, A0{});
        if (int e = check_launch("mm4r_kernel")) return e;
        const int64_t n = (int64_t)nr * O;
        hipLaunchKernelGGL((mm4r_reduce_kernel<TA, TM>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                           as_stream(stream), part, (const TM*)mx, (const TM*)rx_s, (const TM*)bias, (const TA*)rr,
                           (TA*)yr, nr, (int)O, p.nstrips, p.ksplit, epilogue);
        return check_launch("mm4r_reduce_kernel");
      });
    });
    if (rc) return rc;
  }
  return RWKV7MI_OK;
}
