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
#include "common.h"

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
  // d = 8 nibbles n0..n7 (n_{2j} low nibble of byte j); out = [n0,n4,n1,n5,n2,n6,n3,n7] - 8
  f16x8 out;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const uint32_t hv = ((d >> (4 * s)) & 0x000F000Fu) | 0x64006400u;
    f16x2 h = __builtin_bit_cast(f16x2, hv);
    h = h + (f16x2){(_Float16)-1032.0f, (_Float16)-1032.0f};
    out[2 * s] = h[0];
    out[2 * s + 1] = h[1];
  }
  return out;
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
