// wkv7 sequential on-chip scan (gfx950): T steps of the decode update with the
// state resident in registers.
//
// State rows are independent in the DPLR recurrence (row i only reads v[i] and
// the shared key-side vectors), so a head is split into 8 row blocks of 8 rows
// and each row block is one 64-lane wavefront: 8 lanes per row, 8 key columns
// per lane.  Grid = B*H*8 single-wave workgroups (2048 for B=8, H=32), enough
// to fill 256 CUs.  Per 8-token slab the wave stages r, w, k, kk*a, kk and the
// 8 needed v values in LDS and buffers its 8x8 outputs before one store.
//
// Replaces the reference's _recurrent_scan_kernel / _recurrent_scan_rows_kernel
// (rwkv7_hf/fused_recurrent_update.py:232, :454).
#include "common.h"

namespace rwkv7mi {

constexpr int SCAN_N = 64;
constexpr int SCAN_ROWS = 8;   // rows per wave
constexpr int SCAN_SLAB = 8;   // tokens staged per LDS fill

template <typename TA, typename TW>
__global__ __launch_bounds__(64) void wkv7_scan_kernel(
    const TA* __restrict__ r, const TW* __restrict__ w, const TA* __restrict__ k,
    const TA* __restrict__ v, const TA* __restrict__ kk, const TA* __restrict__ a,
    const float* state_in, float* state_out, TA* __restrict__ y,
    int T, int H) {
  __shared__ float s_r[SCAN_SLAB][SCAN_N], s_w[SCAN_SLAB][SCAN_N], s_k[SCAN_SLAB][SCAN_N];
  __shared__ float s_kk[SCAN_SLAB][SCAN_N], s_ka[SCAN_SLAB][SCAN_N];
  __shared__ float s_v[SCAN_SLAB][SCAN_ROWS];
  __shared__ float s_y[SCAN_SLAB][SCAN_ROWS];

  const int rb = blockIdx.x % (SCAN_N / SCAN_ROWS);
  const int bh = blockIdx.x / (SCAN_N / SCAN_ROWS);
  const int b = bh / H;
  const int h = bh % H;
  const int lane = threadIdx.x;
  const int row = rb * SCAN_ROWS + (lane >> 3);
  const int j0 = (lane & 7) * 8;

  float s[8];
  const int64_t soff = ((int64_t)bh * SCAN_N + row) * SCAN_N + j0;
  {
    const float4* src = reinterpret_cast<const float4*>(state_in + soff);
    float4 p = src[0], q = src[1];
    s[0] = p.x; s[1] = p.y; s[2] = p.z; s[3] = p.w;
    s[4] = q.x; s[5] = q.y; s[6] = q.z; s[7] = q.w;
  }

  const int64_t tok_stride = (int64_t)H * SCAN_N;
  const int64_t base = ((int64_t)b * T * H + h) * SCAN_N;  // token 0 of this (b,h)

  for (int t0 = 0; t0 < T; t0 += SCAN_SLAB) {
    const int nt = min(SCAN_SLAB, T - t0);
    // stage the slab: lane = channel
    for (int tt = 0; tt < nt; ++tt) {
      const int64_t off = base + (int64_t)(t0 + tt) * tok_stride + lane;
      float kkv = ld(kk, off);
      s_r[tt][lane] = ld(r, off);
      s_w[tt][lane] = ld(w, off);
      s_k[tt][lane] = ld(k, off);
      s_kk[tt][lane] = kkv;
      s_ka[tt][lane] = kkv * ld(a, off);
      if (lane < SCAN_ROWS) s_v[tt][lane] = ld(v, base + (int64_t)(t0 + tt) * tok_stride + rb * SCAN_ROWS + lane);
    }
    __syncthreads();
    for (int tt = 0; tt < nt; ++tt) {
      float dot = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) dot += s[j] * s_kk[tt][j0 + j];
      dot = group_sum<8>(dot);
      const float vi = s_v[tt][lane >> 3];
      float acc = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        float ns = s[j] * s_w[tt][j0 + j] - dot * s_ka[tt][j0 + j] + vi * s_k[tt][j0 + j];
        s[j] = ns;
        acc += ns * s_r[tt][j0 + j];
      }
      acc = group_sum<8>(acc);
      if ((lane & 7) == 0) s_y[tt][lane >> 3] = acc;
    }
    __syncthreads();
    // write the slab's outputs: lane -> (token lane/8, row lane%8)
    {
      const int tt = lane >> 3;
      const int rr = lane & 7;
      if (tt < nt) y[base + (int64_t)(t0 + tt) * tok_stride + rb * SCAN_ROWS + rr] = from_f32<TA>(s_y[tt][rr]);
    }
    __syncthreads();
  }
  {
    float4* dst = reinterpret_cast<float4*>(state_out + soff);
    dst[0] = make_float4(s[0], s[1], s[2], s[3]);
    dst[1] = make_float4(s[4], s[5], s[6], s[7]);
  }
}

}  // namespace rwkv7mi

using namespace rwkv7mi;

extern "C" int rwkv7mi_wkv7_scan(const void* r, const void* w, const void* k, const void* v,
                                 const void* kk, const void* a, const float* state_in,
                                 float* state_out, void* y, int64_t B, int64_t T, int64_t H, int64_t N,
                                 int act_dtype, int w_dtype, void* stream) {
  if (N != SCAN_N) return fail(RWKV7MI_EINVAL, "wkv7 scan: head size must be 64");
  if (B < 0 || T < 0 || H <= 0) return fail(RWKV7MI_EINVAL, "wkv7 scan: bad B/T/H");
  if (B == 0) return RWKV7MI_OK;
  if (!state_in || !state_out) return fail(RWKV7MI_EINVAL, "wkv7 scan: null state");
  if (T > 0 && (!r || !w || !k || !v || !kk || !a || !y)) return fail(RWKV7MI_EINVAL, "wkv7 scan: null input");
  if ((reinterpret_cast<uintptr_t>(state_in) | reinterpret_cast<uintptr_t>(state_out)) & 15)
    return fail(RWKV7MI_EINVAL, "wkv7 scan: state must be 16-byte aligned");
  if (B * H * 8 > INT32_MAX || T > INT32_MAX) return fail(RWKV7MI_EINVAL, "wkv7 scan: too large");
  return dispatch_dtype(act_dtype, [&](auto ta) {
    using TA = decltype(ta);
    return dispatch_dtype(w_dtype, [&](auto tw) {
      using TW = decltype(tw);
      hipLaunchKernelGGL((wkv7_scan_kernel<TA, TW>), dim3((unsigned)(B * H * 8)), dim3(64), 0,
                         as_stream(stream), (const TA*)r, (const TW*)w, (const TA*)k, (const TA*)v,
                         (const TA*)kk, (const TA*)a, state_in, state_out, (TA*)y, (int)T, (int)H);
      return check_launch("wkv7_scan_kernel");
    });
  });
}
