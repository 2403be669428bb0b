// Prefill MM8 dequant GEMM over the blocked layout (more than 256 rows: long
// prompts), rwkv7_hf/native_quant_mm8.py:468-507 (the route that
// materialises the dequantised weight for rows > fused_max_rows) and the
// prefill projections of rwkv7_hf/native_jit_prefill.py:542-631, 955-1013.
//
// The weight is never materialised.  With W_hat[i,o] = (w + 0.5) ry[i] rx[o]
// + my[i] + mx[o] (native_quant_mm8.py:62-126):
//   y[m,o] = rx[o] (sum_i x[m,i] b[i,o] + 128.5 sum_i x ry)
//          + sum_i x my + mx[o] sum_i x,      b[i,o] = fp16((w[i,o] - 128) ry[i])
// b is built in registers from the MM8 bytes (w - 128 is exact in fp16, one
// packed multiply by ry rounds it once, as the reference's fp16 dequantised
// weight is rounded); the three row sums come out of the same MFMAs as three
// extra output columns (ry, my, 1), exact products with fp32 sums.
//
// Tile: a 512-lane workgroup computes 256 rows x 256 columns (16 column
// groups of the blocked layout).  Eight waves in a 2 x 4 grid each own
// 128 rows x 64 columns (8 x 4 MFMA tiles of v_mfma_f32_16x16x32_f16).  K
// advances 64 inputs per step (one 1 KB half of each 2 KB blocked tile):
//  * x rows go global -> registers -> LDS (double-buffered, one barrier per
//    step; the next step's loads are in flight during this step's MFMAs);
//  * each wave loads its own B bytes (16 bytes per lane and column group:
//    one lane's 16 bytes are the B operands of two consecutive MFMAs) one
//    step ahead, into registers;
//  * ry and my of the step's inputs sit in LDS with the x tile.
// Wave (wm, wn) also computes the extra columns for its M tiles 2wn, 2wn+1.
// The tile order is XCD-aware: a workgroup's linear id L runs on XCD L % 8,
// so tiles are numbered to give each XCD contiguous groups of 4 row tiles x
// 8 column tiles (their x rows and weight columns stay in that XCD's L2).
#include <string>

#include "mm8t_common.h"

namespace rwkv7mi {

constexpr int MM8P_M = 256, MM8P_N = 256, MM8P_KS = 64;
constexpr int MM8P_XS = MM8P_KS + 8;                    // LDS row stride (halfs)
constexpr int MM8P_ABYTES = MM8P_M * MM8P_XS * 2;       // one x buffer
constexpr int MM8P_VBYTES = 2 * MM8P_KS * 2;            // ry, my of one step (fp16)
constexpr int MM8P_LDS = 2 * (MM8P_ABYTES + MM8P_VBYTES);

struct Mm8pBatch {
  Mm8tProb p[MM8T_MAXPROB];
  int rows, I, O, KB;      // KB = ceil(I / 128) blocked tiles per column group
  int mt, nt;              // row / column tiles
  int gm, gn;              // XCD tile group: gm row tiles x gn column tiles
};

// bytes (d0, d1) = 8 consecutive inputs of one column -> fp16 (w - 128) * ry
__device__ __forceinline__ f16x8 mm8p_b_operand(uint32_t d0, uint32_t d1, f16x8 ry) {
  const f16x2 off = {(_Float16)-1152.f, (_Float16)-1152.f};
  f16x2 p0 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, d0, 0x04010400u)) + off;
  f16x2 p1 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, d0, 0x04030402u)) + off;
  f16x2 p2 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, d1, 0x04010400u)) + off;
  f16x2 p3 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, d1, 0x04030402u)) + off;
  const f16x8 w = (f16x8){p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
  return w * ry;
}

__global__ __launch_bounds__(512, 1) void mm8p_kernel(const Mm8pBatch B) {
  using TA = __half;
  const Mm8tProb& P = B.p[blockIdx.y];
  const int I = B.I, O = B.O, M = B.rows;
  // ---- XCD-aware tile number: linear id L on XCD L % 8; XCD x takes the
  // tiles x * per .. (x + 1) * per - 1 of the grouped order
  // (the grouped order pads the tile grid to whole groups; padding tiles exit)
  const int ngm = (B.mt + B.gm - 1) / B.gm, ngn = (B.nt + B.gn - 1) / B.gn;
  const int gsz = B.gm * B.gn;
  const int T = ngm * ngn * gsz;
  const int L = blockIdx.x;
  const int per = (T + 7) / 8;
  const int t = (L % 8) * per + L / 8;
  if (t >= T) return;
  const int grp = t / gsz, gi = t % gsz;
  const int gr = grp / ngn, gc = grp % ngn;
  const int tm = gr * B.gm + gi / B.gn, tn = gc * B.gn + gi % B.gn;
  if (tm >= B.mt || tn >= B.nt) return;
  const int m0 = tm * MM8P_M, n0 = tn * MM8P_N;

  extern __shared__ __align__(16) char smem[];
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int n = lane & 15, kg = lane >> 4;
  const int wm = wave >> 2, wn = wave & 3;
  auto xs = [&](int b) { return reinterpret_cast<_Float16*>(smem + b * (MM8P_ABYTES + MM8P_VBYTES)); };
  auto vs = [&](int b) { return reinterpret_cast<_Float16*>(smem + b * (MM8P_ABYTES + MM8P_VBYTES) + MM8P_ABYTES); };

  // ---- global sources (raw buffer loads; out-of-range offsets read zeros)
  const __amdgpu_buffer_rsrc_t xr = mm8t_rsrc(P.x, (uint32_t)((int64_t)M * I * 2));
  const __amdgpu_buffer_rsrc_t ryr = mm8t_rsrc(P.ry, (uint32_t)(I * 2));
  const __amdgpu_buffer_rsrc_t myr = mm8t_rsrc(P.my, (uint32_t)(I * 2));
  const int ngroups = (O + MM8T_COLS - 1) / MM8T_COLS;
  const uint32_t gbytes = (uint32_t)B.KB * 2048u;
  __amdgpu_buffer_rsrc_t wr[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int g = n0 / MM8T_COLS + 4 * wn + q;
    wr[q] = mm8t_rsrc(P.w + (int64_t)(g < ngroups ? g : 0) * gbytes, g < ngroups ? gbytes : 0u);
  }
  const int nsteps = (I + MM8P_KS - 1) / MM8P_KS;

  // x staging: 256 rows x 64 inputs = 2048 runs of 16 bytes, four per thread
  u32x4 xa[4];
  auto x_issue = [&](int s) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int c = tid + 512 * u;
      const int r = c >> 3, k = s * MM8P_KS + 8 * (c & 7);
      const bool ok = m0 + r < M && k < I;
      xa[u] = mm8t_ld16(xr, ok ? (uint32_t)(((int64_t)(m0 + r) * I + k) * 2) : MM8T_OOB);
    }
  };
  u32x4 va;  // threads 0..7: ry, 8..15: my (16 bytes each)
  auto v_issue = [&](int s) {
    if (tid < 16) {
      const int k = s * MM8P_KS + 8 * (tid & 7);
      va = mm8t_ld16(tid < 8 ? ryr : myr, k < I ? (uint32_t)(k * 2) : MM8T_OOB);
    }
  };
  auto x_store = [&](int b) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int c = tid + 512 * u;
      *reinterpret_cast<u32x4*>(xs(b) + (c >> 3) * MM8P_XS + 8 * (c & 7)) = xa[u];
    }
    if (tid < 16) *reinterpret_cast<u32x4*>(vs(b) + 8 * tid) = va;
  };
  // this wave's B bytes of step s: column group q, lane's 16 bytes of half s%2 of tile s/2
  u32x4 bq[2][4];
  auto b_issue = [&](int s, u32x4 (&b)[4]) {
    const uint32_t off = (uint32_t)(s >> 1) * 2048u + (uint32_t)(s & 1) * 1024u + 16u * (uint32_t)lane;
#pragma unroll
    for (int q = 0; q < 4; ++q) b[q] = mm8t_ld16(wr[q], s < nsteps ? off : MM8T_OOB);
  };

  f32x4 acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int q = 0; q < 4; ++q) acc[i][q] = (f32x4){0.f, 0.f, 0.f, 0.f};
  f32x4 ex[2] = {(f32x4){0.f, 0.f, 0.f, 0.f}, (f32x4){0.f, 0.f, 0.f, 0.f}};

  // prologue: step 0 into LDS buffer 0, step 1's loads in flight
  x_issue(0);
  v_issue(0);
  b_issue(0, bq[0]);
  x_store(0);
  x_issue(1);
  v_issue(1);
  b_issue(1, bq[1]);
  __syncthreads();

  const _Float16 one = (_Float16)1.0f;
  auto step = [&](int s, int b, u32x4 (&bc)[4]) {
    const _Float16* xb = xs(b);
    const _Float16* vb = vs(b);
#pragma unroll
    for (int h = 0; h < 2; ++h) {  // two MFMA K sub-steps of 32 inputs
      // the lane's 8 inputs: 16 kg + 8 h .. +7 of the step
      const int kk = 16 * kg + 8 * h;
      const f16x8 ry8 = *reinterpret_cast<const f16x8*>(vb + kk);
      f16x8 bv[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) bv[q] = mm8p_b_operand(bc[q][2 * h], bc[q][2 * h + 1], ry8);
      f16x8 bx;  // extra columns: 0 = ry, 1 = my, 2 = ones
      {
        const f16x8 my8 = *reinterpret_cast<const f16x8*>(vb + MM8P_KS + kk);
#pragma unroll
        for (int e = 0; e < 8; ++e) bx[e] = n == 0 ? ry8[e] : n == 1 ? my8[e] : n == 2 ? one : (_Float16)0.f;
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const f16x8 a = *reinterpret_cast<const f16x8*>(xb + (128 * wm + 16 * i + n) * MM8P_XS + kk);
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[i][q] = mfma16x16x32(a, bv[q], acc[i][q]);
        if (i == 2 * wn) ex[0] = mfma16x16x32(a, bx, ex[0]);
        if (i == 2 * wn + 1) ex[1] = mfma16x16x32(a, bx, ex[1]);
      }
    }
    (void)s;
  };

  // main loop, two steps per turn (the B ring slot is a compile-time index)
  for (int s = 0; s < nsteps; s += 2) {
    // step s from buffer 0 with bq[0]; step s+1 is in flight (x, v in xa/va, B in bq[1])
    step(s, 0, bq[0]);
    if (s + 2 < nsteps) b_issue(s + 2, bq[0]);
    x_store(1);  // step s+1 (loaded during step s)
    __syncthreads();
    if (s + 2 < nsteps) {
      x_issue(s + 2);
      v_issue(s + 2);
    }
    if (s + 1 < nsteps) {
      step(s + 1, 1, bq[1]);
      if (s + 3 < nsteps) b_issue(s + 3, bq[1]);
      x_store(0);  // step s+2
      __syncthreads();
      if (s + 3 < nsteps) {
        x_issue(s + 3);
        v_issue(s + 3);
      }
    }
  }

  // ---- the extra columns -> LDS row sums (reusing x buffer 0)
  float* rs = reinterpret_cast<float*>(smem);  // [256][3]: sum x ry, sum x my, sum x
  __syncthreads();
  if (n < 3) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) rs[(128 * wm + 16 * (2 * wn + j) + 4 * kg + e) * 3 + n] = ex[j][e];
  }
  __syncthreads();

  // ---- epilogue: lane holds column n of each group, rows 16 i + 4 kg + e
  const __half* rxp = reinterpret_cast<const __half*>(P.rx);
  const __half* mxp = reinterpret_cast<const __half*>(P.mx);
  const __half* bp = reinterpret_cast<const __half*>(P.bias);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int o = n0 + 64 * wn + 16 * q + n;
    if (o >= O) continue;
    const float rxo = ld(rxp, o), mxo = ld(mxp, o), bo = bp ? ld(bp, o) : 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = 128 * wm + 16 * i + 4 * kg + e;
        const int64_t row = m0 + r;
        if (row < M) {
          const float* q3 = rs + r * 3;
          float v = rxo * (acc[i][q][e] + 128.5f * q3[0]) + q3[1] + mxo * q3[2] + bo;
          const int64_t oi = row * O + o;
          if (P.epilogue == RWKV7MI_EPI_RELU2) {
            v = fmaxf(v, 0.f);
            v = v * v;
          } else if (P.epilogue == RWKV7MI_EPI_RESIDUAL) {
            v += ld(reinterpret_cast<const TA*>(P.residual), oi);
          }
          reinterpret_cast<TA*>(P.y)[oi] = from_f32<TA>(v);
        }
      }
  }
}

}  // namespace rwkv7mi

using namespace rwkv7mi;

extern "C" int rwkv7mi_mm8t_gemm_prefill(int nprob, const void* const* x, const uint8_t* const* w_blk,
                                         const void* const* mx, const void* const* rx, const void* const* my,
                                         const void* const* ry, const void* const* bias,
                                         const void* const* residual, void* const* y, const int* epilogue,
                                         int64_t rows, int64_t I, int64_t O, int act_dtype, int meta_dtype,
                                         void* stream) {
  const std::string w("mm8t_gemm_prefill");
  if (nprob < 1 || nprob > MM8T_MAXPROB) return fail(RWKV7MI_EINVAL, w + ": 1..4 problems per launch");
  if (!x || !w_blk || !mx || !rx || !my || !ry || !y || !epilogue) return fail(RWKV7MI_EINVAL, w + ": null array");
  if (rows < 0 || I <= 0 || O <= 0) return fail(RWKV7MI_EINVAL, w + ": bad shape");
  if (rows == 0) return RWKV7MI_OK;
  if (act_dtype != RWKV7MI_F16 || meta_dtype != RWKV7MI_F16)
    return fail(RWKV7MI_EINVAL, w + ": fp16 activations and fp16 metadata only (other dtypes take "
                                    "rwkv7mi_mm8t_gemm_multi in 256-row chunks)");
  if (I % 16) return fail(RWKV7MI_EINVAL, w + ": in_features must be a multiple of 16");
  // x's descriptor spans rows * I * 2 bytes and out-of-range offsets start at 2^31
  if (rows * I * 2 >= (int64_t)MM8T_OOB || (I + 127) / 128 * 2048 * 16 > (int64_t)UINT32_MAX ||
      O > INT32_MAX || rows * O > ((int64_t)1 << 40))
    return fail(RWKV7MI_EINVAL, w + ": too large (split the rows)");
  Mm8pBatch b{};
  for (int i = 0; i < nprob; ++i) {
    Mm8tProb q{x[i], nullptr, w_blk[i], mx[i], rx[i], my[i], ry[i], bias ? bias[i] : nullptr,
               residual ? residual[i] : nullptr, y[i], epilogue[i]};
    if (!q.x || !q.w || !q.mx || !q.rx || !q.my || !q.ry || !q.y) return fail(RWKV7MI_EINVAL, w + ": null pointer");
    if ((reinterpret_cast<uintptr_t>(q.x) | reinterpret_cast<uintptr_t>(q.w) | reinterpret_cast<uintptr_t>(q.my) |
         reinterpret_cast<uintptr_t>(q.ry)) & 15)
      return fail(RWKV7MI_EINVAL, w + ": x, the weights, my and ry must be 16-byte aligned");
    if (q.epilogue < 0 || q.epilogue > 2) return fail(RWKV7MI_EINVAL, w + ": bad epilogue");
    if (q.epilogue == RWKV7MI_EPI_RESIDUAL && !q.residual) return fail(RWKV7MI_EINVAL, w + ": residual missing");
    b.p[i] = q;
  }
  b.rows = (int)rows;
  b.I = (int)I;
  b.O = (int)O;
  b.KB = (int)((I + 127) / 128);
  b.mt = (int)((rows + MM8P_M - 1) / MM8P_M);
  b.nt = (int)((O + MM8P_N - 1) / MM8P_N);
  b.gm = std::min(b.mt, 4);
  b.gn = std::min(b.nt, 8);
  const int64_t T = (int64_t)((b.mt + b.gm - 1) / b.gm) * b.gm * ((b.nt + b.gn - 1) / b.gn) * b.gn;
  if (T > (int64_t)INT32_MAX / 2) return fail(RWKV7MI_EINVAL, w + ": too many tiles");
  const int64_t per = (T + 7) / 8;
  const dim3 grid((unsigned)(per * 8), (unsigned)nprob);
  static std::atomic<uint64_t> raised{0};
  if (int rc = raise_dynamic_lds(reinterpret_cast<const void*>(&mm8p_kernel), MM8P_LDS, raised, "mm8p_kernel"))
    return rc;
  hipLaunchKernelGGL(mm8p_kernel, grid, dim3(512), MM8P_LDS, as_stream(stream), b);
  return check_launch("mm8p_kernel");
}
