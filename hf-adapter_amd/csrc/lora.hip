// RWKV-7 W/A/G/V LoRA projections (rwkv7_hf/fused_lora.py:559 fused_wag_lora,
// :706 fused_wavg_lora; torch form :795-803) as two grouped launches.
//
//   mid_p = act_down_p(x_p @ Wd_p^T)          Wd_p [r_p, D]   (no bias)
//   y_p   = act_up_p(mid_p @ Wu_p^T + b_p)    Wu_p [A, r_p]
//
// The down projections are tall and thin (r_p = 32..128 features over
// D = 4096 inputs): one workgroup per 16-feature tile would put only ~18
// workgroups on the chip, so K is split into `ks` ranges and each workgroup
// writes an fp32 partial tile.  The up kernel sums the partials of its inputs
// in fixed order, applies act_down and rounds to the activation dtype (the
// value the reference's mid tensor holds), stages them in LDS, and runs the
// up projection on v_mfma_f32_16x16x32_f16 — so the split costs no extra
// launch and the result is deterministic.  fp32 / bf16 operands are split
// into fp16 hi + lo as in the dense kernel.
#include "lora_common.h"

namespace rwkv7mi {

// grid (down tiles, ks): partial[p][z][row][n] = sum_{k in range z} x[row,k] Wd[n,k]
template <int MT, typename TA>
__global__ __launch_bounds__(256) void lora_down_kernel(const LoraBatch B, int rows, float* __restrict__ part) {
  __shared__ float s_red[4][16 * MT][17];
  lora_down_tile<MT, TA>(B, rows, part, blockIdx.x, blockIdx.y, threadIdx.x, true, s_red);
}

// grid (up workgroups): y[row, o] = act_up(sum_k mid[row,k] Wu[o,k] + b[o]),
// mid = round_TA(act_down(sum_z partial[z])) staged in LDS once per workgroup,
// then B.tpw output tiles of 16 columns, whole tiles per wave, each wave's next
// tile's weights loaded before this tile's MFMAs.  MT = 4 (up to 64 rows)
// takes ranks up to 128.
template <int MT, typename TA>
__global__ __launch_bounds__(256) void lora_up_kernel(const LoraBatch B, int rows, const float* __restrict__ part) {
  constexpr bool SPLIT = !std::is_same<TA, __half>::value;
  constexpr int RMAX = MT == 4 ? 128 : LORA_MAXR;
  constexpr int RS = RMAX + 8;  // LDS row stride (halfs)
  __shared__ __align__(16) _Float16 mh[16 * MT][RS];
  __shared__ __align__(16) _Float16 ml[SPLIT ? 16 * MT : 1][SPLIT ? RS : 8];
  const int wgi = blockIdx.x;
  const LoraProb& P = B.p[lora_find(B, wgi, true)];
  const int r = P.r;
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(P.wu, (uint32_t)((int64_t)B.A * r * sizeof(TA)));
  const int ntile = (B.A + 15) / 16;
  const int t0 = (wgi - P.tile_u0) * B.tpw;
  const int t1 = min(ntile, t0 + B.tpw);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int l16 = lane & 15, kg = lane >> 4;

  // a tile's up weights for this wave (lane: column 16 tl + l16, rank 32 j + 8 kg ..)
  constexpr int KW = RMAX / 32;
  f16x8 wh[KW], wl[KW];
  auto load_w = [&](int tl) {
#pragma unroll
    for (int j = 0; j < KW; ++j) {
      const int kk = 32 * j + 8 * kg;
      const int o = 16 * tl + l16;
      lora_load8<TA>(wr, (uint32_t)(o * r + kk), tl < t1 && kk < r && o < B.A, wh[j], wl[j]);
    }
  };
  load_w(t0 + wave);  // the wave's first tile overlaps the staging

  // stage mid: fixed-order sum over the K splits, four consecutive elements per
  // 16-byte load, IB groups x 4 splits = 32 loads in flight at a time (each
  // element's sum runs in z order; rows * r is a multiple of 8)
  constexpr int IB = 8;  // 4-element groups per thread and pass
  const int zstride = rows * r;
  const int ngrp = zstride / 4;
  const int r4 = r >> 2;  // 4-element groups per mid row
  const float inv_r4 = 1.0f / (float)r4;
  const __amdgpu_buffer_rsrc_t pr = make_rsrc(part + P.part_off, (uint32_t)(B.ks * zstride * 4));
  for (int g0 = tid; g0 < ngrp; g0 += 256 * IB) {
    float s[IB][4];
#pragma unroll
    for (int ib = 0; ib < IB; ++ib)
#pragma unroll
      for (int e = 0; e < 4; ++e) s[ib][e] = 0.f;
    for (int z0 = 0; z0 < B.ks; z0 += 4) {
      u32x4 t[IB][4];
#pragma unroll
      for (int ib = 0; ib < IB; ++ib) {
        const int g = g0 + 256 * ib;
#pragma unroll
        for (int u = 0; u < 4; ++u)
          t[ib][u] = buf_ld16(pr, z0 + u < B.ks && g < ngrp ? (uint32_t)(((z0 + u) * zstride + 4 * g) * 4)
                                                           : BUF_OOB);
      }
#pragma unroll
      for (int ib = 0; ib < IB; ++ib)
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
          for (int e = 0; e < 4; ++e) s[ib][e] += __uint_as_float(t[ib][u][e]);  // z order; past-the-end terms are +0
    }
#pragma unroll
    for (int ib = 0; ib < IB; ++ib) {
      const int g = g0 + 256 * ib;
      if (g < ngrp) {
        // row = g / r4 from a float reciprocal (g < 2^24) with a one-step fix-up
        int row = (int)((float)g * inv_r4);
        row -= row * r4 > g ? 1 : 0;
        row += (row + 1) * r4 <= g ? 1 : 0;
        const int k0 = 4 * (g - row * r4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float v = to_f32(from_f32<TA>(lora_act_fast(s[ib][e], P.act_d)));
          const _Float16 h = (_Float16)v;
          mh[row][k0 + e] = h;
          if constexpr (SPLIT) ml[row][k0 + e] = (_Float16)(v - (float)h);
        }
      }
    }
  }
  __syncthreads();

  // ---- each wave takes whole output tiles (every rank step), so no
  // cross-wave reduction: tiles t0 + wave, t0 + wave + 4, ...; the wave's mid
  // operands stay in registers for all of them
  const f16x8 zero8 = {0, 0, 0, 0, 0, 0, 0, 0};
  constexpr int KU = RMAX / 32;  // rank steps of 32
  f16x8 amh[MT][KU], aml[SPLIT ? MT : 1][SPLIT ? KU : 1];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int j = 0; j < KU; ++j) {
      const int kk = 32 * j + 8 * kg;
      const int row = 16 * m + l16;  // rows past `rows` only feed discarded D rows
      amh[m][j] = kk < r ? *reinterpret_cast<const f16x8*>(&mh[row][kk]) : zero8;
      if constexpr (SPLIT) aml[m][j] = kk < r ? *reinterpret_cast<const f16x8*>(&ml[row][kk]) : zero8;
    }
  TA* y = reinterpret_cast<TA*>(P.y);
  const TA* bias = reinterpret_cast<const TA*>(P.bu);
  for (int tl = t0 + wave; tl < t1; tl += 4) {
    f16x8 ch[KU], cl[KU];
#pragma unroll
    for (int j = 0; j < KU; ++j) {
      ch[j] = wh[j];
      cl[j] = wl[j];
    }
    load_w(tl + 4);  // the wave's next tile
    f32x4 acc[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      acc[m] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < KU; ++j) {
        if (32 * j < r) {  // (uniform) rank steps past r hold zeros
          acc[m] = mfma16x16x32(amh[m][j], ch[j], acc[m]);
          if constexpr (SPLIT) {
            acc[m] = mfma16x16x32(amh[m][j], cl[j], acc[m]);
            acc[m] = mfma16x16x32(aml[m][j], ch[j], acc[m]);
          }
        }
      }
    }
    // C: lane holds column 16 tl + l16, rows 16 m + 4 kg + e
    const int o = 16 * tl + l16;
    if (o < B.A) {
      const float bo = bias ? to_f32(bias[o]) : 0.f;
#pragma unroll
      for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int row = 16 * m + 4 * kg + e;
          if (row < rows) y[(int64_t)row * B.A + o] = from_f32<TA>(lora_act(acc[m][e] + bo, P.act_u));
        }
    }
  }
}

// Many-row form (prefills): one launch, no workspace.  A workgroup owns
// 64 MT rows of one problem; wave w owns rows 16 MT w .. + 16 MT - 1 (MT
// MFMA row tiles, so every weight operand it loads feeds MT MFMAs) from start
// to end:
//  1. mid = act_down(x Wd^T) over the whole K, MFMA with the rank tiles as
//     N (RT = ceil(r / 16) per row tile), x and Wd streamed from global with
//     the next K step's loads issued before this step's MFMAs;
//  2. mid rounded to the activation dtype (the reference's tensor) into the
//     wave's own LDS rows (hi, and lo for fp32 / bf16);
//  3. y = act_up(mid Wu^T + b) for every output tile of 16 columns, the up
//     weights of the next tiles loaded ahead.
// Waves never read each other's rows, so no workgroup barrier is needed.
template <int RT, int MT, typename TA>
__global__ __launch_bounds__(256) void lora_rows_kernel(const LoraBatch B, int rows) {
  constexpr bool SPLIT = !std::is_same<TA, __half>::value;
  constexpr int MS = 16 * RT + 8;  // LDS row stride of mid (halfs)
  constexpr int WR = 16 * MT;      // rows per wave
  extern __shared__ __align__(16) char lds[];
  _Float16* mh = reinterpret_cast<_Float16*>(lds);  // [4][WR][MS]
  _Float16* ml = mh + 4 * WR * MS;                   // (SPLIT) same shape
  const LoraProb& P = B.p[blockIdx.y];
  const int D = B.D, A = B.A, r = P.r;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int n = lane & 15, kg = lane >> 4;
  const int row0 = blockIdx.x * 4 * WR + WR * wave;
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(P.x, (uint32_t)((int64_t)rows * D * sizeof(TA)));
  const __amdgpu_buffer_rsrc_t dr = make_rsrc(P.wd, (uint32_t)((int64_t)r * D * sizeof(TA)));
  const __amdgpu_buffer_rsrc_t ur = make_rsrc(P.wu, (uint32_t)((int64_t)A * r * sizeof(TA)));
  _Float16* wmh = mh + wave * WR * MS;
  _Float16* wml = ml + wave * WR * MS;

  // ---- 1. down projection, K steps of 32 (lane: row n / rank n, inputs 8kg..)
  f32x4 acc[MT][RT];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int t = 0; t < RT; ++t) acc[m][t] = (f32x4){0.f, 0.f, 0.f, 0.f};
  f16x8 ah[2][MT], al[2][MT], bh[2][RT], bl[2][RT];
  auto load_k = [&](int k0, int sl) {
    const int kk = k0 + 8 * kg;
    const bool kok = kk < D;  // D % 8 == 0
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      const int row = row0 + 16 * m + n;
      lora_load8<TA>(xr, (uint32_t)(row * D + kk), kok && row < rows, ah[sl][m], al[sl][m]);
    }
#pragma unroll
    for (int t = 0; t < RT; ++t)
      lora_load8<TA>(dr, (uint32_t)((16 * t + n) * D + kk), kok && 16 * t + n < r, bh[sl][t], bl[sl][t]);
  };
  auto mfma_k = [&](int sl) {
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int t = 0; t < RT; ++t) {
        acc[m][t] = mfma16x16x32(ah[sl][m], bh[sl][t], acc[m][t]);
        if constexpr (SPLIT) {
          acc[m][t] = mfma16x16x32(ah[sl][m], bl[sl][t], acc[m][t]);
          acc[m][t] = mfma16x16x32(al[sl][m], bh[sl][t], acc[m][t]);
        }
      }
  };
  load_k(0, 0);
  for (int k0 = 0; k0 < D; k0 += 64) {
    load_k(k0 + 32, 1);
    mfma_k(0);
    load_k(k0 + 64, 0);
    mfma_k(1);
  }

  // ---- 2. mid (lane holds rows 16m + 4kg + e of rank column 16t + n)
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int t = 0; t < RT; ++t)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float v = to_f32(from_f32<TA>(lora_act(acc[m][t][e], P.act_d)));
        const _Float16 h = (_Float16)v;
        const int idx = (16 * m + 4 * kg + e) * MS + 16 * t + n;
        wmh[idx] = h;
        if constexpr (SPLIT) wml[idx] = (_Float16)(v - (float)h);
      }
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's mid writes are done
  __builtin_amdgcn_wave_barrier();

  // ---- 3. up projection, output tiles of 16 columns, UT at a time
  constexpr int KU = (16 * RT + 31) / 32;  // K steps of 32 over the rank
  f16x8 mah[MT][KU], mal[MT][KU];
  const f16x8 z8 = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int j = 0; j < KU; ++j) {
      const int kk = 32 * j + 8 * kg;
      const int idx = (16 * m + n) * MS + kk;
      mah[m][j] = kk < r ? *reinterpret_cast<const f16x8*>(wmh + idx) : z8;
      if constexpr (SPLIT) mal[m][j] = kk < r ? *reinterpret_cast<const f16x8*>(wml + idx) : z8;
    }
  TA* y = reinterpret_cast<TA*>(P.y);
  const TA* bias = reinterpret_cast<const TA*>(P.bu);
  const int ntiles = (A + 15) / 16;
  constexpr int UT = 2;  // output tiles per turn
  for (int ot0 = 0; ot0 < ntiles; ot0 += UT) {
    f16x8 uh[UT][KU], ul[UT][KU];
#pragma unroll
    for (int u = 0; u < UT; ++u)
#pragma unroll
      for (int j = 0; j < KU; ++j) {
        const int o = 16 * (ot0 + u) + n, kk = 32 * j + 8 * kg;
        lora_load8<TA>(ur, (uint32_t)(o * r + kk), o < A && kk < r, uh[u][j], ul[u][j]);
      }
#pragma unroll
    for (int u = 0; u < UT; ++u) {
      const int o = 16 * (ot0 + u) + n;
      const float bo = bias && o < A ? to_f32(bias[o]) : 0.f;
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        f32x4 c = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < KU; ++j) {
          c = mfma16x16x32(mah[m][j], uh[u][j], c);
          if constexpr (SPLIT) {
            c = mfma16x16x32(mah[m][j], ul[u][j], c);
            c = mfma16x16x32(mal[m][j], uh[u][j], c);
          }
        }
        if (o < A) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int row = row0 + 16 * m + 4 * kg + e;
            if (row < rows) y[(int64_t)row * A + o] = from_f32<TA>(lora_act(c[e] + bo, P.act_u));
          }
        }
      }
    }
  }
}

template <int RT, int MT, typename TA>
static int lora_rows_go(const LoraBatch& b, int64_t rows, void* stream) {
  constexpr bool SPLIT = !std::is_same<TA, __half>::value;
  constexpr int lds = 4 * 16 * MT * (16 * RT + 8) * 2 * (SPLIT ? 2 : 1);
  static std::atomic<uint64_t> raised{0};
  if (int rc = raise_dynamic_lds(reinterpret_cast<const void*>(&lora_rows_kernel<RT, MT, TA>), lds, raised,
                                 "lora_rows_kernel"))
    return rc;
  const dim3 grid((unsigned)((rows + 64 * MT - 1) / (64 * MT)), (unsigned)b.nprob);
  hipLaunchKernelGGL((lora_rows_kernel<RT, MT, TA>), grid, dim3(256), lds, as_stream(stream), b, (int)rows);
  return check_launch("lora_rows_kernel");
}

}  // namespace rwkv7mi

using namespace rwkv7mi;

extern "C" size_t rwkv7mi_lora_workspace_bytes(int64_t nprob, const int64_t* ranks, int64_t rows, int64_t D) {
  if (nprob < 1 || nprob > 4 || !ranks || rows <= 0 || D <= 0) return 0;
  const int64_t ks = lora_splits(lora_tiles(nprob, ranks), D);
  int64_t sr = 0;
  for (int64_t i = 0; i < nprob; ++i) sr += ranks[i];
  const int64_t nr = rows < LORA_ROWS ? rows : LORA_ROWS;
  return (size_t)(ks * nr * sr) * sizeof(float);
}

static int lora_run(bool up, int64_t nprob, const void* const* xs, const void* const* w_down,
                    const void* const* w_up, const void* const* b_up, void* const* ys, const int64_t* ranks,
                    const int* act_down, const int* act_up, int64_t rows, int64_t D, int64_t A, int act_dtype,
                    void* workspace, size_t workspace_bytes, void* stream) {
  if (nprob < 1 || nprob > 4) return fail(RWKV7MI_EINVAL, "lora_multi: 1..4 problems");
  if (!xs || !w_down || (up && (!w_up || !ys)) || !ranks || !act_down || !act_up)
    return fail(RWKV7MI_EINVAL, "lora_multi: null array");
  if (rows < 0 || D <= 0 || A <= 0 || D % 8 || D > (1 << 20) || A > (1 << 20))
    return fail(RWKV7MI_EINVAL, "lora_multi: bad shape (D a positive multiple of 8)");
  if (rows == 0) return RWKV7MI_OK;
  if (!up && rows > LORA_ROWS) return fail(RWKV7MI_EINVAL, "lora_down_multi: at most 64 rows");
  if (!valid_dtype(act_dtype)) return fail(RWKV7MI_EINVAL, "lora_multi: bad dtype");
  LoraBatch batch{};
  int td = 0, tu = 0;
  int64_t off = 0;
  int rmax = 0;
  for (int i = 0; i < nprob; ++i) rmax = std::max(rmax, (int)ranks[i]);
  // rows per launch pair: 64 (four MFMA row tiles) for ranks up to 128, else 32
  const int64_t chunk = rmax > 128 ? 32 : LORA_ROWS;
  const int64_t nr_max = rows < chunk ? rows : chunk;
  const int tiles_d = (int)lora_tiles(nprob, ranks);
  // up workgroups: each stages its problem's mid once, so several output tiles
  // share it; about one workgroup per compute unit over all problems
  const int ntile_u = (int)((A + 15) / 16);
  // about 128 up workgroups over all problems, at least one tile per wave
  const int tpw = std::min(((ntile_u + 3) / 4) * 4, std::max(4, (int)((nprob * ntile_u / 128 + 3) / 4) * 4));
  // more than 16 rows per chunk: a quarter of the K splits, so each up tile
  // sums four times fewer partials (its staging is the up kernel's cost there)
  const int ks = up && nr_max > 16 ? std::max(1, lora_splits(tiles_d, D) / 4) : lora_splits(tiles_d, D);
  for (int i = 0; i < nprob; ++i) {
    if (!xs[i] || !w_down[i] || (up && (!w_up[i] || !ys[i]))) return fail(RWKV7MI_EINVAL, "lora_multi: null pointer");
    if (ranks[i] <= 0 || ranks[i] % 8 || ranks[i] > LORA_MAXR)
      return fail(RWKV7MI_EINVAL, "lora_multi: rank must be a positive multiple of 8, at most 256");
    if (act_down[i] < 0 || act_down[i] > 2 || act_up[i] < 0 || act_up[i] > 2)
      return fail(RWKV7MI_EINVAL, "lora_multi: activation must be 0 none, 1 tanh or 2 sigmoid");
    if ((reinterpret_cast<uintptr_t>(xs[i]) | reinterpret_cast<uintptr_t>(w_down[i]) |
         reinterpret_cast<uintptr_t>(up ? w_up[i] : nullptr)) & 15)
      return fail(RWKV7MI_EINVAL, "lora_multi: x and weights must be 16-byte aligned");
    batch.p[i] = LoraProb{xs[i], w_down[i], up ? w_up[i] : nullptr, up && b_up ? b_up[i] : nullptr,
                          up ? ys[i] : nullptr, (int)ranks[i],
                          act_down[i], act_up[i], td, tu, off};
    td += (int)((ranks[i] + 15) / 16);
    tu += (ntile_u + tpw - 1) / tpw;
    off += (int64_t)ks * nr_max * ranks[i];
  }
  if ((!up || rows <= LORA_PREFILL_ROWS) && (!workspace || workspace_bytes < (size_t)off * sizeof(float)))
    return fail(RWKV7MI_ESIZE, "lora_multi: workspace too small");
  batch.nprob = (int)nprob;
  batch.D = (int)D;
  batch.A = (int)A;
  batch.tpw = tpw;
  batch.ks = ks;
  batch.kr = (int)((D + ks - 1) / ks);
  batch.kr = (batch.kr + 7) / 8 * 8;
  const size_t esz = act_dtype == RWKV7MI_F32 ? 4 : 2;
  if (up && rows > LORA_PREFILL_ROWS) {
    // many rows: the fused per-row-tile kernel, one launch, no partials
    if (rows * std::max(D, A) * (int64_t)esz > INT32_MAX || A * LORA_MAXR * (int64_t)esz > INT32_MAX)
      return fail(RWKV7MI_EINVAL, "lora_multi: too large");
    const int rt = (rmax + 15) / 16;
    // fp16 with ranks that are multiples of 32: weights shared through LDS, 256 rows per workgroup
    if (act_dtype == RWKV7MI_F16 && lora_seq_supported(batch, rows)) return lora_seq_run(batch, rows, stream);
    return dispatch_dtype(act_dtype, [&](auto ta) {
      using TA = decltype(ta);
      // two row tiles per wave (each weight operand feeds two MFMAs); one for
      // the largest ranks of the split (fp32 / bf16) form, which needs twice the registers
      constexpr bool SPLIT = !std::is_same<TA, __half>::value;
      if (rt <= 2) return lora_rows_go<2, 2, TA>(batch, rows, stream);
      if (rt <= 4) return lora_rows_go<4, 2, TA>(batch, rows, stream);
      if (rt <= 8) return lora_rows_go<8, SPLIT ? 1 : 2, TA>(batch, rows, stream);
      return lora_rows_go<16, 1, TA>(batch, rows, stream);
    });
  }
  float* part = reinterpret_cast<float*>(workspace);
  for (int64_t r0 = 0; r0 < rows; r0 += chunk) {
    const int64_t nr = rows - r0 > chunk ? chunk : rows - r0;
    LoraBatch bb = batch;
    for (int i = 0; i < nprob; ++i) {
      bb.p[i].x = reinterpret_cast<const char*>(batch.p[i].x) + r0 * D * esz;
      if (up) bb.p[i].y = reinterpret_cast<char*>(batch.p[i].y) + r0 * A * esz;
      // partial tiles are packed [ks][nr][r] for this chunk's row count
      int64_t o2 = 0;
      for (int j = 0; j < i; ++j) o2 += (int64_t)ks * nr * ranks[j];
      bb.p[i].part_off = o2;
    }
    const int mt = nr <= 16 ? 1 : nr <= 32 ? 2 : 4;
    int rc = dispatch_dtype(act_dtype, [&](auto ta) {
      using TA = decltype(ta);
      hipStream_t s = as_stream(stream);
#define LORA_GO(MT_)                                                                                    \
  hipLaunchKernelGGL((lora_down_kernel<MT_, TA>), dim3(td, ks), dim3(256), 0, s, bb, (int)nr, part);   \
  if (up)                                                                                               \
  hipLaunchKernelGGL((lora_up_kernel<MT_, TA>), dim3(tu), dim3(256), 0, s, bb, (int)nr, (const float*)part)
      if (mt == 1) {
        LORA_GO(1);
      } else if (mt == 2) {
        LORA_GO(2);
      } else {
        LORA_GO(4);
      }
#undef LORA_GO
      return check_launch("lora_multi");
    });
    if (rc) return rc;
  }
  return RWKV7MI_OK;
}

int rwkv7mi::lora_down_batch(int64_t nprob, const void* const* xs, const void* const* w_down, const int64_t* ranks,
                             int64_t rows, int64_t D, int ks, int act_dtype, LoraBatch* out, int* tiles) {
  if (nprob < 1 || nprob > 4) return fail(RWKV7MI_EINVAL, "lora down: 1..4 problems");
  if (!xs || !w_down || !ranks || !out || !tiles) return fail(RWKV7MI_EINVAL, "lora down: null array");
  if (rows < 1 || rows > LORA_ROWS || D <= 0 || D % 8 || D > (1 << 20) || ks < 1 || ks > D / 8)
    return fail(RWKV7MI_EINVAL, "lora down: 1..64 rows, D a positive multiple of 8, 1 <= ks <= D / 8");
  if (!valid_dtype(act_dtype)) return fail(RWKV7MI_EINVAL, "lora down: bad dtype");
  LoraBatch b{};
  int td = 0;
  int64_t off = 0;
  for (int i = 0; i < nprob; ++i) {
    if (!xs[i] || !w_down[i]) return fail(RWKV7MI_EINVAL, "lora down: null pointer");
    if (ranks[i] <= 0 || ranks[i] % 8 || ranks[i] > LORA_MAXR)
      return fail(RWKV7MI_EINVAL, "lora down: rank must be a positive multiple of 8, at most 256");
    if ((reinterpret_cast<uintptr_t>(xs[i]) | reinterpret_cast<uintptr_t>(w_down[i])) & 15)
      return fail(RWKV7MI_EINVAL, "lora down: x and weights must be 16-byte aligned");
    b.p[i] = LoraProb{xs[i], w_down[i], nullptr, nullptr, nullptr, (int)ranks[i], 0, 0, td, 0, off};
    td += (int)((ranks[i] + 15) / 16);
    off += (int64_t)ks * rows * ranks[i];
  }
  b.nprob = (int)nprob;
  b.D = (int)D;
  b.A = 1;
  b.tpw = 1;
  b.ks = ks;
  b.kr = (int)((D + ks - 1) / ks);
  b.kr = (b.kr + 7) / 8 * 8;
  *out = b;
  *tiles = td;
  return RWKV7MI_OK;
}

extern "C" int rwkv7mi_lora_multi(int64_t nprob, const void* const* xs, const void* const* w_down,
                                  const void* const* w_up, const void* const* b_up, void* const* ys,
                                  const int64_t* ranks, const int* act_down, const int* act_up, int64_t rows,
                                  int64_t D, int64_t A, int act_dtype, void* workspace, size_t workspace_bytes,
                                  void* stream) {
  return lora_run(true, nprob, xs, w_down, w_up, b_up, ys, ranks, act_down, act_up, rows, D, A, act_dtype,
                  workspace, workspace_bytes, stream);
}

extern "C" int rwkv7mi_lora_down_multi(int64_t nprob, const void* const* xs, const void* const* w_down,
                                       const int64_t* ranks, const int* act_down, int64_t rows, int64_t D,
                                       int act_dtype, void* workspace, size_t workspace_bytes, void* stream) {
  int act_up[4] = {0, 0, 0, 0};
  return lora_run(false, nprob, xs, w_down, nullptr, nullptr, nullptr, ranks, act_down, act_up, rows, D, 1,
                  act_dtype, workspace, workspace_bytes, stream);
}
