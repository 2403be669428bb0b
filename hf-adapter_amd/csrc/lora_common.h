// LoRA down projection tile shared by lora.hip (its own launch) and mm8t.hip
// (tail workgroups of the grouped R/K/V GEMV launch at 2..16 rows), see
// lora.hip for the algorithm.
#pragma once
#include "common.h"

namespace rwkv7mi {

enum { LORA_ACT_NONE = 0, LORA_ACT_TANH = 1, LORA_ACT_SIGMOID = 2 };
constexpr int LORA_MAXR = 256;   // largest rank
constexpr int LORA_PREFILL_ROWS = 256;  // above: the fused many-row kernel (no workspace)

struct LoraProb {
  const void* x;
  const void* wd;
  const void* wu;
  const void* bu;
  void* y;
  int r, act_d, act_u, tile_d0, tile_u0;  // tile_u0: first up workgroup (tpw output tiles each)
  int64_t part_off;  // floats
};
struct LoraBatch {
  LoraProb p[4];
  int nprob, D, A, ks, kr;
  int tpw;  // up kernel: output tiles of 16 columns per workgroup
};

// Many-row fp16 form (lora_seq.hip): whether it takes these shapes, and its launch.
bool lora_seq_supported(const LoraBatch& b, int64_t rows);
int lora_seq_run(const LoraBatch& b, int64_t rows, void* stream);

__device__ __forceinline__ float lora_act(float v, int act) {
  if (act == LORA_ACT_TANH) return tanhf(v);
  if (act == LORA_ACT_SIGMOID) return 1.0f / (1.0f + expf(-v));
  return v;
}
// The same with the hardware exp2 / reciprocal for the sigmoid (a few ulp of
// fp32, far below the activation dtype's rounding that follows); tanh keeps
// the library routine (1 - e^-2|v| loses relative accuracy near 0).
__device__ __forceinline__ float lora_act_fast(float v, int act) {
  if (act == LORA_ACT_TANH) return tanhf(v);
  if (act == LORA_ACT_SIGMOID) return __frcp_rn(1.0f + __builtin_amdgcn_exp2f(-1.4426950408889634f * v));
  return v;
}

// 8 consecutive elements at element index e of a buffer (zeros when !ok) as
// fp16 hi (+ lo for fp32 / bf16 sources); unconditional raw buffer loads.
template <typename T>
__device__ __forceinline__ void lora_load8(__amdgpu_buffer_rsrc_t r, uint32_t e, bool ok, f16x8& hi, f16x8& lo) {
  if constexpr (std::is_same<T, __half>::value) {
    hi = __builtin_bit_cast(f16x8, buf_ld16(r, ok ? e * 2u : BUF_OOB));
    lo = (f16x8){0, 0, 0, 0, 0, 0, 0, 0};
  } else {
    float f[8];
    buf_ld8(r, e, ok, (const T*)nullptr, f);
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const _Float16 h = (_Float16)f[q];
      hi[q] = h;
      lo[q] = (_Float16)(f[q] - (float)h);
    }
  }
}

__device__ __forceinline__ int lora_find(const LoraBatch& B, int tile, bool up) {
  int pi = 0;
#pragma unroll
  for (int q = 1; q < 4; ++q)
    if (q < B.nprob && tile >= (up ? B.p[q].tile_u0 : B.p[q].tile_d0)) pi = q;
  return pi;
}

// One (down tile, K range z, rows row0 .. row0 + 16 MT - 1) of the split-K
// down projection:
//   partial[p][z][row][n] = sum_{k in range z} x[row,k] Wd[n,k]
// run by the 256 lanes tid = 0..255 of a workgroup (or of one half of a larger
// one); s_red is this half's [4][16 MT][17] floats of LDS.  Every caller lane
// reaches the one barrier; !valid tiles load and store nothing.
template <int MT, typename TA>
__device__ __forceinline__ void lora_down_tile(const LoraBatch& B, int rows, float* __restrict__ part, int tile,
                                               int z, int tid, bool valid, float (*s_red)[16 * MT][17],
                                               int row0 = 0) {
  constexpr bool SPLIT = !std::is_same<TA, __half>::value;
  const LoraProb& P = B.p[lora_find(B, tile, false)];
  const int D = B.D;
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(valid ? P.x : nullptr, valid ? (uint32_t)((int64_t)rows * D * sizeof(TA)) : 0u);
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(valid ? P.wd : nullptr, valid ? (uint32_t)((int64_t)P.r * D * sizeof(TA)) : 0u);
  const int n0 = (tile - P.tile_d0) * 16;
  const int wave = tid >> 6, lane = tid & 63;
  const int l16 = lane & 15, kg = lane >> 4;
  const int k0 = z * B.kr;
  const int k1 = valid ? min(D, k0 + B.kr) : k0;

  f32x4 acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = (f32x4){0.f, 0.f, 0.f, 0.f};
  // 512-input blocks, each a fully unrolled run of four 32-wide wave steps whose
  // loads are all issued before the MFMAs (steps past the range load zeros)
  for (int c0 = k0; c0 < k1; c0 += 512) {
    f16x8 bh[4], bl[4], ah[4][MT], al[4][MT];
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int kk = c0 + 128 * it + wave * 32 + 8 * kg;
      const bool kok = kk < k1;  // D % 8 == 0
      lora_load8<TA>(wr, (uint32_t)((n0 + l16) * D + kk), kok && n0 + l16 < P.r, bh[it], bl[it]);
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        const int row = row0 + 16 * t + l16;
        lora_load8<TA>(xr, (uint32_t)(row * D + kk), kok && row < rows, ah[it][t], al[it][t]);
      }
    }
#pragma unroll
    for (int it = 0; it < 4; ++it)
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        acc[t] = mfma16x16x32(ah[it][t], bh[it], acc[t]);
        if constexpr (SPLIT) {
          acc[t] = mfma16x16x32(ah[it][t], bl[it], acc[t]);
          acc[t] = mfma16x16x32(al[it][t], bh[it], acc[t]);
        }
      }
  }
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int e = 0; e < 4; ++e) s_red[wave][16 * t + 4 * kg + e][l16] = acc[t][e];
  __syncthreads();
  if (valid) {
    float* dst = part + P.part_off + (int64_t)z * rows * P.r;
    const int nr = min(16 * MT, rows - row0);
    for (int idx = tid; idx < nr * 16; idx += 256) {
      const int row = idx >> 4, nn = idx & 15;
      if (n0 + nn < P.r)
        dst[(int64_t)(row0 + row) * P.r + n0 + nn] =
            ((s_red[0][row][nn] + s_red[1][row][nn]) + s_red[2][row][nn]) + s_red[3][row][nn];
    }
  }
}

// Host: the down-projection batch of up to four problems over `rows` (<= 64)
// rows of D inputs in ks K ranges, partials packed [p][z][row][r_p] from
// `part`; returns RWKV7MI_OK or an error (recorded by fail()).  *tiles: down
// tiles over all problems.
int lora_down_batch(int64_t nprob, const void* const* xs, const void* const* w_down, const int64_t* ranks,
                    int64_t rows, int64_t D, int ks, int act_dtype, LoraBatch* out, int* tiles);

}  // namespace rwkv7mi
