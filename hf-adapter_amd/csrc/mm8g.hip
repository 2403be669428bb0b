// Many-row MM8 dequant GEMM over the blocked layout (see mm8t.hip for the
// layout and the per-launch problem record).
#include <string>

#include <mutex>

#include "mm8t_common.h"
#include "lora_common.h"

// ---------------------------------------------------------------------------
// Many-row MM8 dequant GEMM over the blocked layout (17..256 rows: bsz-64
// decode and short prefills), rwkv7_hf/native_quant_mm8.py:100-126, 468-507.
//
// The GEMV of mm8t.hip tiles 16 rows per workgroup, so more rows stream the
// weights once per 16-row tile.  Here:
//  1. mm8g_prep_kernel computes, once per problem and row, x' = fp16(x ry)
//     (zero-padded to whole 128-input blocks) and the fp32 row sums
//     sum x, sum x my, sum x ry into the workspace;
//  2. mm8g_kernel: one workgroup owns a 64-row tile (four MFMA M tiles share
//     every dequantised B operand), 128 output columns (each of the four waves
//     two 16-column groups, so every LDS A read feeds two MFMAs) and a K range
//     (split s of S).  It copies its x' rows for that range into LDS once (at
//     most 8 K blocks = 1024 inputs), so the main loop has no barriers and the
//     weight ring runs uninterrupted;
//  3. with S > 1 each split writes fp32 partial tiles and mm8g_reduce_kernel
//     adds the splits in order 0..S-1 and applies the epilogue (deterministic,
//     no atomics).
//
// Precision: x' is rounded to fp16 and the weights enter the MFMA as the
// exact integers (w - 128), so the large common part 128.5 sum_i x' of
// (w + 0.5) is added from the fp32 row sum instead:
//   y = rx [sum_i x'_16 (w - 128) + 128.5 sum_i x ry] + sum_i x my + mx sum_i x.
// The fp16 rounding of x' then only touches the centred term.  fp32
// activations keep x' as fp16 hi + lo (x' = hi + lo to ~22 bits, as the
// GEMV stages it) and take two MFMAs per product, in 32-row tiles so the
// doubled LDS copy keeps the 64-row tile's footprint.
namespace rwkv7mi {

constexpr int MM8G_ROWS = 64;   // rows per workgroup tile
constexpr int MM8G_GPW = 2;     // 16-column groups per wave
constexpr int MM8G_COLS = 4 * MM8G_GPW * MM8T_COLS;  // 128 columns per workgroup
constexpr int MM8G_MAXKB = 8;   // K blocks (128 inputs) staged per workgroup
constexpr int MM8G_DEPTH = 4;   // weight ring depth (steps): ~1.5 us of HBM latency at the loop's pace

struct Mm8gBatch {
  Mm8tProb p[MM8T_MAXPROB];
  _Float16* xp;  // [nprob][rows][KB 128] x' = fp16(x ry), zero past I
  _Float16* xl;  // same shape: fp16(x ry - xp), written and read for fp32 activations only
  float* rsum;   // [nprob][rows][3] sum x, sum x my, sum x ry
  float* part;   // [S][nprob][rows][O] fp32 partial products (S > 1)
  int rows, I, O, KB, S, ctiles, nprob;
  int cw;  // workgroups per (problem, split, row tile): column-tile stride
  // Tail workgroups x >= cw S: the decode LoRA down projections (inputs ready
  // when the launch starts) on the CUs the tiles leave free (0: none)
  LoraBatch tl;
  float* tl_part;
  int tl_tiles, tl_wgs;
};

// The tail workgroups' share of the (16-row tile, down tile, K range) units.
// Every lane runs the same trip count (one barrier each).
template <typename TA>
__device__ __forceinline__ void mm8g_lora_tail(const Mm8gBatch& B, char* smem) {
  float(*s_red)[16][17] = reinterpret_cast<float(*)[16][17]>(smem);
  const int per_z = B.tl_tiles * ((B.rows + 15) / 16);
  const int nu = per_z * B.tl.ks;
  for (int u = (int)blockIdx.x - B.cw * B.S; u < nu; u += B.tl_wgs) {
    const int z = u / per_z, rem = u % per_z;
    lora_down_tile<1, TA>(B.tl, B.rows, B.tl_part, rem % B.tl_tiles, z, (int)threadIdx.x, true, s_red,
                          16 * (rem / B.tl_tiles));
    __syncthreads();  // the next unit reuses s_red
  }
}

// bytes (d0, d1) = rows r..r+7 of one column -> fp16 (w - 128) x 8 (exact)
__device__ __forceinline__ f16x8 mm8g_b_operand(uint32_t d0, uint32_t d1) {
  const f16x2 off = {(_Float16)-1152.f, (_Float16)-1152.f};
  f16x2 p0 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, d0, 0x04010400u)) + off;
  f16x2 p1 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, d0, 0x04030402u)) + off;
  f16x2 p2 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, d1, 0x04010400u)) + off;
  f16x2 p3 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, d1, 0x04030402u)) + off;
  return (f16x8){p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

template <typename TA, typename TM>
__device__ __forceinline__ float mm8g_finish(const Mm8tProb& P, float acc, float s_x, float s_xmy, float s_xry,
                                             int64_t row, int o, int O) {
  float v = ld(reinterpret_cast<const TM*>(P.rx), o) * (acc + 128.5f * s_xry) + s_xmy +
            ld(reinterpret_cast<const TM*>(P.mx), o) * s_x;
  if (P.bias) v += ld(reinterpret_cast<const TM*>(P.bias), o);
  if (P.epilogue == RWKV7MI_EPI_RELU2) {
    v = fmaxf(v, 0.f);
    v = v * v;
  } else if (P.epilogue == RWKV7MI_EPI_RESIDUAL) {
    v += ld(reinterpret_cast<const TA*>(P.residual), row * O + o);
  }
  return v;
}

// x' = fp16(x ry) for one (problem, row) per workgroup, zero past I up to the
// whole-block width KB 128, and the row's fp32 sums (lanes in a fixed DPP
// order, then the four waves in order)
template <typename TA, typename TM>
__global__ __launch_bounds__(256) void mm8g_prep_kernel(const Mm8gBatch B) {
  const int p = blockIdx.y;
  const int64_t row = blockIdx.x;
  const Mm8tProb& P = B.p[p];
  const int I = B.I, KBK = B.KB * 128;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const __amdgpu_buffer_rsrc_t xr =
      mm8t_rsrc(reinterpret_cast<const TA*>(P.x) + row * I, (uint32_t)(I * sizeof(TA)));
  const __amdgpu_buffer_rsrc_t ryr = mm8t_rsrc(P.ry, (uint32_t)(I * sizeof(TM)));
  const __amdgpu_buffer_rsrc_t myr = mm8t_rsrc(P.my, (uint32_t)(I * sizeof(TM)));
  _Float16* xo = B.xp + ((int64_t)p * B.rows + row) * KBK;
  _Float16* xlo = B.xl + ((int64_t)p * B.rows + row) * KBK;
  float a = 0.f, b = 0.f, c = 0.f;
  constexpr int PB = 4;  // passes whose loads are in flight together
  for (int k0 = 8 * tid; k0 < KBK; k0 += 8 * 256 * PB) {
    Raw8<TA> xv[PB];
    Raw8<TM> rr[PB], mr[PB];
#pragma unroll
    for (int u = 0; u < PB; ++u) {
      const int k = k0 + 8 * 256 * u;
      const bool valid = k < I;
      xv[u] = mm8t_ld8<TA>(xr, (uint32_t)k, valid);
      rr[u] = mm8t_ld8<TM>(ryr, (uint32_t)k, valid);
      mr[u] = mm8t_ld8<TM>(myr, (uint32_t)k, valid);
    }
#pragma unroll
    for (int u = 0; u < PB; ++u) {
      const int k = k0 + 8 * 256 * u;
      float x[8], rv[8], mv[8];
      mm8t_cvt8(xv[u], x);
      mm8t_cvt8(rr[u], rv);
      mm8t_cvt8(mr[u], mv);
      f16x8 h, l;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float xp = x[e] * rv[e];
        h[e] = (_Float16)xp;
        l[e] = (_Float16)(xp - (float)h[e]);
        a += x[e];
        b += x[e] * mv[e];
        c += xp;
      }
      if (k < KBK) {
        *reinterpret_cast<f16x8*>(xo + k) = h;
        if constexpr (std::is_same<TA, float>::value) *reinterpret_cast<f16x8*>(xlo + k) = l;
      }
    }
  }
  __shared__ float part[4][3];
  a = wave_sum(a);
  b = wave_sum(b);
  c = wave_sum(c);
  if (lane == 0) {
    part[wave][0] = a;
    part[wave][1] = b;
    part[wave][2] = c;
  }
  __syncthreads();
  if (tid < 3)
    B.rsum[((int64_t)p * B.rows + row) * 3 + tid] =
        (part[0][tid] + part[1][tid]) + (part[2][tid] + part[3][tid]);
}

template <typename TA, typename TM, int DEPTH, int NKP>
__global__ __launch_bounds__(256, 2) void mm8g_kernel(const Mm8gBatch B) {
  // NKP: staged K blocks (this split's nkb <= NKP, zero-padded); the main loop
  // is fully unrolled over them so every load-counter wait is exact.
  // Workgroup (x, p, z) takes split s = x % S and the column tiles
  // x / S, x / S + cw, ... of problem p: it stages x' once and streams the
  // weights of all its tiles, the next tile's first steps loading during the
  // current tile's last ones.
  static_assert(NKP % DEPTH == 0 && NKP % 4 == 0, "whole ring turns, whole staging passes");
  constexpr bool LO = std::is_same<TA, float>::value;  // x' as hi + lo
  constexpr int MT = LO ? 2 : 4;                        // MFMA M tiles per workgroup
  constexpr int TROWS = 16 * MT;
  const int p = blockIdx.y;
  const Mm8tProb& P = B.p[p];
  const int I = B.I, O = B.O, KB = B.KB;
  const int s = (int)blockIdx.x % B.S;
  const int c0 = (int)blockIdx.x / B.S;
  const int kb0 = s * KB / B.S, kb1 = (s + 1) * KB / B.S;
  const int nkb = kb1 - kb0;  // K blocks of this split (<= NKP)
  const int row0 = blockIdx.z * TROWS;
  const int nrows = min(TROWS, B.rows - row0);
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int n = lane & 15, kg = lane >> 4;
  const int ngroups = (O + MM8T_COLS - 1) / MM8T_COLS;
  constexpr int XS = 128 * NKP + 8;  // LDS row stride (halfs): rows land 16 bytes apart in the banks
  extern __shared__ __align__(16) char smem[];
  if (B.tl_wgs > 0 && (int)blockIdx.x >= B.cw * B.S) {  // a LoRA-down tail workgroup
    if (blockIdx.y == 0 && blockIdx.z == 0) mm8g_lora_tail<TA>(B, smem);
    return;
  }
  _Float16* xs = reinterpret_cast<_Float16*>(smem);
  _Float16* xsl = xs + TROWS * XS;  // the lo rows (LO only)
  (void)I;

  // ---- this wave's two column groups of tile ct (empty past the last tile)
  const uint32_t gbytes = (uint32_t)KB * 2048u;
  auto grsrc = [&](int ct, int gi) {
    const int g = ct * (MM8G_COLS / MM8T_COLS) + MM8G_GPW * wave + gi;
    const bool ok = ct < B.ctiles && g < ngroups;
    return mm8t_rsrc(P.w + (int64_t)(ok ? g : 0) * gbytes, ok ? gbytes : 0u);
  };
  u32x4 buf[DEPTH][2][2];
  auto load_step = [&](__amdgpu_buffer_rsrc_t r0, __amdgpu_buffer_rsrc_t r1, int j, u32x4 (&b)[2][2]) {
    const uint32_t off = j < nkb ? (uint32_t)(kb0 + j) * 2048u + 16u * (uint32_t)lane : MM8T_OOB;
    b[0][0] = mm8t_ld16(r0, off);
    b[0][1] = mm8t_ld16(r0, off + 1024u);
    b[1][0] = mm8t_ld16(r1, off);
    b[1][1] = mm8t_ld16(r1, off + 1024u);
  };
  __amdgpu_buffer_rsrc_t wr0 = grsrc(c0, 0), wr1 = grsrc(c0, 1);
#pragma unroll
  for (int d = 0; d < DEPTH; ++d) load_step(wr0, wr1, d, buf[d]);

  // ---- copy the x' rows for this split's K range into LDS, every load issued
  // before the first store: wave w takes rows w, w+4, ..., a lane 8
  // consecutive inputs per pass (one 1 KB run per row and pass).  Inputs past
  // the split and rows past the batch stage as zeros.
  {
    const int KBK = KB * 128;
    constexpr int NH = LO ? 2 : 1;      // hi (and lo) copies
    constexpr int RPW = TROWS / 4;      // rows per wave
    constexpr int NIT = NKP / 4;        // passes: 64 lanes x 8 inputs = 4 blocks per pass
    const int kbase = kb0 * 128, kend = kb1 * 128;
    u32x4 v[NH][NIT][RPW];
#pragma unroll
    for (int hl = 0; hl < NH; ++hl) {
      const __amdgpu_buffer_rsrc_t xr = mm8t_rsrc((hl ? B.xl : B.xp) + ((int64_t)p * B.rows + row0) * KBK,
                                                  (uint32_t)nrows * (uint32_t)KBK * 2u);
#pragma unroll
      for (int it = 0; it < NIT; ++it) {
        const int k = kbase + 8 * (lane + 64 * it);
#pragma unroll
        for (int i = 0; i < RPW; ++i) {
          const int r = wave + 4 * i;
          v[hl][it][i] = mm8t_ld16(xr, k < kend && r < nrows ? (uint32_t)(r * KBK + k) * 2u : MM8T_OOB);
        }
      }
    }
#pragma unroll
    for (int hl = 0; hl < NH; ++hl)
#pragma unroll
      for (int it = 0; it < NIT; ++it)
#pragma unroll
        for (int i = 0; i < RPW; ++i)
          *reinterpret_cast<u32x4*>((hl ? xsl : xs) + (wave + 4 * i) * XS + 8 * (lane + 64 * it)) = v[hl][it][i];
  }
  __syncthreads();

  const _Float16* abase = xs + n * XS + 16 * kg;
  const _Float16* albase = xsl + n * XS + 16 * kg;
  for (int ct = c0; ct < B.ctiles; ct += B.cw) {
    const __amdgpu_buffer_rsrc_t nr0 = grsrc(ct + B.cw, 0), nr1 = grsrc(ct + B.cw, 1);
    // ---- per step (one K block) a lane converts its four B operands of each
    // group, refills the ring slot (from the next tile in the last DEPTH
    // steps), then 4 operands x 4 M tiles x 2 groups = 32 MFMAs (eight
    // independent accumulator chains, one shape)
    f32x4 acc[2][MT];
#pragma unroll
    for (int gi = 0; gi < 2; ++gi)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[gi][mt] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < NKP; ++j) {
      const int d = j % DEPTH;
      f16x8 bv[2][4];
#pragma unroll
      for (int gi = 0; gi < 2; ++gi) {
        bv[gi][0] = mm8g_b_operand(buf[d][gi][0][0], buf[d][gi][0][1]);
        bv[gi][1] = mm8g_b_operand(buf[d][gi][0][2], buf[d][gi][0][3]);
        bv[gi][2] = mm8g_b_operand(buf[d][gi][1][0], buf[d][gi][1][1]);
        bv[gi][3] = mm8g_b_operand(buf[d][gi][1][2], buf[d][gi][1][3]);
      }
      if (j + DEPTH < NKP)
        load_step(wr0, wr1, j + DEPTH, buf[d]);
      else
        load_step(nr0, nr1, j + DEPTH - NKP, buf[d]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int hq = 0; hq < 4; ++hq) {
        // operand hq = rows 64 (hq / 2) + 16 kg + 8 (hq % 2) of the block
        const int off = 128 * j + 64 * (hq >> 1) + 8 * (hq & 1);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const f16x8 a = *reinterpret_cast<const f16x8*>(abase + mt * 16 * XS + off);
          acc[0][mt] = mfma16x16x32(a, bv[0][hq], acc[0][mt]);
          acc[1][mt] = mfma16x16x32(a, bv[1][hq], acc[1][mt]);
          if constexpr (LO) {
            const f16x8 al = *reinterpret_cast<const f16x8*>(albase + mt * 16 * XS + off);
            acc[0][mt] = mfma16x16x32(al, bv[0][hq], acc[0][mt]);
            acc[1][mt] = mfma16x16x32(al, bv[1][hq], acc[1][mt]);
          }
        }
      }
    }

    // ---- lane holds column n of each group, rows 16 mt + 4 kg + e
    const int g0 = ct * (MM8G_COLS / MM8T_COLS) + MM8G_GPW * wave;
    if (B.S == 1) {
#pragma unroll
      for (int gi = 0; gi < 2; ++gi) {
        const int o = (g0 + gi) * MM8T_COLS + n;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int r = 16 * mt + 4 * kg + e;
            if (r < nrows && o < O) {
              const int64_t row = row0 + r;
              const float* q = B.rsum + ((int64_t)p * B.rows + row) * 3;
              const float v = mm8g_finish<TA, TM>(P, acc[gi][mt][e], q[0], q[1], q[2], row, o, O);
              reinterpret_cast<TA*>(P.y)[row * O + o] = from_f32<TA>(v);
            }
          }
      }
    } else {
      float* part = B.part + ((int64_t)(s * B.nprob + p) * B.rows + row0) * O;
#pragma unroll
      for (int gi = 0; gi < 2; ++gi) {
        const int o = (g0 + gi) * MM8T_COLS + n;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int r = 16 * mt + 4 * kg + e;
            if (r < nrows && o < O) part[(int64_t)r * O + o] = acc[gi][mt][e];
          }
      }
    }
    wr0 = nr0;
    wr1 = nr1;
  }
}

// y[p][row][o..o+V-1] = epilogue of the splits' partials added in order
// 0..S-1 (V = 4 when O % 4 == 0: float4 loads, four splits in flight)
template <typename TA, typename TM, int V>
__global__ __launch_bounds__(256) void mm8g_reduce_kernel(const Mm8gBatch B) {
  const int p = blockIdx.y;
  const Mm8tProb& P = B.p[p];
  const int O = B.O;
  const int64_t per = (int64_t)B.rows * O;
  const int64_t idx = ((int64_t)blockIdx.x * 256 + threadIdx.x) * V;
  if (idx >= per) return;
  const int64_t row = idx / O;
  const int o = (int)(idx - row * O);
  const int64_t sstride = (int64_t)B.nprob * per;
  const float* part = B.part + (int64_t)p * per + idx;
  float a[V];
#pragma unroll
  for (int v = 0; v < V; ++v) a[v] = 0.f;
  constexpr int SB = 4;  // splits in flight
  for (int s0 = 0; s0 < B.S; s0 += SB) {
    float t[SB][V];
#pragma unroll
    for (int u = 0; u < SB; ++u) {
      if (s0 + u < B.S) {
        if constexpr (V == 4) {
          const float4 q = *reinterpret_cast<const float4*>(part + (s0 + u) * sstride);
          t[u][0] = q.x, t[u][1] = q.y, t[u][2] = q.z, t[u][3] = q.w;
        } else {
          t[u][0] = part[(s0 + u) * sstride];
        }
      } else {
#pragma unroll
        for (int v = 0; v < V; ++v) t[u][v] = 0.f;
      }
    }
#pragma unroll
    for (int u = 0; u < SB; ++u)
#pragma unroll
      for (int v = 0; v < V; ++v) a[v] += t[u][v];  // split order; past-the-end terms are +0
  }
  const float* rsum = B.rsum + ((int64_t)p * B.rows + row) * 3;
  const float s0 = rsum[0], s1 = rsum[1], s2 = rsum[2];
#pragma unroll
  for (int v = 0; v < V; ++v)
    reinterpret_cast<TA*>(P.y)[idx + v] = from_f32<TA>(mm8g_finish<TA, TM>(P, a[v], s0, s1, s2, row, o + v, O));
}

// Split count: explicit, or the fewest (a power of two) that keep every
// workgroup's K range within MM8G_MAXKB blocks.  Fewer, longer splits measured
// faster than more workgroups per CU at every 7.2B bsz-64 shape (the partials
// and the shorter weight streams cost more than the occupancy gains).
static int mm8g_splits(int64_t rows, int64_t I, int64_t O, int nprob, int req) {
  (void)rows, (void)O, (void)nprob;
  const int64_t KB = (I + 127) / 128;
  if (req > 0) return (int)std::min<int64_t>(req, KB);
  int64_t S = 1;
  while (S < KB && (KB + S - 1) / S > MM8G_MAXKB) S *= 2;
  return (int)std::min<int64_t>(S, KB);
}

// Workspace: x' [nprob][rows][KB 128] fp16 | its lo half, same shape (used by
// fp32 activations; reserved for every dtype so the size does not depend on
// it) | row sums [nprob][rows][3] fp32 | partials [S][nprob][rows][O] fp32
// (S > 1), each part 256-byte aligned.
struct Mm8gWs {
  size_t xp, xl, rsum, part, total;
};
static Mm8gWs mm8g_ws_layout(int S, int nprob, int64_t rows, int64_t I, int64_t O) {
  auto up = [](size_t v) { return (v + 255) & ~(size_t)255; };
  Mm8gWs w{};
  w.xp = 0;
  w.xl = up((size_t)nprob * rows * (size_t)((I + 127) / 128) * 128u * 2u);
  w.rsum = 2 * w.xl;
  w.part = w.rsum + up((size_t)nprob * rows * 3u * 4u);
  w.total = w.part + (S > 1 ? up((size_t)S * nprob * rows * O * 4u) : 0);
  return w;
}

}  // namespace rwkv7mi

using namespace rwkv7mi;

extern "C" size_t rwkv7mi_mm8t_gemm_workspace_bytes(int nprob, int64_t rows, int64_t I, int64_t O, int splits) {
  if (nprob < 1 || nprob > MM8T_MAXPROB || rows <= 0 || I <= 0 || O <= 0) return 0;
  return mm8g_ws_layout(mm8g_splits(rows, I, O, nprob, splits), nprob, rows, I, O).total;
}

static int mm8g_run(const char* who, int nprob, const void* const* x, const uint8_t* const* w_blk,
                    const void* const* mx, const void* const* rx, const void* const* my, const void* const* ry,
                    const void* const* bias, const void* const* residual, void* const* y, const int* epilogue,
                    int64_t rows, int64_t I, int64_t O, int act_dtype, int meta_dtype, int splits, void* workspace,
                    size_t workspace_bytes, void* stream, const LoraBatch* tl = nullptr, float* tl_part = nullptr,
                    int tl_tiles = 0) {
  const std::string w(who);
  if (nprob < 1 || nprob > MM8T_MAXPROB) return fail(RWKV7MI_EINVAL, w + ": 1..4 problems per launch");
  if (!x || !w_blk || !mx || !rx || !my || !ry || !y || !epilogue) return fail(RWKV7MI_EINVAL, w + ": null array");
  if (rows < 0 || I <= 0 || O <= 0 || splits < 0) return fail(RWKV7MI_EINVAL, w + ": bad shape");
  if (rows == 0) return RWKV7MI_OK;
  if (I % 16) return fail(RWKV7MI_EINVAL, w + ": in_features must be a multiple of 16");
  const int trows = act_dtype == RWKV7MI_F32 ? MM8G_ROWS / 2 : MM8G_ROWS;  // rows per tile (fp32: hi + lo)
  if (I > (1 << 24) || O > (1 << 24) || rows > 65535LL * trows || rows * std::max(I, O) > INT32_MAX)
    return fail(RWKV7MI_EINVAL, w + ": too large");
  if (!valid_dtype(act_dtype) || !valid_dtype(meta_dtype)) return fail(RWKV7MI_EINVAL, w + ": bad dtype");
  Mm8gBatch b{};
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
  const int S = mm8g_splits(rows, I, O, nprob, splits);
  const int64_t KB = (I + 127) / 128;
  if ((int64_t)MM8G_ROWS * KB * 128 * 2 > INT32_MAX) return fail(RWKV7MI_EINVAL, w + ": too large");
  if ((KB + S - 1) / S > MM8G_MAXKB)
    return fail(RWKV7MI_EINVAL, w + ": splits leave more than 1024 inputs per workgroup");
  const Mm8gWs lay = mm8g_ws_layout(S, nprob, rows, I, O);
  if (!workspace || workspace_bytes < lay.total || (reinterpret_cast<uintptr_t>(workspace) & 255))
    return fail(RWKV7MI_ESIZE, w + ": workspace missing, unaligned or smaller than "
                                   "rwkv7mi_mm8t_gemm_workspace_bytes");
  b.rows = (int)rows;
  b.I = (int)I;
  b.O = (int)O;
  b.KB = (int)KB;
  b.S = S;
  b.nprob = nprob;
  b.ctiles = (int)((O + MM8G_COLS - 1) / MM8G_COLS);
  char* wsb = reinterpret_cast<char*>(workspace);
  b.xp = reinterpret_cast<_Float16*>(wsb + lay.xp);
  b.xl = reinterpret_cast<_Float16*>(wsb + lay.xl);
  b.rsum = reinterpret_cast<float*>(wsb + lay.rsum);
  b.part = S > 1 ? reinterpret_cast<float*>(wsb + lay.part) : nullptr;
  const int nkp = (KB + S - 1) / S <= 4 ? 4 : MM8G_MAXKB;  // staged blocks: one of two kernel instances
  const size_t lds = (size_t)MM8G_ROWS * (size_t)(128 * nkp + 8) * 2u;  // (fp32: half the rows, twice the copies)
  // persistent column tiles: as many workgroups as fit the CUs at once (one per
  // CU with 8 staged blocks, two with 4), the tiles shared out evenly
  const int64_t rtiles = (rows + trows - 1) / trows;
  const int64_t slots = mm8t_cus() * (nkp == 4 ? 2 : 1);
  const int64_t cwmax = std::max<int64_t>(1, slots / ((int64_t)S * nprob * rtiles));
  const int64_t per = (b.ctiles + cwmax - 1) / cwmax;  // tiles per workgroup
  b.cw = (int)((b.ctiles + per - 1) / per);
  int64_t tail = 0;
  if (tl) {
    if (rows > LORA_ROWS || !tl_part || tl_tiles <= 0)
      return fail(RWKV7MI_EINVAL, w + ": the LoRA-down tail takes at most 64 rows");
    const int64_t units = (int64_t)tl_tiles * tl->ks * ((rows + 15) / 16);
    const int64_t free_slots = slots - (int64_t)b.cw * S * nprob * rtiles;
    tail = std::min<int64_t>(units, std::max<int64_t>(free_slots, 8));
    b.tl = *tl;
    b.tl_part = tl_part;
    b.tl_tiles = tl_tiles;
    b.tl_wgs = (int)tail;
  }
  const dim3 grid((unsigned)(b.cw * S + tail), (unsigned)nprob, (unsigned)rtiles);
  return dispatch_dtype(act_dtype, [&](auto ta) {
    using TA = decltype(ta);
    return dispatch_dtype(meta_dtype, [&](auto tm) {
      using TM = decltype(tm);
      // devices whose dynamic LDS limit is raised for each instance
      static std::atomic<uint64_t> raised_max{0}, raised_4{0};
      if (int rc = raise_dynamic_lds(reinterpret_cast<const void*>(&mm8g_kernel<TA, TM, MM8G_DEPTH, MM8G_MAXKB>),
                                     MM8G_ROWS * (128 * MM8G_MAXKB + 8) * 2, raised_max, "mm8g_kernel"))
        return rc;
      if (int rc = raise_dynamic_lds(reinterpret_cast<const void*>(&mm8g_kernel<TA, TM, MM8G_DEPTH, 4>),
                                     MM8G_ROWS * (128 * 4 + 8) * 2, raised_4, "mm8g_kernel"))
        return rc;
      hipLaunchKernelGGL((mm8g_prep_kernel<TA, TM>), dim3((unsigned)rows, (unsigned)nprob), dim3(256), 0,
                         as_stream(stream), b);
      int rc = check_launch("mm8g_prep_kernel");
      if (rc != RWKV7MI_OK) return rc;
      if (nkp == 4)
        hipLaunchKernelGGL((mm8g_kernel<TA, TM, MM8G_DEPTH, 4>), grid, dim3(256), lds, as_stream(stream), b);
      else
        hipLaunchKernelGGL((mm8g_kernel<TA, TM, MM8G_DEPTH, MM8G_MAXKB>), grid, dim3(256), lds, as_stream(stream), b);
      rc = check_launch("mm8g_kernel");
      if (rc != RWKV7MI_OK || S == 1) return rc;
      if (O % 4 == 0) {
        const dim3 rgrid((unsigned)((rows * O / 4 + 255) / 256), (unsigned)nprob);
        hipLaunchKernelGGL((mm8g_reduce_kernel<TA, TM, 4>), rgrid, dim3(256), 0, as_stream(stream), b);
      } else {
        const dim3 rgrid((unsigned)((rows * O + 255) / 256), (unsigned)nprob);
        hipLaunchKernelGGL((mm8g_reduce_kernel<TA, TM, 1>), rgrid, dim3(256), 0, as_stream(stream), b);
      }
      return check_launch("mm8g_reduce_kernel");
    });
  });
}

extern "C" int rwkv7mi_mm8t_gemm_multi(int nprob, const void* const* x, const uint8_t* const* w_blk,
                                       const void* const* mx, const void* const* rx, const void* const* my,
                                       const void* const* ry, const void* const* bias, const void* const* residual,
                                       void* const* y, const int* epilogue, int64_t rows, int64_t I, int64_t O,
                                       int act_dtype, int meta_dtype, int splits, void* workspace,
                                       size_t workspace_bytes, void* stream) {
  return mm8g_run("mm8t_gemm_multi", nprob, x, w_blk, mx, rx, my, ry, bias, residual, y, epilogue, rows, I, O,
                  act_dtype, meta_dtype, splits, workspace, workspace_bytes, stream);
}

extern "C" int rwkv7mi_mm8t_gemm_multi_lora(int nprob, const void* const* x, const uint8_t* const* w_blk,
                                            const void* const* mx, const void* const* rx, const void* const* my,
                                            const void* const* ry, const void* const* bias,
                                            const void* const* residual, void* const* y, const int* epilogue,
                                            int64_t rows, int64_t I, int64_t O, int act_dtype, int meta_dtype,
                                            int splits, void* workspace, size_t workspace_bytes,
                                            int64_t lora_nprob, const void* const* lora_x,
                                            const void* const* lora_w_down, const int64_t* lora_ranks,
                                            int64_t lora_splits, float* lora_part, size_t lora_part_bytes,
                                            void* stream) {
  const char* who = "mm8t_gemm_multi_lora";
  if (rows == 0) return RWKV7MI_OK;
  if (lora_splits < 1 || lora_splits > 64) return fail(RWKV7MI_EINVAL, std::string(who) + ": lora_splits 1..64");
  LoraBatch lb{};
  int tiles = 0;
  if (int rc = lora_down_batch(lora_nprob, lora_x, lora_w_down, lora_ranks, rows, I, (int)lora_splits, act_dtype,
                               &lb, &tiles))
    return rc;
  size_t need = 0;
  for (int64_t i = 0; i < lora_nprob; ++i) need += (size_t)lora_splits * (size_t)rows * (size_t)lora_ranks[i] * 4u;
  if (!lora_part || lora_part_bytes < need || (reinterpret_cast<uintptr_t>(lora_part) & 15))
    return fail(RWKV7MI_ESIZE, std::string(who) + ": LoRA partial buffer missing, unaligned or too small");
  return mm8g_run(who, nprob, x, w_blk, mx, rx, my, ry, bias, residual, y, epilogue, rows, I, O, act_dtype,
                  meta_dtype, splits, workspace, workspace_bytes, stream, &lb, lora_part, tiles);
}

// ---- allocation-free form: the scratch lives in this file's device array
// (one copy per GPU, held until the process ends).  Its host-side name is
// only a stand-in; the device address of each GPU's copy comes from
// hipGetSymbolAddress, taken once per device with that device current.
namespace {
__device__ __align__(256) unsigned char scratch[RWKV7MI_MM8T_GEMM_SCRATCH_BYTES];
std::mutex g_scratch_mu;
void* g_scratch_ptr[64] = {};
}  // namespace

static int mm8g_scratch(void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
    return fail(RWKV7MI_ELAUNCH, "mm8t_gemm_multi_noalloc: no current device");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(RWKV7MI_ELAUNCH, std::string("mm8t_gemm_multi_noalloc: hipGetSymbolAddress failed: ") +
                                       hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return RWKV7MI_OK;
}

extern "C" int rwkv7mi_mm8t_gemm_multi_noalloc(int nprob, const void* const* x, const uint8_t* const* w_blk,
                                               const void* const* mx, const void* const* rx, const void* const* my,
                                               const void* const* ry, const void* const* bias,
                                               const void* const* residual, void* const* y, const int* epilogue,
                                               int64_t rows, int64_t I, int64_t O, int act_dtype, int meta_dtype,
                                               int splits, void* stream) {
  const size_t need = rwkv7mi_mm8t_gemm_workspace_bytes(nprob, rows, I, O, splits);
  if (rows > 0 && need > (size_t)RWKV7MI_MM8T_GEMM_SCRATCH_BYTES)
    return fail(RWKV7MI_ESIZE, "mm8t_gemm_multi_noalloc: the call needs " + std::to_string(need) +
                                   " scratch bytes, more than the library's fixed " +
                                   std::to_string((size_t)RWKV7MI_MM8T_GEMM_SCRATCH_BYTES) +
                                   " (use rwkv7mi_mm8t_gemm_multi with a workspace)");
  void* ws = nullptr;
  if (rows > 0) {
    if (int rc = mm8g_scratch(&ws)) return rc;
  }
  return mm8g_run("mm8t_gemm_multi_noalloc", nprob, x, w_blk, mx, rx, my, ry, bias, residual, y, epilogue, rows, I,
                  O, act_dtype, meta_dtype, splits, ws, (size_t)RWKV7MI_MM8T_GEMM_SCRATCH_BYTES, stream);
}
