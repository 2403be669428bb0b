// MM8 dequant GEMV / small-batch GEMM over OUT-MAJOR weights, for gfx950.
//
// Same format as mm8.hip (rwkv7_hf/native_quant_mm8.py:62-126):
//   W_hat[i,o] = (w[i,o] + 0.5) * ry[i] * rx[o] + my[i] + mx[o]
//   y[b,o] = rx[o] * sum_i x'[b,i] (w[i,o] + 0.5) + sum_i x[b,i] my[i] + mx[o] sum_i x[b,i],
//   x' = x * ry,
// but the MM8 bytes are stored BLOCKED by output-column group: for group g
// (outputs 16g..16g+15) and K block b (inputs 128b..128b+127) one 2048-byte
// tile at byte (g KB + b) 2048, KB = ceil(I / 128), holding at byte
// 1024 h + 16 (16 q + c) + e the weight of output 16g + c, input
// 128b + 64h + 16q + e (h < 2, q < 4, c < 16, e < 16); tails padded with
// zeros.  A wave's step is then one contiguous 2 KB run (two 1 KB loads), the
// access pattern HBM streams fastest; 16 columns x 64 bytes per load (the
// plain [O, I] layout) measured ~25% slower on the 67 MB shapes.
// rwkv7mi_mm8t_block / _unblock convert from and to the reference's [I, O].
// MM4 (BITS = 4) keeps the out-major [O, I/2] layout.
//
// A workgroup owns 16 output columns and ALL of K: no split-K partials, no
// cross-workgroup ordering, deterministic fixed-order sums.
//
// Workgroup = NW (4 or 8) waves, 16 columns, up to 16 batch rows (one MFMA M
// tile).  K is walked in 128-row steps; wave w takes steps w, w+NW, ...  In a step,
// lane (n = l%16, kg = l/16) holds two 16-byte runs of column n, rows
// 16kg..16kg+15 and 64+16kg..64+16kg+15.
// Each 8-byte half is one B operand of v_mfma_f32_16x16x32_f16 (the MFMA's
// logical k = 8kg+e maps to physical row 64h + 16kg + 8q + e; the A operand
// uses the same map), converted to fp16 (w + 0.5) by v_perm + one packed add.
// Weight loads run DEPTH steps ahead of use (DEPTH x 2 KB per wave; about
// 32 KB in flight per CU streams fastest, deeper rings congest HBM), across
// LDS re-staging barriers
// (__syncthreads waits on LDS traffic only).  All global loads are raw buffer
// loads whose out-of-range lanes get an offset past the descriptor's size, so
// the loop is branch-free and the load counter waits stay exact.
//
// x' is staged per K-chunk in LDS as fp16 hi + lo (x' = hi + lo to ~22 bits),
// so each product is two MFMAs with fp32 accumulation.  A rows beyond the
// batch read a duplicate row: MFMA row m of D depends only on A row m, and
// those D rows are never stored.  The per-row sums (sum x, sum x*my) are
// accumulated in fixed thread order during staging.
//
// Up to four problems with the same (rows, I, O) run in one launch
// (blockIdx.y), e.g. the R/K/V projections of one layer.
#include "mm8t_common.h"
#include "lora_common.h"

namespace rwkv7mi {

constexpr int MM8T_SB = 4;  // x' staging groups per load batch
constexpr int MM8T_LDS_X = 72 * 1024;      // x' staging bytes per workgroup (2 workgroups per CU)
constexpr int MM8T_LDS_X_ONE = 144 * 1024; // when the grid is at most one workgroup per CU

// Optional decode prologue (rwkv7_hf/fused_decode_norm_mix.py:39-86, 161-296):
// the activations are built from the residual row x as
//   h = LayerNorm(x),  x_p = h + (prev - h) * mix_p   (rounded to the act dtype)
// inside the x' staging, so no separate mix kernel runs.  Every workgroup
// computes the row statistics itself.  Workgroups past the products (x >= gx,
// y == 0) compute no product: the first writes h (the next token's `prev`) and
// up to four extra mixes of the same h for other consumers; the next `lwgs`
// ones take those extra mixes as inputs of low-rank down projections (the
// decode LoRA), whole-K dot products written as fp32.
struct Mm8tPro {
  const void* prev;  // [rows, I] previous token's LN output
  const void* ln_w;
  const void* ln_b;  // [I]
  void* h_out;       // [rows, I] or null
  const void* aux_mix[4];
  void* aux_out[4];  // [rows, I]
  float eps;
  int naux;
  // LoRA down projections of the extra mixes: lw[a] [lrank[a], I] (act dtype),
  // lout[loff[a] + row * lrank[a] + j] = mix_a[row] . lw[a][j]
  const void* lw[4];
  int lrank[4];
  int64_t loff[4];
  float* lout;
  int lwgs;   // workgroups for them (0: none)
  int lrtot;  // sum of the ranks
};

struct Mm8tBatch {
  Mm8tProb p[MM8T_MAXPROB];
  Mm8tPro pro;
  int rows, I, O, KC;
  int gx;  // product workgroups along x; with the LN-mix prologue one more (x == gx) writes h and the extra mixes
  // Split K (no prologue, 8-bit): S > 1 splits the inputs into S ranges of KC
  // (one LDS chunk each); workgroup x takes range x % S, so its x' is staged
  // once for all its column groups, and writes fp32 partials
  // part[((s * nprob + p) * rows + row) * O + o] for mm8t_split_reduce_kernel.
  int S;
  float* part;
  // Tail workgroups x >= gx (no prologue): the LoRA down projections of the
  // decode step, whose inputs (the w/a/g/v mixes) are ready when this launch
  // starts, on the CUs the products leave free (lora_down_tile; 0: none)
  LoraBatch tl;
  float* tl_part;
  int tl_rows, tl_tiles, tl_wgs;
};

// The tail workgroups' share of the (down tile, K range) units, 256 lanes per
// unit (two units at a time in an eight-wave workgroup); smem holds the units'
// cross-wave sums.  Every lane runs the same trip count (one barrier each).
template <typename TA, int NW>
__device__ __forceinline__ void mm8t_lora_tail(const Mm8tBatch& B, char* smem) {
  constexpr int HALVES = NW * 64 / 256;
  const int h = (int)threadIdx.x >> 8;
  const int tid = (int)threadIdx.x & 255;
  float(*s_red)[16][17] = reinterpret_cast<float(*)[16][17]>(smem) + 4 * h;
  const int nv = B.tl_tiles * B.tl.ks;
  for (int v0 = ((int)blockIdx.x - B.gx) * HALVES; v0 < nv; v0 += B.tl_wgs * HALVES) {
    const int v = v0 + h;
    const bool valid = v < nv;
    const int vv = valid ? v : 0;
    lora_down_tile<1, TA>(B.tl, B.tl_rows, B.tl_part, vv % B.tl_tiles, vv / B.tl_tiles, tid, valid, s_red);
    __syncthreads();  // the next unit reuses s_red
  }
}

// bytes of (d0, d1) = rows r..r+7 of one column -> fp16 [w + 0.5] x 8
__device__ __forceinline__ f16x8 mm8t_b_operand(uint32_t d0, uint32_t d1) {
  const f16x2 half_off = {(_Float16)-1023.5f, (_Float16)-1023.5f};
  f16x2 p0 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, d0, 0x04010400u)) + half_off;
  f16x2 p1 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, d0, 0x04030402u)) + half_off;
  f16x2 p2 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, d1, 0x04010400u)) + half_off;
  f16x2 p3 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, d1, 0x04030402u)) + half_off;
  return (f16x8){p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

// nibbles of dword d = rows r..r+7 of one column (low nibble first) -> fp16
// [u + 0.5] x 8 in the order [0,4,1,5,2,6,3,7] (the x' staging for 4-bit
// weights stores each 8-group in the same order).  fp16 pairs with exponent
// 0x64 hold 1024 + u (nibble in bits 0-3) or 1024 + 16 u (bits 4-7); one
// packed add of -1023.5, or one packed fma by 1/16 with -63.5, gives u + 0.5
// exactly.  9 VALU ops per dword.
__device__ __forceinline__ f16x8 mm4t_b_operand(uint32_t d) {
  const uint32_t d8 = d >> 8;
  const f16x2 a = __builtin_bit_cast(f16x2, and_or(d, 0x000F000Fu, 0x64006400u));
  const f16x2 b = __builtin_bit_cast(f16x2, and_or(d, 0x00F000F0u, 0x64006400u));
  const f16x2 c = __builtin_bit_cast(f16x2, and_or(d8, 0x000F000Fu, 0x64006400u));
  const f16x2 e = __builtin_bit_cast(f16x2, and_or(d8, 0x00F000F0u, 0x64006400u));
  const f16x2 half_off = {(_Float16)-1023.5f, (_Float16)-1023.5f};
  const f16x2 sixteenth = {(_Float16)0.0625f, (_Float16)0.0625f};
  const f16x2 off16 = {(_Float16)-63.5f, (_Float16)-63.5f};
  const f16x2 p0 = a + half_off, p2 = c + half_off;
  const f16x2 p1 = __builtin_elementwise_fma(b, sixteenth, off16);
  const f16x2 p3 = __builtin_elementwise_fma(e, sixteenth, off16);
  return (f16x8){p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

// BITS = 8: MM8 bytes, a step is 128 K rows; BITS = 4: MM4 nibbles packed in
// pairs along K (low nibble = even row), a step is 256 K rows.  Either way a
// step is two 16-byte loads per lane, 128 bytes of each of the 16 columns.
template <typename TA, typename TM, int NW, int CSW, int BITS, bool PRO, int RING, bool DEF = false>
__global__ __launch_bounds__(64 * NW, 8 / NW) void mm8t_kernel(const Mm8tBatch B) {
  // NW waves per workgroup; CSW: steps per wave per K-chunk (KC = RS NW CSW
  // rows).  The chunk body is fully unrolled so the load ring needs no
  // loop-carried waits.
  constexpr int NT = 64 * NW;
  constexpr int DEPTH = CSW < RING ? CSW : RING;
  constexpr int RS = BITS == 8 ? 128 : 256;  // K rows per step
  constexpr int NB = BITS == 8 ? 4 : 8;      // B operands (8 rows each) per step
  const Mm8tProb& P = B.p[blockIdx.y];
  const int I = B.I, O = B.O;
  const int bcol = BITS == 8 ? I : I / 2;  // bytes per column
  constexpr int KC = RS * NW * CSW;
  const int row0 = blockIdx.z * 16;
  const int nrows = min(16, B.rows - row0);
  const int ngroups = (O + MM8T_COLS - 1) / MM8T_COLS;
  const int S = B.S;
  const int gstride = B.gx / S;
  // LN-mix prologue: workgroup x == gx computes no product; it stages the row
  // like the others and writes h and the extra mixes (its twins for the other
  // problems exit at once)
  const bool aux_wg = PRO && (int)blockIdx.x >= B.gx;
  const int lora_i = (int)blockIdx.x - B.gx - 1;  // >= 0: a LoRA-down workgroup
  if (aux_wg && blockIdx.y != 0) return;
  constexpr int XS = KC + 8;  // LDS row stride (halfs)
  extern __shared__ __align__(16) char smem[];
  if constexpr (!PRO && BITS == 8) {
    if (B.tl_wgs > 0 && (int)blockIdx.x >= B.gx) {  // a LoRA-down tail workgroup
      if (blockIdx.y == 0 && blockIdx.z == 0) mm8t_lora_tail<TA, NW>(B, smem);
      return;
    }
  }
  _Float16* xh = reinterpret_cast<_Float16*>(smem);
  _Float16* xl = xh + nrows * XS;
  __shared__ float red[NW][16][17];
  __shared__ float wsum[NW][2];
  __shared__ float wsum2[NW][2][2];  // per-wave staging: [wave][row][sum x, sum x my]
  __shared__ float rsum[16][2];
  __shared__ float wpart[PRO ? 2 : 1][PRO ? NW : 1];  // LN-mix prologue: per-wave partial sums

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar step logic
  const int lane = tid & 63;
  const int n = lane & 15;
  const int kg = lane >> 4;

  // A column group's 16 columns are one contiguous run of ncols * I bytes;
  // groups past the end get an empty descriptor (all loads read zeros).
  const int KBLK = (I + 127) / 128;  // 8-bit: 2 KB tiles per column group
  auto group_rsrc = [&](int g) {
    if constexpr (BITS == 8) {
      const uint32_t gb = (uint32_t)KBLK * 2048u;
      return mm8t_rsrc(P.w + (int64_t)(g < ngroups ? g : 0) * gb, g < ngroups ? gb : 0u);
    }
    const int c0 = g * MM8T_COLS;
    const int nc = g < ngroups ? min(MM8T_COLS, O - c0) : 0;
    return mm8t_rsrc(P.w + (int64_t)(g < ngroups ? c0 : 0) * bcol, (uint32_t)nc * (uint32_t)bcol);
  };
  const __amdgpu_buffer_rsrc_t xr =
      mm8t_rsrc(reinterpret_cast<const TA*>(P.x) + (int64_t)row0 * I, (uint32_t)(nrows * I * sizeof(TA)));
  const __amdgpu_buffer_rsrc_t ryr = mm8t_rsrc(P.ry, (uint32_t)(I * sizeof(TM)));
  const __amdgpu_buffer_rsrc_t myr = mm8t_rsrc(P.my, (uint32_t)(I * sizeof(TM)));
  const uint32_t lane_off = (uint32_t)n * (uint32_t)bcol + 16u * kg;
  // split K: this workgroup's range of inputs starts at kbase (one chunk)
  const int sidx = (int)blockIdx.x % S;
  const int kbase = S > 1 ? sidx * KC : 0;
  const int nchunks = S > 1 ? 1 : (I + KC - 1) / KC;
  const int J = nchunks * CSW;  // steps per wave per column group

  // staging: TPR threads per batch row, fixed for the whole kernel
  int rp2 = 1;
  while (rp2 < nrows) rp2 <<= 1;
  const int TPR = NT / rp2;
  const int sr = tid / TPR;
  const int su = tid % TPR;
  constexpr int NQ = KC >> 3;              // 8-element groups per chunk row
  const int QIT = (NQ + TPR - 1) / TPR;    // uniform trip count
  float sx = 0.f, sxmy = 0.f;

  // x' staging in batches of MM8T_SB groups: issue (loads in flight together),
  // then finish (x' = x ry as fp16 hi + lo into LDS, row sums).  Rows past I
  // stage as zeros.
  constexpr int SB = PRO ? 2 : MM8T_SB;  // staging groups per load batch
  Raw8<TA> rxv[SB];
  Raw8<TM> rrv[SB], rmv[SB];
  // LN-mix prologue operands (act dtype): prev row, this problem's mix, LN w / b
  constexpr int SBP = PRO ? SB : 1;
  float pro_mean = 0.f, pro_rstd = 0.f;  // this thread's row statistics
  Raw8<TA> rpv[SBP], rcv[SBP], rwv[SBP], rbv[SBP], rav[SBP][4];
  // (empty descriptors when the prologue is off: nothing reads them)
  const __amdgpu_buffer_rsrc_t prr =
      mm8t_rsrc(PRO ? reinterpret_cast<const TA*>(B.pro.prev) + (int64_t)row0 * I : nullptr,
                PRO ? (uint32_t)(nrows * I * sizeof(TA)) : 0u);
  const __amdgpu_buffer_rsrc_t mixr = mm8t_rsrc(PRO ? P.mix : nullptr, PRO ? (uint32_t)(I * sizeof(TA)) : 0u);
  const __amdgpu_buffer_rsrc_t lnwr = mm8t_rsrc(PRO ? B.pro.ln_w : nullptr, PRO ? (uint32_t)(I * sizeof(TA)) : 0u);
  const __amdgpu_buffer_rsrc_t lnbr = mm8t_rsrc(PRO ? B.pro.ln_b : nullptr, PRO ? (uint32_t)(I * sizeof(TA)) : 0u);
  __amdgpu_buffer_rsrc_t auxr[4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
    auxr[a] = mm8t_rsrc(PRO && a < B.pro.naux ? B.pro.aux_mix[a] : nullptr,
                        PRO && a < B.pro.naux ? (uint32_t)(I * sizeof(TA)) : 0u);
  auto stage_issue = [&](int kc0, int it0) {
    // x first: the prologue's row statistics wait on these loads only
#pragma unroll
    for (int u = 0; u < SB; ++u) {
      const int q = su + (it0 + u) * TPR;
      const int k = kbase + kc0 + 8 * q;
      rxv[u] = mm8t_ld8<TA>(xr, (uint32_t)(sr * I + k), sr < nrows && q < NQ && k < I);
    }
#pragma unroll
    for (int u = 0; u < SB; ++u) {
      const int q = su + (it0 + u) * TPR;
      const int k = kbase + kc0 + 8 * q;
      const bool valid = sr < nrows && q < NQ && k < I;
      rrv[u] = mm8t_ld8<TM>(ryr, (uint32_t)k, valid);
      rmv[u] = mm8t_ld8<TM>(myr, (uint32_t)k, valid);
      if constexpr (PRO) {
        rpv[u] = mm8t_ld8<TA>(prr, (uint32_t)(sr * I + k), valid);
        rcv[u] = mm8t_ld8<TA>(mixr, (uint32_t)k, valid);
        rwv[u] = mm8t_ld8<TA>(lnwr, (uint32_t)k, valid);
        rbv[u] = mm8t_ld8<TA>(lnbr, (uint32_t)k, valid);
        if (aux_wg) {  // uniform: the product workgroups issue none of these
#pragma unroll
          for (int a = 0; a < 4; ++a) rav[u][a] = mm8t_ld8<TA>(auxr[a], (uint32_t)k, valid && a < B.pro.naux);
        }
      }
    }
  };
  auto stage_finish = [&](int it0) {
#pragma unroll
    for (int u = 0; u < SB; ++u) {
      const int q = su + (it0 + u) * TPR;
      float xv[8], rv[8], mv[8];
      mm8t_cvt8(rxv[u], xv);
      mm8t_cvt8(rrv[u], rv);
      mm8t_cvt8(rmv[u], mv);
      if constexpr (PRO) {
        // x_p = round(h + (prev - h) mix), h = round((x - mean) / std * w + b)
        float pv[8], cv[8], wv[8], bv[8];
        mm8t_cvt8(rpv[u], pv);
        mm8t_cvt8(rcv[u], cv);
        mm8t_cvt8(rwv[u], wv);
        mm8t_cvt8(rbv[u], bv);
        const float mean = pro_mean, rstd = pro_rstd;
        const bool valid = sr < nrows && q < NQ && 8 * q < I;  // one chunk: it starts at k = 0
        float hv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          // h is rounded to the activation dtype before the mix, as the
          // reference's normed tensor is
          hv[e] = to_f32(from_f32<TA>((xv[e] - mean) * rstd * wv[e] + bv[e]));
          xv[e] = valid ? to_f32(from_f32<TA>(hv[e] + (pv[e] - hv[e]) * cv[e])) : 0.f;
        }
        if (aux_wg && valid) {
          const int64_t off = (int64_t)(row0 + sr) * I + 8 * q;
          if (lora_i < 0 && B.pro.h_out) st8(reinterpret_cast<TA*>(B.pro.h_out) + off, hv);
#pragma unroll
          for (int a = 0; a < 4; ++a) {
            if (a < B.pro.naux) {
              float av[8], ov[8];
              mm8t_cvt8(rav[u][a], av);
#pragma unroll
              for (int e = 0; e < 8; ++e) ov[e] = hv[e] + (pv[e] - hv[e]) * av[e];
              if (lora_i < 0)
                st8(reinterpret_cast<TA*>(B.pro.aux_out[a]) + off, ov);
              else  // the LoRA inputs, rounded as the mix tensors are, into LDS
                st8(reinterpret_cast<TA*>(smem) + (int64_t)(a * nrows + sr) * (I + 8) + 8 * q, ov);
            }
          }
        }
      }
      f16x8 hi, lo;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        // 4-bit weights pair rows (e, e+4) in their B operands: store x' as
        // [0,4,1,5,2,6,3,7] so one 16-byte LDS read matches
        const int src = BITS == 8 ? e : (e >> 1) + 4 * (e & 1);
        const float xp = xv[src] * rv[src];
        const _Float16 h = (_Float16)xp;
        hi[e] = h;
        lo[e] = (_Float16)(xp - (float)h);
        sx += xv[e];
        sxmy += xv[e] * mv[e];
      }
      if (sr < nrows && q < NQ && !aux_wg) {  // (the LoRA workgroups keep their mixes there)
        *reinterpret_cast<f16x8*>(xh + sr * XS + 8 * q) = hi;
        *reinterpret_cast<f16x8*>(xl + sr * XS + 8 * q) = lo;
      }
    }
  };

  // Step j of this wave covers K rows RS (wave + NW j) .. +RS-1 of a group,
  // bytes 128 (wave + NW j) .. +127 of each column.  Segments at or beyond the
  // column's bytes (the tail step) read as zeros.
  u32x4 buf[DEPTH][2];
  auto load_step = [&](__amdgpu_buffer_rsrc_t r, int j, u32x4 (&b)[2]) {
    if constexpr (BITS == 8) {
      const int blk = kbase / 128 + wave + NW * j;
      const uint32_t boff = (uint32_t)blk * 2048u + 16u * (uint32_t)lane;
      b[0] = mm8t_ld16(r, blk < KBLK ? boff : MM8T_OOB);
      b[1] = mm8t_ld16(r, blk < KBLK ? boff + 1024u : MM8T_OOB);
      return;
    }
    const int kb = 128 * (wave + NW * j) + 16 * kg;
    const uint32_t off = lane_off + 128u * (uint32_t)(wave + NW * j);
    b[0] = mm8t_ld16(r, kb < bcol ? off : MM8T_OOB);
    b[1] = mm8t_ld16(r, kb + 64 < bcol ? off + 64u : MM8T_OOB);
  };
  // LN-mix prologue: LayerNorm statistics of each staged row from the x
  // registers of the first (only) staging batch, in two passes as the
  // unfused kernel takes them (mean, then the mean squared deviation).  A
  // row's TPR lanes sum with DPP rotations inside 16-lane rows, then across
  // rows and waves; every lane of a row ends with the same value.
  auto row_total = [&](float v, int pass) -> float {
    if (TPR < 16) {
      for (int o = TPR >> 1; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
      return __shfl(v, lane & ~(TPR - 1), 64);
    }
    v += dpp_row_ror<8>(v);
    v += dpp_row_ror<4>(v);
    v += dpp_row_ror<2>(v);
    v += dpp_row_ror<1>(v);
    if (TPR == 16) return __shfl(v, lane & ~15, 64);
    if (TPR == 32) {
      v += __shfl_xor(v, 16, 64);
      return __shfl(v, lane & ~31, 64);
    }
    v = (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
    if (TPR == 64) return v;
    if (lane == 0) wpart[pass][wave] = v;
    __syncthreads();
    const int wpr = TPR >> 6, w0 = (wave / wpr) * wpr;
    float t = 0.f;
    for (int q = 0; q < wpr; ++q) t += wpart[pass][w0 + q];
    return t;
  };
  auto pro_stats = [&]() {
    float xs[SB][8];
    float s1 = 0.f;
#pragma unroll
    for (int u = 0; u < SB; ++u) {
      const int q = su + u * TPR;
      const bool valid = sr < nrows && q < NQ && 8 * q < I;
      mm8t_cvt8(rxv[u], xs[u]);
#pragma unroll
      for (int e = 0; e < 8; ++e) s1 += valid ? xs[u][e] : 0.f;
    }
    pro_mean = row_total(s1, 0) / (float)I;
    float s2 = 0.f;
#pragma unroll
    for (int u = 0; u < SB; ++u) {
      const int q = su + u * TPR;
      const bool valid = sr < nrows && q < NQ && 8 * q < I;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float c = xs[u][e] - pro_mean;
        s2 += valid ? c * c : 0.f;
      }
    }
    pro_rstd = rsqrtf(row_total(s2, 1) / (float)I + B.pro.eps);  // biased variance, as F.layer_norm
  };

  // LoRA-down workgroup i: outputs j = NW i + wave, + NW lwgs, ... of the
  // concatenated ranks; each a whole-K dot product of one weight row (lanes
  // split K in 8-element runs) with the mix staged in LDS, reduced across the
  // wave in a fixed order
  auto lora_down = [&](int li) {
    __syncthreads();
    const TA* lm = reinterpret_cast<const TA*>(smem);
    for (int o = li * NW + wave; o < B.pro.lrtot; o += B.pro.lwgs * NW) {
      int qa = 0, j = o;
      while (qa < 3 && j >= B.pro.lrank[qa]) {
        j -= B.pro.lrank[qa];
        ++qa;
      }
      const __amdgpu_buffer_rsrc_t wrr =
          mm8t_rsrc(reinterpret_cast<const TA*>(B.pro.lw[qa]) + (int64_t)j * I, (uint32_t)(I * sizeof(TA)));
      float acc[2] = {0.f, 0.f};
      for (int k0 = 0; k0 < I; k0 += 512 * 4) {
        Raw8<TA> wv[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int k = k0 + 8 * (lane + 64 * u);
          wv[u] = mm8t_ld8<TA>(wrr, (uint32_t)k, k < I);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int k = k0 + 8 * (lane + 64 * u);
          float w8[8];
          mm8t_cvt8(wv[u], w8);
#pragma unroll
          for (int rr = 0; rr < 2; ++rr) {
            if (rr < nrows && k < I) {
              float x8[8];
              ld8(lm + (int64_t)(qa * nrows + rr) * (I + 8) + k, x8);
#pragma unroll
              for (int e = 0; e < 8; ++e) acc[rr] += w8[e] * x8[e];
            }
          }
        }
      }
#pragma unroll
      for (int rr = 0; rr < 2; ++rr) {
        float v = acc[rr];
        v += dpp_row_ror<8>(v);
        v += dpp_row_ror<4>(v);
        v += dpp_row_ror<2>(v);
        v += dpp_row_ror<1>(v);
        v = (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
        if (rr < nrows && lane == 0) B.pro.lout[B.pro.loff[qa] + (int64_t)(row0 + rr) * B.pro.lrank[qa] + j] = v;
      }
    }
  };

  int g = aux_wg ? ngroups : (int)blockIdx.x / S;       // (the prologue's own workgroup loads nothing)
  __amdgpu_buffer_rsrc_t wr = group_rsrc(g);             // this group
  __amdgpu_buffer_rsrc_t wn = group_rsrc(g + gstride);   // the next one

  // Per-wave staging (8-bit fp16 / bf16, one K chunk, at most two rows, no
  // LN-mix prologue): wave w consumes only the K blocks w + NW j, so it stages
  // just those (its own x' in LDS, its share of the row sums) and no workgroup
  // barrier stands between a wave's loads and its first product.  (With the
  // prologue every wave would need the whole row for the LN statistics; that
  // measured slower than the shared staging.)
  constexpr bool WSOK = BITS == 8 && sizeof(TA) == 2 && !PRO;
  const bool ws = WSOK && nrows <= 2 && nchunks == 1;
  // DEF (instances for 3..16 rows): shared staging of one chunk in two
  // batches: the second batch's loads go out before the products start and
  // it is finished only at step CSW / 2, the first whose K blocks lie in its
  // inputs (it holds inputs [KC / 2, KC); steps jl >= CSW / 2 read blocks
  // >= NW CSW / 2 = KC / (2 RS)), so its load latency overlaps the first
  // steps.  The issue is unconditional (all-invalid loads read zeros when
  // nothing is deferred) so the ring's load-counter waits stay exact.  (Its
  // registers cost one wave per SIMD of occupancy, which the one- and
  // two-row launches keep.)
  const bool defer = DEF && !PRO && !ws && nchunks == 1 && CSW >= 2 && QIT == 2 * SB && NQ % TPR == 0;
  const int last0 = defer ? SB : QIT;  // first iteration of the deferred batch
  float sxw[2] = {0.f, 0.f}, smw[2] = {0.f, 0.f};
  if (ws) {
    constexpr int NRND = (CSW + 3) / 4;  // 64 lanes cover four 128-input blocks per round
    Raw8<TA> wx[NRND][2];
    Raw8<TM> wry[NRND], wmy[NRND];
#pragma unroll
    for (int r = 0; r < NRND; ++r) {
      const int j = 4 * r + (lane >> 4);
      const int k = kbase + 128 * (wave + NW * j) + 8 * (lane & 15);  // global input index
      const bool valid = j < CSW && k < I;
#pragma unroll
      for (int rr = 0; rr < 2; ++rr) wx[r][rr] = mm8t_ld8<TA>(xr, (uint32_t)(rr * I + k), valid && rr < nrows);
      wry[r] = mm8t_ld8<TM>(ryr, (uint32_t)k, valid);
      wmy[r] = mm8t_ld8<TM>(myr, (uint32_t)k, valid);
    }
    __builtin_amdgcn_sched_barrier(0);
    load_step(wr, 0, buf[0]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int r = 0; r < NRND; ++r) {
      const int j = 4 * r + (lane >> 4);
      const int k = 128 * (wave + NW * j) + 8 * (lane & 15);
      float rv[8], mv[8];
      mm8t_cvt8(wry[r], rv);
      mm8t_cvt8(wmy[r], mv);
#pragma unroll
      for (int rr = 0; rr < 2; ++rr) {
        if (rr < nrows) {
          float xv[8];
          mm8t_cvt8(wx[r][rr], xv);  // blocks past I load as zeros
          f16x8 hi, lo;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float xp = xv[e] * rv[e];
            const _Float16 h = (_Float16)xp;
            hi[e] = h;
            lo[e] = (_Float16)(xp - (float)h);
            sxw[rr] += xv[e];
            smw[rr] += xv[e] * mv[e];
          }
          if (j < CSW) {
            *reinterpret_cast<f16x8*>(xh + rr * XS + k) = hi;
            *reinterpret_cast<f16x8*>(xl + rr * XS + k) = lo;
          }
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int d = 1; d < DEPTH; ++d) load_step(wr, d, buf[d]);
    __builtin_amdgcn_sched_barrier(0);
  } else {
  // chunk 0: the first staging batch goes out first, then ONE ring step, and the
  // rest of the ring only once x' is staged.  Every workgroup reads the same
  // x / ry / my lines; issued behind the whole grid's ring fill they would
  // queue behind tens of MB of weight requests (measured: staging 5 us instead
  // of 2 us on the 67 MB shapes), while one step keeps the weights streaming.
  stage_issue(0, 0);
  __builtin_amdgcn_sched_barrier(0);
  load_step(wr, 0, buf[0]);
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (PRO) pro_stats();  // the whole row is in this batch (checked by the host)
  stage_finish(0);
  if (aux_wg) {
    if constexpr (PRO) {
      if (lora_i >= 0) lora_down(lora_i);
    }
    return;
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int d = 1; d < DEPTH; ++d) load_step(wr, d, buf[d]);  // DEPTH <= CSW <= J
  __builtin_amdgcn_sched_barrier(0);
  for (int it0 = SB; it0 < last0; it0 += SB) {
    stage_issue(0, it0);
    stage_finish(it0);
  }
  if constexpr (DEF) stage_issue(0, last0);
  __syncthreads();
  }

  const int arow = n < nrows ? n : nrows - 1;
  // lane kg's 16-byte runs hold rows 16kg.. (8-bit) or 32kg.. (4-bit) of each half step
  const _Float16* ah = xh + arow * XS + (BITS == 8 ? 16 : 32) * kg;
  const _Float16* al = xl + arow * XS + (BITS == 8 ? 16 : 32) * kg;
  const TM* rx = reinterpret_cast<const TM*>(P.rx);
  const TM* mx = reinterpret_cast<const TM*>(P.mx);
  const TM* bias = reinterpret_cast<const TM*>(P.bias);

  // Column groups g = blockIdx.x, + gridDim.x, ...  With one K-chunk, x' stays
  // in LDS for all of them and the ring prefetches the next group's first
  // steps while this one finishes; with several chunks the host launches one
  // group per workgroup.
  for (bool first = true; g < ngroups; g += gstride, first = false) {
    f32x4 acc[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) acc[q] = (f32x4){0.f, 0.f, 0.f, 0.f};

    for (int c = 0; c < nchunks; ++c) {
      if (c > 0) {
        __syncthreads();
        for (int it0 = 0; it0 < QIT; it0 += SB) {
          stage_issue(c * KC, it0);
          stage_finish(it0);
        }
        __syncthreads();
      }
      // ---- this wave's CSW steps of the chunk; the load ring runs DEPTH steps ahead
      const bool last_chunk = c == nchunks - 1;
#pragma unroll
      for (int jl = 0; jl < CSW; ++jl) {
        const int d = jl % DEPTH;
        if constexpr (DEF) {
          if (jl == CSW / 2 && first && defer) {  // the deferred staging batch
            stage_finish(last0);
            __syncthreads();
          }
        }
        // convert this step's bytes first, then refill the same ring slot: the
        // slot is dead once converted, so it keeps its registers
        f16x8 bv[NB];
        if constexpr (BITS == 8) {
          bv[0] = mm8t_b_operand(buf[d][0][0], buf[d][0][1]);
          bv[1] = mm8t_b_operand(buf[d][0][2], buf[d][0][3]);
          bv[2] = mm8t_b_operand(buf[d][1][0], buf[d][1][1]);
          bv[3] = mm8t_b_operand(buf[d][1][2], buf[d][1][3]);
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            bv[q] = mm4t_b_operand(buf[d][0][q]);
            bv[4 + q] = mm4t_b_operand(buf[d][1][q]);
          }
        }
        if (jl + DEPTH < CSW) {
          load_step(wr, c * CSW + jl + DEPTH, buf[d]);
        } else {  // may wrap into the next group's first steps (uniform select)
          const int t = c * CSW + jl + DEPTH;
          load_step(last_chunk ? wn : wr, last_chunk ? t - J : t, buf[d]);
        }
        // keep the refill here: sunk to the end of the body it would leave the
        // ring empty while the body computes
        __builtin_amdgcn_sched_barrier(0);
        const int kl = RS * (wave + NW * jl);
#pragma unroll
        for (int hq = 0; hq < NB; ++hq) {
          // 8-bit: operand hq = rows 64(hq/2) + 16kg + 8(hq%2);
          // 4-bit: operand hq = rows 128(hq/4) + 32kg + 8(hq%4)
          const int off = BITS == 8 ? kl + 64 * (hq >> 1) + 8 * (hq & 1) : kl + 128 * (hq >> 2) + 8 * (hq & 3);
          const f16x8 a_hi = *reinterpret_cast<const f16x8*>(ah + off);
          const f16x8 a_lo = *reinterpret_cast<const f16x8*>(al + off);
          acc[hq & 3] = mfma16x16x32(a_hi, bv[hq], acc[hq & 3]);
          acc[hq & 3] = mfma16x16x32(a_lo, bv[hq], acc[hq & 3]);
        }
      }
    }
    const f32x4 accs = (acc[0] + acc[1]) + (acc[2] + acc[3]);

    if (first && ws) {
      // ---- per-row sums of the per-wave staging: each wave's total, then the
      // waves in order
#pragma unroll
      for (int rr = 0; rr < 2; ++rr) {
        const float a = wave_sum(sxw[rr]), b = wave_sum(smw[rr]);
        if (lane == 0) {
          wsum2[wave][rr][0] = a;
          wsum2[wave][rr][1] = b;
        }
      }
      __syncthreads();
      if (tid < nrows) {
        float a = 0.f, b = 0.f;
        for (int q = 0; q < NW; ++q) {
          a += wsum2[q][tid][0];
          b += wsum2[q][tid][1];
        }
        rsum[tid][0] = a;
        rsum[tid][1] = b;
      }
    } else if (first) {
      // ---- per-row sums (staging is complete): fixed-order butterfly inside
      // each row's lanes, then across waves
      const int width = TPR < 64 ? TPR : 64;
      for (int o = width >> 1; o > 0; o >>= 1) {
        sx += __shfl_xor(sx, o, 64);
        sxmy += __shfl_xor(sxmy, o, 64);
      }
      if (TPR >= 64 && lane == 0) {
        wsum[wave][0] = sx;
        wsum[wave][1] = sxmy;
      }
      __syncthreads();
      if (TPR >= 64) {
        if (tid < nrows) {
          const int wpr = TPR >> 6;  // waves per row
          float a = 0.f, b = 0.f;
          for (int q = 0; q < wpr; ++q) {
            a += wsum[tid * wpr + q][0];
            b += wsum[tid * wpr + q][1];
          }
          rsum[tid][0] = a;
          rsum[tid][1] = b;
        }
      } else if (su == 0 && sr < nrows) {
        rsum[sr][0] = sx;
        rsum[sr][1] = sxmy;
      }
    }
    // ---- wave partial tiles (lane holds col n, rows 4kg + e), then one thread
    // per (row, column) finishes; the barrier pair also fences the previous
    // group's reads of red[]
    __syncthreads();
#pragma unroll
    for (int e = 0; e < 4; ++e) red[wave][4 * kg + e][n] = accs[e];
    __syncthreads();
    if (tid < nrows * MM8T_COLS) {
      const int m = tid >> 4;
      const int cn = tid & 15;
      const int o = g * MM8T_COLS + cn;
      if (o < O) {
        float s = red[0][m][cn];
#pragma unroll
        for (int q = 1; q < NW; ++q) s += red[q][m][cn];
        float v = ld(rx, o) * s + rsum[m][1] + ld(mx, o) * rsum[m][0];
        if (S > 1) {  // this range's share; the reduce kernel adds the ranges, bias and epilogue
          B.part[(((int64_t)sidx * gridDim.y + blockIdx.y) * B.rows + row0 + m) * O + o] = v;
        } else {
          if (bias) v += ld(bias, o);
          const int64_t oi = (int64_t)(row0 + m) * O + o;
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
    wr = wn;
    wn = group_rsrc(g + 2 * gstride);
  }
}


// Split-K finish: y[p][row][o] = epilogue(sum_s part[s][p][row][o] + bias[o]),
// the ranges added in order 0..S-1 (deterministic).  V = 4 when O % 4 == 0.
template <typename TA, typename TM, int V>
__global__ __launch_bounds__(256) void mm8t_split_reduce_kernel(const Mm8tBatch B) {
  const int p = blockIdx.y;
  const Mm8tProb& P = B.p[p];
  const int64_t n = (int64_t)B.rows * B.O;
  const int64_t idx = ((int64_t)blockIdx.x * 256 + threadIdx.x) * V;
  if (idx >= n) return;
  float a[V];
#pragma unroll
  for (int v = 0; v < V; ++v) a[v] = 0.f;
  for (int sp = 0; sp < B.S; ++sp) {
    const float* src = B.part + ((int64_t)sp * gridDim.y + p) * n + idx;
    if constexpr (V == 4) {
      const float4 t = *reinterpret_cast<const float4*>(src);
      a[0] += t.x;
      a[1] += t.y;
      a[2] += t.z;
      a[3] += t.w;
    } else {
      a[0] += src[0];
    }
  }
  const int o0 = (int)(idx % B.O);
  const TM* bias = reinterpret_cast<const TM*>(P.bias);
#pragma unroll
  for (int v = 0; v < V; ++v) {
    float x = a[v];
    if (bias) x += ld(bias, o0 + v);
    if (P.epilogue == RWKV7MI_EPI_RELU2) {
      x = fmaxf(x, 0.f);
      x = x * x;
    } else if (P.epilogue == RWKV7MI_EPI_RESIDUAL) {
      x += ld(reinterpret_cast<const TA*>(P.residual), idx + v);
    }
    reinterpret_cast<TA*>(P.y)[idx + v] = from_f32<TA>(x);
  }
}

// x' staging chunk: the largest power-of-two multiple of 2 RS NW rows (at
// most 32 RS NW, 16 RS NW for the 4-bit eight-wave kernel; RS = K rows per
// step) whose hi/lo copy for the tile's rows fits the LDS budget, and no
// longer than I needs.  A grid of at most one workgroup per CU, or a tile of
// more than four rows (whose staging would otherwise repeat per chunk), uses
// most of the CU's LDS.
static int mm8t_chunk(int64_t rows, int64_t I, int64_t nwg, int nw, int bits) {
  const int64_t nr = rows < 16 ? rows : 16;
  const int64_t rs = bits == 8 ? 128 : 256;
  const int64_t budget = (nwg <= 256 || nr > 4) ? MM8T_LDS_X_ONE : MM8T_LDS_X;
  int64_t kc = 2 * rs * nw;
  if (nr * (kc + 8) * 4 > budget) return 0;  // not even the smallest chunk fits
  const int64_t steps = bits == 4 && nw == 8 ? 16 : 32;  // steps per wave per chunk
  while (kc < I && kc < rs * nw * steps && nr * (2 * kc + 8) * 4 <= budget) kc *= 2;
  return (int)kc;
}

static size_t mm8t_lds(int64_t rows, int KC) {
  const int64_t nr = rows < 16 ? rows : 16;
  return (size_t)nr * (KC + 8) * 4;
}

}  // namespace rwkv7mi

using namespace rwkv7mi;

template <typename TA, typename TM, int NW, int CSW, int BITS, bool PRO, int RING, bool DEF>
static int mm8t_go(dim3 grid, size_t lds, void* stream, const Mm8tBatch& b) {
  static std::atomic<uint64_t> lds_raised{0};  // devices whose dynamic LDS limit is raised for this instance
  if (int rc = raise_dynamic_lds(reinterpret_cast<const void*>(&mm8t_kernel<TA, TM, NW, CSW, BITS, PRO, RING, DEF>),
                                 MM8T_LDS_X_ONE + 1024, lds_raised, "mm8t_kernel"))
    return rc;
  hipLaunchKernelGGL((mm8t_kernel<TA, TM, NW, CSW, BITS, PRO, RING, DEF>), grid, dim3(64 * NW), lds, as_stream(stream),
                     b);
  return check_launch("mm8t_kernel");
}

template <typename TA, typename TM, int NW, int BITS, bool PRO, int RING, bool DEF = false>
static int mm8t_go_csw_ring(dim3 grid, size_t lds, void* stream, const Mm8tBatch& b) {
  switch (b.KC / ((BITS == 8 ? 128 : 256) * NW)) {
    case 2: return mm8t_go<TA, TM, NW, 2, BITS, PRO, RING, DEF>(grid, lds, stream, b);
    case 4: return mm8t_go<TA, TM, NW, 4, BITS, PRO, RING, DEF>(grid, lds, stream, b);
    case 8: return mm8t_go<TA, TM, NW, 8, BITS, PRO, RING, DEF>(grid, lds, stream, b);
    case 16: return mm8t_go<TA, TM, NW, 16, BITS, PRO, RING, DEF>(grid, lds, stream, b);
    default:
      // the 4-bit eight-wave kernel at 32 steps per chunk runs out of
      // registers; its chunks are capped at 16 steps
      if constexpr (BITS == 4 && NW == 8)
        return fail(RWKV7MI_EINVAL, "mm8t_kernel: chunk too long for the 4-bit eight-wave kernel");
      else
        return mm8t_go<TA, TM, NW, 32, BITS, PRO, RING, DEF>(grid, lds, stream, b);
  }
}

// Ring depth: about 32 KB of weight loads in flight per CU (2 KB per wave and
// step).  8-bit: depth 2 with eight resident waves per CU, 4 with four; the
// 4-bit path keeps its depth of 8.  Three or more rows of fp16 / bf16 take
// the instances that defer their second staging batch (DEF).
template <typename TA, typename TM, int NW, int BITS, bool PRO = false>
static int mm8t_go_csw(dim3 grid, size_t lds, void* stream, const Mm8tBatch& b, int waves_per_cu) {
  if constexpr (BITS == 4) {
    return mm8t_go_csw_ring<TA, TM, NW, BITS, PRO, 8>(grid, lds, stream, b);
  } else {
    constexpr bool DEFOK = !PRO && std::is_same<TA, TM>::value && sizeof(TA) == 2;
    if constexpr (DEFOK) {
      // the kernel's staging split: rp2 threads' rows, TPR threads per row,
      // QIT 8-element groups per thread, MM8T_SB per batch; deferral needs one
      // chunk staged in exactly two batches
      int rp2 = 1;
      while (rp2 < std::min(b.rows, 16)) rp2 <<= 1;
      const int tpr = 64 * NW / rp2, nq = b.KC / 8;
      const bool one_chunk = b.KC >= b.I || b.S > 1;
      if (waves_per_cu >= 8 && b.rows >= 3 && one_chunk && nq % tpr == 0 && nq / tpr == 2 * MM8T_SB)
        return mm8t_go_csw_ring<TA, TM, NW, BITS, PRO, 2, true>(grid, lds, stream, b);
    }
    return waves_per_cu >= 8 ? mm8t_go_csw_ring<TA, TM, NW, BITS, PRO, 2>(grid, lds, stream, b)
                             : mm8t_go_csw_ring<TA, TM, NW, BITS, PRO, 4>(grid, lds, stream, b);
  }
}

// compute units of the current device (cached per device)
int64_t rwkv7mi::mm8t_cus() {
  static int64_t cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int n = 0;
    cached[dev] = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0 ? n : 256;
  }
  return cached[dev];
}

// Waves per workgroup and x' chunk of a call.  At most one workgroup per CU:
// eight waves each, so twice the weight bytes are in flight per CU; otherwise
// four-wave workgroups, two per CU.  Without the prologue, an x' too big for
// two workgroups per CU (rows > 4) takes one eight-wave workgroup per CU
// instead of one four-wave one (measured 8-16% faster at 8 rows).  Returns the
// chunk (0: not even the smallest fits).
static int mm8t_plan(int nprob, int64_t rows, int64_t I, int64_t O, int bits, bool pro, int* nw_out) {
  const int64_t nwg = ((O + MM8T_COLS - 1) / MM8T_COLS) * nprob * ((rows + 15) / 16);
  int nw = nwg <= mm8t_cus() ? 8 : 4;
  int kc = mm8t_chunk(rows, I, nwg, nw, bits);
  if (!kc && nw == 8) {
    nw = 4;
    kc = mm8t_chunk(rows, I, nwg, nw, bits);
  }
  if (kc && !pro && nw == 4 && bits == 8 && mm8t_lds(rows, kc) > (size_t)MM8T_LDS_X) {
    const int kc8 = mm8t_chunk(rows, I, nwg, 8, bits);
    if (kc8) {
      nw = 8;
      kc = kc8;
    }
  }
  *nw_out = nw;
  return kc;
}

// Bytes of split-K partials a call needs (0: no split).
static size_t mm8t_part_bytes(int S, int nprob, int64_t rows, int64_t O) {
  return S > 1 ? (size_t)S * (size_t)nprob * (size_t)rows * (size_t)O * 4u : 0;
}

// Split count for a call without the prologue: 1 when x' fits one LDS chunk,
// else one split per chunk (the ranges' x' stays staged for all column groups).
static int mm8t_auto_splits(int64_t I, int KC) { return KC >= I ? 1 : (int)((I + KC - 1) / KC); }

static int mm8t_launch(int nprob, const Mm8tProb* probs, int64_t rows, int64_t I, int64_t O, int act_dtype,
                       int meta_dtype, void* stream, const char* who, int bits = 8, const Mm8tPro* pro = nullptr,
                       void* workspace = nullptr, size_t workspace_bytes = 0, int* splits_out = nullptr,
                       bool defer_reduce = false, const LoraBatch* tl = nullptr, float* tl_part = nullptr,
                       int tl_tiles = 0) {
  const std::string w(who);
  if (nprob < 1 || nprob > MM8T_MAXPROB) return fail(RWKV7MI_EINVAL, w + ": 1..4 problems per launch");
  if (rows < 0 || I <= 0 || O <= 0) return fail(RWKV7MI_EINVAL, w + ": bad shape");
  if (rows == 0) return RWKV7MI_OK;
  if (I % (bits == 8 ? 16 : 32))
    return fail(RWKV7MI_EINVAL, w + (bits == 8 ? ": in_features must be a multiple of 16"
                                               : ": in_features must be a multiple of 32"));
  // buffer descriptors cover 16 columns x I bytes and 16 rows x I activations
  if (I > (1 << 24) || O > INT32_MAX || rows > 65535 * 16) return fail(RWKV7MI_EINVAL, w + ": too large");
  if (!valid_dtype(act_dtype) || !valid_dtype(meta_dtype)) return fail(RWKV7MI_EINVAL, w + ": bad dtype");
  for (int p = 0; p < nprob; ++p) {
    const Mm8tProb& q = probs[p];
    if (!q.x || !q.w || !q.mx || !q.rx || !q.my || !q.ry || !q.y) return fail(RWKV7MI_EINVAL, w + ": null pointer");
    if ((reinterpret_cast<uintptr_t>(q.x) | reinterpret_cast<uintptr_t>(q.w) | reinterpret_cast<uintptr_t>(q.my) |
         reinterpret_cast<uintptr_t>(q.ry)) & 15)
      return fail(RWKV7MI_EINVAL, w + ": x, the weights, my and ry must be 16-byte aligned");
    if (q.epilogue < 0 || q.epilogue > 2) return fail(RWKV7MI_EINVAL, w + ": bad epilogue");
    if (q.epilogue == RWKV7MI_EPI_RESIDUAL && !q.residual) return fail(RWKV7MI_EINVAL, w + ": residual missing");
  }
  Mm8tBatch b{};
  for (int p = 0; p < nprob; ++p) b.p[p] = probs[p];
  if (pro) b.pro = *pro;
  b.rows = (int)rows;
  b.I = (int)I;
  b.O = (int)O;
  const int64_t ngroups = (O + MM8T_COLS - 1) / MM8T_COLS;
  const int64_t rtiles = (rows + 15) / 16;
  const int64_t cus = mm8t_cus();
  int nw = 8;
  b.KC = mm8t_plan(nprob, rows, I, O, bits, pro != nullptr, &nw);
  if (!b.KC) return fail(RWKV7MI_EINVAL, w + ": x' staging does not fit in LDS");
  if (pro) {
    // the prologue takes the row statistics from one staging batch (two
    // 8-element groups per thread): the whole row in one chunk, and
    // 2 * 8 * (threads per row) >= chunk; eight waves double the threads
    auto batches = [&](int nw_, int kc) {
      int64_t rp2 = 1;
      while (rp2 < std::min<int64_t>(rows, 16)) rp2 <<= 1;
      const int64_t tpr = 64 * nw_ / rp2;
      return tpr > 0 ? (kc / 8 + tpr - 1) / tpr : INT64_MAX;
    };
    if (nw == 4 && (b.KC < I || batches(4, b.KC) > 2)) {
      const int kc8 = mm8t_chunk(rows, I, ngroups * nprob * rtiles, 8, bits);
      if (kc8 >= I && batches(8, kc8) <= 2) {
        nw = 8;
        b.KC = kc8;
      }
    }
    if (b.KC < I || batches(nw, b.KC) > 2 || bits != 8)
      return fail(RWKV7MI_EINVAL, w + ": the LN-mix prologue needs the whole row in one staging batch "
                                      "(rows <= 2 at in_features 4096)");
  }
  // split K when x' needs several chunks and the caller gave a workspace for
  // the partials (8-bit, no prologue); otherwise the chunks are re-staged per
  // column group
  int S = 1;
  if (!pro && bits == 8 && workspace) {
    S = mm8t_auto_splits(I, b.KC);
    if (S > 1 && (workspace_bytes < mm8t_part_bytes(S, nprob, rows, O) ||
                  (reinterpret_cast<uintptr_t>(workspace) & 15)))
      return fail(RWKV7MI_ESIZE, w + ": split-K workspace missing, unaligned or smaller than "
                                     "rwkv7mi_mm8t_matmul_workspace_bytes");
  }
  if (tl && (pro || bits != 8 || S != 1 || rows > 16 || !tl_part || tl_tiles <= 0))
    return fail(RWKV7MI_EINVAL, w + ": the LoRA-down tail runs with the 8-bit GEMV of at most 16 rows, "
                                    "without the prologue or split K");
  if (splits_out) *splits_out = S;
  b.S = S;
  b.part = S > 1 ? reinterpret_cast<float*>(workspace) : nullptr;
  size_t lds = mm8t_lds(rows, b.KC);
  int64_t extra = pro ? 1 : 0;  // the prologue's own workgroups (x >= gx, y == 0)
  if (pro && pro->lrtot > 0) {
    // LoRA-down workgroups: two outputs per wave (measured best at the 7.2B
    // ranks: fewer workgroups stream their weights too slowly, more take
    // product slots); their mixes sit in LDS
    b.pro.lwgs = (int)((pro->lrtot + 2 * nw - 1) / (2 * nw));
    extra += b.pro.lwgs;
    lds = std::max<size_t>(lds, (size_t)pro->naux * (size_t)rows * (size_t)(I + 8) * 2u);
    if (lds > (size_t)MM8T_LDS_X_ONE) return fail(RWKV7MI_EINVAL, w + ": the LoRA inputs do not fit in LDS");
  }
  // With x' in one LDS chunk, workgroups loop over column groups: as many as
  // stay resident, split between the problems and row tiles, and then as few
  // as give every workgroup the same number of groups (a launch lasts as long
  // as its busiest workgroup).  At two workgroups per CU the prologue's own
  // workgroups are not counted: they run as a third workgroup on a CU where
  // the kernel's registers allow it (the LN-mix instances do), else in the
  // first free slot (measured faster than shrinking the product grid for
  // them).  At one per CU they take product slots.
  int64_t gx = ngroups;  // column-group workgroups per split
  if (b.KC >= I || S > 1) {
    const int64_t per_cu = nw == 4 && lds <= MM8T_LDS_X ? 2 : 1;
    const int64_t slots = (cus * per_cu - (per_cu == 2 ? 0 : extra)) / (nprob * rtiles * S);
    if (slots >= 1 && slots < gx) {
      const int64_t k = (ngroups + slots - 1) / slots;  // groups per workgroup
      gx = (ngroups + k - 1) / k;
    }
  }
  b.gx = (int)(gx * S);
  if (tl) {
    // the tail: as many workgroups as the products leave slots free (at least
    // eight), two down units at a time in an eight-wave workgroup
    const int64_t halves = nw * 64 / 256;
    const int64_t units = (int64_t)tl_tiles * tl->ks;
    const int64_t per_cu = nw == 4 && lds <= MM8T_LDS_X ? 2 : 1;
    const int64_t free_slots = cus * per_cu - (int64_t)b.gx * nprob * rtiles;
    extra = std::min<int64_t>((units + halves - 1) / halves, std::max<int64_t>(free_slots, 8));
    b.tl = *tl;
    b.tl_part = tl_part;
    b.tl_rows = (int)rows;
    b.tl_tiles = tl_tiles;
    b.tl_wgs = (int)extra;
    lds = std::max(lds, (size_t)halves * 4u * 16u * 17u * 4u);
  }
  dim3 grid((unsigned)(b.gx + extra), (unsigned)nprob, (unsigned)rtiles);
  const int wpc = nw * (nw == 4 && lds <= MM8T_LDS_X ? 2 : 1);  // resident waves per CU
  const int rc = dispatch_dtype(act_dtype, [&](auto ta) {
    using TA = decltype(ta);
    return dispatch_dtype(meta_dtype, [&](auto tm) {
      using TM = decltype(tm);
      if (bits == 4)
        return nw == 8 ? mm8t_go_csw<TA, TM, 8, 4>(grid, lds, stream, b, wpc)
                       : mm8t_go_csw<TA, TM, 4, 4>(grid, lds, stream, b, wpc);
      if (pro) {
        if constexpr (std::is_same<TA, TM>::value && !std::is_same<TA, float>::value)
          return nw == 8 ? mm8t_go_csw<TA, TM, 8, 8, true>(grid, lds, stream, b, wpc)
                         : mm8t_go_csw<TA, TM, 4, 8, true>(grid, lds, stream, b, wpc);
        return fail(RWKV7MI_EINVAL, w + ": the LN-mix prologue takes fp16 or bf16 activations and metadata "
                                        "of the same dtype");
      }
      return nw == 8 ? mm8t_go_csw<TA, TM, 8, 8>(grid, lds, stream, b, wpc)
                     : mm8t_go_csw<TA, TM, 4, 8>(grid, lds, stream, b, wpc);
    });
  });
  if (rc != RWKV7MI_OK || S == 1 || defer_reduce) return rc;
  return dispatch_dtype(act_dtype, [&](auto ta) {
    using TA = decltype(ta);
    return dispatch_dtype(meta_dtype, [&](auto tm) {
      using TM = decltype(tm);
      const int64_t n = rows * O;
      if (O % 4 == 0)
        hipLaunchKernelGGL((mm8t_split_reduce_kernel<TA, TM, 4>), dim3((unsigned)((n / 4 + 255) / 256), nprob),
                           dim3(256), 0, as_stream(stream), b);
      else
        hipLaunchKernelGGL((mm8t_split_reduce_kernel<TA, TM, 1>), dim3((unsigned)((n + 255) / 256), nprob),
                           dim3(256), 0, as_stream(stream), b);
      return check_launch("mm8t_split_reduce_kernel");
    });
  });
}

extern "C" int rwkv7mi_mm8t_matmul(const void* x, const uint8_t* w_blk, const void* mx, const void* rx,
                                   const void* my, const void* ry, const void* bias, const void* residual,
                                   void* y, int64_t rows, int64_t I, int64_t O, int epilogue, int act_dtype,
                                   int meta_dtype, void* stream) {
  Mm8tProb p{x, nullptr, w_blk, mx, rx, my, ry, bias, residual, y, epilogue};
  return mm8t_launch(1, &p, rows, I, O, act_dtype, meta_dtype, stream, "mm8t_matmul");
}

extern "C" int rwkv7mi_mm8t_matmul_multi(int nprob, const void* const* x, const uint8_t* const* w_blk,
                                         const void* const* mx, const void* const* rx, const void* const* my,
                                         const void* const* ry, const void* const* bias,
                                         const void* const* residual, void* const* y, const int* epilogue,
                                         int64_t rows, int64_t I, int64_t O, int act_dtype, int meta_dtype,
                                         void* stream) {
  if (nprob < 1 || nprob > MM8T_MAXPROB) return fail(RWKV7MI_EINVAL, "mm8t_matmul_multi: 1..4 problems per launch");
  if (!x || !w_blk || !mx || !rx || !my || !ry || !y || !epilogue)
    return fail(RWKV7MI_EINVAL, "mm8t_matmul_multi: null array");
  Mm8tProb p[MM8T_MAXPROB];
  for (int i = 0; i < nprob; ++i)
    p[i] = Mm8tProb{x[i], nullptr, w_blk[i], mx[i], rx[i], my[i], ry[i], bias ? bias[i] : nullptr,
                    residual ? residual[i] : nullptr, y[i], epilogue[i]};
  return mm8t_launch(nprob, p, rows, I, O, act_dtype, meta_dtype, stream, "mm8t_matmul_multi");
}

extern "C" size_t rwkv7mi_mm8t_matmul_workspace_bytes(int nprob, int64_t rows, int64_t I, int64_t O) {
  if (nprob < 1 || nprob > MM8T_MAXPROB || rows <= 0 || I <= 0 || O <= 0) return 0;
  int nw = 8;
  const int kc = mm8t_plan(nprob, rows, I, O, 8, false, &nw);
  if (!kc) return 0;
  return mm8t_part_bytes(mm8t_auto_splits(I, kc), nprob, rows, O);
}

extern "C" int rwkv7mi_mm8t_matmul_multi_ws(int nprob, const void* const* x, const uint8_t* const* w_blk,
                                            const void* const* mx, const void* const* rx, const void* const* my,
                                            const void* const* ry, const void* const* bias,
                                            const void* const* residual, void* const* y, const int* epilogue,
                                            int64_t rows, int64_t I, int64_t O, int act_dtype, int meta_dtype,
                                            void* workspace, size_t workspace_bytes, void* stream) {
  if (nprob < 1 || nprob > MM8T_MAXPROB) return fail(RWKV7MI_EINVAL, "mm8t_matmul_multi_ws: 1..4 problems per launch");
  if (!x || !w_blk || !mx || !rx || !my || !ry || !y || !epilogue)
    return fail(RWKV7MI_EINVAL, "mm8t_matmul_multi_ws: null array");
  Mm8tProb p[MM8T_MAXPROB];
  for (int i = 0; i < nprob; ++i)
    p[i] = Mm8tProb{x[i], nullptr, w_blk[i], mx[i], rx[i], my[i], ry[i], bias ? bias[i] : nullptr,
                    residual ? residual[i] : nullptr, y[i], epilogue[i]};
  return mm8t_launch(nprob, p, rows, I, O, act_dtype, meta_dtype, stream, "mm8t_matmul_multi_ws", 8, nullptr,
                     workspace, workspace_bytes);
}

extern "C" int rwkv7mi_mm8t_matmul_multi_lora(int nprob, const void* const* x, const uint8_t* const* w_blk,
                                              const void* const* mx, const void* const* rx, const void* const* my,
                                              const void* const* ry, const void* const* bias,
                                              const void* const* residual, void* const* y, const int* epilogue,
                                              int64_t rows, int64_t I, int64_t O, int act_dtype, int meta_dtype,
                                              int64_t lora_nprob, const void* const* lora_x,
                                              const void* const* lora_w_down, const int64_t* lora_ranks,
                                              int64_t lora_splits, float* lora_part, size_t lora_part_bytes,
                                              void* stream) {
  const char* who = "mm8t_matmul_multi_lora";
  if (nprob < 1 || nprob > MM8T_MAXPROB) return fail(RWKV7MI_EINVAL, std::string(who) + ": 1..4 problems per launch");
  if (!x || !w_blk || !mx || !rx || !my || !ry || !y || !epilogue)
    return fail(RWKV7MI_EINVAL, std::string(who) + ": null array");
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
  Mm8tProb p[MM8T_MAXPROB];
  for (int i = 0; i < nprob; ++i)
    p[i] = Mm8tProb{x[i], nullptr, w_blk[i], mx[i], rx[i], my[i], ry[i], bias ? bias[i] : nullptr,
                    residual ? residual[i] : nullptr, y[i], epilogue[i]};
  return mm8t_launch(nprob, p, rows, I, O, act_dtype, meta_dtype, stream, who, 8, nullptr, nullptr, 0, nullptr,
                     false, &lb, lora_part, tiles);
}

extern "C" int rwkv7mi_mm8t_matmul_partials(const void* x, const uint8_t* w_blk, const void* mx, const void* rx,
                                            const void* my, const void* ry, int64_t rows, int64_t I, int64_t O,
                                            int act_dtype, int meta_dtype, void* workspace, size_t workspace_bytes,
                                            int* splits, void* stream) {
  if (!splits) return fail(RWKV7MI_EINVAL, "mm8t_matmul_partials: null splits");
  if (rwkv7mi_mm8t_matmul_workspace_bytes(1, rows, I, O) == 0)
    return fail(RWKV7MI_EINVAL, "mm8t_matmul_partials: this shape does not split K (use rwkv7mi_mm8t_matmul)");
  // a placeholder output: the split kernels write partials only
  Mm8tProb p{x, nullptr, w_blk, mx, rx, my, ry, nullptr, nullptr, workspace, RWKV7MI_EPI_NONE};
  return mm8t_launch(1, &p, rows, I, O, act_dtype, meta_dtype, stream, "mm8t_matmul_partials", 8, nullptr, workspace,
                     workspace_bytes, splits, true);
}

extern "C" int rwkv7mi_mm8t_lnmix_multi(int nprob, const void* x, const void* prev, const void* ln_w,
                                        const void* ln_b, float eps, const void* const* mix,
                                        const uint8_t* const* w_blk, const void* const* mx, const void* const* rx,
                                        const void* const* my, const void* const* ry, void* const* y,
                                        const int* epilogue, void* h_out, int naux, const void* const* aux_mix,
                                        void* const* aux_out, const void* const* lora_w, const int64_t* lora_ranks,
                                        float* lora_out, int64_t rows, int64_t I, int64_t O, int act_dtype,
                                        void* stream) {
  const char* who = "mm8t_lnmix_multi";
  if (nprob < 1 || nprob > MM8T_MAXPROB) return fail(RWKV7MI_EINVAL, "mm8t_lnmix_multi: 1..4 problems per launch");
  if (!x || !prev || !ln_w || !ln_b || !mix || !w_blk || !mx || !rx || !my || !ry || !y || !epilogue)
    return fail(RWKV7MI_EINVAL, "mm8t_lnmix_multi: null pointer");
  if (naux < 0 || naux > 4 || (naux && (!aux_mix || !aux_out)))
    return fail(RWKV7MI_EINVAL, "mm8t_lnmix_multi: 0..4 extra mixes");
  if (I % 8) return fail(RWKV7MI_EINVAL, "mm8t_lnmix_multi: in_features must be a multiple of 8");
  const uintptr_t al = reinterpret_cast<uintptr_t>(prev) | reinterpret_cast<uintptr_t>(ln_w) |
                       reinterpret_cast<uintptr_t>(ln_b) | reinterpret_cast<uintptr_t>(h_out);
  if (al & 15) return fail(RWKV7MI_EINVAL, "mm8t_lnmix_multi: prev, ln_w, ln_b, h_out must be 16-byte aligned");
  Mm8tPro pro{};
  pro.prev = prev;
  pro.ln_w = ln_w;
  pro.ln_b = ln_b;
  pro.h_out = h_out;
  pro.eps = eps;
  pro.naux = naux;
  for (int a = 0; a < naux; ++a) {
    if (!aux_mix[a] || !aux_out[a] ||
        ((reinterpret_cast<uintptr_t>(aux_mix[a]) | reinterpret_cast<uintptr_t>(aux_out[a])) & 15))
      return fail(RWKV7MI_EINVAL, "mm8t_lnmix_multi: extra mixes must be non-null and 16-byte aligned");
    pro.aux_mix[a] = aux_mix[a];
    pro.aux_out[a] = aux_out[a];
  }
  if (lora_w) {
    if (!naux || !lora_ranks || !lora_out || rows > 2)
      return fail(RWKV7MI_EINVAL, "mm8t_lnmix_multi: the LoRA down projections need the extra mixes, their ranks, "
                                  "an output and at most 2 rows");
    int64_t off = 0;
    for (int a = 0; a < naux; ++a) {
      if (!lora_w[a] || (reinterpret_cast<uintptr_t>(lora_w[a]) & 15) || lora_ranks[a] <= 0 || lora_ranks[a] > 4096)
        return fail(RWKV7MI_EINVAL, "mm8t_lnmix_multi: LoRA down weights must be non-null, 16-byte aligned, "
                                    "with ranks in 1..4096");
      pro.lw[a] = lora_w[a];
      pro.lrank[a] = (int)lora_ranks[a];
      pro.loff[a] = off;
      off += rows * lora_ranks[a];
      pro.lrtot += (int)lora_ranks[a];
    }
    pro.lout = lora_out;
  }
  Mm8tProb p[MM8T_MAXPROB];
  for (int i = 0; i < nprob; ++i) {
    if (!mix[i] || (reinterpret_cast<uintptr_t>(mix[i]) & 15))
      return fail(RWKV7MI_EINVAL, "mm8t_lnmix_multi: mix vectors must be non-null and 16-byte aligned");
    if (epilogue[i] == RWKV7MI_EPI_RESIDUAL)
      return fail(RWKV7MI_EINVAL, "mm8t_lnmix_multi: no residual epilogue on this route");
    p[i] = Mm8tProb{x, mix[i], w_blk[i], mx[i], rx[i], my[i], ry[i], nullptr, nullptr, y[i], epilogue[i]};
  }
  return mm8t_launch(nprob, p, rows, I, O, act_dtype, act_dtype, stream, who, 8, &pro);
}

extern "C" int rwkv7mi_mm4t_matmul(const void* x, const uint8_t* w_t, const void* mx, const void* rx_s,
                                   const void* my, const void* ry_s, const void* bias, const void* residual,
                                   void* y, int64_t rows, int64_t I, int64_t O, int epilogue, int act_dtype,
                                   int meta_dtype, void* stream) {
  Mm8tProb p{x, nullptr, w_t, mx, rx_s, my, ry_s, bias, residual, y, epilogue};
  return mm8t_launch(1, &p, rows, I, O, act_dtype, meta_dtype, stream, "mm4t_matmul", 4);
}

namespace rwkv7mi {
// byte offset of weight (output o, input i) in the blocked 8-bit layout
__host__ __device__ __forceinline__ int64_t mm8t_blk_off(int64_t o, int64_t i, int64_t KB) {
  return ((o >> 4) * KB + (i >> 7)) * 2048 + ((i >> 6) & 1) * 1024 + 16 * (16 * ((i >> 4) & 3) + (o & 15)) + (i & 15);
}

// out[o, i] = (w[o, i] + 0.5) * ry[i] * rx[o] + my[i] + mx[o], fp32 math, one rounding
// (the same expression as mm8_dequant_kernel), from the blocked layout.
template <typename TM, typename TO>
__global__ __launch_bounds__(256) void mm8t_dequant_kernel(const uint8_t* __restrict__ w, const TM* __restrict__ mx,
                                                           const TM* __restrict__ rx, const TM* __restrict__ my,
                                                           const TM* __restrict__ ry, TO* __restrict__ out, int I,
                                                           int O) {
  const int64_t KB = (I + 127) / 128;
  for (int o = blockIdx.y; o < O; o += gridDim.y) {
    const float rxo = to_f32(rx[o]), mxo = to_f32(mx[o]);
    for (int i = (blockIdx.x * 256 + threadIdx.x) * 4; i < I; i += gridDim.x * 256 * 4) {
      // four consecutive inputs (i % 4 == 0) share one 16-byte run
      const uint32_t q = *reinterpret_cast<const uint32_t*>(w + mm8t_blk_off(o, i, KB));
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float wq = (float)((q >> (8 * e)) & 0xffu) + 0.5f;
        out[(int64_t)o * I + i + e] = from_f32<TO>(wq * to_f32(ry[i + e]) * rxo + to_f32(my[i + e]) + mxo);
      }
    }
  }
}

// blocked[tile, 16-byte run] <-> src[o, i] at src + o so + i si (zeros past the edges)
__global__ __launch_bounds__(256) void mm8t_block_kernel(const uint8_t* __restrict__ src, int64_t so, int64_t si,
                                                         int I, int O, uint8_t* __restrict__ blk, int64_t nruns) {
  const int64_t KB = (I + 127) / 128;
  for (int64_t t = blockIdx.x * 256 + threadIdx.x; t < nruns; t += (int64_t)gridDim.x * 256) {
    const int64_t tile = t >> 7, w = t & 127;
    const int64_t o = (tile / KB) * 16 + (w & 15);
    const int64_t i0 = (tile % KB) * 128 + ((w >> 6) & 1) * 64 + ((w >> 4) & 3) * 16;
    uint32_t v[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int e = 0; e < 16; ++e)
      if (o < O && i0 + e < I) v[e >> 2] |= (uint32_t)src[o * so + (i0 + e) * si] << (8 * (e & 3));
    *reinterpret_cast<uint4*>(blk + t * 16) = make_uint4(v[0], v[1], v[2], v[3]);
  }
}

__global__ __launch_bounds__(256) void mm8t_unblock_kernel(const uint8_t* __restrict__ blk, int I, int O,
                                                           uint8_t* __restrict__ dst, int64_t so, int64_t si,
                                                           int64_t nruns) {
  const int64_t KB = (I + 127) / 128;
  for (int64_t t = blockIdx.x * 256 + threadIdx.x; t < nruns; t += (int64_t)gridDim.x * 256) {
    const int64_t tile = t >> 7, w = t & 127;
    const int64_t o = (tile / KB) * 16 + (w & 15);
    const int64_t i0 = (tile % KB) * 128 + ((w >> 6) & 1) * 64 + ((w >> 4) & 3) * 16;
    if (o >= O) continue;
    const uint4 r = *reinterpret_cast<const uint4*>(blk + t * 16);
    const uint32_t v[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int e = 0; e < 16; ++e)
      if (i0 + e < I) dst[o * so + (i0 + e) * si] = (uint8_t)(v[e >> 2] >> (8 * (e & 3)));
  }
}
}  // namespace rwkv7mi

extern "C" size_t rwkv7mi_mm8t_blocked_bytes(int64_t I, int64_t O) {
  if (I <= 0 || O <= 0) return 0;
  return (size_t)((O + 15) / 16) * (size_t)((I + 127) / 128) * 2048u;
}

static int mm8t_relayout(bool to_blocked, const uint8_t* src, uint8_t* dst, int64_t I, int64_t O, int64_t so,
                         int64_t si, void* stream, const char* who) {
  if (I <= 0 || O <= 0 || I > INT32_MAX || O > INT32_MAX) return fail(RWKV7MI_EINVAL, std::string(who) + ": bad shape");
  if (!src || !dst) return fail(RWKV7MI_EINVAL, std::string(who) + ": null pointer");
  const uint8_t* blk = to_blocked ? dst : src;
  if (reinterpret_cast<uintptr_t>(blk) & 15)
    return fail(RWKV7MI_EINVAL, std::string(who) + ": the blocked buffer must be 16-byte aligned");
  const int64_t nruns = (int64_t)(rwkv7mi_mm8t_blocked_bytes(I, O) / 16);
  const unsigned gx = (unsigned)std::min<int64_t>((nruns + 255) / 256, 65536);
  if (to_blocked)
    hipLaunchKernelGGL(mm8t_block_kernel, dim3(gx), dim3(256), 0, as_stream(stream), src, so, si, (int)I, (int)O, dst,
                       nruns);
  else
    hipLaunchKernelGGL(mm8t_unblock_kernel, dim3(gx), dim3(256), 0, as_stream(stream), src, (int)I, (int)O, dst, so,
                       si, nruns);
  return check_launch(who);
}

extern "C" int rwkv7mi_mm8t_block(const uint8_t* src, int64_t stride_o, int64_t stride_i, int64_t I, int64_t O,
                                  uint8_t* w_blk, void* stream) {
  return mm8t_relayout(true, src, w_blk, I, O, stride_o, stride_i, stream, "mm8t_block");
}

extern "C" int rwkv7mi_mm8t_unblock(const uint8_t* w_blk, int64_t I, int64_t O, uint8_t* dst, int64_t stride_o,
                                    int64_t stride_i, void* stream) {
  return mm8t_relayout(false, w_blk, dst, I, O, stride_o, stride_i, stream, "mm8t_unblock");
}

extern "C" int rwkv7mi_mm8t_dequant(const uint8_t* w_blk, const void* mx, const void* rx, const void* my,
                                    const void* ry, void* out, int64_t I, int64_t O, int meta_dtype, int out_dtype,
                                    void* stream) {
  if (I <= 0 || O <= 0 || I % 4 || I > INT32_MAX || O > INT32_MAX) return fail(RWKV7MI_EINVAL, "mm8t_dequant: bad shape");
  if (!w_blk || !mx || !rx || !my || !ry || !out) return fail(RWKV7MI_EINVAL, "mm8t_dequant: null pointer");
  if (reinterpret_cast<uintptr_t>(w_blk) & 15) return fail(RWKV7MI_EINVAL, "mm8t_dequant: w_blk must be 16-byte aligned");
  return dispatch_dtype(meta_dtype, [&](auto tm) {
    using TM = decltype(tm);
    return dispatch_dtype(out_dtype, [&](auto to) {
      using TO = decltype(to);
      const int gx = (int)std::min<int64_t>((I / 4 + 255) / 256, 64);
      hipLaunchKernelGGL((mm8t_dequant_kernel<TM, TO>), dim3(gx, (unsigned)std::min<int64_t>(O, 32768)), dim3(256), 0, as_stream(stream),
                         w_blk, (const TM*)mx, (const TM*)rx, (const TM*)my, (const TM*)ry, (TO*)out, (int)I, (int)O);
      return check_launch("mm8t_dequant_kernel");
    });
  });
}

