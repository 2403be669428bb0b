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
// groups of the blocked layout).  Eight waves (two per SIMD) in a 2 x 4 grid
// each own 128 rows x 64 columns: 8 x 4 MFMA tiles of
// v_mfma_f32_16x16x32_f16 (128 fp32 accumulators per lane; 128 x 128 wave
// tiles would need 256 and spill).  K advances 64 inputs per step (one 1 KB
// half of each 2 KB blocked tile):
//  * every operand of a step goes global -> LDS directly (buffer loads with
//    the lds flag, no registers) into one of three stages; the one barrier
//    per step sits between its two 32-input sub-steps, after which the next
//    step's loads have landed and the previous step's stage takes the loads
//    of the step after next (each step's loads have one step to land);
//  * the MFMAs never wait on a conversion or an LDS read in line: A operands
//    are read two M tiles ahead, the second sub-step's B operands are built
//    between the first sub-step's MFMA groups and the next step's first
//    sub-step operands between the second's;
//  * x rows: a row is 128 bytes whose 16-byte chunk c sits at position
//    c ^ key(row), key(r) = (r % 8) ^ ((r / 8) % 2).  An MFMA A read (lane
//    n + 16 kg: row r0 + n, r0 % 16 == 0, chunk 2 kg + h) then has no LDS
//    bank conflict on gfx950; the plain key r % 8 cost about 4 conflict
//    cycles per read (measured with the SQ_LDS_BANK_CONFLICT counter);
//  * the MM8 bytes: the step's 1 KB half of each of the tile's 16 column
//    groups, as stored (a lane's 16 bytes are the B operands of two
//    consecutive MFMAs), loaded once per workgroup for both row halves;
//  * ry and my of the step's inputs, followed by 64 ones and 64 zeros (rows
//    of 144 bytes, so the four a read touches lie on different banks), so
//    the extra columns' B operand is one LDS read per lane (column 0 reads
//    ry, 1 my, 2 ones, the rest zeros).
// Wave (wm, wn) also computes the extra columns for its M tiles 2wn, 2wn+1
// (their A operands read again from LDS: no per-tile branch in the loop).
// The tile order is XCD-aware: a workgroup's linear id L runs on XCD L % 8,
// so tiles are numbered to give each XCD contiguous groups of 4 row tiles x
// 8 column tiles (their x rows and weight columns stay in that XCD's L2).
#include <string>

#include "mm8t_common.h"

namespace rwkv7mi {

constexpr int MM8P_M = 256, MM8P_N = 256, MM8P_KS = 64;
constexpr int MM8P_XS = MM8P_KS;                        // LDS row (halfs): 128 bytes, 16-byte chunks XOR-swizzled
constexpr int MM8P_ABYTES = MM8P_M * MM8P_XS * 2;       // x rows of one step (32 KB)
constexpr int MM8P_BBYTES = 16 * 1024;                  // MM8 bytes of one step: 16 column groups x 1 KB
constexpr int MM8P_VROW = MM8P_KS + 8;                  // v rows (halfs): 144 bytes, so the four rows the
                                                        // extra-column read touches sit on different banks
constexpr int MM8P_VBYTES = 4 * MM8P_VROW * 2;          // ry, my of one step, then ones, zeros (fp16)
constexpr int MM8P_STAGE = MM8P_ABYTES + MM8P_BBYTES + MM8P_VBYTES;
constexpr int MM8P_NST = 3;                             // pipeline stages (two steps of loads in flight)
constexpr int MM8P_LDS = MM8P_NST * MM8P_STAGE;

struct Mm8pBatch {
  Mm8tProb p[MM8T_MAXPROB];
  int rows, I, O, KB;      // KB = ceil(I / 128) blocked tiles per column group
  int mt, nt;              // row / column tiles
  int gm, gn;              // XCD tile group: gm row tiles x gn column tiles
};

// x row r's 16-byte chunk c sits at position c ^ mm8p_key(r)
__device__ __forceinline__ int mm8p_key(int r) { return (r & 7) ^ ((r >> 3) & 1); }

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

  // ---- global sources (raw buffer loads; out-of-range offsets read zeros)
  const __amdgpu_buffer_rsrc_t xr = mm8t_rsrc(P.x, (uint32_t)((int64_t)M * I * 2));
  const __amdgpu_buffer_rsrc_t ryr = mm8t_rsrc(P.ry, (uint32_t)(I * 2));
  const __amdgpu_buffer_rsrc_t myr = mm8t_rsrc(P.my, (uint32_t)(I * 2));
  const int ngroups = (O + MM8T_COLS - 1) / MM8T_COLS;
  const uint32_t gbytes = (uint32_t)B.KB * 2048u;
  __amdgpu_buffer_rsrc_t wdma[2];  // the two column groups this wave loads for the workgroup
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int g = n0 / MM8T_COLS + 2 * wave + q;
    wdma[q] = mm8t_rsrc(P.w + (int64_t)(g < ngroups ? g : 0) * gbytes, g < ngroups ? gbytes : 0u);
  }
  const int nsteps = (I + MM8P_KS - 1) / MM8P_KS;
  auto xs = [&](int st) { return reinterpret_cast<_Float16*>(smem + st * MM8P_STAGE); };
  auto bs = [&](int st) { return reinterpret_cast<const u32x4*>(smem + st * MM8P_STAGE + MM8P_ABYTES); };
  auto vs = [&](int st) { return reinterpret_cast<_Float16*>(smem + st * MM8P_STAGE + MM8P_ABYTES + MM8P_BBYTES); };
  typedef __attribute__((address_space(3))) void* lds_ptr;

  // loads of step s into stage s % 3 (the LDS writes complete with vmcnt):
  //  * x: wave w, round u writes rows 64 u + 8 w .. +7 (1 KB; lane l lands
  //    at row + l / 8, chunk position l % 8, so it fetches input chunk
  //    (l % 8) ^ key(row + l / 8)); rows past M, inputs past I read zeros;
  //  * B: wave w loads column groups 2w, 2w + 1 (1 KB each);
  //  * ry (lanes 0..7) and my (lanes 8..15): wave 0.
  // Per wave and step: 6 loads, 8 on wave 0.
  auto issue = [&](int s) {
    const int st = s % MM8P_NST;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int r0 = 64 * u + 8 * wave;
      const int r = r0 + (lane >> 3);
      const int k = s * MM8P_KS + 8 * ((lane & 7) ^ mm8p_key(r));
      const bool ok = m0 + r < M && k < I;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_ptr)(xs(st) + r0 * MM8P_XS), 16,
                                               ok ? (int)(((int64_t)(m0 + r) * I + k) * 2) : (int)MM8T_OOB, 0, 0, 0);
    }
    const int boff = s < nsteps ? (s >> 1) * 2048 + (s & 1) * 1024 + 16 * lane : (int)MM8T_OOB;
#pragma unroll
    for (int q = 0; q < 2; ++q)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(wdma[q], (lds_ptr)(bs(st) + 64 * (2 * wave + q)), 16, boff, 0, 0, 0);
    if (wave == 0 && lane < 8) {
      const int k = s * MM8P_KS + 8 * lane;
      const int off = k < I ? k * 2 : (int)MM8T_OOB;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ryr, (lds_ptr)vs(st), 16, off, 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(myr, (lds_ptr)(vs(st) + MM8P_VROW), 16, off, 0, 0, 0);
    }
  };
  // wait until only the newest step's loads may be pending (s_waitcnt
  // vmcnt(6) / vmcnt(8), no expcnt / lgkmcnt wait)
  auto wait_one_step = [&]() {
    if (wave == 0)
      __builtin_amdgcn_s_waitcnt(0x0F78);
    else
      __builtin_amdgcn_s_waitcnt(0x0F76);
  };

  f32x4 acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int q = 0; q < 4; ++q) acc[i][q] = (f32x4){0.f, 0.f, 0.f, 0.f};
  f32x4 ex[2] = {(f32x4){0.f, 0.f, 0.f, 0.f}, (f32x4){0.f, 0.f, 0.f, 0.f}};

  // constant rows of the v part of every stage: 64 ones, 64 zeros
  if (tid < 16 * MM8P_NST) {  // stage tid / 16, 8-half run j = tid % 16 (runs 0..7 ones, 8..15 zeros)
    const int j = tid & 15;
    const _Float16 c = j < 8 ? (_Float16)1.0f : (_Float16)0.0f;
    const f16x8 c8 = (f16x8){c, c, c, c, c, c, c, c};
    *reinterpret_cast<f16x8*>(vs(tid >> 4) + (2 + (j >> 3)) * MM8P_VROW + 8 * (j & 7)) = c8;
  }
  const int xsel = MM8P_VROW * (n < 3 ? n : 3);  // this lane's extra column: ry, my, ones or zeros
  // The lane's raw B bytes of step s (4 column groups, 16 bytes each) and the
  // B operands of one sub-step h built from them (the lane's 8 inputs
  // 16 kg + 8 h .. +7 of the step).
  auto ldb = [&](int s, u32x4 (&braw)[4]) {
#pragma unroll
    for (int q = 0; q < 4; ++q) braw[q] = bs(s % MM8P_NST)[64 * (4 * wn + q) + lane];
  };
  auto ry_of = [&](int s, int h) {
    return *reinterpret_cast<const f16x8*>(vs(s % MM8P_NST) + 16 * kg + 8 * h);
  };

  // prologue: steps 0 and 1 in flight, step 0 landed before the first
  // barrier, its sub-step 0 B operands built
  issue(0);
  issue(1);
  wait_one_step();
  __syncthreads();
  u32x4 braw[4];
  f16x8 bv0[4], bv1[4];
  ldb(0, braw);
  {
    const f16x8 ry0 = ry_of(0, 0);
#pragma unroll
    for (int q = 0; q < 4; ++q) bv0[q] = mm8p_b_operand(braw[q][0], braw[q][1], ry0);
  }

  // Step s: sub-step 0's MFMAs (sub-step 1's B operands built between them),
  // then the barrier after which step s + 1 has landed and step s - 1's stage
  // is free, the loads of step s + 2 into it, and sub-step 1's MFMAs with step
  // s + 1's raw B reads and sub-step 0 conversions between them.  Step s + 1's
  // loads are in flight from the middle of step s - 1 to the middle of step s.
  for (int s = 0; s < nsteps; ++s) {
    const int st = s % MM8P_NST;
    const _Float16* xb = xs(st);
    const _Float16* vb = vs(st);
    // A operands of sub-step h: reads 0..7 are the wave's eight M tiles, 8 and
    // 9 its two extra-column tiles (M tiles 2wn, 2wn + 1, read again)
    auto lda = [&](int h, int i) {
      const int ka = 8 * ((2 * kg + h) ^ mm8p_key(n));  // swizzled chunk of A row (16 j + n): key(n)
      const int mt = i < 8 ? i : 2 * wn + (i - 8);
      return *reinterpret_cast<const f16x8*>(xb + (128 * wm + 16 * mt + n) * MM8P_XS + ka);
    };
    // the sub-step's ten A reads run two ahead of the MFMAs that use them
    // (the read of tile i + 2 is issued before tile i's MFMAs, so its LDS
    // latency hides behind two tiles' MFMAs); `between(i)` runs after tile
    // i's MFMAs
    auto mfmas = [&](int h, const f16x8 (&bv)[4], auto&& between) {
      const f16x8 bx = *reinterpret_cast<const f16x8*>(vb + xsel + 16 * kg + 8 * h);
      f16x8 a = lda(h, 0), an = lda(h, 1);
#pragma unroll
      for (int i = 0; i < 10; ++i) {
        f16x8 ann = an;
        if (i < 8) ann = lda(h, i + 2);
        __builtin_amdgcn_sched_barrier(0);
        if (i < 8) {
#pragma unroll
          for (int q = 0; q < 4; ++q) acc[i][q] = mfma16x16x32(a, bv[q], acc[i][q]);
        } else {
          ex[i - 8] = mfma16x16x32(a, bx, ex[i - 8]);
        }
        between(i);
        __builtin_amdgcn_sched_barrier(0);
        a = an;
        an = ann;
      }
    };
    const f16x8 ry1 = ry_of(s, 1);
    mfmas(0, bv0, [&](int i) {
      if (i < 4) {
        bv1[i] = mm8p_b_operand(braw[i][2], braw[i][3], ry1);
        // keep the conversion here, between the MFMAs (the compiler would
        // otherwise sink it past the barrier to its first use)
        asm volatile("" : "+v"(bv1[i]));
      }
    });
    // vmcnt(0): this wave's loads of step s + 1 have landed (step s + 2 is not
    // issued yet); the barrier makes every wave's loads visible and puts every
    // wave past step s - 1's reads
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();
    issue(s + 2);
    f16x8 ry0;
    mfmas(1, bv1, [&](int i) {
      if (i == 0) {
        ldb(s + 1, braw);
        ry0 = ry_of(s + 1, 0);
      } else if (i >= 2 && i < 6) {
        bv0[i - 2] = mm8p_b_operand(braw[i - 2][0], braw[i - 2][1], ry0);
      }
    });
  }

  // ---- the extra columns -> LDS row sums (reusing stage 0)
  float* rs = reinterpret_cast<float*>(smem);  // [256][3]: sum x ry, sum x my, sum x
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the trailing loads into LDS have landed
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
