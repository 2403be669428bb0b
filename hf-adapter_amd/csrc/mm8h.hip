// Prefill MM8 (more than 256 rows) as the reference computes it: the fp16
// dequantised weight, then one fp16 GEMM.  rwkv7_hf/native_quant_mm8.py:468-507
// takes this route for rows > fused_max_rows (mm8_matmul: dequantize_mm8 at
// native_quant_mm8.py:100-108, then x @ W_hat), as do the prefill projections
// of rwkv7_hf/native_jit_prefill.py:542-631, 955-1013.
//
// 1. mm8h_dequant_kernel writes W_hat[k, o] = ((w + 0.5) ry[k]) rx[o]
//    + my[k] + mx[o] in the activation type, fp16 or bf16 (fp32 arithmetic,
//    one rounding: the bytes rwkv7mi_mm8_dequant writes) into a workspace,
//    in MFMA operand order:
//    [column group g of 16][64-input step sb][sub-step h][lane][8 values],
//    lane n + 16 kg holding inputs 64 sb + 16 kg + 8 h .. +7 of column
//    col(g, n) = 32 (g / 2) + 8 (n / 4) + 4 (g % 2) + n % 4: each pair of
//    groups covers 32 columns, permuted so that the GEMM's output lanes hold
//    8 consecutive columns.  The input order is the lane order of the blocked
//    MM8 layout the decode kernels read (a lane's 16 bytes there are inputs
//    16 kg .. +15 of the step), so each thread turns one such lane's 16 bytes
//    into its two 16-byte records.  O is padded to whole 32-column pairs.
// 2. mm8h_gemm_kernel: y = x W_hat (+ bias) (relu^2 | + residual).  A
//    256-lane workgroup (four waves, one per SIMD) computes 256 rows x 256
//    columns; wave w owns all 256 rows x columns 64 w .. 64 w + 63 (16 x 4
//    tiles of v_mfma_f32_16x16x32_f16, 256 fp32 accumulators per lane in the
//    accumulation registers).  The MFMAs take W_hat as the A operand and x as
//    B, so a lane holds one row (16 i + n) and, across a pair of groups, the
//    8 consecutive columns 32 p + 8 kg .. +7: the epilogue is one 16-byte
//    store (and residual load) per M tile and pair.  K advances 64 inputs
//    per step:
//    * W_hat: each wave loads its own four column groups global -> registers
//      (8 x 16 bytes per lane and step), one step ahead, in two register sets
//      (the loop is unrolled by two; no LDS, no wave reads another's bytes);
//    * x: global -> LDS directly (buffer loads with the lds flag) into three
//      stages, two steps ahead; a row is 128 bytes whose 16-byte chunk c sits
//      at position c ^ key(row), key(r) = (r % 8) ^ ((r / 8) % 2), which
//      leaves the A reads (lane n + 16 kg: row 16 j + n, chunk 2 kg + h) free
//      of LDS bank conflicts on gfx950 (measured with SQ_LDS_BANK_CONFLICT;
//      the plain key r % 8 cost about 4 conflict cycles per read);
//    * A operands are read a whole sub-step ahead (two register sets of 16),
//      so each sub-step's MFMAs cover the next one's LDS reads; the one
//      barrier per step sits between its sub-steps, after the wait for the
//      next step's x rows, whose first A reads follow it;
//    * the global loads are spread over the MFMAs, one after every other M
//      tile (W_hat in sub-step 0, x after the barrier in sub-step 1): issued
//      in bursts they stall the wave while its MFMAs drain (measured: 13-17%
//      of the kernel time per stream).
//    The tile order is XCD-aware: a workgroup's linear id L runs on XCD L % 8,
//    so tiles are numbered to give each XCD contiguous groups of 4 row tiles x
//    8 column tiles (their x rows and weight columns stay in that XCD's L2).
#include <string>

#include "mm8t_common.h"

namespace rwkv7mi {

constexpr int MH_M = 256, MH_N = 256, MH_KS = 64;
constexpr int MH_THREADS = 256;                 // four waves, one per SIMD
constexpr int MH_XS = MH_KS;                    // LDS row (halfs): 128 bytes, 16-byte chunks swizzled
constexpr int MH_STAGE = MH_M * MH_XS * 2;      // x rows of one step (32 KB)
constexpr int MH_NST = 3;                       // x stages (two steps of loads in flight)
constexpr int MH_LDS = MH_NST * MH_STAGE;
constexpr int64_t MH_REC = 2048;                // W_hat bytes per (column group, step): 2 sub-steps x 64 lanes x 16

struct MhProb {
  const void* x;
  const void* wt;    // W_hat in MFMA order (the workspace)
  const void* bias;
  const void* residual;
  void* y;
  int epilogue;
  int vec;  // O % 8 == 0 and y (and the residual) 16-byte aligned: 16-byte output rows
};
struct MhBatch {
  MhProb p[MM8T_MAXPROB];
  int rows, I, O, SB;  // SB = ceil(I / 64) steps
  int mt, nt;          // row / column tiles
  int gm, gn;          // XCD tile group: gm row tiles x gn column tiles
};

__device__ __forceinline__ int mh_key(int r) { return (r & 7) ^ ((r >> 3) & 1); }

// element and 8-vector types of fp16 (__half) and bf16 (__hip_bfloat16) data
template <typename T> struct MhTypes {
  using E = _Float16;
  typedef _Float16 V __attribute__((ext_vector_type(8)));
};
template <> struct MhTypes<__hip_bfloat16> {
  using E = __bf16;
  typedef __bf16 V __attribute__((ext_vector_type(8)));
};

struct MhDeqProb {
  const uint8_t* w;  // blocked MM8 bytes: [ceil(O/16)][ceil(I/128)][2048]
  const void *mx, *rx, *my, *ry;
  void* out;         // [2 ceil(O/32)][SB][2][64][8] of the activation type
};
struct MhDeqBatch {
  MhDeqProb p[MM8T_MAXPROB];
  int I, O, SB, KB;
};

// one thread per (column group, step, lane): the lane's 16 MM8 bytes ->
// its two 8-half records
// The same operand order for an fp16 nn.Linear weight W [O, I] (W_hat[k, o]
// = W[o, k]): one thread per (column group, step, lane) copies the 16
// inputs 16 kg .. +15 of its column into its two records.
struct MhRelBatch {
  const void* w[MM8T_MAXPROB];
  void* out[MM8T_MAXPROB];
  int I, O, SB;
};
template <typename TA>
__global__ __launch_bounds__(256) void mm8h_relayout_kernel(const MhRelBatch R) {
  using E = typename MhTypes<TA>::E;
  using V = typename MhTypes<TA>::V;
  const int p = blockIdx.y;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int ngroups = 2 * ((R.O + 31) / 32);
  if (t >= (int64_t)ngroups * R.SB * 64) return;
  const int lane = (int)(t & 63);
  const int64_t gs = t >> 6;
  const int sb = (int)(gs % R.SB), g = (int)(gs / R.SB);
  const int n = lane & 15, kg = lane >> 4;
  const int o = 32 * (g >> 1) + 8 * (n >> 2) + 4 * (g & 1) + (n & 3);
  const int k0 = 64 * sb + 16 * kg;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    V v;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int k = k0 + 8 * h + j;
      v[j] = o < R.O && k < R.I ? static_cast<const E*>(R.w[p])[(int64_t)o * R.I + k] : (E)0.f;
    }
    *reinterpret_cast<V*>(static_cast<char*>(R.out[p]) + gs * MH_REC + h * 1024 + 16 * lane) = v;
  }
}

template <typename TA>
__global__ __launch_bounds__(256) void mm8h_dequant_kernel(const MhDeqBatch D) {
  using E = typename MhTypes<TA>::E;
  using V = typename MhTypes<TA>::V;
  const MhDeqProb& P = D.p[blockIdx.y];
  const TA *mx = static_cast<const TA*>(P.mx), *rx = static_cast<const TA*>(P.rx);
  const TA *my = static_cast<const TA*>(P.my), *ry = static_cast<const TA*>(P.ry);
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int ngroups = 2 * ((D.O + 31) / 32);
  if (t >= (int64_t)ngroups * D.SB * 64) return;
  const int lane = (int)(t & 63);
  const int64_t gs = t >> 6;
  const int sb = (int)(gs % D.SB), g = (int)(gs / D.SB);
  const int n = lane & 15, kg = lane >> 4;
  const int o = 32 * (g >> 1) + 8 * (n >> 2) + 4 * (g & 1) + (n & 3);
  const int k0 = 64 * sb + 16 * kg;
  const bool ocol = o < D.O;
  // column o's bytes: blocked group o / 16, lane (o % 16) + 16 kg
  const u32x4 raw = ocol ? *reinterpret_cast<const u32x4*>(P.w + ((int64_t)(o >> 4) * D.KB + (sb >> 1)) * 2048 +
                                                            (sb & 1) * 1024 + 16 * ((o & 15) + 16 * kg))
                         : (u32x4){0u, 0u, 0u, 0u};
  const float rxo = ocol ? to_f32(rx[o]) : 0.f, mxo = ocol ? to_f32(mx[o]) : 0.f;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    V v;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int k = k0 + 8 * h + j;
      const uint32_t byte = (raw[2 * h + (j >> 2)] >> (8 * (j & 3))) & 0xffu;
      float x = 0.f;
      if (ocol && k < D.I) {
        const float wq = (float)byte + 0.5f;
        x = wq * to_f32(ry[k]) * rxo + to_f32(my[k]) + mxo;
      }
      v[j] = (E)x;
    }
    *reinterpret_cast<V*>(static_cast<char*>(P.out) + gs * MH_REC + h * 1024 + 16 * lane) = v;
  }
}

// FULLK: I is a multiple of 64 (no step ends inside a 16-byte chunk's range)
template <bool FULLK, typename TA>
__global__ __launch_bounds__(MH_THREADS, 1) void mm8h_gemm_kernel(const MhBatch B) {
  using E = typename MhTypes<TA>::E;
  using V = typename MhTypes<TA>::V;
  const MhProb& P = B.p[blockIdx.y];
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
  const int m0 = tm * MH_M, n0 = tn * MH_N;

  extern __shared__ __align__(16) char smem[];
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int n = lane & 15, kg = lane >> 4;
  const int SB = B.SB;
  const int nsteps = SB + (SB & 1);  // whole step pairs; a padding step reads zeros

  // ---- global sources (raw buffer loads; out-of-range offsets read zeros)
  const __amdgpu_buffer_rsrc_t xr = mm8t_rsrc(P.x, (uint32_t)((int64_t)M * I * 2));
  const int ngroups = 2 * ((O + 31) / 32);
  const int g0 = n0 / 16 + 4 * wave;  // this wave's first column group
  const int gcount = g0 < ngroups ? (ngroups - g0 < 4 ? ngroups - g0 : 4) : 0;
  const __amdgpu_buffer_rsrc_t wr =
      mm8t_rsrc(reinterpret_cast<const char*>(P.wt) + (int64_t)(g0 < ngroups ? g0 : 0) * SB * MH_REC,
                (uint32_t)((int64_t)gcount * SB * MH_REC));
  auto xs = [&](int st) { return reinterpret_cast<E*>(smem + st * MH_STAGE); };
  typedef __attribute__((address_space(3))) void* lds_ptr;

  // x of step s into stage s % 3: wave w, round u writes rows 32 u + 8 w ..
  // +7 (1 KB; lane l lands at row + l / 8, chunk position l % 8, so it
  // fetches input chunk (l % 8) ^ key(row + l / 8)); rows past M, inputs past
  // I read zeros.  8 loads per wave and step.  The lane's byte offsets are
  // fixed per tile (xo); a step adds s * 128 bytes as the scalar offset, and
  // a padding step past the last uses an out-of-range one.  With I not a
  // multiple of 64 the last step's lanes whose chunk lies past I use xl
  // (out of range) instead.
  int xo[8], xl[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const int r = 32 * u + 8 * wave + (lane >> 3);
    const int c = (lane & 7) ^ mh_key(r);
    xo[u] = m0 + r < M ? (int)((int64_t)(m0 + r) * I * 2) + 16 * c : (int)MM8T_OOB;
    xl[u] = FULLK || 64 * (SB - 1) + 8 * c < I ? xo[u] : (int)MM8T_OOB;
  }
  auto issue_x = [&](int s, int u) {
    const int st = s % MH_NST;
    const int r0 = 32 * u + 8 * wave;
    const int so = s < SB ? 128 * s : (int)MM8T_OOB;
    const int vo = FULLK ? xo[u] : (s == SB - 1 ? xl[u] : xo[u]);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_ptr)(xs(st) + r0 * MH_XS), 16, vo, so, 0, 0);
  };
  // W_hat of step s for the wave's group j = 0..3, sub-step h (load 2 j + h
  // of 8): lane offset 16 lane, the rest a scalar offset
  auto issue_w = [&](int s, int j, int h, V (&bw)[4][2]) {
    const int so = s < SB ? (j * SB + s) * (int)MH_REC + h * 1024 : (int)MM8T_OOB;
    bw[j][h] = __builtin_bit_cast(V, __builtin_amdgcn_raw_buffer_load_b128(wr, 16 * lane, so, 0));
  };

  f32x4 acc[16][4];
#pragma unroll
  for (int i = 0; i < 16; ++i)
#pragma unroll
    for (int q = 0; q < 4; ++q) acc[i][q] = (f32x4){0.f, 0.f, 0.f, 0.f};
  // A row offsets (halfs) in sub-steps 0 and 1: row 16 i + n (row % 16 == n),
  // chunk (2 kg + h) ^ key(n)
  const int key = mh_key(n);
  const int abase0 = n * MH_XS + 8 * ((2 * kg) ^ key);
  const int abase1 = n * MH_XS + 8 * ((2 * kg + 1) ^ key);
  auto lda = [&](int st, int h, int i) {
    return *reinterpret_cast<const V*>(xs(st) + (h ? abase1 : abase0) + 16 * i * MH_XS);
  };
  // One sub-step: MFMAs of the 16 M tiles over A operands `a` (read during
  // the previous sub-step) while the next sub-step's 16 A operands are read
  // into `an`, one read per M tile, so every LDS read has a whole sub-step
  // of MFMAs to land.  `load(u)` issues the u-th of the sub-step's eight
  // global loads, one after every other M tile's MFMAs (a burst of loads
  // would stall the wave's issue while its MFMAs drain).
  V a0[16], a1[16];  // A operands of sub-steps 0 and 1
  auto substep = [&](const V (&a)[16], const V (&bw)[4][2], int h, V (&an)[16], int st_n, int h_n,
                     auto&& load) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      an[i] = lda(st_n, h_n, i);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int q = 0; q < 4; ++q) acc[i][q] = mfma16x16x32(bw[q][h], a[i], acc[i][q]);
      if (i % 2 == 0) load(i / 2);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // Step s (its sub-step 0 A operands in a0, read during step s - 1): W_hat
  // of step s landed (issued one step earlier; only step s + 1's x loads,
  // issued after it, may be pending), W_hat of step s + 1 into the other
  // register set, sub-step 0 with sub-step 1's A reads; then the wait for
  // step s + 1's x rows (only the W_hat loads just issued may be pending) and
  // the barrier that makes every wave's rows visible and puts every wave past
  // step s - 1's reads, x of step s + 2 into step s - 1's stage, and sub-step
  // 1 with step s + 1's sub-step 0 A reads.
  auto step = [&](int s, const V (&bw)[4][2], V (&bwn)[4][2]) {
    __builtin_amdgcn_s_waitcnt(0x0F78);  // vmcnt(8)
    __builtin_amdgcn_sched_barrier(0);
    substep(a0, bw, 0, a1, s % MH_NST, 1, [&](int u) { issue_w(s + 1, u >> 1, u & 1, bwn); });
    __builtin_amdgcn_s_waitcnt(0x0F78);  // vmcnt(8)
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    substep(a1, bw, 1, a0, (s + 1) % MH_NST, 0, [&](int u) { issue_x(s + 2, u); });
  };

  // prologue: W_hat of step 0, x of steps 0 and 1 in flight; step 0's rows
  // landed (only step 1's x loads may be pending) and visible, its sub-step
  // 0 A operands read
  V bw0[4][2], bw1[4][2];
#pragma unroll
  for (int u = 0; u < 8; ++u) issue_w(0, u >> 1, u & 1, bw0);
#pragma unroll
  for (int u = 0; u < 8; ++u) issue_x(0, u);
#pragma unroll
  for (int u = 0; u < 8; ++u) issue_x(1, u);
  __builtin_amdgcn_s_waitcnt(0x0F78);  // vmcnt(8)
  __builtin_amdgcn_s_barrier();
#pragma unroll
  for (int i = 0; i < 16; ++i) a0[i] = lda(0, 0, i);
  for (int s = 0; s < nsteps; s += 2) {
    step(s, bw0, bw1);
    step(s + 1, bw1, bw0);
    // keep the tile sums in the accumulation registers across the loop
#pragma unroll
    for (int i = 0; i < 16; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) asm volatile("" : "+a"(acc[i][q]));
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the trailing loads have landed before the waves exit

  // ---- epilogue: lane holds row 16 i + n and, in groups 2 p and 2 p + 1,
  // columns c0 = 32 p + 8 kg .. +3 and c0 + 4 .. +7 of the wave's 64
  const TA* bp = reinterpret_cast<const TA*>(P.bias);
  const bool vec = P.vec;
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int c0 = n0 + 64 * wave + 32 * p + 8 * kg;
    if (c0 >= O) continue;
    float bo[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) bo[e] = bp && c0 + e < O ? to_f32(bp[c0 + e]) : 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int64_t row = m0 + 16 * i + n;
      if (row >= M) continue;
      float v[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[e] = acc[i][2 * p][e] + bo[e];
        v[4 + e] = acc[i][2 * p + 1][e] + bo[4 + e];
      }
      const int64_t oi = row * O + c0;
      if (vec && c0 + 8 <= O) {
        if (P.epilogue == RWKV7MI_EPI_RESIDUAL) {
          const V r = *reinterpret_cast<const V*>(reinterpret_cast<const TA*>(P.residual) + oi);
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] += (float)r[e];
        }
        V o8;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float w = v[e];
          if (P.epilogue == RWKV7MI_EPI_RELU2) {
            w = fmaxf(w, 0.f);
            w = w * w;
          }
          o8[e] = (E)w;
        }
        *reinterpret_cast<V*>(reinterpret_cast<TA*>(P.y) + oi) = o8;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          if (c0 + e >= O) continue;
          float w = v[e];
          if (P.epilogue == RWKV7MI_EPI_RELU2) {
            w = fmaxf(w, 0.f);
            w = w * w;
          } else if (P.epilogue == RWKV7MI_EPI_RESIDUAL) {
            w += ld(reinterpret_cast<const TA*>(P.residual), oi + e);
          }
          reinterpret_cast<TA*>(P.y)[oi + e] = from_f32<TA>(w);
        }
      }
    }
  }
}

}  // namespace rwkv7mi

using namespace rwkv7mi;

extern "C" int64_t rwkv7mi_mm8t_gemm_prefill_ws_bytes(int nprob, int64_t I, int64_t O) {
  if (nprob < 1 || I <= 0 || O <= 0) return 0;
  return (int64_t)nprob * (2 * ((O + 31) / 32)) * ((I + 63) / 64) * MH_REC;
}

namespace rwkv7mi {
// the GEMM over prepared W_hat records (b.p[i].wt), with the tile grid set here
template <typename TA>
static int mh_gemm_launch(MhBatch& b, int nprob, int64_t rows, int64_t I, int64_t O, void* stream,
                          const std::string& w) {
  b.rows = (int)rows;
  b.I = (int)I;
  b.O = (int)O;
  b.SB = (int)((I + 63) / 64);
  b.mt = (int)((rows + MH_M - 1) / MH_M);
  b.nt = (int)((O + MH_N - 1) / MH_N);
  b.gm = std::min(b.mt, 4);
  b.gn = std::min(b.nt, 8);
  const int64_t T = (int64_t)((b.mt + b.gm - 1) / b.gm) * b.gm * ((b.nt + b.gn - 1) / b.gn) * b.gn;
  if (T > (int64_t)INT32_MAX / 2) return fail(RWKV7MI_EINVAL, w + ": too many tiles");
  const int64_t per = (T + 7) / 8;
  auto launch = [&](auto kern, std::atomic<uint64_t>& raised) {
    if (int rc = raise_dynamic_lds(reinterpret_cast<const void*>(kern), MH_LDS, raised, "mm8h_gemm_kernel"))
      return rc;
    hipLaunchKernelGGL(kern, dim3((unsigned)(per * 8), (unsigned)nprob), dim3(MH_THREADS), MH_LDS,
                       as_stream(stream), b);
    return check_launch("mm8h_gemm_kernel");
  };
  static std::atomic<uint64_t> raised_full{0}, raised_part{0};
  return I % 64 == 0 ? launch(&mm8h_gemm_kernel<true, TA>, raised_full)
                      : launch(&mm8h_gemm_kernel<false, TA>, raised_part);
}

// shape, workspace and per-problem checks shared by the two entries
static int mh_check(const std::string& w, int nprob, int64_t rows, int64_t I, int64_t O, void* ws, int64_t ws_bytes) {
  if (nprob < 1 || nprob > MM8T_MAXPROB) return fail(RWKV7MI_EINVAL, w + ": 1..4 problems per launch");
  if (rows < 0 || I <= 0 || O <= 0) return fail(RWKV7MI_EINVAL, w + ": bad shape");
  if (I % 16) return fail(RWKV7MI_EINVAL, w + ": in_features must be a multiple of 16");
  // x's descriptor spans rows * I * 2 bytes and out-of-range offsets start at 2^31;
  // one wave's W_hat descriptor spans 4 groups x SB records
  if (rows * I * 2 >= (int64_t)MM8T_OOB || 4 * ((I + 63) / 64) * MH_REC >= (int64_t)MM8T_OOB || O > INT32_MAX ||
      rows * O > ((int64_t)1 << 40))
    return fail(RWKV7MI_EINVAL, w + ": too large (split the rows)");
  if (rows == 0) return RWKV7MI_OK;
  const int64_t per_prob = (2 * ((O + 31) / 32)) * ((I + 63) / 64) * MH_REC;
  if (!ws || ws_bytes < per_prob * nprob)
    return fail(RWKV7MI_EINVAL, w + ": workspace too small (rwkv7mi_mm8t_gemm_prefill_ws_bytes)");
  if (reinterpret_cast<uintptr_t>(ws) & 15) return fail(RWKV7MI_EINVAL, w + ": workspace must be 16-byte aligned");
  return RWKV7MI_OK;
}

static int mh_prob(const std::string& w, MhProb& q, const void* x, const void* out, const void* bias,
                   const void* res, void* y, int epi, int64_t O) {
  if (!x || !y) return fail(RWKV7MI_EINVAL, w + ": null pointer");
  if (reinterpret_cast<uintptr_t>(x) & 15) return fail(RWKV7MI_EINVAL, w + ": x must be 16-byte aligned");
  if (epi < 0 || epi > 2) return fail(RWKV7MI_EINVAL, w + ": bad epilogue");
  if (epi == RWKV7MI_EPI_RESIDUAL && !res) return fail(RWKV7MI_EINVAL, w + ": residual missing");
  const int vec = O % 8 == 0 && !(reinterpret_cast<uintptr_t>(y) & 15) &&
                  !(epi == RWKV7MI_EPI_RESIDUAL && (reinterpret_cast<uintptr_t>(res) & 15));
  q = MhProb{x, out, bias, res, y, epi, vec};
  return RWKV7MI_OK;
}
}  // namespace rwkv7mi

extern "C" int rwkv7mi_mm8t_gemm_prefill_ws(int nprob, const void* const* x, const uint8_t* const* w_blk,
                                            const void* const* mx, const void* const* rx, const void* const* my,
                                            const void* const* ry, const void* const* bias,
                                            const void* const* residual, void* const* y, const int* epilogue,
                                            int64_t rows, int64_t I, int64_t O, int act_dtype, int meta_dtype,
                                            void* ws, int64_t ws_bytes, void* stream) {
  const std::string w("mm8t_gemm_prefill_ws");
  if (!x || !w_blk || !mx || !rx || !my || !ry || !y || !epilogue) return fail(RWKV7MI_EINVAL, w + ": null array");
  if (!((act_dtype == RWKV7MI_F16 || act_dtype == RWKV7MI_BF16) && meta_dtype == act_dtype))
    return fail(RWKV7MI_EINVAL, w + ": fp16 or bf16 activations with metadata of the same type");
  if (int rc = mh_check(w, nprob, rows, I, O, ws, ws_bytes)) return rc;
  if (rows == 0) return RWKV7MI_OK;
  const int64_t per_prob = rwkv7mi_mm8t_gemm_prefill_ws_bytes(1, I, O);
  MhBatch b{};
  MhDeqBatch d{};
  for (int i = 0; i < nprob; ++i) {
    if (!w_blk[i] || !mx[i] || !rx[i] || !my[i] || !ry[i]) return fail(RWKV7MI_EINVAL, w + ": null pointer");
    if (reinterpret_cast<uintptr_t>(w_blk[i]) & 15) return fail(RWKV7MI_EINVAL, w + ": the weights must be 16-byte aligned");
    void* out = static_cast<char*>(ws) + per_prob * i;
    if (int rc = mh_prob(w, b.p[i], x[i], out, bias ? bias[i] : nullptr, residual ? residual[i] : nullptr, y[i],
                         epilogue[i], O))
      return rc;
    d.p[i] = MhDeqProb{w_blk[i], mx[i], rx[i], my[i], ry[i], out};
  }
  d.I = (int)I;
  d.O = (int)O;
  d.SB = (int)((I + 63) / 64);
  d.KB = (int)((I + 127) / 128);
  const int64_t recs = (2 * ((O + 31) / 32)) * (int64_t)d.SB * 64;
  const dim3 dgrid((unsigned)((recs + 255) / 256), (unsigned)nprob);
  if (act_dtype == RWKV7MI_BF16) {
    hipLaunchKernelGGL(mm8h_dequant_kernel<__hip_bfloat16>, dgrid, dim3(256), 0, as_stream(stream), d);
    if (int rc = check_launch("mm8h_dequant_kernel")) return rc;
    return mh_gemm_launch<__hip_bfloat16>(b, nprob, rows, I, O, stream, w);
  }
  hipLaunchKernelGGL(mm8h_dequant_kernel<__half>, dgrid, dim3(256), 0, as_stream(stream), d);
  if (int rc = check_launch("mm8h_dequant_kernel")) return rc;
  return mh_gemm_launch<__half>(b, nprob, rows, I, O, stream, w);
}

extern "C" int rwkv7mi_dense_gemm_prefill_ws(int nprob, const void* const* x, const void* const* W,
                                             const void* const* bias, const void* const* residual, void* const* y,
                                             const int* epilogue, int64_t rows, int64_t I, int64_t O, int act_dtype,
                                             void* ws, int64_t ws_bytes, void* stream) {
  const std::string w("dense_gemm_prefill_ws");
  if (!x || !W || !y || !epilogue) return fail(RWKV7MI_EINVAL, w + ": null array");
  if (act_dtype != RWKV7MI_F16 && act_dtype != RWKV7MI_BF16)
    return fail(RWKV7MI_EINVAL, w + ": fp16 or bf16 activations and weights");
  if (int rc = mh_check(w, nprob, rows, I, O, ws, ws_bytes)) return rc;
  if (rows == 0) return RWKV7MI_OK;
  const int64_t per_prob = rwkv7mi_mm8t_gemm_prefill_ws_bytes(1, I, O);
  MhBatch b{};
  MhRelBatch r{};
  for (int i = 0; i < nprob; ++i) {
    if (!W[i]) return fail(RWKV7MI_EINVAL, w + ": null pointer");
    void* out = static_cast<char*>(ws) + per_prob * i;
    if (int rc = mh_prob(w, b.p[i], x[i], out, bias ? bias[i] : nullptr, residual ? residual[i] : nullptr, y[i],
                         epilogue[i], O))
      return rc;
    r.w[i] = W[i];
    r.out[i] = out;
  }
  r.I = (int)I;
  r.O = (int)O;
  r.SB = (int)((I + 63) / 64);
  const int64_t recs = (2 * ((O + 31) / 32)) * (int64_t)r.SB * 64;
  const dim3 rgrid((unsigned)((recs + 255) / 256), (unsigned)nprob);
  if (act_dtype == RWKV7MI_BF16) {
    hipLaunchKernelGGL(mm8h_relayout_kernel<__hip_bfloat16>, rgrid, dim3(256), 0, as_stream(stream), r);
    if (int rc = check_launch("mm8h_relayout_kernel")) return rc;
    return mh_gemm_launch<__hip_bfloat16>(b, nprob, rows, I, O, stream, w);
  }
  hipLaunchKernelGGL(mm8h_relayout_kernel<__half>, rgrid, dim3(256), 0, as_stream(stream), r);
  if (int rc = check_launch("mm8h_relayout_kernel")) return rc;
  return mh_gemm_launch<__half>(b, nprob, rows, I, O, stream, w);
}
