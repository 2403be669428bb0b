// Many-row W/A/G/V LoRA for fp16 prefills (rwkv7_hf/fused_lora.py:706
// fused_wavg_lora over B*T rows; torch form :795-803):
//   mid = round(act_down(x Wd^T)),  y = round(act_up(mid Wu^T + b)).
//
// One 1024-lane workgroup owns 256 rows of one problem (wave w: rows
// 16 w .. 16 w + 15) from start to end, so there are no partial sums and no
// workspace.  Both weights are shared by the sixteen waves through LDS: each
// wave loads its share of a stage into registers (three stages ahead), writes
// it to one of two LDS buffers a stage ahead, and one LDS-only barrier per
// stage orders the writes and reads (no wait on global memory at a barrier,
// so loads and stores stay in flight across it).
//  1. down: C^T = Wd x^T on v_mfma_f32_16x16x32_f16, 64 inputs per stage.  The
//     Wd rows (ranks) are the A operand, x rows the B operand (read straight
//     from global, 16 bytes per lane, three stages ahead).  Rank tile t's row
//     i is rank 32 (t / 2) + 8 (i / 4) + 4 (t % 2) + i % 4, so after the loop
//     lane (n, kg) holds ranks 32 s + 8 kg .. + 7 of row n in tiles 2s, 2s+1:
//  2. exactly the B operand of the up projection's k-step s: the mid is
//     activated, rounded and packed in registers (never stored);
//  3. up: C^T = Wu mid^T per group of 64 output columns.  Output tile j's row
//     i is column 32 (j / 2) + 8 (i / 4) + 4 (j % 2) + i % 4 of the group, so
//     lane (n, kg) ends with columns 8 kg .. + 7 (tiles 0, 1) and
//     32 + 8 kg .. + 7 (tiles 2, 3) of row n: two 16-byte stores, each of
//     which writes 64 contiguous bytes of a row from four lanes.  A group's
//     outputs are stored at the start of the next group from one of two
//     register sets, so a store's data registers are rewritten a group later
//     (rewriting them sooner waits for the store).
// LDS rows are 128 or 256 bytes; 16-byte chunk c of row q sits at position
// c ^ key(q), key(q) = (q ^ ((q >> 1) & 4)) & 7: the eight rows an MFMA
// operand read touches per phase, q0 + {0..3, 8..11} for both weights, land
// on eight different chunk positions.
// Ranks are multiples of 32 up to 128; D and A multiples of 256.  Sigmoids use
// the hardware exp2 and reciprocal (lora_act_fast): two per output element
// of the A and V problems would otherwise dominate the up loop's issue.
#include <algorithm>

#include "lora_common.h"

namespace rwkv7mi {

constexpr int LSQ_NW = 16;      // waves per workgroup (one 16-row tile each)
constexpr int LSQ_ROWS = 16 * LSQ_NW;  // rows per workgroup
constexpr int LSQ_KS = 64;      // inputs per down stage
constexpr int LSQ_STAGE = 16384;  // bytes per LDS buffer (128 ranks x 128 B, or 64 columns x 256 B)
constexpr int LSQ_MAXA = 16384;   // up outputs: the whole bias row sits in LDS after the two buffers
constexpr int LSQ_PF = 4;       // register sets per streamed operand (three stages in flight)
constexpr int LSQ_RA = 2;       // LDS operand reads in flight ahead of the MFMAs

__device__ __forceinline__ int lsq_key(int q) { return (q ^ ((q >> 1) & 4)) & 7; }

// LDS-only workgroup barrier: this wave's LDS writes are complete, then the
// barrier; the compiler keeps memory accesses on their side of it.
__device__ __forceinline__ void lsq_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <int RT>
__device__ __forceinline__ void lsq_body(const LoraProb& P, int rows, int D, int A, char* smem) {
  constexpr int KU = RT / 2;                 // up k-steps (32 ranks each)
  constexpr int PITCH = RT > 4 ? 256 : 128;  // Wu LDS row bytes (r * 2 rounded up to 128 or 256)
  const int r = 16 * RT;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15, kg = lane >> 4;
  const int row = blockIdx.x * LSQ_ROWS + 16 * wave + n;  // this lane's row (tile row n)
  // The stage / group part of every global address moves the descriptor's
  // base (scalar), so each lane keeps one fixed offset per stream: range
  // checks stay exact (the records shrink with the base) and the per-stage
  // addresses need no registers.
  const char* const xg = reinterpret_cast<const char*>(P.x);
  const char* const dg = reinterpret_cast<const char*>(P.wd);
  const char* const ug = reinterpret_cast<const char*>(P.wu);
  const uint32_t xbytes = (uint32_t)((int64_t)rows * D * 2), dbytes = (uint32_t)(r * D * 2);

  // ---- 1. down projection
  // Stage s: the Wd rows' 64 inputs, 2 r 16-byte chunks in blocks of 8 rows
  // (1 KB); wave w moves blocks u = w + LSQ_NW i (lane l: row 8 u + l / 8,
  // LDS position l % 8, which holds input chunk (l % 8) ^ key(row)).  The
  // lane's x inputs: row `row`, inputs 64 s + 32 h + 8 kg .. + 7, halves h.
  constexpr int WQ = (2 * RT + LSQ_NW - 1) / LSQ_NW;  // Wd blocks per wave and stage
  const int nst = D / LSQ_KS;
  uint32_t wd_off[WQ];
#pragma unroll
  for (int i = 0; i < WQ; ++i) {
    const int u = wave + LSQ_NW * i;
    const int wrow = 8 * u + (lane >> 3);
    const int wc = (lane & 7) ^ lsq_key(wrow);
    wd_off[i] = u < 2 * RT ? (uint32_t)((wrow * D + 8 * wc) * 2) : BUF_OOB;
  }
  const uint32_t x_off = row < rows ? (uint32_t)((row * D + 8 * kg) * 2) : BUF_OOB;
  auto load_stage = [&](int s, u32x4 (&wreg)[WQ], f16x8 (&xreg)[2]) {
    const int sb = (s < nst ? s : nst) * LSQ_KS * 2;  // past the end: zero records, loads read zeros
    const __amdgpu_buffer_rsrc_t dr = make_rsrc(dg + sb, dbytes - (uint32_t)sb);
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(xg + sb, s < nst ? xbytes - (uint32_t)sb : 0u);
#pragma unroll
    for (int i = 0; i < WQ; ++i) wreg[i] = buf_ld16(dr, s < nst ? wd_off[i] : BUF_OOB);
#pragma unroll
    for (int h = 0; h < 2; ++h) xreg[h] = __builtin_bit_cast(f16x8, buf_ld16(xr, x_off + 64u * h));
  };
  // every block is written (blocks past the rank hold zeros, in rows no read
  // touches; LSQ_NW * WQ <= 16 blocks fit the buffer): no branch in the loop
  auto put_wd = [&](int s, const u32x4 (&wreg)[WQ]) {
#pragma unroll
    for (int i = 0; i < WQ; ++i)
      *reinterpret_cast<u32x4*>(smem + (s & 1) * LSQ_STAGE + (wave + LSQ_NW * i) * 1024 + lane * 16) = wreg[i];
  };
  f32x4 acc[RT];
#pragma unroll
  for (int t = 0; t < RT; ++t) acc[t] = (f32x4){0.f, 0.f, 0.f, 0.f};
  u32x4 wq[LSQ_PF][WQ];
  f16x8 xq[LSQ_PF][2];
#pragma unroll
  for (int s = 0; s < LSQ_PF - 1; ++s) load_stage(s, wq[s], xq[s]);
  put_wd(0, wq[0]);
  lsq_barrier();
  // stage s: Wd of stage s is in LDS buffer s % 2 (visible after the last
  // barrier); write stage s + 1's Wd into the other buffer (every wave is past
  // its stage s - 1 reads), issue stage s + 3's loads, then the MFMAs
  auto stage = [&](int s, const u32x4 (&wnext)[WQ], const f16x8 (&xa)[2], u32x4 (&wfar)[WQ], f16x8 (&xfar)[2]) {
    put_wd(s + 1, wnext);
    load_stage(s + LSQ_PF - 1, wfar, xfar);
    const char* wb = smem + (s & 1) * LSQ_STAGE;
    // the stage's 2 RT A-operand reads (index i = h RT + t) run LSQ_RA ahead
    // of the MFMAs that use them
    auto rd = [&](int i) {
      const int h = i / RT, t = i % RT;
      const int q = 32 * (t >> 1) + 8 * (n >> 2) + 4 * (t & 1) + (n & 3);  // rank of tile row n
      const int c = 4 * h + kg;
      return *reinterpret_cast<const f16x8*>(wb + q * 128 + 16 * (c ^ lsq_key(q)));
    };
    f16x8 ar[LSQ_RA];
#pragma unroll
    for (int i = 0; i < LSQ_RA; ++i) ar[i] = rd(i);
#pragma unroll
    for (int i = 0; i < 2 * RT; ++i) {
      const f16x8 a = ar[i % LSQ_RA];
      if (i + LSQ_RA < 2 * RT) ar[i % LSQ_RA] = rd(i + LSQ_RA);
      __builtin_amdgcn_sched_barrier(0);
      acc[i % RT] = mfma16x16x32(a, xa[i / RT], acc[i % RT]);
      __builtin_amdgcn_sched_barrier(0);
    }
    lsq_barrier();
  };
  static_assert(LSQ_PF == 4, "the stage loop below rotates four register sets");
  for (int s = 0; s < nst; s += 4) {  // the register sets rotate with s % 4 (nst % 4 == 0)
    stage(s, wq[1], xq[0], wq[3], xq[3]);
    stage(s + 1, wq[2], xq[1], wq[0], xq[0]);
    stage(s + 2, wq[3], xq[2], wq[1], xq[1]);
    stage(s + 3, wq[0], xq[3], wq[2], xq[2]);
  }

  // ---- 2. mid: ranks 32 s + 8 kg .. + 7 of row `row`, rounded to fp16
  f16x8 mid[KU];
#pragma unroll
  for (int s = 0; s < KU; ++s)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      mid[s][e] = (_Float16)lora_act_fast(acc[2 * s][e], P.act_d);
      mid[s][4 + e] = (_Float16)lora_act_fast(acc[2 * s + 1][e], P.act_d);
    }

  // ---- 3. up projection, groups of 64 output columns
  // (its per-lane offsets derive from these copies, which the compiler cannot
  // hoist above the down loop: computed early, they would hold registers
  // through it)
  int lane3 = lane, row3 = row;
  asm volatile("" : "+v"(lane3), "+v"(row3));
  // Group g: Wu rows 64 g .. + 63 (row q at q * PITCH, chunk c at position
  // c ^ key(q)): 4 * PITCH / 64 blocks of 1 KB; wave w moves blocks
  // u = w + LSQ_NW i (lane l: chunk 64 u + l, row (64 u + l) / (PITCH / 16)).
  constexpr int CPR = PITCH / 16;                                // chunk positions per row
  constexpr int WUB = 4 * PITCH / 64;                            // 1 KB blocks per group
  constexpr int UQ = (WUB + LSQ_NW - 1) / LSQ_NW;                // blocks per wave
  const int ngr = A / 64;
  const __amdgpu_buffer_rsrc_t br = make_rsrc(P.bu, P.bu ? (uint32_t)(A * 2) : 0u);
  char* const yg = reinterpret_cast<char*>(P.y);
  const uint32_t ybytes = (uint32_t)((int64_t)rows * A * 2);
  const uint32_t y_off = row3 < rows ? (uint32_t)(((int64_t)row3 * A + 8 * (lane3 >> 4)) * 2) : BUF_OOB;
  struct GroupIn {
    u32x4 w[UQ];  // the lane's Wu chunks of one group
  };
  uint32_t wu_off[UQ];
#pragma unroll
  for (int i = 0; i < UQ; ++i) {
    const int u = wave + LSQ_NW * i;
    const int wrow = (64 * u + lane3) / CPR;
    const int wc = ((64 * u + lane3) % CPR) ^ lsq_key(wrow);
    wu_off[i] = u < WUB && 8 * wc < r ? (uint32_t)((wrow * r + 8 * wc) * 2) : BUF_OOB;
  }
  auto load_group = [&](int g, GroupIn& gi) {
    const int gb = (g < ngr ? g : ngr) * 64 * r * 2;
    const __amdgpu_buffer_rsrc_t ur = make_rsrc(ug + gb, (uint32_t)(A * r * 2 - gb));
#pragma unroll
    for (int i = 0; i < UQ; ++i) gi.w[i] = buf_ld16(ur, wu_off[i]);
  };
  auto put_wu = [&](int g, const GroupIn& gi) {
#pragma unroll
    for (int i = 0; i < UQ; ++i)
      *reinterpret_cast<u32x4*>(smem + (g & 1) * LSQ_STAGE + (wave + LSQ_NW * i) * 1024 + lane * 16) = gi.w[i];
  };
  // the bias row (A fp16 values) -> LDS after the two buffers, once
  char* bl = smem + 2 * LSQ_STAGE;
  for (int i = tid; i < A / 8; i += 64 * LSQ_NW)
    *reinterpret_cast<u32x4*>(bl + 16 * i) = buf_ld16(br, (uint32_t)i * 16u);
  GroupIn gq[LSQ_PF];
#pragma unroll
  for (int g = 0; g < LSQ_PF - 1; ++g) load_group(g, gq[g]);
  put_wu(0, gq[0]);
  lsq_barrier();
  // output register sets, group g computes into set g % 2 (stored at the start
  // of group g + 1, rewritten by group g + 2); set 1 starts as the dummy that
  // group 0 stores out of range
  u32x4 dq[2][2];
  dq[1][0] = dq[1][1] = (u32x4){0u, 0u, 0u, 0u};
  // group g's two stores (columns 64 g + 8 kg and 64 g + 32 + 8 kg of row
  // `row`); group -1 (the dummy) has no records, so its stores are dropped
  auto store_group = [&](int g, const u32x4 (&d)[2]) {
    const __amdgpu_buffer_rsrc_t yr = make_rsrc(yg + (g < 0 ? 0 : 128 * g), g < 0 ? 0u : ybytes - 128u * g);
    __builtin_amdgcn_raw_buffer_store_b128(d[0], yr, (int)y_off, 0, 0);
    __builtin_amdgcn_raw_buffer_store_b128(d[1], yr, (int)(y_off + 64u), 0, 0);
  };
  // group g: Wu of group g in LDS buffer g % 2; store group g - 1's outputs
  // (dp; group 0 stores the dummy set), write group g + 1's
  // Wu, issue group g + 3's loads, then the MFMAs and group g's outputs
  auto group = [&](int g, const GroupIn& gnext, GroupIn& gfar, const u32x4 (&dp)[2], u32x4 (&dc)[2]) {
    store_group(g - 1, dp);
    put_wu(g + 1, gnext);
    load_group(g + LSQ_PF - 1, gfar);
    const char* wb = smem + (g & 1) * LSQ_STAGE;
    f32x4 c4[4];  // output tiles
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) c4[jj] = (f32x4){0.f, 0.f, 0.f, 0.f};
    // the group's 4 KU A-operand reads (index i = 4 s + jj) run LSQ_RA ahead
    auto rd = [&](int i) {
      const int s2 = i >> 2, jj = i & 3;
      const int q = 32 * (jj >> 1) + 8 * (n >> 2) + 4 * (jj & 1) + (n & 3);  // group column of tile row n
      const int c = 4 * s2 + kg;
      return *reinterpret_cast<const f16x8*>(wb + q * PITCH + 16 * (c ^ lsq_key(q)));
    };
    constexpr int RA = 4 * KU < LSQ_RA ? 4 * KU : LSQ_RA;
    f16x8 ar[RA];
#pragma unroll
    for (int i = 0; i < RA; ++i) ar[i] = rd(i);
#pragma unroll
    for (int i = 0; i < 4 * KU; ++i) {
      const f16x8 a = ar[i % RA];
      if (i + RA < 4 * KU) ar[i % RA] = rd(i + RA);
      __builtin_amdgcn_sched_barrier(0);
      c4[i & 3] = mfma16x16x32(a, mid[i >> 2], c4[i & 3]);
      __builtin_amdgcn_sched_barrier(0);
    }
    // lane (n, kg): columns 64 g + 32 (jj / 2) + 8 kg + 4 (jj % 2) + e of row
    // `row`; value v = 8 h + 4 (jj % 2) + e of set h = jj / 2
    float bo[16];
    {
      const u32x4 b0 = *reinterpret_cast<const u32x4*>(bl + (64 * g + 8 * kg) * 2);
      const u32x4 b1 = *reinterpret_cast<const u32x4*>(bl + (64 * g + 32 + 8 * kg) * 2);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        f16x2_to_f32(b0[q], bo[2 * q], bo[2 * q + 1]);
        f16x2_to_f32(b1[q], bo[8 + 2 * q], bo[8 + 2 * q + 1]);
      }
    }
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int jj = q >> 1, e = 2 * (q & 1);
      const _Float16 lo = (_Float16)lora_act_fast(c4[jj][e] + bo[2 * q], P.act_u);
      const _Float16 hi = (_Float16)lora_act_fast(c4[jj][e + 1] + bo[2 * q + 1], P.act_u);
      dc[q >> 2][q & 3] =
          (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
    }
    // the stored set stays allocated until here (not reused while its stores run)
    asm volatile("" ::"v"(dp[0]), "v"(dp[1]));
    lsq_barrier();
  };
  for (int g = 0; g < ngr; g += 4) {  // the register sets rotate with g % 4 (ngr % 4 == 0)
    group(g, gq[1], gq[3], dq[1], dq[0]);
    group(g + 1, gq[2], gq[0], dq[0], dq[1]);
    group(g + 2, gq[3], gq[1], dq[1], dq[0]);
    group(g + 3, gq[0], gq[2], dq[0], dq[1]);
  }
  store_group(ngr - 1, dq[1]);  // the last group's outputs (set 1)
}

__global__ __launch_bounds__(1024) void lora_seq_kernel(const LoraBatch B, int rows) {
  extern __shared__ __align__(16) char smem[];
  const LoraProb& P = B.p[blockIdx.y];
  switch (P.r) {  // uniform over the workgroup
    case 32: lsq_body<2>(P, rows, B.D, B.A, smem); break;
    case 64: lsq_body<4>(P, rows, B.D, B.A, smem); break;
    case 96: lsq_body<6>(P, rows, B.D, B.A, smem); break;
    default: lsq_body<8>(P, rows, B.D, B.A, smem); break;
  }
}

bool lora_seq_supported(const LoraBatch& b, int64_t rows) {
  // whole rounds of four down stages and four up groups
  if (b.D % (4 * LSQ_KS) || b.A % 256 || b.A > LSQ_MAXA || rows <= 0) return false;
  // 32-bit buffer offsets for x, y and the weights
  if (rows * std::max(b.D, b.A) * 2 >= (int64_t)BUF_OOB) return false;
  for (int i = 0; i < b.nprob; ++i) {
    const int r = b.p[i].r;
    if (r % 32 || r > 128) return false;
    if ((reinterpret_cast<uintptr_t>(b.p[i].y) | reinterpret_cast<uintptr_t>(b.p[i].bu)) & 15) return false;
  }
  return true;
}

int lora_seq_run(const LoraBatch& b0, int64_t rows, void* stream) {
  // problems by decreasing rank: the grid dispatches problem by problem, so
  // the longest workgroups start first and the short ones fill in behind them
  LoraBatch b = b0;
  std::stable_sort(b.p, b.p + b.nprob, [](const LoraProb& x, const LoraProb& y) { return x.r > y.r; });
  static std::atomic<uint64_t> raised{0};
  const int lds = 2 * LSQ_STAGE + b.A * 2;
  if (int rc = raise_dynamic_lds(reinterpret_cast<const void*>(&lora_seq_kernel), 2 * LSQ_STAGE + LSQ_MAXA * 2, raised,
                                 "lora_seq_kernel"))
    return rc;
  const dim3 grid((unsigned)((rows + LSQ_ROWS - 1) / LSQ_ROWS), (unsigned)b.nprob);
  hipLaunchKernelGGL(lora_seq_kernel, grid, dim3(64 * LSQ_NW), lds, as_stream(stream), b, (int)rows);
  return check_launch("lora_seq_kernel");
}

}  // namespace rwkv7mi
