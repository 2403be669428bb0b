// The W/A/G/V LoRA up projections inside a decode state-update kernel, shared
// by the fp32-state (wkv7_decode.hip) and fp16-state (wkv7_f16.hip) kernels.
//
// The second half of fused_wavg_lora (rwkv7_hf/fused_lora.py:706-886): the down
// projections' fp32 partials (lora.hip, [problem][ks][rows][rank]) are summed
// in fixed order, act_down applied and rounded to the activation dtype (the
// reference's mid tensor); each (batch, head) workgroup then computes only its
// own 64 channels of every up projection, y_p = act_up_p(mid_p Wu_p^T + b_p),
// rounded to the activation dtype as the reference's tensors are.
// Problems: 0 w_raw, 1 a, 2 g, 3 v_gate (the last only with v_mode 2).
// Wave p of a 256-lane workgroup handles problem p end to end (lane c = output
// channel h*64 + c), so its pointers and rank are wave-uniform and it needs no
// barrier until the four results meet for the state update.
#pragma once

#include <string>

#include "common.h"

namespace rwkv7mi {

constexpr int DL_HEAD = 64;
constexpr int DL_MAXR = 128;  // largest rank on this route
constexpr int DL_ZB = 16;     // K-split partials loaded per batch (1 when the sums arrive whole)

struct DecLora {
  const float* part;
  const void* wu[4];
  const void* bu[4];
  int64_t part_off[4];  // floats
  int64_t part_total;   // floats of the whole partial buffer
  int rank[4], act_d[4], act_u[4];
  int nprob, ks, rows;
};

__device__ __forceinline__ float dl_act(float v, int act) {
  if (act == 1) return tanhf(v);
  if (act == 2) return 1.0f / (1.0f + expf(-v));
  return v;
}

// This wave's LoRA problem for batch row b, head h: s_lo[wave][c] = channel
// h*64 + c of the up projection, in fp32 holding a TA value.  `between` runs
// after the first batch of partial loads is issued and before the up weights
// are: the caller's own loads (state rows, vectors) go there, so they are in
// flight together with the LoRA loads without delaying the partials the up
// projection waits on first (loads complete in issue order).
template <typename TA, int ZB, typename Between>
__device__ __forceinline__ void dl_up(const DecLora& LA, int b, int h, int H, int wave, int lane,
                                      float (&s_mid)[4][DL_MAXR], float (&s_lo)[4][DL_HEAD], Between&& between) {
  const bool active = wave < LA.nprob;  // wave-uniform
  const int rp = active ? LA.rank[wave] : 0;
  float pt0[2][ZB];
  {
    const __amdgpu_buffer_rsrc_t pr = make_rsrc(LA.part, (uint32_t)LA.part_total * 4u);
    const uint32_t zs = (uint32_t)(LA.rows * rp);
    const uint32_t base = (uint32_t)((active ? LA.part_off[wave] : 0) + (int64_t)b * rp);
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int zz = 0; zz < ZB; ++zz) {
        const bool ok = lane + 64 * u < rp && zz < LA.ks;
        pt0[u][zz] = buf_ldf(pr, ok ? (base + (uint32_t)zz * zs + lane + 64u * u) * 4u : BUF_OOB);
      }
  }
  between();
  // Up projection of this wave's problem, loaded coalesced: a row of Wu_p
  // (rank elements) is spread over L lanes, 8 elements each (L = rank / 8
  // rounded up to a power of two), so load i reads the 64 / L consecutive
  // rows i * 64 / L .. of the head as one contiguous run.  The lane's row
  // segments are dotted with its 8 mid values and the L lanes of a row then
  // reduce-scatter, which leaves channel c = lq * (64 / L) + lr in lane
  // (lr, lq), lane = lr * L + lq.
  const int r8 = rp >> 3;
  const int L = r8 <= 1 ? 1 : r8 <= 2 ? 2 : r8 <= 4 ? 4 : r8 <= 8 ? 8 : 16;  // wave-uniform
  const int lq = lane & (L - 1), lr = lane / L, rpi = DL_HEAD / L;
  const int cu = lq * rpi + lr;  // the channel this lane finishes
  const void* bu_w = active ? LA.bu[wave] : nullptr;
  const float bias_pre = buf_ld1<TA>(
      make_rsrc(bu_w ? reinterpret_cast<const TA*>(bu_w) + (int64_t)h * DL_HEAD : nullptr,
                bu_w ? DL_HEAD * (uint32_t)sizeof(TA) : 0u),
      (uint32_t)cu, bu_w != nullptr);
  float wseg[DL_MAXR / 8][8];
  {
    const __amdgpu_buffer_rsrc_t wr =
        make_rsrc(active ? LA.wu[wave] : LA.wu[0], (uint32_t)((int64_t)H * DL_HEAD * rp * (int64_t)sizeof(TA)));
#pragma unroll
    for (int i = 0; i < DL_MAXR / 8; ++i) {
      const uint32_t e0 = (uint32_t)((int64_t)(h * DL_HEAD + i * rpi + lr) * rp + 8 * lq);
      buf_ld8(wr, e0, i < L && lq < r8, (const TA*)nullptr, wseg[i]);
    }
  }
  // mid_p[kk] for kk = lane, lane + 64: the rest of the K-split partials (the
  // first ZB splits are in flight since the kernel's start), summed in z order
  {
    const __amdgpu_buffer_rsrc_t pr = make_rsrc(LA.part, (uint32_t)LA.part_total * 4u);
    const uint32_t zs = (uint32_t)(LA.rows * rp);
    const uint32_t base = (uint32_t)((active ? LA.part_off[wave] : 0) + (int64_t)b * rp);
    float acc[2] = {0.f, 0.f};
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int zz = 0; zz < ZB; ++zz) acc[u] += pt0[u][zz];  // past-the-end terms are +0
    for (int z0 = ZB; z0 < LA.ks; z0 += ZB) {
      float t[2][ZB];
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int zz = 0; zz < ZB; ++zz) {
          const bool ok = lane + 64 * u < rp && z0 + zz < LA.ks;
          t[u][zz] = buf_ldf(pr, ok ? (base + (uint32_t)(z0 + zz) * zs + lane + 64u * u) * 4u : BUF_OOB);
        }
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int zz = 0; zz < ZB; ++zz) acc[u] += t[u][zz];
    }
    // every entry of the wave's row is written (zeros past the rank), so the
    // up projection's segments past the rank read zeros
    const int ad = active ? LA.act_d[wave] : 0;
#pragma unroll
    for (int u = 0; u < 2; ++u)
      s_mid[wave][lane + 64 * u] = lane + 64 * u < rp ? to_f32(from_f32<TA>(dl_act(acc[u], ad))) : 0.f;
  }
  // this wave's problem (the wave reads its own s_mid row: LDS operations of
  // one wave complete in order, so no barrier is needed)
  if (active) {
    const float4 m0 = *reinterpret_cast<const float4*>(&s_mid[wave][8 * lq]);
    const float4 m1 = *reinterpret_cast<const float4*>(&s_mid[wave][8 * lq + 4]);
    float pt[DL_MAXR / 8];
#pragma unroll
    for (int i = 0; i < DL_MAXR / 8; ++i)
      pt[i] = ((m0.x * wseg[i][0] + m0.y * wseg[i][1]) + (m0.z * wseg[i][2] + m0.w * wseg[i][3])) +
              ((m1.x * wseg[i][4] + m1.y * wseg[i][5]) + (m1.z * wseg[i][6] + m1.w * wseg[i][7]));
    // reduce-scatter over the row's L lanes: at distance d the lane with bit d
    // of lq set keeps the upper half of its window; pt[0] ends as the total of
    // load lq's row (loads past L read zeros)
#pragma unroll
    for (int d = DL_MAXR / 16; d >= 1; d >>= 1) {
      if (d < L) {
        const bool up = (lq & d) != 0;
#pragma unroll
        for (int j = 0; j < d; ++j) {
          const float keep = up ? pt[j + d] : pt[j];
          const float give = up ? pt[j] : pt[j + d];
          pt[j] = keep + __shfl_xor(give, d, 64);
        }
      }
    }
    float acc = pt[0];
    if (bu_w) acc += bias_pre;
    s_lo[wave][cu] = to_f32(from_f32<TA>(dl_act(acc, LA.act_u[wave])));
  }
}

// Host: the DecLora record of a call, validated (`who` prefixes the messages);
// RWKV7MI_OK or RWKV7MI_EINVAL.  ks = splits, or the split
// rwkv7mi_lora_down_multi uses for these ranks and D when splits is 0.
inline int dl_build(DecLora& la, const char* who, const float* lora_part, int64_t nprob, const int64_t* ranks,
                    const void* const* w_up, const void* const* b_up, const int* act_down, const int* act_up,
                    int64_t D, int64_t splits, int64_t B) {
  const std::string w(who);
  if (!lora_part || !ranks || !w_up || !act_down || !act_up) return fail(RWKV7MI_EINVAL, w + ": null pointer");
  if (nprob != 3 && nprob != 4) return fail(RWKV7MI_EINVAL, w + ": 3 or 4 LoRA problems");
  if (splits < 0 || splits > 4096) return fail(RWKV7MI_EINVAL, w + ": bad lora_splits");
  la = DecLora{};
  la.part = lora_part;
  la.nprob = (int)nprob;
  la.rows = (int)B;
  la.ks = splits ? (int)splits : lora_splits(lora_tiles(nprob, ranks), D);
  int64_t off = 0;
  for (int p = 0; p < nprob; ++p) {
    if (ranks[p] <= 0 || ranks[p] % 8 || ranks[p] > DL_MAXR || !w_up[p])
      return fail(RWKV7MI_EINVAL, w + ": ranks must be positive multiples of 8, at most 128");
    if (act_down[p] < 0 || act_down[p] > 2 || act_up[p] < 0 || act_up[p] > 2)
      return fail(RWKV7MI_EINVAL, w + ": activation must be 0 none, 1 tanh or 2 sigmoid");
    if (reinterpret_cast<uintptr_t>(w_up[p]) & 15) return fail(RWKV7MI_EINVAL, w + ": up weights must be 16-byte aligned");
    la.wu[p] = w_up[p];
    la.bu[p] = b_up ? b_up[p] : nullptr;
    la.rank[p] = (int)ranks[p];
    la.act_d[p] = act_down[p];
    la.act_u[p] = act_up[p];
    la.part_off[p] = off;
    off += (int64_t)la.ks * B * ranks[p];
  }
  la.part_total = off;
  return RWKV7MI_OK;
}

}  // namespace rwkv7mi
