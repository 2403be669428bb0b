/*
 * CPU oracle (TEST INFRASTRUCTURE ONLY) for the rwkv7mi hot path.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * this library, and only as the checker / CPU baseline.  Nothing in the product
 * path (hf-adapter_amd/) links or calls it.
 *
 * Restates, in plain C:
 *   - the DPLR recurrence (rwkv7_hf/fused_recurrent_update.py:757-783 and
 *     :800-844): S' = S diag(w) + (S (-kk)) (kk*a)^T + v k^T, y = S' r,
 *     state [B,H,N,N] with row = value channel, column = key channel; fp64;
 *   - quantize_mm8 (rwkv7_hf/native_quant_mm8.py:62-97) as the same fp32
 *     IEEE op sequence (compiled with -ffp-contract=off, no fast-math);
 *   - quantize_w4_groupwise (rwkv7_hf/sm70_quant.py:502-519), fp32, RNE;
 *   - quantize_mm4 (rwkv7_hf/native_quant_mm4.py:77-105), fp32.
 * fp16 rounding of the packers' metadata is left to numpy (astype float16,
 * round-to-nearest-even), matching torch's .to(float16).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------- wkv7 scan */
/* Inputs [B,T,H,N] as double; state [B,H,N,N] double updated in place;
 * y [B,T,H,N] double.  Heads are independent (parallel over b*h). */
void wkv7_ref_scan_f64(int64_t B, int64_t T, int64_t H, int64_t N, const double* r,
                       const double* w, const double* k, const double* v, const double* kk,
                       const double* a, double* state, double* y) {
#pragma omp parallel for schedule(static)
  for (int64_t bh = 0; bh < B * H; ++bh) {
    const int64_t b = bh / H, h = bh % H;
    double* S = state + bh * N * N;
    double* dot = (double*)malloc(sizeof(double) * N);
    for (int64_t t = 0; t < T; ++t) {
      const int64_t off = ((b * T + t) * H + h) * N;
      const double *rt = r + off, *wt = w + off, *kt = k + off, *vt = v + off, *kkt = kk + off,
                   *at = a + off;
      for (int64_t i = 0; i < N; ++i) {
        double d = 0.0;
        for (int64_t j = 0; j < N; ++j) d += S[i * N + j] * kkt[j];
        dot[i] = d;
      }
      for (int64_t i = 0; i < N; ++i) {
        double acc = 0.0;
        for (int64_t j = 0; j < N; ++j) {
          double s = S[i * N + j] * wt[j] - dot[i] * kkt[j] * at[j] + vt[i] * kt[j];
          S[i * N + j] = s;
          acc += s * rt[j];
        }
        y[off + i] = acc;
      }
    }
    free(dot);
  }
}

/* Same recurrence with fp32 state and fp32 arithmetic (CPU baseline of the
 * sequential scan; inputs already widened to float). */
void wkv7_ref_scan_f32(int64_t B, int64_t T, int64_t H, int64_t N, const float* r, const float* w,
                       const float* k, const float* v, const float* kk, const float* a, float* state,
                       float* y) {
#pragma omp parallel for schedule(static)
  for (int64_t bh = 0; bh < B * H; ++bh) {
    const int64_t b = bh / H, h = bh % H;
    float* S = state + bh * N * N;
    float* dot = (float*)malloc(sizeof(float) * N);
    for (int64_t t = 0; t < T; ++t) {
      const int64_t off = ((b * T + t) * H + h) * N;
      const float *rt = r + off, *wt = w + off, *kt = k + off, *vt = v + off, *kkt = kk + off,
                  *at = a + off;
      for (int64_t i = 0; i < N; ++i) {
        float d = 0.f;
        for (int64_t j = 0; j < N; ++j) d += S[i * N + j] * kkt[j];
        dot[i] = d;
      }
      for (int64_t i = 0; i < N; ++i) {
        float acc = 0.f;
        for (int64_t j = 0; j < N; ++j) {
          float s = S[i * N + j] * wt[j] - dot[i] * kkt[j] * at[j] + vt[i] * kt[j];
          S[i * N + j] = s;
          acc += s * rt[j];
        }
        y[off + i] = acc;
      }
    }
    free(dot);
  }
}

int oracle_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* ------------------------------------------------------------- MM8 packer */
/* W [n,m] fp32 (n = in_features, m = out_features).  Outputs: q [n,m];
 * mx, rx16 [m] and my, ry16 [n] in fp32 (rx16 = rx/16, ry16 = ry/16).
 * Follows rwkv7_hf/native_quant_mm8.py:70-89 op for op. */
void mm8_ref_pack(const float* W, int64_t n, int64_t m, uint8_t* q, float* mx, float* rx16,
                  float* my, float* ry16) {
  float* rx = (float*)malloc(sizeof(float) * m);
  float* ry = (float*)malloc(sizeof(float) * n);
  const int rows_first = n > m;
  /* first and second min */
  if (rows_first) {
    for (int64_t i = 0; i < n; ++i) {
      float mn = INFINITY;
      for (int64_t j = 0; j < m; ++j) mn = fminf(mn, W[i * m + j]);
      my[i] = mn;
    }
    for (int64_t j = 0; j < m; ++j) mx[j] = INFINITY;
    for (int64_t i = 0; i < n; ++i)
      for (int64_t j = 0; j < m; ++j) mx[j] = fminf(mx[j], W[i * m + j] - my[i]);
  } else {
    for (int64_t j = 0; j < m; ++j) mx[j] = INFINITY;
    for (int64_t i = 0; i < n; ++i)
      for (int64_t j = 0; j < m; ++j) mx[j] = fminf(mx[j], W[i * m + j]);
    for (int64_t i = 0; i < n; ++i) {
      float mn = INFINITY;
      for (int64_t j = 0; j < m; ++j) mn = fminf(mn, W[i * m + j] - mx[j]);
      my[i] = mn;
    }
  }
  /* w2 = W - first - second; rx = max(colmax(w2), 1e-8); ry = max(rowmax(w2/rx), 1e-8) */
  for (int64_t j = 0; j < m; ++j) rx[j] = -INFINITY;
  for (int64_t i = 0; i < n; ++i)
    for (int64_t j = 0; j < m; ++j) {
      float w2 = rows_first ? (W[i * m + j] - my[i]) - mx[j] : (W[i * m + j] - mx[j]) - my[i];
      rx[j] = fmaxf(rx[j], w2);
    }
  for (int64_t j = 0; j < m; ++j) rx[j] = fmaxf(rx[j], 1e-8f);
  for (int64_t i = 0; i < n; ++i) {
    float mxv = -INFINITY;
    for (int64_t j = 0; j < m; ++j) {
      float w2 = rows_first ? (W[i * m + j] - my[i]) - mx[j] : (W[i * m + j] - mx[j]) - my[i];
      mxv = fmaxf(mxv, w2 / rx[j]);
    }
    ry[i] = fmaxf(mxv, 1e-8f);
  }
  for (int64_t i = 0; i < n; ++i)
    for (int64_t j = 0; j < m; ++j) {
      float w2 = rows_first ? (W[i * m + j] - my[i]) - mx[j] : (W[i * m + j] - mx[j]) - my[i];
      float w4 = (w2 / rx[j]) / ry[i];
      float c = floorf(w4 * 256.0f);
      c = fminf(fmaxf(c, 0.0f), 255.0f);
      q[i * m + j] = (uint8_t)c;
    }
  for (int64_t j = 0; j < m; ++j) rx16[j] = rx[j] / 16.0f;
  for (int64_t i = 0; i < n; ++i) ry16[i] = ry[i] / 16.0f;
  free(rx);
  free(ry);
}

/* ------------------------------------------------------ W4 group packer */
/* W [o_n, i_n] fp32 -> packed [o_n, i_n/2], scales [o_n, i_n/group] fp32.
 * rwkv7_hf/sm70_quant.py:512-519: s = max(amax|w|/7, 1e-6),
 * q = clamp(round_half_even(w/s), -7, 7) + 8. */
void w4g_ref_pack(const float* W, int64_t o_n, int64_t i_n, int64_t group, uint8_t* packed,
                  float* scales) {
  const int64_t ng = i_n / group;
  for (int64_t o = 0; o < o_n; ++o) {
    for (int64_t g = 0; g < ng; ++g) {
      const float* src = W + o * i_n + g * group;
      float am = 0.f;
      for (int64_t e = 0; e < group; ++e) am = fmaxf(am, fabsf(src[e]));
      float s = fmaxf(am / 7.0f, 1e-6f);
      scales[o * ng + g] = s;
      for (int64_t e = 0; e < group; e += 2) {
        float q0 = nearbyintf(src[e] / s);
        float q1 = nearbyintf(src[e + 1] / s);
        q0 = fminf(fmaxf(q0, -7.f), 7.f) + 8.f;
        q1 = fminf(fmaxf(q1, -7.f), 7.f) + 8.f;
        packed[o * (i_n / 2) + (g * group + e) / 2] = (uint8_t)((int)q0 | ((int)q1 << 4));
      }
    }
  }
}

/* ------------------------------------------------------- MM4 affine packer */
/* W [n, m_pad] fp32 (m_pad even, caller pads with zeros as
 * rwkv7_hf/native_quant_mm4.py:89-92 does).  Same op sequence as MM8 with 16
 * levels: q = clamp(floor(16 w4), 0, 15); packed[i, c] = q[i,2c] | q[i,2c+1] << 4;
 * rx4 = rx/4, ry4 = ry/4. */
void mm4_ref_pack(const float* W, int64_t n, int64_t m, uint8_t* packed, float* mx, float* rx4,
                  float* my, float* ry4) {
  uint8_t* q8 = (uint8_t*)malloc((size_t)(n * m));
  float* rx16 = (float*)malloc(sizeof(float) * m);
  float* ry16 = (float*)malloc(sizeof(float) * n);
  /* reuse the MM8 sequence for the min/max passes, then requantize to 16 levels */
  mm8_ref_pack(W, n, m, q8, mx, rx16, my, ry16);
  const int rows_first = n > m;
  for (int64_t i = 0; i < n; ++i)
    for (int64_t j = 0; j < m; ++j) {
      float rx = rx16[j] * 16.0f, ry = ry16[i] * 16.0f;
      float w2 = rows_first ? (W[i * m + j] - my[i]) - mx[j] : (W[i * m + j] - mx[j]) - my[i];
      float w4 = (w2 / rx) / ry;
      float c = floorf(w4 * 16.0f);
      c = fminf(fmaxf(c, 0.0f), 15.0f);
      q8[i * m + j] = (uint8_t)c;
    }
  for (int64_t i = 0; i < n; ++i)
    for (int64_t c = 0; c < m / 2; ++c)
      packed[i * (m / 2) + c] = (uint8_t)(q8[i * m + 2 * c] | (q8[i * m + 2 * c + 1] << 4));
  for (int64_t j = 0; j < m; ++j) rx4[j] = (rx16[j] * 16.0f) / 4.0f;
  for (int64_t i = 0; i < n; ++i) ry4[i] = (ry16[i] * 16.0f) / 4.0f;
  free(q8);
  free(rx16);
  free(ry16);
}
