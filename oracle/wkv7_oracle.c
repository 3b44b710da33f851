/*
 * TEST INFRASTRUCTURE ONLY -- not part of the product.
 *
 * CPU restatement of the rwkv-rs WKV7 recurrence. The fp32 functions keep the
 * reference kernels' per-row operation order so that they are a faithful
 * stand-in for the reference CubeCL kernels (which cannot be built here: the
 * reference is Rust on Burn/CubeCL from crates.io, and this image has no
 * cargo). Build with -ffp-contract=off so that C evaluates every product and
 * sum with its own rounding, in source order.
 *
 * Reference files (all under /root/reference/crates/rwkv-nn/src/kernels/):
 *   wkv7_common/kernel.rs:6-114    forward kernel
 *   wkv7_common/kernel.rs:116-308  backward kernel
 *   wkv7_infer/kernel.rs:8-114     inference kernel and dither, with F = f32
 *                                  and with F = bf16
 */
#include "wkv7_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* kernel.rs:4 and wkv7_infer/kernel.rs:4-6 */
#define W_SCALE_F (-0.6065306597f)
#define W_SCALE_D (-0.6065306597)
#define TWO_TO_NEG_41 (4.547473508864641e-13f)
#define ROTATOR1 (2654435769u)

/* index of element n of token (b, t, h) in a [B, T, H, N] tensor
 * (kernel.rs:52-55). */
static inline int64_t tok(int64_t T, int64_t H, int64_t N, int64_t b,
                          int64_t t, int64_t h) {
  return ((b * T + t) * H + h) * N;
}

static int bad_shape(int64_t B, int64_t T, int64_t H, int64_t N) {
  return B < 0 || T < 0 || H < 0 || N <= 0;
}

/* ------------------------------------------------------------------------ */
/* fp32 forward, kernel.rs:6-114                                             */
/* ------------------------------------------------------------------------ */
int wkv7o_forward_f32(int64_t B, int64_t T, int64_t H, int64_t N, int64_t C,
                      const float *w, const float *r, const float *k,
                      const float *v, const float *a, const float *b,
                      const float *s0, float *ckpt, float *sa_out, float *y,
                      float *s_T, int nthreads) {
  if (bad_shape(B, T, H, N) || C <= 0 || T % C != 0) return -1;
  const int64_t n_chunks = T / C;
#ifdef _OPENMP
  if (nthreads <= 0) nthreads = omp_get_max_threads();
#pragma omp parallel for num_threads(nthreads) schedule(dynamic, 1)
#endif
  for (int64_t bh = 0; bh < B * H; ++bh) {
    const int64_t bi = bh / H, hi = bh % H;
    /* state[j * N + i]: thread j owns value-row j (kernel.rs:27-42) */
    float *state = (float *)malloc(sizeof(float) * (size_t)(N * N + 6 * N));
    float *sr = state + N * N, *sw = sr + N, *sk = sw + N, *sv = sk + N,
          *sa = sv + N, *sb = sa + N;
    if (s0) {
      memcpy(state, s0 + bh * N * N, sizeof(float) * (size_t)(N * N));
    } else {
      memset(state, 0, sizeof(float) * (size_t)(N * N));
    }
    for (int64_t t = 0; t < T; ++t) {
      const int64_t base = tok(T, H, N, bi, t, hi);
      /* shared-memory fill, kernel.rs:58-65 */
      for (int64_t n = 0; n < N; ++n) {
        sr[n] = r[base + n];
        sk[n] = k[base + n];
        sa[n] = a[base + n];
        sb[n] = b[base + n];
        sv[n] = v[base + n];
        const float w_raw = w[base + n];
        const float w_sig = 1.0f / (1.0f + expf(-w_raw));
        sw[n] = expf(W_SCALE_F * w_sig);
      }
      for (int64_t j = 0; j < N; ++j) {
        float *row = state + j * N;
        /* removal_state = sum_i a_i S[j,i]  (kernel.rs:68-74) */
        float removal_state = 0.0f;
        for (int64_t i = 0; i < N; ++i) removal_state += sa[i] * row[i];
        sa_out[base + j] = removal_state;
        /* update and read-out, kernel.rs:76-87 */
        const float vj = sv[j];
        float yy = 0.0f;
        for (int64_t i = 0; i < N; ++i) {
          row[i] = row[i] * sw[i] + removal_state * sb[i] + sk[i] * vj;
          yy += row[i] * sr[i];
        }
        y[base + j] = yy;
      }
      /* transposed checkpoint, kernel.rs:89-102 */
      if ((t + 1) % C == 0) {
        float *dst = ckpt + (bh * n_chunks + t / C) * N * N;
        for (int64_t j = 0; j < N; ++j)
          for (int64_t i = 0; i < N; ++i) dst[i * N + j] = state[j * N + i];
      }
    }
    if (s_T) memcpy(s_T + bh * N * N, state, sizeof(float) * (size_t)(N * N));
    free(state);
  }
  return 0;
}

/* ------------------------------------------------------------------------ */
/* fp32 backward, kernel.rs:116-308                                          */
/* ------------------------------------------------------------------------ */
int wkv7o_backward_f32(int64_t B, int64_t T, int64_t H, int64_t N, int64_t C,
                       const float *w, const float *r, const float *k,
                       const float *v, const float *a, const float *b,
                       const float *ckpt, const float *sa_in, const float *dy,
                       const float *ds_T, float *dw, float *dr, float *dk,
                       float *dv, float *da, float *db, float *ds0,
                       int nthreads) {
  if (bad_shape(B, T, H, N) || C <= 0 || T % C != 0) return -1;
  const int64_t n_chunks = T / C;
#ifdef _OPENMP
  if (nthreads <= 0) nthreads = omp_get_max_threads();
#pragma omp parallel for num_threads(nthreads) schedule(dynamic, 1)
#endif
  for (int64_t bh = 0; bh < B * H; ++bh) {
    const int64_t bi = bh / H, hi = bh % H;
    const size_t NN = (size_t)(N * N);
    /* Thread i of the reference block holds (kernel.rs:138-162):
     *   st[i*N + x]  = S[x, i]     (state_transposed: key column i)
     *   sg[i*N + x]  = dS[i, x]    (state_grad: value row i)
     *   stg[i*N + x] = dS[x, i]    (state_transposed_grad: key column i) */
    float *st = (float *)malloc(sizeof(float) * (3 * NN + 11 * (size_t)N));
    float *sg = st + NN, *stg = sg + NN;
    float *sh_r = stg + NN, *sh_w = sh_r + N, *sh_k = sh_w + N,
          *sh_v = sh_k + N, *sh_a = sh_v + N, *sh_b = sh_a + N,
          *sh_dy = sh_b + N, *sh_sa = sh_dy + N, *sh_dsa = sh_sa + N,
          *wsig = sh_dsa + N, *dsa_own = wsig + N;
    memset(st, 0, sizeof(float) * NN);
    if (ds_T) {
      const float *g = ds_T + bh * NN;
      for (int64_t i = 0; i < N; ++i)
        for (int64_t x = 0; x < N; ++x) {
          sg[i * N + x] = g[i * N + x];
          stg[i * N + x] = g[x * N + i];
        }
    } else {
      memset(sg, 0, sizeof(float) * NN);
      memset(stg, 0, sizeof(float) * NN);
    }
    for (int64_t t = T - 1; t >= 0; --t) {
      const int64_t base = tok(T, H, N, bi, t, hi);
      /* shared fill, kernel.rs:186-207 */
      for (int64_t n = 0; n < N; ++n) {
        sh_r[n] = r[base + n];
        const float w_sig = 1.0f / (1.0f + expf(-w[base + n]));
        wsig[n] = w_sig;
        sh_w[n] = expf(W_SCALE_F * w_sig);
        sh_k[n] = k[base + n];
        sh_a[n] = a[base + n];
        sh_b[n] = b[base + n];
        sh_v[n] = v[base + n];
        sh_dy[n] = dy[base + n];
        sh_sa[n] = sa_in[base + n];
      }
      /* checkpoint reload, kernel.rs:210-228 */
      if ((t + 1) % C == 0) {
        const float *src = ckpt + (bh * n_chunks + t / C) * (int64_t)NN;
        memcpy(st, src, sizeof(float) * NN);
      }
      /* phase 1, per thread i (kernel.rs:230-272) */
      for (int64_t i = 0; i < N; ++i) {
        float *sti = st + i * N, *sgi = sg + i * N, *stgi = stg + i * N;
        const float r_i = sh_r[i], w_i = sh_w[i], k_i = sh_k[i];
        const float b_i = sh_b[i], dy_i = sh_dy[i];
        float receptance_grad = 0.0f;
        for (int64_t x = 0; x < N; ++x) receptance_grad += sti[x] * sh_dy[x];
        dr[base + i] = receptance_grad;
        const float inverse_w = 1.0f / w_i;
        for (int64_t x = 0; x < N; ++x) {
          sti[x] = (sti[x] - k_i * sh_v[x] - b_i * sh_sa[x]) * inverse_w;
          sgi[x] += dy_i * sh_r[x];
          stgi[x] += r_i * sh_dy[x];
        }
        float wg = 0.0f, kg = 0.0f, vg = 0.0f, bg = 0.0f, dsa = 0.0f;
        for (int64_t x = 0; x < N; ++x) {
          wg += stgi[x] * sti[x];
          kg += stgi[x] * sh_v[x];
          vg += sgi[x] * sh_k[x];
          dsa += sgi[x] * sh_b[x];
          bg += stgi[x] * sh_sa[x];
        }
        dw[base + i] = W_SCALE_F * wg * w_i * wsig[i] * (1.0f - wsig[i]);
        dk[base + i] = kg;
        dv[base + i] = vg;
        db[base + i] = bg;
        dsa_own[i] = dsa;
      }
      /* shared_replaced_state_grad, kernel.rs:274-276 */
      for (int64_t i = 0; i < N; ++i) sh_dsa[i] = dsa_own[i];
      /* phase 2, kernel.rs:280-296 */
      for (int64_t i = 0; i < N; ++i) {
        float *sti = st + i * N, *sgi = sg + i * N, *stgi = stg + i * N;
        float agrad = 0.0f;
        for (int64_t x = 0; x < N; ++x) agrad += sti[x] * sh_dsa[x];
        da[base + i] = agrad;
        const float w_i = sh_w[i], a_i = sh_a[i], dsa = dsa_own[i];
        for (int64_t x = 0; x < N; ++x) {
          sgi[x] = sgi[x] * sh_w[x] + dsa * sh_a[x];
          stgi[x] = stgi[x] * w_i + a_i * sh_dsa[x];
        }
      }
    }
    /* kernel.rs:299-307 */
    if (ds0) memcpy(ds0 + bh * (int64_t)NN, sg, sizeof(float) * NN);
    free(st);
  }
  return 0;
}

/* ------------------------------------------------------------------------ */
/* fp64 forward and BPTT                                                     */
/* ------------------------------------------------------------------------ */
static double sigmoid_d(double x) { return 1.0 / (1.0 + exp(-x)); }

int wkv7o_forward_f64(int64_t B, int64_t T, int64_t H, int64_t N,
                      const double *w, const double *r, const double *k,
                      const double *v, const double *a, const double *b,
                      const double *s0, double *y, double *s_T) {
  if (bad_shape(B, T, H, N)) return -1;
  for (int64_t bh = 0; bh < B * H; ++bh) {
    const int64_t bi = bh / H, hi = bh % H;
    const size_t NN = (size_t)(N * N);
    double *S = (double *)malloc(sizeof(double) * (NN + (size_t)N));
    double *wd = S + NN;
    if (s0) memcpy(S, s0 + bh * (int64_t)NN, sizeof(double) * NN);
    else memset(S, 0, sizeof(double) * NN);
    for (int64_t t = 0; t < T; ++t) {
      const int64_t base = tok(T, H, N, bi, t, hi);
      for (int64_t i = 0; i < N; ++i)
        wd[i] = exp(W_SCALE_D * sigmoid_d(w[base + i]));
      for (int64_t j = 0; j < N; ++j) {
        double *row = S + j * N, sa = 0.0, yy = 0.0;
        for (int64_t i = 0; i < N; ++i) sa += a[base + i] * row[i];
        for (int64_t i = 0; i < N; ++i) {
          row[i] = row[i] * wd[i] + sa * b[base + i] + k[base + i] * v[base + j];
          yy += row[i] * r[base + i];
        }
        y[base + j] = yy;
      }
    }
    if (s_T) memcpy(s_T + bh * (int64_t)NN, S, sizeof(double) * NN);
    free(S);
  }
  return 0;
}

int wkv7o_grad_f64(int64_t B, int64_t T, int64_t H, int64_t N,
                   const double *w, const double *r, const double *k,
                   const double *v, const double *a, const double *b,
                   const double *s0, const double *dy, const double *ds_T,
                   double *dw, double *dr, double *dk, double *dv, double *da,
                   double *db, double *ds0) {
  if (bad_shape(B, T, H, N)) return -1;
  const size_t NN = (size_t)(N * N);
  for (int64_t bh = 0; bh < B * H; ++bh) {
    const int64_t bi = bh / H, hi = bh % H;
    /* states[t+1] = S_t, states[0] = S_{-1} = s0 */
    double *states = (double *)malloc(sizeof(double) * NN * (size_t)(T + 1));
    double *sa = (double *)malloc(sizeof(double) * (size_t)(T * N + 1));
    double *dS = (double *)malloc(sizeof(double) * (NN + 3 * (size_t)N));
    double *wd = dS + NN, *dsa = wd + N, *sig = dsa + N;
    if (s0) memcpy(states, s0 + bh * (int64_t)NN, sizeof(double) * NN);
    else memset(states, 0, sizeof(double) * NN);
    for (int64_t t = 0; t < T; ++t) {
      const int64_t base = tok(T, H, N, bi, t, hi);
      const double *Sp = states + (size_t)t * NN;
      double *Sn = states + (size_t)(t + 1) * NN;
      for (int64_t i = 0; i < N; ++i)
        wd[i] = exp(W_SCALE_D * sigmoid_d(w[base + i]));
      for (int64_t j = 0; j < N; ++j) {
        double acc = 0.0;
        for (int64_t i = 0; i < N; ++i) acc += Sp[j * N + i] * a[base + i];
        sa[t * N + j] = acc;
        for (int64_t i = 0; i < N; ++i)
          Sn[j * N + i] = Sp[j * N + i] * wd[i] + acc * b[base + i] +
                          v[base + j] * k[base + i];
      }
    }
    if (ds_T) memcpy(dS, ds_T + bh * (int64_t)NN, sizeof(double) * NN);
    else memset(dS, 0, sizeof(double) * NN);
    for (int64_t t = T - 1; t >= 0; --t) {
      const int64_t base = tok(T, H, N, bi, t, hi);
      const double *Sp = states + (size_t)t * NN;       /* S_{t-1} */
      const double *Sc = states + (size_t)(t + 1) * NN; /* S_t */
      for (int64_t i = 0; i < N; ++i) {
        sig[i] = sigmoid_d(w[base + i]);
        wd[i] = exp(W_SCALE_D * sig[i]);
      }
      /* y_t = S_t r_t  ->  dS_t += dy_t r_t^T, dr_t = S_t^T dy_t */
      for (int64_t j = 0; j < N; ++j)
        for (int64_t i = 0; i < N; ++i)
          dS[j * N + i] += dy[base + j] * r[base + i];
      for (int64_t i = 0; i < N; ++i) {
        double acc = 0.0;
        for (int64_t j = 0; j < N; ++j) acc += Sc[j * N + i] * dy[base + j];
        dr[base + i] = acc;
      }
      /* S_t = S_{t-1} diag(w) + sa b^T + v k^T */
      for (int64_t i = 0; i < N; ++i) {
        double gw = 0.0, gk = 0.0, gb = 0.0;
        for (int64_t j = 0; j < N; ++j) {
          gw += dS[j * N + i] * Sp[j * N + i];
          gk += dS[j * N + i] * v[base + j];
          gb += dS[j * N + i] * sa[t * N + j];
        }
        dw[base + i] = W_SCALE_D * gw * wd[i] * sig[i] * (1.0 - sig[i]);
        dk[base + i] = gk;
        db[base + i] = gb;
      }
      for (int64_t j = 0; j < N; ++j) {
        double gv = 0.0, gs = 0.0;
        for (int64_t i = 0; i < N; ++i) {
          gv += dS[j * N + i] * k[base + i];
          gs += dS[j * N + i] * b[base + i];
        }
        dv[base + j] = gv;
        dsa[j] = gs;
      }
      /* sa_t = S_{t-1} a_t */
      for (int64_t i = 0; i < N; ++i) {
        double acc = 0.0;
        for (int64_t j = 0; j < N; ++j) acc += Sp[j * N + i] * dsa[j];
        da[base + i] = acc;
      }
      for (int64_t j = 0; j < N; ++j)
        for (int64_t i = 0; i < N; ++i)
          dS[j * N + i] = dS[j * N + i] * wd[i] + dsa[j] * a[base + i];
    }
    if (ds0) memcpy(ds0 + bh * (int64_t)NN, dS, sizeof(double) * NN);
    free(states);
    free(sa);
    free(dS);
  }
  return 0;
}

/* ------------------------------------------------------------------------ */
/* inference, wkv7_infer/kernel.rs:8-114                                     */
/* ------------------------------------------------------------------------ */
float wkv7o_dither(uint32_t seed) {
  const uint32_t mixed = seed * ROTATOR1; /* wrapping u32 multiply */
  int32_t mixed_signed;
  memcpy(&mixed_signed, &mixed, sizeof mixed_signed);
  return (float)mixed_signed * TWO_TO_NEG_41;
}

int wkv7o_infer_f32(int64_t Ba, int64_t T, int64_t H, int64_t N,
                    int64_t full_batch, const float *w, const float *r,
                    const float *k, const float *v, const float *a,
                    const float *b, const int32_t *batch_ids, float *state,
                    const float *mask, const uint32_t *elapsed_t,
                    int use_dither, float *y) {
  if (bad_shape(Ba, T, H, N) || full_batch < 0) return -1;
  for (int64_t bi = 0; bi < Ba; ++bi)
    if (batch_ids[bi] < 0 || batch_ids[bi] >= full_batch) return -2;
  float *sw = (float *)malloc(sizeof(float) * (size_t)N);
  for (int64_t bi = 0; bi < Ba; ++bi) {
    const int64_t slot = batch_ids[bi];
    const uint32_t e_t = elapsed_t ? elapsed_t[slot] : 0u;
    for (int64_t hi = 0; hi < H; ++hi) {
      float *S = state + (slot * H + hi) * N * N;
      uint32_t valid_t = 0;
      for (int64_t t = 0; t < T; ++t) {
        const int64_t base = tok(T, H, N, bi, t, hi);
        if (mask && mask[bi * T + t] == 0.0f) {
          for (int64_t j = 0; j < N; ++j) y[base + j] = 0.0f;
          continue;
        }
        for (int64_t i = 0; i < N; ++i) {
          const float w_sig = 1.0f / (1.0f + expf(-w[base + i]));
          float wd = expf(W_SCALE_F * w_sig);
          if (use_dither) wd += wkv7o_dither(e_t + valid_t);
          sw[i] = wd;
        }
        for (int64_t j = 0; j < N; ++j) {
          float *row = S + j * N;
          float removal_state = 0.0f;
          for (int64_t i = 0; i < N; ++i) removal_state += a[base + i] * row[i];
          const float vj = v[base + j];
          float yy = 0.0f;
          for (int64_t i = 0; i < N; ++i) {
            row[i] = row[i] * sw[i] + removal_state * b[base + i] +
                     k[base + i] * vj;
            yy += row[i] * r[base + i];
          }
          y[base + j] = yy;
        }
        valid_t += 1u;
      }
    }
  }
  free(sw);
  return 0;
}

/* ------------------------------------------------------------------------ */
/* inference with F = bf16, wkv7_infer/kernel.rs:15-114                      */
/* ------------------------------------------------------------------------ */
float wkv7o_round_bf16(float x) {
  uint32_t u;
  memcpy(&u, &x, sizeof u);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu) != 0u) {
    u |= 0x00400000u; /* quiet NaN, payload kept in the upper half */
  } else {
    u += 0x7fffu + ((u >> 16) & 1u); /* ties to even; overflow goes to inf */
  }
  u &= 0xffff0000u;
  memcpy(&x, &u, sizeof x);
  return x;
}

/* One F = bf16 operation: the fp32 result of two bf16 operands, rounded to
 * bf16. A product of two bf16 values is exact in fp32; a sum is rounded twice
 * (fp32, then bf16), which equals one rounding because fp32 carries more than
 * 2 * 8 + 2 significand bits. */
#define BF(x) wkv7o_round_bf16(x)

int wkv7o_infer_bf16(int64_t Ba, int64_t T, int64_t H, int64_t N,
                     int64_t full_batch, const float *w, const float *r,
                     const float *k, const float *v, const float *a,
                     const float *b, const int32_t *batch_ids, float *state,
                     const float *mask, const uint32_t *elapsed_t,
                     int use_dither, float *y) {
  if (bad_shape(Ba, T, H, N) || full_batch < 0) return -1;
  for (int64_t bi = 0; bi < Ba; ++bi)
    if (batch_ids[bi] < 0 || batch_ids[bi] >= full_batch) return -2;
  float *sw = (float *)malloc(sizeof(float) * (size_t)N);
  for (int64_t bi = 0; bi < Ba; ++bi) {
    const int64_t slot = batch_ids[bi];
    const uint32_t e_t = elapsed_t ? elapsed_t[slot] : 0u;
    for (int64_t hi = 0; hi < H; ++hi) {
      float *S = state + (slot * H + hi) * N * N;
      uint32_t valid_t = 0;
      for (int64_t t = 0; t < T; ++t) {
        const int64_t base = tok(T, H, N, bi, t, hi);
        /* kernel.rs:59-62: the mask is an F value compared with 0 */
        if (mask && mask[bi * T + t] == 0.0f) {
          for (int64_t j = 0; j < N; ++j) y[base + j] = 0.0f;
          continue;
        }
        /* kernel.rs:71-78: decay in fp32, dither added in fp32, one cast to F */
        for (int64_t i = 0; i < N; ++i) {
          const float w_sig = 1.0f / (1.0f + expf(-w[base + i]));
          float wd = expf(W_SCALE_F * w_sig);
          if (use_dither) wd += wkv7o_dither(e_t + valid_t);
          sw[i] = BF(wd);
        }
        for (int64_t j = 0; j < N; ++j) {
          float *row = S + j * N;
          /* kernel.rs:81-85: removal_state += removal[i] * state[i], in F */
          float removal_state = 0.0f;
          for (int64_t i = 0; i < N; ++i)
            removal_state = BF(removal_state + BF(a[base + i] * row[i]));
          const float vj = v[base + j];
          float yy = 0.0f;
          /* kernel.rs:90-96: state[i] * w[i] + removal_state * b[i] + k[i] * v,
           * left to right, then y += state[i] * r[i], all in F */
          for (int64_t i = 0; i < N; ++i) {
            const float p0 = BF(row[i] * sw[i]);
            const float p1 = BF(removal_state * b[base + i]);
            const float p2 = BF(k[base + i] * vj);
            row[i] = BF(BF(p0 + p1) + p2);
            yy = BF(yy + BF(row[i] * r[base + i]));
          }
          y[base + j] = yy;
        }
        valid_t += 1u;
      }
    }
  }
  free(sw);
  return 0;
}
