// WKV7 backward recurrence for gfx950, all six input gradients and the
// initial-state gradient in one pass.
//
// Semantics: /root/reference/crates/rwkv-nn/src/kernels/wkv7_common/kernel.rs:116-308
// (wkv7_backward_kernel), per (batch b, head h), t = T-1..0, dS = ds_T or 0:
//   if (t+1) % C == 0: S = checkpoint[t / C]           (exact reload, :210-228)
//   dr_t   = S_t^T dy_t                                             (:230-237)
//   S_{t-1} = (S_t - v k^T - sa b^T) / w~    (rebuild by reversal,  :239-246)
//   dS    += dy r^T                                                 (:248-249)
//   dw~_i  = sum_j dS[j,i] S_{t-1}[j,i];  dk = dS^T v;  db = dS^T sa (:258-265)
//   dv     = dS k;  dsa = dS b
//   dw     = W_SCALE * dw~ * w~ * sigmoid(w) * (1 - sigmoid(w))    (:267-271)
//   da     = S_{t-1}^T dsa                                          (:280-287)
//   dS     = dS diag(w~) + dsa a^T                                  (:289-296)
//   ds0    = dS after t = 0                                         (:299-307)
//
// Design. One 256-thread workgroup per (b, h). Every thread has an own index
// e = 16*wave + 4*g + lo and a segment hi (see wkv7_device.hpp) and plays two
// roles at once:
//   row role:    dSr[m] = dS[e][16*hi+m]   -> row sums dv_e and dsa_e
//   column role: Sc[m]  = S[16*hi+m][e], dSc[m] = dS[16*hi+m][e]
//                -> column sums dr_e, dw~_e, dk_e, db_e, da_e
// so every sum is 16 in-lane products plus a 2-step DPP reduction over the
// four segments, and the operand that varies along the summed index always
// arrives as a DPP quad broadcast. Keeping dS twice (row and column layout)
// costs 3 instructions per element per step; the alternative, cross-wave
// reductions of the five column sums, costs more. The only data exchanged
// between waves is dsa (64 floats, needed by the column role): one LDS vector
// and one barrier per step, whose latency is covered by the column-role work
// scheduled between the write and the barrier.
#include "wkv7_device.hpp"
#include "wkv7_launch.hpp"

namespace wkv7 {
namespace {

constexpr int kTile = 16;   // timesteps per LDS tile

// LDS vectors per timestep (fp32)
enum {
  V_R = 0, V_K, V_B, V_W, V_A,   // key-indexed (row role broadcasts these)
  V_DY, V_V, V_SA,               // value-indexed (column role broadcasts these)
  V_IW,                          // 1 / w~
  V_DWF,                         // W_SCALE * w~ * sig * (1 - sig)
  V_COUNT
};
// staged outputs per timestep
enum { O_DW = 0, O_DR, O_DK, O_DV, O_DA, O_DB, O_COUNT };

// Row role, 8 columns m = 4*S0 .. 4*S0+7 (quad lanes S0, S0+1):
//   dSr[m] += dy_e * r[m];  dv += dSr[m] * k[m];  dsa += dSr[m] * b[m]
#define WKV7_DEF_ROW1(S0, S1)                                                        \
  __device__ __forceinline__ void row1_q##S0(float* d, float& v0, float& v1,         \
                                             float& s0, float& s1, float4 r,          \
                                             float4 k, float4 b, float dye) {         \
    asm("s_nop 1\n\t"                                                                 \
        "v_fmac_f32_dpp %0, %12, %24" WKV7_QP(S0)                                     \
        "v_fmac_f32_dpp %1, %13, %24" WKV7_QP(S0)                                     \
        "v_fmac_f32_dpp %2, %14, %24" WKV7_QP(S0)                                     \
        "v_fmac_f32_dpp %3, %15, %24" WKV7_QP(S0)                                     \
        "v_fmac_f32_dpp %4, %12, %24" WKV7_QP(S1)                                     \
        "v_fmac_f32_dpp %5, %13, %24" WKV7_QP(S1)                                     \
        "v_fmac_f32_dpp %6, %14, %24" WKV7_QP(S1)                                     \
        "v_fmac_f32_dpp %7, %15, %24" WKV7_QP(S1)                                     \
        "v_fmac_f32_dpp %8, %16, %0" WKV7_QP(S0)                                      \
        "v_fmac_f32_dpp %9, %17, %1" WKV7_QP(S0)                                      \
        "v_fmac_f32_dpp %8, %18, %2" WKV7_QP(S0)                                      \
        "v_fmac_f32_dpp %9, %19, %3" WKV7_QP(S0)                                      \
        "v_fmac_f32_dpp %8, %16, %4" WKV7_QP(S1)                                      \
        "v_fmac_f32_dpp %9, %17, %5" WKV7_QP(S1)                                      \
        "v_fmac_f32_dpp %8, %18, %6" WKV7_QP(S1)                                      \
        "v_fmac_f32_dpp %9, %19, %7" WKV7_QP(S1)                                      \
        "v_fmac_f32_dpp %10, %20, %0" WKV7_QP(S0)                                     \
        "v_fmac_f32_dpp %11, %21, %1" WKV7_QP(S0)                                     \
        "v_fmac_f32_dpp %10, %22, %2" WKV7_QP(S0)                                     \
        "v_fmac_f32_dpp %11, %23, %3" WKV7_QP(S0)                                     \
        "v_fmac_f32_dpp %10, %20, %4" WKV7_QP(S1)                                     \
        "v_fmac_f32_dpp %11, %21, %5" WKV7_QP(S1)                                     \
        "v_fmac_f32_dpp %10, %22, %6" WKV7_QP(S1)                                     \
        "v_fmac_f32_dpp %11, %23, %7" WKV7_QP(S1)                                     \
        : "+v"(d[0]), "+v"(d[1]), "+v"(d[2]), "+v"(d[3]), "+v"(d[4]), "+v"(d[5]),    \
          "+v"(d[6]), "+v"(d[7]), "+v"(v0), "+v"(v1), "+v"(s0), "+v"(s1)              \
        : "v"(r.x), "v"(r.y), "v"(r.z), "v"(r.w), "v"(k.x), "v"(k.y), "v"(k.z),       \
          "v"(k.w), "v"(b.x), "v"(b.y), "v"(b.z), "v"(b.w), "v"(dye));                \
  }
WKV7_DEF_ROW1(0, 1)
WKV7_DEF_ROW1(2, 3)

// Row role after dsa is known: dSr[m] = dSr[m] * w~[m] + dsa_e * a[m]
#define WKV7_DEF_ROW2(S0, S1)                                                        \
  __device__ __forceinline__ void row2_q##S0(float* d, float4 w, float4 a,           \
                                             float dsae) {                            \
    asm("s_nop 1\n\t"                                                                 \
        "v_mul_f32_dpp %0, %8, %0" WKV7_QP(S0)                                        \
        "v_mul_f32_dpp %1, %9, %1" WKV7_QP(S0)                                        \
        "v_mul_f32_dpp %2, %10, %2" WKV7_QP(S0)                                       \
        "v_mul_f32_dpp %3, %11, %3" WKV7_QP(S0)                                       \
        "v_mul_f32_dpp %4, %8, %4" WKV7_QP(S1)                                        \
        "v_mul_f32_dpp %5, %9, %5" WKV7_QP(S1)                                        \
        "v_mul_f32_dpp %6, %10, %6" WKV7_QP(S1)                                       \
        "v_mul_f32_dpp %7, %11, %7" WKV7_QP(S1)                                       \
        "v_fmac_f32_dpp %0, %12, %16" WKV7_QP(S0)                                     \
        "v_fmac_f32_dpp %1, %13, %16" WKV7_QP(S0)                                     \
        "v_fmac_f32_dpp %2, %14, %16" WKV7_QP(S0)                                     \
        "v_fmac_f32_dpp %3, %15, %16" WKV7_QP(S0)                                     \
        "v_fmac_f32_dpp %4, %12, %16" WKV7_QP(S1)                                     \
        "v_fmac_f32_dpp %5, %13, %16" WKV7_QP(S1)                                     \
        "v_fmac_f32_dpp %6, %14, %16" WKV7_QP(S1)                                     \
        "v_fmac_f32_dpp %7, %15, %16" WKV7_QP(S1)                                     \
        : "+v"(d[0]), "+v"(d[1]), "+v"(d[2]), "+v"(d[3]), "+v"(d[4]), "+v"(d[5]),    \
          "+v"(d[6]), "+v"(d[7])                                                      \
        : "v"(w.x), "v"(w.y), "v"(w.z), "v"(w.w), "v"(a.x), "v"(a.y), "v"(a.z),       \
          "v"(a.w), "v"(dsae));                                                       \
  }
WKV7_DEF_ROW2(0, 1)
WKV7_DEF_ROW2(2, 3)

// Column role, first half, 4 rows m = 4*S .. 4*S+3 (quad lane S):
//   dr  += S_t[m] * dy[m]
//   S[m] = ((S[m] - v[m] * k_e) - sa[m] * b_e) * (1/w~_e)   -> S_{t-1}
//   dSc[m] += dy[m] * r_e
//   dw~ += dSc[m] * S[m];  dk += dSc[m] * v[m];  db += dSc[m] * sa[m]
#define WKV7_DEF_COL1(S)                                                             \
  __device__ __forceinline__ void col1_q##S(float* c, float* d, float* acc,          \
                                            float4 dy, float4 v, float4 sa,           \
                                            float ke, float be, float iwe,            \
                                            float re) {                               \
    asm("s_nop 1\n\t"                                                                 \
        "v_fmac_f32_dpp %8, %16, %0" WKV7_QP(S)                                       \
        "v_fmac_f32_dpp %9, %17, %1" WKV7_QP(S)                                       \
        "v_fmac_f32_dpp %8, %18, %2" WKV7_QP(S)                                       \
        "v_fmac_f32_dpp %9, %19, %3" WKV7_QP(S)                                       \
        "v_fmac_f32_dpp %0, -%20, %28" WKV7_QP(S)                                     \
        "v_fmac_f32_dpp %1, -%21, %28" WKV7_QP(S)                                     \
        "v_fmac_f32_dpp %2, -%22, %28" WKV7_QP(S)                                     \
        "v_fmac_f32_dpp %3, -%23, %28" WKV7_QP(S)                                     \
        "v_fmac_f32_dpp %0, -%24, %29" WKV7_QP(S)                                     \
        "v_fmac_f32_dpp %1, -%25, %29" WKV7_QP(S)                                     \
        "v_fmac_f32_dpp %2, -%26, %29" WKV7_QP(S)                                     \
        "v_fmac_f32_dpp %3, -%27, %29" WKV7_QP(S)                                     \
        "v_mul_f32_e32 %0, %30, %0\n\t"                                               \
        "v_mul_f32_e32 %1, %30, %1\n\t"                                               \
        "v_mul_f32_e32 %2, %30, %2\n\t"                                               \
        "v_mul_f32_e32 %3, %30, %3\n\t"                                               \
        "v_fmac_f32_dpp %4, %16, %31" WKV7_QP(S)                                      \
        "v_fmac_f32_dpp %5, %17, %31" WKV7_QP(S)                                      \
        "v_fmac_f32_dpp %6, %18, %31" WKV7_QP(S)                                      \
        "v_fmac_f32_dpp %7, %19, %31" WKV7_QP(S)                                      \
        "v_fmac_f32_e32 %10, %4, %0\n\t"                                              \
        "v_fmac_f32_e32 %11, %5, %1\n\t"                                              \
        "v_fmac_f32_e32 %10, %6, %2\n\t"                                              \
        "v_fmac_f32_e32 %11, %7, %3\n\t"                                              \
        "v_fmac_f32_dpp %12, %20, %4" WKV7_QP(S)                                      \
        "v_fmac_f32_dpp %13, %21, %5" WKV7_QP(S)                                      \
        "v_fmac_f32_dpp %12, %22, %6" WKV7_QP(S)                                      \
        "v_fmac_f32_dpp %13, %23, %7" WKV7_QP(S)                                      \
        "v_fmac_f32_dpp %14, %24, %4" WKV7_QP(S)                                      \
        "v_fmac_f32_dpp %15, %25, %5" WKV7_QP(S)                                      \
        "v_fmac_f32_dpp %14, %26, %6" WKV7_QP(S)                                      \
        "v_fmac_f32_dpp %15, %27, %7" WKV7_QP(S)                                      \
        : "+v"(c[0]), "+v"(c[1]), "+v"(c[2]), "+v"(c[3]), "+v"(d[0]), "+v"(d[1]),    \
          "+v"(d[2]), "+v"(d[3]), "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]),           \
          "+v"(acc[3]), "+v"(acc[4]), "+v"(acc[5]), "+v"(acc[6]), "+v"(acc[7])        \
        : "v"(dy.x), "v"(dy.y), "v"(dy.z), "v"(dy.w), "v"(v.x), "v"(v.y), "v"(v.z),   \
          "v"(v.w), "v"(sa.x), "v"(sa.y), "v"(sa.z), "v"(sa.w), "v"(ke), "v"(be),     \
          "v"(iwe), "v"(re));                                                         \
  }
WKV7_DEF_COL1(0)
WKV7_DEF_COL1(1)
WKV7_DEF_COL1(2)
WKV7_DEF_COL1(3)

// Column role, second half, 8 rows m = 4*S0 .. 4*S0+7:
//   da += S_{t-1}[m] * dsa[m];   dSc[m] = dSc[m] * w~_e + dsa[m] * a_e
#define WKV7_DEF_COL2(S0, S1)                                                        \
  __device__ __forceinline__ void col2_q##S0(const float* c, float* d, float& a0,    \
                                             float& a1, float4 dsa, float we,         \
                                             float ae) {                              \
    asm("s_nop 1\n\t"                                                                 \
        "v_fmac_f32_dpp %8, %10, %16" WKV7_QP(S0)                                     \
        "v_fmac_f32_dpp %9, %11, %17" WKV7_QP(S0)                                     \
        "v_fmac_f32_dpp %8, %12, %18" WKV7_QP(S0)                                     \
        "v_fmac_f32_dpp %9, %13, %19" WKV7_QP(S0)                                     \
        "v_fmac_f32_dpp %8, %10, %20" WKV7_QP(S1)                                     \
        "v_fmac_f32_dpp %9, %11, %21" WKV7_QP(S1)                                     \
        "v_fmac_f32_dpp %8, %12, %22" WKV7_QP(S1)                                     \
        "v_fmac_f32_dpp %9, %13, %23" WKV7_QP(S1)                                     \
        "v_mul_f32_e32 %0, %14, %0\n\t"                                               \
        "v_mul_f32_e32 %1, %14, %1\n\t"                                               \
        "v_mul_f32_e32 %2, %14, %2\n\t"                                               \
        "v_mul_f32_e32 %3, %14, %3\n\t"                                               \
        "v_mul_f32_e32 %4, %14, %4\n\t"                                               \
        "v_mul_f32_e32 %5, %14, %5\n\t"                                               \
        "v_mul_f32_e32 %6, %14, %6\n\t"                                               \
        "v_mul_f32_e32 %7, %14, %7\n\t"                                               \
        "v_fmac_f32_dpp %0, %10, %15" WKV7_QP(S0)                                     \
        "v_fmac_f32_dpp %1, %11, %15" WKV7_QP(S0)                                     \
        "v_fmac_f32_dpp %2, %12, %15" WKV7_QP(S0)                                     \
        "v_fmac_f32_dpp %3, %13, %15" WKV7_QP(S0)                                     \
        "v_fmac_f32_dpp %4, %10, %15" WKV7_QP(S1)                                     \
        "v_fmac_f32_dpp %5, %11, %15" WKV7_QP(S1)                                     \
        "v_fmac_f32_dpp %6, %12, %15" WKV7_QP(S1)                                     \
        "v_fmac_f32_dpp %7, %13, %15" WKV7_QP(S1)                                     \
        : "+v"(d[0]), "+v"(d[1]), "+v"(d[2]), "+v"(d[3]), "+v"(d[4]), "+v"(d[5]),    \
          "+v"(d[6]), "+v"(d[7]), "+v"(a0), "+v"(a1)                                  \
        : "v"(dsa.x), "v"(dsa.y), "v"(dsa.z), "v"(dsa.w), "v"(we), "v"(ae),           \
          "v"(c[0]), "v"(c[1]), "v"(c[2]), "v"(c[3]), "v"(c[4]), "v"(c[5]),           \
          "v"(c[6]), "v"(c[7]));                                                      \
  }
WKV7_DEF_COL2(0, 1)
WKV7_DEF_COL2(2, 3)

struct StepOps {
  float4 r, k, b, w, a;      // key-indexed, quad-distributed
  float4 dy, v, sa;          // value-indexed, quad-distributed
  float re, ke, be, we, ae, dye, iwe;   // own index e
};

template <typename Tin>
struct BwdParams {
  const Tin *w, *r, *k, *v, *a, *b, *dy;
  const float* ckpt;
  const float* sa;
  const float* dsT;
  Tin *dw, *dr, *dk, *dv, *da, *db;
  float* ds0;
  int T, H, C;
};

template <typename Tin>
__global__ __launch_bounds__(kThreads) void wkv7_bwd_kernel(BwdParams<Tin> p) {
  __shared__ float4 tile[2][V_COUNT][kTile][16];   // 80 KiB
  __shared__ float ost[2][O_COUNT][kTile][kHead];  // 48 KiB
  __shared__ float4 dsab[2][16];                   // dsa of the step, by parity

  const int h = blockIdx.x, bi = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int L = lane & 15, g = lane >> 4, lo = L & 3, hi = L >> 2;
  const int e = 16 * wave + 4 * g + lo;
  const int sl = tid >> 4, pp = tid & 15;

  const int T = p.T, C = p.C;
  const int64_t bh = (int64_t)bi * p.H + h;
  const int64_t tstride = (int64_t)p.H * kHead;
  const int64_t tok0 = ((int64_t)bi * T * p.H + h) * kHead;

  float dSr[16], Sc[16], dSc[16], Pf[16];
#pragma unroll
  for (int m = 0; m < 16; ++m) Sc[m] = 0.0f;
  if (p.dsT) {
    const float* g0 = p.dsT + bh * (kHead * kHead);
    const float4* row = reinterpret_cast<const float4*>(g0 + e * kHead + 16 * hi);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float4 x = row[q];
      dSr[4 * q] = x.x; dSr[4 * q + 1] = x.y; dSr[4 * q + 2] = x.z; dSr[4 * q + 3] = x.w;
    }
#pragma unroll
    for (int m = 0; m < 16; ++m) dSc[m] = g0[(16 * hi + m) * kHead + e];
  } else {
#pragma unroll
    for (int m = 0; m < 16; ++m) { dSr[m] = 0.0f; dSc[m] = 0.0f; }
  }

  // checkpoint c holds S after step c*C + C - 1, key-major: row e of the
  // checkpoint is column e of S.
  const int64_t nchunks = T / C;
  const float* ckpt_bh = p.ckpt + bh * nchunks * (kHead * kHead) + e * kHead + 16 * hi;
  auto ckload = [&](int64_t c) {
    const float4* src = reinterpret_cast<const float4*>(ckpt_bh + c * (kHead * kHead));
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float4 x = src[q];
      Pf[4 * q] = x.x; Pf[4 * q + 1] = x.y; Pf[4 * q + 2] = x.z; Pf[4 * q + 3] = x.w;
    }
  };
  int64_t next_chunk = nchunks - 1;
  if (next_chunk >= 0) ckload(next_chunk);

  typedef Io<Tin> io;
  typename io::raw pre[7];
  float4 pre_sa;
  auto gload = [&](int t0) {
    if (t0 + sl < T) {
      const int64_t off = tok0 + (int64_t)(t0 + sl) * tstride + 4 * pp;
      pre[0] = io::load(p.w + off);
      pre[1] = io::load(p.r + off);
      pre[2] = io::load(p.k + off);
      pre[3] = io::load(p.v + off);
      pre[4] = io::load(p.a + off);
      pre[5] = io::load(p.b + off);
      pre[6] = io::load(p.dy + off);
      pre_sa = *reinterpret_cast<const float4*>(p.sa + off);
    }
  };
  auto lstore = [&](int buf, int t0) {
    if (t0 + sl < T) {
      const float4 x = io::widen(pre[0]);
      float4 w, iw, dwf;
      const float xs[4] = {x.x, x.y, x.z, x.w};
      float ws[4], iws[4], dws[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float sig = sigmoid_f(xs[c]);
        ws[c] = decay_f(sig);
        iws[c] = 1.0f / ws[c];
        dws[c] = kWScale * ws[c] * sig * (1.0f - sig);
      }
      w = make_float4(ws[0], ws[1], ws[2], ws[3]);
      iw = make_float4(iws[0], iws[1], iws[2], iws[3]);
      dwf = make_float4(dws[0], dws[1], dws[2], dws[3]);
      tile[buf][V_W][sl][pp] = w;
      tile[buf][V_IW][sl][pp] = iw;
      tile[buf][V_DWF][sl][pp] = dwf;
      tile[buf][V_R][sl][pp] = io::widen(pre[1]);
      tile[buf][V_K][sl][pp] = io::widen(pre[2]);
      tile[buf][V_V][sl][pp] = io::widen(pre[3]);
      tile[buf][V_A][sl][pp] = io::widen(pre[4]);
      tile[buf][V_B][sl][pp] = io::widen(pre[5]);
      tile[buf][V_DY][sl][pp] = io::widen(pre[6]);
      tile[buf][V_SA][sl][pp] = pre_sa;
    }
  };
  auto lread = [&](int buf, int s) {
    StepOps o;
    o.r = tile[buf][V_R][s][L];
    o.k = tile[buf][V_K][s][L];
    o.b = tile[buf][V_B][s][L];
    o.w = tile[buf][V_W][s][L];
    o.a = tile[buf][V_A][s][L];
    o.dy = tile[buf][V_DY][s][L];
    o.v = tile[buf][V_V][s][L];
    o.sa = tile[buf][V_SA][s][L];
    o.re = reinterpret_cast<const float*>(tile[buf][V_R][s])[e];
    o.ke = reinterpret_cast<const float*>(tile[buf][V_K][s])[e];
    o.be = reinterpret_cast<const float*>(tile[buf][V_B][s])[e];
    o.we = reinterpret_cast<const float*>(tile[buf][V_W][s])[e];
    o.ae = reinterpret_cast<const float*>(tile[buf][V_A][s])[e];
    o.dye = reinterpret_cast<const float*>(tile[buf][V_DY][s])[e];
    o.iwe = reinterpret_cast<const float*>(tile[buf][V_IW][s])[e];
    return o;
  };

  int until_reload = 0;   // steps until the next checkpoint reload
  int parity = 0;

  auto step = [&](const StepOps& o, int buf, int s) {
    if (until_reload == 0) {   // (t + 1) % C == 0
      until_reload = C;
#pragma unroll
      for (int m = 0; m < 16; ++m) Sc[m] = Pf[m];
      --next_chunk;
      if (next_chunk >= 0) ckload(next_chunk);
    }
    --until_reload;

    // row role: dS row += dy_e r^T; dv_e, dsa_e
    float v0 = 0.0f, v1 = 0.0f, s0 = 0.0f, s1 = 0.0f;
    row1_q0(dSr, v0, v1, s0, s1, o.r, o.k, o.b, o.dye);
    row1_q2(dSr + 8, v0, v1, s0, s1, o.r, o.k, o.b, o.dye);
    const float dv = seg_sum(v0 + v1);
    const float dsa = seg_sum(s0 + s1);
    reinterpret_cast<float*>(dsab[parity])[e] = dsa;
    ost[buf][O_DV][s][e] = dv;

    // column role: dr (from S_t), rebuild S_{t-1}, dS col += dy r_e; dw~, dk, db
    float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    col1_q0(Sc, dSc, acc, o.dy, o.v, o.sa, o.ke, o.be, o.iwe, o.re);
    col1_q1(Sc + 4, dSc + 4, acc, o.dy, o.v, o.sa, o.ke, o.be, o.iwe, o.re);
    col1_q2(Sc + 8, dSc + 8, acc, o.dy, o.v, o.sa, o.ke, o.be, o.iwe, o.re);
    col1_q3(Sc + 12, dSc + 12, acc, o.dy, o.v, o.sa, o.ke, o.be, o.iwe, o.re);
    ost[buf][O_DR][s][e] = seg_sum(acc[0] + acc[1]);
    ost[buf][O_DW][s][e] = seg_sum(acc[2] + acc[3]);
    ost[buf][O_DK][s][e] = seg_sum(acc[4] + acc[5]);
    ost[buf][O_DB][s][e] = seg_sum(acc[6] + acc[7]);

    __syncthreads();   // dsa of every row visible
    const float4 dsa4 = dsab[parity][L];
    parity ^= 1;

    row2_q0(dSr, o.w, o.a, dsa);
    row2_q2(dSr + 8, o.w, o.a, dsa);
    float a0 = 0.0f, a1 = 0.0f;
    col2_q0(Sc, dSc, a0, a1, dsa4, o.we, o.ae);
    col2_q2(Sc + 8, dSc + 8, a0, a1, dsa4, o.we, o.ae);
    ost[buf][O_DA][s][e] = seg_sum(a0 + a1);
  };

  const int ntiles = (T + kTile - 1) / kTile;
  if (ntiles > 0) {
    gload((ntiles - 1) * kTile);
    lstore((ntiles - 1) & 1, (ntiles - 1) * kTile);
  }
  __syncthreads();

  for (int ti = ntiles - 1; ti >= 0; --ti) {
    const int buf = ti & 1;
    const int t0 = ti * kTile;
    const int nst = min(kTile, T - t0);
    if (ti > 0) gload(t0 - kTile);

    StepOps A = lread(buf, nst - 1);
    int s = nst - 1;
    for (; s >= 1; s -= 2) {
      const StepOps Bo = lread(buf, s - 1);
      step(A, buf, s);
      A = lread(buf, max(s - 2, 0));
      step(Bo, buf, s - 1);
    }
    if (s == 0) step(A, buf, 0);

    if (ti > 0) lstore(buf ^ 1, t0 - kTile);
    __syncthreads();
    if (sl < nst) {
      const int64_t off = tok0 + (int64_t)(t0 + sl) * tstride + 4 * pp;
      float4 dw = reinterpret_cast<const float4*>(ost[buf][O_DW][sl])[pp];
      const float4 f = tile[buf][V_DWF][sl][pp];
      dw.x *= f.x; dw.y *= f.y; dw.z *= f.z; dw.w *= f.w;
      io::store(p.dw + off, dw);
      io::store(p.dr + off, reinterpret_cast<const float4*>(ost[buf][O_DR][sl])[pp]);
      io::store(p.dk + off, reinterpret_cast<const float4*>(ost[buf][O_DK][sl])[pp]);
      io::store(p.dv + off, reinterpret_cast<const float4*>(ost[buf][O_DV][sl])[pp]);
      io::store(p.da + off, reinterpret_cast<const float4*>(ost[buf][O_DA][sl])[pp]);
      io::store(p.db + off, reinterpret_cast<const float4*>(ost[buf][O_DB][sl])[pp]);
    }
  }

  if (p.ds0) {
    float4* dst = reinterpret_cast<float4*>(p.ds0 + (bh * kHead + e) * kHead + 16 * hi);
#pragma unroll
    for (int q = 0; q < 4; ++q)
      dst[q] = make_float4(dSr[4 * q], dSr[4 * q + 1], dSr[4 * q + 2], dSr[4 * q + 3]);
  }
}

template <typename Tin>
hipError_t launch_bwd_t(const BackwardDesc& d, hipStream_t stream) {
  BwdParams<Tin> p;
  p.w = static_cast<const Tin*>(d.w);
  p.r = static_cast<const Tin*>(d.r);
  p.k = static_cast<const Tin*>(d.k);
  p.v = static_cast<const Tin*>(d.v);
  p.a = static_cast<const Tin*>(d.a);
  p.b = static_cast<const Tin*>(d.b);
  p.dy = static_cast<const Tin*>(d.dy);
  p.ckpt = d.ckpt;
  p.sa = d.sa;
  p.dsT = d.dsT;
  p.dw = static_cast<Tin*>(d.dw);
  p.dr = static_cast<Tin*>(d.dr);
  p.dk = static_cast<Tin*>(d.dk);
  p.dv = static_cast<Tin*>(d.dv);
  p.da = static_cast<Tin*>(d.da);
  p.db = static_cast<Tin*>(d.db);
  p.ds0 = d.ds0;
  p.T = d.T;
  p.H = d.H;
  p.C = d.C;
  hipLaunchKernelGGL(wkv7_bwd_kernel<Tin>, dim3(d.H, d.B, 1), dim3(kThreads, 1, 1), 0, stream, p);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_backward(const BackwardDesc& d, hipStream_t stream) {
  if (d.B == 0 || d.H == 0) return hipSuccess;
  return d.dtype == Dtype::BF16 ? launch_bwd_t<bf16_t>(d, stream) : launch_bwd_t<float>(d, stream);
}

}  // namespace wkv7
