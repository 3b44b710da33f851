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
// Design. One 512-thread workgroup per (b, h). Thread tid = 16*q + L plays two
// roles on two transposed 2x4 blocks (layout in wkv7_device.hpp):
//   row role:    dSr[d][c] = dS[2q+d][4L+c]   -> row sums dv, dsa of rows 2q, 2q+1
//   column role: Sc[c][d]  = S[4L+c][2q+d],
//                dSc[c][d] = dS[4L+c][2q+d]   -> column sums dr, dw~, dk, db, da
//                                                of columns 2q, 2q+1
// The sixteen lanes of a DPP row (same q) span all 64 columns in the row role
// and all 64 rows in the column role, so every sum is in-lane products plus a
// DPP reduction over the row; sums that are only written out use a
// reduce-scatter (one lane per value) instead of a full reduction. Keeping dS
// twice costs 3 instructions per element per step; reducing the five column
// sums across waves instead would cost more. Every operand arrives as one
// ds_read_b128 of an LDS vector (the thread's four columns for the row role,
// its four rows for the column role) or of a packed per-column-pair record,
// consumed by plain full-rate FMAs. The only data exchanged between waves is
// dsa (64 floats, needed by the column role): one LDS vector and one barrier
// per step, with the column-role work scheduled between write and barrier.
#include "wkv7_device.hpp"
#include "wkv7_launch.hpp"

namespace wkv7 {
namespace {

constexpr int kTile = 8;   // timesteps per LDS tile

// LDS vectors per timestep (fp32, 64 entries)
enum {
  V_R = 0, V_K, V_B, V_W, V_A,   // key-indexed: row role
  V_DY, V_V, V_SA,               // value-indexed: column role (dy also row role)
  V_DWF,                         // W_SCALE * w~ * sig * (1 - sig), used at the flush
  V_COUNT
};
// per-column-pair records for the column role, float4 {x[2p], x[2p+1], y[2p], y[2p+1]}
enum { P_RK = 0, P_BW, P_AI, P_COUNT };   // {r, k}, {b, w~}, {a, 1/w~}
// staged outputs per timestep, in the order the reduce-scatters deliver them
enum { O_DV = 0, O_DR, O_DW, O_DK, O_DB, O_DA, O_COUNT };

__device__ __forceinline__ void unpack4(float* d, float4 x) {
  d[0] = x.x; d[1] = x.y; d[2] = x.z; d[3] = x.w;
}

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
  __shared__ float4 tile[2][V_COUNT][kTile][16];   // 36 KiB
  __shared__ float4 pairs[2][P_COUNT][kTile][32];  // 24 KiB
  __shared__ float ost[2][O_COUNT][kTile][kHead];  // 24 KiB
  __shared__ float4 dsab[2][16];                   // dsa of the step, by parity

  const int h = blockIdx.x, bi = blockIdx.y;
  const int tid = threadIdx.x;
  const int L = tid & 15, q = tid >> 4;
  const int sl = (tid >> 4) & 7, pp = tid & 15;   // staging (threads 0..127)
  const bool stager = tid < 16 * kTile;

  const int T = p.T, C = p.C;
  const int64_t bh = (int64_t)bi * p.H + h;
  const int64_t tstride = (int64_t)p.H * kHead;
  const int64_t tok0 = ((int64_t)bi * T * p.H + h) * kHead;

  float dSr[2][4], Sc[4][2], dSc[4][2], Pf[4][2];
#pragma unroll
  for (int c = 0; c < 4; ++c) { Sc[c][0] = 0.0f; Sc[c][1] = 0.0f; }
  if (p.dsT) {
    const float* g0 = p.dsT + bh * (kHead * kHead);
    unpack4(dSr[0], *reinterpret_cast<const float4*>(g0 + (2 * q) * kHead + 4 * L));
    unpack4(dSr[1], *reinterpret_cast<const float4*>(g0 + (2 * q + 1) * kHead + 4 * L));
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float2 x = *reinterpret_cast<const float2*>(g0 + (4 * L + c) * kHead + 2 * q);
      dSc[c][0] = x.x;
      dSc[c][1] = x.y;
    }
  } else {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      dSr[0][c] = 0.0f; dSr[1][c] = 0.0f; dSc[c][0] = 0.0f; dSc[c][1] = 0.0f;
    }
  }

  // checkpoint c holds S after step c*C + C - 1, key-major ([i][j]): its row
  // 2q+d, entries 4L .. 4L+3, is Sc[0..3][d].
  const int64_t nchunks = T / C;
  const float* ckpt_bh = p.ckpt + (bh * nchunks * kHead + 2 * q) * kHead + 4 * L;
  auto ckload = [&](int64_t c) {
    const float* src = ckpt_bh + c * (kHead * kHead);
    const float4 x0 = *reinterpret_cast<const float4*>(src);
    const float4 x1 = *reinterpret_cast<const float4*>(src + kHead);
    Pf[0][0] = x0.x; Pf[1][0] = x0.y; Pf[2][0] = x0.z; Pf[3][0] = x0.w;
    Pf[0][1] = x1.x; Pf[1][1] = x1.y; Pf[2][1] = x1.z; Pf[3][1] = x1.w;
  };
  int64_t next_chunk = nchunks - 1;
  if (next_chunk >= 0) ckload(next_chunk);

  typedef Io<Tin> io;
  typename io::raw pre[7];
  float4 pre_sa;
  auto gload = [&](int t0) {
    if (stager && t0 + sl < T) {
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
    if (stager && t0 + sl < T) {
      const float4 x = io::widen(pre[0]);
      const float xs[4] = {x.x, x.y, x.z, x.w};
      float ws[4], iws[4], dws[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float sig = sigmoid_f(xs[c]);
        ws[c] = decay_f(sig);
        iws[c] = 1.0f / ws[c];
        dws[c] = kWScale * ws[c] * sig * (1.0f - sig);
      }
      const float4 r = io::widen(pre[1]), k = io::widen(pre[2]), a = io::widen(pre[4]);
      const float4 b = io::widen(pre[5]);
      const float4 w = make_float4(ws[0], ws[1], ws[2], ws[3]);
      const float4 iw = make_float4(iws[0], iws[1], iws[2], iws[3]);
      tile[buf][V_R][sl][pp] = r;
      tile[buf][V_K][sl][pp] = k;
      tile[buf][V_B][sl][pp] = b;
      tile[buf][V_W][sl][pp] = w;
      tile[buf][V_A][sl][pp] = a;
      tile[buf][V_DY][sl][pp] = io::widen(pre[6]);
      tile[buf][V_V][sl][pp] = io::widen(pre[3]);
      tile[buf][V_SA][sl][pp] = pre_sa;
      tile[buf][V_DWF][sl][pp] = make_float4(dws[0], dws[1], dws[2], dws[3]);
      // columns 4pp .. 4pp+3 are column pairs 2pp and 2pp+1
      pairs[buf][P_RK][sl][2 * pp] = make_float4(r.x, r.y, k.x, k.y);
      pairs[buf][P_RK][sl][2 * pp + 1] = make_float4(r.z, r.w, k.z, k.w);
      pairs[buf][P_BW][sl][2 * pp] = make_float4(b.x, b.y, w.x, w.y);
      pairs[buf][P_BW][sl][2 * pp + 1] = make_float4(b.z, b.w, w.z, w.w);
      pairs[buf][P_AI][sl][2 * pp] = make_float4(a.x, a.y, iw.x, iw.y);
      pairs[buf][P_AI][sl][2 * pp + 1] = make_float4(a.z, a.w, iw.z, iw.w);
    }
  };

  int until_reload = 0;   // steps until the next checkpoint reload
  int parity = 0;

  auto step = [&](int buf, int s) {
    if (until_reload == 0) {   // (t + 1) % C == 0, kernel.rs:210-228
      until_reload = C;
#pragma unroll
      for (int c = 0; c < 4; ++c) { Sc[c][0] = Pf[c][0]; Sc[c][1] = Pf[c][1]; }
      --next_chunk;
      if (next_chunk >= 0) ckload(next_chunk);
    }
    --until_reload;

    // row role operands: columns 4L..4L+3, rows 2q, 2q+1
    float rr[4], kk[4], bb[4];
    unpack4(rr, tile[buf][V_R][s][L]);
    unpack4(kk, tile[buf][V_K][s][L]);
    unpack4(bb, tile[buf][V_B][s][L]);
    const float2 dyr = reinterpret_cast<const float2*>(tile[buf][V_DY][s])[q];
    // column role operands: rows 4L..4L+3, columns 2q, 2q+1
    float dy[4], v[4], sa[4];
    unpack4(dy, tile[buf][V_DY][s][L]);
    unpack4(v, tile[buf][V_V][s][L]);
    unpack4(sa, tile[buf][V_SA][s][L]);
    const float4 prk = pairs[buf][P_RK][s][q], pbw = pairs[buf][P_BW][s][q];
    const float4 pai = pairs[buf][P_AI][s][q];
    const float rc[2] = {prk.x, prk.y}, kc[2] = {prk.z, prk.w};
    const float bc[2] = {pbw.x, pbw.y}, wc[2] = {pbw.z, pbw.w};
    const float ac[2] = {pai.x, pai.y}, iwc[2] = {pai.z, pai.w};

    // row role: dS row += dy r^T (kernel.rs:248); dv, dsa (kernel.rs:261-262)
    const float dyd[2] = {dyr.x, dyr.y};
    float dvp[2] = {0.0f, 0.0f};
    float dsa0 = 0.0f, dsa1 = 0.0f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      dSr[0][c] = __builtin_fmaf(dyd[0], rr[c], dSr[0][c]);
      dSr[1][c] = __builtin_fmaf(dyd[1], rr[c], dSr[1][c]);
      dvp[0] = __builtin_fmaf(dSr[0][c], kk[c], dvp[0]);
      dvp[1] = __builtin_fmaf(dSr[1][c], kk[c], dvp[1]);
      dsa0 = __builtin_fmaf(dSr[0][c], bb[c], dsa0);
      dsa1 = __builtin_fmaf(dSr[1][c], bb[c], dsa1);
    }
    row16_sum2(dsa0, dsa1, L);
    if (L == 0) reinterpret_cast<float2*>(dsab[parity])[q] = make_float2(dsa0, dsa1);

    // column role: dr from S_t; rebuild S_{t-1}; dS col += dy r; dw~, dk, db
    float drp[2] = {0.0f, 0.0f}, dwp[2] = {0.0f, 0.0f}, dkp[2] = {0.0f, 0.0f};
    float dbp[2] = {0.0f, 0.0f};
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int d = 0; d < 2; ++d) {
        drp[d] = __builtin_fmaf(Sc[c][d], dy[c], drp[d]);   // kernel.rs:230-237
        // ((S - k v) - b sa) / w~, kernel.rs:239-246
        Sc[c][d] = __builtin_fmaf(-bc[d], sa[c], __builtin_fmaf(-kc[d], v[c], Sc[c][d])) * iwc[d];
        dSc[c][d] = __builtin_fmaf(rc[d], dy[c], dSc[c][d]);   // kernel.rs:249
        dwp[d] = __builtin_fmaf(dSc[c][d], Sc[c][d], dwp[d]);   // kernel.rs:258-264
        dkp[d] = __builtin_fmaf(dSc[c][d], v[c], dkp[d]);
        dbp[d] = __builtin_fmaf(dSc[c][d], sa[c], dbp[d]);
      }
    // dv (rows 2q, 2q+1) and dr, dw~, dk (columns 2q, 2q+1): one lane pair each
    float early[8] = {dvp[0], dvp[1], drp[0], drp[1], dwp[0], dwp[1], dkp[0], dkp[1]};
    row16_scatter<8>(early, L);
    if ((L & 1) == 0) ost[buf][O_DV + (L >> 2)][s][2 * q + ((L >> 1) & 1)] = early[0];

    __syncthreads();   // dsa of every row visible
    float ds[4];
    unpack4(ds, dsab[parity][L]);
    parity ^= 1;

    // row role: dS row = dS row * w~ + dsa a^T (kernel.rs:290-291)
    float ww[4], aa[4];
    unpack4(ww, tile[buf][V_W][s][L]);
    unpack4(aa, tile[buf][V_A][s][L]);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      dSr[0][c] = __builtin_fmaf(dsa0, aa[c], dSr[0][c] * ww[c]);
      dSr[1][c] = __builtin_fmaf(dsa1, aa[c], dSr[1][c] * ww[c]);
    }
    // column role: da = S_{t-1}^T dsa (kernel.rs:280-287); dS col = dS col * w~ + a dsa
    float dap[2] = {0.0f, 0.0f};
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int d = 0; d < 2; ++d) {
        dap[d] = __builtin_fmaf(Sc[c][d], ds[c], dap[d]);
        dSc[c][d] = __builtin_fmaf(ac[d], ds[c], dSc[c][d] * wc[d]);   // kernel.rs:293-294
      }
    // db, da (columns 2q, 2q+1): four lanes each
    float late[4] = {dbp[0], dbp[1], dap[0], dap[1]};
    row16_scatter<4>(late, L);
    if ((L & 3) == 0) ost[buf][O_DB + (L >> 3)][s][2 * q + ((L >> 2) & 1)] = late[0];
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
    for (int s = nst - 1; s >= 0; --s) step(buf, s);
    if (ti > 0) lstore(buf ^ 1, t0 - kTile);
    __syncthreads();
    if (stager && sl < nst) {
      const int64_t off = tok0 + (int64_t)(t0 + sl) * tstride + 4 * pp;
      float4 dw = reinterpret_cast<const float4*>(ost[buf][O_DW][sl])[pp];
      const float4 f = tile[buf][V_DWF][sl][pp];
      dw.x *= f.x; dw.y *= f.y; dw.z *= f.z; dw.w *= f.w;   // kernel.rs:267-271
      io::store(p.dw + off, dw);
      io::store(p.dr + off, reinterpret_cast<const float4*>(ost[buf][O_DR][sl])[pp]);
      io::store(p.dk + off, reinterpret_cast<const float4*>(ost[buf][O_DK][sl])[pp]);
      io::store(p.dv + off, reinterpret_cast<const float4*>(ost[buf][O_DV][sl])[pp]);
      io::store(p.da + off, reinterpret_cast<const float4*>(ost[buf][O_DA][sl])[pp]);
      io::store(p.db + off, reinterpret_cast<const float4*>(ost[buf][O_DB][sl])[pp]);
    }
  }

  if (p.ds0) {   // kernel.rs:299-307
    float* base = p.ds0 + (bh * kHead + 2 * q) * kHead + 4 * L;
    *reinterpret_cast<float4*>(base) = make_float4(dSr[0][0], dSr[0][1], dSr[0][2], dSr[0][3]);
    *reinterpret_cast<float4*>(base + kHead) =
        make_float4(dSr[1][0], dSr[1][1], dSr[1][2], dSr[1][3]);
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
