// WKV7 forward recurrence for gfx950.
//
// Semantics: /root/reference/crates/rwkv-nn/src/kernels/wkv7_common/kernel.rs:6-114
// (wkv7_forward_kernel), per (batch b, head h), t = 0..T-1:
//   w~    = exp(W_SCALE * sigmoid(w_t))
//   sa_j  = sum_i a_i S[j,i]                    (stored: removal_state)
//   S[j,i] = S[j,i] w~_i + sa_j b_i + k_i v_j
//   y_j   = sum_i S[j,i] r_i
//   every C steps: checkpoint S^T (key-major), at the end: s_T = S
//
// Design. One 512-thread workgroup per (b, h); each thread keeps a 2x4 block
// of the state in VGPRs (layout in wkv7_device.hpp). Rows are independent in
// the forward, so the only cross-lane work is the two row sums (sa and y),
// four DPP steps each. Operands are staged through LDS in tiles of 16
// timesteps: threads load one tile with coalesced 8/16-byte loads (one
// timestep of one operand is a 128/256-byte row), widen bf16 to fp32 and
// compute the decay once per element, and the next tile's global loads are in
// flight while the current tile is consumed (double-buffered LDS). Per step a
// thread reads its four columns of w~, a, b, k, r (five ds_read_b128) and its
// two rows of v. y and sa are staged in LDS and written once per tile with
// full-row stores; a checkpoint taken inside a tile is stored at the tile end,
// after the tile's loads have been consumed, so no wait ever covers it.
#include "wkv7_device.hpp"
#include "wkv7_launch.hpp"

namespace wkv7 {
namespace {

constexpr int kTile = 16;   // timesteps per LDS tile

// LDS operand vectors per timestep
enum { V_W = 0, V_R, V_K, V_V, V_A, V_B, V_COUNT };

struct StepOps {
  float4 w, a, b, k, r;   // columns 4L .. 4L+3
  float2 v;               // rows 2q, 2q+1
};

template <typename Tin>
struct FwdParams {
  const Tin *w, *r, *k, *v, *a, *b;
  const float* s0;
  float* ckpt;
  float* sa;
  Tin* y;
  float* sT;
  int T, H, C;
};

template <typename Tin>
__global__ __launch_bounds__(kThreads) void wkv7_fwd_kernel(FwdParams<Tin> p) {
  __shared__ float4 tile[2][V_COUNT][kTile][16];   // 48 KiB
  __shared__ float ost[2][2][kTile][kHead];        // 16 KiB: y, sa

  const int h = blockIdx.x, bi = blockIdx.y;
  const int tid = threadIdx.x;
  const int L = tid & 15, q = tid >> 4;   // columns 4L.., rows 2q, 2q+1
  // staging: threads 0..255 stage w, r, k; threads 256..511 stage v, a, b
  const int st_half = tid >> 8, sl = (tid >> 4) & 15, pp = tid & 15;

  const int T = p.T;
  const int64_t bh = (int64_t)bi * p.H + h;
  const int64_t tstride = (int64_t)p.H * kHead;
  const int64_t tok0 = ((int64_t)bi * T * p.H + h) * kHead;

  float S0[4], S1[4];   // rows 2q and 2q+1, columns 4L .. 4L+3
  if (p.s0) {
    const float* base = p.s0 + (bh * kHead + 2 * q) * kHead + 4 * L;
    const float4 x0 = *reinterpret_cast<const float4*>(base);
    const float4 x1 = *reinterpret_cast<const float4*>(base + kHead);
    S0[0] = x0.x; S0[1] = x0.y; S0[2] = x0.z; S0[3] = x0.w;
    S1[0] = x1.x; S1[1] = x1.y; S1[2] = x1.z; S1[3] = x1.w;
  } else {
#pragma unroll
    for (int c = 0; c < 4; ++c) { S0[c] = 0.0f; S1[c] = 0.0f; }
  }

  typedef Io<Tin> io;
  typename io::raw pre[3];
  const Tin* src0 = st_half ? p.v : p.w;
  const Tin* src1 = st_half ? p.a : p.r;
  const Tin* src2 = st_half ? p.b : p.k;
  auto gload = [&](int t0) {
    if (t0 + sl < T) {
      const int64_t off = tok0 + (int64_t)(t0 + sl) * tstride + 4 * pp;
      pre[0] = io::load(src0 + off);
      pre[1] = io::load(src1 + off);
      pre[2] = io::load(src2 + off);
    }
  };
  auto lstore = [&](int buf, int t0) {
    if (t0 + sl < T) {
      float4 x0 = io::widen(pre[0]);
      if (!st_half) {
        x0.x = decay_f(sigmoid_f(x0.x));
        x0.y = decay_f(sigmoid_f(x0.y));
        x0.z = decay_f(sigmoid_f(x0.z));
        x0.w = decay_f(sigmoid_f(x0.w));
      }
      tile[buf][st_half ? V_V : V_W][sl][pp] = x0;
      tile[buf][st_half ? V_A : V_R][sl][pp] = io::widen(pre[1]);
      tile[buf][st_half ? V_B : V_K][sl][pp] = io::widen(pre[2]);
    }
  };
  auto lread = [&](int buf, int s) {
    StepOps o;
    o.w = tile[buf][V_W][s][L];
    o.a = tile[buf][V_A][s][L];
    o.b = tile[buf][V_B][s][L];
    o.k = tile[buf][V_K][s][L];
    o.r = tile[buf][V_R][s][L];
    o.v = reinterpret_cast<const float2*>(tile[buf][V_V][s])[q];
    return o;
  };

  // checkpoint c: S after step c*C + C - 1, stored key-major ([i][j])
  const int C = p.C;
  const int64_t nchunks = T / C;
  float* ckpt_bh = p.ckpt + (bh * nchunks * kHead + 4 * L) * kHead + 2 * q;
  const bool defer_ckpt = C >= kTile;   // at most one checkpoint per tile
  int until_ckpt = C;
  int64_t chunk = 0;
  bool ck_pending = false;
  float Ck0[4], Ck1[4];
  auto ck_store = [&](int64_t c, const float* a0, const float* a1) {
    float* dst = ckpt_bh + c * (kHead * kHead);
#pragma unroll
    for (int m = 0; m < 4; ++m)
      *reinterpret_cast<float2*>(dst + m * kHead) = make_float2(a0[m], a1[m]);
  };

  auto step = [&](const StepOps& o, int buf, int s) {
    float sa0, sa1, y;
    fwd_step(S0, S1, o.w, o.a, o.b, o.k, o.r, o.v, L, sa0, sa1, y);
    if ((L & 7) == 0) ost[buf][0][s][2 * q + (L >> 3)] = y;
    if (L == 0) reinterpret_cast<float2*>(ost[buf][1][s])[q] = make_float2(sa0, sa1);
    if (--until_ckpt == 0) {   // (t + 1) % C == 0, kernel.rs:89-102
      until_ckpt = C;
      if (defer_ckpt) {
#pragma unroll
        for (int m = 0; m < 4; ++m) { Ck0[m] = S0[m]; Ck1[m] = S1[m]; }
        ck_pending = true;
      } else {
        ck_store(chunk++, S0, S1);
      }
    }
  };

  const int ntiles = (T + kTile - 1) / kTile;
  if (ntiles > 0) {
    gload(0);
    lstore(0, 0);
  }
  __syncthreads();

  for (int ti = 0; ti < ntiles; ++ti) {
    const int buf = ti & 1;
    const int t0 = ti * kTile;
    const int nst = min(kTile, T - t0);
    if (ti + 1 < ntiles) gload(t0 + kTile);

    // Two operand sets alternate so that the reads for step s+1 are in flight
    // while step s computes, without register copies between iterations.
    StepOps A = lread(buf, 0);
    int s = 0;
    for (; s + 1 < nst; s += 2) {
      const StepOps Bo = lread(buf, s + 1);
      step(A, buf, s);
      A = lread(buf, min(s + 2, nst - 1));
      step(Bo, buf, s + 1);
    }
    if (s < nst) step(A, buf, s);

    if (ti + 1 < ntiles) lstore(buf ^ 1, t0 + kTile);
    if (ck_pending) {
      ck_store(chunk++, Ck0, Ck1);
      ck_pending = false;
    }
    __syncthreads();
    if (tid < 256 && sl < nst) {
      const int64_t off = tok0 + (int64_t)(t0 + sl) * tstride + 4 * pp;
      io::store(p.y + off, reinterpret_cast<const float4*>(ost[buf][0][sl])[pp]);
      *reinterpret_cast<float4*>(p.sa + off) = reinterpret_cast<const float4*>(ost[buf][1][sl])[pp];
    }
  }

  if (p.sT) {
    float* base = p.sT + (bh * kHead + 2 * q) * kHead + 4 * L;
    *reinterpret_cast<float4*>(base) = make_float4(S0[0], S0[1], S0[2], S0[3]);
    *reinterpret_cast<float4*>(base + kHead) = make_float4(S1[0], S1[1], S1[2], S1[3]);
  }
}

template <typename Tin>
hipError_t launch_fwd_t(const ForwardDesc& d, hipStream_t stream) {
  FwdParams<Tin> p;
  p.w = static_cast<const Tin*>(d.w);
  p.r = static_cast<const Tin*>(d.r);
  p.k = static_cast<const Tin*>(d.k);
  p.v = static_cast<const Tin*>(d.v);
  p.a = static_cast<const Tin*>(d.a);
  p.b = static_cast<const Tin*>(d.b);
  p.s0 = d.s0;
  p.ckpt = d.ckpt;
  p.sa = d.sa;
  p.y = static_cast<Tin*>(d.y);
  p.sT = d.sT;
  p.T = d.T;
  p.H = d.H;
  p.C = d.C;
  hipLaunchKernelGGL(wkv7_fwd_kernel<Tin>, dim3(d.H, d.B, 1), dim3(kThreads, 1, 1), 0, stream, p);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_forward(const ForwardDesc& d, hipStream_t stream) {
  if (d.B == 0 || d.H == 0) return hipSuccess;
  return d.dtype == Dtype::BF16 ? launch_fwd_t<bf16_t>(d, stream) : launch_fwd_t<float>(d, stream);
}

}  // namespace wkv7
