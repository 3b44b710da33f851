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
// Design. One 256-thread workgroup per (b, h); thread (e, hi) keeps state row
// e, columns 16*hi..16*hi+15 in VGPRs (16 fp32), so the four waves of the
// workgroup cover the 64x64 state with no cross-wave traffic at all: rows are
// independent in the forward. Operands are staged through LDS in tiles of 16
// timesteps: all 256 threads load one tile with coalesced 8/16-byte loads
// (one timestep of one operand is a 128/256-byte row), widen bf16 to fp32 and
// compute the decay once per element, and the next tile's global loads are in
// flight while the current tile is consumed (double-buffered LDS). Per step a
// thread reads five quad-distributed operand vectors (ds_read_b128 each) and
// its own v_e, then does 5 VALU instructions per state element, all with a
// DPP quad broadcast for the column operand, plus two 2-step DPP reductions
// (sa and y over the four segments of a row). y and sa are staged in LDS and
// written once per tile with full-row stores.
#include "wkv7_device.hpp"
#include "wkv7_launch.hpp"

namespace wkv7 {
namespace {

constexpr int kTile = 16;   // timesteps per LDS tile

// LDS operand vectors per timestep
enum { V_W = 0, V_R, V_K, V_V, V_A, V_B, V_COUNT };

struct StepOps {
  float4 w, r, k, a, b;
  float ve;
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
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int L = lane & 15, g = lane >> 4, lo = L & 3, hi = L >> 2;
  const int e = 16 * wave + 4 * g + lo;   // state row owned by this thread
  const int sl = tid >> 4, pp = tid & 15; // staging: timestep, 4-element part

  const int T = p.T;
  const int64_t bh = (int64_t)bi * p.H + h;
  const int64_t tstride = (int64_t)p.H * kHead;
  const int64_t tok0 = ((int64_t)bi * T * p.H + h) * kHead;

  float S[16];
  if (p.s0) {
    const float4* src = reinterpret_cast<const float4*>(p.s0 + (bh * kHead + e) * kHead + 16 * hi);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float4 x = src[q];
      S[4 * q] = x.x; S[4 * q + 1] = x.y; S[4 * q + 2] = x.z; S[4 * q + 3] = x.w;
    }
  } else {
#pragma unroll
    for (int m = 0; m < 16; ++m) S[m] = 0.0f;
  }

  typedef Io<Tin> io;
  typename io::raw pre[V_COUNT];
  auto gload = [&](int t0) {
    if (t0 + sl < T) {
      const int64_t off = tok0 + (int64_t)(t0 + sl) * tstride + 4 * pp;
      pre[V_W] = io::load(p.w + off);
      pre[V_R] = io::load(p.r + off);
      pre[V_K] = io::load(p.k + off);
      pre[V_V] = io::load(p.v + off);
      pre[V_A] = io::load(p.a + off);
      pre[V_B] = io::load(p.b + off);
    }
  };
  auto lstore = [&](int buf, int t0) {
    if (t0 + sl < T) {
      float4 x = io::widen(pre[V_W]);
      x.x = decay_f(sigmoid_f(x.x));
      x.y = decay_f(sigmoid_f(x.y));
      x.z = decay_f(sigmoid_f(x.z));
      x.w = decay_f(sigmoid_f(x.w));
      tile[buf][V_W][sl][pp] = x;
      tile[buf][V_R][sl][pp] = io::widen(pre[V_R]);
      tile[buf][V_K][sl][pp] = io::widen(pre[V_K]);
      tile[buf][V_V][sl][pp] = io::widen(pre[V_V]);
      tile[buf][V_A][sl][pp] = io::widen(pre[V_A]);
      tile[buf][V_B][sl][pp] = io::widen(pre[V_B]);
    }
  };
  auto lread = [&](int buf, int s) {
    StepOps o;
    o.w = tile[buf][V_W][s][L];
    o.r = tile[buf][V_R][s][L];
    o.k = tile[buf][V_K][s][L];
    o.a = tile[buf][V_A][s][L];
    o.b = tile[buf][V_B][s][L];
    o.ve = reinterpret_cast<const float*>(tile[buf][V_V][s])[e];
    return o;
  };

  const int ntiles = (T + kTile - 1) / kTile;
  if (ntiles > 0) {
    gload(0);
    lstore(0, 0);
  }
  __syncthreads();

  int until_ckpt = p.C;
  int64_t chunk = 0;
  const int64_t nchunks = T / p.C;
  float* ckpt_bh = p.ckpt + bh * nchunks * (kHead * kHead) + (16 * hi) * kHead + e;

  auto step = [&](const StepOps& o, int buf, int s) {
    float sa0 = 0.0f, sa1 = 0.0f;
    fwd_sa16(sa0, sa1, o.a, S);
    const float sa = seg_sum(sa0 + sa1);
    float y0 = 0.0f, y1 = 0.0f;
    fwd_upd8_q0(S, y0, y1, o.w, o.b, o.k, o.r, sa, o.ve);
    fwd_upd8_q2(S + 8, y0, y1, o.w, o.b, o.k, o.r, sa, o.ve);
    const float y = seg_sum(y0 + y1);
    ost[buf][0][s][e] = y;
    ost[buf][1][s][e] = sa;
    if (--until_ckpt == 0) {   // (t + 1) % C == 0, kernel.rs:89-102
      until_ckpt = p.C;
      float* dst = ckpt_bh + chunk * (kHead * kHead);
#pragma unroll
      for (int m = 0; m < 16; ++m) dst[m * kHead] = S[m];
      ++chunk;
    }
  };

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
    __syncthreads();
    if (sl < nst) {
      const int64_t off = tok0 + (int64_t)(t0 + sl) * tstride + 4 * pp;
      io::store(p.y + off, reinterpret_cast<const float4*>(ost[buf][0][sl])[pp]);
      *reinterpret_cast<float4*>(p.sa + off) = reinterpret_cast<const float4*>(ost[buf][1][sl])[pp];
    }
  }

  if (p.sT) {
    float4* dst = reinterpret_cast<float4*>(p.sT + (bh * kHead + e) * kHead + 16 * hi);
#pragma unroll
    for (int q = 0; q < 4; ++q)
      dst[q] = make_float4(S[4 * q], S[4 * q + 1], S[4 * q + 2], S[4 * q + 3]);
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
