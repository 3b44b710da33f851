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
// timesteps: the raw rows of the next tile (one timestep of one operand is a
// 128/256-byte row) stream from global memory straight into LDS
// (global_load_lds_dwordx4, no VGPRs involved); at the tile end they are
// widened to fp32 with the decay formed once per element. The loads are in
// flight while the current tile is consumed. Per step a thread reads its four
// columns of w~, a, b, k, r (five ds_read_b128) and its two rows of v. y and
// sa are staged in LDS and written once per tile with full-row stores.
#include "wkv7_device.hpp"
#include "wkv7_launch.hpp"

namespace wkv7 {
namespace {

constexpr int kTile = 16;   // timesteps per LDS tile

// LDS operand vectors per timestep (fp32), and raw rows as loaded
enum { V_W = 0, V_R, V_K, V_V, V_A, V_B, V_COUNT };

struct StepOps {
  float4 w, a, b, k, r;   // columns 4L .. 4L+3
  float2 v;               // rows 2q, 2q+1
};

template <typename Tin>
struct FwdParams {
  const Tin* in[V_COUNT];   // w, r, k, v, a, b (V_* order)
  const float* s0;
  float* ckpt;
  float* sa;
  Tin* y;
  float* sT;
  int T, H, C;
};

// kDefer: C >= kTile, so a tile holds at most one checkpoint, which is kept in
// registers and stored at the tile end instead of in the middle of the steps.
template <typename Tin, bool kDefer>
__global__ __launch_bounds__(kThreads) void wkv7_fwd_kernel(FwdParams<Tin> p) {
  constexpr int kRow = kHead * sizeof(Tin);   // bytes of one raw row
  constexpr int kRawBytes = V_COUNT * kTile * kRow;
  __shared__ float4 tile[V_COUNT][kTile][16];   // 24 KiB
  __shared__ float ost[2][kTile][kHead];        // 8 KiB: y, sa
  __shared__ float4 raw[kRawBytes / 16];        // 12 or 24 KiB

  const int h = blockIdx.x, bi = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63;
  const int L = tid & 15, q = tid >> 4;   // columns 4L.., rows 2q, 2q+1
  // conversion and flush: timestep sl, elements 4pp .. 4pp+3, half cg
  const int cg = tid >> 8, sl = (tid >> 4) & 15, pp = tid & 15;

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
  // Issue the loads of tile [t0, t0+nst) into `raw` (row vec*kTile + step).
  auto issue = [&](int t0, int nst) {
    constexpr int kChunks = kRawBytes / 16;
    for (int c0 = tid - lane; c0 < kChunks; c0 += kThreads) {   // wave-uniform loop
      const int c = c0 + lane;
      const int row = c / (kRow / 16), col = c % (kRow / 16);
      const int step = row % kTile;
      const int vec = __builtin_amdgcn_readfirstlane(c0 / (kRow / 16)) / kTile;
      const Tin* base = p.in[vec];   // kernel-argument array, uniform index
      const char* src =
          reinterpret_cast<const char*>(base + tok0 + (int64_t)(t0 + step) * tstride) + 16 * col;
      if (step < nst) load_lds16(src, &raw[c0]);
    }
  };
  // raw tile -> fp32 vectors; the decay w~ is formed here, once per element
  auto convert = [&](int nst) {
    if (sl >= nst) return;
    const char* rb = reinterpret_cast<const char*>(raw);
    auto rawv = [&](int vec) {
      return io::widen(*reinterpret_cast<const typename io::raw*>(
          rb + (vec * kTile + sl) * kRow + 4 * pp * sizeof(Tin)));
    };
    if (cg == 0) {
      float4 x = rawv(V_W);
      x.x = decay_f(sigmoid_f(x.x));
      x.y = decay_f(sigmoid_f(x.y));
      x.z = decay_f(sigmoid_f(x.z));
      x.w = decay_f(sigmoid_f(x.w));
      tile[V_W][sl][pp] = x;
      tile[V_R][sl][pp] = rawv(V_R);
      tile[V_K][sl][pp] = rawv(V_K);
    } else {
      tile[V_V][sl][pp] = rawv(V_V);
      tile[V_A][sl][pp] = rawv(V_A);
      tile[V_B][sl][pp] = rawv(V_B);
    }
  };
  auto lread = [&](int s) {
    StepOps o;
    o.w = tile[V_W][s][L];
    o.a = tile[V_A][s][L];
    o.b = tile[V_B][s][L];
    o.k = tile[V_K][s][L];
    o.r = tile[V_R][s][L];
    o.v = reinterpret_cast<const float2*>(tile[V_V][s])[q];
    return o;
  };

  // checkpoint c: S after step c*C + C - 1, stored key-major ([i][j])
  const int C = p.C;
  const int64_t nchunks = T / C;
  float* ckpt_bh = p.ckpt + (bh * nchunks * kHead + 4 * L) * kHead + 2 * q;
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

  auto step = [&](const StepOps& o, int s) {
    float sa0, sa1, y;
    fwd_step(S0, S1, o.w, o.a, o.b, o.k, o.r, o.v, L, sa0, sa1, y);
    if ((L & 7) == 0) ost[0][s][2 * q + (L >> 3)] = y;
    if (L == 0) reinterpret_cast<float2*>(ost[1][s])[q] = make_float2(sa0, sa1);
    if (--until_ckpt == 0) {   // (t + 1) % C == 0, kernel.rs:89-102
      until_ckpt = C;
      if constexpr (kDefer) {
#pragma unroll
        for (int m = 0; m < 4; ++m) { Ck0[m] = S0[m]; Ck1[m] = S1[m]; }
        ck_pending = true;
      } else {
        ck_store(chunk++, S0, S1);
      }
    }
  };

  // Tile pipeline. While tile ti is computed, the raw operands of tile ti+1
  // stream into LDS. At the tile end one wait + barrier makes them visible;
  // the outputs of tile ti are flushed and tile ti+1 is converted to fp32, a
  // barrier, and the loads for tile ti+2 are issued.
  const int ntiles = (T + kTile - 1) / kTile;
  auto tile_n = [&](int ti) { return min(kTile, T - ti * kTile); };
  if (ntiles > 0) {
    issue(0, tile_n(0));
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    convert(tile_n(0));
    __syncthreads();
    if (ntiles > 1) issue(kTile, tile_n(1));
  }

  for (int ti = 0; ti < ntiles; ++ti) {
    const int t0 = ti * kTile, nst = tile_n(ti);

    // Two operand sets alternate so that the reads for step s+1 are in flight
    // while step s computes, without register copies between iterations.
    StepOps A = lread(0);
    int s = 0;
    for (; s + 1 < nst; s += 2) {
      const StepOps Bo = lread(s + 1);
      step(A, s);
      A = lread(min(s + 2, nst - 1));
      step(Bo, s + 1);
    }
    if (s < nst) step(A, s);

    if (ck_pending) {
      ck_store(chunk++, Ck0, Ck1);
      ck_pending = false;
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (sl < nst) {   // cg 0 writes y, cg 1 writes sa
      const int64_t off = tok0 + (int64_t)(t0 + sl) * tstride + 4 * pp;
      const float4 x = reinterpret_cast<const float4*>(ost[cg][sl])[pp];
      if (cg == 0) io::store(p.y + off, x);
      else *reinterpret_cast<float4*>(p.sa + off) = x;
    }
    if (ti + 1 < ntiles) convert(tile_n(ti + 1));
    __syncthreads();
    if (ti + 2 < ntiles) issue((ti + 2) * kTile, tile_n(ti + 2));
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
  p.in[V_W] = static_cast<const Tin*>(d.w);
  p.in[V_R] = static_cast<const Tin*>(d.r);
  p.in[V_K] = static_cast<const Tin*>(d.k);
  p.in[V_V] = static_cast<const Tin*>(d.v);
  p.in[V_A] = static_cast<const Tin*>(d.a);
  p.in[V_B] = static_cast<const Tin*>(d.b);
  p.s0 = d.s0;
  p.ckpt = d.ckpt;
  p.sa = d.sa;
  p.y = static_cast<Tin*>(d.y);
  p.sT = d.sT;
  p.T = d.T;
  p.H = d.H;
  p.C = d.C;
  if (d.C >= kTile)
    hipLaunchKernelGGL((wkv7_fwd_kernel<Tin, true>), dim3(d.H, d.B, 1), dim3(kThreads, 1, 1), 0,
                       stream, p);
  else
    hipLaunchKernelGGL((wkv7_fwd_kernel<Tin, false>), dim3(d.H, d.B, 1), dim3(kThreads, 1, 1), 0,
                       stream, p);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_forward(const ForwardDesc& d, hipStream_t stream) {
  if (d.B == 0 || d.H == 0) return hipSuccess;
  return d.dtype == Dtype::BF16 ? launch_fwd_t<bf16_t>(d, stream) : launch_fwd_t<float>(d, stream);
}

}  // namespace wkv7
