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
// of the state in VGPRs (layout and lane-relative row order in
// wkv7_device.hpp). Rows are independent in the forward, so the only
// cross-lane work is the row sums: sa (on the step-to-step dependency chain,
// five DPP operations per step) and y (reduced once per tile for all its
// steps). Operands are staged through LDS in tiles of 16 timesteps: the raw
// rows of the next tile (one timestep of one operand is a 128/256-byte row)
// stream from global memory straight into LDS (global_load_lds_dwordx4, no
// VGPRs involved); at the tile end they are widened to fp32 with the decay
// formed once per element. The loads are in flight while the current tile is
// consumed. Per step a thread reads its four columns of w~, a, b, k, r (five
// ds_read_b128) and its two rows of v. y and sa are staged in LDS and written
// once per tile with full-row stores; checkpoints are transposed through LDS
// and written as full 256-byte rows. The tile end has a fixed cost (waits,
// two barriers, the widening pass), which the 32-step tile amortises.
#include "wkv7_device.hpp"
#include "wkv7_launch.hpp"

namespace wkv7 {
namespace {

constexpr int kTile = 32;   // timesteps per LDS tile

// raw operand rows as loaded (the order of FwdParams::in)
enum { V_W = 0, V_R, V_K, V_V, V_A, V_B, V_COUNT };
// fp32 LDS vectors per timestep: the per-column operands, v, and v with each
// row pair swapped (read by the upper half-rows, which hold (2q+1, 2q))
enum { L_W = 0, L_R, L_K, L_A, L_B, L_V, L_VS, L_COUNT };

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

// Checkpoint placement, fixed at compile time where it can be:
//   kCkTile  C is a multiple of kTile: every tile is full (T is a multiple of
//            C) and a checkpoint falls on a tile end or nowhere;
//   kCkHalf  C == kTile / 2 (the reference's 16) and T a multiple of kTile:
//            full tiles, checkpoints after steps kTile/2 - 1 and kTile - 1;
//   kCkAny   anything else: the last tile may be partial and a checkpoint may
//            fall on any step (stored directly, uncoalesced).
// In the first two modes the steps of a tile form one branch-free block and
// checkpoints go out through an LDS transpose at the tile end.
enum CkMode { kCkAny = 0, kCkTile = 1, kCkHalf = 2 };

template <typename Tin, int kMode>
__global__ __launch_bounds__(kThreads) void wkv7_fwd_kernel(FwdParams<Tin> p) {
  constexpr int kRow = kHead * sizeof(Tin);   // bytes of one raw row
  constexpr int kRawBytes = V_COUNT * kTile * kRow;
  constexpr bool kFull = kMode != kCkAny;       // every tile full, no partial steps
  constexpr int kCkStage = kMode == kCkHalf ? 2 : kMode == kCkTile ? 1 : 0;
  constexpr int kCkPitch = kHead + 4;           // floats per staged row (16-byte aligned)
  // The swapped copy of v is read by the upper half-rows in the same
  // instruction as the plain one by the lower half-rows; it sits 128 bytes off
  // a 256-byte boundary relative to it, so the two fall into different banks.
  __shared__ float4 tile_mem[L_COUNT * kTile * 16 + 8];   // 56 KiB
  __shared__ float ost[2][kTile][kHead];        // 16 KiB: y, sa
  __shared__ float4 raw[kRawBytes / 16];        // 24 or 48 KiB
  __shared__ float ckst[kCkStage > 0 ? kCkStage : 1][kHead][kCkPitch];   // key-major staging

  // row s of LDS vector V
  static_assert(L_VS == L_COUNT - 1, "the shifted vector must be the last one");
  auto tile = [&](int V, int s) -> float4* {
    return tile_mem + (V * kTile + s) * 16 + (V == L_VS ? 8 : 0);
  };
  const int h = blockIdx.x, bi = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63;
  const int L = tid & 15, q = tid >> 4;   // columns 4L.., row pair 2q, 2q+1
  const int up = (L >> 3) & 1;
  const int ro = 2 * q + up, rt = 2 * q + 1 - up;   // own and other row
  // conversion: the decay of elements 2e, 2e+1 (e = tid % 32) of timesteps
  // tid / 32 + 16 u, then half cg widens the other operands' elements
  // 4pp .. 4pp+3 of timesteps sl + 16 u; flush: the same (cg, sl + 16 u, pp)
  const int cg = tid >> 8, sl = (tid >> 4) & 15, pp = tid & 15;
  static_assert(kTile % 16 == 0, "tile passes cover 16 timesteps");

  const int T = p.T, C = p.C;
  const int64_t bh = (int64_t)bi * p.H + h;
  const int64_t tstride = (int64_t)p.H * kHead;
  const int64_t tok0 = ((int64_t)bi * T * p.H + h) * kHead;

  float So[4], St[4];   // own and other row, columns 4L .. 4L+3
  if (p.s0) {
    const float* base = p.s0 + bh * (kHead * kHead) + 4 * L;
    const float4 x0 = *reinterpret_cast<const float4*>(base + ro * kHead);
    const float4 x1 = *reinterpret_cast<const float4*>(base + rt * kHead);
    So[0] = x0.x; So[1] = x0.y; So[2] = x0.z; So[3] = x0.w;
    St[0] = x1.x; St[1] = x1.y; St[2] = x1.z; St[3] = x1.w;
  } else {
#pragma unroll
    for (int c = 0; c < 4; ++c) { So[c] = 0.0f; St[c] = 0.0f; }
  }

  typedef Io<Tin> io;
  // Loads of one tile: 16-byte chunk c0 + lane of `raw` (row vec*kTile +
  // step) for c0 = wave base + kThreads * j. The source of a chunk moves by a
  // whole number of timesteps from tile to tile, so its address at timestep 0
  // and its timestep within the tile are computed once here.
  constexpr int kChunks = kRawBytes / 16;
  constexpr int kIssue = kChunks / kThreads;
  static_assert(kChunks % kThreads == 0, "every wave issues the same number of loads");
  const char* isrc[kIssue];
  int istep[kIssue];
#pragma unroll
  for (int j = 0; j < kIssue; ++j) {
    const int c0 = tid - lane + kThreads * j, c = c0 + lane;
    const int row = c / (kRow / 16), col = c % (kRow / 16);
    istep[j] = row % kTile;
    const Tin* base = p.in[__builtin_amdgcn_readfirstlane(c0 / (kRow / 16)) / kTile];
    isrc[j] = reinterpret_cast<const char*>(base + tok0 + (int64_t)istep[j] * tstride) + 16 * col;
  }
  // Issue the loads of tile [t0, t0+nst) into `raw`.
  auto issue = [&](int t0, int nst) {
    const int64_t shift = (int64_t)t0 * tstride * (int64_t)sizeof(Tin);   // bytes, uniform
#pragma unroll
    for (int j = 0; j < kIssue; ++j)
      if (kMode != kCkAny || istep[j] < nst) load_lds16(isrc[j] + shift, &raw[tid - lane + kThreads * j]);
  };
  // raw tile -> fp32 vectors; the decay w~ is formed here, once per element
  auto convert = [&](int nst) {
    const char* rb = reinterpret_cast<const char*>(raw);
#pragma unroll
    for (int u = 0; u < kTile / 16; ++u) {   // w -> w~, two elements per thread and pass
      const int ws_ = (tid >> 5) + 16 * u, e = tid & 31;
      if (ws_ < nst) {
        float2 x;
        if constexpr (sizeof(Tin) == 2) {
          const uint32_t u = reinterpret_cast<const uint32_t*>(rb + (V_W * kTile + ws_) * kRow)[e];
          x = make_float2(bf16_to_f32(u & 0xffffu), bf16_to_f32(u >> 16));
        } else {
          x = reinterpret_cast<const float2*>(rb + (V_W * kTile + ws_) * kRow)[e];
        }
        reinterpret_cast<float2*>(tile(L_W, ws_))[e] =
            make_float2(decay_f(sigmoid_f(x.x)), decay_f(sigmoid_f(x.y)));
      }
    }
#pragma unroll
    for (int u = 0; u < kTile / 16; ++u) {
      const int st = sl + 16 * u;
      if (st >= nst) break;
      auto rawv = [&](int vec) {
        return io::widen(*reinterpret_cast<const typename io::raw*>(
            rb + (vec * kTile + st) * kRow + 4 * pp * sizeof(Tin)));
      };
      if (cg == 0) {
        tile(L_R, st)[pp] = rawv(V_R);
        tile(L_K, st)[pp] = rawv(V_K);
      } else {
        const float4 v = rawv(V_V);
        tile(L_V, st)[pp] = v;
        tile(L_VS, st)[pp] = make_float4(v.y, v.x, v.w, v.z);
        tile(L_A, st)[pp] = rawv(V_A);
        tile(L_B, st)[pp] = rawv(V_B);
      }
    }
  };
  // (own, other) rows of v for this thread, per step: 32 float2 per step row
  const float2* vrow = reinterpret_cast<const float2*>(tile(up ? L_VS : L_V, 0)) + q;

  // checkpoint c: S after step c*C + C - 1, stored key-major ([i][j]); the
  // thread writes (S[2q][i], S[2q+1][i]) for its four columns i
  float* ckpt_h = p.ckpt + bh * (T / C) * (kHead * kHead);
  auto ck_store = [&](int64_t c) {
    float* dst = ckpt_h + c * (kHead * kHead) + 4 * L * kHead + 2 * q;
#pragma unroll
    for (int m = 0; m < 4; ++m)
      *reinterpret_cast<float2*>(dst + m * kHead) =
          up ? make_float2(St[m], So[m]) : make_float2(So[m], St[m]);
  };
  // the same through LDS: stage the thread's block key-major, then (after a
  // barrier) every thread writes two 16-byte pieces of full rows
  auto ck_stage = [&](int b, const float* o, const float* t) {
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      ckst[b][4 * L + m][ro] = o[m];
      ckst[b][4 * L + m][rt] = t[m];
    }
  };
  auto ck_flush = [&](int b, int64_t c) {
    float* dst = ckpt_h + c * (kHead * kHead);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int e = tid + u * kThreads;    // float4 index in the 64x64 checkpoint
      const int i = e >> 4, j4 = (e & 15) * 4;
      *reinterpret_cast<float4*>(dst + i * kHead + j4) =
          *reinterpret_cast<const float4*>(&ckst[b][i][j4]);
    }
  };
  float Co[4], Ct[4];   // state after step kTile/2 - 1 (kCkHalf)
  int until_ckpt = C;   // steps until the next checkpoint (unaligned C)
  int64_t chunk = 0;

  // Tile pipeline. While tile ti is computed, the raw operands of tile ti+1
  // stream into LDS. At the tile end one wait + barrier makes them visible;
  // the outputs of tile ti are flushed and tile ti+1 is converted to fp32, a
  // barrier, and the loads for tile ti+2 are issued.
  const int ntiles = (T + kTile - 1) / kTile;
  auto tile_n = [&](int ti) { return min(kTile, T - ti * kTile); };
  if (ntiles > 0) {
    issue(0, tile_n(0));
    __builtin_amdgcn_s_waitcnt(0);
    lds_barrier();
    convert(tile_n(0));
    lds_barrier();
    if (ntiles > 1) issue(kTile, tile_n(1));
  }

  for (int ti = 0; ti < ntiles; ++ti) {
    const int t0 = ti * kTile, nst = tile_n(ti);

    // y partials of both rows for every step, [own block | other block]
    float yp[2 * kTile];
    float sav[kTile];   // sa of the own row
#pragma unroll
    for (int s = 0; s < kTile; ++s) {
      if constexpr (!kFull) {
        if (s >= nst) {   // uniform: the last tile may be partial
          yp[s] = yp[kTile + s] = sav[s] = 0.0f;
          continue;
        }
      }
      float sa_t;
      fwd_step(So, St, tile(L_W, s)[L], tile(L_A, s)[L], tile(L_B, s)[L], tile(L_K, s)[L],
               tile(L_R, s)[L], vrow[s * 32], sav[s], sa_t, yp[s], yp[kTile + s]);
      if constexpr (kMode == kCkAny) {
        if (--until_ckpt == 0) {   // (t + 1) % C == 0, kernel.rs:89-102
          until_ckpt = C;
          ck_store(chunk++);
        }
      }
      if constexpr (kMode == kCkHalf) {
        if (s == kTile / 2 - 1) {
#pragma unroll
          for (int m = 0; m < 4; ++m) { Co[m] = So[m]; Ct[m] = St[m]; }
        }
      }
    }
    // y of the own row for steps 2(L&7) and 2(L&7)+1
    row16_reduce_scatter<2 * kTile>(yp, L);
    // y of the own row for steps kTile/8 * (L&7) ..
#pragma unroll
    for (int u = 0; u < kTile / 8; ++u) ost[0][kTile / 8 * (L & 7) + u][ro] = yp[u];
    if ((L & 7) == 0) {
#pragma unroll
      for (int s = 0; s < kTile; ++s) ost[1][s][ro] = sav[s];
    }
    // checkpoints (kernel.rs:89-102) of this tile into the staging buffer
    const bool ck_end = kMode == kCkHalf || (kMode == kCkTile && (t0 + kTile) % C == 0);
    if constexpr (kMode == kCkHalf) ck_stage(1, Co, Ct);
    if (kMode != kCkAny && ck_end) ck_stage(0, So, St);

    // The loads of tile ti+1 have landed once vmcnt reaches 0 (they and the
    // stores of the previous tile end were issued a whole tile ago). Only LDS
    // is fenced by the barriers, so the stores below are not waited for until
    // the next tile end.
    __builtin_amdgcn_s_waitcnt(0);
    lds_barrier();
    if constexpr (kMode == kCkHalf) ck_flush(1, (t0 + kTile) / C - 2);
    if (kMode != kCkAny && ck_end) ck_flush(0, (t0 + kTile) / C - 1);
#pragma unroll
    for (int u = 0; u < kTile / 16; ++u) {   // cg 0 writes y, cg 1 writes sa
      const int st = sl + 16 * u;
      if (st < nst) {
        const int64_t off = tok0 + (int64_t)(t0 + st) * tstride + 4 * pp;
        const float4 x = reinterpret_cast<const float4*>(ost[cg][st])[pp];
        if (cg == 0) io::store(p.y + off, x);
        else *reinterpret_cast<float4*>(p.sa + off) = x;
      }
    }
    if (ti + 1 < ntiles) convert(tile_n(ti + 1));
    lds_barrier();   // converted tile visible; `raw` free for the next loads
    if (ti + 2 < ntiles) issue((ti + 2) * kTile, tile_n(ti + 2));
  }

  if (p.sT) {
    float* base = p.sT + bh * (kHead * kHead) + 4 * L;
    *reinterpret_cast<float4*>(base + ro * kHead) = make_float4(So[0], So[1], So[2], So[3]);
    *reinterpret_cast<float4*>(base + rt * kHead) = make_float4(St[0], St[1], St[2], St[3]);
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
  const dim3 grid(d.H, d.B, 1), block(kThreads, 1, 1);
  if (d.C % kTile == 0)
    hipLaunchKernelGGL((wkv7_fwd_kernel<Tin, kCkTile>), grid, block, 0, stream, p);
  else if (d.C == kTile / 2 && d.T % kTile == 0)
    hipLaunchKernelGGL((wkv7_fwd_kernel<Tin, kCkHalf>), grid, block, 0, stream, p);
  else
    hipLaunchKernelGGL((wkv7_fwd_kernel<Tin, kCkAny>), grid, block, 0, stream, p);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_forward(const ForwardDesc& d, hipStream_t stream) {
  if (d.B == 0 || d.H == 0) return hipSuccess;
  if (!d.kc.step_only) {
    if (chunk_forward_supported(d)) return launch_forward_chunked(d, stream);
    if (chunk_f32_forward_supported(d)) return launch_forward_chunked_f32(d, stream);
  }
  return d.dtype == Dtype::BF16 ? launch_fwd_t<bf16_t>(d, stream) : launch_fwd_t<float>(d, stream);
}

}  // namespace wkv7
